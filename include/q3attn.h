/*
 * q3attn -- MI355X (gfx950) attention for the Qwen3-TTS engine's hot path, as a C ABI.
 *
 * Every pointer is a device pointer owned by the caller.  Every entry point only enqueues kernels
 * on `stream` (a hipStream_t passed as void*; NULL = the legacy default stream): no allocation,
 * no host synchronisation, no blocking copy, so calls are capturable into a HIP graph and two
 * streams may call concurrently as long as they pass distinct output/workspace buffers.
 *
 * Strides are in elements.  Return value: 0 on success, or a negative Q3A_E* code; the message
 * for the last failure on the calling thread is in q3a_last_error().  The library never prints
 * and never aborts.
 */
#ifndef Q3ATTN_H
#define Q3ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define Q3A_OK 0
#define Q3A_EINVAL (-22)  /* bad shape, stride, alignment or argument */
#define Q3A_ELAUNCH (-5)  /* the HIP runtime refused the launch */
#define Q3A_ESPACE (-28)  /* workspace smaller than q3a_paged_decode_workspace_bytes() */

/* ABI version of this header (bumped on any signature change or new entry point); q3a_abi_version() returns the
 * library's.  2: K and V carry separate strides in the prefill and code-predictor entry points.  3: q3a_prefill_append.  4: q3a_paged_decode_append_rope.
 * 5: q3a_prefill_dense_append.  6: q3a_prefill_dense_append_rope, q3a_prefill_append_rope,
 * q3a_cp_attn_append_rope.  7: the decode path codes below (negative split_tokens).  8: per-frame decode plans
 * (q3a_paged_decode_plan_bytes, q3a_paged_decode_plan, Q3A_DECODE_PLANNED). */
#define Q3A_ABI_VERSION 8

/* Decode decomposition codes, passed as split_tokens to the q3a_paged_decode* entry points (0 lets the library
 * choose, a positive multiple of 16 is a fixed split of that many tokens):
 *   Q3A_DECODE_ROW      one workgroup per (row, KV head), the row's tiles over its waves, one launch (tables of at
 *                       most 2,048 tokens)
 *   Q3A_DECODE_CHUNKS   the same kernel over chunks of 128 or more tokens of each row, so one row's tiles spread
 *                       over many workgroups, then a combine launch that merges the chunks' fp32 (m, l, o) records
 *                       (small batches of long rows; tables of at most 131,072 tokens)
 *   Q3A_DECODE_STREAMK  stream-K: a resident grid over all rows' 16-token tiles, then a combine (batch <= 4096)
 * A code that does not take the shape returns Q3A_EINVAL.  Every decomposition computes the same attention; they
 * differ in the order of the fp32 reductions. */
#define Q3A_DECODE_ROW (-1)
#define Q3A_DECODE_CHUNKS (-2)
#define Q3A_DECODE_STREAMK (-3)
/*   Q3A_DECODE_PLANNED  stream-K with the partition, the tile lists and the page ids read from a plan that
 *                       q3a_paged_decode_plan built for this call's cache_seqlens and block table; the workspace
 *                       argument is that plan (see q3a_paged_decode_plan) */
#define Q3A_DECODE_PLANNED (-4)
int q3a_abi_version(void);

/* Message for the last failing call on this thread ("" if none). */
const char* q3a_last_error(void);

/*
 * Talker decode attention over the paged KV pool.
 *
 * Replaces flash_attn_with_kvcache(q, k_cache, v_cache, cache_seqlens=ctx, block_table=bt,
 * softmax_scale=scale, causal=True) at engine/talker.py:77 (fp32 semantics: engine/talker.py:82-88).
 *
 *   q            [B, Hq, D] bf16   row stride q_stride_b, head stride q_stride_h, dim stride 1
 *   k_cache      [num_pages, page_size, Hkv, D] bf16, strides kv_stride_page / kv_stride_tok /
 *   v_cache      kv_stride_head, dim stride 1 (both caches share the strides: the engine allocates the
 *                per-layer pools alike, engine/talker.py:30-31)
 *   cache_seqlens[B] int32   context length of each row (tokens 0..ctx-1 are attended)
 *   block_table  [B, max_pages_per_seq] int32, row stride bt_stride_b: token t of row b lives at
 *                page block_table[b][t / page_size], offset t % page_size
 *   out          [B, Hq, D] bf16   row stride o_stride_b, head stride o_stride_h
 *   workspace    fp32 split-K partials, at least q3a_paged_decode_workspace_bytes() bytes
 *                (uninitialised memory is fine)
 *
 * Query head h reads KV head h / (Hq/Hkv).  softmax is float32.  Rows with ctx <= 0 produce zeros;
 * ctx is clamped to max_pages_per_seq*page_size; a page index outside [0, num_pages) contributes
 * no tokens.  Requirements: D == 128, Hq == 2*Hkv, 1 <= Hkv <= 16, page_size % 16 == 0,
 * 16-byte aligned rows.  split_tokens == 0 lets the library choose the decomposition from the batch and
 * the table capacity max_pages_per_seq*page_size (never from the device-resident lengths): tables of at most
 * 128 tokens and batches of at most 64 rows with tables of at most 2,048 tokens take Q3A_DECODE_ROW, except
 * batches of at most 16 rows with tables of 256 tokens or more, which take Q3A_DECODE_CHUNKS; larger batches
 * take stream-K (a persistent grid sized to the device, balanced over all rows' 16-token tiles; batch <= 4096,
 * larger batches fall back to q3a_paged_decode_default_split()).  The path codes above force one of them;
 * split_tokens > 0 (a multiple of 16, <= 1024) selects one workgroup per (row, split of that many tokens).
 */
int q3a_paged_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                     const void* k_cache, const void* v_cache, int64_t kv_stride_page,
                     int64_t kv_stride_tok, int64_t kv_stride_head, int num_pages, int page_size,
                     const int32_t* cache_seqlens, const int32_t* block_table, int64_t bt_stride_b,
                     int max_pages_per_seq, void* out, int64_t o_stride_b, int64_t o_stride_h,
                     void* workspace, size_t workspace_bytes, int batch, int num_q_heads,
                     int num_kv_heads, int head_dim, float softmax_scale, int split_tokens,
                     void* stream);

/*
 * Per-frame decode plan: the stream-K decomposition of a decode call, computed once and read by every call that
 * shares its cache_seqlens and block table.
 *
 * No reference counterpart as a function: flash-attn 2 recomputes its split scheduling inside every
 * flash_attn_with_kvcache call (engine/talker.py:77, 28 calls per frame from Talker._decode, engine/talker.py:63-80,
 * all with the same ctx and bt, engine/talker.py:107-112); flash-attn 3 exposes the same idea as
 * get_scheduler_metadata / scheduler_metadata.  Here the plan holds the tile prefix sums, every stream-K workgroup's
 * tile range, each wave's first tile list and, for every 16-token tile, its row, offset, valid tokens and page id,
 * so a planned call's waves issue their first K/V loads one memory round trip after launch.
 *
 *   cache_seqlens [batch] int32   as the calls will pass it (plain form: context lengths; append forms: tokens
 *                                 already cached)
 *   block_table   num_tables tables [batch, max_pages_per_seq] int32 (row stride bt_stride_b, table stride
 *                 bt_stride_table): plan t is for table t (one table in the engine; one per layer where each layer
 *                 has its own table)
 *   form          Q3A_PLAN_PLAIN (q3a_paged_decode), Q3A_PLAN_APPEND (q3a_paged_decode_append),
 *                 Q3A_PLAN_APPEND_ROPE (q3a_paged_decode_append_rope)
 *   plans         num_tables plans of q3a_paged_decode_plan_bytes() bytes each, plan t at plans + t * plan_stride
 *                 (bytes; 256-aligned), plans_bytes in all
 *
 * A call uses plan t by passing split_tokens = Q3A_DECODE_PLANNED and the plan as its workspace (with the plan's
 * size as workspace_bytes); it must pass the same cache_seqlens pointer, table t, shape and form, which the library
 * checks on the host (Q3A_EINVAL otherwise).  The plan reflects the lengths and table entries at the time the plan
 * kernel ran: rebuild it (on the same stream, before the calls) whenever either changes.  A planned call also writes
 * its partial records into the plan buffer, so calls that share one plan must not overlap (calls on one stream do
 * not).  Plans exist for the shapes the library decodes with stream-K by itself (split_tokens 0: tables over 128
 * tokens with more than 64 rows, or more than 16 rows of tables over 2,048 tokens) with 8 KV heads, batch <= 4096 and
 * page_size <= 4096; q3a_paged_decode_plan_bytes() returns 0 for other shapes.
 */
#define Q3A_PLAN_PLAIN 0
#define Q3A_PLAN_APPEND 1
#define Q3A_PLAN_APPEND_ROPE 2
size_t q3a_paged_decode_plan_bytes(int batch, int num_kv_heads, int max_pages_per_seq, int page_size);
int q3a_paged_decode_plan(const int32_t* cache_seqlens, const int32_t* block_table, int64_t bt_stride_b,
                          int64_t bt_stride_table, int num_tables, int max_pages_per_seq, int page_size, int batch,
                          int num_kv_heads, int form, void* plans, int64_t plan_stride, size_t plans_bytes,
                          void* stream);

/*
 * Talker decode attention with this step's K/V append fused in.
 *
 * Replaces the pair kc[l].view(-1,8,128).index_copy_(0, slot, k); vc[l]...index_copy_(0, slot, v)
 * (engine/talker.py:72-73) and the attention call after it (engine/talker.py:77), i.e. the
 * flash_attn_with_kvcache(q, k_cache, v_cache, k=k, v=v, cache_seqlens=pos, block_table=bt, ...) form.
 *
 *   k_new, v_new [B, Hkv, D] bf16, row strides kn_stride_b / vn_stride_b, head stride D
 *   cache_seqlens[B] int32   tokens ALREADY in the cache (= the new token's position)
 *   everything else as in q3a_paged_decode (k_cache/v_cache are written)
 *
 * Row b writes k_new[b], v_new[b] into page block_table[b][p / page_size], offset p % page_size with
 * p = cache_seqlens[b], then attends over the p + 1 tokens 0..p; the new token is taken from k_new/v_new
 * directly (the slot's previous contents are never read).  Rows with cache_seqlens < 0, or whose new token
 * would fall past max_pages_per_seq*page_size, are skipped: zero output, nothing written.  A page index
 * outside [0, num_pages) is neither written nor attended.  The page that receives a row's new token must not
 * be read by another row of the same call.  Workspace: q3a_paged_decode_workspace_bytes() as for
 * q3a_paged_decode.
 */
int q3a_paged_decode_append(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k_new,
                            int64_t kn_stride_b, const void* v_new, int64_t vn_stride_b, void* k_cache,
                            void* v_cache, int64_t kv_stride_page, int64_t kv_stride_tok, int64_t kv_stride_head,
                            int num_pages, int page_size, const int32_t* cache_seqlens,
                            const int32_t* block_table, int64_t bt_stride_b, int max_pages_per_seq, void* out,
                            int64_t o_stride_b, int64_t o_stride_h, void* workspace, size_t workspace_bytes,
                            int batch, int num_q_heads, int num_kv_heads, int head_dim, float softmax_scale,
                            int split_tokens, void* stream);

/*
 * q3a_paged_decode_append with the talker's q/k producers fused in: q and k_new arrive as the raw projections and
 * are RMS-normalised and rotated inside the call.
 *
 * Replaces, per layer, rope(rms(q, qn)) and rope(rms(k, kn)) (engine/talker.py:69-70, the functions of
 * engine/ops.py:51-60), the index_copy_ pair (:72-73) and the attention (:77).
 *
 *   q [B, Hq, D], k_new/v_new [B, Hkv, D]   raw bf16 projections (v is used as given), strides as in
 *                                           q3a_paged_decode_append (k_new/v_new heads packed)
 *   q_norm_w, k_norm_w [D] bf16             RMSNorm weights
 *   cos, sin [B, D] bf16                    each row's RoPE table row (the new token's position), row stride
 *                                           cs_stride_b, dims contiguous
 *   eps                                     RMSNorm epsilon (1e-6 in the talker)
 *
 * For each head row x: y = bf16(x * rsqrt(mean(x^2) + eps)) * w, then bf16(y * cos + rot(y) * sin) with
 * rot(y) = (-y[D/2:], y[:D/2]), evaluated in fp32 and rounded once.  The normalised k row is what the slot receives
 * and what the new token is attended with.  Everything else is q3a_paged_decode_append.  Needs split_tokens == 0,
 * head_dim 128 and, above 64 rows, at most 8 KV heads; the norm weights and cos/sin rows 16-byte aligned.
 */
int q3a_paged_decode_append_rope(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k_new,
                                 int64_t kn_stride_b, const void* v_new, int64_t vn_stride_b, const void* q_norm_w,
                                 const void* k_norm_w, const void* cos, const void* sin, int64_t cs_stride_b,
                                 float eps, void* k_cache, void* v_cache, int64_t kv_stride_page,
                                 int64_t kv_stride_tok, int64_t kv_stride_head, int num_pages, int page_size,
                                 const int32_t* cache_seqlens, const int32_t* block_table, int64_t bt_stride_b,
                                 int max_pages_per_seq, void* out, int64_t o_stride_b, int64_t o_stride_h,
                                 void* workspace, size_t workspace_bytes, int batch, int num_q_heads,
                                 int num_kv_heads, int head_dim, float softmax_scale, int split_tokens,
                                 void* stream);

/*
 * q3a_paged_decode without a workspace argument: it allocates nothing and takes no caller buffer beyond q, the
 * caches, the length/table arrays and out.  No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under graph capture, tight serving loops, harnesses that forbid allocation).
 *
 * The workspace is a static 8 MiB device array inside the library, one per GPU, held until the process ends.  Shapes
 * whose workspace (q3a_paged_decode_workspace_bytes) exceeds it are rejected with Q3A_ESPACE; every stream-K call
 * (split_tokens == 0, batch <= 4096) fits on MI355X.  All calls on one GPU share that array: calls that overlap on one
 * GPU (two streams at once) race, calls ordered on one stream do not.  Arguments, semantics and results are those of
 * q3a_paged_decode, bit for bit.
 */
int q3a_paged_decode_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k_cache,
                             const void* v_cache, int64_t kv_stride_page, int64_t kv_stride_tok,
                             int64_t kv_stride_head, int num_pages, int page_size, const int32_t* cache_seqlens,
                             const int32_t* block_table, int64_t bt_stride_b, int max_pages_per_seq, void* out,
                             int64_t o_stride_b, int64_t o_stride_h, int batch, int num_q_heads, int num_kv_heads,
                             int head_dim, float softmax_scale, int split_tokens, void* stream);

/* Bytes of workspace q3a_paged_decode needs for this shape and split (0 if none is needed). */
size_t q3a_paged_decode_workspace_bytes(int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                        int max_pages_per_seq, int page_size, int split_tokens);

/* The fixed split size used for batches beyond the stream-K limit. */
int q3a_paged_decode_default_split(int batch, int num_kv_heads, int max_pages_per_seq,
                                   int page_size);

/*
 * Code-predictor attention over the 16-slot K/V scratch.
 *
 * Replaces cp_attn(q, K, V, n_live, scale) (engine/cp_attn.py:33-39), whose in-graph torch form is
 * engine/code_predictor.py:46-47: slots >= n_live are masked (and never read), scores and softmax
 * are float32, the probabilities are rounded to bf16 before P.V, P.V accumulates in float32.
 *
 *   q   [B, Hq, D] bf16 with row stride q_stride_b (head stride D)
 *   k   [B, Hkv, S, D] bf16 with strides k_stride_b / k_stride_h / k_stride_s (dim stride 1)
 *   v   [B, Hkv, S, D] bf16 with strides v_stride_b / v_stride_h / v_stride_s (dim stride 1)
 *   out [B, Hq*D] bf16 with row stride o_stride_b
 * Requirements: D == 128, Hq == 2*Hkv, 1 <= n_live <= 16, 16-byte aligned pointers and strides,
 * D <= k_stride_s, v_stride_s <= 2^26 elements.
 */
int q3a_cp_attn(const void* q, int64_t q_stride_b, const void* k, int64_t k_stride_b, int64_t k_stride_h,
                int64_t k_stride_s, const void* v, int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_s,
                void* out, int64_t o_stride_b, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                int n_live, float softmax_scale, void* stream);

/*
 * Code-predictor slot write + attention in one launch.
 *
 * Replaces the pair K.index_copy_(2, p, k.unsqueeze(2)); V.index_copy_(2, p, v.unsqueeze(2)) followed by
 * the attention of _post (engine/code_predictor.py:58 then :46-47), with p = n_live - 1: slot p of K/V[b, h]
 * is overwritten with k_new/v_new[b, h] and the query attends over slots 0..p, slot p taken from the new rows.
 *
 *   k_new [B, Hkv, D] bf16, row stride kn_stride_b, head stride D
 *   v_new [B, Hkv, D] bf16, row stride vn_stride_b, head stride D (a view into the qkv projection is fine)
 *   q, k, v, out, strides and requirements as in q3a_cp_attn; k and v are written (slot n_live - 1 only).
 */
int q3a_cp_attn_append(const void* q, int64_t q_stride_b, const void* k_new, int64_t kn_stride_b,
                       const void* v_new, int64_t vn_stride_b, void* k, int64_t k_stride_b, int64_t k_stride_h,
                       int64_t k_stride_s, void* v, int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_s,
                       void* out, int64_t o_stride_b, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                       int n_live, float softmax_scale, void* stream);

/*
 * q3a_cp_attn_append with the step's producers (engine/code_predictor.py:38-43): q and k_new arrive raw (views of
 * the qkv projection: q [B, Hq, D] with head stride D, k_new as in q3a_cp_attn_append) and are RMS-normalised with
 * q_norm_w / k_norm_w [D] and rotated with slot (n_live - 1)'s cos/sin rows [D] (engine/ops.py:51-60 as the compiled
 * _pre evaluates them: y = bf16(x * rsqrt(mean(x^2) + eps)) * w, then bf16(y * cos + rot(y) * sin) rounded once).
 * The normalised k_new is what slot n_live - 1 receives; the rest as q3a_cp_attn_append.  The weights and the
 * cos/sin rows must be 16-byte aligned.
 */
int q3a_cp_attn_append_rope(const void* q, int64_t q_stride_b, const void* k_new, int64_t kn_stride_b,
                            const void* v_new, int64_t vn_stride_b, const void* q_norm_w, const void* k_norm_w,
                            const void* cos, const void* sin, float eps, void* k, int64_t k_stride_b,
                            int64_t k_stride_h, int64_t k_stride_s, void* v, int64_t v_stride_b, int64_t v_stride_h,
                            int64_t v_stride_s, void* out, int64_t o_stride_b, int batch, int num_q_heads,
                            int num_kv_heads, int head_dim, int n_live, float softmax_scale, void* stream);

/*
 * Talker prefill attention (packed variable-length, MFMA).
 *
 * Replaces flash_attn_varlen_func(q, k, v, cu_seqlens_q=cu, cu_seqlens_k=cu, ..., causal=True) at
 * engine/talker.py:169 (fp32 form engine/talker.py:163-167); with cu_seqlens_k != cu_seqlens_q it also covers
 * prefix + new sequences packed by length (the dense flash_attn_func of engine/arrivals.py:148 is
 * q3a_prefill_dense below).  K and V carry their own strides: at engine/talker.py:158-160 k is a fresh
 * [T, 8, 128] tensor (token stride 1024) while v is a view into the qkv projection (token stride 4096).
 *
 *   q       [T, Hq, D] bf16, token stride q_stride_t, head stride q_stride_h; sequence s owns tokens
 *           cu_seqlens_q[s] .. cu_seqlens_q[s+1]-1
 *   k, v    block_table == NULL: packed [Tk, Hkv, D] (token strides k/v_stride_tok, head strides
 *           k/v_stride_head; the page strides are ignored), sequence s owns rows cu_seqlens_k[s] ..
 *           cu_seqlens_k[s+1]-1;
 *           block_table != NULL: the paged pools [num_pages, page_size, Hkv, D] (k/v_stride_page/tok/head), key j
 *           of sequence s at page block_table[s][j / page_size], offset j % page_size, with
 *           Lk = cu_seqlens_k[s+1] - cu_seqlens_k[s] keys
 *   out     [T, Hq, D] bf16 (token stride o_stride_t, head stride o_stride_h)
 * With causal != 0, query i of a sequence sees keys j <= Lk - Lq + i (bottom-right aligned; for Lq == Lk the
 * standard causal mask).  Query rows that see no key are zeros.  Requirements: D == 128, Hq == 2*Hkv,
 * 16-byte aligned rows, strides multiples of 8 elements, K/V token strides in [D, 2^26]; max_seqlen_q >= every Lq.
 */
int q3a_prefill(const void* q, int64_t q_stride_t, int64_t q_stride_h, const int32_t* cu_seqlens_q,
                const void* k, int64_t k_stride_page, int64_t k_stride_tok, int64_t k_stride_head,
                const void* v, int64_t v_stride_page, int64_t v_stride_tok, int64_t v_stride_head,
                int num_pages, int page_size, const int32_t* block_table, int64_t bt_stride_b,
                int max_pages_per_seq, const int32_t* cu_seqlens_k, void* out, int64_t o_stride_t,
                int64_t o_stride_h, int num_seqs, int max_seqlen_q, int num_q_heads, int num_kv_heads,
                int head_dim, float softmax_scale, int causal, void* stream);

/*
 * Talker prefill with the prompt's K/V written into the page pool in the same launch.
 *
 * Replaces the two index_copy_ scatters of engine/talker.py:161-162 (k and v of every prompt token into the pool at
 * the seat's positions 0 .. L-1) together with the attention at engine/talker.py:169.  The attention is
 * q3a_prefill's on the packed k/v (same arguments and result, bit for bit); in addition, the K and V rows of each
 * query token i of sequence s (key position p = Lk - Lq + i, Lq/Lk from cu_seqlens_q/k; p = i for a whole prompt)
 * are stored into k_cache/v_cache [num_pages, page_size, Hkv, D] (strides kv_stride_page/tok/head, shared by the
 * two pools) at page block_table[s][p / page_size], offset p % page_size.  Positions past max_pages_per_seq pages
 * and page ids outside [0, num_pages) are not written.  k/v are the packed [Tk, Hkv, D] rows (token and head
 * strides as in q3a_prefill).  page_size a power of two >= 16; the caches 16-byte aligned, strides multiples of 8
 * elements, token stride >= D, page stride >= page_size * token stride.  The pool rows this call writes must not
 * alias the packed k/v it reads.
 */
int q3a_prefill_append(const void* q, int64_t q_stride_t, int64_t q_stride_h, const int32_t* cu_seqlens_q,
                       const void* k, int64_t k_stride_tok, int64_t k_stride_head, const void* v,
                       int64_t v_stride_tok, int64_t v_stride_head, const int32_t* cu_seqlens_k,
                       void* k_cache, void* v_cache, int64_t kv_stride_page, int64_t kv_stride_tok,
                       int64_t kv_stride_head, int num_pages, int page_size, const int32_t* block_table,
                       int64_t bt_stride_b, int max_pages_per_seq, void* out, int64_t o_stride_t,
                       int64_t o_stride_h, int num_seqs, int max_seqlen_q, int num_q_heads, int num_kv_heads,
                       int head_dim, float softmax_scale, int causal, void* stream);

/*
 * Prefix + new prefill attention on dense [S, R, H, D] tensors (MFMA): the layout flash_attn_func takes at
 * engine/arrivals.py:148 (fp32 form engine/arrivals.py:125-131), with no cumulative-length arrays.
 *
 *   q    [S, Lq, Hq, D] bf16 (sequence/token/head strides q_stride_s/t/h), Lq = seqlen_q
 *   k    [S, Lk, Hkv, D] bf16 (k_stride_s/t/h), Lk = seqlen_k
 *   v    [S, Lk, Hkv, D] bf16 (v_stride_s/t/h)
 *   out  [S, Lq, Hq, D] bf16 (o_stride_s/t/h)
 * With causal != 0, query i sees keys j <= Lk - Lq + i (bottom-right aligned).  Query rows that see no key are
 * zeros.  Requirements as in q3a_prefill (D == 128, Hq == 2*Hkv, 16-byte aligned rows, strides multiples of 8
 * elements, K/V token strides in [D, 2^26]); sequence strides non-negative.
 */
int q3a_prefill_dense(const void* q, int64_t q_stride_s, int64_t q_stride_t, int64_t q_stride_h,
                      const void* k, int64_t k_stride_s, int64_t k_stride_t, int64_t k_stride_h,
                      const void* v, int64_t v_stride_s, int64_t v_stride_t, int64_t v_stride_h,
                      void* out, int64_t o_stride_s, int64_t o_stride_t, int64_t o_stride_h, int num_seqs,
                      int seqlen_q, int seqlen_k, int num_q_heads, int num_kv_heads, int head_dim,
                      float softmax_scale, int causal, void* stream);

/*
 * Fast-admission prefill with the sequences' K/V written into the page pool in the same launch.
 *
 * Replaces the two index_copy_ scatters of engine/arrivals.py:144-145 (every row of K = cat(prefix, new) and of V
 * into the seat's cache positions 0 .. n-1) together with the attention at engine/arrivals.py:148.  The attention is
 * q3a_prefill_dense's on the dense k/v (same arguments and result, bit for bit); in addition, rows first_row ..
 * seqlen_k - 1 of sequence s's K and V (key j at k + s * k_stride_s + j * k_stride_t) are stored into
 * k_cache/v_cache [num_pages, page_size, Hkv, D] (strides kv_stride_page/tok/head, shared by the two pools) at page
 * block_table[s][j / page_size], offset j % page_size.  first_row = 0 writes every row (the engine's call);
 * seqlen_k - seqlen_q writes the new tokens' rows only (a prefix already in the pool).  0 <= first_row <=
 * max(0, seqlen_k - seqlen_q).  Positions past max_pages_per_seq pages and page ids outside [0, num_pages) are not
 * written.  With num_seqs == 0 or seqlen_q == 0 nothing is computed or written.  Pool requirements as in
 * q3a_prefill_append; the pool rows this call writes must not alias the k/v it reads.
 */
int q3a_prefill_dense_append(const void* q, int64_t q_stride_s, int64_t q_stride_t, int64_t q_stride_h,
                             const void* k, int64_t k_stride_s, int64_t k_stride_t, int64_t k_stride_h,
                             const void* v, int64_t v_stride_s, int64_t v_stride_t, int64_t v_stride_h,
                             void* k_cache, void* v_cache, int64_t kv_stride_page, int64_t kv_stride_tok,
                             int64_t kv_stride_head, int num_pages, int page_size, const int32_t* block_table,
                             int64_t bt_stride_b, int max_pages_per_seq, int first_row, void* out,
                             int64_t o_stride_s, int64_t o_stride_t, int64_t o_stride_h, int num_seqs, int seqlen_q,
                             int seqlen_k, int num_q_heads, int num_kv_heads, int head_dim, float softmax_scale,
                             int causal, void* stream);

/*
 * The fast-admission layer's attention block on the caller's stream (engine/arrivals.py:112-118 and
 * 144-148): the producers q = rope(rms(q_raw, q_norm_w)), k = rope(rms(k_raw, k_norm_w)) (engine/ops.py:51-60,
 * evaluated with the rounding of eager bf16 ops: every op rounds to bf16), K = cat(prefix_k, k), V = cat(prefix_v, v)
 * (engine/arrivals.py:118), the two index_copy_ scatters of K and V into the pool (:144-145) and the attention
 * flash_attn_func(q, K, V, causal) (:148).  With n = prefix_len + seqlen_q <= 128 and seqlen_q <= 112 (the
 * admission shape) it is one launch: the attention kernel copies the prefix and new K/V rows from where they are,
 * normalises and rotates the new K rows and q itself, and stores rows first_row .. n-1 into the pool; the workspace
 * is not used.  Otherwise two: the first writes q, K and V into the workspace, the second is
 * q3a_prefill_dense_append on them.
 *
 *   q          [S, R, Hq, D] bf16 raw projections (strides q_stride_s/t/h; a view of the qkv output is fine)
 *   k, v       [S, R, Hkv, D] bf16 raw new keys and the new values (their own strides)
 *   prefix_k/v [num_prefixes, P, Hkv, D] bf16, already normalised and rotated (the registered voice's K/V);
 *              sequence s takes prefix prefix_index[s] (int64), or prefix s when prefix_index is NULL.  An index
 *              outside [0, num_prefixes) reads zeros.
 *   q_norm_w, k_norm_w  [D] bf16;  cos, sin  [R, D] bf16 rows of the new tokens' positions (row stride
 *              rope_stride_t; the same for every sequence, as engine/arrivals.py:109 slices them)
 *   pool, table, first_row (0 <= first_row <= P), out: as q3a_prefill_dense_append
 *   workspace  q3a_prefill_dense_append_rope_workspace_bytes(S, R, P, Hq, Hkv, D) bytes, 16-byte aligned
 * Requirements: D == 128, Hq == 2 * Hkv, Hkv a multiple of 4, 16-byte aligned tensors, strides non-negative multiples
 * of 8 elements.  With num_seqs == 0 or seqlen_q == 0 nothing is computed or written.
 */
size_t q3a_prefill_dense_append_rope_workspace_bytes(int num_seqs, int seqlen_q, int prefix_len, int num_q_heads,
                                                     int num_kv_heads, int head_dim);
int q3a_prefill_dense_append_rope(
    const void* q, int64_t q_stride_s, int64_t q_stride_t, int64_t q_stride_h,
    const void* k, int64_t k_stride_s, int64_t k_stride_t, int64_t k_stride_h,
    const void* v, int64_t v_stride_s, int64_t v_stride_t, int64_t v_stride_h,
    const void* prefix_k, int64_t pk_stride_s, int64_t pk_stride_t, int64_t pk_stride_h,
    const void* prefix_v, int64_t pv_stride_s, int64_t pv_stride_t, int64_t pv_stride_h,
    const int64_t* prefix_index, int64_t num_prefixes,
    const void* q_norm_w, const void* k_norm_w, const void* cos, const void* sin, int64_t rope_stride_t, float eps,
    void* k_cache, void* v_cache, int64_t kv_stride_page, int64_t kv_stride_tok, int64_t kv_stride_head,
    int num_pages, int page_size, const int32_t* block_table, int64_t bt_stride_b, int max_pages_per_seq,
    int first_row, void* out, int64_t o_stride_s, int64_t o_stride_t, int64_t o_stride_h, void* workspace,
    size_t workspace_bytes, int num_seqs, int seqlen_q, int prefix_len, int num_q_heads, int num_kv_heads,
    int head_dim, float softmax_scale, int causal, void* stream);

/*
 * The talker's prompt step with its q/k producers, in two launches (engine/talker.py:157-169): q = rope(rms(q_raw,
 * q_norm_w)) and k = rope(rms(k_raw, k_norm_w)) of every prompt token with the token's own cos/sin row (engine/ops.py:
 * 51-60 as eager bf16 ops: prefill_hidden is not compiled), the index_copy_ pair into the pool (:161-162) and
 * flash_attn_varlen_func(q, k, v, cu, cu, ...) (:169).  Causal: the first launch stores the normalised k rows
 * straight into the pool at their positions; the second is the attention with K read back from the pool, v where it
 * is and the raw q normalised and rotated as it is loaded, and it stores the V rows into the pool.  So the attention
 * sees a key only through a valid table entry: a key whose page id is outside [0, num_pages), or whose position is
 * past the table, attends with zeros for K (the engine's index_copy_ would fail on such a slot).  Not causal: the first launch writes the
 * normalised q and k into the workspace and the second is q3a_prefill_append's attention on them (cu_seqlens for
 * both q and k).
 *
 *   q          [T, Hq, D] bf16 raw projections of the T = total_tokens packed prompt tokens (q_stride_t/h)
 *   k, v       [T, Hkv, D] bf16 raw keys and the values (their own strides)
 *   cos, sin   [T, D] bf16: token t's rows at its position in its sequence (row stride rope_stride_t)
 *   cu_seqlens [num_seqs + 1] int32;  pool, table, out: as q3a_prefill_append
 *   workspace  not causal: q3a_prefill_append_rope_workspace_bytes(T, Hq, Hkv, D) bytes, 16-byte aligned;
 *              causal: unused (may be NULL with workspace_bytes 0)
 * Requirements as q3a_prefill_dense_append_rope.
 */
size_t q3a_prefill_append_rope_workspace_bytes(int total_tokens, int num_q_heads, int num_kv_heads, int head_dim);
int q3a_prefill_append_rope(
    const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k, int64_t k_stride_t, int64_t k_stride_h,
    const void* v, int64_t v_stride_t, int64_t v_stride_h, const void* q_norm_w, const void* k_norm_w,
    const void* cos, const void* sin, int64_t rope_stride_t, float eps, const int32_t* cu_seqlens, void* k_cache,
    void* v_cache, int64_t kv_stride_page, int64_t kv_stride_tok, int64_t kv_stride_head, int num_pages,
    int page_size, const int32_t* block_table, int64_t bt_stride_b, int max_pages_per_seq, void* out,
    int64_t o_stride_t, int64_t o_stride_h, void* workspace, size_t workspace_bytes, int num_seqs, int total_tokens,
    int max_seqlen, int num_q_heads, int num_kv_heads, int head_dim, float softmax_scale, int causal, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* Q3ATTN_H */
