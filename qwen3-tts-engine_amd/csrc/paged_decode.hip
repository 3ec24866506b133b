// Talker paged decode attention for gfx950.
//
// Semantics (engine/talker.py:77, fp32 form engine/talker.py:82-88): for every row b and query
// head h, o[b,h] = softmax(q[b,h] . K[b, h/2, :ctx]^T * scale) . V[b, h/2, :ctx], where token t of
// row b sits in page block_table[b][t / page_size] at offset t % page_size.
//
// Tile engine.  A wave streams 16-token tiles of one KV head: one 16 B buffer load per lane fetches
// 4 tokens x 256 B (lane l: token l/16, dims 8*(l%16)..+8), so a tile is 4 loads of K and 4 of V;
// the loads carry the non-temporal hint and are bounds-checked by the buffer descriptor (tokens
// past the context and invalid pages return zeros without touching memory).  Two register tiles
// alternate so one is in flight while the other is consumed.  Both query heads of the GQA pair
// are applied to every loaded K/V register (bf16 dot2 for q.k, fp32 FMA for p.v).  Each 16-lane
// group keeps its own online-softmax state; the four groups are merged at the end of a segment.
// The tiles a wave will stream are described lane-wise (lane i = tile i: page, offset, valid
// tokens), so the per-tile page lookup is a v_readlane, not a memory access.
//
// Work decomposition (default): stream-K.  The grid is exactly the number of workgroups the GPU
// holds at once; the flattened sequence of (row, tile) pairs is cut into equal contiguous ranges,
// one per workgroup, and every wave of a workgroup streams its KV head over that range.  Rows that
// straddle a range boundary leave partial records (fp32 m, l and the normalised o in 16 bits) in at
// most two slots per workgroup; the combine kernel merges them and writes zeros for ctx == 0 rows.
// Alternative (split_tokens > 0): one workgroup per (row, fixed-size split), partials merged by
// the same kind of combine.  Narrow tables (at most 128 tokens) and small batches (at most 64 rows of up
// to 2,048 tokens) take the row-parallel kernel instead: one workgroup per (row, KV head), the row's tiles
// spread over its waves and merged in LDS, one launch.
//
// Append form (flash_attn_with_kvcache with k=, v=; replaces the index_copy_ pair of
// engine/talker.py:72-73 before the call at :77): cache_seqlens counts the tokens already cached,
// the row attends over cache_seqlens + 1 tokens, and the last one is this step's k/v row.  The wave
// that consumes a row's last tile swaps that token's registers for the k_new/v_new row, writes the
// row into the page slot, and attends with the registers; the slot's old contents are never used.
// In the stream-K kernel a segment's q rows and a row's new k/v rows reach the wave through LDS, copied
// there together with the tile that needs them (see stage_q), so segment starts and row ends never
// drain the tile in flight.
#include <algorithm>
#include <atomic>
#include <mutex>
#include <unordered_map>

#include "q3a_common.h"
#include "../../include/q3attn.h"

namespace q3a {
namespace {

constexpr int kD = 128;
constexpr int kG = 2;                              // query heads per KV head
// Partial record of one (segment, KV head): o = acc / l of both query heads as 16-bit values (fp16; bf16 when
// some |o| would overflow fp16, flagged by negative l), then m[G], l[G] in fp32: 528 bytes, addressed in floats.
constexpr int kPartFloats = kG * kD / 2 + 2 * kG;
constexpr int kPartML = kG * kD / 2;               // float index of m[0]; l[h] at kPartML + kG + h
constexpr int kMaxSplits = 64;
constexpr int kTile = 16;                          // tokens per pipeline stage
constexpr int kMaxSplitTokens = 64 * kTile;        // one VGPR lane per tile of a split
constexpr int kSkMaxRows = 4096;                   // rows the stream-K prologue scans in LDS
constexpr int kSkSlots = 2;                        // partial records per stream-K workgroup
constexpr int kSkMaxGrid = 4096;
constexpr int kOneSplitTokens = 128;               // table capacity up to which rows are never split

struct DecodeArgs {
  const uint16_t* q;
  int64_t q_sb, q_sh;
  const uint16_t* kc;
  const uint16_t* vc;
  int64_t kv_sp, kv_st, kv_sh;
  const uint16_t* k_new;  // append form: [batch, hkv, kD] rows (head stride kD), else unused
  const uint16_t* v_new;
  int64_t kn_sb, vn_sb;
  int num_pages, page_size;
  uint32_t page_bytes;  // byte extent of one page's tokens (bounds of the buffer loads)
  int max_pages;        // table entries per row
  const int32_t* seqlens;
  const int32_t* bt;
  int64_t bt_sb;
  uint16_t* out;
  int64_t o_sb, o_sh;
  float* ws;            // partial records
  int* prefix;          // stream-K: [batch + 1] tile prefix sums
  int* slot_page;       // stream-K append forms: [batch] page id of each row's new-token slot (from the decode kernel)
  // Planned stream-K calls (kPlan): the per-frame plan's workgroup ranges, each wave's first tile list and every
  // tile's entry (see paged_decode_plan_kernel).
  const int* plan_wg;
  const int2* plan_first;
  const int2* plan_tiles;
  const int4* plan_cut;  // the planned combine: cut-row descriptors (row, pieces, overflow base, 0)
  int plan_rec_cap;
  int* plan_claim;       // planned calls: one flag per range, set by the workgroup that takes it (zero between calls)
  int batch, hkv, split_tokens, max_splits, grid;
  int row_per;          // row-parallel path: tiles per wave of the table capacity (the host picks the kernel)
  float scale_log2;
  // Norm/rope form (kRope instantiations): q and the new k rows arrive raw and are normalised and rotated in the
  // kernel (qk_norm_rope16/64): RMSNorm weights [kD] bf16, each row's RoPE cos/sin [kD] bf16 at row stride rs_sb.
  const uint16_t* qn_w;
  const uint16_t* kn_w;
  const uint16_t* rcos;
  const uint16_t* rsin;
  int64_t rs_sb;
  float eps;
};

struct KVTile {
  uint4 k[4];
  uint4 v[4];
};

// Up to 64 tiles of one wave, described lane-wise: consecutive tiles in the stream-K and fixed-split kernels,
// every W-th tile of a row in the row-parallel kernel.
struct TileList {
  int page;    // lane i: page index of tile i
  int off;     // lane i: token offset of tile i inside its page
  int nvalid;  // lane i: valid tokens of tile i (1..16), 0 past the list
  int n;       // number of tiles (uniform)
};

__device__ __forceinline__ int clamp_ctx(const DecodeArgs& a, int c) {
  const int cap = a.max_pages * a.page_size;
  return c < 0 ? 0 : (c > cap ? cap : c);
}

// Tokens row b attends over.  Append form: the cached tokens plus the new one; a row whose new
// token would not fit the table (or with cache_seqlens < 0) is skipped: zero output, nothing written.
template <bool kAppend>
__device__ __forceinline__ int ctx_of(int c, int cap) {
  if constexpr (kAppend) return (c < 0 || c >= cap) ? 0 : c + 1;
  else return c < 0 ? 0 : (c > cap ? cap : c);
}
template <bool kAppend>
__device__ __forceinline__ int row_ctx(const DecodeArgs& a, int b) {
  return ctx_of<kAppend>(a.seqlens[b], a.max_pages * a.page_size);
}

__device__ __forceinline__ int readlane(int v, int lane) { return __builtin_amdgcn_readlane(v, lane); }

// Issues the 8 loads of tile j.  A tile past the list or with an invalid page issues loads against a
// zero-length descriptor (they return zeros and read nothing), so every path issues the same number
// of loads and the compiler's vmcnt bookkeeping stays exact across the ping-pong buffers.
__device__ __forceinline__ void issue_tile(const DecodeArgs& a, const TileList& L, uint32_t lane_off,
                                           int grp, int j, KVTile& T) {
  const int jj = j < L.n ? j : 0;
  const int page = readlane(L.page, jj);
  const int off = readlane(L.off, jj);
  const int nv = j < L.n ? readlane(L.nvalid, jj) : 0;
  const bool ok = nv > 0 && (unsigned)page < (unsigned)a.num_pages;
  const int64_t pbase = ok ? (int64_t)page * a.kv_sp : 0;
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(a.kc + pbase, ok ? a.page_bytes : 0u);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(a.vc + pbase, ok ? a.page_bytes : 0u);
  const uint32_t tok_bytes = (uint32_t)(a.kv_st * 2);
  const uint32_t base = lane_off + (uint32_t)off * tok_bytes;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t o = (4 * i + grp < nv) ? base + (uint32_t)(4 * i) * tok_bytes : kOutOfRange;
    T.k[i] = buffer_load16_stream(rk, o);
    T.v[i] = buffer_load16_stream(rv, o);
  }
}

// Append form, the last tile of a row, once its loads have landed: token nvalid-1 is the new one.  The
// 16 lanes holding it take this step's k/v row instead of the stale slot (its old contents are never
// used) and store that row into the slot; an invalid page is neither written nor attended (tile_update
// masks it).  The two row loads are issued here, at consume time, so they never sit in a register across
// the tile pipeline; the wave waits once per row for them (the fixed-split kernel, one row end per
// workgroup; the stream-K kernel stages the rows instead, take_staged_token).
__device__ __forceinline__ void take_new_token(const DecodeArgs& a, const TileList& L, uint32_t lane_off,
                                               int grp, int g, int j, int row, KVTile& T) {
  const int page = readlane(L.page, j);
  const int off = readlane(L.off, j);
  const int tn = readlane(L.nvalid, j) - 1;
  const int i_new = tn >> 2;
  const bool mine = grp == (tn & 3);
  const bool ok = (unsigned)page < (unsigned)a.num_pages;
  // Uniform bases in SGPRs: the new rows of (row, g), and the slot's page (lane_off already holds the
  // lane's token-in-quad, head and dim offset, so the slot adds only (off + 4*i_new) tokens).
  const uint32_t dim_off = (uint32_t)(threadIdx.x & 15) * 16;
  const __amdgpu_buffer_rsrc_t rkn = make_rsrc(a.k_new + (int64_t)row * a.kn_sb + g * kD, kD * 2);
  const __amdgpu_buffer_rsrc_t rvn = make_rsrc(a.v_new + (int64_t)row * a.vn_sb + g * kD, kD * 2);
  const int64_t pbase = ok ? (int64_t)page * a.kv_sp : 0;
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(a.kc + pbase, ok ? a.page_bytes : 0u);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(a.vc + pbase, ok ? a.page_bytes : 0u);
  const uint32_t slot_off = (uint32_t)((off + 4 * i_new) * a.kv_st * 2);
  // K, then V: one 4-register row live at a time (the other tile of the pipeline is in flight).
  const uint4 kn = buffer_load16_s(rkn, dim_off, 0);
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (i == i_new && mine) T.k[i] = kn;
  if (mine) buffer_store16_s(kn, rk, lane_off, slot_off);
  __builtin_amdgcn_sched_barrier(0);
  const uint4 vn = buffer_load16_s(rvn, dim_off, 0);
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (i == i_new && mine) T.v[i] = vn;
  if (mine) buffer_store16_s(vn, rv, lane_off, slot_off);
  // Drain here (vmcnt(0); expcnt, lgkmcnt untouched) so this once-per-row path rejoins the tile loop
  // with nothing outstanding: the loop's own waits then stay at "this tile only" on every tile.
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __builtin_amdgcn_sched_barrier(0);
}

// ------------------------------------------------------------------------------ segment staging (stream-K)
// Per wave and tile parity, 1 KiB of LDS receives, by direct-to-LDS copies issued together with a tile's K/V
// loads, the q rows of the segment the tile opens (both heads, 512 B; the 16 B-per-lane copy also writes
// zeros over the next 512 B) and, in the append form when the tile ends its row, this step's new k row (at
// kStageNew) and v row (256 B later).  The consumer reads them after the next tile has been issued, from the
// other parity's array, so neither a segment start nor a row end waits for the tile in flight.  Every tile
// issues the q copy (out of bounds when it opens no segment), so each tile puts the same number of operations
// on vmcnt and the compiler's count-based waits stay exact.
constexpr int kStageBytes = 1024;
constexpr int kStageNew = 512;
constexpr int kMaxWaves = 16;
constexpr int kWaitGroup = 0x0F70 | 9;  // s_waitcnt vmcnt(9) (expcnt, lgkmcnt untouched)

__device__ __forceinline__ void stage_q(const DecodeArgs& a, int b, int g, int lane, bool valid, uint8_t* st) {
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.q + (int64_t)b * a.q_sb + (int64_t)(kG * g) * a.q_sh,
                                              valid ? (uint32_t)(((kG - 1) * a.q_sh + kD) * 2) : 0u);
  const uint32_t off = lane < kG * 16 ? (uint32_t)((lane >> 4) * a.q_sh * 2 + (lane & 15) * 16) : kOutOfRange;
  lds_copy16(rq, st, off);
}

__device__ __forceinline__ void stage_new_rows(const DecodeArgs& a, int b, int g, int lane, uint8_t* st) {
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(a.k_new + (int64_t)b * a.kn_sb + g * kD, kD * 2);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(a.v_new + (int64_t)b * a.vn_sb + g * kD, kD * 2);
  lds_copy4(rk, st + kStageNew, (uint32_t)lane * 4);
  lds_copy4(rv, st + kStageNew + kD * 2, (uint32_t)lane * 4);
}

// Norm/rope form: the row's RoPE cos and sin rows (256 B each) follow at kStageRope, copied with the tiles that
// open a segment or end their row.
constexpr int kStageRope = 1024;
constexpr int kStageBytesRope = 1536;

__device__ __forceinline__ void stage_rope(const DecodeArgs& a, int b, int lane, uint8_t* st) {
  lds_copy4(make_rsrc(a.rcos + (int64_t)b * a.rs_sb, kD * 2), st + kStageRope, (uint32_t)lane * 4);
  lds_copy4(make_rsrc(a.rsin + (int64_t)b * a.rs_sb, kD * 2), st + kStageRope + kD * 2, (uint32_t)lane * 4);
}

// Append form, the last tile of a row, read after the next tile was issued: as take_new_token, with the new
// k/v rows taken from the wave's stage.  The slot itself is written by the combine kernel.
__device__ __forceinline__ void take_staged_token(const DecodeArgs& a, const TileList& L, int grp, int j,
                                                  const uint8_t* st, KVTile& T) {
  const int tn = readlane(L.nvalid, j) - 1;
  const int i_new = tn >> 2;
  const bool mine = grp == (tn & 3);
  const int chunk = (int)(threadIdx.x & 15) * 16;
  const uint4 kn = ld16(st + kStageNew + chunk);
  const uint4 vn = ld16(st + kStageNew + kD * 2 + chunk);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (i == i_new && mine) {
      T.k[i] = kn;
      T.v[i] = vn;
    }
  }
  (void)a;
}

__device__ __forceinline__ uint32_t u4get(const uint4& v, int c) {
  return c == 0 ? v.x : (c == 1 ? v.y : (c == 2 ? v.z : v.w));
}

// Online-softmax update of one 16-lane group with its 4 tokens of tile j.
//
// q.k: 4 bf16 dot2 per (token, head) then a 16-lane DPP sum.  p.v: the probabilities are packed to
// bf16 pairs (tokens 0,1 and 2,3) and each output dim takes two dot2 against the matching V pairs
// built with v_perm_b32, the rounding point flash-attention also uses for P.  The running max
// rarely grows after the first tiles, so the rescale of (l, acc) runs only when a lane's max grew.
__device__ __forceinline__ void tile_update(const DecodeArgs& a, const TileList& L, const uint4 (&q)[kG],
                                            const KVTile& T, int j, int grp, float (&m)[kG],
                                            float (&l)[kG], float (&acc)[kG][8]) {
  const int page = readlane(L.page, j);
  const int nv = readlane(L.nvalid, j);
  const bool ok = (unsigned)page < (unsigned)a.num_pages;
  float sc[kG][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int h = 0; h < kG; ++h) {
      float s = dot2_bf16(q[h].x, T.k[i].x, 0.f);
      s = dot2_bf16(q[h].y, T.k[i].y, s);
      s = dot2_bf16(q[h].z, T.k[i].z, s);
      s = dot2_bf16(q[h].w, T.k[i].w, s);
      sc[h][i] = row16_sum(s);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bool valid = ok && (4 * i + grp < nv);
#pragma unroll
    for (int h = 0; h < kG; ++h) sc[h][i] = valid ? sc[h][i] * a.scale_log2 : -INFINITY;
  }
  float mt[kG];
  bool grow = false;
#pragma unroll
  for (int h = 0; h < kG; ++h) {
    mt[h] = fmaxf(fmaxf(sc[h][0], sc[h][1]), fmaxf(sc[h][2], sc[h][3]));
    grow |= mt[h] > m[h];
  }
  if (__any(grow)) {
#pragma unroll
    for (int h = 0; h < kG; ++h) {
      const float mn = fmaxf(m[h], mt[h]);
      const float alpha = fast_exp2(m[h] - mn);
      m[h] = mn;
      l[h] *= alpha;
#pragma unroll
      for (int d = 0; d < 8; ++d) acc[h][d] *= alpha;
    }
  }
  // V pairs: vp[pair][c][0] = (v[2*pair][dim 2c], v[2*pair+1][dim 2c]), [1] for dim 2c+1.
  uint32_t vp[2][4][2];
#pragma unroll
  for (int pr = 0; pr < 2; ++pr) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t v0 = u4get(T.v[2 * pr], c);
      const uint32_t v1 = u4get(T.v[2 * pr + 1], c);
      vp[pr][c][0] = perm_b32(v1, v0, kPermLoLo);
      vp[pr][c][1] = perm_b32(v1, v0, kPermHiHi);
    }
  }
#pragma unroll
  for (int h = 0; h < kG; ++h) {
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = fast_exp2(sc[h][i] - m[h]);
    l[h] += (p[0] + p[1]) + (p[2] + p[3]);
    const uint32_t p01 = pack_bf16x2(p[0], p[1]);
    const uint32_t p23 = pack_bf16x2(p[2], p[3]);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        float x = dot2_bf16(p01, vp[0][c][e], acc[h][2 * c + e]);
        acc[h][2 * c + e] = dot2_bf16(p23, vp[1][c][e], x);
      }
    }
  }
}

__device__ __forceinline__ void reset_state(float (&m)[kG], float (&l)[kG], float (&acc)[kG][8]) {
#pragma unroll
  for (int h = 0; h < kG; ++h) {
    m[h] = kMaxSeed;
    l[h] = 0.f;
#pragma unroll
    for (int d = 0; d < 8; ++d) acc[h][d] = 0.f;
  }
}

// Merge the online-softmax states held by lanes l and l^mask (mask 16 or 32, a compile-time constant at every
// call).  The gfx950 lane swaps (VALU, no LDS crossbar) hand each lane both states, the lower lane's first, so
// both lanes compute the same merge, and lanes 0..15 the same arithmetic as "own state first".
__device__ __forceinline__ void merge_lanes(int mask, float (&m)[kG], float (&l)[kG],
                                            float (&acc)[kG][8]) {
  auto both = [mask](float x) { return mask == 16 ? swap16(x) : swap32(x); };
#pragma unroll
  for (int h = 0; h < kG; ++h) {
    const float2 mm = both(m[h]);
    const float2 ll = both(l[h]);
    const float mn = fmaxf(mm.x, mm.y);
    const float w0 = fast_exp2(mm.x - mn);
    const float w1 = fast_exp2(mm.y - mn);
    l[h] = ll.x * w0 + ll.y * w1;
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const float2 aa = both(acc[h][d]);
      acc[h][d] = aa.x * w0 + aa.y * w1;
    }
    m[h] = mn;
  }
}

__device__ __forceinline__ void store_row8(uint16_t* dst, const float (&x)[8], float scale) {
  uint4 v;
  v.x = pack_bf16x2(x[0] * scale, x[1] * scale);
  v.y = pack_bf16x2(x[2] * scale, x[3] * scale);
  v.z = pack_bf16x2(x[4] * scale, x[5] * scale);
  v.w = pack_bf16x2(x[6] * scale, x[7] * scale);
  *reinterpret_cast<uint4*>(dst) = v;
}

// The (row, head pair) base is uniform, so it lives in the descriptor (SGPRs); the lane adds only its
// 16 B of dims, keeping 64-bit per-lane address pairs out of the kernels' register budget.
__device__ __forceinline__ void load_q(const DecodeArgs& a, int b, int g, int dl, uint4 (&q)[kG]) {
  const __amdgpu_buffer_rsrc_t rq =
      make_rsrc(a.q + (int64_t)b * a.q_sb + (int64_t)(kG * g) * a.q_sh, (uint32_t)(((kG - 1) * a.q_sh + kD) * 2));
#pragma unroll
  for (int h = 0; h < kG; ++h) q[h] = buffer_load16_s(rq, (uint32_t)dl * 2, (uint32_t)(h * a.q_sh * 2));
}

// Lanes 0..15 hold the merged state: the normalised output row of both query heads.
__device__ __forceinline__ void write_output(const DecodeArgs& a, int b, int g, int grp, int dl,
                                             const float (&l)[kG], const float (&acc)[kG][8]) {
  if (grp == 0) {
#pragma unroll
    for (int h = 0; h < kG; ++h)
      store_row8(a.out + b * a.o_sb + (kG * g + h) * a.o_sh + dl, acc[h], l[h] > 0.f ? 1.f / l[h] : 0.f);
  }
}

__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  const _Float16 a = (_Float16)lo, b = (_Float16)hi;
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}
__device__ __forceinline__ float f16_lo(uint32_t w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xFFFFu)); }
__device__ __forceinline__ float f16_hi(uint32_t w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16)); }

// Writes the segment's record (layout at kPartFloats).  The partial records are the decode kernel's largest
// writes and, interleaved with the K/V read stream, cost ~1-2 us per MB (576 rows, 296k context tokens), so o is
// stored normalised in 16 bits: fp16 keeps 11 significant bits (relative error 2^-12 against the bf16 output's
// 2^-9) while the record's largest |o| lies in [2^-6, 2^15]; outside that range (fp16 overflow, or values
// small enough for fp16's fixed absolute resolution to matter) the record is stored in bf16, flagged by
// negative l.
// Every lane holds the merged (m, l, acc) after merge_lanes; lanes 0..15 write o, lane 0 writes (m, l).
__device__ __forceinline__ void write_partial(float* P, int lane, int grp, int dl, const float (&m)[kG],
                                              const float (&l)[kG], const float (&acc)[kG][8]) {
  float inv[kG], big = 0.f;
#pragma unroll
  for (int h = 0; h < kG; ++h) {
    inv[h] = l[h] > 0.f ? 1.f / l[h] : 0.f;
#pragma unroll
    for (int d = 0; d < 8; ++d) big = fmaxf(big, fabsf(acc[h][d] * inv[h]));
  }
  const bool wide = __any(big > 32768.f || big < 0.015625f);
  if (grp == 0) {
#pragma unroll
    for (int h = 0; h < kG; ++h) {
      const float* x = acc[h];
      const float s = inv[h];
      uint4 w;
      if (wide) {
        w.x = pack_bf16x2(x[0] * s, x[1] * s);
        w.y = pack_bf16x2(x[2] * s, x[3] * s);
        w.z = pack_bf16x2(x[4] * s, x[5] * s);
        w.w = pack_bf16x2(x[6] * s, x[7] * s);
      } else {
        w.x = pack_f16x2(x[0] * s, x[1] * s);
        w.y = pack_f16x2(x[2] * s, x[3] * s);
        w.z = pack_f16x2(x[4] * s, x[5] * s);
        w.w = pack_f16x2(x[6] * s, x[7] * s);
      }
      st16(reinterpret_cast<char*>(P) + h * kD * 2 + dl * 2, w);
    }
  }
  if (lane == 0)
    st16(P + kPartML, __builtin_bit_cast(uint4, make_float4(m[0], m[1], wide ? -l[0] : l[0], wide ? -l[1] : l[1])));
}

// Folds a group of up to 8 records (unused entries: m = kMaxSeed, l = 0) into the running (M, L, A): one rescale to
// the group's max, then each record's weight |l| 2^(m - M) (a negative l flags bf16 o values, else fp16).
__device__ __forceinline__ void merge_fold8(const uint2 (&raw)[8], const float (&mr)[8], const float (&lr)[8],
                                            float& M, float& L, float4& A) {
  float mc = M;
#pragma unroll
  for (int u = 0; u < 8; ++u) mc = fmaxf(mc, mr[u]);
  const float alpha = fast_exp2(M - mc);
  L *= alpha;
  A.x *= alpha;
  A.y *= alpha;
  A.z *= alpha;
  A.w *= alpha;
  M = mc;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const bool wide = __builtin_signbit(lr[u]);
    const float w = fabsf(lr[u]) * fast_exp2(mr[u] - M);
    const float4 v = wide ? make_float4(bf16_lo(raw[u].x), bf16_hi(raw[u].x), bf16_lo(raw[u].y), bf16_hi(raw[u].y))
                          : make_float4(f16_lo(raw[u].x), f16_hi(raw[u].x), f16_lo(raw[u].y), f16_hi(raw[u].y));
    L += w;
    A.x = fmaf(v.x, w, A.x);
    A.y = fmaf(v.y, w, A.y);
    A.z = fmaf(v.z, w, A.z);
    A.w = fmaf(v.w, w, A.w);
  }
}

// Merges `count` partial records (rec(i) -> record i) of one (row, KV head) into the output row.
// The whole wave participates; lane l owns query head l/32 and dims 4*(l%32)..+4.  Each lane reads every
// record's (m, l) of its head itself (the 32 lanes of a head read the same words), so the merge needs no
// cross-lane step, and the o, m and l loads of up to 8 records are all in flight at once; records are folded
// in with an online rescale (running max M, running weight L).
template <typename RecFn>
__device__ __forceinline__ void merge_records(const DecodeArgs& a, int b, int g, int lane, int count,
                                              RecFn rec) {
  const int h = lane >> 5;
  const int d0 = (lane & 31) * 4;
  float M = kMaxSeed, L = 0.f;
  float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int s0 = 0; s0 < count; s0 += 8) {
    uint2 raw[8];
    float mr[8], lr[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      raw[u] = make_uint2(0u, 0u);
      mr[u] = kMaxSeed;
      lr[u] = 0.f;
      if (s0 + u < count) {
        const float* P = rec(s0 + u);
        raw[u] = *reinterpret_cast<const uint2*>(reinterpret_cast<const char*>(P) + (h * kD + d0) * 2);
        mr[u] = P[kPartML + h];
        lr[u] = P[kPartML + kG + h];
      }
    }
    merge_fold8(raw, mr, lr, M, L, A);
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  // Non-temporal: with the slot stores below, 200.5 -> 198.9 us per append call at 576 rows (the plain form
  // unchanged within noise).
  u32x2 o;
  o.x = pack_bf16x2(A.x * inv, A.y * inv);
  o.y = pack_bf16x2(A.z * inv, A.w * inv);
  __builtin_nontemporal_store(o, reinterpret_cast<u32x2*>(a.out + b * a.o_sb + (kG * g + h) * a.o_sh + d0));
}

__device__ __forceinline__ void write_zero_row(const DecodeArgs& a, int b, int g, int lane) {
  const int h = lane >> 5;
  const int d0 = (lane & 31) * 4;
  *reinterpret_cast<uint2*>(a.out + b * a.o_sb + (kG * g + h) * a.o_sh + d0) = make_uint2(0u, 0u);
}

// ------------------------------------------------------------------------------ stream-K path
// p / c with 32-bit arithmetic whenever p fits (the tile-range bounds of every call below 2^32 tile-workgroup
// products): the 64-bit division is a chain of ~150 scalar instructions on the prologue's critical path.
__device__ __forceinline__ int64_t udiv_fit(uint64_t p, uint32_t c) {
  return (p >> 32) == 0 ? (int64_t)((uint32_t)p / c) : (int64_t)(p / c);
}
__device__ __forceinline__ int64_t sk_lo(int64_t k, int64_t nt, int64_t grid) {
  return udiv_fit((uint64_t)k * (uint64_t)nt, (uint32_t)grid);
}

// Inclusive prefix sum over the 64 lanes of a wave: four DPP row shifts within each 16 lanes, then the two row
// broadcasts across rows (lanes outside the shifted range or the masked rows add zero).  Seven VALU steps where a
// shuffle-based scan waits for six LDS-crossbar round trips.
__device__ __forceinline__ int wave_scan_incl(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);  // row_bcast:15, into rows 1 and 3
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);  // row_bcast:31, into rows 2 and 3
  return x;
}

// The largest row r in [0, n) with pre[r] <= t, for a wave-uniform t with pre[0] <= t over the non-decreasing pre
// (the rows' first tiles; an empty row shares its successor's), found by the whole wave: each lane tests one row of
// an evenly spaced sample and a ballot counts the sampled rows at or before t, which narrows the range 64-fold per
// LDS round trip (4,096 rows: two round trips, where a binary search waits for twelve).  All lanes must be active.
__device__ __forceinline__ int row_at_or_before(const int* pre, int n, int t, int lane) {
  int lo = 0, hi = n;
  while (hi - lo > 1) {
    const int stride = (hi - lo + 63) >> 6;
    const int r = lo + lane * stride;
    const int k = __builtin_popcountll(__ballot(r < hi && pre[r] <= t));  // lanes 0 .. k-1: rows at or before t
    const int nlo = lo + (k - 1) * stride;
    hi = min(hi, nlo + stride);
    lo = nlo;
  }
  return __builtin_amdgcn_readfirstlane(lo);
}

// Workgroups that take part in a call of NT tiles: at most the resident grid and at most NT (each owns at least one
// tile, so the workgroups covering a row are a contiguous index range, which the combine relies on), and at most
// NT / 4 unless that leaves fewer than min(NT, 8): with one tile each, small batches split every row into
// one-tile partial records that the combine then merges eight at a time (1 row of 1,024 tokens: 20.2 -> 16.0 us).
__device__ __forceinline__ int sk_effective_grid(int grid, int nt) {
  const int g = max(min(nt, 8), (nt + 3) / 4);
  return min(grid, g);
}

constexpr int kFirst = 1;     // tile opens a segment (first tile of the row or of the range)
constexpr int kLast = 2;      // tile closes a segment
constexpr int kRowStart = 4;  // tile is tile 0 of its row
constexpr int kRowEnd = 8;    // tile is the last tile of its row

// Block-wide: each row's clamped context into s_ctx, the exclusive prefix sum of its 16-token tile counts into
// s_prefix[0..B] (s_prefix[B] = NT, the call's tile count), with a DPP scan per wave and one over the waves'
// totals.  Every thread of the block must call it; it ends with a barrier and returns NT.
template <bool kAppend>
__device__ __forceinline__ int sk_tile_scan(const DecodeArgs& a, int* s_ctx, int* s_prefix, int* s_wsum) {
  const int tid = threadIdx.x;
  const int nthr = blockDim.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int B = a.batch;
  const int per = (B + nthr - 1) / nthr;
  const int r0 = min(B, tid * per), r1 = min(B, r0 + per);
  int sum = 0;
  for (int r = r0; r < r1; ++r) {
    const int c = row_ctx<kAppend>(a, r);
    s_ctx[r] = c;
    sum += (c + kTile - 1) / kTile;
  }
  const int x = wave_scan_incl(sum);
  if (lane == 63) s_wsum[wv] = x;
  __syncthreads();
  // This wave's base: the sum of the earlier waves' totals (one LDS read per lane and a second wave scan).
  const int nw = nthr >> 6;
  const int wt = wave_scan_incl(lane < nw ? s_wsum[lane] : 0);
  const int wbase = wv == 0 ? 0 : __builtin_amdgcn_readlane(wt, wv - 1);
  int run = wbase + x - sum;
  for (int r = r0; r < r1; ++r) {
    s_prefix[r] = run;
    run += (s_ctx[r] + kTile - 1) / kTile;
  }
  if (tid == nthr - 1) s_prefix[B] = wbase + x;
  __syncthreads();
  return s_prefix[B];
}

// ------------------------------------------------------------------------------ per-frame plan (stream-K)
// The 28 decode calls of a talker frame share cache_seqlens (and, in the engine, the block table), so the stream-K
// partition, each wave's tile list and the tiles' page ids can be computed once per frame and read by every call:
// a planned call's waves load their first tile list (page ids included) in one round trip, where the unplanned
// prologue waits for cache_seqlens, a block-wide scan, row searches in LDS and then the table.  The plan also says
// where each partial record goes: the records of the c-th cut row (a row whose tiles span several workgroups) start
// at positions 2c and 2c + 1 (its first two pieces; every cut row has at least two), further pieces at an overflow
// position, so the planned combine loads a cut row's first two records beside its descriptor, one round trip.
//
// A tile's entry (int2): x = its page id (as the table holds it), y = row | (offset in page / 16) << 13 |
// valid tokens << 21 | segment flags << 26, with the flags of the wave range that holds the tile.
constexpr int kPlanWgInts = 8;  // per decode workgroup: lo, hi, mid, mid_row, mid_whole, mid_from_lo, rec0, rec1
constexpr int kPlanRowBits = 13;
constexpr int kPlanOffBits = 8;

__device__ __forceinline__ int plan_pack(int row, int off_tiles, int nvalid, int flags) {
  return row | (off_tiles << kPlanRowBits) | (nvalid << (kPlanRowBits + kPlanOffBits)) |
         (flags << (kPlanRowBits + kPlanOffBits + 5));
}

// Record position of piece j of the cut row with index c (ob: its overflow base) among rec_cap cut-row slots.
__device__ __forceinline__ int plan_rec_pos(int c, int j, int ob, int rec_cap) {
  return j < 2 ? 2 * c + j : 2 * rec_cap + ob + (j - 2);
}

// Planned calls take their ranges by XCD (see paged_decode_sk_kernel's claim): range j is one of XCD (j mod 8)'s
// ranges, and with enough tiles per range (NT >= 32 ranges) the ranges of even XCDs are 67/64 and those of odd XCDs
// 61/64 of the mean: at equal work the odd XCDs' workgroups finished ~15 us after the even ones' at 576 rows (per-
// wave XCC_ID stamps).  Measured at 576 rows, us per call against the unplanned call on the same box (191.6-192.3):
// equal ranges claimed the same way -1.0, weights +-1/32 -3.7, +-3/64 -4.5, +-1/16 -2.9 to -4.2, +-5/64 -3.2,
// +-3/32 -1.8, +-1/8 +0.5 (two passes each).  Range k starts at floor(NT W(k) / W(ge)),
// W(k) = 64 k + 3 (k & 1) the summed weights of ranges 0 .. k-1; every range keeps at least 30 tiles, and the ranges
// still cut the tile sequence in order, as the combine's record layout requires.
constexpr int kPlanWScale = 64;  // range weights kPlanWScale +- kPlanWDelta: 67/64 on even XCDs, 61/64 on odd ones
constexpr int kPlanWDelta = 3;
__device__ __forceinline__ bool plan_weighted(int NT, int ge) { return NT >= 32 * ge; }
__device__ __forceinline__ uint64_t plan_w(int k) {
  return (uint64_t)kPlanWScale * (uint64_t)k + (uint64_t)(kPlanWDelta * (k & 1));
}
__device__ __forceinline__ int plan_lo(int k, int NT, int ge) {
  if (!plan_weighted(NT, ge)) return (int)sk_lo(k, NT, ge);
  return (int)((uint64_t)NT * plan_w(k) / plan_w(ge));
}

// Plan t lives at plans + t * plan_stride with the layout of the host's plan_layout.
struct PlanArgs {
  char* plans;
  int64_t plan_stride;
  int64_t bt_stable;  // element stride between the tables
  int64_t wg_off, cut_off, first_off, tiles_off, claim_off;  // byte offsets inside one plan
  int num_tables;
  int halves;
  int rec_cap;        // cut-row descriptors (and pairs of leading record slots) per plan: the decode grid
};

// One launch per frame, 256 threads per workgroup.  Every workgroup scans the rows itself (at most 4,096 ints); the
// tiles, the decode workgroups and the cut rows are spread over the grid.  A tile's thread writes it into every
// table's plan (only the page ids differ between the tables).
template <bool kAppend>
__global__ __launch_bounds__(256) void paged_decode_plan_kernel(const DecodeArgs a, const PlanArgs p) {
  __shared__ int s_ctx[kSkMaxRows];
  __shared__ int s_prefix[kSkMaxRows + 1];
  __shared__ int s_cut[kSkMaxRows + 1];  // per row: cut rows before it | overflow records before it << 16
  __shared__ int s_wsum[16];
  const int NT = sk_tile_scan<kAppend>(a, s_ctx, s_prefix, s_wsum);
  const int ge = sk_effective_grid(a.grid, NT);
  const int B = a.batch;
  const int tid = threadIdx.x;
  const int nthr = blockDim.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  // The range holding tile t: the largest k with plan_lo(k) <= t (equal ranges: ((t + 1) ge - 1) / NT).
  const bool weighted = plan_weighted(NT, ge);
  // Weighted: plan_lo(k) <= t iff W(k) <= M = floor(((t + 1) W(ge) - 1) / NT), and W(k) = 16 k + (k & 1) is increasing
  // with W(M / 16 + 1) > M, so k is M / 16 or one less.
  auto wg_of = [&](int t) {
    if (!weighted) return (int)udiv_fit((uint64_t)(t + 1) * (uint64_t)ge - 1, (uint32_t)NT);
    const int64_t M = (int64_t)(((uint64_t)(t + 1) * plan_w(ge) - 1) / (uint64_t)NT);
    int k = (int)(M / kPlanWScale);
    if ((int64_t)plan_w(k) > M) --k;
    return min(max(k, 0), ge - 1);
  };
  auto row_cut = [&](int r, int& kf, int& nseg) {
    const int p0 = s_prefix[r], p1 = s_prefix[r + 1];
    kf = p1 > p0 ? wg_of(p0) : 0;
    nseg = p1 > p0 ? wg_of(p1 - 1) - kf + 1 : 0;
    return nseg > 1;
  };
  // Second scan: cut rows (low 16 bits) and overflow pieces (high 16 bits) before each row.
  {
    const int per = (B + nthr - 1) / nthr;
    const int r0 = min(B, tid * per), r1 = min(B, r0 + per);
    int sum = 0;
    for (int r = r0; r < r1; ++r) {
      int kf, nseg;
      if (row_cut(r, kf, nseg)) sum += 1 + ((nseg - 2) << 16);
    }
    const int x = wave_scan_incl(sum);
    if (lane == 63) s_wsum[wv] = x;  // (sk_tile_scan's last reads of s_wsum precede its closing barrier)
    __syncthreads();
    const int wt = wave_scan_incl(lane < (nthr >> 6) ? s_wsum[lane] : 0);
    int run = (wv == 0 ? 0 : __builtin_amdgcn_readlane(wt, wv - 1)) + x - sum;
    for (int r = r0; r < r1; ++r) {
      s_cut[r] = run;
      int kf, nseg;
      if (row_cut(r, kf, nseg)) run += 1 + ((nseg - 2) << 16);
    }
    if (tid == nthr - 1) s_cut[B] = run;
    __syncthreads();
  }
  const int ncut = s_cut[B] & 0xFFFF;
  // The largest row r with s_prefix[r] <= t (t < NT; an empty row shares its successor's prefix).
  auto row_of = [&](int t) {
    int lo = 0, hi = B;
    while (hi - lo > 1) {
      const int md = (lo + hi) >> 1;
      if (s_prefix[md] <= t) lo = md; else hi = md;
    }
    return lo;
  };
  auto rec_of = [&](int r, int j) {
    const int c = s_cut[r];
    return plan_rec_pos(c & 0xFFFF, j, c >> 16, p.rec_cap);
  };
  const int stride = gridDim.x * nthr;
  // The three kinds of items start on different workgroups (tiles from the first, workgroup ranges from the last,
  // cut rows from the middle), so that no workgroup's chain holds two kinds; the last two have one item per table.
  const int gx = gridDim.x;
  // Decode workgroup ranges, exactly as the unplanned kernel computes them, and where its two records go; workgroups
  // past the effective grid get an empty range and exit.
  for (int it = (gx - 1 - (int)blockIdx.x) * nthr + tid; it < a.grid * p.num_tables; it += stride) {
    const int w = it % a.grid, tb = it / a.grid;
    int v[kPlanWgInts] = {0, 0, 0, -1, 0, 0, -1, -1};
    if (w < ge) {
      const int lo_w = plan_lo(w, NT, ge), hi_w = plan_lo(w + 1, NT, ge);
      const int mid = p.halves == 2 ? lo_w + (hi_w - lo_w) / 2 : hi_w;
      int mid_row = -1;
      if (p.halves == 2 && lo_w < mid && mid < hi_w) {
        const int r = row_of(mid);
        mid_row = s_prefix[r] < mid ? r : -1;
      }
      v[0] = lo_w;
      v[1] = hi_w;
      v[2] = mid;
      v[3] = mid_row;
      if (mid_row >= 0) {
        v[4] = s_prefix[mid_row] >= lo_w && s_prefix[mid_row + 1] <= hi_w;
        v[5] = s_prefix[mid_row] <= lo_w;
      }
      int kf, nseg;
      // Slot 0: the row holding the range's first tile, when cut (piece w - kf); slot 1: the row holding its last
      // tile, when cut and starting after the first tile (its first piece).
      const int r0 = row_of(lo_w);
      if (row_cut(r0, kf, nseg)) v[6] = rec_of(r0, w - kf);
      const int r1 = row_of(hi_w - 1);
      if (s_prefix[r1] > lo_w && row_cut(r1, kf, nseg)) v[7] = rec_of(r1, 0);
    }
    int4* d = reinterpret_cast<int4*>(p.plans + tb * p.plan_stride + p.wg_off) + 2 * (int64_t)w;
    d[0] = make_int4(v[0], v[1], v[2], v[3]);
    d[1] = make_int4(v[4], v[5], v[6], v[7]);
  }
  // The range flags start at zero; every planned call's combine clears them again.
  if (blockIdx.x == 0) {
    for (int i = tid; i < p.rec_cap * p.num_tables; i += nthr)
      reinterpret_cast<int*>(p.plans + (i / p.rec_cap) * p.plan_stride + p.claim_off)[i % p.rec_cap] = 0;
  }
  // Cut-row descriptors (row, pieces, overflow base, 0), in row order; the slots past the last cut row get row -1.
  const int ncr = B + p.rec_cap;
  for (int it = (((int)blockIdx.x + gx / 2) % gx) * nthr + tid; it < ncr * p.num_tables; it += stride) {
    const int r = it % ncr, tb = it / ncr;
    int4 e;
    int idx;
    if (r < B) {
      int kf, nseg;
      if (!row_cut(r, kf, nseg)) continue;
      idx = s_cut[r] & 0xFFFF;
      e = make_int4(r, nseg, s_cut[r] >> 16, 0);
    } else {
      idx = ncut + (r - B);
      if (idx >= p.rec_cap) continue;
      e = make_int4(-1, 0, 0, 0);
    }
    reinterpret_cast<int4*>(p.plans + tb * p.plan_stride + p.cut_off)[idx] = e;
  }
  // Tiles: the workgroup that holds tile t is wg_of(t).  A tile among the first 64 of its wave's range goes into the
  // wave's first list, a later one into the per-tile entries.
  for (int t = blockIdx.x * nthr + tid; t < NT; t += stride) {
    const int k = wg_of(t);
    const int lo_w = plan_lo(k, NT, ge), hi_w = plan_lo(k + 1, NT, ge);
    const int mid = p.halves == 2 ? lo_w + (hi_w - lo_w) / 2 : hi_w;
    const int half = t >= mid ? 1 : 0;
    const int lo = half ? mid : lo_w, hi = half ? hi_w : mid;
    const int row = row_of(t);
    const int mt = t - s_prefix[row];
    const int ntr = s_prefix[row + 1] - s_prefix[row];
    const int tok = mt * kTile;
    const int pidx = tok / a.page_size;
    const int off = tok - pidx * a.page_size;
    const int nvalid = min(kTile, s_ctx[row] - tok);
    const int flags = ((mt == 0 || t == lo) ? kFirst : 0) | ((mt == ntr - 1 || t == hi - 1) ? kLast : 0) |
                      (mt == 0 ? kRowStart : 0) | (mt == ntr - 1 ? kRowEnd : 0);
    const int y = plan_pack(row, off / kTile, nvalid, flags);
    const int32_t* bt = a.bt + (int64_t)row * a.bt_sb + pidx;
    const int64_t dst = t - lo < 64 ? p.first_off + (((int64_t)k * p.halves + half) * 64 + (t - lo)) * 8
                                    : p.tiles_off + (int64_t)t * 8;
    // All tables' page ids of a pass are loaded before the first store (the compiler cannot move a load above a
    // store that may alias it), unconditionally (a table index past the last reads the last table again: a load
    // under a branch would be waited for at the branch's end): one round trip per 32 tables instead of one per table.
    for (int tb0 = 0; tb0 < p.num_tables; tb0 += 32) {
      int pg[32];
#pragma unroll
      for (int u = 0; u < 32; ++u) pg[u] = bt[(int64_t)min(tb0 + u, p.num_tables - 1) * p.bt_stable];
#pragma unroll
      for (int u = 0; u < 32; ++u)
        if (tb0 + u < p.num_tables)
          *reinterpret_cast<int2*>(p.plans + (tb0 + u) * p.plan_stride + dst) = make_int2(pg[u], y);
    }
  }
}

// kHalves == 2 (8 KV heads): each workgroup runs two waves per KV head, the first taking the first half of the
// workgroup's tile range and the second the other half, so a CU holds one workgroup of 16 waves instead of two of 8.
// The row that straddles the midpoint is merged in LDS (the two waves' states) instead of through two partial
// records in memory, which halves the records: each costs ~1.6 us per MB written inside the call's read stream.
// Every record keeps its meaning for the combine (slot 0: the segment opened at the range start, slot 1: the one
// closed at the range end), and a row held whole by the workgroup is written directly.
//
// kPlan: a planned call (the range and the waves' first tile lists come from the per-frame plan).
template <bool kAppend, bool kRope = false, int kHalves = 1, bool kPlan = false>
__global__ __launch_bounds__(1024) void paged_decode_sk_kernel(const DecodeArgs a) {
  static_assert(kAppend || !kRope, "the norm/rope form is an append form");
  static_assert(kHalves == 1 || kHalves == 2, "one or two waves per KV head");
  // The norm/rope form's larger stages are sized for 8 KV heads (the host rejects more), so two workgroups still
  // share a CU's LDS; with two halves, one workgroup of 16 waves per CU.
  constexpr int kSt = kRope ? kStageBytesRope : kStageBytes;
  constexpr int kW = (kRope && kHalves == 1) ? 8 : kMaxWaves;
  __shared__ int s_ctx[kSkMaxRows];
  __shared__ int s_prefix[kSkMaxRows + 1];
  __shared__ int s_wsum[16];
  // Segment staging, one array per tile parity (see stage_q).
  __shared__ __align__(16) uint8_t s_stage0[kW * kSt];
  __shared__ __align__(16) uint8_t s_stage1[kW * kSt];
  // Norm/rope form: the q-norm and k-norm weights.
  __shared__ __align__(16) uint16_t s_nw[kRope ? 2 : 1][kD];
  // The record of a wave's first segment when that segment is a partial one (the tail of a row cut at the range
  // start), written to the workspace only after the tile loop: in a 576-row, 296k-token call these writes cost
  // 4.5 us inside the read stream and ~1.5 us less at the end of the range.
  __shared__ __align__(16) float s_first[kW][kPartFloats];
  // Two halves: the straddling row's state of each half (o unnormalised in fp32, then m, l), per KV head.
  constexpr int kMidFloats = kG * kD + 2 * kG;
  __shared__ __align__(16) float s_mid[kHalves == 2 ? 2 : 1][kHalves == 2 ? 8 : 1][kMidFloats];
  // Two halves: the outputs of the first kOutRing rows a wave holds whole, staged here and stored after the tile
  // loop, outside the read stream (further rows are stored at once).  Not in the norm/rope form, which has no
  // register left for the count.
  constexpr bool kStageOut = kHalves == 2 && !kRope;
  constexpr int kOutRing = kStageOut ? 4 : 1;
  __shared__ __align__(16) uint32_t s_out[kStageOut ? kW : 1][kOutRing][kG * kD / 2];
  __shared__ int s_out_row[kStageOut ? kW : 1][kOutRing];
  // Planned calls: each wave's first tile list (64 entries and the 512 B its copy zero-fills).
  __shared__ __align__(16) int2 s_plan[kPlan ? kW : 1][kPlan ? 128 : 1];
  int n_out = 0;
  const int tid = threadIdx.x;
  const int nthr = blockDim.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index
  const int half = kHalves == 2 ? (wv >= a.hkv ? 1 : 0) : 0;
  const int g = wv - half * a.hkv;                           // wave-uniform KV head
  const int lane = tid & 63;
  const int grp = lane >> 4;
  const int dl = (lane & 15) * 8;
  const int B = a.batch;

  if constexpr (kRope) {
    // Waves 0 and 1 copy the q-norm and k-norm weights straight into LDS (the first barrier waits for them), so
    // wave 0 reaches the prologue's other loads without waiting for these.
    if (wv < 2 && lane < kD / 8)
      lds_copy16(make_rsrc(wv == 0 ? a.qn_w : a.kn_w, kD * 2), &s_nw[kRope ? (wv & 1) : 0][0], (uint32_t)lane * 16);
  }

  // Prologue: tiles per row and their exclusive prefix sum (block-wide scan).  A planned call reads its range and
  // its waves' first tile lists from the plan instead (one round trip, no scan, no table lookup).
  int NT = 0, ge = 0;
  if constexpr (!kPlan) {
    NT = sk_tile_scan<kAppend>(a, s_ctx, s_prefix, s_wsum);
    if (blockIdx.x == 0) {
      for (int r = tid; r <= B; r += nthr) a.prefix[r] = s_prefix[r];
    }
    ge = sk_effective_grid(a.grid, NT);
    if ((int)blockIdx.x >= ge) return;
  }
  // Planned calls: a workgroup takes the range its XCD's share of the plan holds for it (range j belongs to XCD
  // j mod 8, and the plan weights the ranges by XCD), wherever the dispatcher put it: it reads its XCD id, guesses
  // the range a round-robin placement gives it (workgroup 8i + c on XCD x: range 8i + x) and claims that range's flag
  // with one exchange; on a collision (the placement was not round robin) it takes the next free range.  Every range
  // is taken exactly once (one flag per range, as many workgroups as ranges) and is the same range whoever takes it,
  // so the output does not depend on the placement.  The exchange goes out with the loads of the guessed range and its
  // first tile list, on a flag no other workgroup touches, so it costs no round trip of its own; the planned combine
  // clears the flags for the next call.
  __shared__ int s_claim;
  // Planned calls: the taken range's plan item (kPlanWgInts values), read by one thread with the claim.
  __shared__ int s_pwg[kPlan ? kPlanWgInts : 1];
  [[maybe_unused]] int krange = blockIdx.x;
  [[maybe_unused]] const int* const pwg = s_pwg;
  if constexpr (kPlan) {
    // The kernel arguments of the tile loop are read in the same batch as the claim's: left to itself the compiler
    // reads them after the claim's exchange has returned, one more round trip ahead of the first K/V load.
    __asm__ volatile("" ::"s"(a.q), "s"(a.kc), "s"(a.vc), "s"(a.num_pages), "s"(a.page_bytes), "s"(a.out),
                     "s"(a.ws), "s"(a.hkv), "s"(a.grid), "s"(a.plan_wg), "s"(a.plan_first), "s"(a.plan_claim));
    const int xcc = __builtin_amdgcn_s_getreg(20 | (0 << 6) | (3 << 11)) & 7;  // HW_REG_XCC_ID, bits 0-3
    const int kspec = min((int)(blockIdx.x & ~7u) + xcc, a.grid - 1);
    auto load_list = [&](int k) {
      // The wave's first tile list goes straight into LDS (lanes 0-31 copy 16 B each; the other lanes' out-of-range
      // copies write zeros over the next 512 B): no register holds it through the tile loop.
      lds_copy16(make_rsrc(a.plan_first + ((int64_t)k * kHalves + half) * 64, 64 * sizeof(int2)),
                 &s_plan[kPlan ? wv : 0][0], lane < 32 ? (uint32_t)lane * 16 : kOutOfRange);
    };
    load_list(kspec);
    if (tid == 0) {
      // The guessed range's item is read beside the exchange (one round trip for both); another range's only after
      // a collision.
      const int4* w = reinterpret_cast<const int4*>(a.plan_wg + (int64_t)kspec * kPlanWgInts);
      int4 w0 = w[0], w1 = w[1];
      int got = -1;
      for (int d = 0; d < a.grid && got < 0; ++d) {
        const int k = kspec + d < a.grid ? kspec + d : kspec + d - a.grid;
        if (__hip_atomic_exchange(a.plan_claim + k, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0) got = k;
      }
      if (got >= 0 && got != kspec) {
        w = reinterpret_cast<const int4*>(a.plan_wg + (int64_t)got * kPlanWgInts);
        w0 = w[0];
        w1 = w[1];
      }
      s_claim = got;
      *reinterpret_cast<int4*>(&s_pwg[0]) = w0;
      *reinterpret_cast<int4*>(&s_pwg[kPlan ? 4 : 0]) = w1;
    }
    __syncthreads();
    krange = __builtin_amdgcn_readfirstlane(s_claim);
    if (krange != kspec) {
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the guessed list's copy has landed before it is replaced
      if (krange >= 0) load_list(krange);
    }
    if (krange < 0) return;  // no free range (one flag per launched workgroup: does not happen)
  }
  // The workgroup's tile range [lo_w, hi_w) and, with two halves, its midpoint; the row that runs across the
  // midpoint (tiles mid - 1 and mid in the same row), if any.  Only two values stay live through the tile loop (the
  // kernel is at its register limit): slot0_tile, the tile whose segment is the range's first (record slot 0), and
  // mid_cut_tile, the midpoint when a row runs across it, else -1.
  auto range_of = [&](int& lo_w, int& hi_w, int& mid, int& mid_row) __attribute__((always_inline)) {
    if constexpr (kPlan) {
      lo_w = __builtin_amdgcn_readfirstlane(pwg[0]);
      hi_w = __builtin_amdgcn_readfirstlane(pwg[1]);
      mid = __builtin_amdgcn_readfirstlane(pwg[2]);
      mid_row = __builtin_amdgcn_readfirstlane(pwg[3]);
      return;
    }
    lo_w = (int)sk_lo(blockIdx.x, NT, ge);
    hi_w = (int)sk_lo(blockIdx.x + 1, NT, ge);
    mid = kHalves == 2 ? lo_w + (hi_w - lo_w) / 2 : hi_w;
    mid_row = -1;
    if (kHalves == 2 && lo_w < mid && mid < hi_w) {
      const int r = row_at_or_before(s_prefix, B, mid, lane);  // uniform: a scalar
      mid_row = s_prefix[r] < mid ? r : -1;
    }
  };
  int lo_w, hi_w, mid, mid_row;
  range_of(lo_w, hi_w, mid, mid_row);
  if (kPlan && lo_w >= hi_w) return;  // past the effective grid
  const int lo = half == 0 ? lo_w : mid;                 // this wave's half
  const int hi = half == 0 ? mid : hi_w;
  const int slot0_tile = (half == 0 || mid == lo_w) ? lo : -1;
  const int mid_cut_tile = mid_row >= 0 ? mid : -1;

  const uint32_t lane_off = (uint32_t)((grp * a.kv_st + g * a.kv_sh + dl) * 2);
  float* part = a.ws + (int64_t)blockIdx.x * kSkSlots * a.hkv * kPartFloats;
  // This KV head's record of slot s (0: the piece opened at the range's first tile, 1: the piece cut at its end).
  // A planned call writes it where the plan puts it (the planned combine finds a cut row's records by the row's
  // index among the cut rows); the plan marks a slot the workgroup does not fill with -1.
  auto rec_ptr = [&](int slot) -> float* {
    if constexpr (kPlan) {
      const int pos = pwg[6 + slot];
      return pos >= 0 ? a.ws + ((int64_t)pos * a.hkv + g) * kPartFloats : nullptr;
    }
    return part + (slot * a.hkv + g) * kPartFloats;
  };

  uint8_t* const st0 = s_stage0 + wv * kSt;
  uint8_t* const st1 = s_stage1 + wv * kSt;
  uint4 q[kG];
  float m[kG], l[kG], acc[kG][8];
  reset_state(m, l, acc);
  int seg_row = 0, seg_flags = 0, seg_slot = 0;  // seg_slot 2: the second half's part of the straddling row
  bool first_deferred = false;
  q[0] = q[1] = make_uint4(0u, 0u, 0u, 0u);

  for (int cb = lo; cb < hi; cb += 64) {
    TileList L;
    L.n = min(64, hi - cb);
    L.page = -1;
    L.off = 0;
    L.nvalid = 0;
    int vrow = 0, vflags = 0;
    if constexpr (kPlan) {
      // The wave's first list was loaded with the range; later ones (more than 64 tiles per wave) by one load.
      int2 e = make_int2(-1, 0);
      if (cb == lo) {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the first list's copy (nothing younger is in flight)
        __asm__ volatile("" ::: "memory");
        e = s_plan[kPlan ? wv : 0][lane];
      } else if (lane < L.n) {
        e = a.plan_tiles[cb + lane];
      }
      if (lane < L.n) {
        L.page = e.x;
        vrow = e.y & ((1 << kPlanRowBits) - 1);
        L.off = ((e.y >> kPlanRowBits) & ((1 << kPlanOffBits) - 1)) * kTile;
        L.nvalid = (e.y >> (kPlanRowBits + kPlanOffBits)) & 31;
        vflags = (e.y >> (kPlanRowBits + kPlanOffBits + 5)) & 15;
      }
    }
    // The rows of the list's first and last tiles, by the whole wave; each lane then searches only between them.
    // (Not in the norm/rope form: at its register limit the two bounds spilled.)
    int lo0 = 0, hi0 = B;
    if constexpr (!kRope && !kPlan) {
      lo0 = row_at_or_before(s_prefix, B, cb, lane);
      hi0 = row_at_or_before(s_prefix, B, cb + L.n - 1, lane) + 1;
    }
    if (!kPlan && lane < L.n) {
      const int t = cb + lane;
      int lo_r = lo0, hi_r = hi0;  // largest row with prefix[row] <= t
      while (hi_r - lo_r > 1) {
        const int mid = (lo_r + hi_r) >> 1;
        if (s_prefix[mid] <= t) lo_r = mid; else hi_r = mid;
      }
      const int row = lo_r;
      const int mt = t - s_prefix[row];
      const int ntr = s_prefix[row + 1] - s_prefix[row];
      const int tok = mt * kTile;
      const int pidx = tok / a.page_size;
      L.page = a.bt[(int64_t)row * a.bt_sb + pidx];
      L.off = tok - pidx * a.page_size;
      L.nvalid = min(kTile, s_ctx[row] - tok);
      vrow = row;
      vflags = ((mt == 0 || t == lo) ? kFirst : 0) | ((mt == ntr - 1 || t == hi - 1) ? kLast : 0) |
               (mt == 0 ? kRowStart : 0) | (mt == ntr - 1 ? kRowEnd : 0);
    }

    // Segment bookkeeping for tile j, run before tile j+1 is issued (no memory operand involved).
    auto open_segment = [&](int j) {
      const int fl = readlane(vflags, j);
      if (fl & kFirst) {
        seg_row = readlane(vrow, j);
        seg_flags = fl;
        seg_slot = cb + j == slot0_tile ? 0 : (cb + j == mid_cut_tile ? 2 : 1);
        reset_state(m, l, acc);
      }
    };
    // Consumes tile j after tile j+1 was issued; the segment's q (and the new k/v rows) come from the stage
    // array of tile j's parity, which tile j+1's copies do not touch.
    auto process = [&](KVTile& T, int j, const uint8_t* st) {
      const int fl = readlane(vflags, j);
      if (!kRope && (fl & (kAppend ? (kFirst | kRowEnd) : kFirst))) {
        // The compiler does not order LDS reads after these copies by itself: wait until tile j's group
        // (issued before tile j+1's) has landed.  Tile j+1's group, and the append form's slot stores of
        // the previous tile, are younger; the count is the smallest group (8 loads and the q copy), so
        // the wait is exact when the younger operations are one such group and conservative otherwise.  (The
        // norm/rope form's prep() has already waited for this stage and rewritten it.)
        __builtin_amdgcn_s_waitcnt(kWaitGroup);
        __asm__ volatile("" ::: "memory");
      }
      if (fl & kFirst) {
        q[0] = ld16(st + dl * 2);
        q[1] = ld16(st + kD * 2 + dl * 2);
      }
      if constexpr (kAppend) {
        if (fl & kRowEnd) {
          take_staged_token(a, L, grp, j, st, T);
          // The new token's slot lies in this tile's page: hand its id to the combine kernel, which stores the slot
          // (one wave per row; the combine then needs no table lookup of its own).
          if (g == 0 && lane == 0) a.slot_page[readlane(vrow, j)] = readlane(L.page, j);
        }
      }
      tile_update(a, L, q, T, j, grp, m, l, acc);
      if (fl & kLast) {
        merge_lanes(16, m, l, acc);
        merge_lanes(32, m, l, acc);
        if ((seg_flags & kRowStart) && (fl & kRowEnd)) {
          if (kStageOut && n_out < kOutRing) {
            if (grp == 0) {
              uint32_t* o = s_out[kStageOut ? wv : 0][kStageOut ? n_out : 0];
#pragma unroll
              for (int h = 0; h < kG; ++h) {
                const float s = l[h] > 0.f ? 1.f / l[h] : 0.f;
                const float* x = acc[h];
                st16(o + h * kD / 2 + dl / 2, make_uint4(pack_bf16x2(x[0] * s, x[1] * s), pack_bf16x2(x[2] * s, x[3] * s),
                                                         pack_bf16x2(x[4] * s, x[5] * s), pack_bf16x2(x[6] * s, x[7] * s)));
              }
              s_out_row[kStageOut ? wv : 0][kStageOut ? n_out : 0] = seg_row;
            }
            ++n_out;
          } else {
            write_output(a, seg_row, g, grp, dl, l, acc);
          }
        } else if (kHalves == 2 && mid_cut_tile >= 0 && (half == 0 ? cb + j == mid_cut_tile - 1 : seg_slot == 2)) {
          // The straddling row's part in this half: its state goes to LDS, merged after the loop.
          float* r = s_mid[kHalves == 2 ? half : 0][kHalves == 2 ? g : 0];
          if (grp == 0) {
#pragma unroll
            for (int h = 0; h < kG; ++h) {
              st16(r + h * kD + dl, make_uint4(__float_as_uint(acc[h][0]), __float_as_uint(acc[h][1]),
                                               __float_as_uint(acc[h][2]), __float_as_uint(acc[h][3])));
              st16(r + h * kD + dl + 4, make_uint4(__float_as_uint(acc[h][4]), __float_as_uint(acc[h][5]),
                                                   __float_as_uint(acc[h][6]), __float_as_uint(acc[h][7])));
            }
          }
          if (lane == 0)
            st16(r + kG * kD, __builtin_bit_cast(uint4, make_float4(m[0], m[1], l[0], l[1])));
        } else {
          if (seg_slot == 0) {
            write_partial(&s_first[wv][0], lane, grp, dl, m, l, acc);
            first_deferred = true;
          } else if (float* const P = rec_ptr(1)) {
            write_partial(P, lane, grp, dl, m, l, acc);
          }
        }
      }
    };

    auto issue = [&](int j, KVTile& T, uint8_t* st) {
      const int jj = j < L.n ? j : 0;
      const int fl = j < L.n ? readlane(vflags, jj) : 0;
      const int row = readlane(vrow, jj);
      auto stage = [&]() {
        stage_q(a, row, g, lane, (fl & kFirst) != 0, st);
        if constexpr (kRope) {
          if (fl & (kFirst | kRowEnd)) stage_rope(a, row, lane, st);
        }
        if constexpr (kAppend) {
          if (fl & kRowEnd) stage_new_rows(a, row, g, lane, st);
        }
      };
      // The norm/rope form copies the stage ahead of the tile's loads, so prep() can wait for it with those loads
      // still in flight.
      if constexpr (kRope) stage();
      issue_tile(a, L, lane_off, grp, j, T);
      if constexpr (!kRope) stage();
      // Keep the whole tile's loads ahead of the consumer: no instruction of the next tile_update may
      // be scheduled between them (that would wait for the current tile in the middle of the issue).
      __builtin_amdgcn_sched_barrier(0);
    };
    // Norm/rope form: once the tile before j has been consumed (its registers are free), the q rows tile j opens a
    // segment with and the k row it ends its row with are normalised and rotated in place in tile j's stage, so
    // process() reads them as the plain append form does.  Only tile j's 8 loads are younger than its stage.
    auto prep = [&](int j, uint8_t* st) {
      if constexpr (kRope) {
        if (j >= L.n) return;
        const int fl = readlane(vflags, j);
        if (!(fl & (kFirst | kRowEnd))) return;
        __builtin_amdgcn_s_waitcnt(0x0F70 | 8);
        __asm__ volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        const uint8_t* c = st + kStageRope + dl * 2;
        const uint8_t* sn = c + kD * 2;
        if (fl & kFirst) {
#pragma unroll
          for (int h = 0; h < kG; ++h) {
            const uint4 y = qk_norm_rope16_lds(ld16(st + h * kD * 2 + dl * 2),
                                               reinterpret_cast<const uint8_t*>(&s_nw[0][dl]), c, sn, a.eps);
            if (grp == 0) st16(st + h * kD * 2 + dl * 2, y);
          }
        }
        if (fl & kRowEnd) {
          const uint4 y = qk_norm_rope16_lds(ld16(st + kStageNew + dl * 2),
                                             reinterpret_cast<const uint8_t*>(&s_nw[kRope ? 1 : 0][dl]), c, sn, a.eps);
          if (grp == 0) st16(st + kStageNew + dl * 2, y);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    };

    KVTile A, Bt;
    issue(0, A, st0);
    prep(0, st0);
    for (int j = 0; j < L.n; j += 2) {
      open_segment(j);
      issue(j + 1, Bt, st1);
      process(A, j, st0);
      prep(j + 1, st1);
      if (j + 1 < L.n) open_segment(j + 1);
      issue(j + 2, A, st0);
      if (j + 1 < L.n) process(Bt, j + 1, st1);
      prep(j + 2, st0);
    }
  }
  if (first_deferred && lane < kPartFloats / 4) {
    if (float* const P = rec_ptr(0)) st16(P + lane * 4, ld16(&s_first[wv][lane * 4]));
  }
  if constexpr (kStageOut) {
    if (grp == 0) {
      for (int i = 0; i < n_out; ++i) {
        const int row = s_out_row[wv][i];
#pragma unroll
        for (int h = 0; h < kG; ++h)
          *reinterpret_cast<uint4*>(a.out + row * a.o_sb + (kG * g + h) * a.o_sh + dl) = ld16(&s_out[wv][i][h * kD / 2 + dl / 2]);
      }
    }
  }
  // The last issue() targets tiles past the list; let its (out-of-bounds) copies into LDS land before the
  // wave ends.
  __builtin_amdgcn_s_waitcnt(0x0F70);
  if constexpr (kHalves == 2) {
    // The straddling row: the first half's wave of each KV head merges both halves' states (the same arithmetic as
    // merge_lanes) and writes the row, or, when the row runs past the workgroup's range, its record.
    __syncthreads();
    range_of(lo_w, hi_w, mid, mid_row);
    if (mid_row >= 0 && half == 0) {
      const float* r0 = s_mid[0][kHalves == 2 ? g : 0];
      const float* r1 = s_mid[kHalves == 2 ? 1 : 0][kHalves == 2 ? g : 0];
      const float4 ml0 = __builtin_bit_cast(float4, ld16(r0 + kG * kD));
      const float4 ml1 = __builtin_bit_cast(float4, ld16(r1 + kG * kD));
      const float m0[kG] = {ml0.x, ml0.y}, l0[kG] = {ml0.z, ml0.w};
      const float m1[kG] = {ml1.x, ml1.y}, l1[kG] = {ml1.z, ml1.w};
#pragma unroll
      for (int h = 0; h < kG; ++h) {
        const float mn = fmaxf(m0[h], m1[h]);
        const float w0 = fast_exp2(m0[h] - mn);
        const float w1 = fast_exp2(m1[h] - mn);
        l[h] = l0[h] * w0 + l1[h] * w1;
        m[h] = mn;
        const uint4 a0 = ld16(r0 + h * kD + dl), a1 = ld16(r0 + h * kD + dl + 4);
        const uint4 b0 = ld16(r1 + h * kD + dl), b1 = ld16(r1 + h * kD + dl + 4);
        const uint32_t av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
        const uint32_t bv[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
        for (int d = 0; d < 8; ++d) acc[h][d] = __uint_as_float(av[d]) * w0 + __uint_as_float(bv[d]) * w1;
      }
      // Slot 0 is the segment opened at the range's first tile (the row starts there or before), as the combine
      // expects; slot 1 one that runs past the range's end and started after its first tile.
      const bool from_lo = kPlan ? pwg[5] != 0 : s_prefix[mid_row] <= lo_w;
      if (kPlan ? pwg[4] != 0 : (s_prefix[mid_row] >= lo_w && s_prefix[mid_row + 1] <= hi_w))
        write_output(a, mid_row, g, grp, dl, l, acc);
      else if (float* const P = rec_ptr(from_lo ? 0 : 1))
        write_partial(P, lane, grp, dl, m, l, acc);
    }
  }
}

// One workgroup per row: merges the partial records of rows that straddle workgroup ranges, and
// writes zeros for rows with no context.
//
// Append form: it also writes each row's new k/v row into its page slot.  The decode kernel attends with the staged
// copies and never reads the slot, and no other row reads it in the same call, so the store can wait for this
// kernel, which runs without a read stream to disturb: the same 2.1 MB of 256 B stores cost ~5 us inside the decode
// kernel's read stream (576 rows, 296k tokens).  The slot's page id comes from the decode kernel (the wave holding
// the row's last tile writes it to the workspace), so the slot's loads (the new rows, the row's cache_seqlens, that
// id) all go out with the prefix, one round trip, and the stores come last: the slot write adds no round trip to
// the merge's chain (the table lookup it used to make here was a second one).
template <bool kAppend, bool kRope = false>
__global__ __launch_bounds__(1024) void paged_decode_sk_combine_kernel(const DecodeArgs a) {
  const int b = blockIdx.x;
  const int g = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);  // wave-uniform KV head
  const int lane = threadIdx.x & 63;
  const int p0 = a.prefix[b];
  const int p1 = a.prefix[b + 1];
  const int NT = a.prefix[a.batch];
  // Position c = cache_seqlens[b] receives the new token, unless the row is skipped (row_ctx: c < 0 or c at
  // capacity); an invalid page id receives nothing.  Lane l copies 4 bytes of head g's k and v rows.
  int c = -1, page = -1;
  uint32_t kw = 0u, vw = 0u;
  if constexpr (kAppend) {
    c = a.seqlens[b];
    kw = reinterpret_cast<const uint32_t*>(a.k_new + (int64_t)b * a.kn_sb + g * kD)[lane];
    vw = reinterpret_cast<const uint32_t*>(a.v_new + (int64_t)b * a.vn_sb + g * kD)[lane];
    if constexpr (kRope)  // the same bits the decode kernel attended with (qk_norm_rope16)
      kw = qk_norm_rope64(kw, reinterpret_cast<const uint32_t*>(a.kn_w)[lane],
                          reinterpret_cast<const uint32_t*>(a.rcos + (int64_t)b * a.rs_sb)[lane],
                          reinterpret_cast<const uint32_t*>(a.rsin + (int64_t)b * a.rs_sb)[lane], a.eps);
    if (c >= 0 && c < a.max_pages * a.page_size) page = a.slot_page[b];
  }
  auto store_slot = [&]() {
    if constexpr (kAppend) {
      if ((unsigned)page < (unsigned)a.num_pages) {
        const int pidx = c / a.page_size;
        const int64_t dst = (int64_t)page * a.kv_sp + (int64_t)(c - pidx * a.page_size) * a.kv_st + (int64_t)g * a.kv_sh;
        __builtin_nontemporal_store(kw, reinterpret_cast<uint32_t*>(const_cast<uint16_t*>(a.kc) + dst) + lane);
        __builtin_nontemporal_store(vw, reinterpret_cast<uint32_t*>(const_cast<uint16_t*>(a.vc) + dst) + lane);
      }
    }
  };
  // (G == 0 only when NT == 0, which implies p1 == p0; testing it here keeps the load of prefix[batch] beside the
  // other two, one round trip, instead of behind this branch.)
  const int64_t G = sk_effective_grid(a.grid, NT);
  if (p1 == p0 || G == 0) {
    write_zero_row(a, b, g, lane);
    store_slot();
    return;
  }
  const int kf = (int)udiv_fit((uint64_t)(p0 + 1) * (uint64_t)G - 1, (uint32_t)NT);
  const int kl = (int)udiv_fit((uint64_t)p1 * (uint64_t)G - 1, (uint32_t)NT);
  if (kf != kl) {
    const int first_slot = sk_lo(kf, NT, G) < p0 ? 1 : 0;
    merge_records(a, b, g, lane, kl - kf + 1, [&](int i) -> const float* {
      const int k = kf + i;
      const int slot = i == 0 ? first_slot : 0;
      return a.ws + (((int64_t)k * kSkSlots + slot) * a.hkv + g) * kPartFloats;
    });
  }
  store_slot();
}

// Planned calls: workgroups of kPlanRowsPerWg rows first (zero rows, and in the append forms the new rows' slot
// stores, as in the combine above; every load of the rows goes out at once), then one per possible cut row.  A cut
// row's first two records sit at positions 2c and 2c + 1 (c: its index among the cut rows), so they are loaded beside
// its descriptor, before the row is known: the merge waits for one memory round trip (a second only for rows cut into
// more than two pieces), where the unplanned combine first loads the prefix sums and then the records.  The merge
// itself is merge_records' arithmetic over the same records in the same order, so the output equals the unplanned
// call's on the same ranges bit for bit.
constexpr int kPlanRowsPerWg = 4;

template <bool kAppend, bool kRope = false>
__global__ __launch_bounds__(1024) void paged_decode_plan_combine_kernel(const DecodeArgs a) {
  const int g = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);  // wave-uniform KV head
  const int lane = threadIdx.x & 63;
  const int nrw = (a.batch + kPlanRowsPerWg - 1) / kPlanRowsPerWg;
  if ((int)blockIdx.x < nrw) {
    const int cap = a.max_pages * a.page_size;
    int c[kPlanRowsPerWg], page[kPlanRowsPerWg];
    uint32_t kw[kPlanRowsPerWg], vw[kPlanRowsPerWg];
    uint32_t wk = 0u;
    if constexpr (kRope) wk = reinterpret_cast<const uint32_t*>(a.kn_w)[lane];
#pragma unroll
    for (int u = 0; u < kPlanRowsPerWg; ++u) {
      const int b = min((int)blockIdx.x * kPlanRowsPerWg + u, a.batch - 1);
      c[u] = a.seqlens[b];
      if constexpr (kAppend) {
        kw[u] = reinterpret_cast<const uint32_t*>(a.k_new + (int64_t)b * a.kn_sb + g * kD)[lane];
        vw[u] = reinterpret_cast<const uint32_t*>(a.v_new + (int64_t)b * a.vn_sb + g * kD)[lane];
        page[u] = a.slot_page[b];
        if constexpr (kRope)
          kw[u] = qk_norm_rope64(kw[u], wk, reinterpret_cast<const uint32_t*>(a.rcos + (int64_t)b * a.rs_sb)[lane],
                                 reinterpret_cast<const uint32_t*>(a.rsin + (int64_t)b * a.rs_sb)[lane], a.eps);
      }
    }
#pragma unroll
    for (int u = 0; u < kPlanRowsPerWg; ++u) {
      const int b = (int)blockIdx.x * kPlanRowsPerWg + u;
      if (b >= a.batch) break;
      if constexpr (kAppend) {
        if (c[u] < 0 || c[u] >= cap) {
          write_zero_row(a, b, g, lane);
          continue;
        }
        // (the slot's page id was written by the decode kernel for every row it attended, so it is only read here)
        if ((unsigned)page[u] < (unsigned)a.num_pages) {
          const int pidx = c[u] / a.page_size;
          const int64_t dst = (int64_t)page[u] * a.kv_sp + (int64_t)(c[u] - pidx * a.page_size) * a.kv_st +
                              (int64_t)g * a.kv_sh;
          __builtin_nontemporal_store(kw[u], reinterpret_cast<uint32_t*>(const_cast<uint16_t*>(a.kc) + dst) + lane);
          __builtin_nontemporal_store(vw[u], reinterpret_cast<uint32_t*>(const_cast<uint16_t*>(a.vc) + dst) + lane);
        }
      } else {
        if (ctx_of<false>(c[u], cap) == 0) write_zero_row(a, b, g, lane);
      }
    }
    return;
  }
  const int ci = blockIdx.x - nrw;
  const int4 d = a.plan_cut[ci];
  const int h = lane >> 5;
  const int d0 = (lane & 31) * 4;
  uint2 raw[8];
  float mr[8], lr[8];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const float* P = a.ws + ((int64_t)(2 * ci + u) * a.hkv + g) * kPartFloats;
    raw[u] = *reinterpret_cast<const uint2*>(reinterpret_cast<const char*>(P) + (h * kD + d0) * 2);
    mr[u] = P[kPartML + h];
    lr[u] = P[kPartML + kG + h];
  }
  // The first two records' loads go out with the descriptor's: the empty asm with a memory clobber keeps the compiler
  // from sinking them below the tests on the descriptor, which would make them a second round trip.
  __asm__ volatile("" ::: "memory");
  // The decode kernel's range flags, cleared for the next call on the plan (one per possible range); the store is
  // issued after the loads, so waiting for the descriptor does not wait for it.
  if (threadIdx.x == 0) __hip_atomic_store(a.plan_claim + ci, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const int b = d.x, count = d.y, ob = d.z;
  if (b < 0) return;
  float M = kMaxSeed, L = 0.f;
  float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int s0 = 0; s0 < count; s0 += 8) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (s0 == 0 && u < 2) continue;  // loaded above
      raw[u] = make_uint2(0u, 0u);
      mr[u] = kMaxSeed;
      lr[u] = 0.f;
      if (s0 + u < count) {
        const float* P = a.ws + ((int64_t)plan_rec_pos(ci, s0 + u, ob, a.plan_rec_cap) * a.hkv + g) * kPartFloats;
        raw[u] = *reinterpret_cast<const uint2*>(reinterpret_cast<const char*>(P) + (h * kD + d0) * 2);
        mr[u] = P[kPartML + h];
        lr[u] = P[kPartML + kG + h];
      }
    }
    merge_fold8(raw, mr, lr, M, L, A);
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  u32x2 o;
  o.x = pack_bf16x2(A.x * inv, A.y * inv);
  o.y = pack_bf16x2(A.z * inv, A.w * inv);
  __builtin_nontemporal_store(o, reinterpret_cast<u32x2*>(a.out + b * a.o_sb + (kG * g + h) * a.o_sh + d0));
}

// ------------------------------------------------------------------------------ fixed-split path
template <bool kAppend>
__global__ __launch_bounds__(1024) void paged_decode_split_kernel(const DecodeArgs a) {
  const int b = blockIdx.x;
  const int s = blockIdx.y;
  const int g = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);  // wave-uniform KV head
  const int lane = threadIdx.x & 63;
  const int grp = lane >> 4;
  const int dl = (lane & 15) * 8;

  const int ctx = row_ctx<kAppend>(a, b);
  if (ctx == 0) {
    if (s == 0) write_zero_row(a, b, g, lane);
    return;
  }
  const int ns = (ctx + a.split_tokens - 1) / a.split_tokens;
  if (s >= ns) return;
  const int t0 = s * a.split_tokens;
  const int t1 = min(ctx, t0 + a.split_tokens);

  TileList L;
  L.n = (t1 - t0 + kTile - 1) / kTile;
  L.page = -1;
  L.off = 0;
  L.nvalid = 0;
  if (lane < L.n) {
    const int t = t0 + kTile * lane;
    const int pidx = t / a.page_size;
    L.page = a.bt[(int64_t)b * a.bt_sb + pidx];
    L.off = t - pidx * a.page_size;
    L.nvalid = min(kTile, t1 - t);
  }
  const uint32_t lane_off = (uint32_t)((grp * a.kv_st + g * a.kv_sh + dl) * 2);

  uint4 q[kG];
  load_q(a, b, g, dl, q);
  float m[kG], l[kG], acc[kG][8];
  reset_state(m, l, acc);

  // Append form: the last tile of the last split holds the new token.
  const int tail = (kAppend && s == ns - 1) ? L.n - 1 : -1;
  auto issue = [&](int j, KVTile& T) {
    issue_tile(a, L, lane_off, grp, j, T);
    __builtin_amdgcn_sched_barrier(0);
  };
  auto consume = [&](KVTile& T, int j) {
    if (kAppend && j == tail) take_new_token(a, L, lane_off, grp, g, j, b, T);
    tile_update(a, L, q, T, j, grp, m, l, acc);
  };

  KVTile A, Bt;
  issue(0, A);
  for (int j = 0; j < L.n; j += 2) {
    issue(j + 1, Bt);
    consume(A, j);
    issue(j + 2, A);
    if (j + 1 < L.n) consume(Bt, j + 1);
  }

  merge_lanes(16, m, l, acc);
  merge_lanes(32, m, l, acc);
  if (ns == 1) {
    write_output(a, b, g, grp, dl, l, acc);
  } else {
    write_partial(a.ws + (((int64_t)b * a.max_splits + s) * a.hkv + g) * kPartFloats, lane, grp, dl, m, l, acc);
  }
}

template <bool kAppend>
__global__ __launch_bounds__(1024) void paged_decode_split_combine_kernel(const DecodeArgs a) {
  const int b = blockIdx.x;
  const int g = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);  // wave-uniform KV head
  const int lane = threadIdx.x & 63;
  const int ctx = row_ctx<kAppend>(a, b);
  if (ctx == 0) return;
  const int ns = (ctx + a.split_tokens - 1) / a.split_tokens;
  if (ns <= 1) return;
  merge_records(a, b, g, lane, ns, [&](int s) -> const float* {
    return a.ws + (((int64_t)b * a.max_splits + s) * a.hkv + g) * kPartFloats;
  });
}

// ------------------------------------------------------------------------------ row-parallel path
// Narrow tables (at most kMaxRowTiles tiles of capacity per row, any batch) and small batches (at most
// kRowMaxBatch rows, up to kRowMaxWaves * kRowMaxPer tiles): one workgroup per (row, KV head) whose W waves take
// the row's tiles round-robin (W = the capacity in tiles up to 16, else 8; wave w streams tiles w, w + W, ..., lane i
// of its list describing tile w + i*W), so a row's tiles are spread over up to 16 waves instead of a chain of
// workgroups and a combine.  Everything that does not depend on the context is loaded at once: the row's context,
// the wave's table entries (entries past the context are read but never used), q, and in the append form the new
// k/v rows (parked in the wave's LDS until the tile that needs them); with one tile per wave (kMulti false) the
// call then waits for two round trips.  Each wave reduces its tiles to one online-softmax state (m, l, acc of both
// query heads); wave 0 merges the W states through LDS and writes the row.  No partial records in memory, no second
// kernel; a row with nothing to attend writes zeros (l = 0).
constexpr int kMaxRowTiles = kOneSplitTokens / kTile;
constexpr int kRowMaxWaves = 16;
constexpr int kRowMaxPer = 8;             // rows of up to kRowMaxWaves * kRowMaxPer tiles = 2,048 tokens
constexpr int kRowMaxBatch = 64;            // beyond, stream-K (equal at 128-256 rows, ahead when ragged)
constexpr int kRowRec = kG * kD + 2 * kG;  // floats per wave state: acc[kG][kD], m[kG], l[kG]
// With several tiles per wave the append form needs more than the 128 registers a 16-wave workgroup allows, so both
// forms then run 8 waves of up to 16 tiles (the same decomposition: the append form stays bitwise equal to a scatter
// followed by the plain form).
constexpr int row_max_waves(bool multi) { return multi ? kRowMaxWaves / 2 : kRowMaxWaves; }

//
// Chunked (split-KV) form, for small batches of long rows: the grid gets a third dimension, chunk c of
// CT = W * row_per consecutive tiles, so one row's tiles spread over up to kChunkMax workgroups per KV head
// instead of the W waves of one CU.  Wave w takes tiles c*CT + w + i*W.  A row whose tiles fit one chunk is
// written directly by its chunk-0 workgroup; otherwise every chunk holding tiles of the row writes its merged
// state (fp32 o = sum p.v, m, l of both query heads) as a record, which paged_decode_chunk_combine_kernel merges.
constexpr int kChunkMax = 16;  // records per (row, KV head): the combine loads them all at once

template <bool kAppend, bool kMulti, bool kRope = false>
__global__ __launch_bounds__(64 * row_max_waves(kMulti)) void paged_decode_row_kernel(const DecodeArgs a) {
  static_assert(kAppend || !kRope, "the norm/rope form is an append form");
  __shared__ __align__(16) float rec[kRowMaxWaves][kRowRec];
  __shared__ __align__(16) uint4 snew[kAppend ? kRowMaxWaves : 1][2][kD / 8];  // per wave: the new k and v rows
  const int b = blockIdx.x;
  const int g = blockIdx.y;
  const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int W = (int)(blockDim.x >> 6);
  const int lane = threadIdx.x & 63;
  const int grp = lane >> 4;
  const int dl = (lane & 15) * 8;
  const int CT = W * a.row_per;              // tiles per chunk (the one-launch path: the whole table)
  const int tb = (int)blockIdx.z * CT;       // first tile of this workgroup's chunk

  // Every load that does not depend on the context goes out together with the row's cache_seqlens entry: the
  // table entry of this lane's tile, q, (append form) the new k/v rows, (norm/rope form) the weights and cos/sin.
  // The empty asm with a memory clobber keeps the compiler from sinking them below the exit test of chunks past the
  // row's end, which would put the table and q behind the seqlens round trip.  The kernel arguments these loads
  // and the exit test need are read in one batch (left to itself the compiler reads them in two, a wait between).
  __asm__ volatile("" ::"s"(a.seqlens), "s"(a.bt), "s"(a.bt_sb), "s"(a.max_pages), "s"(a.page_size), "s"(a.row_per),
                   "s"(a.q), "s"(a.q_sb), "s"(a.q_sh), "s"(a.scale_log2), "s"(a.kc), "s"(a.vc), "s"(a.kv_sp),
                   "s"(a.kv_st), "s"(a.kv_sh));
  const int c_row = a.seqlens[b];
  const int cap = a.max_pages * a.page_size;
  const int t = kTile * (tb + w + lane * W);  // first token of this lane's tile
  const int pidx = min(t, cap - 1) / a.page_size;
  const int page = a.bt[(int64_t)b * a.bt_sb + pidx];
  uint4 q[kG];
  load_q(a, b, g, dl, q);
  uint4 rc = make_uint4(0u, 0u, 0u, 0u), rs = rc, qw = rc, kw = rc, kn = rc, vn = rc;
  if constexpr (kRope) {
    rc = ld16(a.rcos + (int64_t)b * a.rs_sb + dl);
    rs = ld16(a.rsin + (int64_t)b * a.rs_sb + dl);
    qw = ld16(a.qn_w + dl);
    if constexpr (kAppend) kw = ld16(a.kn_w + dl);
  }
  if constexpr (kAppend) {
    const uint32_t dim_off = (uint32_t)(lane & 15) * 16;
    kn = buffer_load16_s(make_rsrc(a.k_new + (int64_t)b * a.kn_sb + g * kD, kD * 2), dim_off, 0);
    vn = buffer_load16_s(make_rsrc(a.v_new + (int64_t)b * a.vn_sb + g * kD, kD * 2), dim_off, 0);
  }
  __asm__ volatile("" ::: "memory");
  if constexpr (kRope) {
#pragma unroll
    for (int h = 0; h < kG; ++h) q[h] = qk_norm_rope16(q[h], qw, rc, rs, a.eps);
  }
  if constexpr (kAppend) {
    if constexpr (kRope) kn = qk_norm_rope16(kn, kw, rc, rs, a.eps);
    if (lane < kD / 8) {
      snew[w][0][lane] = kn;
      snew[w][1][lane] = vn;
    }
  }
  const int ctx = ctx_of<kAppend>(c_row, cap);
  const int nrow = (ctx + kTile - 1) / kTile;  // tiles of the row
  const int nch = (nrow + CT - 1) / CT;        // chunks holding tiles of the row
  // Chunks past the row's end have nothing to do (chunk 0 stays: it writes the zero row of an empty one).  The
  // condition is uniform over the workgroup.
  if (blockIdx.z > 0 && (int)blockIdx.z >= nch) return;
  const int nrc = min(nrow - tb, CT);          // tiles of the row in this chunk

  TileList L;
  L.n = nrc > w ? (nrc - w + W - 1) / W : 0;
  L.page = lane < L.n ? page : -1;
  L.off = t - pidx * a.page_size;
  L.nvalid = lane < L.n ? min(kTile, ctx - t) : 0;
  const uint32_t lane_off = (uint32_t)((grp * a.kv_st + g * a.kv_sh + dl) * 2);

  float m[kG], l[kG], acc[kG][8];
  reset_state(m, l, acc);

  // Append form: the row's last tile (this wave's tile jt if it owns it) holds the new token at nvalid - 1; the 16
  // lanes holding it take this step's k/v rows instead of the stale slot, and store them after the loop.
  const int last = nrow - 1 - tb;  // the row's last tile, counted from this chunk's first
  const int jt = (kAppend && nrow > 0 && last >= 0 && last < CT && last % W == w) ? last / W : -1;
  auto issue = [&](int j, KVTile& T) {
    issue_tile(a, L, lane_off, grp, j, T);
    __builtin_amdgcn_sched_barrier(0);
  };
  auto consume = [&](KVTile& T, int j) {
    if constexpr (kAppend) {
      if (j == jt) {
        const int tn = readlane(L.nvalid, j) - 1;
        const uint4 kn = snew[w][0][lane & 15];
        const uint4 vn = snew[w][1][lane & 15];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (i == (tn >> 2) && grp == (tn & 3)) {
            T.k[i] = kn;
            T.v[i] = vn;
          }
        }
      }
    }
    tile_update(a, L, q, T, j, grp, m, l, acc);
  };

  if constexpr (!kMulti) {
    KVTile A;
    issue(0, A);
    consume(A, 0);
  } else {
    KVTile A, Bt;
    issue(0, A);
    for (int j = 0; j < L.n; j += 2) {
      issue(j + 1, Bt);
      consume(A, j);
      issue(j + 2, A);
      if (j + 1 < L.n) consume(Bt, j + 1);
    }
  }
  if constexpr (kAppend) {
    if (jt >= 0) {
      const int pg = readlane(L.page, jt);
      const int tn = readlane(L.nvalid, jt) - 1;
      if (grp == (tn & 3) && (unsigned)pg < (unsigned)a.num_pages) {
        const int64_t pbase = (int64_t)pg * a.kv_sp;
        const uint32_t slot_off = (uint32_t)((readlane(L.off, jt) + 4 * (tn >> 2)) * a.kv_st * 2);
        buffer_store16_s(snew[w][0][lane & 15], make_rsrc(a.kc + pbase, a.page_bytes), lane_off, slot_off);
        buffer_store16_s(snew[w][1][lane & 15], make_rsrc(a.vc + pbase, a.page_bytes), lane_off, slot_off);
      }
    }
  }

  merge_lanes(16, m, l, acc);
  merge_lanes(32, m, l, acc);
  float* r = rec[w];
  if (grp == 0) {
#pragma unroll
    for (int h = 0; h < kG; ++h) {
      st16(r + h * kD + dl, make_uint4(__float_as_uint(acc[h][0]), __float_as_uint(acc[h][1]),
                                       __float_as_uint(acc[h][2]), __float_as_uint(acc[h][3])));
      st16(r + h * kD + dl + 4, make_uint4(__float_as_uint(acc[h][4]), __float_as_uint(acc[h][5]),
                                           __float_as_uint(acc[h][6]), __float_as_uint(acc[h][7])));
    }
  }
  if (lane < kG) {
    r[kG * kD + lane] = lane == 0 ? m[0] : m[1];
    r[kG * kD + kG + lane] = lane == 0 ? l[0] : l[1];
  }
  __syncthreads();
  if (w != 0) return;

  // Wave 0: lane -> (head h = lane / 32, dims 4*(lane%32)..+4), merging the W states.
  const int h = lane >> 5;
  const int d0 = (lane & 31) * 4;
  float M = kMaxSeed;
  for (int v = 0; v < W; ++v) M = fmaxf(M, rec[v][kG * kD + h]);
  float Ls = 0.f, o[4] = {0.f, 0.f, 0.f, 0.f};
  for (int v = 0; v < W; ++v) {
    const float wgt = fast_exp2(rec[v][kG * kD + h] - M);
    Ls += rec[v][kG * kD + kG + h] * wgt;
    const uint4 x = ld16(&rec[v][h * kD + d0]);
    o[0] += __uint_as_float(x.x) * wgt;
    o[1] += __uint_as_float(x.y) * wgt;
    o[2] += __uint_as_float(x.z) * wgt;
    o[3] += __uint_as_float(x.w) * wgt;
  }
  if (nch > 1) {
    // Chunked form, a row spread over several chunks: this chunk's record, [kG][kD] o then m[kG], l[kG] (fp32).
    float* r = a.ws + (((int64_t)b * gridDim.z + blockIdx.z) * a.hkv + g) * kRowRec;
    st16(r + h * kD + d0, make_uint4(__float_as_uint(o[0]), __float_as_uint(o[1]), __float_as_uint(o[2]),
                                     __float_as_uint(o[3])));
    if ((lane & 31) == 0) {
      r[kG * kD + h] = M;
      r[kG * kD + kG + h] = Ls;
    }
    return;
  }
  const float inv = Ls > 0.f ? 1.f / Ls : 0.f;
  uint2 ov;
  ov.x = pack_bf16x2(o[0] * inv, o[1] * inv);
  ov.y = pack_bf16x2(o[2] * inv, o[3] * inv);
  *reinterpret_cast<uint2*>(a.out + b * a.o_sb + (kG * g + h) * a.o_sh + d0) = ov;
}

// Chunked form: one wave per (row, KV head) merges the row's chunk records.  Lane l owns query head l/32 and dims
// 4*(l%32)..+4.  The records of every chunk of the grid are loaded at once, before the row's context is known (the
// combine is one memory round trip); those of chunks past the row's end are stale and are never used.  Rows held by
// one chunk were written by the row kernel.
template <bool kAppend>
__global__ __launch_bounds__(64) void paged_decode_chunk_combine_kernel(const DecodeArgs a) {
  const int b = blockIdx.x;
  const int g = blockIdx.y;
  const int lane = threadIdx.x;
  const int h = lane >> 5;
  const int d0 = (lane & 31) * 4;
  const int nchg = a.max_splits;  // chunks per row in the grid, <= kChunkMax
  const float* base = a.ws + ((int64_t)b * nchg * a.hkv + g) * kRowRec;
  uint4 o[kChunkMax];
  float mr[kChunkMax], lr[kChunkMax];
#pragma unroll
  for (int u = 0; u < kChunkMax; ++u) {
    o[u] = make_uint4(0u, 0u, 0u, 0u);
    mr[u] = kMaxSeed;
    lr[u] = 0.f;
    if (u < nchg) {
      const float* r = base + (int64_t)u * a.hkv * kRowRec;
      o[u] = ld16(r + h * kD + d0);
      mr[u] = r[kG * kD + h];
      lr[u] = r[kG * kD + kG + h];
    }
  }
  const int ctx = row_ctx<kAppend>(a, b);
  const int nch = (ctx + a.split_tokens - 1) / a.split_tokens;
  if (nch <= 1) return;
  float M = kMaxSeed;
#pragma unroll
  for (int u = 0; u < kChunkMax; ++u)
    if (u < nch) M = fmaxf(M, mr[u]);
  float Ls = 0.f, x[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < kChunkMax; ++u) {
    if (u < nch) {
      const float wgt = fast_exp2(mr[u] - M);
      Ls += lr[u] * wgt;
      x[0] += __uint_as_float(o[u].x) * wgt;
      x[1] += __uint_as_float(o[u].y) * wgt;
      x[2] += __uint_as_float(o[u].z) * wgt;
      x[3] += __uint_as_float(o[u].w) * wgt;
    }
  }
  const float inv = Ls > 0.f ? 1.f / Ls : 0.f;
  uint2 ov;
  ov.x = pack_bf16x2(x[0] * inv, x[1] * inv);
  ov.y = pack_bf16x2(x[2] * inv, x[3] * inv);
  *reinterpret_cast<uint2*>(a.out + b * a.o_sb + (kG * g + h) * a.o_sh + d0) = ov;
}

// ------------------------------------------------------------------------------ host side
int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }
size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

int default_split(int batch, int hkv, int max_pages, int page_size) {
  const int64_t max_ctx = (int64_t)max_pages * page_size;
  int split = 64;
  (void)hkv;
  while (split > kTile && (int64_t)batch * ceil_div(max_ctx, split) < 1024) split /= 2;
  while (ceil_div(max_ctx, split) > kMaxSplits && split < kMaxSplitTokens) split *= 2;
  return split;
}

// Workgroups of the stream-K kernel the current device holds at once (cached per device).
// The workspace is sized for the larger of the two forms, so one buffer serves both.  Entries are atomics: two
// host threads may fill the same entry at once (both store the same value).
// form: 0 plain, 1 append, 2 append with the q/k norm and rope.
// Waves per KV head in a stream-K workgroup: two halves of the range for 8 KV heads (16 waves), else one.  Every form
// takes the same decomposition, so the append form stays bitwise equal to a scatter followed by the plain form, and
// the norm/rope form to the append form on normalised q/k.
int sk_halves(int hkv) { return hkv == 8 ? 2 : 1; }

int sk_grid_of(int hkv, int form) {
  static std::atomic<int> cache[64][17][3];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return kSkMaxGrid;
  std::atomic<int>& c = cache[dev][hkv][form];
  const int cached = c.load(std::memory_order_relaxed);
  if (cached > 0) return cached;
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return kSkMaxGrid;
  const int threads = 64 * hkv * sk_halves(hkv);
  hipError_t e;
  if (sk_halves(hkv) == 2)
    e = form == 2   ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, paged_decode_sk_kernel<true, true, 2>, threads, 0)
        : form == 1 ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, paged_decode_sk_kernel<true, false, 2>, threads, 0)
                    : hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, paged_decode_sk_kernel<false, false, 2>, threads, 0);
  else
    e = form == 2   ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, paged_decode_sk_kernel<true, true>, threads, 0)
        : form == 1 ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, paged_decode_sk_kernel<true>, threads, 0)
                    : hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, paged_decode_sk_kernel<false>, threads, 0);
  if (e != hipSuccess) return kSkMaxGrid;
  int g = cus * (per_cu > 0 ? per_cu : 1);
  g = g < 1 ? 1 : (g > kSkMaxGrid ? kSkMaxGrid : g);
  c.store(g, std::memory_order_relaxed);
  return g;
}

int sk_grid(int hkv) {
  const int g0 = sk_grid_of(hkv, 0), g1 = sk_grid_of(hkv, 1), g2 = hkv <= 8 ? sk_grid_of(hkv, 2) : 0;
  return std::max(g0, std::max(g1, g2));
}

// Host copy of sk_effective_grid for a tile-count bound (non-decreasing in the count).
int sk_effective_grid_host(int grid, int64_t nt) {
  const int64_t g = std::max<int64_t>(std::min<int64_t>(nt, 8), (nt + 3) / 4);
  return (int)std::max<int64_t>(1, std::min<int64_t>(grid, g));
}

// The decompositions of one decode call.  split_tokens == 0 lets choose_path pick; Q3A_DECODE_ROW,
// Q3A_DECODE_CHUNKS and Q3A_DECODE_STREAMK (negative codes) ask for one; split_tokens > 0 is the fixed split.
enum class Path { kNone, kRow, kChunks, kStreamK, kFixed };

// Chunked form geometry for a table of cap_tiles tiles: W waves of `per` tiles per chunk, nch chunks per row.
// 128-token chunks (8 waves of one tile) while 16 of them cover the table, then 16 waves of one tile, then 8
// waves of several tiles (two in flight).  False past 64 tiles per wave.
bool chunk_geometry(int64_t cap_tiles, int* W, int* per, int* nch) {
  int w = 8, p = 1;
  if (cap_tiles > (int64_t)kChunkMax * 8) {
    if (cap_tiles <= (int64_t)kChunkMax * 16) {
      w = 16;
    } else {
      p = (int)((cap_tiles + kChunkMax * 8 - 1) / (kChunkMax * 8));
      if (p > 64) return false;
    }
  }
  *W = w;
  *per = p;
  *nch = (int)((cap_tiles + (int64_t)w * p - 1) / ((int64_t)w * p));
  return true;
}

// Batches up to which long rows take the chunked form, and the table capacity (tiles) from which they do.
constexpr int kChunkMaxBatch = 16;
constexpr int kChunkMinTiles = 2 * kMaxRowTiles;

Path choose_path(int batch, int64_t max_ctx, int split_tokens) {
  const int64_t cap_tiles = (max_ctx + kTile - 1) / kTile;
  const bool row_ok = cap_tiles <= kRowMaxWaves * kRowMaxPer;
  int w, p, n;
  const bool chunk_ok = chunk_geometry(cap_tiles, &w, &p, &n);
  switch (split_tokens) {
    case Q3A_DECODE_ROW: return row_ok ? Path::kRow : Path::kNone;
    case Q3A_DECODE_CHUNKS: return chunk_ok ? Path::kChunks : Path::kNone;
    case Q3A_DECODE_STREAMK:
    case Q3A_DECODE_PLANNED: return batch <= kSkMaxRows ? Path::kStreamK : Path::kNone;
    case 0: break;
    default: return split_tokens > 0 ? Path::kFixed : Path::kNone;
  }
  // Narrow tables: one launch.  Small batches of long rows: chunks over many CUs.  Up to 64 rows: the row-parallel
  // kernel.  Beyond: stream-K, and past its row limit the fixed split.
  if (cap_tiles <= kMaxRowTiles) return Path::kRow;
  if (batch <= kChunkMaxBatch && cap_tiles >= kChunkMinTiles && chunk_ok) return Path::kChunks;
  if (batch <= kRowMaxBatch && row_ok) return Path::kRow;
  if (batch <= kSkMaxRows) return Path::kStreamK;
  return Path::kFixed;
}

size_t workspace_bytes(int batch, int hkv, int max_pages, int page_size, int split_tokens) {
  const int64_t max_ctx = (int64_t)max_pages * page_size;
  switch (choose_path(batch, max_ctx, split_tokens)) {
    case Path::kNone:
    case Path::kRow: return 0;
    case Path::kChunks: {
      int w, p, n;
      chunk_geometry((max_ctx + kTile - 1) / kTile, &w, &p, &n);
      return n <= 1 ? 0 : (size_t)batch * n * hkv * kRowRec * sizeof(float);
    }
    case Path::kStreamK:
      return align256((size_t)(batch + 1) * sizeof(int)) + align256((size_t)batch * sizeof(int)) +
             (size_t)sk_grid(hkv) * kSkSlots * hkv * kPartFloats * sizeof(float);
    case Path::kFixed: break;
  }
  if (split_tokens <= 0) split_tokens = default_split(batch, hkv, max_pages, page_size);
  const int max_splits = ceil_div(max_ctx, split_tokens);
  if (max_splits <= 1) return 0;
  return (size_t)batch * max_splits * hkv * kPartFloats * sizeof(float);
}

// Planned stream-K calls.  A plan holds the call's scratch (the new tokens' slot pages, the partial records: two
// leading slots per possible cut row and as many overflow slots) and the plan proper: the decode workgroups' ranges
// and record positions, the cut-row descriptors, each wave's first tile list, and entries for the tiles past them.
// At most grid - 1 rows are cut (each crosses a range boundary), and the records number at most 2 per workgroup.
struct PlanLayout {
  int grid;
  size_t slot_off, rec_off, wg_off, cut_off, claim_off, first_off, tiles_off, bytes;
};

PlanLayout plan_layout(int batch, int hkv, int max_pages, int page_size) {
  const int64_t cap_tiles = ((int64_t)max_pages * page_size + kTile - 1) / kTile;
  PlanLayout L;
  L.grid = sk_effective_grid_host(sk_grid(hkv), (int64_t)batch * cap_tiles);
  L.slot_off = 0;
  L.rec_off = L.slot_off + align256((size_t)batch * sizeof(int));
  L.wg_off = L.rec_off + align256((size_t)4 * L.grid * hkv * kPartFloats * sizeof(float));
  L.cut_off = L.wg_off + align256((size_t)L.grid * kPlanWgInts * sizeof(int));
  L.claim_off = L.cut_off + align256((size_t)L.grid * sizeof(int4));
  L.first_off = L.claim_off + align256((size_t)L.grid * sizeof(int));
  L.tiles_off = L.first_off + align256((size_t)L.grid * sk_halves(hkv) * 64 * sizeof(int2));
  L.bytes = L.tiles_off + align256((size_t)batch * cap_tiles * sizeof(int2));
  return L;
}

// What each plan was built for, keyed by its address: a planned call is checked against it on the host, so a plan
// built for other lengths' pointer, table, shape or form is refused instead of read.
struct PlanInfo {
  int dev, batch, hkv, form, grid, max_pages, page_size;
  const int32_t* seqlens;
  const int32_t* bt;
  int64_t bt_sb;
  size_t bytes;
};
std::mutex g_plan_mu;
std::unordered_map<const void*, PlanInfo> g_plans;

bool find_plan(const void* plan, PlanInfo* out) {
  std::lock_guard<std::mutex> lk(g_plan_mu);
  const auto it = g_plans.find(plan);
  if (it == g_plans.end()) return false;
  *out = it->second;
  return true;
}

}  // namespace
}  // namespace q3a

using namespace q3a;

extern "C" size_t q3a_paged_decode_plan_bytes(int batch, int num_kv_heads, int max_pages_per_seq, int page_size) {
  if (batch <= 0 || batch > kSkMaxRows || num_kv_heads != 8 || max_pages_per_seq <= 0 || page_size <= 0 ||
      page_size % kTile != 0 || page_size > (kTile << kPlanOffBits) ||
      (int64_t)max_pages_per_seq * page_size > ((int64_t)1 << 30))
    return 0;
  // Plans serve the shapes for which the library itself chooses stream-K (small batches take one-launch kernels).
  if (choose_path(batch, (int64_t)max_pages_per_seq * page_size, 0) != Path::kStreamK) return 0;
  return plan_layout(batch, num_kv_heads, max_pages_per_seq, page_size).bytes;
}

extern "C" int q3a_paged_decode_plan(const int32_t* cache_seqlens, const int32_t* block_table, int64_t bt_stride_b,
                                     int64_t bt_stride_table, int num_tables, int max_pages_per_seq, int page_size,
                                     int batch, int num_kv_heads, int form, void* plans, int64_t plan_stride,
                                     size_t plans_bytes, void* stream) {
  const char* who = "paged_decode_plan";
  const size_t need = q3a_paged_decode_plan_bytes(batch, num_kv_heads, max_pages_per_seq, page_size);
  if (need == 0)
    return fail(Q3A_EINVAL,
                "%s: no plan for batch %d, %d KV heads, %d pages of %d tokens (need a shape the library decodes "
                "with stream-K, 1 <= batch <= %d, 8 KV heads, page_size a multiple of %d up to %d)",
                who, batch, num_kv_heads, max_pages_per_seq, page_size, kSkMaxRows, kTile, kTile << kPlanOffBits);
  if (form < Q3A_PLAN_PLAIN || form > Q3A_PLAN_APPEND_ROPE) return fail(Q3A_EINVAL, "%s: form %d unknown", who, form);
  if (!cache_seqlens || !block_table || !plans) return fail(Q3A_EINVAL, "%s: null pointer argument", who);
  if (num_tables < 1 || num_tables > 65535) return fail(Q3A_EINVAL, "%s: num_tables %d outside [1, 65535]", who, num_tables);
  if (bt_stride_b < max_pages_per_seq || (num_tables > 1 && bt_stride_table < (int64_t)batch * bt_stride_b))
    return fail(Q3A_EINVAL, "%s: table strides %lld / %lld overlap", who, (long long)bt_stride_b,
                (long long)bt_stride_table);
  if ((uintptr_t)plans % 256 != 0 || plan_stride % 256 != 0 || (num_tables > 1 && plan_stride < (int64_t)need))
    return fail(Q3A_EINVAL, "%s: plans must be 256-byte aligned with a 256-byte multiple stride >= %zu", who, need);
  if (plans_bytes < (size_t)(num_tables - 1) * (size_t)plan_stride + need)
    return fail(Q3A_ESPACE, "%s: %zu bytes < %zu needed", who, plans_bytes,
                (size_t)(num_tables - 1) * (size_t)plan_stride + need);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(Q3A_ELAUNCH, "%s: no current device", who);
  const PlanLayout L = plan_layout(batch, num_kv_heads, max_pages_per_seq, page_size);
  const int64_t cap_tiles = ((int64_t)max_pages_per_seq * page_size + kTile - 1) / kTile;
  DecodeArgs a{};
  a.seqlens = cache_seqlens;
  a.bt = block_table;
  a.bt_sb = bt_stride_b;
  a.max_pages = max_pages_per_seq;
  a.page_size = page_size;
  a.batch = batch;
  a.hkv = num_kv_heads;
  // The grid the decode kernel of this form launches with (the same rule as launch_decode).
  a.grid = sk_effective_grid_host(sk_grid_of(num_kv_heads, form), (int64_t)batch * cap_tiles);
  PlanArgs p;
  p.plans = static_cast<char*>(plans);
  p.plan_stride = plan_stride;
  p.bt_stable = bt_stride_table;
  p.wg_off = (int64_t)L.wg_off;
  p.cut_off = (int64_t)L.cut_off;
  p.first_off = (int64_t)L.first_off;
  p.tiles_off = (int64_t)L.tiles_off;
  p.claim_off = (int64_t)L.claim_off;
  p.num_tables = num_tables;
  p.halves = sk_halves(num_kv_heads);
  p.rec_cap = L.grid;
  // One thread per tile of the table capacity (at most 64 workgroups; each scans the rows itself).
  // Workgroups of 256 threads, one thread per tile of the table capacity, at most 256 of them (each scans the rows
  // itself): the page-id loads of every table spread over that many CUs (with 28 tables of 576 rows they read 8 MB of
  // table lines, which a few CUs pull far more slowly).
  const int64_t work = std::max<int64_t>((int64_t)batch * cap_tiles, (int64_t)batch + L.grid);
  const int gx = (int)std::min<int64_t>(256, std::max<int64_t>(1, (work + 255) / 256));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (form == Q3A_PLAN_PLAIN)
    hipLaunchKernelGGL(paged_decode_plan_kernel<false>, dim3(gx), dim3(256), 0, st, a, p);
  else
    hipLaunchKernelGGL(paged_decode_plan_kernel<true>, dim3(gx), dim3(256), 0, st, a, p);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(Q3A_ELAUNCH, "%s: launch failed: %s", who, hipGetErrorString(e));
  std::lock_guard<std::mutex> lk(g_plan_mu);
  for (int t = 0; t < num_tables; ++t) {
    const void* key = static_cast<char*>(plans) + (int64_t)t * plan_stride;
    g_plans[key] = PlanInfo{dev, batch, num_kv_heads, form, a.grid, max_pages_per_seq, page_size, cache_seqlens,
                            block_table + (int64_t)t * bt_stride_table, bt_stride_b, need};
  }
  return Q3A_OK;
}

extern "C" int q3a_paged_decode_default_split(int batch, int num_kv_heads, int max_pages_per_seq,
                                              int page_size) {
  if (batch <= 0 || num_kv_heads <= 0 || max_pages_per_seq <= 0 || page_size <= 0) return kTile;
  return default_split(batch, num_kv_heads, max_pages_per_seq, page_size);
}

extern "C" size_t q3a_paged_decode_workspace_bytes(int batch, int num_q_heads, int num_kv_heads,
                                                   int head_dim, int max_pages_per_seq,
                                                   int page_size, int split_tokens) {
  (void)num_q_heads;
  (void)head_dim;
  if (batch <= 0 || num_kv_heads <= 0 || num_kv_heads > 16 || max_pages_per_seq <= 0 || page_size <= 0)
    return 0;
  return workspace_bytes(batch, num_kv_heads, max_pages_per_seq, page_size, split_tokens);
}

// The norm/rope form's extra inputs (q3a_paged_decode_append_rope).
struct NormRope {
  const void* q_norm_w;
  const void* k_norm_w;
  const void* cos;
  const void* sin;
  int64_t cs_stride_b;
  float eps;
};

static int launch_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k_new,
                         int64_t kn_stride_b, const void* v_new, int64_t vn_stride_b, const void* k_cache,
                         const void* v_cache, int64_t kv_stride_page, int64_t kv_stride_tok, int64_t kv_stride_head,
                         int num_pages, int page_size, const int32_t* cache_seqlens, const int32_t* block_table,
                         int64_t bt_stride_b, int max_pages_per_seq, void* out, int64_t o_stride_b,
                         int64_t o_stride_h, void* workspace, size_t workspace_bytes_, int batch, int num_q_heads,
                         int num_kv_heads, int head_dim, float softmax_scale, int split_tokens, void* stream,
                         const char* who, const NormRope* nr = nullptr) {
  const bool append = k_new != nullptr;
  if (batch < 0) return fail(Q3A_EINVAL, "%s: batch %d < 0", who, batch);
  if (batch == 0) return Q3A_OK;
  if (head_dim != kD) return fail(Q3A_EINVAL, "%s: head_dim %d unsupported (need %d)", who, head_dim, kD);
  if (num_kv_heads < 1 || num_kv_heads > 16)
    return fail(Q3A_EINVAL, "%s: num_kv_heads %d outside [1, 16]", who, num_kv_heads);
  if (num_q_heads != kG * num_kv_heads)
    return fail(Q3A_EINVAL, "%s: num_q_heads %d != %d * num_kv_heads %d", who, num_q_heads, kG, num_kv_heads);
  if (page_size <= 0 || page_size % kTile != 0)
    return fail(Q3A_EINVAL, "%s: page_size %d is not a positive multiple of %d", who, page_size, kTile);
  if (num_pages <= 0 || max_pages_per_seq <= 0)
    return fail(Q3A_EINVAL, "%s: num_pages %d / max_pages_per_seq %d must be > 0", who, num_pages, max_pages_per_seq);
  if (!q || !k_cache || !v_cache || !cache_seqlens || !block_table || !out)
    return fail(Q3A_EINVAL, "%s: null pointer argument", who);
  const uintptr_t align = (uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)out |
                          (uintptr_t)k_new | (uintptr_t)v_new;
  if (align % 16 != 0) return fail(Q3A_EINVAL, "%s: q/k_cache/v_cache/out/k_new/v_new must be 16-byte aligned", who);
  if ((q_stride_b | q_stride_h | kv_stride_page | kv_stride_tok | kv_stride_head | o_stride_b | o_stride_h |
       kn_stride_b | vn_stride_b) % 8 != 0)
    return fail(Q3A_EINVAL, "%s: strides must be multiples of 8 elements (16 bytes)", who);
  // q's two head rows of a KV group are read through one buffer descriptor with a 32-bit extent.
  if (q_stride_h <= 0 || ((int64_t)(kG - 1) * q_stride_h + head_dim) * 2 >= ((int64_t)1 << 31))
    return fail(Q3A_EINVAL, "%s: q head stride %lld unsupported (need > 0, head pair extent < 2 GiB)", who,
                (long long)q_stride_h);
  const bool planned = split_tokens == Q3A_DECODE_PLANNED;
  const bool path_code = split_tokens == Q3A_DECODE_ROW || split_tokens == Q3A_DECODE_CHUNKS ||
                         split_tokens == Q3A_DECODE_STREAMK || planned;
  if (!path_code && (split_tokens < 0 || split_tokens % kTile != 0))
    return fail(Q3A_EINVAL, "%s: split_tokens %d is not 0, a path code or a positive multiple of %d", who,
                split_tokens, kTile);
  if (split_tokens > kMaxSplitTokens)
    return fail(Q3A_EINVAL, "%s: split_tokens %d exceeds %d", who, split_tokens, kMaxSplitTokens);
  const int64_t page_extent =
      ((int64_t)(page_size - 1) * kv_stride_tok + (int64_t)(num_kv_heads - 1) * kv_stride_head + head_dim) * 2;
  if (kv_stride_tok <= 0 || kv_stride_head <= 0 || page_extent >= ((int64_t)1 << 31))
    return fail(Q3A_EINVAL, "%s: page extent %lld bytes unsupported (need positive strides, < 2 GiB)", who,
                (long long)page_extent);
  const int64_t max_ctx = (int64_t)max_pages_per_seq * page_size;
  if (max_ctx > (int64_t)1 << 30) return fail(Q3A_EINVAL, "%s: context capacity too large", who);
  const int workspace_split = split_tokens;  // the value the caller sized the workspace with
  const Path path = choose_path(batch, max_ctx, split_tokens);
  if (path == Path::kNone)
    return fail(Q3A_EINVAL, "%s: decode path %d does not take this shape (batch %d, table of %lld tokens)", who,
                split_tokens, batch, (long long)max_ctx);
  // Narrow tables and small batches: one workgroup per (row, KV head) streams the row with up to 16 waves and
  // writes its output, one kernel and no partial records.  Stream-K would cut such rows into short pieces and merge
  // them in a second kernel, whose launch is most of such a call.  Small batches of long rows: the same kernel over
  // chunks of the row, so the row's tiles spread over many CUs, and a combine.
  const bool row = path == Path::kRow;
  const bool chunks = path == Path::kChunks;
  const int cap_tiles = (int)((max_ctx + kTile - 1) / kTile);
  int row_waves = std::min(cap_tiles, row_max_waves(cap_tiles > kRowMaxWaves)), chunk_per = 1, nchunks = 1;
  if (chunks) chunk_geometry(cap_tiles, &row_waves, &chunk_per, &nchunks);
  if (row) split_tokens = cap_tiles * kTile;
  if (chunks) split_tokens = row_waves * chunk_per * kTile;
  const bool sk = path == Path::kStreamK;
  if (sk) split_tokens = 0;
  if (path == Path::kFixed && split_tokens == 0)
    split_tokens = default_split(batch, num_kv_heads, max_pages_per_seq, page_size);
  const int max_splits = sk ? 0 : (chunks ? nchunks : ceil_div(max_ctx, split_tokens));
  if (path == Path::kFixed && max_splits > kMaxSplits)
    return fail(Q3A_EINVAL, "%s: %d splits exceed %d (raise split_tokens)", who, max_splits, kMaxSplits);
  PlanInfo plan{};
  if (planned) {
    // The workspace is a plan: it must have been built (q3a_paged_decode_plan) for this call's lengths, table,
    // shape and form on this device.
    int dev = -1;
    (void)hipGetDevice(&dev);
    const int form = nr != nullptr ? Q3A_PLAN_APPEND_ROPE : (append ? Q3A_PLAN_APPEND : Q3A_PLAN_PLAIN);
    if (workspace == nullptr || !find_plan(workspace, &plan))
      return fail(Q3A_EINVAL, "%s: the workspace is not a decode plan (build it with q3a_paged_decode_plan)", who);
    if (plan.dev != dev || plan.batch != batch || plan.hkv != num_kv_heads || plan.form != form ||
        plan.max_pages != max_pages_per_seq || plan.page_size != page_size || plan.seqlens != cache_seqlens ||
        plan.bt != block_table || plan.bt_sb != bt_stride_b)
      return fail(Q3A_EINVAL,
                  "%s: the plan was built for another call (device %d, batch %d, %d KV heads, form %d, %d pages of %d "
                  "tokens, other cache_seqlens or block table)",
                  who, plan.dev, plan.batch, plan.hkv, plan.form, plan.max_pages, plan.page_size);
    if (workspace_bytes_ < plan.bytes)
      return fail(Q3A_ESPACE, "%s: plan buffer %zu bytes < %zu", who, workspace_bytes_, plan.bytes);
  } else {
    const size_t need = workspace_bytes(batch, num_kv_heads, max_pages_per_seq, page_size, workspace_split);
    if (need > 0 && (workspace == nullptr || workspace_bytes_ < need))
      return fail(Q3A_ESPACE, "%s: workspace %zu bytes < %zu needed", who, workspace_bytes_, need);
    if (need > 0 && (uintptr_t)workspace % 16 != 0)
      return fail(Q3A_EINVAL, "%s: workspace must be 16-byte aligned", who);
  }
  if (nr != nullptr) {
    if (!append) return fail(Q3A_EINVAL, "%s: the norm/rope form needs k_new/v_new", who);
    if (!row && !sk && !chunks)
      return fail(Q3A_EINVAL, "%s: the norm/rope form needs split_tokens <= 0 and batch <= %d", who, kSkMaxRows);
    if (sk && num_kv_heads > 8)
      return fail(Q3A_EINVAL, "%s: the norm/rope form supports at most 8 KV heads (got %d)", who, num_kv_heads);
    if (!nr->q_norm_w || !nr->k_norm_w || !nr->cos || !nr->sin)
      return fail(Q3A_EINVAL, "%s: null norm weight or cos/sin pointer", who);
    if (((uintptr_t)nr->q_norm_w | (uintptr_t)nr->k_norm_w | (uintptr_t)nr->cos | (uintptr_t)nr->sin) % 16 != 0 ||
        nr->cs_stride_b % 8 != 0 || nr->cs_stride_b < 0)
      return fail(Q3A_EINVAL, "%s: norm weights and cos/sin rows must be 16-byte aligned (row stride %lld)", who,
                  (long long)nr->cs_stride_b);
    if (!(nr->eps >= 0.f) || nr->eps > 1.f) return fail(Q3A_EINVAL, "%s: eps %g outside [0, 1]", who, (double)nr->eps);
  }

  DecodeArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_sb = q_stride_b;
  a.q_sh = q_stride_h;
  a.kc = static_cast<const uint16_t*>(k_cache);
  a.vc = static_cast<const uint16_t*>(v_cache);
  a.kv_sp = kv_stride_page;
  a.kv_st = kv_stride_tok;
  a.kv_sh = kv_stride_head;
  a.k_new = static_cast<const uint16_t*>(k_new);
  a.v_new = static_cast<const uint16_t*>(v_new);
  a.kn_sb = kn_stride_b;
  a.vn_sb = vn_stride_b;
  a.num_pages = num_pages;
  a.page_size = page_size;
  a.page_bytes = (uint32_t)page_extent;
  a.seqlens = cache_seqlens;
  a.bt = block_table;
  a.bt_sb = bt_stride_b;
  a.max_pages = max_pages_per_seq;
  a.out = static_cast<uint16_t*>(out);
  a.o_sb = o_stride_b;
  a.o_sh = o_stride_h;
  a.batch = batch;
  a.hkv = num_kv_heads;
  a.split_tokens = split_tokens;
  a.max_splits = max_splits;
  a.row_per = 0;
  a.scale_log2 = softmax_scale * kLog2e;
  const bool rope = nr != nullptr;
  a.qn_w = rope ? static_cast<const uint16_t*>(nr->q_norm_w) : nullptr;
  a.kn_w = rope ? static_cast<const uint16_t*>(nr->k_norm_w) : nullptr;
  a.rcos = rope ? static_cast<const uint16_t*>(nr->cos) : nullptr;
  a.rsin = rope ? static_cast<const uint16_t*>(nr->sin) : nullptr;
  a.rs_sb = rope ? nr->cs_stride_b : 0;
  a.eps = rope ? nr->eps : 0.f;

  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 block(64 * num_kv_heads);
  hipError_t e;
  if (sk) {
    // Launch no more workgroups than the call can use: the tile count is at most rows x table capacity, and the
    // workgroups past sk_effective_grid of the actual count exit after the prologue (every workgroup computes the
    // same effective grid from a.grid, so bounding a.grid here changes no range when the bound holds).
    const int64_t nt_bound = (int64_t)batch * ceil_div(max_ctx, kTile);
    a.grid = sk_grid_of(num_kv_heads, rope ? 2 : (append ? 1 : 0));
    a.grid = sk_effective_grid_host(a.grid, nt_bound);
    a.prefix = static_cast<int*>(workspace);
    const size_t pb = align256((size_t)(batch + 1) * sizeof(int));
    a.slot_page = reinterpret_cast<int*>(static_cast<char*>(workspace) + pb);
    a.ws = reinterpret_cast<float*>(static_cast<char*>(workspace) + pb + align256((size_t)batch * sizeof(int)));
    a.plan_wg = nullptr;
    a.plan_first = nullptr;
    a.plan_tiles = nullptr;
    a.plan_cut = nullptr;
    a.plan_rec_cap = 0;
    a.plan_claim = nullptr;
    if (planned) {
      if (sk_halves(num_kv_heads) != 2 || a.grid != plan.grid)
        return fail(Q3A_EINVAL, "%s: plan grid %d does not match this device's %d", who, plan.grid, a.grid);
      const PlanLayout PL = plan_layout(batch, num_kv_heads, max_pages_per_seq, page_size);
      char* const wsb = static_cast<char*>(workspace);
      a.prefix = nullptr;
      a.slot_page = reinterpret_cast<int*>(wsb + PL.slot_off);
      a.ws = reinterpret_cast<float*>(wsb + PL.rec_off);
      a.plan_wg = reinterpret_cast<const int*>(wsb + PL.wg_off);
      a.plan_cut = reinterpret_cast<const int4*>(wsb + PL.cut_off);
      a.plan_first = reinterpret_cast<const int2*>(wsb + PL.first_off);
      a.plan_tiles = reinterpret_cast<const int2*>(wsb + PL.tiles_off);
      a.plan_rec_cap = PL.grid;
      a.plan_claim = reinterpret_cast<int*>(wsb + PL.claim_off);
      const dim3 block2(2 * 64 * num_kv_heads);
      if (rope)
        hipLaunchKernelGGL((paged_decode_sk_kernel<true, true, 2, true>), dim3(a.grid), block2, 0, st, a);
      else if (append)
        hipLaunchKernelGGL((paged_decode_sk_kernel<true, false, 2, true>), dim3(a.grid), block2, 0, st, a);
      else
        hipLaunchKernelGGL((paged_decode_sk_kernel<false, false, 2, true>), dim3(a.grid), block2, 0, st, a);
      e = hipGetLastError();
      if (e != hipSuccess) return fail(Q3A_ELAUNCH, "%s: planned launch failed: %s", who, hipGetErrorString(e));
      const dim3 cgrid((batch + kPlanRowsPerWg - 1) / kPlanRowsPerWg + PL.grid);
      if (rope)
        hipLaunchKernelGGL((paged_decode_plan_combine_kernel<true, true>), cgrid, block, 0, st, a);
      else if (append)
        hipLaunchKernelGGL(paged_decode_plan_combine_kernel<true>, cgrid, block, 0, st, a);
      else
        hipLaunchKernelGGL(paged_decode_plan_combine_kernel<false>, cgrid, block, 0, st, a);
      e = hipGetLastError();
      if (e != hipSuccess) return fail(Q3A_ELAUNCH, "%s: planned combine launch failed: %s", who, hipGetErrorString(e));
      return Q3A_OK;
    } else if (sk_halves(num_kv_heads) == 2) {
      const dim3 block2(2 * 64 * num_kv_heads);
      if (rope)
        hipLaunchKernelGGL((paged_decode_sk_kernel<true, true, 2>), dim3(a.grid), block2, 0, st, a);
      else if (append)
        hipLaunchKernelGGL((paged_decode_sk_kernel<true, false, 2>), dim3(a.grid), block2, 0, st, a);
      else
        hipLaunchKernelGGL((paged_decode_sk_kernel<false, false, 2>), dim3(a.grid), block2, 0, st, a);
    } else {
      if (rope)
        hipLaunchKernelGGL((paged_decode_sk_kernel<true, true>), dim3(a.grid), block, 0, st, a);
      else if (append)
        hipLaunchKernelGGL(paged_decode_sk_kernel<true>, dim3(a.grid), block, 0, st, a);
      else
        hipLaunchKernelGGL(paged_decode_sk_kernel<false>, dim3(a.grid), block, 0, st, a);
    }
    e = hipGetLastError();
    if (e != hipSuccess) return fail(Q3A_ELAUNCH, "%s: stream-K launch failed: %s", who, hipGetErrorString(e));
    if (rope)
      hipLaunchKernelGGL((paged_decode_sk_combine_kernel<true, true>), dim3(batch), block, 0, st, a);
    else if (append)
      hipLaunchKernelGGL(paged_decode_sk_combine_kernel<true>, dim3(batch), block, 0, st, a);
    else
      hipLaunchKernelGGL(paged_decode_sk_combine_kernel<false>, dim3(batch), block, 0, st, a);
    e = hipGetLastError();
    if (e != hipSuccess) return fail(Q3A_ELAUNCH, "%s: combine launch failed: %s", who, hipGetErrorString(e));
    return Q3A_OK;
  }
  a.grid = 0;
  a.prefix = nullptr;
  a.ws = static_cast<float*>(workspace);
  if (row || chunks) {
    a.row_per = chunks ? chunk_per : (cap_tiles + row_waves - 1) / row_waves;
    const dim3 rgrid(batch, num_kv_heads, chunks ? nchunks : 1), rblock(64 * row_waves);
    if (a.row_per == 1) {
      if (rope)
        hipLaunchKernelGGL((paged_decode_row_kernel<true, false, true>), rgrid, rblock, 0, st, a);
      else if (append)
        hipLaunchKernelGGL((paged_decode_row_kernel<true, false>), rgrid, rblock, 0, st, a);
      else
        hipLaunchKernelGGL((paged_decode_row_kernel<false, false>), rgrid, rblock, 0, st, a);
    } else {
      if (rope)
        hipLaunchKernelGGL((paged_decode_row_kernel<true, true, true>), rgrid, rblock, 0, st, a);
      else if (append)
        hipLaunchKernelGGL((paged_decode_row_kernel<true, true>), rgrid, rblock, 0, st, a);
      else
        hipLaunchKernelGGL((paged_decode_row_kernel<false, true>), rgrid, rblock, 0, st, a);
    }
    e = hipGetLastError();
    if (e != hipSuccess) return fail(Q3A_ELAUNCH, "%s: row launch failed: %s", who, hipGetErrorString(e));
    if (chunks && nchunks > 1) {
      if (append)
        hipLaunchKernelGGL(paged_decode_chunk_combine_kernel<true>, dim3(batch, num_kv_heads), dim3(64), 0, st, a);
      else
        hipLaunchKernelGGL(paged_decode_chunk_combine_kernel<false>, dim3(batch, num_kv_heads), dim3(64), 0, st, a);
      e = hipGetLastError();
      if (e != hipSuccess) return fail(Q3A_ELAUNCH, "%s: chunk combine launch failed: %s", who, hipGetErrorString(e));
    }
    return Q3A_OK;
  }
  if (append)
    hipLaunchKernelGGL(paged_decode_split_kernel<true>, dim3(batch, max_splits), block, 0, st, a);
  else
    hipLaunchKernelGGL(paged_decode_split_kernel<false>, dim3(batch, max_splits), block, 0, st, a);
  e = hipGetLastError();
  if (e != hipSuccess) return fail(Q3A_ELAUNCH, "%s: split launch failed: %s", who, hipGetErrorString(e));
  if (max_splits > 1) {
    if (append)
      hipLaunchKernelGGL(paged_decode_split_combine_kernel<true>, dim3(batch), block, 0, st, a);
    else
      hipLaunchKernelGGL(paged_decode_split_combine_kernel<false>, dim3(batch), block, 0, st, a);
    e = hipGetLastError();
    if (e != hipSuccess) return fail(Q3A_ELAUNCH, "%s: combine launch failed: %s", who, hipGetErrorString(e));
  }
  return Q3A_OK;
}

extern "C" int q3a_paged_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                const void* k_cache, const void* v_cache, int64_t kv_stride_page,
                                int64_t kv_stride_tok, int64_t kv_stride_head, int num_pages,
                                int page_size, const int32_t* cache_seqlens,
                                const int32_t* block_table, int64_t bt_stride_b,
                                int max_pages_per_seq, void* out, int64_t o_stride_b,
                                int64_t o_stride_h, void* workspace, size_t workspace_bytes_,
                                int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                float softmax_scale, int split_tokens, void* stream) {
  return launch_decode(q, q_stride_b, q_stride_h, nullptr, 0, nullptr, 0, k_cache, v_cache, kv_stride_page,
                       kv_stride_tok, kv_stride_head, num_pages, page_size, cache_seqlens, block_table, bt_stride_b,
                       max_pages_per_seq, out, o_stride_b, o_stride_h, workspace, workspace_bytes_, batch,
                       num_q_heads, num_kv_heads, head_dim, softmax_scale, split_tokens, stream, "paged_decode");
}

extern "C" int q3a_paged_decode_append(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                       const void* k_new, int64_t kn_stride_b, const void* v_new,
                                       int64_t vn_stride_b, void* k_cache, void* v_cache,
                                       int64_t kv_stride_page, int64_t kv_stride_tok, int64_t kv_stride_head,
                                       int num_pages, int page_size, const int32_t* cache_seqlens,
                                       const int32_t* block_table, int64_t bt_stride_b, int max_pages_per_seq,
                                       void* out, int64_t o_stride_b, int64_t o_stride_h, void* workspace,
                                       size_t workspace_bytes_, int batch, int num_q_heads, int num_kv_heads,
                                       int head_dim, float softmax_scale, int split_tokens, void* stream) {
  if (!k_new || !v_new) return fail(Q3A_EINVAL, "paged_decode_append: null k_new/v_new");
  return launch_decode(q, q_stride_b, q_stride_h, k_new, kn_stride_b, v_new, vn_stride_b, k_cache, v_cache,
                       kv_stride_page, kv_stride_tok, kv_stride_head, num_pages, page_size, cache_seqlens,
                       block_table, bt_stride_b, max_pages_per_seq, out, o_stride_b, o_stride_h, workspace,
                       workspace_bytes_, batch, num_q_heads, num_kv_heads, head_dim, softmax_scale, split_tokens,
                       stream, "paged_decode_append");
}

extern "C" int q3a_paged_decode_append_rope(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k_new, int64_t kn_stride_b, const void* v_new,
    int64_t vn_stride_b, const void* q_norm_w, const void* k_norm_w, const void* cos, const void* sin,
    int64_t cs_stride_b, float eps, void* k_cache, void* v_cache, int64_t kv_stride_page, int64_t kv_stride_tok,
    int64_t kv_stride_head, int num_pages, int page_size, const int32_t* cache_seqlens, const int32_t* block_table,
    int64_t bt_stride_b, int max_pages_per_seq, void* out, int64_t o_stride_b, int64_t o_stride_h, void* workspace,
    size_t workspace_bytes_, int batch, int num_q_heads, int num_kv_heads, int head_dim, float softmax_scale,
    int split_tokens, void* stream) {
  if (!k_new || !v_new) return fail(Q3A_EINVAL, "paged_decode_append_rope: null k_new/v_new");
  const NormRope nr{q_norm_w, k_norm_w, cos, sin, cs_stride_b, eps};
  return launch_decode(q, q_stride_b, q_stride_h, k_new, kn_stride_b, v_new, vn_stride_b, k_cache, v_cache,
                       kv_stride_page, kv_stride_tok, kv_stride_head, num_pages, page_size, cache_seqlens,
                       block_table, bt_stride_b, max_pages_per_seq, out, o_stride_b, o_stride_h, workspace,
                       workspace_bytes_, batch, num_q_heads, num_kv_heads, head_dim, softmax_scale, split_tokens,
                       stream, "paged_decode_append_rope", &nr);
}

// ------------------------------------------------------------------------------ allocation-free entry point
// For callers that cannot allocate device memory (code under graph capture, tight serving loops, harnesses that
// forbid it): q3a_paged_decode with the workspace taken from this file-scope array instead of the caller.  Each GPU
// the library runs on holds its own copy (kNoAllocScratchBytes) until the process ends.  Its device address comes from
// hipGetSymbolAddress, fetched once per device with that device current; host code never uses the array's name
// as an address.  No byte of it needs to start at zero: the combine kernel reads only what the same call's decode
// kernel wrote (tile prefix sums, partial records).  Every call on one GPU shares the array, so calls that overlap on
// one GPU (two streams at once) race; calls on one stream are ordered and safe.
namespace q3a {
namespace {
constexpr size_t kNoAllocScratchBytes = (size_t)8 << 20;
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];

// The scratch array's device address on the current device (nullptr and a message on failure).
void* scratch_address(const char* who) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    fail(Q3A_ELAUNCH, "%s: no current HIP device (or device index >= %d)", who, kMaxDevices);
    return nullptr;
  }
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p != nullptr) return p;
  void* q = nullptr;
  const hipError_t e = hipGetSymbolAddress(&q, HIP_SYMBOL(scratch));
  if (e != hipSuccess || q == nullptr) {
    fail(Q3A_ELAUNCH, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", who, dev, hipGetErrorString(e));
    return nullptr;
  }
  // Two threads may both look the address up; they store the same value.
  g_scratch_ptr[dev].store(q, std::memory_order_release);
  return q;
}
}  // namespace
}  // namespace q3a

extern "C" int q3a_paged_decode_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k_cache,
                                        const void* v_cache, int64_t kv_stride_page, int64_t kv_stride_tok,
                                        int64_t kv_stride_head, int num_pages, int page_size,
                                        const int32_t* cache_seqlens, const int32_t* block_table, int64_t bt_stride_b,
                                        int max_pages_per_seq, void* out, int64_t o_stride_b, int64_t o_stride_h,
                                        int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                        float softmax_scale, int split_tokens, void* stream) {
  const char* who = "paged_decode_noalloc";
  if (batch < 0) return fail(Q3A_EINVAL, "%s: batch %d < 0", who, batch);
  if (batch == 0) return Q3A_OK;
  if (num_kv_heads < 1 || num_kv_heads > 16)
    return fail(Q3A_EINVAL, "%s: num_kv_heads %d outside [1, 16]", who, num_kv_heads);
  if (page_size <= 0 || max_pages_per_seq <= 0)
    return fail(Q3A_EINVAL, "%s: page_size %d / max_pages_per_seq %d must be > 0", who, page_size, max_pages_per_seq);
  if ((int64_t)max_pages_per_seq * page_size > (int64_t)1 << 30)
    return fail(Q3A_EINVAL, "%s: context capacity too large", who);
  void* ws = scratch_address(who);
  if (ws == nullptr) return Q3A_ELAUNCH;
  const size_t need = workspace_bytes(batch, num_kv_heads, max_pages_per_seq, page_size, split_tokens);
  if (need > kNoAllocScratchBytes)
    return fail(Q3A_ESPACE, "%s: this shape needs %zu bytes of workspace, more than the %zu-byte static scratch "
                "(batch %d, split_tokens %d)", who, need, kNoAllocScratchBytes, batch, split_tokens);
  return launch_decode(q, q_stride_b, q_stride_h, nullptr, 0, nullptr, 0, k_cache, v_cache, kv_stride_page,
                       kv_stride_tok, kv_stride_head, num_pages, page_size, cache_seqlens, block_table, bt_stride_b,
                       max_pages_per_seq, out, o_stride_b, o_stride_h, ws, kNoAllocScratchBytes, batch, num_q_heads,
                       num_kv_heads, head_dim, softmax_scale, split_tokens, stream, who);
}
