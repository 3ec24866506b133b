// Talker prefill attention for gfx950, on MFMA.
//
// Semantics: packed variable-length causal attention.  Sequence s owns query tokens
// [cu_q[s], cu_q[s+1]) of q [T, Hq, D] and keys 0..Lk-1 with Lk = cu_k[s+1] - cu_k[s], read either
// from a packed [Tk, Hkv, D] tensor (token j at row cu_k[s] + j) or from the paged KV pool
// (token j at page block_table[s][j / page_size], offset j % page_size).  Without cu arrays (the dense
// form of flash_attn_func) every sequence has Lq = seqlen_q, Lk = seqlen_k and starts at s times the
// sequence stride of q, K/V and out.  With `causal`, query i
// sees keys j <= Lk - Lq + i (bottom-right alignment).  This covers flash_attn_varlen_func at
// engine/talker.py:169 (cu_q == cu_k, fp32 form engine/talker.py:163-167), the prefix + new form
// of flash_attn_func at engine/arrivals.py:148 (fp32 form engine/arrivals.py:125-131), and both
// read from the pool after the K/V append (engine/talker.py:161-162, engine/arrivals.py:144-145).
//
// Work: one workgroup (4 waves) per (sequence, KV head, 64-query tile); wave w takes tokens 16w..16w+15 of the
// tile for BOTH query heads 2g, 2g+1 of the GQA pair, so every K or V^T operand read from LDS feeds two MFMAs.
// K/V tiles of 32 keys are copied global -> LDS by direct-to-LDS buffer loads (no register staging) into two
// stages, tile t+1 in flight while tile t is consumed, one barrier per tile.  32-key tiles keep the LDS at 32 KiB
// and the registers under 168 per lane, so three workgroups share a CU (64-key tiles: two).  LDS tiles are
// row-major [32 keys][128 dims] with the 16-byte chunks of key k XOR-swizzled by k & 15 (bank-conflict free for both the
// DMA writes and the operand reads).  v_mfma_f32_16x16x32_bf16 layouts: A lane l = row l%16, k 8*(l/16)..+8;
// B lane l = column l%16, same k; C lane l = column l%16, rows 4*(l/16)..+4.
//   S^T = K Q^T  : A = K rows from LDS, B = Q^T (columns = this lane's query token)
//   O^T = V^T P^T: A = V^T from the row-major V tile through ds_read_b64_tr_b16 (a 16-lane transpose read),
//                  B = P^T taken straight from S^T's C registers
// so the softmax statistics, P and the O accumulators of a query token all live on the lanes with that token
// in column l%16; a row's max over a tile needs only two cross-lane steps.
#include <algorithm>
#include <atomic>

#include "q3a_common.h"
#include "../../include/q3attn.h"

namespace q3a {
namespace {

constexpr int kD = 128;
constexpr int kG = 2;  // query heads per KV head (the softmax below is written for exactly two)
constexpr int kQT = 64;        // query tokens per workgroup (16 per wave, both heads)
constexpr int kKT = 32;        // keys per LDS tile
constexpr int kRowB = kD * 2;  // bytes of one key row in an LDS tile
constexpr int kTileB = kKT * kRowB;

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef short v4i16 __attribute__((ext_vector_type(4)));

struct PrefillArgs {
  const uint16_t* q;
  int64_t q_st, q_sh;
  const int32_t* cu_q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t k_sp, k_st, k_sh;  // K and V carry their own strides (k fresh, v a view of the qkv projection)
  int64_t v_sp, v_st, v_sh;
  int num_pages, page_size, page_shift;  // paged: page_size is a power of two >= 16
  const int32_t* bt;  // nullptr: packed K/V
  int64_t bt_sb;
  int max_pages;
  const int32_t* cu_k;
  uint16_t* out;
  int64_t o_st, o_sh;
  // Dense form (cu_q == nullptr): sequence strides and the common lengths.
  int64_t q_ss, k_ss, v_ss, o_ss;
  int dense_lq, dense_lk;
  int causal;
  int hkv;
  float scale_log2;
  // Append forms (q3a_prefill_append, q3a_prefill_dense_append): each query token's K and V rows of its KV head are
  // also written into a page pool at the token's position in its sequence.  pk == nullptr: no write.  p_first >= 0
  // (dense form): the prefix rows p_first .. Lk - Lq - 1 are written as well (by the first query tile's workgroup,
  // or, in the short-key kernel, with every other row from the LDS copy); -1: the query tokens' rows only.
  uint16_t* pk;
  uint16_t* pv;
  int64_t p_sp, p_st, p_sh;
  const int32_t* pbt;
  int64_t pbt_sb;
  int p_pages, p_shift, p_max_pages;
  int p_first;
  // Grouped order (prefill_kernel<true>): sequences in groups of 2^grp_shift, nqt query tiles per sequence.
  int nseq;
  int nqt;
  int grp_shift;
  // Norm/rope q (prefill_kernel<*, true>): q arrives raw and is RMS-normalised with qn and rotated with the cos/sin
  // row of its packed token index (row stride rs_st), with the rounding of eager bf16 ops, as it is loaded.
  const uint16_t* qn;
  const uint16_t* kn;   // the fused admission form (short key ranges): k's weight, then the prefix bank
  const uint16_t* pfk;
  const uint16_t* pfv;
  int64_t pfk_ss, pfk_st, pfk_sh, pfv_ss, pfv_st, pfv_sh;
  const int64_t* pidx;  // nullptr: sequence s takes prefix s; else prefix pidx[s] (outside [0, npre): zeros)
  int64_t npre;
  int P;                // prefix rows; key row j >= P is new row j - P of k/v
  const uint16_t* rcos;
  const uint16_t* rsin;
  int64_t rs_st;
  float eps;
};

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }
__device__ __forceinline__ int readlane(int v, int lane) { return __builtin_amdgcn_readlane(v, lane); }

// 16 bytes per lane from the descriptor straight into LDS at lds + 16 * lane (lanes failing the descriptor's
// bounds write zeros).
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint8_t* lds, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, (int)voff, 0, 0, 0);
}

// Transpose read: within each 16-lane group, lane i receives element i & 3 of the 8-byte words addressed by
// lanes 4k + (i >> 2), k = 0..3.
__device__ __forceinline__ uint2 ldtr(const uint8_t* lds) {
  const v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16*)lds);
  return __builtin_bit_cast(uint2, r);
}

// Waits for this wave's outstanding vector-memory operations (the direct-to-LDS copies); vmcnt(0), the other
// counters untouched.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Three waves per SIMD (<= 168 VGPRs): three workgroups per CU hide each other's prologues and barriers.
template <bool kGrouped, bool kRopeQ = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 3))) void prefill_kernel(const PrefillArgs a) {
  // Two stages of K and V tiles; separate arrays so the compiler can tell the stage being filled from the one
  // being read.
  __shared__ __align__(16) uint8_t sK0[kTileB];
  __shared__ __align__(16) uint8_t sV0[kTileB];
  __shared__ __align__(16) uint8_t sK1[kTileB];
  __shared__ __align__(16) uint8_t sV1[kTileB];

  // Grid x = (sequence, KV head) with the head fastest, z = query tile reversed (slowest): the tiles with the
  // most key tiles (the last ones of each sequence) dispatch first, the short ones fill in last.  Workgroups
  // are handed to the 8 XCDs round-robin in launch order, so with the head fastest every XCD gets the same
  // mix of sequences; with the sequence fastest each XCD got a fixed subset of sequences, and one XCD whose
  // sequences were long stalled the in-order dispatch for all (measured 48 -> 38 us on 32 x U[150,400]).
  // Grouped order, for grids of several rounds of resident workgroups: x = (sequence of the group, KV head),
  // z = (group of 2^grp_shift sequences, query tile reversed), so the groups run one after another, each longest
  // tile first.  The query tiles of a group's sequences then run side by side and share their K/V pages in the L2
  // (up to 16 readers of a page instead of about 3: 32 x 1,024 tokens 205 -> 190 us).
  int s, g, qt;
  if (!kGrouped) {
    s = blockIdx.x / a.hkv;
    g = blockIdx.x - s * a.hkv;
    qt = gridDim.z - 1 - blockIdx.z;
  } else {
    const int G = blockIdx.z / a.nqt;
    qt = a.nqt - 1 - (blockIdx.z - G * a.nqt);
    const int x = blockIdx.x / a.hkv;
    g = blockIdx.x - x * a.hkv;
    s = (G << a.grp_shift) + x;
    if (s >= a.nseq) return;
  }
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int col = lane & 15;
  const int g4 = lane >> 4;

  // The sequence's first 64 page ids depend only on s: fetch them before cu_seqlens so the first tile's
  // loads wait for one memory round trip, not two.
  // Waves 0 and 1 copy K tiles, waves 2 and 3 V tiles (below); each uses its operand's own strides, which are
  // wave-uniform and stay in scalar registers.  The norm/rope-q form reads K paged (the pool, where its producer
  // pass stored the normalised rows) and V packed.
  const bool copies_k = wave < 2;
  const bool paged = a.bt != nullptr && (!kRopeQ || copies_k);
  const int64_t bt_row = (int64_t)s * a.bt_sb;
  const int64_t c_sp = copies_k ? a.k_sp : a.v_sp;
  const int64_t c_st = copies_k ? a.k_st : a.v_st;
  const int64_t c_sh = copies_k ? a.k_sh : a.v_sh;
  int pwin = -1, pwin_base = 0;
  auto load_window = [&](int base) __attribute__((always_inline)) {
    pwin_base = base;
    const int i = base + lane;
    pwin = (paged && i < a.max_pages) ? a.bt[bt_row + i] : -1;
  };
  if (paged) load_window(0);
  // Tile 0's page id for this wave's 16-key group, a scalar load through the constant address space (the table is
  // not written by this kernel): tile 0's copies then wait for it on the scalar counter, not for the window's vector
  // load, which the compiler's count merges with every vector load of the prologue (q, the pool window) in flight.
  int page0 = -1;
  if (paged) {
    typedef __attribute__((address_space(4))) const int32_t cint32;
    const int pi0 = (16 * (wave & 1)) >> a.page_shift;
    if (pi0 < a.max_pages) page0 = ((const cint32*)a.bt)[bt_row + pi0];
  }

  // Element offsets of the sequence's first query/output row and first packed key row.
  int Lq, Lk;
  int64_t qbase, obase, kbase;  // kbase: the first key row of the operand this wave copies
  int64_t krow0, vrow0;         // the first K and V rows (append form)
  int q0 = 0;                   // the sequence's first packed token (the norm/rope form's cos/sin row)
  if (a.cu_q != nullptr) {
    q0 = a.cu_q[s];
    const int k0 = a.cu_k[s];
    Lq = a.cu_q[s + 1] - q0;
    Lk = a.cu_k[s + 1] - k0;
    qbase = (int64_t)q0 * a.q_st;
    obase = (int64_t)q0 * a.o_st;
    kbase = (int64_t)k0 * c_st;
    krow0 = (int64_t)k0 * a.k_st;
    vrow0 = (int64_t)k0 * a.v_st;
  } else {
    Lq = a.dense_lq;
    Lk = a.dense_lk;
    qbase = (int64_t)s * a.q_ss;
    obase = (int64_t)s * a.o_ss;
    kbase = (int64_t)s * (copies_k ? a.k_ss : a.v_ss);
    krow0 = (int64_t)s * a.k_ss;
    vrow0 = (int64_t)s * a.v_ss;
  }
  if (qt * kQT >= Lq) return;
  // Keys past the table are not attended; the norm/rope-q form (K paged, V packed, the prompt's own rows stored
  // from the last tiles) keeps them, and their K reads arrive as zeros (the window entry past the table is -1).
  if (a.bt != nullptr && !kRopeQ) Lk = min(Lk, a.max_pages * a.page_size);
  Lk = max(Lk, 0);

  const int tq = qt * kQT + wave * 16 + col;  // this lane's query token
  const bool qvalid = tq < Lq;
  const int qpos = Lk - Lq + tq;              // last key this token may see when causal

  // Q^T of both heads as B operands of S^T = K Q^T: 4 chunks of 32 dims each.
  bf16x8_t qb[kG][4];
  uint4 x[kG][4], w[4], c[4], sn[4];  // norm/rope-q form: raw q, weight, cos, sin
  if constexpr (!kRopeQ) {
#pragma unroll
    for (int hh = 0; hh < kG; ++hh) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        uint4 xq = make_uint4(0u, 0u, 0u, 0u);
        if (qvalid) xq = ld16(a.q + qbase + (int64_t)tq * a.q_st + (kG * g + hh) * a.q_sh + 32 * kk + 8 * g4);
        qb[hh][kk] = as_bf16x8(xq);
      }
    }
  } else {
    // Raw q, normalised and rotated here (engine/ops.py:51-60 as eager bf16 ops: y = bf16(w * bf16(x * r)),
    // o = bf16(bf16(y * cos) + bf16(rot(y) * sin))).  The lane holds dims 32 kk + 8 g4 .. +8 of its token for
    // kk = 0..3, so the mean of squares is an in-lane sum and two lane swaps over the token's 4 lanes, and the
    // rotate-half partner of chunk kk is chunk kk ^ 2 of the same lane.
    const int64_t crow = (int64_t)(q0 + (qvalid ? tq : 0)) * a.rs_st;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int d0 = 32 * kk + 8 * g4;
      w[kk] = ld16(a.qn + d0);
      c[kk] = make_uint4(0u, 0u, 0u, 0u);
      sn[kk] = c[kk];
      if (qvalid) {
        c[kk] = ld16(a.rcos + crow + d0);
        sn[kk] = ld16(a.rsin + crow + d0);
      }
#pragma unroll
      for (int hh = 0; hh < kG; ++hh) {
        x[hh][kk] = make_uint4(0u, 0u, 0u, 0u);
        if (qvalid) x[hh][kk] = ld16(a.q + qbase + (int64_t)tq * a.q_st + (kG * g + hh) * a.q_sh + d0);
      }
    }
  }

  // Append forms: K and V rows of KV head g go into the pool.  Packed (q3a_prefill_append): the rows of this
  // workgroup's query tokens (positions Lk - Lq + token).  Dense (q3a_prefill_dense_append, p_first >= 0): rows
  // p_first .. Lk - 1 in chunks of 64, chunk c taken by the sequence's query tile c mod nqt, so the prefix rows that
  // no query token owns are spread over the sequence's workgroups too.  In general the rows are loaded here, so they
  // share the prologue's round trip, and stored into the pool after it (lane (r = lane >> 4, c = lane & 15) moves
  // dims 8c..8c+7 of row base + 16 wave + 4i + r); a dense workgroup's further chunks follow the prologue.
  uint4 wk[4], wv[4];
  int64_t wdst[4];
  const bool chunked = a.pk != nullptr && a.p_first >= 0;
  const int nqt_seq = kGrouped ? a.nqt : (int)gridDim.z;
  // With causal masking and a K/V prefix that is a whole number of 32-key tiles (a prompt has none), the query
  // tokens' rows are the last one or two key tiles the workgroup streams; they are stored from LDS after the loop,
  // and the prologue only fetches the table entries of those positions (lane i: page kown0 / page_size + i).
  // (The norm/rope-q form is launched only for whole causal prompts, cu_seqlens_k == cu_seqlens_q: always this case.)
  const bool pool_from_lds =
      kRopeQ || (a.pk != nullptr && !chunked && a.causal && Lk >= Lq && ((Lk - Lq) & (kKT - 1)) == 0);
  const int kown0 = Lk - Lq + qt * kQT;
  int pwo = -1;
  if (pool_from_lds) {
    const int pi = (kown0 >> a.p_shift) + lane;
    if (lane < 8 && pi < a.p_max_pages) pwo = a.pbt[(int64_t)s * a.pbt_sb + pi];
  }
  auto load_rows = [&](int base) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      wk[i] = make_uint4(0u, 0u, 0u, 0u);
      wv[i] = wk[i];
      wdst[i] = -1;
      const int pos = base + wave * 16 + 4 * i + (lane >> 4);
      const int pi = pos >> a.p_shift;
      if (pos >= 0 && pos < Lk && pi < a.p_max_pages) {
        const int page = a.pbt[(int64_t)s * a.pbt_sb + pi];
        wk[i] = ld16(a.k + krow0 + (int64_t)pos * a.k_st + (int64_t)g * a.k_sh + 8 * (lane & 15));
        wv[i] = ld16(a.v + vrow0 + (int64_t)pos * a.v_st + (int64_t)g * a.v_sh + 8 * (lane & 15));
        if ((unsigned)page < (unsigned)a.p_pages)
          wdst[i] = (int64_t)page * a.p_sp + (int64_t)(pos & ((1 << a.p_shift) - 1)) * a.p_st + (int64_t)g * a.p_sh +
                    8 * (lane & 15);
      }
    }
  };
  auto store_rows = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (wdst[i] >= 0) {
        st16(a.pk + wdst[i], wk[i]);
        st16(a.pv + wdst[i], wv[i]);
      }
    }
  };
  if (!kRopeQ && a.pk != nullptr && !pool_from_lds) load_rows(chunked ? a.p_first + qt * kQT : kown0);

  int kend = Lk;
  if (a.causal) {
    const int last = min(Lq - 1, qt * kQT + kQT - 1);
    kend = min(Lk, Lk - Lq + last + 1);
  }
  const int ntiles = kend > 0 ? (kend + kKT - 1) / kKT : 0;
  const int jlim = a.causal ? min(Lk - 1, qpos) : Lk - 1;  // last key this lane's token sees
  // Last key that every token of this wave sees (wave-uniform).
  const int wlim = a.causal ? min(Lk - 1, Lk - Lq + qt * kQT + wave * 16) : Lk - 1;
  // Last key that some token of this wave sees (wave-uniform); -1 when the wave holds no query token.  Tiles past
  // it would add exact zeros, so the wave skips their arithmetic (it still copies and meets every barrier).
  const int wfirst = qt * kQT + wave * 16;
  const int wmax = wfirst >= Lq ? -1 : (a.causal ? min(Lk - 1, Lk - Lq + min(Lq - 1, wfirst + 15)) : Lk - 1);

  // Tile copies.  A 32-key tile is 2 groups of 16 keys and a group never straddles a page (page sizes are
  // powers of two >= 16), so each group has one uniform base address; waves 0 and 1 copy K groups 0 and 1,
  // waves 2 and 3 the V groups, with four direct-to-LDS loads each (instruction i: rows 4i..4i+3 of the group,
  // 1 KiB).  The descriptor covers
  // exactly the group's valid rows of head g: rows past the sequence and groups on an invalid page arrive as
  // zeros.  Lane l of instruction i lands at LDS chunk slot l & 15 of row rr = 4i + (l >> 4), so it fetches
  // global chunk (l & 15) ^ rr: the swizzle is applied on the global side.  Page ids come from a lane-wise
  // window (lane i = table entry pwin_base + i), read with v_readlane; it is refilled once per 64 pages.
  static_assert(kKT == 32 && kQT == 64, "the copy assignment below is for 4 waves and 2 groups per tile");
  const int cgrp = wave & 1;                     // the 16-key group of a tile this wave copies
  const uint16_t* cbase = copies_k ? a.k : a.v;  // waves 0, 1 copy K; waves 2, 3 copy V
  auto group_rsrc = [&](const uint16_t* base, int t, int page) __attribute__((always_inline)) {
    const int j0 = t * kKT + 16 * cgrp;
    const int nv = min(16, Lk - j0);
    bool ok = nv > 0;
    int64_t off = 0;
    if (paged) {
      ok = ok && (unsigned)page < (unsigned)a.num_pages;
      off = (int64_t)page * c_sp + (int64_t)(j0 & (a.page_size - 1)) * c_st;
    } else {
      off = kbase + (int64_t)j0 * c_st;
    }
    return make_rsrc(base + (ok ? off : 0) + (int64_t)g * c_sh, ok ? (uint32_t)(((nv - 1) * c_st + kD) * 2) : 0u);
  };
  uint32_t dma_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int rr = 4 * i + (lane >> 4);
    dma_off[i] = (uint32_t)((rr * c_st + 8 * ((lane & 15) ^ rr)) * 2);
  }
  // Tile 0 (first = true) takes its page id from the scalar load above.
  auto issue = [&](int t, uint8_t* Kst, uint8_t* Vst, bool first = false) __attribute__((always_inline)) {
    int page = 0;
    if (paged && first) {
      page = page0;
    } else if (paged) {
      const int pi = (t * kKT + 16 * cgrp) >> a.page_shift;
      if (pi < pwin_base || pi >= pwin_base + 64) load_window(pi & ~63);
      page = readlane(pwin, pi - pwin_base);
    }
    const __amdgpu_buffer_rsrc_t rc = group_rsrc(cbase, t, page);
    uint8_t* dst = copies_k ? Kst : Vst;
#pragma unroll
    for (int i = 0; i < 4; ++i) dma16(rc, dst + (16 * cgrp + 4 * i) * kRowB, dma_off[i]);
  };

  // Operand read offsets.  K (A of S^T): lane (col, g4) reads key kb*16 + col, logical chunk 4kk + g4, stored at
  // slot (4kk + g4) ^ col.  V^T (A of O^T, transpose read): lane L = lane & 15 of group g4 addresses key
  // key0 + (L >> 2) (key0 = 32 s2 + 16 p + 4 g4), dims 16 db + 4 (L & 3): chunk 2 db + ((L & 3) >> 1), byte
  // (L & 1) * 8, with key & 15 = 4 g4 + (L >> 2) =: rsw.
  uint32_t k_rd[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) k_rd[kk] = (uint32_t)(col * kRowB + (((4 * kk + g4) ^ col) << 4));
  const int rsw = 4 * g4 + ((lane & 15) >> 2);
  const int c_lo = ((lane & 15) & 3) >> 1;
  const uint32_t v_rd = (uint32_t)(rsw * kRowB + (lane & 1) * 8);

  f32x4_t acc[kG][8];
#pragma unroll
  for (int hh = 0; hh < kG; ++hh)
#pragma unroll
    for (int db = 0; db < 8; ++db) acc[hh][db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m[kG] = {kMaxSeed, kMaxSeed}, l[kG] = {0.f, 0.f};

  auto compute = [&](int t, const uint8_t* Ks, const uint8_t* Vs) __attribute__((always_inline)) {
    if (t * kKT > wmax) return;
    // S^T for the tile's 2 blocks of 16 keys, both heads; each K operand is read once.
    f32x4_t st[kG][kKT / 16];
#pragma unroll
    for (int kb = 0; kb < kKT / 16; ++kb) {
#pragma unroll
      for (int hh = 0; hh < kG; ++hh) st[hh][kb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const bf16x8_t kv = as_bf16x8(ld16(Ks + kb * 16 * kRowB + k_rd[kk]));
#pragma unroll
        for (int hh = 0; hh < kG; ++hh)
          st[hh][kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kv, qb[hh][kk], st[hh][kb], 0, 0, 0);
      }
    }
    // Mask: key j is visible to this lane's token iff j <= jlim (= min(Lk - 1, qpos) when causal).
    // Relative to the tile and this lane's key rows that is one compare per score against `lim`.
    // Masked scores become -inf; the running max m is kept in scaled (log2) units.
    // Tiles that every token of the wave sees whole (all but the diagonal one and the sequence's last) skip it.
    if (t * kKT + kKT - 1 > wlim) {
      const int lim = jlim - t * kKT - 4 * g4;
#pragma unroll
      for (int hh = 0; hh < kG; ++hh)
#pragma unroll
        for (int kb = 0; kb < kKT / 16; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) st[hh][kb][i] = (kb * 16 + i <= lim) ? st[hh][kb][i] : -INFINITY;
    }
    bf16x8_t pb[kG][kKT / 32];
    float mx[kG];
#pragma unroll
    for (int hh = 0; hh < kG; ++hh) {
      mx[hh] = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < kKT / 16; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx[hh] = fmaxf(mx[hh], st[hh][kb][i]);
    }
    // Lazy rescale: keep the running max while no token's tile max exceeds it by more than 8 (log2 units), so
    // p = exp2(s * scale - m) <= 256 is exact enough in bf16/fp32 and (l, acc) are rescaled only when a max grows
    // past that margin; one wave vote covers both heads (a head whose max did not grow gets alpha = 1 or a
    // smaller exact shift).  The first tile always sets the max.  The vote tests each lane's own maximum (a token's
    // tile max exceeds the margin iff one of its 4 lanes' does), so the cross-lane reduction runs only when a max
    // grows.
    if (__any(mx[0] * a.scale_log2 > m[0] + 8.f || mx[1] * a.scale_log2 > m[1] + 8.f)) {
#pragma unroll
      for (int hh = 0; hh < kG; ++hh) mx[hh] = max_xor16(max_xor32(mx[hh])) * a.scale_log2;
#pragma unroll
      for (int hh = 0; hh < kG; ++hh) {
        const float mn = fmaxf(m[hh], mx[hh]);
        const float alpha = fast_exp2(m[hh] - mn);
        l[hh] *= alpha;
#pragma unroll
        for (int db = 0; db < 8; ++db) acc[hh][db] = acc[hh][db] * alpha;
        m[hh] = mn;
      }
    }
#pragma unroll
    for (int hh = 0; hh < kG; ++hh) {
      // P^T as the B operand: k slot 8*g4 + i <- key 32*s2 + 4*g4 + i, slot 8*g4 + 4 + i <- key
      // 32*s2 + 16 + 4*g4 + i (blocks 2*s2 and 2*s2+1 of this lane's C registers).
#pragma unroll
      for (int s2 = 0; s2 < kKT / 32; ++s2) {
        float p[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p[i] = fast_exp2(fmaf(st[hh][2 * s2][i], a.scale_log2, -m[hh]));
          p[4 + i] = fast_exp2(fmaf(st[hh][2 * s2 + 1][i], a.scale_log2, -m[hh]));
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) l[hh] += p[i];
        uint4 w;
        w.x = pack_bf16x2(p[0], p[1]);
        w.y = pack_bf16x2(p[2], p[3]);
        w.z = pack_bf16x2(p[4], p[5]);
        w.w = pack_bf16x2(p[6], p[7]);
        pb[hh][s2] = as_bf16x8(w);
      }
    }
    // O^T += V^T P^T: the V^T operand of keys 32 s2 + 4 g4 + (0..3) and 32 s2 + 16 + 4 g4 + (0..3) (the B
    // operand's key order) comes from two transpose reads; each is used for both heads.
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const uint32_t chunk = (uint32_t)((((2 * db) + c_lo) ^ rsw) << 4);
#pragma unroll
      for (int s2 = 0; s2 < kKT / 32; ++s2) {
        const uint2 lo = ldtr(Vs + v_rd + chunk + (32 * s2) * kRowB);
        const uint2 hi = ldtr(Vs + v_rd + chunk + (32 * s2 + 16) * kRowB);
        const bf16x8_t va = as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y));
#pragma unroll
        for (int hh = 0; hh < kG; ++hh)
          acc[hh][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb[hh][s2], acc[hh][db], 0, 0, 0);
      }
    }
  };

  // Stage (t+1) & 1 is filled while tile t is read from stage t & 1; the barrier at the end of each tile both
  // publishes the next tile (every wave has waited for its own copies) and frees the stage just read.
  // The wait is unconditional so that no path into the loop carries outstanding loads (the q fragments): a
  // pending load on any entry path makes the compiler drain every copy before the first MFMA of each tile.
  if (ntiles > 0) issue(0, sK0, sV0, true);
  wait_vmem();
  __syncthreads();
  if constexpr (kRopeQ) {
    // The norm/rope-q form's arithmetic, on the loads the prologue issued beside tile 0's copies.  (Run while the
    // copies are still in flight, before the wait, it measured slower: 56.7 -> 57.5 us per prompt-step call.)
#pragma unroll
    for (int hh = 0; hh < kG; ++hh) {
      float ss = 0.f;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const uint32_t xs[4] = {x[hh][kk].x, x[hh][kk].y, x[hh][kk].z, x[hh][kk].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) ss += bf16_lo(xs[i]) * bf16_lo(xs[i]) + bf16_hi(xs[i]) * bf16_hi(xs[i]);
      }
      const float r = rms_rsqrt(sum_xor32(sum_xor16(ss)), a.eps);
      // chunk pairs (kp, kp + 2): dims d and d + 64
#pragma unroll
      for (int kp = 0; kp < 2; ++kp) {
        const uint32_t xl[4] = {x[hh][kp].x, x[hh][kp].y, x[hh][kp].z, x[hh][kp].w};
        const uint32_t xh[4] = {x[hh][kp + 2].x, x[hh][kp + 2].y, x[hh][kp + 2].z, x[hh][kp + 2].w};
        const uint32_t wl[4] = {w[kp].x, w[kp].y, w[kp].z, w[kp].w};
        const uint32_t wh[4] = {w[kp + 2].x, w[kp + 2].y, w[kp + 2].z, w[kp + 2].w};
        const uint32_t cl[4] = {c[kp].x, c[kp].y, c[kp].z, c[kp].w};
        const uint32_t ch[4] = {c[kp + 2].x, c[kp + 2].y, c[kp + 2].z, c[kp + 2].w};
        const uint32_t sl[4] = {sn[kp].x, sn[kp].y, sn[kp].z, sn[kp].w};
        const uint32_t sh[4] = {sn[kp + 2].x, sn[kp + 2].y, sn[kp + 2].z, sn[kp + 2].w};
        uint32_t ol[4], oh[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float el[2], eh[2];
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2) {
            auto half = [h2](uint32_t v) { return h2 ? bf16_hi(v) : bf16_lo(v); };
            const float yl = round_bf16_1op(half(wl[i]) * round_bf16_1op(half(xl[i]) * r));
            const float yh = round_bf16_1op(half(wh[i]) * round_bf16_1op(half(xh[i]) * r));
            el[h2] = round_bf16_1op(yl * half(cl[i])) + round_bf16_1op(-yh * half(sl[i]));
            eh[h2] = round_bf16_1op(yh * half(ch[i])) + round_bf16_1op(yl * half(sh[i]));
          }
          ol[i] = pack_bf16x2(el[0], el[1]);
          oh[i] = pack_bf16x2(eh[0], eh[1]);
        }
        qb[hh][kp] = as_bf16x8(make_uint4(ol[0], ol[1], ol[2], ol[3]));
        qb[hh][kp + 2] = as_bf16x8(make_uint4(oh[0], oh[1], oh[2], oh[3]));
      }
    }
    // Pin the rotated q here, ahead of the loop state: left to itself the compiler sinks this arithmetic into the
    // loop preheader, beside the live accumulators, where it spills.
#pragma unroll
    for (int hh = 0; hh < kG; ++hh) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        uint4 u = __builtin_bit_cast(uint4, qb[hh][kk]);
        asm volatile("" : "+v"(u.x), "+v"(u.y), "+v"(u.z), "+v"(u.w));
        qb[hh][kk] = as_bf16x8(u);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  if (!kRopeQ && a.pk != nullptr && !pool_from_lds) {
    store_rows();
    if (chunked) {
      for (int c = qt + nqt_seq; a.p_first + c * kQT < Lk; c += nqt_seq) {
        load_rows(a.p_first + c * kQT);
        store_rows();
      }
    }
  }
  for (int t = 0; t < ntiles; t += 2) {
    if (t + 1 < ntiles) issue(t + 1, sK1, sV1);
    compute(t, sK0, sV0);
    wait_vmem();
    __syncthreads();
    if (t + 1 >= ntiles) break;
    if (t + 2 < ntiles) issue(t + 2, sK0, sV0);
    compute(t + 1, sK1, sV1);
    wait_vmem();
    __syncthreads();
  }

  if (pool_from_lds) {
    // Token kown0 + tl's K (part 0) and V (part 1) rows, chunk ch, from the stage its tile was copied into (tile t
    // sits in stage t & 1; its LDS slot c holds global chunk c ^ (row & 15)).  The norm/rope-q form stores the V
    // rows only (its K rows are already in the pool).
    const int kown1 = min(Lk, kown0 + kQT);
    const int pi0 = kown0 >> a.p_shift;
    constexpr int kParts = kRopeQ ? 1 : 2;
#pragma unroll
    for (int it = 0; it < 4 * kParts; ++it) {
      const int idx = tid + 256 * it;
      const int tl = idx >> (3 + kParts);
      const int part = kRopeQ ? 1 : (idx >> 4) & 1;
      const int ch = idx & 15;
      const int key = kown0 + tl;
      const int pi = key >> a.p_shift;
      const int page = __shfl(pwo, min(pi - pi0, 63));
      if (key < kown1 && pi < a.p_max_pages && (unsigned)page < (unsigned)a.p_pages) {
        const int t = key >> 5;
        const int row = key & (kKT - 1);
        const uint8_t* stg = part == 0 ? ((t & 1) ? sK1 : sK0) : ((t & 1) ? sV1 : sV0);
        const uint4 x = ld16(stg + row * kRowB + ((ch ^ (row & 15)) << 4));
        uint16_t* dst = (part == 0 ? a.pk : a.pv) + (int64_t)page * a.p_sp +
                        (int64_t)(key & ((1 << a.p_shift) - 1)) * a.p_st + (int64_t)g * a.p_sh + 8 * ch;
        st16(dst, x);
      }
    }
  }

  // The 4 lanes of a token hold partial sums over disjoint keys.  The output goes out through LDS as whole 256 B
  // head rows (16 B per lane): written straight from the accumulator layout each lane would store 8 B pieces, 32 B
  // of a token row per 4 lanes, which the L2 has to merge.  The stores carry the non-temporal hint: the output is
  // never read here, and kept in the L2 it evicted the K/V pages a sequence's query tiles share (32 x U[150, 400]
  // tokens: 33.6 -> 30.4 us per call).  Each wave stages its 16 tokens x 2 heads (8 KiB) in one
  // of the tile arrays, free once every wave has passed the loop's last barrier (the pool stores above still read
  // them, hence the barrier in that form).  16 B chunks are XOR-swizzled by token, so neither side conflicts.
  if (pool_from_lds) __syncthreads();
  uint8_t* const so = wave == 0 ? sK0 : (wave == 1 ? sV0 : (wave == 2 ? sK1 : sV1));
#pragma unroll
  for (int hh = 0; hh < kG; ++hh) {
    const float lt = sum_xor32(sum_xor16(l[hh]));
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      uint2 w;
      w.x = pack_bf16x2(acc[hh][db][0] * inv, acc[hh][db][1] * inv);
      w.y = pack_bf16x2(acc[hh][db][2] * inv, acc[hh][db][3] * inv);
      const int chunk = 2 * db + (g4 >> 1);
      *reinterpret_cast<uint2*>(so + hh * 16 * kRowB + col * kRowB + ((chunk ^ col) << 4) + (g4 & 1) * 8) = w;
    }
  }
#pragma unroll
  for (int it = 0; it < 4 * kG; ++it) {
    const int hh = it >> 2;
    const int t = 4 * (it & 3) + (lane >> 4);      // token of the wave's 16
    const int c = lane & 15;                       // 16 B chunk of its 256 B row
    const int token = qt * kQT + wave * 16 + t;
    if (token < Lq) {
      const uint4 x = ld16(so + hh * 16 * kRowB + t * kRowB + ((c ^ t) << 4));
      st16_nt(a.out + obase + (int64_t)token * a.o_st + (kG * g + hh) * a.o_sh + 8 * c, x);
    }
  }
}

// ------------------------------------------------------------------------------ short key ranges
// The fast-admission shape (engine/arrivals.py:148: R = 42 new tokens over n = 77 keys) has so little work per
// (sequence, head) that the tiled kernel above is one chain of copy -> barrier -> MFMA -> softmax -> MFMA per key tile
// for a single wave per SIMD.  Here one workgroup, for one query head of a GQA pair, holds the sequence's whole K/V
// range of that KV head in LDS (at most kResMaxTiles tiles of 32 keys, copied at once; the two heads' workgroups
// copy it separately, which halves the LDS operand traffic per CU), and each wave takes 16 query tokens: the tile
// then runs with no copy, wait or barrier, as one pass over all keys (scores of every tile, one row max, P, P.V: no
// running max to carry from tile to tile), and a wave's arithmetic is half the two-head one.  Dense
// form only (seqlen_k <= 128); the query tokens of a sequence are split over workgroups of at most kResMaxGroups
// 16-token groups.
constexpr int kResMaxTiles = 4;
constexpr int kResQ = 16;
constexpr int kResMaxGroups = 16;  // waves per workgroup

// The fused admission form (kRope) runs at most kResRopeWaves waves per workgroup (7 query groups + the store wave):
// with 64 KiB of LDS per workgroup two fit a CU whatever the bound, and the lower bound leaves room in the registers
// for its prologue loads.
constexpr int kResRopeWaves = 8;

template <bool kAppend, bool kRope = false>
__global__ __launch_bounds__(64 * (kRope ? kResRopeWaves : kResMaxGroups)) void prefill_resident_kernel(
    const PrefillArgs a, int ntiles) {
  __shared__ __align__(16) uint8_t sK[kResMaxTiles * kTileB];
  __shared__ __align__(16) uint8_t sV[kResMaxTiles * kTileB];

  const int s = blockIdx.x / a.hkv;
  const int g = blockIdx.x - s * a.hkv;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nwaves = blockDim.x >> 6;
  const int lane = tid & 63;
  const int col = lane & 15;
  const int g4 = lane >> 4;
  const int hh = blockIdx.z & 1;                               // query head 2g + hh
  const int tg = (blockIdx.z >> 1) * kResMaxGroups + wave;     // 16-token query group

  const int Lq = a.dense_lq;
  const int Lk = a.dense_lk;
  const int64_t qbase = (int64_t)s * a.q_ss, obase = (int64_t)s * a.o_ss;

  // Append form: rows p_first .. Lk - 1 of this KV head go into the pool from the LDS copy, K by the workgroup of
  // query head 0 and V by that of query head 1 (first query block only).  When the query groups fit in one
  // workgroup the host adds one wave that holds no query token: it helps with the copies and then makes all the
  // pool stores while the other waves compute; otherwise every wave of the block takes a share.  Lane i holds table
  // entry i (Lk <= 128 keys span at most 8 pages of >= 16); it is loaded beside the copies, so it adds no round trip.
  const bool app = kAppend && (blockIdx.z >> 1) == 0;
  const bool store_wave = kAppend && nwaves > (Lq + kResQ - 1) / kResQ;  // the last wave is the extra one
  int pwo = -1;
  if (app && lane < min(kResMaxTiles * kKT / 16, a.p_max_pages)) pwo = a.pbt[(int64_t)s * a.pbt_sb + lane];

  // Copies: the 16-key groups of K and V (2 per tile and operand) are dealt round-robin to the waves; four
  // direct-to-LDS loads each, same layout and swizzle as the tiled kernel.
  const int ngroups = 4 * ntiles;
  // The copies' kernel arguments (and the append form's table arguments) are read with the others, in one batch:
  // left to itself the compiler reads them after the first batch has returned, one more round trip before the first
  // copy.  (Not in the norm/rope form, whose registers the compiler then splits the first batch over.)
  if constexpr (!kRope) {
    __asm__ volatile("" ::"s"(a.k), "s"(a.v), "s"(a.k_st), "s"(a.k_sh), "s"(a.k_ss), "s"(a.v_st), "s"(a.v_sh),
                     "s"(a.v_ss));
    if constexpr (kAppend) __asm__ volatile("" ::"s"(a.pbt), "s"(a.pbt_sb), "s"(a.p_max_pages));
  }
  const int P = kRope ? a.P : 0;  // fused admission form: key rows below P come from the prefix bank
  int64_t psrc = -1;              // its prefix row (-1: zeros)
  if constexpr (kRope) {
    psrc = a.pidx != nullptr ? a.pidx[s] : s;
    if ((uint64_t)psrc >= (uint64_t)a.npre) psrc = -1;
  }
  for (int c = wave; c < ngroups; c += nwaves) {
    const int op = c & 1;                       // 0: K, 1: V
    const int grp = c >> 1;                     // 16-key group 0 .. 2 ntiles - 1
    const uint16_t* base = op == 0 ? a.k : a.v;
    const int64_t st = op == 0 ? a.k_st : a.v_st;
    const int64_t sh = op == 0 ? a.k_sh : a.v_sh;
    const int64_t ss = op == 0 ? a.k_ss : a.v_ss;
    const int jg = 16 * grp;
    uint8_t* dst = (op == 0 ? sK : sV) + grp * 16 * kRowB;
    if constexpr (!kRope) {
      const int nv = min(16, Lk - jg);
      const bool ok = nv > 0;
      const __amdgpu_buffer_rsrc_t r = make_rsrc(
          base + (ok ? (int64_t)s * ss + (int64_t)jg * st : 0) + (int64_t)g * sh,
          ok ? (uint32_t)(((nv - 1) * st + kD) * 2) : 0u);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rr = 4 * i + (lane >> 4);
        dma16(r, dst + 4 * i * kRowB, (uint32_t)((rr * st + 8 * ((lane & 15) ^ rr)) * 2));
      }
    } else {
      // Rows jg .. jg + 15 from two sources: new rows [max(jg, P), min(jg + 16, Lk)) of k/v (row j - P) here, prefix
      // rows [jg, min(jg + 16, P)) of the bank's row psrc after the q loads (below), once the bank index has arrived.
      // Each lane's copy goes through the descriptor of its row's source, the other masked off, so neither writes
      // the other's rows; rows past a source's range (or a prefix of index -1) arrive as zeros.
      const int j1 = max(jg, P);
      const int nn = min(jg + 16, Lk) - j1;
      const __amdgpu_buffer_rsrc_t rn = make_rsrc(
          nn > 0 ? base + (int64_t)s * ss + (int64_t)(j1 - P) * st + (int64_t)g * sh : base,
          nn > 0 ? (uint32_t)(((nn - 1) * st + kD) * 2) : 0u);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rr = 4 * i + (lane >> 4);
        if (jg + rr >= P)
          dma16(rn, dst + 4 * i * kRowB, (uint32_t)(((jg + rr - j1) * st + 8 * ((lane & 15) ^ rr)) * 2));
      }
    }
  }
  const int tq = tg * kResQ + col;
  const bool qvalid = tq < Lq;
  bf16x8_t qb[4];
  uint4 qx[4], qw[4], qc[4], qs[4];  // fused admission form: raw q, weight, cos, sin
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    uint4 x = make_uint4(0u, 0u, 0u, 0u);
    if (qvalid) x = ld16(a.q + qbase + (int64_t)tq * a.q_st + (kG * g + hh) * a.q_sh + 32 * kk + 8 * g4);
    qb[kk] = as_bf16x8(x);
    if constexpr (kRope) {
      qx[kk] = x;
      qw[kk] = ld16(a.qn + 32 * kk + 8 * g4);
      qc[kk] = make_uint4(0u, 0u, 0u, 0u);
      qs[kk] = qc[kk];
      if (qvalid) {
        qc[kk] = ld16(a.rcos + (int64_t)tq * a.rs_st + 32 * kk + 8 * g4);
        qs[kk] = ld16(a.rsin + (int64_t)tq * a.rs_st + 32 * kk + 8 * g4);
      }
    }
  }
  // Fused admission form: the weight and cos/sin chunks of the first kPf K-row groups this wave normalises (group
  // gi = P / 4 + wave + i nwaves, row 4 gi + lane / 16), loaded beside the copies.
  constexpr int kPf = kRope ? 3 : 1;
  uint4 kw, kc[kPf], ks[kPf];
  if constexpr (kRope) {
    kw = ld16(a.kn + 8 * (lane & 15));
#pragma unroll
    for (int i = 0; i < kPf; ++i) {
      const int r = 4 * ((P >> 2) + wave + i * nwaves) + (lane >> 4);
      const int t = min(max(r - P, 0), Lq - 1);
      kc[i] = ld16(a.rcos + (int64_t)t * a.rs_st + 8 * (lane & 15));
      ks[i] = ld16(a.rsin + (int64_t)t * a.rs_st + 8 * (lane & 15));
    }
    // The prefix rows' copies (16-key groups below P), same assignment of groups to waves as above.
    for (int c = wave; c < ngroups && 16 * (c >> 1) < P; c += nwaves) {
      const int op = c & 1;
      const int jg = 16 * (c >> 1);
      const uint16_t* pbase = op == 0 ? a.pfk : a.pfv;
      const int64_t pst = op == 0 ? a.pfk_st : a.pfv_st;
      const int64_t psh = op == 0 ? a.pfk_sh : a.pfv_sh;
      const int64_t pss = op == 0 ? a.pfk_ss : a.pfv_ss;
      const int np = psrc >= 0 ? min(16, P - jg) : 0;
      const __amdgpu_buffer_rsrc_t rp = make_rsrc(
          np > 0 ? pbase + psrc * pss + (int64_t)jg * pst + (int64_t)g * psh : a.k,
          np > 0 ? (uint32_t)(((np - 1) * pst + kD) * 2) : 0u);
      uint8_t* dst = (op == 0 ? sK : sV) + (c >> 1) * 16 * kRowB;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rr = 4 * i + (lane >> 4);
        if (jg + rr < P) dma16(rp, dst + 4 * i * kRowB, (uint32_t)((rr * pst + 8 * ((lane & 15) ^ rr)) * 2));
      }
    }
  }
  wait_vmem();
  __syncthreads();
  if constexpr (kRope) {
    // The new K rows P .. Lk - 1 normalised and rotated in place (engine/ops.py:51-60 as eager bf16 ops, token
    // j - P's cos/sin row), 16 lanes per row: lane chunk c of row r sits at LDS slot c ^ (r & 15).  Then q, in
    // registers: the lane holds dims 32 kk + 8 g4 .. +8 of its token, so the mean of squares is an in-lane sum and
    // two lane swaps, and the rotate-half partner of chunk kk is chunk kk ^ 2.
    const int ch = lane & 15;
#pragma unroll
    for (int i = 0; i < kPf; ++i) {
      const int gi = (P >> 2) + wave + i * nwaves;
      if (4 * gi >= Lk) break;              // wave-uniform
      const int r = 4 * gi + (lane >> 4);   // < 4 ceil(Lk / 4) <= 128 rows of sK
      uint8_t* p = sK + r * kRowB + ((ch ^ (r & 15)) << 4);
      const uint4 y = qk_norm_rope16_eager(ld16(p), kw, kc[i], ks[i], a.eps);
      if (r >= P && r < Lk) st16(p, y);
    }
    for (int gi = (P >> 2) + wave + kPf * nwaves; 4 * gi < Lk; gi += nwaves) {
      const int r = 4 * gi + (lane >> 4);
      const int t = min(max(r - P, 0), Lq - 1);
      uint8_t* p = sK + r * kRowB + ((ch ^ (r & 15)) << 4);
      const uint4 y = qk_norm_rope16_eager(ld16(p), kw, ld16(a.rcos + (int64_t)t * a.rs_st + 8 * ch),
                                           ld16(a.rsin + (int64_t)t * a.rs_st + 8 * ch), a.eps);
      if (r >= P && r < Lk) st16(p, y);
    }
    float ss = 0.f;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const uint32_t xs[4] = {qx[kk].x, qx[kk].y, qx[kk].z, qx[kk].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) ss += bf16_lo(xs[i]) * bf16_lo(xs[i]) + bf16_hi(xs[i]) * bf16_hi(xs[i]);
    }
    const float rq = rms_rsqrt(sum_xor32(sum_xor16(ss)), a.eps);
#pragma unroll
    for (int kp = 0; kp < 2; ++kp) {
      const uint32_t xl[4] = {qx[kp].x, qx[kp].y, qx[kp].z, qx[kp].w};
      const uint32_t xh[4] = {qx[kp + 2].x, qx[kp + 2].y, qx[kp + 2].z, qx[kp + 2].w};
      const uint32_t wl[4] = {qw[kp].x, qw[kp].y, qw[kp].z, qw[kp].w};
      const uint32_t wh[4] = {qw[kp + 2].x, qw[kp + 2].y, qw[kp + 2].z, qw[kp + 2].w};
      const uint32_t cl[4] = {qc[kp].x, qc[kp].y, qc[kp].z, qc[kp].w};
      const uint32_t chh[4] = {qc[kp + 2].x, qc[kp + 2].y, qc[kp + 2].z, qc[kp + 2].w};
      const uint32_t sl[4] = {qs[kp].x, qs[kp].y, qs[kp].z, qs[kp].w};
      const uint32_t sh[4] = {qs[kp + 2].x, qs[kp + 2].y, qs[kp + 2].z, qs[kp + 2].w};
      uint32_t ol[4], oh[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float el[2], eh[2];
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          auto half = [h2](uint32_t v) { return h2 ? bf16_hi(v) : bf16_lo(v); };
          const float yl = round_bf16(half(wl[i]) * round_bf16(half(xl[i]) * rq));
          const float yh = round_bf16(half(wh[i]) * round_bf16(half(xh[i]) * rq));
          el[h2] = round_bf16(yl * half(cl[i])) + round_bf16(-yh * half(sl[i]));
          eh[h2] = round_bf16(yh * half(chh[i])) + round_bf16(yl * half(sh[i]));
        }
        ol[i] = pack_bf16x2(el[0], el[1]);
        oh[i] = pack_bf16x2(eh[0], eh[1]);
      }
      qb[kp] = as_bf16x8(make_uint4(ol[0], ol[1], ol[2], ol[3]));
      qb[kp + 2] = as_bf16x8(make_uint4(oh[0], oh[1], oh[2], oh[3]));
    }
    wait_vmem();
    __syncthreads();
  }
  if (app) {
    // Rows go out in aligned groups of 4 (lane: row 4 gi + lane / 16, chunk lane % 16), group gi to wave gi mod
    // nwaves.  A group never straddles a page (pages hold >= 16 rows), so its page id is wave-uniform: one
    // v_readlane, no cross-lane shuffle in the chain.  LDS slot c of key row r holds global chunk c ^ (r & 15).
    // Non-temporal stores: 6.93 -> 6.53 us per call on the admission shape (8 x 42 over 77 keys).
    const uint8_t* src = hh == 0 ? sK : sV;
    uint16_t* const dst = hh == 0 ? a.pk : a.pv;
    const int ch = lane & 15;
    const int ng = (Lk + 3) >> 2;
    const int w0 = store_wave ? wave - (nwaves - 1) : wave;   // < 0: a compute wave with the extra one present
    const int ws = store_wave ? 1 : nwaves;
    for (int gi = w0 < 0 ? ng : (a.p_first >> 2) + w0; gi < ng; gi += ws) {
      const int r = 4 * gi + (lane >> 4);
      const int pi = (4 * gi) >> a.p_shift;
      const int page = readlane(pwo, min(pi, 63));
      if (r >= a.p_first && r < Lk && pi < a.p_max_pages && (unsigned)page < (unsigned)a.p_pages)
        st16_nt(dst + (int64_t)page * a.p_sp + (int64_t)(r & ((1 << a.p_shift) - 1)) * a.p_st +
                    (int64_t)g * a.p_sh + 8 * ch,
                ld16(src + r * kRowB + ((ch ^ (r & 15)) << 4)));
    }
  }
  if (tg * kResQ >= Lq) return;                 // a wave with no query token (after the barrier: it copied)

  const int jlim = a.causal ? min(Lk - 1, Lk - Lq + tq) : Lk - 1;
  const int wfirst = tg * kResQ;
  // last key some token of this wave sees, and the last one every token of it sees
  const int wmax = a.causal ? min(Lk - 1, Lk - Lq + min(Lq - 1, wfirst + kResQ - 1)) : Lk - 1;
  const int wlim = a.causal ? min(Lk - 1, Lk - Lq + wfirst) : Lk - 1;
  const int rsw = 4 * g4 + ((lane & 15) >> 2);
  const int c_lo = ((lane & 15) & 3) >> 1;
  const uint32_t v_rd = (uint32_t)(rsw * kRowB + (lane & 1) * 8);

  // One pass over at most 128 keys, no running max: every tile's scores first (independent MFMA chains), one row
  // max, then P and O^T = V^T P^T.  nt = tiles this wave's tokens see (wave-uniform).
  const int nt = min(ntiles, wmax / kKT + 1);
  f32x4_t st[kResMaxTiles][kKT / 16];
#pragma unroll
  for (int t = 0; t < kResMaxTiles; ++t) {
#pragma unroll
    for (int kb = 0; kb < kKT / 16; ++kb) {
      st[t][kb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      if (t < nt) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const bf16x8_t kv =
              as_bf16x8(ld16(sK + t * kTileB + kb * 16 * kRowB + col * kRowB + (((4 * kk + g4) ^ col) << 4)));
          st[t][kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kv, qb[kk], st[t][kb], 0, 0, 0);
        }
      }
    }
  }
  float mx = -INFINITY;
#pragma unroll
  for (int t = 0; t < kResMaxTiles; ++t) {
    if (t < nt) {
      if (t * kKT + kKT - 1 > wlim) {
        // key t*32 + 16 kb + 4 g4 + i is visible to this lane's token iff it is <= jlim
        const int lim = jlim - t * kKT - 4 * g4;
#pragma unroll
        for (int kb = 0; kb < kKT / 16; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) st[t][kb][i] = (kb * 16 + i <= lim) ? st[t][kb][i] : -INFINITY;
      }
#pragma unroll
      for (int kb = 0; kb < kKT / 16; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, st[t][kb][i]);
    }
  }
  // a token that sees no key keeps the finite seed, so its p are exp2(-inf) = 0 and its output is zero
  const float m = fmaxf(kMaxSeed, max_xor16(max_xor32(mx)) * a.scale_log2);
  f32x4_t acc[8];
#pragma unroll
  for (int db = 0; db < 8; ++db) acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float l = 0.f;
#pragma unroll
  for (int t = 0; t < kResMaxTiles; ++t) {
    if (t < nt) {
      float p[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p[i] = fast_exp2(fmaf(st[t][0][i], a.scale_log2, -m));
        p[4 + i] = fast_exp2(fmaf(st[t][1][i], a.scale_log2, -m));
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) l += p[i];
      uint4 w;
      w.x = pack_bf16x2(p[0], p[1]);
      w.y = pack_bf16x2(p[2], p[3]);
      w.z = pack_bf16x2(p[4], p[5]);
      w.w = pack_bf16x2(p[6], p[7]);
      const bf16x8_t pb = as_bf16x8(w);
      const uint8_t* Vs = sV + t * kTileB;
#pragma unroll
      for (int db = 0; db < 8; ++db) {
        const uint32_t chunk = (uint32_t)((((2 * db) + c_lo) ^ rsw) << 4);
        const uint2 lo = ldtr(Vs + v_rd + chunk);
        const uint2 hi = ldtr(Vs + v_rd + chunk + 16 * kRowB);
        acc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y)), pb,
                                                          acc[db], 0, 0, 0);
      }
    }
  }
  // The 4 lanes of a token hold partial sums over disjoint keys.
  l = sum_xor32(sum_xor16(l));
  if (qvalid) {
    const float inv = l > 0.f ? __builtin_amdgcn_rcpf(l) : 0.f;
    uint16_t* o = a.out + obase + (int64_t)tq * a.o_st + (kG * g + hh) * a.o_sh + 4 * g4;
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      uint2 w;
      w.x = pack_bf16x2(acc[db][0] * inv, acc[db][1] * inv);
      w.y = pack_bf16x2(acc[db][2] * inv, acc[db][3] * inv);
      *reinterpret_cast<uint2*>(o + db * 16) = w;
    }
  }
}

// ------------------------------------------------------------------------------ admission producers
// The fast-admission layer's attention inputs (engine/arrivals.py:112-118): q = rope(rms(q_raw, qn)), the new keys
// rope(rms(k_raw, kn)) after the K/V prefix, and the new values after the V prefix, i.e. K = cat(prefix K, new keys)
// and V = cat(prefix V, v) of engine/arrivals.py:118, written dense for the attention that follows.  One 128-dim row
// per 16 lanes (16 B each, the qk_norm_rope16 layout); the row jobs are numbered q rows, new K rows, new V rows,
// prefix K rows, prefix V rows, each block a multiple of 4 rows, so a wave's four rows are all of one kind.
struct AdmitPrepArgs {
  const uint16_t* q;
  int64_t q_ss, q_st, q_sh;
  const uint16_t* k;
  int64_t k_ss, k_st, k_sh;
  const uint16_t* v;
  int64_t v_ss, v_st, v_sh;
  const uint16_t* pk;
  int64_t pk_ss, pk_st, pk_sh;
  const uint16_t* pv;
  int64_t pv_ss, pv_st, pv_sh;
  const int64_t* pidx;  // nullptr: sequence s takes prefix s; else prefix pidx[s] (outside [0, npre): zeros)
  int64_t npre;
  const uint16_t* qn;
  const uint16_t* kn;
  const uint16_t* cs;   // cos/sin rows of the new tokens' positions, row t for token t
  const uint16_t* sn;
  int64_t cs_st;
  float eps;
  uint16_t* qo;  // [S, R, Hq, D]
  uint16_t* ko;  // [S, n, Hkv, D]
  uint16_t* vo;  // [S, n, Hkv, D]
  int R, P, Hq, Hkv;
  int64_t jq, jk, jv, jp, jall;  // job block ends: q | new K | new V | prefix K | prefix V
  // prompt_k_kernel (the prompt step's k rows, R packed tokens): token t belongs to the sequence s with
  // cu[s] <= t < cu[s + 1] (nseq sequences) and its normalised rows go to the page pool at position t - cu[s] of s
  // (table pbt; rows whose page is outside [0, p_pages) or past the table are not stored).
  const int32_t* cu;
  int nseq;
  uint16_t* kpool;
  int64_t p_sp, p_st, p_sh;
  const int32_t* pbt;
  int64_t pbt_sb;
  int p_pages, p_shift, p_max_pages;
};

__global__ __launch_bounds__(256) void admit_prep_kernel(const AdmitPrepArgs a) {
  const int lane = threadIdx.x & 63;
  // The wave's first row job, a multiple of 4 (the job count is below 2^31).  It is wave-uniform, so the block and
  // index decomposition below is done once per wave in 32 bits; the wave's 4 rows differ only in the head (every
  // block's row count and head count are multiples of 4).
  const uint32_t j0 = __builtin_amdgcn_readfirstlane((blockIdx.x * 4u + (threadIdx.x >> 6)) * 4u);
  if (j0 >= (uint32_t)a.jall) return;
  const int hsub = lane >> 4;      // the lane's row of the wave's 4
  const int c8 = 8 * (lane & 15);  // this lane's 8 dims
  const int n = a.P + a.R;
  const uint32_t jq = (uint32_t)a.jq, jk = (uint32_t)a.jk, jv = (uint32_t)a.jv, jp = (uint32_t)a.jp;
  if (j0 < jk) {
    // normalise + rotate: q rows, then the new K rows
    const bool isq = j0 < jq;
    const uint32_t H = isq ? a.Hq : a.Hkv;
    const uint32_t jj = isq ? j0 : j0 - jq, ht = jj / H;
    const int h = (int)(jj - ht * H) + hsub;
    const int t = (int)(ht % (uint32_t)a.R);
    const int64_t sq = ht / (uint32_t)a.R;
    const uint4 x = isq ? ld16(a.q + sq * a.q_ss + (int64_t)t * a.q_st + (int64_t)h * a.q_sh + c8)
                        : ld16(a.k + sq * a.k_ss + (int64_t)t * a.k_st + (int64_t)h * a.k_sh + c8);
    const uint4 w = ld16((isq ? a.qn : a.kn) + c8);
    const uint4 c = ld16(a.cs + (int64_t)t * a.cs_st + c8);
    const uint4 sn = ld16(a.sn + (int64_t)t * a.cs_st + c8);
    const uint4 y = qk_norm_rope16_eager<true>(x, w, c, sn, a.eps);
    if (isq)
      st16(a.qo + ((sq * a.R + t) * a.Hq + h) * kD + c8, y);
    else
      st16(a.ko + ((sq * n + a.P + t) * a.Hkv + h) * kD + c8, y);
  } else if (j0 < jv) {
    const uint32_t jj = j0 - jk, ht = jj / (uint32_t)a.Hkv;  // new V rows
    const int h = (int)(jj - ht * a.Hkv) + hsub;
    const int t = (int)(ht % (uint32_t)a.R);
    const int64_t sq = ht / (uint32_t)a.R;
    st16(a.vo + ((sq * n + a.P + t) * a.Hkv + h) * kD + c8,
         ld16(a.v + sq * a.v_ss + (int64_t)t * a.v_st + (int64_t)h * a.v_sh + c8));
  } else {
    const bool isk = j0 < jp;   // prefix K rows, then prefix V rows
    const uint32_t jj = isk ? j0 - jv : j0 - jp, hr = jj / (uint32_t)a.Hkv;
    const int h = (int)(jj - hr * a.Hkv) + hsub;
    const int r = (int)(hr % (uint32_t)a.P);
    const int64_t sq = hr / (uint32_t)a.P;
    const int64_t src = a.pidx != nullptr ? a.pidx[sq] : sq;
    uint4 x = make_uint4(0u, 0u, 0u, 0u);
    if ((uint64_t)src < (uint64_t)a.npre)
      x = isk ? ld16(a.pk + src * a.pk_ss + (int64_t)r * a.pk_st + (int64_t)h * a.pk_sh + c8)
              : ld16(a.pv + src * a.pv_ss + (int64_t)r * a.pv_st + (int64_t)h * a.pv_sh + c8);
    st16((isk ? a.ko : a.vo) + ((sq * n + r) * a.Hkv + h) * kD + c8, x);
  }
}

// The prompt step's k producer (engine/talker.py:158 as eager bf16 ops): every packed token's Hkv raw k rows
// normalised and rotated with the token's cos/sin row, straight into the pool at the token's position in its
// sequence.  A wave takes kGroups consecutive groups of 4 rows (4 heads of one token, 16 lanes per row in the
// qk_norm_rope16 layout) and issues every group's loads before the first is used, so each wave keeps kGroups KiB of
// rows in flight: with one group per wave the pass was bound by the bytes the resident waves had in flight.  The
// token's sequence comes from one ballot over 64 cu_seqlens entries per group (the lengths are non-decreasing, so
// each ballot is a prefix of the lanes), its page from the table.
constexpr int kPromptKGroups = 2;

__global__ __launch_bounds__(256) void prompt_k_kernel(const AdmitPrepArgs a) {
  constexpr int kGroups = kPromptKGroups;
  typedef __attribute__((address_space(4))) const int32_t cint32;
  const int lane = threadIdx.x & 63;
  const int hsub = lane >> 4;      // the lane's row of a group's 4
  const int c8 = 8 * (lane & 15);  // this lane's 8 dims
  const uint32_t per_tok = (uint32_t)a.Hkv >> 2;
  const uint32_t ngroups = (uint32_t)a.R * per_tok;  // below 2^31 (checked on the host)
  const uint32_t g0 = __builtin_amdgcn_readfirstlane((blockIdx.x * 4u + (threadIdx.x >> 6)) * (uint32_t)kGroups);
  if (g0 >= ngroups) return;
  // The sequence boundaries first (up to 63 sequences in one load; more take the loop below), then the rows: the
  // first wait covers the boundaries alone, and the page ids (scalar loads) are in flight with the rows.
  const bool one_load = a.nseq < 64;
  const int cfirst = one_load ? (lane <= a.nseq ? a.cu[lane] : 0x7fffffff) : 0;
  int t[kGroups], h[kGroups];
  uint4 x[kGroups], c[kGroups], sn[kGroups];
  const uint4 w = ld16(a.kn + c8);
#pragma unroll
  for (int i = 0; i < kGroups; ++i) {
    const uint32_t g = min(g0 + (uint32_t)i, ngroups - 1u);  // a wave's tail groups repeat the last one, unstored
    t[i] = (int)(g / per_tok);
    h[i] = (int)(g - (uint32_t)t[i] * per_tok) * 4 + hsub;
    x[i] = ld16(a.k + (int64_t)t[i] * a.k_st + (int64_t)h[i] * a.k_sh + c8);
    c[i] = ld16(a.cs + (int64_t)t[i] * a.cs_st + c8);
    sn[i] = ld16(a.sn + (int64_t)t[i] * a.cs_st + c8);
  }
  // The sequence of each group's token (wave-uniform): the last s in 0..nseq with cu[s] <= t.  The lengths are
  // non-decreasing, so each ballot is a prefix of the lanes.
  int sidx[kGroups], start[kGroups];
#pragma unroll
  for (int i = 0; i < kGroups; ++i) sidx[i] = -1, start[i] = 0;
  if (one_load) {
#pragma unroll
    for (int i = 0; i < kGroups; ++i) {
      const int nle = __popcll(__ballot(cfirst <= t[i]));
      if (nle > 0) {
        sidx[i] = nle - 1;
        start[i] = __builtin_amdgcn_readlane(cfirst, nle - 1);
      }
    }
  } else {
    for (int base = 0; base <= a.nseq; base += 64) {
      const int j = base + lane;
      const int cj = j <= a.nseq ? a.cu[j] : 0x7fffffff;
      bool more = false;
#pragma unroll
      for (int i = 0; i < kGroups; ++i) {
        const int nle = __popcll(__ballot(cj <= t[i]));
        if (nle > 0) {
          sidx[i] = base + nle - 1;
          start[i] = __builtin_amdgcn_readlane(cj, nle - 1);
        }
        more = more || nle == 64;
      }
      if (!more) break;
    }
  }
  int64_t dst[kGroups];
#pragma unroll
  for (int i = 0; i < kGroups; ++i) {
    dst[i] = -1;
    const int pos = t[i] - start[i];
    const int pi = pos >> a.p_shift;
    if (g0 + (uint32_t)i < ngroups && sidx[i] >= 0 && sidx[i] < a.nseq && pos >= 0 && pi < a.p_max_pages) {
      const int page = ((const cint32*)a.pbt)[(int64_t)sidx[i] * a.pbt_sb + pi];  // the table is read-only here
      if ((unsigned)page < (unsigned)a.p_pages)
        dst[i] = (int64_t)page * a.p_sp + (int64_t)(pos & ((1 << a.p_shift) - 1)) * a.p_st + (int64_t)h[i] * a.p_sh +
                 c8;
    }
  }
#pragma unroll
  for (int i = 0; i < kGroups; ++i) {
    const uint4 y = qk_norm_rope16_eager<true>(x[i], w, c[i], sn[i], a.eps);
    if (dst[i] >= 0) st16(a.kpool + dst[i], y);
  }
}

}  // namespace
}  // namespace q3a

using namespace q3a;

// Checks shared by both entry points; returns Q3A_OK or an error code with the message set.
static int check_common(const void* q, const void* k, const void* v, const void* out, int64_t q_st, int64_t q_sh,
                        int64_t k_st, int64_t k_sh, int64_t v_st, int64_t v_sh, int64_t o_st, int64_t o_sh,
                        int num_q_heads, int num_kv_heads, int head_dim, const char* who) {
  if (head_dim != kD) return fail(Q3A_EINVAL, "%s: head_dim %d unsupported (need %d)", who, head_dim, kD);
  if (num_kv_heads < 1 || num_q_heads != kG * num_kv_heads)
    return fail(Q3A_EINVAL, "%s: num_q_heads %d must be %d * num_kv_heads %d", who, num_q_heads, kG, num_kv_heads);
  if (!q || !k || !v || !out) return fail(Q3A_EINVAL, "%s: null pointer argument", who);
  const uintptr_t align = (uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out;
  if (align % 16 != 0) return fail(Q3A_EINVAL, "%s: q/k/v/out must be 16-byte aligned", who);
  if ((q_st | q_sh | k_st | k_sh | v_st | v_sh | o_st | o_sh) % 8 != 0)
    return fail(Q3A_EINVAL, "%s: strides must be multiples of 8 elements (16 bytes)", who);
  const int64_t lim = (int64_t)1 << 26;
  if (k_st < head_dim || k_sh < 0 || k_st > lim || v_st < head_dim || v_sh < 0 || v_st > lim)
    return fail(Q3A_EINVAL, "%s: token strides %lld/%lld must be in [head_dim, 2^26] and head strides >= 0", who,
                (long long)k_st, (long long)v_st);
  return Q3A_OK;
}

// Workgroups of prefill_kernel the current device holds at once (cached per device; two host threads may fill an
// entry at once, both with the same value).  768 on MI355X (3 per CU).
static int resident_slots() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 768;
  const int cached = cache[dev].load(std::memory_order_relaxed);
  if (cached > 0) return cached;
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, prefill_kernel<false>, 256, 0) != hipSuccess)
    return 768;
  const int n = std::max(1, cus * std::max(1, per_cu));
  cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

static int launch(const PrefillArgs& args, int num_seqs, int max_seqlen_q, void* stream, const char* who) {
  const int nqt = (max_seqlen_q + kQT - 1) / kQT;
  if ((int64_t)num_seqs * args.hkv > 0x7fffffff || nqt > 65535)
    return fail(Q3A_EINVAL, "%s: grid too large (%d seqs x %d KV heads x %d query tiles)", who, num_seqs, args.hkv,
                nqt);
  // Work order.  A grid of at most about three rounds of resident workgroups (3 per CU) runs all sequences'
  // query tiles longest first: the longest key-tile chains start at once, and the call's tail is made of short
  // tiles (32 x U[150, 400] tokens: 34.8 us, against 36.1 grouped).  Larger grids run in groups of sequences
  // with at most 64 query tiles in all (8 of up to 448 tokens, 4 of 1,024), about what one XCD holds at once,
  // so the K/V pages a group's query tiles share stay in the L2 (32 x 1,024: 205 -> 190 us, 64 x U[150, 400]:
  // 61.5 -> 57.0).
  PrefillArgs a = args;
  a.nseq = num_seqs;
  a.nqt = nqt;
  a.grp_shift = 0;
  while (a.grp_shift < 6 && (nqt << (a.grp_shift + 1)) <= 64) ++a.grp_shift;
  const int ngroups = (num_seqs + (1 << a.grp_shift) - 1) >> a.grp_shift;
  const bool grouped = (int64_t)num_seqs * nqt * a.hkv > 3 * resident_slots() && ngroups > 1 &&
                       (int64_t)ngroups * nqt <= 65535;
  const dim3 ggrid((1u << a.grp_shift) * a.hkv, 1, ngroups * nqt), grid(num_seqs * a.hkv, 1, nqt);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (a.qn != nullptr) {
    if (grouped) hipLaunchKernelGGL((prefill_kernel<true, true>), ggrid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((prefill_kernel<false, true>), grid, dim3(256), 0, st, a);
  } else {
    if (grouped) hipLaunchKernelGGL((prefill_kernel<true, false>), ggrid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((prefill_kernel<false, false>), grid, dim3(256), 0, st, a);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(Q3A_ELAUNCH, "%s: launch failed: %s", who, hipGetErrorString(e));
  return Q3A_OK;
}

// Pool-side checks shared by the append entry points.
static int check_pool(const void* k_cache, const void* v_cache, int64_t kv_stride_page, int64_t kv_stride_tok,
                      int64_t kv_stride_head, int num_pages, int page_size, const int32_t* block_table,
                      int max_pages_per_seq, int head_dim, const char* who) {
  if (!k_cache || !v_cache || !block_table) return fail(Q3A_EINVAL, "%s: null pointer argument", who);
  if (page_size < 16 || (page_size & (page_size - 1)) != 0)
    return fail(Q3A_EINVAL, "%s: page_size %d must be a power of two >= 16", who, page_size);
  if (num_pages <= 0 || max_pages_per_seq <= 0)
    return fail(Q3A_EINVAL, "%s: num_pages and max_pages_per_seq must be > 0", who);
  if (((uintptr_t)k_cache | (uintptr_t)v_cache) % 16 != 0)
    return fail(Q3A_EINVAL, "%s: k_cache/v_cache must be 16-byte aligned", who);
  if ((kv_stride_page | kv_stride_tok | kv_stride_head) % 8 != 0 || kv_stride_tok < head_dim || kv_stride_head < 0 ||
      kv_stride_page < (int64_t)page_size * kv_stride_tok)
    return fail(Q3A_EINVAL, "%s: cache strides (page %lld, token %lld, head %lld) unsupported", who,
                (long long)kv_stride_page, (long long)kv_stride_tok, (long long)kv_stride_head);
  return Q3A_OK;
}

static void set_pool(PrefillArgs& a, void* k_cache, void* v_cache, int64_t kv_stride_page, int64_t kv_stride_tok,
                     int64_t kv_stride_head, int num_pages, int page_size, const int32_t* block_table,
                     int64_t bt_stride_b, int max_pages_per_seq, int first_row) {
  a.pk = static_cast<uint16_t*>(k_cache);
  a.pv = static_cast<uint16_t*>(v_cache);
  a.p_sp = kv_stride_page;
  a.p_st = kv_stride_tok;
  a.p_sh = kv_stride_head;
  a.pbt = block_table;
  a.pbt_sb = bt_stride_b;
  a.p_pages = num_pages;
  a.p_shift = 0;
  while ((1 << a.p_shift) < page_size) ++a.p_shift;
  a.p_max_pages = max_pages_per_seq;
  a.p_first = first_row;
}

extern "C" int q3a_prefill(const void* q, int64_t q_stride_t, int64_t q_stride_h, const int32_t* cu_seqlens_q,
                           const void* k, int64_t k_stride_page, int64_t k_stride_tok, int64_t k_stride_head,
                           const void* v, int64_t v_stride_page, int64_t v_stride_tok, int64_t v_stride_head,
                           int num_pages, int page_size, const int32_t* block_table, int64_t bt_stride_b,
                           int max_pages_per_seq, const int32_t* cu_seqlens_k, void* out, int64_t o_stride_t,
                           int64_t o_stride_h, int num_seqs, int max_seqlen_q, int num_q_heads, int num_kv_heads,
                           int head_dim, float softmax_scale, int causal, void* stream) {
  if (num_seqs < 0 || max_seqlen_q < 0) return fail(Q3A_EINVAL, "prefill: negative num_seqs/max_seqlen_q");
  if (num_seqs == 0 || max_seqlen_q == 0) return Q3A_OK;
  if (!cu_seqlens_q || !cu_seqlens_k) return fail(Q3A_EINVAL, "prefill: null pointer argument");
  int rc = check_common(q, k, v, out, q_stride_t, q_stride_h, k_stride_tok, k_stride_head, v_stride_tok,
                        v_stride_head, o_stride_t, o_stride_h, num_q_heads, num_kv_heads, head_dim, "prefill");
  if (rc != Q3A_OK) return rc;
  if (block_table != nullptr) {
    if (page_size <= 0 || num_pages <= 0 || max_pages_per_seq <= 0)
      return fail(Q3A_EINVAL, "prefill: paged K/V needs page_size, num_pages and max_pages_per_seq > 0");
    if ((k_stride_page | v_stride_page) % 8 != 0)
      return fail(Q3A_EINVAL, "prefill: page strides must be multiples of 8 elements");
    if (page_size < 16 || (page_size & (page_size - 1)) != 0)
      return fail(Q3A_EINVAL, "prefill: page_size %d must be a power of two >= 16", page_size);
  }

  PrefillArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.q_st = q_stride_t;
  a.q_sh = q_stride_h;
  a.cu_q = cu_seqlens_q;
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.k_sp = k_stride_page;
  a.k_st = k_stride_tok;
  a.k_sh = k_stride_head;
  a.v_sp = v_stride_page;
  a.v_st = v_stride_tok;
  a.v_sh = v_stride_head;
  a.num_pages = num_pages;
  a.page_size = page_size;
  a.page_shift = 0;
  while (block_table != nullptr && (1 << a.page_shift) < page_size) ++a.page_shift;
  a.bt = block_table;
  a.bt_sb = bt_stride_b;
  a.max_pages = max_pages_per_seq;
  a.cu_k = cu_seqlens_k;
  a.out = static_cast<uint16_t*>(out);
  a.o_st = o_stride_t;
  a.o_sh = o_stride_h;
  a.causal = causal ? 1 : 0;
  a.scale_log2 = softmax_scale * kLog2e;
  a.hkv = num_kv_heads;
  return launch(a, num_seqs, max_seqlen_q, stream, "prefill");
}

// q3a_prefill_append with the caller's extra fields in a (the norm/rope-q form's weight and cos/sin tables).
static int prefill_append_impl(PrefillArgs& a, const void* q, int64_t q_stride_t, int64_t q_stride_h,
                               const int32_t* cu_seqlens_q, const void* k, int64_t k_stride_tok, int64_t k_stride_head,
                               const void* v, int64_t v_stride_tok, int64_t v_stride_head, const int32_t* cu_seqlens_k,
                               void* k_cache, void* v_cache, int64_t kv_stride_page, int64_t kv_stride_tok,
                               int64_t kv_stride_head, int num_pages, int page_size, const int32_t* block_table,
                               int64_t bt_stride_b, int max_pages_per_seq, void* out, int64_t o_stride_t,
                               int64_t o_stride_h, int num_seqs, int max_seqlen_q, int num_q_heads, int num_kv_heads,
                               int head_dim, float softmax_scale, int causal, void* stream, const char* who) {
  if (num_seqs < 0 || max_seqlen_q < 0) return fail(Q3A_EINVAL, "%s: negative num_seqs/max_seqlen_q", who);
  if (num_seqs == 0 || max_seqlen_q == 0) return Q3A_OK;
  if (!cu_seqlens_q || !cu_seqlens_k) return fail(Q3A_EINVAL, "%s: null pointer argument", who);
  int rc = check_common(q, k, v, out, q_stride_t, q_stride_h, k_stride_tok, k_stride_head, v_stride_tok,
                        v_stride_head, o_stride_t, o_stride_h, num_q_heads, num_kv_heads, head_dim, who);
  if (rc != Q3A_OK) return rc;
  rc = check_pool(k_cache, v_cache, kv_stride_page, kv_stride_tok, kv_stride_head, num_pages, page_size, block_table,
                  max_pages_per_seq, head_dim, who);
  if (rc != Q3A_OK) return rc;

  a.q = static_cast<const uint16_t*>(q);
  a.q_st = q_stride_t;
  a.q_sh = q_stride_h;
  a.cu_q = cu_seqlens_q;
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.k_st = k_stride_tok;
  a.k_sh = k_stride_head;
  a.v_st = v_stride_tok;
  a.v_sh = v_stride_head;
  a.bt = nullptr;                  // attention reads the packed k/v
  a.cu_k = cu_seqlens_k;
  a.out = static_cast<uint16_t*>(out);
  a.o_st = o_stride_t;
  a.o_sh = o_stride_h;
  a.causal = causal ? 1 : 0;
  a.scale_log2 = softmax_scale * kLog2e;
  a.hkv = num_kv_heads;
  set_pool(a, k_cache, v_cache, kv_stride_page, kv_stride_tok, kv_stride_head, num_pages, page_size, block_table,
           bt_stride_b, max_pages_per_seq, -1);
  if (a.qn != nullptr) {
    // The norm/rope-q form reads K from the pool, where the producer pass stored the normalised rows (V packed).
    a.k = static_cast<const uint16_t*>(k_cache);
    a.k_sp = kv_stride_page;
    a.k_st = kv_stride_tok;
    a.k_sh = kv_stride_head;
    a.bt = block_table;
    a.bt_sb = bt_stride_b;
    a.max_pages = max_pages_per_seq;
    a.num_pages = num_pages;
    a.page_size = page_size;
    a.page_shift = a.p_shift;
  }
  return launch(a, num_seqs, max_seqlen_q, stream, who);
}

extern "C" int q3a_prefill_append(const void* q, int64_t q_stride_t, int64_t q_stride_h, const int32_t* cu_seqlens_q,
                                  const void* k, int64_t k_stride_tok, int64_t k_stride_head, const void* v,
                                  int64_t v_stride_tok, int64_t v_stride_head, const int32_t* cu_seqlens_k,
                                  void* k_cache, void* v_cache, int64_t kv_stride_page, int64_t kv_stride_tok,
                                  int64_t kv_stride_head, int num_pages, int page_size, const int32_t* block_table,
                                  int64_t bt_stride_b, int max_pages_per_seq, void* out, int64_t o_stride_t,
                                  int64_t o_stride_h, int num_seqs, int max_seqlen_q, int num_q_heads, int num_kv_heads,
                                  int head_dim, float softmax_scale, int causal, void* stream) {
  PrefillArgs a{};
  return prefill_append_impl(a, q, q_stride_t, q_stride_h, cu_seqlens_q, k, k_stride_tok, k_stride_head, v,
                             v_stride_tok, v_stride_head, cu_seqlens_k, k_cache, v_cache, kv_stride_page, kv_stride_tok,
                             kv_stride_head, num_pages, page_size, block_table, bt_stride_b, max_pages_per_seq, out,
                             o_stride_t, o_stride_h, num_seqs, max_seqlen_q, num_q_heads, num_kv_heads, head_dim,
                             softmax_scale, causal, stream, "prefill_append");
}

// The dense form with an optional pool write (a.pk set by the caller).
static int prefill_dense_impl(PrefillArgs& a, const void* q, int64_t q_stride_s, int64_t q_stride_t,
                              int64_t q_stride_h, const void* k, int64_t k_stride_s, int64_t k_stride_t,
                              int64_t k_stride_h, const void* v, int64_t v_stride_s, int64_t v_stride_t,
                              int64_t v_stride_h, void* out, int64_t o_stride_s, int64_t o_stride_t,
                              int64_t o_stride_h, int num_seqs, int seqlen_q, int seqlen_k, int num_q_heads,
                              int num_kv_heads, int head_dim, float softmax_scale, int causal, void* stream,
                              const char* who) {
  int rc = check_common(q, k, v, out, q_stride_t, q_stride_h, k_stride_t, k_stride_h, v_stride_t, v_stride_h,
                        o_stride_t, o_stride_h, num_q_heads, num_kv_heads, head_dim, who);
  if (rc != Q3A_OK) return rc;
  if ((q_stride_s | k_stride_s | v_stride_s | o_stride_s) % 8 != 0 || q_stride_s < 0 || k_stride_s < 0 ||
      v_stride_s < 0 || o_stride_s < 0)
    return fail(Q3A_EINVAL, "%s: sequence strides must be non-negative multiples of 8 elements", who);

  a.q = static_cast<const uint16_t*>(q);
  a.q_st = q_stride_t;
  a.q_sh = q_stride_h;
  a.q_ss = q_stride_s;
  a.cu_q = nullptr;
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.k_st = k_stride_t;
  a.k_sh = k_stride_h;
  a.k_ss = k_stride_s;
  a.v_st = v_stride_t;
  a.v_sh = v_stride_h;
  a.v_ss = v_stride_s;
  a.bt = nullptr;
  a.cu_k = nullptr;
  a.out = static_cast<uint16_t*>(out);
  a.o_st = o_stride_t;
  a.o_sh = o_stride_h;
  a.o_ss = o_stride_s;
  a.dense_lq = seqlen_q;
  a.dense_lk = seqlen_k;
  a.causal = causal ? 1 : 0;
  a.scale_log2 = softmax_scale * kLog2e;
  a.hkv = num_kv_heads;
  if (seqlen_k <= kResMaxTiles * kKT) {
    // Short key range: the whole K/V range of a (sequence, KV head) in LDS, one wave per 16 tokens and query head.
    const int ntiles = seqlen_k > 0 ? (seqlen_k + kKT - 1) / kKT : 0;
    const int ngroups = (seqlen_q + kResQ - 1) / kResQ;
    const int nblk = (ngroups + kResMaxGroups - 1) / kResMaxGroups;
    const int waves = ngroups < kResMaxGroups ? ngroups : kResMaxGroups;
    if ((int64_t)num_seqs * num_kv_heads > 0x7fffffff || 2 * nblk > 65535)
      return fail(Q3A_EINVAL, "%s: grid too large (%d seqs x %d KV heads x %d query blocks)", who, num_seqs,
                  num_kv_heads, nblk);
    // The append form is its own instantiation: its store loop changes the plain kernel's schedule (5.36 -> 5.87 us
    // on the admission shape when shared).  With fewer than 16 query groups it runs one extra wave for the stores.
    if (a.kn != nullptr)
      hipLaunchKernelGGL((prefill_resident_kernel<true, true>), dim3(num_seqs * num_kv_heads, 1, 2 * nblk),
                         dim3(64 * (waves + (ngroups < kResMaxGroups ? 1 : 0))), 0, static_cast<hipStream_t>(stream),
                         a, ntiles);
    else if (a.pk != nullptr)
      hipLaunchKernelGGL(prefill_resident_kernel<true>, dim3(num_seqs * num_kv_heads, 1, 2 * nblk),
                         dim3(64 * (waves + (ngroups < kResMaxGroups ? 1 : 0))), 0, static_cast<hipStream_t>(stream),
                         a, ntiles);
    else
      hipLaunchKernelGGL(prefill_resident_kernel<false>, dim3(num_seqs * num_kv_heads, 1, 2 * nblk), dim3(64 * waves),
                         0, static_cast<hipStream_t>(stream), a, ntiles);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(Q3A_ELAUNCH, "%s: launch failed: %s", who, hipGetErrorString(e));
    return Q3A_OK;
  }
  return launch(a, num_seqs, seqlen_q, stream, who);
}

extern "C" int q3a_prefill_dense(const void* q, int64_t q_stride_s, int64_t q_stride_t, int64_t q_stride_h,
                                 const void* k, int64_t k_stride_s, int64_t k_stride_t, int64_t k_stride_h,
                                 const void* v, int64_t v_stride_s, int64_t v_stride_t, int64_t v_stride_h,
                                 void* out, int64_t o_stride_s, int64_t o_stride_t, int64_t o_stride_h, int num_seqs,
                                 int seqlen_q, int seqlen_k, int num_q_heads, int num_kv_heads, int head_dim,
                                 float softmax_scale, int causal, void* stream) {
  if (num_seqs < 0 || seqlen_q < 0 || seqlen_k < 0)
    return fail(Q3A_EINVAL, "prefill_dense: negative num_seqs/seqlen_q/seqlen_k");
  if (num_seqs == 0 || seqlen_q == 0) return Q3A_OK;
  PrefillArgs a{};
  return prefill_dense_impl(a, q, q_stride_s, q_stride_t, q_stride_h, k, k_stride_s, k_stride_t, k_stride_h, v,
                            v_stride_s, v_stride_t, v_stride_h, out, o_stride_s, o_stride_t, o_stride_h, num_seqs,
                            seqlen_q, seqlen_k, num_q_heads, num_kv_heads, head_dim, softmax_scale, causal, stream,
                            "prefill_dense");
}

extern "C" int q3a_prefill_dense_append(const void* q, int64_t q_stride_s, int64_t q_stride_t, int64_t q_stride_h,
                                        const void* k, int64_t k_stride_s, int64_t k_stride_t, int64_t k_stride_h,
                                        const void* v, int64_t v_stride_s, int64_t v_stride_t, int64_t v_stride_h,
                                        void* k_cache, void* v_cache, int64_t kv_stride_page, int64_t kv_stride_tok,
                                        int64_t kv_stride_head, int num_pages, int page_size,
                                        const int32_t* block_table, int64_t bt_stride_b, int max_pages_per_seq,
                                        int first_row, void* out, int64_t o_stride_s, int64_t o_stride_t,
                                        int64_t o_stride_h, int num_seqs, int seqlen_q, int seqlen_k, int num_q_heads,
                                        int num_kv_heads, int head_dim, float softmax_scale, int causal,
                                        void* stream) {
  const char* who = "prefill_dense_append";
  if (num_seqs < 0 || seqlen_q < 0 || seqlen_k < 0)
    return fail(Q3A_EINVAL, "%s: negative num_seqs/seqlen_q/seqlen_k", who);
  if (first_row < 0 || first_row > std::max(0, seqlen_k - seqlen_q))
    return fail(Q3A_EINVAL, "%s: first_row %d must lie in [0, max(0, seqlen_k - seqlen_q) = %d]", who, first_row,
                std::max(0, seqlen_k - seqlen_q));
  if (num_seqs == 0 || seqlen_q == 0) return Q3A_OK;
  int rc = check_pool(k_cache, v_cache, kv_stride_page, kv_stride_tok, kv_stride_head, num_pages, page_size,
                      block_table, max_pages_per_seq, head_dim, who);
  if (rc != Q3A_OK) return rc;
  PrefillArgs a{};
  set_pool(a, k_cache, v_cache, kv_stride_page, kv_stride_tok, kv_stride_head, num_pages, page_size, block_table,
           bt_stride_b, max_pages_per_seq, first_row);
  return prefill_dense_impl(a, q, q_stride_s, q_stride_t, q_stride_h, k, k_stride_s, k_stride_t, k_stride_h, v,
                            v_stride_s, v_stride_t, v_stride_h, out, o_stride_s, o_stride_t, o_stride_h, num_seqs,
                            seqlen_q, seqlen_k, num_q_heads, num_kv_heads, head_dim, softmax_scale, causal, stream,
                            who);
}

// The producer launch shared by the rope entry points (the job block ends in p must be set).
static int launch_prep(const AdmitPrepArgs& p, void* stream, const char* who) {
  // Every job block is a multiple of Hkv rows; with Hkv a multiple of 4 each wave's four rows are of one kind.
  if (p.Hkv % 4 != 0) return fail(Q3A_EINVAL, "%s: num_kv_heads %d must be a multiple of 4", who, p.Hkv);
  if (p.jall >= ((int64_t)1 << 31)) return fail(Q3A_EINVAL, "%s: grid too large (%lld row jobs)", who, (long long)p.jall);
  const int64_t waves = p.jall / 4;
  const int64_t blocks = (waves + 3) / 4;
  if (blocks == 0) return Q3A_OK;
  hipLaunchKernelGGL(admit_prep_kernel, dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream), p);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(Q3A_ELAUNCH, "%s: producer launch failed: %s", who, hipGetErrorString(e));
  return Q3A_OK;
}

static int launch_prompt_k(const AdmitPrepArgs& p, void* stream, const char* who) {
  if (p.Hkv % 4 != 0) return fail(Q3A_EINVAL, "%s: num_kv_heads %d must be a multiple of 4", who, p.Hkv);
  const int64_t groups = (int64_t)p.R * (p.Hkv / 4);
  if (groups >= ((int64_t)1 << 31) - 64) return fail(Q3A_EINVAL, "%s: grid too large (%lld row groups)", who, (long long)groups);
  const int64_t waves = (groups + kPromptKGroups - 1) / kPromptKGroups;
  const int64_t blocks = (waves + 3) / 4;
  if (blocks == 0) return Q3A_OK;
  hipLaunchKernelGGL(prompt_k_kernel, dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream), p);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(Q3A_ELAUNCH, "%s: producer launch failed: %s", who, hipGetErrorString(e));
  return Q3A_OK;
}

// Workspace of q3a_prefill_dense_append_rope: the normalised q [S, R, Hq, D] and the dense K, V [S, P + R, Hkv, D],
// each part 256-byte aligned.
static size_t admit_ws_part(int64_t elems) { return (size_t)((elems * 2 + 255) / 256 * 256); }

extern "C" size_t q3a_prefill_dense_append_rope_workspace_bytes(int num_seqs, int seqlen_q, int prefix_len,
                                                                int num_q_heads, int num_kv_heads, int head_dim) {
  if (num_seqs <= 0 || seqlen_q <= 0 || prefix_len < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0)
    return 0;
  const int64_t n = (int64_t)prefix_len + seqlen_q;
  return admit_ws_part((int64_t)num_seqs * seqlen_q * num_q_heads * head_dim) +
         2 * admit_ws_part((int64_t)num_seqs * n * num_kv_heads * head_dim);
}

extern "C" int q3a_prefill_dense_append_rope(
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
    int head_dim, float softmax_scale, int causal, void* stream) {
  const char* who = "prefill_dense_append_rope";
  if (num_seqs < 0 || seqlen_q < 0 || prefix_len < 0)
    return fail(Q3A_EINVAL, "%s: negative num_seqs/seqlen_q/prefix_len", who);
  if (first_row < 0 || first_row > prefix_len)
    return fail(Q3A_EINVAL, "%s: first_row %d must lie in [0, prefix_len = %d]", who, first_row, prefix_len);
  if (num_seqs == 0 || seqlen_q == 0) return Q3A_OK;
  if (head_dim != kD) return fail(Q3A_EINVAL, "%s: head_dim %d unsupported (need %d)", who, head_dim, kD);
  if (num_kv_heads < 1 || num_q_heads != kG * num_kv_heads)
    return fail(Q3A_EINVAL, "%s: num_q_heads %d must be %d * num_kv_heads %d", who, num_q_heads, kG, num_kv_heads);
  if (num_kv_heads % 4 != 0) return fail(Q3A_EINVAL, "%s: num_kv_heads %d must be a multiple of 4", who, num_kv_heads);
  if (!q || !k || !v || !q_norm_w || !k_norm_w || !cos || !sin || !out || !workspace ||
      (prefix_len > 0 && (!prefix_k || !prefix_v)))
    return fail(Q3A_EINVAL, "%s: null pointer argument", who);
  const uintptr_t align = (uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)prefix_k | (uintptr_t)prefix_v |
                          (uintptr_t)q_norm_w | (uintptr_t)k_norm_w | (uintptr_t)cos | (uintptr_t)sin |
                          (uintptr_t)workspace;
  if (align % 16 != 0) return fail(Q3A_EINVAL, "%s: tensors and the workspace must be 16-byte aligned", who);
  if ((q_stride_s | q_stride_t | q_stride_h | k_stride_s | k_stride_t | k_stride_h | v_stride_s | v_stride_t |
       v_stride_h | pk_stride_s | pk_stride_t | pk_stride_h | pv_stride_s | pv_stride_t | pv_stride_h | rope_stride_t) %
          8 != 0 ||
      q_stride_s < 0 || q_stride_t < 0 || q_stride_h < 0 || k_stride_s < 0 || k_stride_t < 0 || k_stride_h < 0 ||
      v_stride_s < 0 || v_stride_t < 0 || v_stride_h < 0 || pk_stride_s < 0 || pk_stride_t < 0 || pk_stride_h < 0 ||
      pv_stride_s < 0 || pv_stride_t < 0 || pv_stride_h < 0 || rope_stride_t < 0)
    return fail(Q3A_EINVAL, "%s: strides must be non-negative multiples of 8 elements", who);
  if (prefix_len > 0 && num_prefixes < 1) return fail(Q3A_EINVAL, "%s: num_prefixes must be >= 1", who);
  // The short-key kernel addresses a 16-row group of the prefix bank through one buffer descriptor with a 32-bit
  // extent ((15 * token stride + head_dim) * 2 bytes), the bound k and v get in check_common.
  const int64_t lim = (int64_t)1 << 26;
  if (prefix_len > 0 && (pk_stride_t < head_dim || pk_stride_t > lim || pv_stride_t < head_dim || pv_stride_t > lim))
    return fail(Q3A_EINVAL, "%s: prefix token strides %lld/%lld must be in [head_dim, 2^26]", who,
                (long long)pk_stride_t, (long long)pv_stride_t);
  const size_t need = q3a_prefill_dense_append_rope_workspace_bytes(num_seqs, seqlen_q, prefix_len, num_q_heads,
                                                                    num_kv_heads, head_dim);
  if (workspace_bytes < need)
    return fail(Q3A_EINVAL, "%s: workspace of %zu bytes, need %zu", who, workspace_bytes, need);
  int rc = check_pool(k_cache, v_cache, kv_stride_page, kv_stride_tok, kv_stride_head, num_pages, page_size,
                      block_table, max_pages_per_seq, head_dim, who);
  if (rc != Q3A_OK) return rc;

  const int n = prefix_len + seqlen_q;
  const int64_t S = num_seqs;
  if (n <= kResMaxTiles * kKT && (seqlen_q + kResQ - 1) / kResQ + 1 <= kResRopeWaves) {
    // Short key range (the admission shape): one launch.  The resident kernel copies the prefix rows from the bank
    // and the new rows from k/v, normalises and rotates the new K rows in LDS and q in registers, then stores the
    // pool rows and attends; the workspace is not used.
    PrefillArgs a{};
    set_pool(a, k_cache, v_cache, kv_stride_page, kv_stride_tok, kv_stride_head, num_pages, page_size, block_table,
             bt_stride_b, max_pages_per_seq, first_row);
    a.qn = static_cast<const uint16_t*>(q_norm_w);
    a.kn = static_cast<const uint16_t*>(k_norm_w);
    a.rcos = static_cast<const uint16_t*>(cos);
    a.rsin = static_cast<const uint16_t*>(sin);
    a.rs_st = rope_stride_t;
    a.eps = eps;
    a.pfk = static_cast<const uint16_t*>(prefix_k);
    a.pfv = static_cast<const uint16_t*>(prefix_v);
    a.pfk_ss = pk_stride_s; a.pfk_st = pk_stride_t; a.pfk_sh = pk_stride_h;
    a.pfv_ss = pv_stride_s; a.pfv_st = pv_stride_t; a.pfv_sh = pv_stride_h;
    a.pidx = prefix_index;
    a.npre = prefix_index != nullptr ? num_prefixes : S;
    a.P = prefix_len;
    return prefill_dense_impl(a, q, q_stride_s, q_stride_t, q_stride_h, k, k_stride_s, k_stride_t, k_stride_h, v,
                              v_stride_s, v_stride_t, v_stride_h, out, o_stride_s, o_stride_t, o_stride_h, num_seqs,
                              seqlen_q, n, num_q_heads, num_kv_heads, head_dim, softmax_scale, causal, stream, who);
  }
  AdmitPrepArgs p{};
  p.q = static_cast<const uint16_t*>(q);
  p.q_ss = q_stride_s; p.q_st = q_stride_t; p.q_sh = q_stride_h;
  p.k = static_cast<const uint16_t*>(k);
  p.k_ss = k_stride_s; p.k_st = k_stride_t; p.k_sh = k_stride_h;
  p.v = static_cast<const uint16_t*>(v);
  p.v_ss = v_stride_s; p.v_st = v_stride_t; p.v_sh = v_stride_h;
  p.pk = static_cast<const uint16_t*>(prefix_k);
  p.pk_ss = pk_stride_s; p.pk_st = pk_stride_t; p.pk_sh = pk_stride_h;
  p.pv = static_cast<const uint16_t*>(prefix_v);
  p.pv_ss = pv_stride_s; p.pv_st = pv_stride_t; p.pv_sh = pv_stride_h;
  p.pidx = prefix_index;
  p.npre = prefix_index != nullptr ? num_prefixes : S;
  p.qn = static_cast<const uint16_t*>(q_norm_w);
  p.kn = static_cast<const uint16_t*>(k_norm_w);
  p.cs = static_cast<const uint16_t*>(cos);
  p.sn = static_cast<const uint16_t*>(sin);
  p.cs_st = rope_stride_t;
  p.eps = eps;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  p.qo = reinterpret_cast<uint16_t*>(ws);
  p.ko = reinterpret_cast<uint16_t*>(ws + admit_ws_part(S * seqlen_q * num_q_heads * kD));
  p.vo = reinterpret_cast<uint16_t*>(reinterpret_cast<uint8_t*>(p.ko) + admit_ws_part(S * n * num_kv_heads * kD));
  p.R = seqlen_q;
  p.P = prefix_len;
  p.Hq = num_q_heads;
  p.Hkv = num_kv_heads;
  p.jq = S * seqlen_q * num_q_heads;
  p.jk = p.jq + S * seqlen_q * num_kv_heads;
  p.jv = p.jk + S * seqlen_q * num_kv_heads;
  p.jp = p.jv + S * prefix_len * num_kv_heads;
  p.jall = p.jp + S * prefix_len * num_kv_heads;
  rc = launch_prep(p, stream, who);
  if (rc != Q3A_OK) return rc;

  PrefillArgs a{};
  set_pool(a, k_cache, v_cache, kv_stride_page, kv_stride_tok, kv_stride_head, num_pages, page_size, block_table,
           bt_stride_b, max_pages_per_seq, first_row);
  return prefill_dense_impl(a, p.qo, (int64_t)seqlen_q * num_q_heads * kD, (int64_t)num_q_heads * kD, kD, p.ko,
                            (int64_t)n * num_kv_heads * kD, (int64_t)num_kv_heads * kD, kD, p.vo,
                            (int64_t)n * num_kv_heads * kD, (int64_t)num_kv_heads * kD, kD, out, o_stride_s, o_stride_t,
                            o_stride_h, num_seqs, seqlen_q, n, num_q_heads, num_kv_heads, head_dim, softmax_scale,
                            causal, stream, who);
}

// Workspace of q3a_prefill_append_rope when not causal: the normalised q [T, Hq, D] and k [T, Hkv, D] (v is read
// where it is).  The causal form uses none.
extern "C" size_t q3a_prefill_append_rope_workspace_bytes(int total_tokens, int num_q_heads, int num_kv_heads,
                                                          int head_dim) {
  if (total_tokens <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0) return 0;
  return admit_ws_part((int64_t)total_tokens * num_q_heads * head_dim) +
         admit_ws_part((int64_t)total_tokens * num_kv_heads * head_dim);
}

extern "C" int q3a_prefill_append_rope(
    const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k, int64_t k_stride_t, int64_t k_stride_h,
    const void* v, int64_t v_stride_t, int64_t v_stride_h, const void* q_norm_w, const void* k_norm_w,
    const void* cos, const void* sin, int64_t rope_stride_t, float eps, const int32_t* cu_seqlens, void* k_cache,
    void* v_cache, int64_t kv_stride_page, int64_t kv_stride_tok, int64_t kv_stride_head, int num_pages,
    int page_size, const int32_t* block_table, int64_t bt_stride_b, int max_pages_per_seq, void* out,
    int64_t o_stride_t, int64_t o_stride_h, void* workspace, size_t workspace_bytes, int num_seqs, int total_tokens,
    int max_seqlen, int num_q_heads, int num_kv_heads, int head_dim, float softmax_scale, int causal, void* stream) {
  const char* who = "prefill_append_rope";
  if (num_seqs < 0 || total_tokens < 0 || max_seqlen < 0)
    return fail(Q3A_EINVAL, "%s: negative num_seqs/total_tokens/max_seqlen", who);
  if (num_seqs == 0 || total_tokens == 0 || max_seqlen == 0) return Q3A_OK;
  if (head_dim != kD) return fail(Q3A_EINVAL, "%s: head_dim %d unsupported (need %d)", who, head_dim, kD);
  if (num_kv_heads < 1 || num_q_heads != kG * num_kv_heads)
    return fail(Q3A_EINVAL, "%s: num_q_heads %d must be %d * num_kv_heads %d", who, num_q_heads, kG, num_kv_heads);
  // Causal, nothing goes through the workspace (k rows straight into the pool, q normalised in the attention).
  const bool uses_ws = causal == 0;
  if (!q || !k || !v || !q_norm_w || !k_norm_w || !cos || !sin || !cu_seqlens || !out || (uses_ws && !workspace))
    return fail(Q3A_EINVAL, "%s: null pointer argument", who);
  const uintptr_t align = (uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)q_norm_w | (uintptr_t)k_norm_w |
                          (uintptr_t)cos | (uintptr_t)sin | (uses_ws ? (uintptr_t)workspace : 0);
  if (align % 16 != 0) return fail(Q3A_EINVAL, "%s: tensors and the workspace must be 16-byte aligned", who);
  if ((q_stride_t | q_stride_h | k_stride_t | k_stride_h | v_stride_t | v_stride_h | rope_stride_t) % 8 != 0 ||
      q_stride_t < 0 || q_stride_h < 0 || k_stride_t < 0 || k_stride_h < 0 || v_stride_t < 0 || v_stride_h < 0 ||
      rope_stride_t < 0)
    return fail(Q3A_EINVAL, "%s: strides must be non-negative multiples of 8 elements", who);
  const size_t need = q3a_prefill_append_rope_workspace_bytes(total_tokens, num_q_heads, num_kv_heads, head_dim);
  if (uses_ws && workspace_bytes < need)
    return fail(Q3A_EINVAL, "%s: workspace of %zu bytes, need %zu", who, workspace_bytes, need);
  int rc = check_pool(k_cache, v_cache, kv_stride_page, kv_stride_tok, kv_stride_head, num_pages, page_size,
                      block_table, max_pages_per_seq, head_dim, who);
  if (rc != Q3A_OK) return rc;
  // The attention's own checks, before the producer pass writes anything (K read back from the pool).
  rc = check_common(q, k_cache, v, out, q_stride_t, q_stride_h, kv_stride_tok, kv_stride_head, v_stride_t, v_stride_h,
                    o_stride_t, o_stride_h, num_q_heads, num_kv_heads, head_dim, who);
  if (rc != Q3A_OK) return rc;

  // The producers over all T tokens as one sequence with no prefix: token t takes rope row t; no V rows (the
  // attention reads v where it is).  Causal: k rows only, stored straight into the pool at each token's position in
  // its sequence (cu_seqlens), where the attention kernel reads them back as paged K; it normalises and rotates q
  // as it loads it and stores only the V rows into the pool (from the last tiles it streams).  Otherwise q and k
  // rows into the workspace, and the plain append form on them.
  const int64_t T = total_tokens;
  const bool q_in_kernel = causal != 0;
  AdmitPrepArgs p{};
  p.q = static_cast<const uint16_t*>(q);
  p.q_st = q_stride_t; p.q_sh = q_stride_h;
  p.k = static_cast<const uint16_t*>(k);
  p.k_st = k_stride_t; p.k_sh = k_stride_h;
  p.v = static_cast<const uint16_t*>(v);
  p.v_st = v_stride_t; p.v_sh = v_stride_h;
  p.qn = static_cast<const uint16_t*>(q_norm_w);
  p.kn = static_cast<const uint16_t*>(k_norm_w);
  p.cs = static_cast<const uint16_t*>(cos);
  p.sn = static_cast<const uint16_t*>(sin);
  p.cs_st = rope_stride_t;
  p.eps = eps;
  p.R = total_tokens;
  p.P = 0;
  p.Hq = num_q_heads;
  p.Hkv = num_kv_heads;
  if (q_in_kernel) {
    p.cu = cu_seqlens;
    p.nseq = num_seqs;
    p.kpool = static_cast<uint16_t*>(k_cache);
    p.p_sp = kv_stride_page;
    p.p_st = kv_stride_tok;
    p.p_sh = kv_stride_head;
    p.pbt = block_table;
    p.pbt_sb = bt_stride_b;
    p.p_pages = num_pages;
    p.p_shift = 0;
    while ((1 << p.p_shift) < page_size) ++p.p_shift;
    p.p_max_pages = max_pages_per_seq;
    rc = launch_prompt_k(p, stream, who);
  } else {
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    p.qo = reinterpret_cast<uint16_t*>(ws);
    p.ko = reinterpret_cast<uint16_t*>(ws + admit_ws_part(T * num_q_heads * kD));
    p.jq = T * num_q_heads;
    p.jk = p.jq + T * num_kv_heads;
    p.jv = p.jk;
    p.jp = p.jv;
    p.jall = p.jv;
    rc = launch_prep(p, stream, who);
  }
  if (rc != Q3A_OK) return rc;
  PrefillArgs a{};
  if (q_in_kernel) {
    a.qn = p.qn;
    a.rcos = p.cs;
    a.rsin = p.sn;
    a.rs_st = rope_stride_t;
    a.eps = eps;
    return prefill_append_impl(a, q, q_stride_t, q_stride_h, cu_seqlens, k_cache, kv_stride_tok, kv_stride_head, v,
                               v_stride_t, v_stride_h, cu_seqlens, k_cache, v_cache, kv_stride_page, kv_stride_tok,
                               kv_stride_head, num_pages, page_size, block_table, bt_stride_b, max_pages_per_seq, out,
                               o_stride_t, o_stride_h, num_seqs, max_seqlen, num_q_heads, num_kv_heads, head_dim,
                               softmax_scale, causal, stream, who);
  }
  return prefill_append_impl(a, p.qo, (int64_t)num_q_heads * kD, kD, cu_seqlens, p.ko, (int64_t)num_kv_heads * kD, kD,
                             v, v_stride_t, v_stride_h, cu_seqlens, k_cache, v_cache, kv_stride_page, kv_stride_tok,
                             kv_stride_head, num_pages, page_size, block_table, bt_stride_b, max_pages_per_seq, out,
                             o_stride_t, o_stride_h, num_seqs, max_seqlen, num_q_heads, num_kv_heads, head_dim,
                             softmax_scale, causal, stream, who);
}
