// Talker prefill attention for gfx950, on MFMA.
//
// Semantics: packed variable-length causal attention.  Sequence s owns query tokens
// [cu_q[s], cu_q[s+1]) of q [T, Hq, D] and keys 0..Lk-1 with Lk = cu_k[s+1] - cu_k[s], read either
// from a packed [Tk, Hkv, D] tensor (token j at row cu_k[s] + j) or from the paged KV pool
// (token j at page block_table[s][j / page_size], offset j % page_size).  With `causal`, query i
// sees keys j <= Lk - Lq + i (bottom-right alignment).  This covers flash_attn_varlen_func at
// engine/talker.py:169 (cu_q == cu_k, fp32 form engine/talker.py:163-167), the prefix + new form
// of flash_attn_func at engine/arrivals.py:148 (fp32 form engine/arrivals.py:125-131), and both
// read from the pool after the K/V append (engine/talker.py:161-162, engine/arrivals.py:144-145).
//
// Work: one workgroup (4 waves) per (sequence, 64-query tile, KV head); wave w takes tokens 16w..16w+15 of
// the tile for BOTH query heads 2g, 2g+1 of the GQA pair, so every K or V^T operand read from LDS feeds two
// MFMAs.  Key tiles of 64 are staged in LDS (K row-major with padding, V transposed and swizzled); the next
// tile is prefetched into registers while the current one is consumed.  v_mfma_f32_16x16x32_bf16 layouts:
// A lane l = row l%16, k 8*(l/16)..+8; B lane l = column l%16, same k; C lane l = column l%16, rows
// 4*(l/16)..+4.
//   S^T = K Q^T  : A = K (rows = keys), B = Q^T (columns = this lane's query token)
//   O^T = V^T P^T: A = V^T from LDS, B = P^T taken straight from S^T's C registers
// so the softmax statistics, P and the O accumulators of a query token all live on the lanes with
// that token in column l%16; a row's max over a tile needs only two cross-lane steps.
#include "q3a_common.h"
#include "../../include/q3attn.h"

namespace q3a {
namespace {

constexpr int kD = 128;
constexpr int kG = 2;
constexpr int kQT = 64;        // query tokens per workgroup (16 per wave, both heads)
constexpr int kKT = 64;        // keys per LDS tile
constexpr int kKs = kD + 8;    // K tile row stride in LDS (bf16 elements, padded)
constexpr int kVs = kKT + 8;   // V^T tile row stride in LDS (bf16 elements, padded)

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;

struct PrefillArgs {
  const uint16_t* q;
  int64_t q_st, q_sh;
  const int32_t* cu_q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t kv_sp, kv_st, kv_sh;
  int num_pages, page_size, page_shift;  // paged: page_size is a power of two >= 16
  const int32_t* bt;  // nullptr: packed K/V
  int64_t bt_sb;
  int max_pages;
  const int32_t* cu_k;
  uint16_t* out;
  int64_t o_st, o_sh;
  int causal;
  float scale_log2;
};

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }
__device__ __forceinline__ int readlane(int v, int lane) { return __builtin_amdgcn_readlane(v, lane); }

// V^T tile swizzle: key k of dim row r is stored at column k ^ vswz(r).  It moves whole 4-key quads (bits 2-5
// of k), so 8-byte reads of 4 consecutive keys stay contiguous; with the 72-element row stride it makes both
// the transposed stores (16 rows x 4 quads per wave) and the MFMA operand reads free of LDS bank conflicts.
__device__ __forceinline__ int vswz(int r) { return (((r >> 3) & 3) << 2) ^ (((r >> 5) & 3) << 4); }

__global__ __launch_bounds__(256) void prefill_kernel(const PrefillArgs a) {
  __shared__ __align__(16) uint16_t Ks[kKT * kKs];
  __shared__ __align__(16) uint16_t Vt[kD * kVs];

  // Grid (sequence, KV head, query tile) with the query tile slowest and reversed: the tiles with the most
  // key tiles (the last ones of each sequence) dispatch first for every head, the short ones fill in last.
  const int s = blockIdx.x;
  const int g = blockIdx.y;
  const int qt = gridDim.z - 1 - blockIdx.z;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int col = lane & 15;
  const int g4 = lane >> 4;

  // The sequence's first 64 page ids depend only on s: fetch them before cu_seqlens so the first tile's
  // loads wait for one memory round trip, not two.
  const bool paged = a.bt != nullptr;
  const int64_t bt_row = (int64_t)s * a.bt_sb;
  int pwin = -1, pwin_base = 0;
  auto load_window = [&](int base) __attribute__((always_inline)) {
    pwin_base = base;
    const int i = base + lane;
    pwin = (paged && i < a.max_pages) ? a.bt[bt_row + i] : -1;
  };
  if (paged) load_window(0);

  const int q0 = a.cu_q[s];
  const int Lq = a.cu_q[s + 1] - q0;
  if (qt * kQT >= Lq) return;
  const int k0 = a.cu_k[s];
  int Lk = a.cu_k[s + 1] - k0;
  if (a.bt != nullptr) Lk = min(Lk, a.max_pages * a.page_size);
  Lk = max(Lk, 0);

  const int tq = qt * kQT + wave * 16 + col;  // this lane's query token
  const bool qvalid = tq < Lq;
  const int qpos = Lk - Lq + tq;              // last key this token may see when causal

  // Q^T of both heads as B operands of S^T = K Q^T: 4 chunks of 32 dims each.
  bf16x8_t qb[kG][4];
#pragma unroll
  for (int hh = 0; hh < kG; ++hh) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      uint4 x = make_uint4(0u, 0u, 0u, 0u);
      if (qvalid) x = ld16(a.q + (int64_t)(q0 + tq) * a.q_st + (kG * g + hh) * a.q_sh + 32 * kk + 8 * g4);
      qb[hh][kk] = as_bf16x8(x);
    }
  }

  int kend = Lk;
  if (a.causal) {
    const int last = min(Lq - 1, qt * kQT + kQT - 1);
    kend = min(Lk, Lk - Lq + last + 1);
  }
  const int ntiles = kend > 0 ? (kend + kKT - 1) / kKT : 0;
  const int jlim = a.causal ? min(Lk - 1, qpos) : Lk - 1;  // last key this lane's token sees

  // Tile loads.  A 64-key tile is 4 groups of 16 keys and a group never straddles a page (page sizes are
  // powers of two >= 16), so each group has one uniform base address: all K/V loads are raw buffer loads
  // against a descriptor covering exactly the group's valid rows of head g (rows past the sequence, and
  // groups on an invalid page, read as zeros without touching memory).  No per-lane address math.
  //   K: thread t loads key 16r + (t >> 4), dims 8 (t & 15), for r = 0..3.
  //   V: wave w loads group w: keys 16w + 4((t >> 4) & 3) + b, b = 0..3, dims 8 (t & 15): each thread
  //      holds 4 consecutive keys x 8 dims, the shape of its transposed LDS store.
  // Page ids come from a lane-wise window (lane i = table entry pwin_base + i), read with v_readlane, so
  // a tile costs one memory round trip; the window is refilled once per 64 pages.
  // Descriptor of group r of tile t given the group's page id (uniform).
  auto group_rsrc = [&](const uint16_t* base, int t, int r, int page) __attribute__((always_inline)) {
    const int j0 = t * kKT + 16 * r;
    const int nv = min(16, Lk - j0);
    bool ok = nv > 0;
    int64_t off = 0;
    if (paged) {
      ok = ok && (unsigned)page < (unsigned)a.num_pages;
      off = (int64_t)page * a.kv_sp + (int64_t)(j0 & (a.page_size - 1)) * a.kv_st;
    } else {
      off = (int64_t)(k0 + j0) * a.kv_st;
    }
    return make_rsrc(base + (ok ? off : 0) + (int64_t)g * a.kv_sh, ok ? (uint32_t)(((nv - 1) * a.kv_st + kD) * 2) : 0u);
  };

  const uint32_t k_off = (uint32_t)(((tid >> 4) * a.kv_st + 8 * (tid & 15)) * 2);
  const uint32_t v_off = (uint32_t)((4 * ((tid >> 4) & 3) * a.kv_st + 8 * (tid & 15)) * 2);
  const uint32_t tok_bytes = (uint32_t)(a.kv_st * 2);
  uint4 kr[4], vr[4];
  auto load_tile = [&](int t) __attribute__((always_inline)) {
    // All page ids first: reading the window register waits for its load, and a wait placed between the
    // K/V loads would also wait for the loads issued before it.
    int pg[4] = {0, 0, 0, 0};
    int pgv = 0;
    if (paged) {
      const int pf = (t * kKT) >> a.page_shift;
      const int pl = (t * kKT + kKT - 1) >> a.page_shift;
      if (pf < pwin_base || pl >= pwin_base + 64) load_window(pf);
#pragma unroll
      for (int r = 0; r < 4; ++r) pg[r] = readlane(pwin, ((t * kKT + 16 * r) >> a.page_shift) - pwin_base);
      pgv = readlane(pwin, ((t * kKT + 16 * wave) >> a.page_shift) - pwin_base);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) kr[r] = buffer_load16(group_rsrc(a.k, t, r, pg[r]), k_off);
    const __amdgpu_buffer_rsrc_t rv = group_rsrc(a.v, t, wave, pgv);
#pragma unroll
    for (int b = 0; b < 4; ++b) vr[b] = buffer_load16(rv, v_off + b * tok_bytes);
  };
  auto store_tile = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < 4; ++r) st16(&Ks[((tid >> 4) + 16 * r) * kKs + 8 * (tid & 15)], kr[r]);
    // V transposed: for each of this thread's 8 dims, its 4 keys as one 8-byte row segment.
    const int kq = 16 * wave + 4 * ((tid >> 4) & 3);
    const int d0 = 8 * (tid & 15);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t w0 = c == 0 ? vr[0].x : c == 1 ? vr[0].y : c == 2 ? vr[0].z : vr[0].w;
      const uint32_t w1 = c == 0 ? vr[1].x : c == 1 ? vr[1].y : c == 2 ? vr[1].z : vr[1].w;
      const uint32_t w2 = c == 0 ? vr[2].x : c == 1 ? vr[2].y : c == 2 ? vr[2].z : vr[2].w;
      const uint32_t w3 = c == 0 ? vr[3].x : c == 1 ? vr[3].y : c == 2 ? vr[3].z : vr[3].w;
      uint2 lo, hi;
      lo.x = perm_b32(w1, w0, kPermLoLo);
      lo.y = perm_b32(w3, w2, kPermLoLo);
      hi.x = perm_b32(w1, w0, kPermHiHi);
      hi.y = perm_b32(w3, w2, kPermHiHi);
      const int r0 = d0 + 2 * c;
      *reinterpret_cast<uint2*>(&Vt[r0 * kVs + (kq ^ vswz(r0))]) = lo;
      *reinterpret_cast<uint2*>(&Vt[(r0 + 1) * kVs + (kq ^ vswz(r0 + 1))]) = hi;
    }
  };

  f32x4_t acc[kG][8];
#pragma unroll
  for (int hh = 0; hh < kG; ++hh)
#pragma unroll
    for (int db = 0; db < 8; ++db) acc[hh][db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m[kG] = {kMaxSeed, kMaxSeed}, l[kG] = {0.f, 0.f};

  if (ntiles > 0) load_tile(0);
  for (int t = 0; t < ntiles; ++t) {
    __syncthreads();
    store_tile();
    __syncthreads();
    if (t + 1 < ntiles) load_tile(t + 1);

    // S^T for the tile's 4 blocks of 16 keys, both heads; each K operand is read once.
    f32x4_t st[kG][4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
      for (int hh = 0; hh < kG; ++hh) st[hh][kb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const bf16x8_t kv = as_bf16x8(ld16(&Ks[(kb * 16 + col) * kKs + 32 * kk + 8 * g4]));
#pragma unroll
        for (int hh = 0; hh < kG; ++hh)
          st[hh][kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kv, qb[hh][kk], st[hh][kb], 0, 0, 0);
      }
    }
    // Mask: key j is visible to this lane's token iff j <= jlim (= min(Lk - 1, qpos) when causal).
    // Relative to the tile and this lane's key rows that is one compare per score against `lim`.
    // Masked scores become -inf; the running max m is kept in scaled (log2) units.
    const int lim = jlim - t * kKT - 4 * g4;
    bf16x8_t pb[kG][2];
#pragma unroll
    for (int hh = 0; hh < kG; ++hh) {
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          st[hh][kb][i] = (kb * 16 + i <= lim) ? st[hh][kb][i] : -INFINITY;
          mx = fmaxf(mx, st[hh][kb][i]);
        }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      mx *= a.scale_log2;
      // Lazy rescale: keep the running max while no token's tile max exceeds it by more than 8 (log2
      // units), so p = exp2(s * scale - m) <= 256 is exact enough in bf16/fp32 and (l, acc) are rescaled
      // only when a max grows past that margin.  The first tile always sets the max.
      if (__any(mx > m[hh] + 8.f)) {
        const float mn = fmaxf(m[hh], mx);
        const float alpha = fast_exp2(m[hh] - mn);
        l[hh] *= alpha;
#pragma unroll
        for (int db = 0; db < 8; ++db) {
          acc[hh][db][0] *= alpha;
          acc[hh][db][1] *= alpha;
          acc[hh][db][2] *= alpha;
          acc[hh][db][3] *= alpha;
        }
        m[hh] = mn;
      }
      // P^T as the B operand: k slot 8*g4 + i <- key 32*s2 + 4*g4 + i, slot 8*g4 + 4 + i <- key
      // 32*s2 + 16 + 4*g4 + i (blocks 2*s2 and 2*s2+1 of this lane's C registers).
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
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
    // O^T += V^T P^T; V^T rows are dims, the same key order as the B operand; each V^T operand is
    // read once for both heads.
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const int vr_row = db * 16 + col;
      const uint16_t* vrow = &Vt[vr_row * kVs];
      const int sw = vswz(vr_row);
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const uint2 lo = *reinterpret_cast<const uint2*>(vrow + ((32 * s2 + 4 * g4) ^ sw));
        const uint2 hi = *reinterpret_cast<const uint2*>(vrow + ((32 * s2 + 4 * g4 + 16) ^ sw));
        const bf16x8_t va = as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y));
#pragma unroll
        for (int hh = 0; hh < kG; ++hh)
          acc[hh][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb[hh][s2], acc[hh][db], 0, 0, 0);
      }
    }
  }

  // The 4 lanes of a token hold partial sums over disjoint keys.
#pragma unroll
  for (int hh = 0; hh < kG; ++hh) {
    float lt = l[hh];
    lt += __shfl_xor(lt, 16);
    lt += __shfl_xor(lt, 32);
    if (qvalid) {
      const float inv = lt > 0.f ? 1.f / lt : 0.f;
      uint16_t* o = a.out + (int64_t)(q0 + tq) * a.o_st + (kG * g + hh) * a.o_sh + 4 * g4;
#pragma unroll
      for (int db = 0; db < 8; ++db) {
        uint2 w;
        w.x = pack_bf16x2(acc[hh][db][0] * inv, acc[hh][db][1] * inv);
        w.y = pack_bf16x2(acc[hh][db][2] * inv, acc[hh][db][3] * inv);
        *reinterpret_cast<uint2*>(o + db * 16) = w;
      }
    }
  }
}

}  // namespace
}  // namespace q3a

using namespace q3a;

extern "C" int q3a_prefill(const void* q, int64_t q_stride_t, int64_t q_stride_h, const int32_t* cu_seqlens_q,
                           const void* k, const void* v, int64_t kv_stride_page, int64_t kv_stride_tok,
                           int64_t kv_stride_head, int num_pages, int page_size, const int32_t* block_table,
                           int64_t bt_stride_b, int max_pages_per_seq, const int32_t* cu_seqlens_k, void* out,
                           int64_t o_stride_t, int64_t o_stride_h, int num_seqs, int max_seqlen_q,
                           int num_q_heads, int num_kv_heads, int head_dim, float softmax_scale, int causal,
                           void* stream) {
  if (num_seqs < 0 || max_seqlen_q < 0) return fail(Q3A_EINVAL, "prefill: negative num_seqs/max_seqlen_q");
  if (num_seqs == 0 || max_seqlen_q == 0) return Q3A_OK;
  if (head_dim != kD) return fail(Q3A_EINVAL, "prefill: head_dim %d unsupported (need %d)", head_dim, kD);
  if (num_kv_heads < 1 || num_q_heads != kG * num_kv_heads)
    return fail(Q3A_EINVAL, "prefill: num_q_heads %d must be %d * num_kv_heads %d", num_q_heads, kG, num_kv_heads);
  if (!q || !k || !v || !cu_seqlens_q || !cu_seqlens_k || !out) return fail(Q3A_EINVAL, "prefill: null pointer argument");
  const uintptr_t align = (uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out;
  if (align % 16 != 0) return fail(Q3A_EINVAL, "prefill: q/k/v/out must be 16-byte aligned");
  if ((q_stride_t | q_stride_h | kv_stride_tok | kv_stride_head | o_stride_t | o_stride_h) % 8 != 0)
    return fail(Q3A_EINVAL, "prefill: strides must be multiples of 8 elements (16 bytes)");
  if (kv_stride_tok < head_dim || kv_stride_head < 0 || kv_stride_tok > ((int64_t)1 << 26))
    return fail(Q3A_EINVAL, "prefill: token stride %lld must be in [head_dim, 2^26] and head stride >= 0",
                (long long)kv_stride_tok);
  if (block_table != nullptr) {
    if (page_size <= 0 || num_pages <= 0 || max_pages_per_seq <= 0)
      return fail(Q3A_EINVAL, "prefill: paged K/V needs page_size, num_pages and max_pages_per_seq > 0");
    if (kv_stride_page % 8 != 0) return fail(Q3A_EINVAL, "prefill: page stride must be a multiple of 8 elements");
    if (page_size < 16 || (page_size & (page_size - 1)) != 0)
      return fail(Q3A_EINVAL, "prefill: page_size %d must be a power of two >= 16", page_size);
  }
  const int nqt = (max_seqlen_q + kQT - 1) / kQT;
  if (num_seqs > 0x7fffffff || nqt > 65535 || num_kv_heads > 65535)
    return fail(Q3A_EINVAL, "prefill: grid too large (%d seqs x %d query tiles)", num_seqs, nqt);

  PrefillArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_st = q_stride_t;
  a.q_sh = q_stride_h;
  a.cu_q = cu_seqlens_q;
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.kv_sp = kv_stride_page;
  a.kv_st = kv_stride_tok;
  a.kv_sh = kv_stride_head;
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
  hipLaunchKernelGGL(prefill_kernel, dim3(num_seqs, num_kv_heads, nqt), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(Q3A_ELAUNCH, "prefill: launch failed: %s", hipGetErrorString(e));
  return Q3A_OK;
}
