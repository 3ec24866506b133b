// Talker paged decode attention for gfx950.
//
// Semantics (engine/talker.py:77, fp32 form engine/talker.py:82-88): for every row b and query
// head h, o[b,h] = softmax(q[b,h] . K[b, h/2, :ctx]^T * scale) . V[b, h/2, :ctx], where token t of
// row b sits in page block_table[b][t / page_size] at offset t % page_size.
//
// Work decomposition.  One workgroup = (row b, split s) with one wave per KV head.  A split is
// `split_tokens` consecutive context tokens; rows shorter than that have one split and write the
// output directly, longer rows write fp32 partials (running max m, sum l, unnormalised o) that the
// combine kernel merges.  Inside a wave, one load instruction fetches 4 tokens x 256 B of one KV
// head (lane l: token l/16, dims 8*(l%16)..+8, 16 B per lane), so a page of 16 tokens is 4
// instructions for K and 4 for V, and the 8 waves of the workgroup together sweep each 32 KiB page
// contiguously.  Both query heads of the GQA pair are applied to every K/V register the wave loads.
// Each 16-lane group keeps its own online-softmax state over the tokens it saw; the four groups
// are merged once at the end of the split.  The next 16-token tile is loaded while the current
// one is computed.
#include "q3a_common.h"
#include "../../include/q3attn.h"

namespace q3a {
namespace {

constexpr int kD = 128;
constexpr int kG = 2;                              // query heads per KV head
constexpr int kPartFloats = kG * kD + 2 * kG;      // acc[G][D], m[G], l[G]
constexpr int kMaxSplits = 64;
constexpr int kTile = 16;                          // tokens per pipeline stage

struct DecodeArgs {
  const uint16_t* q;
  int64_t q_sb, q_sh;
  const uint16_t* kc;
  const uint16_t* vc;
  int64_t kv_sp, kv_st, kv_sh;
  int num_pages, page_size;
  const int32_t* seqlens;
  const int32_t* bt;
  int64_t bt_sb;
  int max_pages;
  uint16_t* out;
  int64_t o_sb, o_sh;
  float* ws;
  int hkv, split_tokens, max_splits;
  float scale_log2;
};

struct KVTile {
  uint4 k[4];
  uint4 v[4];
};

__device__ __forceinline__ int row_ctx(const DecodeArgs& a, int b) {
  const int c = a.seqlens[b];
  const int cap = a.max_pages * a.page_size;
  return c < 0 ? 0 : (c > cap ? cap : c);
}

// Loads the 16-token tile starting at context token t (t % 16 == 0) for KV head g.  Tokens at or
// past t1 and tokens of an out-of-range page are not read and come back as zeros.
__device__ __forceinline__ bool load_tile(const DecodeArgs& a, int b, int g, int grp, int dl, int t,
                                          int t1, KVTile& T) {
  const int pidx = t / a.page_size;
  const int off = t - pidx * a.page_size;
  const int page = a.bt[(int64_t)b * a.bt_sb + pidx];
  const bool page_ok = (unsigned)page < (unsigned)a.num_pages;
  const int64_t base = (int64_t)page * a.kv_sp + (int64_t)g * a.kv_sh + dl;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int tok = 4 * i + grp;
    if (page_ok && t + tok < t1) {
      const int64_t o = base + (int64_t)(off + tok) * a.kv_st;
      T.k[i] = *reinterpret_cast<const uint4*>(a.kc + o);
      T.v[i] = *reinterpret_cast<const uint4*>(a.vc + o);
    } else {
      T.k[i] = make_uint4(0u, 0u, 0u, 0u);
      T.v[i] = make_uint4(0u, 0u, 0u, 0u);
    }
  }
  return page_ok;
}

__device__ __forceinline__ uint32_t u4get(const uint4& v, int c) {
  return c == 0 ? v.x : (c == 1 ? v.y : (c == 2 ? v.z : v.w));
}

// Online-softmax update of one 16-lane group with its 4 tokens of the tile.
__device__ __forceinline__ void tile_update(const uint4 (&q)[kG], const KVTile& T, int t, int t1,
                                            int grp, bool page_ok, float scale_log2,
                                            float (&m)[kG], float (&l)[kG],
                                            float (&acc)[kG][8]) {
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
    const bool valid = page_ok && (t + 4 * i + grp < t1);
#pragma unroll
    for (int h = 0; h < kG; ++h) sc[h][i] = valid ? sc[h][i] * scale_log2 : -INFINITY;
  }
  float vf[4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t w = u4get(T.v[i], c);
      vf[i][2 * c] = bf16_lo(w);
      vf[i][2 * c + 1] = bf16_hi(w);
    }
  }
#pragma unroll
  for (int h = 0; h < kG; ++h) {
    const float mt = fmaxf(fmaxf(sc[h][0], sc[h][1]), fmaxf(sc[h][2], sc[h][3]));
    const float mn = fmaxf(m[h], mt);
    const float alpha = fast_exp2(m[h] - mn);
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = fast_exp2(sc[h][i] - mn);
    l[h] = l[h] * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
    m[h] = mn;
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      float x = acc[h][d] * alpha;
#pragma unroll
      for (int i = 0; i < 4; ++i) x = fmaf(p[i], vf[i][d], x);
      acc[h][d] = x;
    }
  }
}

// Merge the online-softmax states held by lanes l and l^mask (mask 16 or 32).
__device__ __forceinline__ void merge_lanes(int mask, float (&m)[kG], float (&l)[kG],
                                            float (&acc)[kG][8]) {
#pragma unroll
  for (int h = 0; h < kG; ++h) {
    const float mo = __shfl_xor(m[h], mask);
    const float lo = __shfl_xor(l[h], mask);
    const float mn = fmaxf(m[h], mo);
    const float ws = fast_exp2(m[h] - mn);
    const float wo = fast_exp2(mo - mn);
    l[h] = l[h] * ws + lo * wo;
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const float ao = __shfl_xor(acc[h][d], mask);
      acc[h][d] = acc[h][d] * ws + ao * wo;
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

__global__ __launch_bounds__(1024) void paged_decode_split_kernel(const DecodeArgs a) {
  const int b = blockIdx.x;
  const int s = blockIdx.y;
  const int g = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int grp = lane >> 4;
  const int dl = (lane & 15) * 8;

  const int ctx = row_ctx(a, b);
  if (ctx == 0) {
    if (s == 0 && grp == 0) {
      const float z[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int h = 0; h < kG; ++h) store_row8(a.out + b * a.o_sb + (kG * g + h) * a.o_sh + dl, z, 0.f);
    }
    return;
  }
  const int ns = (ctx + a.split_tokens - 1) / a.split_tokens;
  if (s >= ns) return;
  const int t0 = s * a.split_tokens;
  const int t1 = min(ctx, t0 + a.split_tokens);

  uint4 q[kG];
#pragma unroll
  for (int h = 0; h < kG; ++h)
    q[h] = *reinterpret_cast<const uint4*>(a.q + b * a.q_sb + (kG * g + h) * a.q_sh + dl);

  float m[kG], l[kG], acc[kG][8];
#pragma unroll
  for (int h = 0; h < kG; ++h) {
    m[h] = kMaxSeed;
    l[h] = 0.f;
#pragma unroll
    for (int d = 0; d < 8; ++d) acc[h][d] = 0.f;
  }

  KVTile cur, nxt;
  bool ok_cur = load_tile(a, b, g, grp, dl, t0, t1, cur);
  for (int t = t0; t < t1; t += kTile) {
    bool ok_nxt = false;
    if (t + kTile < t1) ok_nxt = load_tile(a, b, g, grp, dl, t + kTile, t1, nxt);
    tile_update(q, cur, t, t1, grp, ok_cur, a.scale_log2, m, l, acc);
    cur = nxt;
    ok_cur = ok_nxt;
  }

  merge_lanes(16, m, l, acc);
  merge_lanes(32, m, l, acc);

  if (ns == 1) {
    if (grp == 0) {
#pragma unroll
      for (int h = 0; h < kG; ++h)
        store_row8(a.out + b * a.o_sb + (kG * g + h) * a.o_sh + dl, acc[h], l[h] > 0.f ? 1.f / l[h] : 0.f);
    }
    return;
  }
  float* P = a.ws + (((int64_t)b * a.max_splits + s) * a.hkv + g) * kPartFloats;
  if (grp == 0) {
#pragma unroll
    for (int h = 0; h < kG; ++h) {
      float4* dst = reinterpret_cast<float4*>(P + h * kD + dl);
      dst[0] = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
      dst[1] = make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < kG; ++h) {
      P[kG * kD + h] = m[h];
      P[kG * kD + kG + h] = l[h];
    }
  }
}

// Merges the split partials of rows that have more than one split.  One workgroup per row, one
// wave per KV head; lane l owns query head 2g + l/32 and dims 4*(l%32)..+4.
__global__ __launch_bounds__(1024) void paged_decode_combine_kernel(const DecodeArgs a) {
  const int b = blockIdx.x;
  const int g = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int ctx = row_ctx(a, b);
  if (ctx == 0) return;
  const int ns = (ctx + a.split_tokens - 1) / a.split_tokens;
  if (ns <= 1) return;
  const float* base = a.ws + ((int64_t)b * a.max_splits * a.hkv + g) * kPartFloats;
  const int64_t sstride = (int64_t)a.hkv * kPartFloats;

  // Pass 1: lane j < ns reads split j's (m, l) for both heads; wave max and weighted sum.
  float mj[kG], lj[kG];
#pragma unroll
  for (int h = 0; h < kG; ++h) {
    mj[h] = kMaxSeed;
    lj[h] = 0.f;
  }
  if (lane < ns) {
    const float* P = base + lane * sstride;
#pragma unroll
    for (int h = 0; h < kG; ++h) {
      mj[h] = P[kG * kD + h];
      lj[h] = P[kG * kD + kG + h];
    }
  }
  float M[kG], wj[kG], L[kG];
#pragma unroll
  for (int h = 0; h < kG; ++h) {
    float x = mj[h];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
    M[h] = x;
    wj[h] = lane < ns ? fast_exp2(mj[h] - x) : 0.f;
    float y = lj[h] * wj[h];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) y += __shfl_xor(y, off);
    L[h] = y;
  }

  // Pass 2: weighted sum of the unnormalised partial outputs.
  const int h = lane >> 5;
  const int d0 = (lane & 31) * 4;
  const float lsel = h == 0 ? L[0] : L[1];
  const float wsel_inv = lsel > 0.f ? 1.f / lsel : 0.f;
  float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 8
  for (int s = 0; s < ns; ++s) {
    const float w0 = __shfl(wj[0], s);
    const float w1 = __shfl(wj[1], s);
    const float w = h == 0 ? w0 : w1;
    const float4 v = *reinterpret_cast<const float4*>(base + s * sstride + h * kD + d0);
    A.x = fmaf(v.x, w, A.x);
    A.y = fmaf(v.y, w, A.y);
    A.z = fmaf(v.z, w, A.z);
    A.w = fmaf(v.w, w, A.w);
  }
  uint2 o;
  o.x = pack_bf16x2(A.x * wsel_inv, A.y * wsel_inv);
  o.y = pack_bf16x2(A.z * wsel_inv, A.w * wsel_inv);
  *reinterpret_cast<uint2*>(a.out + b * a.o_sb + (kG * g + h) * a.o_sh + d0) = o;
}

int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

int default_split(int batch, int hkv, int max_pages, int page_size) {
  const int64_t max_ctx = (int64_t)max_pages * page_size;
  int split = 64;
  (void)hkv;
  while (split > kTile && (int64_t)batch * ceil_div(max_ctx, split) < 1024) split /= 2;
  while (ceil_div(max_ctx, split) > kMaxSplits) split *= 2;
  return split;
}

}  // namespace
}  // namespace q3a

using namespace q3a;

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
  if (batch <= 0 || num_kv_heads <= 0 || max_pages_per_seq <= 0 || page_size <= 0) return 0;
  if (split_tokens <= 0) split_tokens = default_split(batch, num_kv_heads, max_pages_per_seq, page_size);
  const int max_splits = ceil_div((int64_t)max_pages_per_seq * page_size, split_tokens);
  if (max_splits <= 1) return 0;
  return (size_t)batch * max_splits * num_kv_heads * kPartFloats * sizeof(float);
}

extern "C" int q3a_paged_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                const void* k_cache, const void* v_cache, int64_t kv_stride_page,
                                int64_t kv_stride_tok, int64_t kv_stride_head, int num_pages,
                                int page_size, const int32_t* cache_seqlens,
                                const int32_t* block_table, int64_t bt_stride_b,
                                int max_pages_per_seq, void* out, int64_t o_stride_b,
                                int64_t o_stride_h, void* workspace, size_t workspace_bytes,
                                int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                float softmax_scale, int split_tokens, void* stream) {
  if (batch < 0) return fail(Q3A_EINVAL, "paged_decode: batch %d < 0", batch);
  if (batch == 0) return Q3A_OK;
  if (head_dim != kD) return fail(Q3A_EINVAL, "paged_decode: head_dim %d unsupported (need %d)", head_dim, kD);
  if (num_kv_heads < 1 || num_kv_heads > 16)
    return fail(Q3A_EINVAL, "paged_decode: num_kv_heads %d outside [1, 16]", num_kv_heads);
  if (num_q_heads != kG * num_kv_heads)
    return fail(Q3A_EINVAL, "paged_decode: num_q_heads %d != %d * num_kv_heads %d", num_q_heads, kG, num_kv_heads);
  if (page_size <= 0 || page_size % kTile != 0)
    return fail(Q3A_EINVAL, "paged_decode: page_size %d is not a positive multiple of %d", page_size, kTile);
  if (num_pages <= 0 || max_pages_per_seq <= 0)
    return fail(Q3A_EINVAL, "paged_decode: num_pages %d / max_pages_per_seq %d must be > 0", num_pages, max_pages_per_seq);
  if (!q || !k_cache || !v_cache || !cache_seqlens || !block_table || !out)
    return fail(Q3A_EINVAL, "paged_decode: null pointer argument");
  const uintptr_t align = (uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)out;
  if (align % 16 != 0) return fail(Q3A_EINVAL, "paged_decode: q/k_cache/v_cache/out must be 16-byte aligned");
  if ((q_stride_b | q_stride_h | kv_stride_page | kv_stride_tok | kv_stride_head | o_stride_b | o_stride_h) % 8 != 0)
    return fail(Q3A_EINVAL, "paged_decode: strides must be multiples of 8 elements (16 bytes)");
  if (split_tokens == 0) split_tokens = default_split(batch, num_kv_heads, max_pages_per_seq, page_size);
  if (split_tokens < kTile || split_tokens % kTile != 0)
    return fail(Q3A_EINVAL, "paged_decode: split_tokens %d is not a positive multiple of %d", split_tokens, kTile);
  const int64_t max_ctx = (int64_t)max_pages_per_seq * page_size;
  if (max_ctx > (int64_t)1 << 30) return fail(Q3A_EINVAL, "paged_decode: context capacity too large");
  const int max_splits = ceil_div(max_ctx, split_tokens);
  if (max_splits > kMaxSplits)
    return fail(Q3A_EINVAL, "paged_decode: %d splits exceed %d (raise split_tokens)", max_splits, kMaxSplits);
  const size_t need = q3a_paged_decode_workspace_bytes(batch, num_q_heads, num_kv_heads, head_dim,
                                                       max_pages_per_seq, page_size, split_tokens);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return fail(Q3A_ESPACE, "paged_decode: workspace %zu bytes < %zu needed", workspace_bytes, need);
  if (need > 0 && (uintptr_t)workspace % 16 != 0)
    return fail(Q3A_EINVAL, "paged_decode: workspace must be 16-byte aligned");

  DecodeArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_sb = q_stride_b;
  a.q_sh = q_stride_h;
  a.kc = static_cast<const uint16_t*>(k_cache);
  a.vc = static_cast<const uint16_t*>(v_cache);
  a.kv_sp = kv_stride_page;
  a.kv_st = kv_stride_tok;
  a.kv_sh = kv_stride_head;
  a.num_pages = num_pages;
  a.page_size = page_size;
  a.seqlens = cache_seqlens;
  a.bt = block_table;
  a.bt_sb = bt_stride_b;
  a.max_pages = max_pages_per_seq;
  a.out = static_cast<uint16_t*>(out);
  a.o_sb = o_stride_b;
  a.o_sh = o_stride_h;
  a.ws = static_cast<float*>(workspace);
  a.hkv = num_kv_heads;
  a.split_tokens = split_tokens;
  a.max_splits = max_splits;
  a.scale_log2 = softmax_scale * kLog2e;

  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 block(64 * num_kv_heads);
  hipLaunchKernelGGL(paged_decode_split_kernel, dim3(batch, max_splits), block, 0, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(Q3A_ELAUNCH, "paged_decode: split launch failed: %s", hipGetErrorString(e));
  if (max_splits > 1) {
    hipLaunchKernelGGL(paged_decode_combine_kernel, dim3(batch), block, 0, st, a);
    e = hipGetLastError();
    if (e != hipSuccess) return fail(Q3A_ELAUNCH, "paged_decode: combine launch failed: %s", hipGetErrorString(e));
  }
  return Q3A_OK;
}
