// Code-predictor attention over the 16-slot K/V scratch, for gfx950.
//
// Semantics (engine/cp_attn.py:13-30; in-graph torch form engine/code_predictor.py:46-47): for
// row b and KV head g, the two query heads 2g, 2g+1 attend over slots 0..n_live-1 of K/V[b, g];
// scores and softmax in float32, probabilities rounded to bf16, P.V accumulated in float32,
// output rounded to bf16.  Slots >= n_live are never read.
//
// The append form also takes this step's k/v rows: slot n_live-1 of K/V[b, g] is written from them
// (the K.index_copy_ / V.index_copy_ of engine/code_predictor.py:58) by the same wave that attends,
// which uses the new rows straight from registers.
//
// One wave per (row, KV head).  Scores: lane l takes slots l/8 and 8 + l/8 and an eighth of the head
// dimension of each (4 x 16 B loads; the 8 lanes of a slot pair read 128 contiguous bytes, a whole
// cache line, per instruction) and reduces with three DPP steps; q is loaded once per wave and handed
// to those lanes with ds_bpermute.  P.V: lane l owns output dims 2l, 2l+1 of both query heads and walks the slots up to
// n_live rounded up to a multiple of 4 (one instantiation per multiple); each slot is one 256 B
// coalesced load and the slot's probability is broadcast with v_readlane.  All loads of the wave are issued before the first use, without branches: the
// scratch rows go through a buffer descriptor whose extent ends at the last row read, so the loads
// of dead slots return zeros without touching memory.  Cross-row reductions use the gfx950 lane
// swaps.
#include "q3a_common.h"
#include "../../include/q3attn.h"

namespace q3a {
namespace {

constexpr int kD = 128;
constexpr int kG = 2;
constexpr int kSlots = 16;
constexpr int kWavesPerBlock = 4;

struct CpArgs {
  const uint16_t* q;
  int64_t q_sb;
  uint16_t* k;  // written only at slot n_live - 1, and only when k_new != nullptr
  uint16_t* v;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  const uint16_t* k_new;  // optional [B, Hkv, D] rows for slot n_live - 1 (row strides kn_sb / vn_sb,
  const uint16_t* v_new;  // head stride D)
  int64_t kn_sb, vn_sb;
  uint16_t* out;
  int64_t o_sb;
  int pairs, hkv, n_live;
  float scale_log2;
  // Norm/rope form: q and the new k arrive raw and are RMS-normalised (q_norm_w / k_norm_w) and rotated with the
  // step's cos/sin row in the kernel.
  const uint16_t* qn;
  const uint16_t* kn;
  const uint16_t* cs;
  const uint16_t* sn;
  float eps;
};

// The 16 bytes lane `src` holds (ds_bpermute: the LDS crossbar, no LDS storage).  All lanes must be active.
__device__ __forceinline__ uint4 bpermute16(const uint4& v, int src) {
  const int addr = src * 4;
  return make_uint4((uint32_t)__builtin_amdgcn_ds_bpermute(addr, (int)v.x), (uint32_t)__builtin_amdgcn_ds_bpermute(addr, (int)v.y),
                    (uint32_t)__builtin_amdgcn_ds_bpermute(addr, (int)v.z), (uint32_t)__builtin_amdgcn_ds_bpermute(addr, (int)v.w));
}

// kNV: slots whose V rows are loaded and walked by P.V, n_live rounded up to a multiple of 4 (one instantiation
// each, so every load stays unconditional and the slot loop fully unrolled).
template <bool kAppend, int kNV, bool kRope = false>
__global__ __launch_bounds__(64 * kWavesPerBlock) void cp_attn_kernel(const CpArgs a) {
  static_assert(kAppend || !kRope, "the norm/rope form is an append form");
  const int wave = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  // Every argument the wave uses is read before the exit test of the waves past the last (row, head) pair: left to
  // itself the compiler reads the pair count alone, waits, and only then the rest, two more argument round trips
  // ahead of the first memory load.
  __asm__ volatile("" ::"s"(a.q), "s"(a.k), "s"(a.v), "s"(a.out), "s"(a.q_sb), "s"(a.k_sb), "s"(a.k_sh), "s"(a.k_ss),
                   "s"(a.v_sb), "s"(a.v_sh), "s"(a.v_ss), "s"(a.o_sb), "s"(a.hkv), "s"(a.n_live), "s"(a.scale_log2));
  if constexpr (kAppend) __asm__ volatile("" ::"s"(a.k_new), "s"(a.v_new), "s"(a.kn_sb), "s"(a.vn_sb));
  if constexpr (kRope) __asm__ volatile("" ::"s"(a.qn), "s"(a.kn), "s"(a.cs), "s"(a.sn), "s"(a.eps));
  if (wave >= a.pairs) return;
  const int b = __builtin_amdgcn_readfirstlane(wave / a.hkv);
  const int g = __builtin_amdgcn_readfirstlane(wave - b * a.hkv);
  const int lane = threadIdx.x & 63;
  // Lane (s8, c) = (lane >> 3, lane & 7) holds slots s8 and 8 + s8, dims 8c..8c+7 and 64+8c..64+8c+7 of each, so
  // every K load instruction reads 8 slots x 128 contiguous bytes: whole 128 B lines.
  const int s8 = lane >> 3;
  const int c = lane & 7;
  const bool liveA = s8 < a.n_live;
  const bool liveB = 8 + s8 < a.n_live;

  uint16_t* kb = a.k + (int64_t)b * a.k_sb + (int64_t)g * a.k_sh;
  uint16_t* vb = a.v + (int64_t)b * a.v_sb + (int64_t)g * a.v_sh;
  const uint16_t* qb = a.q + (int64_t)b * a.q_sb + (int64_t)(kG * g) * kD;
  const int last = a.n_live - 1;
  const int n_read = kAppend ? last : a.n_live;
  const uint32_t krow_b = (uint32_t)a.k_ss * 2;
  const uint32_t vrow_b = (uint32_t)a.v_ss * 2;
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(kb, n_read > 0 ? (uint32_t)(n_read - 1) * krow_b + kD * 2 : 0u);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(vb, n_read > 0 ? (uint32_t)(n_read - 1) * vrow_b + kD * 2 : 0u);

  uint4 kr[4], qr[kG][2];
  uint32_t vr[kNV], vn = 0u;
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(qb, kG * kD * 2);
  uint4 qc = buffer_load16(rq, lane < kG * 16 ? (uint32_t)lane * 16 : kOutOfRange);
  const __amdgpu_buffer_rsrc_t rkn =
      kAppend ? make_rsrc(a.k_new + (int64_t)b * a.kn_sb + (int64_t)g * kD, kD * 2) : rk;
  const __amdgpu_buffer_rsrc_t rvn =
      kAppend ? make_rsrc(a.v_new + (int64_t)b * a.vn_sb + (int64_t)g * kD, kD * 2) : rv;
  // The new k row sits on lanes kKL .. kKL + 15 (16 B each); the norm/rope form puts it beside q's lanes 0..31, so
  // one qk_norm_rope16 pass transforms both.
  constexpr int kKL = kRope ? 32 : 0;
  uint4 knc = make_uint4(0u, 0u, 0u, 0u);
  // Norm/rope form: the new k row and lane l's 16 B chunk (dims 8 (l % 16)..+8) of the weights and of the step's
  // cos/sin row are loaded right after q, ahead of the K/V slots, so the transform waits for these loads only and
  // runs while the slot loads are in flight (loaded after them, it waited for every load: +1.1 us per call).
  uint4 wn, rc, rs;
  if constexpr (kRope) {
    knc = buffer_load16(rkn, (unsigned)(lane - kKL) < 16u ? (uint32_t)(lane - kKL) * 16 : kOutOfRange);
    const int c16 = 8 * (lane & 15);
    wn = ld16((lane < 32 ? a.qn : a.kn) + c16);
    rc = ld16(a.cs + c16);
    rs = ld16(a.sn + c16);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j)
    kr[j] = buffer_load16(rk, (uint32_t)(s8 + 8 * (j >> 1)) * krow_b + (uint32_t)(8 * c + 64 * (j & 1)) * 2);
  if constexpr (kAppend && !kRope)
    knc = buffer_load16(rkn, (unsigned)(lane - kKL) < 16u ? (uint32_t)(lane - kKL) * 16 : kOutOfRange);
#pragma unroll
  for (int s = 0; s < kNV; ++s)
    vr[s] = __builtin_amdgcn_raw_buffer_load_b32(rv, lane * 4, (int)((uint32_t)s * vrow_b), 0);
  if constexpr (kAppend) vn = __builtin_amdgcn_raw_buffer_load_b32(rvn, lane * 4, 0, 0);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (kRope) {
    // q of heads 2g, 2g+1 on lanes 0..31 and the new k row on lanes 32..47, each row on 16 lanes in the layout
    // qk_norm_rope16 takes: one pass normalises and rotates all three rows (lanes 48..63 transform zeros and are
    // not read).  The rope is rounded once, as the compiled _pre evaluates it (engine/code_predictor.py:38-43).
    const uint4 y = qk_norm_rope16(lane < 32 ? qc : knc, wn, rc, rs, a.eps);
    qc = y;
    knc = y;
  }
#pragma unroll
  for (int h = 0; h < kG; ++h) {
    qr[h][0] = bpermute16(qc, 16 * h + c);
    qr[h][1] = bpermute16(qc, 16 * h + 8 + c);
  }
  if constexpr (kAppend) {
    const uint4 kn0 = bpermute16(knc, kKL + c), kn1 = bpermute16(knc, kKL + 8 + c);
    if (s8 == last) {
      kr[0] = kn0;
      kr[1] = kn1;
    }
    if (8 + s8 == last) {
      kr[2] = kn0;
      kr[3] = kn1;
    }
    const __amdgpu_buffer_rsrc_t wk = make_rsrc(kb + (int64_t)last * a.k_ss, kD * 2);
    // Non-temporal slot and output stores (the lines stream out instead of staying dirty in the L2): 6.83 -> 6.79 us
    // per call in the 512-row frame.
    __builtin_amdgcn_raw_buffer_store_b128(
        __builtin_bit_cast(u32x4, knc), wk,
        (int)((unsigned)(lane - kKL) < 16u ? (uint32_t)(lane - kKL) * 16 : kOutOfRange), 0, kCacheNT);
    // The new v row (the youngest load) is swapped in and stored after the scores (below), so the scores wait for
    // the K loads only, not for every V load.
  }

  auto dot16 = [](const uint4& q0, const uint4& k0, const uint4& q1, const uint4& k1) {
    float x = dot2_bf16(q0.x, k0.x, 0.f);
    x = dot2_bf16(q0.y, k0.y, x);
    x = dot2_bf16(q0.z, k0.z, x);
    x = dot2_bf16(q0.w, k0.w, x);
    x = dot2_bf16(q1.x, k1.x, x);
    x = dot2_bf16(q1.y, k1.y, x);
    x = dot2_bf16(q1.z, k1.z, x);
    return dot2_bf16(q1.w, k1.w, x);
  };
  float pa[kG], pb[kG];
#pragma unroll
  for (int h = 0; h < kG; ++h) {
    float xa = dot16(qr[h][0], kr[0], qr[h][1], kr[1]);
    float xb = dot16(qr[h][0], kr[2], qr[h][1], kr[3]);
    // sum over the 8 lanes of a slot pair (xor 1, xor 2, then the quads' halves)
    xa = quad_sum(xa);
    xa += dpp_f32<kDppHalfMirror>(xa);
    xb = quad_sum(xb);
    xb += dpp_f32<kDppHalfMirror>(xb);
    xa = liveA ? xa * a.scale_log2 : -INFINITY;
    xb = liveB ? xb * a.scale_log2 : -INFINITY;
    // max and sum over the 16 slots: 8-lane-uniform values, 8 groups per wave
    float mx = fmaxf(xa, xb);
    mx = fmaxf(mx, dpp_f32<kDppRor8>(mx));
    mx = max_xor32(max_xor16(mx));
    const float ea = fast_exp2(xa - mx);
    const float eb = fast_exp2(xb - mx);
    float z = ea + eb;
    z += dpp_f32<kDppRor8>(z);
    z = sum_xor32(sum_xor16(z));
    const float r = __builtin_amdgcn_rcpf(z);
    pa[h] = round_bf16(ea * r);
    pb[h] = round_bf16(eb * r);
  }

  if constexpr (kAppend) {
#pragma unroll
    for (int s = 0; s < kNV; ++s)
      if (s == last) vr[s] = vn;
    __builtin_amdgcn_raw_buffer_store_b32(vn, make_rsrc(vb + (int64_t)last * a.v_ss, kD * 2), lane * 4, 0, kCacheNT);
  }
  float o[kG][2];
#pragma unroll
  for (int h = 0; h < kG; ++h) o[h][0] = o[h][1] = 0.f;
#pragma unroll
  for (int s = 0; s < kNV; ++s) {
    const float lo = bf16_lo(vr[s]);
    const float hi = bf16_hi(vr[s]);
#pragma unroll
    for (int h = 0; h < kG; ++h) {
      const float src = s < 8 ? pa[h] : pb[h];
      const float ps = __builtin_bit_cast(
          float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, src), 8 * (s & 7)));
      o[h][0] = fmaf(ps, lo, o[h][0]);
      o[h][1] = fmaf(ps, hi, o[h][1]);
    }
  }
  uint16_t* ob = a.out + (int64_t)b * a.o_sb + (int64_t)(kG * g) * kD;
#pragma unroll
  for (int h = 0; h < kG; ++h)
    __builtin_nontemporal_store(pack_bf16x2(o[h][0], o[h][1]), reinterpret_cast<uint32_t*>(ob + h * kD + 2 * lane));
}

}  // namespace
}  // namespace q3a

using namespace q3a;

static int cp_launch(const void* q, int64_t q_stride_b, void* k, int64_t k_stride_b, int64_t k_stride_h,
                     int64_t k_stride_s, void* v, int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_s,
                     const void* k_new, const void* v_new, int64_t kn_stride_b, int64_t vn_stride_b, void* out,
                     int64_t o_stride_b, int batch, int num_q_heads, int num_kv_heads, int head_dim, int n_live,
                     float softmax_scale, void* stream, const char* who, const void* q_norm_w = nullptr,
                     const void* k_norm_w = nullptr, const void* cos = nullptr, const void* sin = nullptr,
                     float eps = 0.f) {
  if (batch < 0) return fail(Q3A_EINVAL, "%s: batch %d < 0", who, batch);
  if (batch == 0) return Q3A_OK;
  if (head_dim != kD) return fail(Q3A_EINVAL, "%s: head_dim %d unsupported (need %d)", who, head_dim, kD);
  if (num_kv_heads < 1 || num_q_heads != kG * num_kv_heads)
    return fail(Q3A_EINVAL, "%s: num_q_heads %d must be %d * num_kv_heads %d", who, num_q_heads, kG, num_kv_heads);
  if (n_live < 1 || n_live > kSlots) return fail(Q3A_EINVAL, "%s: n_live %d outside [1, %d]", who, n_live, kSlots);
  if (!q || !k || !v || !out) return fail(Q3A_EINVAL, "%s: null pointer argument", who);
  const uintptr_t align = (uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out | (uintptr_t)k_new |
                          (uintptr_t)v_new;
  if (align % 16 != 0) return fail(Q3A_EINVAL, "%s: q/K/V/out/k_new/v_new must be 16-byte aligned", who);
  if ((q_stride_b | k_stride_b | k_stride_h | k_stride_s | v_stride_b | v_stride_h | v_stride_s | o_stride_b |
       kn_stride_b | vn_stride_b) % 8 != 0)
    return fail(Q3A_EINVAL, "%s: strides must be multiples of 8 elements (16 bytes)", who);
  const int64_t pairs = (int64_t)batch * num_kv_heads;
  if (pairs > ((int64_t)1 << 30)) return fail(Q3A_EINVAL, "%s: batch too large", who);
  const int64_t lim = (int64_t)1 << 26;
  if (k_stride_s < head_dim || k_stride_s > lim || v_stride_s < head_dim || v_stride_s > lim)
    return fail(Q3A_EINVAL, "%s: slot strides %lld/%lld must be in [head_dim, 2^26] elements", who,
                (long long)k_stride_s, (long long)v_stride_s);

  CpArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_sb = q_stride_b;
  a.k = static_cast<uint16_t*>(k);
  a.v = static_cast<uint16_t*>(v);
  a.k_sb = k_stride_b;
  a.k_sh = k_stride_h;
  a.k_ss = k_stride_s;
  a.v_sb = v_stride_b;
  a.v_sh = v_stride_h;
  a.v_ss = v_stride_s;
  a.k_new = static_cast<const uint16_t*>(k_new);
  a.v_new = static_cast<const uint16_t*>(v_new);
  a.kn_sb = kn_stride_b;
  a.vn_sb = vn_stride_b;
  a.out = static_cast<uint16_t*>(out);
  a.o_sb = o_stride_b;
  a.pairs = (int)pairs;
  a.hkv = num_kv_heads;
  a.n_live = n_live;
  a.scale_log2 = softmax_scale * kLog2e;
  const bool rope = q_norm_w != nullptr;
  a.qn = static_cast<const uint16_t*>(q_norm_w);
  a.kn = static_cast<const uint16_t*>(k_norm_w);
  a.cs = static_cast<const uint16_t*>(cos);
  a.sn = static_cast<const uint16_t*>(sin);
  a.eps = eps;
  const int blocks = (int)((pairs + kWavesPerBlock - 1) / kWavesPerBlock);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(blocks), block(64 * kWavesPerBlock);
  const int nv = (n_live + 3) / 4;
  if (rope) {
    if (nv == 1) hipLaunchKernelGGL((cp_attn_kernel<true, 4, true>), grid, block, 0, st, a);
    else if (nv == 2) hipLaunchKernelGGL((cp_attn_kernel<true, 8, true>), grid, block, 0, st, a);
    else if (nv == 3) hipLaunchKernelGGL((cp_attn_kernel<true, 12, true>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((cp_attn_kernel<true, 16, true>), grid, block, 0, st, a);
  } else if (k_new != nullptr) {
    if (nv == 1) hipLaunchKernelGGL((cp_attn_kernel<true, 4>), grid, block, 0, st, a);
    else if (nv == 2) hipLaunchKernelGGL((cp_attn_kernel<true, 8>), grid, block, 0, st, a);
    else if (nv == 3) hipLaunchKernelGGL((cp_attn_kernel<true, 12>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((cp_attn_kernel<true, 16>), grid, block, 0, st, a);
  } else {
    if (nv == 1) hipLaunchKernelGGL((cp_attn_kernel<false, 4>), grid, block, 0, st, a);
    else if (nv == 2) hipLaunchKernelGGL((cp_attn_kernel<false, 8>), grid, block, 0, st, a);
    else if (nv == 3) hipLaunchKernelGGL((cp_attn_kernel<false, 12>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((cp_attn_kernel<false, 16>), grid, block, 0, st, a);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(Q3A_ELAUNCH, "%s: launch failed: %s", who, hipGetErrorString(e));
  return Q3A_OK;
}

extern "C" int q3a_cp_attn(const void* q, int64_t q_stride_b, const void* k, int64_t k_stride_b, int64_t k_stride_h,
                           int64_t k_stride_s, const void* v, int64_t v_stride_b, int64_t v_stride_h,
                           int64_t v_stride_s, void* out, int64_t o_stride_b, int batch, int num_q_heads,
                           int num_kv_heads, int head_dim, int n_live, float softmax_scale, void* stream) {
  return cp_launch(q, q_stride_b, const_cast<void*>(k), k_stride_b, k_stride_h, k_stride_s, const_cast<void*>(v),
                   v_stride_b, v_stride_h, v_stride_s, nullptr, nullptr, 0, 0, out, o_stride_b, batch, num_q_heads,
                   num_kv_heads, head_dim, n_live, softmax_scale, stream, "cp_attn");
}

extern "C" int q3a_cp_attn_append(const void* q, int64_t q_stride_b, const void* k_new, int64_t kn_stride_b,
                                  const void* v_new, int64_t vn_stride_b, void* k, int64_t k_stride_b,
                                  int64_t k_stride_h, int64_t k_stride_s, void* v, int64_t v_stride_b,
                                  int64_t v_stride_h, int64_t v_stride_s, void* out, int64_t o_stride_b, int batch,
                                  int num_q_heads, int num_kv_heads, int head_dim, int n_live, float softmax_scale,
                                  void* stream) {
  if (!k_new || !v_new) return fail(Q3A_EINVAL, "cp_attn_append: null k_new/v_new");
  return cp_launch(q, q_stride_b, k, k_stride_b, k_stride_h, k_stride_s, v, v_stride_b, v_stride_h, v_stride_s,
                   k_new, v_new, kn_stride_b, vn_stride_b, out, o_stride_b, batch, num_q_heads, num_kv_heads,
                   head_dim, n_live, softmax_scale, stream, "cp_attn_append");
}

extern "C" int q3a_cp_attn_append_rope(const void* q, int64_t q_stride_b, const void* k_new, int64_t kn_stride_b,
                                       const void* v_new, int64_t vn_stride_b, const void* q_norm_w,
                                       const void* k_norm_w, const void* cos, const void* sin, float eps, void* k,
                                       int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_s, void* v,
                                       int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_s, void* out,
                                       int64_t o_stride_b, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                       int n_live, float softmax_scale, void* stream) {
  const char* who = "cp_attn_append_rope";
  if (!k_new || !v_new) return fail(Q3A_EINVAL, "%s: null k_new/v_new", who);
  if (!q_norm_w || !k_norm_w || !cos || !sin) return fail(Q3A_EINVAL, "%s: null norm weight or cos/sin row", who);
  if (((uintptr_t)q_norm_w | (uintptr_t)k_norm_w | (uintptr_t)cos | (uintptr_t)sin) % 16 != 0)
    return fail(Q3A_EINVAL, "%s: norm weights and cos/sin rows must be 16-byte aligned", who);
  return cp_launch(q, q_stride_b, k, k_stride_b, k_stride_h, k_stride_s, v, v_stride_b, v_stride_h, v_stride_s,
                   k_new, v_new, kn_stride_b, vn_stride_b, out, o_stride_b, batch, num_q_heads, num_kv_heads,
                   head_dim, n_live, softmax_scale, stream, who, q_norm_w, k_norm_w, cos, sin, eps);
}
