// Shared device helpers and host error plumbing for the q3attn HIP library (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q3a {

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;

constexpr float kLog2e = 1.4426950408889634f;
// Running-max seed: finite, so exp2(m_old - m_new) never evaluates (-inf) - (-inf).
constexpr float kMaxSeed = -1.0e30f;

// ---------------------------------------------------------------------------------- arithmetic
// a.lo*b.lo + a.hi*b.hi + c with bf16 pairs and an fp32 accumulator (v_dot2c_f32_bf16).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

__device__ __forceinline__ float bf16_lo(uint32_t x) { return __uint_as_float(x << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t x) { return __uint_as_float(x & 0xffff0000u); }

// Two floats -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// Byte permute (v_perm_b32): bytes 0-3 of `lo` and 4-7 of `hi`, selected by `sel`.
__device__ __forceinline__ uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}
// (lo half of a, lo half of b) and (hi half of a, hi half of b) as bf16 pairs.
constexpr uint32_t kPermLoLo = 0x05040100u;
constexpr uint32_t kPermHiHi = 0x07060302u;

// Round a float to the nearest bf16 value (round to nearest even), returned as float.
__device__ __forceinline__ float round_bf16(float x) {
  return __uint_as_float(pack_bf16x2(x, 0.f) << 16);
}

// The same rounding in one instruction: v_cvt_pk_bf16_f32 with bf16(x) in the high half and bf16(+0) = 0 in the low
// half is bf16(x)'s fp32 bit pattern.  The compiler lowers every C form of it to a conversion into the low half plus
// a shift or permute, so it is written as assembly; the scheduler then knows nothing of its latency.  Used where
// chains of eager roundings are issue-bound (the prompt step's q prologue and its k producer pass: 62.1 -> 59.0 us per
// layer call); in the short-key admission kernel it measured slower (9.46 -> 9.85 us), which keeps round_bf16.
__device__ __forceinline__ float round_bf16_1op(float x) {
  float r;
  asm("v_cvt_pk_bf16_f32 %0, 0, %1" : "=v"(r) : "v"(x));
  return r;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------------------------- buffer loads
// Raw buffer resource (gfx9 family word 3).  Loads whose byte offset + 16 exceeds num_records
// return zeros and do not touch memory, so a tile's tail tokens and invalid pages cost no traffic.
constexpr int kBufferWord3 = 0x00020000;
constexpr uint32_t kOutOfRange = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufferWord3);
}

__device__ __forceinline__ uint4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, 0));
}

// Uniform part of the offset in an SGPR (soffset), per-lane part in a VGPR.
__device__ __forceinline__ uint4 buffer_load16_s(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, uint32_t s_off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, (int)s_off, 0));
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// 16-byte loads/stores through a vector type.  A plain `uint4` assignment from memory is a struct copy
// (a memcpy in the IR) that can leave the destination array in private (scratch) memory; these stay in
// registers.
__device__ __forceinline__ uint4 ld16(const void* p) {
  return __builtin_bit_cast(uint4, *reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void st16(void* p, uint4 v) { *reinterpret_cast<u32x4*>(p) = __builtin_bit_cast(u32x4, v); }
// The same store with the non-temporal hint: the line streams out instead of staying dirty in the L2.
__device__ __forceinline__ void st16_nt(void* p, uint4 v) {
  __builtin_nontemporal_store(__builtin_bit_cast(u32x4, v), reinterpret_cast<u32x4*>(p));
}
__device__ __forceinline__ void buffer_store16_s(uint4 v, __amdgpu_buffer_rsrc_t r, uint32_t byte_off,
                                                 uint32_t s_off) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, (int)byte_off, (int)s_off, 0);
}

// Direct-to-LDS copies (buffer_load ... lds): lane i's `bytes` (4 or 16) land at lds + bytes * i, with no
// register staging; lanes failing the descriptor's bounds write zeros.  `lds` must be wave-uniform.  The
// copies count on vmcnt like loads, and the compiler's waits before an LDS read cover only the copies into the
// same __shared__ array, so a copy into one array can stay in flight while another array is read.
typedef __attribute__((address_space(3))) void* lds_ptr_t;
__device__ __forceinline__ void lds_copy16(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t byte_off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds, 16, (int)byte_off, 0, 0, 0);
}
__device__ __forceinline__ void lds_copy4(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t byte_off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds, 4, (int)byte_off, 0, 0, 0);
}

// Streaming variant with the non-temporal hint (`nt`): data read exactly once (the K/V pages of a
// decode call) bypasses cache retention, which measured ~12% more HBM read bandwidth on MI355X
// than plain loads for the same access pattern.
constexpr int kCacheNT = 2;
__device__ __forceinline__ uint4 buffer_load16_stream(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, kCacheNT));
}

// ---------------------------------------------------------------------------------- lane moves
// DPP lane permutations within 16-lane rows.  All lanes of the wave must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7-i within each 8 lanes
constexpr int kDppMirror = 0x140;      // lane i <-> 15-i within each 16 lanes

// Sum over each aligned group of 16 lanes; every lane of the group gets the same bits.
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_f32<kDppXor1>(x);
  x += dpp_f32<kDppXor2>(x);
  x += dpp_f32<kDppHalfMirror>(x);
  x += dpp_f32<kDppMirror>(x);
  return x;
}

// Sum over each aligned quad of lanes.
__device__ __forceinline__ float quad_sum(float x) {
  x += dpp_f32<kDppXor1>(x);
  x += dpp_f32<kDppXor2>(x);
  return x;
}

// For values that are uniform within each quad: combine the 4 quads of a 16-lane row.
__device__ __forceinline__ float quads_sum(float x) {
  x += dpp_f32<kDppHalfMirror>(x);
  x += dpp_f32<kDppMirror>(x);
  return x;
}
__device__ __forceinline__ float quads_max(float x) {
  x = fmaxf(x, dpp_f32<kDppHalfMirror>(x));
  x = fmaxf(x, dpp_f32<kDppMirror>(x));
  return x;
}

// x + (x of lane l ^ 32) and x + (x of lane l ^ 16), and the same for max, with the gfx950 lane swaps (VALU
// operations, not the LDS crossbar): with x in both operands, one result holds x and the other the partner's x.
__device__ __forceinline__ float2 swap32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float2 swap16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor32(float x) { const float2 r = swap32(x); return r.x + r.y; }
__device__ __forceinline__ float sum_xor16(float x) { const float2 r = swap16(x); return r.x + r.y; }
__device__ __forceinline__ float max_xor32(float x) { const float2 r = swap32(x); return fmaxf(r.x, r.y); }
__device__ __forceinline__ float max_xor16(float x) { const float2 r = swap16(x); return fmaxf(r.x, r.y); }

// ---------------------------------------------------------------------------------- qk-norm + RoPE
// One 128-dim bf16 head row x, its RMSNorm weight w and the row's RoPE cos/sin (engine/ops.py:51-60, the talker's
// q/k producers at engine/talker.py:69-70 and the code predictor's at engine/code_predictor.py:38-43), as the
// compiled callers evaluate them (torch.compile'd Talker._decode and CodePredictor._pre, whose generated kernels
// keep the whole chain in fp32 and round once at the store; the explicit cast inside rms is not materialised):
//   y = (x * rsqrt(mean(x^2) + eps)) * w            (fp32)
//   o = bf16(y * cos + rot(y) * sin),  rot(y) = (-y[64:], y[:64])   (two fp32 products and an fp32 sum, not fused)
// Contraction into FMA is off in these helpers so the products round as separate multiplies.  The sum of squares
// follows one binary tree over the dims in index order (pairs, pairs of pairs, ...), so the 16-lane layout (8 dims per
// lane, used where a row meets the tile engine) and the 64-lane layout (2 dims per lane, used where a row is stored)
// give the same bits.  All lanes of the wave must be active.
constexpr int kDppRor8 = 0x128;  // row_ror:8 (lane i <- lane i^8 within each 16 lanes)

__device__ __forceinline__ float rms_rsqrt(float sumsq, float eps) {
  return __builtin_amdgcn_rsqf(sumsq * (1.0f / 128.0f) + eps);
}

// Lane l of each aligned 16-lane group holds dims 8*(l%16)..+8 of its row (x, w, cos, sin alike).
__device__ __forceinline__ uint4 qk_norm_rope16(uint4 x, uint4 w, uint4 c, uint4 s, float eps) {
#pragma clang fp contract(off)
  const uint32_t xs[4] = {x.x, x.y, x.z, x.w}, ws[4] = {w.x, w.y, w.z, w.w};
  const uint32_t cs[4] = {c.x, c.y, c.z, c.w}, ss[4] = {s.x, s.y, s.z, s.w};
  float v[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = bf16_lo(xs[i]);
    v[2 * i + 1] = bf16_hi(xs[i]);
  }
  float p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = v[2 * i] * v[2 * i] + v[2 * i + 1] * v[2 * i + 1];
  const float r = rms_rsqrt(row16_sum((p[0] + p[1]) + (p[2] + p[3])), eps);
  const bool lo = (threadIdx.x & 8) == 0;  // dims 0..63: rot = -y[d + 64]
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float y[2], out[2];
    y[0] = (v[2 * i] * r) * bf16_lo(ws[i]);
    y[1] = (v[2 * i + 1] * r) * bf16_hi(ws[i]);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const float yp = dpp_f32<kDppRor8>(y[e]);
      const float cv = e ? bf16_hi(cs[i]) : bf16_lo(cs[i]);
      const float sv = e ? bf16_hi(ss[i]) : bf16_lo(ss[i]);
      out[e] = y[e] * cv + (lo ? -yp : yp) * sv;
    }
    o[i] = pack_bf16x2(out[0], out[1]);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// The same producers as eager bf16 torch ops evaluate them (engine/ops.py:51-60 outside torch.compile; the
// admission layer runs this way by default, engine/arrivals.py:57-61): every op rounds to bf16,
//   y = bf16(w * bf16(x * rsqrt(mean(x^2) + eps))),  o = bf16(bf16(y * cos) + bf16(rot(y) * sin)).
// Layout and reduction tree as qk_norm_rope16.  kOneOpRound: each rounding is round_bf16_1op (same bits).
template <bool kOneOpRound = false>
__device__ __forceinline__ uint4 qk_norm_rope16_eager(uint4 x, uint4 w, uint4 c, uint4 s, float eps) {
  auto rb = [](float v) { return kOneOpRound ? round_bf16_1op(v) : round_bf16(v); };
  const uint32_t xs[4] = {x.x, x.y, x.z, x.w}, ws[4] = {w.x, w.y, w.z, w.w};
  const uint32_t cs[4] = {c.x, c.y, c.z, c.w}, ss[4] = {s.x, s.y, s.z, s.w};
  float p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float v0 = bf16_lo(xs[i]), v1 = bf16_hi(xs[i]);
    p[i] = v0 * v0 + v1 * v1;
  }
  const float r = rms_rsqrt(row16_sum((p[0] + p[1]) + (p[2] + p[3])), eps);
  const bool lo = (threadIdx.x & 8) == 0;  // dims 0..63: rot = -y[d + 64]
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float out[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const float xv = e ? bf16_hi(xs[i]) : bf16_lo(xs[i]);
      const float wv = e ? bf16_hi(ws[i]) : bf16_lo(ws[i]);
      const float y = rb(wv * rb(xv * r));
      const float yp = dpp_f32<kDppRor8>(y);
      const float cv = e ? bf16_hi(cs[i]) : bf16_lo(cs[i]);
      const float sv = e ? bf16_hi(ss[i]) : bf16_lo(ss[i]);
      out[e] = rb(y * cv) + rb((lo ? -yp : yp) * sv);
    }
    o[i] = pack_bf16x2(out[0], out[1]);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// qk_norm_rope16 with the weight and cos/sin chunks read from LDS a word at a time (the lane's 16 B chunk at w, c,
// s), for kernels whose tile pipeline leaves few registers free: same arithmetic, same bits.
__device__ __forceinline__ uint4 qk_norm_rope16_lds(uint4 x, const uint8_t* w, const uint8_t* c, const uint8_t* s,
                                                    float eps) {
#pragma clang fp contract(off)
  const uint32_t xs[4] = {x.x, x.y, x.z, x.w};
  float p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float v0 = bf16_lo(xs[i]), v1 = bf16_hi(xs[i]);
    p[i] = v0 * v0 + v1 * v1;
  }
  const float r = rms_rsqrt(row16_sum((p[0] + p[1]) + (p[2] + p[3])), eps);
  const bool lo = (threadIdx.x & 8) == 0;
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t ww = *reinterpret_cast<const uint32_t*>(w + 4 * i);
    const uint32_t cw = *reinterpret_cast<const uint32_t*>(c + 4 * i);
    const uint32_t sw = *reinterpret_cast<const uint32_t*>(s + 4 * i);
    const float y0 = (bf16_lo(xs[i]) * r) * bf16_lo(ww);
    const float y1 = (bf16_hi(xs[i]) * r) * bf16_hi(ww);
    const float p0 = dpp_f32<kDppRor8>(y0), p1 = dpp_f32<kDppRor8>(y1);
    o[i] = pack_bf16x2(y0 * bf16_lo(cw) + (lo ? -p0 : p0) * bf16_lo(sw),
                       y1 * bf16_hi(cw) + (lo ? -p1 : p1) * bf16_hi(sw));
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// Lane l holds dims 2l, 2l+1 of the row.
__device__ __forceinline__ uint32_t qk_norm_rope64(uint32_t x, uint32_t w, uint32_t c, uint32_t s, float eps) {
#pragma clang fp contract(off)
  const float v0 = bf16_lo(x), v1 = bf16_hi(x);
  const float p = row16_sum(v0 * v0 + v1 * v1);
  const float r = rms_rsqrt(sum_xor32(sum_xor16(p)), eps);
  const float y0 = (v0 * r) * bf16_lo(w);
  const float y1 = (v1 * r) * bf16_hi(w);
  const float2 e0 = swap32(y0), e1 = swap32(y1);  // (lane l & ~32's value, lane l | 32's value)
  const bool lo = (threadIdx.x & 32) == 0;
  const float yp0 = lo ? e0.y : e0.x, yp1 = lo ? e1.y : e1.x;
  const float o0 = y0 * bf16_lo(c) + (lo ? -yp0 : yp0) * bf16_lo(s);
  const float o1 = y1 * bf16_hi(c) + (lo ? -yp1 : yp1) * bf16_hi(s);
  return pack_bf16x2(o0, o1);
}

}  // namespace q3a

// ---------------------------------------------------------------------------------- host side
namespace q3a {
// Records a message for q3a_last_error() on this thread and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
}  // namespace q3a
