// HBM read probes for gfx950: measurement infrastructure beside the q3attn library (built into libq3probe.so; not
// part of the attention ABI).  They answer "what read rate does this access pattern reach on this GPU", so a kernel's
// achieved bandwidth can be set against a measured ceiling as well as against the 8 TB/s datasheet peak.
//
// q3p_stream_read: every 16-byte word of a buffer once, grid-stride, 16 B per lane per load, with or without the
//   non-temporal hint.
// q3p_tile_read: the talker decode's K/V access pattern.  A resident grid cuts a flattened list of 16-token tiles
//   (page id, valid tokens; rows one after another) into equal contiguous ranges (or, with flags, the planned
//   decode's XCD-weighted ranges, each taken by a workgroup of its XCD); the workgroup's wave g streams KV
//   head g of each tile in its range: 4 loads of K and 4 of V per tile, lane l fetching token 4i + l/16, dims
//   8 (l % 16) .. +8 (256 B head rows at the token stride), through a buffer descriptor covering exactly one page, so
//   tokens past the tile's valid count and invalid pages are bounds-failed loads; non-temporal; tile j+1 issued before
//   tile j is consumed.  Consuming a tile folds its words into an XOR, which the kernel stores only if it equals a
//   value the caller chose to be impossible in practice (so the loads cannot be removed).
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int kD = 128;
constexpr uint32_t kOutOfRange = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

template <int kAux>
__device__ __forceinline__ uint4 load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kAux));
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t fold(uint4 v) { return v.x ^ v.y ^ v.z ^ v.w; }
__device__ __forceinline__ uint32_t fold(u32x4 v) { return v.x ^ v.y ^ v.z ^ v.w; }

template <bool kNT>
__device__ __forceinline__ u32x4 ld(const u32x4* p) {
  if constexpr (kNT) return __builtin_nontemporal_load(p);
  return *p;
}

template <bool kNT>
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* buf, size_t n16, uint32_t magic,
                                                          uint32_t* sink) {
  uint32_t acc = 0;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  // Four independent loads in flight per lane.
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const u32x4 a = ld<kNT>(buf + i), b = ld<kNT>(buf + i + stride);
    const u32x4 c = ld<kNT>(buf + i + 2 * stride), d = ld<kNT>(buf + i + 3 * stride);
    acc ^= fold(a) ^ fold(b) ^ fold(c) ^ fold(d);
  }
  for (; i < n16; i += stride) acc ^= fold(ld<kNT>(buf + i));
  if (acc == magic) sink[blockIdx.x] = acc;
}

struct TileArgs {
  const uint16_t* kc;
  const uint16_t* vc;
  int64_t kv_sp, kv_st, kv_sh;   // element strides of a page, a token, a head
  uint32_t page_bytes;           // byte extent of one page's tokens
  int num_pages;
  const int2* tiles;             // [nt]: (page id, valid tokens 1..16)
  int nt, grid;
  int* flags;                    // nullptr: equal ranges by workgroup index; else one zeroed flag per range (below)
  uint32_t magic;
  uint32_t* sink;
};

struct Tile {
  uint4 k[4], v[4];
};

__device__ __forceinline__ void issue(const TileArgs& a, int2 t, uint32_t lane_off, int grp, Tile& T) {
  const bool ok = t.y > 0 && (unsigned)t.x < (unsigned)a.num_pages;
  const int64_t pbase = ok ? (int64_t)t.x * a.kv_sp : 0;
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(a.kc + pbase, ok ? a.page_bytes : 0u);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(a.vc + pbase, ok ? a.page_bytes : 0u);
  const uint32_t tok_bytes = (uint32_t)(a.kv_st * 2);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t o = (4 * i + grp < t.y) ? lane_off + (uint32_t)(4 * i) * tok_bytes : kOutOfRange;
    T.k[i] = load16<2>(rk, o);
    T.v[i] = load16<2>(rv, o);
  }
}

// Range k of the XCD-weighted split (as the planned decode's): ranges of even index 67/64 of the mean, odd 61/64,
// with at least 4 tiles per range (the probe's resident grid is larger than the decode's); equal ranges otherwise.
__device__ __forceinline__ int range_lo(int k, int nt, int grid, bool weighted) {
  if (!weighted) return (int)((int64_t)k * nt / grid);
  const uint64_t wk = 64ull * (uint64_t)k + 3ull * (uint64_t)(k & 1), wg = 64ull * (uint64_t)grid + 3ull * (uint64_t)(grid & 1);
  return (int)((uint64_t)nt * wk / wg);
}

__global__ __launch_bounds__(1024) void tile_read_kernel(const TileArgs a) {
  const int g = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int grp = lane >> 4;
  // With flags, the workgroup takes range j mod 8 == its XCD id the way the planned decode does: it guesses the range a
  // round-robin placement gives it, prefetches that range's first tile entries and claims the range's flag with one
  // exchange (a collision takes the next free flag); ranges weighted by XCD.
  __shared__ int s_claim;
  int k = blockIdx.x;
  bool weighted = false;
  int2 pre = make_int2(-1, 0);
  int kspec = -1;
  if (a.flags != nullptr) {
    const int xcc = __builtin_amdgcn_s_getreg(20 | (0 << 6) | (3 << 11)) & 7;  // HW_REG_XCC_ID, bits 0-3
    weighted = a.nt >= 4 * a.grid;
    kspec = min((int)(blockIdx.x & ~7u) + xcc, a.grid - 1);
    const int lo_s = range_lo(kspec, a.nt, a.grid, weighted), hi_s = range_lo(kspec + 1, a.nt, a.grid, weighted);
    if (lane < min(64, hi_s - lo_s)) pre = a.tiles[lo_s + lane];
    if (threadIdx.x == 0) {
      int got = -1;
      for (int d = 0; d < a.grid && got < 0; ++d) {
        const int kk = kspec + d < a.grid ? kspec + d : kspec + d - a.grid;
        if (__hip_atomic_exchange(a.flags + kk, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0) got = kk;
      }
      s_claim = got;
    }
    __syncthreads();
    k = s_claim;
    if (k < 0) return;
  }
  const int lo = range_lo(k, a.nt, a.grid, weighted);
  const int hi = range_lo(k + 1, a.nt, a.grid, weighted);
  const uint32_t lane_off = (uint32_t)((grp * a.kv_st + g * a.kv_sh + (lane & 15) * 8) * 2);
  uint32_t acc = 0;
  for (int cb = lo; cb < hi; cb += 64) {
    const int n = min(64, hi - cb);
    // lane i describes tile cb + i (the first list of a correctly guessed range was prefetched)
    const int2 mine = (cb == lo && k == kspec) ? (lane < n ? pre : make_int2(-1, 0))
                                               : (lane < n ? a.tiles[cb + lane] : make_int2(-1, 0));
    auto tile = [&](int j) {
      const int jj = j < n ? j : 0;
      int2 t;
      t.x = __builtin_amdgcn_readlane(mine.x, jj);
      t.y = j < n ? __builtin_amdgcn_readlane(mine.y, jj) : 0;
      return t;
    };
    Tile A, B;
    issue(a, tile(0), lane_off, grp, A);
    for (int j = 0; j < n; j += 2) {
      issue(a, tile(j + 1), lane_off, grp, B);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc ^= fold(A.k[i]) ^ fold(A.v[i]);
      issue(a, tile(j + 2), lane_off, grp, A);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc ^= fold(B.k[i]) ^ fold(B.v[i]);
    }
  }
  if (acc == a.magic) a.sink[blockIdx.x] = acc;
}

}  // namespace

// Reads n16 16-byte words of buf (16-byte aligned) with `grid` workgroups of 256 threads; nt selects the
// non-temporal hint.  sink: at least `grid` words, written only when a lane's XOR equals magic.  0 or a HIP error.
extern "C" int q3p_stream_read(const void* buf, size_t n16, int grid, int nt, uint32_t magic, uint32_t* sink,
                               void* stream) {
  if (!buf || !sink || grid <= 0) return (int)hipErrorInvalidValue;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (nt)
    hipLaunchKernelGGL(stream_read_kernel<true>, dim3(grid), dim3(256), 0, s, static_cast<const u32x4*>(buf), n16,
                       magic, sink);
  else
    hipLaunchKernelGGL(stream_read_kernel<false>, dim3(grid), dim3(256), 0, s, static_cast<const u32x4*>(buf), n16,
                       magic, sink);
  return (int)hipGetLastError();
}

// Streams the K/V head rows of nt tiles (tiles: [nt] int2 of (page id, valid tokens)) from the paged pools
// [num_pages, 16, hkv, 128] bf16 (16-token pages) with `grid` workgroups of 64 * hkv threads, each over an equal contiguous
// range of the list.  sink: at least `grid` words.  0 or a HIP error.
// flags: nullptr, or `grid` ints that are zero at launch (q3p_clear_flags): the XCD-weighted ranges taken by XCD.
extern "C" int q3p_tile_read(const void* k_cache, const void* v_cache, int64_t kv_stride_page, int64_t kv_stride_tok,
                             int64_t kv_stride_head, int num_pages, int page_size, int hkv, const int32_t* tiles,
                             int nt, int grid, uint32_t magic, uint32_t* sink, int* flags, void* stream) {
  // A tile is one whole 16-token page (its loads start at token 0 of the page).
  if (!k_cache || !v_cache || !tiles || !sink || nt < 0 || grid <= 0 || hkv < 1 || hkv > 16 || page_size != 16)
    return (int)hipErrorInvalidValue;
  if (nt == 0) return 0;
  TileArgs a;
  a.kc = static_cast<const uint16_t*>(k_cache);
  a.vc = static_cast<const uint16_t*>(v_cache);
  a.kv_sp = kv_stride_page;
  a.kv_st = kv_stride_tok;
  a.kv_sh = kv_stride_head;
  a.page_bytes = (uint32_t)(((int64_t)(page_size - 1) * kv_stride_tok + (int64_t)(hkv - 1) * kv_stride_head + kD) * 2);
  a.num_pages = num_pages;
  a.tiles = reinterpret_cast<const int2*>(tiles);
  a.nt = nt;
  a.grid = grid;
  a.magic = magic;
  a.sink = sink;
  a.flags = flags;
  hipLaunchKernelGGL(tile_read_kernel, dim3(grid), dim3(64 * hkv), 0, static_cast<hipStream_t>(stream), a);
  return (int)hipGetLastError();
}

__global__ __launch_bounds__(256) void clear_kernel(int* flags, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) flags[i] = 0;
}

// Zeroes n ints (the range flags of q3p_tile_read calls) with a kernel (capturable, no memset node).
extern "C" int q3p_clear_flags(int* flags, int n, void* stream) {
  if (!flags || n < 0) return (int)hipErrorInvalidValue;
  if (n == 0) return 0;
  hipLaunchKernelGGL(clear_kernel, dim3((n + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream), flags, n);
  return (int)hipGetLastError();
}

// Workgroups of each probe kernel one GPU holds at once (occupancy x CUs), for sizing a resident grid.
extern "C" int q3p_resident_grid(int which, int hkv) {
  int dev = 0, cus = 0, per = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return -1;
  const hipError_t e = which == 0
                           ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, stream_read_kernel<true>, 256, 0)
                           : hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, tile_read_kernel, 64 * hkv, 0);
  if (e != hipSuccess) return -1;
  return cus * per;
}
