// Byte-plane spill codec for gfx950 (bit-exact).
//
// A 16-bit element is treated as two bytes, never as a number, so every bit
// pattern (NaN payloads, subnormals, signed zeros) survives.  Plane `lo` holds
// byte 0 of each element and plane `hi` byte 1, in element order: the layout of
// the reference's vpack codec, lo = raw[0::2], hi = raw[1::2]
// (formats/packed.py:49-50, 277-282), merged back as raw[0::2] = lo,
// raw[1::2] = hi (formats/packed.py:376-378).
//
// Each thread moves 16 elements per step: two 16-byte loads in, one 16-byte
// store per plane out, with v_perm_b32 doing the byte selection.  The kernels
// are HBM-bound (2 bytes read + 2 bytes written per element).
//
// Page checksums (spill integrity; this build's own, the reference has none):
// the slot kernels can also sum, per listed slot, a position-keyed word hash
// of the slot's bytes: 32-bit word j of the slot contributes
// fmix32(word + j * 0x9E3779B9) and the contributions add mod 2^32.  fmix32 is
// MurmurHash3's 32-bit finaliser, a bijection, so changing any one word
// always changes the sum, and a word moved to another position is keyed
// differently.  The split sums the pool slot it reads, the merge sums the
// words it reassembles, and voom_page_sums_verify compares the two.
#include "common.h"

namespace voom {
namespace {

constexpr int kThreads = 256;
constexpr int kElemsPerThread = 16;

// From two dwords (elements e0..e3, little endian) select the low bytes
// {e0.lo, e1.lo, e2.lo, e3.lo} and the high bytes {e0.hi, ..., e3.hi}.
__device__ __forceinline__ uint32_t lo_bytes(uint32_t w0, uint32_t w1) {
  return __builtin_amdgcn_perm(w1, w0, 0x06040200u);
}
__device__ __forceinline__ uint32_t hi_bytes(uint32_t w0, uint32_t w1) {
  return __builtin_amdgcn_perm(w1, w0, 0x07050301u);
}
// Inverse: interleave low-plane dword L and high-plane dword H into the first
// (elements 0,1) and second (elements 2,3) element dwords.
__device__ __forceinline__ uint32_t join_first(uint32_t L, uint32_t H) {
  return __builtin_amdgcn_perm(H, L, 0x05010400u);
}
__device__ __forceinline__ uint32_t join_second(uint32_t L, uint32_t H) {
  return __builtin_amdgcn_perm(H, L, 0x07030602u);
}

__device__ __forceinline__ uint32_t fmix32(uint32_t h) {
  h ^= h >> 16;
  h *= 0x85ebca6bu;
  h ^= h >> 13;
  h *= 0xc2b2ae35u;
  h ^= h >> 16;
  return h;
}

constexpr uint32_t kWordKey = 0x9E3779B9u;

// Hash contribution of the 8 words of one 16-element group; word0 is the
// index of the group's first word inside the slot.
__device__ __forceinline__ uint32_t group_sum(const u32x4& a, const u32x4& b, uint32_t word0) {
  uint32_t s = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    s += fmix32(a[k] + (word0 + k) * kWordKey);
    s += fmix32(b[k] + (word0 + 4 + k) * kWordKey);
  }
  return s;
}

// Sum over the wavefront, then one atomic add per wavefront into *dst
// (integer addition: the result does not depend on the order).
__device__ __forceinline__ void wave_add_to(uint32_t v, uint32_t* dst) {
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) v += static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), o));
  if ((threadIdx.x & (kWave - 1)) == 0) atomicAdd(dst, v);
}

__device__ __forceinline__ void split16(const uint16_t* __restrict__ src,
                                        uint8_t* __restrict__ lo, uint8_t* __restrict__ hi,
                                        u32x4* a_out = nullptr, u32x4* b_out = nullptr) {
  const u32x4 a = *reinterpret_cast<const u32x4*>(src);
  const u32x4 b = *reinterpret_cast<const u32x4*>(src + 8);
  if (a_out != nullptr) {
    *a_out = a;
    *b_out = b;
  }
  u32x4 l, h;
  l[0] = lo_bytes(a[0], a[1]);
  l[1] = lo_bytes(a[2], a[3]);
  l[2] = lo_bytes(b[0], b[1]);
  l[3] = lo_bytes(b[2], b[3]);
  h[0] = hi_bytes(a[0], a[1]);
  h[1] = hi_bytes(a[2], a[3]);
  h[2] = hi_bytes(b[0], b[1]);
  h[3] = hi_bytes(b[2], b[3]);
  *reinterpret_cast<u32x4*>(lo) = l;
  *reinterpret_cast<u32x4*>(hi) = h;
}

__device__ __forceinline__ void merge16(const uint8_t* __restrict__ lo,
                                        const uint8_t* __restrict__ hi,
                                        uint16_t* __restrict__ dst, u32x4* a_out = nullptr,
                                        u32x4* b_out = nullptr) {
  const u32x4 l = *reinterpret_cast<const u32x4*>(lo);
  const u32x4 h = *reinterpret_cast<const u32x4*>(hi);
  u32x4 a, b;
  a[0] = join_first(l[0], h[0]);
  a[1] = join_second(l[0], h[0]);
  a[2] = join_first(l[1], h[1]);
  a[3] = join_second(l[1], h[1]);
  b[0] = join_first(l[2], h[2]);
  b[1] = join_second(l[2], h[2]);
  b[2] = join_first(l[3], h[3]);
  b[3] = join_second(l[3], h[3]);
  *reinterpret_cast<u32x4*>(dst) = a;
  *reinterpret_cast<u32x4*>(dst + 8) = b;
  if (a_out != nullptr) {
    *a_out = a;
    *b_out = b;
  }
}

// Contiguous split: vector body over n16 groups of 16 elements, then a scalar
// tail handled by the first threads.
__global__ __launch_bounds__(kThreads) void split_kernel(const uint16_t* __restrict__ src,
                                                         uint8_t* __restrict__ lo,
                                                         uint8_t* __restrict__ hi, size_t n) {
  const size_t n16 = n / kElemsPerThread;
  const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
  for (size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; i < n16;
       i += stride) {
    split16(src + i * kElemsPerThread, lo + i * kElemsPerThread, hi + i * kElemsPerThread);
  }
  const size_t tail = n16 * kElemsPerThread;
  const size_t gi = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (gi < n - tail) {
    const uint16_t e = src[tail + gi];
    lo[tail + gi] = static_cast<uint8_t>(e & 0xff);
    hi[tail + gi] = static_cast<uint8_t>(e >> 8);
  }
}

__global__ __launch_bounds__(kThreads) void merge_kernel(const uint8_t* __restrict__ lo,
                                                         const uint8_t* __restrict__ hi,
                                                         uint16_t* __restrict__ dst, size_t n) {
  const size_t n16 = n / kElemsPerThread;
  const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
  for (size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; i < n16;
       i += stride) {
    merge16(lo + i * kElemsPerThread, hi + i * kElemsPerThread, dst + i * kElemsPerThread);
  }
  const size_t tail = n16 * kElemsPerThread;
  const size_t gi = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (gi < n - tail) {
    dst[tail + gi] = static_cast<uint16_t>(lo[tail + gi] | (static_cast<uint16_t>(hi[tail + gi]) << 8));
  }
}

// Slot-gathering split: blockIdx.y walks the listed slots, blockIdx.x/threads
// walk the 16-element groups inside one slot.  With SUMS, listed slot i's
// checksum is added into sums[i] (which the caller zeroes).
template <bool SUMS>
__global__ __launch_bounds__(kThreads) void split_slots_kernel(
    const uint16_t* __restrict__ pool, const int32_t* __restrict__ slots, size_t slot_elems,
    int num_slots, uint8_t* __restrict__ lo, uint8_t* __restrict__ hi,
    uint32_t* __restrict__ sums) {
  const int i = blockIdx.y;
  const int slot = slots[i];
  if (static_cast<unsigned>(slot) >= static_cast<unsigned>(num_slots)) return;
  const uint16_t* src = pool + static_cast<size_t>(slot) * slot_elems;
  uint8_t* lo_i = lo + static_cast<size_t>(i) * slot_elems;
  uint8_t* hi_i = hi + static_cast<size_t>(i) * slot_elems;
  const size_t groups = slot_elems / kElemsPerThread;
  uint32_t acc = 0;
  for (size_t gidx = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; gidx < groups;
       gidx += static_cast<size_t>(gridDim.x) * kThreads) {
    if constexpr (SUMS) {
      u32x4 a, b;
      split16(src + gidx * kElemsPerThread, lo_i + gidx * kElemsPerThread,
              hi_i + gidx * kElemsPerThread, &a, &b);
      acc += group_sum(a, b, static_cast<uint32_t>(gidx * 8));
    } else {
      split16(src + gidx * kElemsPerThread, lo_i + gidx * kElemsPerThread,
              hi_i + gidx * kElemsPerThread);
    }
  }
  if constexpr (SUMS) wave_add_to(acc, sums + i);
}

template <bool SUMS>
__global__ __launch_bounds__(kThreads) void merge_slots_kernel(
    const uint8_t* __restrict__ lo, const uint8_t* __restrict__ hi, uint16_t* __restrict__ pool,
    const int32_t* __restrict__ slots, size_t slot_elems, int num_slots,
    uint32_t* __restrict__ sums) {
  const int i = blockIdx.y;
  const int slot = slots[i];
  if (static_cast<unsigned>(slot) >= static_cast<unsigned>(num_slots)) return;
  uint16_t* dst = pool + static_cast<size_t>(slot) * slot_elems;
  const uint8_t* lo_i = lo + static_cast<size_t>(i) * slot_elems;
  const uint8_t* hi_i = hi + static_cast<size_t>(i) * slot_elems;
  const size_t groups = slot_elems / kElemsPerThread;
  uint32_t acc = 0;
  for (size_t gidx = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; gidx < groups;
       gidx += static_cast<size_t>(gridDim.x) * kThreads) {
    if constexpr (SUMS) {
      u32x4 a, b;
      merge16(lo_i + gidx * kElemsPerThread, hi_i + gidx * kElemsPerThread,
              dst + gidx * kElemsPerThread, &a, &b);
      acc += group_sum(a, b, static_cast<uint32_t>(gidx * 8));
    } else {
      merge16(lo_i + gidx * kElemsPerThread, hi_i + gidx * kElemsPerThread,
              dst + gidx * kElemsPerThread);
    }
  }
  if constexpr (SUMS) wave_add_to(acc, sums + i);
}

// status[0] counts mismatching checksums; the first mismatch also stores
// ``tag`` (non-zero) into status[1] when it is still 0.
__global__ __launch_bounds__(kThreads) void verify_sums_kernel(
    const uint32_t* __restrict__ expected, const uint32_t* __restrict__ got, int n, int tag,
    int32_t* __restrict__ status) {
  const int i = blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  if (expected[i] != got[i]) {
    atomicAdd(status, 1);
    atomicCAS(status + 1, 0, tag);
  }
}

unsigned grid_for(size_t n16) {
  // Enough workgroups to fill 256 CUs several times over; the kernels loop.
  const size_t want = (n16 + kThreads - 1) / kThreads;
  const size_t cap = static_cast<size_t>(device_cu_count()) * 16;
  const size_t g = want < cap ? want : cap;
  return static_cast<unsigned>(g > 0 ? g : 1);
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace
}  // namespace voom

using namespace voom;

extern "C" int voom_byteplane_split(const void* src, void* lo, void* hi, size_t n_elems,
                                    hipStream_t stream) {
  if (n_elems == 0) return VOOM_OK;
  VOOM_REQUIRE(src && lo && hi, "byteplane_split: null pointer");
  VOOM_REQUIRE(aligned16(src) && aligned16(lo) && aligned16(hi),
               "byteplane_split: buffers must be 16-byte aligned");
  hipLaunchKernelGGL(split_kernel, dim3(grid_for(n_elems / kElemsPerThread + 1)), dim3(kThreads),
                     0, stream, static_cast<const uint16_t*>(src), static_cast<uint8_t*>(lo),
                     static_cast<uint8_t*>(hi), n_elems);
  return VOOM_LAUNCH_CHECK("byteplane_split: launch");
}

extern "C" int voom_byteplane_merge(const void* lo, const void* hi, void* dst, size_t n_elems,
                                    hipStream_t stream) {
  if (n_elems == 0) return VOOM_OK;
  VOOM_REQUIRE(dst && lo && hi, "byteplane_merge: null pointer");
  VOOM_REQUIRE(aligned16(dst) && aligned16(lo) && aligned16(hi),
               "byteplane_merge: buffers must be 16-byte aligned");
  hipLaunchKernelGGL(merge_kernel, dim3(grid_for(n_elems / kElemsPerThread + 1)), dim3(kThreads),
                     0, stream, static_cast<const uint8_t*>(lo), static_cast<const uint8_t*>(hi),
                     static_cast<uint16_t*>(dst), n_elems);
  return VOOM_LAUNCH_CHECK("byteplane_merge: launch");
}

extern "C" int voom_byteplane_split_slots(const void* pool, const int32_t* slots, int n_slots,
                                          size_t slot_bytes, int num_slots, void* lo, void* hi,
                                          uint32_t* sums, hipStream_t stream) {
  if (n_slots == 0) return VOOM_OK;
  VOOM_REQUIRE(pool && slots && lo && hi, "byteplane_split_slots: null pointer");
  VOOM_REQUIRE(n_slots > 0 && n_slots <= 65535, "byteplane_split_slots: n_slots %d not in [0, 65535]",
               n_slots);
  VOOM_REQUIRE(slot_bytes > 0 && slot_bytes % 64 == 0,
               "byteplane_split_slots: slot_bytes %zu must be a positive multiple of 64",
               slot_bytes);
  VOOM_REQUIRE(num_slots > 0, "byteplane_split_slots: empty pool");
  VOOM_REQUIRE(aligned16(pool) && aligned16(lo) && aligned16(hi),
               "byteplane_split_slots: buffers must be 16-byte aligned");
  VOOM_REQUIRE(reinterpret_cast<uintptr_t>(sums) % 4 == 0,
               "byteplane_split_slots: sums must be 4-byte aligned");
  const size_t elems = slot_bytes / 2;
  const size_t groups = elems / kElemsPerThread;
  size_t gx = (groups + kThreads - 1) / kThreads;
  if (gx > 64) gx = 64;
  const dim3 grid(static_cast<unsigned>(gx), n_slots);
  const auto* src = static_cast<const uint16_t*>(pool);
  auto* l = static_cast<uint8_t*>(lo);
  auto* h = static_cast<uint8_t*>(hi);
  if (sums != nullptr) {
    hipLaunchKernelGGL(split_slots_kernel<true>, grid, dim3(kThreads), 0, stream, src, slots,
                       elems, num_slots, l, h, sums);
  } else {
    hipLaunchKernelGGL(split_slots_kernel<false>, grid, dim3(kThreads), 0, stream, src, slots,
                       elems, num_slots, l, h, sums);
  }
  return VOOM_LAUNCH_CHECK("byteplane_split_slots: launch");
}

extern "C" int voom_byteplane_merge_slots(const void* lo, const void* hi, void* pool,
                                          const int32_t* slots, int n_slots, size_t slot_bytes,
                                          int num_slots, uint32_t* sums, hipStream_t stream) {
  if (n_slots == 0) return VOOM_OK;
  VOOM_REQUIRE(pool && slots && lo && hi, "byteplane_merge_slots: null pointer");
  VOOM_REQUIRE(n_slots > 0 && n_slots <= 65535, "byteplane_merge_slots: n_slots %d not in [0, 65535]",
               n_slots);
  VOOM_REQUIRE(slot_bytes > 0 && slot_bytes % 64 == 0,
               "byteplane_merge_slots: slot_bytes %zu must be a positive multiple of 64",
               slot_bytes);
  VOOM_REQUIRE(num_slots > 0, "byteplane_merge_slots: empty pool");
  VOOM_REQUIRE(aligned16(pool) && aligned16(lo) && aligned16(hi),
               "byteplane_merge_slots: buffers must be 16-byte aligned");
  VOOM_REQUIRE(reinterpret_cast<uintptr_t>(sums) % 4 == 0,
               "byteplane_merge_slots: sums must be 4-byte aligned");
  const size_t elems = slot_bytes / 2;
  const size_t groups = elems / kElemsPerThread;
  size_t gx = (groups + kThreads - 1) / kThreads;
  if (gx > 64) gx = 64;
  const dim3 grid(static_cast<unsigned>(gx), n_slots);
  const auto* l = static_cast<const uint8_t*>(lo);
  const auto* h = static_cast<const uint8_t*>(hi);
  auto* dst = static_cast<uint16_t*>(pool);
  if (sums != nullptr) {
    hipLaunchKernelGGL(merge_slots_kernel<true>, grid, dim3(kThreads), 0, stream, l, h, dst,
                       slots, elems, num_slots, sums);
  } else {
    hipLaunchKernelGGL(merge_slots_kernel<false>, grid, dim3(kThreads), 0, stream, l, h, dst,
                       slots, elems, num_slots, sums);
  }
  return VOOM_LAUNCH_CHECK("byteplane_merge_slots: launch");
}

extern "C" int voom_page_sums_verify(const uint32_t* expected, const uint32_t* got, int n,
                                     int tag, int32_t* status, hipStream_t stream) {
  if (n == 0) return VOOM_OK;
  VOOM_REQUIRE(expected && got && status, "page_sums_verify: null pointer");
  VOOM_REQUIRE(n > 0 && tag != 0, "page_sums_verify: n %d, tag %d (must be non-zero)", n, tag);
  hipLaunchKernelGGL(verify_sums_kernel, dim3((n + kThreads - 1) / kThreads), dim3(kThreads), 0,
                     stream, expected, got, n, tag, status);
  return VOOM_LAUNCH_CHECK("page_sums_verify: launch");
}
