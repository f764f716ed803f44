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

// ---- spill records: pool slots <-> a record in pinned host memory -----------
//
// One workgroup owns one (tensor, listed slot) unit at a time and walks the
// units grid-stride, so a slot's checksum is reduced inside the workgroup and
// stored (merge: compared) once, with no atomics on the record.  The record
// side uses buffer accesses with cache policy sc0|sc1 (system scope): stores
// write through to host memory and loads do not hit lines the GPU cached
// earlier.  Measured on MI355X with 64 workgroups: 57.1 GB/s device to host
// and 57.3 GB/s host to device, the rate of the copy engines (57.0 / 57.1).

constexpr int kRecMaxTensors = 4;
constexpr int kRecWorkgroups = 64;
constexpr int kHostPolicy = 1 | 16;  // sc0 | sc1
constexpr int kRecUnroll = 4;        // 16-element groups per thread in flight

struct RecTensor {
  uint16_t* pool;
  uint32_t half;       // bytes of one plane of one slot (= elements per slot)
  int32_t num_slots;
  uint64_t lo, hi;     // offsets of the tensor's low / high plane part in the record
  uint64_t sums;       // offset of the tensor's checksum row
};

struct RecArgs {
  RecTensor t[kRecMaxTensors];
  uint8_t* rec;
  const int32_t* slots;
  int n_tensors;
  int n_slots;
  int first;
};

// a.t[t] for a wave-uniform t without dynamic indexing of the argument block
__device__ __forceinline__ RecTensor rec_tensor(const RecArgs& a, int t) {
  switch (t) {
    case 0: return a.t[0];
    case 1: return a.t[1];
    case 2: return a.t[2];
    default: return a.t[3];
  }
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t host_rsrc(uint8_t* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(base, static_cast<short>(0), bytes, 0x00020000);
}

// Sum over the workgroup, the same value in every thread.
__device__ __forceinline__ uint32_t block_sum(uint32_t v, uint32_t* red) {
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) v += static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), o));
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  uint32_t s = 0;
#pragma unroll
  for (int w = 0; w < kThreads / kWave; ++w) s += red[w];
  __syncthreads();
  return s;
}

// One unit of the spill: the slot's planes (and checksum) into record slot r.
template <bool SUMS>
__device__ __forceinline__ void spill_unit(const RecArgs& a, const RecTensor& d, int slot,
                                           size_t r, uint32_t* red) {
  const uint16_t* src = d.pool + static_cast<size_t>(slot) * d.half;
  const auto lo = host_rsrc(a.rec + d.lo + r * d.half, d.half);
  const auto hi = host_rsrc(a.rec + d.hi + r * d.half, d.half);
  const int groups = static_cast<int>(d.half / kElemsPerThread);
  uint32_t acc = 0;
  for (int g0 = threadIdx.x; g0 < groups; g0 += kRecUnroll * kThreads) {
    u32x4 x[kRecUnroll], y[kRecUnroll];
#pragma unroll
    for (int k = 0; k < kRecUnroll; ++k) {
      const int g = g0 + k * kThreads;
      if (g < groups) {
        x[k] = *reinterpret_cast<const u32x4*>(src + g * kElemsPerThread);
        y[k] = *reinterpret_cast<const u32x4*>(src + g * kElemsPerThread + 8);
      }
    }
#pragma unroll
    for (int k = 0; k < kRecUnroll; ++k) {
      const int g = g0 + k * kThreads;
      if (g < groups) {
        const u32x4 l = {lo_bytes(x[k][0], x[k][1]), lo_bytes(x[k][2], x[k][3]),
                         lo_bytes(y[k][0], y[k][1]), lo_bytes(y[k][2], y[k][3])};
        const u32x4 h = {hi_bytes(x[k][0], x[k][1]), hi_bytes(x[k][2], x[k][3]),
                         hi_bytes(y[k][0], y[k][1]), hi_bytes(y[k][2], y[k][3])};
        __builtin_amdgcn_raw_buffer_store_b128(l, lo, g * 16, 0, kHostPolicy);
        __builtin_amdgcn_raw_buffer_store_b128(h, hi, g * 16, 0, kHostPolicy);
        if constexpr (SUMS) acc += group_sum(x[k], y[k], static_cast<uint32_t>(g * 8));
      }
    }
  }
  if constexpr (SUMS) {
    const uint32_t s = block_sum(acc, red);
    if (threadIdx.x == 0) {
      __builtin_amdgcn_raw_buffer_store_b32(s, host_rsrc(a.rec + d.sums + r * 4, 4), 0, 0,
                                            kHostPolicy);
    }
  }
}

// One unit of the reload: record slot r back into the pool slot, its
// checksum compared with the record's (mismatches counted into status).
template <bool SUMS>
__device__ __forceinline__ void reload_unit(const RecArgs& a, const RecTensor& d, int slot,
                                            size_t r, uint32_t* red, int tag, int32_t* status) {
  uint16_t* dst = d.pool + static_cast<size_t>(slot) * d.half;
  const auto lo = host_rsrc(a.rec + d.lo + r * d.half, d.half);
  const auto hi = host_rsrc(a.rec + d.hi + r * d.half, d.half);
  const int groups = static_cast<int>(d.half / kElemsPerThread);
  uint32_t acc = 0;
  for (int g0 = threadIdx.x; g0 < groups; g0 += kRecUnroll * kThreads) {
    u32x4 l[kRecUnroll], h[kRecUnroll];
#pragma unroll
    for (int k = 0; k < kRecUnroll; ++k) {
      const int g = g0 + k * kThreads;
      if (g < groups) {
        l[k] = __builtin_amdgcn_raw_buffer_load_b128(lo, g * 16, 0, kHostPolicy);
        h[k] = __builtin_amdgcn_raw_buffer_load_b128(hi, g * 16, 0, kHostPolicy);
      }
    }
#pragma unroll
    for (int k = 0; k < kRecUnroll; ++k) {
      const int g = g0 + k * kThreads;
      if (g < groups) {
        const u32x4 x = {join_first(l[k][0], h[k][0]), join_second(l[k][0], h[k][0]),
                         join_first(l[k][1], h[k][1]), join_second(l[k][1], h[k][1])};
        const u32x4 y = {join_first(l[k][2], h[k][2]), join_second(l[k][2], h[k][2]),
                         join_first(l[k][3], h[k][3]), join_second(l[k][3], h[k][3])};
        *reinterpret_cast<u32x4*>(dst + g * kElemsPerThread) = x;
        *reinterpret_cast<u32x4*>(dst + g * kElemsPerThread + 8) = y;
        if constexpr (SUMS) acc += group_sum(x, y, static_cast<uint32_t>(g * 8));
      }
    }
  }
  if constexpr (SUMS) {
    const uint32_t s = block_sum(acc, red);
    if (threadIdx.x == 0) {
      const uint32_t want = __builtin_amdgcn_raw_buffer_load_b32(
          host_rsrc(a.rec + d.sums + r * 4, 4), 0, 0, kHostPolicy);
      if (want != s) {
        atomicAdd(status, 1);
        atomicCAS(status + 1, 0, tag);
      }
    }
  }
}

// Unit u = (tensor u / n_slots, listed slot u % n_slots); workgroup b takes
// units b, b + G, b + 2G, ... (G = gridDim.x).  The slot list may live in
// pinned host memory (no upload copy between record launches), so each batch
// of the workgroup's next kThreads units reads its slot ids with one load per
// thread into LDS before the units run.
template <bool SPILL, bool SUMS>
__global__ __launch_bounds__(kThreads) void record_kernel(RecArgs a, int tag,
                                                          int32_t* __restrict__ status) {
  __shared__ uint32_t red[kThreads / kWave];
  __shared__ int batch[kThreads];
  const int units = a.n_tensors * a.n_slots;
  const int G = static_cast<int>(gridDim.x);
  // system-scope loads: the host may have rewritten the list since an
  // earlier kernel read the same addresses
  const auto list = host_rsrc(reinterpret_cast<uint8_t*>(const_cast<int32_t*>(a.slots)),
                              static_cast<uint32_t>(a.n_slots) * 4u);
  for (int base = blockIdx.x; base < units; base += G * kThreads) {
    const int mine = base + static_cast<int>(threadIdx.x) * G;
    batch[threadIdx.x] =
        mine < units ? static_cast<int>(__builtin_amdgcn_raw_buffer_load_b32(
                           list, (mine % a.n_slots) * 4, 0, kHostPolicy))
                     : -1;
    __syncthreads();
    for (int j = 0; j < kThreads; ++j) {
      const int u = base + j * G;
      if (u >= units) break;
      const int t = u / a.n_slots;
      const RecTensor d = rec_tensor(a, t);
      const int slot = uniform(batch[j]);
      if (static_cast<unsigned>(slot) >= static_cast<unsigned>(d.num_slots)) continue;
      const size_t r = static_cast<size_t>(a.first) + (u - t * a.n_slots);
      if constexpr (SPILL) {
        spill_unit<SUMS>(a, d, slot, r, red);
      } else {
        reload_unit<SUMS>(a, d, slot, r, red, tag, status);
      }
    }
    __syncthreads();  // every thread is done with this batch before the next is staged
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

namespace voom {
namespace {

// Resolves `p` (n bytes, named `name` in errors) to the address a kernel
// uses for it: pinned host memory, or device memory of the current device.
// Pageable memory (which a kernel cannot touch), managed memory and a range
// running past the end of its allocation are refused.
int device_view(const void* p, size_t n, uint8_t** out, const char* what, const char* name) {
  hipPointerAttribute_t at;
  if (hipPointerGetAttributes(&at, p) != hipSuccess) {
    (void)hipGetLastError();
    return set_error(VOOM_EINVAL, "%s: %s is neither pinned host nor device memory", what, name);
  }
  if (at.type != hipMemoryTypeHost && at.type != hipMemoryTypeDevice) {
    return set_error(VOOM_EINVAL, "%s: %s must be pinned host or device memory (type %d)", what,
                     name, static_cast<int>(at.type));
  }
  if (at.type == hipMemoryTypeDevice) {
    int dev = -1;
    if (int rc = check_hip(hipGetDevice(&dev), what)) return rc;
    VOOM_REQUIRE(at.device == dev, "%s: %s lives on device %d, current device is %d", what, name,
                 at.device, dev);
  }
  void* start = nullptr;
  size_t size = 0;
  if (hipPointerGetAttribute(&start, HIP_POINTER_ATTRIBUTE_RANGE_START_ADDR,
                             reinterpret_cast<hipDeviceptr_t>(const_cast<void*>(p))) != hipSuccess ||
      hipPointerGetAttribute(&size, HIP_POINTER_ATTRIBUTE_RANGE_SIZE,
                             reinterpret_cast<hipDeviceptr_t>(const_cast<void*>(p))) != hipSuccess) {
    (void)hipGetLastError();
    return set_error(VOOM_EINVAL, "%s: cannot find the %s's allocation", what, name);
  }
  const uintptr_t lo = reinterpret_cast<uintptr_t>(start);
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  VOOM_REQUIRE(a >= lo && n <= size - (a - lo),
               "%s: %s of %zu bytes runs past the end of its allocation", what, name, n);
  VOOM_REQUIRE(at.devicePointer != nullptr, "%s: %s has no device address", what, name);
  *out = static_cast<uint8_t*>(at.devicePointer);
  return VOOM_OK;
}

// Validates a record call and fills the kernel arguments.
int record_args(const void* const* pools, const size_t* slot_bytes, const int* num_slots,
                int n_tensors, const int32_t* slots, int n_slots, const void* record,
                int rec_slots, int first, bool sums, RecArgs* a, const char* what) {
  VOOM_REQUIRE(pools && slot_bytes && num_slots && slots && record, "%s: null pointer", what);
  VOOM_REQUIRE(n_tensors >= 1 && n_tensors <= kRecMaxTensors, "%s: n_tensors %d not in [1, %d]",
               what, n_tensors, kRecMaxTensors);
  VOOM_REQUIRE(n_slots >= 0 && first >= 0 && rec_slots >= 0 &&
                   static_cast<long long>(first) + n_slots <= rec_slots,
               "%s: listed slots [%d, %d + %d) outside the record's %d slots", what, first, first,
               n_slots, rec_slots);
  VOOM_REQUIRE(n_slots < (1 << 28), "%s: %d slots, at most 2^28 - 1 per call", what, n_slots);
  size_t half_sum = 0;
  for (int t = 0; t < n_tensors; ++t) {
    VOOM_REQUIRE(slot_bytes[t] > 0 && slot_bytes[t] % 64 == 0 && slot_bytes[t] < (1ull << 31),
                 "%s: slot_bytes[%d] = %zu must be a positive multiple of 64 below 2^31", what, t,
                 slot_bytes[t]);
    VOOM_REQUIRE(pools[t] != nullptr && aligned16(pools[t]), "%s: pool %d null or not 16-byte "
                 "aligned", what, t);
    VOOM_REQUIRE(num_slots[t] > 0, "%s: pool %d is empty", what, t);
    half_sum += slot_bytes[t] / 2;
  }
  VOOM_REQUIRE(aligned16(record), "%s: record must be 16-byte aligned", what);
  const size_t R = static_cast<size_t>(rec_slots);
  const size_t bytes = 2 * R * half_sum + (sums ? 4 * R * n_tensors : 0);
  uint8_t* rec = nullptr;
  if (int rc = device_view(record, bytes, &rec, what, "record")) return rc;
  uint8_t* slot_list = nullptr;
  VOOM_REQUIRE(reinterpret_cast<uintptr_t>(slots) % 4 == 0, "%s: slots must be 4-byte aligned",
               what);
  if (n_slots > 0) {
    if (int rc = device_view(slots, 4 * static_cast<size_t>(n_slots), &slot_list, what,
                             "slot list")) {
      return rc;
    }
  }
  *a = RecArgs{};
  size_t lo = 0;
  for (int t = 0; t < n_tensors; ++t) {
    RecTensor& d = a->t[t];
    d.pool = static_cast<uint16_t*>(const_cast<void*>(pools[t]));
    d.half = static_cast<uint32_t>(slot_bytes[t] / 2);
    d.num_slots = num_slots[t];
    d.lo = lo;
    d.hi = R * half_sum + lo;
    d.sums = 2 * R * half_sum + 4 * R * t;
    lo += R * d.half;
  }
  a->rec = rec;
  a->slots = reinterpret_cast<const int32_t*>(slot_list);
  a->n_tensors = n_tensors;
  a->n_slots = n_slots;
  a->first = first;
  return VOOM_OK;
}

unsigned record_grid(int n_tensors, int n_slots) {
  const int units = n_tensors * n_slots;
  return static_cast<unsigned>(units < kRecWorkgroups ? units : kRecWorkgroups);
}

}  // namespace
}  // namespace voom

extern "C" int voom_spill_record(const void* const* pools, const size_t* slot_bytes,
                                 const int* num_slots, int n_tensors, const int32_t* slots,
                                 int n_slots, void* record, int rec_slots, int first,
                                 int with_sums, hipStream_t stream) {
  RecArgs a;
  if (int rc = record_args(pools, slot_bytes, num_slots, n_tensors, slots, n_slots, record,
                           rec_slots, first, with_sums != 0, &a, "spill_record")) {
    return rc;
  }
  if (n_slots == 0) return VOOM_OK;
  const dim3 grid(record_grid(n_tensors, n_slots));
  if (with_sums) {
    hipLaunchKernelGGL((record_kernel<true, true>), grid, dim3(kThreads), 0, stream, a, 0,
                       nullptr);
  } else {
    hipLaunchKernelGGL((record_kernel<true, false>), grid, dim3(kThreads), 0, stream, a, 0,
                       nullptr);
  }
  return VOOM_LAUNCH_CHECK("spill_record: launch");
}

extern "C" int voom_reload_record(const void* record, int rec_slots, int first,
                                  void* const* pools, const size_t* slot_bytes,
                                  const int* num_slots, int n_tensors, const int32_t* slots,
                                  int n_slots, int tag, int32_t* status, hipStream_t stream) {
  RecArgs a;
  if (int rc = record_args(const_cast<const void* const*>(pools), slot_bytes, num_slots, n_tensors,
                           slots, n_slots, record, rec_slots, first, tag != 0, &a,
                           "reload_record")) {
    return rc;
  }
  VOOM_REQUIRE(tag == 0 || status != nullptr, "reload_record: a tag needs a status buffer");
  if (n_slots == 0) return VOOM_OK;
  const dim3 grid(record_grid(n_tensors, n_slots));
  if (tag != 0) {
    hipLaunchKernelGGL((record_kernel<false, true>), grid, dim3(kThreads), 0, stream, a, tag,
                       status);
  } else {
    hipLaunchKernelGGL((record_kernel<false, false>), grid, dim3(kThreads), 0, stream, a, 0,
                       status);
  }
  return VOOM_LAUNCH_CHECK("reload_record: launch");
}

extern "C" int voom_copy_rows(void* dst, size_t dst_pitch, const void* src, size_t src_pitch,
                              size_t width, size_t rows, hipStream_t stream) {
  if (width == 0 || rows == 0) return VOOM_OK;
  VOOM_REQUIRE(dst && src, "copy_rows: null pointer");
  VOOM_REQUIRE(width <= dst_pitch && width <= src_pitch,
               "copy_rows: width %zu exceeds a pitch (dst %zu, src %zu)", width, dst_pitch,
               src_pitch);
  return check_hip(hipMemcpy2DAsync(dst, dst_pitch, src, src_pitch, width, rows, hipMemcpyDefault,
                                    stream),
                   "copy_rows: hipMemcpy2DAsync");
}

extern "C" int voom_record_prepare(void) {
  // The first launch of a kernel in a process sets up its function object on
  // the host (about a millisecond per kernel); resolving the record kernels'
  // attributes here does that ahead of the first spill.
  const void* kernels[] = {
      reinterpret_cast<const void*>(&record_kernel<true, true>),
      reinterpret_cast<const void*>(&record_kernel<true, false>),
      reinterpret_cast<const void*>(&record_kernel<false, true>),
      reinterpret_cast<const void*>(&record_kernel<false, false>),
  };
  for (const void* k : kernels) {
    hipFuncAttributes attr;
    if (int rc = check_hip(hipFuncGetAttributes(&attr, k), "record_prepare")) return rc;
  }
  return VOOM_OK;
}
