// Calibration kernel for the benchmark: the time one launch needs to stream a
// buffer from HBM, the floor any single kernel reading that many bytes runs
// into (launch, first-byte latency, ramp).  No counterpart in the reference.
#include "common.h"

namespace voom {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;

// Each thread XORs 16-byte words, kUnroll loads in flight per lane, grid
// stride; each wavefront folds its XOR into sink[workgroup], so no load is
// dead.  Ordinary loads: over a single 16.8 MB pass they measured 4.7 us
// against 5.3 us for non-temporal ones.
__global__ __launch_bounds__(kThreads) void stream_read_kernel(const u32x4* __restrict__ p,
                                                               size_t n16,
                                                               uint32_t* __restrict__ sink) {
  const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
  size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
  uint32_t acc = 0;
  for (; i + (kUnroll - 1) * stride < n16; i += kUnroll * stride) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = p[i + u * stride];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  for (; i < n16; i += stride) {
    const u32x4 v = p[i];
    acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) acc ^= static_cast<uint32_t>(__shfl_xor(static_cast<int>(acc), o));
  if ((threadIdx.x & (kWave - 1)) == 0) atomicXor(sink + blockIdx.x, acc);
}

}  // namespace
}  // namespace voom

using namespace voom;

extern "C" int voom_stream_read(const void* src, size_t n_bytes, uint32_t* sink, int workgroups,
                                hipStream_t stream) {
  VOOM_REQUIRE(src && sink, "stream_read: null pointer");
  VOOM_REQUIRE(reinterpret_cast<uintptr_t>(src) % 16 == 0 && n_bytes % 16 == 0,
               "stream_read: buffer must be 16-byte aligned and a multiple of 16 bytes");
  VOOM_REQUIRE(workgroups > 0 && workgroups <= (1 << 20), "stream_read: workgroups %d",
               workgroups);
  if (n_bytes == 0) return VOOM_OK;
  hipLaunchKernelGGL(stream_read_kernel, dim3(static_cast<unsigned>(workgroups)), dim3(kThreads),
                     0, stream, static_cast<const u32x4*>(src), n_bytes / 16, sink);
  return VOOM_LAUNCH_CHECK("stream_read: launch");
}

namespace voom {
namespace {

// Row gather: wavefront v (of all the grid's) reads rows v, v + V, ... of the
// index list, each row_bytes (a multiple of 1 KiB) at base + idx[r] *
// row_bytes -- and the same row of base2 when given -- one 1 KiB piece per
// instruction, four rows in flight.
__global__ __launch_bounds__(kThreads) void gather_read_kernel(const uint8_t* __restrict__ base,
                                                               const uint8_t* __restrict__ base2,
                                                               size_t row_bytes,
                                                               const int32_t* __restrict__ idx,
                                                               int n_rows, int n_base_rows,
                                                               uint32_t* __restrict__ sink) {
  const int lane = threadIdx.x & (kWave - 1);
  const int waves = static_cast<int>(gridDim.x) * (kThreads / kWave);
  const int wv = static_cast<int>(blockIdx.x) * (kThreads / kWave) + threadIdx.x / kWave;
  const int pieces = static_cast<int>(row_bytes / 1024);
  const int tensors = base2 != nullptr ? 2 : 1;
  uint32_t acc = 0;
  for (int r0 = wv; r0 < n_rows; r0 += 4 * waves) {
    u32x4 v[4][2][4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int r = r0 + u * waves;
      int row = r < n_rows ? idx[r] : 0;
      row = static_cast<unsigned>(row) < static_cast<unsigned>(n_base_rows) ? row : 0;
      const size_t off = static_cast<size_t>(row) * row_bytes + 16 * lane;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint8_t* src = (t == 0 ? base : base2) + off;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          v[u][t][p] = (r < n_rows && t < tensors && p < pieces)
                           ? *reinterpret_cast<const u32x4*>(src + 1024 * p)
                           : u32x4{0u, 0u, 0u, 0u};
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int p = 0; p < 4; ++p) acc ^= v[u][t][p][0] ^ v[u][t][p][1] ^ v[u][t][p][2] ^ v[u][t][p][3];
      }
    }
  }
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) acc ^= static_cast<uint32_t>(__shfl_xor(static_cast<int>(acc), o));
  if (lane == 0) atomicXor(sink + blockIdx.x, acc);
}

}  // namespace
}  // namespace voom

extern "C" int voom_gather_read(const void* base, const void* base2, size_t row_bytes,
                                int n_base_rows, const int32_t* idx, int n_rows, uint32_t* sink,
                                int workgroups, hipStream_t stream) {
  VOOM_REQUIRE(base && idx && sink, "gather_read: null pointer");
  VOOM_REQUIRE(reinterpret_cast<uintptr_t>(base2) % 16 == 0, "gather_read: base2 not 16-byte aligned");
  VOOM_REQUIRE(row_bytes > 0 && row_bytes % 1024 == 0 && row_bytes <= 4096,
               "gather_read: row_bytes %zu must be 1, 2, 3 or 4 KiB", row_bytes);
  VOOM_REQUIRE(reinterpret_cast<uintptr_t>(base) % 16 == 0, "gather_read: base not 16-byte aligned");
  VOOM_REQUIRE(n_rows >= 0 && n_base_rows > 0 && workgroups > 0 && workgroups <= (1 << 20),
               "gather_read: bad sizes");
  if (n_rows == 0) return VOOM_OK;
  hipLaunchKernelGGL(gather_read_kernel, dim3(static_cast<unsigned>(workgroups)), dim3(kThreads),
                     0, stream, static_cast<const uint8_t*>(base), static_cast<const uint8_t*>(base2),
                     row_bytes, idx, n_rows, n_base_rows, sink);
  return VOOM_LAUNCH_CHECK("gather_read: launch");
}
