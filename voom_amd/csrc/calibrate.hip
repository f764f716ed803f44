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
