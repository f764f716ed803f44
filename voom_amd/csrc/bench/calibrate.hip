// Calibration kernels for the benchmark (libvoom_calibrate.so, not the
// paged-KV library): the time one launch needs to stream a
// buffer from HBM, the floor any single kernel reading that many bytes runs
// into (launch, first-byte latency, ramp).  No counterpart in the reference.
#include "../common.h"
#include "../../../include/voom_calibrate.h"

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

namespace voom {
namespace {

// Latent tile stream: the data movement of the MLA latent kernel
// (mla_group64_kernel) with no arithmetic.  Workgroup (sequence b, range r,
// group g) -- the `groups` workgroups of a range placed on one XCD, as the
// latent kernel places its head groups -- copies its 64 query rows and then
// the 64-token tiles of its range into LDS with direct-to-LDS loads, two tile
// buffers, the next tile's 18 loads per wavefront issued when the current one
// has landed, and at the end writes 64 rows of 512 fp16 (the bytes of one
// head group's partial rows).  Tiles are 64 rows of 576 bf16 at the start of
// a 64-token page (table[b][t]); rows past ctx read as zeros.
constexpr int kTrLat = 576;
constexpr int kTrRowBytes = kTrLat * 2;
constexpr int kTrLoads = 18;  // 1 KiB direct-to-LDS loads per wavefront and tile

__device__ __forceinline__ int tr_swizzle(int r) { return ((r >> 2) ^ (((r >> 1) & 1) << 2)) & 7; }

__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void tile_read_kernel(const uint16_t* __restrict__ pool, int num_slots,
                      const int32_t* __restrict__ table, const uint16_t* __restrict__ q,
                      int max_pages, int ctx, int ranges, int groups,
                      uint16_t* __restrict__ rows_out, uint32_t* __restrict__ sink) {
  typedef __attribute__((address_space(3))) void lds_void;
  __shared__ __attribute__((aligned(16))) uint16_t tile[2][64 * kTrLat];
  const int lane = threadIdx.x & (kWave - 1);
  const int w = uniform(threadIdx.x / kWave);
  const int n_tasks = static_cast<int>(gridDim.x) / groups;
  const int bid = blockIdx.x;
  int task, g;
  if (n_tasks % 8 == 0) {
    const int local = bid >> 3;
    g = local % groups;
    task = (local / groups) * 8 + (bid & 7);
  } else {
    g = bid % groups;
    task = bid / groups;
  }
  const int b = task / ranges;
  const int range = task - b * ranges;
  const int n_tiles = (ctx + 63) / 64;
  const int per = (n_tiles + ranges - 1) / ranges;
  const int t_lo = range * per;
  const int t_hi = t_lo + per < n_tiles ? t_lo + per : n_tiles;
  // rows 8 w + lane / 8 (+ 32), chunk (lane & 7) ^ swizzle: the latent kernel's layout
  const int row = 8 * w + (lane >> 3);
  const int col = 16 * ((lane & 7) ^ tr_swizzle(row));
  const int off0 = row * kTrRowBytes + col;
  const int off1 = off0 + 32 * kTrRowBytes;
  auto issue = [&](__amdgpu_buffer_rsrc_t r, uint16_t* dst) {
#pragma unroll
    for (int k = 0; k < kTrLoads; ++k) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)(dst + (w + 4 * k) * 512), 16,
                                               ((k & 1) ? off1 : off0) + 128 * (k >> 1), 0, 0, 0);
    }
  };
  auto tile_src = [&](int t) {
    int slot = table[static_cast<size_t>(b) * max_pages + t];
    slot = static_cast<unsigned>(slot) < static_cast<unsigned>(num_slots) ? slot : 0;
    int valid = ctx - 64 * t;
    valid = valid > 64 ? 64 : valid;
    return __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(pool) + static_cast<size_t>(slot) * 64 * kTrLat, static_cast<short>(0),
        valid * kTrRowBytes, 0x00020000);
  };
  if (q != nullptr) {
    issue(__builtin_amdgcn_make_buffer_rsrc(
              const_cast<uint16_t*>(q) + (static_cast<size_t>(b) * groups + g) * 64 * kTrLat,
              static_cast<short>(0), 64 * kTrRowBytes, 0x00020000),
          tile[1]);
  }
  if (t_lo < t_hi) issue(tile_src(t_lo), tile[0]);
  uint32_t acc = 0;
  for (int t = t_lo; t < t_hi; ++t) {
    wait_vmem_all();
    lds_barrier();
    if (t + 1 < t_hi) issue(tile_src(t + 1), tile[(t + 1 - t_lo) & 1]);
    acc ^= *reinterpret_cast<const uint32_t*>(tile[(t - t_lo) & 1] + 8 * lane + 512 * w);
    lds_barrier();
  }
  wait_vmem_all();
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) acc ^= static_cast<uint32_t>(__shfl_xor(static_cast<int>(acc), o));
  uint16_t* po = rows_out + static_cast<size_t>(bid) * 64 * 512;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    *reinterpret_cast<u32x4*>(po + (16 * w + i) * 512 + 8 * lane) = u32x4{acc, acc, acc, acc};
  }
  if (threadIdx.x == 0) sink[bid] = acc;
}

}  // namespace
}  // namespace voom

extern "C" int voom_tile_read(const void* pool, int num_slots, const int32_t* table,
                              const void* q, int batch, int max_pages, int ctx, int ranges,
                              int groups, void* rows_out, uint32_t* sink, hipStream_t stream) {
  VOOM_REQUIRE(pool && table && rows_out && sink, "tile_read: null pointer");
  VOOM_REQUIRE(batch > 0 && ranges > 0 && (groups == 1 || groups == 2) && num_slots > 0 &&
                   max_pages > 0 && ctx > 0 && ctx <= 64 * max_pages,
               "tile_read: bad sizes (batch %d ranges %d groups %d ctx %d max_pages %d)", batch,
               ranges, groups, ctx, max_pages);
  VOOM_REQUIRE(static_cast<long long>(num_slots) * 64 * kTrRowBytes < (1LL << 40),
               "tile_read: pool too large");
  const long long grid = static_cast<long long>(batch) * ranges * groups;
  VOOM_REQUIRE(grid <= (1 << 20), "tile_read: %lld workgroups", grid);
  hipLaunchKernelGGL(tile_read_kernel, dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, stream,
                     static_cast<const uint16_t*>(pool), num_slots, table,
                     static_cast<const uint16_t*>(q), max_pages, ctx, ranges, groups,
                     static_cast<uint16_t*>(rows_out), sink);
  return VOOM_LAUNCH_CHECK("tile_read: launch");
}
