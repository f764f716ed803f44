// Bounds checks of the index inputs of the attention kernels (debug mode).
//
// The attention kernels never fault on a bad index: a slot or page id out of
// range reads slot 0, a position outside the RoPE tables is clamped.  That
// keeps a malformed call from taking the GPU down, but it turns a caller's
// bug into plausible numbers.  The reference raises instead -- the pool's
// IndexError/ValueError on bad page ids (runtime/kv_cache.py:305-310,
// 357-476) and the kernel wrapper's ValueError on a bad geometry
// (runtime/pic_attention.py:197-213).  These kernels give the host the same
// answer for the index arrays: each counts the entries an attention call
// would read out of range into a caller-zeroed int32 status vector, and the
// host layer turns non-zero counts into ValueError.  Nothing traps; every
// workgroup exits normally.  Counts are reduced per wavefront and added with
// one vector atomic per wavefront.
#include "common.h"

namespace voom {
namespace {

constexpr int kChkThreads = 256;

// Adds this lane's count to *dst once per wavefront.
__device__ __forceinline__ void wave_count_add(int32_t* dst, int n) {
  const float total = wave_sum_uniform(static_cast<float>(n));
  if ((threadIdx.x & (kWave - 1)) == 0 && total > 0.f)
    atomicAdd(dst, static_cast<int32_t>(total));
}

// Thread per (sequence, table column); a column counts when it lies inside
// the sequence's context.  status[0]: slot ids outside [0, num_slots) inside
// a context; status[1]: context lengths outside [0, max_pages * page_tokens]
// (counted once per sequence, by column 0).
__global__ __launch_bounds__(kChkThreads) void check_table_kernel(
    const int32_t* table, const int32_t* ctx, int32_t* status, int batch, int max_pages,
    int page_tokens, int num_slots) {
  int bad_slot = 0, bad_ctx = 0;
  const long long n = static_cast<long long>(batch) * max_pages;
  for (long long i = blockIdx.x * static_cast<long long>(kChkThreads) + threadIdx.x; i < n;
       i += static_cast<long long>(gridDim.x) * kChkThreads) {
    const int b = static_cast<int>(i / max_pages);
    const int p = static_cast<int>(i - static_cast<long long>(b) * max_pages);
    const int c = ctx[b];
    const long long cap = static_cast<long long>(max_pages) * page_tokens;
    if (p == 0 && (c < 0 || c > cap)) ++bad_ctx;
    const long long used = c <= 0 ? 0 : (static_cast<long long>(c) + page_tokens - 1) / page_tokens;
    if (p < used) {
      const int s = table[i];
      if (static_cast<unsigned>(s) >= static_cast<unsigned>(num_slots)) ++bad_slot;
    }
  }
  wave_count_add(status + 0, bad_slot);
  wave_count_add(status + 1, bad_ctx);
}

// Thread per selected entry (the sparse latent contraction reads position p
// of sequence b through table column p / page_tokens).  status[0]: slot ids
// outside [0, num_slots) that a used position reads; status[2]: used
// positions outside [0, max_pages * page_tokens); status[3]: sel_lens outside
// [0, k] (counted by entry 0).
__global__ __launch_bounds__(kChkThreads) void check_selection_kernel(
    const int32_t* sel, const int32_t* sel_lens, const int32_t* table, int32_t* status,
    int batch, int k, int max_pages, int page_tokens, int num_slots) {
  int bad_slot = 0, bad_pos = 0, bad_len = 0;
  const long long n = static_cast<long long>(batch) * k;
  for (long long i = blockIdx.x * static_cast<long long>(kChkThreads) + threadIdx.x; i < n;
       i += static_cast<long long>(gridDim.x) * kChkThreads) {
    const int b = static_cast<int>(i / k);
    const int j = static_cast<int>(i - static_cast<long long>(b) * k);
    const int len = sel_lens[b];
    if (j == 0 && (len < 0 || len > k)) ++bad_len;
    if (j < len) {
      const int pos = sel[i];
      if (pos < 0 || pos / page_tokens >= max_pages) {
        ++bad_pos;
      } else {
        const int s = table[static_cast<long long>(b) * max_pages + pos / page_tokens];
        if (static_cast<unsigned>(s) >= static_cast<unsigned>(num_slots)) ++bad_slot;
      }
    }
  }
  wave_count_add(status + 0, bad_slot);
  wave_count_add(status + 2, bad_pos);
  wave_count_add(status + 3, bad_len);
}

// Thread per key.  status[0]: page ids of the keys' table entries outside
// [0, num_pages) (one count per key that reads one); status[1]: key positions
// outside [0, max_position).
__global__ __launch_bounds__(kChkThreads) void check_pf_kernel(
    const int32_t* table, const int32_t* kpos, int32_t* status, int num_keys, int block_size,
    int num_pages, int max_position) {
  int bad_page = 0, bad_pos = 0;
  for (long long i = blockIdx.x * static_cast<long long>(kChkThreads) + threadIdx.x;
       i < num_keys; i += static_cast<long long>(gridDim.x) * kChkThreads) {
    const int page = table[i / block_size];
    if (static_cast<unsigned>(page) >= static_cast<unsigned>(num_pages)) ++bad_page;
    const int p = kpos[i];
    if (p < 0 || p >= max_position) ++bad_pos;
  }
  wave_count_add(status + 0, bad_page);
  wave_count_add(status + 1, bad_pos);
}

unsigned check_grid(long long n) {
  long long g = (n + kChkThreads - 1) / kChkThreads;
  if (g > 1024) g = 1024;
  return static_cast<unsigned>(g < 1 ? 1 : g);
}

}  // namespace
}  // namespace voom

using namespace voom;

extern "C" int voom_check_block_table(const int32_t* block_table, const int32_t* ctx_lens,
                                      int32_t* status, int batch, int max_pages,
                                      int page_tokens, int num_slots, hipStream_t stream) {
  VOOM_REQUIRE(block_table && ctx_lens && status, "check_block_table: null pointer argument");
  VOOM_REQUIRE(batch > 0 && max_pages > 0 && page_tokens > 0 && num_slots >= 0,
               "check_block_table: bad geometry");
  hipLaunchKernelGGL(check_table_kernel,
                     dim3(check_grid(static_cast<long long>(batch) * max_pages)),
                     dim3(kChkThreads), 0, stream, block_table, ctx_lens, status, batch,
                     max_pages, page_tokens, num_slots);
  return VOOM_LAUNCH_CHECK("check_block_table: launch");
}

extern "C" int voom_check_selection(const int32_t* sel, const int32_t* sel_lens,
                                    const int32_t* block_table, int32_t* status, int batch,
                                    int k, int max_pages, int page_tokens, int num_slots,
                                    hipStream_t stream) {
  VOOM_REQUIRE(sel && sel_lens && block_table && status, "check_selection: null pointer argument");
  VOOM_REQUIRE(batch > 0 && k > 0 && max_pages > 0 && page_tokens > 0 && num_slots >= 0,
               "check_selection: bad geometry");
  hipLaunchKernelGGL(check_selection_kernel,
                     dim3(check_grid(static_cast<long long>(batch) * k)), dim3(kChkThreads), 0,
                     stream, sel, sel_lens, block_table, status, batch, k, max_pages,
                     page_tokens, num_slots);
  return VOOM_LAUNCH_CHECK("check_selection: launch");
}

extern "C" int voom_check_position_free_pages(const int32_t* block_table,
                                              const int32_t* key_positions, int32_t* status,
                                              int num_keys, int block_size, int num_pages,
                                              int max_position, hipStream_t stream) {
  VOOM_REQUIRE(status, "check_position_free_pages: null status");
  VOOM_REQUIRE(num_keys >= 0 && block_size > 0 && num_pages >= 0 && max_position > 0,
               "check_position_free_pages: bad geometry");
  if (num_keys == 0) return VOOM_OK;
  VOOM_REQUIRE(block_table && key_positions, "check_position_free_pages: null key arrays");
  hipLaunchKernelGGL(check_pf_kernel, dim3(check_grid(num_keys)), dim3(kChkThreads), 0, stream,
                     block_table, key_positions, status, num_keys, block_size, num_pages,
                     max_position);
  return VOOM_LAUNCH_CHECK("check_position_free_pages: launch");
}
