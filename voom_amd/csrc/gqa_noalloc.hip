// Allocation-free variant of voom_paged_gqa_decode for callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).  It has no counterpart in the reference.
#include <mutex>

#include "common.h"

// ---------------------------------------------------------------------------
// Allocation-free decode: the split partials live in a file-scope device
// array instead of a caller workspace.  Each device holds its own copy of the
// array for the life of the process; its address is resolved once per device
// with hipGetSymbolAddress and only that address is handed to kernels.  The
// partials kernel writes every slot the combine later reads, so nothing needs
// clearing between calls.  Calls that overlap on one device share the array
// and race.
namespace voom {
namespace {

constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of this device's scratch array (resolved on first use).
int scratch_address(hipStream_t stream, void** out) {
  int dev = -1;
  int rc = check_hip(hipGetDevice(&dev), "paged_gqa_decode_noalloc: hipGetDevice");
  if (rc) return rc;
  VOOM_REQUIRE(dev >= 0 && dev < kMaxDevices, "paged_gqa_decode_noalloc: device %d", dev);
  if (stream != nullptr) {
    int sdev = -1;
    rc = check_hip(hipStreamGetDevice(stream, &sdev), "paged_gqa_decode_noalloc: stream device");
    if (rc) return rc;
    VOOM_REQUIRE(sdev == dev,
                 "paged_gqa_decode_noalloc: stream is on device %d, current device is %d",
                 sdev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    rc = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)),
                   "paged_gqa_decode_noalloc: hipGetSymbolAddress(scratch)");
    if (rc) return rc;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return VOOM_OK;
}

}  // namespace
}  // namespace voom

using namespace voom;

extern "C" size_t voom_paged_gqa_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int voom_paged_gqa_decode_noalloc(const void* q, const void* k_pool,
                                             const void* v_pool, const int32_t* block_table,
                                             const int32_t* ctx_lens, void* out, float* lse_out,
                                             int batch, int num_q_heads, int num_kv_heads,
                                             int head_dim, int page_tokens, int max_pages,
                                             int num_slots, float scale, int num_splits,
                                             hipStream_t stream) {
  const char* who = "paged_gqa_decode_noalloc";
  VOOM_REQUIRE(batch > 0 && num_q_heads > 0 && num_kv_heads > 0 && head_dim > 0,
               "%s: bad geometry", who);
  const size_t need = voom_paged_gqa_workspace_bytes(batch, num_q_heads, num_kv_heads,
                                                      head_dim, num_splits);
  VOOM_REQUIRE(need <= kNoAllocScratchBytes,
               "%s: the split partials need %zu bytes, more than the %zu-byte scratch array "
               "(fewer sequences or splits, or voom_paged_gqa_decode with a workspace)",
               who, need, kNoAllocScratchBytes);
  void* ws = nullptr;
  const int rc = scratch_address(stream, &ws);
  if (rc) return rc;
  return voom_paged_gqa_decode(q, k_pool, v_pool, block_table, ctx_lens, out, lse_out, ws,
                               kNoAllocScratchBytes, batch, num_q_heads, num_kv_heads,
                               head_dim, page_tokens, max_pages, num_slots, scale, num_splits,
                               stream);
}
