// Page writes (append) and logical gathers for the device page pools.
//
// K pool [slots, NKV, PT, D] is token-major; V pool [slots, NKV, PT/VB, D, VB]
// with VB = min(PT, 32) keeps each 32-token block of a page transposed (V^T,
// one 64-byte row of 32 tokens per dim) so decode attention reads every block
// of K and V as one contiguous run and feeds V^T straight into MFMA operands.  Appending is a
// 16-byte row store for K and a 32-element-strided column store for V; both
// are tiny next to attention (one token per step).
#include "common.h"

namespace voom {
namespace {

constexpr int kThreads = 256;

// Element offset of V(token off, dim d) inside the V^T blocks of one head
// page: block off / VB of [D, VB], VB = 1 << vb_shift = min(PT, 32).
__device__ __forceinline__ size_t v_offset(size_t head_page, int pt_shift, int vb_shift,
                                           int off, int D, int d) {
  const size_t blk = (head_page << (pt_shift - vb_shift)) + (off >> vb_shift);
  return ((blk * D + d) << vb_shift) + (off & ((1 << vb_shift) - 1));
}

// One thread per (b, h, t, 8-dim chunk) of the new tokens.
__global__ __launch_bounds__(kThreads) void append_kernel(
    const uint16_t* __restrict__ k_new, const uint16_t* __restrict__ v_new,
    uint16_t* __restrict__ k_pool, uint16_t* __restrict__ v_pool,
    const int32_t* __restrict__ table, const int32_t* __restrict__ positions, int B, int NKV,
    int L, int D, int pt_shift, int max_pages, int num_slots) {
  const int chunks = D / 8;
  const long long total = static_cast<long long>(B) * NKV * L * chunks;
  const long long idx = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
  if (idx >= total) return;
  const int c = static_cast<int>(idx % chunks);
  long long rest = idx / chunks;
  const int t = static_cast<int>(rest % L);
  rest /= L;
  const int h = static_cast<int>(rest % NKV);
  const int b = static_cast<int>(rest / NKV);
  const int pos = positions[b] + t;
  if (pos < 0) return;
  const int page = pos >> pt_shift;
  if (page >= max_pages) return;
  const int off = pos & ((1 << pt_shift) - 1);
  const int slot = table[static_cast<size_t>(b) * max_pages + page];
  if (static_cast<unsigned>(slot) >= static_cast<unsigned>(num_slots)) return;
  const size_t src = ((static_cast<size_t>(b) * NKV + h) * L + t) * D + c * 8;
  const size_t head_page = static_cast<size_t>(slot) * NKV + h;
  // K row store.
  *reinterpret_cast<u32x4*>(k_pool + ((head_page << pt_shift) + off) * D + c * 8) =
      *reinterpret_cast<const u32x4*>(k_new + src);
  // V column store (transposed page).
  const u32x4 v = *reinterpret_cast<const u32x4*>(v_new + src);
  const int vb_shift = pt_shift < 5 ? pt_shift : 5;
  uint16_t* vcol = v_pool + v_offset(head_page, pt_shift, vb_shift, off, D, c * 8);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t w = v[e >> 1];
    vcol[e << vb_shift] = static_cast<uint16_t>((e & 1) ? (w >> 16) : (w & 0xffff));
  }
}

// One thread per (b, h, position, 8-dim chunk) of the logical output.
__global__ __launch_bounds__(kThreads) void gather_kernel(
    const uint16_t* __restrict__ k_pool, const uint16_t* __restrict__ v_pool,
    const int32_t* __restrict__ table, uint16_t* __restrict__ k_out,
    uint16_t* __restrict__ v_out, int B, int NKV, int S, int D, int pt_shift, int max_pages,
    int num_slots) {
  const int chunks = D / 8;
  const long long total = static_cast<long long>(B) * NKV * S * chunks;
  const long long idx = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
  if (idx >= total) return;
  const int c = static_cast<int>(idx % chunks);
  long long rest = idx / chunks;
  const int pos = static_cast<int>(rest % S);
  rest /= S;
  const int h = static_cast<int>(rest % NKV);
  const int b = static_cast<int>(rest / NKV);
  const size_t dst = ((static_cast<size_t>(b) * NKV + h) * S + pos) * D + c * 8;
  const int page = pos >> pt_shift;
  const int off = pos & ((1 << pt_shift) - 1);
  const int slot = page < max_pages ? table[static_cast<size_t>(b) * max_pages + page] : -1;
  if (static_cast<unsigned>(slot) >= static_cast<unsigned>(num_slots)) {
    const u32x4 z = {0u, 0u, 0u, 0u};
    *reinterpret_cast<u32x4*>(k_out + dst) = z;
    *reinterpret_cast<u32x4*>(v_out + dst) = z;
    return;
  }
  const size_t head_page = static_cast<size_t>(slot) * NKV + h;
  *reinterpret_cast<u32x4*>(k_out + dst) =
      *reinterpret_cast<const u32x4*>(k_pool + ((head_page << pt_shift) + off) * D + c * 8);
  const int vb_shift = pt_shift < 5 ? pt_shift : 5;
  const uint16_t* vcol = v_pool + v_offset(head_page, pt_shift, vb_shift, off, D, c * 8);
  u32x4 v;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    v[w] = static_cast<uint32_t>(vcol[(2 * w) << vb_shift]) |
           (static_cast<uint32_t>(vcol[(2 * w + 1) << vb_shift]) << 16);
  }
  *reinterpret_cast<u32x4*>(v_out + dst) = v;
}

// Token-row pages (the MLA latent cache): pool [slots, PT, W].  One thread per
// (b, t, 16-byte chunk) of the rows being written or read.
__global__ __launch_bounds__(kThreads) void append_rows_kernel(
    const uint16_t* __restrict__ src, uint16_t* __restrict__ pool,
    const int32_t* __restrict__ table, const int32_t* __restrict__ positions, int B, int L,
    int W, int pt_shift, int max_pages, int num_slots) {
  const int chunks = W / 8;
  const long long total = static_cast<long long>(B) * L * chunks;
  const long long idx = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
  if (idx >= total) return;
  const int c = static_cast<int>(idx % chunks);
  const long long rest = idx / chunks;
  const int t = static_cast<int>(rest % L);
  const int b = static_cast<int>(rest / L);
  const int pos = positions[b] + t;
  if (pos < 0) return;
  const int page = pos >> pt_shift;
  if (page >= max_pages) return;
  const int slot = table[static_cast<size_t>(b) * max_pages + page];
  if (static_cast<unsigned>(slot) >= static_cast<unsigned>(num_slots)) return;
  const size_t off = (pos & ((1 << pt_shift) - 1));
  *reinterpret_cast<u32x4*>(pool + ((static_cast<size_t>(slot) << pt_shift) + off) * W + c * 8) =
      *reinterpret_cast<const u32x4*>(src + (static_cast<size_t>(b) * L + t) * W + c * 8);
}

__global__ __launch_bounds__(kThreads) void gather_rows_kernel(
    const uint16_t* __restrict__ pool, const int32_t* __restrict__ table,
    uint16_t* __restrict__ dst, int B, int S, int W, int pt_shift, int max_pages, int num_slots) {
  const int chunks = W / 8;
  const long long total = static_cast<long long>(B) * S * chunks;
  const long long idx = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
  if (idx >= total) return;
  const int c = static_cast<int>(idx % chunks);
  const long long rest = idx / chunks;
  const int pos = static_cast<int>(rest % S);
  const int b = static_cast<int>(rest / S);
  const int page = pos >> pt_shift;
  const int slot = page < max_pages ? table[static_cast<size_t>(b) * max_pages + page] : -1;
  u32x4 v = {0u, 0u, 0u, 0u};
  if (static_cast<unsigned>(slot) < static_cast<unsigned>(num_slots)) {
    const size_t off = pos & ((1 << pt_shift) - 1);
    v = *reinterpret_cast<const u32x4*>(pool + ((static_cast<size_t>(slot) << pt_shift) + off) * W +
                                        c * 8);
  }
  *reinterpret_cast<u32x4*>(dst + (static_cast<size_t>(b) * S + pos) * W + c * 8) = v;
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace
}  // namespace voom

using namespace voom;

extern "C" int voom_append_kv(const void* k_new, const void* v_new, void* k_pool, void* v_pool,
                              const int32_t* block_table, const int32_t* positions, int batch,
                              int num_kv_heads, int new_tokens, int head_dim, int page_tokens,
                              int max_pages, int num_slots, hipStream_t stream) {
  VOOM_REQUIRE(k_new && v_new && k_pool && v_pool && block_table && positions,
               "append_kv: null pointer");
  VOOM_REQUIRE(batch > 0 && num_kv_heads > 0 && new_tokens >= 0 && max_pages > 0 &&
                   num_slots > 0,
               "append_kv: bad geometry");
  VOOM_REQUIRE(head_dim > 0 && head_dim % 8 == 0, "append_kv: head_dim %d not a multiple of 8",
               head_dim);
  VOOM_REQUIRE(is_pow2(page_tokens) && page_tokens <= 4096,
               "append_kv: page_tokens %d must be a power of two <= 4096", page_tokens);
  VOOM_REQUIRE(aligned16(k_new) && aligned16(v_new) && aligned16(k_pool) && aligned16(v_pool),
               "append_kv: buffers must be 16-byte aligned");
  if (new_tokens == 0) return VOOM_OK;
  const long long total =
      static_cast<long long>(batch) * num_kv_heads * new_tokens * (head_dim / 8);
  const dim3 grid(static_cast<unsigned>((total + kThreads - 1) / kThreads));
  hipLaunchKernelGGL(append_kernel, grid, dim3(kThreads), 0, stream,
                     static_cast<const uint16_t*>(k_new), static_cast<const uint16_t*>(v_new),
                     static_cast<uint16_t*>(k_pool), static_cast<uint16_t*>(v_pool), block_table,
                     positions, batch, num_kv_heads, new_tokens, head_dim, ilog2(page_tokens),
                     max_pages, num_slots);
  return VOOM_LAUNCH_CHECK("append_kv: launch");
}

extern "C" int voom_gather_kv(const void* k_pool, const void* v_pool, const int32_t* block_table,
                              void* k_out, void* v_out, int batch, int num_kv_heads, int seq_len,
                              int head_dim, int page_tokens, int max_pages, int num_slots,
                              hipStream_t stream) {
  VOOM_REQUIRE(k_pool && v_pool && block_table && k_out && v_out, "gather_kv: null pointer");
  VOOM_REQUIRE(batch > 0 && num_kv_heads > 0 && seq_len >= 0 && max_pages > 0 && num_slots > 0,
               "gather_kv: bad geometry");
  VOOM_REQUIRE(head_dim > 0 && head_dim % 8 == 0, "gather_kv: head_dim %d not a multiple of 8",
               head_dim);
  VOOM_REQUIRE(is_pow2(page_tokens) && page_tokens <= 4096,
               "gather_kv: page_tokens %d must be a power of two <= 4096", page_tokens);
  VOOM_REQUIRE(aligned16(k_out) && aligned16(v_out) && aligned16(k_pool) && aligned16(v_pool),
               "gather_kv: buffers must be 16-byte aligned");
  if (seq_len == 0) return VOOM_OK;
  const long long total = static_cast<long long>(batch) * num_kv_heads * seq_len * (head_dim / 8);
  const dim3 grid(static_cast<unsigned>((total + kThreads - 1) / kThreads));
  hipLaunchKernelGGL(gather_kernel, grid, dim3(kThreads), 0, stream,
                     static_cast<const uint16_t*>(k_pool), static_cast<const uint16_t*>(v_pool),
                     block_table, static_cast<uint16_t*>(k_out), static_cast<uint16_t*>(v_out),
                     batch, num_kv_heads, seq_len, head_dim, ilog2(page_tokens), max_pages,
                     num_slots);
  return VOOM_LAUNCH_CHECK("gather_kv: launch");
}

extern "C" int voom_append_rows(const void* src, void* pool, const int32_t* block_table,
                                const int32_t* positions, int batch, int new_tokens,
                                int row_elems, int page_tokens, int max_pages, int num_slots,
                                hipStream_t stream) {
  VOOM_REQUIRE(src && pool && block_table && positions, "append_rows: null pointer");
  VOOM_REQUIRE(batch > 0 && new_tokens >= 0 && max_pages > 0 && num_slots > 0,
               "append_rows: bad geometry");
  VOOM_REQUIRE(row_elems > 0 && row_elems % 8 == 0,
               "append_rows: row_elems %d not a multiple of 8", row_elems);
  VOOM_REQUIRE(is_pow2(page_tokens) && page_tokens <= 4096,
               "append_rows: page_tokens %d must be a power of two <= 4096", page_tokens);
  VOOM_REQUIRE(aligned16(src) && aligned16(pool), "append_rows: buffers must be 16-byte aligned");
  if (new_tokens == 0) return VOOM_OK;
  const long long total = static_cast<long long>(batch) * new_tokens * (row_elems / 8);
  hipLaunchKernelGGL(append_rows_kernel, dim3(static_cast<unsigned>((total + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, stream, static_cast<const uint16_t*>(src),
                     static_cast<uint16_t*>(pool), block_table, positions, batch, new_tokens,
                     row_elems, ilog2(page_tokens), max_pages, num_slots);
  return VOOM_LAUNCH_CHECK("append_rows: launch");
}

extern "C" int voom_gather_rows(const void* pool, const int32_t* block_table, void* dst, int batch,
                                int seq_len, int row_elems, int page_tokens, int max_pages,
                                int num_slots, hipStream_t stream) {
  VOOM_REQUIRE(pool && block_table && dst, "gather_rows: null pointer");
  VOOM_REQUIRE(batch > 0 && seq_len >= 0 && max_pages > 0 && num_slots > 0,
               "gather_rows: bad geometry");
  VOOM_REQUIRE(row_elems > 0 && row_elems % 8 == 0,
               "gather_rows: row_elems %d not a multiple of 8", row_elems);
  VOOM_REQUIRE(is_pow2(page_tokens) && page_tokens <= 4096,
               "gather_rows: page_tokens %d must be a power of two <= 4096", page_tokens);
  VOOM_REQUIRE(aligned16(pool) && aligned16(dst), "gather_rows: buffers must be 16-byte aligned");
  if (seq_len == 0) return VOOM_OK;
  const long long total = static_cast<long long>(batch) * seq_len * (row_elems / 8);
  hipLaunchKernelGGL(gather_rows_kernel, dim3(static_cast<unsigned>((total + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, stream, static_cast<const uint16_t*>(pool), block_table,
                     static_cast<uint16_t*>(dst), batch, seq_len, row_elems, ilog2(page_tokens),
                     max_pages, num_slots);
  return VOOM_LAUNCH_CHECK("gather_rows: launch");
}
