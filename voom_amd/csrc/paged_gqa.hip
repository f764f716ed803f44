// Paged GQA decode attention for gfx950.
//
// One query token per sequence attends over its logical KV, which lives in
// fixed-size pages scattered through a shared device pool and is addressed
// through a per-sequence block table.  This replaces the reference's decode
// step, which concatenates every page of the layer (runtime/kv_paged.py:164-181)
// and then calls MLX SDPA with the GQA broadcast (runtime/layer_runner.py:
// 179-180); the page indexing follows the reference's Metal paged kernel
// (runtime/pic_attention.py:60-65) with V stored as transposed 32-token blocks
// inside a page: V pool [slots, NKV, PT/32, D, 32], so a wavefront's K block
// (32 x D) and V^T block (D x 32) are each one contiguous 64*D-byte run.
//
// Work decomposition (balanced split-K over 32-token blocks):
//   A "unit" is one 32-token block of one (sequence, kv-head) segment.  The
//   units of all segments are laid end to end, (b, kvh, block) in that order,
//   and wavefront w of W takes units [w*U/W, (w+1)*U/W).  Every wavefront
//   therefore streams the same number of KV bytes whatever the context
//   lengths, and it emits one partial softmax state (m, l, o) per segment
//   piece it touches into slot (segment + w) of the workspace.  The slots of a
//   segment are contiguous, so the reduce kernel finds them arithmetically.
//
// Per 32-token block a wavefront issues 2*(D/32) K loads and D/16 V loads of
// 16 bytes per lane that land directly in MFMA operand registers:
//   scores^T[token][head] = K[token][:] . Q^T          v_mfma_f32_16x16x32_bf16
//   out^T[dim][head]     += V^T[dim][token] . P^T      v_mfma_f32_16x16x32_bf16
// with the GQA heads of one KV head in the N dimension (<= 16), so each K/V
// byte is read from HBM once for all heads that share it.  The 16 token rows of
// the two score tiles are permuted (tile t row 4g+r holds token 8g+4t+r) so
// that the score accumulators of lane group g are exactly the 8 consecutive
// tokens that the P^T operand of the same lane needs: no lane shuffles are
// required between the two products.
#include "common.h"

namespace voom {
namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / kWave;
constexpr int kMaxBatch = 1024;
constexpr int kBlockTokens = 32;

// Pipeline depth (32-token blocks in flight per wavefront) and the occupancy
// target handed to the register allocator, per head_dim.
#ifndef VOOM_GQA_NBUF_128
#define VOOM_GQA_NBUF_128 3
#endif
#ifndef VOOM_GQA_WAVES_PER_EU_128
#define VOOM_GQA_WAVES_PER_EU_128 1
#endif
// Cache policy (buffer-load aux bits) of the K and V streams.  Every byte of
// a block is read exactly once and the blocks are contiguous, so both streams
// load non-temporal (aux bit 1): measured 6.37 TB/s for the partials kernel
// against 5.6 TB/s with ordinary loads at the Llama-3-8B 32k shape.
#ifndef VOOM_GQA_K_CACHE_POLICY
#define VOOM_GQA_K_CACHE_POLICY 2
#endif
#ifndef VOOM_GQA_CACHE_POLICY
#define VOOM_GQA_CACHE_POLICY 2
#endif
#ifndef VOOM_GQA_SPLITS_PER_CU
#define VOOM_GQA_SPLITS_PER_CU 4
#endif
constexpr int kNbuf128 = VOOM_GQA_NBUF_128;
constexpr int kWavesPerEu128 = VOOM_GQA_WAVES_PER_EU_128;
#ifndef VOOM_GQA_NBUF_64
#define VOOM_GQA_NBUF_64 3
#endif
constexpr int kNbuf64 = VOOM_GQA_NBUF_64;
constexpr int kWavesPerEu64 = 2;

// Exclusive prefix sum of per-sequence 32-token block counts into seg[0..B].
// Requires blockDim.x == kThreads; ends with a barrier.
__device__ void build_block_prefix(const int32_t* __restrict__ ctx_lens, int B,
                                   int cap_tokens, int* seg, int* wave_tot) {
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1);
  const int wv = t / kWave;
  int carry = 0;
  for (int base = 0; base < B; base += kThreads) {
    const int i = base + t;
    int n = 0;
    if (i < B) {
      int c = ctx_lens[i];
      c = c < 0 ? 0 : (c > cap_tokens ? cap_tokens : c);
      n = (c + kBlockTokens - 1) / kBlockTokens;
    }
    const int x = wave_inclusive_scan(n, lane);
    if (lane == kWave - 1) wave_tot[wv] = x;
    __syncthreads();
    int pre = carry;
    for (int k = 0; k < wv; ++k) pre += wave_tot[k];
    if (i < B) seg[i] = pre + x - n;
    int chunk = 0;
    for (int k = 0; k < kWavesPerBlock; ++k) chunk += wave_tot[k];
    __syncthreads();
    carry += chunk;
  }
  if (t == 0) seg[B] = carry;
  __syncthreads();
}

template <int D>
struct BlockRegs {
  u32x4 k[2][D / 32];  // two 16-token score tiles x (D/32) k-steps
  u32x4 v[D / 16];     // D/16 dimension tiles of V^T, 8 tokens per lane
};

struct SegmentArgs {
  const uint16_t* __restrict__ k_pool;
  const uint16_t* __restrict__ v_pool;
  const int32_t* __restrict__ table_row;
  int n_pages;   // pages addressable through table_row
  int kvh;
  int nkv;
  int pt_shift;  // log2(page_tokens)
  int num_slots;
  int ctx;       // tokens of this sequence (clamped to table capacity)
};

// Buffer resource covering one head-page: out-of-range offsets read as zero,
// so no load of a well-formed call can leave the page.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t page_rsrc(const uint16_t* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), static_cast<short>(0),
                                           bytes, 0x00020000);
}

// Lane-constant byte offsets of the MFMA operand loads inside a 32-token block.
struct LaneOffsets {
  int k;  // K row (8*(i16/4) + i16%4) x D + 8g, in bytes
  int v;  // V^T row i16 x PT + 8g, in bytes
};

// Loads block bi of the segment into r.  A block past the end of the piece
// (bi >= bhi) is issued against an empty descriptor: the loads complete with
// zeros and move no bytes, which keeps the pipeline's wait counts
// branch-free without re-reading memory.
template <int D>
__device__ __forceinline__ void load_block(BlockRegs<D>& r, const SegmentArgs& a, int bi,
                                           int bhi, int& tab_base, int& tab, int lane,
                                           const LaneOffsets& lo) {
  const bool live = bi < bhi;
  if (!live) bi = bhi - 1;
  const int sub_shift = a.pt_shift - 5;
  const int page = bi >> sub_shift;
  const int sub = bi & ((1 << sub_shift) - 1);
  if (page >= tab_base + kWave) {
    tab_base = page;
    const int p = tab_base + lane;
    tab = p < a.n_pages ? a.table_row[p] : 0;
    // Wait here, on this rare path, for the window.  Without it the compiler
    // cannot tell at the readlane below whether a table load is outstanding,
    // and waits for every load in flight there -- the blocks the ring has
    // prefetched included -- on every block.
    wait_vmem_all();
  }
  int slot = __builtin_amdgcn_readlane(tab, page - tab_base);
  if (static_cast<unsigned>(slot) >= static_cast<unsigned>(a.num_slots)) slot = 0;
  const size_t head_page = static_cast<size_t>(slot) * a.nkv + a.kvh;
  const int page_elems = D << a.pt_shift;
  const int page_bytes = live ? page_elems * 2 : 0;
  const __amdgpu_buffer_rsrc_t kr = page_rsrc(a.k_pool + head_page * page_elems, page_bytes);
  const __amdgpu_buffer_rsrc_t vr = page_rsrc(a.v_pool + head_page * page_elems, page_bytes);
  const int k_sub = sub * kBlockTokens * D * 2;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int s = 0; s < D / 32; ++s) {
      r.k[t][s] = __builtin_amdgcn_raw_buffer_load_b128(kr, lo.k + (4 * t * D + 32 * s) * 2,
                                                        k_sub, VOOM_GQA_K_CACHE_POLICY);
    }
  }
  const int v_sub = k_sub;  // V^T blocks are [D, 32]: same bytes per block as K
  const int v_tile = 16 * kBlockTokens * 2;
#pragma unroll
  for (int n = 0; n < D / 16; ++n) {
    r.v[n] = __builtin_amdgcn_raw_buffer_load_b128(vr, lo.v, v_sub + n * v_tile,
                                                   VOOM_GQA_CACHE_POLICY);
  }
}

template <int D>
struct SoftmaxState {
  f32x4 acc[D / 16];
  float m;
  float l;
};

template <int D>
__device__ __forceinline__ void compute_block(const BlockRegs<D>& r, const u32x4* qop,
                                              SoftmaxState<D>& st, int valid,
                                              float scale_log2e, int lane) {
  const int g = lane >> 4;
  f32x4 s0 = {0.f, 0.f, 0.f, 0.f};
  f32x4 s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < D / 32; ++s) {
    const bf16x8 qb = __builtin_bit_cast(bf16x8, qop[s]);
    s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, r.k[0][s]), qb,
                                                 s0, 0, 0, 0);
    s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, r.k[1][s]), qb,
                                                 s1, 0, 0, 0);
  }
  // Lane (head j, group g) now holds tokens 8g+e, e = 0..7, of this block.
  float x[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    x[e] = s0[e] * scale_log2e;
    x[4 + e] = s1[e] * scale_log2e;
  }
  u32x4 vv[D / 16];
#pragma unroll
  for (int n = 0; n < D / 16; ++n) vv[n] = r.v[n];
  if (valid < kBlockTokens) {
    // Tail block: tokens past the context are garbage (possibly NaN) in the
    // pool, so they are removed by selection, never by arithmetic.
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (8 * g + e >= valid) x[e] = -INFINITY;
    }
#pragma unroll
    for (int n = 0; n < D / 16; ++n) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const bool lo_ok = 8 * g + 2 * w < valid;
        const bool hi_ok = 8 * g + 2 * w + 1 < valid;
        const unsigned mask = (lo_ok ? 0x0000ffffu : 0u) | (hi_ok ? 0xffff0000u : 0u);
        vv[n][w] &= mask;
      }
    }
  }
  float mb = x[0];
#pragma unroll
  for (int e = 1; e < 8; ++e) mb = fmaxf(mb, x[e]);
  mb = wave_max_across_groups(mb);
  const float m_new = fmaxf(st.m, mb);
  const float alpha = fast_exp2(st.m - m_new);
  float p[8];
  float psum = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) p[e] = fast_exp2(x[e] - m_new);
  u32x4 pk;
  pk[0] = pack_bf16x2(p[0], p[1]);
  pk[1] = pack_bf16x2(p[2], p[3]);
  pk[2] = pack_bf16x2(p[4], p[5]);
  pk[3] = pack_bf16x2(p[6], p[7]);
  // The normaliser sums the same bf16-rounded weights the MFMA consumes, so
  // the output is an exact convex combination of V rows up to fp32 rounding.
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    psum += __builtin_bit_cast(float, pk[w] << 16) + __builtin_bit_cast(float, pk[w] & 0xffff0000u);
  }
  st.l = st.l * alpha + psum;
  st.m = m_new;
  const bf16x8 pb = __builtin_bit_cast(bf16x8, pk);
#pragma unroll
  for (int n = 0; n < D / 16; ++n) {
    st.acc[n] *= alpha;
    st.acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, vv[n]), pb,
                                                        st.acc[n], 0, 0, 0);
  }
}

template <int D, int NBUF, int WAVES_PER_EU>
__global__ __launch_bounds__(kThreads, WAVES_PER_EU) void gqa_decode_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_pool,
    const uint16_t* __restrict__ v_pool, const int32_t* __restrict__ block_table,
    const int32_t* __restrict__ ctx_lens, float* __restrict__ part_o,
    float* __restrict__ part_ml, int B, int NKV, int G, int max_pages, int pt_shift,
    int num_slots, float scale_log2e, int W) {
  __shared__ int seg[kMaxBatch + 1];
  __shared__ int wave_tot[kWavesPerBlock];
  const int cap_tokens = max_pages << pt_shift;
  build_block_prefix(ctx_lens, B, cap_tokens, seg, wave_tot);

  const int lane = threadIdx.x & (kWave - 1);
  // Wave-uniform values are pinned to scalar registers: LDS reads are
  // per-lane as far as the compiler knows, and the buffer descriptors built
  // from them must be scalar.
  const int w = blockIdx.x * kWavesPerBlock + uniform(threadIdx.x / kWave);
  const long long U = static_cast<long long>(uniform(seg[B])) * NKV;
  // Never more wavefronts than units: every active wavefront then owns at
  // least one unit, which the reduce kernel relies on.
  const int We = static_cast<int>(U < W ? U : W);
  if (w >= We) return;
  long long u0 = static_cast<long long>(w) * U / We;
  const long long u1 = static_cast<long long>(w + 1) * U / We;

  // Sequence holding unit u0: the largest b with NKV*seg[b] <= u0.
  int lo = 0, hi = B - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (static_cast<long long>(uniform(seg[mid])) * NKV <= u0) lo = mid; else hi = mid - 1;
  }
  int b = lo;
  int nb = uniform(seg[b + 1]) - uniform(seg[b]);
  int kvh = static_cast<int>((u0 - static_cast<long long>(uniform(seg[b])) * NKV) / nb);
  long long S = static_cast<long long>(uniform(seg[b])) * NKV + static_cast<long long>(kvh) * nb;

  const int NQ = NKV * G;
  const int i16 = lane & 15;
  const int g = lane >> 4;
  const bool head_ok = i16 < G;
  LaneOffsets lofs;
  lofs.k = ((8 * (i16 >> 2) + (i16 & 3)) * D + 8 * g) * 2;
  lofs.v = ((i16 * kBlockTokens) + 8 * g) * 2;

  while (true) {
    const long long send = S + nb;
    const int blo = static_cast<int>(u0 - S);
    const int bhi = static_cast<int>((u1 < send ? u1 : send) - S);

    SegmentArgs a;
    a.k_pool = k_pool;
    a.v_pool = v_pool;
    a.table_row = block_table + static_cast<size_t>(b) * max_pages;
    a.n_pages = max_pages;
    a.kvh = kvh;
    a.nkv = NKV;
    a.pt_shift = pt_shift;
    a.num_slots = num_slots;
    const int ctx = uniform(ctx_lens[b]);
    a.ctx = ctx > cap_tokens ? cap_tokens : ctx;

    // Q^T operand: lane (head j, group g) holds q[j][32s + 8g .. +8].
    u32x4 qop[D / 32];
    const uint16_t* qh = q + (static_cast<size_t>(b) * NQ + kvh * G + (head_ok ? i16 : 0)) * D;
#pragma unroll
    for (int s = 0; s < D / 32; ++s) {
      const u32x4 z = {0u, 0u, 0u, 0u};
      qop[s] = head_ok ? *reinterpret_cast<const u32x4*>(qh + 32 * s + 8 * g) : z;
    }

    SoftmaxState<D> st;
#pragma unroll
    for (int n = 0; n < D / 16; ++n) st.acc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
    st.m = -INFINITY;
    st.l = 0.f;

    int tab_base = -(1 << 30);
    int tab = 0;
    // NBUF-deep register ring: block bi+NBUF-1 is requested while block bi is
    // consumed.  Every ring slot is loaded unconditionally (prefetches past
    // the piece are empty loads), so the waitcnt before each compute never
    // depends on a branch.
    BlockRegs<D> ring[NBUF];
#pragma unroll
    for (int j = 0; j < NBUF - 1; ++j) {
      load_block<D>(ring[j], a, blo + j, bhi, tab_base, tab, lane, lofs);
    }
    int bi = blo;
    bool done = false;
    while (!done) {
#pragma unroll
      for (int j = 0; j < NBUF; ++j) {
        if (!done) {
          const int pf = bi + NBUF - 1;
          load_block<D>(ring[(j + NBUF - 1) % NBUF], a, pf, bhi, tab_base, tab, lane, lofs);
          compute_block<D>(ring[j], qop, st, a.ctx - bi * kBlockTokens, scale_log2e, lane);
          done = ++bi >= bhi;
        }
      }
    }

    const float l_tot = wave_sum_across_groups(st.l);
    const long long pidx = static_cast<long long>(b) * NKV + kvh + w;
    if (head_ok) {
      float* po = part_o + (pidx * G + i16) * D;
#pragma unroll
      for (int n = 0; n < D / 16; ++n) {
        *reinterpret_cast<f32x4*>(po + 16 * n + 4 * g) = st.acc[n];
      }
      if (g == 0) {
        part_ml[(pidx * G + i16) * 2 + 0] = st.m;
        part_ml[(pidx * G + i16) * 2 + 1] = l_tot;
      }
    }

    u0 = u1 < send ? u1 : send;
    if (u0 >= u1) break;
    S = send;
    if (++kvh == NKV) {
      kvh = 0;
      do {
        ++b;
      } while (b < B - 1 && uniform(seg[b + 1]) == uniform(seg[b]));
      nb = uniform(seg[b + 1]) - uniform(seg[b]);
    }
  }
}

// Short contexts: one workgroup per (sequence, kv head) segment.  Its SW
// wavefronts take an equal share of the segment's 32-token blocks with the
// partials kernel's block loop, leave their softmax states in LDS, and merge
// them into the bf16 output (and LSE) themselves -- one launch and no
// workspace, where the split-K pair of kernels costs two launches of
// mostly fixed latency when a segment has only a few dozen blocks.
template <int D, int NBUF, int SW>
__global__ __launch_bounds__(SW * kWave) void gqa_segment_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_pool,
    const uint16_t* __restrict__ v_pool, const int32_t* __restrict__ block_table,
    const int32_t* __restrict__ ctx_lens, uint16_t* __restrict__ out,
    float* __restrict__ lse_out, int NKV, int G, int max_pages, int pt_shift, int num_slots,
    float scale_log2e) {
  __shared__ float red_o[SW][16][D];
  __shared__ float red_m[SW][16];
  __shared__ float red_l[SW][16];
  const int lane = threadIdx.x & (kWave - 1);
  const int wl = uniform(threadIdx.x / kWave);
  const int b = blockIdx.x / NKV;
  const int kvh = blockIdx.x - b * NKV;
  const int NQ = NKV * G;
  const int i16 = lane & 15;
  const int g = lane >> 4;
  const bool head_ok = i16 < G;
  // Loads that do not depend on the context length issue before it arrives:
  // the q operands and, for tables of at most 64 pages, the whole table row
  // (one memory round trip fewer before the first page load).
  u32x4 qop[D / 32];
  {
    const uint16_t* qh = q + (static_cast<size_t>(b) * NQ + kvh * G + (head_ok ? i16 : 0)) * D;
#pragma unroll
    for (int s = 0; s < D / 32; ++s) {
      const u32x4 z = {0u, 0u, 0u, 0u};
      qop[s] = head_ok ? *reinterpret_cast<const u32x4*>(qh + 32 * s + 8 * g) : z;
    }
  }
  int tab_base = -(1 << 30);
  int tab = 0;
  if (max_pages <= kWave) {
    tab_base = 0;
    tab = lane < max_pages ? block_table[static_cast<size_t>(b) * max_pages + lane] : 0;
  }
  const int cap_tokens = max_pages << pt_shift;
  int ctx = uniform(ctx_lens[b]);
  ctx = ctx < 0 ? 0 : (ctx > cap_tokens ? cap_tokens : ctx);
  const int nb = (ctx + kBlockTokens - 1) / kBlockTokens;
  const int blo = wl * nb / SW;
  const int bhi = (wl + 1) * nb / SW;

  LaneOffsets lofs;
  lofs.k = ((8 * (i16 >> 2) + (i16 & 3)) * D + 8 * g) * 2;
  lofs.v = ((i16 * kBlockTokens) + 8 * g) * 2;
  SegmentArgs a;
  a.k_pool = k_pool;
  a.v_pool = v_pool;
  a.table_row = block_table + static_cast<size_t>(b) * max_pages;
  a.n_pages = max_pages;
  a.kvh = kvh;
  a.nkv = NKV;
  a.pt_shift = pt_shift;
  a.num_slots = num_slots;
  a.ctx = ctx;

  SoftmaxState<D> st;
#pragma unroll
  for (int n = 0; n < D / 16; ++n) st.acc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
  st.m = -INFINITY;
  st.l = 0.f;
  if (blo < bhi) {
    BlockRegs<D> ring[NBUF];
#pragma unroll
    for (int j = 0; j < NBUF - 1; ++j) {
      load_block<D>(ring[j], a, blo + j, bhi, tab_base, tab, lane, lofs);
    }
    int bi = blo;
    bool done = false;
    while (!done) {
#pragma unroll
      for (int j = 0; j < NBUF; ++j) {
        if (!done) {
          const int pf = bi + NBUF - 1;
          load_block<D>(ring[(j + NBUF - 1) % NBUF], a, pf, bhi, tab_base, tab, lane, lofs);
          compute_block<D>(ring[j], qop, st, a.ctx - bi * kBlockTokens, scale_log2e, lane);
          done = ++bi >= bhi;
        }
      }
    }
  }
  const float l_tot = wave_sum_across_groups(st.l);
  if (head_ok) {
#pragma unroll
    for (int n = 0; n < D / 16; ++n) {
#pragma unroll
      for (int r = 0; r < 4; ++r) red_o[wl][i16][16 * n + 4 * g + r] = st.acc[n][r];
    }
    if (g == 0) {
      red_m[wl][i16] = st.m;
      red_l[wl][i16] = l_tot;
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < G * D; idx += SW * kWave) {
    const int h = idx / D;
    const int d = idx - h * D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < SW; ++w) M = fmaxf(M, red_m[w][h]);
    const size_t row = static_cast<size_t>(b) * NQ + kvh * G + h;
    if (M == -INFINITY) {  // no tokens
      out[row * D + d] = 0;
      if (lse_out != nullptr && d == 0) lse_out[row] = -INFINITY;
      continue;
    }
    float L = 0.f;
    float o = 0.f;
#pragma unroll
    for (int w = 0; w < SW; ++w) {
      const float mw = red_m[w][h];
      const float wt = mw == -INFINITY ? 0.f : fast_exp2(mw - M);
      L += red_l[w][h] * wt;
      o += red_o[w][h][d] * wt;
    }
    out[row * D + d] = f2bf(o * (1.f / L));
    if (lse_out != nullptr && d == 0) lse_out[row] = (M + __log2f(L)) * 0.6931471805599453f;
  }
}

// Wavefront of the split holding unit u (the last w with w*U/W <= u).
__device__ __forceinline__ long long wave_of_unit(long long u, long long U, int W) {
  return ((u + 1) * W - 1) / U;
}

// One wavefront per (sequence, q-head): merges the partial states of the
// wavefronts that shared the head's KV segment.
template <int D>
__global__ __launch_bounds__(kThreads) void gqa_reduce_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_ml,
    const int32_t* __restrict__ ctx_lens, uint16_t* __restrict__ out,
    float* __restrict__ lse_out, int B, int NKV, int G, int max_pages, int pt_shift, int W) {
  constexpr int DPL = D / kWave;  // dims per lane
  const int lane = threadIdx.x & (kWave - 1);
  const int task = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
  const int NQ = NKV * G;
  if (task >= B * NQ) return;
  const int b = task / NQ;
  const int hq = task - b * NQ;
  const int kvh = hq / G;
  const int j = hq - kvh * G;
  const int s = b * NKV + kvh;

  // This wavefront's own block prefix (no LDS, no barrier): blocks before
  // sequence b, blocks of b, and the total, 64 sequences per step.
  const int cap_tokens = max_pages << pt_shift;
  int seg_b = 0;
  int nb = 0;
  int total = 0;
  for (int base = 0; base < B; base += kWave) {
    const int i = base + lane;
    int nblk = 0;
    if (i < B) {
      int c = ctx_lens[i];
      c = c < 0 ? 0 : (c > cap_tokens ? cap_tokens : c);
      nblk = (c + kBlockTokens - 1) / kBlockTokens;
    }
    const int x = wave_inclusive_scan(nblk, lane);
    if (b >= base && b < base + kWave) {
      seg_b = total + __builtin_amdgcn_readlane(x - nblk, b - base);
      nb = __builtin_amdgcn_readlane(nblk, b - base);
    }
    total += __builtin_amdgcn_readlane(x, kWave - 1);
  }
  uint16_t* ob = out + static_cast<size_t>(task) * D;
  if (nb == 0) {
#pragma unroll
    for (int d = 0; d < DPL; ++d) ob[lane * DPL + d] = 0;
    if (lse_out != nullptr && lane == 0) lse_out[task] = -INFINITY;
    return;
  }
  const long long U = static_cast<long long>(total) * NKV;
  const int We = static_cast<int>(U < W ? U : W);
  const long long us = static_cast<long long>(seg_b) * NKV + static_cast<long long>(kvh) * nb;
  const long long p0 = s + wave_of_unit(us, U, We);
  const int n = static_cast<int>(wave_of_unit(us + nb - 1, U, We) + s - p0) + 1;

  // Single pass over batches of kBatch partials.  Every load of a batch --
  // lane i's (m, l) of partial i and all kBatch partial rows of this lane's
  // dims -- is issued before the first use, so a batch costs one memory
  // round trip; the batch maximum then rescales the running state.  Indices
  // past n are clamped to the last partial (always written) and weighted 0.
  constexpr int kBatch = D == 128 ? 32 : 64;
  const float2* ml2 = reinterpret_cast<const float2*>(part_ml);
  float M = -INFINITY;
  float L = 0.f;
  float acc[DPL];
#pragma unroll
  for (int d = 0; d < DPL; ++d) acc[d] = 0.f;
  for (int i0 = 0; i0 < n; i0 += kBatch) {
    const int i = i0 + lane;
    const bool live = lane < kBatch && i < n;
    const float2 mi = ml2[(p0 + (live ? i : n - 1)) * G + j];
    float v[kBatch][DPL];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int k = i0 + u < n ? i0 + u : n - 1;
      const float* po = part_o + ((p0 + k) * G + j) * D + lane * DPL;
      if constexpr (DPL == 2) {
        const float2 t = *reinterpret_cast<const float2*>(po);
        v[u][0] = t.x;
        v[u][1] = t.y;
      } else {
#pragma unroll
        for (int d = 0; d < DPL; ++d) v[u][d] = po[d];
      }
    }
    // Keep the scheduler from sinking each load next to its use (which would
    // serialise kBatch round trips): everything above issues first.
    __builtin_amdgcn_sched_barrier(0);
    // cross-lane work by DPP moves and v_readlane (no LDS crossbar trips)
    const float Mc = wave_max_uniform(live ? mi.x : -INFINITY);
    const float Mn = fmaxf(M, Mc);
    const float rescale = fast_exp2(M - Mn);
    const float wl = live ? fast_exp2(mi.x - Mn) : 0.f;
    const float Lc = wave_sum_uniform(live ? mi.y * wl : 0.f);
    L = L * rescale + Lc;
    M = Mn;
#pragma unroll
    for (int d = 0; d < DPL; ++d) acc[d] *= rescale;
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const float wk = __builtin_bit_cast(
          float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), u));
#pragma unroll
      for (int d = 0; d < DPL; ++d) acc[d] += v[u][d] * wk;
    }
  }
  const float inv = 1.f / L;
#pragma unroll
  for (int d = 0; d < DPL; ++d) ob[lane * DPL + d] = f2bf(acc[d] * inv);
  if (lse_out != nullptr && lane == 0) lse_out[task] = (M + __log2f(L)) * 0.6931471805599453f;
}

__global__ __launch_bounds__(kThreads) void merge_states_kernel(
    const uint16_t* __restrict__ oa, const float* __restrict__ la,
    const uint16_t* __restrict__ ob, const float* __restrict__ lb, uint16_t* __restrict__ out,
    float* __restrict__ lse_out, int rows, int D) {
  const long long idx = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
  if (idx >= static_cast<long long>(rows) * D) return;
  const int row = static_cast<int>(idx / D);
  const float a = la[row];
  const float c = lb[row];
  const float m = fmaxf(a, c);
  float res;
  float lse;
  if (m == -INFINITY) {
    res = 0.f;
    lse = -INFINITY;
  } else {
    const float wa = __expf(a - m);
    const float wb = __expf(c - m);
    res = (bf2f(oa[idx]) * wa + bf2f(ob[idx]) * wb) / (wa + wb);
    lse = m + __logf(wa + wb);
  }
  out[idx] = f2bf(res);
  if (lse_out != nullptr && idx % D == 0) lse_out[row] = lse;
}

// Folds one bf16 attention state (o_b, lse_b) over a key set disjoint from the
// accumulator's into an fp32 running state (o_acc, lse_acc), in place.  One
// wavefront per row: its lanes read the row's running LSE in the same load
// instruction, before lane 0 stores the new one, so the in-place update has no
// cross-thread hazard.  With ``init`` the state is set to (o_b, lse_b).  The
// running output is never re-rounded to bf16, so folding many chunks does not
// accumulate rounding error; the caller rounds once at the end.
__global__ __launch_bounds__(kThreads) void fold_state_kernel(
    float* __restrict__ o_acc, float* __restrict__ lse_acc, const uint16_t* __restrict__ ob,
    const float* __restrict__ lb, int rows, int D, int init) {
  const int row = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  if (row >= rows) return;
  float* o = o_acc + static_cast<size_t>(row) * D;
  const uint16_t* b = ob + static_cast<size_t>(row) * D;
  const float c = lb[row];
  if (init) {
    for (int d = lane; d < D; d += kWave) o[d] = bf2f(b[d]);
    if (lane == 0) lse_acc[row] = c;
    return;
  }
  const float a = lse_acc[row];
  const float m = fmaxf(a, c);
  if (m == -INFINITY) {  // both key sets empty: the state stays (0, -inf)
    for (int d = lane; d < D; d += kWave) o[d] = 0.f;
    return;
  }
  const float wa = __expf(a - m);
  const float wb = __expf(c - m);
  const float inv = 1.f / (wa + wb);
  for (int d = lane; d < D; d += kWave) o[d] = (o[d] * wa + bf2f(b[d]) * wb) * inv;
  if (lane == 0) lse_acc[row] = m + __logf(wa + wb);
}

size_t part_slots(int batch, int num_kv_heads, int num_splits) {
  return static_cast<size_t>(batch) * num_kv_heads + static_cast<size_t>(num_splits);
}

}  // namespace
}  // namespace voom

using namespace voom;

extern "C" int voom_paged_gqa_default_splits(void) {
  return device_cu_count() * VOOM_GQA_SPLITS_PER_CU;
}

extern "C" size_t voom_paged_gqa_workspace_bytes(int batch, int num_q_heads, int num_kv_heads,
                                                 int head_dim, int num_splits) {
  if (batch <= 0 || num_kv_heads <= 0 || num_q_heads <= 0 || head_dim <= 0) return 0;
  if (num_splits <= 0) num_splits = voom_paged_gqa_default_splits();
  const size_t G = static_cast<size_t>(num_q_heads / num_kv_heads);
  const size_t slots = part_slots(batch, num_kv_heads, num_splits);
  const size_t o_bytes = slots * G * head_dim * sizeof(float);
  const size_t ml_bytes = slots * G * 2 * sizeof(float);
  return ((o_bytes + 255) & ~size_t(255)) + ml_bytes;
}

namespace voom {
namespace {

// Validated geometry and workspace carving shared by the decode halves.
struct GqaPlan {
  int B, NQ, NKV, G, D, max_pages, pt_shift, num_splits;
  float* part_o;
  float* part_ml;
};

int plan_gqa(const char* who, void* workspace, size_t ws_bytes, int batch, int num_q_heads,
             int num_kv_heads, int head_dim, int page_tokens, int max_pages, int num_splits,
             GqaPlan* p) {
  VOOM_REQUIRE(workspace != nullptr, "%s: null workspace", who);
  VOOM_REQUIRE(batch > 0 && batch <= kMaxBatch, "%s: batch %d not in [1, %d]", who, batch,
               kMaxBatch);
  VOOM_REQUIRE(num_kv_heads > 0 && num_q_heads > 0 && num_q_heads % num_kv_heads == 0,
               "%s: num_q_heads %d not a multiple of num_kv_heads %d", who, num_q_heads,
               num_kv_heads);
  const int G = num_q_heads / num_kv_heads;
  VOOM_REQUIRE(G <= 16, "%s: GQA group %d exceeds 16", who, G);
  VOOM_REQUIRE(head_dim == 64 || head_dim == 128, "%s: head_dim %d unsupported (64 or 128)",
               who, head_dim);
  VOOM_REQUIRE(is_pow2(page_tokens) && page_tokens >= 32 && page_tokens <= 4096,
               "%s: page_tokens %d must be a power of two in [32, 4096]", who, page_tokens);
  VOOM_REQUIRE(max_pages > 0, "%s: empty block table", who);
  VOOM_REQUIRE(static_cast<long long>(max_pages) * page_tokens < (1LL << 30),
               "%s: table capacity too large", who);
  if (num_splits <= 0) num_splits = voom_paged_gqa_default_splits();
  VOOM_REQUIRE(num_splits <= (1 << 22), "%s: num_splits %d too large", who, num_splits);
  const size_t need = voom_paged_gqa_workspace_bytes(batch, num_q_heads, num_kv_heads,
                                                      head_dim, num_splits);
  VOOM_REQUIRE(ws_bytes >= need, "%s: workspace %zu bytes < required %zu", who, ws_bytes,
               need);
  VOOM_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0,
               "%s: workspace must be 16-byte aligned", who);
  const size_t slots = part_slots(batch, num_kv_heads, num_splits);
  const size_t o_bytes = slots * G * head_dim * sizeof(float);
  p->B = batch;
  p->NQ = num_q_heads;
  p->NKV = num_kv_heads;
  p->G = G;
  p->D = head_dim;
  p->max_pages = max_pages;
  p->pt_shift = ilog2(page_tokens);
  p->num_splits = num_splits;
  p->part_o = static_cast<float*>(workspace);
  p->part_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                        ((o_bytes + 255) & ~size_t(255)));
  return VOOM_OK;
}

int launch_partials(const GqaPlan& p, const void* q, const void* k_pool, const void* v_pool,
                    const int32_t* block_table, const int32_t* ctx_lens, int num_slots,
                    float scale, hipStream_t stream) {
  const float scale_log2e = scale * 1.4426950408889634f;
  const dim3 grid((p.num_splits + kWavesPerBlock - 1) / kWavesPerBlock);
  const auto* qq = static_cast<const uint16_t*>(q);
  const auto* kp = static_cast<const uint16_t*>(k_pool);
  const auto* vp = static_cast<const uint16_t*>(v_pool);
  if (p.D == 128) {
    hipLaunchKernelGGL((gqa_decode_kernel<128, kNbuf128, kWavesPerEu128>), grid,
                       dim3(kThreads), 0, stream, qq, kp, vp, block_table, ctx_lens, p.part_o,
                       p.part_ml, p.B, p.NKV, p.G, p.max_pages, p.pt_shift, num_slots,
                       scale_log2e, p.num_splits);
  } else {
    hipLaunchKernelGGL((gqa_decode_kernel<64, kNbuf64, kWavesPerEu64>), grid, dim3(kThreads),
                       0, stream, qq, kp, vp, block_table, ctx_lens, p.part_o, p.part_ml, p.B,
                       p.NKV, p.G, p.max_pages, p.pt_shift, num_slots, scale_log2e,
                       p.num_splits);
  }
  return VOOM_LAUNCH_CHECK("paged_gqa: partials kernel launch");
}

// Block tables of at most this many tokens per sequence use the one-launch
// segment kernel when the caller leaves the split count to the library.  A
// segment streams through one CU (about 39 GB/s), so its time grows by ~6.5 ns
// per token at D = 64; measured against partials + combine at the default
// split count for 3 to 384 segments, the segment kernel wins or ties at 1,024
// tokens and loses from 1,536 (4,096 tokens, 3 segments: 29.7 against 12.9 us).
constexpr long long kSegmentKernelTokens = 1024;
// Wavefronts per segment workgroup.
#ifndef VOOM_GQA_SEGMENT_WAVES
#define VOOM_GQA_SEGMENT_WAVES 4
#endif
constexpr int kSegmentWaves = VOOM_GQA_SEGMENT_WAVES;

int launch_segments(const GqaPlan& p, const void* q, const void* k_pool, const void* v_pool,
                    const int32_t* block_table, const int32_t* ctx_lens, int num_slots,
                    float scale, void* out, float* lse_out, hipStream_t stream) {
  const float scale_log2e = scale * 1.4426950408889634f;
  const dim3 grid(static_cast<unsigned>(p.B * p.NKV));
  const auto* qq = static_cast<const uint16_t*>(q);
  const auto* kp = static_cast<const uint16_t*>(k_pool);
  const auto* vp = static_cast<const uint16_t*>(v_pool);
  auto* oo = static_cast<uint16_t*>(out);
  constexpr int SW = kSegmentWaves;
  if (p.D == 128) {
    hipLaunchKernelGGL((gqa_segment_kernel<128, kNbuf128, SW>), grid, dim3(SW * kWave), 0, stream,
                       qq, kp, vp, block_table, ctx_lens, oo, lse_out, p.NKV, p.G, p.max_pages,
                       p.pt_shift, num_slots, scale_log2e);
  } else {
    hipLaunchKernelGGL((gqa_segment_kernel<64, kNbuf64, SW>), grid, dim3(SW * kWave), 0, stream,
                       qq, kp, vp, block_table, ctx_lens, oo, lse_out, p.NKV, p.G, p.max_pages,
                       p.pt_shift, num_slots, scale_log2e);
  }
  return VOOM_LAUNCH_CHECK("paged_gqa: segment kernel launch");
}

int launch_combine(const GqaPlan& p, const int32_t* ctx_lens, void* out, float* lse_out,
                   hipStream_t stream) {
  const dim3 grid((p.B * p.NQ + kWavesPerBlock - 1) / kWavesPerBlock);
  auto* oo = static_cast<uint16_t*>(out);
  if (p.D == 128) {
    hipLaunchKernelGGL((gqa_reduce_kernel<128>), grid, dim3(kThreads), 0, stream, p.part_o,
                       p.part_ml, ctx_lens, oo, lse_out, p.B, p.NKV, p.G, p.max_pages,
                       p.pt_shift, p.num_splits);
  } else {
    hipLaunchKernelGGL((gqa_reduce_kernel<64>), grid, dim3(kThreads), 0, stream, p.part_o,
                       p.part_ml, ctx_lens, oo, lse_out, p.B, p.NKV, p.G, p.max_pages,
                       p.pt_shift, p.num_splits);
  }
  return VOOM_LAUNCH_CHECK("paged_gqa: combine kernel launch");
}

int check_partials_args(const char* who, const void* q, const void* k_pool,
                        const void* v_pool, const int32_t* block_table,
                        const int32_t* ctx_lens, int num_slots) {
  VOOM_REQUIRE(q && k_pool && v_pool && block_table && ctx_lens,
               "%s: null pointer argument", who);
  VOOM_REQUIRE(num_slots > 0, "%s: empty page pool", who);
  VOOM_REQUIRE(reinterpret_cast<uintptr_t>(q) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(k_pool) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(v_pool) % 16 == 0,
               "%s: q and pools must be 16-byte aligned", who);
  return VOOM_OK;
}

}  // namespace
}  // namespace voom

extern "C" int voom_paged_gqa_decode(const void* q, const void* k_pool, const void* v_pool,
                                     const int32_t* block_table, const int32_t* ctx_lens,
                                     void* out, float* lse_out, void* workspace,
                                     size_t ws_bytes, int batch, int num_q_heads,
                                     int num_kv_heads, int head_dim, int page_tokens,
                                     int max_pages, int num_slots, float scale,
                                     int num_splits, hipStream_t stream) {
  const char* who = "paged_gqa_decode";
  int rc = check_partials_args(who, q, k_pool, v_pool, block_table, ctx_lens, num_slots);
  if (rc) return rc;
  VOOM_REQUIRE(out != nullptr, "%s: null output", who);
  const bool auto_splits = num_splits <= 0;
  GqaPlan p;
  rc = plan_gqa(who, workspace, ws_bytes, batch, num_q_heads, num_kv_heads, head_dim,
                page_tokens, max_pages, num_splits, &p);
  if (rc) return rc;
  if (auto_splits && static_cast<long long>(max_pages) * page_tokens <= kSegmentKernelTokens) {
    return launch_segments(p, q, k_pool, v_pool, block_table, ctx_lens, num_slots, scale,
                           out, lse_out, stream);
  }
  rc = launch_partials(p, q, k_pool, v_pool, block_table, ctx_lens, num_slots, scale, stream);
  if (rc) return rc;
  return launch_combine(p, ctx_lens, out, lse_out, stream);
}

extern "C" int voom_paged_gqa_partials(const void* q, const void* k_pool, const void* v_pool,
                                       const int32_t* block_table, const int32_t* ctx_lens,
                                       void* workspace, size_t ws_bytes, int batch,
                                       int num_q_heads, int num_kv_heads, int head_dim,
                                       int page_tokens, int max_pages, int num_slots,
                                       float scale, int num_splits, hipStream_t stream) {
  const char* who = "paged_gqa_partials";
  int rc = check_partials_args(who, q, k_pool, v_pool, block_table, ctx_lens, num_slots);
  if (rc) return rc;
  GqaPlan p;
  rc = plan_gqa(who, workspace, ws_bytes, batch, num_q_heads, num_kv_heads, head_dim,
                page_tokens, max_pages, num_splits, &p);
  if (rc) return rc;
  return launch_partials(p, q, k_pool, v_pool, block_table, ctx_lens, num_slots, scale, stream);
}

extern "C" int voom_paged_gqa_combine(const int32_t* ctx_lens, void* out, float* lse_out,
                                      void* workspace, size_t ws_bytes, int batch,
                                      int num_q_heads, int num_kv_heads, int head_dim,
                                      int page_tokens, int max_pages, int num_splits,
                                      hipStream_t stream) {
  const char* who = "paged_gqa_combine";
  VOOM_REQUIRE(ctx_lens && out, "%s: null pointer argument", who);
  GqaPlan p;
  const int rc = plan_gqa(who, workspace, ws_bytes, batch, num_q_heads, num_kv_heads,
                          head_dim, page_tokens, max_pages, num_splits, &p);
  if (rc) return rc;
  return launch_combine(p, ctx_lens, out, lse_out, stream);
}

extern "C" int voom_merge_attn_states(const void* o_a, const float* lse_a, const void* o_b,
                                      const float* lse_b, void* out, float* lse_out, int rows,
                                      int head_dim, hipStream_t stream) {
  VOOM_REQUIRE(o_a && lse_a && o_b && lse_b && out, "merge_attn_states: null pointer");
  VOOM_REQUIRE(rows >= 0 && head_dim > 0, "merge_attn_states: bad shape");
  if (rows == 0) return VOOM_OK;
  const long long n = static_cast<long long>(rows) * head_dim;
  const dim3 grid(static_cast<unsigned>((n + kThreads - 1) / kThreads));
  hipLaunchKernelGGL(merge_states_kernel, grid, dim3(kThreads), 0, stream,
                     static_cast<const uint16_t*>(o_a), lse_a,
                     static_cast<const uint16_t*>(o_b), lse_b, static_cast<uint16_t*>(out),
                     lse_out, rows, head_dim);
  return VOOM_LAUNCH_CHECK("merge_attn_states: launch");
}

extern "C" int voom_fold_attn_state(float* o_acc, float* lse_acc, const void* o_b,
                                    const float* lse_b, int rows, int head_dim, int init,
                                    hipStream_t stream) {
  VOOM_REQUIRE(o_acc && lse_acc && o_b && lse_b, "fold_attn_state: null pointer");
  VOOM_REQUIRE(rows >= 0 && head_dim > 0, "fold_attn_state: bad shape");
  if (rows == 0) return VOOM_OK;
  const dim3 grid(static_cast<unsigned>((rows + kWavesPerBlock - 1) / kWavesPerBlock));
  hipLaunchKernelGGL(fold_state_kernel, grid, dim3(kThreads), 0, stream, o_acc, lse_acc,
                     static_cast<const uint16_t*>(o_b), lse_b, rows, head_dim, init ? 1 : 0);
  return VOOM_LAUNCH_CHECK("fold_attn_state: launch");
}
