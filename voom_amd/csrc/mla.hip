// Absorbed-MLA paged decode (latent contraction) for gfx950.
//
// Restates the latent part of the reference's _mla_absorbed_attention
// (runtime/glm.py:133-164): with q_lat = [q_nope . W_UK | q_rope] per head,
//   scores[h, t] = q_lat[h] . lat[t]            (576-wide, fp32, * scale)
//   p            = softmax_t(scores), rounded to bf16 (glm.py:159-161)
//   weighted_c[h] = sum_t p[h, t] * lat[t, :512]  (bf16 result)
// over a latent cache kept in 64-token pages ([slots, page_tokens, 576]) and
// addressed through a block table.  The absorption GEMMs (q_nope . W_UK and
// weighted_c . W_UV) stay outside, in hipBLASLt.
//
// 128 heads share one latent row, so the contraction is MFMA work:
//   scores^T [tokens x heads] = Lat [tokens x 576] . Q^T      v_mfma_f32_16x16x32_bf16
//   out^T    [dims x heads]  += C^T [dims x tokens] . P^T     v_mfma_f32_16x16x32_bf16
// Decomposition: one workgroup (4 wavefronts) per (sequence, token range,
// group of 32 heads).  The four head groups of a range are placed on the same
// XCD so the latent tiles they all read are served from that XCD's L2.
// Per 64-token tile: the tile is staged in LDS (register prefetch of the next
// tile overlaps the current one's math); wavefront w computes the scores of
// tokens 16w..16w+15 for all 32 heads, the page maximum is combined through
// LDS, P is written to LDS in bf16, and wavefront w accumulates dims
// 128w..128w+127 of out^T for all 32 heads (accumulators stay in registers
// for the whole range).  The C^T operand is read from the token-major tile
// with 16-bit LDS reads; lane group g takes tokens g, g+4, ..., g+28 of a
// 32-token step, which keeps those reads free of bank conflicts, and P is
// stored in the same token order so its operand is one 16-byte read.
#include "common.h"

namespace voom {
namespace {

constexpr int kThreads = 256;
constexpr int kLat = 576;          // kv_lora_rank 512 + rope dim 64
constexpr int kC = 512;
constexpr int kHeadsPerGroup = 32;
constexpr int kTile = 64;          // tokens per tile
constexpr int kRow = kLat + 8;     // LDS row stride in bf16 elements (1168 B, 16 B aligned)
constexpr int kChunksPerRow = kLat * 2 / 16;  // 72 sixteen-byte chunks per token
constexpr int kChunksPerThread = kTile * kChunksPerRow / kThreads;  // 18
constexpr int kQSteps = kLat / 32;  // 18 k-steps of the score MFMA

__device__ __forceinline__ int perm_pos(int t) {
  // Position of token t (0..31 within a 32-token step) in the P row: token
  // 4e+g is stored at 8g+e, so lane group g reads its 8 tokens contiguously.
  return 8 * (t & 3) + (t >> 2);
}

struct MlaArgs {
  const uint16_t* __restrict__ q;        // [B, H, 576]
  const uint16_t* __restrict__ lat;      // [slots, PT, 576]
  const int32_t* __restrict__ table;     // [B, max_pages]
  const int32_t* __restrict__ ctx_lens;  // [B]
  float* __restrict__ part_o;            // [B, NR, H, 512]
  float* __restrict__ part_ml;           // [B, NR, H, 2]
  int B, H, NR, max_pages, pt_shift, num_slots;
  float scale_log2e;
};

__global__ __launch_bounds__(kThreads, 1) void mla_latent_kernel(MlaArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t tile[kTile * kRow];
  __shared__ __attribute__((aligned(16))) uint16_t p_lds[kHeadsPerGroup * kTile];
  __shared__ float pmax[4][kHeadsPerGroup];
  __shared__ float psum[4][kHeadsPerGroup];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int i16 = lane & 15;
  const int g = lane >> 4;
  const int NHG = a.H / kHeadsPerGroup;

  // Block -> (task = sequence x range, head group); head groups of one task
  // share bid % 8, i.e. the same XCD.
  const int n_tasks = a.B * a.NR;
  int task, hg;
  const int bid = blockIdx.x;
  if (n_tasks % 8 == 0) {
    const int xcd = bid & 7;
    const int local = bid >> 3;
    hg = local % NHG;
    task = (local / NHG) * 8 + xcd;
  } else {
    hg = bid % NHG;
    task = bid / NHG;
  }
  const int b = task / a.NR;
  const int range = task - b * a.NR;
  const int tiles_per_page = 1 << (a.pt_shift - 6);
  int ctx = a.ctx_lens[b];
  const int cap = a.max_pages << a.pt_shift;
  ctx = ctx < 0 ? 0 : (ctx > cap ? cap : ctx);
  const int n_tiles = (ctx + kTile - 1) / kTile;
  const int per = (n_tiles + a.NR - 1) / a.NR;
  const int t_lo = range * per;
  const int t_hi = (t_lo + per < n_tiles) ? t_lo + per : n_tiles;
  const int head0 = hg * kHeadsPerGroup;
  const int32_t* trow = a.table + static_cast<size_t>(b) * a.max_pages;

  // Q^T operands for both head tiles, all 18 k-steps: lane (head i16, group g)
  // holds q[head][32s + 8g .. +8].
  u32x4 qop[2][kQSteps];
#pragma unroll
  for (int ht = 0; ht < 2; ++ht) {
    const uint16_t* qh = a.q + (static_cast<size_t>(b) * a.H + head0 + 16 * ht + i16) * kLat;
#pragma unroll
    for (int s = 0; s < kQSteps; ++s) {
      qop[ht][s] = *reinterpret_cast<const u32x4*>(qh + 32 * s + 8 * g);
    }
  }

  f32x4 acc[8][2];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    acc[dt][0] = f32x4{0.f, 0.f, 0.f, 0.f};
    acc[dt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  float m_run[2] = {-INFINITY, -INFINITY};  // per head tile: head 16ht + i16
  float l_run[2] = {0.f, 0.f};

  auto tile_base = [&](int t) -> const uint16_t* {
    const int page = t / tiles_per_page;
    const int sub = t - page * tiles_per_page;
    int slot = trow[page];
    if (static_cast<unsigned>(slot) >= static_cast<unsigned>(a.num_slots)) slot = 0;
    return a.lat + ((static_cast<size_t>(slot) << a.pt_shift) + sub * kTile) * kLat;
  };

  u32x4 pre[kChunksPerThread];
  auto prefetch = [&](int t) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(tile_base(t)),
                                          static_cast<short>(0), kTile * kLat * 2, 0x00020000);
#pragma unroll
    for (int k = 0; k < kChunksPerThread; ++k) {
      pre[k] = __builtin_amdgcn_raw_buffer_load_b128(r, (tid + kThreads * k) * 16, 0, 0);
    }
  };
  auto stage = [&](int t) {
    const int valid = ctx - t * kTile;
#pragma unroll
    for (int k = 0; k < kChunksPerThread; ++k) {
      const int c = tid + kThreads * k;
      const int tok = c / kChunksPerRow;
      const int col = c - tok * kChunksPerRow;
      u32x4 v = pre[k];
      if (tok >= valid) v = u32x4{0u, 0u, 0u, 0u};  // tokens past the context
      *reinterpret_cast<u32x4*>(tile + tok * kRow + col * 8) = v;
    }
  };

  if (t_lo < t_hi) prefetch(t_lo);
  for (int t = t_lo; t < t_hi; ++t) {
    __syncthreads();  // previous tile fully consumed
    stage(t);
    if (t + 1 < t_hi) prefetch(t + 1);
    __syncthreads();

    // ---- scores: tokens 16w..16w+15 x 32 heads ----
    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
    const uint16_t* arow = tile + (16 * w + i16) * kRow + 8 * g;
#pragma unroll
    for (int s = 0; s < kQSteps; ++s) {
      const bf16x8 av = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(arow + 32 * s));
      s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, __builtin_bit_cast(bf16x8, qop[0][s]), s0,
                                                   0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, __builtin_bit_cast(bf16x8, qop[1][s]), s1,
                                                   0, 0, 0);
    }
    // lane (head i16, group g) holds tokens 16w + 4g + r, r = 0..3
    const int valid = ctx - t * kTile;
    float x[2][4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool ok = 16 * w + 4 * g + r < valid;
      x[0][r] = ok ? s0[r] * a.scale_log2e : -INFINITY;
      x[1][r] = ok ? s1[r] * a.scale_log2e : -INFINITY;
    }
#pragma unroll
    for (int ht = 0; ht < 2; ++ht) {
      float mx = fmaxf(fmaxf(x[ht][0], x[ht][1]), fmaxf(x[ht][2], x[ht][3]));
      mx = wave_max_across_groups(mx);
      if (g == 0) pmax[w][16 * ht + i16] = mx;
    }
    __syncthreads();

    float alpha[2];
#pragma unroll
    for (int ht = 0; ht < 2; ++ht) {
      const int hh = 16 * ht + i16;
      const float mp = fmaxf(fmaxf(pmax[0][hh], pmax[1][hh]), fmaxf(pmax[2][hh], pmax[3][hh]));
      const float mn = fmaxf(m_run[ht], mp);
      alpha[ht] = fast_exp2(m_run[ht] - mn);
      m_run[ht] = mn;
      float ps = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = fast_exp2(x[ht][r] - mn);
        const uint16_t pb = f2bf(p);
        ps += bf2f(pb);
        const int tok = 16 * w + 4 * g + r;  // 0..63
        p_lds[hh * kTile + 32 * (tok >> 5) + perm_pos(tok & 31)] = pb;
      }
      ps = wave_sum_across_groups(ps);
      if (g == 0) psum[w][hh] = ps;
    }
    __syncthreads();

#pragma unroll
    for (int ht = 0; ht < 2; ++ht) {
      const int hh = 16 * ht + i16;
      l_run[ht] = l_run[ht] * alpha[ht] + (psum[0][hh] + psum[1][hh] + psum[2][hh] + psum[3][hh]);
    }

    // ---- out^T[dims 128w.., heads] += C^T . P^T ----
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      acc[dt][0] *= alpha[0];
      acc[dt][1] *= alpha[1];
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const bf16x8 pb0 = __builtin_bit_cast(
          bf16x8, *reinterpret_cast<const u32x4*>(p_lds + i16 * kTile + 32 * ks + 8 * g));
      const bf16x8 pb1 = __builtin_bit_cast(
          bf16x8, *reinterpret_cast<const u32x4*>(p_lds + (16 + i16) * kTile + 32 * ks + 8 * g));
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const int dim = 128 * w + 16 * dt + i16;
        const uint16_t* col = tile + (32 * ks + g) * kRow + dim;
        u32x4 cv;
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          const uint32_t lo = col[(8 * e2) * kRow];      // token 32ks + 4(2e2) + g
          const uint32_t hi = col[(8 * e2 + 4) * kRow];  // token 32ks + 4(2e2+1) + g
          cv[e2] = lo | (hi << 16);
        }
        const bf16x8 av = __builtin_bit_cast(bf16x8, cv);
        acc[dt][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, pb0, acc[dt][0], 0, 0, 0);
        acc[dt][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, pb1, acc[dt][1], 0, 0, 0);
      }
    }
  }

  // ---- partial state of this (sequence, range, head group) ----
  const size_t pbase = (static_cast<size_t>(b) * a.NR + range) * a.H + head0;
#pragma unroll
  for (int ht = 0; ht < 2; ++ht) {
    const int hh = 16 * ht + i16;
    float* po = a.part_o + (pbase + hh) * kC + 128 * w + 4 * g;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      *reinterpret_cast<f32x4*>(po + 16 * dt) = acc[dt][ht];
    }
    if (w == 0 && g == 0) {
      a.part_ml[(pbase + hh) * 2 + 0] = m_run[ht];
      a.part_ml[(pbase + hh) * 2 + 1] = l_run[ht];
    }
  }
}

// One wavefront per (sequence, head): merge the NR range partials.
__global__ __launch_bounds__(kThreads) void mla_reduce_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_ml,
    uint16_t* __restrict__ out, float* __restrict__ lse_out, int B, int H, int NR) {
  const int lane = threadIdx.x & 63;
  const int task = blockIdx.x * (kThreads / 64) + uniform(threadIdx.x >> 6);
  if (task >= B * H) return;
  const int b = task / H;
  const int h = task - b * H;
  float M = -INFINITY;
  for (int r = 0; r < NR; ++r) {
    M = fmaxf(M, part_ml[((static_cast<size_t>(b) * NR + r) * H + h) * 2]);
  }
  constexpr int DPL = kC / 64;
  float accv[DPL];
#pragma unroll
  for (int d = 0; d < DPL; ++d) accv[d] = 0.f;
  float L = 0.f;
  if (M != -INFINITY) {
    for (int r = 0; r < NR; ++r) {
      const size_t p = (static_cast<size_t>(b) * NR + r) * H + h;
      const float m = part_ml[p * 2];
      if (m == -INFINITY) continue;
      const float wgt = fast_exp2(m - M);
      L += part_ml[p * 2 + 1] * wgt;
      const float* po = part_o + p * kC + lane * DPL;
#pragma unroll
      for (int d = 0; d < DPL; ++d) accv[d] += po[d] * wgt;
    }
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  uint16_t* ob = out + static_cast<size_t>(task) * kC + lane * DPL;
#pragma unroll
  for (int d = 0; d < DPL; ++d) ob[d] = f2bf(accv[d] * inv);
  if (lse_out != nullptr && lane == 0) {
    lse_out[task] = L > 0.f ? (M + __log2f(L)) * 0.6931471805599453f : -INFINITY;
  }
}

int default_ranges(int B, int H) {
  const int wgs_per_range = B * (H / kHeadsPerGroup);
  int nr = (device_cu_count() + wgs_per_range - 1) / wgs_per_range;
  return nr < 1 ? 1 : nr;
}

}  // namespace
}  // namespace voom

using namespace voom;

extern "C" size_t voom_mla_workspace_bytes(int batch, int num_heads, int num_ranges) {
  if (batch <= 0 || num_heads <= 0) return 0;
  if (num_ranges <= 0) num_ranges = default_ranges(batch, num_heads);
  const size_t n = static_cast<size_t>(batch) * num_ranges * num_heads;
  return ((n * kC * sizeof(float) + 255) & ~size_t(255)) + n * 2 * sizeof(float);
}

extern "C" int voom_mla_absorbed_decode(const void* q_lat, const void* lat_pool,
                                        const int32_t* block_table, const int32_t* ctx_lens,
                                        void* out_c, float* lse_out, void* workspace,
                                        size_t ws_bytes, int batch, int num_heads,
                                        int latent_dim, int c_dim, int page_tokens, int max_pages,
                                        int num_slots, float scale, int num_ranges,
                                        hipStream_t stream) {
  VOOM_REQUIRE(q_lat && lat_pool && block_table && ctx_lens && out_c && workspace,
               "mla_absorbed_decode: null pointer argument");
  VOOM_REQUIRE(latent_dim == kLat && c_dim == kC,
               "mla_absorbed_decode: latent %d / c_dim %d unsupported (576 / 512)", latent_dim,
               c_dim);
  VOOM_REQUIRE(batch > 0 && num_heads > 0 && num_heads % kHeadsPerGroup == 0,
               "mla_absorbed_decode: num_heads %d must be a positive multiple of 32", num_heads);
  VOOM_REQUIRE(is_pow2(page_tokens) && page_tokens >= kTile && page_tokens <= 4096,
               "mla_absorbed_decode: page_tokens %d must be a power of two in [64, 4096]",
               page_tokens);
  VOOM_REQUIRE(max_pages > 0 && num_slots > 0, "mla_absorbed_decode: empty table or pool");
  VOOM_REQUIRE(static_cast<long long>(max_pages) * page_tokens < (1LL << 30),
               "mla_absorbed_decode: table capacity too large");
  if (num_ranges <= 0) num_ranges = default_ranges(batch, num_heads);
  const size_t need = voom_mla_workspace_bytes(batch, num_heads, num_ranges);
  VOOM_REQUIRE(ws_bytes >= need, "mla_absorbed_decode: workspace %zu bytes < required %zu",
               ws_bytes, need);
  VOOM_REQUIRE(reinterpret_cast<uintptr_t>(q_lat) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(lat_pool) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(workspace) % 16 == 0,
               "mla_absorbed_decode: q, pool and workspace must be 16-byte aligned");
  const long long grid = static_cast<long long>(batch) * num_ranges * (num_heads / kHeadsPerGroup);
  VOOM_REQUIRE(grid < (1LL << 31), "mla_absorbed_decode: grid too large");

  const size_t n = static_cast<size_t>(batch) * num_ranges * num_heads;
  MlaArgs a;
  a.q = static_cast<const uint16_t*>(q_lat);
  a.lat = static_cast<const uint16_t*>(lat_pool);
  a.table = block_table;
  a.ctx_lens = ctx_lens;
  a.part_o = static_cast<float*>(workspace);
  a.part_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                       ((n * kC * sizeof(float) + 255) & ~size_t(255)));
  a.B = batch;
  a.H = num_heads;
  a.NR = num_ranges;
  a.max_pages = max_pages;
  a.pt_shift = ilog2(page_tokens);
  a.num_slots = num_slots;
  a.scale_log2e = scale * 1.4426950408889634f;
  hipLaunchKernelGGL(mla_latent_kernel, dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0,
                     stream, a);
  int rc = VOOM_LAUNCH_CHECK("mla_absorbed_decode: latent kernel launch");
  if (rc) return rc;
  const unsigned red_grid = static_cast<unsigned>((batch * num_heads + 3) / 4);
  hipLaunchKernelGGL(mla_reduce_kernel, dim3(red_grid), dim3(kThreads), 0, stream, a.part_o,
                     a.part_ml, static_cast<uint16_t*>(out_c), lse_out, batch, num_heads,
                     num_ranges);
  return VOOM_LAUNCH_CHECK("mla_absorbed_decode: reduce kernel launch");
}
