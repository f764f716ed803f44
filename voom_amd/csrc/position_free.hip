// Position-free paged attention for gfx950.
//
// Restates the reference's position_free_paged_attention (runtime/
// pic_attention.py:22-232): keys are stored *before* RoPE in physical pages
// [pages, NKV, BLOCK, D] (V in the same layout), a block table maps the
// logical sequence to pages (a page id may repeat: that is the sharing
// primitive), and every key is rotated at its logical position while the
// attention runs.  Per the reference:
//   q      [B, NQ, TQ, D]  already rotated
//   key k  rotated with fp32 cos/sin tables [max_pos, D/2] (NeoX rotate-half)
//          and rounded to bf16 before the dot product (:81-90)
//   mask   a key attends iff k_positions[k] <= q_positions[tq]     (:57-58)
//   out    softmax(q.k * scale) . v, zeros when no key is visible   (:117-128)
//
// MI355X mapping.  Segments are (batch row, kv head); the GQA heads and the
// TQ queries of a segment form the N = G*TQ <= 16 columns of one MFMA tile,
// so each key byte is read once for all of them.  A segment's 32-key blocks
// are split over several wavefronts (split-K), each leaving a partial
// softmax state that pf_reduce_kernel merges.  Per 32-key block a wavefront:
//   - looks up the 32 page rows and positions (one key per lane),
//   - loads its K rows as MFMA A operands (16 bytes per lane per k-step),
//     rotates them in registers -- dims d and d + D/2 sit in k-steps s and
//     s + D/64 of the same lane -- and rounds them to bf16,
//   - scores^T[key][column] = K_rot . Q^T with v_mfma_f32_16x16x32_bf16,
//   - stages the 32 V rows in its own LDS slice and reads V^T operands back
//     with ds_read_b64_tr_b16, so out^T += V^T . P^T needs no V^T storage.
// The two 16-key score tiles leave lane (column j, group g) holding keys
// 4g + r and 16 + 4g + r; the transposed V reads address exactly those rows,
// so P^T is used straight from the score registers.
#include "common.h"

namespace voom {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kKeys = 32;  // keys per block
constexpr int kCols = 16;  // MFMA N: (head, query) columns of a segment

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

struct PfArgs {
  const uint16_t* q;         // [B, NQ, TQ, D]
  const uint16_t* k_pages;   // [P, NKV, BLOCK, D]
  const uint16_t* v_pages;   // [P, NKV, BLOCK, D]
  const int32_t* table;      // [ceil(TK / BLOCK)]
  const int32_t* k_pos;      // [TK]
  const int32_t* q_pos;      // [TQ]
  const float* cos_t;        // [max_pos, D/2]
  const float* sin_t;        // [max_pos, D/2]
  float* part_o;             // [waves, 16, D]
  float* part_ml;            // [waves, 16, 2]
  int B, NQ, TQ, NKV, G, BLOCK, P, TK, max_pos, splits;
  float scale_log2e;
};

template <int D>
__global__ __launch_bounds__(kThreads) void pf_attention_kernel(PfArgs a) {
  constexpr int KS = D / 32;     // k-steps of the score MFMA
  constexpr int HS = D / 64;     // k-steps in one rotary half
  constexpr int DT = D / 16;     // dim tiles of out^T
  constexpr int kVRow = D + 8;   // LDS row stride of the staged V rows (elements)
  __shared__ __attribute__((aligned(16))) uint16_t v_stage[kWaves][kKeys * kVRow];

  const int lane = threadIdx.x & (kWave - 1);
  const int wl = uniform(threadIdx.x / kWave);
  const int wave = blockIdx.x * kWaves + wl;
  const int n_seg = a.B * a.NKV;
  if (wave >= n_seg * a.splits) return;
  const int seg = wave / a.splits;
  const int split = wave - seg * a.splits;
  const int b = seg / a.NKV;
  const int kvh = seg - b * a.NKV;
  const int nb = (a.TK + kKeys - 1) / kKeys;
  const int blo = static_cast<int>(static_cast<long long>(split) * nb / a.splits);
  const int bhi = static_cast<int>(static_cast<long long>(split + 1) * nb / a.splits);

  const int i16 = lane & 15;
  const int g = lane >> 4;
  const int NC = a.G * a.TQ;
  const bool col_ok = i16 < NC;
  const int cj = col_ok ? i16 / a.TQ : 0;     // head within the group
  const int ctq = col_ok ? i16 - cj * a.TQ : 0;  // query
  const int qpos = a.q_pos[ctq];

  // Q^T operand: lane (column i16, group g) holds q[head][tq][32s + 8g .. +8]
  u32x4 qop[KS];
  {
    const uint16_t* qh =
        a.q + ((static_cast<size_t>(b) * a.NQ + kvh * a.G + cj) * a.TQ + ctq) * D;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const u32x4 z = {0u, 0u, 0u, 0u};
      qop[s] = col_ok ? *reinterpret_cast<const u32x4*>(qh + 32 * s + 8 * g) : z;
    }
  }

  f32x4 acc[DT];
#pragma unroll
  for (int d = 0; d < DT; ++d) acc[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;
  float l_lane = 0.f;
  uint16_t* vs = v_stage[wl];

  for (int bi = blo; bi < bhi; ++bi) {
    // ---- key rows and positions, one key per lane (lanes 32..63 mirror) ----
    const int key = bi * kKeys + (lane & 31);
    const bool kvalid = key < a.TK;
    long long row = 0;
    int kpos = 0;
    if (kvalid) {
      const int blk = key / a.BLOCK;
      int page = a.table[blk];
      page = static_cast<unsigned>(page) < static_cast<unsigned>(a.P) ? page : 0;
      row = (static_cast<long long>(page) * a.NKV + kvh) * a.BLOCK + (key - blk * a.BLOCK);
      kpos = a.k_pos[key];
      kpos = kpos < 0 ? 0 : (kpos >= a.max_pos ? a.max_pos - 1 : kpos);
    }
    const int row_lo = static_cast<int>(row & 0xffffffff);
    const int row_hi = static_cast<int>(row >> 32);

    // ---- V rows into this wave's LDS slice (coalesced 16-byte chunks) ----
    constexpr int kChunks = kKeys * D / 8;
#pragma unroll
    for (int c0 = 0; c0 < kChunks; c0 += kWave) {
      const int c = c0 + lane;
      const int r = c / (D / 8);
      const int col = c - r * (D / 8);
      const long long vr = (static_cast<long long>(__shfl(row_hi, r)) << 32) |
                           static_cast<unsigned>(__shfl(row_lo, r));
      const u32x4 val = *reinterpret_cast<const u32x4*>(a.v_pages + vr * D + 8 * col);
      *reinterpret_cast<u32x4*>(vs + r * kVRow + 8 * col) = val;
    }

    // ---- scores of the two 16-key tiles, keys rotated in registers ----
    f32x4 sc[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int kk = 16 * t + i16;
      const long long kr = (static_cast<long long>(__shfl(row_hi, kk)) << 32) |
                           static_cast<unsigned>(__shfl(row_lo, kk));
      const int p = __shfl(kpos, kk);
      const uint16_t* krow = a.k_pages + kr * D;
      u32x4 kv[KS];
#pragma unroll
      for (int s = 0; s < KS; ++s) kv[s] = *reinterpret_cast<const u32x4*>(krow + 32 * s + 8 * g);
      const float* cr = a.cos_t + static_cast<size_t>(p) * (D / 2);
      const float* sr = a.sin_t + static_cast<size_t>(p) * (D / 2);
#pragma unroll
      for (int s = 0; s < HS; ++s) {
        const f32x4 c0 = *reinterpret_cast<const f32x4*>(cr + 32 * s + 8 * g);
        const f32x4 c1 = *reinterpret_cast<const f32x4*>(cr + 32 * s + 8 * g + 4);
        const f32x4 s0 = *reinterpret_cast<const f32x4*>(sr + 32 * s + 8 * g);
        const f32x4 s1 = *reinterpret_cast<const f32x4*>(sr + 32 * s + 8 * g + 4);
        const float cs[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
        const float sn[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
        u32x4 lo_out, hi_out;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t xa = kv[s][w];
          const uint32_t xb = kv[s + HS][w];
          float ra[2], rb[2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const float av = __builtin_bit_cast(float, h ? (xa & 0xffff0000u) : (xa << 16));
            const float bv = __builtin_bit_cast(float, h ? (xb & 0xffff0000u) : (xb << 16));
            const int e = 2 * w + h;
            ra[h] = av * cs[e] - bv * sn[e];
            rb[h] = bv * cs[e] + av * sn[e];
          }
          lo_out[w] = pack_bf16x2(ra[0], ra[1]);
          hi_out[w] = pack_bf16x2(rb[0], rb[1]);
        }
        kv[s] = lo_out;
        kv[s + HS] = hi_out;
      }
      f32x4 acc_s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        acc_s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kv[s]),
                                                        __builtin_bit_cast(bf16x8, qop[s]),
                                                        acc_s, 0, 0, 0);
      }
      sc[t] = acc_s;
    }

    // ---- mask, online softmax; lane (column i16, group g) holds keys
    //      16t + 4g + r ----
    float x[2][4];
    float mb = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kk = 16 * t + 4 * g + r;
        // the cross-lane read runs in every lane: a lane it reads from must
        // be active, so it stays outside the short-circuit condition
        const int kp = __shfl(kpos, kk);
        const bool vis = col_ok && bi * kKeys + kk < a.TK && kp <= qpos;
        x[t][r] = vis ? sc[t][r] * a.scale_log2e : -INFINITY;
        mb = fmaxf(mb, x[t][r]);
      }
    }
    mb = wave_max_across_groups(mb);
    const float m_new = fmaxf(m_run, mb);
    const float alpha = m_new == m_run ? 1.f : fast_exp2(m_run - m_new);
    m_run = m_new;
    u32x4 pk;
    float ps = 0.f;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      float p[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) p[r] = x[t][r] == -INFINITY ? 0.f : fast_exp2(x[t][r] - m_new);
      const uint32_t w0 = pack_bf16x2(p[0], p[1]);
      const uint32_t w1 = pack_bf16x2(p[2], p[3]);
      pk[2 * t] = w0;
      pk[2 * t + 1] = w1;
      ps += __builtin_bit_cast(float, w0 << 16) + __builtin_bit_cast(float, w0 & 0xffff0000u) +
            __builtin_bit_cast(float, w1 << 16) + __builtin_bit_cast(float, w1 & 0xffff0000u);
    }
    l_lane = l_lane * alpha + ps;

    // ---- out^T[dims][columns] += V^T . P^T ----
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // V rows are in LDS
#pragma unroll
    for (int d = 0; d < DT; ++d) acc[d] *= alpha;
    const bf16x8 pb = __builtin_bit_cast(bf16x8, pk);
    // lane i16 of group g addresses key row 4g + i16/4 (and +16) at dims
    // 16dt + 4*(i16%4): after the transpose lane l holds keys 4g..4g+3 (and
    // 16 + 4g..) of dim 16dt + l%16
    const uint16_t* vb = vs + (4 * g + (i16 >> 2)) * kVRow + 4 * (i16 & 3);
#pragma unroll
    for (int d = 0; d < DT; ++d) {
      const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(vb + 16 * d));
      const bf16x4 hi =
          __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(vb + 16 * kVRow + 16 * d));
      const bf16x8 av = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      acc[d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, pb, acc[d], 0, 0, 0);
    }
    // the next block overwrites the slice: its reads must have completed
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }

  const float l_tot = wave_sum_across_groups(l_lane);
  if (col_ok) {
    float* po = a.part_o + (static_cast<size_t>(wave) * kCols + i16) * D + 4 * g;
#pragma unroll
    for (int d = 0; d < DT; ++d) *reinterpret_cast<f32x4*>(po + 16 * d) = acc[d];
    if (g == 0) {
      a.part_ml[(static_cast<size_t>(wave) * kCols + i16) * 2 + 0] = m_run;
      a.part_ml[(static_cast<size_t>(wave) * kCols + i16) * 2 + 1] = l_tot;
    }
  }
}

// One wavefront per (segment, column): merges the segment's split partials
// and writes out[b][head][tq][:] (zeros when no key was visible).
template <int D>
__global__ __launch_bounds__(kThreads) void pf_reduce_kernel(PfArgs a, uint16_t* out) {
  constexpr int DPL = D / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int task = blockIdx.x * kWaves + uniform(threadIdx.x / kWave);
  const int NC = a.G * a.TQ;
  if (task >= a.B * a.NKV * NC) return;
  const int seg = task / NC;
  const int n = task - seg * NC;
  const int b = seg / a.NKV;
  const int kvh = seg - b * a.NKV;
  const int j = n / a.TQ;
  const int tq = n - j * a.TQ;
  float M = -INFINITY;
  for (int s = 0; s < a.splits; ++s) {
    M = fmaxf(M, a.part_ml[((static_cast<size_t>(seg) * a.splits + s) * kCols + n) * 2]);
  }
  float L = 0.f;
  float acc[DPL];
#pragma unroll
  for (int d = 0; d < DPL; ++d) acc[d] = 0.f;
  if (M != -INFINITY) {
    for (int s = 0; s < a.splits; ++s) {
      const size_t p = (static_cast<size_t>(seg) * a.splits + s) * kCols + n;
      const float m = a.part_ml[p * 2];
      if (m == -INFINITY) continue;
      const float w = fast_exp2(m - M);
      L += a.part_ml[p * 2 + 1] * w;
      const float* po = a.part_o + p * D + lane * DPL;
#pragma unroll
      for (int d = 0; d < DPL; ++d) acc[d] += po[d] * w;
    }
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  uint16_t* o =
      out + ((static_cast<size_t>(b) * a.NQ + kvh * a.G + j) * a.TQ + tq) * D + lane * DPL;
#pragma unroll
  for (int d = 0; d < DPL; ++d) o[d] = f2bf(acc[d] * inv);
}

int pf_splits(int B, int NKV, int TK, int num_splits) {
  const int nb = (TK + kKeys - 1) / kKeys;
  int s = num_splits > 0 ? num_splits
                         : (4 * device_cu_count() + B * NKV - 1) / (B * NKV);
  if (s > nb) s = nb;
  return s < 1 ? 1 : s;
}

}  // namespace
}  // namespace voom

using namespace voom;

extern "C" size_t voom_position_free_workspace_bytes(int batch, int num_kv_heads, int head_dim,
                                                     int num_keys, int num_splits) {
  if (batch <= 0 || num_kv_heads <= 0 || head_dim <= 0 || num_keys < 0) return 0;
  const size_t waves =
      static_cast<size_t>(batch) * num_kv_heads * pf_splits(batch, num_kv_heads, num_keys, num_splits);
  const size_t o = waves * kCols * head_dim * sizeof(float);
  return ((o + 255) & ~size_t(255)) + waves * kCols * 2 * sizeof(float);
}

extern "C" int voom_position_free_attention(
    const void* q, const void* k_pages, const void* v_pages, const int32_t* block_table,
    const int32_t* key_positions, const int32_t* query_positions, const float* cos_table,
    const float* sin_table, void* out, void* workspace, size_t ws_bytes, int batch,
    int num_q_heads, int num_queries, int num_kv_heads, int head_dim, int block_size,
    int num_pages, int num_keys, int max_position, float scale, int num_splits,
    hipStream_t stream) {
  const char* who = "position_free_attention";
  VOOM_REQUIRE(q && k_pages && v_pages && out && workspace && query_positions && cos_table &&
                   sin_table,
               "%s: null pointer argument", who);
  VOOM_REQUIRE(num_keys == 0 || (block_table && key_positions), "%s: null key arrays", who);
  VOOM_REQUIRE(batch > 0 && num_queries > 0 && num_kv_heads > 0 && num_q_heads > 0 &&
                   num_q_heads % num_kv_heads == 0,
               "%s: unsupported head or position geometry", who);
  const int G = num_q_heads / num_kv_heads;
  VOOM_REQUIRE(G * num_queries <= kCols,
               "%s: heads per kv head x queries = %d exceeds %d", who, G * num_queries, kCols);
  VOOM_REQUIRE(head_dim == 64 || head_dim == 128, "%s: head_dim %d unsupported (64 or 128)",
               who, head_dim);
  VOOM_REQUIRE(block_size > 0 && num_pages > 0 && num_keys >= 0 && max_position > 0,
               "%s: bad page or position geometry", who);
  const int splits = pf_splits(batch, num_kv_heads, num_keys, num_splits);
  const size_t need =
      voom_position_free_workspace_bytes(batch, num_kv_heads, head_dim, num_keys, splits);
  VOOM_REQUIRE(ws_bytes >= need, "%s: workspace %zu bytes < required %zu", who, ws_bytes, need);
  VOOM_REQUIRE(reinterpret_cast<uintptr_t>(q) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(k_pages) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(v_pages) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(cos_table) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(sin_table) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(workspace) % 16 == 0,
               "%s: tensors must be 16-byte aligned", who);
  const long long waves = static_cast<long long>(batch) * num_kv_heads * splits;
  VOOM_REQUIRE(waves < (1LL << 30), "%s: grid too large", who);

  PfArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k_pages = static_cast<const uint16_t*>(k_pages);
  a.v_pages = static_cast<const uint16_t*>(v_pages);
  a.table = block_table;
  a.k_pos = key_positions;
  a.q_pos = query_positions;
  a.cos_t = cos_table;
  a.sin_t = sin_table;
  a.part_o = static_cast<float*>(workspace);
  const size_t o = static_cast<size_t>(waves) * kCols * head_dim * sizeof(float);
  a.part_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) + ((o + 255) & ~size_t(255)));
  a.B = batch;
  a.NQ = num_q_heads;
  a.TQ = num_queries;
  a.NKV = num_kv_heads;
  a.G = G;
  a.BLOCK = block_size;
  a.P = num_pages;
  a.TK = num_keys;
  a.max_pos = max_position;
  a.splits = splits;
  a.scale_log2e = scale * 1.4426950408889634f;
  const dim3 grid(static_cast<unsigned>((waves + kWaves - 1) / kWaves));
  const dim3 grid_red(
      static_cast<unsigned>((static_cast<long long>(batch) * num_kv_heads * G * num_queries +
                             kWaves - 1) / kWaves));
  auto* oo = static_cast<uint16_t*>(out);
  if (head_dim == 128) {
    hipLaunchKernelGGL(pf_attention_kernel<128>, grid, dim3(kThreads), 0, stream, a);
    const int rc = VOOM_LAUNCH_CHECK("position_free_attention: kernel launch");
    if (rc) return rc;
    hipLaunchKernelGGL(pf_reduce_kernel<128>, grid_red, dim3(kThreads), 0, stream, a, oo);
  } else {
    hipLaunchKernelGGL(pf_attention_kernel<64>, grid, dim3(kThreads), 0, stream, a);
    const int rc = VOOM_LAUNCH_CHECK("position_free_attention: kernel launch");
    if (rc) return rc;
    hipLaunchKernelGGL(pf_reduce_kernel<64>, grid_red, dim3(kThreads), 0, stream, a, oo);
  }
  return VOOM_LAUNCH_CHECK("position_free_attention: reduce launch");
}
