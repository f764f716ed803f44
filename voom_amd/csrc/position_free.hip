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

// Table entry and raw logical position of key `key` (one per lane).  The
// loads are unconditional -- a key past the end reads entry 0, so a wavefront
// issues the same number of loads every block -- and only the loads: the
// arithmetic on them waits for pf_key_finish, so a wait for these loads never
// covers loads issued after them.  Requires TK > 0.
__device__ __forceinline__ void pf_key_load(const PfArgs& a, int key, int& page, int& pos) {
  const int k = key < a.TK ? key : 0;
  page = a.table[k / a.BLOCK];
  pos = a.k_pos[k];
}

// Page row of `key` for kv head `kvh` (split in 32-bit halves for the
// cross-lane reads) and its position clamped into the tables.  A key past the
// end gets row 0 and position 0; page ids out of range read page 0.
__device__ __forceinline__ void pf_key_finish(const PfArgs& a, int kvh, int key, int page,
                                              int pos, int& row_lo, int& row_hi, int& kpos) {
  long long row = 0;
  kpos = 0;
  if (key < a.TK) {
    const int blk = key / a.BLOCK;
    page = static_cast<unsigned>(page) < static_cast<unsigned>(a.P) ? page : 0;
    row = (static_cast<long long>(page) * a.NKV + kvh) * a.BLOCK + (key - blk * a.BLOCK);
    kpos = pos < 0 ? 0 : (pos >= a.max_pos ? a.max_pos - 1 : pos);
  }
  row_lo = static_cast<int>(row & 0xffffffff);
  row_hi = static_cast<int>(row >> 32);
}

__device__ __forceinline__ long long pf_row_of(int row_lo, int row_hi, int src) {
  return (static_cast<long long>(__shfl(row_hi, src)) << 32) |
         static_cast<unsigned>(__shfl(row_lo, src));
}

// One workgroup per (batch row, split, group of HW kv heads); wavefront w
// takes kv head HW * group + w.  All HW wavefronts walk the same key blocks,
// so a block's cos/sin rows are loaded once per workgroup into a shared LDS
// tile (double-buffered, one barrier per block) while every wavefront keeps
// its own K rows in registers and stages its own V rows in a private LDS
// slice.  Block i + 1's K and V rows, and its cos/sin rows, are in flight
// while block i is computed; table entries are fetched two blocks ahead.
// Partials are indexed (segment * splits + split).
template <int D, int HW>
__global__ __launch_bounds__(HW * kWave) __attribute__((amdgpu_waves_per_eu(2)))
void pf_attention_kernel(PfArgs a) {
  constexpr int KS = D / 32;     // k-steps of the score MFMA
  constexpr int HS = D / 64;     // k-steps in one rotary half
  constexpr int DT = D / 16;     // dim tiles of out^T
  constexpr int kVRow = D + 8;   // LDS row stride of the staged V rows (elements)
  constexpr int kVLoads = kKeys * D / 8 / kWave;  // 16-byte V chunks per lane
  constexpr int CPR = D / 8;     // 16-byte chunks in one cos (or sin) row of D/2 floats
  constexpr int kCsPerThread = kKeys * 2 * CPR / (HW * kWave);
  static_assert(kCsPerThread * HW * kWave == kKeys * 2 * CPR, "cos/sin tile split");
  __shared__ __attribute__((aligned(16))) uint16_t v_stage[HW][kKeys * kVRow];
  // [buffer][key][cos, sin][chunk]: chunk c of key r sits at c ^ (r % CPR), so
  // the 16 lanes that read one chunk of 16 different keys hit distinct banks
  __shared__ f32x4 cs_stage[2][kKeys][2][CPR];

  const int lane = threadIdx.x & (kWave - 1);
  const int wl = uniform(threadIdx.x / kWave);
  const int groups = a.NKV / HW;
  const int kg = blockIdx.x % groups;
  const int rest = blockIdx.x / groups;
  const int split = rest % a.splits;
  const int b = rest / a.splits;
  const int kvh = kg * HW + wl;
  const int seg = b * a.NKV + kvh;
  const size_t pidx = static_cast<size_t>(seg) * a.splits + split;
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
  const int klane = lane & 31;  // the key this lane looks up (lanes 32..63 mirror)
  uint16_t* vs = v_stage[wl];

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

  // K and V rows are read once per call: non-temporal loads (measured 37.7 ->
  // 36.7 us per call at 32,768 keys).
  auto load_k = [&](int rlo, int rhi, u32x4 (&kk)[2][KS]) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const uint16_t* krow = a.k_pages + pf_row_of(rlo, rhi, 16 * t + i16) * D;
#pragma unroll
      for (int s = 0; s < KS; ++s)
        kk[t][s] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(krow + 32 * s + 8 * g));
    }
  };
  auto load_v = [&](int rlo, int rhi, u32x4 (&vv)[kVLoads]) {
#pragma unroll
    for (int u = 0; u < kVLoads; ++u) {
      const int c = u * kWave + lane;
      const int r = c / (D / 8);
      const int col = c - r * (D / 8);
      vv[u] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4*>(a.v_pages + pf_row_of(rlo, rhi, r) * D + 8 * col));
    }
  };
  // V rows, coalesced 16-byte chunks, into this wave's LDS slice
  auto store_v = [&](const u32x4 (&vv)[kVLoads]) {
#pragma unroll
    for (int u = 0; u < kVLoads; ++u) {
      const int c = u * kWave + lane;
      const int r = c / (D / 8);
      const int col = c - r * (D / 8);
      *reinterpret_cast<u32x4*>(vs + r * kVRow + 8 * col) = vv[u];
    }
  };
  // this thread's share of a block's cos/sin rows: chunk id -> (key, table, chunk)
  auto load_cs = [&](int kp, f32x4 (&cr)[kCsPerThread]) {
#pragma unroll
    for (int i = 0; i < kCsPerThread; ++i) {
      const int cid = static_cast<int>(threadIdx.x) + i * HW * kWave;
      const int key = cid / (2 * CPR);
      const int tab = (cid / CPR) & 1;
      const int ch = cid & (CPR - 1);
      const int p = __shfl(kp, key);
      const float* src = (tab ? a.sin_t : a.cos_t) + static_cast<size_t>(p) * (D / 2) + 4 * ch;
      cr[i] = *reinterpret_cast<const f32x4*>(src);
    }
  };
  auto store_cs = [&](int buf, const f32x4 (&cr)[kCsPerThread]) {
#pragma unroll
    for (int i = 0; i < kCsPerThread; ++i) {
      const int cid = static_cast<int>(threadIdx.x) + i * HW * kWave;
      const int key = cid / (2 * CPR);
      const int tab = (cid / CPR) & 1;
      const int ch = cid & (CPR - 1);
      cs_stage[buf][key][tab][ch ^ (key & (CPR - 1))] = cr[i];
    }
  };

  f32x4 acc[DT];
#pragma unroll
  for (int d = 0; d < DT; ++d) acc[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;
  float l_lane = 0.f;

  // ---- prologue: block blo resident (K in registers; V and cos/sin in
  //      LDS), block blo + 1's table entries loaded ----
  int rA_lo = 0, rA_hi = 0, kA = 0;   // rows / position of block bi
  int pgB = 0, psB = 0;               // raw table entry / position of block bi + 1
  u32x4 kc[2][KS];  // K rows of block bi (block bi + 1's once scored)
  if (blo < bhi) {
    int pg, ps;
    pf_key_load(a, blo * kKeys + klane, pg, ps);
    pf_key_finish(a, kvh, blo * kKeys + klane, pg, ps, rA_lo, rA_hi, kA);
    pf_key_load(a, blo + 1 < bhi ? (blo + 1) * kKeys + klane : a.TK, pgB, psB);
    f32x4 c0[kCsPerThread];
    u32x4 v0[kVLoads];
    load_cs(kA, c0);
    load_v(rA_lo, rA_hi, v0);
    load_k(rA_lo, rA_hi, kc);
    store_cs(blo & 1, c0);
    store_v(v0);
  }
  // nothing of the prologue stays in flight into the loop, so the loop's
  // waits count only its own loads
  wait_vmem_all();
  lds_barrier();

  for (int bi = blo; bi < bhi; ++bi) {
    const bool more = bi + 1 < bhi;
    // ---- issue: table entries two ahead, then block bi + 1's rows.  Every
    //      load issues every block; past the split's end they read key
    //      row 0 / table entry 0 (one cache line), so the wait counts stay
    //      exact ----
    int pgC, psC;
    pf_key_load(a, bi + 2 < bhi ? (bi + 2) * kKeys + klane : a.TK, pgC, psC);
    int rB_lo, rB_hi, kB;
    pf_key_finish(a, kvh, more ? (bi + 1) * kKeys + klane : a.TK, pgB, psB, rB_lo, rB_hi,
                  kB);
    u32x4 vn[kVLoads];
    f32x4 cn[kCsPerThread];
    // cos/sin and V now (they are waited for at the end of this block); K
    // once this block's keys are scored and their registers are free
    load_cs(kB, cn);
    load_v(rB_lo, rB_hi, vn);
    int kp[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int r = 0; r < 4; ++r) kp[t][r] = __shfl(kA, 16 * t + 4 * g + r);
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- rotate the keys in registers, score the two 16-key tiles ----
    const int buf = bi & 1;
    f32x4 sc[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int key = 16 * t + i16;
      const int sw = key & (CPR - 1);
#pragma unroll
      for (int s = 0; s < HS; ++s) {
        const int c0 = 8 * s + 2 * g;
        const f32x4 cA = cs_stage[buf][key][0][c0 ^ sw];
        const f32x4 cB = cs_stage[buf][key][0][(c0 + 1) ^ sw];
        const f32x4 sA = cs_stage[buf][key][1][c0 ^ sw];
        const f32x4 sB = cs_stage[buf][key][1][(c0 + 1) ^ sw];
        u32x4 lo_out, hi_out;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t xa = kc[t][s][w];
          const uint32_t xb = kc[t][s + HS][w];
          float ra[2], rb[2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const float av = __builtin_bit_cast(float, h ? (xa & 0xffff0000u) : (xa << 16));
            const float bv = __builtin_bit_cast(float, h ? (xb & 0xffff0000u) : (xb << 16));
            const int e = 2 * w + h;
            const float c = e < 4 ? cA[e] : cB[e - 4];
            const float sv = e < 4 ? sA[e] : sB[e - 4];
            ra[h] = av * c - bv * sv;
            rb[h] = bv * c + av * sv;
          }
          lo_out[w] = pack_bf16x2(ra[0], ra[1]);
          hi_out[w] = pack_bf16x2(rb[0], rb[1]);
        }
        kc[t][s] = lo_out;
        kc[t][s + HS] = hi_out;
      }
      f32x4 acc_s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        acc_s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kc[t][s]),
                                                        __builtin_bit_cast(bf16x8, qop[s]),
                                                        acc_s, 0, 0, 0);
      }
      sc[t] = acc_s;
    }
    load_k(rB_lo, rB_hi, kc);

    // ---- mask, online softmax; lane (column i16, group g) holds keys
    //      16t + 4g + r ----
    float x[2][4];
    float mb = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kk = 16 * t + 4 * g + r;
        const bool vis = col_ok && bi * kKeys + kk < a.TK && kp[t][r] <= qpos;
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

    // ---- block bi + 1's V rows into the slice once this block's reads of
    //      it are done, its cos/sin into the other buffer; after the barrier
    //      every wave has finished with this block's tiles ----
    if (more) {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      store_v(vn);
      store_cs(buf ^ 1, cn);
    }
    lds_barrier();
    rA_lo = rB_lo;
    rA_hi = rB_hi;
    kA = kB;
    pgB = pgC;
    psB = psC;
  }

  const float l_tot = wave_sum_across_groups(l_lane);
  if (col_ok) {
    float* po = a.part_o + (pidx * kCols + i16) * D + 4 * g;
#pragma unroll
    for (int d = 0; d < DT; ++d) *reinterpret_cast<f32x4*>(po + 16 * d) = acc[d];
    if (g == 0) {
      a.part_ml[(pidx * kCols + i16) * 2 + 0] = m_run;
      a.part_ml[(pidx * kCols + i16) * 2 + 1] = l_tot;
    }
  }
}

// One workgroup per (segment, column, 32-dim slice of the output row): its
// kRedWaves wavefronts each merge a contiguous share of the segment's split
// partials, then wave 0 merges their states and writes the slice of
// out[b][head][tq][:] (zeros when no key was visible).  Spreading a row over
// D/32 workgroups spreads the partial reads over that many more CUs.  Lane
// (r, j) of a wavefront reads dims 4j..4j+3 of the slice for split r of each
// group of kRedRows consecutive splits; a batch of kRedIters groups is loaded
// before its first use (one memory round trip), and the batch maximum
// rescales the running state.  A split with no visible key left m = -inf and
// weighs 0.
constexpr int kRedWaves = 4;
constexpr int kRedDims = 32;                  // output dims per workgroup
constexpr int kRedCols = kRedDims / 4;        // lanes across one slice (float4 each)
constexpr int kRedRows = kWave / kRedCols;    // splits per wave-wide load
constexpr int kRedIters = 8;                  // wave-wide loads per batch

template <int D>
__global__ __launch_bounds__(kRedWaves * kWave) void pf_reduce_kernel(PfArgs a, uint16_t* out) {
  constexpr int kSlices = D / kRedDims;
  __shared__ float st_ml[kRedWaves][2];
  __shared__ __attribute__((aligned(16))) f32x4 st_o[kRedWaves][kRedCols];
  const int lane = threadIdx.x & (kWave - 1);
  const int wl = uniform(threadIdx.x / kWave);
  const int NC = a.G * a.TQ;
  const int slice = blockIdx.x % kSlices;
  const int task = blockIdx.x / kSlices;
  const int seg = task / NC;
  const int n = task - seg * NC;
  const int r = lane / kRedCols;
  const int j = lane - r * kRedCols;
  const int s0 = static_cast<int>(static_cast<long long>(wl) * a.splits / kRedWaves);
  const int cnt = static_cast<int>(static_cast<long long>(wl + 1) * a.splits / kRedWaves) - s0;
  const size_t first = static_cast<size_t>(seg) * a.splits + s0;
  const float2* ml2 = reinterpret_cast<const float2*>(a.part_ml);
  const int dim0 = slice * kRedDims + 4 * j;

  float M = -INFINITY;
  float L = 0.f;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int i0 = 0; i0 < cnt; i0 += kRedRows * kRedIters) {
    float2 ml[kRedIters];
    f32x4 o[kRedIters];
#pragma unroll
    for (int u = 0; u < kRedIters; ++u) {
      const int i = i0 + u * kRedRows + r;
      const size_t p = (first + (i < cnt ? i : cnt - 1)) * kCols + n;
      ml[u] = ml2[p];
      o[u] = *reinterpret_cast<const f32x4*>(a.part_o + p * D + dim0);
    }
    // everything above issues before the first use
    __builtin_amdgcn_sched_barrier(0);
    float Mc = -INFINITY;
#pragma unroll
    for (int u = 0; u < kRedIters; ++u) {
      const bool live = i0 + u * kRedRows + r < cnt;
      if (live) Mc = fmaxf(Mc, ml[u].x);
    }
    Mc = wave_max_uniform(Mc);  // DPP moves + v_readlane, no LDS crossbar trips
    const float Mn = fmaxf(M, Mc);
    if (Mn == -INFINITY) continue;  // wave-uniform: nothing visible yet
    const float rescale = M == -INFINITY ? 0.f : fast_exp2(M - Mn);
    float Lc = 0.f;
    acc *= rescale;
#pragma unroll
    for (int u = 0; u < kRedIters; ++u) {
      const bool live = i0 + u * kRedRows + r < cnt && ml[u].x != -INFINITY;
      const float w = live ? fast_exp2(ml[u].x - Mn) : 0.f;
      acc += o[u] * w;
      Lc += ml[u].y * w;
    }
    // each split's l is held by all kRedCols lanes of its row: count lane j == 0
    Lc = wave_sum_uniform(j == 0 ? Lc : 0.f);
    L = L * rescale + Lc;
    M = Mn;
  }
  // rows of one wave share M: the lanes of a column sum their rows
#pragma unroll
  for (int x = kRedCols; x < kWave; x <<= 1) {
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] += __shfl_xor(acc[e], x);
  }
  if (lane == 0) {
    st_ml[wl][0] = M;
    st_ml[wl][1] = L;
  }
  if (r == 0) st_o[wl][j] = acc;
  __syncthreads();
  if (wl != 0 || r != 0) return;
  float Mt = -INFINITY;
#pragma unroll
  for (int k = 0; k < kRedWaves; ++k) Mt = fmaxf(Mt, st_ml[k][0]);
  float Lt = 0.f;
  f32x4 res = {0.f, 0.f, 0.f, 0.f};
  if (Mt != -INFINITY) {
#pragma unroll
    for (int k = 0; k < kRedWaves; ++k) {
      const float mk = st_ml[k][0];
      const float wk = mk == -INFINITY ? 0.f : fast_exp2(mk - Mt);
      Lt += st_ml[k][1] * wk;
      res += st_o[k][j] * wk;
    }
  }
  const float inv = Lt > 0.f ? 1.f / Lt : 0.f;
  const int b = seg / a.NKV;
  const int kvh = seg - b * a.NKV;
  const int hj = n / a.TQ;
  const int tq = n - hj * a.TQ;
  uint16_t* ob =
      out + ((static_cast<size_t>(b) * a.NQ + kvh * a.G + hj) * a.TQ + tq) * D + dim0;
  const uint32_t w0 = pack_bf16x2(res[0] * inv, res[1] * inv);
  const uint32_t w1 = pack_bf16x2(res[2] * inv, res[3] * inv);
  *reinterpret_cast<uint2*>(ob) = make_uint2(w0, w1);
}

template <int D>
void launch_pf_attention(int hw, dim3 grid, dim3 block, hipStream_t stream, const PfArgs& a) {
  switch (hw) {
    case 8: hipLaunchKernelGGL((pf_attention_kernel<D, 8>), grid, block, 0, stream, a); break;
    case 4: hipLaunchKernelGGL((pf_attention_kernel<D, 4>), grid, block, 0, stream, a); break;
    case 2: hipLaunchKernelGGL((pf_attention_kernel<D, 2>), grid, block, 0, stream, a); break;
    default: hipLaunchKernelGGL((pf_attention_kernel<D, 1>), grid, block, 0, stream, a); break;
  }
}

int pf_splits(int B, int NKV, int TK, int num_splits) {
  const int nb = (TK + kKeys - 1) / kKeys;
  int s = num_splits > 0 ? num_splits
                         : (8 * device_cu_count() + B * NKV - 1) / (B * NKV);
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
  VOOM_REQUIRE(block_size > 0 && num_pages > 0 && num_keys >= 0 && num_keys <= (1 << 30) &&
                   max_position > 0,
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
                   reinterpret_cast<uintptr_t>(workspace) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(out) % 16 == 0,
               "%s: tensors must be 16-byte aligned", who);
  const long long waves = static_cast<long long>(batch) * num_kv_heads * splits;
  VOOM_REQUIRE(waves < (1LL << 30) &&
                   static_cast<long long>(batch) * num_kv_heads * G * num_queries * 4 < (1LL << 31),
               "%s: grid too large", who);

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
  // kv heads per workgroup: the largest of 8, 4, 2, 1 that divides NKV
  const int hw = num_kv_heads % 8 == 0 ? 8 : num_kv_heads % 4 == 0 ? 4 : num_kv_heads % 2 == 0 ? 2 : 1;
  const dim3 grid(static_cast<unsigned>(waves / hw));
  const dim3 block(static_cast<unsigned>(hw * kWave));
  const dim3 grid_red(static_cast<unsigned>(static_cast<long long>(batch) * num_kv_heads * G *
                                            num_queries * (head_dim / kRedDims)));
  auto* oo = static_cast<uint16_t*>(out);
  if (head_dim == 128) {
    launch_pf_attention<128>(hw, grid, block, stream, a);
  } else {
    launch_pf_attention<64>(hw, grid, block, stream, a);
  }
  const int rc = VOOM_LAUNCH_CHECK("position_free_attention: kernel launch");
  if (rc) return rc;
  if (head_dim == 128) {
    hipLaunchKernelGGL(pf_reduce_kernel<128>, grid_red, dim3(kRedWaves * kWave), 0, stream, a,
                       oo);
  } else {
    hipLaunchKernelGGL(pf_reduce_kernel<64>, grid_red, dim3(kRedWaves * kWave), 0, stream, a,
                       oo);
  }
  return VOOM_LAUNCH_CHECK("position_free_attention: reduce launch");
}
