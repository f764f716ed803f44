// Position-free paged attention for gfx950.
//
// Restates the reference's position_free_paged_attention (runtime/
// pic_attention.py:22-232): keys are stored *before* RoPE in physical pages
// [pages, NKV, BLOCK, D] (V in the same layout), a block table maps the
// logical sequence to pages (a page id may repeat: that is the sharing
// primitive), and every key is rotated at its logical position while the
// attention runs.  Per the reference:
//   q      [B, NQ, TQ, D]  already rotated, element type T (bf16, fp16, fp32)
//   key k  rotated with cos/sin tables [max_pos, D/2] (fp32 or T; NeoX
//          rotate-half) in fp32 and rounded to T before the dot product
//          (:81-90)
//   mask   a key attends iff k_positions[k] <= q_positions[tq]     (:57-58)
//   out    softmax(q.k * scale) . v, zeros when no key is visible   (:117-128)
// Like the Metal kernel, any number of queries and any GQA group is served.
//
// Two attention kernels leave split partials (m, l, o) that pf_reduce_kernel
// merges:
//   pf_attention_kernel  bf16 pages, D in {64, 128}: MFMA.  Segments are
//                        (batch row, kv head); 16 (head, query) columns of a
//                        segment form the N dimension of one MFMA tile, so each
//                        key byte is read once for all of them.
//   pf_generic_kernel    every other element type and head dim (fp32 and fp16
//                        pages, D any multiple of 32 up to 256): fp32 VALU
//                        over LDS-staged 32-key blocks, no rounding of P.
// A segment with more columns than one pass holds (16 for the MFMA kernel,
// 4096 / D for the generic one) runs as several column passes.  The passes of
// one piece of work are launched next to each other on the same XCD, so the
// second pass reads the pages from that XCD's L2.
//
// MFMA kernel, per 32-key block a wavefront:
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

#include <limits.h>

namespace voom {
namespace {

constexpr int kKeys = 32;  // keys per block
constexpr int kCols = 16;  // MFMA N: (head, query) columns of one pass
constexpr float kLog2e = 1.4426950408889634f;

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

// ---- element types (the VOOM_DTYPE_* codes) --------------------------------
struct EBf16 {
  typedef uint16_t raw;
  __device__ static float load(const raw* p) { return bf2f(*p); }
  __device__ static float round(float x) { return bf2f(f2bf(x)); }
  __device__ static void store4(raw* p, f32x4 v) {
    *reinterpret_cast<uint2*>(p) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
  }
};
struct EF16 {
  typedef uint16_t raw;
  __device__ static float h2f(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
  }
  __device__ static uint16_t f2h(float x) {  // round to nearest even
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
  }
  __device__ static float load(const raw* p) { return h2f(*p); }
  __device__ static float round(float x) { return h2f(f2h(x)); }
  __device__ static void store4(raw* p, f32x4 v) {
    const uint32_t w0 = f2h(v[0]) | (static_cast<uint32_t>(f2h(v[1])) << 16);
    const uint32_t w1 = f2h(v[2]) | (static_cast<uint32_t>(f2h(v[3])) << 16);
    *reinterpret_cast<uint2*>(p) = make_uint2(w0, w1);
  }
};
struct EF32 {
  typedef float raw;
  __device__ static float load(const raw* p) { return *p; }
  __device__ static float round(float x) { return x; }
  __device__ static void store4(raw* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }
};

// Four consecutive table entries as loaded (raw) and as fp32 (cvt): the MFMA
// kernel keeps the raw chunk in registers while it is in flight and converts
// it when it is stored to LDS.
template <typename TT> struct TabChunk;
template <> struct TabChunk<EF32> {
  typedef f32x4 raw;
  __device__ static raw load(const void* base, size_t off) {
    return *reinterpret_cast<const f32x4*>(static_cast<const float*>(base) + off);
  }
  __device__ static f32x4 cvt(raw r) { return r; }
};
template <> struct TabChunk<EBf16> {
  typedef u32x2 raw;
  __device__ static raw load(const void* base, size_t off) {
    return *reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(base) + off);
  }
  __device__ static f32x4 cvt(raw r) {
    return f32x4{__builtin_bit_cast(float, r[0] << 16),
                 __builtin_bit_cast(float, r[0] & 0xffff0000u),
                 __builtin_bit_cast(float, r[1] << 16),
                 __builtin_bit_cast(float, r[1] & 0xffff0000u)};
  }
};

struct PfArgs {
  const void* q;             // [B, NQ, TQ, D]
  const void* k_pages;       // [P, NKV, BLOCK, D]
  const void* v_pages;       // [P, NKV, BLOCK, D]
  const int32_t* table;      // [ceil(TK / BLOCK)]
  const int32_t* k_pos;      // [TK]
  const int32_t* q_pos;      // [TQ]
  const void* cos_t;         // [max_pos, D/2]
  const void* sin_t;         // [max_pos, D/2]
  float* part_o;             // [B * NKV * splits, NCP, D]
  float* part_ml;            // [B * NKV * splits, NCP, 2]
  int B, NQ, TQ, NKV, G, D, BLOCK, P, TK, max_pos, splits;
  int NC;      // columns of a segment: G * TQ
  int ncg;     // columns per pass
  int passes;  // ceil(NC / ncg)
  int NCP;     // passes * ncg: partial rows per (segment, split)
  int nwork;   // workgroups of one pass
  float scale, scale_log2e;
};

// Work item and column pass of this workgroup.  With several passes, the
// passes of one work item get consecutive groups of eight workgroup ids at
// the same position in the group, i.e. the same XCD at about the same time
// (workgroups go to the XCDs round-robin), so every pass after the first
// reads the pages from that XCD's L2.  Ids past the last work item return
// false (a whole workgroup, before any barrier).
__device__ __forceinline__ bool pf_work(const PfArgs& a, int& w, int& pass) {
  const int bid = static_cast<int>(blockIdx.x);
  if (a.passes == 1) {
    w = bid;
    pass = 0;
    return true;
  }
  const int r = bid >> 3;
  pass = r % a.passes;
  w = (r / a.passes) * 8 + (bid & 7);
  return w < a.nwork;
}

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

// One workgroup per (batch row, split, group of HW kv heads, column pass);
// wavefront w takes kv head HW * group + w.  All HW wavefronts walk the same
// key blocks, so a block's cos/sin rows are loaded once per workgroup into a
// shared LDS tile (double-buffered, one barrier per block) while every
// wavefront keeps its own K rows in registers and stages its own V rows in a
// private LDS slice.  Block i + 1's K and V rows, and its cos/sin rows, are in
// flight while block i is computed; table entries are fetched two blocks
// ahead.  Partials are indexed (segment * splits + split, pass * 16 + column).
// (With 2 or 1 wavefronts per workgroup each thread stages 4-8x the cos/sin
// chunks of the 8-wavefront shape; those variants get the whole register file.)
template <int D, int HW, typename TT>
__global__ __launch_bounds__(HW * kWave) __attribute__((amdgpu_waves_per_eu(HW >= 4 ? 2 : 1)))
void pf_attention_kernel(PfArgs a) {
  constexpr int KS = D / 32;     // k-steps of the score MFMA
  constexpr int HS = D / 64;     // k-steps in one rotary half
  constexpr int DT = D / 16;     // dim tiles of out^T
  constexpr int kVRow = D + 8;   // LDS row stride of the staged V rows (elements)
  constexpr int kVLoads = kKeys * D / 8 / kWave;  // 16-byte V chunks per lane
  constexpr int CPR = D / 8;     // 4-entry chunks in one cos (or sin) row of D/2 entries
  constexpr int kCsPerThread = kKeys * 2 * CPR / (HW * kWave);
  static_assert(kCsPerThread * HW * kWave == kKeys * 2 * CPR, "cos/sin tile split");
  typedef TabChunk<TT> TC;
  __shared__ __attribute__((aligned(16))) uint16_t v_stage[HW][kKeys * kVRow];
  // [buffer][key][cos, sin][chunk]: chunk c of key r sits at c ^ (r % CPR), so
  // the 16 lanes that read one chunk of 16 different keys hit distinct banks
  __shared__ f32x4 cs_stage[2][kKeys][2][CPR];

  int w, pass;
  if (!pf_work(a, w, pass)) return;
  const uint16_t* q16 = static_cast<const uint16_t*>(a.q);
  const uint16_t* kpg = static_cast<const uint16_t*>(a.k_pages);
  const uint16_t* vpg = static_cast<const uint16_t*>(a.v_pages);
  const int lane = threadIdx.x & (kWave - 1);
  const int wl = uniform(threadIdx.x / kWave);
  const int groups = a.NKV / HW;
  const int kg = w % groups;
  const int rest = w / groups;
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
  const int col = pass * kCols + i16;  // (head, query) column of the segment
  const bool col_ok = col < a.NC;
  const int cj = col_ok ? col / a.TQ : 0;      // head within the group
  const int ctq = col_ok ? col - cj * a.TQ : 0;  // query
  const int qpos = a.q_pos[ctq];
  const int klane = lane & 31;  // the key this lane looks up (lanes 32..63 mirror)
  uint16_t* vs = v_stage[wl];

  // Q^T operand: lane (column i16, group g) holds q[head][tq][32s + 8g .. +8]
  u32x4 qop[KS];
  {
    const uint16_t* qh =
        q16 + ((static_cast<size_t>(b) * a.NQ + kvh * a.G + cj) * a.TQ + ctq) * D;
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
      const uint16_t* krow = kpg + pf_row_of(rlo, rhi, 16 * t + i16) * D;
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
      const int cc = c - r * (D / 8);
      vv[u] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4*>(vpg + pf_row_of(rlo, rhi, r) * D + 8 * cc));
    }
  };
  // V rows, coalesced 16-byte chunks, into this wave's LDS slice
  auto store_v = [&](const u32x4 (&vv)[kVLoads]) {
#pragma unroll
    for (int u = 0; u < kVLoads; ++u) {
      const int c = u * kWave + lane;
      const int r = c / (D / 8);
      const int cc = c - r * (D / 8);
      *reinterpret_cast<u32x4*>(vs + r * kVRow + 8 * cc) = vv[u];
    }
  };
  // this thread's share of a block's cos/sin rows: chunk id -> (key, table, chunk)
  auto load_cs = [&](int kp, typename TC::raw (&cr)[kCsPerThread]) {
#pragma unroll
    for (int i = 0; i < kCsPerThread; ++i) {
      const int cid = static_cast<int>(threadIdx.x) + i * HW * kWave;
      const int key = cid / (2 * CPR);
      const int tab = (cid / CPR) & 1;
      const int ch = cid & (CPR - 1);
      const int p = __shfl(kp, key);
      cr[i] = TC::load(tab ? a.sin_t : a.cos_t, static_cast<size_t>(p) * (D / 2) + 4 * ch);
    }
  };
  auto store_cs = [&](int buf, const typename TC::raw (&cr)[kCsPerThread]) {
#pragma unroll
    for (int i = 0; i < kCsPerThread; ++i) {
      const int cid = static_cast<int>(threadIdx.x) + i * HW * kWave;
      const int key = cid / (2 * CPR);
      const int tab = (cid / CPR) & 1;
      const int ch = cid & (CPR - 1);
      cs_stage[buf][key][tab][ch ^ (key & (CPR - 1))] = TC::cvt(cr[i]);
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
    typename TC::raw c0[kCsPerThread];
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
    typename TC::raw cn[kCsPerThread];
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
        for (int wv = 0; wv < 4; ++wv) {
          const uint32_t xa = kc[t][s][wv];
          const uint32_t xb = kc[t][s + HS][wv];
          float ra[2], rb[2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const float av = __builtin_bit_cast(float, h ? (xa & 0xffff0000u) : (xa << 16));
            const float bv = __builtin_bit_cast(float, h ? (xb & 0xffff0000u) : (xb << 16));
            const int e = 2 * wv + h;
            const float c = e < 4 ? cA[e] : cB[e - 4];
            const float sv = e < 4 ? sA[e] : sB[e - 4];
            ra[h] = av * c - bv * sv;
            rb[h] = bv * c + av * sv;
          }
          lo_out[wv] = pack_bf16x2(ra[0], ra[1]);
          hi_out[wv] = pack_bf16x2(rb[0], rb[1]);
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
    const size_t row = pidx * a.NCP + col;
    float* po = a.part_o + row * D + 4 * g;
#pragma unroll
    for (int d = 0; d < DT; ++d) *reinterpret_cast<f32x4*>(po + 16 * d) = acc[d];
    if (g == 0) {
      a.part_ml[row * 2 + 0] = m_run;
      a.part_ml[row * 2 + 1] = l_tot;
    }
  }
}

// ---- generic kernel ---------------------------------------------------------
constexpr int kGenThreads = 256;
constexpr int kGenAcc = 16;                     // output values per thread
constexpr int kGenOut = kGenThreads * kGenAcc;  // columns * D of one pass
constexpr int kGenMaxD = 256;

// LDS of the generic kernel, in 4-byte words, for head dim D and ncg columns.
struct GenLds {
  int kr, vr, qs, ss, mcol, lcol, acol, qp, kpv, kpt, krow;  // word offsets
  int words;
};
__host__ __device__ inline GenLds gen_lds(int D, int ncg) {
  GenLds s;
  s.kr = 0;                              // [32][D + 4] rotated keys, rounded to T
  s.vr = s.kr + kKeys * (D + 4);         // [32][D]
  s.qs = s.vr + kKeys * D;               // [ncg][D] q * scale
  s.ss = s.qs + ncg * D;                 // [ncg][32] scores (log2 units), then P
  s.mcol = s.ss + ncg * kKeys;           // [ncg] running maximum
  s.lcol = s.mcol + ncg;                 // [ncg] running sum
  s.acol = s.lcol + ncg;                 // [ncg] this block's rescale
  s.qp = s.acol + ncg;                   // [ncg] query position (INT_MIN: no column)
  s.kpv = s.qp + ncg;                    // [32] key position for the mask
  s.kpt = s.kpv + kKeys;                 // [32] key position clamped into the tables
  s.krow = (s.kpt + kKeys + 1) & ~1;     // [32] int64 page rows
  s.words = s.krow + 2 * kKeys;
  return s;
}

// One workgroup of 256 threads per (batch row, kv head, split, column pass).
// Per 32-key block: thread t < 32 resolves key t's page row and position; the
// keys are rotated in fp32, rounded to T and staged in LDS with the V rows
// (one pair of rotary dims per thread step, coalesced over dims); every score
// is an fp32 dot product over LDS (thread = (key, column)); each half-wave
// runs one column's online-softmax step; then thread t owns output values
// t + 256 i (i < 16) of the pass's [columns][D] block and adds P . V over the
// 32 keys.  P stays fp32, as in the reference kernel.
template <typename E, typename TT>
__global__ __launch_bounds__(kGenThreads) void pf_generic_kernel(PfArgs a) {
  extern __shared__ __attribute__((aligned(16))) float gsm[];
  int w, pass;
  if (!pf_work(a, w, pass)) return;
  typedef typename E::raw R;
  typedef typename TT::raw TR;
  const int D = a.D;
  const int H = D / 2;
  const int KR = D + 4;
  const int ncg = a.ncg;
  const GenLds L = gen_lds(D, ncg);
  float* kr = gsm + L.kr;
  float* vr = gsm + L.vr;
  float* qs = gsm + L.qs;
  float* ss = gsm + L.ss;
  float* mcol = gsm + L.mcol;
  float* lcol = gsm + L.lcol;
  float* acol = gsm + L.acol;
  int* qp = reinterpret_cast<int*>(gsm + L.qp);
  int* kpv = reinterpret_cast<int*>(gsm + L.kpv);
  int* kpt = reinterpret_cast<int*>(gsm + L.kpt);
  long long* krow = reinterpret_cast<long long*>(gsm + L.krow);

  const R* qg = static_cast<const R*>(a.q);
  const R* kpg = static_cast<const R*>(a.k_pages);
  const R* vpg = static_cast<const R*>(a.v_pages);
  const TR* cos_t = static_cast<const TR*>(a.cos_t);
  const TR* sin_t = static_cast<const TR*>(a.sin_t);
  const int t = threadIdx.x;
  const int kvh = w % a.NKV;
  const int rest = w / a.NKV;
  const int split = rest % a.splits;
  const int b = rest / a.splits;
  const size_t pidx = static_cast<size_t>(b * a.NKV + kvh) * a.splits + split;
  const int nb = (a.TK + kKeys - 1) / kKeys;
  const int blo = static_cast<int>(static_cast<long long>(split) * nb / a.splits);
  const int bhi = static_cast<int>(static_cast<long long>(split + 1) * nb / a.splits);
  const int n0 = pass * ncg;
  const int ncols = min(ncg, a.NC - n0);

  for (int e = t; e < ncg * D; e += kGenThreads) {
    const int c = e / D;
    const int d = e - c * D;
    float v = 0.f;
    if (c < ncols) {
      const int n = n0 + c;
      const int j = n / a.TQ;
      const int tq = n - j * a.TQ;
      v = E::load(qg + ((static_cast<size_t>(b) * a.NQ + kvh * a.G + j) * a.TQ + tq) * D + d) *
          a.scale;
    }
    qs[e] = v;
  }
  for (int c = t; c < ncg; c += kGenThreads) {
    mcol[c] = -INFINITY;
    lcol[c] = 0.f;
    qp[c] = c < ncols ? a.q_pos[(n0 + c) % a.TQ] : INT_MIN;
  }
  float acc[kGenAcc];
#pragma unroll
  for (int i = 0; i < kGenAcc; ++i) acc[i] = 0.f;

  for (int bi = blo; bi < bhi; ++bi) {
    __syncthreads();  // the previous block's LDS reads are done
    if (t < kKeys) {
      const int key = bi * kKeys + t;
      long long row = 0;
      int pv = INT_MAX, pt = 0;
      if (key < a.TK) {
        const int blk = key / a.BLOCK;
        int page = a.table[blk];
        page = static_cast<unsigned>(page) < static_cast<unsigned>(a.P) ? page : 0;
        row = (static_cast<long long>(page) * a.NKV + kvh) * a.BLOCK + (key - blk * a.BLOCK);
        pv = a.k_pos[key];
        pt = pv < 0 ? 0 : (pv >= a.max_pos ? a.max_pos - 1 : pv);
      }
      krow[t] = row;
      kpv[t] = pv;
      kpt[t] = pt;
    }
    __syncthreads();
    for (int p = t; p < kKeys * H; p += kGenThreads) {
      const int key = p / H;
      const int d = p - key * H;
      const R* kk = kpg + krow[key] * D;
      const float x = E::load(kk + d);
      const float y = E::load(kk + d + H);
      const size_t to = static_cast<size_t>(kpt[key]) * H + d;
      const float c = TT::load(cos_t + to);
      const float s = TT::load(sin_t + to);
      kr[key * KR + d] = E::round(x * c - y * s);
      kr[key * KR + d + H] = E::round(y * c + x * s);
    }
    for (int e = t; e < kKeys * D; e += kGenThreads) {
      const int key = e / D;
      vr[e] = E::load(vpg + krow[key] * D + (e - key * D));
    }
    __syncthreads();
    {
      const int sk = t & (kKeys - 1);
      const f32x4* kq = reinterpret_cast<const f32x4*>(kr + sk * KR);
      const bool key_ok = bi * kKeys + sk < a.TK;
      for (int c = t / kKeys; c < ncg; c += kGenThreads / kKeys) {
        const f32x4* qq = reinterpret_cast<const f32x4*>(qs + c * D);
        float s = 0.f;
        for (int d4 = 0; d4 < D / 4; ++d4) {
          const f32x4 x = kq[d4];
          const f32x4 y = qq[d4];
          s = fmaf(x[0], y[0], s);
          s = fmaf(x[1], y[1], s);
          s = fmaf(x[2], y[2], s);
          s = fmaf(x[3], y[3], s);
        }
        ss[c * kKeys + sk] = key_ok && kpv[sk] <= qp[c] ? s * kLog2e : -INFINITY;
      }
    }
    __syncthreads();
    {
      const int l32 = t & (kKeys - 1);
      for (int c = t / kKeys; c < ncg; c += kGenThreads / kKeys) {
        const float x = ss[c * kKeys + l32];
        float mx = x;
#pragma unroll
        for (int o = kKeys / 2; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kKeys));
        const float mo = mcol[c];
        const float mn = fmaxf(mo, mx);
        const float p = x == -INFINITY ? 0.f : fast_exp2(x - mn);
        ss[c * kKeys + l32] = p;
        float sum = p;
#pragma unroll
        for (int o = kKeys / 2; o > 0; o >>= 1) sum += __shfl_xor(sum, o, kKeys);
        if (l32 == 0) {
          const float al = mn == mo ? 1.f : fast_exp2(mo - mn);
          acol[c] = al;
          lcol[c] = lcol[c] * al + sum;
          mcol[c] = mn;
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kGenAcc; ++i) {
      const int e = t + kGenThreads * i;
      if (e < ncg * D) {
        const int c = e / D;
        const int d = e - c * D;
        const f32x4* pc = reinterpret_cast<const f32x4*>(ss + c * kKeys);
        float s = acc[i] * acol[c];
#pragma unroll
        for (int k4 = 0; k4 < kKeys / 4; ++k4) {
          const f32x4 pp = pc[k4];
          s = fmaf(pp[0], vr[(4 * k4 + 0) * D + d], s);
          s = fmaf(pp[1], vr[(4 * k4 + 1) * D + d], s);
          s = fmaf(pp[2], vr[(4 * k4 + 2) * D + d], s);
          s = fmaf(pp[3], vr[(4 * k4 + 3) * D + d], s);
        }
        acc[i] = s;
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kGenAcc; ++i) {
    const int e = t + kGenThreads * i;
    if (e < ncols * D) {
      const int c = e / D;
      a.part_o[(pidx * a.NCP + n0 + c) * D + (e - c * D)] = acc[i];
    }
  }
  for (int c = t; c < ncols; c += kGenThreads) {
    a.part_ml[(pidx * a.NCP + n0 + c) * 2 + 0] = mcol[c];
    a.part_ml[(pidx * a.NCP + n0 + c) * 2 + 1] = lcol[c];
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

template <typename E>
__global__ __launch_bounds__(kRedWaves * kWave) void pf_reduce_kernel(PfArgs a,
                                                                      typename E::raw* out) {
  __shared__ float st_ml[kRedWaves][2];
  __shared__ __attribute__((aligned(16))) f32x4 st_o[kRedWaves][kRedCols];
  const int D = a.D;
  const int slices = D / kRedDims;
  const int lane = threadIdx.x & (kWave - 1);
  const int wl = uniform(threadIdx.x / kWave);
  const int slice = blockIdx.x % slices;
  const int task = blockIdx.x / slices;
  const int seg = task / a.NC;
  const int n = task - seg * a.NC;
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
      const size_t p = (first + (i < cnt ? i : cnt - 1)) * a.NCP + n;
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
  E::store4(out + ((static_cast<size_t>(b) * a.NQ + kvh * a.G + hj) * a.TQ + tq) * D + dim0,
            res * inv);
}

template <int D, typename TT>
void launch_pf_attention(int hw, dim3 grid, dim3 block, hipStream_t stream, const PfArgs& a) {
  switch (hw) {
    case 8: hipLaunchKernelGGL((pf_attention_kernel<D, 8, TT>), grid, block, 0, stream, a); break;
    case 4: hipLaunchKernelGGL((pf_attention_kernel<D, 4, TT>), grid, block, 0, stream, a); break;
    case 2: hipLaunchKernelGGL((pf_attention_kernel<D, 2, TT>), grid, block, 0, stream, a); break;
    default: hipLaunchKernelGGL((pf_attention_kernel<D, 1, TT>), grid, block, 0, stream, a); break;
  }
}

// How one call is cut: which kernel, columns per pass, passes, splits and the
// workspace it needs.  voom_position_free_workspace_bytes and the call share
// it, so the two always agree.
struct PfPlan {
  bool mfma;
  int hw;      // kv heads per workgroup (MFMA kernel)
  int ncg, passes, ncp, splits;
  size_t o_bytes, ws_bytes;
};

PfPlan pf_plan(int B, int NQ, int TQ, int NKV, int D, int TK, int dtype, int num_splits) {
  PfPlan p;
  const int NC = NQ / NKV * TQ;
  p.mfma = dtype == VOOM_DTYPE_BF16 && (D == 64 || D == 128);
  p.hw = NKV % 8 == 0 ? 8 : NKV % 4 == 0 ? 4 : NKV % 2 == 0 ? 2 : 1;
  p.ncg = p.mfma ? kCols : (NC < kGenOut / D ? NC : kGenOut / D);
  p.passes = (NC + p.ncg - 1) / p.ncg;
  p.ncp = p.passes * p.ncg;
  const int nb = (TK + kKeys - 1) / kKeys;
  // default: 8 wavefronts per CU for the MFMA kernel, 2 workgroups of 4
  // wavefronts per CU for the generic one
  const long long target = p.mfma ? 8LL * device_cu_count() : 2LL * device_cu_count();
  const long long per = static_cast<long long>(B) * NKV * p.passes;
  long long s = num_splits > 0 ? num_splits : (target + per - 1) / per;
  if (s > nb) s = nb;
  p.splits = s < 1 ? 1 : static_cast<int>(s);
  const size_t rows = static_cast<size_t>(B) * NKV * p.splits * p.ncp;
  p.o_bytes = (rows * D * sizeof(float) + 255) & ~size_t(255);
  p.ws_bytes = p.o_bytes + rows * 2 * sizeof(float);
  return p;
}

bool pf_dtype_ok(int dt) {
  return dt == VOOM_DTYPE_BF16 || dt == VOOM_DTYPE_F16 || dt == VOOM_DTYPE_F32;
}

// Launches the generic kernel with `lds` bytes of dynamic LDS (up to 85 KB at
// head_dim 256), raising the kernel's dynamic-LDS limit first when the
// request is above the 64 KB default.
template <typename E, typename TT>
int launch_pf_generic_tt(dim3 grid, size_t lds, hipStream_t stream, const PfArgs& a) {
  if (lds > 65536) {
    const int rc = check_hip(
        hipFuncSetAttribute(reinterpret_cast<const void*>(&pf_generic_kernel<E, TT>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)),
        "position_free_attention: dynamic LDS limit");
    if (rc) return rc;
  }
  hipLaunchKernelGGL((pf_generic_kernel<E, TT>), grid, dim3(kGenThreads), lds, stream, a);
  return VOOM_LAUNCH_CHECK("position_free_attention: kernel launch");
}

template <typename E>
int launch_pf_generic(int table_dtype, dim3 grid, size_t lds, hipStream_t stream,
                      const PfArgs& a) {
  return table_dtype == VOOM_DTYPE_F32 ? launch_pf_generic_tt<E, EF32>(grid, lds, stream, a)
                                       : launch_pf_generic_tt<E, E>(grid, lds, stream, a);
}

}  // namespace
}  // namespace voom

using namespace voom;

extern "C" size_t voom_position_free_workspace_bytes(int batch, int num_q_heads, int num_queries,
                                                     int num_kv_heads, int head_dim,
                                                     int num_keys, int dtype, int num_splits) {
  if (batch <= 0 || num_q_heads <= 0 || num_queries <= 0 || num_kv_heads <= 0 ||
      num_q_heads % num_kv_heads || head_dim <= 0 || head_dim % 32 || head_dim > kGenMaxD ||
      num_keys < 0 || !pf_dtype_ok(dtype))
    return 0;
  return pf_plan(batch, num_q_heads, num_queries, num_kv_heads, head_dim, num_keys, dtype,
                 num_splits)
      .ws_bytes;
}

extern "C" int voom_position_free_attention(
    const void* q, const void* k_pages, const void* v_pages, const int32_t* block_table,
    const int32_t* key_positions, const int32_t* query_positions, const void* cos_table,
    const void* sin_table, void* out, void* workspace, size_t ws_bytes, int batch,
    int num_q_heads, int num_queries, int num_kv_heads, int head_dim, int block_size,
    int num_pages, int num_keys, int max_position, int dtype, int table_dtype, float scale,
    int num_splits, hipStream_t stream) {
  const char* who = "position_free_attention";
  VOOM_REQUIRE(q && k_pages && v_pages && out && workspace && query_positions && cos_table &&
                   sin_table,
               "%s: null pointer argument", who);
  VOOM_REQUIRE(num_keys == 0 || (block_table && key_positions), "%s: null key arrays", who);
  VOOM_REQUIRE(batch > 0 && num_queries > 0 && num_kv_heads > 0 && num_q_heads > 0 &&
                   num_q_heads % num_kv_heads == 0,
               "%s: unsupported head or position geometry", who);
  VOOM_REQUIRE(head_dim > 0 && head_dim % 32 == 0 && head_dim <= kGenMaxD,
               "%s: head_dim %d unsupported (a multiple of 32 up to %d)", who, head_dim,
               kGenMaxD);
  VOOM_REQUIRE(pf_dtype_ok(dtype), "%s: unsupported element type code %d", who, dtype);
  VOOM_REQUIRE(table_dtype == VOOM_DTYPE_F32 || table_dtype == dtype,
               "%s: RoPE cache must be FP32 or match the Q/K/V dtype", who);
  VOOM_REQUIRE(block_size > 0 && num_pages > 0 && num_keys >= 0 && num_keys <= (1 << 30) &&
                   max_position > 0,
               "%s: bad page or position geometry", who);
  const PfPlan p = pf_plan(batch, num_q_heads, num_queries, num_kv_heads, head_dim, num_keys,
                           dtype, num_splits);
  VOOM_REQUIRE(ws_bytes >= p.ws_bytes, "%s: workspace %zu bytes < required %zu", who, ws_bytes,
               p.ws_bytes);
  VOOM_REQUIRE(reinterpret_cast<uintptr_t>(q) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(k_pages) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(v_pages) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(cos_table) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(sin_table) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(workspace) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(out) % 16 == 0,
               "%s: tensors must be 16-byte aligned", who);
  const int G = num_q_heads / num_kv_heads;
  const long long NC = static_cast<long long>(G) * num_queries;
  const long long segs = static_cast<long long>(batch) * num_kv_heads;
  const long long nwork = segs * p.splits / (p.mfma ? p.hw : 1);
  const long long grid_x = p.passes == 1 ? nwork : (nwork + 7) / 8 * 8 * p.passes;
  VOOM_REQUIRE(NC < (1LL << 24) && grid_x < (1LL << 30) && segs * NC * (head_dim / 32) < (1LL << 31),
               "%s: grid too large", who);

  PfArgs a;
  a.q = q;
  a.k_pages = k_pages;
  a.v_pages = v_pages;
  a.table = block_table;
  a.k_pos = key_positions;
  a.q_pos = query_positions;
  a.cos_t = cos_table;
  a.sin_t = sin_table;
  a.part_o = static_cast<float*>(workspace);
  a.part_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) + p.o_bytes);
  a.B = batch;
  a.NQ = num_q_heads;
  a.TQ = num_queries;
  a.NKV = num_kv_heads;
  a.G = G;
  a.D = head_dim;
  a.BLOCK = block_size;
  a.P = num_pages;
  a.TK = num_keys;
  a.max_pos = max_position;
  a.splits = p.splits;
  a.NC = static_cast<int>(NC);
  a.ncg = p.ncg;
  a.passes = p.passes;
  a.NCP = p.ncp;
  a.nwork = static_cast<int>(nwork);
  a.scale = scale;
  a.scale_log2e = scale * kLog2e;
  const dim3 grid(static_cast<unsigned>(grid_x));
  int rc;
  if (p.mfma) {
    const dim3 block(static_cast<unsigned>(p.hw * kWave));
    const bool f32_tab = table_dtype == VOOM_DTYPE_F32;
    if (head_dim == 128) {
      if (f32_tab) launch_pf_attention<128, EF32>(p.hw, grid, block, stream, a);
      else launch_pf_attention<128, EBf16>(p.hw, grid, block, stream, a);
    } else {
      if (f32_tab) launch_pf_attention<64, EF32>(p.hw, grid, block, stream, a);
      else launch_pf_attention<64, EBf16>(p.hw, grid, block, stream, a);
    }
    rc = VOOM_LAUNCH_CHECK("position_free_attention: kernel launch");
  } else {
    const size_t lds = static_cast<size_t>(gen_lds(head_dim, p.ncg).words) * 4;
    if (dtype == VOOM_DTYPE_F32) rc = launch_pf_generic<EF32>(table_dtype, grid, lds, stream, a);
    else if (dtype == VOOM_DTYPE_F16) rc = launch_pf_generic<EF16>(table_dtype, grid, lds, stream, a);
    else rc = launch_pf_generic<EBf16>(table_dtype, grid, lds, stream, a);
  }
  if (rc) return rc;
  const dim3 grid_red(static_cast<unsigned>(segs * NC * (head_dim / kRedDims)));
  const dim3 block_red(kRedWaves * kWave);
  if (dtype == VOOM_DTYPE_F32) {
    hipLaunchKernelGGL(pf_reduce_kernel<EF32>, grid_red, block_red, 0, stream, a,
                       static_cast<float*>(out));
  } else if (dtype == VOOM_DTYPE_F16) {
    hipLaunchKernelGGL(pf_reduce_kernel<EF16>, grid_red, block_red, 0, stream, a,
                       static_cast<uint16_t*>(out));
  } else {
    hipLaunchKernelGGL(pf_reduce_kernel<EBf16>, grid_red, block_red, 0, stream, a,
                       static_cast<uint16_t*>(out));
  }
  return VOOM_LAUNCH_CHECK("position_free_attention: reduce launch");
}
