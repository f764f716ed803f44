// DeepSeek Sparse Attention selection for gfx950: the lightning indexer's
// scores over the cached index keys and the top-k of each row, as the
// reference computes them for a decode step (runtime/glm_dsa.py:113-166):
//
//   score[s] = sum_j w[j] * relu(scale * (q_idx[j] . k_idx[s]))     fp32
//   keep the k highest scores of keys s < n (causal), indices ascending
//
// w already carries the reference's n_heads^-0.5 and scale is
// head_dim^-0.5 (:147-150).  The top-k set matches argpartition + sort
// (:156-160); among keys whose scores tie at the k-th value the lowest
// indices are kept, where argpartition leaves the choice open.
//
// Scores (HBM-bound: 256 B of index key per key for 32 heads x 128 dims,
// ~32 flop per byte):  scores^T tiles [16 heads x 16 keys] =
// Q [heads x 128] . K^T with v_mfma_f32_16x16x32_bf16 -- the bf16 products
// are exact in fp32, as in the reference's fp32 einsum over bf16 values; lane
// (key i16, group g) then holds heads 4g + r of its key, so relu, the head
// weights and the head sum stay in registers plus two cross-group adds.
//
// Top-k: one workgroup of 1024 threads per row.  Scores map to order-
// preserving 32-bit keys; three radix passes (11, 11 and 10 bits) with LDS
// histograms find the k-th largest key T and how many keys equal to T to
// keep.  Two ordered passes then write the selection: each wavefront owns a
// contiguous index range, counts its keys above T and equal to T, and after
// an exclusive scan over wavefronts writes its indices in order, so the
// output is sorted without a sort.
#include "common.h"

namespace voom {
namespace {

constexpr int kDsaDim = 128;           // index head dim
constexpr int kDsaSteps = kDsaDim / 32;  // k-steps of the score MFMA
constexpr int kScoreThreads = 256;
constexpr int kScoreWaves = kScoreThreads / kWave;
constexpr int kKeysPerIter = 64;       // 4 key tiles per wave-iteration
constexpr int kItersPerWave = 2;
constexpr int kKeysPerWave = kKeysPerIter * kItersPerWave;
constexpr int kKeysPerGroup = kKeysPerWave * kScoreWaves;  // 512 keys per workgroup

struct DsaScoreArgs {
  const uint16_t* q;     // [B, NH, 128] bf16
  const float* w;        // [B, NH] fp32
  const uint16_t* k;     // [B, cap, 128] bf16
  const int32_t* lens;   // [B]
  float* scores;         // [B, cap]
  int B, NH, cap;
  float scale;
};

template <int NHT>  // 16-head tiles
__global__ __launch_bounds__(kScoreThreads) void dsa_scores_kernel(DsaScoreArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wl = uniform(threadIdx.x / kWave);
  const int b = blockIdx.y;
  int n = a.lens[b];
  n = uniform(n < 0 ? 0 : (n > a.cap ? a.cap : n));
  const int key0 = blockIdx.x * kKeysPerGroup + wl * kKeysPerWave;
  if (key0 >= n) return;
  const int i16 = lane & 15;
  const int g = lane >> 4;

  // A operand (index queries): lane (head 16ht + i16, group g) holds
  // q[head][32s + 8g .. +8]; the head weights of the rows this lane's
  // accumulators hold: heads 16ht + 4g + r.
  u32x4 qop[NHT][kDsaSteps];
  float wr[NHT][4];
#pragma unroll
  for (int ht = 0; ht < NHT; ++ht) {
    const uint16_t* qh = a.q + (static_cast<size_t>(b) * a.NH + 16 * ht + i16) * kDsaDim;
#pragma unroll
    for (int s = 0; s < kDsaSteps; ++s) {
      qop[ht][s] = *reinterpret_cast<const u32x4*>(qh + 32 * s + 8 * g);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) wr[ht][r] = a.w[static_cast<size_t>(b) * a.NH + 16 * ht + 4 * g + r];
  }
  const uint16_t* kb = a.k + static_cast<size_t>(b) * a.cap * kDsaDim;
  float* sb = a.scores + static_cast<size_t>(b) * a.cap;

  // B operands (index keys): lane (key i16, group g) holds k[key][32s + 8g ..];
  // both iterations' rows are loaded before the first MFMA.  Keys past n read
  // key n - 1 and are not written.
  u32x4 kop[kItersPerWave][4][kDsaSteps];
#pragma unroll
  for (int it = 0; it < kItersPerWave; ++it) {
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      int key = key0 + it * kKeysPerIter + 16 * tt + i16;
      key = key < n ? key : n - 1;
      const uint16_t* kr = kb + static_cast<size_t>(key) * kDsaDim + 8 * g;
#pragma unroll
      for (int s = 0; s < kDsaSteps; ++s) kop[it][tt][s] = *reinterpret_cast<const u32x4*>(kr + 32 * s);
    }
  }
#pragma unroll
  for (int it = 0; it < kItersPerWave; ++it) {
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      float v = 0.f;
#pragma unroll
      for (int ht = 0; ht < NHT; ++ht) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < kDsaSteps; ++s) {
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, qop[ht][s]),
                                                        __builtin_bit_cast(bf16x8, kop[it][tt][s]),
                                                        acc, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) v += wr[ht][r] * fmaxf(acc[r] * a.scale, 0.f);
      }
      v = wave_sum_across_groups(v);
      const int key = key0 + it * kKeysPerIter + 16 * tt + i16;
      if (g == 0 && key < n) sb[key] = v;
    }
  }
}

// ---------------------------------------------------------------- top-k ----

constexpr int kTopkThreads = 1024;
constexpr int kTopkWaves = kTopkThreads / kWave;

// Order-preserving map of fp32 onto uint32: a > b  <=>  key(a) > key(b), and
// -0 maps like +0 (they compare equal, so they tie).
__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  u = u == 0x80000000u ? 0u : u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Exclusive scan of one int per thread over the workgroup; returns the
// workgroup total in `total`.  `tmp` holds kTopkWaves ints of LDS.
__device__ __forceinline__ int block_exclusive_scan(int x, int* tmp, int& total) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  const int inc = wave_inclusive_scan(x, lane);
  if (lane == kWave - 1) tmp[wv] = inc;
  __syncthreads();
  int before = 0;
  total = 0;
#pragma unroll
  for (int k = 0; k < kTopkWaves; ++k) {
    const int t = tmp[k];
    before += k < wv ? t : 0;
    total += t;
  }
  __syncthreads();
  return before + inc - x;
}

__global__ __launch_bounds__(kTopkThreads) void dsa_topk_kernel(const float* __restrict__ scores,
                                                                const int32_t* __restrict__ lens,
                                                                int32_t* __restrict__ sel,
                                                                int32_t* __restrict__ sel_lens,
                                                                int cap, int K) {
  __shared__ int hist[2048];
  __shared__ int scan_tmp[kTopkWaves];
  __shared__ int found[2];
  __shared__ int wave_gt[kTopkWaves];
  __shared__ int wave_eq[kTopkWaves];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wv = tid / kWave;
  const int b = blockIdx.x;
  int n = lens[b];
  n = n < 0 ? 0 : (n > cap ? cap : n);
  const float* sb = scores + static_cast<size_t>(b) * cap;
  int32_t* ob = sel + static_cast<size_t>(b) * K;
  if (n <= K) {  // every key is selected
    for (int i = tid; i < n; i += kTopkThreads) ob[i] = i;
    if (tid == 0) sel_lens[b] = n;
    return;
  }

  // ---- radix select of the K-th largest key ----
  uint32_t prefix = 0;
  uint32_t pmask = 0;
  int kk = K;  // keys still to take at or below the current prefix
#pragma unroll 1
  for (int p = 0; p < 3; ++p) {
    const int shift = p == 0 ? 21 : (p == 1 ? 10 : 0);
    const int bins = p == 2 ? 1024 : 2048;
    for (int i = tid; i < bins; i += kTopkThreads) hist[i] = 0;
    __syncthreads();
    for (int i = tid; i < n; i += kTopkThreads) {
      const uint32_t u = order_key(sb[i]);
      if ((u & pmask) == prefix) atomicAdd(&hist[(u >> shift) & (bins - 1)], 1);
    }
    __syncthreads();
    // bins in descending order: thread t holds bins - 1 - (E t + e), e < E
    const int E = bins / kTopkThreads;
    int c[2] = {0, 0};
    int mine = 0;
    for (int e = 0; e < E; ++e) {
      c[e] = hist[bins - 1 - (E * tid + e)];
      mine += c[e];
    }
    int total;
    int run = block_exclusive_scan(mine, scan_tmp, total);
    for (int e = 0; e < E; ++e) {
      if (run < kk && run + c[e] >= kk) {
        found[0] = bins - 1 - (E * tid + e);  // the digit
        found[1] = run;                       // keys above it
      }
      run += c[e];
    }
    __syncthreads();
    const int d = found[0];
    kk -= found[1];
    prefix |= static_cast<uint32_t>(d) << shift;
    pmask |= static_cast<uint32_t>(bins - 1) << shift;
    __syncthreads();
  }
  const uint32_t T = prefix;  // keys > T are all kept, kk of the keys == T

  // ---- ordered write: wave wv owns [lo, hi), 64 indices per step ----
  const int per = ((n + kTopkWaves - 1) / kTopkWaves + kWave - 1) / kWave * kWave;
  const int lo = wv * per;
  const int hi = lo + per < n ? lo + per : n;
  int gt = 0;
  int eq = 0;
  for (int i0 = lo; i0 < hi; i0 += kWave) {
    const int i = i0 + lane;
    const uint32_t u = i < hi ? order_key(sb[i]) : 0u;
    gt += __popcll(__ballot(i < hi && u > T));
    eq += __popcll(__ballot(i < hi && u == T));
  }
  if (lane == 0) {
    wave_gt[wv] = gt;
    wave_eq[wv] = eq;
  }
  __syncthreads();
  int gt_before = 0;
  int eq_before = 0;
  for (int k = 0; k < wv; ++k) {
    gt_before += wave_gt[k];
    eq_before += wave_eq[k];
  }
  int out = gt_before + (eq_before < kk ? eq_before : kk);  // selections before this wave
  int eq_seen = eq_before;
  for (int i0 = lo; i0 < hi; i0 += kWave) {
    const int i = i0 + lane;
    const uint32_t u = i < hi ? order_key(sb[i]) : 0u;
    const bool is_gt = i < hi && u > T;
    const bool is_eq = i < hi && u == T;
    const unsigned long long eq_mask = __ballot(is_eq);
    const int eq_rank = eq_seen + __popcll(eq_mask & ((1ull << lane) - 1ull));
    const bool take = is_gt || (is_eq && eq_rank < kk);
    const unsigned long long take_mask = __ballot(take);
    if (take) ob[out + __popcll(take_mask & ((1ull << lane) - 1ull))] = i;
    out += __popcll(take_mask);
    eq_seen += __popcll(eq_mask);
  }
  if (tid == 0) sel_lens[b] = K;
}

}  // namespace
}  // namespace voom

using namespace voom;

extern "C" int voom_dsa_index_scores(const void* q_idx, const float* w_head, const void* k_idx,
                                     const int32_t* lens, float* scores, int batch,
                                     int num_heads, int head_dim, int cap, float scale,
                                     hipStream_t stream) {
  const char* who = "dsa_index_scores";
  VOOM_REQUIRE(q_idx && w_head && k_idx && lens && scores, "%s: null pointer argument", who);
  VOOM_REQUIRE(head_dim == kDsaDim, "%s: index head_dim %d unsupported (128)", who, head_dim);
  VOOM_REQUIRE(num_heads % 16 == 0 && num_heads >= 16 && num_heads <= 64,
               "%s: index heads %d unsupported (16, 32, 48 or 64)", who, num_heads);
  VOOM_REQUIRE(batch > 0 && batch < 65536 && cap > 0, "%s: bad batch or capacity", who);
  VOOM_REQUIRE(reinterpret_cast<uintptr_t>(q_idx) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(k_idx) % 16 == 0,
               "%s: q and k must be 16-byte aligned", who);
  DsaScoreArgs a;
  a.q = static_cast<const uint16_t*>(q_idx);
  a.w = w_head;
  a.k = static_cast<const uint16_t*>(k_idx);
  a.lens = lens;
  a.scores = scores;
  a.B = batch;
  a.NH = num_heads;
  a.cap = cap;
  a.scale = scale;
  const dim3 grid(static_cast<unsigned>((cap + kKeysPerGroup - 1) / kKeysPerGroup),
                  static_cast<unsigned>(batch));
  switch (num_heads / 16) {
    case 1: hipLaunchKernelGGL(dsa_scores_kernel<1>, grid, dim3(kScoreThreads), 0, stream, a); break;
    case 2: hipLaunchKernelGGL(dsa_scores_kernel<2>, grid, dim3(kScoreThreads), 0, stream, a); break;
    case 3: hipLaunchKernelGGL(dsa_scores_kernel<3>, grid, dim3(kScoreThreads), 0, stream, a); break;
    default: hipLaunchKernelGGL(dsa_scores_kernel<4>, grid, dim3(kScoreThreads), 0, stream, a); break;
  }
  return VOOM_LAUNCH_CHECK("dsa_index_scores: kernel launch");
}

extern "C" int voom_dsa_topk(const float* scores, const int32_t* lens, int32_t* sel,
                             int32_t* sel_lens, int batch, int cap, int k, hipStream_t stream) {
  const char* who = "dsa_topk";
  VOOM_REQUIRE(scores && lens && sel && sel_lens, "%s: null pointer argument", who);
  VOOM_REQUIRE(batch > 0 && cap > 0 && k > 0, "%s: bad batch, capacity or k", who);
  hipLaunchKernelGGL(dsa_topk_kernel, dim3(static_cast<unsigned>(batch)), dim3(kTopkThreads), 0,
                     stream, scores, lens, sel, sel_lens, cap, k);
  return VOOM_LAUNCH_CHECK("dsa_topk: kernel launch");
}
