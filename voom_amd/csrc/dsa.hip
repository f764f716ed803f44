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
// Top-k, two launches per call: (1) chunk workgroups (4,096 keys each) each
// place the same threshold T0 at a fixed rank of a strided sample of the row
// and move the keys >= T0, with their indices and in index order, to
// per-chunk slots -- the row is read once, by many CUs; (2) one workgroup
// per row gathers the candidates into LDS (at most 16,384)
// and runs the exact selection there: radix passes of up to 11 bits below the
// leading bits every candidate shares find the k-th largest key T and how
// many keys equal to T to keep, and an ordered write -- each wavefront owns a
// contiguous range, counts its keys above and equal to T, and after an
// exclusive scan over wavefronts writes its indices -- leaves the output
// sorted without a sort.  Scores map to order-preserving 32-bit keys.  When
// the sample misjudges the row (fewer than k or more than 16,384
// candidates), the same exact selection runs over the row in memory.
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
  // every load above issues before the first MFMA (one memory round trip)
  __builtin_amdgcn_sched_barrier(0);
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
constexpr int kRadixBits = 12;                     // digit width of the radix select
constexpr int kRadixBins = 1 << kRadixBits;
constexpr int kBinsPerThread = kRadixBins / kTopkThreads;
static_assert(kBinsPerThread == 4, "one int4 of histogram bins per thread");
constexpr int kChunksPerThread = 2;                // select kernel: up to 2048 chunks

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

constexpr int kCandCap = 16384;  // candidate keys held in LDS
constexpr int kSample = 4096;    // keys sampled to place the threshold
constexpr int kChunkKeys = 4096; // keys per compaction workgroup

// Radix select over `count` keys read by key(i): the rank-th largest key T
// (rank >= 1) and how many keys equal to T belong to the top `rank` (kk).
// The digits start below the leading bits that every key shares: scores of
// one row share their sign and most of their exponent, and a first digit over
// those bits would send every key to a handful of histogram bins, serialising
// the LDS atomics.  The shared bits come from the keys' range [lo, hi], passed
// in when the caller knows it (range_known) or found by a min/max reduction.
// Passes of kRadixBits bits then walk down to bit 0 (or stop after
// max_passes > 0 passes: T is then the lower edge of the crossing bin, a key
// bound with at least `rank` keys at or above it, and kk is meaningless); a
// thread adds runs of equal bins as one atomic.  Three barriers per pass:
// after the histogram; after each thread has taken (and zeroed, for the next
// pass) its int4 of bins and each wavefront has left its scan total; after
// the thread holding the crossing has written it.  (Zeroing the histogram and
// the scan as separate steps cost six barriers a pass, 5.5 k cycles; one
// wavefront scanning every bin hit 32-way LDS bank conflicts.)
// found[] holds the result, scan_tmp kTopkWaves ints; hist must hold
// kRadixBins ints, 16-byte aligned.
template <typename KeyFn>
__device__ void radix_select(KeyFn key, int count, int rank, int* hist, int* scan_tmp, int* found,
                             bool range_known, uint32_t lo_k, uint32_t hi_k, int max_passes,
                             uint32_t& T, int& kk_out) {
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wv = tid / kWave;
  int4* hist4 = reinterpret_cast<int4*>(hist);
  hist4[tid] = make_int4(0, 0, 0, 0);
  if (range_known) {
    __syncthreads();  // bins zero
  } else {
    if (tid == 0) {
      found[0] = static_cast<int>(0xFFFFFFFFu);
      found[1] = 0;
    }
    lo_k = 0xFFFFFFFFu;
    hi_k = 0u;
    for (int i = tid; i < count; i += kTopkThreads) {
      const uint32_t u = key(i);
      lo_k = u < lo_k ? u : lo_k;
      hi_k = u > hi_k ? u : hi_k;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const uint32_t a = static_cast<uint32_t>(__shfl_xor(static_cast<int>(lo_k), o));
      const uint32_t b = static_cast<uint32_t>(__shfl_xor(static_cast<int>(hi_k), o));
      lo_k = a < lo_k ? a : lo_k;
      hi_k = b > hi_k ? b : hi_k;
    }
    __syncthreads();  // found[] and hist initialised
    if (lane == 0) {
      atomicMin(reinterpret_cast<unsigned int*>(&found[0]), lo_k);
      atomicMax(reinterpret_cast<unsigned int*>(&found[1]), hi_k);
    }
    __syncthreads();
    lo_k = static_cast<uint32_t>(found[0]);
    hi_k = static_cast<uint32_t>(found[1]);
  }
  // bits above `top` are common to every key
  int top = 31 - __clz(static_cast<int>(lo_k ^ hi_k));  // -1 when all keys are equal
  uint32_t prefix = top < 31 ? (hi_k & ~((2u << (top < 0 ? 0 : top)) - 1u)) : 0u;
  if (top < 0) prefix = hi_k;
  uint32_t pmask = top < 31 ? ~((2u << (top < 0 ? 0 : top)) - 1u) : 0u;
  if (top < 0) pmask = 0xFFFFFFFFu;
  int kk = rank;
  int passes = 0;
#pragma unroll 1
  while (top >= 0 && (max_passes <= 0 || passes < max_passes)) {
    const int width = top + 1 < kRadixBits ? top + 1 : kRadixBits;
    const int shift = top + 1 - width;
    const int bins = 1 << width;
    int run_bin = -1;
    int run_n = 0;
    for (int i = tid; i < count; i += kTopkThreads) {
      const uint32_t u = key(i);
      if ((u & pmask) == prefix) {
        const int bin = static_cast<int>((u >> shift) & static_cast<uint32_t>(bins - 1));
        if (bin != run_bin) {
          if (run_n) atomicAdd(&hist[run_bin], run_n);
          run_bin = bin;
          run_n = 0;
        }
        ++run_n;
      }
    }
    if (run_n) atomicAdd(&hist[run_bin], run_n);
    __syncthreads();  // histogram complete (found[] of the previous pass read)
    // thread t owns the int4 of bins base .. base + 3, base = kRadixBins - 4 (t + 1),
    // taken in descending order
    const int q4 = kRadixBins / kBinsPerThread - 1 - tid;
    const int4 h = hist4[q4];
    hist4[q4] = make_int4(0, 0, 0, 0);
    const int base = q4 * kBinsPerThread;
    const int c[kBinsPerThread] = {h.w, h.z, h.y, h.x};
    const int mine = h.x + h.y + h.z + h.w;
    const int inc = wave_inclusive_scan(mine, lane);
    if (lane == kWave - 1) scan_tmp[wv] = inc;
    __syncthreads();  // wave totals in scan_tmp, bins zero again
    int run = inc - mine;
#pragma unroll
    for (int k = 0; k < kTopkWaves; ++k) run += k < wv ? scan_tmp[k] : 0;
#pragma unroll
    for (int e = 0; e < kBinsPerThread; ++e) {
      if (run < kk && run + c[e] >= kk) {
        found[0] = base + kBinsPerThread - 1 - e;
        found[1] = run;
      }
      run += c[e];
    }
    __syncthreads();  // result in found[]
    const int d = found[0];
    kk -= found[1];
    prefix |= static_cast<uint32_t>(d) << shift;
    pmask |= static_cast<uint32_t>(bins - 1) << shift;
    top = shift - 1;
    ++passes;
  }
  __syncthreads();  // found[] read by every thread before anyone reuses it
  T = prefix;
  kk_out = kk;
}

// Ordered selection write: keys i < count in index order; every key > T and
// the first kk keys == T go to out[] in that order, as idx(i).  Wavefront w
// owns a contiguous range of i; counts, an exclusive scan over wavefronts,
// then ballots place each index.
template <typename KeyFn, typename IdxFn>
__device__ void ordered_write(KeyFn key, IdxFn idx, int count, uint32_t T, int kk, int* wave_gt,
                              int* wave_eq, int32_t* out) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  const int per = ((count + kTopkWaves - 1) / kTopkWaves + kWave - 1) / kWave * kWave;
  const int lo = wv * per;
  const int hi = lo + per < count ? lo + per : count;
  int gt = 0;
  int eq = 0;
  for (int i0 = lo; i0 < hi; i0 += kWave) {
    const int i = i0 + lane;
    const uint32_t u = i < hi ? key(i) : 0u;
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
  int pos = gt_before + (eq_before < kk ? eq_before : kk);  // selections before this wave
  int eq_seen = eq_before;
  for (int i0 = lo; i0 < hi; i0 += kWave) {
    const int i = i0 + lane;
    const uint32_t u = i < hi ? key(i) : 0u;
    const bool is_gt = i < hi && u > T;
    const bool is_eq = i < hi && u == T;
    const unsigned long long eq_mask = __ballot(is_eq);
    const int eq_rank = eq_seen + __popcll(eq_mask & ((1ull << lane) - 1ull));
    const bool take = is_gt || (is_eq && eq_rank < kk);
    const unsigned long long take_mask = __ballot(take);
    if (take) out[pos + __popcll(take_mask & ((1ull << lane) - 1ull))] = idx(i);
    pos += __popcll(take_mask);
    eq_seen += __popcll(eq_mask);
  }
  __syncthreads();
}

// Workspace of the top-k (per row): the threshold T0, per-chunk candidate
// counts and largest candidate keys, and per-chunk candidate slots of (key,
// index) pairs.
struct TopkWs {
  uint32_t* t0;     // [B]
  int* counts;      // [B, chunks]
  uint32_t* cmax;   // [B, chunks]
  uint2* cand;      // [B, chunks, kChunkKeys]
  int chunks;
};

__host__ __device__ inline int topk_chunks(int cap) { return (cap + kChunkKeys - 1) / kChunkKeys; }

// 1. Threshold and compaction, one launch: one workgroup per chunk of
// kChunkKeys keys of a row.  Each workgroup places the row's threshold T0
// itself -- every one from the same sample with the same exact select, so all
// agree -- while its chunk's keys are in flight, then moves every key >= T0,
// with its index and in index order, to the chunk's slots.  Rows of at most
// kCandCap keys take every key as a candidate (T0 = 0).  Longer rows: T0 is
// the key of rank 1.5 x (the sample's share of k) + 32 in a sample of kSample
// keys (runs of 4 adjacent keys spread evenly over a 16-byte aligned row, else
// single keys at an even stride), placed by two passes of the radix select in
// LDS: the lower edge of the bin (24 bits below the sample's shared leading
// bits) that holds that rank -- about 1.5 k candidates, with margin.  Each
// workgroup also records its candidates' largest key, which with T0 bounds
// the select kernel's keys.  (As separate launches, the one-workgroup
// threshold kernel took 9.2 us and the compaction 5.0 us behind it.)
template <bool VEC>
__global__ __launch_bounds__(kTopkThreads) void dsa_topk_compact_kernel(
    const float* __restrict__ scores, const int32_t* __restrict__ lens, TopkWs ws, int cap,
    int K) {
  __shared__ uint32_t sample[kSample];
  __shared__ __align__(16) int hist[kRadixBins];
  __shared__ int scan_tmp[kTopkWaves];
  __shared__ uint32_t wave_max[kTopkWaves];
  __shared__ int found[2];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wv = tid / kWave;
  const int b = blockIdx.y;
  const int chunk = blockIdx.x;
  int n = lens[b];
  n = n < 0 ? 0 : (n > cap ? cap : n);
  if (n <= K) return;  // the select kernel takes every key; nothing to compact
  const int c0 = chunk * kChunkKeys;
  if (c0 >= n) return;
  const float* sb = scores + static_cast<size_t>(b) * cap;

  // this chunk's keys c0 + 4 tid .. + 3, loaded first so that they are in
  // flight while the threshold is placed
  static_assert(kChunkKeys == 4 * kTopkThreads, "four keys of the chunk per thread");
  const int i = c0 + 4 * tid;
  float v[4];
  if (VEC && i + 3 < n) {
    const f32x4 t = *reinterpret_cast<const f32x4*>(sb + i);
    v[0] = t[0]; v[1] = t[1]; v[2] = t[2]; v[3] = t[3];
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = i + e < n ? sb[i + e] : 0.f;
  }

  uint32_t T0 = 0u;
  if (n > kCandCap) {
    constexpr int kPer = kSample / kTopkThreads;
    float sv[kPer];
    if (VEC) {
      static_assert(kSample / kTopkThreads == 4, "one float4 of sample keys per thread");
      // runs of kPer adjacent keys, one 16-byte load per thread, spread evenly
      // over the row (n > kCandCap, so every run lies inside it)
      const int j0 =
          static_cast<int>(static_cast<long long>(tid) * n / kTopkThreads) & ~(kPer - 1);
      const float4 f = *reinterpret_cast<const float4*>(sb + j0);
      sv[0] = f.x;
      sv[1] = f.y;
      sv[2] = f.z;
      sv[3] = f.w;
    } else {
#pragma unroll
      for (int k = 0; k < kPer; ++k) {
        const int j = tid + k * kTopkThreads;
        sv[k] = sb[static_cast<int>(static_cast<long long>(j) * n / kSample)];
      }
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) sample[tid * kPer + k] = order_key(sv[k]);
    __syncthreads();
    long long r = (static_cast<long long>(K) * kSample + n - 1) / n;
    r = r + r / 2 + 32;
    const int want = static_cast<int>(r > kSample ? kSample : r);
    int unused;
    radix_select([&](int k) { return sample[k]; }, kSample, want, hist, scan_tmp, found,
                 false, 0u, 0u, 2, T0, unused);
  }
  if (chunk == 0 && tid == 0) ws.t0[b] = T0;

  // keys >= T0 in index order: a scan over the workgroup places each thread's
  // candidates; the same barrier collects the chunk's largest candidate key
  bool in[4];
  int cnt = 0;
  uint32_t mx = 0u;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t u = order_key(v[e]);
    in[e] = i + e < n && u >= T0;
    cnt += in[e] ? 1 : 0;
    mx = in[e] && u > mx ? u : mx;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const uint32_t y = static_cast<uint32_t>(__shfl_xor(static_cast<int>(mx), o));
    mx = y > mx ? y : mx;
  }
  const int inc = wave_inclusive_scan(cnt, lane);
  if (lane == kWave - 1) scan_tmp[wv] = inc;
  if (lane == 0) wave_max[wv] = mx;
  __syncthreads();
  int at = inc - cnt;
  int all = 0;
  uint32_t cmax = 0u;
#pragma unroll
  for (int k = 0; k < kTopkWaves; ++k) {
    const int t = scan_tmp[k];
    at += k < wv ? t : 0;
    all += t;
    cmax = wave_max[k] > cmax ? wave_max[k] : cmax;
  }
  uint2* slots = ws.cand + (static_cast<size_t>(b) * ws.chunks + chunk) * kChunkKeys;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if (in[e]) {
      slots[at] = make_uint2(order_key(v[e]), static_cast<uint32_t>(i + e));
      ++at;
    }
  }
  if (tid == 0) {
    ws.counts[static_cast<size_t>(b) * ws.chunks + chunk] = all;
    ws.cmax[static_cast<size_t>(b) * ws.chunks + chunk] = cmax;
  }
}

// 3. Select: one workgroup per row.  The chunks' candidates, in chunk order
// (index order), go to LDS when there are between k and kCandCap of them;
// the exact selection and the ordered write run there.  Otherwise -- a
// threshold that the sample misplaced -- the exact selection runs over the
// row in memory.
__global__ __launch_bounds__(kTopkThreads) void dsa_topk_select_kernel(
    const float* __restrict__ scores, const int32_t* __restrict__ lens, TopkWs ws,
    int32_t* __restrict__ sel, int32_t* __restrict__ sel_lens, int cap, int K) {
  __shared__ uint32_t cand_key[kCandCap];
  __shared__ int32_t cand_idx[kCandCap];
  __shared__ __align__(16) int hist[kRadixBins];
  __shared__ int scan_tmp[kTopkWaves];
  __shared__ int found[2];
  __shared__ int wave_gt[kTopkWaves];
  __shared__ int wave_eq[kTopkWaves];
  __shared__ uint32_t wave_max[kTopkWaves];
  __shared__ int chunk_off[kChunksPerThread * kTopkThreads + 1];
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
  // candidate offsets of the row's chunks (up to 2048 chunks in LDS), and the
  // largest candidate key, which with T0 bounds every candidate
  const int nch = (n + kChunkKeys - 1) / kChunkKeys;
  const int* cnt = ws.counts + static_cast<size_t>(b) * ws.chunks;
  const uint32_t* cmx = ws.cmax + static_cast<size_t>(b) * ws.chunks;
  const uint32_t t0 = ws.t0[b];
  int C = 0;
  bool fits = nch <= kChunksPerThread * kTopkThreads;
  if (fits) {
    int c2[kChunksPerThread];
    int mine = 0;
    uint32_t m2 = 0u;
#pragma unroll
    for (int e = 0; e < kChunksPerThread; ++e) {
      const int ch = kChunksPerThread * tid + e;
      c2[e] = ch < nch ? cnt[ch] : 0;
      const uint32_t m = ch < nch ? cmx[ch] : 0u;
      m2 = m > m2 ? m : m2;
      mine += c2[e];
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const uint32_t y = static_cast<uint32_t>(__shfl_xor(static_cast<int>(m2), o));
      m2 = y > m2 ? y : m2;
    }
    if (lane == 0) wave_max[wv] = m2;  // read after the scan's barriers
    int total;
    int run = block_exclusive_scan(mine, scan_tmp, total);
#pragma unroll
    for (int e = 0; e < kChunksPerThread; ++e) {
      const int ch = kChunksPerThread * tid + e;
      if (ch < nch) chunk_off[ch] = run;
      run += c2[e];
    }
    if (tid == 0) chunk_off[nch] = total;
    C = total;
    fits = C >= K && C <= kCandCap;
    __syncthreads();
  }
  uint32_t T;
  int kk;
  if (fits) {
    // flat candidate j -> its chunk by binary search over the offsets; every
    // thread's loads (at most kCandCap / kTopkThreads) are issued before the
    // first is stored to LDS, so the gather costs one memory round trip
    constexpr int kPerThread = kCandCap / kTopkThreads;
    uint2 e[kPerThread];
#pragma unroll
    for (int r = 0; r < kPerThread; ++r) {
      const int j = tid + r * kTopkThreads;
      if (j < C) {
        int lo = 0, hi = nch;
        while (hi - lo > 1) {
          const int mid = (lo + hi) >> 1;
          if (chunk_off[mid] <= j) lo = mid; else hi = mid;
        }
        e[r] = ws.cand[(static_cast<size_t>(b) * ws.chunks + lo) * kChunkKeys +
                       (j - chunk_off[lo])];
      }
    }
#pragma unroll
    for (int r = 0; r < kPerThread; ++r) {
      const int j = tid + r * kTopkThreads;
      if (j < C) {
        cand_key[j] = e[r].x;
        cand_idx[j] = static_cast<int32_t>(e[r].y);
      }
    }
    __syncthreads();
    uint32_t hi = 0u;
#pragma unroll
    for (int k = 0; k < kTopkWaves; ++k) hi = wave_max[k] > hi ? wave_max[k] : hi;
    auto lds_key = [&](int i) { return cand_key[i]; };
    auto lds_idx = [&](int i) { return cand_idx[i]; };
    radix_select(lds_key, C, K, hist, scan_tmp, found, true, t0, hi, 0, T, kk);
    ordered_write(lds_key, lds_idx, C, T, kk, wave_gt, wave_eq, ob);
  } else {
    auto mem_key = [&](int i) { return order_key(sb[i]); };
    radix_select(mem_key, n, K, hist, scan_tmp, found, false, 0u, 0u, 0, T, kk);
    ordered_write(mem_key, [](int i) { return i; }, n, T, kk, wave_gt, wave_eq, ob);
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

extern "C" size_t voom_dsa_topk_workspace_bytes(int batch, int cap) {
  if (batch <= 0 || cap <= 0) return 0;
  const size_t chunks = static_cast<size_t>(topk_chunks(cap));
  return ((static_cast<size_t>(batch) * 4 + 255) & ~size_t(255)) +
         2 * ((static_cast<size_t>(batch) * chunks * 4 + 255) & ~size_t(255)) +
         static_cast<size_t>(batch) * chunks * kChunkKeys * sizeof(uint2);
}

extern "C" int voom_dsa_topk(const float* scores, const int32_t* lens, int32_t* sel,
                             int32_t* sel_lens, void* workspace, size_t ws_bytes, int batch,
                             int cap, int k, hipStream_t stream) {
  const char* who = "dsa_topk";
  VOOM_REQUIRE(scores && lens && sel && sel_lens && workspace, "%s: null pointer argument", who);
  VOOM_REQUIRE(batch > 0 && batch < 65536 && cap > 0 && k > 0, "%s: bad batch, capacity or k",
               who);
  const size_t need = voom_dsa_topk_workspace_bytes(batch, cap);
  VOOM_REQUIRE(ws_bytes >= need, "%s: workspace %zu bytes < required %zu", who, ws_bytes, need);
  VOOM_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0,
               "%s: workspace must be 16-byte aligned", who);
  TopkWs ws;
  ws.chunks = topk_chunks(cap);
  char* p = static_cast<char*>(workspace);
  const size_t t0_bytes = (static_cast<size_t>(batch) * 4 + 255) & ~size_t(255);
  const size_t per_chunk_bytes = (static_cast<size_t>(batch) * ws.chunks * 4 + 255) & ~size_t(255);
  ws.t0 = reinterpret_cast<uint32_t*>(p);
  ws.counts = reinterpret_cast<int*>(p + t0_bytes);
  ws.cmax = reinterpret_cast<uint32_t*>(p + t0_bytes + per_chunk_bytes);
  ws.cand = reinterpret_cast<uint2*>(p + t0_bytes + 2 * per_chunk_bytes);
  const bool vec = cap % 4 == 0 && reinterpret_cast<uintptr_t>(scores) % 16 == 0;
  const dim3 cgrid(static_cast<unsigned>(ws.chunks), static_cast<unsigned>(batch));
  if (vec) {
    hipLaunchKernelGGL(dsa_topk_compact_kernel<true>, cgrid, dim3(kTopkThreads), 0, stream,
                       scores, lens, ws, cap, k);
  } else {
    hipLaunchKernelGGL(dsa_topk_compact_kernel<false>, cgrid, dim3(kTopkThreads), 0, stream,
                       scores, lens, ws, cap, k);
  }
  int rc = VOOM_LAUNCH_CHECK("dsa_topk: threshold + compaction kernel launch");
  if (rc) return rc;
  hipLaunchKernelGGL(dsa_topk_select_kernel, dim3(static_cast<unsigned>(batch)),
                     dim3(kTopkThreads), 0, stream, scores, lens, ws, sel, sel_lens, cap, k);
  return VOOM_LAUNCH_CHECK("dsa_topk: select kernel launch");
}
