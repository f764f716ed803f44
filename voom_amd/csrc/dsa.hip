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
// Top-k, one launch per call: chunk workgroups (4,096 keys each) each place
// the same threshold T0 at a fixed rank of a strided sample of the row and
// move the keys >= T0, with their indices and in index order, to per-chunk
// slots -- the row is read once, by many CUs; the row's last chunk workgroup
// to finish (an arrival counter in the workspace) gathers the candidates (at
// most 16,384) into registers and runs the exact selection there: radix
// passes over offsets from the candidates' smallest key find the k-th largest
// key T and how many keys equal to T to keep, and an ordered write -- each
// wavefront owns a contiguous range of candidates, counts its keys above and
// equal to T, and after a prefix over wavefronts writes its indices -- leaves
// the output sorted without a sort.  Scores map to order-preserving 32-bit
// keys.  When the sample misjudges the row (fewer than k or more than 16,384
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
constexpr int kChunksPerThread = 2;                // up to 2048 chunks per row
constexpr int kCandCap = 16384;                    // candidates selected from registers
constexpr int kRegKeys = kCandCap / kTopkThreads;  // candidates per thread
constexpr int kSample = 4096;                      // keys sampled to place the threshold
constexpr int kChunkKeys = 4096;                   // keys per chunk workgroup
constexpr int kWaveKeys = kChunkKeys / (kTopkThreads / kWave);  // 256 keys per wavefront
// rows of at most this many chunks (512 Ki keys) compact each wavefront's
// keys into its own 256-slot segment: as many segments as the selection's
// offset scan takes (two per thread)
constexpr int kSegChunks = kChunksPerThread * kTopkThreads / (kTopkThreads / kWave);
static_assert(kChunkKeys == 4 * kTopkThreads, "four keys of the chunk per thread");
static_assert(kSample == 4 * kTopkThreads, "four sample keys per thread");

// Order-preserving map of fp32 onto uint32: a > b  <=>  key(a) > key(b), and
// -0 maps like +0 (they compare equal, so they tie).
__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  u = u == 0x80000000u ? 0u : u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, false));
}

// Largest and smallest of a uint32 over the 64 lanes, the same in every lane
// (quad swaps and row mirrors by DPP, then the four rows read out).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  uint32_t t;
  t = dpp_u32<0xB1>(v);  v = t > v ? t : v;
  t = dpp_u32<0x4E>(v);  v = t > v ? t : v;
  t = dpp_u32<0x141>(v); v = t > v ? t : v;
  t = dpp_u32<0x140>(v); v = t > v ? t : v;
  uint32_t r = 0u;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t x = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 16 * k));
    r = x > r ? x : r;
  }
  return r;
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  return ~wave_max_u32(~v);
}

// Exclusive scan of one int per thread over the workgroup; returns the
// workgroup total in `total`.  `tmp` holds kTopkWaves ints of LDS; the
// caller passes a barrier before anything writes `tmp` again.
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
  return before + inc - x;
}

// Radix select over keys held in registers: thread t holds up to N keys,
// key[r] in use iff r < nregs (the same in every thread) and bit r of
// `valid`, every one within [lo, hi].  The top `rank` keys (1 <= rank <= the
// number of keys) are then every key > T and the first kk keys equal to T:
// T is the rank-th largest key and kk how many keys equal to it belong to
// the top `rank`, or -- when after some pass the rank takes every key of the
// crossing bin, which ends the select there -- T is one below that bin's
// lower edge and kk is 0.  With max_passes > 0 the passes may stop early -- after
// max_passes passes, or after any pass whose crossing bin holds at most
// `enough` keys: T is then the lower edge of the bin holding the rank-th
// largest key (at least `rank` keys are >= T, at most rank - 1 + enough) and
// kk is meaningless.
//
// Bins are offsets from the range's lower end: a pass over [base, base +
// span] counts (key - base) >> shift in 2^width bins, width = min(bits of
// span, kRadixBits), so the bins cover the keys' range however many leading
// bits its ends share (scores on both sides of a power of two share none,
// yet may lie close together); the bin holding the rank-th largest key is
// the next range.  A range narrower than 2^24 takes two passes.
//
// Per pass: the histogram (LDS atomics); a barrier; thread t takes bins 4 q4
// .. 4 q4 + 3 (q4 = 1023 - t, so the bins run in descending order over the
// threads), clears the same int4 of the other histogram buffer, and each
// wavefront scans its counts (DPP) and leaves its total; a barrier;
// wavefront 0 alone finds the crossing -- the totals name the wavefront whose
// bins hold it, whose 256 bins it reads and scans -- and leaves it in
// found[]; a barrier.  (Every wavefront finding it for itself saves that
// barrier but costs more: sixteen wavefronts share four SIMDs.)  The two
// buffers alternate between passes, so pass p's is cleared in pass p + 1,
// after every wavefront has passed pass p.
// hist2: 2 * kRadixBins ints, 16-byte aligned, both buffers zero (the
// caller clears them before a barrier it passes anyway: a barrier of its own
// here cost ~0.3 us per call); totals: kTopkWaves ints, 16-byte aligned;
// found: 3 ints.  Every wavefront must have finished with them since its
// last barrier.
template <int N>
__device__ void radix_select_regs(const uint32_t (&key)[N], uint32_t valid, int nregs, int rank,
                                  int* hist2, int* totals, int* found, uint32_t lo, uint32_t hi,
                                  int max_passes, int enough, uint32_t& T, int& kk_out) {
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wv = tid / kWave;
  int4* h4 = reinterpret_cast<int4*>(hist2);
  uint32_t base = lo;
  uint32_t span = hi - lo;
  int kk = rank;
#pragma unroll 1
  for (int pass = 0; span != 0u && (max_passes <= 0 || pass < max_passes); ++pass) {
    const int cur = pass & 1;
    int* hist = hist2 + cur * kRadixBins;
    const int bits = 32 - __clz(static_cast<int>(span));
    const int width = bits < kRadixBits ? bits : kRadixBits;
    const int shift = bits - width;
#pragma unroll
    for (int r = 0; r < N; ++r) {
      if (r < nregs) {
        const uint32_t d = key[r] - base;
        if (((valid >> r) & 1u) && d <= span) atomicAdd(&hist[d >> shift], 1);
      }
    }
    __syncthreads();  // histogram complete
    const int q4 = kRadixBins / 4 - 1 - tid;
    const int4 h = reinterpret_cast<const int4*>(hist)[q4];
    h4[(cur ^ 1) * (kRadixBins / 4) + q4] = make_int4(0, 0, 0, 0);
    const int mine = h.x + h.y + h.z + h.w;
    const int inc = wave_inclusive_scan(mine, lane);
    if (lane == kWave - 1) totals[wv] = inc;
    __syncthreads();  // wavefront totals in LDS; the other buffer clear
    if (wv == 0) {
      // cw: the wavefront whose bins hold the crossing; above: the keys in
      // the (higher) bins of the wavefronts before it
      int cw = 0;
      int above = 0;
      int cum = 0;
#pragma unroll
      for (int k4 = 0; k4 < kTopkWaves / 4; ++k4) {
        const int4 t = reinterpret_cast<const int4*>(totals)[k4];
        const int tk[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          cum += tk[e];
          if (cum < kk) {
            cw = 4 * k4 + e + 1;
            above = cum;
          }
        }
      }
      const int cq4 = kRadixBins / 4 - 1 - (cw * kWave + lane);
      const int4 hc = reinterpret_cast<const int4*>(hist)[cq4];
      const int c[kBinsPerThread] = {hc.w, hc.z, hc.y, hc.x};  // bins 4 cq4 + 3 .. 4 cq4
      const int m = hc.x + hc.y + hc.z + hc.w;
      int run = above + wave_inclusive_scan(m, lane) - m;  // keys in higher bins
#pragma unroll
      for (int e = 0; e < kBinsPerThread; ++e) {
        if (run < kk && run + c[e] >= kk) {  // exactly one bin of one lane
          found[0] = 4 * cq4 + 3 - e;
          found[1] = run;
          found[2] = c[e];
        }
        run += c[e];
      }
    }
    __syncthreads();  // crossing in found[]
    const uint32_t off = static_cast<uint32_t>(found[0]) << shift;
    kk -= found[1];
    base += off;
    const uint32_t bin_m1 = (1u << shift) - 1u;
    span = span - off < bin_m1 ? span - off : bin_m1;
    if (max_passes > 0 && found[2] <= enough) break;
    if (max_passes <= 0 && span != 0u && found[2] == kk && base != 0u) {
      // the rank takes every key of the crossing bin: the selection is
      // every key >= the bin's lower edge, and no narrower pass is needed
      T = base - 1u;
      kk_out = 0;
      return;
    }
  }
  T = base;
  kk_out = kk;
}

// Ordered selection write from registers: key[r] / idx[r] of thread (wave w,
// lane l) is candidate w * per + 64 r + l, candidates in index order, in use
// iff r < nregs (the same in every thread) and bit r of `valid`.  Every key >
// T and the first kk keys == T go to out[] in index order: counts per
// wavefront, a prefix over the wavefronts, then ballots place each index.
// counts: 2 * kTopkWaves ints of LDS, 16-byte aligned.
template <int N>
__device__ void ordered_write_regs(const uint32_t (&key)[N], const int32_t (&idx)[N],
                                   uint32_t valid, int nregs, uint32_t T, int kk, int* counts,
                                   int32_t* out) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  int gt = 0;
  int eq = 0;
#pragma unroll
  for (int r = 0; r < N; ++r) {
    if (r < nregs) {
      const bool v = (valid >> r) & 1u;
      gt += __popcll(__ballot(v && key[r] > T));
      eq += __popcll(__ballot(v && key[r] == T));
    }
  }
  if (lane == 0) {
    counts[wv] = gt;
    counts[kTopkWaves + wv] = eq;
  }
  __syncthreads();
  int gt_before = 0;
  int eq_before = 0;
#pragma unroll
  for (int k4 = 0; k4 < kTopkWaves / 4; ++k4) {
    const int4 g = reinterpret_cast<const int4*>(counts)[k4];
    const int4 q = reinterpret_cast<const int4*>(counts + kTopkWaves)[k4];
    gt_before += (4 * k4 < wv ? g.x : 0) + (4 * k4 + 1 < wv ? g.y : 0) +
                 (4 * k4 + 2 < wv ? g.z : 0) + (4 * k4 + 3 < wv ? g.w : 0);
    eq_before += (4 * k4 < wv ? q.x : 0) + (4 * k4 + 1 < wv ? q.y : 0) +
                 (4 * k4 + 2 < wv ? q.z : 0) + (4 * k4 + 3 < wv ? q.w : 0);
  }
  int pos = gt_before + (eq_before < kk ? eq_before : kk);  // selections before this wave
  int eq_seen = eq_before;
  const unsigned long long below = (1ull << lane) - 1ull;
#pragma unroll
  for (int r = 0; r < N; ++r) {
    if (r < nregs) {
      const bool v = (valid >> r) & 1u;
      const bool is_gt = v && key[r] > T;
      const bool is_eq = v && key[r] == T;
      const unsigned long long eq_mask = __ballot(is_eq);
      const int eq_rank = eq_seen + __popcll(eq_mask & below);
      const bool take = is_gt || (is_eq && eq_rank < kk);
      const unsigned long long take_mask = __ballot(take);
      if (take) out[pos + __popcll(take_mask & below)] = idx[r];
      pos += __popcll(take_mask);
      eq_seen += __popcll(eq_mask);
    }
  }
}

// Radix select over keys read by key(i), i < count, from memory: the
// fallback for a row whose sampled threshold left fewer than k or more than
// kCandCap candidates.  Same digits and result as radix_select_regs (exact:
// no pass limit), one histogram buffer and three barriers per pass; the
// range comes from a min/max pass over the keys.  hist: kRadixBins ints,
// 16-byte aligned; scan_tmp kTopkWaves ints; found 2 ints.
template <typename KeyFn>
__device__ void radix_select_mem(KeyFn key, int count, int rank, int* hist, int* scan_tmp,
                                 int* found, uint32_t& T, int& kk_out) {
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wv = tid / kWave;
  int4* hist4 = reinterpret_cast<int4*>(hist);
  hist4[tid] = make_int4(0, 0, 0, 0);
  uint32_t lo = 0xFFFFFFFFu;
  uint32_t hi = 0u;
  for (int i = tid; i < count; i += kTopkThreads) {
    const uint32_t u = key(i);
    lo = u < lo ? u : lo;
    hi = u > hi ? u : hi;
  }
  lo = wave_min_u32(lo);
  hi = wave_max_u32(hi);
  if (lane == 0) {
    scan_tmp[wv] = static_cast<int>(lo);
    found[0] = 0;
  }
  __syncthreads();
  uint32_t l2 = 0xFFFFFFFFu;
#pragma unroll
  for (int k = 0; k < kTopkWaves; ++k) {
    const uint32_t x = static_cast<uint32_t>(scan_tmp[k]);
    l2 = x < l2 ? x : l2;
  }
  __syncthreads();
  if (lane == 0) scan_tmp[wv] = static_cast<int>(hi);
  __syncthreads();
  uint32_t h2 = 0u;
#pragma unroll
  for (int k = 0; k < kTopkWaves; ++k) {
    const uint32_t x = static_cast<uint32_t>(scan_tmp[k]);
    h2 = x > h2 ? x : h2;
  }
  __syncthreads();
  uint32_t base = l2;
  uint32_t span = h2 - l2;
  int kk = rank;
#pragma unroll 1
  while (span != 0u) {
    const int bits = 32 - __clz(static_cast<int>(span));
    const int width = bits < kRadixBits ? bits : kRadixBits;
    const int shift = bits - width;
    for (int i = tid; i < count; i += kTopkThreads) {
      const uint32_t d = key(i) - base;
      if (d <= span) atomicAdd(&hist[d >> shift], 1);
    }
    __syncthreads();  // histogram complete
    const int q4 = kRadixBins / 4 - 1 - tid;
    const int4 h = hist4[q4];
    hist4[q4] = make_int4(0, 0, 0, 0);
    const int c[kBinsPerThread] = {h.w, h.z, h.y, h.x};
    const int mine = h.x + h.y + h.z + h.w;
    const int inc = wave_inclusive_scan(mine, lane);
    if (lane == kWave - 1) scan_tmp[wv] = inc;
    __syncthreads();  // wave totals in scan_tmp, bins clear again
    int run = inc - mine;
#pragma unroll
    for (int k = 0; k < kTopkWaves; ++k) run += k < wv ? scan_tmp[k] : 0;
#pragma unroll
    for (int e = 0; e < kBinsPerThread; ++e) {
      if (run < kk && run + c[e] >= kk) {
        found[0] = 4 * q4 + 3 - e;
        found[1] = run;
      }
      run += c[e];
    }
    __syncthreads();  // crossing in found[]
    const uint32_t off = static_cast<uint32_t>(found[0]) << shift;
    kk -= found[1];
    base += off;
    const uint32_t bin_m1 = (1u << shift) - 1u;
    span = span - off < bin_m1 ? span - off : bin_m1;
  }
  __syncthreads();  // found[] read by every thread before anyone reuses it
  T = base;
  kk_out = kk;
}

// Ordered selection write over keys read from memory (the fallback's):
// keys i < count in index order; every key > T and the first kk keys == T go
// to out[] in that order, as idx(i).  Wavefront w owns a contiguous range of
// i; counts, a prefix over wavefronts, then ballots place each index.
template <typename KeyFn, typename IdxFn>
__device__ void ordered_write_mem(KeyFn key, IdxFn idx, int count, uint32_t T, int kk, int* wave_gt,
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
  int pos = gt_before + (eq_before < kk ? eq_before : kk);
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
}

// Workspace of the top-k (per row): the arrival counter of the row's chunk
// workgroups (zero between calls), per-chunk candidate counts and largest
// candidate keys, and per-chunk candidate slots of (key, index) pairs.
struct TopkWs {
  int* arrive;      // [B]
  int* counts;      // [B, chunks * 16]: candidates per segment (16 per chunk, or 1)
  uint32_t* cmax;   // [B, chunks * 16]: largest candidate key per segment
  uint2* cand;      // [B, chunks, kChunkKeys]
  int chunks;
};

__host__ __device__ inline int topk_chunks(int cap) { return (cap + kChunkKeys - 1) / kChunkKeys; }

// The top-k of a row, one launch: one workgroup per chunk of kChunkKeys keys.
//
// 1. Threshold.  Each workgroup places the row's threshold T0 itself -- every
//    one from the same sample with the same passes, so all agree -- while its
//    chunk's keys are in flight.  Rows of at most kCandCap keys take every key
//    as a candidate (T0 = 0).  Longer rows: T0 is the lower edge of the bin
//    holding the key of rank 1.5 x (the sample's share of k) + 32 in a sample
//    of kSample keys (runs of 4 adjacent keys spread evenly over a 16-byte
//    aligned row, else single keys at an even stride) -- after one pass of
//    radix_select_regs (bins of the sample's span / 4096) when that bin holds
//    at most 32 sample keys, else after a second (span / 2^24): about 1.5 k
//    + 32 n / kSample candidates (4,100-4,800 for k = 2048 of 131,072 keys).
// 2. Compaction.  Keys >= T0 move, with their indices and in index order,
//    to the chunk's slots, with a count and a largest key per segment: each
//    wavefront's own 256-slot segment (rows of at most kSegChunks chunks),
//    else one segment per chunk.
// 3. Selection, by the row's last workgroup to finish (an arrival counter;
//    its stores released to every XCD before the count, the others' acquired
//    after it): between k and kCandCap candidates are gathered, in segment
//    (so index) order, straight into registers, kRegKeys per thread, through
//    an LDS table of their slots; the exact select over the range [T0,
//    largest candidate] and the ordered write run from there.  Otherwise --
//    a threshold the sample misplaced -- the exact selection runs over the
//    row in memory.
// The counter is back at zero when the launch ends.
template <bool VEC>
__global__ __launch_bounds__(kTopkThreads) void dsa_topk_kernel(
    const float* __restrict__ scores, const int32_t* __restrict__ lens, TopkWs ws,
    int32_t* __restrict__ sel, int32_t* __restrict__ sel_lens, int cap, int K) {
  __shared__ __align__(16) int hist2[2 * kRadixBins];
  __shared__ __align__(16) int totals[kTopkWaves];
  __shared__ __align__(16) int scan_tmp[kTopkWaves];
  __shared__ __align__(16) uint32_t wave_red[2 * kTopkWaves];
  __shared__ int slot_of[kCandCap];  // candidate j -> its slot in the row's slots
  __shared__ __align__(16) int wcount[2 * kTopkWaves];
  __shared__ int found[3];
  __shared__ int is_last;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wv = tid / kWave;
  const int b = blockIdx.y;
  const int chunk = blockIdx.x;
  int n = lens[b];
  n = n < 0 ? 0 : (n > cap ? cap : n);
  int32_t* ob = sel + static_cast<size_t>(b) * K;
  if (n <= K) {  // every key is selected
    if (chunk == 0) {
      for (int i = tid; i < n; i += kTopkThreads) ob[i] = i;
      if (tid == 0) sel_lens[b] = n;
    }
    return;
  }
  const int nch = (n + kChunkKeys - 1) / kChunkKeys;
  const int c0 = chunk * kChunkKeys;
  if (c0 >= n) return;
  const float* sb = scores + static_cast<size_t>(b) * cap;

  // this chunk's keys c0 + 4 tid .. + 3, in flight while T0 is placed
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
    uint32_t sk[4];
    if (VEC) {
      // runs of 4 adjacent keys, one 16-byte load per thread, spread evenly
      // over the row (n > kCandCap, so every run lies inside it)
      const int j0 = static_cast<int>(static_cast<long long>(tid) * n / kTopkThreads) & ~3;
      const f32x4 f = *reinterpret_cast<const f32x4*>(sb + j0);
#pragma unroll
      for (int k = 0; k < 4; ++k) sk[k] = order_key(f[k]);
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int j = tid + k * kTopkThreads;
        sk[k] = order_key(sb[static_cast<int>(static_cast<long long>(j) * n / kSample)]);
      }
    }
    uint32_t lo = sk[0];
    uint32_t hi = sk[0];
#pragma unroll
    for (int k = 1; k < 4; ++k) {
      lo = sk[k] < lo ? sk[k] : lo;
      hi = sk[k] > hi ? sk[k] : hi;
    }
    lo = wave_min_u32(lo);
    hi = wave_max_u32(hi);
    if (lane == 0) {
      wave_red[wv] = lo;
      wave_red[kTopkWaves + wv] = hi;
    }
    // the select's histograms, cleared under the same barrier
    reinterpret_cast<int4*>(hist2)[tid] = make_int4(0, 0, 0, 0);
    reinterpret_cast<int4*>(hist2)[tid + kRadixBins / 4] = make_int4(0, 0, 0, 0);
    __syncthreads();
    lo = 0xFFFFFFFFu;
    hi = 0u;
#pragma unroll
    for (int k = 0; k < kTopkWaves; ++k) {
      lo = wave_red[k] < lo ? wave_red[k] : lo;
      hi = wave_red[kTopkWaves + k] > hi ? wave_red[kTopkWaves + k] : hi;
    }
    long long r = (static_cast<long long>(K) * kSample + n - 1) / n;
    r = r + r / 2 + 32;
    const int want = static_cast<int>(r > kSample ? kSample : r);
    int unused;
    // a second pass only when the first one's crossing bin holds more than
    // 32 sample keys (about 1,000 more candidates than the rank asks for)
    radix_select_regs(sk, 0xFu, 4, want, hist2, totals, found, lo, hi, 2, 32, T0, unused);
  }

  // keys >= T0 in index order.  Rows of at most kSegChunks chunks: each
  // wavefront moves its 256 keys' candidates into its own 256-slot segment
  // of the chunk's slots (a wave scan, no barrier) and leaves the segment's
  // count and largest key.  Longer rows: a scan over the workgroup places
  // the chunk's candidates densely (one segment of 4096 slots), and the
  // same barrier collects the chunk's largest.
  const bool per_wave = nch <= kSegChunks;
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
  mx = wave_max_u32(mx);
  const int inc = wave_inclusive_scan(cnt, lane);
  int at = inc - cnt;
  uint2* slots = ws.cand + (static_cast<size_t>(b) * ws.chunks + chunk) * kChunkKeys;
  // the row's segment counts and largest keys: [chunks * 16] per row
  const size_t seg_row = static_cast<size_t>(b) * ws.chunks * kTopkWaves;
  if (per_wave) {
    slots += kWaveKeys * wv;
    if (lane == kWave - 1) {  // inc: the wavefront's count; mx is uniform
      ws.counts[seg_row + kTopkWaves * chunk + wv] = inc;
      ws.cmax[seg_row + kTopkWaves * chunk + wv] = mx;
    }
  } else {
    if (lane == kWave - 1) scan_tmp[wv] = inc;
    if (lane == 0) wave_red[wv] = mx;
    __syncthreads();
    int all = 0;
    uint32_t cmax = 0u;
#pragma unroll
    for (int k4 = 0; k4 < kTopkWaves / 4; ++k4) {
      const int4 t4 = reinterpret_cast<const int4*>(scan_tmp)[k4];
      const uint4 m4 = reinterpret_cast<const uint4*>(wave_red)[k4];
      const int t[4] = {t4.x, t4.y, t4.z, t4.w};
      const uint32_t m[4] = {m4.x, m4.y, m4.z, m4.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        at += 4 * k4 + e < wv ? t[e] : 0;
        all += t[e];
        cmax = m[e] > cmax ? m[e] : cmax;
      }
    }
    if (tid == 0) {
      ws.counts[seg_row + chunk] = all;
      ws.cmax[seg_row + chunk] = cmax;
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if (in[e]) {
      slots[at] = make_uint2(order_key(v[e]), static_cast<uint32_t>(i + e));
      ++at;
    }
  }

  // Publish, then count the arrival: every wavefront waits for its stores to
  // reach its XCD's L2, one release fence writes that L2 back for the other
  // XCDs, and the last workgroup to arrive acquires theirs.
  wait_vmem_all();
  __syncthreads();
  if (tid == 0) {
    __threadfence();
    const int last = atomicAdd(&ws.arrive[b], 1) == nch - 1;
    if (last) {
      atomicExch(&ws.arrive[b], 0);  // zero again for the next call
      __threadfence();
    }
    is_last = last;
  }
  __syncthreads();
  if (!is_last) return;
  // the exact select's histograms, cleared now: the barrier after the chunk
  // offsets below also orders this
  reinterpret_cast<int4*>(hist2)[tid] = make_int4(0, 0, 0, 0);
  reinterpret_cast<int4*>(hist2)[tid + kRadixBins / 4] = make_int4(0, 0, 0, 0);

  // ---- selection over the row's candidates ----
  // The segments' counts (in index order) give each candidate its slot: a
  // scan over the workgroup, then the thread holding segment s writes the
  // slots of candidates off[s] .. off[s + 1] - 1 into slot_of; the segments'
  // largest keys give the largest candidate, which with T0 bounds them all.
  const int nseg = per_wave ? nch * kTopkWaves : nch;
  const int seg_keys = per_wave ? kWaveKeys : kChunkKeys;
  const int* cnt_row = ws.counts + static_cast<size_t>(b) * ws.chunks * kTopkWaves;
  const uint32_t* cmx_row = ws.cmax + static_cast<size_t>(b) * ws.chunks * kTopkWaves;
  int C = 0;
  uint32_t hi = 0u;
  bool fits = nseg <= kChunksPerThread * kTopkThreads;
  if (fits) {
    int c2[kChunksPerThread];
    int mine = 0;
    uint32_t m2 = 0u;
#pragma unroll
    for (int e = 0; e < kChunksPerThread; ++e) {
      const int sg = kChunksPerThread * tid + e;
      c2[e] = sg < nseg ? cnt_row[sg] : 0;
      const uint32_t m = sg < nseg ? cmx_row[sg] : 0u;
      m2 = m > m2 ? m : m2;
      mine += c2[e];
    }
    m2 = wave_max_u32(m2);
    if (lane == 0) wave_red[wv] = m2;  // read after the scan's barrier
    int total;
    int run = block_exclusive_scan(mine, scan_tmp, total);
#pragma unroll
    for (int k = 0; k < kTopkWaves; ++k) hi = wave_red[k] > hi ? wave_red[k] : hi;
    C = total;
    fits = C >= K && C <= kCandCap;
    if (fits) {
#pragma unroll
      for (int e = 0; e < kChunksPerThread; ++e) {
        const int base = (kChunksPerThread * tid + e) * seg_keys;
        for (int k = 0; k < c2[e]; ++k) slot_of[run + k] = base + k;
        run += c2[e];
      }
    }
    __syncthreads();  // slot_of complete
  }
  uint32_t T;
  int kk;
  if (fits) {
    // wavefront w holds candidates w * per .. + per - 1, 64 per register
    // (nregs registers), each lane's slots read from slot_of.  Every load is
    // issued before the first is used: one memory round trip.
    const int per = ((C + kTopkWaves - 1) / kTopkWaves + kWave - 1) / kWave * kWave;
    const int nregs = per / kWave;
    const int j0 = wv * per;
    const uint2* cand_row = ws.cand + static_cast<size_t>(b) * ws.chunks * kChunkKeys;
    uint2 e[kRegKeys];
    uint32_t valid = 0u;
#pragma unroll
    for (int r = 0; r < kRegKeys; ++r) {
      e[r] = make_uint2(0u, 0u);
      if (r < nregs) {
        const int j = j0 + kWave * r + lane;
        if (j < C) {
          e[r] = cand_row[slot_of[j]];
          valid |= 1u << r;
        }
      }
    }
    uint32_t key[kRegKeys];
    int32_t idx[kRegKeys];
#pragma unroll
    for (int r = 0; r < kRegKeys; ++r) {
      key[r] = e[r].x;
      idx[r] = static_cast<int32_t>(e[r].y);
    }
    radix_select_regs(key, valid, nregs, K, hist2, totals, found, T0, hi, 0, 0, T, kk);
    ordered_write_regs(key, idx, valid, nregs, T, kk, wcount, ob);
  } else {
    auto mem_key = [&](int i) { return order_key(sb[i]); };
    radix_select_mem(mem_key, n, K, hist2, scan_tmp, found, T, kk);
    ordered_write_mem(mem_key, [](int i) { return i; }, n, T, kk, wcount, wcount + kTopkWaves, ob);
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
         2 * ((static_cast<size_t>(batch) * chunks * kTopkWaves * 4 + 255) & ~size_t(255)) +
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
  const size_t arrive_bytes = (static_cast<size_t>(batch) * 4 + 255) & ~size_t(255);
  const size_t per_chunk_bytes =
      (static_cast<size_t>(batch) * ws.chunks * kTopkWaves * 4 + 255) & ~size_t(255);
  ws.arrive = reinterpret_cast<int*>(p);
  ws.counts = reinterpret_cast<int*>(p + arrive_bytes);
  ws.cmax = reinterpret_cast<uint32_t*>(p + arrive_bytes + per_chunk_bytes);
  ws.cand = reinterpret_cast<uint2*>(p + arrive_bytes + 2 * per_chunk_bytes);
  const bool vec = cap % 4 == 0 && reinterpret_cast<uintptr_t>(scores) % 16 == 0;
  const dim3 grid(static_cast<unsigned>(ws.chunks), static_cast<unsigned>(batch));
  if (vec) {
    hipLaunchKernelGGL(dsa_topk_kernel<true>, grid, dim3(kTopkThreads), 0, stream, scores, lens,
                       ws, sel, sel_lens, cap, k);
  } else {
    hipLaunchKernelGGL(dsa_topk_kernel<false>, grid, dim3(kTopkThreads), 0, stream, scores, lens,
                       ws, sel, sel_lens, cap, k);
  }
  return VOOM_LAUNCH_CHECK("dsa_topk: kernel launch");
}
