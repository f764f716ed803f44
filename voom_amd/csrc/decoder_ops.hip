// Fused per-token ops of the config-1 decoder harness (a Llama-style block
// around the paged attention), so that one decode step is a short chain of
// launches: the residual add + RMSNorm, RoPE of q and k together with the
// split of the fused qkv projection into the attention layouts, SwiGLU, and
// the one-token projections (GEMV, optionally with SwiGLU fused).
// They restate the block math of runtime/layer_runner.py (rms_norm :263,309,
// rope :99-103, _silu_mul :43-46 and :188) with Hugging Face LlamaForCausalLM's
// cast order -- the reference its parity tests use:
//   rms_norm:  y = bf16(w * bf16(x * rsqrt(mean(x^2) + eps)))   stats in fp32
//   rope:      rotate-half, fp32 products from fp32 cos/sin tables, bf16 out
//   swiglu:    bf16(bf16(g / (1 + exp(-g))) * u)
// All memory-bound; each kernel reads and writes its rows once.
#include "common.h"

namespace voom {
namespace {

constexpr int kRowThreads = 256;

// 16-byte chunk at col of bf16(x + delta) (of x alone without delta).
__device__ __forceinline__ u32x4 add_chunk(const uint16_t* __restrict__ x,
                                           const uint16_t* __restrict__ delta, int col) {
  u32x4 a = *reinterpret_cast<const u32x4*>(x + col);
  if (delta) {
    const u32x4 d = *reinterpret_cast<const u32x4*>(delta + col);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float lo = bf2f(static_cast<uint16_t>(a[w] & 0xffffu)) +
                       bf2f(static_cast<uint16_t>(d[w] & 0xffffu));
      const float hi = bf2f(static_cast<uint16_t>(a[w] >> 16)) +
                       bf2f(static_cast<uint16_t>(d[w] >> 16));
      a[w] = pack_bf16x2(lo, hi);
    }
  }
  return a;
}

// Sum of squares of one chunk's 8 values added to ss, in element order with
// explicit fused multiply-adds.  The row statistics of every kernel here are
// built the same way -- lane l of one wavefront takes chunks l, l + 64, ...
// in order, then the lanes are summed by wave_sum_uniform (and
// 1 / sqrt(ss / hidden + eps)) -- so a fused normalisation is bit-identical
// to add_rms_norm_kernel's.
__device__ __forceinline__ float chunk_sumsq(u32x4 a, float ss) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float lo = bf2f(static_cast<uint16_t>(a[w] & 0xffffu));
    const float hi = bf2f(static_cast<uint16_t>(a[w] >> 16));
    ss = __builtin_fmaf(lo, lo, ss);
    ss = __builtin_fmaf(hi, hi, ss);
  }
  return ss;
}
__device__ __forceinline__ float rms_inv(float ss_lane, int hidden, float eps) {
  const float ss = wave_sum_uniform(ss_lane);
  return 1.f / sqrtf(ss / static_cast<float>(hidden) + eps);
}
// bf16(w * bf16(v * inv)) for one chunk, as packed bf16.
__device__ __forceinline__ u32x4 norm_chunk(u32x4 a, u32x4 wv, float inv) {
  u32x4 o;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float n0 = bf2f(f2bf(bf2f(static_cast<uint16_t>(a[w] & 0xffffu)) * inv));
    const float n1 = bf2f(f2bf(bf2f(static_cast<uint16_t>(a[w] >> 16)) * inv));
    o[w] = pack_bf16x2(bf2f(static_cast<uint16_t>(wv[w] & 0xffffu)) * n0,
                       bf2f(static_cast<uint16_t>(wv[w] >> 16)) * n1);
  }
  return o;
}

// One workgroup per row of `hidden` bf16 values (hidden % 8 == 0, <= 8192).
// With delta, the row first becomes bf16(x + delta) and is written back.
// Wavefront 0 computes the row statistics in the canonical order above.
__global__ __launch_bounds__(kRowThreads) void add_rms_norm_kernel(
    uint16_t* __restrict__ x, const uint16_t* __restrict__ delta,
    const uint16_t* __restrict__ weight, uint16_t* __restrict__ out, int hidden, float eps) {
  __shared__ float s_inv;
  const size_t row = blockIdx.x;
  uint16_t* xr = x + row * hidden;
  const uint16_t* dr = delta ? delta + row * hidden : nullptr;
  uint16_t* orow = out + row * hidden;
  const int chunks = hidden / 8;
  if (threadIdx.x < kWave) {
    float ss = 0.f;
    for (int c = threadIdx.x; c < chunks; c += kWave) ss = chunk_sumsq(add_chunk(xr, dr, 8 * c), ss);
    const float inv = rms_inv(ss, hidden, eps);
    if (threadIdx.x == 0) s_inv = inv;
  }
  __syncthreads();  // every read of the unmodified row is done
  const float inv = s_inv;
  for (int c = threadIdx.x; c < chunks; c += kRowThreads) {
    const u32x4 a = add_chunk(xr, dr, 8 * c);
    if (dr) *reinterpret_cast<u32x4*>(xr + 8 * c) = a;
    const u32x4 wv = *reinterpret_cast<const u32x4*>(weight + 8 * c);
    *reinterpret_cast<u32x4*>(orow + 8 * c) = norm_chunk(a, wv, inv);
  }
}

// qkv [B * L, (nq + 2 nkv) * hd] -> q [B, nq, L, hd], k and v [B, nkv, L, hd];
// q and k rotated (rotate-half) with the fp32 tables cos/sin [L, hd]
// (cos[i] = cos[i + hd/2]).  One thread per (row, head, dim pair).
__global__ __launch_bounds__(kRowThreads) void rope_split_kernel(
    const uint16_t* __restrict__ qkv, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, uint16_t* __restrict__ q, uint16_t* __restrict__ k,
    uint16_t* __restrict__ v, int B, int L, int nq, int nkv, int hd) {
  const int half = hd / 2;
  const int heads = nq + 2 * nkv;
  const long long idx = static_cast<long long>(blockIdx.x) * kRowThreads + threadIdx.x;
  const long long total = static_cast<long long>(B) * L * heads * half;
  if (idx >= total) return;
  const int i = static_cast<int>(idx % half);
  const long long rh = idx / half;
  const int h = static_cast<int>(rh % heads);
  const int row = static_cast<int>(rh / heads);
  const int b = row / L;
  const int l = row - b * L;
  const uint16_t* src = qkv + (static_cast<size_t>(row) * heads + h) * hd;
  const float x1 = bf2f(src[i]);
  const float x2 = bf2f(src[i + half]);
  uint16_t* dst;
  if (h < nq) {
    dst = q + ((static_cast<size_t>(b) * nq + h) * L + l) * hd;
  } else if (h < nq + nkv) {
    dst = k + ((static_cast<size_t>(b) * nkv + (h - nq)) * L + l) * hd;
  } else {
    dst = v + ((static_cast<size_t>(b) * nkv + (h - nq - nkv)) * L + l) * hd;
    dst[i] = src[i];
    dst[i + half] = src[i + half];
    return;
  }
  {
    // x * cos + rotate_half(x) * sin with each product and the sum rounded as
    // separate fp32 ops (no fused multiply-add), as torch evaluates it
#pragma clang fp contract(off)
    const float c0 = cos_t[static_cast<size_t>(l) * hd + i];
    const float s0 = sin_t[static_cast<size_t>(l) * hd + i];
    const float c1 = cos_t[static_cast<size_t>(l) * hd + i + half];
    const float s1 = sin_t[static_cast<size_t>(l) * hd + i + half];
    const float a0 = x1 * c0;
    const float b0 = -x2 * s0;
    const float a1 = x2 * c1;
    const float b1 = x1 * s1;
    dst[i] = f2bf(a0 + b0);
    dst[i + half] = f2bf(a1 + b1);
  }
}

// gate_up [rows, 2 I] (gate first) -> out [rows, I]; 8 values per thread.
__global__ __launch_bounds__(kRowThreads) void silu_mul_kernel(
    const uint16_t* __restrict__ gate_up, uint16_t* __restrict__ out, int rows, int inter) {
  const long long idx = static_cast<long long>(blockIdx.x) * kRowThreads + threadIdx.x;
  const int per_row = inter / 8;
  if (idx >= static_cast<long long>(rows) * per_row) return;
  const int row = static_cast<int>(idx / per_row);
  const int c = static_cast<int>(idx - static_cast<long long>(row) * per_row) * 8;
  const uint16_t* gr = gate_up + static_cast<size_t>(row) * 2 * inter;
  const u32x4 g = *reinterpret_cast<const u32x4*>(gr + c);
  const u32x4 u = *reinterpret_cast<const u32x4*>(gr + inter + c);
  u32x4 o;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    float r[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const float gv = bf2f(static_cast<uint16_t>(e ? g[w] >> 16 : g[w] & 0xffffu));
      const float uv = bf2f(static_cast<uint16_t>(e ? u[w] >> 16 : u[w] & 0xffffu));
      const float s = bf2f(f2bf(gv / (1.f + expf(-gv))));
      r[e] = s * uv;
    }
    o[w] = pack_bf16x2(r[0], r[1]);
  }
  *reinterpret_cast<u32x4*>(out + static_cast<size_t>(row) * inter + c) = o;
}

// One-token projection: y[r] = bf16(sum_k W[r][k] x[k]) with W [N, K] bf16
// row-major (a torch Linear weight), x [K], fp32 sums.  Decode runs these at
// one row of activations, where a GEMM tiling reads the weights at a fraction
// of the bandwidth; here each wavefront takes 4 weight rows, every lane holds
// KC 16-byte chunks of x (chunks lane, lane + 64, ...) in registers and reads
// the same chunks of its 4 rows (coalesced 1 KB per row per step, all 4 x KC
// loads in flight, non-temporal: each weight byte is used once per token),
// and the 4 dot products are summed across the lanes.
// SWIGLU: W is the fused [gate; up] weight [2I, K] and y [I] is
// bf16(bf16(silu(g)) * u) with g, u the bf16-rounded projections of rows r
// and I + r -- the projection followed by silu_mul_kernel's math; a wave then
// takes 2 gate and the 2 matching up rows.
// The projection input of one lane: chunks lane, lane + 64, ... of x (and of
// delta and ln when the residual-add + RMSNorm prologue is on).  The raw
// loads are issued first, then the weight loads, then the input is finished
// while the weights are still in flight: the prologue costs no second memory
// round trip.
template <int KC>
struct GemvInput {
  u32x4 x[KC], d[KC], ln[KC];
};

template <int KC, bool NORM>
__device__ __forceinline__ void gemv_fetch_x(const uint16_t* __restrict__ x,
                                             const uint16_t* __restrict__ delta,
                                             const uint16_t* __restrict__ ln, int chunks, int lane,
                                             GemvInput<KC>& in) {
  // every lane loads (lanes past the row reread its last chunk and are
  // masked later): straight-line loads let the compiler wait for exactly
  // the ones it needs
  const uint16_t* d = delta ? delta : x;
#pragma unroll
  for (int j = 0; j < KC; ++j) {
    const int c = min(lane + kWave * j, chunks - 1);
    in.x[j] = *reinterpret_cast<const u32x4*>(x + 8 * c);
    if (NORM) {
      in.d[j] = *reinterpret_cast<const u32x4*>(d + 8 * c);
      in.ln[j] = *reinterpret_cast<const u32x4*>(ln + 8 * c);
    }
  }
}

// Plain (ln == nullptr): the input is x.  Otherwise it is add_rms_norm_kernel's
// output, bit for bit: v = bf16(x + delta) (x without delta), input =
// bf16(ln * bf16(v * rsqrt(mean(v^2) + eps))), with v also stored to x_out
// (when given) by one wavefront of the grid.
template <int KC, bool NORM>
__device__ __forceinline__ void gemv_finish_x(const GemvInput<KC>& in, bool has_delta, float eps,
                                              uint16_t* __restrict__ x_out, bool writer, int k,
                                              int lane, float (&xv)[KC][8]) {
  const int chunks = k / 8;
  u32x4 v[KC];
#pragma unroll
  for (int j = 0; j < KC; ++j) {
    v[j] = lane + kWave * j < chunks ? in.x[j] : u32x4{0u, 0u, 0u, 0u};
    if (NORM) {
      // the sum is formed either way and selected: a branch here lets the
      // compiler sink the delta loads into it, behind a wait for the weights
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float lo = bf2f(static_cast<uint16_t>(v[j][w] & 0xffffu)) +
                         bf2f(static_cast<uint16_t>(in.d[j][w] & 0xffffu));
        const float hi = bf2f(static_cast<uint16_t>(v[j][w] >> 16)) +
                         bf2f(static_cast<uint16_t>(in.d[j][w] >> 16));
        const uint32_t sum = pack_bf16x2(lo, hi);
        v[j][w] = has_delta ? sum : v[j][w];
      }
    }
  }
  if (NORM) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < KC; ++j) {
      if (lane + kWave * j < chunks) ss = chunk_sumsq(v[j], ss);
    }
    const float inv = rms_inv(ss, k, eps);
#pragma unroll
    for (int j = 0; j < KC; ++j) {
      const int c = lane + kWave * j;
      if (c < chunks) {
        if (writer && x_out) *reinterpret_cast<u32x4*>(x_out + 8 * c) = v[j];
        v[j] = norm_chunk(v[j], in.ln[j], inv);
      }
    }
  }
#pragma unroll
  for (int j = 0; j < KC; ++j) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      xv[j][2 * e] = bf2f(static_cast<uint16_t>(v[j][e] & 0xffffu));
      xv[j][2 * e + 1] = bf2f(static_cast<uint16_t>(v[j][e] >> 16));
    }
  }
}

// Loads of 4 weight rows (non-temporal: each weight byte is read once per
// token).
template <int KC>
__device__ __forceinline__ void gemv_fetch_w(const uint16_t* __restrict__ w, const int (&rows)[4],
                                             int k, int chunks, int lane, u32x4 (&wv)[4][KC]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint16_t* wr = w + static_cast<size_t>(rows[i]) * k;
#pragma unroll
    for (int j = 0; j < KC; ++j) {
      const int c = min(lane + kWave * j, chunks - 1);  // see gemv_fetch_x
      wv[i][j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr + 8 * c));
    }
  }
}

// Dot products of the 4 weight rows with x, summed over the wave (every lane
// gets the 4 sums); chunks past the row (lane + 64 j >= chunks) add nothing.
template <int KC>
__device__ __forceinline__ void gemv_dot4(const u32x4 (&wv)[4][KC], const float (&xv)[KC][8],
                                          int chunks, int lane, float (&acc)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < KC; ++j) {
      if (lane + kWave * j >= chunks) continue;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s += bf2f(static_cast<uint16_t>(wv[i][j][e] & 0xffffu)) * xv[j][2 * e];
        s += bf2f(static_cast<uint16_t>(wv[i][j][e] >> 16)) * xv[j][2 * e + 1];
      }
    }
    acc[i] = wave_sum_uniform(s);
  }
}

// One wavefront's projection of rows[0..3]: input fetch, weight fetch, input
// finish, dot products.
template <int KC, bool NORM>
__device__ __forceinline__ void gemv_rows(const uint16_t* __restrict__ w,
                                          const uint16_t* __restrict__ x,
                                          const uint16_t* __restrict__ delta,
                                          const uint16_t* __restrict__ ln, float eps,
                                          uint16_t* __restrict__ x_out, bool writer,
                                          const int (&rows)[4], int k, int lane,
                                          float (&acc)[4]) {
  const int chunks = k / 8;
  GemvInput<KC> in;
  gemv_fetch_x<KC, NORM>(x, delta, ln, chunks, lane, in);
  u32x4 wv[4][KC];
  gemv_fetch_w<KC>(w, rows, k, chunks, lane, wv);
  float xv[KC][8];
  gemv_finish_x<KC, NORM>(in, delta != nullptr, eps, x_out, writer, k, lane, xv);
  gemv_dot4<KC>(wv, xv, chunks, lane, acc);
}

template <int KC, bool SWIGLU, bool NORM>
__global__ __launch_bounds__(kRowThreads) void gemv_kernel(
    const uint16_t* __restrict__ w, const uint16_t* __restrict__ x,
    const uint16_t* __restrict__ delta, const uint16_t* __restrict__ ln, float eps,
    uint16_t* __restrict__ x_out, uint16_t* __restrict__ y, int n, int k) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = blockIdx.x * (kRowThreads / kWave) + (threadIdx.x / kWave);
  // rows of this wave: plain 4r..4r+3; SwiGLU gate 2r, 2r+1 and up n + 2r, n + 2r + 1
  // (rows past the end read row `first` again; their sums are not stored)
  const int first = SWIGLU ? 2 * wave : 4 * wave;
  if (first >= n) return;
  int rows[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int local = SWIGLU ? (i & 1) : i;
    const int r = first + local < n ? first + local : first;
    rows[i] = SWIGLU && i >= 2 ? n + r : r;
  }
  float acc[4];
  gemv_rows<KC, NORM>(w, x, delta, ln, eps, x_out, wave == 0, rows, k, lane, acc);
  if (lane == 0) {
    if (SWIGLU) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        if (first + i < n) {
          const float g = bf2f(f2bf(acc[i]));
          const float u = bf2f(f2bf(acc[2 + i]));
          const float sg = bf2f(f2bf(g / (1.f + expf(-g))));
          y[first + i] = f2bf(sg * u);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (first + i < n) y[first + i] = f2bf(acc[i]);
      }
    }
  }
}

// The fused qkv projection of one decode token [(nq + 2 nkv) hd, k] . x, the
// RoPE of its q and k heads and the page write of k and v: wave w of head h
// takes rows d, d + 1, d + hd/2, d + hd/2 + 1 of the head (d = 2 (w % (hd/4))),
// so both halves of each rotated pair are in the wave.  The projection is
// rounded to bf16 before the rotation and the rotation rounds each product
// and the sum (rope_split_kernel's formula), so q, k and v are bit-identical
// to the projection, voom_rope_split and voom_append_kv in sequence.  k and v
// land at position *pos of the sequence through its block-table row, in the
// pool layouts of voom_append_kv.
template <int KC, bool NORM>
__global__ __launch_bounds__(kRowThreads) void qkv_rope_append_kernel(
    const uint16_t* __restrict__ w, const uint16_t* __restrict__ x,
    const uint16_t* __restrict__ delta, const uint16_t* __restrict__ ln, float eps,
    uint16_t* __restrict__ x_out,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t, uint16_t* __restrict__ q,
    uint16_t* __restrict__ k_pool, uint16_t* __restrict__ v_pool,
    const int32_t* __restrict__ table_row, const int32_t* __restrict__ pos_ptr, int nq, int nkv,
    int hd, int k, int pt_shift, int max_pages, int num_slots, int rope_rows) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = blockIdx.x * (kRowThreads / kWave) + (threadIdx.x / kWave);
  const int half = hd / 2;
  const int per_head = half / 2;
  const int h = wave / per_head;
  if (h >= nq + 2 * nkv) return;
  const int d = 2 * (wave - h * per_head);
  const int rows[4] = {h * hd + d, h * hd + d + 1, h * hd + d + half, h * hd + d + half + 1};
  float acc[4];
  gemv_rows<KC, NORM>(w, x, delta, ln, eps, x_out, wave == 0, rows, k, lane, acc);
  if (lane >= 2) return;
  // lane e handles dims d + e and d + e + half
  const float x1 = bf2f(f2bf(acc[lane]));
  const float x2 = bf2f(f2bf(acc[2 + lane]));
  const int i = d + lane;
  uint16_t o1, o2;
  if (h < nq + nkv) {
#pragma clang fp contract(off)
    if (rope_rows > 0) {  // tables: the row of the token's position (clamped)
      const int r = min(max(*pos_ptr, 0), rope_rows - 1);
      cos_t += static_cast<size_t>(r) * hd;
      sin_t += static_cast<size_t>(r) * hd;
    }
    const float a0 = x1 * cos_t[i];
    const float b0 = -x2 * sin_t[i];
    const float a1 = x2 * cos_t[i + half];
    const float b1 = x1 * sin_t[i + half];
    o1 = f2bf(a0 + b0);
    o2 = f2bf(a1 + b1);
  } else {
    o1 = f2bf(x1);
    o2 = f2bf(x2);
  }
  if (h < nq) {
    q[static_cast<size_t>(h) * hd + i] = o1;
    q[static_cast<size_t>(h) * hd + i + half] = o2;
    return;
  }
  const int pos = *pos_ptr;
  if (pos < 0) return;
  const int page = pos >> pt_shift;
  if (page >= max_pages) return;
  const int slot = table_row[page];
  if (static_cast<unsigned>(slot) >= static_cast<unsigned>(num_slots)) return;
  const int off = pos & ((1 << pt_shift) - 1);
  const bool is_k = h < nq + nkv;
  const int kvh = is_k ? h - nq : h - nq - nkv;
  const size_t head_page = static_cast<size_t>(slot) * nkv + kvh;
  if (is_k) {
    uint16_t* kr = k_pool + ((head_page << pt_shift) + off) * hd;
    kr[i] = o1;
    kr[i + half] = o2;
  } else {
    const int vb_shift = pt_shift < 5 ? pt_shift : 5;
    const size_t blk = (head_page << (pt_shift - vb_shift)) + (off >> vb_shift);
    const int col = off & ((1 << vb_shift) - 1);
    v_pool[((blk * hd + i) << vb_shift) + col] = o1;
    v_pool[((blk * hd + i + half) << vb_shift) + col] = o2;
  }
}

// Greedy sampling key of one bf16 logit: larger keys are larger logits, and
// among equal logits the lower index; -0 counts as +0 and every NaN as the
// largest value, as torch.argmax orders them.
__device__ __forceinline__ uint64_t logit_key(uint16_t bits, int idx) {
  if ((bits & 0x7fffu) == 0) bits = 0;
  if ((bits & 0x7f80u) == 0x7f80u && (bits & 0x7fu)) bits = 0x7fc0u;
  const uint32_t f = static_cast<uint32_t>(bits) << 16;
  const uint32_t ordered = f ^ ((f >> 31) ? 0xffffffffu : 0x80000000u);
  return (static_cast<uint64_t>(ordered) << 32) | (0xffffffffu - static_cast<uint32_t>(idx));
}

// The lm_head projection of one row with its argmax: each wavefront projects
// 4 vocabulary rows (the GEMV above, optional final-norm prologue), keys its
// bf16 logits and the workgroup's best key goes to keys[blockIdx.x].  No
// logits are stored.
template <int KC, bool NORM>
__global__ __launch_bounds__(kRowThreads) void gemv_argmax_kernel(
    const uint16_t* __restrict__ w, const uint16_t* __restrict__ x,
    const uint16_t* __restrict__ delta, const uint16_t* __restrict__ ln, float eps,
    uint64_t* __restrict__ keys, int n, int k) {
  __shared__ uint64_t s_key[kRowThreads / kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int wib = threadIdx.x / kWave;
  const int first = 4 * (blockIdx.x * (kRowThreads / kWave) + wib);
  uint64_t best = 0;  // below every real key
  if (first < n) {  // uniform over the wavefront
    int rows[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) rows[i] = first + i < n ? first + i : first;
    float acc[4];
    gemv_rows<KC, NORM>(w, x, delta, ln, eps, nullptr, false, rows, k, lane, acc);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (first + i < n) {
        const uint64_t key = logit_key(f2bf(acc[i]), first + i);
        best = key > best ? key : best;
      }
    }
  }
  if (lane == 0) s_key[wib] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t m = s_key[0];
#pragma unroll
    for (int i = 1; i < kRowThreads / kWave; ++i) m = s_key[i] > m ? s_key[i] : m;
    keys[blockIdx.x] = m;
  }
}

// One workgroup: the best of nkeys keys; its index goes to token[0] and,
// when given, token_copy[0].
__global__ __launch_bounds__(kRowThreads) void argmax_finish_kernel(
    const uint64_t* __restrict__ keys, int nkeys, int64_t* __restrict__ token,
    int64_t* __restrict__ token_copy) {
  __shared__ uint64_t s_key[kRowThreads];
  constexpr int kPer = 16;  // loads in flight per thread
  uint64_t m = 0;
  for (int base = 0; base < nkeys; base += kPer * kRowThreads) {
    uint64_t v[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i = base + j * kRowThreads + threadIdx.x;
      v[j] = i < nkeys ? keys[i] : 0;
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) m = v[j] > m ? v[j] : m;
  }
  s_key[threadIdx.x] = m;
  __syncthreads();
  for (int h = kRowThreads / 2; h >= 1; h >>= 1) {
    if (threadIdx.x < h) {
      const uint64_t o = s_key[threadIdx.x + h];
      if (o > s_key[threadIdx.x]) s_key[threadIdx.x] = o;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const int64_t idx = static_cast<int64_t>(0xffffffffu - static_cast<uint32_t>(s_key[0]));
    token[0] = idx;
    if (token_copy) token_copy[0] = idx;
  }
}

template <bool SWIGLU, bool NORM>
void launch_gemv_kc(int kc, dim3 grid, const uint16_t* w, const uint16_t* x, const uint16_t* delta,
                    const uint16_t* ln, float eps, uint16_t* x_out, uint16_t* y, int n, int k,
                    hipStream_t stream) {
#define VOOM_GEMV(KC_)                                                                       \
  hipLaunchKernelGGL((gemv_kernel<KC_, SWIGLU, NORM>), grid, dim3(kRowThreads), 0, stream, w, x, \
                     delta, ln, eps, x_out, y, n, k)
  switch (kc) {
    case 1: VOOM_GEMV(1); break;
    case 2: VOOM_GEMV(2); break;
    case 3: VOOM_GEMV(3); break;
    default: VOOM_GEMV(4); break;
  }
#undef VOOM_GEMV
}

template <bool SWIGLU>
int launch_gemv(const uint16_t* w, const uint16_t* x, const uint16_t* delta, const uint16_t* ln,
                float eps, uint16_t* x_out, uint16_t* y, int n, int k, hipStream_t stream) {
  const int rows_per_wave = SWIGLU ? 2 : 4;
  const long long waves = (static_cast<long long>(n) + rows_per_wave - 1) / rows_per_wave;
  const dim3 grid(static_cast<unsigned>((waves + kRowThreads / kWave - 1) / (kRowThreads / kWave)));
  const int kc = (k / 8 + kWave - 1) / kWave;
  if (ln)
    launch_gemv_kc<SWIGLU, true>(kc, grid, w, x, delta, ln, eps, x_out, y, n, k, stream);
  else
    launch_gemv_kc<SWIGLU, false>(kc, grid, w, x, delta, ln, eps, x_out, y, n, k, stream);
  return VOOM_LAUNCH_CHECK("gemv: kernel launch");
}

}  // namespace
}  // namespace voom

using namespace voom;

namespace {
// Shared checks of the residual-add + RMSNorm prologue arguments.
int check_norm_prologue(const char* who, const void* x, const void* delta, const void* ln_weight,
                        const void* x_out) {
  VOOM_REQUIRE(ln_weight != nullptr || (delta == nullptr && x_out == nullptr),
               "%s: delta and x_out need ln_weight", who);
  VOOM_REQUIRE(x_out == nullptr || (x_out != x && x_out != delta),
               "%s: x_out must not alias x or delta", who);
  VOOM_REQUIRE(reinterpret_cast<uintptr_t>(delta) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(ln_weight) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(x_out) % 16 == 0,
               "%s: delta, ln_weight and x_out must be 16-byte aligned", who);
  return 0;
}
}  // namespace

extern "C" int voom_qkv_rope_append(const void* w_qkv, const void* x, const void* delta,
                                    const void* ln_weight, float eps, void* x_out,
                                    const float* cos_row, const float* sin_row, void* q,
                                    void* k_pool, void* v_pool, const int32_t* table_row,
                                    const int32_t* position, int num_q_heads, int num_kv_heads,
                                    int head_dim, int k, int page_tokens, int max_pages,
                                    int num_slots, int rope_rows, hipStream_t stream) {
  const char* who = "qkv_rope_append";
  VOOM_REQUIRE(w_qkv && x && cos_row && sin_row && q && k_pool && v_pool && table_row && position,
               "%s: null pointer argument", who);
  if (int rc = check_norm_prologue(who, x, delta, ln_weight, x_out)) return rc;
  VOOM_REQUIRE(num_q_heads > 0 && num_kv_heads > 0 && head_dim > 0 && head_dim % 4 == 0,
               "%s: bad head geometry", who);
  VOOM_REQUIRE(k > 0 && k % 8 == 0 && k <= 8 * kWave * 4,
               "%s: k %d must be a positive multiple of 8 up to %d", who, k, 8 * kWave * 4);
  VOOM_REQUIRE(is_pow2(page_tokens) && page_tokens <= 4096 && max_pages > 0 && num_slots > 0,
               "%s: bad page geometry", who);
  VOOM_REQUIRE(rope_rows >= 0, "%s: rope_rows must be >= 0", who);
  VOOM_REQUIRE(reinterpret_cast<uintptr_t>(w_qkv) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(x) % 16 == 0,
               "%s: weight and x must be 16-byte aligned", who);
  const long long waves = static_cast<long long>(num_q_heads + 2 * num_kv_heads) * (head_dim / 4);
  const dim3 grid(static_cast<unsigned>((waves + kRowThreads / kWave - 1) / (kRowThreads / kWave)));
  const int kc = (k / 8 + kWave - 1) / kWave;
  const auto* wq = static_cast<const uint16_t*>(w_qkv);
  const auto* xv = static_cast<const uint16_t*>(x);
  auto* qo = static_cast<uint16_t*>(q);
  auto* kp = static_cast<uint16_t*>(k_pool);
  auto* vp = static_cast<uint16_t*>(v_pool);
  const auto* dv = static_cast<const uint16_t*>(delta);
  const auto* lw = static_cast<const uint16_t*>(ln_weight);
  auto* xo = static_cast<uint16_t*>(x_out);
  const int pts = ilog2(page_tokens);
#define VOOM_QRA_N(KC_, NORM_)                                                             \
  hipLaunchKernelGGL((qkv_rope_append_kernel<KC_, NORM_>), grid, dim3(kRowThreads), 0, stream, \
                     wq, xv, dv, lw, eps, xo, cos_row, sin_row, qo, kp, vp, table_row,         \
                     position, num_q_heads, num_kv_heads, head_dim, k, pts, max_pages,         \
                     num_slots, rope_rows)
#define VOOM_QRA(KC_)      \
  if (lw)                  \
    VOOM_QRA_N(KC_, true); \
  else                     \
    VOOM_QRA_N(KC_, false)
  switch (kc) {
    case 1: VOOM_QRA(1); break;
    case 2: VOOM_QRA(2); break;
    case 3: VOOM_QRA(3); break;
    default: VOOM_QRA(4); break;
  }
#undef VOOM_QRA
#undef VOOM_QRA_N
  return VOOM_LAUNCH_CHECK("qkv_rope_append: kernel launch");
}

extern "C" int voom_gemv_bf16(const void* weight, const void* x, void* y, int n, int k,
                              int swiglu, hipStream_t stream) {
  return voom_add_rms_norm_gemv(x, nullptr, nullptr, 0.f, nullptr, weight, y, n, k, swiglu,
                                stream);
}

extern "C" int voom_add_rms_norm_gemv(const void* x, const void* delta, const void* ln_weight,
                                      float eps, void* x_out, const void* weight, void* y, int n,
                                      int k, int swiglu, hipStream_t stream) {
  const char* who = "gemv_bf16";
  VOOM_REQUIRE(weight && x && y, "%s: null pointer argument", who);
  if (int rc = check_norm_prologue(who, x, delta, ln_weight, x_out)) return rc;
  VOOM_REQUIRE(n > 0 && k > 0 && k % 8 == 0 && k <= 8 * kWave * 4,
               "%s: k %d must be a positive multiple of 8 up to %d", who, k, 8 * kWave * 4);
  VOOM_REQUIRE(n < (1 << 28), "%s: n %d too large", who, n);
  VOOM_REQUIRE(reinterpret_cast<uintptr_t>(weight) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(y) % 2 == 0,
               "%s: weight and x must be 16-byte aligned", who);
  const auto* w = static_cast<const uint16_t*>(weight);
  const auto* xv = static_cast<const uint16_t*>(x);
  auto* yv = static_cast<uint16_t*>(y);
  const auto* dv = static_cast<const uint16_t*>(delta);
  const auto* lw = static_cast<const uint16_t*>(ln_weight);
  auto* xo = static_cast<uint16_t*>(x_out);
  return swiglu ? launch_gemv<true>(w, xv, dv, lw, eps, xo, yv, n, k, stream)
                : launch_gemv<false>(w, xv, dv, lw, eps, xo, yv, n, k, stream);
}

extern "C" int voom_lm_head_argmax(const void* x, const void* delta, const void* ln_weight,
                                   float eps, const void* weight, int n, int k, void* workspace,
                                   size_t ws_bytes, int64_t* token, int64_t* token_copy,
                                   hipStream_t stream) {
  const char* who = "lm_head_argmax";
  VOOM_REQUIRE(x && weight && workspace && token, "%s: null pointer argument", who);
  if (int rc = check_norm_prologue(who, x, delta, ln_weight, nullptr)) return rc;
  VOOM_REQUIRE(n > 0 && n < (1 << 28) && k > 0 && k % 8 == 0 && k <= 8 * kWave * 4,
               "%s: k %d must be a positive multiple of 8 up to %d", who, k, 8 * kWave * 4);
  VOOM_REQUIRE(reinterpret_cast<uintptr_t>(weight) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(workspace) % 8 == 0,
               "%s: weight and x must be 16-byte aligned, workspace 8-byte", who);
  const int rows_per_block = 4 * (kRowThreads / kWave);
  const int blocks = (n + rows_per_block - 1) / rows_per_block;
  VOOM_REQUIRE(ws_bytes >= static_cast<size_t>(blocks) * 8, "%s: workspace needs %d bytes", who,
               blocks * 8);
  const auto* w = static_cast<const uint16_t*>(weight);
  const auto* xv = static_cast<const uint16_t*>(x);
  const auto* dv = static_cast<const uint16_t*>(delta);
  const auto* lw = static_cast<const uint16_t*>(ln_weight);
  auto* keys = static_cast<uint64_t*>(workspace);
  const int kc = (k / 8 + kWave - 1) / kWave;
#define VOOM_GA(KC_, NORM_)                                                                   \
  hipLaunchKernelGGL((gemv_argmax_kernel<KC_, NORM_>), dim3(blocks), dim3(kRowThreads), 0,      \
                     stream, w, xv, dv, lw, eps, keys, n, k)
#define VOOM_GA_KC(KC_) \
  if (lw)               \
    VOOM_GA(KC_, true); \
  else                  \
    VOOM_GA(KC_, false)
  switch (kc) {
    case 1: VOOM_GA_KC(1); break;
    case 2: VOOM_GA_KC(2); break;
    case 3: VOOM_GA_KC(3); break;
    default: VOOM_GA_KC(4); break;
  }
#undef VOOM_GA_KC
#undef VOOM_GA
  if (int rc = VOOM_LAUNCH_CHECK("lm_head_argmax: projection launch")) return rc;
  hipLaunchKernelGGL(argmax_finish_kernel, dim3(1), dim3(kRowThreads), 0, stream, keys, blocks,
                     token, token_copy);
  return VOOM_LAUNCH_CHECK("lm_head_argmax: finish launch");
}

extern "C" int voom_add_rms_norm(void* x, const void* delta, const void* weight, void* out,
                                 int rows, int hidden, float eps, hipStream_t stream) {
  const char* who = "add_rms_norm";
  VOOM_REQUIRE(x && weight && out, "%s: null pointer argument", who);
  VOOM_REQUIRE(rows > 0 && hidden > 0 && hidden % 8 == 0 && hidden <= 8192,
               "%s: hidden %d must be a multiple of 8 up to 8192", who, hidden);
  VOOM_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(weight) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(out) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(delta) % 16 == 0,
               "%s: tensors must be 16-byte aligned", who);
  hipLaunchKernelGGL(add_rms_norm_kernel, dim3(static_cast<unsigned>(rows)), dim3(kRowThreads),
                     0, stream, static_cast<uint16_t*>(x), static_cast<const uint16_t*>(delta),
                     static_cast<const uint16_t*>(weight), static_cast<uint16_t*>(out), hidden,
                     eps);
  return VOOM_LAUNCH_CHECK("add_rms_norm: kernel launch");
}

extern "C" int voom_rope_split(const void* qkv, const float* cos_table, const float* sin_table,
                               void* q, void* k, void* v, int batch, int seq, int num_q_heads,
                               int num_kv_heads, int head_dim, hipStream_t stream) {
  const char* who = "rope_split";
  VOOM_REQUIRE(qkv && cos_table && sin_table && q && k && v, "%s: null pointer argument", who);
  VOOM_REQUIRE(batch > 0 && seq > 0 && num_q_heads > 0 && num_kv_heads > 0 && head_dim > 0 &&
                   head_dim % 2 == 0,
               "%s: bad geometry", who);
  const long long total =
      static_cast<long long>(batch) * seq * (num_q_heads + 2 * num_kv_heads) * (head_dim / 2);
  VOOM_REQUIRE(total < (1LL << 40), "%s: too large", who);
  hipLaunchKernelGGL(rope_split_kernel,
                     dim3(static_cast<unsigned>((total + kRowThreads - 1) / kRowThreads)),
                     dim3(kRowThreads), 0, stream, static_cast<const uint16_t*>(qkv), cos_table,
                     sin_table, static_cast<uint16_t*>(q), static_cast<uint16_t*>(k),
                     static_cast<uint16_t*>(v), batch, seq, num_q_heads, num_kv_heads, head_dim);
  return VOOM_LAUNCH_CHECK("rope_split: kernel launch");
}

extern "C" int voom_silu_mul(const void* gate_up, void* out, int rows, int intermediate,
                             hipStream_t stream) {
  const char* who = "silu_mul";
  VOOM_REQUIRE(gate_up && out, "%s: null pointer argument", who);
  VOOM_REQUIRE(rows > 0 && intermediate > 0 && intermediate % 8 == 0,
               "%s: intermediate %d must be a positive multiple of 8", who, intermediate);
  VOOM_REQUIRE(reinterpret_cast<uintptr_t>(gate_up) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(out) % 16 == 0,
               "%s: tensors must be 16-byte aligned", who);
  const long long total = static_cast<long long>(rows) * (intermediate / 8);
  hipLaunchKernelGGL(silu_mul_kernel,
                     dim3(static_cast<unsigned>((total + kRowThreads - 1) / kRowThreads)),
                     dim3(kRowThreads), 0, stream, static_cast<const uint16_t*>(gate_up),
                     static_cast<uint16_t*>(out), rows, intermediate);
  return VOOM_LAUNCH_CHECK("silu_mul: kernel launch");
}
