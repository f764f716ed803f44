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
// Decomposition: one workgroup (8 wavefronts, 2 per SIMD) per (sequence,
// token range, group of 64 heads; 32 when the head count is not a multiple of
// 64).  The head groups of a range are placed on the same XCD so the latent
// tiles they all read are served from that XCD's L2; with 64 heads a tile
// pulled into LDS serves twice as many heads as with 32.
// Per 64-token tile: buffer loads deliver the tile straight into LDS (no
// register staging; the next tile streams into the second buffer while the
// current one is used).  The 4 token tiles x 4 head tiles of scores are split
// over the wavefronts (2 token tiles of one head tile each), with the latent
// rows of a k-step read two steps ahead of their MFMAs; the tile maximum of a
// head is combined through LDS, P is written to LDS in bf16, and wavefront w
// accumulates dims 64w..64w+63 of out^T for all heads of the group
// (accumulators stay in registers for the whole range).  The softmax
// normaliser is kept per lane and summed across lanes and wavefronts once,
// after the last tile.  The C^T operand comes from the token-major tile through
// ds_read_b64_tr_b16: in each 16-lane group, lane l receives element l%4 of
// the 8-byte rows addressed by lanes 4c + l/4 (c = 0..3), so two transposed
// reads give a lane the 8 tokens of one latent dim.  LDS rows are unpadded
// (72 sixteen-byte chunks) with chunk bits 1-2 XOR-swizzled by row bits 1-3
// (tile_swizzle), which keeps both the row reads of the score MFMA and the
// transposed reads free of bank conflicts.
#include "common.h"

namespace voom {
namespace {

constexpr int kThreads = 256;
constexpr int kLat = 576;          // kv_lora_rank 512 + rope dim 64
constexpr int kC = 512;
constexpr int kTile = 64;          // tokens per tile
constexpr int kChunksPerRow = kLat * 2 / 16;  // 72 sixteen-byte chunks per token
constexpr int kRow = kChunksPerRow * 8;        // LDS row stride in bf16 elements
constexpr int kTileChunks = kTile * kChunksPerRow;  // 4608 = 72 x 64
constexpr int kLoadsPerTile = kTileChunks / 64;     // 72 wave-wide 16-byte loads
constexpr int kQSteps = kLat / 32;  // 18 k-steps of the score MFMA
constexpr int kHgTile = 16;  // per-head products: output columns per 16x16x32 MFMA tile
constexpr int kHgStep = 32;  // per-head products: k per MFMA
constexpr int kPRow = kTile + 16;   // P row stride (160 B = 10 chunks): the 16 head rows
                                    // of a 32-lane read phase fall on distinct banks

// LDS tile swizzle: chunk c of token row r is stored at chunk c ^ tile_swizzle(r)
// of the row (row bits 1-3 flip chunk bits 1-2; chunks 64..71 stay in place
// as a group).  Measured on gfx950: ds_read_b128 serves 32 lanes per phase
// in 8-byte halves over 128 four-byte banks, ds_read_b64_tr_b16 32 lanes per
// phase over 64 banks.  With this swizzle the score reads (rows 16x + 0..15,
// chunks 4s + g) and the transposed reads (rows 8g + 0..3 of two lane groups,
// 32 bytes each) both touch every bank once per phase; a row padded to 73
// chunks cost 4 and 2 conflict cycles per instruction respectively.
__device__ __forceinline__ int tile_swizzle(int r) {
  return ((((r >> 1) ^ (r >> 2)) & 1) << 1) | (((r >> 3) & 1) << 2);
}

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

struct MlaArgs {
  const uint16_t* __restrict__ q;        // [B, H, 576]
  const uint16_t* __restrict__ lat;      // [slots, PT, 576]
  const int32_t* __restrict__ table;     // [B, max_pages]
  const int32_t* __restrict__ ctx_lens;  // [B] (sparse: selected counts)
  float* __restrict__ part_o;            // [B, NR, H, 512] fp32 sums (32-head groups)
  void* __restrict__ part_o16;           // [B, NR, H, 512] fp16 rows (64-head groups)
  float* __restrict__ part_ml;           // [B, NR, H, 2] (m, l); 64-head groups: [.., 4] (m, l, e bytes, 0)
  const int32_t* __restrict__ sel;       // sparse: [B, sel_stride] positions, ascending
  int B, H, NR, max_pages, pt_shift, num_slots, sel_stride;
  uint32_t pool_bytes;                   // sparse: bytes of the latent pool (< 4 GiB)
  float scale_log2e;
};

constexpr int kMlaThreads = 512;  // 8 wavefronts, 2 per SIMD
constexpr int kPre = 4;           // sparse: tiles per range at most
constexpr int kMlaWaves = kMlaThreads / 64;
constexpr int kLoadsPerWave = (kLoadsPerTile + kMlaWaves - 1) / kMlaWaves;

// HG heads per workgroup (32 or 64).  With HG = 64 each latent tile that a
// workgroup pulls from L2 into LDS serves twice as many heads, which halves
// the L2-to-LDS traffic per HBM byte -- the path this kernel waits on.
//
// Scores: the 4 token tiles x NHT head tiles of a 64-token tile are spread
// over the 8 wavefronts, HTW head tiles x TTW token tiles each.  A latent row
// read from LDS feeds HTW MFMAs; a wave holds q for HTW head tiles.  HTW = 1:
// q for two head tiles (2 x 18 k-steps) would exceed the 256 registers a
// wavefront has at 2 per SIMD.
//
// SPARSE: the context of sequence b is the list of positions sel[b][0..n)
// (the DSA top-k, runtime/glm.py:280-289) instead of positions 0..ctx-1.
// Row j of tile t is position sel[b][64t + j]; each lane resolves one of the
// tile's positions through the block table to a byte offset in the pool, and
// the direct-to-LDS loads take per-lane offsets into one descriptor over the
// whole pool, so the selected rows are gathered on the way into LDS with no
// intermediate copy.  Rows past n, and the padding chunks, use an offset past
// the descriptor's end and land as zeros.
template <int HG, bool SPARSE>
__global__ __launch_bounds__(kMlaThreads) void mla_latent_kernel(MlaArgs a) {
  constexpr int HTW = 1;
  constexpr int NHT = HG / 16;               // 16-head tiles in the group
  constexpr int TTW = 4 * NHT / (8 * HTW);   // token tiles per wavefront
  constexpr int WPH = 4 / TTW;               // wavefronts sharing one head tile's 64 tokens
  static_assert(TTW * HTW * 8 == 4 * NHT, "score tiles must split evenly");
  __shared__ __attribute__((aligned(16))) uint16_t tile_a[kTile * kRow];
  __shared__ __attribute__((aligned(16))) uint16_t tile_b[kTile * kRow];
  __shared__ __attribute__((aligned(16))) uint16_t p_lds[HG * kPRow];
  __shared__ float pmax[WPH][HG];
  __shared__ float psum[WPH][HG];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = uniform(tid >> 6);   // 0..7
  const int qt0 = (w % (NHT / HTW)) * HTW;  // score MFMA: head tiles qt0 .. qt0+HTW-1
  const int wg = w / (NHT / HTW);           // score MFMA: token tiles wg*TTW .. +TTW-1
  const int i16 = lane & 15;
  const int g = lane >> 4;
  const int NHG = a.H / HG;

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
  int ctx = a.ctx_lens[b];
  const int cap = SPARSE ? a.sel_stride : a.max_pages << a.pt_shift;
  ctx = uniform(ctx < 0 ? 0 : (ctx > cap ? cap : ctx));
  const int n_tiles = (ctx + kTile - 1) / kTile;
  const int per = (n_tiles + a.NR - 1) / a.NR;
  const int t_lo = range * per;
  const int t_hi = (t_lo + per < n_tiles) ? t_lo + per : n_tiles;
  const int head0 = hg * HG;
  const int32_t* trow = a.table + static_cast<size_t>(b) * a.max_pages;

  // Q^T operands of this wave's head tiles, all 18 k-steps: lane (head i16,
  // group g) holds q[head][32s + 8g .. +8].
  u32x4 qop[HTW][kQSteps];
#pragma unroll
  for (int k = 0; k < HTW; ++k) {
    const uint16_t* qh =
        a.q + (static_cast<size_t>(b) * a.H + head0 + 16 * (qt0 + k) + i16) * kLat;
#pragma unroll
    for (int s = 0; s < kQSteps; ++s) {
      qop[k][s] = *reinterpret_cast<const u32x4*>(qh + 32 * s + 8 * g);
    }
  }

  f32x4 acc[4][NHT];  // out^T tiles: dims 64w + 16dt.., head tile ht
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
    for (int ht = 0; ht < NHT; ++ht) acc[dt][ht] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  float m_run[NHT];  // per head tile: head 16ht + i16, common to all waves
#pragma unroll
  for (int ht = 0; ht < NHT; ++ht) m_run[ht] = -INFINITY;
  // m_run of this wave's own head tiles kept apart: qt0 is known only at run
  // time, and indexing m_run with it would move the array to scratch memory.
  float m_own[HTW];
  // Softmax normaliser of the own head tiles, per lane (its tokens only): the
  // lanes and the wavefronts sharing a head are summed once, after the loop.
  float l_lane[HTW];
#pragma unroll
  for (int k = 0; k < HTW; ++k) {
    m_own[k] = -INFINITY;
    l_lane[k] = 0.f;
  }

  // Lane-constant source offsets of this wave's direct-to-LDS loads: load i
  // (i = w, w+8, ...) fills LDS chunks 64i..64i+63 of the tile; LDS chunk
  // (row, col) holds bytes 16 * (col ^ tile_swizzle(row)) of token row.
  // Source offset of load k.
  auto src_off_of = [&](int k) {
    const int j = 64 * (w + kMlaWaves * k) + lane;
    const int row = j / kChunksPerRow;
    const int col = j - row * kChunksPerRow;
    return (row * kChunksPerRow + (col ^ tile_swizzle(row))) * 16;
  };
  int src_off[kLoadsPerWave];
#pragma unroll
  for (int k = 0; k < kLoadsPerWave; ++k) src_off[k] = src_off_of(k);

  // Block-table entries of the range's pages, one per lane, refreshed every 64
  // pages: slot lookups inside the loop are register reads, not memory trips.
  const int tile_shift = a.pt_shift - 6;
  int tab_base = -(1 << 30);
  int tab = 0;
  // Issues the loads of tile t into LDS buffer dst; tokens at or past the
  // context end read as zeros (the descriptor covers only valid rows).
  // SPARSE: byte offset of the pool row behind position `pos` (sentinel past
  // the descriptor for no row).
  auto row_offset = [&](int pos, int slot) -> uint32_t {
    if (pos < 0) return 0xFFFFFFF0u;
    if (static_cast<unsigned>(slot) >= static_cast<unsigned>(a.num_slots)) slot = 0;
    const long long row = (static_cast<long long>(slot) << a.pt_shift) +
                          (pos & ((1 << a.pt_shift) - 1));
    return static_cast<uint32_t>(row * (kLat * 2));
  };
  // SPARSE: the range's tiles (at most kPre, the host sizes the ranges so)
  // have their rows resolved up front into LDS -- all positions, then all
  // table entries: two round trips for the range instead of two per tile.
  // Wave 0 resolves, every wave reads.
  __shared__ uint32_t pre_off[SPARSE ? kPre : 1][kTile];
  if constexpr (SPARSE) {
    if (w == 0) {
      int pos[kPre];
#pragma unroll
      for (int k = 0; k < kPre; ++k) {
        const int tok = (t_lo + k) * kTile + lane;
        pos[k] = (t_lo + k < t_hi && tok < ctx)
                     ? a.sel[static_cast<size_t>(b) * a.sel_stride + tok]
                     : -1;
      }
      int slot[kPre];
#pragma unroll
      for (int k = 0; k < kPre; ++k) {
        const int page = pos[k] >> a.pt_shift;
        slot[k] = (pos[k] >= 0 && page < a.max_pages) ? trow[page] : 0;
      }
#pragma unroll
      for (int k = 0; k < kPre; ++k) pre_off[k][lane] = row_offset(pos[k], slot[k]);
    }
    lds_barrier();
  }

  auto load_tile = [&](int t, uint16_t* dst) {
    if constexpr (SPARSE) {
      // row r of tile t: the offset resolved in the prologue (a sparse range
      // has at most kPre tiles)
      const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint16_t*>(a.lat), static_cast<short>(0), static_cast<int>(a.pool_bytes),
          0x00020000);
#pragma unroll
      for (int k = 0; k < kLoadsPerWave; ++k) {
        const int i = w + kMlaWaves * k;
        const int j = 64 * i + lane;
        const int row = j / kChunksPerRow;  // < kTile: the loads cover the tile exactly
        const int col = j - row * kChunksPerRow;
        const uint32_t base = pre_off[(t - t_lo) & (kPre - 1)][row];
        const uint32_t off = base != 0xFFFFFFF0u
                                 ? base + static_cast<uint32_t>(col ^ tile_swizzle(row)) * 16
                                 : 0xFFFFFFF0u;
        if (i < kLoadsPerTile) {
          __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)(dst + i * 64 * 8), 16,
                                                   static_cast<int>(off), 0, 0, 0);
        }
      }
      return;
    }
    const int page = t >> tile_shift;
    const int sub = t - (page << tile_shift);
    if (page >= tab_base + 64) {
      tab_base = page;
      tab = tab_base + lane < a.max_pages ? trow[tab_base + lane] : 0;
    }
    int slot = __builtin_amdgcn_readlane(tab, page - tab_base);
    if (static_cast<unsigned>(slot) >= static_cast<unsigned>(a.num_slots)) slot = 0;
    const uint16_t* base = a.lat + ((static_cast<size_t>(slot) << a.pt_shift) + sub * kTile) * kLat;
    int valid = ctx - t * kTile;
    valid = valid > kTile ? kTile : valid;
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(base), static_cast<short>(0), valid * kLat * 2, 0x00020000);
#pragma unroll
    for (int k = 0; k < kLoadsPerWave; ++k) {
      const int i = w + kMlaWaves * k;
      if (i < kLoadsPerTile) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)(dst + i * 64 * 8), 16,
                                                 src_off[k], 0, 0, 0);
      }
    }
  };

  // One tile of work on LDS buffer `tile` while tile t+1 streams into `next`.
  auto step = [&](int t, const uint16_t* tile, uint16_t* next) {
    // This wave's loads of tile t have landed; after the barrier every wave's
    // have, and every wave is done with the other buffer (tile t-1).  The
    // wait is the builtin (wait_vmem_all), not inline asm: with an asm wait
    // the compiler still counted the q operand loads from before the loop as
    // pending and waited before every score MFMA -- in effect for the whole
    // next tile, which is issued just before (7 % of the kernel).
    wait_vmem_all();
    lds_barrier();
    if (t + 1 < t_hi) load_tile(t + 1, next);

    // ---- scores: TTW token tiles x HTW head tiles ----
    const int valid = ctx - t * kTile;
    float x[TTW][HTW][4];
    {
      // The latent rows of k-step s + kAhead are read while the MFMAs of
      // step s run, so no MFMA waits on a read issued just before it.
      constexpr int kAhead = 2;
      // Row 16x + i16, logical chunk 4s + g sits at chunk 4(s ^ flip) + lo:
      // the swizzle of rows 16x + i16 depends on i16 only.
      const int sw = tile_swizzle(i16);
      const int lo = g ^ (sw & 2);
      const int flip = sw >> 2;
      const uint16_t* arow[TTW];
      f32x4 sc[TTW][HTW];
      u32x4 ring[kAhead + 1][TTW];
#pragma unroll
      for (int j = 0; j < TTW; ++j) {
        arow[j] = tile + (16 * (wg * TTW + j) + i16) * kRow + 8 * lo;
#pragma unroll
        for (int k = 0; k < HTW; ++k) sc[j][k] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
      // element offset of k-step s: 32 * (s ^ flip)
      auto kstep = [&](int s) { return 32 * s + ((s & 1) ? -32 : 32) * flip; };
#pragma unroll
      for (int s = 0; s < kAhead; ++s) {
#pragma unroll
        for (int j = 0; j < TTW; ++j) ring[s][j] = *reinterpret_cast<const u32x4*>(arow[j] + kstep(s));
      }
#pragma unroll
      for (int s = 0; s < kQSteps; ++s) {
        if (s + kAhead < kQSteps) {
#pragma unroll
          for (int j = 0; j < TTW; ++j) {
            ring[(s + kAhead) % (kAhead + 1)][j] =
                *reinterpret_cast<const u32x4*>(arow[j] + kstep(s + kAhead));
          }
        }
#pragma unroll
        for (int j = 0; j < TTW; ++j) {
#pragma unroll
          for (int k = 0; k < HTW; ++k) {
            sc[j][k] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(bf16x8, ring[s % (kAhead + 1)][j]),
                __builtin_bit_cast(bf16x8, qop[k][s]), sc[j][k], 0, 0, 0);
          }
        }
      }
      // lane (head 16(qt0+k) + i16, group g) holds tokens 16tt + 4g + r, r = 0..3
#pragma unroll
      for (int j = 0; j < TTW; ++j) {
        const int tt = wg * TTW + j;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const bool ok = 16 * tt + 4 * g + r < valid;
#pragma unroll
          for (int k = 0; k < HTW; ++k) x[j][k][r] = ok ? sc[j][k][r] * a.scale_log2e : -INFINITY;
        }
      }
    }
#pragma unroll
    for (int k = 0; k < HTW; ++k) {
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < TTW; ++j) {
#pragma unroll
        for (int r = 0; r < 4; ++r) mx = fmaxf(mx, x[j][k][r]);
      }
      mx = wave_max_across_groups(mx);
      if (g == 0) pmax[wg][16 * (qt0 + k) + i16] = mx;
    }
    lds_barrier();

    float alpha[NHT];
#pragma unroll
    for (int ht = 0; ht < NHT; ++ht) {
      const int hh = 16 * ht + i16;
      float mp = pmax[0][hh];
#pragma unroll
      for (int k = 1; k < WPH; ++k) mp = fmaxf(mp, pmax[k][hh]);
      const float mn = fmaxf(m_run[ht], mp);
      alpha[ht] = fast_exp2(m_run[ht] - mn);
      m_run[ht] = mn;
    }
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
      for (int ht = 0; ht < NHT; ++ht) acc[dt][ht] *= alpha[ht];
    }
#pragma unroll
    for (int k = 0; k < HTW; ++k) {
      const int hh = 16 * (qt0 + k) + i16;
      float mp = pmax[0][hh];
#pragma unroll
      for (int kk = 1; kk < WPH; ++kk) mp = fmaxf(mp, pmax[kk][hh]);
      const float mn = fmaxf(m_own[k], mp);
      const float alpha_own = fast_exp2(m_own[k] - mn);
      m_own[k] = mn;
      float ps = 0.f;
#pragma unroll
      for (int j = 0; j < TTW; ++j) {
        const int tt = wg * TTW + j;
        float p[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) p[r] = fast_exp2(x[j][k][r] - m_own[k]);
        const uint32_t w0 = pack_bf16x2(p[0], p[1]);
        const uint32_t w1 = pack_bf16x2(p[2], p[3]);
        // P row of head hh: tokens 16tt+4g .. +3 in natural order
        *reinterpret_cast<u32x2*>(p_lds + hh * kPRow + 16 * tt + 4 * g) = u32x2{w0, w1};
        ps += __builtin_bit_cast(float, w0 << 16) + __builtin_bit_cast(float, w0 & 0xffff0000u) +
              __builtin_bit_cast(float, w1 << 16) + __builtin_bit_cast(float, w1 & 0xffff0000u);
      }
      l_lane[k] = l_lane[k] * alpha_own + ps;
    }
    lds_barrier();

    // ---- out^T[dims 64w.., heads] += C^T . P^T ----
    // Transposed-read addresses: lane k of a 16-lane group supplies token row
    // 8g + (k/4) (+4 for the second read) at dims 4*(k%4) of the dim tile.
    const int trow_tok = 8 * g + (i16 >> 2);
    const int tcol = 4 * (i16 & 3);
    // The swizzle of those rows permutes the four 16-dim tiles of the wave's
    // 64 dims: tile dt is stored at dt ^ x.
    const int x_lo = tile_swizzle(trow_tok) >> 1;
    const int x_hi = tile_swizzle(trow_tok + 4) >> 1;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      bf16x8 pb[NHT];
#pragma unroll
      for (int ht = 0; ht < NHT; ++ht) {
        pb[ht] = __builtin_bit_cast(
            bf16x8,
            *reinterpret_cast<const u32x4*>(p_lds + (16 * ht + i16) * kPRow + 32 * ks + 8 * g));
      }
      const uint16_t* trb = tile + (32 * ks + trow_tok) * kRow + 64 * w + tcol;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
            (lds_bf16x4*)(trb + 16 * (dt ^ x_lo)));
        const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
            (lds_bf16x4*)(trb + 4 * kRow + 16 * (dt ^ x_hi)));
        const bf16x8 av = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
        for (int ht = 0; ht < NHT; ++ht) {
          acc[dt][ht] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, pb[ht], acc[dt][ht], 0, 0, 0);
        }
      }
    }
  };

  // The two buffers are distinct LDS objects and the loop is unrolled by two,
  // so every LDS read provably misses the buffer being filled and the loads
  // of the next tile stay in flight across the current tile's reads.
  if (t_lo < t_hi) load_tile(t_lo, tile_a);
  for (int t = t_lo; t < t_hi; t += 2) {
    step(t, tile_a, tile_b);
    if (t + 1 < t_hi) step(t + 1, tile_b, tile_a);
  }

  // ---- partial state of this (sequence, range, head group) ----
  const size_t pbase = (static_cast<size_t>(b) * a.NR + range) * a.H + head0;
#pragma unroll
  for (int ht = 0; ht < NHT; ++ht) {
    const int hh = 16 * ht + i16;
    float* po = a.part_o + (pbase + hh) * kC + 64 * w + 4 * g;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      *reinterpret_cast<f32x4*>(po + 16 * dt) = acc[dt][ht];
    }
  }
  // normaliser: lanes of a wave, then the WPH wavefronts sharing each head
#pragma unroll
  for (int k = 0; k < HTW; ++k) {
    const float l = wave_sum_across_groups(l_lane[k]);
    if (g == 0) psum[wg][16 * (qt0 + k) + i16] = l;
  }
  lds_barrier();
  if (w == 0 && g == 0) {
#pragma unroll
    for (int ht = 0; ht < NHT; ++ht) {
      const int hh = 16 * ht + i16;
      float l = psum[0][hh];
#pragma unroll
      for (int k = 1; k < WPH; ++k) l += psum[k][hh];
      a.part_ml[(pbase + hh) * 2 + 0] = m_run[ht];
      a.part_ml[(pbase + hh) * 2 + 1] = l;
    }
  }
}

// ------------------------------------------- 64-head groups, 32x32 tiles ----
// mla_group64_kernel: the latent contraction for head groups of 64 with four
// wavefronts (one per SIMD, so each has the SIMD's whole register file) and
// v_mfma_f32_32x32x16_bf16, whose 32x32 output tile halves the LDS operand
// bytes per flop of the 16x16 shape.  Per 64-token tile:
//   scores  wave w: tokens 32(w>>1).., heads 32(w&1)..   A = latent rows (LDS),
//           B = q (registers, all 36 k-steps)
//   P.V     wave w: dims 128w..128w+127 x all 64 heads   A = C^T (transposed
//           LDS reads), B = P (LDS)
// Two barriers per tile: one after the tile has landed, one after P is
// written.  The softmax uses one reference maximum M per head for the whole
// token range, the maximum of the range's first tile (shared by the four
// wavefronts), so P of a tile is formed before its maximum is known across
// wavefronts and the accumulators are never rescaled: P = 2^(x - M) stays
// below 2^kBig, and a tile that would exceed that -- in practice never after
// the first -- starts the range over with the raised M.  Every wavefront
// reads the same tile maxima from LDS, so all four take the same branches.
constexpr int kGThreads = 256;
constexpr int kGWaves = 4;
constexpr int kGLoads = kLoadsPerTile / kGWaves;  // 18 direct-to-LDS loads per wave and tile
constexpr int kGPRow = kTile + 8;                 // P row stride: 144 B, conflict-free rows
constexpr int kGSteps = kLat / 16;                // 36 k-steps of the score MFMA
constexpr float kBig = 64.f;
static_assert(kLoadsPerTile % kGWaves == 0, "loads split evenly over the wavefronts");

typedef float f32x16 __attribute__((ext_vector_type(16)));

// Chunk c of token row r is stored at chunk c ^ group_swizzle(r).  The score
// reads (32 consecutive rows, one chunk) and the transposed reads (rows
// 4k..4k+3, four adjacent chunks) then spread over all banks: rows r and r+4j
// differ in bits 0-2 of the swizzle for j = 1..7, and rows r and r+2 in bit 2.
__device__ __forceinline__ int group_swizzle(int r) {
  return ((r >> 2) ^ (((r >> 1) & 1) << 2)) & 7;
}

// Build knobs of mla_group64_kernel (measured defaults): k-steps of latent
// rows read ahead of the score MFMAs, P.V steps of C^T read ahead, and one
// next-tile load issued every VOOM_MLA_LOAD_EVERY score k-steps.
#ifndef VOOM_MLA_SCORE_AHEAD
#define VOOM_MLA_SCORE_AHEAD 5
#endif
#ifndef VOOM_MLA_PV_AHEAD
#define VOOM_MLA_PV_AHEAD 2
#endif
#ifndef VOOM_MLA_LOAD_EVERY
#define VOOM_MLA_LOAD_EVERY 2
#endif
static_assert((kLat / 16 + VOOM_MLA_LOAD_EVERY - 1) / VOOM_MLA_LOAD_EVERY >= kLoadsPerTile / 4,
              "every next-tile load must fall on a score k-step");
static_assert(VOOM_MLA_SCORE_AHEAD >= 1 && VOOM_MLA_PV_AHEAD >= 1, "read-ahead of at least one step");

template <bool SPARSE>
__global__ __launch_bounds__(kGThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void mla_group64_kernel(MlaArgs a) {
  constexpr int HG = 64;
  __shared__ __attribute__((aligned(16))) uint16_t tile_a[kTile * kRow];
  __shared__ __attribute__((aligned(16))) uint16_t tile_b[kTile * kRow];
  __shared__ __attribute__((aligned(16))) uint16_t p_lds[HG * kGPRow];
  // per tile parity and head: the four partial maxima of the tile
  __shared__ __attribute__((aligned(16))) float tmax_lds[2][HG][4];
  __shared__ float lsum_lds[2][HG];
  __shared__ uint32_t pre_off[SPARSE ? kPre : 1][kTile];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = uniform(tid >> 6);  // 0..3
  const int th = w >> 1;            // score tokens 32 th ..
  const int hh = w & 1;             // score heads 32 hh ..
  const int l32 = lane & 31;
  const int lh = lane >> 5;
  const int NHG = a.H / HG;

  const int n_tasks = a.B * a.NR;
  int task, hg;
  const int bid = blockIdx.x;
  if (n_tasks % 8 == 0) {
    // the head groups of one (sequence, range) share bid % 8: the same XCD
    const int local = bid >> 3;
    hg = local % NHG;
    task = (local / NHG) * 8 + (bid & 7);
  } else {
    hg = bid % NHG;
    task = bid / NHG;
  }
  const int b = task / a.NR;
  const int range = task - b * a.NR;
  int ctx = a.ctx_lens[b];
  const int cap = SPARSE ? a.sel_stride : a.max_pages << a.pt_shift;
  ctx = uniform(ctx < 0 ? 0 : (ctx > cap ? cap : ctx));
  const int n_tiles = (ctx + kTile - 1) / kTile;
  const int per = (n_tiles + a.NR - 1) / a.NR;
  const int t_lo = range * per;
  const int t_hi = (t_lo + per < n_tiles) ? t_lo + per : n_tiles;
  const int head0 = hg * HG;
  const int32_t* trow = a.table + static_cast<size_t>(b) * a.max_pages;

  // B operand of the scores: lane (head 32 hh + l32, half lh) holds
  // q[head][16 s + 8 lh .. + 8] for all 36 k-steps.
  u32x4 qop[kGSteps];  // filled from LDS below

  f32x16 acc[4][2];  // out^T: dims 128 w + 32 dt .., heads 32 ht + l32
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
    for (int ht = 0; ht < 2; ++ht) acc[dt][ht] = f32x16{};
  }
  // Reference maxima (log2 units) of heads l32 and 32 + l32, the same in
  // every wavefront; the normaliser of the score head (32 hh + l32) over this
  // lane's tokens, relative to M.
  float M[2] = {-INFINITY, -INFINITY};
  float l_run = 0.f;

  // LDS tile layout: nine column blocks of 8 chunks (128 bytes of a row)
  // for all 64 rows, 8 KiB each; row r of block cb holds chunks 8 cb .. 8 cb
  // + 7 of token row r at r * 128 bytes, chunk c at position c ^
  // group_swizzle(r).  A direct-to-LDS load fills 1 KiB, i.e. rows 8 g ..
  // 8 g + 7 of one block: load k of wave w covers block k >> 1, rows 8 w +
  // 32 (k & 1) + lane / 8, so its source offset is one of two per-lane bases
  // plus 128 (k >> 1) -- the swizzle of those rows does not depend on k.
  const int ld_row = 8 * w + (lane >> 3);
  const int ld_col = 16 * ((lane & 7) ^ group_swizzle(ld_row));
  const int ld_base0 = ld_row * (kLat * 2) + ld_col;
  const int ld_base1 = ld_base0 + 32 * (kLat * 2);

  // The group's q rows (64 x 576, contiguous in memory) go through the
  // second tile buffer in the tile layout: one coalesced stream instead of 36
  // row-strided loads per wavefront, and the score operands are then read
  // with the conflict-free pattern of the latent rows (row 32 hh + l32).
  auto load_q = [&]() {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(a.q + (static_cast<size_t>(b) * a.H + head0) * kLat),
        static_cast<short>(0), HG * kLat * 2, 0x00020000);
#pragma unroll
    for (int k = 0; k < kGLoads; ++k) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)(tile_b + (w + kGWaves * k) * 512), 16,
                                               ((k & 1) ? ld_base1 : ld_base0) + 128 * (k >> 1),
                                               0, 0, 0);
    }
  };

  if constexpr (SPARSE) {
    // q needs no selection: its loads go out first, under the selection ->
    // table -> row offset chain
    load_q();
    if (w == 0) {
      // Both lookups load unconditionally (index 0 where there is nothing to
      // look up), so each is one batch of loads with one wait; loads under a
      // branch were waited for one by one.
      int pos[kPre];
#pragma unroll
      for (int k = 0; k < kPre; ++k) {
        const int tok = (t_lo + k) * kTile + lane;
        const bool used = t_lo + k < t_hi && tok < ctx;
        const int p = a.sel[static_cast<size_t>(b) * a.sel_stride + (used ? tok : 0)];
        pos[k] = used ? p : -1;
      }
      int tab_slot[kPre];
#pragma unroll
      for (int k = 0; k < kPre; ++k) {
        const int page = pos[k] >> a.pt_shift;
        tab_slot[k] = trow[pos[k] >= 0 && page < a.max_pages ? page : 0];
      }
#pragma unroll
      for (int k = 0; k < kPre; ++k) {
        // a position past the table reads from slot 0 (the slot an invalid
        // table entry falls back to); no position: a row of zeros
        const int page = pos[k] >> a.pt_shift;
        int slot = (pos[k] >= 0 && page < a.max_pages) ? tab_slot[k] : 0;
        if (static_cast<unsigned>(slot) >= static_cast<unsigned>(a.num_slots)) slot = 0;
        pre_off[k][lane] =
            pos[k] < 0 ? 0xFFFFFFF0u
                       : static_cast<uint32_t>(((static_cast<long long>(slot) << a.pt_shift) +
                                                (pos[k] & ((1 << a.pt_shift) - 1))) *
                                               (kLat * 2));
      }
    }
    lds_barrier();
  }

  // Source of a tile's direct-to-LDS loads: a buffer descriptor and two
  // per-lane offsets (rows 8 w + lane / 8 and 32 rows further); load k adds
  // 128 (k >> 1) bytes.  Rows past the context, and a tile that does not
  // exist, read as zeros: their offsets lie past the descriptor's range
  // (0xFFFF0000 and above, which no pool or tile range reaches).
  const int tile_shift = a.pt_shift - 6;
  int tab_base = -(1 << 30);
  int tab = 0;
  auto tile_src = [&](int t, uint32_t (&off)[2]) -> __amdgpu_buffer_rsrc_t {
    if (t >= t_hi) {
      off[0] = off[1] = 0xFFFF0000u;
      return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.lat), static_cast<short>(0),
                                               0, 0x00020000);
    }
    if constexpr (SPARSE) {
      const uint32_t* po = pre_off[(t - t_lo) & (kPre - 1)];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const uint32_t rb = po[ld_row + 32 * i];
        off[i] = rb != 0xFFFFFFF0u ? rb + static_cast<uint32_t>(ld_col) : 0xFFFF0000u;
      }
      return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.lat), static_cast<short>(0),
                                               static_cast<int>(a.pool_bytes), 0x00020000);
    }
    const int page = t >> tile_shift;
    const int sub = t - (page << tile_shift);
    if (page < tab_base || page >= tab_base + 64) {
      tab_base = page;
      tab = tab_base + lane < a.max_pages ? trow[tab_base + lane] : 0;
    }
    int slot = __builtin_amdgcn_readlane(tab, page - tab_base);
    if (static_cast<unsigned>(slot) >= static_cast<unsigned>(a.num_slots)) slot = 0;
    const uint16_t* base =
        a.lat + ((static_cast<size_t>(slot) << a.pt_shift) + sub * kTile) * kLat;
    int valid = ctx - t * kTile;
    valid = valid > kTile ? kTile : valid;
    off[0] = static_cast<uint32_t>(ld_base0);
    off[1] = static_cast<uint32_t>(ld_base1);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), static_cast<short>(0),
                                             valid * kLat * 2, 0x00020000);
  };
  auto load_tile = [&](int t, uint16_t* dst) {
    uint32_t off[2];
    const __amdgpu_buffer_rsrc_t r = tile_src(t, off);
#pragma unroll
    for (int k = 0; k < kGLoads; ++k) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)(dst + (w + kGWaves * k) * 512), 16,
                                               static_cast<int>(off[k & 1] + 128 * (k >> 1)), 0,
                                               0, 0);
    }
  };

  // Per-lane parts of the LDS addresses (in bf16 elements; a block is 4096).
  // Scores: row 32 th + l32 (its swizzle depends on l32 only), logical chunk
  // 2 s + lh, i.e. block s >> 2, chunk 2 (s & 3) + lh within it.
  const int sw_row = group_swizzle(l32);
  int a_off[4];  // k-step s = 4 i + j: element offset 4096 i + a_off[j]
#pragma unroll
  for (int j = 0; j < 4; ++j) a_off[j] = (32 * th + l32) * 64 + 8 * ((2 * j + lh) ^ sw_row);
  // Transposed reads: in 16-lane group G, lane i16 addresses token row
  // 16 ks + 8 (G >> 1) + 4 h + (i16 >> 2) at dims 128 w + 32 dt + 16 (G & 1) +
  // 4 (i16 & 3), i.e. block 2 w + (dt >> 1), chunk 4 (dt & 1) + 2 (G & 1) +
  // (i16 & 3) / 2; the swizzle of that row is (4 (ks & 1) + 2 (G >> 1) + h) ^
  // 4 (i16 >> 3).
  const int G = lane >> 4;
  const int i16 = lane & 15;
  // The lane-dependent part depends on ks & 1, h and dt & 1 only (eight
  // registers); ks >> 1 adds 32 rows and dt >> 1 one block.
  int tr_base[2][2][2];
#pragma unroll
  for (int k1 = 0; k1 < 2; ++k1) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int d1 = 0; d1 < 2; ++d1) {
        const int row = 16 * k1 + 8 * (G >> 1) + 4 * h + (i16 >> 2);
        const int sw = ((4 * k1 + 2 * (G >> 1) + h) ^ (4 * (i16 >> 3))) & 7;
        const int chunk = 4 * d1 + 2 * (G & 1) + ((i16 & 3) >> 1);
        tr_base[k1][h][d1] = 4096 * 2 * w + row * 64 + 8 * (chunk ^ sw) + 4 * (i16 & 1);
      }
    }
  }
  auto tr_off = [&](int ks, int h, int dt) {
    return tr_base[ks & 1][h][dt & 1] + 2048 * (ks >> 1) + 4096 * (dt >> 1);
  };

  // Instruction-group order for the scheduler (masks of
  // __builtin_amdgcn_sched_group_barrier).
  constexpr int kMfma = 0x008, kVmemRead = 0x020, kDsRead = 0x100;

  // One tile on LDS buffer `tile` while tile t + 1 streams into `next`;
  // false: the range has to start over (see below).
  const int t_first = t_lo;
  // Reference check of tile tp: its tile maxima against M (kept in LDS by
  // tile parity, so that the check of tile t - 1 can be made during tile t).
  auto too_big = [&](int tp) {
    float tm[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(&tmax_lds[tp & 1][32 * k + l32][0]);
      tm[k] = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
    }
    if (__builtin_amdgcn_ballot_w64(tm[0] > M[0] + kBig || tm[1] > M[1] + kBig) == 0) return false;
    M[0] = fmaxf(M[0], tm[0]);
    M[1] = fmaxf(M[1], tm[1]);
    return true;
  };

  auto step = [&](int t, const uint16_t* tile, uint16_t* next) -> bool {
    wait_vmem_all();
    lds_barrier();
    uint32_t noff[2];
    const __amdgpu_buffer_rsrc_t nsrc = tile_src(t + 1, noff);

    // ---- scores: 32 tokens x 32 heads, one accumulator chain (dependent
    // 32x32 MFMAs issue back to back).  The latent rows of k-step s + kAhead
    // are read while the MFMA of step s runs, and the next tile's 18 loads go
    // out one every two k-steps: issued in one burst, they stall the wave
    // until the memory pipeline has taken them. ----
    f32x16 sc = f32x16{};
    {
      constexpr int kAhead = VOOM_MLA_SCORE_AHEAD;
      u32x4 ring[kAhead];
#pragma unroll
      for (int s = 0; s < kAhead; ++s) {
        ring[s] = *reinterpret_cast<const u32x4*>(tile + 4096 * (s >> 2) + a_off[s & 3]);
      }
      __builtin_amdgcn_sched_group_barrier(kDsRead, kAhead, 0);
#pragma unroll
      for (int s = 0; s < kGSteps; ++s) {
        const bf16x8 av = __builtin_bit_cast(bf16x8, ring[s % kAhead]);
        const bf16x8 qv = __builtin_bit_cast(bf16x8, qop[s]);
        if (s + kAhead < kGSteps) {
          const int n = s + kAhead;
          ring[s % kAhead] = *reinterpret_cast<const u32x4*>(tile + 4096 * (n >> 2) + a_off[n & 3]);
          __builtin_amdgcn_sched_group_barrier(kDsRead, 1, 0);
        }
        sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, qv, sc, 0, 0, 0);
        __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
        if (s % VOOM_MLA_LOAD_EVERY == 0 && s / VOOM_MLA_LOAD_EVERY < kGLoads) {
          const int k = s / VOOM_MLA_LOAD_EVERY;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              nsrc, (lds_void*)(next + (w + kGWaves * k) * 512), 16,
              static_cast<int>(noff[k & 1] + 128 * (k >> 1)), 0, 0, 0);
          __builtin_amdgcn_sched_group_barrier(kVmemRead, 1, 0);
        }
      }
    }
    // The previous tile's reference check, deferred to here so that its LDS
    // reads were hidden behind the score MFMAs; a failure drops this tile too.
    if (t - 1 > t_first && too_big(t - 1)) return false;

    // lane (head 32 hh + l32) holds tokens 32 th + 4 lh + (8 (r >> 2) + (r & 3))
    // as raw dot products; the scale (> 0) is applied inside the exponent.
    // Only the last tile of a sequence has rows past its end.
    float x[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) x[r] = sc[r];
    if (ctx - t * kTile < kTile) {
      const int lim = ctx - t * kTile - (32 * th + 4 * lh);
#pragma unroll
      for (int r = 0; r < 16; ++r) x[r] = 8 * (r >> 2) + (r & 3) < lim ? x[r] : -INFINITY;
    }
    float mloc = x[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mloc = fmaxf(mloc, x[r]);
    // the maximum of this lane's 16 tokens (log2 units); the four lanes
    // holding a head's 64 tokens (th, lh) each leave theirs
    tmax_lds[t & 1][32 * hh + l32][2 * th + lh] = mloc * a.scale_log2e;

    uint16_t* prow = p_lds + (32 * hh + l32) * kGPRow + 32 * th + 4 * lh;
    auto write_p = [&](float m) {
      float ps = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float e[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) e[i] = fast_exp2(__builtin_fmaf(x[4 * q + i], a.scale_log2e, -m));
        const uint32_t w0 = pack_bf16x2(e[0], e[1]);
        const uint32_t w1 = pack_bf16x2(e[2], e[3]);
        *reinterpret_cast<u32x2*>(prow + 8 * q) = u32x2{w0, w1};
        ps = sum_bf16x2(w1, sum_bf16x2(w0, ps));
      }
      return ps;
    };

    // ---- operands of P.V: C^T by transposed reads of the tile, P from LDS
    // once every wavefront has written it.  The C^T operand of step (ks, dt)
    // is read two steps ahead, P one k-step ahead. ----
    constexpr int kCAhead = VOOM_MLA_PV_AHEAD;
    bf16x8 pb[2][2];
    bf16x8 cv[kCAhead + 1];
    auto read_c = [&](int i) {  // step i = 4 ks + dt
      const int ks = i >> 2, dt = i & 3;
      const bf16x4 lo =
          __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(tile + tr_off(ks, 0, dt)));
      const bf16x4 hi =
          __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(tile + tr_off(ks, 1, dt)));
      cv[i % (kCAhead + 1)] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    };
    auto read_p = [&](int ks) {
#pragma unroll
      for (int ht = 0; ht < 2; ++ht) {
        pb[ks & 1][ht] = __builtin_bit_cast(
            bf16x8, *reinterpret_cast<const u32x4*>(p_lds + (32 * ht + l32) * kGPRow + 16 * ks +
                                                    8 * lh));
      }
    };
    if (t == t_first) {
      // first tile of the range: the reference maximum comes from it, so the
      // maxima are exchanged before P is formed (one more barrier)
      lds_barrier();
      too_big(t);
    }
    const float ps = write_p(hh ? M[1] : M[0]);
    lds_barrier();
    read_p(0);
#pragma unroll
    for (int i = 0; i < kCAhead; ++i) read_c(i);

    // ---- out^T[dims 128 w .., heads] += C^T . P^T, 16 tokens per k-step ----
    __builtin_amdgcn_sched_group_barrier(kDsRead, 2 + 2 * kCAhead, 1);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int ks = i >> 2, dt = i & 3;
      if (i + kCAhead < 16) {
        read_c(i + kCAhead);
        __builtin_amdgcn_sched_group_barrier(kDsRead, 2, 1);
      }
      if (dt == 0 && ks + 1 < 4) {
        read_p(ks + 1);
        __builtin_amdgcn_sched_group_barrier(kDsRead, 2, 1);
      }
#pragma unroll
      for (int ht = 0; ht < 2; ++ht) {
        acc[dt][ht] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cv[i % (kCAhead + 1)], pb[ks & 1][ht],
                                                              acc[dt][ht], 0, 0, 0);
        __builtin_amdgcn_sched_group_barrier(kMfma, 1, 1);
      }
    }
    l_run += ps;
    return true;
  };

  // A restart (a tile more than 2^kBig above the reference of the first)
  // drops the range's sums and runs it again from its first tile with the
  // raised reference, which no tile of the range can exceed by that much
  // again before a still higher one: M grows by more than kBig per restart,
  // so the loop ends.  The accumulators are only ever zeroed or fed to MFMAs,
  // which keeps them in accumulation registers.
  //
  // The first tile's loads are issued right behind q's (dense: its table
  // lookup first, as that load's wait would also wait for q; sparse: q went
  // out before the row offsets were looked up), and only q is waited for
  // before its rows are read out, so the tile's latency overlaps that.
  {
    uint32_t off[2];
    const __amdgpu_buffer_rsrc_t r0 = tile_src(t_lo, off);  // empty past t_hi
    if constexpr (!SPARSE) load_q();
#pragma unroll
    for (int k = 0; k < kGLoads; ++k) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r0, (lds_void*)(tile_a + (w + kGWaves * k) * 512),
                                               16, static_cast<int>(off[k & 1] + 128 * (k >> 1)),
                                               0, 0, 0);
    }
    static_assert(kGLoads == 18, "the wait below counts the first tile's 18 loads");
    __builtin_amdgcn_s_waitcnt(0x4F72);  // gfx9 encoding: vmcnt 18 (q landed), lgkmcnt 15
    lds_barrier();
#pragma unroll
    for (int s = 0; s < kGSteps; ++s) {
      qop[s] = *reinterpret_cast<const u32x4*>(tile_b + 4096 * (s >> 2) + a_off[s & 3] +
                                               (hh - th) * 32 * 64);
    }
  }
  for (bool first_pass = true;; first_pass = false) {
    int t = t_lo;
    bool ok = true;
    if (!first_pass) load_tile(t, tile_a);
    while (ok && t < t_hi) {
      ok = step(t, tile_a, tile_b);
      if (ok && t + 1 < t_hi) ok = step(t + 1, tile_b, tile_a);
      t += 2;
    }
    if (ok && t_hi - 1 > t_lo) {
      // the last tile's check (the others were made one tile later)
      lds_barrier();
      ok = !too_big(t_hi - 1);
    }
    if (ok) break;
    wait_vmem_all();  // loads issued before the restart
    lds_barrier();
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
      for (int ht = 0; ht < 2; ++ht) acc[dt][ht] = f32x16{};
    }
    l_run = 0.f;
  }

  // ---- partial state of this (sequence, range, head group) ----
  // Written as normalised rows o = acc / l in fp16.  Wavefront w scales its
  // dims 128 w .. 128 w + 127 of a (range, head) row by 2^-e_w so that their
  // largest magnitude lies in [2^14, 2^15) (no exchange of maxima between
  // wavefronts); the statistics hold (m, l) and, one signed byte each in the
  // third word, e_0 .. e_3: half the bytes of fp32 sums, at 11 significant bits
  // (the reduce multiplies 2^e back).  The rows go through LDS so that each
  // store instruction writes 1 KiB of one row.
  const size_t pbase = (static_cast<size_t>(b) * a.NR + range) * a.H + head0;
  const float lw = l_run + __shfl_xor(l_run, 32);
  if (lh == 0) lsum_lds[th][32 * hh + l32] = lw;
  wait_vmem_all();  // the last step's (empty) next-tile loads write tile_b
  lds_barrier();
  constexpr int kStageRow = kC + 8;  // fp16 elements per staged row (1040 bytes)
  _Float16* stage = reinterpret_cast<_Float16*>(tile_a);
  uint8_t* e_lds = reinterpret_cast<uint8_t*>(&tmax_lds[0][0][0]);  // [64 heads][4 wavefronts]
  float lrow[2];
#pragma unroll
  for (int ht = 0; ht < 2; ++ht) {
    const int h = 32 * ht + l32;
    const float l = lsum_lds[0][h] + lsum_lds[1][h];
    lrow[ht] = l;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    float mx = 0.f;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, fabsf(acc[dt][ht][r]));
    }
    mx *= inv;
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    // e = ilogb(mx) - 14, within [-100, 113]: mx 2^-e in [2^14, 2^15), so a
    // quarter of small values keeps 11 bits instead of falling into fp16's
    // subnormals (a zero quarter takes -100; non-finite rows take 0)
    const int eb = static_cast<int>((__builtin_bit_cast(uint32_t, mx) >> 23) & 0xff) - 127;
    const int ex = eb == 128 ? 0 : (eb < -86 ? -100 : eb - 14);
    if (lh == 0) e_lds[4 * h + w] = static_cast<uint8_t>(static_cast<int8_t>(ex));
    const float f = inv * __builtin_bit_cast(float, static_cast<uint32_t>(127 - ex) << 23);
    typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 v = f32x4{acc[dt][ht][4 * q], acc[dt][ht][4 * q + 1], acc[dt][ht][4 * q + 2],
                              acc[dt][ht][4 * q + 3]} * f;
        *reinterpret_cast<f16x4*>(stage + h * kStageRow + 128 * w + 32 * dt + 8 * q + 4 * lh) =
            __builtin_convertvector(v, f16x4);
      }
    }
  }
  lds_barrier();
  // wavefront w stores heads 16 w .. 16 w + 15, one 1 KiB row per instruction
  _Float16* po = static_cast<_Float16*>(a.part_o16) + pbase * kC;
#pragma unroll
  for (int i = 0; i < HG / kGWaves; ++i) {
    const int h = (HG / kGWaves) * w + i;
    *reinterpret_cast<u32x4*>(po + static_cast<size_t>(h) * kC + 8 * lane) =
        *reinterpret_cast<const u32x4*>(stage + h * kStageRow + 8 * lane);
  }
  if (w == 0) {
    // lane = head: heads l32 and 32 + l32 sit in lanes l32 and l32 + 32
    const uint32_t ebits = reinterpret_cast<const uint32_t*>(e_lds)[lane];
    reinterpret_cast<f32x4*>(a.part_ml)[pbase + lane] =
        f32x4{lh ? M[1] : M[0], lh ? lrow[1] : lrow[0], __builtin_bit_cast(float, ebits), 0.f};
  }
}

// Merge of the NR range partials of (sequence b, head h) by one wavefront:
// lane r holds range r's statistics; the partial rows of a batch of ranges
// are all loaded before the first is used (one memory round trip per batch).
// F16 = false: rows are fp32 sums relative to 2^m, stats (m, l).
// F16 = true: rows are fp16 o 2^-e with o = sum / l, stats (m, l, e bytes, 0)
// with one e per 128-dim quarter of the row; the weight of the row's quarter
// is then 2^(m - M) l 2^e.  Lane `lane` ends with dims
// 8 lane .. 8 lane + 7 of sum_r weight_r row_r in acc, and M, L such that the
// merged row is acc / L with log-sum-exp M + log2 L (log2 units).
constexpr int kDPL = kC / 64;  // 8 dims per lane

// 2^e for the signed byte at bit qsh of an fp16 partial's exponent word
// (e in [-100, 113]): the scale of the 128-dim quarter that lane `lane` of a
// merge reads (qsh = 8 (lane / 16)).
__device__ __forceinline__ float quarter_scale(uint32_t ebits, int qsh) {
  const int e = static_cast<int8_t>(static_cast<uint8_t>(ebits >> qsh));
  return __builtin_bit_cast(float, static_cast<uint32_t>(127 + e) << 23);
}
template <bool F16>
__device__ __forceinline__ void merge_ranges(const void* __restrict__ part_o,
                                             const float* __restrict__ part_ml, int b, int h,
                                             int H, int NR, int lane, f32x4 (&acc)[kDPL / 4],
                                             float& M, float& L) {
  constexpr int kBatch = 8;
  M = -INFINITY;
  L = 0.f;
#pragma unroll
  for (int c = 0; c < kDPL / 4; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int r0 = 0; r0 < NR; r0 += 64) {
    const int r = r0 + lane;
    const size_t ri = (static_cast<size_t>(b) * NR + r) * H + h;
    float m = -INFINITY, l = 0.f;
    uint32_t ebits = 0;
    if (r < NR) {
      if constexpr (F16) {
        const f32x4 v = reinterpret_cast<const f32x4*>(part_ml)[ri];
        m = v[0];
        l = v[1];
        // the element goes through a scalar first: this compiler's bit cast of
        // a vector element reads element 0
        const float e = v[2];
        ebits = __builtin_bit_cast(uint32_t, e);
      } else {
        const float2 v = reinterpret_cast<const float2*>(part_ml)[ri];
        m = v.x;
        l = v.y;
      }
    }
    // cross-lane work by DPP moves and v_readlane (no LDS crossbar trips)
    const float Mc = wave_max_uniform(m);
    const float Mn = fmaxf(M, Mc);
    if (Mn == -INFINITY) continue;  // no tokens in any range so far
    const float rescale = fast_exp2(M - Mn);
    const float wl = m == -INFINITY ? 0.f : fast_exp2(m - Mn);
    const float Lc = wave_sum_uniform(l * wl);
    L = L * rescale + Lc;
    M = Mn;
#pragma unroll
    for (int c = 0; c < kDPL / 4; ++c) acc[c] *= rescale;
    // weight of a row: fp32 sums 2^(m - M); fp16 rows 2^(m - M) l, times 2^e
    // of the quarter this lane reads
    const float wrow = F16 ? wl * l : wl;
    const int cnt = NR - r0 < 64 ? NR - r0 : 64;
    for (int k0 = 0; k0 < cnt; k0 += kBatch) {
      f32x4 v[kBatch][kDPL / 4];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int k = k0 + u < cnt ? k0 + u : cnt - 1;
        const size_t row = ((static_cast<size_t>(b) * NR + r0 + k) * H + h) * kC + lane * kDPL;
        if constexpr (F16) {
          typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
          const f16x8 x = *reinterpret_cast<const f16x8*>(static_cast<const _Float16*>(part_o) + row);
          v[u][0] = f32x4{static_cast<float>(x[0]), static_cast<float>(x[1]),
                          static_cast<float>(x[2]), static_cast<float>(x[3])};
          v[u][1] = f32x4{static_cast<float>(x[4]), static_cast<float>(x[5]),
                          static_cast<float>(x[6]), static_cast<float>(x[7])};
        } else {
          const f32x4* po = reinterpret_cast<const f32x4*>(static_cast<const float*>(part_o) + row);
#pragma unroll
          for (int c = 0; c < kDPL / 4; ++c) v[u][c] = po[c];
        }
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        float wk = k0 + u < cnt ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                      __builtin_bit_cast(int, wrow), k0 + u))
                                : 0.f;
        if constexpr (F16) {
          wk *= quarter_scale(__builtin_amdgcn_readlane(ebits, k0 + u), 8 * (lane >> 4));
        }
        // a range without tokens has weight 0 and an all-zero row
#pragma unroll
        for (int c = 0; c < kDPL / 4; ++c) acc[c] += v[u][c] * wk;
      }
    }
  }
}

// At most kSmallRanges fp16 range partials (the usual case): the statistics
// and every partial row are loaded before any is used -- one memory round
// trip, where merge_ranges waits for the statistics before it loads a row --
// and combined with the same arithmetic in the same order as merge_ranges
// (weights 2^(m - M) l 2^e, lane r holding range r; rows r >= NR are copies
// of row NR - 1 with weight 0), so both give the same bits.
constexpr int kSmallRanges = 16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

struct SmallRanges {
  f32x4 st;  // lane r < NR: (m, l, e bytes, 0) of range r
  f16x8 rows[kSmallRanges];
};

__device__ __forceinline__ void load_small_ranges(const void* __restrict__ part_o16,
                                                  const float* __restrict__ part_ml, int b,
                                                  int h, int H, int NR, int lane,
                                                  SmallRanges& sr) {
  sr.st = f32x4{-INFINITY, 0.f, 0.f, 0.f};
  if (lane < NR) {
    sr.st = reinterpret_cast<const f32x4*>(part_ml)[(static_cast<size_t>(b) * NR + lane) * H + h];
  }
#pragma unroll
  for (int r = 0; r < kSmallRanges; ++r) {
    const int rr = r < NR ? r : NR - 1;
    sr.rows[r] = *reinterpret_cast<const f16x8*>(
        static_cast<const _Float16*>(part_o16) +
        ((static_cast<size_t>(b) * NR + rr) * H + h) * kC + lane * kDPL);
  }
}

__device__ __forceinline__ void combine_small_ranges(const SmallRanges& sr, int NR, int lane,
                                                     f32x4 (&acc)[kDPL / 4], float& M, float& L) {
  const float m = sr.st[0], l = sr.st[1];
  const float e = sr.st[2];  // through a scalar, as in merge_ranges
  const uint32_t ebits = __builtin_bit_cast(uint32_t, e);
  M = wave_max_uniform(m);
  const float wl = m == -INFINITY ? 0.f : fast_exp2(m - M);
  L = wave_sum_uniform(l * wl);
  const float wrow = wl * l;
  acc[0] = acc[1] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (M == -INFINITY) return;  // no tokens in any range
#pragma unroll
  for (int r = 0; r < kSmallRanges; ++r) {
    const float wk =
        r < NR ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wrow), r)) *
                     quarter_scale(__builtin_amdgcn_readlane(ebits, r), 8 * (lane >> 4))
               : 0.f;
    const f16x8& x = sr.rows[r];
    acc[0] += f32x4{static_cast<float>(x[0]), static_cast<float>(x[1]), static_cast<float>(x[2]),
                    static_cast<float>(x[3])} * wk;
    acc[1] += f32x4{static_cast<float>(x[4]), static_cast<float>(x[5]), static_cast<float>(x[6]),
                    static_cast<float>(x[7])} * wk;
  }
}

// The merged row as bf16 (dims 8 lane .. + 7, one 16-byte word per lane).
__device__ __forceinline__ u32x4 merged_row_bf16(const f32x4 (&acc)[kDPL / 4], float L) {
  const float inv = L > 0.f ? 1.f / L : 0.f;
  return u32x4{pack_bf16x2(acc[0][0] * inv, acc[0][1] * inv),
               pack_bf16x2(acc[0][2] * inv, acc[0][3] * inv),
               pack_bf16x2(acc[1][0] * inv, acc[1][1] * inv),
               pack_bf16x2(acc[1][2] * inv, acc[1][3] * inv)};
}

__device__ __forceinline__ float merged_lse(float M, float L) {
  return L > 0.f ? (M + __log2f(L)) * 0.6931471805599453f : -INFINITY;
}

// One wavefront per (sequence, head): merges the range partials into
// weighted_c [B, H, 512] bf16 (and the log-sum-exp).
template <bool F16>
__global__ __launch_bounds__(kThreads) void mla_reduce_kernel(
    const void* __restrict__ part_o, const float* __restrict__ part_ml,
    uint16_t* __restrict__ out, float* __restrict__ lse_out, int B, int H, int NR) {
  const int lane = threadIdx.x & 63;
  const int task = blockIdx.x * (kThreads / 64) + uniform(threadIdx.x >> 6);
  if (task >= B * H) return;
  const int b = task / H;
  const int h = task - b * H;
  f32x4 acc[kDPL / 4];
  float M, L;
  if (F16 && NR <= kSmallRanges) {
    SmallRanges sr;
    load_small_ranges(part_o, part_ml, b, h, H, NR, lane, sr);
    combine_small_ranges(sr, NR, lane, acc, M, L);
  } else {
    merge_ranges<F16>(part_o, part_ml, b, h, H, NR, lane, acc, M, L);
  }
  *reinterpret_cast<u32x4*>(out + static_cast<size_t>(task) * kC + lane * kDPL) =
      merged_row_bf16(acc, L);
  if (lse_out != nullptr && lane == 0) lse_out[task] = merged_lse(M, L);
}

// Merge and output projection fused, one workgroup per head (64-head-group
// partials): weighted_c [b, h, :] for every sequence b, rounded to bf16 as the
// reference rounds it (runtime/glm.py:162-164), then y [b, h, :dv] =
// weighted_c . W_UV (runtime/glm.py:200-202) on v_mfma_f32_16x16x32_bf16 with
// the sequences as the M = 16 dimension.  W_UV[h] (packed as for
// voom_mla_head_gemv, dv <= 128: at most 128 KiB) streams into LDS from the
// first instruction on, beside the partial rows the merge reads, so one
// launch replaces the merge and the projection's weight stream.  Eight
// wavefronts: wavefront w merges sequences w, w + 8, then projects column
// tiles w, w + 8.
constexpr int kRpMaxTiles = 8;                 // dv <= 128
constexpr int kRpSteps = kC / kHgStep;         // 16 k-steps over the 512 latent dims
constexpr int kRpThreads = 512;                // 8 wavefronts: one per sequence, one per tile
__global__ __launch_bounds__(kRpThreads) void mla_reduce_project_kernel(
    const void* __restrict__ part_o16, const float* __restrict__ part_ml,
    const uint16_t* __restrict__ w_uv, uint16_t* __restrict__ y, uint16_t* __restrict__ wc_out,
    float* __restrict__ lse_out, int B, int H, int NR, int DV, int NT, int splits) {
  __shared__ __attribute__((aligned(16))) uint16_t wl[kRpMaxTiles * kRpSteps * 512];
  __shared__ __attribute__((aligned(16))) uint16_t wcs[16][kC + 8];
  // workgroups h + H part (same XCD for every part of a head when H % 8 == 0,
  // so the parts' reads of the head's partial rows meet in one L2) split the
  // head's column tiles; each merges all rows, part 0 writes weighted_c / lse
  const int h = blockIdx.x % H;
  const int part = blockIdx.x / H;
  const int tpp = (NT + splits - 1) / splits;  // column tiles per part
  const int nt_lo = part * tpp;
  const int nt_hi = nt_lo + tpp < NT ? nt_lo + tpp : NT;
  const int lane = threadIdx.x & 63;
  const int w = uniform(threadIdx.x >> 6);
  constexpr int kWaves = kRpThreads / kWave;
  // The merge's loads go out first (statistics and, for up to kSmallRanges
  // ranges, every partial row), then the weight stream: the merge waits only
  // for its own loads, which the wait counter drains in issue order.
  const int bw = w < B ? w : 0;  // wavefronts past B merge row 0 and keep nothing
  const bool small = NR <= kSmallRanges;
  SmallRanges sr;
  if (small) load_small_ranges(part_o16, part_ml, bw, h, H, NR, lane, sr);
  {
    // this part's tiles: blocks nt_lo * 16 .. nt_hi * 16 (1 KiB each) of the head
    const int blocks = (nt_hi - nt_lo) * kRpSteps;
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(w_uv + (static_cast<size_t>(h) * NT + nt_lo) * kRpSteps * 512),
        static_cast<short>(0), blocks * 1024, 0x00020000);
    for (int i = w; i < blocks; i += kWaves) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)(wl + i * 512), 16, i * 1024 + lane * 16,
                                               0, 0, 0);
    }
  }
  for (int b = w; b < B; b += kWaves) {
    f32x4 acc[kDPL / 4];
    float M, L;
    if (small && b == w) {
      combine_small_ranges(sr, NR, lane, acc, M, L);  // the rows loaded at kernel start
    } else {
      merge_ranges<true>(part_o16, part_ml, b, h, H, NR, lane, acc, M, L);
    }
    const u32x4 row = merged_row_bf16(acc, L);
    *reinterpret_cast<u32x4*>(&wcs[b][lane * kDPL]) = row;
    const size_t task = static_cast<size_t>(b) * H + h;
    if (part == 0 && wc_out != nullptr) {
      *reinterpret_cast<u32x4*>(wc_out + task * kC + lane * kDPL) = row;
    }
    if (part == 0 && lse_out != nullptr && lane == 0) lse_out[task] = merged_lse(M, L);
  }
  wait_vmem_all();  // this wave's weight loads; the barrier makes it everyone's
  lds_barrier();
  const int bq = lane & 15;
  const int kq = 8 * (lane >> 4);
  for (int nt = nt_lo + w; nt < nt_hi; nt += kWaves) {
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < kRpSteps; ++s) {
      const u32x4 av = bq < B ? *reinterpret_cast<const u32x4*>(&wcs[bq][kHgStep * s + kq])
                              : u32x4{0u, 0u, 0u, 0u};
      const u32x4 bv =
          *reinterpret_cast<const u32x4*>(wl + ((nt - nt_lo) * kRpSteps + s) * 512 + lane * 8);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av),
                                                    __builtin_bit_cast(bf16x8, bv), acc, 0, 0, 0);
    }
    const int n = kHgTile * nt + (lane & 15);
    if (n < DV) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 4 * (lane >> 4) + r;
        if (row < B) y[(static_cast<size_t>(row) * H + h) * DV + n] = f2bf(acc[r]);
      }
    }
  }
}

// Heads per workgroup for a head count: 64 when it divides, else 32.
int heads_per_group(int H) { return H % 64 == 0 ? 64 : 32; }

int default_ranges(int B, int H) {
  const int wgs_per_range = B * (H / heads_per_group(H));
  int nr = (device_cu_count() + wgs_per_range - 1) / wgs_per_range;
  return nr < 1 ? 1 : nr;
}

// Latent kernel (dense or sparse) and the range reduce.
int launch_mla(const MlaArgs& a, int hg, bool sparse, long long grid, uint16_t* out,
               float* lse_out, hipStream_t stream) {
  const dim3 g(static_cast<unsigned>(grid));
  if (hg == 64) {
    if (sparse) {
      hipLaunchKernelGGL((mla_group64_kernel<true>), g, dim3(kGThreads), 0, stream, a);
    } else {
      hipLaunchKernelGGL((mla_group64_kernel<false>), g, dim3(kGThreads), 0, stream, a);
    }
  } else {
    if (sparse) {
      hipLaunchKernelGGL((mla_latent_kernel<32, true>), g, dim3(kMlaThreads), 0, stream, a);
    } else {
      hipLaunchKernelGGL((mla_latent_kernel<32, false>), g, dim3(kMlaThreads), 0, stream, a);
    }
  }
  int rc = VOOM_LAUNCH_CHECK("mla: latent kernel launch");
  if (rc) return rc;
  const unsigned red_grid = static_cast<unsigned>((a.B * a.H + 3) / 4);
  if (hg == 64) {
    hipLaunchKernelGGL(mla_reduce_kernel<true>, dim3(red_grid), dim3(kThreads), 0, stream,
                       static_cast<const void*>(a.part_o16), a.part_ml, out, lse_out, a.B, a.H, a.NR);
  } else {
    hipLaunchKernelGGL(mla_reduce_kernel<false>, dim3(red_grid), dim3(kThreads), 0, stream,
                       static_cast<const void*>(a.part_o), a.part_ml, out, lse_out, a.B, a.H, a.NR);
  }
  return VOOM_LAUNCH_CHECK("mla: reduce kernel launch");
}

// Latent kernel (64-head groups) and the fused merge + output projection.
int launch_mla_project(const MlaArgs& a, long long grid, const void* w_uv_packed, int dv,
                       void* y, uint16_t* wc_out, float* lse_out, hipStream_t stream) {
  hipLaunchKernelGGL((mla_group64_kernel<false>), dim3(static_cast<unsigned>(grid)),
                     dim3(kGThreads), 0, stream, a);
  int rc = VOOM_LAUNCH_CHECK("mla: latent kernel launch");
  if (rc) return rc;
  const int nt = (dv + kHgTile - 1) / kHgTile;
  // two parts per head when there are at least two column tiles: twice the
  // workgroups for the weight stream
  const int splits = nt >= 2 ? 2 : 1;
  hipLaunchKernelGGL(mla_reduce_project_kernel, dim3(static_cast<unsigned>(a.H * splits)),
                     dim3(kRpThreads), 0, stream, static_cast<const void*>(a.part_o16), a.part_ml,
                     static_cast<const uint16_t*>(w_uv_packed), static_cast<uint16_t*>(y), wc_out,
                     lse_out, a.B, a.H, a.NR, dv, nt, splits);
  return VOOM_LAUNCH_CHECK("mla: merge + projection kernel launch");
}

// Ranges for a selection of at most sel_stride positions: one per two 64-row
// tiles (a selection is short, and every range costs a partial row per head
// that the reduce reads back) unless the dense default is lower, and never so
// few that a range holds more than kPre tiles.
int sparse_min_ranges(int sel_stride) {
  const int tiles = (sel_stride + kTile - 1) / kTile;
  return (tiles + kPre - 1) / kPre;
}

int sparse_ranges(int B, int H, int sel_stride) {
  const int by_tiles = (sel_stride + 2 * kTile - 1) / (2 * kTile);
  int nr = default_ranges(B, H);
  nr = nr < by_tiles ? nr : by_tiles;
  const int lo = sparse_min_ranges(sel_stride);
  return nr < lo ? lo : (nr < 1 ? 1 : nr);
}

// ------------------------------------------------------ per-head products ----
// y[b, h, n] = sum_k x[b, h, k] w[h, k, n] for the few query rows of a decode
// step (B <= 16): q_nope . W_UK and weighted_c . W_UV^T of absorbed MLA.  The
// work is a weight stream (2 x 16.8 MB at config 5 against 1 MB of rows), and
// fp32 FMAs over it would cost as much VALU time as the stream takes, so the
// products run on v_mfma_f32_16x16x32_bf16 with the batch as the (padded)
// M = 16 dimension: A = x rows, B = a 32 x 16 block of w.
//
// Weights are packed once (voom_mla_pack_head_weights) in MFMA operand order:
// for head h, column tile nt (16 columns) and k-step s (32 rows) a 1 KiB
// block in which lane l holds w[32 s + 8 (l / 16) + e][16 nt + l % 16],
// e = 0..7 -- every weight load is one contiguous 1 KiB per wavefront.  K and
// N are zero-padded to multiples of 32 and 16.
constexpr int kHgChunk = 16;    // k-steps whose weight loads are issued together

// Packs w [H, K, N] (bf16) into [H, Np / 16, Kp / 32, 64, 8].
__global__ __launch_bounds__(kThreads) void pack_head_weights_kernel(
    const uint16_t* __restrict__ w, uint16_t* __restrict__ wp, int H, int K, int N, int NT,
    int KS) {
  const long long total = static_cast<long long>(H) * NT * KS * 64;
  const long long p = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
  if (p >= total) return;
  const int l = static_cast<int>(p & 63);
  long long r = p >> 6;
  const int s = static_cast<int>(r % KS);
  r /= KS;
  const int nt = static_cast<int>(r % NT);
  const int h = static_cast<int>(r / NT);
  const int n = kHgTile * nt + (l & 15);
  const int k0 = kHgStep * s + 8 * (l >> 4);
  uint32_t v[4];
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const int ka = k0 + e, kb = k0 + e + 1;
    const uint32_t lo = (ka < K && n < N) ? w[(static_cast<size_t>(h) * K + ka) * N + n] : 0u;
    const uint32_t hi = (kb < K && n < N) ? w[(static_cast<size_t>(h) * K + kb) * N + n] : 0u;
    v[e >> 1] = lo | (hi << 16);
  }
  *reinterpret_cast<u32x4*>(wp + p * 8) = u32x4{v[0], v[1], v[2], v[3]};
}

// Each wavefront takes TPW adjacent 16-column tiles of one head and walks K in
// chunks of KC k-steps; the TPW x KC = 16 weight loads of a chunk (16 KiB per
// wavefront) are all issued before its first MFMA, and the x operands of a
// k-step serve all TPW tiles.  Four wavefronts per workgroup, no LDS and no
// barriers.  Lane l's x operand is row b = l % 16 (zero for b >= B) at k =
// 32 s + 8 (l / 16) .. + 7; a 16 x 16 result has lane l holding column l % 16
// of rows 4 (l / 16) .. + 3.  tail (optional): tail[b, h, 0 .. tail_cols) is
// copied to y[b, h, N ..] by the first wavefront of each head (q_rope beside
// q_nope . W_UK in q_lat).
template <int KC, int TPW>
__global__ __launch_bounds__(kThreads) void head_gemv_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wp, uint16_t* __restrict__ y,
    const uint16_t* __restrict__ tail, int B, int H, int K, int N, int NT, int KS, int x_stride,
    int y_stride, int x_vec, int tail_cols, int tail_stride) {
  static_assert(KC * TPW == kHgChunk, "16 weight loads per chunk");
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = blockIdx.x * (kThreads / kWave) + uniform(threadIdx.x / kWave);
  const int h = blockIdx.y;
  if (tail != nullptr && wave == 0) {
    for (int c = lane; c < tail_cols; c += kWave) {
      for (int bb = 0; bb < B; ++bb) {
        y[(static_cast<size_t>(bb) * H + h) * y_stride + N + c] =
            tail[(static_cast<size_t>(bb) * H + h) * tail_stride + c];
      }
    }
  }
  const int nt0 = wave * TPW;
  if (nt0 >= NT) return;
  const int b = lane & 15;
  const int kq = 8 * (lane >> 4);
  const uint16_t* xr = x + (static_cast<size_t>(b < B ? b : 0) * H + h) * x_stride;
  f32x4 acc[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < KS; s0 += KC) {
    u32x4 wq[TPW][KC];
    u32x4 xq[KC];
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      // tiles past NT and k-steps past KS reread a valid block, unused
      const int nt = nt0 + j < NT ? nt0 + j : NT - 1;
      const u32x4* wt = reinterpret_cast<const u32x4*>(wp) +
                        (static_cast<size_t>(h) * NT + nt) * KS * 64 + lane;
#pragma unroll
      for (int i = 0; i < KC; ++i) {
        const int s = s0 + i < KS ? s0 + i : KS - 1;
        wq[j][i] = __builtin_nontemporal_load(wt + static_cast<size_t>(s) * 64);
      }
    }
#pragma unroll
    for (int i = 0; i < KC; ++i) {
      const int k = kHgStep * (s0 + i) + kq;
      if (x_vec) {
        // rows 16-byte aligned with K % 8 == 0: whole 8-element pieces
        xq[i] = (b < B && k < K) ? *reinterpret_cast<const u32x4*>(xr + k)
                                 : u32x4{0u, 0u, 0u, 0u};
      } else {
        uint32_t v[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          const uint32_t lo = (b < B && k + e < K) ? xr[k + e] : 0u;
          const uint32_t hi = (b < B && k + e + 1 < K) ? xr[k + e + 1] : 0u;
          v[e >> 1] = lo | (hi << 16);
        }
        xq[i] = u32x4{v[0], v[1], v[2], v[3]};
      }
    }
#pragma unroll
    for (int i = 0; i < KC; ++i) {
      if (s0 + i < KS) {
#pragma unroll
        for (int j = 0; j < TPW; ++j) {
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xq[i]),
                                                           __builtin_bit_cast(bf16x8, wq[j][i]),
                                                           acc[j], 0, 0, 0);
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int n = kHgTile * (nt0 + j) + (lane & 15);
    if (nt0 + j < NT && n < N) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 4 * (lane >> 4) + r;
        if (row < B) y[(static_cast<size_t>(row) * H + h) * y_stride + n] = f2bf(acc[j][r]);
      }
    }
  }
}

int launch_head_gemv(const void* x, const void* w_packed, void* y, const void* tail, int batch,
                     int num_heads, int k, int n, int x_stride, int y_stride, int tail_cols,
                     int tail_stride, hipStream_t stream) {
  const int nt = (n + kHgTile - 1) / kHgTile;
  const int ks = (k + kHgStep - 1) / kHgStep;
  const int x_vec = (k % 8 == 0 && x_stride % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0);
  // short K: several tiles per wavefront share each x operand
  const int tpw = ks <= 4 ? 4 : (ks <= 8 ? 2 : 1);
  const int waves = (nt + tpw - 1) / tpw;
  const dim3 grid(static_cast<unsigned>((waves + kThreads / kWave - 1) / (kThreads / kWave)),
                  static_cast<unsigned>(num_heads));
  const auto* xv = static_cast<const uint16_t*>(x);
  const auto* wv = static_cast<const uint16_t*>(w_packed);
  auto* yv = static_cast<uint16_t*>(y);
  const auto* tv = static_cast<const uint16_t*>(tail);
  if (tpw == 4) {
    hipLaunchKernelGGL((head_gemv_kernel<4, 4>), grid, dim3(kThreads), 0, stream, xv, wv, yv, tv,
                       batch, num_heads, k, n, nt, ks, x_stride, y_stride, x_vec, tail_cols,
                       tail_stride);
  } else if (tpw == 2) {
    hipLaunchKernelGGL((head_gemv_kernel<8, 2>), grid, dim3(kThreads), 0, stream, xv, wv, yv, tv,
                       batch, num_heads, k, n, nt, ks, x_stride, y_stride, x_vec, tail_cols,
                       tail_stride);
  } else {
    hipLaunchKernelGGL((head_gemv_kernel<16, 1>), grid, dim3(kThreads), 0, stream, xv, wv, yv, tv,
                       batch, num_heads, k, n, nt, ks, x_stride, y_stride, x_vec, tail_cols,
                       tail_stride);
  }
  return VOOM_LAUNCH_CHECK("mla_head_gemv: kernel launch");
}

}  // namespace
}  // namespace voom

using namespace voom;

namespace voom {
namespace {
// Workspace of n = batch x ranges x heads partial rows: the rows (fp32 sums
// for 32-head groups, fp16 for 64-head groups), 256-byte aligned, then the
// per-row statistics ((m, l), or (m, l, e, 0) with the fp16 rows).
size_t partial_rows_bytes(size_t n, int H) {
  const size_t row = heads_per_group(H) == 64 ? kC * 2 : kC * sizeof(float);
  return (n * row + 255) & ~size_t(255);
}
size_t partial_bytes(size_t n, int H) {
  return partial_rows_bytes(n, H) + n * (heads_per_group(H) == 64 ? 4 : 2) * sizeof(float);
}
void set_partials(MlaArgs& a, void* workspace, size_t n) {
  a.part_o = static_cast<float*>(workspace);
  a.part_o16 = workspace;
  a.part_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) + partial_rows_bytes(n, a.H));
}
}  // namespace
}  // namespace voom

extern "C" size_t voom_mla_sparse_workspace_bytes(int batch, int num_heads, int sel_stride,
                                                  int num_ranges) {
  if (batch <= 0 || num_heads <= 0 || sel_stride <= 0) return 0;
  if (num_ranges <= 0) num_ranges = sparse_ranges(batch, num_heads, sel_stride);
  return partial_bytes(static_cast<size_t>(batch) * num_ranges * num_heads, num_heads);
}

extern "C" size_t voom_mla_workspace_bytes(int batch, int num_heads, int num_ranges) {
  if (batch <= 0 || num_heads <= 0) return 0;
  if (num_ranges <= 0) num_ranges = default_ranges(batch, num_heads);
  return partial_bytes(static_cast<size_t>(batch) * num_ranges * num_heads, num_heads);
}

namespace voom {
namespace {
// Checks of the dense latent decode's arguments; fills `a` and the grid.
int prepare_dense(const char* who, const void* q_lat, const void* lat_pool,
                  const int32_t* block_table, const int32_t* ctx_lens, void* workspace,
                  size_t ws_bytes, int batch, int num_heads, int latent_dim, int c_dim,
                  int page_tokens, int max_pages, int num_slots, float scale, int num_ranges,
                  MlaArgs& a, long long& grid) {
  VOOM_REQUIRE(q_lat && lat_pool && block_table && ctx_lens && workspace,
               "%s: null pointer argument", who);
  VOOM_REQUIRE(latent_dim == kLat && c_dim == kC, "%s: latent %d / c_dim %d unsupported (576 / 512)",
               who, latent_dim, c_dim);
  VOOM_REQUIRE(batch > 0 && num_heads > 0 && num_heads % 32 == 0,
               "%s: num_heads %d must be a positive multiple of 32", who, num_heads);
  VOOM_REQUIRE(is_pow2(page_tokens) && page_tokens >= kTile && page_tokens <= 4096,
               "%s: page_tokens %d must be a power of two in [64, 4096]", who, page_tokens);
  VOOM_REQUIRE(max_pages > 0 && num_slots > 0, "%s: empty table or pool", who);
  VOOM_REQUIRE(scale > 0.f && scale < INFINITY, "%s: scale %g must be positive", who,
               static_cast<double>(scale));
  VOOM_REQUIRE(static_cast<long long>(max_pages) * page_tokens < (1LL << 30),
               "%s: table capacity too large", who);
  if (num_ranges <= 0) num_ranges = default_ranges(batch, num_heads);
  const size_t need = voom_mla_workspace_bytes(batch, num_heads, num_ranges);
  VOOM_REQUIRE(ws_bytes >= need, "%s: workspace %zu bytes < required %zu", who, ws_bytes, need);
  VOOM_REQUIRE(reinterpret_cast<uintptr_t>(q_lat) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(lat_pool) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(workspace) % 16 == 0,
               "%s: q, pool and workspace must be 16-byte aligned", who);
  const int hg = heads_per_group(num_heads);
  grid = static_cast<long long>(batch) * num_ranges * (num_heads / hg);
  VOOM_REQUIRE(grid < (1LL << 31), "%s: grid too large", who);
  a.q = static_cast<const uint16_t*>(q_lat);
  a.lat = static_cast<const uint16_t*>(lat_pool);
  a.table = block_table;
  a.ctx_lens = ctx_lens;
  a.B = batch;
  a.H = num_heads;
  set_partials(a, workspace, static_cast<size_t>(batch) * num_ranges * num_heads);
  a.NR = num_ranges;
  a.max_pages = max_pages;
  a.pt_shift = ilog2(page_tokens);
  a.num_slots = num_slots;
  a.scale_log2e = scale * 1.4426950408889634f;
  a.sel = nullptr;
  a.sel_stride = 0;
  a.pool_bytes = 0;
  return VOOM_OK;
}
}  // namespace
}  // namespace voom

extern "C" int voom_mla_absorbed_decode(const void* q_lat, const void* lat_pool,
                                        const int32_t* block_table, const int32_t* ctx_lens,
                                        void* out_c, float* lse_out, void* workspace,
                                        size_t ws_bytes, int batch, int num_heads,
                                        int latent_dim, int c_dim, int page_tokens, int max_pages,
                                        int num_slots, float scale, int num_ranges,
                                        hipStream_t stream) {
  const char* who = "mla_absorbed_decode";
  VOOM_REQUIRE(out_c != nullptr, "%s: null pointer argument", who);
  MlaArgs a;
  long long grid = 0;
  const int rc = prepare_dense(who, q_lat, lat_pool, block_table, ctx_lens, workspace, ws_bytes,
                               batch, num_heads, latent_dim, c_dim, page_tokens, max_pages,
                               num_slots, scale, num_ranges, a, grid);
  if (rc) return rc;
  return launch_mla(a, heads_per_group(num_heads), false, grid, static_cast<uint16_t*>(out_c),
                    lse_out, stream);
}

extern "C" int voom_mla_absorbed_decode_project(
    const void* q_lat, const void* lat_pool, const int32_t* block_table, const int32_t* ctx_lens,
    const void* w_uv_packed, int dv, void* y, void* wc_out, float* lse_out, void* workspace,
    size_t ws_bytes, int batch, int num_heads, int latent_dim, int c_dim, int page_tokens,
    int max_pages, int num_slots, float scale, int num_ranges, hipStream_t stream) {
  const char* who = "mla_absorbed_decode_project";
  VOOM_REQUIRE(w_uv_packed && y, "%s: null pointer argument", who);
  VOOM_REQUIRE(num_heads % 64 == 0, "%s: num_heads %d must be a multiple of 64", who, num_heads);
  VOOM_REQUIRE(batch <= 16, "%s: batch %d must be at most 16", who, batch);
  VOOM_REQUIRE(dv >= 1 && dv <= kRpMaxTiles * kHgTile, "%s: dv %d must be 1..%d", who, dv,
               kRpMaxTiles * kHgTile);
  VOOM_REQUIRE(reinterpret_cast<uintptr_t>(w_uv_packed) % 16 == 0,
               "%s: w_uv_packed must be 16-byte aligned", who);
  MlaArgs a;
  long long grid = 0;
  const int rc = prepare_dense(who, q_lat, lat_pool, block_table, ctx_lens, workspace, ws_bytes,
                               batch, num_heads, latent_dim, c_dim, page_tokens, max_pages,
                               num_slots, scale, num_ranges, a, grid);
  if (rc) return rc;
  return launch_mla_project(a, grid, w_uv_packed, dv, y, static_cast<uint16_t*>(wc_out), lse_out,
                            stream);
}

extern "C" int voom_mla_sparse_decode(const void* q_lat, const void* lat_pool,
                                      const int32_t* block_table, const int32_t* sel,
                                      const int32_t* sel_lens, void* out_c, float* lse_out,
                                      void* workspace, size_t ws_bytes, int batch, int num_heads,
                                      int latent_dim, int c_dim, int page_tokens, int max_pages,
                                      int num_slots, int sel_stride, float scale, int num_ranges,
                                      hipStream_t stream) {
  const char* who = "mla_sparse_decode";
  VOOM_REQUIRE(q_lat && lat_pool && block_table && sel && sel_lens && out_c && workspace,
               "%s: null pointer argument", who);
  VOOM_REQUIRE(latent_dim == kLat && c_dim == kC, "%s: latent %d / c_dim %d unsupported (576 / 512)",
               who, latent_dim, c_dim);
  VOOM_REQUIRE(batch > 0 && num_heads > 0 && num_heads % 32 == 0,
               "%s: num_heads %d must be a positive multiple of 32", who, num_heads);
  VOOM_REQUIRE(is_pow2(page_tokens) && page_tokens >= kTile && page_tokens <= 4096,
               "%s: page_tokens %d must be a power of two in [64, 4096]", who, page_tokens);
  VOOM_REQUIRE(max_pages > 0 && num_slots > 0 && sel_stride > 0, "%s: empty table, pool or selection",
               who);
  VOOM_REQUIRE(scale > 0.f && scale < INFINITY, "%s: scale %g must be positive", who,
               static_cast<double>(scale));
  const unsigned long long pool =
      static_cast<unsigned long long>(num_slots) * page_tokens * kLat * 2;
  VOOM_REQUIRE(pool < 0xFFFF0000ull,
               "%s: latent pool of %llu bytes exceeds the 4 GiB a gathered load can address", who,
               pool);
  if (num_ranges <= 0) num_ranges = sparse_ranges(batch, num_heads, sel_stride);
  VOOM_REQUIRE(num_ranges >= sparse_min_ranges(sel_stride),
               "%s: %d ranges leave more than %d tiles per range (at least %d needed)", who,
               num_ranges, kPre, sparse_min_ranges(sel_stride));
  const size_t need = voom_mla_workspace_bytes(batch, num_heads, num_ranges);
  VOOM_REQUIRE(ws_bytes >= need, "%s: workspace %zu bytes < required %zu", who, ws_bytes, need);
  VOOM_REQUIRE(reinterpret_cast<uintptr_t>(q_lat) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(lat_pool) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(workspace) % 16 == 0,
               "%s: q, pool and workspace must be 16-byte aligned", who);
  const int hg = heads_per_group(num_heads);
  const long long grid = static_cast<long long>(batch) * num_ranges * (num_heads / hg);
  VOOM_REQUIRE(grid < (1LL << 31), "%s: grid too large", who);

  const size_t n = static_cast<size_t>(batch) * num_ranges * num_heads;
  MlaArgs a;
  a.q = static_cast<const uint16_t*>(q_lat);
  a.lat = static_cast<const uint16_t*>(lat_pool);
  a.table = block_table;
  a.ctx_lens = sel_lens;
  a.sel = sel;
  a.B = batch;
  a.H = num_heads;
  set_partials(a, workspace, n);
  a.NR = num_ranges;
  a.max_pages = max_pages;
  a.pt_shift = ilog2(page_tokens);
  a.num_slots = num_slots;
  a.sel_stride = sel_stride;
  a.pool_bytes = static_cast<uint32_t>(pool);
  a.scale_log2e = scale * 1.4426950408889634f;
  return launch_mla(a, hg, true, grid, static_cast<uint16_t*>(out_c), lse_out, stream);
}

extern "C" size_t voom_mla_head_weights_bytes(int num_heads, int k, int n) {
  if (num_heads <= 0 || k <= 0 || n <= 0) return 0;
  const size_t nt = (n + kHgTile - 1) / kHgTile;
  const size_t ks = (k + kHgStep - 1) / kHgStep;
  return static_cast<size_t>(num_heads) * nt * ks * 64 * 8 * 2;
}

extern "C" int voom_mla_pack_head_weights(const void* w, void* w_packed, int num_heads, int k,
                                          int n, hipStream_t stream) {
  const char* who = "mla_pack_head_weights";
  VOOM_REQUIRE(w && w_packed, "%s: null pointer argument", who);
  VOOM_REQUIRE(num_heads >= 1 && k >= 1 && n >= 1, "%s: empty weights", who);
  VOOM_REQUIRE(reinterpret_cast<uintptr_t>(w_packed) % 16 == 0, "%s: w_packed must be 16-byte aligned",
               who);
  const int nt = (n + kHgTile - 1) / kHgTile;
  const int ks = (k + kHgStep - 1) / kHgStep;
  const long long total = static_cast<long long>(num_heads) * nt * ks * 64;
  VOOM_REQUIRE(total / kThreads < (1LL << 31), "%s: weights too large", who);
  hipLaunchKernelGGL(pack_head_weights_kernel, dim3(static_cast<unsigned>((total + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, stream, static_cast<const uint16_t*>(w),
                     static_cast<uint16_t*>(w_packed), num_heads, k, n, nt, ks);
  return VOOM_LAUNCH_CHECK("mla_pack_head_weights: kernel launch");
}

extern "C" int voom_mla_head_gemv(const void* x, const void* w_packed, void* y, int batch,
                                  int num_heads, int k, int n, int x_stride, int y_stride,
                                  hipStream_t stream) {
  const char* who = "mla_head_gemv";
  VOOM_REQUIRE(x && w_packed && y, "%s: null pointer argument", who);
  VOOM_REQUIRE(batch >= 1 && batch <= 16 && num_heads >= 1, "%s: batch must be 1..16", who);
  VOOM_REQUIRE(k >= 1 && n >= 1, "%s: k %d and n %d must be positive", who, k, n);
  VOOM_REQUIRE(x_stride >= k && y_stride >= n, "%s: row strides below k / n", who);
  VOOM_REQUIRE(reinterpret_cast<uintptr_t>(w_packed) % 16 == 0,
               "%s: w_packed must be 16-byte aligned", who);
  return launch_head_gemv(x, w_packed, y, nullptr, batch, num_heads, k, n, x_stride, y_stride, 0,
                          0, stream);
}

extern "C" int voom_mla_absorb_query(const void* q_nope, const void* q_rope, const void* w_uk_packed,
                                     void* q_lat, int batch, int num_heads, int dn, int c_dim,
                                     int rope_dim, hipStream_t stream) {
  const char* who = "mla_absorb_query";
  VOOM_REQUIRE(q_nope && q_rope && w_uk_packed && q_lat, "%s: null pointer argument", who);
  VOOM_REQUIRE(batch >= 1 && batch <= 16 && num_heads >= 1, "%s: batch must be 1..16", who);
  VOOM_REQUIRE(dn >= 1 && c_dim >= 1 && rope_dim >= 0, "%s: empty dimensions", who);
  VOOM_REQUIRE(reinterpret_cast<uintptr_t>(w_uk_packed) % 16 == 0,
               "%s: w_uk_packed must be 16-byte aligned", who);
  return launch_head_gemv(q_nope, w_uk_packed, q_lat, rope_dim > 0 ? q_rope : nullptr, batch,
                          num_heads, dn, c_dim, dn, c_dim + rope_dim, rope_dim, rope_dim, stream);
}
