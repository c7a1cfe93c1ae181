// Triangle multiplicative update (TriMul) on gfx950, built on the MFMA GEMM
// main loop of gemm_core.hpp with the gating / LayerNorm work fused into
// GEMM prologues and epilogues.
//
// Stock math (openfold3/core/model/layers/triangular_multiplicative_update.py
// :1263-1284 and :734-760; LayerNorm openfold3/core/model/primitives/
// normalization.py:54-78, f32 statistics, eps 1e-5):
//   zln = LN_in(z);  a = mask * sigmoid(zln Wag^T) * (zln Wap^T);  b likewise
//   outgoing: x[c,i,j] = sum_k a[i,k,c] b[j,k,c];  incoming: sum_k a[k,i,c] b[k,j,c]
//   out = (LN_out(x) Wz^T) * sigmoid(gl),  gl = zln Wg^T
//
// Storage (C == H channels, natural rows rho = (b*N + r)*N + s of z [B,N,N,C]):
//   z, zln, gl, out, dz, dy: [R][C] bf16 row-major; xln [R][H];
//   dproj5 [R][5H] with column blocks [d a_p | d a_g | d b_p | d b_g | d gl]
//   (the row order of W5 = [W_ap; W_ag; W_bp; W_bg; W_g]);
//   a, b (and da, db): channel-major "stored" matrices A_c[i][k], B_c[j][k]
//   with plane size N*Np (row pitch Np = N rounded up to 8, pad columns
//   zero): outgoing A_c[i][k] = a[i,k,c]; incoming A_c[i][k] = a[k,i,c], so
//   both directions contract as the NT GEMM x_c = A_c B_c^T;
//   x, dx: channel-major [B*H][N][Np] in natural (i, j) order.
// The projection kernels walk rows in stored-matrix order m (position
// p = m % NN of batch item m / NN): the natural row is m itself (outgoing) or
// the transposed position (incoming), read through the GEMM's row gather.
//
// Kernels of one direction:
//   forward:  tm_ln_rows (LN_in) -> tm_in_proj_fwd (a, b, gl) -> GEMM x ->
//             tm_ln_planes (LN_out) -> tm_out_proj<fwd> (out)
//   backward: tm_out_proj<bwd> (dy, d gl) -> tm_ln_bwd<planes> (dx, LN_out
//             partials) -> GEMMs da, db -> tm_in_proj_bwd (d a_p .. d b_g)
//             -> tm_ln_bwd<rows> (dz, LN_in partials) -> split-K weight
//             GEMMs -> fixed-order folds.
// 32-deep k stages: every TriMul GEMM has K = C or 5H (small).
#define TPF_GEMM_GK 32
#include <type_traits>

#include "common.hpp"
#include "gemm_core.hpp"
#include "tpf_gemm.hpp"
#include "tpf_status.hpp"

namespace tpf {

struct TmGeom {
  int B, N, Np, H;
  int64_t NN;  // N*N positions per batch item
  int64_t PS;  // N*Np elements per channel-major plane
  int64_t R;   // B*N*N rows (< 2^30)
  int outgoing;
  int ntg;     // gated 128-column weight tiles per branch (64 channels each)
  FastDiv div_n, div_nn;
};

constexpr int kSP = 136;  // bf16 pitch of 128-wide LDS staging tiles
// LDS of a kernel = max(main loop ring, epilogue staging).
// LDS of a kernel whose epilogue staging reuses its NS-stage GEMM ring.
// Block walk of the persistent row kernels: a workgroup runs the virtual
// blocks [bbeg, bend) and pb(blk) is the 32-row block a virtual block reads:
// one contiguous range per workgroup, or (strided) blocks g, g + G, ... for
// workgroup g of G, which keeps the grid on a compact window of rows.  Each
// kernel takes the walk measured faster for it at N = 384 (strided: LN_in
// backward 59.2 -> 55.8 us, output projection 23.8 -> 21.4 us; contiguous:
// the projection backward, whose 64-byte plane stores of consecutive blocks
// merge, 71.6 against 79.7 us, the projection forward and the output
// backward).  Either walk depends on the shape and grid only.
#define TM_BLOCKS_CONTIGUOUS(nblocks)                                            \
  const int64_t per = ((nblocks) + gridDim.x - 1) / gridDim.x;                   \
  const int64_t bbeg = blockIdx.x * per;                                         \
  const int64_t bend = bbeg + per < (nblocks) ? bbeg + per : (nblocks);          \
  auto pb = [&](int64_t v) { return v; }
#define TM_BLOCKS_STRIDED(nblocks)                                               \
  const int64_t bbeg = 0;                                                        \
  const int64_t bend =                                                           \
      blockIdx.x < (nblocks) ? ((nblocks) - blockIdx.x + gridDim.x - 1) / gridDim.x : 0; \
  auto pb = [&](int64_t v) { return v * (int64_t)gridDim.x + blockIdx.x; }

// Tile size of the channel contractions (forward x = A B^T, backward dA and
// dB): 192 x 192 when N is a multiple of 192 (N = 384: 4 tiles per channel
// instead of 9, one round of 512 workgroups on 256 CUs instead of 2.25, and
// 1.5x the MFMA work per loaded byte; measured 27.6 -> 25.8 us forward and
// 61.3 -> 55.6 us dA + dB at N = 384, 186 -> 163 and 330 -> 277 us at
// N = 768), else 128 x 128.  Every output element
// is summed over k in the same order whatever the tile, so the choice changes
// no bit of the results.
inline int tm_contract_tile(int64_t N) { return N % 192 == 0 ? 192 : 128; }

constexpr int lds_bytes(int epilogue, int ns = kGNS) {
  return epilogue > gemm_ring_bytes(ns) ? epilogue : gemm_ring_bytes(ns);
}
// Ring depths per kernel (measured): the short-K projections keep two
// stages (occupancy), the long-K / large-epilogue kernels take more.
constexpr int kInProjBwdNS = 3, kOutProjNS = 4;
constexpr int kLnOutBwdNS = 2;
constexpr int kInProjLds = lds_bytes((64 + 128) * kSP * 2, kInProjBwdNS);  // d tile + [dp | dg] tile
constexpr int kOutProjLds = lds_bytes(2 * 128 * kSP * 2, kOutProjNS);  // gate + dout tiles
constexpr int kLnOutBwdLds = lds_bytes(128 * kSP * 2, kLnOutBwdNS);  // x tile

// Element offset of position p = i*N + j inside a channel-major plane.
__device__ __forceinline__ int64_t tm_plane_off(const TmGeom& g, int64_t p) {
  if (g.Np == g.N) return p;
  const uint32_t i = fdiv((uint32_t)p, g.div_n);
  return (int64_t)i * g.Np + ((uint32_t)p - i * (uint32_t)g.N);
}
// Batch item and position of row m.
__device__ __forceinline__ void tm_bp(const TmGeom& g, int64_t m, int64_t& b, int64_t& p) {
  const uint32_t bb = fdiv((uint32_t)m, g.div_nn);
  b = bb;
  p = (uint32_t)m - bb * (uint32_t)g.NN;
}
// Natural row of stored-order row m.
__device__ __forceinline__ int64_t tm_phys_row(const TmGeom& g, int64_t m) {
  if (g.outgoing) return m;
  int64_t b, p;
  tm_bp(g, m, b, p);
  const uint32_t i = fdiv((uint32_t)p, g.div_n), k = (uint32_t)p - i * (uint32_t)g.N;
  return b * g.NN + (int64_t)k * g.N + i;
}

// ---------------------------------------------------------------------------
// Weight packing (per call, tiny): the f32 module weights to bf16 GEMM
// operands.
//   Wp tile t < 2*ntg (branch t / ntg, channel block q = t % ntg): rows
//   [p c0..c0+31 | g c0..c0+31 | p c0+32..c0+63 | g c0+32..c0+63], c0 = 64q,
//   so the wave holding output columns 64wn.. sees p and g of the same 32
//   channels in its two accumulator columns (the projection backward's B
//   operand).
//   W5 = [W_ap; W_ag; W_bp; W_bg; W_g] [5H][C] (the reference's d_w5 order;
//   also the forward projections' stationary operand);
//   Wz = W_z [C][H]; W5t = W5^T [C][5H] and Wzt = W_z^T [H][C] (stationary
//   operands of the LN_in / LN_out backward kernels).  Missing channels are
//   zero rows.
// ---------------------------------------------------------------------------
struct TmWeights {
  const float* ap;
  const float* ag;
  const float* bp;
  const float* bg;
  const float* g;
  const float* z;
};

__global__ __launch_bounds__(256) void tm_pack_weights_kernel(TmWeights w, __bf16* __restrict__ wp,
                                                              __bf16* __restrict__ w5,
                                                              __bf16* __restrict__ wz,
                                                              __bf16* __restrict__ w5t,
                                                              __bf16* __restrict__ wzt, int C,
                                                              int ntg) {
  const int cpr = C / 8;
  const int wp_rows = 2 * ntg * 128;
  const int64_t total = (int64_t)(wp_rows + 6 * C) * cpr;
  const float* const mats[5] = {w.ap, w.ag, w.bp, w.bg, w.g};
  // W5^T [C][5C] (C x 5C / 8 chunks) and Wz^T [H][C] (H x C / 8 chunks)
  // after the row-copied part.
  const int64_t t5 = total + (int64_t)C * 5 * cpr;
  for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < t5 + (int64_t)C * cpr;
       idx += (int64_t)gridDim.x * 256) {
    // The transposed parts take consecutive source columns on consecutive
    // lanes (coalesced loads; the 16-byte stores are the scattered side).
    if (idx >= t5) {
      const int64_t j = idx - t5;
      const int h = (int)(j % C), c0 = 8 * (int)(j / C);
      bf16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = f2bf(w.z[(int64_t)(c0 + e) * C + h]);
      st8(wzt + (int64_t)h * C + c0, o);
      continue;
    }
    if (idx >= total) {
      const int64_t j = idx - total;
      const int c = (int)(j % C), k0 = 8 * (int)(j / C);
      bf16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int k = k0 + e;
        o[e] = f2bf(mats[k / C][(int64_t)(k % C) * C + c]);
      }
      st8(w5t + (int64_t)c * 5 * C + k0, o);
      continue;
    }
    const int row = (int)(idx / cpr), ch = (int)(idx % cpr);
    const float* src = nullptr;
    __bf16* dst;
    if (row < wp_rows) {
      dst = wp + (int64_t)row * C + ch * 8;
      const int t = row / 128, rr = row % 128;
      const int br = t / ntg, q = t % ntg;
      const int c = 64 * q + 32 * (rr / 64) + (rr & 31);
      const bool isg = (rr >> 5) & 1;
      if (c < C) src = (br ? (isg ? w.bg : w.bp) : (isg ? w.ag : w.ap)) + (int64_t)c * C;
    } else if (row < wp_rows + 5 * C) {
      const int j = row - wp_rows, blk = j / C, c = j % C;
      dst = w5 + (int64_t)j * C + ch * 8;
      src = mats[blk] + (int64_t)c * C;
    } else {
      const int c = row - wp_rows - 5 * C;
      dst = wz + (int64_t)c * C + ch * 8;
      src = w.z + (int64_t)c * C;
    }
    bf16x8 o = zero8();
    if (src) {
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = f2bf(src[ch * 8 + e]);
    }
    st8(dst, o);
  }
}

// ---------------------------------------------------------------------------
// LN_in over rows of z (16 lanes per row, 8 channels per lane).  A thread
// handles kLnRowsRPT rows 16 apart, their loads issued together.
// ---------------------------------------------------------------------------
constexpr int kLnRowsRPT = 2;
// Workgroups of the LN_in launch: one per 16 * kLnRowsRPT rows (the kernel
// also walks grid-stride, loading its next rows while it normalises the
// current ones, when launched with fewer; 8 or 16 workgroups per CU measured
// no faster at N = 384).
static inline int64_t tm_ln_rows_grid(int64_t R) {
  return (R + 16 * kLnRowsRPT - 1) / (16 * kLnRowsRPT);
}
template <int C>
__global__ __launch_bounds__(256) void tm_ln_rows_kernel(const __bf16* __restrict__ z,
                                                         const float* __restrict__ w,
                                                         const float* __restrict__ bias,
                                                         __bf16* __restrict__ out,
                                                         float* __restrict__ mean_out,
                                                         float* __restrict__ rstd_out, int64_t R) {
  const int l16 = threadIdx.x & 15;
  const bool chan = l16 < C / 8;
  const int64_t nb = (R + 16 * kLnRowsRPT - 1) / (16 * kLnRowsRPT);
  // The lane's 8 LayerNorm weights and biases.
  f32x4 wv[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}}, bv[2] = {wv[0], wv[1]};
  if (chan) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      wv[h] = *reinterpret_cast<const f32x4*>(w + l16 * 8 + 4 * h);
      bv[h] = *reinterpret_cast<const f32x4*>(bias + l16 * 8 + 4 * h);
    }
  }
  // Rows of block blk: row0 + 16 k.  Loads are unconditional (rows past R
  // re-read row R - 1, lanes past C read channel 0) so the loads of the next
  // block stay in flight while the current one is normalised.
  auto load = [&](int64_t blk, bf16x8 (&v)[kLnRowsRPT]) {
    const int64_t row0 = blk * 16 * kLnRowsRPT + (threadIdx.x >> 4);
#pragma unroll
    for (int k = 0; k < kLnRowsRPT; ++k) {
      const int64_t row = min(row0 + 16 * k, R - 1);
      v[k] = ld8(z + row * C + (chan ? l16 * 8 : 0));
    }
  };
  bf16x8 nxt[kLnRowsRPT];
  int64_t blk = blockIdx.x;
  load(blk, nxt);
#pragma unroll 1
  for (; blk < nb; blk += gridDim.x) {
    float x[kLnRowsRPT][8];
#pragma unroll
    for (int k = 0; k < kLnRowsRPT; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) x[k][e] = chan ? bf2f(nxt[k][e]) : 0.f;
    if (blk + gridDim.x < nb) load(blk + gridDim.x, nxt);
    const int64_t row0 = blk * 16 * kLnRowsRPT + (threadIdx.x >> 4);
#pragma unroll
    for (int k = 0; k < kLnRowsRPT; ++k) {
      const int64_t row = row0 + 16 * k;
      const bool act = (row < R) && chan;
      float s = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) s += x[k][e];
      s = row16_sum(s);
      const float mean = s * (1.f / C);
      float v2 = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = act ? x[k][e] - mean : 0.f;
        v2 = fmaf(d, d, v2);
      }
      v2 = row16_sum(v2);
      const float rstd = rsqrtf(v2 * (1.f / C) + 1e-5f);
      if (act) {
        bf16x8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e)
          o[e] = f2bf((x[k][e] - mean) * rstd * wv[e >> 2][e & 3] + bv[e >> 2][e & 3]);
        st8(out + row * C + l16 * 8, o);
        if (l16 == 0) {
          mean_out[row] = mean;
          rstd_out[row] = rstd;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// LN_out over the channels of the channel-major product x, written as
// row-major xln.  Workgroup = 128 positions (natural order) x up to 128
// channels; wave = (64-position half wv / 2) x (64-channel half wv % 2);
// lane = (8-position group pg = lane % 8, 8-channel group lane / 8): it
// reads its 8 channels' 16-byte position runs (128-byte runs per plane
// along pg) and keeps the 8 x 8 block in registers, so no LDS transpose is
// needed.  Per-position sums over channels: the 8 channel groups of a wave
// by lane exchanges, the two channel halves through LDS; mean first, then
// the centred sum of squares.  Each thread then writes its 8 channels of
// its 8 rows as 16-byte stores, so a store instruction covers 8 rows x 128
// contiguous bytes (16 rows x 64 bytes with 16 position groups per wave:
// 17.3 -> 16.4 us at N=384, C=128).
// ---------------------------------------------------------------------------
// Workgroups of the LN_out launch per batch: a grid-stride walk over the
// 128-position tiles at 2 workgroups per CU (over all batches), each loading
// its next tile while it normalises the current one.  Tiles are independent,
// so the results do not depend on the grid.
constexpr int kLnPlanesWgsPerCu = 2;
static inline int64_t tm_ln_planes_grid(int64_t NN, int64_t B) {
  const int64_t nt = (NN + 127) / 128;
  const int64_t cap = ((int64_t)device_cus() * kLnPlanesWgsPerCu + B - 1) / B;
  return nt < cap ? nt : cap;
}
template <int H>
__global__ __launch_bounds__(256) void tm_ln_planes_kernel(const __bf16* __restrict__ x,
                                                           const float* __restrict__ w,
                                                           const float* __restrict__ bias,
                                                           __bf16* __restrict__ xln,
                                                           float* __restrict__ mean_out,
                                                           float* __restrict__ rstd_out,
                                                           TmGeom g) {
  constexpr int T = 128;  // positions per tile
  __shared__ float red[2][4][8][8];
  const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63, b = blockIdx.y;
  const int pg = lane & 7, cg = (lane >> 3) + 8 * (wv & 1);
  const int p0 = 64 * (wv >> 1) + pg * 8;  // first position in the tile
  const bool chan = cg * 8 < H;
  const int64_t nt = (g.NN + T - 1) / T;
  const bool vec = g.Np == g.N;
  const int cgl = chan ? cg : 0;
  float wc[8], bc[8];
  {
    const f32x4 w0 = *reinterpret_cast<const f32x4*>(w + cgl * 8);
    const f32x4 w1 = *reinterpret_cast<const f32x4*>(w + cgl * 8 + 4);
    const f32x4 b0 = *reinterpret_cast<const f32x4*>(bias + cgl * 8);
    const f32x4 b1 = *reinterpret_cast<const f32x4*>(bias + cgl * 8 + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      wc[i] = w0[i]; wc[4 + i] = w1[i];
      bc[i] = b0[i]; bc[4 + i] = b1[i];
    }
  }
  // v[c][e]: channel cg*8 + c, position pb + e of tile t.  Full tiles of
  // unpadded planes load unconditionally, 16 bytes per channel.
  auto load = [&](int64_t t, bf16x8 (&v)[8]) {
    const int64_t pb = t * T + p0;
    if (vec && pb + 8 <= g.NN) {
#pragma unroll
      for (int c = 0; c < 8; ++c) v[c] = ld8(x + ((int64_t)b * H + cgl * 8 + c) * g.PS + pb);
    } else {
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const __bf16* plane = x + ((int64_t)b * H + cgl * 8 + c) * g.PS;
#pragma unroll
        for (int e = 0; e < 8; ++e)
          v[c][e] = pb + e < g.NN ? plane[tm_plane_off(g, pb + e)] : static_cast<__bf16>(0.f);
      }
    }
  };
  // Sum over all channels of q[e] (this thread's 8 channels already summed);
  // the two sums of a tile use the two halves of `red`, so one barrier each.
  auto channel_sum = [&](float (&q)[8], int half) {
#pragma unroll
    for (int e = 0; e < 8; ++e) q[e] = xor32_sum(xor16_sum(q[e] + dpp_f<kDppXor8>(q[e])));
    if ((lane & 56) == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) red[half][wv][pg][e] = q[e];
    }
    __syncthreads();
    const int w0 = wv & 2;
#pragma unroll
    for (int e = 0; e < 8; ++e) q[e] = red[half][w0][pg][e] + red[half][w0 + 1][pg][e];
  };
  bf16x8 nxt[8];
  int64_t t = blockIdx.x;
  if (t < nt) load(t, nxt);
#pragma unroll 1
  for (; t < nt; t += gridDim.x) {
    bf16x8 v[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) v[c] = chan ? nxt[c] : zero8();
    if (t + gridDim.x < nt) load(t + gridDim.x, nxt);
    const int64_t pb = t * T + p0;  // first position of this thread
    float mean[8], rstd[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float s = 0.f;
#pragma unroll
      for (int c = 0; c < 8; ++c) s += bf2f(v[c][e]);
      mean[e] = s;
    }
    // red[0] was last read before the previous tile's second barrier, red[1]
    // before this tile's first: no barrier is needed between tiles.
    channel_sum(mean, 0);
#pragma unroll
    for (int e = 0; e < 8; ++e) mean[e] *= 1.f / H;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float s = 0.f;
      if (chan) {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          const float d = bf2f(v[c][e]) - mean[e];
          s = fmaf(d, d, s);
        }
      }
      rstd[e] = s;
    }
    channel_sum(rstd, 1);
#pragma unroll
    for (int e = 0; e < 8; ++e) rstd[e] = rsqrtf(rstd[e] * (1.f / H) + 1e-5f);
    if (chan) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (pb + e >= g.NN) continue;
        bf16x8 o;
#pragma unroll
        for (int c = 0; c < 8; ++c) o[c] = f2bf((bf2f(v[c][e]) - mean[e]) * rstd[e] * wc[c] + bc[c]);
        st8(xln + ((int64_t)b * g.NN + pb + e) * H + cg * 8, o);
      }
    }
    if (cg == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (pb + e < g.NN) {
          mean_out[(int64_t)b * g.NN + pb + e] = mean[e];
          rstd_out[(int64_t)b * g.NN + pb + e] = rstd[e];
        }
    }
  }
}

// Accumulator coordinates of this lane inside the 128 x 128 tile.
struct AccPos {
  int rl, hl, wm, wn;
  __device__ __forceinline__ AccPos() {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    rl = lane & 31; hl = lane >> 5; wm = w >> 1; wn = w & 1;
  }
  __device__ __forceinline__ int row(int i, int r) const {
    return 64 * wm + 32 * i + 8 * (r >> 2) + 4 * hl + (r & 3);
  }
  __device__ __forceinline__ int col(int j) const { return 64 * wn + 32 * j + rl; }
};

// Copy a [128 rows][ncols] bf16 LDS tile (pitch kSP) to rows rho_s[row] of a
// row-major global matrix (pitch ld, column offset c0); rows < 0 skipped.
__device__ __forceinline__ void tm_store_rows(const __bf16* S, int ncols, const int64_t* rho_s,
                                              __bf16* __restrict__ dst, int64_t ld, int c0) {
  const int cpr = ncols / 8;
  for (int idx = threadIdx.x; idx < 128 * 16; idx += 256) {
    const int row = idx >> 4, ch = idx & 15;
    const int64_t rho = rho_s[row];
    if (rho >= 0 && ch < cpr)
      st8(dst + rho * ld + c0 + ch * 8, *reinterpret_cast<const bf16x8*>(&S[row * kSP + ch * 8]));
  }
}

// Store an LDS tile S[c * kSP + pos] of [nch channels][128 positions] to
// channel-major planes (plane b*H + c0 + c, position of tile row m0 + pos
// within its batch item).
__device__ __forceinline__ void tm_store_planes(const __bf16* S, int nch, __bf16* planes,
                                                const TmGeom& g, int64_t m0, int c0) {
  for (int idx = threadIdx.x; idx < nch * 16; idx += 256) {
    const int cl = idx >> 4, chn = idx & 15;
    const int c = c0 + cl;
    if (c >= g.H) continue;
    const int64_t mb = m0 + 8 * chn;
    const __bf16* s = S + cl * kSP + 8 * chn;
    if (g.Np == g.N && mb + 7 < g.R) {
      // NN is a multiple of 64 here, so the 8 positions share a batch item.
      int64_t b, p;
          tm_bp(g, mb, b, p);
      st8(planes + ((int64_t)b * g.H + c) * g.PS + p, *reinterpret_cast<const bf16x8*>(s));
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int64_t m = mb + e;
        if (m < g.R) {
          int64_t b, p;
          tm_bp(g, m, b, p);
          planes[((int64_t)b * g.H + c) * g.PS + tm_plane_off(g, p)] = s[e];
        }
      }
    }
  }
}

// Register staging of an epilogue operand tile: fetched from HBM before the
// GEMM main loop (so its latency overlaps the main loop) and written to LDS
// after it.  Chunk k of thread t is tile chunk idx = t + 256 k.
struct RegTile {
  bf16x8 v[8];
};
// [128 rows][ncols] of a row-major matrix, natural rows m0 + row.
__device__ __forceinline__ void fetch_rows(RegTile& t, const __bf16* __restrict__ src, int64_t ld,
                                           int ncols, int64_t m0, int64_t R) {
  const int cpr = ncols / 8;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int idx = threadIdx.x + 256 * k;
    const int row = idx >> 4, ch = idx & 15;
    const int64_t m = m0 + row;
    t.v[k] = (ch < cpr && m < R) ? ld8(src + m * ld + ch * 8) : zero8();
  }
}
__device__ __forceinline__ void put_rows(__bf16* S, const RegTile& t) {
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int idx = threadIdx.x + 256 * k;
    *reinterpret_cast<bf16x8*>(&S[(idx >> 4) * kSP + (idx & 15) * 8]) = t.v[k];
  }
}
// [nch channels][128 positions] of channel-major planes (channels c0 + c,
// positions of tile rows m0 ..); nch * 16 <= 2048.
__device__ __forceinline__ void fetch_planes(RegTile& t, const __bf16* __restrict__ planes,
                                             const TmGeom& g, int nch, int64_t m0, int c0) {
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int idx = threadIdx.x + 256 * k;
    const int cl = idx >> 4, chn = idx & 15;
    const int c = c0 + cl;
    const int64_t mb = m0 + 8 * chn;
    bf16x8 v = zero8();
    if (cl < nch && c < g.H) {
      if (g.Np == g.N && mb + 7 < g.R) {
        int64_t b, p;
          tm_bp(g, mb, b, p);
        v = ld8(planes + ((int64_t)b * g.H + c) * g.PS + p);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int64_t m = mb + e;
          if (m < g.R) {
            int64_t b, p;
          tm_bp(g, m, b, p);
            v[e] = planes[((int64_t)b * g.H + c) * g.PS + tm_plane_off(g, p)];
          }
        }
      }
    }
    t.v[k] = v;
  }
}
__device__ __forceinline__ void put_planes(__bf16* S, const RegTile& t, int nch) {
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int idx = threadIdx.x + 256 * k;
    const int cl = idx >> 4, chn = idx & 15;
    if (cl < nch) *reinterpret_cast<bf16x8*>(&S[cl * kSP + 8 * chn]) = t.v[k];
  }
}

// ---------------------------------------------------------------------------
// Forward input projections, weight-stationary.  One wave per 16 channels
// (C / 16 waves) holds the bf16 rows of W_ap, W_ag, W_bp, W_bg and W_g for
// its channels in registers (the B operands of v_mfma_f32_16x16x32_bf16) for
// the whole kernel; workgroups are persistent and walk 32-row blocks of zln
// in stored row order.
//   * loads: the first half of the waves stream each block's rows straight
//     into a 4-deep LDS ring (buffer_load ... lds, three blocks ahead; the
//     chunk order within a row is rotated by the row so the A-fragment
//     reads are conflict-free) and the block's mask values beside them;
//     these waves issue no stores, so their vmcnt waits cover loads only;
//   * stores: the second half of the waves copy each block's staged outputs
//     (a and b as [channel][32 positions], gl as [32 rows][channel], double
//     buffered in LDS) to HBM as 64-byte plane segments and 2C-byte rows.
// One barrier per block.
//   16x16x32 layouts: A lane l holds A[l % 16][8 (l / 16) ..+8]; B lane l
//   holds B[8 (l / 16) ..+8][l % 16]; C register r of lane l is
//   C[4 (l / 16) + r][l % 16].
// ---------------------------------------------------------------------------
__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
// Direct 4-byte buffer -> LDS load: lane i writes dst_base + 4 i.
__device__ __forceinline__ void buf2lds4(i32x4 rsrc, uint32_t voff, void* dst_base) {
  const unsigned lds = __builtin_amdgcn_readfirstlane(lds_offset(dst_base));
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds"
               :: "s"(lds), "v"(voff), "s"(rsrc) : "memory", "m0");
}

// Depth of the zln block ring (blocks in flight: kInFwdDepth - 2).
constexpr int kInFwdDepth = 4;
template <int C, bool PAD>
__global__ __launch_bounds__(4 * C) void tm_in_proj_fwd_kernel(
    const __bf16* __restrict__ zln, const __bf16* __restrict__ w5, const float* __restrict__ mask,
    __bf16* __restrict__ a_pl, __bf16* __restrict__ b_pl, __bf16* __restrict__ gl, TmGeom g,
    int64_t nblocks) {
  constexpr int NW = C / 16;         // waves
  constexpr int CPR = C / 8;         // 16-byte chunks per row
  constexpr int KS = C / 32;         // 32-deep k steps
  constexpr int PP = 40;             // plane staging pitch (bf16): 32 positions + pad
  constexpr int GP = C + 8;          // gl staging pitch (bf16)
  __shared__ __attribute__((aligned(1024))) __bf16 As[kInFwdDepth][32 * C];
  __shared__ __attribute__((aligned(256))) float Ms[kInFwdDepth][64];
  __shared__ __attribute__((aligned(16))) __bf16 Sp[2][2][C * PP];  // [buf][a | b][ch][pos]
  __shared__ __attribute__((aligned(16))) __bf16 Sg[2][32 * GP];    // [buf][pos][ch]

  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int l16 = lane & 15, lg = lane >> 4;
  const int ch = 16 * w + l16;  // this lane's output channel
  const bool loader = w < NW / 2;

  // Stationary B operands: W5 rows (proj * C + ch), k chunk 4 ks + lg.
  bf16x8 wf[5][KS];
#pragma unroll
  for (int p = 0; p < 5; ++p)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) wf[p][ks] = ld8(w5 + ((int64_t)p * C + ch) * C + 8 * (4 * ks + lg));

  const i32x4 rs_z = buffer_rsrc(zln);
  const i32x4 rs_m = buffer_rsrc(mask);
  const __amdgpu_buffer_rsrc_t rs_a = __builtin_amdgcn_make_buffer_rsrc(a_pl, 0, 0x7FFFFFFF, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs_b = __builtin_amdgcn_make_buffer_rsrc(b_pl, 0, 0x7FFFFFFF, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs_g = __builtin_amdgcn_make_buffer_rsrc(gl, 0, 0x7FFFFFFF, 0x00020000);
  // Workgroup c takes the contiguous blocks [c per, (c + 1) per).
  TM_BLOCKS_CONTIGUOUS(nblocks);
  // Loader: instruction j of wave w fills LDS chunks (2 w + j) * 64 + lane
  // (row ci / CPR, slot ci % CPR) with global chunk (slot - row) mod CPR.
  auto issue = [&](int64_t blk) {
    const int stage = (int)(blk % kInFwdDepth);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int ci = (2 * w + j) * 64 + lane;
      const int r = ci / CPR, slot = ci % CPR;
      const int gc = (slot - r % CPR + CPR) % CPR;
      const int64_t m = pb(blk) * 32 + r;
      const bool ok = blk < bend && m < g.R;
      const uint32_t off = ok ? (uint32_t)((tm_phys_row(g, m) * C + 8 * gc) * 2) : kBufOOB;
      buf2lds16(rs_z, off, &As[stage][(2 * w + j) * 512]);
    }
    if (w == 0) {
      const int64_t m = pb(blk) * 32 + lane;
      const bool ok = lane < 32 && blk < bend && m < g.R;
      buf2lds4(rs_m, ok ? (uint32_t)(tm_phys_row(g, m) * 4) : kBufOOB, &Ms[stage][0]);
    }
  };
  auto mma = [&](int64_t blk, f32x4 (&acc)[5][2]) {
#pragma unroll
    for (int p = 0; p < 5; ++p)
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) acc[p][rt] = f32x4{0.f, 0.f, 0.f, 0.f};
    const __bf16* A = As[blk % kInFwdDepth];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        const int row = 16 * rt + l16;
        const bf16x8 af =
            *reinterpret_cast<const bf16x8*>(&A[row * C + 8 * ((4 * ks + lg + row) % CPR)]);
#pragma unroll
        for (int p = 0; p < 5; ++p) acc[p][rt] = mfma16(af, wf[p][ks], acc[p][rt]);
      }
  };
  // Epilogue of block blk: a = mask s(g_a) p_a, b likewise, gl -> staging.
  auto epilogue = [&](int64_t blk, const f32x4 (&acc)[5][2]) {
    const int sb = (int)(blk & 1);
    __bf16* Sa = Sp[sb][0];
    __bf16* Sb = Sp[sb][1];
    __bf16* G = Sg[sb];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int r0 = 16 * rt + 4 * lg;
      const f32x4 mk = *reinterpret_cast<const f32x4*>(&Ms[blk % kInFwdDepth][r0]);
      bf16x4 va, vb;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        va[e] = f2bf(mk[e] * sigmoidf(acc[1][rt][e]) * acc[0][rt][e]);
        vb[e] = f2bf(mk[e] * sigmoidf(acc[3][rt][e]) * acc[2][rt][e]);
        G[(r0 + e) * GP + ch] = f2bf(acc[4][rt][e]);
      }
      *reinterpret_cast<bf16x4*>(&Sa[ch * PP + r0]) = va;
      *reinterpret_cast<bf16x4*>(&Sb[ch * PP + r0]) = vb;
    }
  };
  auto stores = [&](int64_t blk) {
    // 12 C 16-byte chunks per block over the 2 C storing threads: all LDS
    // reads first, then the stores (buffer stores; rows past the end are
    // dropped through an out-of-range offset, so there are no branches).
    const int sb = (int)(blk & 1);
    const __bf16* G = Sg[sb];
    const int st = tid - 2 * C;
    const int64_t mb0 = pb(blk) * 32;
    bf16x8 v[6];
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int q = st + 2 * C * it;
      const int t = it >> 1, c = (q - 4 * C * t) >> 2, part = q & 3;
      v[it] = *reinterpret_cast<const bf16x8*>(&Sp[sb][t][c * PP + 8 * part]);
    }
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int q = st + 2 * C * it, row = q / CPR, c8 = q % CPR;
      v[4 + it] = *reinterpret_cast<const bf16x8*>(&G[row * GP + 8 * c8]);
    }
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int q = st + 2 * C * it;       // < 8C: a then b, (channel, 8-position part)
      const int t = it >> 1;
      const int c = (q - 4 * C * t) >> 2, part = q & 3;
      const int64_t mb = mb0 + 8 * part;
      if (!PAD) {
        // N % 8 == 0: the 8 positions are contiguous in one plane row.
        int64_t bb, pp;
        tm_bp(g, mb < g.R ? mb : 0, bb, pp);
        const uint32_t off = mb < g.R ? (uint32_t)((((int64_t)bb * g.H + c) * g.PS + pp) * 2) : kBufOOB;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v[it]), t ? rs_b : rs_a, off, 0, 0);
      } else {
        __bf16* planes = t ? b_pl : a_pl;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int64_t m = mb + e;
          if (m < g.R) {
            int64_t bb, pp;
            tm_bp(g, m, bb, pp);
            planes[((int64_t)bb * g.H + c) * g.PS + tm_plane_off(g, pp)] = v[it][e];
          }
        }
      }
    }
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int q = st + 2 * C * it;       // < 4C: (row, chunk)
      const int row = q / CPR, c8 = q % CPR;
      const int64_t m = mb0 + row;
      const uint32_t off = m < g.R ? (uint32_t)((tm_phys_row(g, m) * C + 8 * c8) * 2) : kBufOOB;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v[4 + it]), rs_g, off, 0, 0);
    }
  };
  // Pipeline: iteration blk issues the loads of blk + 3, multiplies blk + 1
  // while finishing blk's epilogue, waits for blk + 2's loads, then the
  // storing waves write blk's outputs.
  if (loader) {
#pragma unroll
    for (int d = 0; d < kInFwdDepth - 1; ++d) issue(bbeg + d);
    // blocks bbeg, bbeg + 1 landed
    if (w == 0) wait_vmcnt<3 * (kInFwdDepth - 3)>(); else wait_vmcnt<2 * (kInFwdDepth - 3)>();
  }
  __syncthreads();
  f32x4 acc0[5][2], acc1[5][2];
  mma(bbeg, acc0);
  int64_t blk = bbeg;
  auto iter = [&](f32x4 (&cur)[5][2], f32x4 (&nxt)[5][2]) {
    if (loader) issue(blk + kInFwdDepth - 1);
    // The two waves sharing a SIMD (w, w + NW / 2) take the two halves in
    // opposite order, so one's MFMAs overlap the other's epilogue VALU.
    if (loader) {
      if (blk + 1 < bend) mma(blk + 1, nxt);
      epilogue(blk, cur);
    } else {
      epilogue(blk, cur);
      if (blk + 1 < bend) mma(blk + 1, nxt);
    }
    if (loader) {
      if (w == 0) wait_vmcnt<3 * (kInFwdDepth - 3)>(); else wait_vmcnt<2 * (kInFwdDepth - 3)>();   // block blk + 2 landed
    }
    __syncthreads();
    if (!loader) stores(blk);
    ++blk;
  };
#pragma unroll 1
  while (blk < bend) {
    iter(acc0, acc1);
    if (blk >= bend) break;
    iter(acc1, acc0);
  }
  // The ring loads issued past the last block still write LDS: let them land
  // before the workgroup releases its LDS.
  if (loader) wait_vmcnt<0>();
}

// ---------------------------------------------------------------------------
// Input projections, backward, weight-stationary (N % 8 == 0).  The same
// persistent walk over 32-row blocks as the forward, with W_ap, W_ag, W_bp,
// W_bg rows of the wave's 16 channels in registers as the A operand, so the
// accumulators come out transposed (register r of lane l: channel
// 16 w + 4 (l / 16) + r, row l % 16) and each lane owns 4 consecutive
// channels of one row: the dproj5 row segments are 8-byte LDS writes.  Per
// block the loading waves stream zln rows, the da / db plane segments
// ([channel][32 positions], 64 bytes each) and the mask into a 4-deep LDS
// ring; d is read back transposed (ds_read_b64_tr_b16).  Outputs
// d a_p = d s(g_a), d a_g = d p_a s (1 - s), likewise for b, go through one
// LDS staging tile [32 rows][4C] and are stored as 8C-byte row segments of
// dproj5 by the storing waves.  Two barriers per block (staging reuse).
// ---------------------------------------------------------------------------
// 32-bit forms of the row / plane index helpers (R < 2^30 rows and plane
// tensors below 2^30 elements, both checked by tm_geom).
__device__ __forceinline__ uint32_t tm_phys_row32(const TmGeom& g, uint32_t m) {
  if (g.outgoing) return m;
  const uint32_t b = fdiv(m, g.div_nn), p = m - b * (uint32_t)g.NN;
  const uint32_t i = fdiv(p, g.div_n), k = p - i * (uint32_t)g.N;
  return b * (uint32_t)g.NN + k * (uint32_t)g.N + i;
}
// Element offset of stored row m in channel plane c (N % 8 == 0: Np == N).
__device__ __forceinline__ uint32_t tm_plane_elem32(const TmGeom& g, uint32_t m, int c) {
  const uint32_t b = fdiv(m, g.div_nn), p = m - b * (uint32_t)g.NN;
  return (b * (uint32_t)g.H + (uint32_t)c) * (uint32_t)g.PS + p;
}

constexpr int kInBwdDepth = 4;
template <int C>
__global__ __launch_bounds__(4 * C) void tm_in_proj_bwd_ws_kernel(
    const __bf16* __restrict__ zln, const __bf16* __restrict__ w5, const float* __restrict__ mask,
    const __bf16* __restrict__ da, const __bf16* __restrict__ db, __bf16* __restrict__ dproj5,
    TmGeom g, int64_t nblocks) {
  constexpr int NW = C / 16;         // waves
  constexpr int CPR = C / 8;         // 16-byte chunks per zln row
  constexpr int KS = C / 32;         // 32-deep k steps
  constexpr int SOP = 4 * C + 8;     // staging pitch (bf16)
  __shared__ __attribute__((aligned(1024))) __bf16 As[kInBwdDepth][32 * C];
  __shared__ __attribute__((aligned(1024))) __bf16 Ds[kInBwdDepth][2 * C * 32];  // [t][ch][pos]
  __shared__ __attribute__((aligned(256))) float Ms[kInBwdDepth][64];
  __shared__ __attribute__((aligned(16))) __bf16 So[32 * SOP];                   // [row][4C]

  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int l16 = lane & 15, lg = lane >> 4;
  const bool loader = w < NW / 2;

  // Stationary A operands: W5 rows (proj * C + 16 w + l16), k chunk 4 ks + lg.
  bf16x8 wf[4][KS];
#pragma unroll
  for (int p = 0; p < 4; ++p)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      wf[p][ks] = ld8(w5 + ((int64_t)p * C + 16 * w + l16) * C + 8 * (4 * ks + lg));

  const i32x4 rs_z = buffer_rsrc(zln);
  const i32x4 rs_m = buffer_rsrc(mask);
  const i32x4 rs_da = buffer_rsrc(da);
  const i32x4 rs_db = buffer_rsrc(db);
  const __amdgpu_buffer_rsrc_t rs_o = __builtin_amdgcn_make_buffer_rsrc(dproj5, 0, 0x7FFFFFFF, 0x00020000);
  TM_BLOCKS_CONTIGUOUS(nblocks);
  // Loads of a block per loading wave: 2 zln, 4 plane-segment, (wave 0) 1 mask.
  auto issue = [&](int64_t blk) {
    const int stage = (int)(blk % kInBwdDepth);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int ci = (2 * w + j) * 64 + lane;
      const int r = ci / CPR, slot = ci % CPR;
      const int gc = (slot - r % CPR + CPR) % CPR;
      const uint32_t m = (uint32_t)pb(blk) * 32 + r;
      const bool ok = blk < bend && m < (uint32_t)g.R;
      const uint32_t off = ok ? (tm_phys_row32(g, m) * C + 8 * gc) * 2 : kBufOOB;
      buf2lds16(rs_z, off, &As[stage][(2 * w + j) * 512]);
    }
    // Plane chunks gi = (4 w + j) * 64 + lane over [t][channel][4 parts].
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int gi = (4 * w + j) * 64 + lane;
      const int t = (4 * w + j) * 64 / (4 * C), rem = gi - t * 4 * C;  // t wave-uniform
      const int c = rem >> 2, part = rem & 3;
      const uint32_t mb = (uint32_t)pb(blk) * 32 + 8 * part;
      const bool ok = blk < bend && mb < (uint32_t)g.R;
      const uint32_t off = ok ? tm_plane_elem32(g, mb, c) * 2 : kBufOOB;
      // The first 4C chunks are da, the rest db (each wave's 4 instructions
      // stay within one tensor: 4C is a multiple of 256).
      buf2lds16(t ? rs_db : rs_da, off, &Ds[stage][(4 * w + j) * 512]);
    }
    if (w == 0) {
      const uint32_t m = (uint32_t)pb(blk) * 32 + lane;
      const bool ok = lane < 32 && blk < bend && m < (uint32_t)g.R;
      buf2lds4(rs_m, ok ? tm_phys_row32(g, m) * 4 : kBufOOB, &Ms[stage][0]);
    }
  };
  auto mma = [&](int64_t blk, f32x4 (&acc)[4][2]) {
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) acc[p][rt] = f32x4{0.f, 0.f, 0.f, 0.f};
    const __bf16* A = As[blk % kInBwdDepth];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        const int row = 16 * rt + l16;
        const bf16x8 zf =
            *reinterpret_cast<const bf16x8*>(&A[row * C + 8 * ((4 * ks + lg + row) % CPR)]);
#pragma unroll
        for (int p = 0; p < 4; ++p) acc[p][rt] = mfma16(wf[p][ks], zf, acc[p][rt]);
      }
  };
  // d for (channels 16 w + 4 lg + e, row 16 rt + l16) from the [ch][pos]
  // plane tile: lane L of a 16-lane group supplies row 16 w + 4 lg + L / 4,
  // columns 16 rt + 4 (L % 4) .. + 3.
  auto epilogue = [&](int64_t blk, const f32x4 (&acc)[4][2]) {
    const int stage = (int)(blk % kInBwdDepth);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        const __bf16* src = &Ds[stage][(t * C + 16 * w + 4 * lg + (l16 >> 2)) * 32 + 16 * rt + 4 * (l16 & 3)];
        const bf16x4 dv = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)src);
        const int row = 16 * rt + l16;
        const float mk = Ms[stage][row];
        bf16x4 dp, dg;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float d = bf2f(dv[e]) * mk;
          const float p = acc[2 * t][rt][e];
          const float sg = sigmoidf(acc[2 * t + 1][rt][e]);
          dp[e] = f2bf(d * sg);
          dg[e] = f2bf(d * p * sg * (1.f - sg));
        }
        const int col = 16 * w + 4 * lg;
        *reinterpret_cast<bf16x4*>(&So[row * SOP + (2 * t) * C + col]) = dp;
        *reinterpret_cast<bf16x4*>(&So[row * SOP + (2 * t + 1) * C + col]) = dg;
      }
  };
  auto stores = [&](int64_t blk) {
    // 16 C chunks (32 rows x C / 2) over the 2 C storing threads, four LDS
    // reads ahead of their stores.
    const int st = tid - 2 * C;
    const int64_t mb0 = pb(blk) * 32;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      bf16x8 v[4];
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int q = st + 2 * C * (4 * h + it), row = q / (C / 2), k = q % (C / 2);
        v[it] = *reinterpret_cast<const bf16x8*>(&So[row * SOP + 8 * k]);
      }
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int q = st + 2 * C * (4 * h + it), row = q / (C / 2), k = q % (C / 2);
        const uint32_t m = (uint32_t)mb0 + row;
        const uint32_t off = m < (uint32_t)g.R ? (tm_phys_row32(g, m) * 5 * C + 8 * k) * 2 : kBufOOB;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v[it]), rs_o, off, 0, 0);
      }
    }
  };
  if (loader) {
#pragma unroll
    for (int d = 0; d < kInBwdDepth - 1; ++d) issue(bbeg + d);
    // blocks bbeg, bbeg + 1 landed
    if (w == 0) wait_vmcnt<7 * (kInBwdDepth - 3)>(); else wait_vmcnt<6 * (kInBwdDepth - 3)>();
  }
  __syncthreads();
  f32x4 acc0[4][2], acc1[4][2];
  mma(bbeg, acc0);
  int64_t blk = bbeg;
  auto iter = [&](f32x4 (&cur)[4][2], f32x4 (&nxt)[4][2]) {
    if (loader) issue(blk + kInBwdDepth - 1);
    if (blk + 1 < bend) mma(blk + 1, nxt);
    __syncthreads();  // the staging tile of blk - 1 has been read
    epilogue(blk, cur);
    if (loader) {     // block blk + 2 landed
      if (w == 0) wait_vmcnt<7 * (kInBwdDepth - 3)>(); else wait_vmcnt<6 * (kInBwdDepth - 3)>();
    }
    __syncthreads();
    if (!loader) stores(blk);
    ++blk;
  };
#pragma unroll 1
  while (blk < bend) {
    iter(acc0, acc1);
    if (blk >= bend) break;
    iter(acc1, acc0);
  }
  // The ring loads issued past the last block still write LDS: let them land
  // before the workgroup releases its LDS.
  if (loader) wait_vmcnt<0>();
}

// ---------------------------------------------------------------------------
// Input projections, backward (stored row order): recompute p, g for 64
// channels of branch a or b and write d p = d * mask * s(g),
// d g = d * mask * p * s(g) (1 - s(g)) into dproj5, d = da / db.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256, 2) void tm_in_proj_bwd_kernel(
    const __bf16* __restrict__ zln, const __bf16* __restrict__ wp, const float* __restrict__ mask,
    const __bf16* __restrict__ a_pl, const __bf16* __restrict__ b_pl,
    __bf16* __restrict__ dproj5, TmGeom g, int C) {
  __shared__ __attribute__((aligned(1024))) char smem[kInProjLds];
  __shared__ float mask_s[128];
  __shared__ int64_t rho_s[128];
  const int H = g.H;
  const int tn = 2 * g.ntg;
  const int64_t tm = (g.R + 127) / 128;
  const int64_t T = xcd_order(tm * tn);
  if (T < 0) return;
  const int nt = (int)(T % tn);
  const int64_t m0 = (T / tn) * 128;
  if (threadIdx.x < 128) {
    const int64_t m = m0 + threadIdx.x;
    const int64_t rho = m < g.R ? tm_phys_row(g, m) : -1;
    rho_s[threadIdx.x] = rho;
    mask_s[threadIdx.x] = rho >= 0 ? mask[rho] : 0.f;
  }
  GemmOperand A{zln, C, (int)g.R, g.outgoing ? 0 : g.N, g.div_n, g.div_nn};
  GemmOperand W{wp, C, 2 * g.ntg * 128, 0, {}, {}};
  RegTile dreg;
  fetch_planes(dreg, (nt / g.ntg) ? b_pl : a_pl, g, 64, m0, 64 * (nt % g.ntg));
  f32x16 acc[2][2];
  gemm_tile<true, true, kInProjBwdNS>(A, W, (int)m0, nt * 128, 0, C, smem, acc);
  const AccPos ap;
  __bf16* S0 = reinterpret_cast<__bf16*>(smem);
  const int br = nt / g.ntg, q = nt % g.ntg;
  const int cl = 32 * ap.wn + ap.rl;  // channel 64q + cl
  // Backward: d tile [64 ch][128 pos] in S0, outputs [128 rows][dp 64 | dg 64] in So.
  __bf16* So = S0 + 64 * kSP;
  put_planes(S0, dreg, 64);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = ap.row(i, r);
      const float d = bf2f(S0[cl * kSP + row]) * mask_s[row];
      const float p = acc[i][0][r];
      const float s = sigmoidf(acc[i][1][r]);
      So[row * kSP + cl] = f2bf(d * s);
      So[row * kSP + 64 + cl] = f2bf(d * p * s * (1.f - s));
    }
  __syncthreads();
  const int nvalid = min(64, H - 64 * q) / 8;  // 8-channel chunks inside H
  for (int idx = threadIdx.x; idx < 128 * 16; idx += 256) {
    const int row = idx >> 4, k = idx & 15, isg = k >> 3, c8 = k & 7;
    const int64_t rho = rho_s[row];
    if (rho < 0 || c8 >= nvalid) continue;
    const int col = (2 * br + isg) * H + 64 * q + 8 * c8;
    st8(dproj5 + rho * 5 * H + col, *reinterpret_cast<const bf16x8*>(&So[row * kSP + isg * 64 + 8 * c8]));
  }
}

// ---------------------------------------------------------------------------
// Output projection backward, tile GEMM (N % 8 != 0; otherwise the fused
// tm_out_bwd_ws_kernel runs): y = xln Wz^T recomputed (natural rows),
// dy = dout s(gl) (row-major) and d gl = dout y s(gl) (1 - s(gl)) into the
// last block of dproj5.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256, 2) void tm_out_proj_bwd_kernel(
    const __bf16* __restrict__ xln, const __bf16* __restrict__ p_out,
    const __bf16* __restrict__ gl, const __bf16* __restrict__ dout,
    __bf16* __restrict__ dy, __bf16* __restrict__ dproj5, TmGeom g, int C) {
  constexpr int kStage = 128 * kSP * 2;
  __shared__ __attribute__((aligned(1024))) char smem[kOutProjLds];
  __shared__ int64_t rho_s[128];
  const int H = g.H;
  const int64_t T = xcd_order((g.R + 127) / 128);
  if (T < 0) return;
  const int64_t m0 = T * 128;
  if (threadIdx.x < 128) rho_s[threadIdx.x] = m0 + threadIdx.x < g.R ? m0 + threadIdx.x : -1;
  GemmOperand A{xln, H, (int)g.R, 0, {}, {}};
  GemmOperand W{p_out, H, C, 0, {}, {}};
  RegTile greg, dreg;
  fetch_rows(greg, gl, C, C, m0, g.R);
  fetch_rows(dreg, dout, C, C, m0, g.R);
  f32x16 acc[2][2];
  gemm_tile<true, true, kOutProjNS>(A, W, (int)m0, 0, 0, H, smem, acc);
  const AccPos ap;
  __bf16* Sg = reinterpret_cast<__bf16*>(smem);
  __bf16* Sd = reinterpret_cast<__bf16*>(smem + kStage);
  put_rows(Sg, greg);
  put_rows(Sd, dreg);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = ap.col(j);
      if (col >= C) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int o = ap.row(i, r) * kSP + col;
        const float s = sigmoidf(bf2f(Sg[o]));
        const float y = acc[i][j][r];
        const float go = bf2f(Sd[o]);
        Sd[o] = f2bf(go * s);
        Sg[o] = f2bf(go * y * s * (1.f - s));
      }
    }
  __syncthreads();
  tm_store_rows(Sd, C, rho_s, dy, C, 0);
  tm_store_rows(Sg, C, rho_s, dproj5, 5 * H, 4 * H);
}

// ---------------------------------------------------------------------------
// LN_out backward fused onto the GEMM that produces its input gradient
// (natural rows): G = dy Wz (A = dy [R][C], B = Wz read MN), x from the
// channel-major planes, dx written to planes;
//   g = G * gamma;  dx = rstd (g - mean(g) - xhat mean(g xhat));
//   per-tile partials d gamma = sum G xhat, d beta = sum G into
//   lnp[tile][2][W] (W channels).
// The epilogue works on the accumulators in registers: the x tile sits in
// LDS as [channel][row], so 8-byte reads give each lane the 4 consecutive
// rows of one accumulator column; row sums are reduced across the 32 columns of
// a wave with a transposing butterfly and across the two column waves in
// LDS, column sums across the two row halves with a lane swap and across
// the row waves in LDS.  All reductions run in a fixed order.
// ---------------------------------------------------------------------------

// x values of acc[i][j] rows 4*rq .. 4*rq+3 (of this lane's 16 registers).
__device__ __forceinline__ bf16x4 tm_x4(const __bf16* Xt, const AccPos& ap, int i, int j, int rq) {
  const int row = 64 * ap.wm + 32 * i + 8 * rq + 4 * ap.hl;
  return *reinterpret_cast<const bf16x4*>(Xt + ap.col(j) * kSP + row);
}

// One level of the transposing butterfly: lanes exchange half of their
// 2*HALF partial sums with lane ^ HALF and keep the half selected by that
// lane bit (constant indices only, so the arrays stay in registers).
template <int HALF>
__device__ __forceinline__ void tm_butterfly(float* a, float* b, int lane) {
  const bool up = (lane & HALF) != 0;
#pragma unroll
  for (int k = 0; k < HALF; ++k) {
    const float sa = up ? a[k] : a[k + HALF];
    const float sb = up ? b[k] : b[k + HALF];
    const float ra = butterfly_partner<HALF>(sa, lane);
    const float rb = butterfly_partner<HALF>(sb, lane);
    a[k] = (up ? a[k + HALF] : a[k]) + ra;
    b[k] = (up ? b[k + HALF] : b[k]) + rb;
  }
}

// Row totals of per-wave partial sums P [2][NWV][32] (quantity, wave, row)
// in LDS, for the four rows r0 .. r0 + 3 that all 16 lanes of a lane group
// share: lane 8 q + v of the group reads wave v's partials of quantity q
// (zeros for v >= NWV), the 8 lanes of a quantity are summed on DPP and the
// two quantities swapped across the group's halves.  s0 / s1 are the totals
// of quantity 0 / 1 (the same bits on every lane).
template <int NWV>
__device__ __forceinline__ void wave_row_sums(const float* P, int r0, int lane, f32x4& s0,
                                              f32x4& s1) {
  static_assert(NWV >= 1 && NWV <= 8, "waves per lane group");
  const int v = lane & 7, q = (lane >> 3) & 1;
  f32x4 r = f32x4{0.f, 0.f, 0.f, 0.f};
  if (v < NWV) r = *reinterpret_cast<const f32x4*>(&P[(q * NWV + v) * 32 + r0]);
  f32x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    r[e] = lanes_sum<8>(r[e]);
    o[e] = dpp_f<kDppXor8>(r[e]);
  }
  s0 = q ? o : r;
  s1 = q ? r : o;
}

__global__ __launch_bounds__(256, 2) void tm_ln_out_bwd_kernel(
    const __bf16* __restrict__ a_op, int64_t a_ld, const __bf16* __restrict__ w_op, int K,
    const __bf16* __restrict__ xsrc, const float* __restrict__ mean, const float* __restrict__ rstd,
    const float* __restrict__ gamma, __bf16* __restrict__ dst, float* __restrict__ lnp,
    TmGeom g, int W) {
  __shared__ __attribute__((aligned(1024))) char smem[kLnOutBwdLds];
  __shared__ __attribute__((aligned(16))) float mean_s[128], rstd_s[128];
  __shared__ __attribute__((aligned(16))) float rsum[2][2][128];  // [quantity][wn][row]
  __shared__ float csum[2][2][128];                               // [quantity][wm][col]
  const int tid = threadIdx.x;
  const int64_t T = xcd_order((g.R + 127) / 128);
  if (T < 0) return;
  const int64_t m0 = T * 128;
  if (tid < 128) {
    const int64_t m = m0 + tid;
    const bool ok = m < g.R;
    mean_s[tid] = ok ? mean[m] : 0.f;
    rstd_s[tid] = ok ? rstd[m] : 0.f;
  }
  GemmOperand A{a_op, a_ld, (int)g.R, 0, {}, {}};
  GemmOperand B{w_op, W, W, 0, {}, {}};
  RegTile xreg;
  fetch_planes(xreg, xsrc, g, 128, m0, 0);
  f32x16 acc[2][2];
  gemm_tile<true, false, kLnOutBwdNS>(A, B, (int)m0, 0, 0, K, smem, acc);
  __bf16* Xt = reinterpret_cast<__bf16*>(smem);  // [ch][row]
  put_planes(Xt, xreg, 128);
  __syncthreads();
  const AccPos ap;
  const int lane = tid & 63;
  float gam[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) gam[j] = ap.col(j) < W ? gamma[ap.col(j)] : 0.f;
  // Pass 1: per-row partial sums over this lane's two columns, per-column
  // partial sums over this lane's 32 rows.
  float rs_g[32], rs_gx[32];
  float cs_g[2] = {0.f, 0.f}, cs_gx[2] = {0.f, 0.f};
#pragma unroll
  for (int t = 0; t < 32; ++t) { rs_g[t] = 0.f; rs_gx[t] = 0.f; }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      const int row0 = 64 * ap.wm + 32 * i + 8 * rq + 4 * ap.hl;
      const f32x4 mu = *reinterpret_cast<const f32x4*>(&mean_s[row0]);
      const f32x4 rs = *reinterpret_cast<const f32x4*>(&rstd_s[row0]);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const bf16x4 xv = tm_x4(Xt, ap, i, j, rq);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * rq + e;
          const float G = acc[i][j][r];
          const float xh = (bf2f(xv[e]) - mu[e]) * rs[e];
          const float gv = G * gam[j];
          rs_g[16 * i + r] += gv;
          rs_gx[16 * i + r] = fmaf(gv, xh, rs_gx[16 * i + r]);
          cs_g[j] += G;
          cs_gx[j] = fmaf(G, xh, cs_gx[j]);
        }
      }
    }
  // Transposing butterfly over the 32 columns of the wave: lane rl ends with
  // the full sums of value index t = rl.
  tm_butterfly<16>(rs_g, rs_gx, lane);
  tm_butterfly<8>(rs_g, rs_gx, lane);
  tm_butterfly<4>(rs_g, rs_gx, lane);
  tm_butterfly<2>(rs_g, rs_gx, lane);
  tm_butterfly<1>(rs_g, rs_gx, lane);
  {
    const int t = ap.rl, i = t >> 4, r = t & 15;
    const int row = ap.row(i, r);
    rsum[0][ap.wn][row] = rs_g[0];
    rsum[1][ap.wn][row] = rs_gx[0];
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const float a0 = xor32_sum(cs_g[j]), a1 = xor32_sum(cs_gx[j]);
    if (ap.hl == 0) {
      csum[0][ap.wm][ap.col(j)] = a0;
      csum[1][ap.wm][ap.col(j)] = a1;
    }
  }
  __syncthreads();
  if (tid < W) {
    float* part = lnp + T * 2 * W;
    part[tid] = csum[1][0][tid] + csum[1][1][tid];
    part[W + tid] = csum[0][0][tid] + csum[0][1][tid];
  }
  // Pass 2: dx in place of x (each element is read and written by one lane).
  const float invW = 1.f / W;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      const int row0 = 64 * ap.wm + 32 * i + 8 * rq + 4 * ap.hl;
      const f32x4 mu = *reinterpret_cast<const f32x4*>(&mean_s[row0]);
      const f32x4 rs = *reinterpret_cast<const f32x4*>(&rstd_s[row0]);
      const f32x4 sg0 = *reinterpret_cast<const f32x4*>(&rsum[0][0][row0]);
      const f32x4 sg1 = *reinterpret_cast<const f32x4*>(&rsum[0][1][row0]);
      const f32x4 sx0 = *reinterpret_cast<const f32x4*>(&rsum[1][0][row0]);
      const f32x4 sx1 = *reinterpret_cast<const f32x4*>(&rsum[1][1][row0]);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const bf16x4 xv = tm_x4(Xt, ap, i, j, rq);
        bf16x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float mg = (sg0[e] + sg1[e]) * invW, mgx = (sx0[e] + sx1[e]) * invW;
          const float xh = (bf2f(xv[e]) - mu[e]) * rs[e];
          const float gv = acc[i][j][4 * rq + e] * gam[j];
          o[e] = f2bf(rs[e] * (gv - mg - xh * mgx));
        }
        *reinterpret_cast<bf16x4*>(Xt + ap.col(j) * kSP + row0) = o;
      }
    }
  __syncthreads();
  tm_store_planes(Xt, 128, dst, g, m0, 0);
}

// ---------------------------------------------------------------------------
// LN_in backward, weight-stationary: G = dproj5 W5 (K = 5H) and the LayerNorm
// backward of LN_in, per 32-row block of natural rows, persistent workgroups
// of C / 16 waves.  Wave w = (channel group cg = w / 2 of 32 channels, k half
// kh = w % 2) holds the W5^T rows of its 32 channels over its half of K (B
// operands of v_mfma_f32_32x32x16_bf16) for the whole kernel, so each dproj5
// fragment read from LDS feeds a 32 x 32 product: every block's dproj5 tile is
// read from LDS C / 32 times instead of C / 16.  The loading waves stream each
// block's dproj5 rows (chunks rotated by row, so fragment reads are
// conflict-free) into a 3-deep LDS ring and its z rows and row statistics
// into a 2-deep one.  The two k halves of a channel group meet through LDS:
// each wave keeps the accumulator registers of 8 of its lane's 16 rows and
// hands the other 8 to its partner, so a lane ends with G[row][channel
// 32 cg + lane % 32] for rows 16 kh + 8 g + 4 (lane / 32) + e (g < 2, e < 4),
// the sum (k half 0) + (k half 1).  z is read back transposed to match.  Row
// sums of g = G gamma and g xhat are reduced across a group's 32 channels
// with a transposing butterfly and across the groups in LDS (fixed order);
// dz = rstd (g - mean(g) - xhat mean(g xhat)) is staged in LDS and stored as
// full rows by the storing waves.  The d gamma / d beta column sums of each
// lane stay in registers over all of a workgroup's blocks and are written
// once per workgroup to lnp [workgroup][2][C] (d gamma, d beta).
// ---------------------------------------------------------------------------
constexpr int kLnInDepth = 3;
template <int C>
__global__ __launch_bounds__(4 * C) void tm_ln_in_bwd_ws_kernel(
    const __bf16* __restrict__ dproj5, const __bf16* __restrict__ w5t,
    const __bf16* __restrict__ z, const float* __restrict__ mean, const float* __restrict__ rstd,
    const float* __restrict__ gamma, __bf16* __restrict__ dz, float* __restrict__ lnp, TmGeom g,
    int64_t nblocks) {
  constexpr int NW = C / 16;         // waves
  constexpr int NG = C / 32;         // channel groups
  constexpr int K = 5 * C;           // contraction depth
  constexpr int KC = K / 8;          // 16-byte chunks per dproj5 row
  constexpr int KH = KC / 2;         // chunks per k half
  constexpr int KT = K / 32;         // 16-deep MFMA steps per k half
  constexpr int CPR = C / 8;         // 16-byte chunks per z row
  constexpr int SP = C + 8;          // dz staging pitch (bf16)
  constexpr int PI = 32 * KC / 64 / (NW / 2);  // dproj5 load instructions per loading wave
  constexpr int XB = NG * 2 * 8 * 64 * 4;      // k-half exchange [cg][kh][register][lane] f32
  constexpr int OB = 32 * SP * 2;              // dz staging tile
  __shared__ __attribute__((aligned(1024))) __bf16 Ps[kLnInDepth][32 * K];
  __shared__ __attribute__((aligned(1024))) __bf16 Zs[2][32 * C];
  __shared__ __attribute__((aligned(256))) float Ss[2][2][64];           // mean | rstd
  __shared__ __attribute__((aligned(16))) float Rs[2][NG][32];           // row sums [q][group][row]
  // The exchange is read before the block's row-sum barrier and the staging
  // tile written after it, so the two share memory.
  __shared__ __attribute__((aligned(16))) char XO[XB > OB ? XB : OB];
  float* const X = reinterpret_cast<float*>(XO);
  __bf16* const So = reinterpret_cast<__bf16*>(XO);
  static_assert(PI * 64 * (NW / 2) == 32 * KC, "dproj5 loads split evenly");
  static_assert(KC % 2 == 0 && KH % 2 == 0, "k halves of whole MFMA steps");

  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int l16 = lane & 15, l32 = lane & 31, hl = lane >> 5, q = lane >> 4;
  const int cg = w >> 1, kh = w & 1;
  const int ch = 32 * cg + l32;
  const bool loader = w < NW / 2;

  bf16x8 wf[KT];
#pragma unroll
  for (int t = 0; t < KT; ++t) wf[t] = ld8(w5t + (int64_t)ch * K + 8 * (kh * KH + 2 * t + hl));
  const float gam = gamma[ch];

  const i32x4 rs_p = buffer_rsrc(dproj5);
  const i32x4 rs_z = buffer_rsrc(z);
  const i32x4 rs_mu = buffer_rsrc(mean);
  const i32x4 rs_rs = buffer_rsrc(rstd);
  const __amdgpu_buffer_rsrc_t rs_o = __builtin_amdgcn_make_buffer_rsrc(dz, 0, 0x7FFFFFFF, 0x00020000);
  TM_BLOCKS_STRIDED(nblocks);
  // Loads per block and loading wave: 2 z instructions and, by wave 0, the
  // two statistics rows (load j < 2, block blk, into the 2-deep ring), then PI
  // dproj5 instructions (load j >= 2, into the 3-deep ring).
  auto load = [&](int j, int64_t blk) {
    if (j < 2) {
      const int stage = (int)(blk & 1);
      const int ci = (2 * w + j) * 64 + lane;
      const int r = ci / CPR, slot = ci % CPR;
      const int gc = (slot - r % CPR + CPR) % CPR;
      const uint32_t m = (uint32_t)pb(blk) * 32 + r;
      const bool ok = blk < bend && m < (uint32_t)g.R;
      buf2lds16(rs_z, ok ? (m * C + 8 * gc) * 2 : kBufOOB, &Zs[stage][(2 * w + j) * 512]);
      if (j == 1 && w == 0) {
        const uint32_t mr = (uint32_t)pb(blk) * 32 + lane;
        const bool okr = lane < 32 && blk < bend && mr < (uint32_t)g.R;
        buf2lds4(rs_mu, okr ? mr * 4 : kBufOOB, &Ss[stage][0][0]);
        buf2lds4(rs_rs, okr ? mr * 4 : kBufOOB, &Ss[stage][1][0]);
      }
    } else {
      const int stage = (int)(blk % kLnInDepth);
      const int ci = (PI * w + j - 2) * 64 + lane;
      const int r = ci / KC, slot = ci % KC;
      const int gc = (slot - r % KC + KC) % KC;
      const uint32_t m = (uint32_t)pb(blk) * 32 + r;
      const bool ok = blk < bend && m < (uint32_t)g.R;
      buf2lds16(rs_p, ok ? (m * K + 8 * gc) * 2 : kBufOOB, &Ps[stage][(PI * w + j - 2) * 512]);
    }
  };
  constexpr int NL = PI + 2;
  float cgs = 0.f, cgx = 0.f;  // this lane's channel: sum G, sum G xhat over its rows
  if (loader) {
#pragma unroll
    for (int j = 0; j < NL; ++j) load(j, bbeg);
#pragma unroll
    for (int j = 2; j < NL; ++j) load(j, bbeg + 1);
  }
#pragma unroll 1
  for (int64_t blk = bbeg; blk < bend; ++blk) {
    const int sp = (int)(blk % kLnInDepth), sz = (int)(blk & 1);
    // Issued since block blk's loads: at most block blk + 1's dproj5 (the
    // last PI loads of the previous iteration).
    if (loader) wait_vmcnt<PI>();
    __syncthreads();
    // This k half's partial G: rows 8 (r / 4) + 4 hl + r % 4, channel ch.
    // The loading waves spread the next blocks' loads (z of blk + 1, then
    // dproj5 of blk + 2) over the MFMA chain, whose stalls hide their issue.
    f32x16 acc = zero16();
    const __bf16* P = Ps[sp];
    auto chain = [&](auto with_loads) {
#pragma unroll
      for (int t = 0; t < KT; ++t) {
        const int gc = kh * KH + 2 * t + hl;
        const bf16x8 pf = *reinterpret_cast<const bf16x8*>(&P[l32 * K + 8 * ((gc + l32) % KC)]);
        acc = mfma32(pf, wf[t], acc);
        if constexpr (decltype(with_loads)::value) {
#pragma unroll
          for (int j = 0; j < NL; ++j)
            if (j * KT / NL == t) load(j, j < 2 ? blk + 1 : blk + 2);
        }
      }
    };
    if (loader) chain(std::true_type{});
    else chain(std::false_type{});
    // Registers 8 kh .. 8 kh + 7 stay (rows 16 kh + 8 g + 4 hl + e), the
    // other eight go to the partner wave.
    float G[8];
    {
      float* xs = X + (cg * 2 + kh) * 8 * 64 + lane;
      if (kh == 0) {
#pragma unroll
        for (int j = 0; j < 8; ++j) xs[j * 64] = acc[8 + j];
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) xs[j * 64] = acc[j];
      }
      __syncthreads();
      const float* xr = X + (cg * 2 + (kh ^ 1)) * 8 * 64 + lane;
      if (kh == 0) {
#pragma unroll
        for (int j = 0; j < 8; ++j) G[j] = acc[j] + xr[j * 64];
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) G[j] = xr[j * 64] + acc[8 + j];
      }
    }
    // x for the same (row, channel) pairs: lane L of a 16-lane group reads
    // row r0 + L / 4, channels 32 cg + 16 (q % 2) + 4 (L % 4) .. + 3 (rotated chunk).
    float xh[8], gv[8], a[8], b[8];
#pragma unroll
    for (int gg = 0; gg < 2; ++gg) {
      const int r0 = 16 * kh + 8 * gg + 4 * hl;
      const int rr = r0 + (l16 >> 2);
      const int cc = 32 * cg + 16 * (q & 1) + 4 * (l16 & 3);
      const __bf16* src = &Zs[sz][rr * C + 8 * (((cc >> 3) + rr) % CPR) + (cc & 7)];
      const bf16x4 xv = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)src);
      const f32x4 mu = *reinterpret_cast<const f32x4*>(&Ss[sz][0][r0]);
      const f32x4 rsd = *reinterpret_cast<const f32x4*>(&Ss[sz][1][r0]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = 4 * gg + e;
        xh[i] = (bf2f(xv[e]) - mu[e]) * rsd[e];
        gv[i] = G[i] * gam;
        a[i] = gv[i];
        b[i] = gv[i] * xh[i];
        cgs += G[i];
        cgx = fmaf(G[i], xh[i], cgx);
      }
    }
    // Row sums over the 32 channels of this group: lanes with l16 = t < 8
    // end with value t (row 16 kh + 8 (t / 4) + 4 hl + t % 4), summed over
    // the 16 lanes of their group and the 16 of the neighbouring group.
    tm_butterfly<4>(a, b, lane);
    tm_butterfly<2>(a, b, lane);
    tm_butterfly<1>(a, b, lane);
    a[0] = xor16_sum(a[0] + dpp_f<kDppXor8>(a[0]));
    b[0] = xor16_sum(b[0] + dpp_f<kDppXor8>(b[0]));
    if ((lane & 24) == 0) {
      const int t = l16, row = 16 * kh + 8 * (t >> 2) + 4 * hl + (t & 3);
      Rs[0][cg][row] = a[0];
      Rs[1][cg][row] = b[0];
    }
    __syncthreads();
    const float invC = 1.f / C;
#pragma unroll
    for (int gg = 0; gg < 2; ++gg) {
      const int r0 = 16 * kh + 8 * gg + 4 * hl;
      const f32x4 rsd = *reinterpret_cast<const f32x4*>(&Ss[sz][1][r0]);
      f32x4 sg, sx;
      wave_row_sums<NG>(&Rs[0][0][0], r0, lane, sg, sx);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = 4 * gg + e;
        const float o = rsd[e] * (gv[i] - sg[e] * invC - xh[i] * (sx[e] * invC));
        So[(r0 + e) * SP + ch] = f2bf(o);
      }
    }
    __syncthreads();
    if (!loader) {
      // 4 C chunks (32 rows x C / 8) over the 2 C storing threads.
      const int st = tid - 2 * C;
      bf16x8 v[2];
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        const int qq = st + 2 * C * it, row = qq / CPR, k = qq % CPR;
        v[it] = *reinterpret_cast<const bf16x8*>(&So[row * SP + 8 * k]);
      }
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        const int qq = st + 2 * C * it, row = qq / CPR, k = qq % CPR;
        const uint32_t m = (uint32_t)pb(blk) * 32 + row;
        const uint32_t off = m < (uint32_t)g.R ? (m * C + 8 * k) * 2 : kBufOOB;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v[it]), rs_o, off, 0, 0);
      }
    }
  }
  // The ring loads issued past the last block still write LDS: let them land
  // before the workgroup releases its LDS.
  if (loader) wait_vmcnt<0>();
  // Column sums: the two row halves of a lane's channel (lanes l, l ^ 32),
  // then the two k-half waves of the group through LDS, k half 0 first.
  cgs = xor32_sum(cgs);
  cgx = xor32_sum(cgx);
  __syncthreads();
  if (kh == 1 && hl == 0) {
    Rs[0][cg][l32] = cgx;
    Rs[1][cg][l32] = cgs;
  }
  __syncthreads();
  if (kh == 0 && hl == 0) {
    lnp[(int64_t)blockIdx.x * 2 * C + ch] = cgx + Rs[0][cg][l32];
    lnp[(int64_t)blockIdx.x * 2 * C + C + ch] = cgs + Rs[1][cg][l32];
  }
}

// ---------------------------------------------------------------------------
// Output projection backward and LN_out backward in one persistent,
// weight-stationary kernel (N % 8 == 0), per 32-row block of natural rows:
//   y = xln Wz^T (recomputed), s = s(gl):  dy = dout s,  d gl = dout y s (1 - s);
//   G = dy Wz, then the LN_out backward of x (planes) into dx (planes).
// Wave w owns channels 16 w .. 16 w + 15 of both products: its rows of Wz
// (A operand of the first, which forms y^T) and of Wz^T (B operand of the
// second) stay in registers.  In the first product register r of lane l
// holds row l % 16, channel 16 w + 4 (l / 16) + r, so gl and dout are read
// and dy / d gl written as 4-channel runs; in the second, row 4 (l / 16) + r,
// channel 16 w + l % 16 (+ 16 rows per row tile).  The loading waves stream
// each block's xln, gl and dout rows (chunk-rotated) and x plane segments
// ([channel][32 positions]) and the LN_out statistics into a 3-deep LDS
// ring.  dy (the
// second product's A operand), d gl and dx are staged in LDS and stored by
// the storing waves: dy rows, d gl into the last block of dproj5, dx plane
// segments.  Row sums of the LayerNorm backward are reduced across each
// wave's 16 channels with a transposing butterfly and across the waves in
// LDS (fixed order); the d gamma / d beta column sums stay in registers for
// all of a workgroup's blocks and go to lnp [workgroup][2][C].
// ---------------------------------------------------------------------------
constexpr int kOutBwdDepth = 3;
template <int C>
__global__ __launch_bounds__(4 * C) void tm_out_bwd_ws_kernel(
    const __bf16* __restrict__ xln, const __bf16* __restrict__ wz, const __bf16* __restrict__ wzt,
    const __bf16* __restrict__ gl, const __bf16* __restrict__ dout, const __bf16* __restrict__ x,
    const float* __restrict__ mean, const float* __restrict__ rstd, const float* __restrict__ gamma,
    __bf16* __restrict__ dproj5, __bf16* __restrict__ dx, float* __restrict__ lnp,
    float* __restrict__ wzp, TmGeom g, int64_t nblocks) {
  constexpr int NW = C / 16;         // waves
  constexpr int CPR = C / 8;         // 16-byte chunks per row
  constexpr int KS = C / 32;         // 32-deep k steps
  constexpr int RP = C + 8;          // row staging pitch (bf16)
  constexpr int PP = 40;             // plane staging pitch (bf16)
  constexpr int HT = C / 16;         // 16-channel tiles of the xln side of dWz
  constexpr int TILE = 32 * C;       // elements of one [32][C] (or [C][32]) tile
  __shared__ __attribute__((aligned(1024))) __bf16 Rg[kOutBwdDepth][4][TILE];  // xln | gl | dout | x
  __shared__ __attribute__((aligned(256))) float Ss[kOutBwdDepth][2][64];      // mean | rstd
  __shared__ __attribute__((aligned(16))) float Rs[2][NW][32];
  __shared__ __attribute__((aligned(16))) __bf16 Dy[32 * RP];
  __shared__ __attribute__((aligned(16))) __bf16 Dg[32 * RP];
  __shared__ __attribute__((aligned(16))) __bf16 Dx[C * PP];

  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int l16 = lane & 15, lg = lane >> 4;
  const int ch = 16 * w + l16;
  const bool loader = w < NW / 2;

  bf16x8 wf[KS], wtf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    wf[ks] = ld8(wz + (int64_t)ch * C + 8 * (4 * ks + lg));
    wtf[ks] = ld8(wzt + (int64_t)ch * C + 8 * (4 * ks + lg));
  }
  const float gam = gamma[ch];

  const i32x4 rs_in[3] = {buffer_rsrc(xln), buffer_rsrc(gl), buffer_rsrc(dout)};
  const i32x4 rs_x = buffer_rsrc(x);
  const i32x4 rs_mu = buffer_rsrc(mean);
  const i32x4 rs_rs = buffer_rsrc(rstd);
  const __amdgpu_buffer_rsrc_t rs_dp = __builtin_amdgcn_make_buffer_rsrc(dproj5, 0, 0x7FFFFFFF, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs_dx = __builtin_amdgcn_make_buffer_rsrc(dx, 0, 0x7FFFFFFF, 0x00020000);
  TM_BLOCKS_CONTIGUOUS(nblocks);
  // Loads per block and loading wave: 2 instructions for each of xln, gl,
  // dout (rows, chunk-rotated) and x (plane segments); wave 0 also loads the
  // two statistics rows.
  auto issue = [&](int64_t blk) {
    const int stage = (int)(blk % kOutBwdDepth);
#pragma unroll
    for (int t = 0; t < 3; ++t)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int ci = (2 * w + j) * 64 + lane;
        const int r = ci / CPR, slot = ci % CPR;
        const int gc = (slot - r % CPR + CPR) % CPR;
        const uint32_t m = (uint32_t)pb(blk) * 32 + r;
        const bool ok = blk < bend && m < (uint32_t)g.R;
        buf2lds16(rs_in[t], ok ? (m * C + 8 * gc) * 2 : kBufOOB, &Rg[stage][t][(2 * w + j) * 512]);
      }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int ci = (2 * w + j) * 64 + lane;  // (channel ci / 4, 8-position part ci % 4)
      const int c = ci >> 2, part = ci & 3;
      const uint32_t mb = (uint32_t)pb(blk) * 32 + 8 * part;
      const bool ok = blk < bend && mb < (uint32_t)g.R;
      buf2lds16(rs_x, ok ? tm_plane_elem32(g, mb, c) * 2 : kBufOOB, &Rg[stage][3][(2 * w + j) * 512]);
    }
    if (w == 0) {
      const uint32_t m = (uint32_t)pb(blk) * 32 + lane;
      const bool ok = lane < 32 && blk < bend && m < (uint32_t)g.R;
      buf2lds4(rs_mu, ok ? m * 4 : kBufOOB, &Ss[stage][0][0]);
      buf2lds4(rs_rs, ok ? m * 4 : kBufOOB, &Ss[stage][1][0]);
    }
  };

  float cg = 0.f, cgx = 0.f;
  // dWz partial of this workgroup's rows: dWz[o][h] = sum_r dy[r][o] xln[r][h]
  // with dy^T (wave w's 16 output channels) as the A operand and xln as the
  // B operand, both column fragments of the row-major LDS tiles (32 rows =
  // the MFMA's k); register e of lane l: o = 16 w + 4 lg + e, h = 16 j + l16.
  f32x4 dwz[HT];
#pragma unroll
  for (int j = 0; j < HT; ++j) dwz[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // Column fragment of 4 rows r0 .. r0 + 3 x 16 columns c0 .. c0 + 15 of a
  // row-major tile (element (r, c) at off(r, c)): lane j of each 16-lane
  // group receives { M[r0 + e][c0 + j] : e = 0..3 } (ds_read_b64_tr_b16).
  auto col4 = [&](const __bf16* M, auto off, int r0, int c0) {
    const int r = r0 + (l16 >> 2), c = c0 + 4 * (l16 & 3);
    return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)&M[off(r, c)]);
  };
  auto dy_off = [](int r, int c) { return r * RP + c; };
  auto xl_off = [](int r, int c) { return r * C + 8 * (((c >> 3) + r) % CPR) + (c & 7); };
  if (loader) {
    issue(bbeg);
    issue(bbeg + 1);
  }
#pragma unroll 1
  for (int64_t blk = bbeg; blk < bend; ++blk) {
    const int stage = (int)(blk % kOutBwdDepth);
    if (loader) {  // block blk landed (block blk + 1 may be in flight)
      if (w == 0) wait_vmcnt<10>(); else wait_vmcnt<8>();
    }
    __syncthreads();
    if (loader) issue(blk + 2);
    // y^T = Wz xln^T (the weight rows as the A operand): register e of lane
    // l holds y[row 16 rt + l16][channel 16 w + 4 lg + e], so gl and dout are
    // plain 8-byte reads of the row tiles and dy / d gl 8-byte writes.
    f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    const __bf16* Xl = Rg[stage][0];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        const int row = 16 * rt + l16;
        const bf16x8 af =
            *reinterpret_cast<const bf16x8*>(&Xl[row * C + 8 * ((4 * ks + lg + row) % CPR)]);
        acc[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[ks], af, acc[rt], 0, 0, 0);
      }
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int row = 16 * rt + l16, cc = 16 * w + 4 * lg;
      const int off = row * C + 8 * (((cc >> 3) + row) % CPR) + (cc & 7);
      const bf16x4 gv4 = *reinterpret_cast<const bf16x4*>(&Rg[stage][1][off]);
      const bf16x4 go4 = *reinterpret_cast<const bf16x4*>(&Rg[stage][2][off]);
      bf16x4 vy, vg;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float sg = sigmoidf(bf2f(gv4[e]));
        const float go = bf2f(go4[e]);
        vy[e] = f2bf(go * sg);
        vg[e] = f2bf(go * acc[rt][e] * sg * (1.f - sg));
      }
      *reinterpret_cast<bf16x4*>(&Dy[row * RP + cc]) = vy;
      *reinterpret_cast<bf16x4*>(&Dg[row * RP + cc]) = vg;
    }
    __syncthreads();
    // G = dy Wz, then the LayerNorm backward (channel ch of LN_out).
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) acc[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        const bf16x8 af = *reinterpret_cast<const bf16x8*>(&Dy[(16 * rt + l16) * RP + 8 * (4 * ks + lg)]);
        acc[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, wtf[ks], acc[rt], 0, 0, 0);
      }
    {
      const bf16x8 dyt = cat8(col4(Dy, dy_off, 8 * lg, 16 * w), col4(Dy, dy_off, 8 * lg + 4, 16 * w));
      const __bf16* Xl2 = Rg[stage][0];
#pragma unroll
      for (int j = 0; j < HT; ++j) {
        const bf16x8 xb = cat8(col4(Xl2, xl_off, 8 * lg, 16 * j), col4(Xl2, xl_off, 8 * lg + 4, 16 * j));
        dwz[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(dyt, xb, dwz[j], 0, 0, 0);
      }
    }
    float xh[2][4], gv[2][4], a[8], b[8];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int r0 = 16 * rt + 4 * lg;
      const bf16x4 xv = *reinterpret_cast<const bf16x4*>(&Rg[stage][3][ch * 32 + r0]);
      const f32x4 mu = *reinterpret_cast<const f32x4*>(&Ss[stage][0][r0]);
      const f32x4 rsd = *reinterpret_cast<const f32x4*>(&Ss[stage][1][r0]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xh[rt][e] = (bf2f(xv[e]) - mu[e]) * rsd[e];
        const float G = acc[rt][e];
        gv[rt][e] = G * gam;
        a[4 * rt + e] = gv[rt][e];
        b[4 * rt + e] = gv[rt][e] * xh[rt][e];
        cg += G;
        cgx = fmaf(G, xh[rt][e], cgx);
      }
    }
    tm_butterfly<4>(a, b, lane);
    tm_butterfly<2>(a, b, lane);
    tm_butterfly<1>(a, b, lane);
    a[0] += dpp_f<kDppXor8>(a[0]);
    b[0] += dpp_f<kDppXor8>(b[0]);
    if (l16 < 8) {
      const int t = l16, row = 16 * (t >> 2) + 4 * lg + (t & 3);
      Rs[0][w][row] = a[0];
      Rs[1][w][row] = b[0];
    }
    __syncthreads();
    const float invC = 1.f / C;
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int r0 = 16 * rt + 4 * lg;
      const f32x4 rsd = *reinterpret_cast<const f32x4*>(&Ss[stage][1][r0]);
      f32x4 sg, sx;
      wave_row_sums<NW>(&Rs[0][0][0], r0, lane, sg, sx);
      bf16x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        o[e] = f2bf(rsd[e] * (gv[rt][e] - sg[e] * invC - xh[rt][e] * (sx[e] * invC)));
      *reinterpret_cast<bf16x4*>(&Dx[ch * PP + r0]) = o;
    }
    __syncthreads();
    if (!loader) {
      // d gl rows (into dproj5's last block), dx plane segments: 4 C chunks
      // each over the 2 C storing threads.
      const int st = tid - 2 * C;
      bf16x8 v[6];
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        const int q = st + 2 * C * it, row = q / CPR, k = q % CPR;
        v[2 + it] = *reinterpret_cast<const bf16x8*>(&Dg[row * RP + 8 * k]);
        v[4 + it] = *reinterpret_cast<const bf16x8*>(&Dx[(q >> 2) * PP + 8 * (q & 3)]);
      }
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        const int q = st + 2 * C * it, row = q / CPR, k = q % CPR;
        const uint32_t m = (uint32_t)pb(blk) * 32 + row;
        const bool ok = m < (uint32_t)g.R;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v[2 + it]), rs_dp,
                                               ok ? (m * 5 * C + 4 * C + 8 * k) * 2 : kBufOOB, 0, 0);
        const uint32_t mb = (uint32_t)pb(blk) * 32 + 8 * (q & 3);
        __builtin_amdgcn_raw_buffer_store_b128(
            __builtin_bit_cast(u32x4, v[4 + it]), rs_dx,
            mb < (uint32_t)g.R ? tm_plane_elem32(g, mb, q >> 2) * 2 : kBufOOB, 0, 0);
      }
    }
  }
  // The ring loads issued past the last block still write LDS: let them land
  // before the workgroup releases its LDS.
  if (loader) wait_vmcnt<0>();
  cg = xor32_sum(xor16_sum(cg));
  cgx = xor32_sum(xor16_sum(cgx));
  if (lg == 0) {
    lnp[(int64_t)blockIdx.x * 2 * C + ch] = cgx;
    lnp[(int64_t)blockIdx.x * 2 * C + C + ch] = cg;
  }
  float* wp = wzp + (int64_t)blockIdx.x * C * C;
#pragma unroll
  for (int j = 0; j < HT; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) wp[(16 * w + 4 * lg + e) * C + 16 * j + l16] = dwz[j][e];
}

// ---------------------------------------------------------------------------
// Output projection forward, weight-stationary (N % 8 == 0 not required:
// rows are natural, row-major): out = (xln Wz^T) s(gl), persistent
// workgroups of C / 16 waves over 32-row blocks.  Wave w holds the Wz rows of
// channels 16 w .. 16 w + 15 (B operands of v_mfma_f32_16x16x32_bf16); the
// loading waves stream xln and gl rows (chunk-rotated) into a 4-deep LDS
// ring; gl is read back transposed to match the accumulators; out is staged
// as [row][channel] and stored as full rows by the storing waves.
// ---------------------------------------------------------------------------
constexpr int kOutFwdDepth = 4;
template <int C>
__global__ __launch_bounds__(4 * C) void tm_out_proj_fwd_ws_kernel(
    const __bf16* __restrict__ xln, const __bf16* __restrict__ wz, const __bf16* __restrict__ gl,
    __bf16* __restrict__ out, TmGeom g, int64_t nblocks) {
  constexpr int NW = C / 16;         // waves
  constexpr int CPR = C / 8;         // 16-byte chunks per row
  constexpr int KS = C / 32;         // 32-deep k steps
  constexpr int RP = C + 8;          // staging pitch (bf16)
  __shared__ __attribute__((aligned(1024))) __bf16 Rg[kOutFwdDepth][2][32 * C];  // xln | gl
  __shared__ __attribute__((aligned(16))) __bf16 Or[2][32 * RP];

  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int l16 = lane & 15, lg = lane >> 4;
  const int ch = 16 * w + l16;
  const bool loader = w < NW / 2;

  bf16x8 wf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) wf[ks] = ld8(wz + (int64_t)ch * C + 8 * (4 * ks + lg));
  const i32x4 rs_in[2] = {buffer_rsrc(xln), buffer_rsrc(gl)};
  const __amdgpu_buffer_rsrc_t rs_o = __builtin_amdgcn_make_buffer_rsrc(out, 0, 0x7FFFFFFF, 0x00020000);
  TM_BLOCKS_STRIDED(nblocks);
  // Loads per block and loading wave: 2 instructions each for xln and gl.
  auto issue = [&](int64_t blk) {
    const int stage = (int)(blk % kOutFwdDepth);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int ci = (2 * w + j) * 64 + lane;
        const int r = ci / CPR, slot = ci % CPR;
        const int gc = (slot - r % CPR + CPR) % CPR;
        const uint32_t m = (uint32_t)pb(blk) * 32 + r;
        const bool ok = blk < bend && m < (uint32_t)g.R;
        buf2lds16(rs_in[t], ok ? (m * C + 8 * gc) * 2 : kBufOOB, &Rg[stage][t][(2 * w + j) * 512]);
      }
  };
  if (loader) {
#pragma unroll
    for (int d = 0; d < kOutFwdDepth - 1; ++d) issue(bbeg + d);
    wait_vmcnt<4 * (kOutFwdDepth - 2)>();  // block bbeg landed
  }
  __syncthreads();
#pragma unroll 1
  for (int64_t blk = bbeg; blk < bend; ++blk) {
    const int stage = (int)(blk % kOutFwdDepth);
    const int sb = (int)(blk & 1);
    if (loader) issue(blk + kOutFwdDepth - 1);
    f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    const __bf16* Xl = Rg[stage][0];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        const int row = 16 * rt + l16;
        const bf16x8 af =
            *reinterpret_cast<const bf16x8*>(&Xl[row * C + 8 * ((4 * ks + lg + row) % CPR)]);
        acc[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, wf[ks], acc[rt], 0, 0, 0);
      }
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      // gl for rows 16 rt + 4 lg + e, channel ch: lane L of a 16-lane group
      // reads row 16 rt + 4 lg + L / 4, channels 16 w + 4 (L % 4) .. + 3.
      const int rr = 16 * rt + 4 * lg + (l16 >> 2);
      const int cc = 16 * w + 4 * (l16 & 3);
      const bf16x4 gv4 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
          (lds_bf16x4*)&Rg[stage][1][rr * C + 8 * (((cc >> 3) + rr) % CPR) + (cc & 7)]);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        Or[sb][(16 * rt + 4 * lg + e) * RP + ch] = f2bf(acc[rt][e] * sigmoidf(bf2f(gv4[e])));
    }
    if (loader) wait_vmcnt<4 * (kOutFwdDepth - 2)>();  // block blk + 1 landed
    __syncthreads();
    if (!loader) {
      // 4 C chunks (32 rows x C / 8) over the 2 C storing threads.
      const int st = tid - 2 * C;
      bf16x8 v[2];
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        const int q = st + 2 * C * it, row = q / CPR, k = q % CPR;
        v[it] = *reinterpret_cast<const bf16x8*>(&Or[sb][row * RP + 8 * k]);
      }
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        const int q = st + 2 * C * it, row = q / CPR, k = q % CPR;
        const uint32_t m = (uint32_t)pb(blk) * 32 + row;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v[it]), rs_o,
                                               m < (uint32_t)g.R ? (m * C + 8 * k) * 2 : kBufOOB, 0, 0);
      }
    }
  }
  // The ring loads issued past the last block still write LDS: let them land
  // before the workgroup releases its LDS.
  if (loader) wait_vmcnt<0>();
}

// Zero-fill (used instead of hipMemsetAsync so callers may capture graphs).
__global__ __launch_bounds__(256) void zero_u32_kernel(uint32_t* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    p[i] = 0u;
}

static int zero_fill(void* p, int64_t bytes, hipStream_t s, const char* fn) {
  const int64_t n = bytes / 4;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  if (blocks < 1) return TPF_OK;
  hipLaunchKernelGGL(zero_u32_kernel, dim3((unsigned)blocks), dim3(256), 0, s, (uint32_t*)p, n);
  return check_launch(fn);
}

}  // namespace tpf

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
using namespace tpf;

// Whether the kernels' 32-bit buffer offsets cover a B x N x N x C pair:
// every row tensor of C channels and every channel-major plane tensor within
// a 2 GiB window, and row indices within int32 / 2; the backward also holds
// dproj5, rows of 5 C channels.
static bool tm_extent_ok(int64_t B, int64_t N, int64_t C, bool backward) {
  if (B < 1 || N < 1 || B > INT32_MAX || N > INT32_MAX / 8) return false;
  const int64_t Np = (N + 7) / 8 * 8;
  const double R = (double)B * (double)N * (double)N;
  if (R > (double)(INT32_MAX / 2)) return false;
  const double lim = (double)kBufOOB;
  const int64_t pitch = backward ? 5 * C : C;
  return R * (double)pitch * 2 < lim && (double)B * C * N * Np * 2 < lim;
}

static int tm_geom(TmGeom* g, int64_t B, int64_t N, int64_t C, int outgoing, const char* fn,
                   bool backward) {
  if (B < 1 || N < 1) return set_error(TPF_ERR_SHAPE, "%s: B and N must be positive", fn);
  if (C != 32 && C != 64 && C != 96 && C != 128)
    return set_error(TPF_ERR_SHAPE, "%s: C=%lld must be one of 32, 64, 96, 128", fn, (long long)C);
  const int64_t Np = (N + 7) / 8 * 8;
  const int64_t R = B * N * N;
  if (!tm_extent_ok(B, N, C, backward))
    return set_error(TPF_ERR_SHAPE,
                     "%s: B=%lld N=%lld C=%lld too large (a %s tensor would exceed 2 GiB)", fn,
                     (long long)B, (long long)N, (long long)C,
                     backward ? "pair, plane or dproj5" : "pair or plane");
  g->B = (int)B; g->N = (int)N; g->Np = (int)Np; g->H = (int)C;
  g->NN = N * N; g->PS = N * Np; g->R = R; g->outgoing = outgoing ? 1 : 0;
  g->ntg = (int)((C + 63) / 64);
  g->div_n = make_fastdiv((uint32_t)N);
  g->div_nn = make_fastdiv((uint32_t)(N * N));
  return TPF_OK;
}

static int64_t align256(int64_t v) { return (v + 255) / 256 * 256; }
static int64_t tm_wp_rows(int64_t C) { return 2 * ((C + 63) / 64) * 128; }
static int64_t tm_weights_bytes(int64_t C) {
  return align256(tm_wp_rows(C) * C * 2) + 2 * align256(5 * C * C * 2) + 2 * align256(C * C * 2);
}

// Packed bf16 weights at the start of a workspace.
struct TmPacked {
  __bf16* wp;
  __bf16* w5;
  __bf16* wz;
  __bf16* w5t;
  __bf16* wzt;
};
static TmPacked tm_packed(void* ws, int64_t C) {
  char* p = (char*)ws;
  TmPacked k;
  k.wp = (__bf16*)p;
  p += align256(tm_wp_rows(C) * C * 2);
  k.w5 = (__bf16*)p;
  p += align256(5 * C * C * 2);
  k.wz = (__bf16*)p;
  p += align256(C * C * 2);
  k.w5t = (__bf16*)p;
  p += align256(5 * C * C * 2);
  k.wzt = (__bf16*)p;
  return k;
}

static int tm_pack(const TmWeights& w, const TmPacked& k, int C, int ntg, hipStream_t s,
                   const char* fn) {
  const int64_t chunks = (tm_wp_rows(C) + 12 * C) * (C / 8);
  hipLaunchKernelGGL(tm_pack_weights_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0,
                     s, w, k.wp, k.w5, k.wz, k.w5t, k.wzt, C, ntg);
  return check_launch(fn);
}

static unsigned tm_grid(int64_t tiles) { return (unsigned)((tiles + 7) / 8 * 8); }


#define TM_DISPATCH_C(C, KERNEL, GRID, ...)                                                   \
  switch (C) {                                                                               \
    case 32: hipLaunchKernelGGL(KERNEL<32>, GRID, dim3(256), 0, s, __VA_ARGS__); break;     \
    case 64: hipLaunchKernelGGL(KERNEL<64>, GRID, dim3(256), 0, s, __VA_ARGS__); break;     \
    case 96: hipLaunchKernelGGL(KERNEL<96>, GRID, dim3(256), 0, s, __VA_ARGS__); break;     \
    default: hipLaunchKernelGGL(KERNEL<128>, GRID, dim3(256), 0, s, __VA_ARGS__); break;    \
  }

extern "C" {

int64_t tpf_trimul_plane_pitch(int64_t N) { return (N + 7) / 8 * 8; }

int tpf_trimul_shape_supported(int64_t B, int64_t N, int64_t C, int backward) {
  if (C != 32 && C != 64 && C != 96 && C != 128) return 0;
  return tm_extent_ok(B, N, C, backward != 0) ? 1 : 0;
}

int64_t tpf_trimul_forward_workspace_bytes(int64_t C) { return tm_weights_bytes(C); }

int tpf_trimul_forward_bf16(const void* z, const float* mask, const float* w_ap, const float* w_ag,
                            const float* w_bp, const float* w_bg, const float* w_g,
                            const float* w_z, const float* ln_in_w, const float* ln_in_b,
                            const float* ln_out_w, const float* ln_out_b, int outgoing, int64_t B,
                            int64_t N, int64_t C, void* out, void* zln, void* gate, void* a,
                            void* b, void* x, void* xln, float* mean_in, float* rstd_in,
                            float* mean_out, float* rstd_out, void* workspace,
                            int64_t workspace_bytes, void* stream) {
  const char* fn = "tpf_trimul_forward_bf16";
  TmGeom g;
  int rc = tm_geom(&g, B, N, C, outgoing, fn, false);
  if (rc) return rc;
  if (!z || !mask || !w_ap || !w_ag || !w_bp || !w_bg || !w_g || !w_z || !ln_in_w || !ln_in_b ||
      !ln_out_w || !ln_out_b || !out || !zln || !gate || !a || !b || !x || !xln || !mean_in ||
      !rstd_in || !mean_out || !rstd_out || !workspace)
    return set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  if (workspace_bytes < tm_weights_bytes(C))
    return set_error(TPF_ERR_ARG, "%s: workspace %lld < required %lld", fn,
                     (long long)workspace_bytes, (long long)tm_weights_bytes(C));
  hipStream_t s = (hipStream_t)stream;
  const TmPacked k = tm_packed(workspace, C);
  const TmWeights w{w_ap, w_ag, w_bp, w_bg, w_g, w_z};
  if ((rc = tm_pack(w, k, (int)C, g.ntg, s, fn))) return rc;
  if (g.Np != g.N) {
    // The contraction reads whole rows of Np; pad columns must be zero.  It
    // stores only the N real columns of x, so x's pad is cleared too: the
    // saved state is then a function of the inputs alone.
    if ((rc = zero_fill(a, B * C * g.PS * 2, s, fn))) return rc;
    if ((rc = zero_fill(b, B * C * g.PS * 2, s, fn))) return rc;
    if ((rc = zero_fill(x, B * C * g.PS * 2, s, fn))) return rc;
  }
  TM_DISPATCH_C(C, tm_ln_rows_kernel, dim3((unsigned)tm_ln_rows_grid(g.R)), (const __bf16*)z, ln_in_w,
                ln_in_b, (__bf16*)zln, mean_in, rstd_in, g.R);
  if ((rc = check_launch("tpf_trimul_forward_bf16(ln_in)"))) return rc;
  const int64_t tiles = (g.R + 127) / 128;
  {
    // Persistent: one workgroup of C / 16 waves per CU share at C = 128.
    const int64_t nblk = (g.R + 31) / 32;
    const int64_t cap = (int64_t)device_cus() * (128 / C);
    const unsigned grid = (unsigned)(nblk < cap ? nblk : cap);
    switch (C) {
#define TM_IN_FWD(CC)                                                                           \
  case CC:                                                                                      \
    if (g.Np == g.N)                                                                            \
      hipLaunchKernelGGL((tm_in_proj_fwd_kernel<CC, false>), dim3(grid), dim3(4 * CC), 0, s,    \
                         (const __bf16*)zln, k.w5, mask, (__bf16*)a, (__bf16*)b, (__bf16*)gate, \
                         g, nblk);                                                              \
    else                                                                                        \
      hipLaunchKernelGGL((tm_in_proj_fwd_kernel<CC, true>), dim3(grid), dim3(4 * CC), 0, s,     \
                         (const __bf16*)zln, k.w5, mask, (__bf16*)a, (__bf16*)b, (__bf16*)gate, \
                         g, nblk);                                                              \
    break;
      TM_IN_FWD(32) TM_IN_FWD(64) TM_IN_FWD(96) TM_IN_FWD(128)
#undef TM_IN_FWD
    }
  }
  if ((rc = check_launch("tpf_trimul_forward_bf16(in_proj)"))) return rc;
  GemmArgs ga{};
  ga.A = (const __bf16*)a; ga.a_ld = g.Np; ga.a_bs = g.PS;
  ga.B = (const __bf16*)b; ga.b_ld = g.Np; ga.b_bs = g.PS;
  ga.C = x; ga.c_ld = g.Np; ga.c_bs = g.PS;
  ga.M = (int)N; ga.N = (int)N; ga.K = g.Np; ga.ksplit = 1; ga.k_chunk = g.Np; ga.alpha = 1.f;
  if ((rc = gemm_launch(ga, 1, 1, 0, (int)(B * C), s, "tpf_trimul_forward_bf16(contract)",
                        tm_contract_tile(N))))
    return rc;
  TM_DISPATCH_C(C, tm_ln_planes_kernel, dim3((unsigned)tm_ln_planes_grid(g.NN, B), (unsigned)B),
                (const __bf16*)x, ln_out_w, ln_out_b, (__bf16*)xln, mean_out, rstd_out, g);
  if ((rc = check_launch("tpf_trimul_forward_bf16(ln_out)"))) return rc;
  {
    const int64_t nblk = (g.R + 31) / 32;
    const int64_t cap = (int64_t)device_cus() * (128 / C);
    const unsigned grid = (unsigned)(nblk < cap ? nblk : cap);
    switch (C) {
#define TM_OUT_FWD(CC)                                                                          \
  case CC:                                                                                      \
    hipLaunchKernelGGL(tm_out_proj_fwd_ws_kernel<CC>, dim3(grid), dim3(4 * CC), 0, s,           \
                       (const __bf16*)xln, k.wz, (const __bf16*)gate, (__bf16*)out, g, nblk);   \
    break;
      TM_OUT_FWD(32) TM_OUT_FWD(64) TM_OUT_FWD(96) TM_OUT_FWD(128)
#undef TM_OUT_FWD
    }
  }
  return check_launch("tpf_trimul_forward_bf16(out_proj)");
}

// Backward workspace (each region 256-byte aligned): packed weights, dy
// [R][C], dproj5 [R][5H], dx / da / db channel-major planes, LN_out
// parameter partials [tiles][2][C], LN_in parameter partials [<= R/32][2][C],
// split-K partials of dW5 and dWz.
static int tm_split(int64_t R, int64_t per, int cap) {
  int64_t s = R / per;
  if (s < 1) s = 1;
  if (s > cap) s = cap;
  return (int)s;
}
// dWz on the split-K GEMM (N % 8 != 0) takes K ranges of 2304 rows
// (measured at N = 384: 576-row ranges cost 18 us more per out + in step, in
// the larger fold).  dW5 takes as many K ranges as fill one round of 512
// workgroups with its ceil(5C / 128) x ceil(C / 128) output tiles (at least
// 256 rows each): shape-only, so its fold order is the same on any device.
static int tm_w5_splits(int64_t R, int64_t C) {
  const int64_t tiles = ((5 * C + 127) / 128) * ((C + 127) / 128);
  return tm_split(R, 256, (int)(512 / tiles));
}
static int tm_wz_splits(int64_t R) { return tm_split(R, 2304, 64); }
// Workgroups of the persistent backward kernels that leave per-workgroup
// partials (LN parameter and dWz sums): a fixed plan of 256 CUs, so the
// partition of the rows, and every summation order, depends on the shape
// only (the same bits on any device).
constexpr int64_t kTmPlanCus = 256;
static int64_t tm_bwd_grid(int64_t R, int64_t C) {
  const int64_t nblk = (R + 31) / 32, cap = kTmPlanCus * (128 / C);
  return nblk < cap ? nblk : cap;
}

int64_t tpf_trimul_backward_workspace_bytes(int64_t B, int64_t N, int64_t C) {
  const int64_t Np = (N + 7) / 8 * 8, R = B * N * N;
  const int64_t tiles = (R + 127) / 128;
  int64_t t = tm_weights_bytes(C);
  t += align256(R * C * 2);                        // dy
  t += align256(R * 5 * C * 2);                    // dproj5
  t += 3 * align256(B * C * N * Np * 2);           // dx, da, db
  t += align256((R + 31) / 32 * 2 * C * 4);        // LN_out parameter partials (tiles or workgroups)
  t += align256((R + 31) / 32 * 2 * C * 4);        // LN_in parameter partials (per workgroup)
  t += align256((int64_t)tm_w5_splits(R, C) * 5 * C * C * 4);
  const int64_t wz_parts = tm_wz_splits(R) > tm_bwd_grid(R, C) ? tm_wz_splits(R) : tm_bwd_grid(R, C);
  t += align256(wz_parts * C * C * 4);  // dWz partials (split-K GEMM or per workgroup)
  return t;
}

}  // extern "C"

// The TriMul backward; the five H x C row blocks of the W5 gradient
// (ap, ag, bp, bg, g) land at w5dst[0..4].
static int trimul_backward_impl(
    const void* grad_out, const void* z, const float* mask, const float* w_ap,
    const float* w_ag, const float* w_bp, const float* w_bg, const float* w_g, const float* w_z,
    const float* ln_in_w, const float* ln_out_w, const void* zln, const void* gate, const void* a,
    const void* b, const void* x, const void* xln, const float* mean_in, const float* rstd_in,
    const float* mean_out, const float* rstd_out, int outgoing, int64_t B, int64_t N, int64_t C,
    void* dz, float* const w5dst[5], float* d_w_z, float* d_ln_in_w, float* d_ln_in_b,
    float* d_ln_out_w, float* d_ln_out_b, void* workspace, int64_t workspace_bytes, void* stream,
    const char* fn) {
  float* const d_w5 = w5dst[0];
  TmGeom g;
  int rc = tm_geom(&g, B, N, C, outgoing, fn, true);
  if (rc) return rc;
  if (!grad_out || !z || !mask || !w_ap || !w_ag || !w_bp || !w_bg || !w_g || !w_z || !ln_in_w ||
      !ln_out_w || !zln || !gate || !a || !b || !x || !xln || !mean_in || !rstd_in || !mean_out ||
      !rstd_out || !dz || !d_w5 || !w5dst[1] || !w5dst[2] || !w5dst[3] || !w5dst[4] || !d_w_z ||
      !d_ln_in_w || !d_ln_in_b || !d_ln_out_w || !d_ln_out_b || !workspace)
    return set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  const int64_t need = tpf_trimul_backward_workspace_bytes(B, N, C);
  if (workspace_bytes < need)
    return set_error(TPF_ERR_ARG, "%s: workspace %lld < required %lld", fn,
                     (long long)workspace_bytes, (long long)need);
  hipStream_t s = (hipStream_t)stream;
  const int64_t R = g.R, H = C;
  const int64_t tiles = (R + 127) / 128;
  const int s5 = tm_w5_splits(R, C), sz = tm_wz_splits(R);
  const TmPacked k = tm_packed(workspace, C);
  const TmWeights w{w_ap, w_ag, w_bp, w_bg, w_g, w_z};
  char* wp_ = (char*)workspace + tm_weights_bytes(C);
  auto take = [&](int64_t bytes) { char* p = wp_; wp_ += align256(bytes); return p; };
  __bf16* dy = (__bf16*)take(R * C * 2);
  __bf16* dproj5 = (__bf16*)take(R * 5 * H * 2);
  const int64_t plane_bytes = B * C * g.PS * 2;
  __bf16* dx = (__bf16*)take(plane_bytes);
  __bf16* da = (__bf16*)take(plane_bytes);
  __bf16* db = (__bf16*)take(plane_bytes);
  float* lnp = (float*)take((R + 31) / 32 * 2 * C * 4);
  float* lnin = (float*)take((R + 31) / 32 * 2 * C * 4);
  float* w5p = (float*)take((int64_t)s5 * 5 * C * C * 4);
  float* wzp = (float*)take((int64_t)(sz > tm_bwd_grid(R, C) ? sz : tm_bwd_grid(R, C)) * C * C * 4);
  if ((rc = tm_pack(w, k, (int)C, g.ntg, s, fn))) return rc;
  // Pad columns of dx are read by the dA GEMM (K = Np) and must be zero.
  if (g.Np != g.N && (rc = zero_fill(dx, plane_bytes, s, fn))) return rc;
  const unsigned grid_rows = tm_grid(tiles);
  int lnp_splits = (int)tiles;  // LN_out parameter partials
  if (g.Np == g.N) {
    // Output projection backward + LN_out backward in one pass.
    const int64_t nblk = (R + 31) / 32;
    lnp_splits = (int)tm_bwd_grid(R, C);
    switch (C) {
#define TM_OUT_BWD(CC)                                                                          \
  case CC:                                                                                      \
    hipLaunchKernelGGL(tm_out_bwd_ws_kernel<CC>, dim3(lnp_splits), dim3(4 * CC), 0, s,          \
                       (const __bf16*)xln, k.wz, k.wzt, (const __bf16*)gate,                    \
                       (const __bf16*)grad_out, (const __bf16*)x, mean_out, rstd_out, ln_out_w, \
                       dproj5, dx, lnp, wzp, g, nblk);                                          \
    break;
      TM_OUT_BWD(32) TM_OUT_BWD(64) TM_OUT_BWD(96) TM_OUT_BWD(128)
#undef TM_OUT_BWD
    }
    if ((rc = check_launch("tpf_trimul_backward_bf16(out_proj + ln_out_bwd)"))) return rc;
  } else {
    hipLaunchKernelGGL(tm_out_proj_bwd_kernel, dim3(grid_rows), dim3(256), 0, s,
                       (const __bf16*)xln, k.wz, (const __bf16*)gate, (const __bf16*)grad_out,
                       dy, dproj5, g, (int)C);
    if ((rc = check_launch("tpf_trimul_backward_bf16(out_proj)"))) return rc;
    hipLaunchKernelGGL(tm_ln_out_bwd_kernel, dim3(grid_rows), dim3(256), 0, s, (const __bf16*)dy,
                       (int64_t)C, k.wz, (int)C, (const __bf16*)x, mean_out,
                       rstd_out, ln_out_w, dx, lnp, g, (int)H);
    if ((rc = check_launch("tpf_trimul_backward_bf16(ln_out_bwd)"))) return rc;
  }
  // Contraction backward: dA_c = dX_c B_c, dB_c = dX_c^T A_c (stored layouts).
  GemmArgs ga{};
  ga.A = dx; ga.a_ld = g.Np; ga.a_bs = g.PS;
  ga.B = (const __bf16*)b; ga.b_ld = g.Np; ga.b_bs = g.PS;
  ga.C = da; ga.c_ld = g.Np; ga.c_bs = g.PS;
  ga.M = (int)N; ga.N = (int)N; ga.K = g.Np; ga.ksplit = 1; ga.k_chunk = g.Np; ga.alpha = 1.f;
  // K = Np runs over dX's zero pad columns; the matching rows of B_c past N
  // do not exist (past the last plane they are past the tensor): read zeros.
  ga.b_kmax = (int)N;
  GemmArgs gb{};
  gb.A = dx; gb.a_ld = g.Np; gb.a_bs = g.PS;
  gb.B = (const __bf16*)a; gb.b_ld = g.Np; gb.b_bs = g.PS;
  gb.C = db; gb.c_ld = g.Np; gb.c_bs = g.PS;
  gb.M = (int)N; gb.N = (int)N; gb.K = (int)N; gb.ksplit = 1; gb.k_chunk = (int)N; gb.alpha = 1.f;
  // dA and dB in one launch (2 x B*C batched tiles keep the tail short).
  ga.batch = (int)(B * C);
  gb.batch = (int)(B * C);
  if ((rc = gemm_launch_pair(ga, 1, 0, gb, 0, 0, 0, s, "tpf_trimul_backward_bf16(dA, dB)",
                             tm_contract_tile(N))))
    return rc;
  if (g.Np == g.N) {
    const int64_t nblk = (R + 31) / 32;
    const int64_t cap = (int64_t)device_cus() * (128 / C);
    const unsigned grid = (unsigned)(nblk < cap ? nblk : cap);
    switch (C) {
#define TM_IN_BWD(CC)                                                                            \
  case CC:                                                                                       \
    hipLaunchKernelGGL(tm_in_proj_bwd_ws_kernel<CC>, dim3(grid), dim3(4 * CC), 0, s,             \
                       (const __bf16*)zln, k.w5, mask, (const __bf16*)da, (const __bf16*)db,     \
                       dproj5, g, nblk);                                                         \
    break;
      TM_IN_BWD(32) TM_IN_BWD(64) TM_IN_BWD(96) TM_IN_BWD(128)
#undef TM_IN_BWD
    }
  } else {
    hipLaunchKernelGGL(tm_in_proj_bwd_kernel, dim3(tm_grid(tiles * 2 * g.ntg)), dim3(256), 0, s,
                       (const __bf16*)zln, k.wp, mask, da, db, dproj5, g, (int)C);
  }
  if ((rc = check_launch("tpf_trimul_backward_bf16(in_proj)"))) return rc;
  const int64_t ln_blk = (R + 31) / 32;
  const int ln_grid = (int)tm_bwd_grid(R, C);
  switch (C) {
#define TM_LN_IN(CC)                                                                            \
  case CC:                                                                                      \
    hipLaunchKernelGGL(tm_ln_in_bwd_ws_kernel<CC>, dim3(ln_grid), dim3(4 * CC), 0, s,           \
                       (const __bf16*)dproj5, k.w5t, (const __bf16*)z, mean_in, rstd_in,        \
                       ln_in_w, (__bf16*)dz, lnin, g, ln_blk);                                  \
    break;
    TM_LN_IN(32) TM_LN_IN(64) TM_LN_IN(96) TM_LN_IN(128)
#undef TM_LN_IN
  }
  if ((rc = check_launch("tpf_trimul_backward_bf16(ln_in_bwd)"))) return rc;
  // Weight gradients over all rows: MN operands straight from the row-major
  // tensors, split-K + fixed-order fold.
  GemmArgs gw{};
  gw.A = dproj5; gw.a_ld = 5 * H; gw.a_bs = 0;
  gw.B = (const __bf16*)zln; gw.b_ld = C; gw.b_bs = 0;
  gw.C = w5p; gw.c_ld = C; gw.c_bs = 0; gw.c_split = 5 * C * C;
  gw.M = (int)(5 * H); gw.N = (int)C; gw.K = (int)R; gw.ksplit = s5;
  gw.k_chunk = (int)((R + s5 - 1) / s5); gw.alpha = 1.f;
  GemmArgs gz{};
  gz.A = dy; gz.a_ld = C; gz.a_bs = 0;
  gz.B = (const __bf16*)xln; gz.b_ld = H; gz.b_bs = 0;
  gz.C = wzp; gz.c_ld = H; gz.c_bs = 0; gz.c_split = C * H;
  gz.M = (int)C; gz.N = (int)H; gz.K = (int)R; gz.ksplit = sz;
  gz.k_chunk = (int)((R + sz - 1) / sz); gz.alpha = 1.f;
  gw.batch = 1;
  gz.batch = 1;
  const bool wz_fused = g.Np == g.N;  // tm_out_bwd_ws_kernel left per-workgroup dWz partials
  if (wz_fused) {
    if ((rc = gemm_launch_wgrad(gw, s, "tpf_trimul_backward_bf16(dW5)"))) return rc;
  } else {
    // dW5 and dWz are independent split-K GEMMs of ~300 tiles each: one
    // launch keeps both in flight together.
    if ((rc = gemm_launch_pair_wgrad(gw, gz, s, "tpf_trimul_backward_bf16(dW5, dWz)")))
      return rc;
  }
  // The four weight-gradient folds in one launch per pass; the LayerNorm
  // partials ([tiles][ln_out_w | ln_out_b] and [workgroups][ln_in_w |
  // ln_in_b]) land directly in the four parameter gradients.
  // The W5 partials fold as two segments: rows ap | ag | bp | bg (four
  // H x C pieces) and g; each element's fold is the same either way.
  FoldSegs f{};
  f.nseg = 5;
  f.part[0] = w5p; f.n[0] = 4 * H * C; f.stride[0] = 5 * C * C; f.splits[0] = s5;
  f.piece[0] = H * C;
  for (int j = 0; j < 4; ++j) f.dst[0][j] = w5dst[j];
  f.part[4] = w5p + 4 * H * C; f.n[4] = C * C; f.stride[4] = 5 * C * C; f.splits[4] = s5;
  f.piece[4] = C * C; f.dst[4][0] = w5dst[4];
  f.part[1] = wzp; f.n[1] = C * H; f.stride[1] = C * H; f.splits[1] = wz_fused ? lnp_splits : sz;
  f.piece[1] = C * H; f.dst[1][0] = d_w_z;
  f.part[2] = lnp; f.n[2] = 2 * C; f.stride[2] = 2 * C; f.splits[2] = lnp_splits;
  f.piece[2] = C;
  f.dst[2][0] = d_ln_out_w; f.dst[2][1] = d_ln_out_b;
  f.part[3] = lnin; f.n[3] = 2 * C; f.stride[3] = 2 * C; f.splits[3] = ln_grid;
  f.piece[3] = C;
  f.dst[3][0] = d_ln_in_w; f.dst[3][1] = d_ln_in_b;
  return fold_multi(f, s, fn);
}

extern "C" {

int tpf_trimul_backward_bf16(const void* grad_out, const void* z, const float* mask,
                             const float* w_ap, const float* w_ag, const float* w_bp,
                             const float* w_bg, const float* w_g, const float* w_z,
                             const float* ln_in_w, const float* ln_out_w, const void* zln,
                             const void* gate, const void* a, const void* b, const void* x,
                             const void* xln, const float* mean_in, const float* rstd_in,
                             const float* mean_out, const float* rstd_out, int outgoing, int64_t B,
                             int64_t N, int64_t C, void* dz, float* d_w5, float* d_w_z,
                             float* d_ln_in_w, float* d_ln_in_b, float* d_ln_out_w,
                             float* d_ln_out_b, void* workspace, int64_t workspace_bytes,
                             void* stream) {
  const int64_t hc = C * C;  // H = C
  float* const w5dst[5] = {d_w5, d_w5 ? d_w5 + hc : nullptr, d_w5 ? d_w5 + 2 * hc : nullptr,
                           d_w5 ? d_w5 + 3 * hc : nullptr, d_w5 ? d_w5 + 4 * hc : nullptr};
  return trimul_backward_impl(grad_out, z, mask, w_ap, w_ag, w_bp, w_bg, w_g, w_z, ln_in_w,
                              ln_out_w, zln, gate, a, b, x, xln, mean_in, rstd_in, mean_out,
                              rstd_out, outgoing, B, N, C, dz, w5dst, d_w_z, d_ln_in_w, d_ln_in_b,
                              d_ln_out_w, d_ln_out_b, workspace, workspace_bytes, stream,
                              "tpf_trimul_backward_bf16");
}

int tpf_trimul_backward_named_bf16(
    const void* grad_out, const void* z, const float* mask, const float* w_ap, const float* w_ag,
    const float* w_bp, const float* w_bg, const float* w_g, const float* w_z,
    const float* ln_in_w, const float* ln_out_w, const void* zln, const void* gate, const void* a,
    const void* b, const void* x, const void* xln, const float* mean_in, const float* rstd_in,
    const float* mean_out, const float* rstd_out, int outgoing, int64_t B, int64_t N, int64_t C,
    void* dz, float* d_p_in, float* d_g_in, float* d_w_g, float* d_w_z, float* d_ln_in_w,
    float* d_ln_in_b, float* d_ln_out_w, float* d_ln_out_b, void* workspace,
    int64_t workspace_bytes, void* stream) {
  const int64_t hc = C * C;  // H = C
  float* const w5dst[5] = {d_p_in, d_g_in, d_p_in ? d_p_in + hc : nullptr,
                           d_g_in ? d_g_in + hc : nullptr, d_w_g};
  return trimul_backward_impl(grad_out, z, mask, w_ap, w_ag, w_bp, w_bg, w_g, w_z, ln_in_w,
                              ln_out_w, zln, gate, a, b, x, xln, mean_in, rstd_in, mean_out,
                              rstd_out, outgoing, B, N, C, dz, w5dst, d_w_z, d_ln_in_w, d_ln_in_b,
                              d_ln_out_w, d_ln_out_b, workspace, workspace_bytes, stream,
                              "tpf_trimul_backward_named_bf16");
}

}  // extern "C"
