// Triangle multiplicative update (TriMul) on gfx950: fused row-tile kernels
// around the channel-batched MFMA contraction of csrc/gemm.hip.
//
// Stock math (openfold3/core/model/layers/triangular_multiplicative_update.py
// :1263-1284 and :734-760; LayerNorm openfold3/core/model/primitives/
// normalization.py:54-78, f32 statistics, eps 1e-5):
//   zln = LN_in(z);  a = mask * sigmoid(zln Wag^T) * (zln Wap^T);  b likewise
//   outgoing: x[c,i,j] = sum_k a[i,k,c] b[j,k,c];  incoming: sum_k a[k,i,c] b[k,j,c]
//   out = (LN_out(x) Wz^T) * sigmoid(zln Wg^T)
//
// Storage (C == H channels, rows rho = (b*N + r)*N + s of z [B,N,N,C]):
//   z, zln, out, dz: [R][C] bf16 row-major; dgl (output-gate logit grad)
//   [R][H].  Weight-gradient operands are stored transposed, [channel][Rp]
//   (Rp = R rounded up to 8, pad zero): dy^T, xln^T, zln^T and dproj5^T
//   whose channel blocks are [d p_in (2H) | d g_in (2H) | d g_out (H)].
//   a, b (and da, db) channel-major "stored" matrices A_c[i][k], B_c[j][k]
//   with plane size N*Np (row pitch Np = N rounded up to 8, pad columns
//   zero): outgoing A_c[i][k] = a[i,k,c]; incoming A_c[i][k] = a[k,i,c].
//   Both directions then contract as x_c = A_c B_c^T (an NT GEMM).
//   x, dx: channel-major [B*H][N][Np] in natural (i, j) order.
// A tile is 64 positions of one batch item; for a/b tiles the position p is
// i*N + k of the stored matrix, so stores are contiguous in both directions.
#include "common.hpp"
#include "tpf_gemm.hpp"
#include "tpf_status.hpp"

namespace tpf {

struct TmGeom {
  int B, N, Np;
  int64_t NN;     // N*N positions per batch item
  int64_t PS;     // N*Np elements per channel-major plane
  int outgoing;
};

// Source row (b, r, s) of stored-matrix position p = i*N + k.
__device__ __forceinline__ int64_t tm_src_row(const TmGeom& g, int b, int64_t p) {
  if (g.outgoing) return (int64_t)b * g.NN + p;
  const int64_t i = p / g.N, k = p % g.N;  // A_c[i][k] = a[k, i, c]
  return (int64_t)b * g.NN + k * g.N + i;
}
// Element offset of position p = i*N + j inside a channel-major plane.
__device__ __forceinline__ int64_t tm_plane_off(const TmGeom& g, int64_t p) {
  return (g.Np == g.N) ? p : (p / g.N) * g.Np + (p % g.N);
}

// LayerNorm of 64 rows (4 threads per row) into an LDS bf16 tile.
// rows[i] < 0 marks a padding row (written as zeros).  Returns nothing;
// optionally stores mean/rstd and the normalised rows to global memory.
template <int C>
__device__ __forceinline__ void tm_layernorm_tile(const __bf16* __restrict__ src,
                                                  const int64_t* rows, const float* __restrict__ w,
                                                  const float* __restrict__ bias, __bf16* Ts,
                                                  int pitch, float* __restrict__ mean_out,
                                                  float* __restrict__ rstd_out,
                                                  __bf16* __restrict__ save) {
  constexpr int CPT = C / 4;  // channels per thread (multiple of 8)
  const int tid = threadIdx.x, row = tid >> 2, part = tid & 3;
  const int64_t rho = rows[row];
  float x[CPT];
  if (rho >= 0) {
#pragma unroll
    for (int c8 = 0; c8 < CPT / 8; ++c8) {
      bf16x8 v = ld8(src + rho * C + part * CPT + c8 * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[c8 * 8 + e] = bf2f(v[e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < CPT; ++e) x[e] = 0.f;
  }
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < CPT; ++e) s += x[e];
  s += __shfl_xor(s, 1);
  s += __shfl_xor(s, 2);
  const float mean = s * (1.f / C);
  float v2 = 0.f;
#pragma unroll
  for (int e = 0; e < CPT; ++e) { const float d = x[e] - mean; v2 = fmaf(d, d, v2); }
  v2 += __shfl_xor(v2, 1);
  v2 += __shfl_xor(v2, 2);
  const float rstd = rsqrtf(v2 * (1.f / C) + 1e-5f);
#pragma unroll
  for (int c8 = 0; c8 < CPT / 8; ++c8) {
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int c = part * CPT + c8 * 8 + e;
      o[e] = rho >= 0 ? f2bf((x[c8 * 8 + e] - mean) * rstd * w[c] + bias[c]) : f2bf(0.f);
    }
    *reinterpret_cast<bf16x8*>(&Ts[row * pitch + part * CPT + c8 * 8]) = o;
    if (save && rho >= 0) st8(save + rho * C + part * CPT + c8 * 8, o);
  }
  if (part == 0 && rho >= 0 && mean_out) {
    mean_out[rho] = mean;
    rstd_out[rho] = rstd;
  }
}

// acc += A(32 rows of LDS tile, K=KD) * W[n0 + lane col][0..KD)^T
template <int KD>
__device__ __forceinline__ f32x16 tile_mm(const __bf16* As, int pitch, int row0,
                                          const __bf16* __restrict__ W, int ldw, int n, f32x16 acc) {
  const int lane = threadIdx.x & 63, rl = lane & 31, hl = lane >> 5;
#pragma unroll
  for (int s = 0; s < KD / 16; ++s) {
    bf16x8 a = *reinterpret_cast<const bf16x8*>(&As[(row0 + rl) * pitch + 16 * s + 8 * hl]);
    bf16x8 b = ld8(W + (int64_t)n * ldw + 16 * s + 8 * hl);
    acc = mfma32(a, b, acc);
  }
  return acc;
}

// ---------------------------------------------------------------------------
// Forward stage 1: LN_in, the four branch projections, gating and mask.
// Wave w: rows 32*(w&1).., branch w>>1 (0 = a, 1 = b).
// ---------------------------------------------------------------------------
template <int C>
__global__ __launch_bounds__(256) void tm_in_fwd_kernel(
    const __bf16* __restrict__ z, const float* __restrict__ mask,
    const __bf16* __restrict__ p_in, const __bf16* __restrict__ g_in,
    const float* __restrict__ ln_w, const float* __restrict__ ln_b, __bf16* __restrict__ a_out,
    __bf16* __restrict__ b_out, __bf16* __restrict__ zln, float* __restrict__ mean_in,
    float* __restrict__ rstd_in, TmGeom g) {
  constexpr int H = C, P = C + 8;
  __shared__ __attribute__((aligned(16))) __bf16 Zs[64 * P];
  __shared__ int64_t rows[64];
  const int tid = threadIdx.x, b = blockIdx.y;
  const int64_t p0 = (int64_t)blockIdx.x * 64;
  if (tid < 64) rows[tid] = (p0 + tid < g.NN) ? tm_src_row(g, b, p0 + tid) : -1;
  __syncthreads();
  tm_layernorm_tile<C>(z, rows, ln_w, ln_b, Zs, P, mean_in, rstd_in, zln);
  __syncthreads();

  const int w = tid >> 6, lane = tid & 63, rl = lane & 31, hl = lane >> 5;
  const int rb = w & 1, br = w >> 1;
  __bf16* dst = br ? b_out : a_out;
  float mk[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = rb * 32 + 8 * (r >> 2) + 4 * hl + (r & 3);
    mk[r] = rows[row] >= 0 ? mask[rows[row]] : 0.f;
  }
  for (int cb = 0; cb < H / 32; ++cb) {
    const int n = cb * 32 + rl;
    f32x16 ap = tile_mm<C>(Zs, P, rb * 32, p_in + (int64_t)br * H * C, C, n, zero16());
    f32x16 ag = tile_mm<C>(Zs, P, rb * 32, g_in + (int64_t)br * H * C, C, n, zero16());
    __bf16* plane = dst + ((int64_t)b * H + n) * g.PS;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t p = p0 + rb * 32 + 8 * j + 4 * hl;
      float val[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) val[i] = mk[4 * j + i] * sigmoidf(ag[4 * j + i]) * ap[4 * j + i];
      if (g.Np == g.N && (g.NN & 3) == 0 && p + 3 < g.NN) {
        bf16x4 v4;
#pragma unroll
        for (int i = 0; i < 4; ++i) v4[i] = f2bf(val[i]);
        *reinterpret_cast<bf16x4*>(plane + p) = v4;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (p + i < g.NN) plane[tm_plane_off(g, p + i)] = f2bf(val[i]);
      }
    }
  }
}

// Load a channel-major [H][T positions] tile of x (natural order) as bf16
// into LDS Xb[c * pitch + pp]; zeros past the end of the plane.
template <int H, int T>
__device__ __forceinline__ void tm_load_chmajor(const __bf16* __restrict__ x, const TmGeom& g,
                                                int b, int64_t p0, __bf16* Xb, int pitch) {
  const bool vec = (g.Np == g.N) && (g.NN % 8 == 0) && (p0 + T <= g.NN);
  if (vec) {
    for (int idx = threadIdx.x; idx < H * (T / 8); idx += 256) {
      const int c = idx / (T / 8), ch = idx % (T / 8);
      bf16x8 v = ld8(x + ((int64_t)b * H + c) * g.PS + p0 + ch * 8);
      *reinterpret_cast<bf16x8*>(&Xb[c * pitch + ch * 8]) = v;
    }
  } else {
    for (int idx = threadIdx.x; idx < H * T; idx += 256) {
      const int c = idx / T, pp = idx % T;
      const int64_t p = p0 + pp;
      Xb[c * pitch + pp] = (p < g.NN) ? x[((int64_t)b * H + c) * g.PS + tm_plane_off(g, p)]
                                      : static_cast<__bf16>(0.f);
    }
  }
}

// Store 4 values at consecutive row indices tau..tau+3 of a transposed
// [channel][Rp] buffer row; rows >= lim (end of the batch item) are skipped.
__device__ __forceinline__ void st4_rows(__bf16* __restrict__ row_base, int64_t tau, int64_t R,
                                         const float (&v)[4]) {
  if ((tau & 3) == 0 && tau + 3 < R) {
    bf16x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = f2bf(v[i]);
    *reinterpret_cast<bf16x4*>(row_base + tau) = o;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (tau + i < R) row_base[tau + i] = f2bf(v[i]);
  }
}

// Write an LDS tile S[row * pitch + c] (T rows x NC channels) transposed to
// dst[(c0 + c) * Rp + tau0 + row] for rows with tau0 + row < R (R = end of
// the batch item's rows).
template <int NC, int T>
__device__ __forceinline__ void tm_store_transposed(const __bf16* S, int pitch, __bf16* __restrict__ dst,
                                                    int c0, int64_t Rp, int64_t tau0, int64_t R) {
  const bool vec = (tau0 % 8 == 0) && (tau0 + T <= R);
  for (int idx = threadIdx.x; idx < NC * (T / 8); idx += 256) {
    const int c = idx / (T / 8), ch = idx % (T / 8);
    __bf16* d = dst + (int64_t)(c0 + c) * Rp + tau0 + ch * 8;
    if (vec) {
      bf16x8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = S[(ch * 8 + e) * pitch + c];
      st8(d, v);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (tau0 + ch * 8 + e < R) d[e] = S[(ch * 8 + e) * pitch + c];
    }
  }
}

// ---------------------------------------------------------------------------
// Forward stage 3: LN_out over the channel-major product, output projection
// and the sigmoid output gate from zln.  Rows in natural order.
// ---------------------------------------------------------------------------
template <int C>
__global__ __launch_bounds__(256) void tm_out_fwd_kernel(
    const __bf16* __restrict__ x, const __bf16* __restrict__ zln,
    const __bf16* __restrict__ p_out, const __bf16* __restrict__ g_out,
    const float* __restrict__ ln_w, const float* __restrict__ ln_b, __bf16* __restrict__ out,
    __bf16* __restrict__ xln, float* __restrict__ mean_out, float* __restrict__ rstd_out,
    TmGeom g) {
  constexpr int H = C, P = C + 8, XP = 64 + 8;
  __shared__ __attribute__((aligned(16))) __bf16 Xb[H * XP];
  __shared__ __attribute__((aligned(16))) __bf16 Xs[64 * P];
  __shared__ __attribute__((aligned(16))) __bf16 Zs[64 * P];
  const int tid = threadIdx.x, b = blockIdx.y;
  const int64_t p0 = (int64_t)blockIdx.x * 64;
  tm_load_chmajor<H, 64>(x, g, b, p0, Xb, XP);
  for (int idx = tid; idx < 64 * (C / 8); idx += 256) {
    const int row = idx / (C / 8), c8 = (idx % (C / 8)) * 8;
    const int64_t p = p0 + row;
    bf16x8 v = (p < g.NN) ? ld8(zln + ((int64_t)b * g.NN + p) * C + c8) : zero8();
    *reinterpret_cast<bf16x8*>(&Zs[row * P + c8]) = v;
  }
  __syncthreads();
  {  // LN over channels of each row: 4 threads per row.
    constexpr int CPT = H / 4;
    const int row = tid >> 2, part = tid & 3;
    const int64_t p = p0 + row;
    float xv[CPT];
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < CPT; ++e) { xv[e] = bf2f(Xb[(part * CPT + e) * XP + row]); s += xv[e]; }
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    const float mean = s * (1.f / H);
    float v2 = 0.f;
#pragma unroll
    for (int e = 0; e < CPT; ++e) { const float d = xv[e] - mean; v2 = fmaf(d, d, v2); }
    v2 += __shfl_xor(v2, 1);
    v2 += __shfl_xor(v2, 2);
    const float rstd = rsqrtf(v2 * (1.f / H) + 1e-5f);
    const int64_t rho = (int64_t)b * g.NN + p;
#pragma unroll
    for (int c8 = 0; c8 < CPT / 8; ++c8) {
      bf16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int c = part * CPT + c8 * 8 + e;
        o[e] = f2bf((xv[c8 * 8 + e] - mean) * rstd * ln_w[c] + ln_b[c]);
      }
      *reinterpret_cast<bf16x8*>(&Xs[row * P + part * CPT + c8 * 8]) = o;
      if (xln && p < g.NN) st8(xln + rho * H + part * CPT + c8 * 8, o);
    }
    if (part == 0 && p < g.NN && mean_out) { mean_out[rho] = mean; rstd_out[rho] = rstd; }
  }
  __syncthreads();
  const int w = tid >> 6, lane = tid & 63, rl = lane & 31, hl = lane >> 5;
  const int rb = w & 1;
  for (int cb = w >> 1; cb < C / 32; cb += 2) {
    const int n = cb * 32 + rl;
    f32x16 y = tile_mm<H>(Xs, P, rb * 32, p_out, H, n, zero16());
    f32x16 gl = tile_mm<C>(Zs, P, rb * 32, g_out, C, n, zero16());
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t p = p0 + rb * 32 + 8 * (r >> 2) + 4 * hl + (r & 3);
      if (p < g.NN) out[((int64_t)b * g.NN + p) * C + n] = f2bf(y[r] * sigmoidf(gl[r]));
    }
  }
}

// ---------------------------------------------------------------------------
// Backward stage 1 (32-row tiles, natural row order): output gate, output
// projection and LN_out backward.
//   dy = dout * s(gl); dgl = dout * y * s(gl) (1 - s(gl));  d_xln = dy Wz
//   dx = rstd * (g - mean(g) - xhat * mean(g * xhat)),  g = d_xln * gamma_out
// Writes dx channel-major, dgl row-major [R][H], dy^T and xln^T as
// [channel][Rp] (K-contiguous operands of the weight-gradient GEMM), and
// per-workgroup partials of d gamma_out / d beta_out.
// ---------------------------------------------------------------------------
template <int C>
__global__ __launch_bounds__(256) void tm_out_bwd_kernel(
    const __bf16* __restrict__ dout, const __bf16* __restrict__ x,
    const __bf16* __restrict__ xln, const __bf16* __restrict__ zln,
    const float* __restrict__ mean_out, const float* __restrict__ rstd_out,
    const __bf16* __restrict__ p_out, const __bf16* __restrict__ g_out,
    const __bf16* __restrict__ p_out_t, const float* __restrict__ ln_w,
    __bf16* __restrict__ dy_t, __bf16* __restrict__ xln_t, __bf16* __restrict__ dgl,
    __bf16* __restrict__ dx, float* __restrict__ dgamma_part, float* __restrict__ dbeta_part,
    TmGeom g, int64_t Rp) {
  constexpr int H = C, T = 32, P = C + 8, XP = T + 8, GP = H + 4;
  __shared__ __attribute__((aligned(16))) __bf16 Xb[H * XP];     // x tile, channel-major
  __shared__ __attribute__((aligned(16))) __bf16 XZ[2 * T * P];  // xln | zln, later d_xln f32
  __shared__ __attribute__((aligned(16))) __bf16 Ds[T * P];      // dy tile
  __shared__ __attribute__((aligned(16))) __bf16 Dx[H * XP];     // dx tile, channel-major
  __shared__ float mst[T], rst[T];
  __bf16* Xs = XZ;
  __bf16* Zs = XZ + T * P;
  float* Gf = reinterpret_cast<float*>(XZ);
  const int tid = threadIdx.x, b = blockIdx.y;
  const int64_t p0 = (int64_t)blockIdx.x * T;
  // Transposed stores stop at the end of this batch item's rows.
  const int64_t lim = (int64_t)b * g.NN + g.NN;
  const int64_t tau0 = (int64_t)b * g.NN + p0;
  tm_load_chmajor<H, T>(x, g, b, p0, Xb, XP);
  for (int idx = tid; idx < T * (C / 8); idx += 256) {
    const int row = idx / (C / 8), c8 = (idx % (C / 8)) * 8;
    const bool ok = p0 + row < g.NN;
    const int64_t rho = tau0 + row;
    *reinterpret_cast<bf16x8*>(&Zs[row * P + c8]) = ok ? ld8(zln + rho * C + c8) : zero8();
    *reinterpret_cast<bf16x8*>(&Xs[row * P + c8]) = ok ? ld8(xln + rho * H + c8) : zero8();
  }
  if (tid < T) {
    const bool ok = p0 + tid < g.NN;
    mst[tid] = ok ? mean_out[tau0 + tid] : 0.f;
    rst[tid] = ok ? rstd_out[tau0 + tid] : 0.f;
  }
  __syncthreads();
  tm_store_transposed<H, T>(Xs, P, xln_t, 0, Rp, tau0, lim);
  const int w = tid >> 6, lane = tid & 63, rl = lane & 31, hl = lane >> 5;
  for (int cb = w; cb < C / 32; cb += 4) {
    const int n = cb * 32 + rl;
    f32x16 y = tile_mm<H>(Xs, P, 0, p_out, H, n, zero16());
    f32x16 gl = tile_mm<C>(Zs, P, 0, g_out, C, n, zero16());
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float dyv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * j + i, row = 8 * j + 4 * hl + i;
        const bool ok = p0 + row < g.NN;
        const int64_t rho = tau0 + row;
        const float go = ok ? bf2f(dout[rho * C + n]) : 0.f;
        const float sg = sigmoidf(gl[r]);
        dyv[i] = go * sg;
        Ds[row * P + n] = f2bf(dyv[i]);
        if (ok) dgl[rho * H + n] = f2bf(go * y[r] * sg * (1.f - sg));
      }
      st4_rows(dy_t + (int64_t)n * Rp, tau0 + 8 * j + 4 * hl, lim, dyv);
    }
  }
  __syncthreads();
  // d_xln (T x H) = dy (T x C) * Wz (C x H); B operand = rows of Wz^T.
  {
    f32x16 d = zero16();
    const bool has = w < H / 32;
    if (has) d = tile_mm<C>(Ds, P, 0, p_out_t, C, w * 32 + rl, d);
    if (has) {
#pragma unroll
      for (int r = 0; r < 16; ++r) Gf[(8 * (r >> 2) + 4 * hl + (r & 3)) * GP + w * 32 + rl] = d[r];
    }
  }
  __syncthreads();
  {  // LN_out backward: 8 threads per row.
    constexpr int CPT = H / 8;
    const int row = tid >> 3, part = tid & 7;
    const float mean = mst[row], rstd = rst[row];
    float sg = 0.f, sgx = 0.f;
#pragma unroll
    for (int e = 0; e < CPT; ++e) {
      const int c = part * CPT + e;
      const float xh = (bf2f(Xb[c * XP + row]) - mean) * rstd;
      const float gv = Gf[row * GP + c] * ln_w[c];
      sg += gv;
      sgx = fmaf(gv, xh, sgx);
    }
#pragma unroll
    for (int m = 1; m < 8; m <<= 1) { sg += __shfl_xor(sg, m); sgx += __shfl_xor(sgx, m); }
    sg *= 1.f / H;
    sgx *= 1.f / H;
#pragma unroll
    for (int e = 0; e < CPT; ++e) {
      const int c = part * CPT + e;
      const float xh = (bf2f(Xb[c * XP + row]) - mean) * rstd;
      const float gv = Gf[row * GP + c] * ln_w[c];
      Dx[c * XP + row] = f2bf(rstd * (gv - sg - xh * sgx));
    }
  }
  __syncthreads();
  {
    const bool vec = (g.Np == g.N) && (g.NN % 8 == 0) && (p0 + T <= g.NN);
    for (int idx = tid; idx < H * (T / 8); idx += 256) {
      const int c = idx / (T / 8), ch = idx % (T / 8);
      __bf16* plane = dx + ((int64_t)b * H + c) * g.PS;
      if (vec) {
        st8(plane + p0 + ch * 8, *reinterpret_cast<const bf16x8*>(&Dx[c * XP + ch * 8]));
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int64_t p = p0 + ch * 8 + e;
          if (p < g.NN) plane[tm_plane_off(g, p)] = Dx[c * XP + ch * 8 + e];
        }
      }
    }
  }
  if (tid < H) {
    float sgm = 0.f, sbt = 0.f;
    for (int row = 0; row < T; ++row) {
      const float gr = Gf[row * GP + tid];
      const float xh = (bf2f(Xb[tid * XP + row]) - mst[row]) * rst[row];
      sgm = fmaf(gr, xh, sgm);
      sbt += gr;
    }
    const int64_t blk = (int64_t)b * gridDim.x + blockIdx.x;
    dgamma_part[blk * 4 * H + tid] = sgm;
    dbeta_part[blk * 4 * H + tid] = sbt;
  }
}

// ---------------------------------------------------------------------------
// Backward stage 3 (32-row tiles in stored-matrix order): gate / mask
// backward of the four branch projections (recomputed from zln),
// d_zln = dproj5 * W5, LN_in backward.  Writes dproj5^T and zln^T as
// [channel][Rp] in tile order (K-contiguous weight-gradient operands).
// ---------------------------------------------------------------------------
template <int C>
__global__ __launch_bounds__(256) void tm_in_bwd_kernel(
    const __bf16* __restrict__ z, const __bf16* __restrict__ zln, const float* __restrict__ mask,
    const __bf16* __restrict__ p_in, const __bf16* __restrict__ g_in,
    const __bf16* __restrict__ da, const __bf16* __restrict__ db,
    const __bf16* __restrict__ dgl, const __bf16* __restrict__ w5_t,
    const float* __restrict__ mean_in, const float* __restrict__ rstd_in,
    const float* __restrict__ ln_w, __bf16* __restrict__ dproj5_t, __bf16* __restrict__ zln_t,
    __bf16* __restrict__ dz, float* __restrict__ dgamma_part, float* __restrict__ dbeta_part,
    TmGeom g, int64_t Rp) {
  constexpr int H = C, T = 32, P = C + 8, PP = 5 * H + 8, GP = C + 4;
  __shared__ __attribute__((aligned(16))) __bf16 Zs[T * P];
  __shared__ __attribute__((aligned(16))) __bf16 Ps[T * PP];  // later: d_zln | xhat (f32)
  __shared__ int64_t rows[T];
  __shared__ float mst[T], rst[T];
  float* Gf = reinterpret_cast<float*>(Ps);
  float* Xh = Gf + T * GP;
  const int tid = threadIdx.x, b = blockIdx.y;
  const int64_t p0 = (int64_t)blockIdx.x * T;
  // Transposed stores stop at the end of this batch item's rows.
  const int64_t lim = (int64_t)b * g.NN + g.NN;
  const int64_t tau0 = (int64_t)b * g.NN + p0;
  if (tid < T) {
    const int64_t rho = (p0 + tid < g.NN) ? tm_src_row(g, b, p0 + tid) : -1;
    rows[tid] = rho;
    mst[tid] = rho >= 0 ? mean_in[rho] : 0.f;
    rst[tid] = rho >= 0 ? rstd_in[rho] : 0.f;
  }
  __syncthreads();
  for (int idx = tid; idx < T * (C / 8); idx += 256) {
    const int row = idx / (C / 8), c8 = (idx % (C / 8)) * 8;
    const int64_t rho = rows[row];
    *reinterpret_cast<bf16x8*>(&Zs[row * P + c8]) = rho >= 0 ? ld8(zln + rho * C + c8) : zero8();
    *reinterpret_cast<bf16x8*>(&Ps[row * PP + 4 * H + c8]) =
        rho >= 0 ? ld8(dgl + rho * H + c8) : zero8();
  }
  __syncthreads();
  tm_store_transposed<C, T>(Zs, P, zln_t, 0, Rp, tau0, lim);
  tm_store_transposed<H, T>(Ps + 4 * H, PP, dproj5_t, 4 * H, Rp, tau0, lim);
  const int w = tid >> 6, lane = tid & 63, rl = lane & 31, hl = lane >> 5;
  const int br = w >> 1;
  const __bf16* dsrc = br ? db : da;
  float mk[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = 8 * (r >> 2) + 4 * hl + (r & 3);
    mk[r] = rows[row] >= 0 ? mask[rows[row]] : 0.f;
  }
  const bool vec = (g.Np == g.N) && (g.NN % 4 == 0);
  for (int cb = w & 1; cb < H / 32; cb += 2) {
    const int n = cb * 32 + rl;
    f32x16 ap = tile_mm<C>(Zs, P, 0, p_in + (int64_t)br * H * C, C, n, zero16());
    f32x16 ag = tile_mm<C>(Zs, P, 0, g_in + (int64_t)br * H * C, C, n, zero16());
    const __bf16* plane = dsrc + ((int64_t)b * H + n) * g.PS;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t pj = p0 + 8 * j + 4 * hl;
      float dv[4];
      if (vec && pj + 3 < g.NN) {
        bf16x4 v4 = ld4(plane + pj);
#pragma unroll
        for (int i = 0; i < 4; ++i) dv[i] = bf2f(v4[i]);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) dv[i] = (pj + i < g.NN) ? bf2f(plane[tm_plane_off(g, pj + i)]) : 0.f;
      }
      float dpv[4], dgv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * j + i, row = 8 * j + 4 * hl + i;
        const float sg = sigmoidf(ag[r]);
        dpv[i] = dv[i] * mk[r] * sg;
        dgv[i] = dv[i] * mk[r] * ap[r] * sg * (1.f - sg);
        Ps[row * PP + br * H + n] = f2bf(dpv[i]);
        Ps[row * PP + 2 * H + br * H + n] = f2bf(dgv[i]);
      }
      st4_rows(dproj5_t + (int64_t)(br * H + n) * Rp, tau0 + 8 * j + 4 * hl, lim, dpv);
      st4_rows(dproj5_t + (int64_t)(2 * H + br * H + n) * Rp, tau0 + 8 * j + 4 * hl, lim, dgv);
    }
  }
  __syncthreads();
  {  // d_zln (T x C) = dproj5 (T x 5H) * W5 (5H x C); B operand rows of W5^T.
    f32x16 d = zero16();
    const bool has = w < C / 32;
    if (has) d = tile_mm<5 * H>(Ps, PP, 0, w5_t, 5 * H, w * 32 + rl, d);
    __syncthreads();  // Ps is overwritten by Gf below
    if (has) {
#pragma unroll
      for (int r = 0; r < 16; ++r) Gf[(8 * (r >> 2) + 4 * hl + (r & 3)) * GP + w * 32 + rl] = d[r];
    }
  }
  __syncthreads();
  {  // LN_in backward: 8 threads per row, 4-channel vectors.
    constexpr int CPT = C / 8;
    const int row = tid >> 3, part = tid & 7;
    const int64_t rho = rows[row];
    const bool ok = rho >= 0;
    const float mean = mst[row], rstd = rst[row];
    float xh[CPT];
#pragma unroll
    for (int c4 = 0; c4 < CPT / 4; ++c4) {
      bf16x4 v = ok ? ld4(z + rho * C + part * CPT + c4 * 4) : bf16x4{};
#pragma unroll
      for (int e = 0; e < 4; ++e) xh[c4 * 4 + e] = ok ? (bf2f(v[e]) - mean) * rstd : 0.f;
    }
    float sg = 0.f, sgx = 0.f;
#pragma unroll
    for (int e = 0; e < CPT; ++e) {
      const int c = part * CPT + e;
      const float gv = Gf[row * GP + c] * ln_w[c];
      sg += gv;
      sgx = fmaf(gv, xh[e], sgx);
      Xh[row * GP + c] = xh[e];
    }
#pragma unroll
    for (int m = 1; m < 8; m <<= 1) { sg += __shfl_xor(sg, m); sgx += __shfl_xor(sgx, m); }
    sg *= 1.f / C;
    sgx *= 1.f / C;
#pragma unroll
    for (int c4 = 0; c4 < CPT / 4; ++c4) {
      bf16x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int c = part * CPT + c4 * 4 + e;
        const float gv = Gf[row * GP + c] * ln_w[c];
        o[e] = f2bf(rstd * (gv - sg - xh[c4 * 4 + e] * sgx));
      }
      if (ok) *reinterpret_cast<bf16x4*>(dz + rho * C + part * CPT + c4 * 4) = o;
    }
  }
  __syncthreads();
  if (tid < C) {
    float sgm = 0.f, sbt = 0.f;
    for (int row = 0; row < T; ++row) {
      const float gr = Gf[row * GP + tid];
      sgm = fmaf(gr, Xh[row * GP + tid], sgm);
      sbt += gr;
    }
    const int64_t blk = (int64_t)b * gridDim.x + blockIdx.x;
    dgamma_part[blk * 4 * C + tid] = sgm;
    dbeta_part[blk * 4 * C + tid] = sbt;
  }
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
  hipLaunchKernelGGL(zero_u32_kernel, dim3((unsigned)blocks), dim3(256), 0, s, (uint32_t*)p, n);
  return check_launch(fn);
}

}  // namespace tpf

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
using namespace tpf;

static int tm_geom(TmGeom* g, int64_t B, int64_t N, int64_t C, int outgoing, const char* fn) {
  if (B < 1 || N < 1) return set_error(TPF_ERR_SHAPE, "%s: B and N must be positive", fn);
  if (C != 32 && C != 64 && C != 96 && C != 128)
    return set_error(TPF_ERR_SHAPE, "%s: C=%lld must be one of 32, 64, 96, 128", fn, (long long)C);
  if (N > 46340) return set_error(TPF_ERR_SHAPE, "%s: N=%lld too large", fn, (long long)N);
  g->B = (int)B; g->N = (int)N; g->Np = (int)((N + 7) / 8 * 8);
  g->NN = N * N; g->PS = N * (int64_t)g->Np; g->outgoing = outgoing ? 1 : 0;
  if ((g->NN + 63) / 64 > INT32_MAX || B > 65535)
    return set_error(TPF_ERR_SHAPE, "%s: grid too large", fn);
  return TPF_OK;
}

#define TM_DISPATCH(C, KERNEL, GRID, ...)                                                     \
  switch (C) {                                                                               \
    case 32: hipLaunchKernelGGL(KERNEL<32>, GRID, dim3(256), 0, s, __VA_ARGS__); break;     \
    case 64: hipLaunchKernelGGL(KERNEL<64>, GRID, dim3(256), 0, s, __VA_ARGS__); break;     \
    case 96: hipLaunchKernelGGL(KERNEL<96>, GRID, dim3(256), 0, s, __VA_ARGS__); break;     \
    default: hipLaunchKernelGGL(KERNEL<128>, GRID, dim3(256), 0, s, __VA_ARGS__); break;    \
  }

extern "C" {

int64_t tpf_trimul_plane_pitch(int64_t N) { return (N + 7) / 8 * 8; }

int tpf_trimul_forward_bf16(const void* z, const float* mask, const void* p_in, const void* g_in,
                            const void* p_out, const void* g_out, const float* ln_in_w,
                            const float* ln_in_b, const float* ln_out_w, const float* ln_out_b,
                            int outgoing, int64_t B, int64_t N, int64_t C, void* out, void* zln,
                            void* a, void* b, void* x, void* xln, float* mean_in, float* rstd_in,
                            float* mean_out, float* rstd_out, void* stream) {
  const char* fn = "tpf_trimul_forward_bf16";
  TmGeom g;
  int rc = tm_geom(&g, B, N, C, outgoing, fn);
  if (rc) return rc;
  if (!z || !mask || !p_in || !g_in || !p_out || !g_out || !ln_in_w || !ln_in_b || !ln_out_w ||
      !ln_out_b || !out || !zln || !a || !b || !x || !mean_in || !rstd_in)
    return set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  hipStream_t s = (hipStream_t)stream;
  if (g.Np != g.N) {
    // The contraction reads whole rows of Np; pad columns must be zero.
    if ((rc = zero_fill(a, B * C * g.PS * 2, s, fn))) return rc;
    if ((rc = zero_fill(b, B * C * g.PS * 2, s, fn))) return rc;
  }
  dim3 grid((unsigned)((g.NN + 63) / 64), (unsigned)B);
  TM_DISPATCH(C, tm_in_fwd_kernel, grid, (const __bf16*)z, mask, (const __bf16*)p_in,
              (const __bf16*)g_in, ln_in_w, ln_in_b, (__bf16*)a, (__bf16*)b, (__bf16*)zln,
              mean_in, rstd_in, g);
  if ((rc = check_launch("tpf_trimul_forward_bf16(in)"))) return rc;
  GemmArgs ga{};
  ga.A = (const __bf16*)a; ga.a_ld = g.Np; ga.a_bs = g.PS;
  ga.B = (const __bf16*)b; ga.b_ld = g.Np; ga.b_bs = g.PS;
  ga.C = x; ga.c_ld = g.Np; ga.c_bs = g.PS;
  ga.M = (int)N; ga.N = (int)N; ga.K = g.Np; ga.ksplit = 1; ga.k_chunk = g.Np; ga.alpha = 1.f;
  if ((rc = gemm_launch(ga, 1, 1, 0, (int)(B * C), s, "tpf_trimul_forward_bf16(contract)")))
    return rc;
  TM_DISPATCH(C, tm_out_fwd_kernel, grid, (const __bf16*)x, (const __bf16*)zln,
              (const __bf16*)p_out, (const __bf16*)g_out, ln_out_w, ln_out_b, (__bf16*)out,
              (__bf16*)xln, mean_out, rstd_out, g);
  return check_launch("tpf_trimul_forward_bf16(out)");
}

// Backward workspace (each region 256-byte aligned):
//   dy^T [C][Rp], xln^T [H][Rp], dproj5^T [5H][Rp], zln^T [C][Rp] (Rp = R
//   rounded up to 8; K-contiguous weight-gradient operands), dgl [R][H],
//   dx / da / db channel-major planes, LN parameter partials, split-K
//   partials of dW5 and dWz.
static int64_t align256(int64_t v) { return (v + 255) / 256 * 256; }

static int trimul_wgrad_splits(int64_t R) {
  int64_t s = R / 2048;
  if (s < 1) s = 1;
  if (s > 64) s = 64;
  return (int)s;
}

static int64_t tm_bwd_blocks(int64_t B, int64_t N) { return B * ((N * N + 31) / 32); }

int64_t tpf_trimul_backward_workspace_bytes(int64_t B, int64_t N, int64_t C) {
  const int64_t Np = (N + 7) / 8 * 8, R = B * N * N, Rp = (R + 7) / 8 * 8;
  const int64_t blocks = tm_bwd_blocks(B, N);
  const int64_t splits = trimul_wgrad_splits(R);
  int64_t t = 0;
  t += align256(C * Rp * 2);                      // dy^T
  t += align256(C * Rp * 2);                      // xln^T
  t += align256(5 * C * Rp * 2);                  // dproj5^T
  t += align256(C * Rp * 2);                      // zln^T
  t += align256(R * C * 2);                       // dgl
  t += 3 * align256(B * C * N * Np * 2);          // dx, da, db
  t += align256(blocks * 4 * C * 4);              // LN parameter partials [blocks][4][C]
  t += align256(4 * C * 4);                       // folded LN parameter grads
  t += align256(splits * 5 * C * C * 4);          // dW5 partials
  t += align256(splits * C * C * 4);              // dWz partials
  return t;
}

int tpf_trimul_backward_bf16(const void* grad_out, const void* z, const float* mask,
                             const void* p_in, const void* g_in, const void* p_out_t,
                             const void* w5_t, const void* p_out, const void* g_out,
                             const float* ln_in_w, const float* ln_out_w, const void* zln,
                             const void* a, const void* b, const void* x, const void* xln,
                             const float* mean_in, const float* rstd_in, const float* mean_out,
                             const float* rstd_out, int outgoing, int64_t B, int64_t N, int64_t C,
                             void* dz, float* d_w5, float* d_p_out, float* d_ln_in_w,
                             float* d_ln_in_b, float* d_ln_out_w, float* d_ln_out_b,
                             void* workspace, int64_t workspace_bytes, void* stream) {
  const char* fn = "tpf_trimul_backward_bf16";
  TmGeom g;
  int rc = tm_geom(&g, B, N, C, outgoing, fn);
  if (rc) return rc;
  if (!grad_out || !z || !mask || !p_in || !g_in || !p_out_t || !w5_t || !p_out || !g_out ||
      !ln_in_w || !ln_out_w || !zln || !a || !b || !x || !xln || !mean_in || !rstd_in ||
      !mean_out || !rstd_out || !dz || !d_w5 || !d_p_out || !d_ln_in_w || !d_ln_in_b ||
      !d_ln_out_w || !d_ln_out_b || !workspace)
    return set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  const int64_t need = tpf_trimul_backward_workspace_bytes(B, N, C);
  if (workspace_bytes < need)
    return set_error(TPF_ERR_ARG, "%s: workspace %lld < required %lld", fn,
                     (long long)workspace_bytes, (long long)need);
  hipStream_t s = (hipStream_t)stream;
  const int64_t R = B * N * N, Rp = (R + 7) / 8 * 8, H = C;
  const int64_t blocks = tm_bwd_blocks(B, N);
  const int splits = trimul_wgrad_splits(R);
  char* wp = (char*)workspace;
  auto take = [&](int64_t bytes) { char* p = wp; wp += align256(bytes); return p; };
  __bf16* dy_t = (__bf16*)take(C * Rp * 2);
  __bf16* xln_t = (__bf16*)take(C * Rp * 2);
  __bf16* dproj5_t = (__bf16*)take(5 * C * Rp * 2);
  __bf16* zln_t = (__bf16*)take(C * Rp * 2);
  __bf16* dgl = (__bf16*)take(R * C * 2);
  const int64_t plane_bytes = B * C * g.PS * 2;
  __bf16* dx = (__bf16*)take(plane_bytes);
  __bf16* da = (__bf16*)take(plane_bytes);
  __bf16* db = (__bf16*)take(plane_bytes);
  float* lnp = (float*)take(blocks * 4 * C * 4);
  float* lnf = (float*)take(4 * C * 4);
  float *dgo = lnp, *dbo = lnp + C, *dgi = lnp + 2 * C, *dbi = lnp + 3 * C;
  float* w5p = (float*)take((int64_t)splits * 5 * C * C * 4);
  float* wzp = (float*)take((int64_t)splits * C * C * 4);
  // Pad columns of K-contiguous GEMM operands must read as zero.
  if (g.Np != g.N && (rc = zero_fill(dx, plane_bytes, s, fn))) return rc;
  if (Rp != R) {
    if ((rc = zero_fill(dy_t, (int64_t)((char*)dgl - (char*)dy_t), s, fn))) return rc;
  }
  dim3 grid((unsigned)((g.NN + 31) / 32), (unsigned)B);
  TM_DISPATCH(C, tm_out_bwd_kernel, grid, (const __bf16*)grad_out, (const __bf16*)x,
              (const __bf16*)xln, (const __bf16*)zln, mean_out, rstd_out, (const __bf16*)p_out,
              (const __bf16*)g_out, (const __bf16*)p_out_t, ln_out_w, dy_t, xln_t, dgl, dx, dgo,
              dbo, g, Rp);
  if ((rc = check_launch("tpf_trimul_backward_bf16(out)"))) return rc;
  // Contraction backward: dA_c = dX_c B_c, dB_c = dX_c^T A_c (stored layouts).
  GemmArgs ga{};
  ga.A = dx; ga.a_ld = g.Np; ga.a_bs = g.PS;
  ga.B = (const __bf16*)b; ga.b_ld = g.Np; ga.b_bs = g.PS;
  ga.C = da; ga.c_ld = g.Np; ga.c_bs = g.PS;
  ga.M = (int)N; ga.N = (int)N; ga.K = g.Np; ga.ksplit = 1; ga.k_chunk = g.Np; ga.alpha = 1.f;
  if ((rc = gemm_launch(ga, 1, 0, 0, (int)(B * C), s, "tpf_trimul_backward_bf16(dA)"))) return rc;
  GemmArgs gb{};
  gb.A = dx; gb.a_ld = g.Np; gb.a_bs = g.PS;
  gb.B = (const __bf16*)a; gb.b_ld = g.Np; gb.b_bs = g.PS;
  gb.C = db; gb.c_ld = g.Np; gb.c_bs = g.PS;
  gb.M = (int)N; gb.N = (int)N; gb.K = (int)N; gb.ksplit = 1; gb.k_chunk = (int)N; gb.alpha = 1.f;
  if ((rc = gemm_launch(gb, 0, 0, 0, (int)(B * C), s, "tpf_trimul_backward_bf16(dB)"))) return rc;
  TM_DISPATCH(C, tm_in_bwd_kernel, grid, (const __bf16*)z, (const __bf16*)zln, mask,
              (const __bf16*)p_in, (const __bf16*)g_in, da, db, dgl, (const __bf16*)w5_t,
              mean_in, rstd_in, ln_in_w, dproj5_t, zln_t, (__bf16*)dz, dgi, dbi, g, Rp);
  if ((rc = check_launch("tpf_trimul_backward_bf16(in)"))) return rc;
  // Weight gradients over all rows: K-contiguous split-K GEMMs + fixed-order fold.
  const int k_chunk = (int)((Rp + splits - 1) / splits);
  GemmArgs gw{};
  gw.A = dproj5_t; gw.a_ld = Rp; gw.a_bs = 0;
  gw.B = zln_t; gw.b_ld = Rp; gw.b_bs = 0;
  gw.C = w5p; gw.c_ld = C; gw.c_bs = 0; gw.c_split = 5 * C * C;
  gw.M = (int)(5 * H); gw.N = (int)C; gw.K = (int)Rp; gw.ksplit = splits; gw.k_chunk = k_chunk;
  gw.alpha = 1.f;
  if ((rc = gemm_launch(gw, 1, 1, 1, 1, s, "tpf_trimul_backward_bf16(dW5)"))) return rc;
  GemmArgs gz = gw;
  gz.A = dy_t;
  gz.B = xln_t;
  gz.C = wzp; gz.c_ld = H; gz.c_split = C * H;
  gz.M = (int)C; gz.N = (int)H;
  if ((rc = gemm_launch(gz, 1, 1, 1, 1, s, "tpf_trimul_backward_bf16(dWz)"))) return rc;
  if ((rc = fold_launch(w5p, d_w5, 5 * C * C, 5 * C * C, splits, s, fn))) return rc;
  if ((rc = fold_launch(wzp, d_p_out, C * H, C * H, splits, s, fn))) return rc;
  if ((rc = fold_launch(lnp, lnf, 4 * C, 4 * C, (int)blocks, s, fn))) return rc;
  float* outs[4] = {d_ln_out_w, d_ln_out_b, d_ln_in_w, d_ln_in_b};
  for (int i = 0; i < 4; ++i)
    if (hipMemcpyAsync(outs[i], lnf + i * C, C * 4, hipMemcpyDeviceToDevice, s) != hipSuccess)
      return set_error(TPF_ERR_LAUNCH, "%s: copy of LN parameter gradients failed", fn);
  return TPF_OK;
}

}  // extern "C"
