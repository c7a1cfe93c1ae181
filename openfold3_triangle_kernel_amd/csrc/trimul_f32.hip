// FP32 triangle multiplicative update, inference only (gfx950 FP32 MFMA).
//
// The contract of the reference's pure-FP32 TriMul
// (openfold3/core/kernels/turbopairformer/turbopairformer_trimul_fp32.py:155-400):
//   zln = LN_in(z) (optional affine, eps);  p_* / g_* = zln W^T (+ bias);
//   a = mask sigmoid(a_g) a_p, b = mask sigmoid(b_g) b_p;
//   x_c = A_c B_c^T (outgoing: A_c[i][k] = a[i,k,c]; incoming: a[k,i,c]);
//   out = (LN_out(x) W_z^T (+ b_z)) * sigmoid(zln W_g^T (+ b_g)).
// All storage and arithmetic in FP32 (v_mfma_f32_32x32x2_f32).
//
// Layouts (R = B*N*N rows, C4 / H4 = C / H rounded up to 4, zero padded):
//   zln, gate [R][C4]; xln [R][H4]; a, b, x channel-major [B*H][N][Np]
//   (Np = N rounded up to 4, pad columns zero); out [R][C] (exact C).
// Kernels: tm32_ln_rows (LN_in) -> tm32_in_proj (GEMM + gates, a / b planes
// and the output gate) -> FP32 GEMM x -> tm32_ln_planes (LN_out) ->
// tm32_out_proj (GEMM + bias + gate).
#include "common.hpp"
#include "gemm_core.hpp"
#include "gemm_core_f32.hpp"
#include "tpf_gemm.hpp"
#include "tpf_status.hpp"

namespace tpf {

struct Tm32Geom {
  int B, N, Np, C, C4, H, H4;
  int64_t NN, PS, R;
  int outgoing;
  int ntg;    // gated 128-column weight tiles per branch (64 channels each)
  int ntgo;   // output-gate 128-column tiles
  FastDiv div_n, div_nn;
};

struct Tm32Weights {
  const float* w[6];  // ap, ag, bp, bg, g [.., C]; z [C, H]
  const float* b[6];  // optional biases (nullptr = none)
};

// Packed operands: Wp [(2*ntg + ntgo)*128][C4] with per-row bias bp, and
// Wz [C][H4] with bias bz.  Gated tile t < 2*ntg (branch t / ntg, block
// q = t % ntg): rows [p c0..c0+31 | g c0..c0+31 | p c0+32.. | g c0+32..],
// c0 = 64q, so a wave's two accumulator columns hold p and g of the same
// channels; tiles 2*ntg.. hold W_g.  Missing channels are zero rows.
__global__ __launch_bounds__(256) void tm32_pack_kernel(Tm32Weights w, float* __restrict__ wp,
                                                        float* __restrict__ bp,
                                                        float* __restrict__ wz,
                                                        float* __restrict__ bz, Tm32Geom g) {
  const int wp_rows = (2 * g.ntg + g.ntgo) * 128;
  const int64_t total = (int64_t)wp_rows * g.C4 + (int64_t)g.C * g.H4 + wp_rows + g.C;
  for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * 256) {
    int64_t i = idx;
    if (i < (int64_t)wp_rows * g.C4 + wp_rows) {
      const bool is_bias = i >= (int64_t)wp_rows * g.C4;
      const int row = is_bias ? (int)(i - (int64_t)wp_rows * g.C4) : (int)(i / g.C4);
      const int col = is_bias ? 0 : (int)(i % g.C4);
      const int t = row / 128, rr = row % 128;
      int mat = -1, c = 0;
      if (t < 2 * g.ntg) {
        const int br = t / g.ntg, q = t % g.ntg;
        c = 64 * q + 32 * (rr / 64) + (rr & 31);
        const int isg = (rr >> 5) & 1;
        if (c < g.H) mat = 2 * br + isg;  // ap, ag, bp, bg
      } else {
        c = 128 * (t - 2 * g.ntg) + rr;
        if (c < g.C) mat = 4;
      }
      float v = 0.f;
      if (mat >= 0) {
        if (is_bias) v = w.b[mat] ? w.b[mat][c] : 0.f;
        else if (col < g.C) v = w.w[mat][(int64_t)c * g.C + col];
      }
      if (is_bias) bp[row] = v;
      else wp[(int64_t)row * g.C4 + col] = v;
    } else {
      i -= (int64_t)wp_rows * g.C4 + wp_rows;
      if (i < (int64_t)g.C * g.H4) {
        const int c = (int)(i / g.H4), h = (int)(i % g.H4);
        wz[i] = h < g.H ? w.w[5][(int64_t)c * g.H + h] : 0.f;
      } else {
        const int c = (int)(i - (int64_t)g.C * g.H4);
        bz[c] = w.b[5] ? w.b[5][c] : 0.f;
      }
    }
  }
}

// One wave per row: LN over the first C entries of a row of pitch ld_in,
// written with pitch ld_out (pad columns zero).  gamma / beta nullable.
__global__ __launch_bounds__(256) void tm32_ln_rows_kernel(const float* __restrict__ x,
                                                           int64_t ld_in, int C,
                                                           const float* __restrict__ gamma,
                                                           const float* __restrict__ beta,
                                                           float eps, float* __restrict__ y,
                                                           int64_t ld_out, int64_t R) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= R) return;
  const float* xr = x + row * ld_in;
  float s = 0.f;
  for (int c = lane; c < C; c += 64) s += xr[c];
  s = lanes_sum<64>(s);
  const float mean = s / C;
  float v2 = 0.f;
  for (int c = lane; c < C; c += 64) {
    const float d = xr[c] - mean;
    v2 = fmaf(d, d, v2);
  }
  v2 = lanes_sum<64>(v2);
  const float rstd = 1.f / sqrtf(v2 / C + eps);
  float* yr = y + row * ld_out;
  for (int c = lane; c < ld_out; c += 64) {
    float o = 0.f;
    if (c < C) {
      o = (xr[c] - mean) * rstd;
      if (gamma) o *= gamma[c];
      if (beta) o += beta[c];
    }
    yr[c] = o;
  }
}

// LN_out over the H channels of the channel-major product: 32 positions
// (natural order) per workgroup, 8 threads per position for the statistics,
// rows of xln written channel-fastest.
__global__ __launch_bounds__(256) void tm32_ln_planes_kernel(const float* __restrict__ x,
                                                             const float* __restrict__ gamma,
                                                             const float* __restrict__ beta,
                                                             float eps, float* __restrict__ xln,
                                                             Tm32Geom g) {
  constexpr int T = 32, XP = T + 1;
  __shared__ float Xs[256 * XP];  // [channel][position], H <= 256
  __shared__ float mu_s[T], rs_s[T];
  const int tid = threadIdx.x, b = blockIdx.y;
  const int64_t p0 = (int64_t)blockIdx.x * T;
  for (int idx = tid; idx < g.H * T; idx += 256) {
    const int c = idx / T, pp = idx % T;
    const int64_t p = p0 + pp;
    float v = 0.f;
    if (p < g.NN) {
      const uint32_t i = fdiv((uint32_t)p, g.div_n);
      v = x[((int64_t)b * g.H + c) * g.PS + (int64_t)i * g.Np + ((uint32_t)p - i * (uint32_t)g.N)];
    }
    Xs[c * XP + pp] = v;
  }
  __syncthreads();
  {
    const int pp = tid >> 3, part = tid & 7;
    float s = 0.f;
    for (int c = part; c < g.H; c += 8) s += Xs[c * XP + pp];
    s = lanes_sum<8>(s);
    const float mean = s / g.H;
    float v2 = 0.f;
    for (int c = part; c < g.H; c += 8) {
      const float d = Xs[c * XP + pp] - mean;
      v2 = fmaf(d, d, v2);
    }
    v2 = lanes_sum<8>(v2);
    if (part == 0) {
      mu_s[pp] = mean;
      rs_s[pp] = 1.f / sqrtf(v2 / g.H + eps);
    }
  }
  __syncthreads();
  for (int idx = tid; idx < T * g.H4; idx += 256) {
    const int pp = idx / g.H4, c = idx % g.H4;
    const int64_t p = p0 + pp;
    if (p >= g.NN) continue;
    float o = 0.f;
    if (c < g.H) {
      o = (Xs[c * XP + pp] - mu_s[pp]) * rs_s[pp];
      if (gamma) o *= gamma[c];
      if (beta) o += beta[c];
    }
    xln[((int64_t)b * g.NN + p) * g.H4 + c] = o;
  }
}

// Vector forms of the two LayerNorms (used when the shapes allow 16-byte
// accesses).  Rows: 16 lanes per row, 16 rows per workgroup; lane l holds
// the float4 chunks l, l + 16, ... of its row in registers (C <= 64 * NV).
template <int NV>
__global__ __launch_bounds__(256) void tm32_ln_rows_vec_kernel(const float* __restrict__ x,
                                                               int64_t ld_in, int C,
                                                               const float* __restrict__ gamma,
                                                               const float* __restrict__ beta,
                                                               float eps, float* __restrict__ y,
                                                               int64_t ld_out, int64_t R) {
  const int l = threadIdx.x & 15;
  const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const bool ok = row < R;
  const int n4 = C / 4;
  f32x4 v[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int c4 = k * 16 + l;
    v[k] = (ok && c4 < n4) ? *reinterpret_cast<const f32x4*>(x + row * ld_in + c4 * 4)
                           : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < NV; ++k) s += (v[k][0] + v[k][1]) + (v[k][2] + v[k][3]);
  s = lanes_sum<16>(s);
  const float mean = s / C;
  float v2 = 0.f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    if (k * 16 + l >= n4) continue;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float d = v[k][e] - mean;
      v2 = fmaf(d, d, v2);
    }
  }
  v2 = lanes_sum<16>(v2);
  const float rstd = 1.f / sqrtf(v2 / C + eps);
  if (!ok) return;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int c4 = k * 16 + l;
    if (c4 >= n4) continue;
    const f32x4 gm = gamma ? *reinterpret_cast<const f32x4*>(gamma + c4 * 4) : f32x4{1.f, 1.f, 1.f, 1.f};
    const f32x4 bt = beta ? *reinterpret_cast<const f32x4*>(beta + c4 * 4) : f32x4{0.f, 0.f, 0.f, 0.f};
    f32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = (v[k][e] - mean) * rstd * gm[e] + bt[e];
    *reinterpret_cast<f32x4*>(y + row * ld_out + c4 * 4) = o;
  }
}

// Planes: 64 positions per workgroup (N % 4 == 0, so 4 consecutive positions
// share one row of the plane); float4 loads along positions, LDS
// [channel][position] with pitch 65, 4 threads per position for the
// statistics, float4 stores of 4 channels.
__global__ __launch_bounds__(256) void tm32_ln_planes_vec_kernel(const float* __restrict__ x,
                                                                 const float* __restrict__ gamma,
                                                                 const float* __restrict__ beta,
                                                                 float eps, float* __restrict__ xln,
                                                                 Tm32Geom g) {
  constexpr int T = 64, XP = T + 1;
  __shared__ float Xs[256 * XP];  // [channel][position], H <= 256
  __shared__ float mu_s[T], rs_s[T];
  const int tid = threadIdx.x, b = blockIdx.y;
  const int64_t p0 = (int64_t)blockIdx.x * T;
  for (int idx = tid; idx < g.H * (T / 4); idx += 256) {
    const int c = idx / (T / 4), q4 = idx % (T / 4);
    const int64_t p = p0 + 4 * q4;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (p < g.NN) {
      const uint32_t i = fdiv((uint32_t)p, g.div_n);
      v = *reinterpret_cast<const f32x4*>(
          x + ((int64_t)b * g.H + c) * g.PS + (int64_t)i * g.Np + ((uint32_t)p - i * (uint32_t)g.N));
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) Xs[c * XP + 4 * q4 + e] = v[e];
  }
  __syncthreads();
  {
    const int pp = tid >> 2, part = tid & 3;
    float s = 0.f;
    for (int c = part; c < g.H; c += 4) s += Xs[c * XP + pp];
    s = lanes_sum<4>(s);
    const float mean = s / g.H;
    float v2 = 0.f;
    for (int c = part; c < g.H; c += 4) {
      const float d = Xs[c * XP + pp] - mean;
      v2 = fmaf(d, d, v2);
    }
    v2 = lanes_sum<4>(v2);
    if (part == 0) {
      mu_s[pp] = mean;
      rs_s[pp] = 1.f / sqrtf(v2 / g.H + eps);
    }
  }
  __syncthreads();
  const int h4n = g.H4 / 4;
  for (int idx = tid; idx < T * h4n; idx += 256) {
    const int pp = idx / h4n, c0 = 4 * (idx % h4n);
    const int64_t p = p0 + pp;
    if (p >= g.NN) continue;
    f32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = c0 + e;
      float t = 0.f;
      if (c < g.H) {
        t = (Xs[c * XP + pp] - mu_s[pp]) * rs_s[pp];
        if (gamma) t *= gamma[c];
        if (beta) t += beta[c];
      }
      o[e] = t;
    }
    *reinterpret_cast<f32x4*>(xln + ((int64_t)b * g.NN + p) * g.H4 + c0) = o;
  }
}

// Planes, register-resident: workgroup = 64 positions x all channels;
// thread = (4-position group pg = tid % 16, channel group cg = tid / 16 of
// CPT channels).  Each thread issues all of its CPT float4 loads at once and
// keeps the CPT x 4 block in registers; per-position channel sums go through
// the 4 channel groups of a wave by shuffles and the 4 waves through LDS in
// fixed order (mean first, then the centred sum of squares).  Rows of xln
// are written as float4 runs of the thread's channels (pad channels up to
// H4 as zeros).  Needs N % 4 == 0 and H <= 16 * CPT.
template <int CPT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 8))) void tm32_ln_planes_reg_kernel(
    const float* __restrict__ x, const float* __restrict__ gamma, const float* __restrict__ beta,
    float eps, float* __restrict__ xln, Tm32Geom g) {
  constexpr int T = 64;
  __shared__ float red[2][4][16][4];  // [pass][wave][position group][position]
  const int tid = threadIdx.x, wv = tid >> 6, b = blockIdx.y;
  const int pg = tid & 15, cg = tid >> 4;
  const int64_t pb = (int64_t)blockIdx.x * T + 4 * pg;  // first position of this thread
  const bool pos_ok = pb < g.NN;                       // NN % 4 == 0: all 4 or none
  const int c0 = cg * CPT;
  int64_t off = 0;
  if (pos_ok) {
    const uint32_t i = fdiv((uint32_t)pb, g.div_n);
    off = (int64_t)i * g.Np + ((uint32_t)pb - i * (uint32_t)g.N);
  }
  float v[CPT][4];
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    f32x4 t = {0.f, 0.f, 0.f, 0.f};
    if (pos_ok && c0 + c < g.H)
      t = *reinterpret_cast<const f32x4*>(x + ((int64_t)b * g.H + c0 + c) * g.PS + off);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[c][e] = t[e];
  }
  const float invH = 1.f / g.H;
  float mean[4], rstd[4];
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    float q[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float a = 0.f;
#pragma unroll
      for (int c = 0; c < CPT; ++c) {
        if (pass == 0) {
          a += v[c][e];
        } else if (c0 + c < g.H) {
          const float d = v[c][e] - mean[e];
          a = fmaf(d, d, a);
        }
      }
      a = xor32_sum(xor16_sum(a));
      q[e] = a;
    }
    if ((tid & 48) == 0) {
#pragma unroll
      for (int e = 0; e < 4; ++e) red[pass][wv][pg][e] = q[e];
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float t = ((red[pass][0][pg][e] + red[pass][1][pg][e]) + red[pass][2][pg][e]) +
                      red[pass][3][pg][e];
      if (pass == 0) mean[e] = t * invH;
      else rstd[e] = 1.f / sqrtf(t * invH + eps);
    }
  }
  if (!pos_ok || c0 >= g.H4) return;
#pragma unroll
  for (int c4 = 0; c4 < CPT / 4; ++c4) {
    if (c0 + 4 * c4 >= g.H4) continue;
    float gm[4], bt[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int c = c0 + 4 * c4 + k;
      gm[k] = c < g.H ? (gamma ? gamma[c] : 1.f) : 0.f;
      bt[k] = c < g.H ? (beta ? beta[c] : 0.f) : 0.f;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      f32x4 o;
#pragma unroll
      for (int k = 0; k < 4; ++k) o[k] = (v[4 * c4 + k][e] - mean[e]) * rstd[e] * gm[k] + bt[k];
      *reinterpret_cast<f32x4*>(xln + ((int64_t)b * g.NN + pb + e) * g.H4 + c0 + 4 * c4) = o;
    }
  }
}

// Hardware exp and reciprocal (each within a few ulp: far inside the FP32
// mode's 1e-4 bound); the IEEE division made the gating epilogue VALU-bound.
__device__ __forceinline__ float sigmoid_f32(float x) { return sigmoidf(x); }

// Input projections in stored row order m (natural row = gather of m for
// the incoming direction).  Gated tiles write a / b planes; output-gate
// tiles write sigmoid(g) row-major.
__global__ __launch_bounds__(256, 2) void tm32_in_proj_kernel(
    const float* __restrict__ zln, const float* __restrict__ wp, const float* __restrict__ bp,
    const float* __restrict__ mask, float* __restrict__ a_pl, float* __restrict__ b_pl,
    float* __restrict__ gate, Tm32Geom g) {
  constexpr int SP = 132;  // f32 pitch of the [64 channel][128 position] staging tile
  __shared__ __attribute__((aligned(1024))) char smem[kFMainLdsBytes];
  __shared__ float mask_s[128];
  __shared__ int64_t rho_s[128];
  const int tn = 2 * g.ntg + g.ntgo;
  const int64_t tm = (g.R + 127) / 128;
  const int64_t T = xcd_order(tm * tn);
  if (T < 0) return;
  const int nt = (int)(T % tn);
  const int64_t m0 = (T / tn) * 128;
  if (threadIdx.x < 128) {
    const int64_t m = m0 + threadIdx.x;
    int64_t rho = -1;
    if (m < g.R) {
      rho = m;
      if (!g.outgoing) {
        const uint32_t bb = fdiv((uint32_t)m, g.div_nn), p = (uint32_t)m - bb * (uint32_t)g.NN;
        const uint32_t i = fdiv(p, g.div_n), k = p - i * (uint32_t)g.N;
        rho = (int64_t)bb * g.NN + (int64_t)k * g.N + i;
      }
    }
    rho_s[threadIdx.x] = rho;
    mask_s[threadIdx.x] = rho >= 0 ? mask[rho] : 0.f;
  }
  GemmOperandF32 A{zln, g.C4, (int)g.R, g.outgoing ? 0 : g.N, g.div_n, g.div_nn};
  GemmOperandF32 W{wp, g.C4, tn * 128, 0, {}, {}};
  f32x16 acc[2][2];
  gemm_tile_f32<true, true>(A, W, (int)m0, nt * 128, 0, g.C4, smem, acc);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int rl = lane & 31, hl = lane >> 5, wm = w >> 1, wn = w & 1;
  if (nt >= 2 * g.ntg) {  // output gate: sigmoid(zln W_g^T + b_g), row-major [R][C4]
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = nt * 128 + 64 * wn + 32 * j + rl;
      const int c = col - 2 * g.ntg * 128;
      if (c >= g.C) continue;
      const float bias = bp[col];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = 64 * wm + 32 * i + 8 * (r >> 2) + 4 * hl + (r & 3);
          const int64_t rho = rho_s[row];
          if (rho >= 0) gate[rho * g.C4 + c] = sigmoid_f32(acc[i][j][r] + bias);
        }
    }
    return;
  }
  const int br = nt / g.ntg, q = nt % g.ntg;
  const int cl = 32 * wn + rl;  // channel 64q + cl
  const float biasp = bp[nt * 128 + 64 * wn + rl], biasg = bp[nt * 128 + 64 * wn + 32 + rl];
  float* S = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = 64 * wm + 32 * i + 8 * (r >> 2) + 4 * hl + (r & 3);
      S[cl * SP + row] = mask_s[row] * sigmoid_f32(acc[i][1][r] + biasg) * (acc[i][0][r] + biasp);
    }
  __syncthreads();
  float* planes = br ? b_pl : a_pl;
  for (int idx = threadIdx.x; idx < 64 * 32; idx += 256) {
    const int c_l = idx >> 5, chn = idx & 31;
    const int c = 64 * q + c_l;
    if (c >= g.H) continue;
    const int64_t mb = m0 + 4 * chn;
    const float* s = S + c_l * SP + 4 * chn;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t m = mb + e;
      if (m >= g.R) break;
      const uint32_t bb = fdiv((uint32_t)m, g.div_nn), p = (uint32_t)m - bb * (uint32_t)g.NN;
      const uint32_t i = fdiv(p, g.div_n);
      planes[((int64_t)bb * g.H + c) * g.PS + (int64_t)i * g.Np + (p - i * (uint32_t)g.N)] = s[e];
    }
  }
}

// out[rho][c] = (xln W_z^T + b_z)[rho][c] * gate[rho][c], natural rows.
__global__ __launch_bounds__(256, 2) void tm32_out_proj_kernel(
    const float* __restrict__ xln, const float* __restrict__ wz, const float* __restrict__ bz,
    const float* __restrict__ gate, float* __restrict__ out, Tm32Geom g) {
  __shared__ __attribute__((aligned(1024))) char smem[kFMainLdsBytes];
  const int tn = (g.C + 127) / 128;
  const int64_t T = xcd_order(((g.R + 127) / 128) * tn);
  if (T < 0) return;
  const int nt = (int)(T % tn);
  const int64_t m0 = (T / tn) * 128;
  GemmOperandF32 A{xln, g.H4, (int)g.R, 0, {}, {}};
  GemmOperandF32 W{wz, g.H4, g.C, 0, {}, {}};
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int rl = lane & 31, hl = lane >> 5, wm = w >> 1, wn = w & 1;
  // The gate values of this lane's accumulator elements are loaded before
  // the main loop, so their latency overlaps it.
  float gv[2][2][16];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int c = nt * 128 + 64 * wn + 32 * j + rl;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t rho = m0 + 64 * wm + 32 * i + 8 * (r >> 2) + 4 * hl + (r & 3);
        gv[j][i][r] = (c < g.C && rho < g.R) ? gate[rho * g.C4 + c] : 0.f;
      }
  }
  f32x16 acc[2][2];
  gemm_tile_f32<true, true>(A, W, (int)m0, nt * 128, 0, g.H4, smem, acc);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int c = nt * 128 + 64 * wn + 32 * j + rl;
    if (c >= g.C) continue;
    const float bias = bz[c];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t rho = m0 + 64 * wm + 32 * i + 8 * (r >> 2) + 4 * hl + (r & 3);
        if (rho < g.R) out[rho * g.C + c] = (acc[i][j][r] + bias) * gv[j][i][r];
      }
  }
}

__global__ __launch_bounds__(256) void tm32_zero_kernel(float* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    p[i] = 0.f;
}

}  // namespace tpf

using namespace tpf;

static int64_t a256f(int64_t v) { return (v + 255) / 256 * 256; }

static int tm32_geom(Tm32Geom* g, int64_t B, int64_t N, int64_t C, int64_t H, int outgoing,
                     const char* fn) {
  if (B < 1 || N < 1 || C < 1 || H < 1)
    return set_error(TPF_ERR_SHAPE, "%s: B, N, C and H must be positive", fn);
  if (C > 512 || H > 256)
    return set_error(TPF_ERR_SHAPE, "%s: C=%lld (max 512) or H=%lld (max 256) too large", fn,
                     (long long)C, (long long)H);
  const int64_t Np = (N + 3) / 4 * 4, R = B * N * N;
  const int64_t C4 = (C + 3) / 4 * 4, H4 = (H + 3) / 4 * 4;
  if (R * (C4 > H4 ? C4 : H4) * 4 >= (int64_t)kBufOOB || B * H * N * Np * 4 >= (int64_t)kBufOOB ||
      R > INT32_MAX / 2)
    return set_error(TPF_ERR_SHAPE, "%s: B=%lld N=%lld too large", fn, (long long)B, (long long)N);
  g->B = (int)B; g->N = (int)N; g->Np = (int)Np; g->C = (int)C; g->C4 = (int)C4;
  g->H = (int)H; g->H4 = (int)H4; g->NN = N * N; g->PS = N * Np; g->R = R;
  g->outgoing = outgoing ? 1 : 0;
  g->ntg = (int)((H + 63) / 64);
  g->ntgo = (int)((C + 127) / 128);
  g->div_n = make_fastdiv((uint32_t)N);
  g->div_nn = make_fastdiv((uint32_t)(N * N));
  return TPF_OK;
}

struct Tm32Work {
  float *wp, *bp, *wz, *bz, *zln, *gate, *a, *b, *x, *xln;
};

// Workspace: packed weights, zln and gate logits [R, C4], the a and b
// planes [B, H, N, Np], and the product and its LayerNorm for one chunk of
// output rows: x [H, rows, Np], xln [rows * N, H4] (rows = row_chunk).
static int64_t tm32_layout(const Tm32Geom& g, int64_t row_chunk, char* base, Tm32Work* w) {
  const int64_t wp_rows = (int64_t)(2 * g.ntg + g.ntgo) * 128;
  const int64_t planes = (int64_t)g.B * g.H * g.PS;
  int64_t off = 0;
  auto take = [&](int64_t bytes) { char* p = base ? base + off : nullptr; off += a256f(bytes); return (float*)p; };
  Tm32Work t;
  t.wp = take(wp_rows * g.C4 * 4);
  t.bp = take(wp_rows * 4);
  t.wz = take((int64_t)g.C * g.H4 * 4);
  t.bz = take((int64_t)g.C * 4);
  t.zln = take(g.R * g.C4 * 4);
  t.gate = take(g.R * g.C4 * 4);
  t.a = take(planes * 4);
  t.b = take(planes * 4);
  t.x = take((int64_t)g.H * row_chunk * g.Np * 4);
  t.xln = take(row_chunk * g.N * g.H4 * 4);
  if (w) *w = t;
  return off;
}

extern "C" {

int64_t tpf_trimul_forward_f32_workspace_bytes_chunked(int64_t B, int64_t N, int64_t C, int64_t H,
                                                       int64_t row_chunk) {
  Tm32Geom g;
  if (tm32_geom(&g, B, N, C, H, 1, "tpf_trimul_forward_f32_workspace_bytes")) return -1;
  if (row_chunk < 1) return -1;
  return tm32_layout(g, row_chunk < N ? row_chunk : N, nullptr, nullptr);
}

int64_t tpf_trimul_forward_f32_workspace_bytes(int64_t B, int64_t N, int64_t C, int64_t H) {
  return tpf_trimul_forward_f32_workspace_bytes_chunked(B, N, C, H, N);
}

int tpf_trimul_forward_f32_chunked(const float* z, const float* mask, const float* w_ap, const float* w_ag,
                           const float* w_bp, const float* w_bg, const float* w_g,
                           const float* w_z, const float* b_ap, const float* b_ag,
                           const float* b_bp, const float* b_bg, const float* b_g,
                           const float* b_z, const float* ln_in_w, const float* ln_in_b,
                           double ln_in_eps, const float* ln_out_w, const float* ln_out_b,
                           double ln_out_eps, int outgoing, int64_t B, int64_t N, int64_t C,
                           int64_t H, int64_t row_chunk, float* out, void* workspace,
                           int64_t workspace_bytes, void* stream) {
  const char* fn = "tpf_trimul_forward_f32";
  Tm32Geom g;
  int rc = tm32_geom(&g, B, N, C, H, outgoing, fn);
  if (rc) return rc;
  if (row_chunk < 1) return set_error(TPF_ERR_ARG, "%s: row_chunk must be positive", fn);
  if (row_chunk > N) row_chunk = N;
  if (!z || !mask || !w_ap || !w_ag || !w_bp || !w_bg || !w_g || !w_z || !out || !workspace)
    return set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  if (!(ln_in_eps > 0) || !(ln_out_eps > 0))
    return set_error(TPF_ERR_ARG, "%s: LayerNorm eps must be positive", fn);
  const int64_t need = tm32_layout(g, row_chunk, nullptr, nullptr);
  if (workspace_bytes < need)
    return set_error(TPF_ERR_ARG, "%s: workspace %lld < required %lld", fn,
                     (long long)workspace_bytes, (long long)need);
  hipStream_t s = (hipStream_t)stream;
  Tm32Work wk;
  tm32_layout(g, row_chunk, (char*)workspace, &wk);
  Tm32Weights w{{w_ap, w_ag, w_bp, w_bg, w_g, w_z}, {b_ap, b_ag, b_bp, b_bg, b_g, b_z}};
  hipLaunchKernelGGL(tm32_pack_kernel, dim3(1024), dim3(256), 0, s, w, wk.wp, wk.bp, wk.wz, wk.bz, g);
  if ((rc = check_launch(fn))) return rc;
  if (g.Np != g.N) {  // contraction reads whole rows of Np: pad columns must be zero
    // a and b are adjacent regions ending where x begins.
    hipLaunchKernelGGL(tm32_zero_kernel, dim3(8192), dim3(256), 0, s, wk.a, (int64_t)(wk.x - wk.a));
    if ((rc = check_launch(fn))) return rc;
  }
  const bool rows_vec = C % 4 == 0 && ((uintptr_t)z | (uintptr_t)ln_in_w | (uintptr_t)ln_in_b) % 16 == 0;
  const int nv = (int)((C / 4 + 15) / 16);  // float4 chunks per lane (C <= 512: <= 8)
  if (rows_vec) {
    const dim3 grid((unsigned)((g.R + 15) / 16));
#define TM32_LN_ROWS(NV)                                                                       \
  hipLaunchKernelGGL(tm32_ln_rows_vec_kernel<NV>, grid, dim3(256), 0, s, z, (int64_t)C, (int)C,  \
                     ln_in_w, ln_in_b, (float)ln_in_eps, wk.zln, (int64_t)g.C4, g.R)
    if (nv <= 1) TM32_LN_ROWS(1);
    else if (nv <= 2) TM32_LN_ROWS(2);
    else if (nv <= 4) TM32_LN_ROWS(4);
    else TM32_LN_ROWS(8);
#undef TM32_LN_ROWS
  } else {
    hipLaunchKernelGGL(tm32_ln_rows_kernel, dim3((unsigned)((g.R + 3) / 4)), dim3(256), 0, s, z,
                       (int64_t)C, (int)C, ln_in_w, ln_in_b, (float)ln_in_eps, wk.zln,
                       (int64_t)g.C4, g.R);
  }
  if ((rc = check_launch(fn))) return rc;
  const int64_t tiles = (g.R + 127) / 128;
  const int64_t ptiles = tiles * (2 * g.ntg + g.ntgo);
  hipLaunchKernelGGL(tm32_in_proj_kernel, dim3((unsigned)((ptiles + 7) / 8 * 8)), dim3(256), 0, s,
                     wk.zln, wk.wp, wk.bp, mask, wk.a, wk.b, wk.gate, g);
  if ((rc = check_launch(fn))) return rc;
  // Contraction, LN_out and the output projection over chunks of output
  // rows i (every element keeps its full K = N reduction and its own
  // LayerNorm and projection: the results do not depend on the chunking).
  for (int64_t bb = 0; bb < B; ++bb) {
    for (int64_t i0 = 0; i0 < N; i0 += row_chunk) {
      const int64_t rows = N - i0 < row_chunk ? N - i0 : row_chunk;
      GemmArgsF32 ga{};
      ga.A = wk.a + bb * g.H * g.PS + i0 * g.Np; ga.a_ld = g.Np; ga.a_bs = g.PS;
      ga.B = wk.b + bb * g.H * g.PS; ga.b_ld = g.Np; ga.b_bs = g.PS;
      ga.C = wk.x; ga.c_ld = g.Np; ga.c_bs = rows * g.Np;
      ga.M = (int)rows; ga.N = g.N; ga.K = g.Np; ga.alpha = 1.f; ga.bias = nullptr;
      if ((rc = gemm_f32_launch(ga, 1, 1, (int)H, s, "tpf_trimul_forward_f32(contract)"))) return rc;
      // The chunk as a one-batch problem of rows * N positions.
      Tm32Geom gc = g;
      gc.B = 1; gc.NN = rows * N; gc.PS = rows * g.Np; gc.R = rows * N;
      const int64_t r0 = bb * g.NN + i0 * N;  // first pair row of the chunk
      if (N % 4 == 0 && g.Np % 4 == 0 && H <= 128)
        hipLaunchKernelGGL(tm32_ln_planes_reg_kernel<8>, dim3((unsigned)((gc.NN + 63) / 64), 1u),
                           dim3(256), 0, s, wk.x, ln_out_w, ln_out_b, (float)ln_out_eps, wk.xln, gc);
      else if (N % 4 == 0 && g.Np % 4 == 0 && H <= 256)
        hipLaunchKernelGGL(tm32_ln_planes_reg_kernel<16>, dim3((unsigned)((gc.NN + 63) / 64), 1u),
                           dim3(256), 0, s, wk.x, ln_out_w, ln_out_b, (float)ln_out_eps, wk.xln, gc);
      else if (N % 4 == 0 && g.Np % 4 == 0)
        hipLaunchKernelGGL(tm32_ln_planes_vec_kernel, dim3((unsigned)((gc.NN + 63) / 64), 1u),
                           dim3(256), 0, s, wk.x, ln_out_w, ln_out_b, (float)ln_out_eps, wk.xln, gc);
      else
        hipLaunchKernelGGL(tm32_ln_planes_kernel, dim3((unsigned)((gc.NN + 31) / 32), 1u),
                           dim3(256), 0, s, wk.x, ln_out_w, ln_out_b, (float)ln_out_eps, wk.xln, gc);
      if ((rc = check_launch(fn))) return rc;
      const int64_t otiles = (gc.R + 127) / 128 * ((C + 127) / 128);
      hipLaunchKernelGGL(tm32_out_proj_kernel, dim3((unsigned)((otiles + 7) / 8 * 8)), dim3(256), 0,
                         s, wk.xln, wk.wz, wk.bz, wk.gate + r0 * g.C4, out + r0 * C, gc);
      if ((rc = check_launch(fn))) return rc;
    }
  }
  return TPF_OK;
}

int tpf_trimul_forward_f32(const float* z, const float* mask, const float* w_ap, const float* w_ag,
                           const float* w_bp, const float* w_bg, const float* w_g,
                           const float* w_z, const float* b_ap, const float* b_ag,
                           const float* b_bp, const float* b_bg, const float* b_g,
                           const float* b_z, const float* ln_in_w, const float* ln_in_b,
                           double ln_in_eps, const float* ln_out_w, const float* ln_out_b,
                           double ln_out_eps, int outgoing, int64_t B, int64_t N, int64_t C,
                           int64_t H, float* out, void* workspace, int64_t workspace_bytes,
                           void* stream) {
  return tpf_trimul_forward_f32_chunked(z, mask, w_ap, w_ag, w_bp, w_bg, w_g, w_z, b_ap, b_ag,
                                        b_bp, b_bg, b_g, b_z, ln_in_w, ln_in_b, ln_in_eps, ln_out_w,
                                        ln_out_b, ln_out_eps, outgoing, B, N, C, H, N, out,
                                        workspace, workspace_bytes, stream);
}

}  // extern "C"
