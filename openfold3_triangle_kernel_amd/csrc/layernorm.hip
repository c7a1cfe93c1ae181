// LayerNorm over the channels of bf16 pair rows, with FP32 statistics.
//
// The pair stack normalises every pair row before its projections
// (openfold3/core/model/layers/triangular_attention.py:160-170 with the
// FP32-statistics LayerNorm of openfold3/core/model/primitives/normalization.py:54-78).
// A row is C contiguous bf16 channels; the rows of a [B, I, J] pair grid are
// addressed through element strides (sb, si, sj), so the transposed view the
// ending-node module normalises is read in place.  The normalised output and
// the statistics are written in logical (contiguous) row order.
//
// Layout per launch: L lanes share one row, each lane owns K chunks of 8
// channels (chunk j = k*L + lane), 256 threads hold 256/L rows.  Both kernels
// stream each row once from HBM: the forward reads 2C bytes and writes 2C
// (+8 for the statistics), the backward reads x and dy (4C) and writes dx
// (2C).  dgamma / dbeta come from per-workgroup partials over a grid whose
// size depends only on R (fixed row order inside a workgroup, fixed-order
// fold afterwards), so the parameter gradients are deterministic.

#include "common.hpp"
#include "tpf_gemm.hpp"
#include "tpf_status.hpp"

namespace tpf {

struct LnRows {
  int64_t R;
  FastDiv div_j, div_i;  // r -> (b, i, j)
  int64_t sb, si, sj;    // element strides of the strided operand
};

__device__ __forceinline__ int64_t ln_row_offset(const LnRows& g, uint32_t r) {
  const uint32_t t = fdiv(r, g.div_j);
  const uint32_t j = r - t * g.div_j.d;
  const uint32_t b = fdiv(t, g.div_i);
  const uint32_t i = t - b * g.div_i.d;
  return (int64_t)b * g.sb + (int64_t)i * g.si + (int64_t)j * g.sj;
}

// A workgroup normalises two groups of RPB rows (rows 2 * blockIdx.x * RPB
// + u * RPB + slot, u = 0, 1): both rows' loads are issued before either
// row's sums, so each thread keeps twice the bytes in flight (one row per
// thread measured 4.6 TB/s at 589,824 rows of 128 channels).
template <int L, int K>
__global__ __launch_bounds__(256) void ln_fwd_bf16_kernel(const __bf16* __restrict__ x,
                                                          const float* __restrict__ w,
                                                          const float* __restrict__ bias,
                                                          __bf16* __restrict__ y,
                                                          float* __restrict__ mean_out,
                                                          float* __restrict__ rstd_out,
                                                          LnRows g, int C, float eps) {
  constexpr int RPB = 256 / L;
  const int lane = threadIdx.x % L;
  const int n8 = C / 8;
  int64_t row[2];
  bool row_ok[2];
  const __bf16* xr[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    row[u] = ((int64_t)blockIdx.x * 2 + u) * RPB + threadIdx.x / L;
    row_ok[u] = row[u] < g.R;
    xr[u] = x + (row_ok[u] ? ln_row_offset(g, (uint32_t)row[u]) : 0);
  }
  // The affine parameters are loaded as vectors next to the rows, so every
  // load of the thread is in flight at once.
  float wv[K][8], bv[K][8];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int ch = k * L + lane;
    f32x4 w0 = {1.f, 1.f, 1.f, 1.f}, w1 = w0, b0 = {0.f, 0.f, 0.f, 0.f}, b1 = b0;
    if (ch < n8) {
      if (w) {
        w0 = *(const f32x4*)(w + ch * 8);
        w1 = *(const f32x4*)(w + ch * 8 + 4);
      }
      if (bias) {
        b0 = *(const f32x4*)(bias + ch * 8);
        b1 = *(const f32x4*)(bias + ch * 8 + 4);
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      wv[k][e] = w0[e];
      wv[k][e + 4] = w1[e];
      bv[k][e] = b0[e];
      bv[k][e + 4] = b1[e];
    }
  }
  float v[2][K][8];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int ch = k * L + lane;
      if (row_ok[u] && ch < n8) {
        const bf16x8 t = ld8(xr[u] + ch * 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[u][k][e] = bf2f(t[e]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[u][k][e] = 0.f;
      }
    }
  const float inv_c = 1.f / (float)C;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < K; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) s += v[u][k][e];
    s = lanes_sum<L>(s);
    const float mean = s * inv_c;
    float q = 0.f;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const bool ok = k * L + lane < n8;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = ok ? v[u][k][e] - mean : 0.f;
        q = fmaf(d, d, q);
      }
    }
    q = lanes_sum<L>(q);
    const float rstd = rsqrtf(q * inv_c + eps);
    if (!row_ok[u]) continue;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int ch = k * L + lane;
      if (ch >= n8) continue;
      bf16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        o[e] = f2bf(fmaf((v[u][k][e] - mean) * rstd, wv[k][e], bv[k][e]));
      st8(y + row[u] * C + ch * 8, o);
    }
    if (lane == 0) {
      mean_out[row[u]] = mean;
      rstd_out[row[u]] = rstd;
    }
  }
}

// dx = rstd * (g - mean(g) - xhat * mean(g * xhat)), g = dy * w,
// xhat = (x - mean) * rstd; dgamma += dy * xhat, dbeta += dy.  Workgroup
// `blk` of G takes row groups blk, blk + G, ... in ascending order; its RPB
// row slots are summed in slot order through LDS into part[blk][2][C].
template <int L, int K>
__global__ __launch_bounds__(256) void ln_bwd_bf16_kernel(
    const __bf16* __restrict__ dy, const __bf16* __restrict__ x, const float* __restrict__ mean_in,
    const float* __restrict__ rstd_in, const float* __restrict__ w, __bf16* __restrict__ dx,
    float* __restrict__ part, LnRows gx, LnRows gdx, int C, int want_params) {
  constexpr int RPB = 256 / L;
  extern __shared__ float red[];  // [RPB][2][C]
  const int lane = threadIdx.x % L;
  const int slot = threadIdx.x / L;
  const int n8 = C / 8;
  const int64_t groups = (gx.R + RPB - 1) / RPB;
  const float inv_c = 1.f / (float)C;
  float wv[K][8], dgam[K][8], dbet[K][8];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int ch = k * L + lane;
    f32x4 w0 = {1.f, 1.f, 1.f, 1.f}, w1 = w0;
    if (w && ch < n8) {
      w0 = *(const f32x4*)(w + ch * 8);
      w1 = *(const f32x4*)(w + ch * 8 + 4);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      wv[k][e] = w0[e];
      wv[k][e + 4] = w1[e];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      dgam[k][e] = 0.f;
      dbet[k][e] = 0.f;
    }
  }
  // Two row groups per iteration: both rows' loads are issued before either
  // row's arithmetic.  Rows are still folded into the partials in ascending
  // group order.
  for (int64_t grp = blockIdx.x; grp < groups; grp += 2 * (int64_t)gridDim.x) {
    int64_t rows[2] = {grp * RPB + slot, (grp + gridDim.x) * RPB + slot};
    bool ok_row[2];
    bf16x8 xt[2][K], dt[2][K];
    float mu[2], rs[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      ok_row[u] = (u == 0 || grp + gridDim.x < groups) && rows[u] < gx.R;
      mu[u] = 0.f;
      rs[u] = 0.f;
      if (!ok_row[u]) continue;
      const __bf16* xr = x + ln_row_offset(gx, (uint32_t)rows[u]);
      const __bf16* dyr = dy + rows[u] * C;
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int ch = k * L + lane;
        if (ch < n8) {
          xt[u][k] = ld8(xr + ch * 8);
          dt[u][k] = ld8(dyr + ch * 8);
        }
      }
      mu[u] = mean_in[rows[u]];
      rs[u] = rstd_in[rows[u]];
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      // Lanes of one row share ok_row, so the shuffles below stay within
      // fully active row groups.
      if (!ok_row[u]) continue;
      float xh[K][8], gg[K][8];
      float s1 = 0.f, s2 = 0.f;
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const bool ok = k * L + lane < n8;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = ok ? bf2f(dt[u][k][e]) : 0.f;
          xh[k][e] = ok ? (bf2f(xt[u][k][e]) - mu[u]) * rs[u] : 0.f;
          gg[k][e] = d * wv[k][e];
          s1 += gg[k][e];
          s2 = fmaf(gg[k][e], xh[k][e], s2);
          dgam[k][e] = fmaf(d, xh[k][e], dgam[k][e]);
          dbet[k][e] += d;
        }
      }
      s1 = lanes_sum<L>(s1);
      s2 = lanes_sum<L>(s2);
      const float m1 = s1 * inv_c, m2 = s2 * inv_c;
      __bf16* dxr = dx + ln_row_offset(gdx, (uint32_t)rows[u]);
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int ch = k * L + lane;
        if (ch >= n8) continue;
        bf16x8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = f2bf(rs[u] * (gg[k][e] - m1 - xh[k][e] * m2));
        st8(dxr + ch * 8, o);
      }
    }
  }
  if (!want_params) return;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int ch = k * L + lane;
    if (ch >= n8) continue;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      red[(slot * 2 + 0) * C + ch * 8 + e] = dgam[k][e];
      red[(slot * 2 + 1) * C + ch * 8 + e] = dbet[k][e];
    }
  }
  __syncthreads();
  for (int c = threadIdx.x; c < 2 * C; c += 256) {
    float acc = red[c];
    for (int s = 1; s < RPB; ++s) acc += red[s * 2 * C + c];
    part[(int64_t)blockIdx.x * 2 * C + c] = acc;
  }
}

namespace {

constexpr int kLnMaxC = 2048;

struct LnShape {
  int L, K;
};

LnShape ln_shape(int C) {
  const int n8 = C / 8;
  if (n8 > 64) return {64, (n8 + 63) / 64};
  int L = 1;
  while (L < n8) L <<= 1;
  return {L, 1};
}

int ln_bwd_grid(int64_t R, int L) {
  const int64_t groups = (R + 256 / L - 1) / (256 / L);
  return (int)(groups < 2048 ? groups : 2048);
}

int ln_rows(int64_t B, int64_t I, int64_t J, int64_t sb, int64_t si, int64_t sj, LnRows* g,
            const char* fn) {
  if (B < 1 || I < 1 || J < 1) return set_error(TPF_ERR_SHAPE, "%s: empty row grid", fn);
  const int64_t R = B * I * J;
  if (R > INT32_MAX || I > INT32_MAX || J > INT32_MAX)
    return set_error(TPF_ERR_SHAPE, "%s: more than 2^31 rows", fn);
  if ((sb | si | sj) % 8 != 0 || sb < 0 || si < 0 || sj < 0)
    return set_error(TPF_ERR_ARG, "%s: row strides must be non-negative multiples of 8", fn);
  g->R = R;
  g->div_j = make_fastdiv((uint32_t)J);
  g->div_i = make_fastdiv((uint32_t)I);
  g->sb = sb;
  g->si = si;
  g->sj = sj;
  return TPF_OK;
}

int ln_check_c(int64_t C, const char* fn) {
  if (C < 8 || C > kLnMaxC || C % 8 != 0)
    return set_error(TPF_ERR_SHAPE, "%s: C must be a multiple of 8 in [8, %d]", fn, kLnMaxC);
  return TPF_OK;
}

}  // namespace

#define TPF_LN_DISPATCH(KERNEL, GRID, SMEM, ...)                                                \
  do {                                                                                          \
    const LnShape sh = ln_shape((int)C);                                                        \
    switch (sh.L * 8 + sh.K) {                                                                  \
      case 1 * 8 + 1: hipLaunchKernelGGL((KERNEL<1, 1>), GRID(1), dim3(256), SMEM(1), s, __VA_ARGS__); break;    \
      case 2 * 8 + 1: hipLaunchKernelGGL((KERNEL<2, 1>), GRID(2), dim3(256), SMEM(2), s, __VA_ARGS__); break;    \
      case 4 * 8 + 1: hipLaunchKernelGGL((KERNEL<4, 1>), GRID(4), dim3(256), SMEM(4), s, __VA_ARGS__); break;    \
      case 8 * 8 + 1: hipLaunchKernelGGL((KERNEL<8, 1>), GRID(8), dim3(256), SMEM(8), s, __VA_ARGS__); break;    \
      case 16 * 8 + 1: hipLaunchKernelGGL((KERNEL<16, 1>), GRID(16), dim3(256), SMEM(16), s, __VA_ARGS__); break; \
      case 32 * 8 + 1: hipLaunchKernelGGL((KERNEL<32, 1>), GRID(32), dim3(256), SMEM(32), s, __VA_ARGS__); break; \
      case 64 * 8 + 1: hipLaunchKernelGGL((KERNEL<64, 1>), GRID(64), dim3(256), SMEM(64), s, __VA_ARGS__); break; \
      case 64 * 8 + 2: hipLaunchKernelGGL((KERNEL<64, 2>), GRID(64), dim3(256), SMEM(64), s, __VA_ARGS__); break; \
      case 64 * 8 + 3: hipLaunchKernelGGL((KERNEL<64, 3>), GRID(64), dim3(256), SMEM(64), s, __VA_ARGS__); break; \
      case 64 * 8 + 4: hipLaunchKernelGGL((KERNEL<64, 4>), GRID(64), dim3(256), SMEM(64), s, __VA_ARGS__); break; \
      default: return set_error(TPF_ERR_SHAPE, "%s: unsupported C=%lld", fn, (long long)C);    \
    }                                                                                           \
  } while (0)

}  // namespace tpf

using namespace tpf;

extern "C" int tpf_layer_norm_forward_bf16(const void* x, int64_t B, int64_t I, int64_t J,
                                           int64_t sb, int64_t si, int64_t sj, int64_t C,
                                           const float* w, const float* b, double eps, void* y,
                                           float* mean, float* rstd, void* stream) {
  const char* fn = "tpf_layer_norm_forward_bf16";
  if (!x || !y || !mean || !rstd) return set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  int rc = ln_check_c(C, fn);
  if (rc) return rc;
  LnRows g{};
  if ((rc = ln_rows(B, I, J, sb, si, sj, &g, fn))) return rc;
  if (!(eps > 0.0)) return set_error(TPF_ERR_ARG, "%s: eps must be positive", fn);
  if (((uintptr_t)x | (uintptr_t)y | (uintptr_t)w | (uintptr_t)b) % 16 != 0)
    return set_error(TPF_ERR_ARG, "%s: x, y, w and b must be 16-byte aligned", fn);
  hipStream_t s = (hipStream_t)stream;
#define TPF_LN_FGRID(L) dim3((unsigned)((g.R + 512 / (L) - 1) / (512 / (L))))
#define TPF_LN_NOSMEM(L) 0
  TPF_LN_DISPATCH(ln_fwd_bf16_kernel, TPF_LN_FGRID, TPF_LN_NOSMEM, (const __bf16*)x, w, b,
                  (__bf16*)y, mean, rstd, g, (int)C, (float)eps);
#undef TPF_LN_FGRID
  return check_launch(fn);
}

extern "C" int64_t tpf_layer_norm_backward_workspace_bytes(int64_t R, int64_t C) {
  if (R < 1 || C < 8 || C > tpf::kLnMaxC || C % 8) return -1;
  const LnShape sh = ln_shape((int)C);
  return ((int64_t)ln_bwd_grid(R, sh.L) * 2 * C * 4 + 255) / 256 * 256;
}

extern "C" int tpf_layer_norm_backward_bf16(const void* dy, const void* x, int64_t B, int64_t I,
                                            int64_t J, int64_t sb, int64_t si, int64_t sj,
                                            int64_t dsb, int64_t dsi, int64_t dsj, int64_t C,
                                            const float* mean, const float* rstd, const float* w,
                                            void* dx, float* dw, float* db, void* workspace,
                                            int64_t workspace_bytes, void* stream) {
  const char* fn = "tpf_layer_norm_backward_bf16";
  if (!dy || !x || !mean || !rstd || !dx) return set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  if ((dw == nullptr) != (db == nullptr))
    return set_error(TPF_ERR_ARG, "%s: dw and db are both given or both null", fn);
  int rc = ln_check_c(C, fn);
  if (rc) return rc;
  LnRows gx{}, gdx{};
  if ((rc = ln_rows(B, I, J, sb, si, sj, &gx, fn))) return rc;
  if ((rc = ln_rows(B, I, J, dsb, dsi, dsj, &gdx, fn))) return rc;
  if (((uintptr_t)x | (uintptr_t)dy | (uintptr_t)dx | (uintptr_t)w) % 16 != 0)
    return set_error(TPF_ERR_ARG, "%s: x, dy, dx and w must be 16-byte aligned", fn);
  const int want = dw != nullptr;
  const int64_t need = tpf_layer_norm_backward_workspace_bytes(gx.R, C);
  if (want && (!workspace || workspace_bytes < need))
    return set_error(TPF_ERR_ARG, "%s: workspace needs %lld bytes", fn, (long long)need);
  float* part = (float*)workspace;
  hipStream_t s = (hipStream_t)stream;
  const int grid = ln_bwd_grid(gx.R, ln_shape((int)C).L);
#define TPF_LN_BGRID(L) dim3((unsigned)grid)
#define TPF_LN_BSMEM(L) (want ? (size_t)(256 / (L)) * 2 * C * 4 : 0)
  TPF_LN_DISPATCH(ln_bwd_bf16_kernel, TPF_LN_BGRID, TPF_LN_BSMEM, (const __bf16*)dy,
                  (const __bf16*)x, mean, rstd, w, (__bf16*)dx, part, gx, gdx, (int)C, want);
#undef TPF_LN_BGRID
#undef TPF_LN_BSMEM
  if ((rc = check_launch(fn))) return rc;
  if (!want) return TPF_OK;
  if ((rc = fold_launch(part, dw, C, 2 * C, grid, s, fn))) return rc;
  return fold_launch(part + C, db, C, 2 * C, grid, s, fn);
}
