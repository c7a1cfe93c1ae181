// Internal interface of the batched MFMA GEMM (csrc/gemm.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.hpp"

namespace tpf {

struct GemmArgs {
  const __bf16* A; int64_t a_bs, a_ld;   // batch stride, leading dimension
  const __bf16* B; int64_t b_bs, b_ld;
  void* C; int64_t c_bs, c_ld, c_split;  // c_split: element offset between K splits
  int M, N, K;
  int ksplit, k_chunk;                   // K range of split s: [s*k_chunk, (s+1)*k_chunk)
  float alpha;
  int a_gather_n;                        // KC row gather of A (0 = none), see gemm_core.hpp
  FastDiv a_div_n, a_div_nn;             // set by gemm_launch when a_gather_n > 0
  int batch;                             // set by gemm_launch
  int b_kmax;                            // MN B: k rows that exist (0 = all K)
};

// FP32 variant (gemm_core_f32.hpp); bias (nullable) is added per column n.
struct GemmArgsF32 {
  const float* A; int64_t a_bs, a_ld;
  const float* B; int64_t b_bs, b_ld;
  float* C; int64_t c_bs, c_ld;
  int M, N, K;
  float alpha;
  const float* bias;
  int a_gather_n;
  FastDiv a_div_n, a_div_nn;
  int batch;
};

// a_kc / b_kc: operand is K-contiguous (1) or MN-contiguous (0).  tm: square
// tile size, 128 or 192 (192 instantiated for the TriMul contraction layouts:
// bf16 out, (1, 1) alone and the (1, 0) + (0, 0) pair).
int gemm_launch(const GemmArgs& g, int a_kc, int b_kc, int out_f32, int batch,
                hipStream_t stream, const char* fn, int tm = 128);
// Two GEMMs in one launch (g.batch of each, 0 meaning 1), each with its own
// operand layout; instantiated for the layout pairs TriMul uses.
int gemm_launch_pair(const GemmArgs& g0, int a_kc0, int b_kc0, const GemmArgs& g1, int a_kc1,
                     int b_kc1, int out_f32, hipStream_t stream, const char* fn, int tm = 128);
// Split-K weight-gradient products (both operands MN-contiguous, f32 output):
// one problem, or two in one launch (gemm_wgrad.hip).
int gemm_launch_wgrad(const GemmArgs& g, hipStream_t stream, const char* fn);
int gemm_launch_pair_wgrad(const GemmArgs& g0, const GemmArgs& g1, hipStream_t stream,
                           const char* fn);
int gemm_f32_launch(const GemmArgsF32& g, int a_kc, int b_kc, int batch, hipStream_t stream,
                    const char* fn);
int fold_launch(const float* part, float* out, int64_t n, int64_t stride, int splits,
                hipStream_t stream, const char* fn);

// Up to kFoldMaxSegs independent fixed-order folds in one launch (fold_launch
// is the one-segment case).  Segment sg folds `splits` partial vectors of n
// floats spaced `stride` apart into dst[sg][i / piece][i % piece]; the
// partials are left unchanged.
constexpr int kFoldMaxSegs = 5;
struct FoldSegs {
  const float* part[kFoldMaxSegs];
  float* dst[kFoldMaxSegs][4];
  int64_t n[kFoldMaxSegs], stride[kFoldMaxSegs], piece[kFoldMaxSegs];
  int splits[kFoldMaxSegs], gbase[kFoldMaxSegs];
  int ranges[kFoldMaxSegs];  // set by fold_multi
  int vec[kFoldMaxSegs];     // set by fold_multi: 4 elements per thread
  int nseg;
};
int fold_multi(FoldSegs f, hipStream_t stream, const char* fn);
// y[R, N] = x[R, K] W^T on the weight-stationary row kernel (rowgemm.hip)
// when the shape has an instance; false (nothing launched) otherwise.  W is
// [N, K] (w_kc = 1) or [K, N] (w_kc = 0) with leading dimension ldw.
bool rowgemm_try(const __bf16* x, int64_t ldx, const __bf16* w, int w_kc, int64_t ldw, __bf16* y,
                 int64_t ldy, int64_t R, int64_t N, int64_t K, hipStream_t stream, int* rc,
                 const char* fn);

// Fused d_og = dout W_o with the backward of the module's output gate
// (rowgemm.hip): writes d_o, the gate gradient and delta of the pair rows.
bool rowgemm_gate_supported(int64_t C, int64_t H, int64_t D);
int rowgemm_gate_bwd(const __bf16* dout, const __bf16* w_o, int64_t C, const __bf16* o,
                     const __bf16* res, const __bf16* gate, int64_t gpitch, __bf16* d_o,
                     float* delta, __bf16* dgate, int64_t dpitch, int64_t B, int64_t N, int64_t H,
                     int64_t D, int og_t, hipStream_t stream, const char* fn);

}  // namespace tpf
