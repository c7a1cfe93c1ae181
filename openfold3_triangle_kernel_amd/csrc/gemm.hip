// Batched bf16 GEMM on gfx950 MFMA for the TriMul channel contraction, its
// backward products and the split-K weight-gradient products.
//
//   C[z][m][n] = alpha * sum_k A[z](m, k) * B[z](n, k)
//
// A and B are each given either K-contiguous ("KC": X[r * ld + k]) or
// MN-contiguous ("MN": X[k * ld + r]); the main loop (gemm_core.hpp) reads
// both layouts straight into LDS and feeds the MFMA from there.  C is
// row-major (n contiguous) in bf16 or f32.  Split-K writes f32 partials at
// C + split * c_split and a fixed-order fold kernel sums them
// (deterministic, no atomics).
// Stage shape of this translation unit (measured on the TriMul contraction
// and its dA / dB products: 32-deep k-steps, three stages in flight); the
// split-K weight-gradient products use their own shape (gemm_wgrad.hip).
#define TPF_GEMM_GK 32
#define TPF_GEMM_NS 3
#define TPF_GEMM_IMPL gk32
#include "gemm_impl.hpp"

namespace tpf {

using namespace gk32;

// Several fixed-order folds in one launch.  Segment sg owns workgroups
// [gbase[sg], gbase[sg + 1]); a workgroup covers 256 / RC consecutive
// element groups x RC ranges of splits (RC = ranges[sg], a power of two
// chosen so that a range holds at most kFoldRangeSplits splits); an element
// group is 4 consecutive elements read as one 16-byte load when the segment's sizes and
// pointers allow it (vec[sg]), else one element.  Thread (range r, group i)
// sums splits [r * per, min((r + 1) * per, splits)) in ascending order with
// up to 16 of its loads in flight, and the ranges meet in LDS in the fixed order
// ((r0 + r1) + r2) + ...; element i of the segment lands in
// dst[i / piece][i % piece].  Every element's order depends only on the
// shapes (the grouping changes no sum).
// Splits per range: 32 (two batches of 16 loads per thread) measured
// 13.8 -> 12.2 us against 16 on the TriMul weight-gradient fold at N=768
// (8 and 4: 18.3 and 26.8 us; 64: 13.9 us), 14.4 -> 12.8 us at N=384.
constexpr int kFoldRangeSplits = 32;

template <int EPT>
__device__ __forceinline__ void fold_multi_body(const FoldSegs& f, int sg) {
  typedef float VT __attribute__((ext_vector_type(EPT)));
  __shared__ VT red[256];
  const int rc = f.ranges[sg], epw = 256 / rc;
  const int r = threadIdx.x / epw, el = threadIdx.x - r * epw;
  const int64_t i = ((int64_t)((int)blockIdx.x - f.gbase[sg]) * epw + el) * EPT;
  const bool act = i < f.n[sg];
  const int splits = f.splits[sg];
  const int per = (splits + rc - 1) / rc;
  const int s0 = r * per, s1 = min(splits, s0 + per);
  const float* part = f.part[sg];
  const int64_t stride = f.stride[sg];
  VT acc = (VT)0.f;
  if (act && s0 < s1) {
    // Up to 16 loads go out together, then they are added in ascending
    // order.
    for (int s = s0; s < s1; s += 16) {
      VT v[16];
#pragma unroll
      for (int e = 0; e < 16; ++e)
        if (s + e < s1) v[e] = *reinterpret_cast<const VT*>(part + (int64_t)(s + e) * stride + i);
#pragma unroll
      for (int e = 0; e < 16; ++e)
        if (s + e < s1) acc = (s + e == s0) ? v[e] : acc + v[e];
    }
  }
  red[threadIdx.x] = acc;
  __syncthreads();
  if (r != 0 || !act) return;
  for (int q = 1; q < rc; ++q)
    if (q * per < splits) acc += red[q * epw + el];
  const int64_t pc = i / f.piece[sg];
  *reinterpret_cast<VT*>(f.dst[sg][pc] + (i - pc * f.piece[sg])) = acc;
}

__global__ __launch_bounds__(256) void fold_multi_kernel(FoldSegs f) {
  int sg = 0;
  while (sg + 1 < f.nseg && (int)blockIdx.x >= f.gbase[sg + 1]) ++sg;
  if (f.vec[sg])
    fold_multi_body<4>(f, sg);
  else
    fold_multi_body<1>(f, sg);
}

// The weight-gradient fold contract of the reference
// (trimul_wgrad_fixed_fold, turbopairformer_trimul_cuda.cu:200-217, 2050-2089):
// accumulator[e] = (((init + p[0][e]) + p[1][e]) + ...) + p[chunks-1][e] in
// round-to-nearest FP32, init = 0 (initialize) or the accumulator's value.
template <bool INIT>
__global__ __launch_bounds__(256) void wgrad_fixed_fold_kernel(const float* __restrict__ part,
                                                               int chunks, int64_t n,
                                                               float* __restrict__ acc) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  float sum = INIT ? 0.f : acc[i];
  int c = 0;
  for (; c + 8 <= chunks; c += 8) {  // 8 loads in flight, added in ascending order
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = part[(int64_t)(c + e) * n + i];
#pragma unroll
    for (int e = 0; e < 8; ++e) sum = __fadd_rn(sum, v[e]);
  }
  for (; c < chunks; ++c) sum = __fadd_rn(sum, part[(int64_t)c * n + i]);
  acc[i] = sum;
}

int fold_multi(FoldSegs f, hipStream_t stream, const char* fn) {
  if (f.nseg < 1 || f.nseg > kFoldMaxSegs) return set_error(TPF_ERR_ARG, "%s: bad fold segments", fn);
  int64_t blocks = 0;
  for (int sg = 0; sg < f.nseg; ++sg) {
    if (f.splits[sg] < 1 || f.n[sg] < 1 || f.piece[sg] < 1)
      return set_error(TPF_ERR_ARG, "%s: bad fold segment", fn);
    int rc = 1;
    while (rc < 64 && (f.splits[sg] + rc - 1) / rc > kFoldRangeSplits) rc *= 2;
    f.ranges[sg] = rc;
    bool vec = f.n[sg] % 4 == 0 && f.stride[sg] % 4 == 0 && f.piece[sg] % 4 == 0 &&
               (uintptr_t)f.part[sg] % 16 == 0;
    for (int pc = 0; pc < 4 && vec; ++pc)
      if ((int64_t)pc * f.piece[sg] < f.n[sg] && (uintptr_t)f.dst[sg][pc] % 16 != 0) vec = false;
    f.vec[sg] = vec ? 1 : 0;
    f.gbase[sg] = (int)blocks;
    const int64_t per_wg = (int64_t)(256 / rc) * (vec ? 4 : 1);
    blocks += (f.n[sg] + per_wg - 1) / per_wg;
  }
  if (blocks > 0x7fffffff) return set_error(TPF_ERR_ARG, "%s: fold grid too large", fn);
  hipLaunchKernelGGL(fold_multi_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, f);
  return check_launch(fn);
}

int gemm_launch(const GemmArgs& g0, int a_kc, int b_kc, int out_f32, int batch,
                hipStream_t stream, const char* fn, int tm) {
  GemmArgs g = g0;
  int rc = gemm_prepare(g, a_kc, b_kc, out_f32, batch, fn);
  if (rc) return rc;
  if (tm == 192) {
    if (a_kc != 1 || b_kc != 1 || out_f32)
      return set_error(TPF_ERR_ARG, "%s: 192 tiles not instantiated for this layout", fn);
    const int64_t blocks = (gemm_tiles(g, 192) + 7) / 8 * 8;
    if (blocks > INT32_MAX) return set_error(TPF_ERR_SHAPE, "%s: GEMM grid too large", fn);
    hipLaunchKernelGGL((gemm_bf16_kernel<true, true, false, 192>), dim3((unsigned)blocks),
                       dim3(256), 0, stream, g);
    return check_launch(fn);
  }
  if (tm != 128) return set_error(TPF_ERR_ARG, "%s: tile size %d", fn, tm);
  dim3 grid((unsigned)((gemm_tiles(g) + 7) / 8 * 8));
#define TPF_GEMM_CASE(AK, BK, OF)                                                            \
  if (a_kc == AK && b_kc == BK && out_f32 == OF) {                                            \
    hipLaunchKernelGGL((gemm_bf16_kernel<AK, BK, OF>), grid, dim3(256), 0, stream, g);         \
    return check_launch(fn);                                                                  \
  }
  TPF_GEMM_CASE(1, 1, 0)
  TPF_GEMM_CASE(1, 1, 1)
  TPF_GEMM_CASE(1, 0, 0)
  TPF_GEMM_CASE(1, 0, 1)
  TPF_GEMM_CASE(0, 1, 0)
  TPF_GEMM_CASE(0, 1, 1)
  TPF_GEMM_CASE(0, 0, 0)
  TPF_GEMM_CASE(0, 0, 1)
#undef TPF_GEMM_CASE
  return set_error(TPF_ERR_ARG, "%s: bad GEMM layout flags", fn);
}

int gemm_launch_pair(const GemmArgs& p0, int a_kc0, int b_kc0, const GemmArgs& p1, int a_kc1,
                     int b_kc1, int out_f32, hipStream_t stream, const char* fn, int tm) {
  GemmArgs g0 = p0, g1 = p1;
  int rc = gemm_prepare(g0, a_kc0, b_kc0, out_f32, p0.batch > 0 ? p0.batch : 1, fn);
  if (rc) return rc;
  if ((rc = gemm_prepare(g1, a_kc1, b_kc1, out_f32, p1.batch > 0 ? p1.batch : 1, fn))) return rc;
  if (tm != 128 && tm != 192) return set_error(TPF_ERR_ARG, "%s: tile size %d", fn, tm);
  const int64_t blocks = (gemm_tiles(g0, tm) + 7) / 8 * 8 + (gemm_tiles(g1, tm) + 7) / 8 * 8;
  if (blocks > INT32_MAX) return set_error(TPF_ERR_SHAPE, "%s: GEMM grid too large", fn);
  dim3 grid((unsigned)blocks);
#define TPF_GEMM_PAIR_CASE(A0, B0, A1, B1, OF, TM)                                            \
  if (a_kc0 == A0 && b_kc0 == B0 && a_kc1 == A1 && b_kc1 == B1 && out_f32 == OF && tm == TM) { \
    hipLaunchKernelGGL((gemm_bf16_pair_kernel<A0, B0, A1, B1, OF, TM>), grid, dim3(256), 0,     \
                       stream, g0, g1);                                                       \
    return check_launch(fn);                                                                  \
  }
  TPF_GEMM_PAIR_CASE(1, 0, 0, 0, 0, 128)  // TriMul contraction backward (dA, dB)
  TPF_GEMM_PAIR_CASE(1, 0, 0, 0, 0, 192)
#undef TPF_GEMM_PAIR_CASE
  return set_error(TPF_ERR_ARG, "%s: GEMM pair layout not instantiated", fn);
}

int fold_launch(const float* part, float* out, int64_t n, int64_t stride, int splits,
                hipStream_t stream, const char* fn) {
  FoldSegs f{};
  f.nseg = 1;
  f.part[0] = part; f.n[0] = n; f.stride[0] = stride; f.splits[0] = splits;
  f.piece[0] = n; f.dst[0][0] = out;
  return fold_multi(f, stream, fn);
}

}  // namespace tpf

extern "C" int tpf_gemm_bf16(const void* A, int a_kc, int64_t a_ld, int64_t a_bs, const void* B,
                             int b_kc, int64_t b_ld, int64_t b_bs, void* C, int out_f32,
                             int64_t c_ld, int64_t c_bs, int64_t M, int64_t N, int64_t K,
                             int64_t batch, double alpha, void* stream) {
  if (!A || !B || !C) return tpf::set_error(TPF_ERR_ARG, "tpf_gemm_bf16: null pointer");
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX)
    return tpf::set_error(TPF_ERR_SHAPE, "tpf_gemm_bf16: dimension exceeds int32");
  // Tall row-major products with a small weight (the pair-row projections)
  // run on the weight-stationary row kernel; the choice depends on the
  // operand shapes only, so rows give the same bits in any row chunking.
  if (batch == 1 && !out_f32 && a_kc == 1 && alpha == 1.0) {
    int rc = TPF_OK;
    if (tpf::rowgemm_try((const __bf16*)A, a_ld, (const __bf16*)B, b_kc, b_ld, (__bf16*)C, c_ld, M,
                         N, K, (hipStream_t)stream, &rc, "tpf_gemm_bf16"))
      return rc;
  }
  tpf::GemmArgs g{};
  g.A = (const __bf16*)A; g.a_ld = a_ld; g.a_bs = a_bs;
  g.B = (const __bf16*)B; g.b_ld = b_ld; g.b_bs = b_bs;
  g.C = C; g.c_ld = c_ld; g.c_bs = c_bs; g.c_split = 0;
  g.M = (int)M; g.N = (int)N; g.K = (int)K; g.ksplit = 1; g.k_chunk = (int)K;
  g.alpha = (float)alpha;
  return tpf::gemm_launch(g, a_kc, b_kc, out_f32, (int)batch, (hipStream_t)stream, "tpf_gemm_bf16");
}


extern "C" int tpf_trimul_wgrad_fixed_fold(const float* partials, int64_t chunks, int64_t elements,
                                           float* accumulator, int initialize, void* stream) {
  const char* fn = "tpf_trimul_wgrad_fixed_fold";
  if (!partials || !accumulator) return tpf::set_error(TPF_ERR_ARG, "%s: null pointer", fn);
  if (chunks < 1 || chunks > INT32_MAX || elements < 1)
    return tpf::set_error(TPF_ERR_SHAPE, "%s: chunks and elements must be positive", fn);
  if ((elements + 255) / 256 > INT32_MAX)
    return tpf::set_error(TPF_ERR_SHAPE, "%s: too many elements", fn);
  const char* pa = (const char*)partials;
  const char* ac = (const char*)accumulator;
  if (ac < pa + chunks * elements * 4 && pa < ac + elements * 4)
    return tpf::set_error(TPF_ERR_ARG, "%s: accumulator overlaps the partials", fn);
  const dim3 grid((unsigned)((elements + 255) / 256));
  if (initialize)
    hipLaunchKernelGGL(tpf::wgrad_fixed_fold_kernel<true>, grid, dim3(256), 0, (hipStream_t)stream,
                       partials, (int)chunks, elements, accumulator);
  else
    hipLaunchKernelGGL(tpf::wgrad_fixed_fold_kernel<false>, grid, dim3(256), 0,
                       (hipStream_t)stream, partials, (int)chunks, elements, accumulator);
  return tpf::check_launch(fn);
}
