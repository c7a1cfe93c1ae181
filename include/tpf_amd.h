/*
 * TurboPairFormer on MI355X (gfx950): C ABI of libtpf_amd.so.
 *
 * Plain pointers, 64-bit sizes and a hipStream_t passed as void*.  Every
 * entry point launches asynchronously on the given stream, never
 * synchronises, and returns 0 on success or a TPF_ERR_* code; the message
 * of the last failure on the calling thread is tpf_last_error().  Shapes are
 * validated before any launch (the reference raises on the same conditions
 * through TORCH_CHECK, e.g. turbopairformer_triangle_forward.cu:1835-1897).
 * Callers allocate every output and workspace buffer.
 *
 * Dtypes: "bf16" pointers are bfloat16 arrays; "f32" are float arrays.
 */
#ifndef TPF_AMD_H
#define TPF_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  TPF_OK = 0,
  TPF_ERR_ARG = 1,    /* null pointer, workspace too small, bad flag */
  TPF_ERR_SHAPE = 2,  /* unsupported or inconsistent dimensions */
  TPF_ERR_LAUNCH = 3, /* the HIP runtime rejected a launch */
};

/* Message of the last failed call on this thread ("" if none). */
const char* tpf_last_error(void);
/* ABI revision of this header (8). */
int tpf_abi_version(void);

/* ------------------------------------------------------------------------
 * Triangle attention with pair bias.
 *
 * layout: bit flags.  q, k, v: bf16 [B, O, H, N, D] in one shared storage
 *   order: head-major (contiguous) or, with TPF_QKV_SEQ_MAJOR, sequence-major
 *   (a contiguous [B, O, N, H, D] buffer viewed as [B, O, H, N, D]).
 * mask: f32 [B, O, N] additive (0 keeps, -inf drops).
 * bias: bf16 [bias_batches, H, N, N], bias_batches in {1, B} (1 = shared),
 *   contiguous or, with TPF_BIAS_TRANSPOSED, the transpose over its last two
 *   axes of a contiguous one (bias[bb, h, q, k] stored at
 *   ((bb * H + h) * N + k) * N + q: the ending node's transposed pair bias,
 *   read in place).
 * out: bf16 [B, O, N, H, D].  lse, delta: f32 [B, O, H, N].
 * Requirements: N % 64 == 0 (pad on the host with -inf mask entries),
 * D % 8 == 0 and 8 <= D <= 64, B*O <= 65535.  scale = 1/sqrt(D_true): when
 * the host zero-pads D it passes the unpadded D's scale.
 * ---------------------------------------------------------------------- */

enum {
  TPF_QKV_SEQ_MAJOR = 1,   /* q, k, v (and dq, dk, dv) in sequence-major storage */
  TPF_BIAS_TRANSPOSED = 2, /* bias given as the transpose of a contiguous tensor */
  TPF_DBIAS_BF16 = 4,      /* backward: dbias is bf16 (the f32 fold rounded once), stored
                              in the bias's own order (transposed with TPF_BIAS_TRANSPOSED) */
};

/* Bytes of device workspace tpf_attn_forward_bf16 needs (the bias in f32,
 * prescaled by 1/scale). */
int64_t tpf_attn_forward_workspace_bytes(int64_t B, int64_t H, int64_t N, int64_t bias_batches);

/* Forward: out and the per-row logsumexp (-inf for a fully masked row,
 * whose output is 0).  Replaces turbopairformer_triangle_forward_out
 * (openfold3/core/kernels/turbopairformer/turbopairformer_triangle_forward.cu:1960-1990). */
int tpf_attn_forward_bf16(const void* q, const void* k, const void* v, const float* mask,
                          const void* bias, void* out, float* lse, void* workspace,
                          int64_t workspace_bytes, int64_t B, int64_t O, int64_t H, int64_t N,
                          int64_t D, int layout, int64_t bias_batches, double scale,
                          void* stream);

/* Forward that also writes the shadow residual: residual bf16 [B, O, N, H, D]
 * = bf16(O_f32 - f32(out)), the part of the f32 output the bf16 store of out
 * drops.  The backward's delta then pairs dO with out + residual
 * (tpf_attn_delta_shadow_bf16).  Replaces turbopairformer_triangle_forward_shadow_out
 * (openfold3/core/kernels/turbopairformer/turbopairformer_triangle_forward.cu:1960-1990,
 * selected by OPENFOLD3_SR_SHADOW, turbopairformer_triangle_attention.py:247-262). */
int tpf_attn_forward_shadow_bf16(const void* q, const void* k, const void* v, const float* mask,
                                 const void* bias, void* out, float* lse, void* residual,
                                 void* workspace, int64_t workspace_bytes, int64_t B, int64_t O,
                                 int64_t H, int64_t N, int64_t D, int layout,
                                 int64_t bias_batches, double scale, void* stream);

/* Forward that allocates nothing: the same kernels as tpf_attn_forward_bf16,
 * with the prescaled-bias scratch in a static per-GPU device array of 16 MiB
 * (bias_batches * H * N * N <= 4,194,304; larger problems are rejected with
 * TPF_ERR_SHAPE) instead of a caller workspace.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (different streams) race and must be serialised by the caller.  The
 * array's address is looked up once per device on that device's first call. */
int tpf_attn_forward_noalloc_bf16(const void* q, const void* k, const void* v, const float* mask,
                                  const void* bias, void* out, float* lse, int64_t B, int64_t O,
                                  int64_t H, int64_t N, int64_t D, int layout,
                                  int64_t bias_batches, double scale, void* stream);

/* delta = rowsum(f32(dout) * f32(out)) for dout/out bf16 [B, O, N, H, D].
 * Replaces turbopairformer_triangle_delta_out
 * (openfold3/core/kernels/turbopairformer/turbopairformer_triangle_delta.cu:292-342). */
int tpf_attn_delta_bf16(const void* dout, const void* out, float* delta, int64_t B, int64_t O,
                        int64_t H, int64_t N, int64_t D, void* stream);

/* delta = rowsum(f32(dout) * (f32(out) + f32(residual))), residual from
 * tpf_attn_forward_shadow_bf16.  Replaces turbopairformer_triangle_delta_shadow_out
 * (openfold3/core/kernels/turbopairformer/turbopairformer_triangle_delta.cu:343-416). */
int tpf_attn_delta_shadow_bf16(const void* dout, const void* out, const void* residual,
                               float* delta, int64_t B, int64_t O, int64_t H, int64_t N,
                               int64_t D, void* stream);

/* Bytes of device workspace of the one-slab backward plan (dQ partials of
 * every outer row, one f32 dBias partial per run of outer groups, the
 * prescaled bias and the row statistics).  tpf_attn_backward_main_bf16 /
 * _finish_bf16 need this much. */
int64_t tpf_attn_backward_workspace_bytes(int64_t B, int64_t O, int64_t H, int64_t N,
                                          int64_t D);

/* Workspace bytes of the backward plan under a budget: the full plan when it
 * fits, otherwise slabs of consecutive runs of outer rows whose dQ partials
 * fit (each slab's dQ folded before the next reuses the space; dBias partials
 * stay resident, so every summation order, and every result bit, is that of
 * the full plan).  Below the one-run minimum the minimum is returned (it
 * exceeds the budget), as the reference's planner returns its irreducible
 * tile.  tpf_attn_backward_bf16 and tpf_attn_backward_fused_bf16 accept any
 * workspace of at least the minimum and plan their slabs from its size.
 * Replaces workspace_plan / sr_workspace_plan
 * (openfold3/core/kernels/turbopairformer/turbopairformer_triangle_dq_dbias.py:149-300,569-669),
 * whose 256 MiB budget bounds its dBias leaves. */
int64_t tpf_attn_backward_workspace_bytes_budget(int64_t B, int64_t O, int64_t H, int64_t N,
                                                 int64_t D, int64_t budget_bytes);
/* Slabs the backward runs in for a workspace of workspace_bytes (0 when it
 * is below the minimum; -1 for non-positive sizes). */
int tpf_attn_backward_slab_count(int64_t B, int64_t O, int64_t H, int64_t N, int64_t D,
                                 int64_t workspace_bytes);

/* Single-reconstruction backward: dq, dk, dv (bf16, same storage order as
 * q) and dbias (f32 [bias_batches, H, N, N], summed over every (b, o) that
 * shares the bias; with TPF_DBIAS_BF16 the same sums rounded to bf16 and
 * stored in the bias's order), all reduced in fixed orders that depend on
 * the problem shape only (not on the device's CU count or the workspace
 * size): bitwise reproducible on any gfx950 device and for any budget.
 * Replaces turbopairformer_triangle_sr_backward_out
 * (openfold3/core/kernels/turbopairformer/turbopairformer_triangle_dq_dbias.cu:2526-2648)
 * together with its planner (turbopairformer_triangle_dq_dbias.py:466-566)
 * and the broadcast dBias reduction (:1788-1825, .py:326-376). */
int tpf_attn_backward_bf16(const void* q, const void* k, const void* v, const void* dout,
                           const float* lse, const float* delta, const float* mask,
                           const void* bias, void* dq, void* dk, void* dv, void* dbias,
                           void* workspace, int64_t workspace_bytes, int64_t B, int64_t O,
                           int64_t H, int64_t N, int64_t D, int layout, int64_t bias_batches,
                           double scale, void* stream);

/* The two stages of tpf_attn_backward_bf16, for callers that time or
 * schedule them separately: the reconstruction kernel (dk, dv and the
 * partials in workspace) and the fixed-order folds of the dQ / dBias
 * partials.  Same split as the reference's sr_leaf_kernel / finalizer /
 * dq_reduce launches (turbopairformer_triangle_dq_dbias.cu:2358-2499). */
int tpf_attn_backward_main_bf16(const void* q, const void* k, const void* v, const void* dout,
                                const float* lse, const float* delta, const float* mask,
                                const void* bias, void* dk, void* dv, void* workspace,
                                int64_t workspace_bytes, int64_t B, int64_t O, int64_t H,
                                int64_t N, int64_t D, int layout, int64_t bias_batches,
                                double scale, void* stream);
int tpf_attn_backward_finish_bf16(void* dq, void* dbias, const void* workspace, int64_t B,
                                  int64_t O, int64_t H, int64_t N, int64_t D, int layout,
                                  int64_t bias_batches, double scale, void* stream);

/* The whole backward from the forward's outputs in three launches: delta
 * (rowsum(f32(dout) * (f32(out) + f32(residual))), residual nullable),
 * the row statistics and the prescaled bias in one kernel, then the
 * reconstruction kernel and the folds.  Same results as
 * tpf_attn_delta[_shadow]_bf16 followed by tpf_attn_backward_bf16 (the
 * delta values never leave the workspace).  No single counterpart in the
 * reference, whose facade launches delta_out / delta_shadow_out and
 * sr_backward_out back to back (turbopairformer_triangle_attention.py:287-304). */
int tpf_attn_backward_fused_bf16(const void* q, const void* k, const void* v, const void* dout,
                                 const void* out, const void* residual, const float* lse,
                                 const float* mask, const void* bias, void* dq, void* dk,
                                 void* dv, void* dbias, void* workspace, int64_t workspace_bytes,
                                 int64_t B, int64_t O, int64_t H, int64_t N, int64_t D,
                                 int layout, int64_t bias_batches, double scale, void* stream);

/* Split backward route for direct callers (not on the facade path), from
 * caller-supplied lse and delta, in the layouts and flags of
 * tpf_attn_backward_bf16 (TPF_DBIAS_BF16 excluded).
 *
 * dK / dV only: dk, dv bf16 in Q/K/V storage order.  With delta_true
 * (nullable, f32 [B, O, H, N]) the call also forms delta_true = sum_k P dP
 * of each query row: per-64-key-block f32 partials in delta_true_partials
 * ([B, O, H, ceil(N/64), N], tpf_attn_dkdv_delta_true_partial_elements
 * floats, 16-byte aligned) folded in ascending block order.  dS uses the
 * supplied delta either way.  dk and dv are bitwise those of
 * tpf_attn_backward_bf16 on the same inputs.  Replaces
 * turbopairformer_triangle_dkdv_out / _dkdv_delta_true_out
 * (openfold3/core/kernels/turbopairformer/turbopairformer_triangle_dkdv.py:101-174). */
int64_t tpf_attn_dkdv_workspace_bytes(int64_t B, int64_t O, int64_t H, int64_t N, int64_t D,
                                      int64_t bias_batches);
int64_t tpf_attn_dkdv_delta_true_partial_elements(int64_t B, int64_t O, int64_t H, int64_t N);
int tpf_attn_dkdv_bf16(const void* q, const void* k, const void* v, const void* dout,
                       const float* lse, const float* delta, const float* mask, const void* bias,
                       void* dk, void* dv, float* delta_true_partials, float* delta_true,
                       void* workspace, int64_t workspace_bytes, int64_t B, int64_t O, int64_t H,
                       int64_t N, int64_t D, int layout, int64_t bias_batches, double scale,
                       void* stream);
/* dQ / dBias only: dq bf16 in Q's storage order and dbias f32 per batch item
 * [B, H, N, N] (a bias shared by the batch still gets one gradient per
 * item; the caller reduces a broadcast).  Workspace and slabs as
 * tpf_attn_backward_bf16 (its size queries apply); dq and each batch's
 * dbias are bitwise that route's.  Replaces turbopairformer_triangle_dq_dbias_out
 * (openfold3/core/kernels/turbopairformer/turbopairformer_triangle_dq_dbias.py:379-463). */
int64_t tpf_attn_dq_dbias_workspace_bytes(int64_t B, int64_t O, int64_t H, int64_t N, int64_t D);
int tpf_attn_dq_dbias_bf16(const void* q, const void* k, const void* v, const void* dout,
                           const float* lse, const float* delta, const float* mask,
                           const void* bias, void* dq, float* dbias, void* workspace,
                           int64_t workspace_bytes, int64_t B, int64_t O, int64_t H, int64_t N,
                           int64_t D, int layout, int64_t bias_batches, double scale,
                           void* stream);

/* FP32 forward (inference): q, k, v, bias f32 in the layouts above (layout:
 * TPF_QKV_SEQ_MAJOR only; the bias is contiguous), out f32
 * [B, O, N, H, D], lse (nullable) f32 [B, O, H, N].  Requirements: N % 64 == 0,
 * D % 4 == 0 and 4 <= D <= 64.  Products and sums in FP32 MFMA.
 * Replaces turbopairformer_attention_fp32_forward
 * (openfold3/core/kernels/turbopairformer/turbopairformer_attention_fp32.py:139-224). */
int64_t tpf_attn_forward_f32_workspace_bytes(int64_t B, int64_t H, int64_t N,
                                             int64_t bias_batches);
int tpf_attn_forward_f32(const float* q, const float* k, const float* v, const float* mask,
                         const float* bias, float* out, float* lse, void* workspace,
                         int64_t workspace_bytes, int64_t B, int64_t O, int64_t H, int64_t N,
                         int64_t D, int layout, int64_t bias_batches, double scale,
                         void* stream);

/* ------------------------------------------------------------------------
 * Triangle multiplicative update (C == H in {32, 64, 96, 128}).
 *
 * z: bf16 [B, N, N, C]; mask: f32 [B, N, N].
 * Weights (f32, the module's parameters): w_ap, w_ag, w_bp, w_bg [H, C],
 * w_g [C, C], w_z [C, H]; LayerNorm weights f32 [C].  Both entry points
 * pack them into bf16 GEMM operands inside the workspace.
 * Saved state written by the forward (R = B*N*N rows): zln [R, C], gate =
 * output-gate logits zln W_g^T [R, C], a, b [B*H, N*Np] (channel-major
 * stored matrices, Np = tpf_trimul_plane_pitch(N)), x [B*H, N, Np], xln
 * [R, H], mean/rstd f32 [R].
 * ---------------------------------------------------------------------- */

/* Row pitch Np (N rounded up to 8) of the channel-major a / b / x buffers. */
int64_t tpf_trimul_plane_pitch(int64_t N);

/* 1 when the bf16 TriMul kernels take a [B, N, N, C] pair (C in {32, 64, 96,
 * 128}): every [B*N*N, C] row tensor and [B*C, N, Np] plane tensor below
 * 2 GiB (the kernels' 32-bit buffer offsets), and, for the backward
 * (backward != 0), the [B*N*N, 5C] dproj5 scratch too (at C = 128: N <= 2896
 * forward, N <= 1295 backward, B = 1); else 0.  Host-only, no launch.  The
 * reference's kernels index in 64 bits (check_pair_extent,
 * turbopairformer_trimul_cuda.cu:147-166); larger pairs take the stock path
 * through check_stable_trimul_support. */
int tpf_trimul_shape_supported(int64_t B, int64_t N, int64_t C, int backward);

/* Bytes of device workspace tpf_trimul_forward_bf16 needs (packed bf16 weights). */
int64_t tpf_trimul_forward_workspace_bytes(int64_t C);

/* Forward: LN_in + projections + gates (trimul_in_fwd), the channel
 * contraction (the reference's torch.bmm), LN_out + projection + gate
 * (trimul_out_fwd).  outgoing = 1: x_ij = sum_k a_ik b_jk; 0: sum_k a_ki b_kj.
 * Replaces trimul_in_fwd / torch.bmm / trimul_out_fwd of
 * _trimul_forward_impl (openfold3/core/kernels/turbopairformer/turbopairformer_trimul.py:184-292;
 * kernels turbopairformer_trimul_cuda.cu:615-1166, 1191-1530). */
int tpf_trimul_forward_bf16(const void* z, const float* mask, const float* w_ap, const float* w_ag,
                            const float* w_bp, const float* w_bg, const float* w_g,
                            const float* w_z, const float* ln_in_w, const float* ln_in_b,
                            const float* ln_out_w, const float* ln_out_b, int outgoing, int64_t B,
                            int64_t N, int64_t C, void* out, void* zln, void* gate, void* a,
                            void* b, void* x, void* xln, float* mean_in, float* rstd_in,
                            float* mean_out, float* rstd_out, void* workspace,
                            int64_t workspace_bytes, void* stream);

int64_t tpf_trimul_backward_workspace_bytes(int64_t B, int64_t N, int64_t C);

/* Backward: dz (bf16) and every parameter gradient in f32 with fixed-order
 * reductions.  d_w5 is [5H, C] in the order [w_ap; w_ag; w_bp; w_bg; w_g]
 * (the reference's d_w5), d_w_z [C, H].
 * Replaces _trimul_backward_combined_impl
 * (openfold3/core/kernels/turbopairformer/turbopairformer_trimul.py:295-392) with its
 * kernels sig_mul_bwd_out, transpose_ln_bwd, trimul_gate_split_bwd,
 * ln_bwd_dx, ln_bwd_dgb, trimul_wgrad_fixed_fold
 * (turbopairformer_trimul_cuda.cu:196-560, 1532-2160) and its cuBLAS GEMMs. */
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
                             void* stream);
/* tpf_trimul_backward_bf16 with the W5 gradient delivered as the gradients
 * of turbo_trimul's named weights (README.md:137-143, `p_in_weight`,
 * `g_in_weight`, `g_out_weight`): d_p_in [2H, C] = [d w_ap; d w_bp], d_g_in
 * [2H, C] = [d w_ag; d w_bg], d_w_g [C, C].  The fold writes each row block
 * straight to its place (same values, bit for bit, as the d_w5 rows), so
 * the caller needs no row gather. */
int tpf_trimul_backward_named_bf16(
    const void* grad_out, const void* z, const float* mask, const float* w_ap, const float* w_ag,
    const float* w_bp, const float* w_bg, const float* w_g, const float* w_z,
    const float* ln_in_w, const float* ln_out_w, const void* zln, const void* gate, const void* a,
    const void* b, const void* x, const void* xln, const float* mean_in, const float* rstd_in,
    const float* mean_out, const float* rstd_out, int outgoing, int64_t B, int64_t N, int64_t C,
    void* dz, float* d_p_in, float* d_g_in, float* d_w_g, float* d_w_z, float* d_ln_in_w,
    float* d_ln_in_b, float* d_ln_out_w, float* d_ln_out_b, void* workspace,
    int64_t workspace_bytes, void* stream);

/* Weight gradient of a linear layer over R rows, dW[m][n] = sum_r dy[r][m] x[r][n]
 * (dy [R, M], x [R, N] row-major bf16 with leading dimensions ld_dy, ld_x;
 * dW f32 [M, N]), split over R with a fixed-order fold.  Used for the pair
 * stack's projection weights (R = B*N^2), the products the reference leaves
 * to torch / cuBLAS (openfold3/core/model/layers/triangular_attention.py:160-243). */
int64_t tpf_wgrad_bf16_workspace_bytes(int64_t R, int64_t M, int64_t N);
int tpf_wgrad_bf16(const void* dy, int64_t ld_dy, const void* x, int64_t ld_x, int64_t R,
                   int64_t M, int64_t N, float* dw, void* workspace, int64_t workspace_bytes,
                   void* stream);

/* FP32 TriMul forward (inference).  z f32 [B, N, N, C] (rows contiguous),
 * mask f32 [B, N, N]; weights f32 w_ap, w_ag, w_bp, w_bg [H, C], w_g [C, C],
 * w_z [C, H]; biases (each nullable) [H] / [C]; LayerNorm affine
 * parameters nullable, with their eps.  out f32 [B, N, N, C].  C <= 512,
 * H <= 256.  Replaces run_trimul_fp32
 * (openfold3/core/kernels/turbopairformer/turbopairformer_trimul_fp32.py:155-400). */
int64_t tpf_trimul_forward_f32_workspace_bytes(int64_t B, int64_t N, int64_t C, int64_t H);
int tpf_trimul_forward_f32(const float* z, const float* mask, const float* w_ap, const float* w_ag,
                           const float* w_bp, const float* w_bg, const float* w_g,
                           const float* w_z, const float* b_ap, const float* b_ag,
                           const float* b_bp, const float* b_bg, const float* b_g,
                           const float* b_z, const float* ln_in_w, const float* ln_in_b,
                           double ln_in_eps, const float* ln_out_w, const float* ln_out_b,
                           double ln_out_eps, int outgoing, int64_t B, int64_t N, int64_t C,
                           int64_t H, float* out, void* workspace, int64_t workspace_bytes,
                           void* stream);
/* tpf_trimul_forward_f32 with the contraction, LN_out and output projection
 * run over chunks of row_chunk output rows i (per batch item), so the product
 * scratch is [H, row_chunk, N] instead of [B, H, N, N]; the outputs are
 * bitwise those of the unchunked call.  Replaces the output_row_chunk_size
 * path of run_trimul_fp32
 * (openfold3/core/kernels/turbopairformer/turbopairformer_trimul_fp32.py:203-221,344-345). */
int64_t tpf_trimul_forward_f32_workspace_bytes_chunked(int64_t B, int64_t N, int64_t C, int64_t H,
                                                       int64_t row_chunk);
int tpf_trimul_forward_f32_chunked(const float* z, const float* mask, const float* w_ap,
                                   const float* w_ag, const float* w_bp, const float* w_bg,
                                   const float* w_g, const float* w_z, const float* b_ap,
                                   const float* b_ag, const float* b_bp, const float* b_bg,
                                   const float* b_g, const float* b_z, const float* ln_in_w,
                                   const float* ln_in_b, double ln_in_eps, const float* ln_out_w,
                                   const float* ln_out_b, double ln_out_eps, int outgoing,
                                   int64_t B, int64_t N, int64_t C, int64_t H, int64_t row_chunk,
                                   float* out, void* workspace, int64_t workspace_bytes,
                                   void* stream);

/* Batched bf16 MFMA GEMM C[z] = alpha * A[z] B[z]^T with each operand
 * K-contiguous (x_kc = 1: X[r*ld + k]) or MN-contiguous (0: X[k*ld + r]);
 * C row-major, bf16 (out_f32 = 0) or f32.  The channel contraction of
 * TriMul, which the reference delegates to cuBLAS through torch.bmm
 * (turbopairformer_trimul.py:244-249, 355-362). */
int tpf_gemm_bf16(const void* A, int a_kc, int64_t a_ld, int64_t a_bs, const void* B, int b_kc,
                  int64_t b_ld, int64_t b_bs, void* C, int out_f32, int64_t c_ld, int64_t c_bs,
                  int64_t M, int64_t N, int64_t K, int64_t batch, double alpha, void* stream);

/* Fixed-order FP32 fold of weight-gradient partials [chunks, elements]:
 * accumulator[e] = (((init + p[0][e]) + p[1][e]) + ...) + p[chunks-1][e],
 * each add rounded to nearest, init = 0 when initialize != 0 else the
 * accumulator's current value (bitwise equal to an ascending FP32 add_ over
 * the chunks).  The accumulator must not overlap the partials.  Replaces
 * trimul_wgrad_fixed_fold
 * (openfold3/core/kernels/turbopairformer/turbopairformer_trimul_cuda.cu:200-217, 2050-2089). */
int tpf_trimul_wgrad_fixed_fold(const float* partials, int64_t chunks, int64_t elements,
                                float* accumulator, int initialize, void* stream);

/* Batched FP32 MFMA GEMM C[z] = alpha * A[z] B[z]^T + bias (bias per column,
 * nullable), operands K- or MN-contiguous as tpf_gemm_bf16, C row-major f32.
 * The strict-FP32 products of the reference's FP32 TriMul
 * (turbopairformer_trimul_fp32.py:336-360). */
int tpf_gemm_f32(const float* A, int a_kc, int64_t a_ld, int64_t a_bs, const float* B, int b_kc,
                 int64_t b_ld, int64_t b_bs, float* C, int64_t c_ld, int64_t c_bs, int64_t M,
                 int64_t N, int64_t K, int64_t batch, double alpha, const float* bias,
                 void* stream);

/* LayerNorm over the C contiguous bf16 channels of each row of a [B, I, J]
 * pair grid, FP32 statistics.  x rows are addressed through element strides
 * (sb, si, sj) (multiples of 8), so a transposed view is read in place; y
 * [B*I*J, C], mean and rstd [B*I*J] are written in logical row order.  w / b
 * (f32 [C]) are nullable (no affine).  8 <= C <= 2048, C % 8 == 0.  Replaces
 * the module's torch LayerNorm with FP32 statistics
 * (openfold3/core/model/primitives/normalization.py:54-78, applied at
 * openfold3/core/model/layers/triangular_attention.py:160-170). */
int tpf_layer_norm_forward_bf16(const void* x, int64_t B, int64_t I, int64_t J, int64_t sb,
                                int64_t si, int64_t sj, int64_t C, const float* w,
                                const float* b, double eps, void* y, float* mean, float* rstd,
                                void* stream);

/* Its backward: dy [B*I*J, C] logical row order, x with strides (sb, si, sj)
 * and dx written with strides (dsb, dsi, dsj); dw / db f32 [C] (both null to
 * skip the parameter gradients) from fixed-order partials in the workspace. */
int64_t tpf_layer_norm_backward_workspace_bytes(int64_t R, int64_t C);
int tpf_layer_norm_backward_bf16(const void* dy, const void* x, int64_t B, int64_t I, int64_t J,
                                 int64_t sb, int64_t si, int64_t sj, int64_t dsb, int64_t dsi,
                                 int64_t dsj, int64_t C, const float* mean, const float* rstd,
                                 const float* w, void* dx, float* dw, float* db, void* workspace,
                                 int64_t workspace_bytes, void* stream);

/* Attention core of the triangle-attention module over pair rows (row
 * (b, i, j) = pair (i, j); plane i attends over j).  q, k, v are head-major
 * planes qkv [3][B][N][H][N][D] bf16 (q | k | v, as tpf_pair_projection_bf16
 * writes them); rest [B*N*N][rest_pitch] bf16 holds per pair row the gate
 * logits (H*D) | the pair bias (H) | pad; mask f32 [B, N, N] additive.
 * flags: TPF_PAIR_BIAS_TRANSPOSED selects bias[h, q, k] = rest[b, k, q, HD + h]
 * instead of rest[b, q, k, HD + h]; TPF_PAIR_OG_TRANSPOSED stores og
 * (forward) and reads d_og (backward) of pair row (i, j) at row (j, i), so the
 * ending node's module output leaves its output projection in the caller's
 * pair order.  Forward writes o [B, N, N, H*D], lse [B, N, H, N] f32 and the
 * gated og = o * sigmoid(gate).  Backward takes d_og and writes the whole
 * projection gradient row into dproj [B*N*N][dproj_pitch] = q | k | v | gate
 * | bias | pad (pad zeroed).  residual (nullable, bf16 like o): when given,
 * the forward writes o's shadow residual there and the backward forms delta
 * from o + residual, as the standalone shadow entry points do.  Replaces the
 * module glue around the kernel
 * (openfold3/core/model/layers/triangular_attention.py:160-243 with
 * openfold3/core/model/primitives/attention.py:640-692: q/k/v/gate/bias
 * projections split into views, gating, and the gradient concatenation). */
enum {
  TPF_PAIR_BIAS_TRANSPOSED = 1, /* pair bias read as bias[h, q, k] = rest[b, k, q, HD + h] */
  TPF_PAIR_OG_TRANSPOSED = 2    /* og / d_og rows in transposed pair order */
};
int64_t tpf_attn_pair_forward_workspace_bytes(int64_t B, int64_t N, int64_t H);
int tpf_attn_pair_forward_bf16(const void* qkv, const void* rest, int64_t rest_pitch,
                               const float* mask, int flags, void* o, float* lse, void* og,
                               void* residual, void* workspace, int64_t workspace_bytes,
                               int64_t B, int64_t N, int64_t H, int64_t D, double scale,
                               void* stream);
int64_t tpf_attn_pair_backward_workspace_bytes(int64_t B, int64_t N, int64_t H, int64_t D);
int tpf_attn_pair_backward_bf16(const void* qkv, const void* rest, int64_t rest_pitch,
                                const float* mask, int flags, const void* o, const float* lse,
                                const void* residual, const void* d_og, void* dproj,
                                int64_t dproj_pitch, void* workspace, int64_t workspace_bytes,
                                int64_t B, int64_t N, int64_t H, int64_t D, double scale,
                                void* stream);
/* tpf_attn_pair_backward_bf16 from the module's upstream gradient instead of
 * d_og: dout [B*N*N, C] bf16 (rows in the caller's pair order, transposed
 * with TPF_PAIR_OG_TRANSPOSED) and the output projection weight w_o [C, H*D]
 * bf16 (out = og w_o^T).  The product d_og = dout w_o runs on the
 * weight-stationary row kernel with the gate backward (d_o, the gate
 * gradient, delta) in its epilogue, so d_og never reaches memory; results
 * are bitwise those of tpf_gemm_bf16 (dout, w_o) followed by
 * tpf_attn_pair_backward_bf16.  Same workspace.  Supported when C = 128, D in
 * {8, 16, 32, 64} and H*D a multiple of 16 up to 128
 * (tpf_attn_pair_backward_dout_supported).  Replaces the same module glue
 * (openfold3/core/model/primitives/attention.py:640-692: linear_o's input
 * gradient and the gating backward). */
int tpf_attn_pair_backward_dout_supported(int64_t C, int64_t H, int64_t D);
int tpf_attn_pair_backward_dout_bf16(const void* qkv, const void* rest, int64_t rest_pitch,
                                     const float* mask, int flags, const void* o,
                                     const float* lse, const void* residual, const void* dout,
                                     const void* w_o, int64_t C, void* dproj, int64_t dproj_pitch,
                                     void* workspace, int64_t workspace_bytes, int64_t B,
                                     int64_t N, int64_t H, int64_t D, double scale, void* stream);

/* The projection of the triangle-attention module, x [B*N*N, C] times
 * W_all^T (W_all [P, C] = W_q; W_k; W_v; W_gate; W_bias; 0), with its output
 * split as the pair-row core reads it: columns q | k | v into head-major
 * planes qkv [3][B][N][H][N][D], the remaining P - 3*H*D columns (gate | bias
 * | pad) into rows rest [B*N*N][P - 3*H*D].  bf16 in and out, f32
 * accumulation, on the weight-stationary row kernel; supported when C = 128,
 * P is a multiple of 16 up to 640 with P - 3*H*D >= 8 a multiple of 8, N a
 * multiple of 32 and D a multiple of 8 (tpf_pair_projection_supported).  No
 * reference counterpart as one call: the module's linear projections
 * (openfold3/core/model/layers/triangular_attention.py:160-243). */
int tpf_pair_projection_supported(int64_t P, int64_t C, int64_t N, int64_t H, int64_t D);
int tpf_pair_projection_bf16(const void* x, const void* w, int64_t B, int64_t N, int64_t C,
                             int64_t P, int64_t H, int64_t D, void* qkv, void* rest,
                             void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TPF_AMD_H */
