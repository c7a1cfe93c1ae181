"""Drop-in OpenFold3 pair-stack modules backed by the MI355X kernels.

``TriangleAttention`` (``TriangleAttentionStartingNode`` /
``TriangleAttentionEndingNode``) and ``TriangleMultiplicativeUpdate`` (with
the ``TriangleMultiplicationOutgoing`` / ``Incoming`` subclasses) register the
same parameters under the same names as OpenFold3's modules
(``openfold3/core/model/layers/triangular_attention.py:35-75`` with the
``Attention`` primitive of ``openfold3/core/model/primitives/attention.py``,
and ``openfold3/core/model/layers/triangular_multiplicative_update.py:700-830``),
so a ``state_dict`` of the stock module loads unchanged, and take the same
forward arguments (``triangular_attention.py:245-258``,
``triangular_multiplicative_update.py:1187-1197``).  Routing follows the
reference's ``use_stable_*`` policy (``attention.py:520-692``,
``triangular_multiplicative_update.py:62-120``), with the stable kernels
selected by default here:

* attention, stable: LayerNorm (FP32 statistics; the BF16 LayerNorm kernel),
  the additive mask ``inf * (mask - 1)``, one projection GEMM for q / k / v,
  the gate and the pair bias ``linear_z``; for N a multiple of 64 the
  pair-row core (``tpf_attn_pair_*``: attention and gate read the projection
  rows in place, gradients land in one projection-gradient buffer), else the
  triangle-attention facade on sequence-major views; ``linear_o``.  The
  projection weight gradients (contractions over all B*N^2 pair rows) run on
  the split-K MFMA GEMM.  FP32 activations under ``torch.no_grad()`` take
  the FP32 inference kernel; FP32 training inputs take the stock FP32 math
  unless ``set_tpf_bf16_cast_for_fp32_training(True)``.
* TriMul, stable: ``run_trimul_fp32`` for FP32 inference, else
  ``run_stable_trimul`` (BF16 kernels, autograd) when
  ``check_stable_trimul_support`` accepts the module.
* An unsupported stable request raises under strict mode and otherwise logs
  once and runs the stock PyTorch math (``routing.py``);
  ``use_stable_*=False`` selects the stock math directly.  The reference's
  other backends (DeepSpeed, cuEquivariance, Triton, LMA, Protenix) do not
  exist in this build and raise.
"""

from __future__ import annotations

import math

import torch
from torch import nn

from . import _native, routing
from .attention import (
    _device_ctx,
    is_turbopairformer_supported,
    shadow_enabled,
    turbopairformer_triangle_attention,
)
from .attention_fp32 import turbopairformer_attention_fp32
from .layernorm import layer_norm_bf16
from .trimul import check_stable_trimul_support, run_stable_trimul
from .trimul_fp32 import run_trimul_fp32


def _reject_backends(**flags) -> None:
    for name, value in flags.items():
        if value:
            raise ValueError(f"{name} is not available in this build (MI355X kernels only)")


def _fp32_compute(x: torch.Tensor) -> bool:
    return x.dtype == torch.float32 and (
        not torch.is_autocast_enabled("cuda") or torch.get_autocast_dtype("cuda") == torch.float32)


def _stock_layer_norm(ln: nn.LayerNorm, x: torch.Tensor) -> torch.Tensor:
    w = None if ln.weight is None else ln.weight.float()
    b = None if ln.bias is None else ln.bias.float()
    return nn.functional.layer_norm(x.float(), ln.normalized_shape, w, b, ln.eps).to(x.dtype)


def _stock_linear(layer: nn.Linear, x: torch.Tensor) -> torch.Tensor:
    b = None if layer.bias is None else layer.bias.to(x.dtype)
    return nn.functional.linear(x, layer.weight.to(x.dtype), b)


def _layer_norm(ln: nn.LayerNorm, x: torch.Tensor) -> torch.Tensor:
    """LayerNorm with FP32 statistics, returned in the input dtype
    (``openfold3/core/model/primitives/normalization.py:54-78``); BF16 CUDA
    activations run on the LayerNorm kernel (strided rows read in place)."""
    C = x.shape[-1]
    if x.is_cuda and x.dtype == torch.bfloat16 and C % 8 == 0 and 8 <= C <= 2048:
        return layer_norm_bf16(x, ln.weight, ln.bias, ln.eps)
    w = None if ln.weight is None else ln.weight.float()
    b = None if ln.bias is None else ln.bias.float()
    return nn.functional.layer_norm(x.float(), ln.normalized_shape, w, b, ln.eps).to(x.dtype)


def _fp32_inference(x: torch.Tensor) -> bool:
    return x.dtype == torch.float32 and not torch.is_grad_enabled()


def _wgrad(dy2: torch.Tensor, x2: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """dW = dy2^T x2 over all rows on the split-K MFMA GEMM (f32 accumulate)."""
    R, M = dy2.shape
    K = x2.shape[1]
    dw32 = torch.empty((M, K), device=x2.device, dtype=torch.float32)
    ws_bytes = int(_native.query("tpf_wgrad_bf16_workspace_bytes", R, M, K))
    ws = torch.empty(ws_bytes, device=x2.device, dtype=torch.uint8)
    with _device_ctx(x2.device):
        _native.call("tpf_wgrad_bf16", dy2.data_ptr(), dy2.stride(0), x2.data_ptr(),
                     x2.stride(0), R, M, K, dw32.data_ptr(), ws.data_ptr(), ws_bytes,
                     _native.stream_of(x2))
    return dw32.to(dtype)


def _mm(a: torch.Tensor, b: torch.Tensor, b_kc: bool) -> torch.Tensor:
    """Row GEMM of the pair-row modules on the bf16 MFMA GEMM
    (``tpf_gemm_bf16``): ``a [R, K] @ b.t()`` for ``b [N, K]`` (b_kc) or
    ``a @ b`` for ``b [K, N]``, f32 accumulation, bf16 out.  Operands are
    made contiguous; a feature size that is not a multiple of 8 (16-byte
    rows) takes torch's matmul."""
    a = a.contiguous()
    b = b.contiguous()
    R, K = a.shape
    N = b.shape[0] if b_kc else b.shape[1]
    if a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16 or K % 8 or N % 8:
        return a @ (b.t() if b_kc else b)
    out = torch.empty((R, N), device=a.device, dtype=torch.bfloat16)
    with _device_ctx(a.device):
        _native.call("tpf_gemm_bf16", a.data_ptr(), 1, K, 0, b.data_ptr(), int(b_kc),
                     b.stride(0), 0, out.data_ptr(), 0, N, 0, R, N, K, 1, 1.0,
                     _native.stream_of(a))
    return out


def _pair_projection(x2: torch.Tensor, wa: torch.Tensor, B: int, N: int, H: int, D: int):
    """x2 [R, C] @ wa^T split as the pair-row core reads it: q | k | v as
    head-major planes [3, B, N, H, N, D] and gate | bias | pad as rows
    [R, P - 3 H D], in one pass of the row GEMM (``tpf_pair_projection_bf16``)
    where the shape has an instance, else through the tile GEMM and a copy."""
    R, C = x2.shape
    P, hc = wa.shape[0], H * D
    dev = x2.device
    qkv = torch.empty((3, B, N, H, N, D), device=dev, dtype=torch.bfloat16)
    if _native.query("tpf_pair_projection_supported", P, C, N, H, D):
        rest = torch.empty((R, P - 3 * hc), device=dev, dtype=torch.bfloat16)
        x2 = x2.contiguous()
        with _device_ctx(dev):
            _native.call("tpf_pair_projection_bf16", x2.data_ptr(), wa.data_ptr(), B, N, C, P, H,
                         D, qkv.data_ptr(), rest.data_ptr(), _native.stream_of(x2))
        return qkv, rest
    proj = _mm(x2, wa, True)
    qkv.copy_(proj[:, :3 * hc].view(B, N, N, 3, H, D).permute(3, 0, 1, 4, 2, 5))
    return qkv, proj[:, 3 * hc:].contiguous()


def _pair_flags(transpose_bias: bool, og_t: bool) -> int:
    """Flags of the pair-row entry points (TPF_PAIR_BIAS_TRANSPOSED = 1,
    TPF_PAIR_OG_TRANSPOSED = 2)."""
    return (1 if transpose_bias else 0) | (2 if og_t else 0)


class _PairAttentionCore(torch.autograd.Function):
    """Projection -> triangle attention -> gate -> output projection of the
    triangle-attention module over BF16 pair rows, with explicit buffers.

    One GEMM forms x W_all^T (W_all rows q | k | v | gate | bias | pad) and
    stores q, k, v as head-major planes qkv [3, B, N, H, N, D] (the layout the
    attention kernels stream as contiguous tiles) and gate | bias | pad as
    rows ``rest`` [R, P - 3 H D] (``_pair_projection``);
    ``tpf_attn_pair_forward_bf16`` reads them in place and writes o and
    og = o * sigmoid(gate); out = og W_o^T.
    The backward's ``tpf_attn_pair_backward_bf16`` writes every column of the
    projection gradient row (gate, q, k, v, bias, zeroed pad) into one
    buffer, so dx = dproj W_all and dW_all = dproj^T x are single GEMMs.

    ``og_t`` (the ending node, whose x rows are the transposed pair order):
    og is stored in the caller's pair order, so ``out`` leaves the output
    projection in that order and the module returns it without a transposed
    copy; the backward reads d_og in the same order.
    """

    @staticmethod
    def forward(ctx, x, w_all, w_o, mask_add, H, D, transpose_bias, og_t=False):
        B, N, _, C = x.shape
        P = w_all.shape[0]
        R, hc = B * N * N, H * D
        dev = x.device
        x2 = x.reshape(R, C)
        wa = w_all.to(torch.bfloat16)
        wo = w_o.to(torch.bfloat16).contiguous()
        qkv, rest = _pair_projection(x2, wa, B, N, H, D)
        o = torch.empty((R, hc), device=dev, dtype=torch.bfloat16)
        og = torch.empty_like(o)
        lse = torch.empty((B, N, H, N), device=dev, dtype=torch.float32)
        ws_bytes = int(_native.query("tpf_attn_pair_forward_workspace_bytes", B, N, H))
        ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
        scale = 1.0 / math.sqrt(D)
        # Shadow residual of o (the facade's OPENFOLD3_SR_SHADOW policy): the
        # backward's delta then sees o's f32 value.
        res = torch.empty_like(o) if shadow_enabled() else None
        with _device_ctx(dev):
            _native.call("tpf_attn_pair_forward_bf16", qkv.data_ptr(), rest.data_ptr(),
                         rest.shape[1], mask_add.data_ptr(), _pair_flags(transpose_bias, og_t),
                         o.data_ptr(), lse.data_ptr(), og.data_ptr(), _native.ptr(res),
                         ws.data_ptr(), ws_bytes, B, N, H, D, scale, _native.stream_of(o))
        out = _mm(og, wo, True)
        ctx.save_for_backward(x2, wa, wo, qkv, rest, o, og, lse, mask_add, res)
        ctx.dims = (B, N, H, D, C, P, _pair_flags(transpose_bias, og_t), scale)
        ctx.w_dtypes = (w_all.dtype, w_o.dtype)
        ctx.set_materialize_grads(False)
        return out.view(B, N, N, C)

    @staticmethod
    def backward(ctx, dout):
        if dout is None:
            return (None,) * 8
        x2, wa, wo, qkv, rest, o, og, lse, mask_add, res = ctx.saved_tensors
        B, N, H, D, C, P, flags, scale = ctx.dims
        R = B * N * N
        dev = x2.device
        dout2 = dout.reshape(R, C).to(torch.bfloat16).contiguous()
        dw_o = _wgrad(dout2, og, ctx.w_dtypes[1]) if ctx.needs_input_grad[2] else None
        dproj = torch.empty((R, P), device=dev, dtype=torch.bfloat16)
        ws_bytes = int(_native.query("tpf_attn_pair_backward_workspace_bytes", B, N, H, D))
        ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
        common = (qkv.data_ptr(), rest.data_ptr(), rest.shape[1], mask_add.data_ptr(), flags,
                  o.data_ptr(), lse.data_ptr(), _native.ptr(res))
        tail = (dproj.data_ptr(), P, ws.data_ptr(), ws_bytes, B, N, H, D, scale,
                _native.stream_of(dproj))
        with _device_ctx(dev):
            if _native.query("tpf_attn_pair_backward_dout_supported", C, H, D):
                # d_og = dout W_o with the gate backward in its epilogue.
                _native.call("tpf_attn_pair_backward_dout_bf16", *common, dout2.data_ptr(),
                             wo.data_ptr(), C, *tail)
            else:
                d_og = _mm(dout2, wo, False)
                _native.call("tpf_attn_pair_backward_bf16", *common, d_og.data_ptr(), *tail)
        dx = _mm(dproj, wa, False).view(B, N, N, C) if ctx.needs_input_grad[0] else None
        dw_all = _wgrad(dproj, x2, ctx.w_dtypes[0]) if ctx.needs_input_grad[1] else None
        return dx, dw_all, dw_o, None, None, None, None, None


class _ProjLinear(torch.autograd.Function):
    """y = x W^T for BF16 activations over B*N^2 rows, whose weight gradient
    dW = dy^T x (K = rows) runs on the split-K MFMA GEMM (tpf_wgrad_bf16)."""

    @staticmethod
    def forward(ctx, x, w):
        wb = w.to(x.dtype)
        ctx.save_for_backward(x, wb)
        ctx.w_dtype = w.dtype
        return _mm(x.reshape(-1, x.shape[-1]), wb, True).view(*x.shape[:-1], wb.shape[0])

    @staticmethod
    def backward(ctx, dy):
        x, wb = ctx.saved_tensors
        dx = dw = None
        if ctx.needs_input_grad[0]:
            dx = _mm(dy.reshape(-1, dy.shape[-1]).to(torch.bfloat16), wb, False).view(
                *dy.shape[:-1], wb.shape[1])
        if ctx.needs_input_grad[1]:
            M, K = wb.shape
            dy2 = dy.reshape(-1, M).to(torch.bfloat16).contiguous()
            dw = _wgrad(dy2, x.reshape(-1, K).contiguous(), ctx.w_dtype)
        return dx, dw


def _mm_f32(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """``a [R, K] @ b.t()`` for FP32 ``b [N, K]`` on the FP32 MFMA GEMM
    (``tpf_gemm_f32``, strict FP32: no TF32-style rounding)."""
    a = a.contiguous()
    b = b.contiguous()
    R, K = a.shape
    N = b.shape[0]
    out = torch.empty((R, N), device=a.device, dtype=torch.float32)
    with _device_ctx(a.device):
        _native.call("tpf_gemm_f32", a.data_ptr(), 1, K, 0, b.data_ptr(), 1, K, 0, out.data_ptr(),
                     N, 0, R, N, K, 1, 1.0, None, _native.stream_of(a))
    return out


def _linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """Projection over the pair rows on the MFMA GEMMs: BF16 activations
    (feature sizes multiples of 8) with the split-K weight gradient under
    autograd, FP32 inference on the FP32 GEMM; anything else (CPU, other
    dtypes or sizes) takes torch.  Each output row depends only on its input
    row, so row chunks give the same bits."""
    if x.is_cuda and x.numel() > 0 and w.shape[0] % 8 == 0 and w.shape[1] % 8 == 0:
        if x.dtype == torch.bfloat16:
            if torch.is_grad_enabled():
                return _ProjLinear.apply(x, w)
            y = _mm(x.reshape(-1, x.shape[-1]), w.to(torch.bfloat16), True)
            return y.view(*x.shape[:-1], w.shape[0])
        if x.dtype == torch.float32 and not torch.is_grad_enabled() and w.dtype == torch.float32:
            return _mm_f32(x.reshape(-1, x.shape[-1]), w).view(*x.shape[:-1], w.shape[0])
    return nn.functional.linear(x, w.to(x.dtype))


class _MHA(nn.Module):
    """The parameter container of OpenFold3's ``Attention`` for triangle
    attention (no biases, gating on): linear_{q,k,v,o,g}."""

    def __init__(self, c_in: int, c_hidden: int, no_heads: int):
        super().__init__()
        self.c_hidden = c_hidden
        self.no_heads = no_heads
        self.linear_q = nn.Linear(c_in, c_hidden * no_heads, bias=False)
        self.linear_k = nn.Linear(c_in, c_hidden * no_heads, bias=False)
        self.linear_v = nn.Linear(c_in, c_hidden * no_heads, bias=False)
        self.linear_o = nn.Linear(c_hidden * no_heads, c_in, bias=False)
        self.linear_g = nn.Linear(c_in, c_hidden * no_heads, bias=False)


class TriangleAttention(nn.Module):
    """Triangle attention around the starting (or ending) node."""

    def __init__(self, c_in: int, c_hidden: int, no_heads: int, starting: bool = True,
                 inf: float = 1e9):
        super().__init__()
        self.c_in = c_in
        self.c_hidden = c_hidden
        self.no_heads = no_heads
        self.starting = starting
        self.inf = inf
        self.layer_norm = nn.LayerNorm(c_in)
        self.linear_z = nn.Linear(c_in, no_heads, bias=False)
        self.mha = _MHA(c_in, c_hidden, no_heads)

    def forward(self, x: torch.Tensor, mask: torch.Tensor | None = None,
                transpose_bias: bool = False, chunk_size: int | None = None,
                use_deepspeed_evo_attention: bool = False,
                use_cueq_triangle_kernels: bool = False,
                use_triton_triangle_kernels: bool = False,
                use_stable_triangle_attention: bool = True, use_lma: bool = False,
                inplace_safe: bool = False,
                use_protenix_triangle_attention: bool = False) -> torch.Tensor:
        """x: [*, I, J, C_in]; mask: [*, I, J] (1 keep, 0 drop).

        ``chunk_size`` (inference only on the stable route, as the reference's
        ``triangular_attention.py:114-158, 322-327``) runs the projections,
        attention, gate and output projection over chunks of outer rows with
        the full pair bias; the output is bitwise the unchunked one.
        ``inplace_safe`` only saves memory in the reference and is accepted.
        """
        _reject_backends(use_deepspeed_evo_attention=use_deepspeed_evo_attention,
                         use_cueq_triangle_kernels=use_cueq_triangle_kernels,
                         use_triton_triangle_kernels=use_triton_triangle_kernels,
                         use_lma=use_lma,
                         use_protenix_triangle_attention=use_protenix_triangle_attention)
        if mask is None:
            mask = x.new_ones(x.shape[:-1])
        if not self.starting:
            x = x.transpose(-2, -3)
            mask = mask.transpose(-1, -2)
        if self._stable_route(x, use_stable_triangle_attention):
            if chunk_size is not None:
                if chunk_size < 1:
                    raise ValueError("chunk_size must be positive")
                if torch.is_grad_enabled() and (x.requires_grad or any(
                        p.requires_grad for p in self.parameters())):
                    raise ValueError(
                        "stable Triangle Attention chunking is inference-only; "
                        "use eval() with gradients disabled outside checkpointing")
            out = self._stable_forward(x, mask, transpose_bias, chunk_size)
        else:
            out = self._stock_forward(x, mask, transpose_bias)
        if not self.starting:
            out = out.transpose(-2, -3)
        return out

    def _stable_route(self, x: torch.Tensor, use_stable: bool) -> bool:
        """The reference's route choice (``attention.py:520-595``)."""
        if not use_stable:
            return False
        native_fp32_inference = _fp32_inference(x)
        if _fp32_compute(x) and not native_fp32_inference and \
                not routing.tpf_bf16_cast_for_fp32_training():
            return False
        reasons = []
        if not x.is_cuda:
            reasons.append("requires GPU inputs")
        if self.c_hidden > 64:
            reasons.append("head dimension exceeds 64")
        if x.shape[-2] < (1 if native_fp32_inference else 2):
            reasons.append("sequence length is below 2")
        if reasons:
            if native_fp32_inference:
                raise ValueError("unsupported TurboPairFormer FP32 inference attention: "
                                 + "; ".join(reasons))
            routing.report_fallback(type(self).__qualname__, tuple(x.shape), "; ".join(reasons))
            return False
        return True

    def _stock_forward(self, x, mask, transpose_bias):
        """The stock module math (``triangular_attention.py:352-409`` with
        ``Attention._prep_qkv`` / ``_wrap_up``): softmax in FP32."""
        routing.note_stock_call()
        m = self.mha
        H, c = m.no_heads, m.c_hidden
        x = _stock_layer_norm(self.layer_norm, x)
        mask_bias = (self.inf * (mask.to(x.dtype) - 1))[..., :, None, None, :]
        zb = _stock_linear(self.linear_z, x)
        tri = zb.permute(*range(zb.dim() - 3), *(zb.dim() + p for p in
                                                  ((-1, -2, -3) if transpose_bias else (-1, -3, -2))))
        tri = tri.unsqueeze(-4)

        def heads(t):
            return t.reshape(t.shape[:-1] + (H, c)).transpose(-2, -3)

        q = heads(_stock_linear(m.linear_q, x)) / math.sqrt(c)
        k, v = heads(_stock_linear(m.linear_k, x)), heads(_stock_linear(m.linear_v, x))
        s = (q @ k.transpose(-1, -2)).float() + mask_bias.float() + tri.float()
        o = (torch.softmax(s, -1).to(v.dtype) @ v).transpose(-2, -3)
        g = torch.sigmoid(_stock_linear(m.linear_g, x)).reshape(o.shape)
        return _stock_linear(m.linear_o, (o * g).flatten(-2))

    def _stable_forward(self, x, mask, transpose_bias, chunk_size=None):
        x = _layer_norm(self.layer_norm, x)
        mask_bias = (self.inf * (mask.float() - 1))[..., :, None, None, :]
        m = self.mha
        H, c = m.no_heads, m.c_hidden
        if chunk_size is not None and chunk_size < x.shape[-3]:
            return self._chunked_forward(x, mask_bias, transpose_bias, chunk_size)
        # One projection GEMM for q, k, v, the gate and the pair bias.  Rows are
        # padded to a multiple of 64 outputs (128-byte aligned projection rows
        # for the pair-row core) or of 8 (per-projection route); the pad
        # outputs are unused.
        hc = H * c
        prefix = x.shape[:-3]
        N = x.shape[-2]
        pair_core = (x.dtype == torch.bfloat16 and x.is_cuda and x.shape[-3] == N
                     and N % 64 == 0 and c % 8 == 0 and 8 <= c <= 64 and H <= 16
                     and self.c_in % 8 == 0 and x.numel() > 0)
        pad = (-(4 * hc + H)) % (64 if pair_core else 8)
        w_all = torch.cat([m.linear_q.weight, m.linear_k.weight, m.linear_v.weight,
                           m.linear_g.weight, self.linear_z.weight]
                          + ([self.linear_z.weight.new_zeros(pad, self.c_in)] if pad else []))
        if pair_core:
            B = math.prod(prefix)
            mask_add = mask_bias.reshape(B, N, N).contiguous()
            # The ending node's x is the transposed view of the caller's
            # pair rows: the core returns its output in the caller's order,
            # handed back as the transposed view the caller transposes again
            # (no copy, and a contiguous result).
            og_t = not self.starting
            out = _PairAttentionCore.apply(x.reshape(B, N, N, self.c_in), w_all,
                                           m.linear_o.weight, mask_add, H, c,
                                           bool(transpose_bias), og_t)
            out = out.reshape(x.shape)
            return out.transpose(-2, -3) if og_t else out
        proj = _linear(x, w_all)
        # split (not slicing): its backward is one concatenation of the part
        # gradients instead of a zero-filled full-size buffer per part.
        qp, kp, vp, gp, zb, *_ = torch.split(proj, [hc, hc, hc, hc, H] + ([pad] if pad else []), -1)
        perm = (-1, -2, -3) if transpose_bias else (-1, -3, -2)
        tri_bias = zb.permute(*range(zb.dim() - 3), *(zb.dim() + p for p in perm)).unsqueeze(-4)

        def heads(t):  # [*, I, J, H*c] -> [*, I, H, J, c]
            return t.reshape(t.shape[:-1] + (H, c)).transpose(-2, -3)

        q, k, v = heads(qp), heads(kp), heads(vp)
        o = self._attend(q, k, v, mask_bias, tri_bias, x.dtype, _fp32_inference(x))
        if o is None:
            return self._stock_forward_from_ln(x, mask_bias, tri_bias, q, k, v, gp)
        g = torch.sigmoid(gp).reshape(o.shape)
        return _linear((o * g).flatten(-2), m.linear_o.weight)

    def _attend(self, q, k, v, mask_bias, tri_bias, x_dtype, fp32_inference):
        """Attention core on sequence-major q / k / v views (or None when the
        bf16 kernel's verdict rejects the case)."""
        if fp32_inference:
            return turbopairformer_attention_fp32(q, k, v, mask_bias, tri_bias.float())
        args = (q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16), mask_bias,
                tri_bias.to(torch.bfloat16))
        ok, reason = is_turbopairformer_supported(*args)
        if not ok:
            routing.report_fallback(type(self).__qualname__, tuple(q.shape), reason)
            return None
        return turbopairformer_triangle_attention(*args).to(x_dtype)

    def _chunked_forward(self, x, mask_bias, transpose_bias, chunk_size):
        """Inference over chunks of outer rows (reference ``_chunk_stable``,
        ``triangular_attention.py:114-158``): the pair bias of every pair is
        projected once; each chunk projects its rows' q / k / v / gate, runs
        attention over its planes with the full bias, gates and projects its
        output rows.  Per-row GEMMs and per-plane attention make the output
        bitwise that of the unchunked call."""
        m = self.mha
        H, c = m.no_heads, m.c_hidden
        hc = H * c
        outer = x.shape[-3]
        zb = _linear(x, self.linear_z.weight) if H % 8 == 0 else None
        if zb is None:  # pad the bias projection to 8 outputs (16-byte rows)
            wz = torch.cat([self.linear_z.weight,
                            self.linear_z.weight.new_zeros((-H) % 8, self.c_in)])
            zb = _linear(x, wz)[..., :H]
        perm = (-1, -2, -3) if transpose_bias else (-1, -3, -2)
        tri_bias = zb.permute(*range(zb.dim() - 3), *(zb.dim() + p for p in perm)).unsqueeze(-4)
        w_qkvg = torch.cat([m.linear_q.weight, m.linear_k.weight, m.linear_v.weight,
                            m.linear_g.weight])
        fp32_inf = _fp32_inference(x)

        def heads(t):  # [*, I, J, H*c] -> [*, I, H, J, c]
            return t.reshape(t.shape[:-1] + (H, c)).transpose(-2, -3)

        out = None
        for start in range(0, outer, chunk_size):
            rows = slice(start, min(start + chunk_size, outer))
            xs = x[..., rows, :, :]
            proj = _linear(xs, w_qkvg)
            qp, kp, vp, gp = torch.split(proj, [hc, hc, hc, hc], -1)
            q, k, v = heads(qp), heads(kp), heads(vp)
            mb = mask_bias[..., rows, :, :, :]
            o = self._attend(q, k, v, mb, tri_bias, x.dtype, fp32_inf)
            if o is None:
                o_rows = self._stock_forward_from_ln(xs, mb, tri_bias, q, k, v, gp)
            else:
                g = torch.sigmoid(gp).reshape(o.shape)
                o_rows = _linear((o * g).flatten(-2), m.linear_o.weight)
            if out is None:
                out = o_rows.new_empty(x.shape[:-1] + (o_rows.shape[-1],))
            out[..., rows, :, :] = o_rows
        return out

    def _stock_forward_from_ln(self, x, mask_bias, tri_bias, q, k, v, gp):
        """Stock attention on projections already formed (the reference's
        fallback after a failed support verdict, ``attention.py:675-692``)."""
        routing.note_stock_call()
        c = self.mha.c_hidden
        s = ((q / math.sqrt(c)) @ k.transpose(-1, -2)).float() + mask_bias.float() + tri_bias.float()
        o = (torch.softmax(s, -1).to(v.dtype) @ v).transpose(-2, -3)
        g = torch.sigmoid(gp).reshape(o.shape)
        return _linear((o * g).flatten(-2), self.mha.linear_o.weight)


TriangleAttentionStartingNode = TriangleAttention


class TriangleAttentionEndingNode(TriangleAttention):
    """Triangle attention around the ending node (``triangular_attention.py:413``)."""

    def __init__(self, c_in: int, c_hidden: int, no_heads: int, inf: float = 1e9):
        super().__init__(c_in, c_hidden, no_heads, starting=False, inf=inf)


class TriangleMultiplicativeUpdate(nn.Module):
    """Triangle multiplicative update (outgoing or incoming edges)."""

    def __init__(self, c_z: int, c_hidden: int, _outgoing: bool = True):
        super().__init__()
        self.c_z = c_z
        self.c_hidden = c_hidden
        self._outgoing = _outgoing
        # Registration order of the stock module: linear_g, linear_z, the two
        # LayerNorms, then the four branch projections.
        self.linear_g = nn.Linear(c_z, c_z, bias=False)
        self.linear_z = nn.Linear(c_hidden, c_z, bias=False)
        self.layer_norm_in = nn.LayerNorm(c_z)
        self.layer_norm_out = nn.LayerNorm(c_hidden)
        self.linear_a_p = nn.Linear(c_z, c_hidden, bias=False)
        self.linear_a_g = nn.Linear(c_z, c_hidden, bias=False)
        self.linear_b_p = nn.Linear(c_z, c_hidden, bias=False)
        self.linear_b_g = nn.Linear(c_z, c_hidden, bias=False)

    def forward(self, z: torch.Tensor, mask: torch.Tensor | None = None,
                inplace_safe: bool = False, use_cueq_triangle_kernels: bool = False,
                use_triton_triangle_kernels: bool = False,
                use_stable_triangle_multiplicative: bool = True,
                _add_with_inplace: bool = False,
                _inplace_chunk_size: int | None = 256) -> torch.Tensor:
        """z: [*, N, N, C_z]; mask: [*, N, N].  Returns the update; the stock
        route with ``inplace_safe`` and ``_add_with_inplace`` returns z + update
        (the reference overwrites z with it)."""
        _reject_backends(use_cueq_triangle_kernels=use_cueq_triangle_kernels,
                         use_triton_triangle_kernels=use_triton_triangle_kernels)
        if use_stable_triangle_multiplicative:
            # FP32 inference owns the site (triangular_multiplicative_update.py:64-84):
            # unsupported metadata raises instead of falling back.
            if z.is_cuda and _fp32_inference(z) and _fp32_compute(z):
                return run_trimul_fp32(self, z, mask)
            ok, reason = check_stable_trimul_support(self, z, mask)
            if ok:
                return run_stable_trimul(self, z, mask)
            routing.report_fallback(type(self).__qualname__, tuple(z.shape), reason)
        out = self._stock_forward(z, mask)
        if inplace_safe and _add_with_inplace:
            out = z + out
        return out

    def _stock_forward(self, z, mask):
        """The stock module math (``triangular_multiplicative_update.py:1262-1284``)."""
        routing.note_stock_call()
        if mask is None:
            mask = z.new_ones(z.shape[:-1])
        mask = mask.to(z.dtype).unsqueeze(-1)
        zl = _stock_layer_norm(self.layer_norm_in, z)
        a = mask * torch.sigmoid(_stock_linear(self.linear_a_g, zl)) * _stock_linear(self.linear_a_p, zl)
        b = mask * torch.sigmoid(_stock_linear(self.linear_b_g, zl)) * _stock_linear(self.linear_b_p, zl)
        eq = "...ikc,...jkc->...ijc" if self._outgoing else "...kic,...kjc->...ijc"
        x = torch.einsum(eq, a.float(), b.float()).to(z.dtype)
        x = _stock_layer_norm(self.layer_norm_out, x)
        return _stock_linear(self.linear_z, x) * torch.sigmoid(_stock_linear(self.linear_g, zl))


class TriangleMultiplicationOutgoing(TriangleMultiplicativeUpdate):
    def __init__(self, c_z: int, c_hidden: int):
        super().__init__(c_z, c_hidden, _outgoing=True)


class TriangleMultiplicationIncoming(TriangleMultiplicativeUpdate):
    def __init__(self, c_z: int, c_hidden: int):
        super().__init__(c_z, c_hidden, _outgoing=False)


__all__ = [
    "TriangleAttention",
    "TriangleAttentionEndingNode",
    "TriangleAttentionStartingNode",
    "TriangleMultiplicationIncoming",
    "TriangleMultiplicationOutgoing",
    "TriangleMultiplicativeUpdate",
]
