"""The Python boundary on CPU with a fake native backend.

As in the reference's fake-backend route test
(openfold3/tests/core/kernels/test_turbopairformer_sr_policy.py:68-132), the
native calls are replaced: here by a fake that evaluates the numpy oracle on
the raw buffers the facade hands to the C ABI.  This checks the host logic --
validation, D/N padding, storage orders, batch flattening, bias broadcast and
gradient routing -- end to end without a GPU.
"""

import ctypes
import math

import numpy as np
import pytest
import torch

from oracle.attention import attention_backward, attention_forward
from tests._util import attention_case, max_rel


def _arr(ptr, shape, dtype):
    n = int(np.prod(shape))
    ct = {np.uint16: ctypes.c_uint16, np.float32: ctypes.c_float}[dtype]
    return np.ctypeslib.as_array(ctypes.cast(ptr, ctypes.POINTER(ct)), (n,)).reshape(shape)


def _bf2f(a):
    return (a.astype(np.uint32) << 16).view(np.float32)


def _f2bf(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


class FakeBackend:
    """Implements the attention entry points on host memory with the oracle."""

    def __init__(self):
        self.calls = []
        self.layouts = []
        self.shadow = []

    def _bias(self, ptr, Bb, H, N, layout):
        b = _bf2f(_arr(ptr, (Bb, H, N, N), np.uint16))
        if layout & 2:  # TPF_BIAS_TRANSPOSED: storage holds bias[..., k, q]
            b = np.swapaxes(b, -1, -2)
        return b[:, None]

    def _qkv(self, ptr, B, O, H, N, D, seq_major):
        if seq_major:
            return np.swapaxes(_bf2f(_arr(ptr, (B, O, N, H, D), np.uint16)), 2, 3)
        return _bf2f(_arr(ptr, (B, O, H, N, D), np.uint16))

    def __call__(self, name, *a):
        self.calls.append(name)
        if name in ("tpf_attn_forward_bf16", "tpf_attn_forward_shadow_bf16"):
            if name == "tpf_attn_forward_bf16":
                q, k, v, mask, bias, out, lse, ws, wsb, B, O, H, N, D, sm, Bb, scale, _ = a
                res = None
            else:
                q, k, v, mask, bias, out, lse, res, ws, wsb, B, O, H, N, D, sm, Bb, scale, _ = a
            Q, K, V = (self._qkv(p, B, O, H, N, D, sm & 1) for p in (q, k, v))
            M = _arr(mask, (B, O, N), np.float32).reshape(B, O, 1, 1, N)
            Bi = self._bias(bias, Bb, H, N, sm)
            o, l, _ = attention_forward(Q, K, V, M, Bi, scale=scale)
            ob = _f2bf(o)
            _arr(out, (B, O, N, H, D), np.uint16)[...] = ob
            _arr(lse, (B, O, H, N), np.float32)[...] = l
            if res is not None:
                _arr(res, (B, O, N, H, D), np.uint16)[...] = _f2bf(o.astype(np.float32) - _bf2f(ob))
        elif name in ("tpf_attn_delta_bf16", "tpf_attn_delta_shadow_bf16"):
            if name == "tpf_attn_delta_bf16":
                do, out, delta, B, O, H, N, D, _ = a
                res = None
            else:
                do, out, res, delta, B, O, H, N, D, _ = a
            dO = _bf2f(_arr(do, (B, O, N, H, D), np.uint16))
            Ov = _bf2f(_arr(out, (B, O, N, H, D), np.uint16))
            if res is not None:
                Ov = Ov + _bf2f(_arr(res, (B, O, N, H, D), np.uint16))
            _arr(delta, (B, O, H, N), np.float32)[...] = np.swapaxes((dO * Ov).sum(-1), 2, 3)
        elif name in ("tpf_attn_backward_bf16", "tpf_attn_backward_fused_bf16"):
            if name == "tpf_attn_backward_bf16":
                (q, k, v, do, lse, delta, mask, bias, dq, dk, dv, dbias, ws, wsb, B, O, H, N, D,
                 sm, Bb, scale, _) = a
            else:
                (q, k, v, do, out, res, lse, mask, bias, dq, dk, dv, dbias, ws, wsb, B, O, H, N,
                 D, sm, Bb, scale, _) = a
                self.shadow.append(bool(res))
            Q, K, V = (self._qkv(p, B, O, H, N, D, sm & 1) for p in (q, k, v))
            M = _arr(mask, (B, O, N), np.float32).reshape(B, O, 1, 1, N)
            Bi = self._bias(bias, Bb, H, N, sm)
            self.layouts.append(sm)
            dO = _bf2f(_arr(do, (B, O, N, H, D), np.uint16))
            gq, gk, gv, gb = attention_backward(Q, K, V, M, Bi, dO, scale=scale)
            for ptr, g in ((dq, gq), (dk, gk), (dv, gv)):
                if sm & 1:
                    _arr(ptr, (B, O, N, H, D), np.uint16)[...] = _f2bf(np.swapaxes(g, 2, 3))
                else:
                    _arr(ptr, (B, O, H, N, D), np.uint16)[...] = _f2bf(g)
            if sm & 4:  # TPF_DBIAS_BF16: bf16 in the bias's storage order
                g = gb[:, 0].astype(np.float32)
                if sm & 2:
                    g = np.swapaxes(g, -1, -2)
                _arr(dbias, (Bb, H, N, N), np.uint16)[...] = _f2bf(g)
            else:
                _arr(dbias, (Bb, H, N, N), np.float32)[...] = gb[:, 0]
        else:
            raise AssertionError(name)
        return 0


@pytest.fixture
def fake(monkeypatch):
    from openfold3_triangle_kernel_amd import _native, attention

    backend = FakeBackend()
    monkeypatch.setattr(attention, "_device_supported", lambda t: (True, ""))
    monkeypatch.setattr(_native, "call", backend)
    monkeypatch.setattr(_native, "query", lambda name, *a: 256)
    attention._SUPPORT_CACHE.clear()
    yield backend
    attention._SUPPORT_CACHE.clear()


def _grads(q, k, v, mask, bias, dout, seq_major=False, bias_prefix=None):
    from openfold3_triangle_kernel_amd import turbopairformer_triangle_attention

    if seq_major:
        q, k, v = (t.transpose(-2, -3).contiguous().transpose(-2, -3) for t in (q, k, v))
    tq, tk, tv = (t.to(torch.bfloat16).detach().requires_grad_(True) for t in (q, k, v))
    tb = bias.to(torch.bfloat16).detach().requires_grad_(True)
    out = turbopairformer_triangle_attention(tq, tk, tv, mask, tb)
    out.backward(dout.to(torch.bfloat16))
    return [t.detach().float().numpy() for t in (out, tq.grad, tk.grad, tv.grad, tb.grad)]


@pytest.mark.parametrize("shape,seq_major", [((1, 3, 2, 20, 12), False), ((2, 2, 2, 64, 16), True),
                                             ((1, 2, 3, 70, 8), False)])
def test_facade_padding_and_layouts(fake, shape, seq_major):
    case = attention_case(*shape, mask_frac=0.2, seed=4)
    q, k, v, mask, bias, dout = case
    got = _grads(q, k, v, mask, bias, dout, seq_major)
    ref_o, _, _ = attention_forward(*(t.numpy() for t in (q, k, v, mask, bias)))
    ref = [ref_o, *attention_backward(*(t.numpy() for t in (q, k, v, mask, bias, dout)))]
    for g, r in zip(got, ref):
        assert g.shape == r.shape
        assert max_rel(g, r) < 1e-2
    assert fake.calls.count("tpf_attn_backward_fused_bf16") == 1


def test_facade_batch_prefix_and_broadcast_bias(fake):
    g = torch.Generator().manual_seed(2)
    B1, B2, O, H, N, D = 2, 2, 2, 2, 64, 8
    q, k, v = (torch.randn(B1, B2, O, H, N, D, generator=g).bfloat16().float() for _ in range(3))
    bias = torch.randn(B1, 1, 1, H, N, N, generator=g).bfloat16().float()  # broadcast over B2
    mask = torch.zeros(1, B2, O, 1, 1, N)
    dout = torch.randn(B1, B2, O, N, H, D, generator=g).bfloat16().float()
    got = _grads(q, k, v, mask, bias, dout)
    ref_o, _, _ = attention_forward(q.numpy(), k.numpy(), v.numpy(), mask.numpy(), bias.numpy())
    *_, ref_db = attention_backward(q.numpy(), k.numpy(), v.numpy(), mask.numpy(), bias.numpy(),
                                    dout.numpy())
    assert got[0].shape == (B1, B2, O, N, H, D)
    assert got[4].shape == tuple(bias.shape)
    assert max_rel(got[0], ref_o) < 1e-2
    assert max_rel(got[4], ref_db) < 1e-2


def test_fp32_bias_gets_fp32_grad(fake):
    q, k, v, mask, bias, dout = attention_case(1, 2, 2, 64, 8, seed=1)
    from openfold3_triangle_kernel_amd import turbopairformer_triangle_attention

    tq, tk, tv = (t.bfloat16().requires_grad_(True) for t in (q, k, v))
    tb = bias.clone().requires_grad_(True)
    out = turbopairformer_triangle_attention(tq, tk, tv, mask, tb)
    out.float().sum().backward()
    assert tb.grad.dtype == torch.float32 and tb.grad.shape == tb.shape


def test_invocation_count_and_turbo_attention_defaults(fake):
    from openfold3_triangle_kernel_amd import attention, turbo_attention

    before = attention.invocation_count()
    q, k, v, mask, bias, dout = attention_case(1, 2, 2, 64, 8, seed=1)
    out = turbo_attention(q.bfloat16(), k.bfloat16(), v.bfloat16(), pair_bias=bias.bfloat16())
    assert out.shape == (1, 2, 64, 2, 8)
    assert attention.invocation_count() == before + 1
    with pytest.raises(ValueError, match="pair_bias is required"):
        turbo_attention(q.bfloat16(), k.bfloat16(), v.bfloat16(), pair_bias=None)


@pytest.mark.parametrize("mutate,msg", [
    (lambda a: a.update(q=a["q"].half()), "BF16"),
    (lambda a: a.update(q=a["q"].float()), "FP32"),
    (lambda a: a.update(q=a["q"][..., :1, :, :]), "k shape must match q"),
    (lambda a: a.update(q=torch.zeros(1, 2, 2, 64, 72, dtype=torch.bfloat16),
                        k=torch.zeros(1, 2, 2, 64, 72, dtype=torch.bfloat16),
                        v=torch.zeros(1, 2, 2, 64, 72, dtype=torch.bfloat16)), "D<=64"),
    (lambda a: a.update(res_mask=a["res_mask"][..., :10]), "res_mask tail"),
    (lambda a: a.update(res_mask=a["res_mask"].bool()), "floating additive mask"),
    (lambda a: a.update(pair_bias=a["pair_bias"][..., :10]), "pair_bias tail"),
    (lambda a: a.update(res_mask=a["res_mask"].clone().requires_grad_(True)), "must not require"),
])
def test_unsupported_cases_raise_before_launch(fake, mutate, msg):
    from openfold3_triangle_kernel_amd import turbopairformer_triangle_attention

    q, k, v, mask, bias, _ = attention_case(1, 2, 2, 64, 8, seed=1)
    args = dict(q=q.bfloat16(), k=k.bfloat16(), v=v.bfloat16(), res_mask=mask, pair_bias=bias.bfloat16())
    mutate(args)
    with pytest.raises(ValueError, match=msg):
        turbopairformer_triangle_attention(**args)
    assert fake.calls == []


def test_sr_backward_flag_zero_raises(fake, monkeypatch):
    from openfold3_triangle_kernel_amd import turbopairformer_triangle_attention

    q, k, v, mask, bias, _ = attention_case(1, 2, 2, 64, 8, seed=1)
    monkeypatch.setenv("TURBOPAIRFORMER_SR_BACKWARD", "0")
    with pytest.raises(ValueError, match="SR_BACKWARD=0"):
        turbopairformer_triangle_attention(q.bfloat16(), k.bfloat16(), v.bfloat16(), mask, bias.bfloat16())
    monkeypatch.setenv("TURBOPAIRFORMER_SR_BACKWARD", "1")
    monkeypatch.setenv("OPENFOLD3_SR_BACKWARD", "0")  # canonical name takes precedence
    turbopairformer_triangle_attention(q.bfloat16(), k.bfloat16(), v.bfloat16(), mask, bias.bfloat16())


def test_product_path_fails_loudly_without_library(monkeypatch, tmp_path):
    from openfold3_triangle_kernel_amd import _native

    monkeypatch.setattr(_native, "LIB_PATH", tmp_path / "missing.so")
    monkeypatch.setattr(_native, "_LIB", None)
    with pytest.raises(RuntimeError, match="not built"):
        _native.library()


@pytest.mark.parametrize("canonical,legacy,expect_shadow", [
    (None, None, True),          # reference default: OPENFOLD3_SR_SHADOW=1
    (None, "0", False),
    ("1", "0", True),            # canonical name takes precedence
    ("0", None, False),
])
def test_shadow_residual_policy_routes_entry_points(fake, monkeypatch, canonical, legacy,
                                                    expect_shadow):
    """The shadow flag selects the residual-saving forward and the residual
    delta, as the reference's OPENFOLD3_SR_SHADOW does
    (turbopairformer_triangle_attention.py:247-262)."""
    for name, value in (("TURBOPAIRFORMER_SR_SHADOW", canonical), ("OPENFOLD3_SR_SHADOW", legacy)):
        if value is None:
            monkeypatch.delenv(name, raising=False)
        else:
            monkeypatch.setenv(name, value)
    case = attention_case(1, 2, 2, 64, 16, mask_frac=0.1, seed=9)
    got = _grads(*case)
    used = set(fake.calls)
    # The forward saves the residual and the fused backward's delta pairs it
    # with out (a non-null residual argument).
    assert ("tpf_attn_forward_shadow_bf16" in used) == expect_shadow
    assert ("tpf_attn_forward_bf16" in used) == (not expect_shadow)
    assert fake.shadow == [expect_shadow]
    q, k, v, mask, bias, dout = (t.numpy() for t in case)
    ref = attention_backward(q, k, v, mask, bias, dout)
    for g, r in zip(got[1:], ref):
        assert max_rel(g, r) <= 2e-2


def test_shadow_flag_rejects_other_values(fake, monkeypatch):
    monkeypatch.setenv("TURBOPAIRFORMER_SR_SHADOW", "yes")
    case = attention_case(1, 2, 2, 64, 16, seed=1)
    with pytest.raises(ValueError, match="SR_SHADOW"):
        _grads(*case)


def test_fp32_q_delegates_to_fp32_inference(monkeypatch):
    """FP32 q routes the verdict and the call to the FP32 implementation
    (reference turbopairformer_triangle_attention.py:144-150, 362-370)."""
    from openfold3_triangle_kernel_amd import attention, attention_fp32

    attention._SUPPORT_CACHE.clear()
    seen = {}
    monkeypatch.setattr(attention_fp32, "is_attention_fp32_supported",
                        lambda *a: (True, "fp32 verdict"))

    def fake_fp32(q, k, v, m, b):
        seen["called"] = True
        return torch.zeros(q.shape[:-3] + (q.shape[-2], q.shape[-3], q.shape[-1]))

    monkeypatch.setattr(attention_fp32, "turbopairformer_attention_fp32", fake_fp32)
    q = torch.randn(1, 2, 2, 8, 4)
    mask = torch.zeros(1, 2, 1, 1, 8)
    bias = torch.zeros(1, 1, 2, 8, 8)
    with torch.no_grad():
        assert attention.is_turbopairformer_supported(q, q, q, mask, bias) == (True, "fp32 verdict")
        out = attention.turbopairformer_triangle_attention(q, q, q, mask, bias)
    assert seen["called"] and out.shape == (1, 2, 8, 2, 4)
    attention._SUPPORT_CACHE.clear()


def test_transposed_bias_view_is_read_in_place(fake):
    """The ending node passes bias.transpose(-1, -2) of a contiguous tensor: the
    facade hands its storage to the kernels with TPF_BIAS_TRANSPOSED instead of
    copying it, and the gradient comes back in the view's shape."""
    from openfold3_triangle_kernel_amd import turbopairformer_triangle_attention

    q, k, v, mask, bias, dout = attention_case(1, 3, 2, 64, 16, mask_frac=0.1, seed=17)
    base = bias.transpose(-1, -2).contiguous().to(torch.bfloat16).requires_grad_(True)
    view = base.transpose(-1, -2)
    assert not view.is_contiguous()
    tq, tk, tv = (t.to(torch.bfloat16).requires_grad_(True) for t in (q, k, v))
    out = turbopairformer_triangle_attention(tq, tk, tv, mask, view)
    out.backward(dout.to(torch.bfloat16))
    assert fake.layouts and fake.layouts[-1] & 2
    ref_out, _, _ = attention_forward(q.numpy(), k.numpy(), v.numpy(), mask.numpy(),
                                      view.detach().float().numpy())
    ref = attention_backward(q.numpy(), k.numpy(), v.numpy(), mask.numpy(),
                             view.detach().float().numpy(), dout.numpy())
    assert max_rel(out.detach().float().numpy(), ref_out) <= 2e-2
    assert max_rel(base.grad.float().numpy(), np.swapaxes(ref[3], -1, -2)) <= 2e-2
