"""Pin the attention oracle: hand-derived backward vs torch autograd of an
independent forward, and the invariants the kernels must honour."""

import math

import numpy as np
import pytest
import torch

from oracle.attention import attention_backward, attention_forward
from tests._util import attention_case


def _torch_attention(q, k, v, mask, bias):
    # Literal restatement of attention.py:176-217 with q pre-scaled (:347-368),
    # -inf masks mapped to a large finite value as in aot_numeric_smoke.py:30-36.
    mask = torch.where(torch.isinf(mask), torch.full_like(mask, -1e4), mask)
    s = torch.einsum("...qc,...kc->...qk", q / math.sqrt(q.shape[-1]), k) + mask + bias
    return torch.einsum("...qk,...kc->...qc", torch.softmax(s, -1), v).transpose(-2, -3)


@pytest.mark.parametrize("shape,kw", [
    ((1, 3, 2, 16, 8), dict(mask_frac=0.25)),
    ((2, 2, 3, 24, 12), dict(mask_tail=5)),
])
def test_backward_matches_autograd(shape, kw):
    q, k, v, mask, bias, dout = attention_case(*shape, **kw, seed=11)
    tq, tk, tv, tb = (t.double().requires_grad_(True) for t in (q, k, v, bias))
    out = _torch_attention(tq, tk, tv, mask.double(), tb)
    out.backward(dout.double())
    o, _, _ = attention_forward(q, k, v, mask, bias)
    grads = attention_backward(q, k, v, mask, bias, dout)
    np.testing.assert_allclose(o, out.detach().numpy(), rtol=1e-9, atol=1e-10)
    for g, t in zip(grads, (tq, tk, tv, tb)):
        np.testing.assert_allclose(g, t.grad.numpy(), rtol=1e-8, atol=1e-10)


def test_brute_force_tiny():
    rng = np.random.default_rng(0)
    q, k, v = (rng.standard_normal((1, 1, 1, 3, 2)) for _ in range(3))
    mask = np.array([0.0, -np.inf, 0.0]).reshape(1, 1, 1, 1, 3)
    bias = rng.standard_normal((1, 1, 1, 3, 3))
    out, lse, _ = attention_forward(q, k, v, mask, bias)
    for i in range(3):
        s = [q[0, 0, 0, i] @ k[0, 0, 0, j] / math.sqrt(2) + bias[0, 0, 0, i, j] for j in (0, 2)]
        w = np.exp(s) / np.exp(s).sum()
        np.testing.assert_allclose(out[0, 0, i, 0], w[0] * v[0, 0, 0, 0] + w[1] * v[0, 0, 0, 2])
        np.testing.assert_allclose(lse[0, 0, 0, i], np.log(np.exp(s).sum()))


def test_fully_masked_rows_give_zero_output_and_grads():
    q, k, v, mask, bias, dout = (t.numpy() for t in attention_case(1, 3, 2, 16, 8, full_planes=1))
    out, lse, _ = attention_forward(q, k, v, mask, bias)
    assert np.all(out[:, 0] == 0) and np.all(np.isneginf(lse[:, 0]))
    dq, dk, dv, _ = attention_backward(q, k, v, mask, bias, dout)
    for g in (dq, dk, dv):
        assert np.all(g[:, 0] == 0)


def test_dbias_is_sum_over_outer_rows():
    q, k, v, mask, bias, dout = (t.numpy() for t in attention_case(2, 3, 2, 8, 4, mask_frac=0.2))
    _, _, _, db = attention_backward(q, k, v, mask, bias, dout)
    acc = np.zeros_like(db)
    for b in range(2):
        for o in range(3):
            sl = (slice(b, b + 1), slice(o, o + 1))
            *_, dbo = attention_backward(q[sl], k[sl], v[sl], mask[sl], bias, dout[sl])
            acc += dbo
    np.testing.assert_allclose(db, acc, rtol=1e-10, atol=1e-12)


def test_ending_node_is_starting_node_on_transposed_pair():
    # TriangleAttention ending node = starting node on z^T (triangular_attention.py:358-360,406-407)
    from oracle.modules import triangle_attention_module

    rng = np.random.default_rng(1)
    C, c, H = 16, 4, 2
    params = {"layer_norm_w": rng.standard_normal(C), "layer_norm_b": rng.standard_normal(C),
              "linear_z": rng.standard_normal((H, C)) * 0.3}
    for n in ("linear_q", "linear_k", "linear_v", "linear_g"):
        params[n] = rng.standard_normal((H * c, C)) * 0.3
    params["linear_o"] = rng.standard_normal((C, H * c)) * 0.3
    x = rng.standard_normal((1, 6, 6, C))
    end = triangle_attention_module(x, params, H, starting=False)
    start_t = triangle_attention_module(np.swapaxes(x, 1, 2), params, H, starting=True)
    np.testing.assert_allclose(end, np.swapaxes(start_t, 1, 2), rtol=1e-12, atol=1e-12)


def test_padding_invariance():
    q, k, v, mask, bias, dout = (t.numpy() for t in attention_case(1, 2, 2, 10, 8, mask_frac=0.2))
    out, _, _ = attention_forward(q, k, v, mask, bias)
    def pad(t, axis, n):
        widths = [(0, 0)] * t.ndim
        widths[axis] = (0, n)
        return np.pad(t, widths)
    qp, kp, vp = (pad(t, -2, 6) for t in (q, k, v))
    mp = np.concatenate([mask, np.full(mask.shape[:-1] + (6,), -np.inf)], -1)
    bp = pad(pad(bias, -1, 6), -2, 6)
    outp, _, _ = attention_forward(qp, kp, vp, mp, bp)
    np.testing.assert_allclose(outp[:, :, :10], out, rtol=1e-12, atol=1e-12)
