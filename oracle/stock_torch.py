"""Stock OpenFold3 PyTorch math, FP32, for the CPU baseline -- TEST INFRASTRUCTURE ONLY.

This is the path the kernels replace, restated with torch ops so that it can
be timed on the host cores beside the GPU (``bench.py``'s ``cpu_baseline``
leg) and pinned to the numpy oracle (tests/test_oracle_stock_torch.py).  The
product package never imports it.

* ``attention_stock``: OpenFold3's attention core ``_attention``
  (openfold3/core/model/primitives/attention.py:176-217) with q pre-scaled by
  1/sqrt(D) as ``_prep_qkv`` does (:347-368), the mask and pair bias as its
  two additive biases, and the output transposed to [*, O, N, H, D] as
  ``_wrap_up`` / ``attention_chunked_trainable`` do (:273-277).  With
  ``chunk`` set it runs outer-row chunks one after the other, the stock
  chunked path (:221-278); for a training step each chunk's forward and
  backward run together, so peak memory stays one chunk's scores.
* ``trimul_stock``: TriangleMultiplicativeUpdate's forward
  (openfold3/core/model/layers/triangular_multiplicative_update.py:1263-1284)
  with OpenFold3's LayerNorm (primitives/normalization.py:54-78; eps 1e-5).
"""

from __future__ import annotations

import math

import torch


def attention_stock(q, k, v, res_mask, pair_bias):
    """out [*, O, N, H, D] = softmax(q k^T / sqrt(D) + mask + bias) v."""
    scale = 1.0 / math.sqrt(q.shape[-1])
    s = torch.einsum("...qc,...kc->...qk", q * scale, k)
    s = s + res_mask
    s = s + pair_bias
    p = torch.softmax(s, dim=-1)
    o = torch.einsum("...qk,...kc->...qc", p, v)
    return o.transpose(-2, -3)


def attention_stock_train_step(q, k, v, res_mask, pair_bias, d_out, chunk=None):
    """Forward + backward of ``attention_stock`` with cotangent ``d_out``.

    Returns (out, dq, dk, dv, dbias).  ``chunk`` splits the outer dimension
    (dim -4 of q); dbias accumulates over chunks in chunk order.
    """
    O = q.shape[-4]
    chunk = chunk or O
    outs, dqs, dks, dvs = [], [], [], []
    dbias = torch.zeros_like(pair_bias)
    for s0 in range(0, O, chunk):
        sl = (Ellipsis, slice(s0, s0 + chunk), slice(None), slice(None), slice(None))
        qc, kc, vc = (t[sl].detach().requires_grad_(True) for t in (q, k, v))
        mc = res_mask[sl] if res_mask.shape[-4] != 1 else res_mask
        bc = pair_bias.detach().requires_grad_(True)
        out = attention_stock(qc, kc, vc, mc, bc)
        gq, gk, gv, gb = torch.autograd.grad(out, (qc, kc, vc, bc), d_out[sl])
        outs.append(out.detach())
        dqs.append(gq)
        dks.append(gk)
        dvs.append(gv)
        dbias += gb
    cat = lambda ts: torch.cat(ts, dim=-4)  # noqa: E731
    return cat(outs), cat(dqs), cat(dks), cat(dvs), dbias


def layer_norm(x, w, b, eps=1e-5):
    return torch.nn.functional.layer_norm(x, (x.shape[-1],), w, b, eps)


def trimul_stock(z, mask, w, outgoing):
    """TriMul forward; ``w`` holds w_ap, w_ag, w_bp, w_bg [H, C], w_g [C, C],
    w_z [C, H] and the LayerNorm affines g_in, b_in [C], g_out, b_out [H]."""
    zl = layer_norm(z, w["g_in"], w["b_in"])
    m = mask.unsqueeze(-1)
    a = m * torch.sigmoid(zl @ w["w_ag"].t()) * (zl @ w["w_ap"].t())
    b = m * torch.sigmoid(zl @ w["w_bg"].t()) * (zl @ w["w_bp"].t())
    eq = "...ikc,...jkc->...ijc" if outgoing else "...kic,...kjc->...ijc"
    x = torch.einsum(eq, a, b)
    x = layer_norm(x, w["g_out"], w["b_out"])
    return (x @ w["w_z"].t()) * torch.sigmoid(zl @ w["w_g"].t())
