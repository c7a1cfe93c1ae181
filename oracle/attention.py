"""Triangle attention oracle (numpy) -- TEST INFRASTRUCTURE ONLY.

Restates the reference's triangle attention math:
  * stock OpenFold3 attention core ``_attention``
    (openfold3/core/model/primitives/attention.py:176-217) with the scale of
    ``_prep_qkv`` (:347-368) applied to Q and the output transpose of
    ``Attention.forward`` (:732);
  * the FP64 oracle of the release smoke tool
    (tools/aot_numeric_smoke.py:39-48), autograd gradients in closed form;
  * the kernel contract for fully masked rows
    (turbopairformer_triangle_forward.cu:35-37, 431-433): output 0, LSE -inf,
    and therefore zero gradients.

Shapes: q, k, v ``[*B, O, H, N, D]``; res_mask ``[*B, O, 1, 1, N]``;
pair_bias ``[*Bb, 1, H, N, N]`` broadcastable to the prefix; output
``[*B, O, N, H, D]``; lse ``[*B, O, H, N]``.

Parity pinning: see oracle/__init__.py and tests/test_oracle_attention.py.
"""

from __future__ import annotations

import numpy as np


def _swap(x: np.ndarray) -> np.ndarray:
    return np.swapaxes(x, -1, -2)


def attention_forward(q, k, v, res_mask, pair_bias, scale=None, dtype=np.float64):
    """Return (out [*B,O,N,H,D], lse [*B,O,H,N], p [*B,O,H,N,N]).

    ``scale`` defaults to 1/sqrt(D) (q is unscaled, as in the reference
    contract ``turbopairformer_triangle_attention.py:15-17``).
    """
    q, k, v = (np.asarray(t, dtype=dtype) for t in (q, k, v))
    mask = np.asarray(res_mask, dtype=dtype)
    bias = np.asarray(pair_bias, dtype=dtype)
    d = q.shape[-1]
    if scale is None:
        scale = 1.0 / np.sqrt(d)
    s = np.matmul(q, _swap(k)) * dtype(scale)
    s = s + mask + bias  # mask [...,O,1,1,N], bias [...,1,H,N,N]
    m = s.max(axis=-1, keepdims=True)
    full = ~np.isfinite(m)
    m_safe = np.where(full, 0.0, m).astype(dtype)
    with np.errstate(invalid="ignore"):
        e = np.exp(s - m_safe)
    e = np.where(np.isnan(e), 0.0, e).astype(dtype)
    l = e.sum(axis=-1, keepdims=True)
    with np.errstate(invalid="ignore", divide="ignore"):
        p = np.where(l > 0, e / np.where(l > 0, l, 1.0), 0.0).astype(dtype)
    o = np.matmul(p, v)  # [..., O, H, N, D]
    out = np.swapaxes(o, -2, -3)  # [..., O, N, H, D]
    with np.errstate(divide="ignore"):
        lse = np.where(l[..., 0] > 0, m_safe[..., 0] + np.log(np.where(l[..., 0] > 0, l[..., 0], 1.0)), -np.inf)
    return out, lse.astype(dtype), p


def _reduce_to(grad: np.ndarray, shape: tuple) -> np.ndarray:
    """Sum a broadcast gradient back to ``shape`` (numpy broadcasting rules)."""
    lead = grad.ndim - len(shape)
    if lead:
        grad = grad.sum(axis=tuple(range(lead)))
    axes = tuple(i for i, s in enumerate(shape) if s == 1 and grad.shape[i] != 1)
    if axes:
        grad = grad.sum(axis=axes, keepdims=True)
    return grad


def attention_backward(q, k, v, res_mask, pair_bias, d_out, scale=None, dtype=np.float64):
    """Return (dq, dk, dv, dbias) for loss = <d_out, out>.

    Closed form of the autograd graph of ``attention_forward``:
    dV = P^T dO, dP = dO V^T, delta = rowsum(dO * O), dS = P (dP - delta),
    dQ = scale dS K, dK = scale dS^T Q, dBias = sum over broadcast axes of dS.
    """
    q, k, v = (np.asarray(t, dtype=dtype) for t in (q, k, v))
    d = q.shape[-1]
    if scale is None:
        scale = 1.0 / np.sqrt(d)
    out, _, p = attention_forward(q, k, v, res_mask, pair_bias, scale, dtype)
    do = np.swapaxes(np.asarray(d_out, dtype=dtype), -2, -3)  # [..., O, H, N, D]
    o = np.swapaxes(out, -2, -3)
    dv = np.matmul(_swap(p), do)
    dp = np.matmul(do, _swap(v))
    delta = (do * o).sum(axis=-1, keepdims=True)
    ds = p * (dp - delta)
    dq = np.matmul(ds, k) * dtype(scale)
    dk = np.matmul(_swap(ds), q) * dtype(scale)
    dbias = _reduce_to(ds, np.shape(pair_bias))
    return dq, dk, dv, dbias


def attention_flops(B, O, H, N, D) -> dict:
    """Algorithmic matmul flops: fwd 4*P*N^2*D, bwd 10*P*N^2*D (P = B*O*H)."""
    planes = B * O * H
    fwd = 4.0 * planes * N * N * D
    bwd = 10.0 * planes * N * N * D
    return {"fwd": fwd, "bwd": bwd, "total": fwd + bwd}
