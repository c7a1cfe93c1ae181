"""TriMul oracle (numpy): forward and hand-derived backward -- TEST INFRASTRUCTURE ONLY.

Restates the stock OpenFold3 triangle multiplicative update:
  * TriangleMultiplicativeUpdate.forward
    (openfold3/core/model/layers/triangular_multiplicative_update.py:1263-1284),
  * _combine_projections (:734-760): outgoing x[i,j] = sum_k a[i,k] b[j,k],
    incoming x[i,j] = sum_k a[k,i] b[k,j], per channel,
  * LayerNorm (openfold3/core/model/primitives/normalization.py:54-78),
    biased variance, eps 1e-5, computed in f32 or wider,
  * Linear without bias (openfold3/core/model/primitives/linear.py:138-143),
with the named-weight mapping of the cuEquivariance call site (:1228-1250).

The backward is derived by hand (chain rule through LN, gates, contraction)
and pinned against torch autograd of an independent torch forward in
tests/test_oracle_trimul.py.
"""

from __future__ import annotations

import numpy as np

EPS = 1e-5


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def layer_norm(x, w, b, eps=EPS):
    """Return (y, xhat, rstd) over the last axis."""
    mean = x.mean(axis=-1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
    rstd = 1.0 / np.sqrt(var + eps)
    xhat = (x - mean) * rstd
    return xhat * w + b, xhat, rstd


def layer_norm_backward(dy, xhat, rstd, w):
    """Return (dx, dw, db) of y = xhat*w + b for upstream dy (last-axis LN)."""
    g = dy * w
    dx = rstd * (g - g.mean(axis=-1, keepdims=True) - xhat * (g * xhat).mean(axis=-1, keepdims=True))
    red = tuple(range(dy.ndim - 1))
    return dx, (dy * xhat).sum(axis=red), dy.sum(axis=red)


def _contract(a, b, outgoing):
    """Channel-batched pair product via matmul on channel-first copies."""
    ac = np.moveaxis(a, -1, -3)  # [..., C, N, N]
    bc = np.moveaxis(b, -1, -3)
    if outgoing:
        x = ac @ np.swapaxes(bc, -1, -2)  # x_c = a_c b_c^T
    else:
        x = np.swapaxes(ac, -1, -2) @ bc  # x_c = a_c^T b_c
    return np.moveaxis(x, -3, -1)


def trimul_forward(z, mask, w, outgoing, dtype=np.float64, eps_in=EPS, eps_out=EPS):
    """Forward of the stock module.

    ``w`` maps names to arrays: w_ap, w_ag, w_bp, w_bg [H, C]; w_g [C, C];
    w_z [C, H]; g_in, b_in [C]; g_out, b_out [H]; optional linear biases
    bias_ap, bias_ag, bias_bp, bias_bg [H], bias_g, bias_z [C] (the AF2
    layouts the reference's FP32 path accepts,
    ``turbopairformer_trimul_fp32.py:91-152``).  ``mask`` is [..., N, N].
    Returns (out, cache) where cache holds what the backward needs.
    """
    z = np.asarray(z, dtype=dtype)
    W = {k: np.asarray(v, dtype=dtype) for k, v in w.items()}
    m = np.asarray(mask, dtype=dtype)[..., None]

    def lin(x, name):
        y = x @ W["w_" + name].T
        return y + W["bias_" + name] if "bias_" + name in W else y

    zln, xh_in, rstd_in = layer_norm(z, W["g_in"], W["b_in"], eps_in)
    ap, ag = lin(zln, "ap"), lin(zln, "ag")
    bp, bg = lin(zln, "bp"), lin(zln, "bg")
    sa, sb = sigmoid(ag), sigmoid(bg)
    a = m * sa * ap
    b = m * sb * bp
    x = _contract(a, b, outgoing)
    xln, xh_out, rstd_out = layer_norm(x, W["g_out"], W["b_out"], eps_out)
    y = lin(xln, "z")
    sg = sigmoid(lin(zln, "g"))
    out = y * sg
    cache = dict(W=W, m=m, zln=zln, xh_in=xh_in, rstd_in=rstd_in, ap=ap, bp=bp, sa=sa, sb=sb,
                 a=a, b=b, x=x, xln=xln, xh_out=xh_out, rstd_out=rstd_out, y=y, sg=sg,
                 outgoing=outgoing)
    return out, cache


def trimul_backward(dout, cache):
    """Gradients of <dout, out> w.r.t. z and every weight (same names as ``w``)."""
    W, m = cache["W"], cache["m"]
    dout = np.asarray(dout, dtype=cache["zln"].dtype)
    red = tuple(range(dout.ndim - 1))
    sg, y = cache["sg"], cache["y"]
    dy = dout * sg
    dgl = dout * y * sg * (1.0 - sg)
    grads = {}
    grads["w_z"] = np.einsum("rc,rh->ch", dy.reshape(-1, dy.shape[-1]),
                             cache["xln"].reshape(-1, cache["xln"].shape[-1]))
    d_xln = dy @ W["w_z"]
    dx, grads["g_out"], grads["b_out"] = layer_norm_backward(d_xln, cache["xh_out"],
                                                             cache["rstd_out"], W["g_out"])
    a, b = cache["a"], cache["b"]
    dxc = np.moveaxis(dx, -1, -3)
    ac, bc = np.moveaxis(a, -1, -3), np.moveaxis(b, -1, -3)
    if cache["outgoing"]:
        da = dxc @ bc                                  # da_ik = sum_j dx_ij b_jk
        db = np.swapaxes(dxc, -1, -2) @ ac             # db_jk = sum_i dx_ij a_ik
    else:
        da = bc @ np.swapaxes(dxc, -1, -2)             # da_ki = sum_j b_kj dx_ij
        db = ac @ dxc                                  # db_kj = sum_i a_ki dx_ij
    da, db = np.moveaxis(da, -3, -1), np.moveaxis(db, -3, -1)
    sa, sb, ap, bp = cache["sa"], cache["sb"], cache["ap"], cache["bp"]
    d_ap = da * m * sa
    d_ag = da * m * ap * sa * (1.0 - sa)
    d_bp = db * m * sb
    d_bg = db * m * bp * sb * (1.0 - sb)
    zln = cache["zln"]
    zf = zln.reshape(-1, zln.shape[-1])
    for name, d in (("w_ap", d_ap), ("w_ag", d_ag), ("w_bp", d_bp), ("w_bg", d_bg), ("w_g", dgl)):
        grads[name] = d.reshape(-1, d.shape[-1]).T @ zf
    d_zln = d_ap @ W["w_ap"] + d_ag @ W["w_ag"] + d_bp @ W["w_bp"] + d_bg @ W["w_bg"] + dgl @ W["w_g"]
    dz, grads["g_in"], grads["b_in"] = layer_norm_backward(d_zln, cache["xh_in"], cache["rstd_in"],
                                                          W["g_in"])
    del red
    return dz, grads


def trimul_flops(B, N, C) -> dict:
    """Algorithmic matmul flops (H == C): in-proj 2*R*C*5H (4 branch + output
    gate), contraction 2*H*N^3 per batch item, out-proj 2*R*H*C; bwd = 2 x fwd."""
    R = B * N * N
    H = C
    fwd = 2.0 * R * C * 5 * H + 2.0 * B * H * N ** 3 + 2.0 * R * H * C
    return {"fwd": fwd, "bwd": 2 * fwd, "total": 3 * fwd}
