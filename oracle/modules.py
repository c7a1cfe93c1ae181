"""Numpy restatements of OpenFold3's pair-stack modules -- TEST INFRASTRUCTURE ONLY.

Used to pin the oracles against the reference's committed module snapshots
(openfold3/tests/test_data/snapshots/test_triangular_{attention,
multiplicative_update}/*/test_shape_cpu_*.npz, copied into tests/golden/).

* ``triangle_attention_module`` follows TriangleAttention.forward
  (openfold3/core/model/layers/triangular_attention.py:352-409) and the stock
  Attention path (openfold3/core/model/primitives/attention.py:347-384, 732):
  LN, mask bias inf*(mask-1), pair bias linear_z permuted to [*,1,H,I,J],
  q/k/v projections, attention (oracle.attention), sigmoid gate, linear_o;
  the ending-node variant transposes the pair input and output.
* ``trimul_module`` is oracle.trimul.trimul_forward with the module's weights.
"""

from __future__ import annotations

import numpy as np

from .attention import attention_forward
from .trimul import layer_norm, sigmoid, trimul_forward


def triangle_attention_module(x, params, no_heads, starting=True, mask=None, inf=1e9,
                              dtype=np.float64):
    """params: layer_norm_w/b [C], linear_z [H, C], q/k/v/g [H*c, C], o [C, H*c]."""
    x = np.asarray(x, dtype=dtype)
    P = {k: np.asarray(v, dtype=dtype) for k, v in params.items()}
    if mask is None:
        mask = np.ones(x.shape[:-1], dtype=dtype)
    if not starting:
        x = np.swapaxes(x, -2, -3)
        mask = np.swapaxes(mask, -1, -2)
    x, _, _ = layer_norm(x, P["layer_norm_w"], P["layer_norm_b"])
    mask_bias = (inf * (mask - 1))[..., :, None, None, :]          # [*, I, 1, 1, J]
    tri = x @ P["linear_z"].T                                       # [*, I, J, H]
    tri = np.moveaxis(tri, -1, -3)[..., None, :, :, :]              # [*, 1, H, I, J]
    H = no_heads
    q = (x @ P["linear_q"].T)
    k = (x @ P["linear_k"].T)
    v = (x @ P["linear_v"].T)
    c = q.shape[-1] // H
    q, k, v = (np.swapaxes(t.reshape(t.shape[:-1] + (H, c)), -2, -3) for t in (q, k, v))
    o, _, _ = attention_forward(q, k, v, mask_bias, tri, scale=1.0 / np.sqrt(c), dtype=dtype)
    g = sigmoid(x @ P["linear_g"].T).reshape(o.shape)                # [*, I, J, H, c]
    o = (o * g).reshape(o.shape[:-2] + (H * c,))
    out = o @ P["linear_o"].T
    if not starting:
        out = np.swapaxes(out, -2, -3)
    return out


def trimul_module(z, mask, params, outgoing=True, dtype=np.float64):
    """params keys: linear_a_p/a_g/b_p/b_g [H, C], linear_g [C, C], linear_z [C, H],
    layer_norm_in_w/b [C], layer_norm_out_w/b [H]."""
    w = dict(w_ap=params["linear_a_p"], w_ag=params["linear_a_g"], w_bp=params["linear_b_p"],
             w_bg=params["linear_b_g"], w_g=params["linear_g"], w_z=params["linear_z"],
             g_in=params["layer_norm_in_w"], b_in=params["layer_norm_in_b"],
             g_out=params["layer_norm_out_w"], b_out=params["layer_norm_out_b"])
    out, _ = trimul_forward(z, mask, w, outgoing, dtype=dtype)
    return out
