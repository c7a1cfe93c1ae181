"""Pins the torch restatement of the stock math (oracle/stock_torch.py, the
CPU baseline's path) to the numpy oracle, in FP64, chunked and unchunked."""

import numpy as np
import torch

from oracle.attention import attention_backward, attention_forward
from oracle.stock_torch import attention_stock_train_step, trimul_stock
from oracle.trimul import trimul_forward


def test_attention_stock_matches_oracle_chunked():
    g = torch.Generator().manual_seed(3)
    B, O, H, N, D = 1, 6, 2, 24, 8
    q, k, v = (torch.randn(B, O, H, N, D, generator=g, dtype=torch.float64) for _ in range(3))
    mask = torch.zeros(B, O, 1, 1, N, dtype=torch.float64)
    mask[..., 20:] = float("-inf")
    bias = torch.randn(1, 1, H, N, N, generator=g, dtype=torch.float64)
    dout = torch.randn(B, O, N, H, D, generator=g, dtype=torch.float64)
    ref_out, _, _ = attention_forward(q.numpy(), k.numpy(), v.numpy(), mask.numpy(), bias.numpy())
    ref = [ref_out, *attention_backward(q.numpy(), k.numpy(), v.numpy(), mask.numpy(),
                                        bias.numpy(), dout.numpy())]
    for chunk in (None, 4):
        got = attention_stock_train_step(q, k, v, mask, bias, dout, chunk=chunk)
        for a, r in zip(got, ref):
            assert a.shape == r.shape
            assert np.allclose(a.numpy(), r, rtol=1e-9, atol=1e-11)


def test_trimul_stock_matches_oracle():
    g = torch.Generator().manual_seed(4)
    C = 8
    w = {n: torch.randn(C, C, generator=g, dtype=torch.float64) / 3
         for n in ("w_ap", "w_ag", "w_bp", "w_bg", "w_g", "w_z")}
    w.update({"g_in": 1 + 0.1 * torch.randn(C, generator=g, dtype=torch.float64),
              "b_in": 0.1 * torch.randn(C, generator=g, dtype=torch.float64),
              "g_out": 1 + 0.1 * torch.randn(C, generator=g, dtype=torch.float64),
              "b_out": 0.1 * torch.randn(C, generator=g, dtype=torch.float64)})
    z = torch.randn(2, 7, 7, C, generator=g, dtype=torch.float64)
    m = (torch.rand(2, 7, 7, generator=g) > 0.2).double()
    for outgoing in (True, False):
        ref, _ = trimul_forward(z.numpy(), m.numpy(), {n: t.numpy() for n, t in w.items()},
                                outgoing)
        assert np.allclose(trimul_stock(z, m, w, outgoing).numpy(), ref, rtol=1e-10, atol=1e-12)
