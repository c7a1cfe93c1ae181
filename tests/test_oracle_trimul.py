"""Pin the TriMul oracle: forward vs a literal torch restatement of the stock
module code, hand-derived backward vs torch autograd."""

import numpy as np
import pytest
import torch

from oracle.trimul import trimul_backward, trimul_forward


def _permute_final_dims(t, inds):
    zero_index = -1 * len(inds)
    first = list(range(len(t.shape[:zero_index])))
    return t.permute(first + [zero_index + i for i in inds])


def _torch_trimul(z, mask, w, outgoing):
    # Literal structure of triangular_multiplicative_update.py:1263-1284 and
    # _combine_projections :734-760 (permute_final_dims + matmul).
    ln = lambda x, g, b: torch.nn.functional.layer_norm(x, (x.shape[-1],), g, b, 1e-5)
    m = mask.unsqueeze(-1)
    zz = ln(z, w["g_in"], w["b_in"])
    a = m * torch.sigmoid(zz @ w["w_ag"].T) * (zz @ w["w_ap"].T)
    b = m * torch.sigmoid(zz @ w["w_bg"].T) * (zz @ w["w_bp"].T)
    if outgoing:
        a2, b2 = _permute_final_dims(a, (2, 0, 1)), _permute_final_dims(b, (2, 1, 0))
    else:
        a2, b2 = _permute_final_dims(a, (2, 1, 0)), _permute_final_dims(b, (2, 0, 1))
    x = _permute_final_dims(torch.matmul(a2, b2), (1, 2, 0))
    x = ln(x, w["g_out"], w["b_out"]) @ w["w_z"].T
    return x * torch.sigmoid(zz @ w["w_g"].T)


def _weights(rng, C, H):
    w = {n: rng.standard_normal((H, C)) / np.sqrt(C) for n in ("w_ap", "w_ag", "w_bp", "w_bg")}
    w["w_g"] = rng.standard_normal((C, C)) / np.sqrt(C)
    w["w_z"] = rng.standard_normal((C, H)) / np.sqrt(H)
    w["g_in"], w["b_in"] = 1 + 0.1 * rng.standard_normal(C), 0.1 * rng.standard_normal(C)
    w["g_out"], w["b_out"] = 1 + 0.1 * rng.standard_normal(H), 0.1 * rng.standard_normal(H)
    return w


@pytest.mark.parametrize("outgoing", [True, False])
@pytest.mark.parametrize("H", [8, 5])
def test_forward_backward_match_torch(outgoing, H):
    rng = np.random.default_rng(7)
    B, N, C = 2, 7, 8
    z = rng.standard_normal((B, N, N, C))
    mask = (rng.random((B, N, N)) > 0.2).astype(np.float64)
    w = _weights(rng, C, H)
    tw = {k: torch.tensor(v, requires_grad=True) for k, v in w.items()}
    tz = torch.tensor(z, requires_grad=True)
    tout = _torch_trimul(tz, torch.tensor(mask), tw, outgoing)
    dout = rng.standard_normal(tout.shape)
    tout.backward(torch.tensor(dout))
    out, cache = trimul_forward(z, mask, w, outgoing)
    np.testing.assert_allclose(out, tout.detach().numpy(), rtol=1e-10, atol=1e-12)
    dz, grads = trimul_backward(dout, cache)
    np.testing.assert_allclose(dz, tz.grad.numpy(), rtol=1e-8, atol=1e-11)
    for k in w:
        np.testing.assert_allclose(grads[k], tw[k].grad.numpy(), rtol=1e-8, atol=1e-11, err_msg=k)


def test_masked_rows_do_not_feed_the_product():
    rng = np.random.default_rng(3)
    B, N, C = 1, 5, 4
    w = _weights(rng, C, C)
    z = rng.standard_normal((B, N, N, C))
    mask = np.ones((B, N, N))
    mask[0, 2, :] = 0
    out1, c1 = trimul_forward(z, mask, w, True)
    z2 = z.copy()
    z2[0, 2, :] += 5.0  # masked row: only its own output gate may change
    out2, c2 = trimul_forward(z2, mask, w, True)
    np.testing.assert_allclose(c1["x"], c2["x"], rtol=0, atol=1e-12)


def test_forward_with_linear_biases_and_eps_matches_torch_modules():
    """Pins the optional-bias / eps extension of trimul_forward against an
    independent torch restatement built from nn.Linear / nn.LayerNorm."""
    import torch

    from oracle.trimul import trimul_forward

    torch.manual_seed(3)
    C, H, N = 12, 10, 7
    lin = {n: torch.nn.Linear(C, H, dtype=torch.float64) for n in ("ap", "ag", "bp", "bg")}
    lin["g"] = torch.nn.Linear(C, C, dtype=torch.float64)
    lin["z"] = torch.nn.Linear(H, C, dtype=torch.float64)
    ln_in = torch.nn.LayerNorm(C, eps=1e-3, dtype=torch.float64)
    ln_out = torch.nn.LayerNorm(H, eps=1e-4, dtype=torch.float64)
    with torch.no_grad():
        for t in (ln_in.weight, ln_in.bias, ln_out.weight, ln_out.bias):
            t.normal_()
    z = torch.randn(2, N, N, C, dtype=torch.float64)
    mask = (torch.rand(2, N, N) > 0.2).double()
    for outgoing in (True, False):
        with torch.no_grad():
            zl = ln_in(z)
            a = mask[..., None] * torch.sigmoid(lin["ag"](zl)) * lin["ap"](zl)
            b = mask[..., None] * torch.sigmoid(lin["bg"](zl)) * lin["bp"](zl)
            eq = "bikc,bjkc->bijc" if outgoing else "bkic,bkjc->bijc"
            ref = lin["z"](ln_out(torch.einsum(eq, a, b))) * torch.sigmoid(lin["g"](zl))
        w = {"g_in": ln_in.weight.detach().numpy(), "b_in": ln_in.bias.detach().numpy(),
             "g_out": ln_out.weight.detach().numpy(), "b_out": ln_out.bias.detach().numpy()}
        for n, l in lin.items():
            w["w_" + n] = l.weight.detach().numpy()
            w["bias_" + n] = l.bias.detach().numpy()
        got, _ = trimul_forward(z.numpy(), mask.numpy(), w, outgoing, eps_in=1e-3, eps_out=1e-4)
        np.testing.assert_allclose(got, ref.numpy(), rtol=1e-10, atol=1e-10)
