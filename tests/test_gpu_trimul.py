"""GPU parity of TriMul (C-ABI kernels) against the numpy FP64 oracle.

Tolerance (north star): bf16 output and every gradient at max-rel <= 2e-2,
max-rel = max|got - ref| / max|ref|, oracle evaluated on the same
bf16-rounded z and the same f32 weights.
"""

import numpy as np
import pytest
import torch

from oracle.trimul import trimul_backward, trimul_forward
from tests._util import max_rel

TOL = 2e-2


def trimul_case(B, N, C, seed=0, mask_frac=0.1):
    g = torch.Generator().manual_seed(seed)
    H = C
    z = torch.randn(B, N, N, C, generator=g).to(torch.bfloat16).float()
    mask = (torch.rand(B, N, N, generator=g) > mask_frac).float()
    w = {
        "w_ap": torch.randn(H, C, generator=g) / C ** 0.5,
        "w_ag": torch.randn(H, C, generator=g) / C ** 0.5,
        "w_bp": torch.randn(H, C, generator=g) / C ** 0.5,
        "w_bg": torch.randn(H, C, generator=g) / C ** 0.5,
        "w_g": torch.randn(C, C, generator=g) / C ** 0.5,
        "w_z": torch.randn(C, H, generator=g) / H ** 0.5,
        "g_in": 1 + 0.1 * torch.randn(C, generator=g),
        "b_in": 0.1 * torch.randn(C, generator=g),
        "g_out": 1 + 0.1 * torch.randn(H, generator=g),
        "b_out": 0.1 * torch.randn(H, generator=g),
    }
    dout = torch.randn(B, N, N, C, generator=g).to(torch.bfloat16).float()
    return z, mask, w, dout


def run_turbo(z, mask, w, dout, outgoing, dev):
    from openfold3_triangle_kernel_amd import turbo_trimul

    tz = z.to(dev, torch.bfloat16).requires_grad_(True)
    tw = {k: v.to(dev).requires_grad_(True) for k, v in w.items()}
    p_in = torch.cat([tw["w_ap"], tw["w_bp"]], 0)
    g_in = torch.cat([tw["w_ag"], tw["w_bg"]], 0)
    out = turbo_trimul(tz, "outgoing" if outgoing else "incoming", mask.to(dev),
                       tw["g_in"], tw["b_in"], p_in, g_in, tw["g_out"], tw["b_out"],
                       tw["w_z"], tw["w_g"])
    out.backward(dout.to(dev, torch.bfloat16))
    torch.cuda.synchronize()
    got = {"out": out, "dz": tz.grad}
    got.update({k: t.grad for k, t in tw.items()})
    return {k: v.detach().float().cpu().numpy() for k, v in got.items()}


# N % 8 == 0 runs the persistent weight-stationary kernels (B = 2 crosses a
# batch item inside the walk; N = 200 gives workgroups several 32-row blocks
# and an uneven last share), other N the tile kernels.  N % 192 == 0 runs
# the channel contractions on 192 x 192 tiles (128 x 128 otherwise).
CASES = [(1, 64, 128), (1, 128, 128), (2, 33, 64), (1, 101, 32), (1, 113, 96), (1, 17, 128),
         (2, 48, 64), (1, 72, 96), (1, 40, 32), (1, 200, 128), (1, 192, 64), (2, 192, 32)]


@pytest.mark.gpu
@pytest.mark.parametrize("outgoing", [True, False], ids=["outgoing", "incoming"])
@pytest.mark.parametrize("B,N,C", CASES, ids=[f"B{b}N{n}C{c}" for b, n, c in CASES])
def test_trimul_matches_oracle(gpu, B, N, C, outgoing):
    print(f"[trimul parity] B={B} N={N} C={C} outgoing={outgoing}", flush=True)
    z, mask, w, dout = trimul_case(B, N, C, seed=N + C)
    got = run_turbo(z, mask, w, dout, outgoing, gpu)
    out, cache = trimul_forward(z.numpy(), mask.numpy(), {k: v.numpy() for k, v in w.items()},
                                outgoing)
    dz, grads = trimul_backward(dout.numpy(), cache)
    ref = {"out": out, "dz": dz, **grads}
    errs = {k: max_rel(got[k], ref[k]) for k in ref}
    print({k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    for k, e in errs.items():
        assert e <= TOL, f"{k}: max-rel {e:.3e} > {TOL}"


@pytest.mark.gpu
def test_trimul_bitwise_replay(gpu):
    z, mask, w, dout = trimul_case(1, 96, 128, seed=9)
    a = run_turbo(z, mask, w, dout, True, gpu)
    b = run_turbo(z, mask, w, dout, True, gpu)
    for k in a:
        assert np.array_equal(a[k], b[k]), k


@pytest.mark.gpu
@pytest.mark.parametrize("outgoing", [True, False], ids=["outgoing", "incoming"])
def test_named_weight_gradients_equal_d_w5_rows(gpu, outgoing):
    """turbo_trimul's gradients of p_in / g_in / g_out (written in place by
    tpf_trimul_backward_named_bf16's fold) are bitwise the matching row
    blocks of the op route's d_w5 [ap; ag; bp; bg; g]."""
    from openfold3_triangle_kernel_amd import trimul as tm

    z, mask, w, dout = trimul_case(1, 64, 64, seed=4)
    got = run_turbo(z, mask, w, dout, outgoing, gpu)
    zb = z.to(gpu, torch.bfloat16)
    names = ("w_ap", "w_ag", "w_bp", "w_bg", "w_g", "w_z")
    res = torch.ops.openfold3_turbopairformer._trimul_fwd_v1(
        zb, mask.to(gpu), *[w[k].to(gpu) for k in names], w["g_in"].to(gpu),
        w["b_in"].to(gpu), w["g_out"].to(gpu), w["b_out"].to(gpu), outgoing, True)
    out, z_ln, gate, a, b, x, xln, mi, ri, mo, ro = res
    d_w5 = tm._trimul_bwd_v1(dout.to(gpu, torch.bfloat16), zb, mask.to(gpu), z_ln, gate, a, b, x,
                             xln, mi, ri, mo, ro, *[w[k].to(gpu) for k in names],
                             w["g_in"].to(gpu), w["g_out"].to(gpu), out, outgoing)[1]
    rows = d_w5.view(5, 64, 64).cpu().numpy()
    for i, k in enumerate(("w_ap", "w_ag", "w_bp", "w_bg", "w_g")):
        assert np.array_equal(got[k], rows[i]), k


@pytest.mark.gpu
@pytest.mark.parametrize("outgoing", [1, 0], ids=["outgoing", "incoming"])
def test_trimul_backward_ignores_memory_past_the_planes(gpu, outgoing):
    """N % 8 != 0: the dA contraction runs K over the plane pitch Np (dX's zero
    pad columns), whose rows of B_c past N do not exist -- past the last plane
    they lie outside the tensor.  Here the memory right after a and b holds
    non-finite values: every gradient must stay finite and equal the run with
    clean memory (the kernels must not read there)."""
    from openfold3_triangle_kernel_amd import _native

    B, N, C = 1, 50, 128
    print(f"[trimul pad tail] N={N} outgoing={outgoing}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(3)
    z = torch.randn(B, N, N, C, device=gpu, generator=g).bfloat16()
    mask = (torch.rand(B, N, N, device=gpu, generator=g) > 0.1).float()
    w = [torch.randn(C, C, device=gpu, generator=g) / C ** 0.5 for _ in range(6)]
    ln = [torch.ones(C, device=gpu), torch.zeros(C, device=gpu)] * 2
    dout = torch.randn(B, N, N, C, device=gpu, generator=g).bfloat16()
    Np = int(_native.query("tpf_trimul_plane_pitch", N))
    rows, pn = B * N * N, B * C * N * Np
    P = lambda t: t.data_ptr()  # noqa: E731

    def run(tail):
        E = lambda *s, dt=torch.bfloat16: torch.empty(*s, device=gpu, dtype=dt)  # noqa: E731
        # a and b at the start of buffers whose remainder holds `tail`.
        ab = torch.full((2, pn + 8 * Np), tail, device=gpu, dtype=torch.bfloat16)
        a, b = ab[0], ab[1]
        out, zln, gate, x, xln = E(rows, C), E(rows, C), E(rows, C), E(pn), E(rows, C)
        st = [E(rows, dt=torch.float32) for _ in range(4)]
        wsf = E(int(_native.query("tpf_trimul_forward_workspace_bytes", C)), dt=torch.uint8)
        wsb = E(int(_native.query("tpf_trimul_backward_workspace_bytes", B, N, C)), dt=torch.uint8)
        grads = [E(rows, C), E(5 * C, C, dt=torch.float32), E(C, C, dt=torch.float32)]
        grads += [E(C, dt=torch.float32) for _ in range(4)]
        s = torch.cuda.current_stream().cuda_stream
        _native.call("tpf_trimul_forward_bf16", P(z), P(mask), *map(P, w), *map(P, ln), outgoing,
                     B, N, C, P(out), P(zln), P(gate), P(a), P(b), P(x), P(xln), *map(P, st),
                     P(wsf), wsf.numel(), s)
        _native.call("tpf_trimul_backward_bf16", P(dout), P(z), P(mask), *map(P, w), P(ln[0]),
                     P(ln[2]), P(zln), P(gate), P(a), P(b), P(x), P(xln), *map(P, st), outgoing,
                     B, N, C, *map(P, grads), P(wsb), wsb.numel(), s)
        torch.cuda.synchronize()
        return grads

    clean = run(0.0)
    dirty = run(float("inf"))
    for c, d in zip(clean, dirty):
        assert torch.isfinite(d.float()).all()
        assert torch.equal(c, d)
