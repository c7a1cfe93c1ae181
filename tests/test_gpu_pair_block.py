"""Config 5: the pair-stack block through the drop-in modules at N=768.

The block of the reference's pairformer (openfold3/core/model/latent/
base_blocks.py:311-431) applies, residually and in order, TriMul outgoing,
TriMul incoming, triangle attention around the starting node and around the
ending node (H=4, D=32, pair bias projected from z).  Here it runs in BF16
through the kernels (modules in ``openfold3_triangle_kernel_amd.modules``)
and, as the reference, in FP32 through the same modules' stock math
(``use_stable_*=False``; that math is pinned to the reference's committed
module snapshots in tests/test_modules_cpu.py), on the same bf16-representable
weights N(0, 1/sqrt(fan_in)) and input z ~ N(0, 1) [1, 768, 768, 128].

Gate (north star): the block output, dz and every parameter gradient at
max-rel <= 2e-2 against the FP32 stock block.
"""

import math

import pytest
import torch

TOL = 2e-2


def _block(dev, dtype):
    from openfold3_triangle_kernel_amd import (
        TriangleAttention,
        TriangleMultiplicationIncoming,
        TriangleMultiplicationOutgoing,
    )

    torch.manual_seed(5)
    C = 128
    mods = [TriangleMultiplicationOutgoing(C, C), TriangleMultiplicationIncoming(C, C),
            TriangleAttention(C, 32, 4, starting=True), TriangleAttention(C, 32, 4, starting=False)]
    for mo in mods:
        for p in mo.parameters():
            if p.dim() == 2:
                p.data = (torch.randn_like(p) / math.sqrt(p.shape[1])).bfloat16().float()
    return [mo.to(dev, dtype) for mo in mods]


def _run(mods, z, mask, dout, stable):
    zt = z.detach().requires_grad_(True)
    h = zt
    for mo in mods:
        if hasattr(mo, "mha"):
            upd = mo(h, mask, use_stable_triangle_attention=stable)
        else:
            upd = mo(h, mask, use_stable_triangle_multiplicative=stable)
        h = h + upd
    params = [p for mo in mods for p in mo.parameters()]
    grads = torch.autograd.grad(h, [zt] + params, dout)
    return [h.detach()] + [g.detach() for g in grads]


@pytest.mark.gpu
def test_config5_pair_block_n768(gpu):
    from openfold3_triangle_kernel_amd import stock_invocation_count

    N, C = 768, 128
    print(f"[pair block] config 5 N={N} C={C}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(50)
    z = torch.randn(1, N, N, C, device=gpu, generator=g).bfloat16()
    mask = torch.ones(1, N, N, device=gpu)
    dout = torch.randn(1, N, N, C, device=gpu, generator=g).bfloat16()

    mods_b = _block(gpu, torch.bfloat16)
    before = stock_invocation_count()
    got = _run(mods_b, z, mask.bfloat16(), dout, stable=True)
    assert stock_invocation_count() == before, "the BF16 block must run the kernels"
    torch.cuda.synchronize()

    mods_f = _block(gpu, torch.float32)
    ref = _run(mods_f, z.float(), mask, dout.float(), stable=False)
    names = ["out", "dz"] + [f"{type(mo).__name__}[{i}].{n}" for i, mo in enumerate(mods_f)
                             for n, _ in mo.named_parameters()]
    worst = 0.0
    fails = []
    for name, a, b in zip(names, got, ref):
        err = ((a.float() - b).abs().max() / b.abs().max()).item()
        worst = max(worst, err)
        print(f"pair block {name} max-rel {err:.3e}", flush=True)
        if not err <= TOL:
            fails.append(f"{name}: {err:.3e}")
    assert not fails, "; ".join(fails)
