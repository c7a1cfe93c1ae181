"""Drop-in modules on the GPU against the reference's committed module
snapshots (``tests/golden/snapshots``, built exactly as the reference's
tests build them: seed 123, every parameter ~ N(0, 0.01) in registration
order, x = rand(2, 22, 22, 128)).

BF16 route (training kernels): max-rel <= 2e-2; FP32 inference route:
max-rel <= 1e-4 (the snapshots are FP32 CPU outputs).
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from tests._util import max_rel

GOLD = Path(__file__).resolve().parent / "golden" / "snapshots"


def _attention_module(starting):
    from openfold3_triangle_kernel_amd import TriangleAttention

    torch.manual_seed(123)
    m = TriangleAttention(128, 12, 4, starting=starting)
    for p in m.parameters():
        p.data.normal_(std=0.01)
    x = torch.rand((2, 22, 22, 128))
    return m, x


@pytest.mark.gpu
@pytest.mark.parametrize("starting", [True, False])
def test_triangle_attention_module_snapshot(gpu, starting):
    m, x = _attention_module(starting)
    ref = np.load(GOLD / f"tri_att_cpu_starting_{starting}.npz")["output"]
    m = m.to(gpu)
    print(f"module tri-att starting={starting}", flush=True)
    with torch.no_grad():
        out32 = m(x.to(gpu))                                   # FP32 inference kernel
    assert max_rel(out32.cpu().numpy(), ref) <= 1e-4
    mb = m.to(torch.bfloat16)
    xb = x.to(gpu, torch.bfloat16).requires_grad_(True)
    outb = mb(xb)                                              # BF16 training kernels
    outb.float().square().mean().backward()
    assert max_rel(outb.detach().float().cpu().numpy(), ref) <= 2e-2
    assert xb.grad is not None and torch.isfinite(xb.grad).all()
    assert all(p.grad is not None for p in mb.parameters())


@pytest.mark.gpu
def test_trimul_module_snapshot_fp32(gpu):
    from openfold3_triangle_kernel_amd import TriangleMultiplicationOutgoing

    torch.manual_seed(123)
    m = TriangleMultiplicationOutgoing(128, 11)
    for p in m.parameters():
        p.data.normal_(std=0.01)
    x = torch.rand((2, 22, 22, 128))
    mask = torch.randint(0, 2, size=(2, 22, 22))
    ref = np.load(GOLD / "tri_mul_outgoing_cpu.npz")["output"]
    m = m.to(gpu)
    with torch.no_grad():
        out = m(x.to(gpu), mask.to(gpu).float())
    assert max_rel(out.cpu().numpy(), ref) <= 1e-4
    # The BF16 training kernels need c_hidden == c_z: this module is rejected loudly.
    with pytest.raises(ValueError, match="c_hidden == c_z"):
        m(x.to(gpu).requires_grad_(True), mask.to(gpu).float())
