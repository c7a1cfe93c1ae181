"""Drop-in module adapters: parameter names, order and shapes match the
OpenFold3 modules (CPU, no kernels run)."""

import torch

from openfold3_triangle_kernel_amd import (
    TriangleAttention,
    TriangleMultiplicationIncoming,
    TriangleMultiplicationOutgoing,
)


def test_triangle_attention_state_dict_layout():
    m = TriangleAttention(128, 32, 4, starting=False)
    names = [(n, tuple(p.shape)) for n, p in m.named_parameters()]
    assert names == [
        ("layer_norm.weight", (128,)), ("layer_norm.bias", (128,)), ("linear_z.weight", (4, 128)),
        ("mha.linear_q.weight", (128, 128)), ("mha.linear_k.weight", (128, 128)),
        ("mha.linear_v.weight", (128, 128)), ("mha.linear_o.weight", (128, 128)),
        ("mha.linear_g.weight", (128, 128)),
    ]


def test_trimul_state_dict_layout():
    out = TriangleMultiplicationOutgoing(128, 64)
    assert out._outgoing and not TriangleMultiplicationIncoming(128, 64)._outgoing
    names = [(n, tuple(p.shape)) for n, p in out.named_parameters()]
    assert names == [
        ("linear_g.weight", (128, 128)), ("linear_z.weight", (128, 64)),
        ("layer_norm_in.weight", (128,)), ("layer_norm_in.bias", (128,)),
        ("layer_norm_out.weight", (64,)), ("layer_norm_out.bias", (64,)),
        ("linear_a_p.weight", (64, 128)), ("linear_a_g.weight", (64, 128)),
        ("linear_b_p.weight", (64, 128)), ("linear_b_g.weight", (64, 128)),
    ]
    sd = out.state_dict()
    fresh = TriangleMultiplicationOutgoing(128, 64)
    fresh.load_state_dict(sd)
    for k, v in fresh.state_dict().items():
        assert torch.equal(v, sd[k])


# --- routing (use_stable_* flags, strict mode, fallback logging) -----------

from pathlib import Path  # noqa: E402

import numpy as np  # noqa: E402
import pytest  # noqa: E402

GOLD = Path(__file__).resolve().parent / "golden" / "snapshots"


def _snapshot_attention(starting):
    torch.manual_seed(123)
    m = TriangleAttention(128, 12, 4, starting=starting)
    for p in m.parameters():
        p.data.normal_(std=0.01)
    return m, torch.rand((2, 22, 22, 128))


@pytest.mark.parametrize("starting", [True, False])
def test_stock_attention_route_matches_reference_snapshot(starting):
    """use_stable_triangle_attention=False runs the stock math; it reproduces
    the reference module's committed FP32 CPU output."""
    from openfold3_triangle_kernel_amd import stock_invocation_count

    m, x = _snapshot_attention(starting)
    ref = np.load(GOLD / f"tri_att_cpu_starting_{starting}.npz")["output"]
    before = stock_invocation_count()
    with torch.no_grad():
        out = m(x, use_stable_triangle_attention=False)
    assert stock_invocation_count() == before + 1
    assert np.abs(out.numpy() - ref).max() <= 1e-5 * np.abs(ref).max()


def test_stock_trimul_route_matches_reference_snapshot():
    torch.manual_seed(123)
    m = TriangleMultiplicationOutgoing(128, 11)
    for p in m.parameters():
        p.data.normal_(std=0.01)
    x = torch.rand((2, 22, 22, 128))
    mask = torch.randint(0, 2, size=(2, 22, 22))
    ref = np.load(GOLD / "tri_mul_outgoing_cpu.npz")["output"]
    with torch.no_grad():
        out = m(x, mask.float(), use_stable_triangle_multiplicative=False)
    assert np.abs(out.numpy() - ref).max() <= 1e-5 * np.abs(ref).max()
    with torch.no_grad():
        added = m(x, mask.float(), inplace_safe=True, _add_with_inplace=True,
                  use_stable_triangle_multiplicative=False)
    assert torch.allclose(added, x + out)


def test_stable_route_fallback_logging_and_strict_mode(caplog):
    """An unsupported stable request (CPU tensors) logs once and runs the stock
    math; strict mode raises instead (attention.py:586-595, 675-692)."""
    from openfold3_triangle_kernel_amd import set_turbopairformer_strict, stock_invocation_count

    m, x = _snapshot_attention(True)
    x.requires_grad_(True)
    m = m.to(torch.bfloat16)
    xb = x.detach().bfloat16().requires_grad_(True)
    before = stock_invocation_count()
    with caplog.at_level("WARNING"):
        m(xb)
        m(xb)
    assert stock_invocation_count() == before + 2
    assert sum("fallback to stock" in r.getMessage() for r in caplog.records) == 1
    set_turbopairformer_strict(True)
    try:
        with pytest.raises(RuntimeError, match="strict route"):
            m(xb)
        t = TriangleMultiplicationOutgoing(128, 128).to(torch.bfloat16)
        with pytest.raises(RuntimeError, match="strict route"):
            t(xb)
    finally:
        set_turbopairformer_strict(False)


def test_fp32_inference_and_backend_flags():
    """FP32 inference owns the site: an unsupported case raises (no fallback);
    the reference's other backends are absent and raise."""
    m, x = _snapshot_attention(True)
    with torch.no_grad(), pytest.raises(ValueError, match="FP32 inference"):
        m(x)
    for flag in ("use_deepspeed_evo_attention", "use_cueq_triangle_kernels",
                 "use_triton_triangle_kernels", "use_lma", "use_protenix_triangle_attention"):
        with pytest.raises(ValueError, match="not available"):
            m(x, **{flag: True})
    t = TriangleMultiplicationOutgoing(128, 128)
    with pytest.raises(ValueError, match="not available"):
        t(x, use_cueq_triangle_kernels=True)
