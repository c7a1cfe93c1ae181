"""TriMul boundary contracts on CPU: op schemas (the reference's exact
strings), fake kernels, first-order-only backward, weight mapping and the
support verdict."""

import types

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import openfold3_triangle_kernel_amd  # noqa: F401  registers the ops

# openfold3/tests/test_turbopairformer_trimul_custom_op.py:26-40
FORWARD_SCHEMA = (
    "openfold3_turbopairformer::_trimul_fwd_v1(Tensor z_bf, Tensor mask_f, "
    "Tensor w_ap, Tensor w_ag, Tensor w_bp, Tensor w_bg, Tensor w_g, "
    "Tensor w_z, Tensor g_in, Tensor b_in, Tensor g_out, Tensor b_out, "
    "bool outgoing, bool save_state) -> (Tensor, Tensor, Tensor, Tensor, "
    "Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)"
)
BACKWARD_SCHEMA = (
    "openfold3_turbopairformer::_trimul_bwd_v1(Tensor grad_out, Tensor z_bf, "
    "Tensor mask_f, Tensor z_ln, Tensor gate, Tensor a, Tensor b, Tensor x, "
    "Tensor xlnT, Tensor mean_in, Tensor rstd_in, Tensor mean_out, "
    "Tensor rstd_out, Tensor w_ap, Tensor w_ag, Tensor w_bp, Tensor w_bg, "
    "Tensor w_g, Tensor w_z, Tensor g_in, Tensor g_out, Tensor out, "
    "bool outgoing) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)"
)


def test_schemas_match_reference():
    ops = torch.ops.openfold3_turbopairformer
    assert str(ops._trimul_fwd_v1.default._schema) == FORWARD_SCHEMA
    assert str(ops._trimul_bwd_v1.default._schema) == BACKWARD_SCHEMA


def _inputs(B=1, N=20, C=32):
    z = torch.zeros(B, N, N, C, dtype=torch.bfloat16)
    mask = torch.ones(B, N, N)
    w = [torch.zeros(C, C) for _ in range(6)]
    ln = [torch.ones(C), torch.zeros(C), torch.ones(C), torch.zeros(C)]
    return z, mask, w, ln


def test_fake_kernels_describe_shapes():
    z, mask, w, ln = _inputs()
    with FakeTensorMode() as mode:
        fz, fm = mode.from_tensor(z), mode.from_tensor(mask)
        fw = [mode.from_tensor(t) for t in w]
        fl = [mode.from_tensor(t) for t in ln]
        outs = torch.ops.openfold3_turbopairformer._trimul_fwd_v1(fz, fm, *fw, *fl, True, True)
        assert outs[0].shape == z.shape and outs[0].dtype == torch.bfloat16
        assert outs[3].shape == (32, 20 * 24)  # channel-major stored matrix, pitch 24
        assert outs[5].shape == (32, 20, 24)
        grads = torch.ops.openfold3_turbopairformer._trimul_bwd_v1(
            mode.from_tensor(z), fz, fm, outs[1], outs[2], outs[3], outs[4], outs[5], outs[6],
            outs[7], outs[8], outs[9], outs[10], *fw, fl[0], fl[2], outs[0], True)
        assert grads[0].shape == z.shape
        assert grads[1].shape == (5 * 32, 32) and grads[1].dtype == torch.float32


def test_second_order_gradients_are_rejected():
    from openfold3_triangle_kernel_amd import trimul

    with pytest.raises(RuntimeError, match="first-order"):
        trimul._trimul_bwd_v1_backward(None)


def _module(C=32, H=32, bias=False, eps=1e-5, outgoing=True):
    lin = lambda i, o: types.SimpleNamespace(weight=torch.zeros(o, i), bias=torch.zeros(o) if bias else None)
    ln = lambda c: types.SimpleNamespace(weight=torch.ones(c), bias=torch.zeros(c), eps=eps)
    return types.SimpleNamespace(linear_a_p=lin(C, H), linear_a_g=lin(C, H), linear_b_p=lin(C, H),
                                 linear_b_g=lin(C, H), linear_g=lin(C, C), linear_z=lin(H, C),
                                 layer_norm_in=ln(C), layer_norm_out=ln(H), _outgoing=outgoing)


class _Meta(torch.Tensor):
    pass


@pytest.mark.parametrize("mod_kw,z_shape,reason", [
    (dict(H=16), (1, 8, 8, 32), "c_hidden == c_z"),
    (dict(C=48, H=48), (1, 8, 8, 48), "channels"),
    (dict(bias=True), (1, 8, 8, 32), "bias"),
    (dict(eps=1e-6), (1, 8, 8, 32), "eps"),
])
def test_support_verdicts(monkeypatch, mod_kw, z_shape, reason):
    from openfold3_triangle_kernel_amd import trimul

    z = torch.zeros(z_shape, dtype=torch.bfloat16, device="meta")
    monkeypatch.setattr(torch.Tensor, "device", property(lambda self: torch.device("cuda")), raising=False)
    ok, why = trimul.check_stable_trimul_support(_module(**mod_kw), z, None)
    assert not ok and reason in why


def test_turbo_trimul_rejects_bad_direction_and_shapes():
    from openfold3_triangle_kernel_amd import turbo_trimul

    z = torch.zeros(1, 8, 8, 32, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="direction"):
        turbo_trimul(z, direction="sideways")
    with pytest.raises(ValueError, match="p_in_weight"):
        turbo_trimul(z, p_in_weight=torch.zeros(32, 32))


def test_eager_trimul_rejects_host_tensors_before_any_launch(monkeypatch):
    """Eager calls run the op implementations directly (not through the CUDA-only
    custom-op dispatch): host tensors must be refused before a pointer reaches
    the library.  The native entry points are replaced by a tripwire."""
    from openfold3_triangle_kernel_amd import _native, turbo_trimul

    def tripwire(*args, **kwargs):
        raise AssertionError("a native entry point was called with host tensors")

    monkeypatch.setattr(_native, "call", tripwire)
    z = torch.zeros(1, 8, 8, 32, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU tensors"):
        turbo_trimul(z)
    with pytest.raises(RuntimeError, match="GPU tensors"):
        turbo_trimul(z.requires_grad_(True))
