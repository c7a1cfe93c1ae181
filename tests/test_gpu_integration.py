"""Framework integration of the drop-in path on the GPU, after the
reference's custom-op tests (``openfold3/tests/test_turbopairformer_trimul_custom_op.py``):

* ``torch.library.opcheck`` on ``_trimul_fwd_v1`` / ``_trimul_bwd_v1``
  (schema, fake kernel, autograd registration, AOT dispatch; ``:641-718``);
* fake-kernel metadata equal to the real outputs' (``:721-770``);
* ``torch.compile(fullgraph=True, backend="aot_eager")`` over the supported
  TriMul route bitwise equal to eager, forward and backward, also with
  ``dynamic=True`` across sequence lengths (``:781-857``);
* activation checkpointing through the drop-in modules gives the same
  gradients, bitwise (the kernels are deterministic);
* ``chunk_size`` on the attention module only bounds memory in the
  reference (``triangular_attention.py:245-258``): outputs are unchanged.
"""

import copy

import pytest
import torch
from torch.utils.checkpoint import checkpoint


def _trimul_module(channels, outgoing, device, seed):
    from openfold3_triangle_kernel_amd import (
        TriangleMultiplicationIncoming,
        TriangleMultiplicationOutgoing,
    )

    torch.manual_seed(seed)
    cls = TriangleMultiplicationOutgoing if outgoing else TriangleMultiplicationIncoming
    m = cls(channels, channels)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if "layer_norm" in name and name.endswith("weight"):
                p.copy_(1.0 + 0.1 * torch.randn_like(p))
            else:
                p.normal_(std=channels ** -0.5 if p.dim() == 2 else 0.1)
    return m.to(device)


def _fwd_inputs(m, z, mask, outgoing, save_state=True):
    return (
        z, mask,
        m.linear_a_p.weight, m.linear_a_g.weight, m.linear_b_p.weight, m.linear_b_g.weight,
        m.linear_g.weight, m.linear_z.weight,
        m.layer_norm_in.weight, m.layer_norm_in.bias,
        m.layer_norm_out.weight, m.layer_norm_out.bias,
        outgoing, save_state,
    )


@pytest.mark.gpu
@pytest.mark.parametrize("outgoing", [False, True])
@pytest.mark.parametrize("channels,seq", [(32, 64), (128, 65)])
def test_trimul_custom_ops_pass_opcheck(gpu, channels, seq, outgoing):
    from openfold3_triangle_kernel_amd import trimul

    print(f"opcheck C={channels} N={seq} outgoing={outgoing}", flush=True)
    m = _trimul_module(channels, outgoing, gpu, 2026 + channels + seq + int(outgoing))
    z = torch.randn(1, seq, seq, channels, device=gpu, dtype=torch.bfloat16)
    mask = torch.ones(1, seq, seq, device=gpu)
    inputs = _fwd_inputs(m, z.requires_grad_(True), mask, outgoing)
    res = torch.library.opcheck(trimul._trimul_fwd_v1, inputs, raise_exception=True)
    assert all(v == "SUCCESS" for v in res.values()), res

    with torch.no_grad():
        o = trimul._trimul_fwd_v1(*inputs)
    bwd_inputs = (
        torch.randn_like(o[0]), inputs[0], inputs[1], *o[1:11], *inputs[2:8],
        inputs[8], inputs[10], o[0], outgoing,
    )
    bwd_inputs = tuple(t.detach() if isinstance(t, torch.Tensor) else t for t in bwd_inputs)
    res = torch.library.opcheck(
        trimul._trimul_bwd_v1, bwd_inputs,
        test_utils=("test_schema", "test_faketensor", "test_aot_dispatch_dynamic"),
        raise_exception=True,
    )
    assert all(v == "SUCCESS" for v in res.values()), res


@pytest.mark.gpu
@pytest.mark.parametrize("save_state", [False, True])
def test_trimul_fake_forward_metadata_matches_real(gpu, save_state):
    from torch._subclasses.fake_tensor import FakeTensorMode

    from openfold3_triangle_kernel_amd import trimul

    m = _trimul_module(32, True, gpu, 2525 + int(save_state))
    z = torch.randn(1, 17, 17, 32, device=gpu, dtype=torch.bfloat16)
    mask = torch.ones(1, 17, 17, device=gpu)
    tensors = tuple(t.detach() for t in _fwd_inputs(m, z, mask, True)[:12])
    with torch.no_grad():
        real = trimul._trimul_fwd_v1(*tensors, True, save_state)
    mode = FakeTensorMode()
    fakes = tuple(mode.from_tensor(t) for t in tensors)
    with mode, torch.no_grad():
        fake = trimul._trimul_fwd_v1(*fakes, True, save_state)
    assert len(real) == len(fake) == 11
    for r, f in zip(real, fake):
        assert (r.shape, r.dtype, r.device, r.stride()) == (f.shape, f.dtype, f.device, f.stride())
    ptrs = [t.data_ptr() for t in real if t.numel()]
    assert len(set(ptrs)) == len(ptrs), "forward outputs must not alias"
    # save_state=False keeps the schema but returns the backward-only state
    # (z_ln, xln, mean_out, rstd_out) with zero rows (reference
    # turbopairformer_trimul.py:532-546).
    saved_rows = 17 * 17 if save_state else 0
    for i in (1, 6, 9, 10):
        assert real[i].shape[0] == saved_rows, (i, tuple(real[i].shape))
    if not save_state:
        with_state = trimul._trimul_fwd_v1(*tensors, True, True)
        assert torch.equal(real[0], with_state[0]), "inference output must not depend on save_state"


@pytest.mark.gpu
def test_trimul_save_state_false_rejects_gradients(gpu):
    """Reference turbopairformer_trimul.py:689-692: no saved state, no backward."""
    m = _trimul_module(32, True, gpu, 77)
    z = torch.randn(1, 16, 16, 32, device=gpu, dtype=torch.bfloat16, requires_grad=True)
    mask = torch.ones(1, 16, 16, device=gpu)
    with pytest.raises(RuntimeError, match="save_state=True"):
        torch.ops.openfold3_turbopairformer._trimul_fwd_v1(*_fwd_inputs(m, z, mask, True, False))


class _Route(torch.nn.Module):
    """The supported stable route as one module (what the reference compiles)."""

    def __init__(self, inner):
        super().__init__()
        self.inner = inner

    def forward(self, z, mask):
        from openfold3_triangle_kernel_amd import run_stable_trimul

        return run_stable_trimul(self.inner, z, mask)


def _receipt(model, z, mask, grad_out):
    zz = z.detach().clone().requires_grad_(True)
    model.zero_grad(set_to_none=True)
    out = model(zz, mask)
    out.backward(grad_out)
    grads = [p.grad.detach().clone() for p in model.parameters()]
    return [out.detach().clone(), zz.grad.detach().clone(), *grads]


def _assert_bitwise(a, b):
    assert len(a) == len(b)
    for i, (x, y) in enumerate(zip(a, b)):
        assert x.dtype == y.dtype and x.shape == y.shape, i
        assert torch.equal(x, y), f"tensor {i} differs"


@pytest.mark.gpu
@pytest.mark.parametrize("outgoing", [False, True])
@pytest.mark.parametrize("channels,seq", [(32, 64), (128, 65)])
def test_trimul_fullgraph_compile_matches_eager(gpu, channels, seq, outgoing):
    print(f"compile aot_eager C={channels} N={seq} outgoing={outgoing}", flush=True)
    torch.compiler.reset()
    eager = _Route(_trimul_module(channels, outgoing, gpu, 3030 + channels + seq + int(outgoing)))
    compiled = torch.compile(copy.deepcopy(eager), backend="aot_eager", fullgraph=True)
    z = torch.randn(1, seq, seq, channels, device=gpu, dtype=torch.bfloat16)
    mask = (torch.rand(1, seq, seq, device=gpu) > 0.1).float()
    grad_out = torch.randn_like(z)
    _assert_bitwise(_receipt(eager, z, mask, grad_out), _receipt(compiled, z, mask, grad_out))


@pytest.mark.gpu
@pytest.mark.parametrize("outgoing", [False, True])
def test_trimul_dynamic_fullgraph_across_sequence_lengths(gpu, outgoing):
    torch.compiler.reset()
    eager = _Route(_trimul_module(32, outgoing, gpu, 3737 + int(outgoing)))
    compiled = torch.compile(copy.deepcopy(eager), backend="aot_eager", fullgraph=True,
                             dynamic=True)
    for seq in (127, 129):
        print(f"dynamic compile N={seq} outgoing={outgoing}", flush=True)
        z = torch.randn(1, seq, seq, 32, device=gpu, dtype=torch.bfloat16)
        mask = torch.ones(1, seq, seq, device=gpu)
        grad_out = torch.randn_like(z)
        _assert_bitwise(_receipt(eager, z, mask, grad_out), _receipt(compiled, z, mask, grad_out))


class _Checkpointed(torch.nn.Module):
    def __init__(self, inner):
        super().__init__()
        self.inner = inner

    def forward(self, z, mask):
        return checkpoint(self.inner, z, mask, use_reentrant=False)


@pytest.mark.gpu
@pytest.mark.parametrize("outgoing", [False, True])
def test_trimul_module_activation_checkpointing(gpu, outgoing):
    m = _trimul_module(128, outgoing, gpu, 41 + int(outgoing)).to(torch.bfloat16)
    z = torch.randn(2, 48, 48, 128, device=gpu, dtype=torch.bfloat16)
    mask = (torch.rand(2, 48, 48, device=gpu) > 0.2).to(torch.bfloat16)
    grad_out = torch.randn_like(z)

    class _Plain(torch.nn.Module):
        def __init__(self, inner):
            super().__init__()
            self.inner = inner

        def forward(self, z, mask):
            return self.inner(z, mask)

    _assert_bitwise(_receipt(_Plain(m), z, mask, grad_out),
                    _receipt(_Checkpointed(m), z, mask, grad_out))


def _attention_module(starting, device, seed):
    from openfold3_triangle_kernel_amd import TriangleAttention

    torch.manual_seed(seed)
    m = TriangleAttention(128, 32, 4, starting=starting)
    with torch.no_grad():
        for p in m.parameters():
            p.normal_(std=0.05)
    return m.to(device, torch.bfloat16)


@pytest.mark.gpu
@pytest.mark.parametrize("starting", [True, False])
def test_attention_module_activation_checkpointing(gpu, starting):
    m = _attention_module(starting, gpu, 77 + int(starting))
    x = torch.randn(1, 64, 64, 128, device=gpu, dtype=torch.bfloat16)
    mask = (torch.rand(1, 64, 64, device=gpu) > 0.1).to(torch.bfloat16)
    grad_out = torch.randn_like(x)

    class _Plain(torch.nn.Module):
        def __init__(self, inner):
            super().__init__()
            self.inner = inner

        def forward(self, x, mask):
            return self.inner(x, mask)

    _assert_bitwise(_receipt(_Plain(m), x, mask, grad_out),
                    _receipt(_Checkpointed(m), x, mask, grad_out))


@pytest.mark.gpu
@pytest.mark.parametrize("chunk_size", [None, 4, 16])
def test_attention_module_chunk_size_leaves_output_unchanged(gpu, chunk_size):
    m = _attention_module(True, gpu, 91)
    x = torch.randn(1, 48, 48, 128, device=gpu, dtype=torch.bfloat16)
    mask = (torch.rand(1, 48, 48, device=gpu) > 0.1).to(torch.bfloat16)
    with torch.no_grad():
        ref = m(x, mask)
        out = m(x, mask, chunk_size=chunk_size, inplace_safe=chunk_size is not None)
    assert torch.equal(ref, out)


@pytest.mark.gpu
@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_turbo_trimul_no_grad_matches_autograd_forward(gpu, direction):
    """Without autograd the public operator skips the saved state; the output
    is bitwise the one of the differentiable call."""
    from openfold3_triangle_kernel_amd import turbo_trimul

    g = torch.Generator(device=gpu).manual_seed(5)
    C, N = 64, 40
    z = torch.randn(1, N, N, C, device=gpu, generator=g).to(torch.bfloat16)
    w = dict(p_in_weight=torch.randn(2 * C, C, device=gpu, generator=g) / 8,
             g_in_weight=torch.randn(2 * C, C, device=gpu, generator=g) / 8,
             p_out_weight=torch.randn(C, C, device=gpu, generator=g) / 8,
             g_out_weight=torch.randn(C, C, device=gpu, generator=g) / 8)
    mask = (torch.rand(1, N, N, device=gpu, generator=g) > 0.1).float()
    with torch.no_grad():
        ref = turbo_trimul(z, direction, mask, **w)
    wg = {k: v.clone().requires_grad_(True) for k, v in w.items()}
    out = turbo_trimul(z.clone().requires_grad_(True), direction, mask, **wg)
    assert torch.equal(ref, out.detach())
    out.float().sum().backward()
    assert all(t.grad is not None for t in wg.values())
