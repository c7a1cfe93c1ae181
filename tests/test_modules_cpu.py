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
