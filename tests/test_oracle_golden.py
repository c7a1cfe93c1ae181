"""Pin the numpy oracle against the reference's committed module snapshots.

The reference tests build the module under torch.manual_seed(123), re-initialise
every parameter with normal_(std=0.01) in registration order, then draw the
inputs.  Module construction consumes torch RNG through nn.Linear's own
reset_parameters (kaiming_uniform_); the reference's truncated-normal init uses
numpy/scipy RNG and leaves the torch stream untouched.  We replay exactly that
torch consumption with plain torch.nn.Linear objects of the same shapes and
order, then evaluate the numpy restatement of the module (oracle.modules).
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle.modules import triangle_attention_module, trimul_module

GOLD = Path(__file__).resolve().parent / "golden" / "snapshots"
TOL = dict(atol=1e-4, rtol=1e-4)  # the reference test's own tolerance


def _linear_rng(in_dim, out_dim):
    return torch.nn.Linear(in_dim, out_dim, bias=False)


@pytest.mark.parametrize("starting", [True, False])
def test_triangle_attention_snapshot(starting):
    torch.manual_seed(123)
    c_z, c, heads = 128, 12, 4
    # Registration order: layer_norm.{weight,bias}, linear_z, mha.linear_{q,k,v,o,g}.
    shapes = [("layer_norm_w", (c_z,)), ("layer_norm_b", (c_z,))]
    lin = [("linear_z", c_z, heads), ("linear_q", c_z, c * heads), ("linear_k", c_z, c * heads),
           ("linear_v", c_z, c * heads), ("linear_o", c * heads, c_z), ("linear_g", c_z, c * heads)]
    for _, i, o in lin:
        _linear_rng(i, o)
    params = {}
    for name, shp in shapes:
        params[name] = torch.empty(shp).normal_(std=0.01)
    for name, i, o in lin:
        params[name] = torch.empty(o, i).normal_(std=0.01)
    x = torch.rand((2, 22, 22, c_z))
    out = triangle_attention_module(x.numpy(), {k: v.numpy() for k, v in params.items()}, heads,
                                    starting=starting)
    ref = np.load(GOLD / f"tri_att_cpu_starting_{starting}.npz")["output"]
    np.testing.assert_allclose(out, ref, **TOL)


def test_trimul_outgoing_snapshot():
    torch.manual_seed(123)
    c_z, c = 128, 11
    # Construction: linear_g, linear_z, (layer norms), linear_{a_p,a_g,b_p,b_g}.
    for i, o in ((c_z, c_z), (c, c_z), (c_z, c), (c_z, c), (c_z, c), (c_z, c)):
        _linear_rng(i, o)
    order = [("linear_g", (c_z, c_z)), ("linear_z", (c_z, c)), ("layer_norm_in_w", (c_z,)),
             ("layer_norm_in_b", (c_z,)), ("layer_norm_out_w", (c,)), ("layer_norm_out_b", (c,)),
             ("linear_a_p", (c, c_z)), ("linear_a_g", (c, c_z)), ("linear_b_p", (c, c_z)),
             ("linear_b_g", (c, c_z))]
    params = {name: torch.empty(shp).normal_(std=0.01).numpy() for name, shp in order}
    x = torch.rand((2, 22, 22, c_z))
    mask = torch.randint(0, 2, size=(2, 22, 22))
    out = trimul_module(x.numpy(), mask.numpy(), params, outgoing=True)
    ref = np.load(GOLD / "tri_mul_outgoing_cpu.npz")["output"]
    np.testing.assert_allclose(out, ref, **TOL)
