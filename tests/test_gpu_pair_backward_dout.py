"""The fused pair-row backward (tpf_attn_pair_backward_dout_bf16) through the
C ABI: d_og = dout W_o on the weight-stationary row kernel with the output
gate's backward (d_o, the gate gradient, delta) in its epilogue must give the
whole projection-gradient row bitwise equal to the two-step route it
replaces, tpf_gemm_bf16 (dout, W_o) then tpf_attn_pair_backward_bf16, whose
results the module tests pin against the stock FP32 module math.  Both node
orders (og rows plain or transposed), shadow residual on and off, and every
supported head width."""

import math

import pytest
import torch

from openfold3_triangle_kernel_amd import _native

CASES = [
    # B, N, H, D, og_t, shadow
    (1, 64, 4, 32, False, True),
    (1, 64, 4, 32, True, True),
    (2, 64, 2, 16, True, False),
    (1, 128, 2, 64, False, False),
    (1, 64, 8, 16, True, True),
    (1, 64, 1, 16, False, True),
    (1, 128, 16, 8, True, False),
]


def _call(name, *args):
    _native.call(name, *args)


@pytest.mark.gpu
@pytest.mark.parametrize("B,N,H,D,og_t,shadow", CASES,
                         ids=lambda v: str(int(v)) if isinstance(v, bool) else str(v))
def test_pair_backward_from_dout_matches_two_step(gpu, B, N, H, D, og_t, shadow):
    C, hc = 128, H * D
    R = B * N * N
    rest_pitch = (hc + H + 7) // 8 * 8
    P = 3 * hc + rest_pitch
    assert _native.query("tpf_attn_pair_backward_dout_supported", C, H, D)
    g = torch.Generator(device=gpu).manual_seed(1000 * N + 10 * H + D)

    def rnd(*shape, std=1.0):
        return (torch.randn(*shape, generator=g, device=gpu) * std).bfloat16()

    qkv = rnd(3, B, N, H, N, D)
    rest = rnd(R, rest_pitch)
    mask = torch.where(torch.rand(B, N, N, generator=g, device=gpu) < 0.1,
                       torch.tensor(-1e9, device=gpu), torch.tensor(0.0, device=gpu))
    mask[..., 0] = 0.0  # no fully masked row
    flags = 2 if og_t else 0
    o = torch.empty(R, hc, device=gpu, dtype=torch.bfloat16)
    og = torch.empty_like(o)
    res = torch.empty_like(o) if shadow else None
    lse = torch.empty(B, N, H, N, device=gpu, dtype=torch.float32)
    fws = int(_native.query("tpf_attn_pair_forward_workspace_bytes", B, N, H))
    fw = torch.empty(fws, device=gpu, dtype=torch.uint8)
    scale = 1.0 / math.sqrt(D)
    stream = _native.stream_of(o)
    print(f"pair backward from dout: B={B} N={N} H={H} D={D} og_t={og_t} shadow={shadow}",
          flush=True)
    _call("tpf_attn_pair_forward_bf16", qkv.data_ptr(), rest.data_ptr(), rest_pitch,
          mask.data_ptr(), flags, o.data_ptr(), lse.data_ptr(), og.data_ptr(), _native.ptr(res),
          fw.data_ptr(), fws, B, N, H, D, scale, stream)
    dout = rnd(R, C)
    w_o = rnd(C, hc, std=0.1)
    bws = int(_native.query("tpf_attn_pair_backward_workspace_bytes", B, N, H, D))
    common = (qkv.data_ptr(), rest.data_ptr(), rest_pitch, mask.data_ptr(), flags, o.data_ptr(),
              lse.data_ptr(), _native.ptr(res))
    outs = []
    for fused in (False, True):
        dproj = torch.full((R, P), 7.0, device=gpu, dtype=torch.bfloat16)
        ws = torch.empty(bws, device=gpu, dtype=torch.uint8)
        tail = (dproj.data_ptr(), P, ws.data_ptr(), bws, B, N, H, D, scale, stream)
        if fused:
            _call("tpf_attn_pair_backward_dout_bf16", *common, dout.data_ptr(), w_o.data_ptr(), C,
                  *tail)
        else:
            d_og = torch.empty(R, hc, device=gpu, dtype=torch.bfloat16)
            _call("tpf_gemm_bf16", dout.data_ptr(), 1, C, 0, w_o.data_ptr(), 0, hc, 0,
                  d_og.data_ptr(), 0, hc, 0, R, hc, C, 1, 1.0, stream)
            _call("tpf_attn_pair_backward_bf16", *common, d_og.data_ptr(), *tail)
        outs.append(dproj)
    torch.cuda.synchronize()
    assert torch.isfinite(outs[0].float()).all()
    assert torch.equal(outs[0], outs[1])


@pytest.mark.gpu
def test_pair_backward_from_dout_rejects_unsupported(gpu):
    """A head width without an instance is refused before any launch."""
    assert not _native.query("tpf_attn_pair_backward_dout_supported", 128, 4, 24)
    t = torch.zeros(1024, device=gpu, dtype=torch.bfloat16)
    p = t.data_ptr()
    with pytest.raises(RuntimeError, match="no fused instance"):
        _call("tpf_attn_pair_backward_dout_bf16", p, p, 104, p, 0, p, p, None, p, p, 128, p, 400,
              p, 0, 1, 64, 4, 24, 0.2, _native.stream_of(t))
