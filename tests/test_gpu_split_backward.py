"""The split backward route for direct callers (``split_backward.py``): dK / dV
with ``delta_true``, and dQ / per-batch dBias, from the forward's lse and a
caller-supplied delta.

* bitwise equal to the single-reconstruction backward (``tpf_attn_backward_bf16``)
  on the same lse / delta: dk, dv, dq, and dBias for a per-batch bias (each
  batch folds its own runs in both routes);
* every gradient within the bf16 tolerance of the FP64 oracle, including a
  shared bias with per-batch dBias (oracle: dS summed over that batch's
  outer rows) and a fully masked outer row;
* ``delta_true`` = sum_k P dP per query row, pinned to the closed form
  rowsum(dO * O) of the FP64 oracle's exact output (sum_k P_k (dO . v_k) =
  dO . sum_k P_k v_k), with exact zeros on fully masked rows;
* the reference release smoke's two "classic" cases
  (``tools/aot_numeric_smoke.py:130-139``: N=384 D=24, N=256 D=64 with two
  fully masked planes; no shadow residual) through forward + delta + the
  split route, held to its rule rel_L2 <= 1.1 * rel_L2(stock) + 1e-6.
"""

import math

import numpy as np
import pytest
import torch

from oracle.attention import attention_backward, attention_forward
from tests._util import attention_case, max_rel, record


def _npf(t):
    return t.detach().double().cpu().numpy()


def _forward_rows(q, k, v, mask, bias, dout, bb):
    """Kernel forward (out, lse) and delta = rowsum(dO * out), no residual."""
    from openfold3_triangle_kernel_amd import _native

    B, O, H, N, D = q.shape
    out = torch.empty(B, O, N, H, D, device=q.device, dtype=torch.bfloat16)
    lse = torch.empty(B, O, H, N, device=q.device, dtype=torch.float32)
    delta = torch.empty_like(lse)
    ws_n = int(_native.query("tpf_attn_forward_workspace_bytes", B, H, N, bb))
    ws = torch.empty(ws_n, device=q.device, dtype=torch.uint8)
    st = _native.stream_of(q)
    _native.call("tpf_attn_forward_bf16", q.data_ptr(), k.data_ptr(), v.data_ptr(), mask.data_ptr(),
                 bias.data_ptr(), out.data_ptr(), lse.data_ptr(), ws.data_ptr(), ws_n, B, O, H, N,
                 D, 0, bb, 1.0 / math.sqrt(D), st)
    _native.call("tpf_attn_delta_bf16", dout.data_ptr(), out.data_ptr(), delta.data_ptr(), B, O, H,
                 N, D, st)
    return out, lse, delta


def _sr_backward(q, k, v, mask, bias, dout, lse, delta, bb):
    from openfold3_triangle_kernel_amd import _native

    B, O, H, N, D = q.shape
    dq, dk, dv = (torch.empty_like(q) for _ in range(3))
    dbias = torch.empty(bb, H, N, N, device=q.device, dtype=torch.float32)
    ws_n = int(_native.query("tpf_attn_backward_workspace_bytes", B, O, H, N, D))
    ws = torch.empty(ws_n, device=q.device, dtype=torch.uint8)
    _native.call("tpf_attn_backward_bf16", q.data_ptr(), k.data_ptr(), v.data_ptr(),
                 dout.data_ptr(), lse.data_ptr(), delta.data_ptr(), mask.data_ptr(),
                 bias.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dbias.data_ptr(),
                 ws.data_ptr(), ws_n, B, O, H, N, D, 0, bb, 1.0 / math.sqrt(D),
                 _native.stream_of(q))
    return dq, dk, dv, dbias


def _bitwise(a, b):
    return torch.equal(a.contiguous().view(torch.uint8), b.contiguous().view(torch.uint8))


def _case(gpu, B, O, H, N, D, per_batch_bias, seed):
    q, k, v, mask, bias, dout = attention_case(B, O, H, N, D, mask_tail=16, random_tail=True,
                                               mask_frac=0.05, seed=seed)
    mask[:, 1] = float("-inf")  # one fully masked outer row per batch item
    if per_batch_bias:
        g = torch.Generator().manual_seed(seed + 100)
        bias = torch.randn(B, 1, H, N, N, generator=g).bfloat16().float()
    dev = dict(device=gpu)
    qd, kd, vd = (t.to(**dev).bfloat16() for t in (q, k, v))
    bias_d = bias.to(**dev).bfloat16().contiguous()
    return (q, k, v, mask, bias, dout), (qd, kd, vd, mask.to(**dev).contiguous(), bias_d,
                                         dout.to(**dev).bfloat16().contiguous())


@pytest.mark.gpu
@pytest.mark.parametrize("D,N", [(32, 128), (64, 192), (24, 128)])
@pytest.mark.parametrize("per_batch_bias", [True, False], ids=["bias_per_batch", "bias_shared"])
def test_split_route_matches_sr_and_oracle(gpu, D, N, per_batch_bias):
    from openfold3_triangle_kernel_amd.split_backward import (
        turbopairformer_triangle_dkdv,
        turbopairformer_triangle_dq_dbias,
    )

    B, O, H = 2, 9, 4
    print(f"[split] B={B} O={O} H={H} N={N} D={D} per_batch_bias={per_batch_bias}", flush=True)
    host, (q, k, v, mask, bias, dout) = _case(gpu, B, O, H, N, D, per_batch_bias, seed=D + N)
    bb = B if per_batch_bias else 1
    bias_in = bias if per_batch_bias else bias.expand(B, 1, H, N, N)
    out, lse, delta = _forward_rows(q, k, v, mask, bias, dout, bb)
    dk, dv, dtrue = turbopairformer_triangle_dkdv(q, k, v, dout, lse, delta, mask, bias_in,
                                                  emit_delta_true=True)
    dq, dbias = turbopairformer_triangle_dq_dbias(q, k, v, dout, lse, delta, mask, bias_in)
    torch.cuda.synchronize()
    assert dbias.shape == (B, 1, H, N, N) and dbias.dtype == torch.float32
    sq, sk, sv, sdb = _sr_backward(q, k, v, mask, bias, dout, lse, delta, bb)
    torch.cuda.synchronize()
    assert _bitwise(dk, sk) and _bitwise(dv, sv), "dK / dV differ from the SR backward"
    assert _bitwise(dq, sq), "dQ differs from the SR backward"
    if per_batch_bias:
        assert _bitwise(dbias.reshape(B, H, N, N), sdb), "dBias differs from the SR backward"

    # FP64 oracle on the bf16-rounded inputs; dBias per batch item.
    qh, kh, vh, mh, bh, doh = (t.double().numpy() for t in host)
    bias_full = np.broadcast_to(bh, (B, 1, H, N, N))
    ref_out, _, _ = attention_forward(qh, kh, vh, mh, bias_full)
    rdq, rdk, rdv, rdb = attention_backward(qh, kh, vh, mh, bias_full, doh)
    for name, got, ref in (("dq", dq, rdq), ("dk", dk, rdk), ("dv", dv, rdv),
                           ("dbias", dbias, rdb)):
        err = max_rel(_npf(got), ref)
        print(f"  {name} max-rel {err:.2e}", flush=True)
        assert err <= 2e-2, f"{name}: {err:.3e}"

    # delta_true against the closed form rowsum(dO * O_exact).
    o64 = np.swapaxes(ref_out, -2, -3)                 # [B, O, H, N, D]
    do64 = np.swapaxes(doh, -2, -3)
    want = (do64 * o64).sum(-1)                        # [B, O, H, N]
    got = _npf(dtrue)
    assert np.all(got[:, 1] == 0), "fully masked rows must give delta_true = 0"
    err = float(np.linalg.norm(got - want) / np.linalg.norm(want))
    print(f"  delta_true rel-L2 vs rowsum(dO * O_exact) {err:.2e}", flush=True)
    assert err <= 1e-3, err
    # The caller's delta (from the bf16 output) differs from it at bf16 level.
    assert float(np.abs(_npf(delta) - got).max()) > 0.0


@pytest.mark.gpu
def test_dkdv_without_delta_true_and_supplied_buffers(gpu):
    from openfold3_triangle_kernel_amd.split_backward import (
        delta_true_partial_elements,
        turbopairformer_triangle_dkdv,
        turbopairformer_triangle_dq_dbias,
    )

    B, O, H, N, D = 1, 5, 4, 128, 32
    _, (q, k, v, mask, bias, dout) = _case(gpu, B, O, H, N, D, False, seed=3)
    out, lse, delta = _forward_rows(q, k, v, mask, bias, dout, 1)
    dk, dv = turbopairformer_triangle_dkdv(q, k, v, dout, lse, delta, mask, bias)
    parts = torch.empty(delta_true_partial_elements(N, H, B, outer=O), device=gpu)
    bk, bv_, bt = torch.empty_like(q), torch.empty_like(q), torch.empty(B, O, H, N, device=gpu)
    r = turbopairformer_triangle_dkdv(q, k, v, dout, lse, delta, mask, bias, out_dk=bk, out_dv=bv_,
                                      emit_delta_true=True, delta_true_partials=parts,
                                      out_delta_true=bt)
    assert r[0] is bk and r[1] is bv_ and r[2] is bt
    ws = torch.empty(1024, device=gpu, dtype=torch.bfloat16)  # below the plan's minimum
    with pytest.raises(ValueError, match="workspace"):
        turbopairformer_triangle_dq_dbias(q, k, v, dout, lse, delta, mask, bias, workspace=ws)
    dq1, db1 = turbopairformer_triangle_dq_dbias(q, k, v, dout, lse, delta, mask, bias,
                                                 debug_full_plane=True)
    dq2, db2 = turbopairformer_triangle_dq_dbias(q, k, v, dout, lse, delta, mask, bias,
                                                 workspace_budget_bytes=1)
    torch.cuda.synchronize()
    assert _bitwise(dk, bk) and _bitwise(dv, bv_)
    assert _bitwise(dq1, dq2) and _bitwise(db1, db2), "slabbed dq_dbias differs"
    with pytest.raises(ValueError, match="requires"):
        turbopairformer_triangle_dkdv(q, k, v, dout, lse, delta, mask, bias, emit_delta_true=True,
                                      delta_true_partials=parts[:10])


# (name, B, O, H, N, D, mask_frac, full_planes): tools/aot_numeric_smoke.py:130-139
CLASSIC = [
    ("classic N=384 D=24", 1, 4, 4, 384, 24, 0.2, 0),
    ("classic N=256 D=64 full planes", 1, 6, 4, 256, 64, 0.2, 2),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", CLASSIC, ids=[c[0] for c in CLASSIC])
def test_classic_smoke_cases_through_split_route(gpu, case):
    from openfold3_triangle_kernel_amd.split_backward import (
        turbopairformer_triangle_dkdv,
        turbopairformer_triangle_dq_dbias,
    )
    from tests.test_gpu_numerics import _inputs, _rel, _stock

    name, B, O, H, N, D, frac, full = case
    print(f"[classic] {name}", flush=True)
    inputs = _inputs(B, O, H, N, D, frac, full)
    q, k, v, mask, bias, dout = (t.to(gpu) for t in inputs)
    mask = mask.contiguous()
    out, lse, delta = _forward_rows(q, k, v, mask, bias, dout, 1)
    dk, dv = turbopairformer_triangle_dkdv(q, k, v, dout, lse, delta, mask,
                                           bias.expand(B, 1, H, N, N))
    dq, dbias = turbopairformer_triangle_dq_dbias(q, k, v, dout, lse, delta, mask,
                                                  bias.expand(B, 1, H, N, N))
    torch.cuda.synchronize()
    got = [_npf(t) for t in (out, dq, dk, dv, dbias.sum(0, keepdim=True))]
    assert all(np.isfinite(t).all() for t in got)
    stock = _stock(q, k, v, mask, bias, dout)
    qh, kh, vh, mh, bh, doh = (t.float().numpy() for t in inputs)
    ref_out, _, _ = attention_forward(qh, kh, vh, mh, bh)
    ref = [ref_out, *attention_backward(qh, kh, vh, mh, bh, doh)]
    if full:
        for t in got[:4]:
            assert np.all(t[:, :full] == 0), f"{name}: fully masked planes must be zero"
        got[0], stock[0], ref[0] = got[0][:, full:], stock[0][:, full:], ref[0][:, full:]
    rows = {}
    for i, label in enumerate(("out", "dq", "dk", "dv", "dbias")):
        e, es = _rel(got[i], ref[i]), _rel(stock[i], ref[i])
        rows[label] = {"ours": e, "stock": es, "limit": 1.1 * es + 1e-6}
        print(f"  {label}: {e:.2e} / stock {es:.2e}", flush=True)
    record("attention_release_gate_rel_l2", f"{name} (split route, no shadow)", rows)
    for label, r in rows.items():
        assert r["ours"] <= r["limit"], f"{name} {label}: {r}"
