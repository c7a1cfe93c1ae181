#!/usr/bin/env python3
"""Benchmark of the TurboPairFormer hot path on one MI355X.

Metric: tri-attn fwd+bwd ms & TFLOP/s at N=384, H=4, D=32
bf16; TriMul fwd+bwd ms.

A step is one pass of the hot path over one batch of synthetic input:
  * triangle attention fwd+bwd, starting node and ending node (config 3:
    q, k, v [1,384,4,384,32] ~ N(0,1), pair_bias 2*N(0,1) [1,1,4,384,384],
    res_mask with a random 0-32 key -inf tail per outer row; the ending node
    runs the same op on the pair transposed over its two N axes, with the
    bias as a transposed view);
  * TriMul outgoing + incoming fwd+bwd (config 4: z [1,384,384,128] ~ N(0,1),
    LN weights 1/0, projections ~ N(0, 1/sqrt(128)), mask all ones), timed
    as its own loop and reported under "trimul".
``value`` is the attention fwd+bwd throughput in algorithmic TFLOP/s
(14*B*O*H*N^2*D per variant), inputs resident in HBM before timing; step
times are the median of per-step HIP-event times over exactly ``--steps``
steps after ``--warmup`` untimed ones (defaults 50 and 10).

Also reported: config 5 (attention at N=768, H=4 D=32 and H=8 D=64, and the
pair-stack block TriMul-out -> TriMul-in -> TriAtt-start -> TriAtt-end
through the modules; ``--no-config5`` skips it), the FP32 inference mode,
the roofline of the dominant kernel (the attention backward kernel, timed
alone with HIP events on the launching stream) and a CPU baseline (the stock
PyTorch math in FP32 on the host cores, configs 1, 3 and 4 in full).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
HBM_PEAK_GBPS = 8000.0           # MI355X HBM3E

B, O, H, N, D = 1, 384, 4, 384, 32
TM_N, TM_C = 384, 128
PROBE_PASSES = 6


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-trimul", action="store_true")
    ap.add_argument("--no-fp32", action="store_true", help="skip the FP32 inference-mode timings")
    ap.add_argument("--no-config5", action="store_true",
                    help="skip config 5 (attention at N=768: H=4 D=32 and H=8 D=64, and the "
                         "pair-stack block through the modules); for profiling runs whose kernel "
                         "trace should hold only the config-3 / config-4 launches")
    ap.add_argument("--kernel-reps", type=int, default=20)
    ap.add_argument("--probe", choices=("attention", "trimul", "pair-block"),
                    help="launch a 256 MiB calibration copy, then two fwd+bwd passes of one path "
                         "(attention: config 3 starting node; trimul: config 4 outgoing + incoming) "
                         "six times and exit: the program that the per-kernel rocprofv3 counter passes "
                         "profile (the last pass is the steady-state one)")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="launch a 256 MiB calibration copy and one attention backward kernel, "
                         "then exit (the program profiled by the FETCH_SIZE / WRITE_SIZE passes)")
    return ap.parse_args()


def gpu_time(torch, fn, steps, warmup):
    """Run ``warmup`` untimed steps, then exactly ``steps`` timed ones, each
    bracketed by HIP events on the current stream; the whole timed region is
    bracketed by device synchronisation.  Returns the median and mean step
    time in ms (median: the GPU clock ramps over the first seconds)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    t0 = time.perf_counter()
    for a, b in ev:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    ts = sorted(a.elapsed_time(b) for a, b in ev)
    return {"median": ts[len(ts) // 2], "mean": sum(ts) / len(ts), "wall": wall}


def trimul_inputs(torch, dev, seed=1):
    """Config 4: z [1,384,384,128] ~ N(0,1) bf16, LN weights 1 / 0, projections
    ~ N(0, 1/sqrt(128)) in the named-argument layout, mask all ones."""
    g = torch.Generator(device=dev).manual_seed(seed)
    C = TM_C
    z = torch.randn(1, TM_N, TM_N, C, device=dev, generator=g).to(torch.bfloat16).requires_grad_(True)
    sd = 1.0 / math.sqrt(C)
    wts = dict(
        norm_in_weight=torch.ones(C, device=dev), norm_in_bias=torch.zeros(C, device=dev),
        p_in_weight=torch.randn(2 * C, C, device=dev, generator=g) * sd,
        g_in_weight=torch.randn(2 * C, C, device=dev, generator=g) * sd,
        norm_out_weight=torch.ones(C, device=dev), norm_out_bias=torch.zeros(C, device=dev),
        p_out_weight=torch.randn(C, C, device=dev, generator=g) * sd,
        g_out_weight=torch.randn(C, C, device=dev, generator=g) * sd,
    )
    wts = {kk: vv.requires_grad_(True) for kk, vv in wts.items()}
    mask = torch.ones(1, TM_N, TM_N, device=dev)
    dout = torch.randn(1, TM_N, TM_N, C, device=dev, generator=g).to(torch.bfloat16)
    return z, wts, mask, dout


def pair_block_setup(torch, dev):
    """Config 5's pair block through the drop-in modules (TriMul out, TriMul
    in, triangle attention starting and ending node, residual adds) at
    N = 768, C = 128, H = 4, D = 32; returns its fwd+bwd step and the state
    that keeps its tensors alive."""
    from openfold3_triangle_kernel_amd import (
        TriangleAttention,
        TriangleMultiplicationIncoming,
        TriangleMultiplicationOutgoing,
    )

    torch.manual_seed(5)
    Np, Cz = 768, 128
    mods = [TriangleMultiplicationOutgoing(Cz, Cz), TriangleMultiplicationIncoming(Cz, Cz),
            TriangleAttention(Cz, 32, 4, starting=True), TriangleAttention(Cz, 32, 4, starting=False)]
    for mo in mods:
        for prm in mo.parameters():
            if prm.dim() == 2:
                torch.nn.init.normal_(prm, std=1.0 / math.sqrt(prm.shape[1]))
    mods = [mo.to(dev, torch.bfloat16) for mo in mods]
    zp = torch.randn(1, Np, Np, Cz, device=dev).to(torch.bfloat16).requires_grad_(True)
    mp = torch.ones(1, Np, Np, device=dev, dtype=torch.bfloat16)
    params = [zp] + [prm for mo in mods for prm in mo.parameters()]

    # A fixed upstream gradient (seeded N(0,1) bf16) drives the backward, as
    # the measurement rules allow (autograd.grad with a fixed grad_out): the
    # block is timed without an FP32 loss's elementwise passes.
    g = torch.Generator(device=dev).manual_seed(6)
    dh = torch.randn(1, Np, Np, Cz, device=dev, generator=g).to(torch.bfloat16)

    def block_step():
        h = zp
        for mo in mods:
            h = h + mo(h, mp)
        torch.autograd.grad(h, params, dh)

    return block_step, (zp, mods, params, dh)


def probe(torch, dev, target):
    """Calibration copy (256 MiB read + 256 MiB written), then six fwd+bwd
    passes of one path, for per-kernel counter passes (the last pass runs
    with warm clocks and caches)."""
    from openfold3_triangle_kernel_amd import turbo_trimul, turbopairformer_triangle_attention

    src = torch.ones(64 * 1024 * 1024, device=dev, dtype=torch.float32)  # 256 MiB
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    if target == "pair-block":
        block_step, _state = pair_block_setup(torch, dev)
        for _ in range(PROBE_PASSES):
            block_step()
    elif target == "attention":
        q, k, v, bias, mask, dout = attention_inputs(torch, dev)
        xs = [t.detach().requires_grad_(True) for t in (q, k, v, bias)]
        for _ in range(PROBE_PASSES):
            out = turbopairformer_triangle_attention(xs[0], xs[1], xs[2], mask, xs[3])
            torch.autograd.grad(out, xs, dout)
    else:
        z, wts, mask, dout = trimul_inputs(torch, dev)
        params = [z] + list(wts.values())
        for _ in range(PROBE_PASSES):
            for direction in ("outgoing", "incoming"):
                o = turbo_trimul(z, direction, mask, **wts)
                torch.autograd.grad(o, params, dout)
    torch.cuda.synchronize()
    print(f"probe {target}: copy 268435456 B read + 268435456 B written; {PROBE_PASSES} fwd+bwd "
          "passes", flush=True)


def attention_inputs(torch, dev, seed=0):
    g = torch.Generator(device=dev).manual_seed(seed)
    q, k, v = (torch.randn(B, O, H, N, D, device=dev, generator=g).to(torch.bfloat16) for _ in range(3))
    bias = (torch.randn(1, 1, H, N, N, device=dev, generator=g) * 2).to(torch.bfloat16)
    tails = torch.randint(0, 33, (B, O), device=dev, generator=g)
    ar = torch.arange(N, device=dev)
    mask = torch.where(ar[None, None, :] >= (N - tails)[..., None], float("-inf"), 0.0)
    mask = mask.reshape(B, O, 1, 1, N).float()
    dout = torch.randn(B, O, N, H, D, device=dev, generator=g).to(torch.bfloat16)
    return q, k, v, bias, mask, dout


def dominant_kernel(torch, _native, dev, q, k, v, bias, mask, dout):
    """Inputs, forward state and workspace of one attention backward launch
    (starting node); returns a closure that launches the backward kernel."""
    stream = torch.cuda.current_stream().cuda_stream
    scale = 1.0 / math.sqrt(D)
    out = torch.empty(B, O, N, H, D, device=dev, dtype=torch.bfloat16)
    lse = torch.empty(B, O, H, N, device=dev, dtype=torch.float32)
    delta = torch.empty_like(lse)
    mflat = mask.reshape(B, O, N).contiguous()
    bflat = bias.reshape(1, H, N, N).contiguous()
    fws_bytes = int(_native.query("tpf_attn_forward_workspace_bytes", B, H, N, 1))
    fws = torch.empty(fws_bytes, device=dev, dtype=torch.uint8)
    _native.call("tpf_attn_forward_bf16", q.data_ptr(), k.data_ptr(), v.data_ptr(), mflat.data_ptr(),
                 bflat.data_ptr(), out.data_ptr(), lse.data_ptr(), fws.data_ptr(), fws_bytes,
                 B, O, H, N, D, 0, 1, scale, stream)
    _native.call("tpf_attn_delta_bf16", dout.data_ptr(), out.data_ptr(), delta.data_ptr(), B, O, H, N, D,
                 stream)
    dk, dv = torch.empty_like(q), torch.empty_like(q)
    ws_bytes = int(_native.query("tpf_attn_backward_workspace_bytes", B, O, H, N, D))
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)

    def bwd_main():
        _native.call("tpf_attn_backward_main_bf16", q.data_ptr(), k.data_ptr(), v.data_ptr(),
                     dout.data_ptr(), lse.data_ptr(), delta.data_ptr(), mflat.data_ptr(),
                     bflat.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), ws_bytes,
                     B, O, H, N, D, 0, 1, scale, stream)

    return bwd_main


def main():
    args = parse()
    if args.gpus != 1:
        print(
            f"bench.py: --gpus {args.gpus} is not supported; this build measures one MI355X "
            "(the hot path has no collectives: one GPU's share is the whole kernel workload)",
            file=sys.stderr,
        )
        sys.exit(2)
    import torch

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from openfold3_triangle_kernel_amd import _native, turbo_trimul, turbopairformer_triangle_attention

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.probe:
        probe(torch, dev, args.probe)
        return

    # ---------------- attention: starting + ending node -----------------
    q, k, v, bias, mask, dout = attention_inputs(torch, dev)
    if args.traffic_probe:
        bwd_main = dominant_kernel(torch, _native, dev, q, k, v, bias, mask, dout)
        src = torch.ones(64 * 1024 * 1024, device=dev, dtype=torch.float32)  # 256 MiB
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        bwd_main()
        torch.cuda.synchronize()
        print("traffic probe: copy 268435456 B read + 268435456 B written; one attn_bwd launch", flush=True)
        return

    # Ending node: the same op on the pair transposed over its two N axes.
    qe, ke, ve = (t.transpose(1, 3).contiguous() for t in (q, k, v))
    mask_e = mask.clone()
    bias_e = bias.transpose(-1, -2)  # transposed view (reference transpose_bias path)
    dout_e = dout.clone()
    variants = [
        [t.detach().requires_grad_(True) for t in (q, k, v)] + [bias.detach().requires_grad_(True), mask, dout],
        [t.detach().requires_grad_(True) for t in (qe, ke, ve)]
        + [bias_e.detach().requires_grad_(True), mask_e, dout_e],
    ]

    def attn_step():
        for vq, vk, vv, vb, vm, vd in variants:
            out = turbopairformer_triangle_attention(vq, vk, vv, vm, vb)
            torch.autograd.grad(out, (vq, vk, vv, vb), vd)

    at = gpu_time(torch, attn_step, args.steps, args.warmup)
    ms_step, wall_ms = at["median"], at["wall"]
    attn_flops = 2 * 14.0 * B * O * H * N * N * D  # two variants
    attn_tflops = attn_flops / (ms_step * 1e-3) / 1e12
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    # Forward-only timing (starting node) for the breakdown.
    with torch.no_grad():
        fwd_ms = gpu_time(torch, lambda: turbopairformer_triangle_attention(q, k, v, mask, bias),
                          args.steps, 3)["median"]

    # ------------- dominant kernel: attention backward, alone -------------
    bwd_main = dominant_kernel(torch, _native, dev, q, k, v, bias, mask, dout)
    for _ in range(3):
        bwd_main()
    torch.cuda.synchronize()
    e0.record()
    for _ in range(args.kernel_reps):
        bwd_main()
    e1.record()
    torch.cuda.synchronize()
    bwd_kernel_ms = e0.elapsed_time(e1) / args.kernel_reps
    bwd_flops = 10.0 * B * O * H * N * N * D
    achieved = bwd_flops / (bwd_kernel_ms * 1e-3) / 1e12
    roofline = {
        "kernel": "attn_bwd_kernel<32> (timed with its attn_bwd_prep_kernel launch)",
        "bound": "mfma",
        "achieved": round(achieved, 2),
        "peak": MFMA_BF16_PEAK_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4),
        "traffic": traffic_bytes(),
        "avg_launch_us": round(bwd_kernel_ms * 1e3, 2),
        "flops_per_launch": bwd_flops,
    }

    # ------------- config 5 attention shapes (starting node) -------------
    config5_attention = None
    if not args.no_config5:
        config5_attention = []
        reps = max(10, args.steps // 4)
        for H5, D5 in ((4, 32), (8, 64)):
            N5 = 768
            g5 = torch.Generator(device=dev).manual_seed(5)
            qkv5 = [torch.randn(1, N5, H5, N5, D5, device=dev, generator=g5).to(torch.bfloat16)
                    .requires_grad_(True) for _ in range(3)]
            bias5 = torch.randn(1, 1, H5, N5, N5, device=dev, generator=g5).to(torch.bfloat16)
            bias5.requires_grad_(True)
            mask5 = torch.zeros(1, N5, 1, 1, N5, device=dev)
            dout5 = torch.randn(1, N5, N5, H5, D5, device=dev, generator=g5).to(torch.bfloat16)

            def step5():
                o5 = turbopairformer_triangle_attention(*qkv5, mask5, bias5)
                torch.autograd.grad(o5, (*qkv5, bias5), dout5)

            ms5 = gpu_time(torch, step5, reps, 3)["median"]
            fl5 = 14.0 * N5 * H5 * N5 * N5 * D5
            config5_attention.append({"N": N5, "O": N5, "H": H5, "D": D5, "ms_fwd_bwd": round(ms5, 3),
                                      "tflops": round(fl5 / (ms5 * 1e-3) / 1e12, 2), "steps": reps})
            del qkv5, bias5, mask5, dout5
        torch.cuda.empty_cache()

    # --------------------------- TriMul ----------------------------------
    trimul = None
    if not args.no_trimul:
        C = TM_C
        z, wts, tm_mask, tm_dout = trimul_inputs(torch, dev)
        params = [z] + list(wts.values())

        def tm_step():
            for direction in ("outgoing", "incoming"):
                o = turbo_trimul(z, direction, tm_mask, **wts)
                torch.autograd.grad(o, params, tm_dout)

        tm_ms = gpu_time(torch, tm_step, args.steps, args.warmup)["median"]
        R = TM_N * TM_N
        tm_fwd_flops = 2.0 * R * C * 5 * C + 2.0 * C * TM_N ** 3 + 2.0 * R * C * C
        tm_flops = 2 * 3 * tm_fwd_flops
        # Per-stage roofline sum_s max(F_s / P_mfma, B_s / BW_hbm) with the
        # minimum bytes of each direction (12 U forward, 20 U backward, U =
        # rows * C * 2 B); at C = 128 every stage is HBM-bound (the
        # contraction's 14.5 GFLOP take 5.8 us at the MFMA peak against 14 us
        # for its 3 U), so the sum is the byte term.
        U = TM_N * TM_N * C * 2
        roof_ms = 2 * 32 * U / (HBM_PEAK_GBPS * 1e9) * 1e3
        trimul = {
            "ms_fwd_bwd_out_plus_in": round(tm_ms, 4),
            "tflops": round(tm_flops / (tm_ms * 1e-3) / 1e12, 2),
            "flops": tm_flops,
            "roofline_ms": round(roof_ms, 4),
            "roofline_frac": round(roof_ms / tm_ms, 4),
            "roofline_basis": "sum over stages of max(F/P, B/BW); minimum bytes 12U fwd + 20U bwd "
                              "per direction at 8 TB/s (all stages HBM-bound at C=128)",
            "traffic": trimul_traffic_bytes(),
            "min_bytes": int(2 * 32 * U),
            "config": {"N": TM_N, "C": C, "H": C, "directions": ["outgoing", "incoming"]},
        }

    # ------------------- FP32 inference mode (no autograd) ---------------
    fp32 = None
    if not args.no_fp32:
        from types import SimpleNamespace

        from openfold3_triangle_kernel_amd import run_trimul_fp32, turbopairformer_attention_fp32

        with torch.no_grad():
            qf, kf, vf, bf = (t.float() for t in (q, k, v, bias))
            for _ in range(2):
                turbopairformer_attention_fp32(qf, kf, vf, mask, bf)
            torch.cuda.synchronize()
            e0.record()
            for _ in range(args.steps):
                turbopairformer_attention_fp32(qf, kf, vf, mask, bf)
            e1.record()
            torch.cuda.synchronize()
            att32_ms = e0.elapsed_time(e1) / args.steps
            del qf, kf, vf, bf
            C = TM_C
            g32 = torch.Generator(device=dev).manual_seed(2)

            def lin(i, o):
                layer = torch.nn.Linear(i, o, bias=False, device=dev)
                with torch.no_grad():
                    layer.weight.copy_(torch.randn(o, i, device=dev, generator=g32) / math.sqrt(i))
                return layer

            mod = SimpleNamespace(c_z=C, c_hidden=C, _outgoing=True,
                                  linear_a_p=lin(C, C), linear_a_g=lin(C, C),
                                  linear_b_p=lin(C, C), linear_b_g=lin(C, C),
                                  linear_g=lin(C, C), linear_z=lin(C, C),
                                  layer_norm_in=torch.nn.LayerNorm(C, device=dev),
                                  layer_norm_out=torch.nn.LayerNorm(C, device=dev))
            z32 = torch.randn(1, TM_N, TM_N, C, device=dev, generator=g32)
            m32 = torch.ones(1, TM_N, TM_N, device=dev)

            def tm32_step():
                for outgoing in (True, False):
                    mod._outgoing = outgoing
                    run_trimul_fp32(mod, z32, m32)

            tm32_step()
            torch.cuda.synchronize()
            e0.record()
            for _ in range(args.steps):
                tm32_step()
            e1.record()
            torch.cuda.synchronize()
            tm32_ms = e0.elapsed_time(e1) / args.steps
        att32_flops = 4.0 * B * O * H * N * N * D
        tm32_flops = 2 * (2.0 * TM_N * TM_N * C * 5 * C + 2.0 * C * TM_N ** 3 + 2.0 * TM_N * TM_N * C * C)
        fp32 = {
            "attention_fwd_ms": round(att32_ms, 4),
            "attention_fwd_tflops": round(att32_flops / (att32_ms * 1e-3) / 1e12, 2),
            "trimul_fwd_out_plus_in_ms": round(tm32_ms, 4),
            "trimul_fwd_tflops": round(tm32_flops / (tm32_ms * 1e-3) / 1e12, 2),
            "peak_fp32_mfma_tflops": 157.3,
            "note": "inference-only FP32 mode (no autograd), config 3 starting node / config 4",
        }

    # ------------- config 5: pair-stack block at N=768 (modules) -----------
    pair_block = None
    if not args.no_config5:
        block_step, pb_state = pair_block_setup(torch, dev)
        blk_ms = gpu_time(torch, block_step, max(10, args.steps // 4), 3)["median"]
        pair_block = {
            "ms_fwd_bwd": round(blk_ms, 3),
            "config": {"N": 768, "C": 128, "blocks": ["trimul_out", "trimul_in", "tri_att_start",
                                                      "tri_att_end"], "H": 4, "D": 32},
            "note": "config 5: residual pair block through the drop-in modules (bf16 params; "
                    "LayerNorm, projections, attention core, gate and TriMul in the HIP kernels, "
                    "the residual adds in torch); backward driven by a fixed bf16 grad_out",
        }
        del pb_state

    # -------------------------- CPU baseline -----------------------------
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline()

    line = {
        "metric": "tri-attn fwd+bwd ms & TFLOP/s (N=384,H=4,D=32 bf16); TriMul fwd+bwd ms",
        "value": round(attn_tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) inputs of the config-3/config-4 shapes)",
        "config": {
            "workload": "triangle attention fwd+bwd, starting + ending node (config 3)",
            "B": B, "O": O, "H": H, "N": N, "D": D,
            "parallelism": "single GPU",
        },
        "attention": {
            "ms_fwd_bwd_start_plus_end": round(ms_step, 4),
            "ms_mean": round(at["mean"], 4),
            "timing": "median of per-step HIP-event times",
            "ms_fwd_start": round(fwd_ms, 4),
            "host_wall_ms_per_step": round(wall_ms, 4),
            "mfma_frac": round(attn_tflops / MFMA_BF16_PEAK_TFLOPS, 4),
        },
        "trimul": trimul,
        "config5_attention": config5_attention,
        "fp32_inference": fp32,
        "pair_block": pair_block,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                            "attn_bwd_N384_H4_D32_traffic.json")


def traffic_bytes():
    """HBM bytes per launch of the attention backward kernel, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE passes over ``bench.py --traffic-probe``,
    each scaled by the same counter's reading on a 256 MiB copy (None when the
    summary is absent)."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        return int(t["fetch_bytes_calibrated"] + t["write_bytes_calibrated"])
    except (OSError, KeyError, ValueError):
        return None


TRIMUL_TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                                   "trimul_N384_C128_traffic.json")


def trimul_traffic_bytes():
    """HBM bytes of one TriMul out + in fwd + bwd step, summed over the
    library's kernels from the committed FETCH_SIZE / WRITE_SIZE passes over
    ``bench.py --probe trimul`` (None when the summary is absent)."""
    try:
        with open(TRIMUL_TRAFFIC_FILE) as f:
            t = json.load(f)
        return int(t["fetch_bytes_calibrated"] + t["write_bytes_calibrated"])
    except (OSError, KeyError, ValueError):
        return None


def _cpu_threads() -> int:
    """Host cores this process may run on (the cgroup / affinity share)."""
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1


def _median_time(fn, reps, warmup):
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2] * 1e3, ts


def cpu_baseline():
    """The stock PyTorch math in FP32 on the host cores (oracle/stock_torch.py,
    a restatement of OpenFold3's ``_attention`` and TriMul forward with
    autograd for the backward), on the same seeded workloads:

    * config 1 in full: attention fwd+bwd [1,64,4,64,32], mask zeros;
    * config 3 in full: attention fwd+bwd, starting + ending node
      [1,384,4,384,32], chunked over the outer rows (the stock chunked path);
    * config 4 in full: TriMul outgoing + incoming fwd+bwd [1,384,384,128].

    Median of 5 timed runs after 2 warm-ups each; ``value`` is config 3 in
    the headline unit (TFLOP/s), so it sits beside the GPU figure.
    """
    import torch

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle.stock_torch import attention_stock_train_step, trimul_stock

    cores = _cpu_threads()
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(0)
    reps, warm = 5, 2

    def attn_case(O_, N_, bias_scale, tail):
        q_, k_, v_ = (torch.randn(1, O_, H, N_, D, generator=g) for _ in range(3))
        b_ = torch.randn(1, 1, H, N_, N_, generator=g) * bias_scale
        m_ = torch.zeros(1, O_, 1, 1, N_)
        if tail:
            tails = torch.randint(0, tail + 1, (O_,), generator=g)
            for o_ in range(O_):
                if int(tails[o_]):
                    m_[0, o_, ..., N_ - int(tails[o_]):] = float("-inf")
        d_ = torch.randn(1, O_, N_, H, D, generator=g)
        return q_, k_, v_, m_, b_, d_

    # Config 1.
    c1 = attn_case(64, 64, 1.0, 0)
    c1_ms, _ = _median_time(lambda: attention_stock_train_step(*c1), reps, warm)
    # Config 3: starting node and ending node (transposed pair, transposed bias).
    q3, k3, v3, m3, b3, d3 = attn_case(O, N, 2.0, 32)
    q3e, k3e, v3e = (t.transpose(1, 3).contiguous() for t in (q3, k3, v3))
    b3e = b3.transpose(-1, -2).contiguous()

    def c3_step():
        attention_stock_train_step(q3, k3, v3, m3, b3, d3, chunk=64)
        attention_stock_train_step(q3e, k3e, v3e, m3, b3e, d3, chunk=64)

    c3_ms, _ = _median_time(c3_step, reps, warm)
    c3_flops = 2 * 14.0 * B * O * H * N * N * D
    # Config 4: TriMul out + in.
    C = TM_C
    z = torch.randn(1, TM_N, TM_N, C, generator=g).requires_grad_(True)
    sd = 1.0 / math.sqrt(C)
    w = {n: (torch.randn(C, C, generator=g) * sd).requires_grad_(True)
         for n in ("w_ap", "w_ag", "w_bp", "w_bg", "w_g", "w_z")}
    w.update({n: (torch.ones(C) if n.startswith("g") else torch.zeros(C)).requires_grad_(True)
              for n in ("g_in", "b_in", "g_out", "b_out")})
    tm_mask = torch.ones(1, TM_N, TM_N)
    tm_dout = torch.randn(1, TM_N, TM_N, C, generator=g)
    params = [z] + list(w.values())

    def c4_step():
        for outgoing in (True, False):
            out = trimul_stock(z, tm_mask, w, outgoing)
            torch.autograd.grad(out, params, tm_dout)

    c4_ms, _ = _median_time(c4_step, reps, warm)
    return {
        "value": round(c3_flops / (c3_ms * 1e-3) / 1e12, 5),
        "unit": "TFLOP/s",
        "cores": int(cores),
        "kind": "port",
        "sample": "stock OpenFold3 math in FP32 on the host (oracle/stock_torch.py), config 3 in "
                  "full: attention fwd+bwd, starting + ending node, chunked over 64 outer rows; "
                  f"median of {reps} after {warm} warm-ups",
        "config1_attention_ms": round(c1_ms, 3),
        "config3_attention_ms": round(c3_ms, 1),
        "config4_trimul_out_plus_in_ms": round(c4_ms, 1),
        "torch_threads": torch.get_num_threads(),
    }


if __name__ == "__main__":
    main()
