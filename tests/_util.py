"""Shared helpers for the test-suite: seeded inputs and error metrics."""

from __future__ import annotations

import numpy as np
import torch


def max_rel(got, ref) -> float:
    """max |got - ref| / max |ref|  (the tolerance metric used throughout)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    denom = np.abs(ref).max()
    if denom == 0:
        return float(np.abs(got).max())
    return float(np.abs(got - ref).max() / denom)


def rel_l2(got, ref) -> float:
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30))


def attention_case(B, O, H, N, D, *, mask_tail=0, mask_frac=0.0, full_planes=0,
                   bias_scale=1.0, seed=0, random_tail=False):
    """Seeded bf16-representable attention inputs (CPU tensors, float32 values).

    mask_tail: last ``mask_tail`` keys set to -inf for every outer row;
    random_tail: per-outer-row random 0..mask_tail key tail set to -inf;
    mask_frac: random fraction of keys set to -inf;
    full_planes: first ``full_planes`` outer rows fully masked.
    """
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(B, O, H, N, D, generator=g).to(torch.bfloat16).float() for _ in range(3))
    bias = (torch.randn(1, 1, H, N, N, generator=g) * bias_scale).to(torch.bfloat16).float()
    mask = torch.zeros(B, O, 1, 1, N)
    if mask_tail and not random_tail:
        mask[..., N - mask_tail:] = float("-inf")
    if mask_tail and random_tail:
        tails = torch.randint(0, mask_tail + 1, (B, O), generator=g)
        for b in range(B):
            for o in range(O):
                t = int(tails[b, o])
                if t:
                    mask[b, o, ..., N - t:] = float("-inf")
    if mask_frac:
        mask[torch.rand(B, O, 1, 1, N, generator=g) < mask_frac] = float("-inf")
    if full_planes:
        mask[:, :full_planes] = float("-inf")
    dout = torch.randn(B, O, N, H, D, generator=g).to(torch.bfloat16).float()
    if full_planes:
        dout[:, :full_planes] = 0
    return q, k, v, mask, bias, dout


def record(name: str, key: str, values: dict) -> None:
    """Merge ``{key: values}`` into ``$TPF_NUMERICS_OUT/<name>.json`` when that
    environment variable names a directory (GPU runs set it so the measured
    error figures are kept as a record); otherwise do nothing."""
    import json
    import os

    out = os.environ.get("TPF_NUMERICS_OUT")
    if not out:
        return
    os.makedirs(out, exist_ok=True)
    path = os.path.join(out, f"{name}.json")
    data = {}
    if os.path.exists(path):
        with open(path) as f:
            data = json.load(f)
    data[key] = values
    with open(path, "w") as f:
        json.dump(data, f, indent=1, sort_keys=True)
