"""C-ABI contract without a GPU: the library loads, exports every symbol that
include/tpf_amd.h declares with the argument counts the ctypes binding uses,
and rejects bad shapes with a status code and message before any launch."""

import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "tpf_amd.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"\b(?:int|int64_t|const char\*)\s+(tpf_\w+)\s*\(([^)]*)\)\s*;", text):
        args = [a for a in m.group(2).split(",") if a.strip() and a.strip() != "void"]
        decls[m.group(1)] = len(args)
    return decls


@pytest.fixture(scope="module")
def lib():
    from openfold3_triangle_kernel_amd import _native

    return _native.library()


def test_header_declares_entry_points():
    decls = _declared()
    assert {"tpf_attn_forward_bf16", "tpf_attn_backward_bf16", "tpf_trimul_forward_bf16",
            "tpf_trimul_backward_bf16", "tpf_last_error"} <= set(decls)


def test_library_exports_every_declared_symbol(lib):
    from openfold3_triangle_kernel_amd import _native

    decls = _declared()
    for name, nargs in decls.items():
        assert hasattr(lib, name), f"{name} not exported"
        assert name in _native.SIGNATURES, f"{name} missing from the ctypes binding"
        assert len(_native.SIGNATURES[name][1]) == nargs, f"{name}: arg count mismatch"
    assert lib.tpf_abi_version() == 8


def test_shape_errors_are_reported_without_launch(lib):
    from openfold3_triangle_kernel_amd import _native

    with pytest.raises(RuntimeError, match="multiple of 64"):
        _native.call("tpf_attn_forward_bf16", 16, 16, 16, 16, 16, 16, 16, 16, 1 << 30, 1, 2, 4, 100,
                     32, 0, 1, 0.1767, None)
    with pytest.raises(RuntimeError, match="D=20"):
        _native.call("tpf_attn_forward_bf16", 16, 16, 16, 16, 16, 16, 16, 16, 1 << 30, 1, 2, 4, 128,
                     20, 0, 1, 0.2, None)
    with pytest.raises(RuntimeError, match="null pointer"):
        _native.call("tpf_attn_forward_bf16", None, 16, 16, 16, 16, 16, 16, 16, 1 << 30, 1, 2, 4,
                     128, 32, 0, 1, 0.2, None)
    with pytest.raises(RuntimeError, match="bias batch"):
        _native.call("tpf_attn_forward_bf16", 16, 16, 16, 16, 16, 16, 16, 16, 1 << 30, 2, 2, 4, 128,
                     32, 0, 3, 0.2, None)
    with pytest.raises(RuntimeError, match="C=48"):
        _native.call("tpf_trimul_forward_bf16", *([16] * 12), 1, 1, 64, 48, *([16] * 12), 1 << 20, None)
    with pytest.raises(RuntimeError, match="workspace"):
        _native.call("tpf_attn_backward_bf16", *([16] * 13), 0, 1, 4, 4, 128, 32, 0, 1, 0.2, None)
    with pytest.raises(RuntimeError, match="multiple of 8"):
        _native.call("tpf_layer_norm_forward_bf16", 16, 1, 4, 4, 0, 48, 12, 12, None, None, 1e-5,
                     16, 16, 16, None)
    with pytest.raises(RuntimeError, match="strides"):
        _native.call("tpf_layer_norm_forward_bf16", 16, 1, 4, 4, 0, 20, 5, 16, None, None, 1e-5,
                     16, 16, 16, None)
    with pytest.raises(RuntimeError, match="both given or both null"):
        _native.call("tpf_layer_norm_backward_bf16", 16, 16, 1, 4, 4, 0, 64, 16, 0, 64, 16, 16, 16,
                     16, None, 16, 16, None, 16, 1 << 20, None)
    with pytest.raises(RuntimeError, match="workspace"):
        _native.call("tpf_layer_norm_backward_bf16", 16, 16, 1, 4, 4, 0, 64, 16, 0, 64, 16, 16, 16,
                     16, None, 16, 16, 16, 16, 8, None)


def test_trimul_shape_supported_boundaries(lib):
    """The bf16 TriMul extent: a tensor fits the kernels' 32-bit buffer
    windows when its bytes stay below 2^31.  Forward: [B*N*N, C] rows and
    [B*C, N, Np] planes; backward also [B*N*N, 5C] rows.  The boundaries
    below follow from that closed form, e.g. at C = 128, B = 1 the largest
    forward N has N^2 * 128 * 2 < 2^31 (2896^2 * 256 = 2,147,024,896)."""
    from openfold3_triangle_kernel_amd import _native

    def ok(B, N, C, bwd):
        return _native.query("tpf_trimul_shape_supported", B, N, C, bwd)

    def fits(B, N, C, bwd):
        Np = (N + 7) // 8 * 8
        rows = B * N * N * (5 * C if bwd else C) * 2
        planes = B * C * N * Np * 2
        return int(rows < 2**31 and planes < 2**31 and B * N * N <= (2**31 - 1) // 2)

    assert ok(1, 2896, 128, 0) == 1 and ok(1, 2897, 128, 0) == 0
    assert ok(1, 1295, 128, 1) == 1 and ok(1, 1296, 128, 1) == 0
    assert ok(1, 768, 128, 1) == 1 and ok(2, 2048, 128, 0) == 0
    assert ok(1, 64, 48, 0) == 0 and ok(0, 64, 128, 0) == 0
    for B, N, C in ((1, 1831, 64), (1, 1832, 64), (3, 1672, 32), (1, 4095, 32), (2, 1025, 96)):
        for bwd in (0, 1):
            assert ok(B, N, C, bwd) == fits(B, N, C, bwd), (B, N, C, bwd)

    # The host layer's traceable restatement agrees with the library.
    from openfold3_triangle_kernel_amd.trimul import _extent_fits

    for B in (1, 2, 3):
        for N in (1, 64, 1295, 1296, 1831, 1832, 2048, 2896, 2897, 4095, 4096):
            for C in (32, 64, 96, 128):
                for bwd in (0, 1):
                    assert int(_extent_fits(B, N, C, bool(bwd))) == ok(B, N, C, bwd), (B, N, C, bwd)


def test_workspace_sizes(lib):
    from openfold3_triangle_kernel_amd import _native

    ws = _native.query("tpf_attn_backward_workspace_bytes", 1, 384, 4, 384, 32)
    dq = 3 * 384 * 4 * 384 * 32 * 2  # bf16 dQ partial per 128-key block (D <= 32)
    db = 20 * 4 * 384 * 384 * 4  # f32 dBias partial per run of 5 outer groups (20 runs)
    rest = 4 * 384 * 384 * 4 + 2 * 384 * 4 * 384 * 4  # prescaled bias, two row statistics
    assert ws == dq + db + rest
    assert _native.query("tpf_trimul_plane_pitch", 113) == 120
    assert _native.query("tpf_trimul_plane_pitch", 384) == 384
    assert _native.query("tpf_trimul_backward_workspace_bytes", 1, 384, 128) > 0
    # LayerNorm parameter partials: at most 2048 workgroups x [dgamma | dbeta]
    assert _native.query("tpf_layer_norm_backward_workspace_bytes", 384 * 384, 128) == 2048 * 2 * 128 * 4
    assert _native.query("tpf_layer_norm_backward_workspace_bytes", 16, 128) == 1 * 2 * 128 * 4
    assert _native.query("tpf_layer_norm_backward_workspace_bytes", 16, 12) == -1


def test_backward_workspace_budget_plan(lib):
    """The budgeted plan: the full plan when it fits, otherwise slabs whose
    workspace stays within the budget, down to a one-run minimum that is
    returned (and exceeds the budget) for budgets below it."""
    from openfold3_triangle_kernel_amd import _native

    for shape in ((1, 384, 4, 384, 32), (1, 768, 8, 768, 64), (2, 130, 4, 128, 32)):
        full = _native.query("tpf_attn_backward_workspace_bytes", *shape)
        assert _native.query("tpf_attn_backward_workspace_bytes_budget", *shape, full) == full
        assert _native.query("tpf_attn_backward_slab_count", *shape, full) == 1
        minimum = _native.query("tpf_attn_backward_workspace_bytes_budget", *shape, 1)
        assert 0 < minimum < full
        assert _native.query("tpf_attn_backward_slab_count", *shape, minimum - 1) == 0
        last = 1
        for frac in (0.9, 0.6, 0.4, 0.2):
            budget = max(minimum, int(full * frac))
            ws = _native.query("tpf_attn_backward_workspace_bytes_budget", *shape, budget)
            assert minimum <= ws <= budget
            slabs = _native.query("tpf_attn_backward_slab_count", *shape, ws)
            assert slabs >= last  # fewer bytes never means fewer slabs
            last = slabs
    # Config 5's H=8, D=64 attention needs 7.46 GB in one slab; 4 GiB gives two.
    ws = _native.query("tpf_attn_backward_workspace_bytes_budget", 1, 768, 8, 768, 64, 4 << 30)
    assert ws <= 4 << 30
    assert _native.query("tpf_attn_backward_slab_count", 1, 768, 8, 768, 64, ws) == 2


def test_pair_backward_dout_instances(lib):
    """Head shapes the fused d_og + gate-backward row kernel serves (C = 128,
    D in {8, 16, 32, 64}, H*D a multiple of 16 up to 128); others take the
    two-step route."""
    from openfold3_triangle_kernel_amd import _native

    q = lambda C, H, D: _native.query("tpf_attn_pair_backward_dout_supported", C, H, D)
    assert q(128, 4, 32) and q(128, 2, 64) and q(128, 16, 8) and q(128, 1, 16)
    assert not q(64, 4, 32) and not q(128, 4, 24) and not q(128, 8, 32) and not q(128, 1, 8)
