"""ctypes binding of the gfx950 C-ABI library ``libtpf_amd.so``.

The library is the only compute path: there is no CPU or PyTorch fallback.
Loading fails with a RuntimeError naming the missing file when the library
has not been built, and every entry point's status code is turned into a
RuntimeError carrying the library's own message.

Loading is behind a lock and cached per process, mirroring the fail-closed
loader of the reference (openfold3/core/kernels/turbopairformer/_aot_runtime.py:273-321),
without its manifest/hash attestation (the library is built in-tree).
"""

from __future__ import annotations

import contextlib
import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libtpf_amd.so"

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int
_F64 = ctypes.c_double

# name -> (restype, argtypes).  Must match include/tpf_amd.h.
SIGNATURES: dict[str, tuple] = {
    "tpf_abi_version": (_I32, []),
    "tpf_last_error": (ctypes.c_char_p, []),
    "tpf_attn_forward_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64]),
    "tpf_attn_forward_bf16": (
        _I32,
        [_P] * 8 + [_I64] * 6 + [_I32, _I64, _F64, _P],
    ),
    "tpf_attn_forward_shadow_bf16": (
        _I32,
        [_P] * 9 + [_I64] * 6 + [_I32, _I64, _F64, _P],
    ),
    "tpf_attn_forward_noalloc_bf16": (
        _I32,
        [_P] * 7 + [_I64] * 5 + [_I32, _I64, _F64, _P],
    ),
    "tpf_attn_delta_bf16": (_I32, [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P]),
    "tpf_attn_delta_shadow_bf16": (_I32, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P]),
    "tpf_attn_backward_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64, _I64]),
    "tpf_attn_backward_workspace_bytes_budget": (_I64, [_I64, _I64, _I64, _I64, _I64, _I64]),
    "tpf_attn_backward_slab_count": (_I32, [_I64, _I64, _I64, _I64, _I64, _I64]),
    "tpf_attn_backward_bf16": (
        _I32,
        [_P] * 13 + [_I64] * 6 + [_I32, _I64, _F64, _P],
    ),
    "tpf_attn_backward_fused_bf16": (
        _I32,
        [_P] * 14 + [_I64] * 6 + [_I32, _I64, _F64, _P],
    ),
    "tpf_attn_backward_main_bf16": (
        _I32,
        [_P] * 11 + [_I64] * 6 + [_I32, _I64, _F64, _P],
    ),
    "tpf_attn_backward_finish_bf16": (
        _I32,
        [_P, _P, _P] + [_I64] * 5 + [_I32, _I64, _F64, _P],
    ),
    "tpf_attn_dkdv_workspace_bytes": (_I64, [_I64] * 6),
    "tpf_attn_dkdv_delta_true_partial_elements": (_I64, [_I64] * 4),
    "tpf_attn_dkdv_bf16": (
        _I32,
        [_P] * 13 + [_I64] * 6 + [_I32, _I64, _F64, _P],
    ),
    "tpf_attn_dq_dbias_workspace_bytes": (_I64, [_I64] * 5),
    "tpf_attn_dq_dbias_bf16": (
        _I32,
        [_P] * 11 + [_I64] * 6 + [_I32, _I64, _F64, _P],
    ),
    "tpf_gemm_bf16": (
        _I32,
        [_P, _I32, _I64, _I64, _P, _I32, _I64, _I64, _P, _I32, _I64, _I64, _I64, _I64, _I64,
         _I64, _F64, _P],
    ),
    "tpf_attn_pair_forward_workspace_bytes": (_I64, [_I64, _I64, _I64]),
    "tpf_attn_pair_forward_bf16": (
        _I32, [_P, _P, _I64, _P, _I32, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F64,
               _P]),
    "tpf_attn_pair_backward_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64]),
    "tpf_attn_pair_backward_bf16": (
        _I32, [_P, _P, _I64, _P, _I32, _P, _P, _P, _P, _P, _I64, _P, _I64, _I64, _I64, _I64,
               _I64, _F64, _P]),
    "tpf_attn_pair_backward_dout_supported": (_I32, [_I64] * 3),
    "tpf_attn_pair_backward_dout_bf16": (
        _I32, [_P, _P, _I64, _P, _I32, _P, _P, _P, _P, _P, _I64, _P, _I64, _P, _I64, _I64, _I64,
               _I64, _I64, _F64, _P]),
    "tpf_pair_projection_supported": (_I32, [_I64] * 5),
    "tpf_pair_projection_bf16": (_I32, [_P, _P] + [_I64] * 6 + [_P, _P, _P]),
    "tpf_layer_norm_forward_bf16": (_I32, [_P] + [_I64] * 7 + [_P, _P, _F64, _P, _P, _P, _P]),
    "tpf_layer_norm_backward_workspace_bytes": (_I64, [_I64, _I64]),
    "tpf_layer_norm_backward_bf16": (_I32, [_P, _P] + [_I64] * 10 + [_P] * 7 + [_I64, _P]),
    "tpf_attn_forward_f32_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64]),
    "tpf_attn_forward_f32": (
        _I32,
        [_P] * 8 + [_I64] * 6 + [_I32, _I64, _F64, _P],
    ),
    "tpf_gemm_f32": (
        _I32,
        [_P, _I32, _I64, _I64, _P, _I32, _I64, _I64, _P, _I64, _I64, _I64, _I64, _I64, _I64,
         _F64, _P, _P],
    ),
    "tpf_trimul_forward_f32_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64]),
    "tpf_trimul_forward_f32": (
        _I32,
        [_P] * 16 + [_F64, _P, _P, _F64, _I32, _I64, _I64, _I64, _I64, _P, _P, _I64, _P],
    ),
    "tpf_trimul_forward_f32_workspace_bytes_chunked": (_I64, [_I64, _I64, _I64, _I64, _I64]),
    "tpf_trimul_forward_f32_chunked": (
        _I32,
        [_P] * 16 + [_F64, _P, _P, _F64, _I32, _I64, _I64, _I64, _I64, _I64, _P, _P, _I64, _P],
    ),
    "tpf_wgrad_bf16_workspace_bytes": (_I64, [_I64, _I64, _I64]),
    "tpf_wgrad_bf16": (_I32, [_P, _I64, _P, _I64, _I64, _I64, _I64, _P, _P, _I64, _P]),
    "tpf_trimul_wgrad_fixed_fold": (_I32, [_P, _I64, _I64, _P, _I32, _P]),
    "tpf_trimul_plane_pitch": (_I64, [_I64]),
    "tpf_trimul_shape_supported": (_I32, [_I64, _I64, _I64, _I32]),
    "tpf_trimul_forward_workspace_bytes": (_I64, [_I64]),
    "tpf_trimul_forward_bf16": (
        _I32,
        [_P] * 12 + [_I32, _I64, _I64, _I64] + [_P] * 12 + [_I64, _P],
    ),
    "tpf_trimul_backward_workspace_bytes": (_I64, [_I64, _I64, _I64]),
    "tpf_trimul_backward_bf16": (
        _I32,
        [_P] * 21 + [_I32, _I64, _I64, _I64] + [_P] * 8 + [_I64, _P],
    ),
    "tpf_trimul_backward_named_bf16": (
        _I32,
        [_P] * 21 + [_I32, _I64, _I64, _I64] + [_P] * 10 + [_I64, _P],
    ),
}

_LOCK = threading.Lock()
_LIB: ctypes.CDLL | None = None


def library() -> ctypes.CDLL:
    """Load (once) and return the C-ABI library; raise if it is not built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"TurboPairFormer MI355X library not built: {LIB_PATH} is missing "
                    "(run `python -m openfold3_triangle_kernel_amd.build`)"
                )
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _LIB = lib
    return _LIB


def call(name: str, *args) -> int:
    """Invoke an entry point and raise RuntimeError on a non-zero status."""
    lib = library()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.tpf_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed (status {rc}): {msg}")
    return rc


def query(name: str, *args):
    """Invoke a value-returning entry point (sizes, versions)."""
    return getattr(library(), name)(*args)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor) -> int:
    """The current HIP stream of the tensor's device (0 = null stream off-GPU)."""
    dev = t.device
    if dev.type != "cuda":
        return 0
    if _RAW_STREAM is not None and dev.index is not None:
        return _RAW_STREAM(dev.index)  # no Stream object per call
    return torch.cuda.current_stream(dev).cuda_stream


_NO_SWITCH = contextlib.nullcontext()


def device_ctx(device: torch.device):
    """Make ``device`` current for a native call; no switch (and no guard
    object) when it already is, which is the common case."""
    if device.type != "cuda" or device.index is None or device.index == torch.cuda.current_device():
        return _NO_SWITCH
    return torch.cuda.device(device)
