"""Model-level routing policy of the drop-in modules.

Mirrors the reference's policy around its stable kernels:

* strict mode (``openfold3/core/utils/distributed_contract.py:46-80``): when
  enabled, a stable request that the kernels do not support raises instead
  of falling back to the stock PyTorch math;
* fallback logging (``openfold3/core/model/primitives/attention.py:675-692``,
  ``openfold3/core/model/layers/triangular_multiplicative_update.py:62-120``):
  otherwise the fallback is logged once per (site, reason) and the module
  runs its stock math;
* FP32 training inputs of triangle attention take the stock FP32 math unless
  the BF16 cast is selected (``attention.py:105-113, 520-548``).

Counters let tests lock the routing: ``stock_invocation_count`` counts stock
executions, the kernel facades count their own invocations.
"""

from __future__ import annotations

import logging

_STRICT = False
_BF16_CAST_FOR_FP32_TRAINING = False
_LOGGED: set = set()
_STOCK_CALLS = 0

_LOG = logging.getLogger(__name__)


def set_turbopairformer_strict(enabled: bool) -> None:
    """Make unsupported stable requests fatal (True) or logged fallbacks (False)."""
    global _STRICT
    _STRICT = bool(enabled)


def turbopairformer_strict_enabled() -> bool:
    return _STRICT


def set_tpf_bf16_cast_for_fp32_training(enabled: bool) -> None:
    """Choose the BF16 kernels (True) or the stock FP32 math (False) for FP32
    triangle-attention inputs outside FP32 inference."""
    global _BF16_CAST_FOR_FP32_TRAINING
    _BF16_CAST_FOR_FP32_TRAINING = bool(enabled)


def tpf_bf16_cast_for_fp32_training() -> bool:
    return _BF16_CAST_FOR_FP32_TRAINING


def report_fallback(site: str, shape: tuple, reason: str) -> None:
    """Raise under strict mode; otherwise log the fallback once per (site, reason)."""
    if _STRICT:
        raise RuntimeError(
            f"TurboPairFormer strict route rejected a stock fallback for {site} at shape "
            f"{tuple(shape)}: {reason}"
        )
    key = (site, reason)
    if key not in _LOGGED:
        _LOGGED.add(key)
        _LOG.warning("TurboPairFormer fallback to stock for %s at shape %s: %s", site,
                     tuple(shape), reason)


def note_stock_call() -> None:
    global _STOCK_CALLS
    _STOCK_CALLS += 1


def stock_invocation_count() -> int:
    return _STOCK_CALLS


__all__ = [
    "report_fallback",
    "set_tpf_bf16_cast_for_fp32_training",
    "set_turbopairformer_strict",
    "stock_invocation_count",
    "tpf_bf16_cast_for_fp32_training",
    "turbopairformer_strict_enabled",
]
