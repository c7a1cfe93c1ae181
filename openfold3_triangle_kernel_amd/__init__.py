"""TurboPairFormer triangle attention and triangle multiplicative update on MI355X.

From-scratch gfx950 implementation of the two TurboPairFormer operators behind
OpenFold3's TriangleAttention / TriangleMultiplicativeUpdate modules.  All
compute runs in hand-written HIP kernels in ``libtpf_amd.so`` (C ABI,
``include/tpf_amd.h``); there is no CPU or PyTorch fallback.
"""

from .attention import (
    invocation_count,
    is_turbopairformer_supported,
    turbo_attention,
    turbopairformer_triangle_attention,
)

__all__ = [
    "invocation_count",
    "is_turbopairformer_supported",
    "turbo_attention",
    "turbopairformer_triangle_attention",
]

from .trimul import (  # noqa: E402
    check_stable_trimul_support,
    run_stable_trimul,
    trimul_wgrad_fixed_fold,
    turbo_trimul,
)

__all__ += ["check_stable_trimul_support", "run_stable_trimul", "trimul_wgrad_fixed_fold",
            "turbo_trimul"]

from .attention_fp32 import is_attention_fp32_supported, turbopairformer_attention_fp32  # noqa: E402

__all__ += ["is_attention_fp32_supported", "turbopairformer_attention_fp32"]

from .trimul_fp32 import run_trimul_fp32  # noqa: E402

__all__ += ["run_trimul_fp32"]

from .modules import (  # noqa: E402
    TriangleAttention,
    TriangleAttentionEndingNode,
    TriangleAttentionStartingNode,
    TriangleMultiplicationIncoming,
    TriangleMultiplicationOutgoing,
    TriangleMultiplicativeUpdate,
)

__all__ += ["TriangleAttention", "TriangleAttentionEndingNode", "TriangleAttentionStartingNode",
            "TriangleMultiplicationIncoming", "TriangleMultiplicationOutgoing",
            "TriangleMultiplicativeUpdate"]

from .routing import (  # noqa: E402
    set_tpf_bf16_cast_for_fp32_training,
    set_turbopairformer_strict,
    stock_invocation_count,
    turbopairformer_strict_enabled,
)

__all__ += ["set_tpf_bf16_cast_for_fp32_training", "set_turbopairformer_strict",
            "stock_invocation_count", "turbopairformer_strict_enabled"]

from .layernorm import layer_norm_bf16  # noqa: E402

__all__ += ["layer_norm_bf16"]
