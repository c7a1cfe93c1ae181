"""CPU oracle for the TurboPairFormer hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the reference algorithms that the gfx950
kernels implement.  It is the checker, never the thing measured or shipped:
only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import it.  The product package
``openfold3_triangle_kernel_amd`` never imports it and has no CPU fallback.

Modules:
  attention  -- triangle attention forward / backward (closed form).
  trimul     -- LayerNorm and the triangle multiplicative update, forward and
                hand-derived backward.
  modules    -- restatements of OpenFold3's TriangleAttention and
                TriangleMultiplicationOutgoing/Incoming modules (projections,
                gating, transposes), used to pin the oracle against the
                reference's committed module snapshots.

How each function is pinned (see tests/test_oracle_*.py):
  * against the reference's committed golden vectors (module snapshots
    ``openfold3/tests/test_data/snapshots/test_triangular_{attention,
    multiplicative_update}/*/test_shape_cpu_*.npz``, copied as data into
    ``tests/golden/``);
  * hand-derived backward formulas against torch autograd of an independent
    forward written with torch ops (a different differentiation method);
  * invariants: softmax rows sum to 1, fully masked rows give zero output and
    zero gradients, ending node == starting node on transposed inputs,
    padding invariance, dBias == sum over outer rows of dS (brute force).
"""
