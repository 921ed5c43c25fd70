"""CPU oracle for the fp8 decode/prefill op pack -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference package
``custom_esimd_kernels_vllm`` computes for its hot path (fp8-weight GEMV /
GEMM, fused residual-add + RMSNorm) and the closed forms of the ops that the
reference lacks (per-token fp8 quantisation, a8w8 GEMM, gelu_and_mul,
QK-norm + RoPE).  Every function cites the reference file:line it follows
(paths are relative to the reference repository root).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker or the timed
CPU baseline.  The product path (``esimd_learning_amd`` and the
``custom_esimd_kernels_vllm`` torch ops) never imports it and has no CPU
fallback: a missing HIP library is an error there.

Pinning (what checks each oracle function against something other than
itself) is listed per module in its docstring; the tests that perform the
pins live in ``tests/test_oracle_fp8.py`` (codec) and ``tests/test_oracle_ops.py`` (ops).
"""

from . import fp8, gemv, norm, act, gemm, layer  # noqa: F401
