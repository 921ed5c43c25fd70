"""custom_esimd_kernels_vllm -- MI355X (gfx950) build.

Same import surface as the reference package
(reference python/custom_esimd_kernels_vllm/__init__.py:1-11): importing it
loads the two extension modules, which register the
``torch.ops.custom_esimd_kernels_vllm`` ops, and re-exports the wrappers.
There is no fallback: if the HIP build is missing the import fails.
"""

import torch  # noqa: F401  (loads libtorch before the extension modules)

from custom_esimd_kernels_vllm import custom_esimd_kernels  # noqa: F401
from custom_esimd_kernels_vllm import custom_esimd_kernels_gemm  # noqa: F401

from custom_esimd_kernels_vllm.ops import (  # noqa: F401
    esimd_gemv_fp8_pern,
    esimd_gemv_fp8_pert,
    esimd_fused_add_rms_norm_batched,
    esimd_gemm_fp8_pert,
    esimd_gemv_fp8_pern_fused,
    esimd_gemv_fp8_pert_fused,
    esimd_fused_add_rms_norm_quant_fp8,
    esimd_per_token_quant_fp8,
    esimd_gelu_and_mul,
    esimd_gemv_fp8_gelu_and_mul,
    esimd_fused_add_rms_norm_gemv_fp8,
    esimd_fused_add_rms_norm_quant_gemv_fp8,
    esimd_qk_norm_rope,
    esimd_gemv_fp8_qk_norm_rope,
    gemv_tail_counters,
    esimd_gemv_fp8_add_rms_norm_defer,
    esimd_gemv_fp8_add_rms_norm_defer_groups,
    esimd_defer_norm_shift,
    esimd_gemv_fp8_pern_rs,
    esimd_gemv_fp8_gelu_and_mul_rs,
    esimd_gemv_fp8_qk_norm_rope_rs,
    esimd_gemm_fp8_a8w8,
    esimd_gemm_fp8_a8w8_gelu_and_mul,
)
