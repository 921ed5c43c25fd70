"""The drop-in boundary on the torch side (CPU): schemas and failure modes.

The reference's four schemas must be registered verbatim
(reference csrc/xpu/torch_extension.cc:9-18, torch_extension_gemm.cc:11-13),
the wrappers must keep their names and parameters
(reference python/custom_esimd_kernels_vllm/ops.py:7-67), and calling an op
with CPU tensors must fail loudly rather than fall back.
"""

import inspect

import pytest
import torch

import esimd_learning_amd

REFERENCE_SCHEMAS = {
    "esimd_gemv_fp8_pern": "esimd_gemv_fp8_pern(Tensor input, Tensor weight, Tensor weight_scale, "
                           "Tensor output, int N, int K) -> Tensor",
    "esimd_gemv_fp8_pert": "esimd_gemv_fp8_pert(Tensor input, Tensor weight, Tensor weight_scale, "
                           "Tensor output) -> Tensor",
    "esimd_fused_add_rms_norm_batched": "esimd_fused_add_rms_norm_batched(Tensor hidden_states, "
                                        "Tensor residual, Tensor weight, float eps) -> Tensor",
    "esimd_gemm_fp8_pert": "esimd_gemm_fp8_pert(Tensor input, Tensor weight, Tensor weight_scale, "
                           "Tensor output) -> Tensor",
}


@pytest.fixture(scope="module")
def pkg():
    assert esimd_learning_amd.built(), "extension not built"
    return esimd_learning_amd.ops()


def test_reference_schemas_verbatim(pkg):
    for name, schema in REFERENCE_SCHEMAS.items():
        op = getattr(torch.ops.custom_esimd_kernels_vllm, name).default
        assert str(op._schema) == "custom_esimd_kernels_vllm::" + schema


def test_new_ops_registered(pkg):
    for name in ("esimd_fused_add_rms_norm_quant_fp8", "esimd_per_token_quant_fp8", "esimd_gelu_and_mul",
                 "esimd_qk_norm_rope", "esimd_gemm_fp8_a8w8", "esimd_gemv_fp8_pern_fused",
                 "esimd_gemv_fp8_pert_fused", "esimd_gemv_fp8_gelu_and_mul",
                 "esimd_gemm_fp8_a8w8_gelu_and_mul", "esimd_fused_add_rms_norm_gemv_fp8",
                 "esimd_fused_add_rms_norm_quant_gemv_fp8", "esimd_gemv_fp8_qk_norm_rope"):
        op = getattr(torch.ops.custom_esimd_kernels_vllm, name).default
        assert "!" in str(op._schema)     # written tensors carry alias annotations


def test_wrapper_signatures(pkg):
    assert list(inspect.signature(pkg.esimd_gemv_fp8_pern).parameters) == \
        ["input", "weight", "weight_scale", "output", "N", "K"]
    assert list(inspect.signature(pkg.esimd_gemv_fp8_pert).parameters) == \
        ["input", "weight", "weight_scale", "output"]
    assert list(inspect.signature(pkg.esimd_fused_add_rms_norm_batched).parameters) == \
        ["hidden_states", "residual", "weight", "eps"]
    assert list(inspect.signature(pkg.esimd_gemm_fp8_pert).parameters) == \
        ["input", "weight", "weight_scale", "output"]
    assert pkg.custom_esimd_kernels.__name__.endswith("custom_esimd_kernels")
    assert pkg.custom_esimd_kernels_gemm.__name__.endswith("custom_esimd_kernels_gemm")


def test_cpu_tensors_fail_loudly(pkg):
    x = torch.zeros(1, 64, dtype=torch.float16)
    w = torch.zeros(8, 64, dtype=torch.float8_e4m3fn)
    y = torch.zeros(1, 8, dtype=torch.float16)
    with pytest.raises(NotImplementedError):
        pkg.esimd_gemv_fp8_pern(x, w, torch.ones(8), y, 8, 64)
    with pytest.raises(NotImplementedError):
        pkg.esimd_fused_add_rms_norm_batched(x, x.clone(), torch.ones(64, dtype=torch.float16), 1e-6)
