// torch_extension.cpp -- op registration of module custom_esimd_kernels.
//
// The first three schemas are the reference's, verbatim
// (csrc/xpu/torch_extension.cc:9-18), registered on the CUDA dispatch key,
// which is where PyTorch-ROCm puts HIP tensors.  The new ops follow in the
// same namespace, with alias annotations on the tensors they write.
#include <Python.h>
#include <torch/library.h>

#include "torch_ops.h"

TORCH_LIBRARY(custom_esimd_kernels_vllm, m) {
  m.def("esimd_gemv_fp8_pern(Tensor input, Tensor weight, Tensor weight_scale, "
        "Tensor output, int N, int K) -> Tensor");
  m.impl("esimd_gemv_fp8_pern", c10::DispatchKey::CUDA, &esimd_gemv_fp8_pern);

  m.def("esimd_gemv_fp8_pert(Tensor input, Tensor weight, Tensor weight_scale, "
        "Tensor output) -> Tensor");
  m.impl("esimd_gemv_fp8_pert", c10::DispatchKey::CUDA, &esimd_gemv_fp8_pert);

  m.def("esimd_fused_add_rms_norm_batched(Tensor hidden_states, Tensor residual, "
        "Tensor weight, float eps) -> Tensor");
  m.impl("esimd_fused_add_rms_norm_batched", c10::DispatchKey::CUDA, &esimd_fused_add_rms_norm_batched);

  // ---- new ops ----
  m.def("esimd_gemv_fp8_pern_fused(Tensor input, Tensor[] weights, Tensor[] weight_scales, "
        "Tensor(a!)[] outputs) -> ()");
  m.impl("esimd_gemv_fp8_pern_fused", c10::DispatchKey::CUDA, &esimd_gemv_fp8_pern_fused);

  m.def("esimd_gemv_fp8_pert_fused(Tensor input, Tensor[] weights, Tensor[] weight_scales, "
        "Tensor(a!)[] outputs) -> ()");
  m.impl("esimd_gemv_fp8_pert_fused", c10::DispatchKey::CUDA, &esimd_gemv_fp8_pert_fused);

  m.def("esimd_fused_add_rms_norm_quant_fp8(Tensor hidden_states, Tensor(a!) residual, Tensor weight, "
        "float eps, Tensor(b!) out_q, Tensor(c!) out_scale) -> ()");
  m.impl("esimd_fused_add_rms_norm_quant_fp8", c10::DispatchKey::CUDA, &esimd_fused_add_rms_norm_quant_fp8);

  m.def("esimd_per_token_quant_fp8(Tensor input, Tensor(a!) out_q, Tensor(b!) out_scale) -> ()");
  m.impl("esimd_per_token_quant_fp8", c10::DispatchKey::CUDA, &esimd_per_token_quant_fp8);

  m.def("esimd_gelu_and_mul(Tensor(a!) out, Tensor input) -> ()");
  m.impl("esimd_gelu_and_mul", c10::DispatchKey::CUDA, &esimd_gelu_and_mul);

  m.def("esimd_gemv_fp8_gelu_and_mul(Tensor input, Tensor weight, Tensor weight_scale, "
        "Tensor(a!) output) -> ()");
  m.impl("esimd_gemv_fp8_gelu_and_mul", c10::DispatchKey::CUDA, &esimd_gemv_fp8_gelu_and_mul);

  m.def("esimd_fused_add_rms_norm_gemv_fp8(Tensor hidden_states, Tensor residual, Tensor weight, float eps, "
        "Tensor(a!) residual_out, Tensor w, Tensor w_scale, Tensor(b!) output, bool gelu_and_mul=False) -> ()");
  m.impl("esimd_fused_add_rms_norm_gemv_fp8", c10::DispatchKey::CUDA, &esimd_fused_add_rms_norm_gemv_fp8);

  m.def("esimd_fused_add_rms_norm_quant_gemv_fp8(Tensor hidden_states, Tensor residual, Tensor weight, "
        "float eps, Tensor(a!) residual_out, Tensor(b!) out_q, Tensor(c!) out_scale, Tensor b, Tensor b_scale, "
        "Tensor(d!) output, bool gelu_and_mul=False) -> ()");
  m.impl("esimd_fused_add_rms_norm_quant_gemv_fp8", c10::DispatchKey::CUDA, &esimd_fused_add_rms_norm_quant_gemv_fp8);

  m.def("esimd_qk_norm_rope(Tensor(a!) q, Tensor(b!) k, Tensor q_weight, Tensor k_weight, "
        "Tensor positions, float eps, float theta, bool is_neox) -> ()");
  m.impl("esimd_qk_norm_rope", c10::DispatchKey::CUDA, &esimd_qk_norm_rope);

  m.def("esimd_gemv_fp8_qk_norm_rope(Tensor input, Tensor weight, Tensor weight_scale, Tensor(a!) output, "
        "Tensor q_weight, Tensor k_weight, Tensor positions, int n_q, int n_k, float eps, float theta, "
        "bool is_neox, Tensor(b!) counters, Tensor(c!)? q_out=None) -> ()");
  m.impl("esimd_gemv_fp8_qk_norm_rope", c10::DispatchKey::CUDA, &esimd_gemv_fp8_qk_norm_rope);

  m.def("esimd_gemv_fp8_add_rms_norm_defer_groups(int N) -> int", &esimd_gemv_fp8_add_rms_norm_defer_groups);
  m.def("esimd_defer_norm_shift(float max_abs_norm_weight) -> int", &esimd_defer_norm_shift);
  m.def("esimd_gemv_fp8_add_rms_norm_defer(Tensor input, Tensor weight, Tensor weight_scale, Tensor(a!) residual, "
        "Tensor norm_weight, Tensor(b!) output, Tensor(c!) row_ss, int norm_shift=0) -> ()");
  m.impl("esimd_gemv_fp8_add_rms_norm_defer", c10::DispatchKey::CUDA, &esimd_gemv_fp8_add_rms_norm_defer);

  m.def("esimd_gemv_fp8_pern_rs(Tensor input, Tensor weight, Tensor weight_scale, Tensor(a!) output, "
        "Tensor row_ss, float eps) -> ()");
  m.impl("esimd_gemv_fp8_pern_rs", c10::DispatchKey::CUDA, &esimd_gemv_fp8_pern_rs);

  m.def("esimd_gemv_fp8_gelu_and_mul_rs(Tensor input, Tensor weight, Tensor weight_scale, Tensor(a!) output, "
        "Tensor row_ss, float eps) -> ()");
  m.impl("esimd_gemv_fp8_gelu_and_mul_rs", c10::DispatchKey::CUDA, &esimd_gemv_fp8_gelu_and_mul_rs);

  m.def("esimd_gemv_fp8_qk_norm_rope_rs(Tensor input, Tensor weight, Tensor weight_scale, Tensor(a!) output, "
        "Tensor q_weight, Tensor k_weight, Tensor positions, int n_q, int n_k, float eps, float theta, "
        "bool is_neox, Tensor(b!) counters, Tensor row_ss, float row_eps, Tensor(c!)? q_out=None) -> ()");
  m.impl("esimd_gemv_fp8_qk_norm_rope_rs", c10::DispatchKey::CUDA, &esimd_gemv_fp8_qk_norm_rope_rs);
}

PyMODINIT_FUNC PyInit_custom_esimd_kernels() {
  static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "custom_esimd_kernels", nullptr, 0, nullptr};
  return PyModule_Create(&module);
}
