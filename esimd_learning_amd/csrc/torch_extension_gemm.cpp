// torch_extension_gemm.cpp -- op registration of module custom_esimd_kernels_gemm.
//
// esimd_gemm_fp8_pert keeps the reference's schema verbatim
// (csrc/xpu/torch_extension_gemm.cc:11-13), added as a library fragment so
// that this module loads after custom_esimd_kernels, as in the reference.
#include <Python.h>
#include <torch/library.h>

#include "torch_ops.h"

TORCH_LIBRARY_FRAGMENT(custom_esimd_kernels_vllm, m) {
  m.def("esimd_gemm_fp8_pert(Tensor input, Tensor weight, Tensor weight_scale, "
        "Tensor output) -> Tensor");
  m.impl("esimd_gemm_fp8_pert", c10::DispatchKey::CUDA, &esimd_gemm_fp8_pert);

  // ---- new ops ----
  m.def("esimd_gemm_fp8_a8w8(Tensor a, Tensor a_scale, Tensor b, Tensor b_scale, "
        "Tensor(a!) output) -> Tensor(a!)");
  m.impl("esimd_gemm_fp8_a8w8", c10::DispatchKey::CUDA, &esimd_gemm_fp8_a8w8);

  m.def("esimd_gemm_fp8_a8w8_gelu_and_mul(Tensor a, Tensor a_scale, Tensor b, Tensor b_scale, "
        "Tensor(a!) output) -> ()");
  m.impl("esimd_gemm_fp8_a8w8_gelu_and_mul", c10::DispatchKey::CUDA, &esimd_gemm_fp8_a8w8_gelu_and_mul);
}

PyMODINIT_FUNC PyInit_custom_esimd_kernels_gemm() {
  static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "custom_esimd_kernels_gemm", nullptr, 0, nullptr};
  return PyModule_Create(&module);
}
