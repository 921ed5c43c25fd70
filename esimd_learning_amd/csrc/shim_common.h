// shim_common.h -- helpers shared by the torch shims (host C++ only).
#pragma once

#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include "cek.h"

namespace cek_shim {

inline void* current_stream(const at::Tensor& t) {
  return reinterpret_cast<void*>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

// Activation dtype code; fp16 and bf16 are the only activation types.
inline int io_code(at::ScalarType s) {
  return s == at::ScalarType::BFloat16 ? CEK_BF16 : CEK_F16;
}
inline bool is_io(at::ScalarType s) {
  return s == at::ScalarType::Half || s == at::ScalarType::BFloat16;
}

// fp8 encoding of a weight tensor, as the reference's get_fp8_mode
// (csrc/xpu/esimd_kernel.sycl:14-16): e5m2 if the dtype says so, else e4m3.
inline int fp8_code(const at::Tensor& w) {
  return w.scalar_type() == at::ScalarType::Float8_e5m2 ? CEK_E5M2 : CEK_E4M3;
}

inline void check_fp8_weight(const at::Tensor& w, const char* op) {
  TORCH_CHECK(w.element_size() == 1, op, ": weight must be an 8-bit (fp8) tensor, got ", w.scalar_type());
}

inline void check_device(const at::Tensor& t, const at::Tensor& ref, const char* op, const char* name) {
  TORCH_CHECK(t.is_cuda(), op, ": ", name, " must be a GPU tensor");
  TORCH_CHECK(t.device() == ref.device(), op, ": ", name, " is on ", t.device(), " but input is on ",
              ref.device());
}

inline void check_contig(const at::Tensor& t, const char* op, const char* name) {
  TORCH_CHECK(t.is_contiguous(), op, ": ", name, " must be contiguous");
}

inline void check_rc(int rc, const char* op) {
  if (rc == CEK_OK) return;
  TORCH_CHECK(false, op, ": ", cek_error_string(rc), rc == CEK_ERR_HIP ? " -- " : "",
              rc == CEK_ERR_HIP ? cek_last_hip_error() : "");
}

}  // namespace cek_shim
