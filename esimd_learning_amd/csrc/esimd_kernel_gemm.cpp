// esimd_kernel_gemm.cpp -- torch shims of the GEMM ops (takes over the
// reference's csrc/xpu/esimd_kernel_gemm.sycl).
//
// esimd_gemm_fp8_pert keeps the reference's contract (fp16|bf16 input and
// output of one dtype, fp8 weight, fp32 scalar scale, N and K from the weight,
// M from the input).  The reference converts bf16 input to fp16 and back
// around its fp16-only kernels (esimd_kernel_gemm.sycl:43-48,61-63); here the
// kernels take bf16 directly, so no temporaries are allocated.
#include "torch_ops.h"

#include "shim_common.h"

using namespace cek_shim;

at::Tensor esimd_gemm_fp8_pert(at::Tensor input, at::Tensor weight, at::Tensor weight_scale,
                               at::Tensor output) {
  const char* op = "esimd_gemm_fp8_pert";
  TORCH_CHECK(is_io(input.scalar_type()), op, ": input must be fp16 or bf16");
  TORCH_CHECK(is_io(output.scalar_type()), op, ": output must be fp16 or bf16");
  TORCH_CHECK(input.scalar_type() == output.scalar_type(), op, ": input and output must have the same dtype");
  check_fp8_weight(weight, op);
  TORCH_CHECK(weight.dim() == 2, op, ": weight must be [N, K]");
  check_device(weight, input, op, "weight");
  check_device(weight_scale, input, op, "weight_scale");
  check_device(output, input, op, "output");
  check_contig(input, op, "input");
  check_contig(weight, op, "weight");
  check_contig(output, op, "output");
  TORCH_CHECK(weight_scale.scalar_type() == at::ScalarType::Float && weight_scale.numel() >= 1, op,
              ": weight_scale must be an fp32 scalar tensor");
  const int64_t N = weight.size(0), K = weight.size(1);
  TORCH_CHECK(N > 0 && K > 0, op, ": weight must be non-empty");
  TORCH_CHECK(input.numel() % K == 0, op, ": input's element count must be a multiple of K");
  const int64_t M = input.numel() / K;
  TORCH_CHECK(output.numel() >= M * N, op, ": output must hold M*N elements");
  c10::OptionalDeviceGuard guard(input.device());
  const auto* sp = static_cast<const float*>(weight_scale.data_ptr());
  // shapes with too few tiles split K: fp32 partials in a workspace from the
  // caching allocator (no kernel runs to allocate or clear it)
  const int64_t need = cek_gemm_fp8_pert_workspace_size(M, N, K);
  if (need > 0) {
    at::Tensor ws = at::empty({(need + 3) / 4}, weight_scale.options());
    check_rc(cek_gemm_fp8_pert_ws(input.data_ptr(), weight.data_ptr(), sp, output.data_ptr(), M, N, K,
                                  io_code(input.scalar_type()), fp8_code(weight), ws.data_ptr(), need,
                                  current_stream(input)),
             op);
  } else {
    check_rc(cek_gemm_fp8_pert(input.data_ptr(), weight.data_ptr(), sp, output.data_ptr(), M, N, K,
                               io_code(input.scalar_type()), fp8_code(weight), current_stream(input)),
             op);
  }
  return output;
}

at::Tensor esimd_gemm_fp8_a8w8(at::Tensor a, at::Tensor a_scale, at::Tensor b, at::Tensor b_scale,
                               at::Tensor output) {
  const char* op = "esimd_gemm_fp8_a8w8";
  TORCH_CHECK(a.element_size() == 1 && b.element_size() == 1, op, ": a and b must be 8-bit (e4m3) tensors");
  TORCH_CHECK(a.scalar_type() != at::ScalarType::Float8_e5m2 && b.scalar_type() != at::ScalarType::Float8_e5m2, op,
              ": a and b must be e4m3");
  TORCH_CHECK(a_scale.scalar_type() == at::ScalarType::Float && b_scale.scalar_type() == at::ScalarType::Float, op,
              ": scales must be fp32");
  TORCH_CHECK(is_io(output.scalar_type()), op, ": output must be fp16 or bf16");
  TORCH_CHECK(a.dim() == 2 && b.dim() == 2 && a.size(1) == b.size(1), op, ": a [M, K] and b [N, K] required");
  for (auto* t : {&a_scale, &b, &b_scale, &output}) check_device(*t, a, op, "operand");
  check_contig(a, op, "a");
  check_contig(b, op, "b");
  check_contig(a_scale, op, "a_scale");
  check_contig(b_scale, op, "b_scale");
  check_contig(output, op, "output");
  const int64_t M = a.size(0), K = a.size(1), N = b.size(0);
  TORCH_CHECK(K % 16 == 0, op, ": K must be a multiple of 16");
  TORCH_CHECK(a_scale.numel() == M && b_scale.numel() == N, op, ": a_scale [M] and b_scale [N] required");
  TORCH_CHECK(output.numel() == M * N, op, ": output must be [M, N]");
  c10::OptionalDeviceGuard guard(a.device());
  const auto* ap = static_cast<const uint8_t*>(a.data_ptr());
  const auto* sap = static_cast<const float*>(a_scale.data_ptr());
  const auto* bp = static_cast<const uint8_t*>(b.data_ptr());
  const auto* sbp = static_cast<const float*>(b_scale.data_ptr());
  // shapes with too few tiles split K: fp32 partials in a workspace from the
  // caching allocator (no kernel runs to allocate or clear it)
  const int64_t need = cek_gemm_fp8_a8w8_workspace_size(M, N, K);
  if (need > 0) {
    at::Tensor ws = at::empty({(need + 3) / 4}, a_scale.options());
    check_rc(cek_gemm_fp8_a8w8_ws(ap, sap, bp, sbp, output.data_ptr(), M, N, K, io_code(output.scalar_type()),
                                  ws.data_ptr(), need, current_stream(a)),
             op);
  } else {
    check_rc(cek_gemm_fp8_a8w8(ap, sap, bp, sbp, output.data_ptr(), M, N, K, io_code(output.scalar_type()),
                               current_stream(a)),
             op);
  }
  return output;
}

// a8w8 gate/up GEMM over a merged [2d, K] e4m3 weight with gelu_and_mul fused
// into the epilogue: output[m, i] = gelu_tanh(g[m, i]) * u[m, i], g and u the
// rounded outputs of weight rows i and d + i.  Decode batches (M <= 16) take
// the fused kernel; other shapes run esimd_gemm_fp8_a8w8's kernels into a
// workspace and then gelu_and_mul (the same values).
void esimd_gemm_fp8_a8w8_gelu_and_mul(at::Tensor a, at::Tensor a_scale, at::Tensor b, at::Tensor b_scale,
                                      at::Tensor output) {
  const char* op = "esimd_gemm_fp8_a8w8_gelu_and_mul";
  TORCH_CHECK(a.element_size() == 1 && b.element_size() == 1, op, ": a and b must be 8-bit (e4m3) tensors");
  TORCH_CHECK(a.scalar_type() != at::ScalarType::Float8_e5m2 && b.scalar_type() != at::ScalarType::Float8_e5m2, op,
              ": a and b must be e4m3");
  TORCH_CHECK(a_scale.scalar_type() == at::ScalarType::Float && b_scale.scalar_type() == at::ScalarType::Float, op,
              ": scales must be fp32");
  TORCH_CHECK(is_io(output.scalar_type()), op, ": output must be fp16 or bf16");
  TORCH_CHECK(a.dim() == 2 && b.dim() == 2 && a.size(1) == b.size(1), op, ": a [M, K] and b [2d, K] required");
  TORCH_CHECK(b.size(0) % 2 == 0, op, ": b must have an even number of rows (gate rows, then up rows)");
  for (auto* t : {&a_scale, &b, &b_scale, &output}) check_device(*t, a, op, "operand");
  check_contig(a, op, "a");
  check_contig(b, op, "b");
  check_contig(a_scale, op, "a_scale");
  check_contig(b_scale, op, "b_scale");
  check_contig(output, op, "output");
  const int64_t M = a.size(0), K = a.size(1), d = b.size(0) / 2;
  TORCH_CHECK(K % 16 == 0, op, ": K must be a multiple of 16");
  TORCH_CHECK(a_scale.numel() == M && b_scale.numel() == 2 * d, op, ": a_scale [M] and b_scale [2d] required");
  TORCH_CHECK(output.numel() == M * d, op, ": output must be [M, d]");
  c10::OptionalDeviceGuard guard(a.device());
  void* st = current_stream(a);
  const int io = io_code(output.scalar_type());
  const auto* ap = static_cast<const uint8_t*>(a.data_ptr());
  const auto* sa = static_cast<const float*>(a_scale.data_ptr());
  const auto* bp = static_cast<const uint8_t*>(b.data_ptr());
  const auto* sb = static_cast<const float*>(b_scale.data_ptr());
  int rc = M <= 16 ? cek_gemv_fp8_gelu_and_mul(ap, sa, bp, sb, output.data_ptr(), M, d, K, io, CEK_E4M3, CEK_F32, st)
                   : CEK_ERR_UNSUPPORTED;
  if (rc == CEK_ERR_UNSUPPORTED && M > 0 && d > 0) {
    at::Tensor gu = at::empty({M, 2 * d}, output.options());
    check_rc(cek_gemm_fp8_a8w8(ap, sa, bp, sb, gu.data_ptr(), M, 2 * d, K, io, st), op);
    rc = cek_gelu_and_mul(output.data_ptr(), gu.data_ptr(), M, d, 2 * d, d, io, st);
  }
  check_rc(rc, op);
}
