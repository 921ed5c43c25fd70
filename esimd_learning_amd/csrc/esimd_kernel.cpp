// esimd_kernel.cpp -- torch shims of the GEMV, norm, quant, activation and
// RoPE ops (takes over the reference's csrc/xpu/esimd_kernel.sycl).
//
// Every shim: dtype checks with the reference's messages, then the checks the
// reference leaves out (device, contiguity, sizes), a device guard, the
// current HIP stream of the input's device, and one C-ABI call.  Outputs are
// written in place and returned as the reference does; nothing synchronises.
#include "torch_ops.h"

#include <ATen/MemoryOverlap.h>

#include <algorithm>
#include <vector>

#include "shim_common.h"

using namespace cek_shim;

static void check_gemv_io(const at::Tensor& input, const at::Tensor& output, const char* op) {
  TORCH_CHECK(is_io(input.scalar_type()), op, ": input must be fp16 or bf16");
  TORCH_CHECK(is_io(output.scalar_type()), op, ": output must be fp16 or bf16");
  TORCH_CHECK(input.scalar_type() == output.scalar_type(), op, ": input and output must have the same dtype");
}

// Rows of `input` that the op computes.  The reference kernels compute row 0
// only (csrc/xpu/esimd_kernels/fp8_GEMV_v2.h:62-75); here every row that both
// input and output hold, i.e. a superset that equals the reference for M = 1.
static int64_t gemv_rows(const at::Tensor& input, const at::Tensor& output, int64_t N, int64_t K) {
  return std::min(input.numel() / K, output.numel() / N);
}

static void run_gemv(const at::Tensor& input, const at::Tensor& weight, const at::Tensor& scale,
                     const at::Tensor& output, int64_t N, int64_t K, bool per_tensor, const char* op) {
  check_gemv_io(input, output, op);
  check_fp8_weight(weight, op);
  check_device(weight, input, op, "weight");
  check_device(scale, input, op, "weight_scale");
  check_device(output, input, op, "output");
  check_contig(input, op, "input");
  check_contig(weight, op, "weight");
  check_contig(output, op, "output");
  check_contig(scale, op, "weight_scale");
  TORCH_CHECK(N > 0 && K > 0, op, ": N and K must be positive");
  TORCH_CHECK(weight.numel() >= N * K, op, ": weight holds ", weight.numel(), " elements, need N*K = ", N * K);
  TORCH_CHECK(input.numel() >= K, op, ": input holds fewer than K elements");
  TORCH_CHECK(output.numel() >= N, op, ": output holds fewer than N elements");
  int scale_code = CEK_F32;
  if (per_tensor) {
    TORCH_CHECK(scale.scalar_type() == at::ScalarType::Float && scale.numel() >= 1, op,
                ": weight_scale must be an fp32 scalar tensor");
  } else {
    const auto st = scale.scalar_type();
    TORCH_CHECK(st == at::ScalarType::Half || st == at::ScalarType::BFloat16 || st == at::ScalarType::Float, op,
                ": weight_scale must be fp16, bf16 or fp32");
    TORCH_CHECK(scale.numel() >= N, op, ": weight_scale must hold N elements");
    scale_code = st == at::ScalarType::Float ? CEK_F32 : (st == at::ScalarType::Half ? CEK_F16 : CEK_BF16);
  }
  const int64_t M = gemv_rows(input, output, N, K);
  c10::OptionalDeviceGuard guard(input.device());
  void* st = current_stream(input);
  const int io = io_code(input.scalar_type());
  const int fmt = fp8_code(weight);
  // Up to 16 rows the decode GEMV kernels; more rows the w8a16 GEMM, which
  // streams the weights once for all of them.
  const int rc = per_tensor ? cek_gemv_fp8_pert(input.data_ptr(), weight.data_ptr(),
                                                static_cast<const float*>(scale.data_ptr()), output.data_ptr(), M, N,
                                                K, io, fmt, st)
                            : cek_gemv_fp8_pern(input.data_ptr(), weight.data_ptr(), scale.data_ptr(),
                                                output.data_ptr(), M, N, K, io, fmt, scale_code, st);
  check_rc(rc, op);
}

at::Tensor esimd_gemv_fp8_pern(at::Tensor input, at::Tensor weight, at::Tensor weight_scale,
                               at::Tensor output, int64_t N, int64_t K) {
  run_gemv(input, weight, weight_scale, output, N, K, false, "esimd_gemv_fp8_pern");
  return output;
}

at::Tensor esimd_gemv_fp8_pert(at::Tensor input, at::Tensor weight, at::Tensor weight_scale,
                               at::Tensor output) {
  TORCH_CHECK(weight.dim() == 2, "esimd_gemv_fp8_pert: weight must be [N, K]");
  run_gemv(input, weight, weight_scale, output, weight.size(0), weight.size(1), true, "esimd_gemv_fp8_pert");
  return output;
}

// Fused GEMVs sharing `input`: one launch per group of up to 8 matrices.
static void run_gemv_fused(const at::Tensor& input, const std::vector<at::Tensor>& weights,
                           const std::vector<at::Tensor>& scales, const std::vector<at::Tensor>& outputs,
                           bool per_tensor, const char* op) {
  TORCH_CHECK(!weights.empty() && weights.size() == scales.size() && weights.size() == outputs.size(), op,
              ": weights, weight_scales and outputs must be non-empty lists of one length");
  TORCH_CHECK(is_io(input.scalar_type()), op, ": input must be fp16 or bf16");
  TORCH_CHECK(input.is_cuda(), op, ": input must be a GPU tensor");
  check_contig(input, op, "input");
  const int64_t K = weights[0].dim() == 2 ? weights[0].size(1) : -1;
  TORCH_CHECK(K > 0 && input.numel() % K == 0, op, ": weights must be [N_i, K] with input [M, K]");
  const int64_t M = input.numel() / K;
  TORCH_CHECK(M <= 16, op, ": at most 16 activation rows");
  const int fmt = fp8_code(weights[0]);
  int scale_code = CEK_F32;
  for (size_t i = 0; i < weights.size(); ++i) {
    const auto& w = weights[i];
    const auto& sc = scales[i];
    const auto& y = outputs[i];
    check_fp8_weight(w, op);
    TORCH_CHECK(fp8_code(w) == fmt, op, ": all weights must share one fp8 format");
    TORCH_CHECK(w.dim() == 2 && w.size(1) == K, op, ": every weight must be [N_i, K]");
    check_device(w, input, op, "weight");
    check_device(sc, input, op, "weight_scale");
    check_device(y, input, op, "output");
    check_contig(w, op, "weight");
    check_contig(sc, op, "weight_scale");
    check_contig(y, op, "output");
    TORCH_CHECK(y.scalar_type() == input.scalar_type(), op, ": outputs must have the input's dtype");
    TORCH_CHECK(y.numel() == M * w.size(0), op, ": output ", i, " must be [M, N_i]");
    if (per_tensor) {
      TORCH_CHECK(sc.scalar_type() == at::ScalarType::Float && sc.numel() >= 1, op,
                  ": weight_scales must be fp32 scalar tensors");
    } else {
      const auto st = sc.scalar_type();
      TORCH_CHECK(st == at::ScalarType::Half || st == at::ScalarType::BFloat16 || st == at::ScalarType::Float, op,
                  ": weight_scales must be fp16, bf16 or fp32");
      const int code = st == at::ScalarType::Float ? CEK_F32 : (st == at::ScalarType::Half ? CEK_F16 : CEK_BF16);
      TORCH_CHECK(i == 0 || code == scale_code, op, ": all weight_scales must share one dtype");
      scale_code = code;
      TORCH_CHECK(sc.numel() >= w.size(0), op, ": weight_scale ", i, " must hold N_i elements");
    }
  }
  c10::OptionalDeviceGuard guard(input.device());
  void* st = current_stream(input);
  for (size_t b = 0; b < weights.size(); b += 8) {
    const int cnt = (int)std::min<size_t>(8, weights.size() - b);
    const void* wp[8];
    const void* sp[8];
    void* yp[8];
    int64_t ns[8];
    for (int i = 0; i < cnt; ++i) {
      wp[i] = weights[b + i].data_ptr();
      sp[i] = scales[b + i].data_ptr();
      yp[i] = outputs[b + i].data_ptr();
      ns[i] = weights[b + i].size(0);
    }
    const int io = io_code(input.scalar_type());
    int rc = per_tensor ? cek_gemv_fp8_pert_multi(input.data_ptr(), cnt, wp, reinterpret_cast<const float* const*>(sp),
                                                  yp, ns, M, K, io, fmt, st)
                        : cek_gemv_fp8_pern_multi(input.data_ptr(), cnt, wp, sp, yp, ns, M, K, io, fmt, scale_code, st);
    check_rc(rc, op);
  }
}

void esimd_gemv_fp8_pern_fused(at::Tensor input, std::vector<at::Tensor> weights,
                               std::vector<at::Tensor> weight_scales, std::vector<at::Tensor> outputs) {
  run_gemv_fused(input, weights, weight_scales, outputs, false, "esimd_gemv_fp8_pern_fused");
}

void esimd_gemv_fp8_pert_fused(at::Tensor input, std::vector<at::Tensor> weights,
                               std::vector<at::Tensor> weight_scales, std::vector<at::Tensor> outputs) {
  run_gemv_fused(input, weights, weight_scales, outputs, true, "esimd_gemv_fp8_pert_fused");
}

static void check_norm(const at::Tensor& h, const at::Tensor& r, const at::Tensor& w, const char* op) {
  TORCH_CHECK(is_io(h.scalar_type()), op, ": hidden_states must be fp16 or bf16");
  TORCH_CHECK(r.scalar_type() == h.scalar_type() && w.scalar_type() == h.scalar_type(), op,
              ": residual and weight must have the dtype of hidden_states");
  check_device(r, h, op, "residual");
  check_device(w, h, op, "weight");
  check_contig(h, op, "hidden_states");
  check_contig(r, op, "residual");
  check_contig(w, op, "weight");
  TORCH_CHECK(h.dim() >= 1 && h.size(-1) > 0, op, ": hidden_states must have a non-empty last dimension");
  TORCH_CHECK(r.numel() == h.numel(), op, ": residual must match hidden_states");
  TORCH_CHECK(w.numel() == h.size(-1), op, ": weight must have hidden_states.size(-1) elements");
}

at::Tensor esimd_fused_add_rms_norm_batched(at::Tensor hidden_states, at::Tensor residual,
                                            at::Tensor weight, double eps) {
  const char* op = "esimd_fused_add_rms_norm_batched";
  check_norm(hidden_states, residual, weight, op);
  const int64_t H = hidden_states.size(-1);
  const int64_t rows = hidden_states.numel() / H;
  c10::OptionalDeviceGuard guard(hidden_states.device());
  check_rc(cek_fused_add_rms_norm(hidden_states.data_ptr(), residual.data_ptr(), weight.data_ptr(), rows, H,
                                  (float)eps, io_code(hidden_states.scalar_type()), current_stream(hidden_states)),
           op);
  return hidden_states;
}

static void check_quant_out(const at::Tensor& ref, const at::Tensor& q, const at::Tensor& s, int64_t rows,
                            const char* op) {
  TORCH_CHECK(q.element_size() == 1, op, ": out_q must be an 8-bit tensor (float8_e4m3fn or uint8)");
  TORCH_CHECK(q.scalar_type() != at::ScalarType::Float8_e5m2, op, ": out_q must be e4m3, not e5m2");
  TORCH_CHECK(s.scalar_type() == at::ScalarType::Float, op, ": out_scale must be fp32");
  check_device(q, ref, op, "out_q");
  check_device(s, ref, op, "out_scale");
  check_contig(q, op, "out_q");
  check_contig(s, op, "out_scale");
  TORCH_CHECK(q.numel() == ref.numel(), op, ": out_q must have as many elements as the input");
  TORCH_CHECK(s.numel() == rows, op, ": out_scale must have one element per token (", rows, ")");
}

void esimd_fused_add_rms_norm_quant_fp8(at::Tensor hidden_states, at::Tensor residual, at::Tensor weight,
                                        double eps, at::Tensor out_q, at::Tensor out_scale) {
  const char* op = "esimd_fused_add_rms_norm_quant_fp8";
  check_norm(hidden_states, residual, weight, op);
  const int64_t H = hidden_states.size(-1);
  const int64_t rows = hidden_states.numel() / H;
  check_quant_out(hidden_states, out_q, out_scale, rows, op);
  c10::OptionalDeviceGuard guard(hidden_states.device());
  check_rc(cek_fused_add_rms_norm_quant_fp8(hidden_states.data_ptr(), residual.data_ptr(), weight.data_ptr(), rows,
                                            H, (float)eps, io_code(hidden_states.scalar_type()),
                                            static_cast<uint8_t*>(out_q.data_ptr()),
                                            static_cast<float*>(out_scale.data_ptr()), current_stream(hidden_states)),
           op);
}

void esimd_per_token_quant_fp8(at::Tensor input, at::Tensor out_q, at::Tensor out_scale) {
  const char* op = "esimd_per_token_quant_fp8";
  TORCH_CHECK(is_io(input.scalar_type()), op, ": input must be fp16 or bf16");
  TORCH_CHECK(input.is_cuda(), op, ": input must be a GPU tensor");
  check_contig(input, op, "input");
  TORCH_CHECK(input.dim() >= 1 && input.size(-1) > 0, op, ": input must have a non-empty last dimension");
  const int64_t H = input.size(-1);
  const int64_t rows = input.numel() / H;
  check_quant_out(input, out_q, out_scale, rows, op);
  c10::OptionalDeviceGuard guard(input.device());
  check_rc(cek_per_token_quant_fp8(input.data_ptr(), rows, H, io_code(input.scalar_type()),
                                   static_cast<uint8_t*>(out_q.data_ptr()), static_cast<float*>(out_scale.data_ptr()),
                                   current_stream(input)),
           op);
}

void esimd_gelu_and_mul(at::Tensor out, at::Tensor input) {
  const char* op = "esimd_gelu_and_mul";
  TORCH_CHECK(is_io(input.scalar_type()) && out.scalar_type() == input.scalar_type(), op,
              ": input and out must be fp16 or bf16 of the same dtype");
  check_device(out, input, op, "out");
  TORCH_CHECK(input.dim() >= 1 && input.size(-1) % 2 == 0, op, ": input's last dimension must be even");
  const int64_t d = input.size(-1) / 2;
  TORCH_CHECK(out.size(-1) == d, op, ": out's last dimension must be half of input's");
  TORCH_CHECK(input.stride(-1) == 1 && out.stride(-1) == 1, op, ": last dimensions must be contiguous");
  // Rows may be strided (e.g. a view into a wider buffer); leading dims flatten.
  const int64_t T = input.numel() / input.size(-1);
  TORCH_CHECK(out.numel() / d == T, op, ": out and input must have the same number of rows");
  const int64_t xs = input.dim() >= 2 ? input.stride(-2) : 2 * d;
  const int64_t os = out.dim() >= 2 ? out.stride(-2) : d;
  if (input.dim() > 2) TORCH_CHECK(input.is_contiguous(), op, ": >2-D input must be contiguous");
  if (out.dim() > 2) TORCH_CHECK(out.is_contiguous(), op, ": >2-D out must be contiguous");
  c10::OptionalDeviceGuard guard(input.device());
  check_rc(cek_gelu_and_mul(out.data_ptr(), input.data_ptr(), T, d, xs, os, io_code(input.scalar_type()),
                            current_stream(input)),
           op);
}

// Gate/up GEMV over a merged [2d, K] weight with gelu_and_mul fused into its
// epilogue: output[m, i] = gelu_tanh(g[m, i]) * u[m, i], g and u the GEMV's
// rounded outputs of rows i and d + i.  Up to 16 rows go to the fused
// kernel; shapes it does not cover, and more rows, run the GEMV into a
// workspace and then gelu_and_mul (the same values).
void esimd_gemv_fp8_gelu_and_mul(at::Tensor input, at::Tensor weight, at::Tensor weight_scale, at::Tensor output) {
  const char* op = "esimd_gemv_fp8_gelu_and_mul";
  check_gemv_io(input, output, op);
  check_fp8_weight(weight, op);
  check_device(weight, input, op, "weight");
  check_device(weight_scale, input, op, "weight_scale");
  check_device(output, input, op, "output");
  check_contig(input, op, "input");
  check_contig(weight, op, "weight");
  check_contig(weight_scale, op, "weight_scale");
  check_contig(output, op, "output");
  TORCH_CHECK(weight.dim() == 2 && weight.size(0) % 2 == 0 && weight.size(0) > 0 && weight.size(1) > 0, op,
              ": weight must be [2d, K]");
  const int64_t d = weight.size(0) / 2, K = weight.size(1);
  TORCH_CHECK(input.size(-1) == K, op, ": input must be [M, K]");
  const int64_t M = input.numel() / K;
  TORCH_CHECK(output.size(-1) == d && output.numel() == M * d, op, ": output must be [M, d]");
  const auto sdt = weight_scale.scalar_type();
  TORCH_CHECK(sdt == at::ScalarType::Half || sdt == at::ScalarType::BFloat16 || sdt == at::ScalarType::Float, op,
              ": weight_scale must be fp16, bf16 or fp32");
  TORCH_CHECK(weight_scale.numel() == 2 * d, op, ": weight_scale must hold 2d elements");
  const int scale_code = sdt == at::ScalarType::Float ? CEK_F32 : (sdt == at::ScalarType::Half ? CEK_F16 : CEK_BF16);
  c10::OptionalDeviceGuard guard(input.device());
  void* st = current_stream(input);
  const int io = io_code(input.scalar_type());
  const int fmt = fp8_code(weight);
  const size_t esz = input.element_size();
  if (M > 16) {
    // the GEMV over all rows at once (weights streamed once), then gelu_and_mul
    at::Tensor gu = at::empty({M, 2 * d}, input.options());
    check_rc(cek_gemv_fp8_pern(input.data_ptr(), weight.data_ptr(), weight_scale.data_ptr(), gu.data_ptr(), M, 2 * d,
                               K, io, fmt, scale_code, st),
             op);
    check_rc(cek_gelu_and_mul(output.data_ptr(), gu.data_ptr(), M, d, 2 * d, d, io, st), op);
    return;
  }
  at::Tensor gu;  // workspace of the unfused path, [16, 2d]
  for (int64_t m0 = 0; m0 < M; m0 += 16) {
    const int64_t mb = std::min<int64_t>(16, M - m0);
    const char* x = static_cast<const char*>(input.data_ptr()) + m0 * K * esz;
    char* y = static_cast<char*>(output.data_ptr()) + m0 * d * esz;
    int rc = cek_gemv_fp8_gelu_and_mul(x, nullptr, weight.data_ptr(), weight_scale.data_ptr(), y, mb, d, K, io, fmt,
                                       scale_code, st);
    if (rc == CEK_ERR_UNSUPPORTED) {
      if (!gu.defined()) gu = at::empty({16, 2 * d}, input.options());
      check_rc(cek_gemv_fp8_pern(x, weight.data_ptr(), weight_scale.data_ptr(), gu.data_ptr(), mb, 2 * d, K, io, fmt,
                                 scale_code, st),
               op);
      rc = cek_gelu_and_mul(y, gu.data_ptr(), mb, d, 2 * d, d, io, st);
    }
    check_rc(rc, op);
  }
}

// q / k are [T, n * hd] or [T, n, hd] views (rows may be strided, heads
// contiguous within a row), modified in place.
static int64_t rows_and_stride(const at::Tensor& t, int64_t hd, int64_t& n_heads, const char* op,
                               const char* name) {
  TORCH_CHECK(t.dim() == 2 || t.dim() == 3, op, ": ", name, " must be [T, n*hd] or [T, n, hd]");
  TORCH_CHECK(t.stride(-1) == 1, op, ": ", name, "'s last dimension must be contiguous");
  if (t.dim() == 3) {
    TORCH_CHECK(t.size(2) == hd && t.stride(1) == hd, op, ": ", name, " heads must be contiguous of size hd");
    n_heads = t.size(1);
  } else {
    TORCH_CHECK(t.size(1) % hd == 0, op, ": ", name, "'s width must be a multiple of head_dim");
    n_heads = t.size(1) / hd;
  }
  return t.stride(0);
}

void esimd_qk_norm_rope(at::Tensor q, at::Tensor k, at::Tensor q_weight, at::Tensor k_weight, at::Tensor positions,
                        double eps, double theta, bool is_neox) {
  const char* op = "esimd_qk_norm_rope";
  TORCH_CHECK(is_io(q.scalar_type()), op, ": q must be fp16 or bf16");
  TORCH_CHECK(k.scalar_type() == q.scalar_type() && q_weight.scalar_type() == q.scalar_type() &&
                  k_weight.scalar_type() == q.scalar_type(),
              op, ": q, k and the weights must share one dtype");
  TORCH_CHECK(positions.scalar_type() == at::ScalarType::Long, op, ": positions must be int64");
  check_device(k, q, op, "k");
  check_device(q_weight, q, op, "q_weight");
  check_device(k_weight, q, op, "k_weight");
  check_device(positions, q, op, "positions");
  check_contig(q_weight, op, "q_weight");
  check_contig(k_weight, op, "k_weight");
  check_contig(positions, op, "positions");
  const int64_t hd = q_weight.numel();
  TORCH_CHECK(k_weight.numel() == hd, op, ": q_weight and k_weight must both have head_dim elements");
  TORCH_CHECK(hd > 0 && hd % 2 == 0 && hd <= 512, op, ": head_dim must be even and <= 512");
  int64_t nq = 0, nk = 0;
  const int64_t qs = rows_and_stride(q, hd, nq, op, "q");
  const int64_t ks = rows_and_stride(k, hd, nk, op, "k");
  const int64_t T = q.size(0);
  TORCH_CHECK(k.size(0) == T && positions.numel() == T, op, ": q, k and positions must have T rows");
  c10::OptionalDeviceGuard guard(q.device());
  check_rc(cek_qk_norm_rope(q.data_ptr(), k.data_ptr(), q_weight.data_ptr(), k_weight.data_ptr(),
                            static_cast<const int64_t*>(positions.data_ptr()), T, nq, nk, hd, qs, ks, (float)eps,
                            (float)theta, is_neox ? 1 : 0, io_code(q.scalar_type()), current_stream(q)),
           op);
}

// ---- add+RMSNorm (+ quant) fused into the GEMV that consumes it ----
// residual_out = hidden + residual; the normed rows (or their e4m3 codes and
// scales) feed the GEMV (or the gate/up GEMV with gelu_and_mul).  Decode
// batches of up to four rows run as one launch; other shapes, and a
// residual_out that aliases the inputs, run the norm op on a copy and then
// the GEMV op (the same values).
// The norm kernels update their residual argument in place: residual_out
// takes residual's values first (nothing to copy when it is residual).
static void seed_residual_out(at::Tensor& residual_out, const at::Tensor& residual) {
  if (at::get_overlap_status(residual_out, residual) != at::MemOverlapStatus::Full) residual_out.copy_(residual);
}

static void check_norm_gemv_common(const at::Tensor& h, const at::Tensor& r, const at::Tensor& nw,
                                   const at::Tensor& r_out, const at::Tensor& w, const at::Tensor& ws,
                                   const at::Tensor& y, bool glu, const char* op, int64_t& M, int64_t& N,
                                   int64_t& K) {
  check_norm(h, r, nw, op);
  TORCH_CHECK(r_out.scalar_type() == h.scalar_type() && r_out.numel() == h.numel(), op,
              ": residual_out must match hidden_states");
  check_device(r_out, h, op, "residual_out");
  check_contig(r_out, op, "residual_out");
  check_fp8_weight(w, op);
  check_device(w, h, op, "weight");
  check_device(ws, h, op, "weight_scale");
  check_device(y, h, op, "output");
  check_contig(w, op, "weight");
  check_contig(ws, op, "weight_scale");
  check_contig(y, op, "output");
  K = h.size(-1);
  M = h.numel() / K;
  TORCH_CHECK(w.dim() == 2 && w.size(1) == K && w.size(0) > 0, op, ": weight must be [N, K] with K = hidden size");
  N = w.size(0);
  TORCH_CHECK(!glu || N % 2 == 0, op, ": with gelu_and_mul the weight must have 2d rows");
  TORCH_CHECK(y.scalar_type() == h.scalar_type(), op, ": output must have the dtype of hidden_states");
  TORCH_CHECK(y.numel() == M * (glu ? N / 2 : N), op, ": output must be [M, ", glu ? "d" : "N", "]");
}

void esimd_fused_add_rms_norm_gemv_fp8(at::Tensor hidden_states, at::Tensor residual, at::Tensor weight, double eps,
                                       at::Tensor residual_out, at::Tensor w, at::Tensor w_scale, at::Tensor output,
                                       bool gelu_and_mul) {
  const char* op = "esimd_fused_add_rms_norm_gemv_fp8";
  int64_t M, N, K;
  check_norm_gemv_common(hidden_states, residual, weight, residual_out, w, w_scale, output, gelu_and_mul, op, M, N, K);
  const auto sdt = w_scale.scalar_type();
  TORCH_CHECK(sdt == at::ScalarType::Half || sdt == at::ScalarType::BFloat16 || sdt == at::ScalarType::Float, op,
              ": weight_scale must be fp16, bf16 or fp32");
  TORCH_CHECK(w_scale.numel() == N, op, ": weight_scale must hold N elements");
  const int scale_code = sdt == at::ScalarType::Float ? CEK_F32 : (sdt == at::ScalarType::Half ? CEK_F16 : CEK_BF16);
  c10::OptionalDeviceGuard guard(hidden_states.device());
  void* st = current_stream(hidden_states);
  const int io = io_code(hidden_states.scalar_type());
  const int fmt = fp8_code(w);
  int rc = cek_add_rms_norm_gemv_fp8(hidden_states.data_ptr(), residual.data_ptr(), weight.data_ptr(), (float)eps,
                                     residual_out.data_ptr(), nullptr, nullptr, nullptr, w.data_ptr(),
                                     w_scale.data_ptr(), output.data_ptr(), M, N, K, gelu_and_mul ? 1 : 0, io, fmt,
                                     scale_code, st);
  if (rc != CEK_ERR_UNSUPPORTED) {
    check_rc(rc, op);
    return;
  }
  // two launches: the norm in place on copies, then the GEMV
  at::Tensor x = hidden_states.clone();
  seed_residual_out(residual_out, residual);
  check_rc(cek_fused_add_rms_norm(x.data_ptr(), residual_out.data_ptr(), weight.data_ptr(), M, K, (float)eps, io, st),
           op);
  if (gelu_and_mul) esimd_gemv_fp8_gelu_and_mul(x.view({M, K}), w, w_scale, output.view({M, N / 2}));
  else run_gemv(x, w, w_scale, output, N, K, false, op);
}

void esimd_fused_add_rms_norm_quant_gemv_fp8(at::Tensor hidden_states, at::Tensor residual, at::Tensor weight,
                                             double eps, at::Tensor residual_out, at::Tensor out_q,
                                             at::Tensor out_scale, at::Tensor b, at::Tensor b_scale,
                                             at::Tensor output, bool gelu_and_mul) {
  const char* op = "esimd_fused_add_rms_norm_quant_gemv_fp8";
  int64_t M, N, K;
  check_norm_gemv_common(hidden_states, residual, weight, residual_out, b, b_scale, output, gelu_and_mul, op, M, N, K);
  TORCH_CHECK(b.scalar_type() != at::ScalarType::Float8_e5m2, op, ": b must be e4m3");
  TORCH_CHECK(b_scale.scalar_type() == at::ScalarType::Float && b_scale.numel() == N, op,
              ": b_scale must be fp32 [N]");
  check_quant_out(hidden_states, out_q, out_scale, M, op);
  c10::OptionalDeviceGuard guard(hidden_states.device());
  void* st = current_stream(hidden_states);
  const int io = io_code(hidden_states.scalar_type());
  auto* q = static_cast<uint8_t*>(out_q.data_ptr());
  auto* qs = static_cast<float*>(out_scale.data_ptr());
  int rc = cek_add_rms_norm_gemv_fp8(hidden_states.data_ptr(), residual.data_ptr(), weight.data_ptr(), (float)eps,
                                     residual_out.data_ptr(), nullptr, q, qs, b.data_ptr(), b_scale.data_ptr(),
                                     output.data_ptr(), M, N, K, gelu_and_mul ? 1 : 0, io, CEK_E4M3, CEK_F32, st);
  if (rc != CEK_ERR_UNSUPPORTED) {
    check_rc(rc, op);
    return;
  }
  // two launches: norm + quant (hidden only read), then the a8w8 product.
  // hidden is read after residual_out has been seeded with residual, so it
  // is read from a copy when residual_out shares its memory.
  const at::Tensor h = at::get_overlap_status(residual_out, hidden_states) == at::MemOverlapStatus::No
                           ? hidden_states
                           : hidden_states.clone();
  seed_residual_out(residual_out, residual);
  check_rc(cek_fused_add_rms_norm_quant_fp8(h.data_ptr(), residual_out.data_ptr(), weight.data_ptr(), M, K,
                                            (float)eps, io, q, qs, st),
           op);
  const auto* bp = static_cast<const uint8_t*>(b.data_ptr());
  const auto* sb = static_cast<const float*>(b_scale.data_ptr());
  if (!gelu_and_mul) {
    check_rc(cek_gemm_fp8_a8w8(q, qs, bp, sb, output.data_ptr(), M, N, K, io, st), op);
    return;
  }
  rc = M <= 16 ? cek_gemv_fp8_gelu_and_mul(q, qs, bp, sb, output.data_ptr(), M, N / 2, K, io, CEK_E4M3, CEK_F32, st)
               : CEK_ERR_UNSUPPORTED;
  if (rc == CEK_ERR_UNSUPPORTED) {
    at::Tensor gu = at::empty({M, N}, output.options());
    check_rc(cek_gemm_fp8_a8w8(q, qs, bp, sb, gu.data_ptr(), M, N, K, io, st), op);
    rc = cek_gelu_and_mul(output.data_ptr(), gu.data_ptr(), M, N / 2, N, N / 2, io, st);
  }
  check_rc(rc, op);
}

// ---- GEMV with the consuming op fused into its last workgroup ----
// counters: int32 on the device, zero before the first call, left zero by
// every call (64 * (1 + ceil(N / 256)) for add+RMSNorm, 64 * (n_q + n_k)
// for QK-norm+RoPE: counters 256 bytes apart); calls that may overlap in
// time need their own.  Shapes the fused launch does not take
// run the GEMV op, then the norm / RoPE op (the same values).
static void check_counters(const at::Tensor& c, const at::Tensor& ref, int64_t need, const char* op) {
  TORCH_CHECK(c.scalar_type() == at::ScalarType::Int, op, ": counters must be int32");
  check_device(c, ref, op, "counters");
  check_contig(c, op, "counters");
  TORCH_CHECK(c.numel() >= need, op, ": counters must hold ", need, " elements");
}

static int scale_code_of(const at::Tensor& scale, int64_t N, const char* op) {
  const auto st = scale.scalar_type();
  TORCH_CHECK(st == at::ScalarType::Half || st == at::ScalarType::BFloat16 || st == at::ScalarType::Float, op,
              ": weight_scale must be fp16, bf16 or fp32");
  TORCH_CHECK(scale.numel() >= N, op, ": weight_scale must hold N elements");
  return st == at::ScalarType::Float ? CEK_F32 : (st == at::ScalarType::Half ? CEK_F16 : CEK_BF16);
}

// q_out (optional, [M, n_q hd] of the input's dtype): also receives the
// rotated q heads, as a copy of output's q columns would.
static void* check_q_out(const c10::optional<at::Tensor>& q_out, const at::Tensor& input, int64_t M, int64_t n_q,
                         int64_t hd, const char* op) {
  if (!q_out.has_value() || !q_out->defined()) return nullptr;
  TORCH_CHECK(q_out->scalar_type() == input.scalar_type(), op, ": q_out must have the input's dtype");
  check_device(*q_out, input, op, "q_out");
  check_contig(*q_out, op, "q_out");
  TORCH_CHECK(q_out->numel() == M * n_q * hd, op, ": q_out must be [M, n_q * head_dim]");
  return q_out->data_ptr();
}

void esimd_gemv_fp8_qk_norm_rope(at::Tensor input, at::Tensor weight, at::Tensor weight_scale, at::Tensor output,
                                 at::Tensor q_weight, at::Tensor k_weight, at::Tensor positions, int64_t n_q,
                                 int64_t n_k, double eps, double theta, bool is_neox, at::Tensor counters,
                                 c10::optional<at::Tensor> q_out) {
  const char* op = "esimd_gemv_fp8_qk_norm_rope";
  check_gemv_io(input, output, op);
  check_fp8_weight(weight, op);
  for (const auto* t : {&weight_scale, &output, &q_weight, &k_weight, &positions})
    check_device(*t, input, op, "operand");
  check_contig(input, op, "input");
  check_contig(weight, op, "weight");
  check_contig(weight_scale, op, "weight_scale");
  check_contig(output, op, "output");
  check_contig(q_weight, op, "q_weight");
  check_contig(k_weight, op, "k_weight");
  check_contig(positions, op, "positions");
  TORCH_CHECK(weight.dim() == 2 && weight.size(0) > 0 && weight.size(1) > 0, op, ": weight must be [N, K]");
  const int64_t N = weight.size(0), K = weight.size(1);
  TORCH_CHECK(input.size(-1) == K, op, ": input must be [M, K]");
  const int64_t M = input.numel() / K;
  TORCH_CHECK(output.numel() == M * N, op, ": output must be [M, N]");
  TORCH_CHECK(q_weight.scalar_type() == input.scalar_type() && k_weight.scalar_type() == input.scalar_type(), op,
              ": q_weight and k_weight must have the input's dtype");
  TORCH_CHECK(positions.scalar_type() == at::ScalarType::Long && positions.numel() == M, op,
              ": positions must be int64 [M]");
  const int64_t hd = q_weight.numel();
  TORCH_CHECK(k_weight.numel() == hd && hd > 0 && hd % 2 == 0 && hd <= 512, op,
              ": q_weight and k_weight must both have head_dim (even, <= 512) elements");
  TORCH_CHECK(n_q >= 0 && n_k >= 0 && (n_q + n_k) * hd <= N, op, ": the q and k heads must fit in the output row");
  check_counters(counters, input, 64 * (n_q + n_k), op);
  void* qo = check_q_out(q_out, input, M, n_q, hd, op);
  const int scale_code = scale_code_of(weight_scale, N, op);
  c10::OptionalDeviceGuard guard(input.device());
  void* st = current_stream(input);
  const int io = io_code(input.scalar_type());
  const int rc = cek_gemv_fp8_qk_norm_rope(
      input.data_ptr(), weight.data_ptr(), weight_scale.data_ptr(), output.data_ptr(), q_weight.data_ptr(),
      k_weight.data_ptr(), static_cast<const int64_t*>(positions.data_ptr()), n_q, n_k, hd, (float)eps, (float)theta,
      is_neox ? 1 : 0, static_cast<int*>(counters.data_ptr()), qo, M, N, K, io, fp8_code(weight), scale_code, st);
  if (rc != CEK_ERR_UNSUPPORTED) {
    check_rc(rc, op);
    return;
  }
  run_gemv(input, weight, weight_scale, output, N, K, false, op);
  if (n_q + n_k == 0) return;
  auto* y = static_cast<char*>(output.data_ptr());
  check_rc(cek_qk_norm_rope(y, y + n_q * hd * output.element_size(), q_weight.data_ptr(), k_weight.data_ptr(),
                            static_cast<const int64_t*>(positions.data_ptr()), M, n_q, n_k, hd, N, N, (float)eps,
                            (float)theta, is_neox ? 1 : 0, io, st),
           op);
  if (qo) q_out->view({M, n_q * hd}).copy_(output.view({M, N}).narrow(1, 0, n_q * hd));
}

// Deferred RMSNorm between two decode GEMVs (up to four rows, e4m3
// weights).  The producer GEMV (e.g. o_proj) adds its rounded output into
// the residual in place, writes output = residual * norm_weight * 2^-shift
// (the norm without its 1 / rms; the shift keeps it finite) and row_ss
// [M, G], G = defer_groups(N), the sums of squares of the unrounded sums
// times 2^-shift over G equal runs of columns; the consumer ops below (the
// plain GEMV, gate/up with gelu_and_mul, QKV with QK-norm + RoPE) take that
// output and row_ss and scale their rows by rsqrt(sum / K + eps), with
// eps * 4^-shift for the norm's eps.  No fallback: shapes the kernels do not
// take raise, and the caller runs the unfused ops.
static void check_defer_common(const at::Tensor& input, const at::Tensor& weight, const at::Tensor& weight_scale,
                               const at::Tensor& output, const char* op, int64_t& M, int64_t& N, int64_t& K) {
  check_gemv_io(input, output, op);
  check_fp8_weight(weight, op);
  check_device(weight, input, op, "weight");
  check_device(weight_scale, input, op, "weight_scale");
  check_device(output, input, op, "output");
  check_contig(input, op, "input");
  check_contig(weight, op, "weight");
  check_contig(weight_scale, op, "weight_scale");
  check_contig(output, op, "output");
  TORCH_CHECK(weight.dim() == 2 && weight.size(0) > 0 && weight.size(1) > 0, op, ": weight must be [N, K]");
  N = weight.size(0);
  K = weight.size(1);
  TORCH_CHECK(input.size(-1) == K, op, ": input must be [M, K]");
  M = input.numel() / K;
}

static void check_row_ss(const at::Tensor& row_ss, const at::Tensor& input, int64_t M, const char* op) {
  TORCH_CHECK(row_ss.scalar_type() == at::ScalarType::Float, op, ": row_ss must be fp32");
  check_device(row_ss, input, op, "row_ss");
  check_contig(row_ss, op, "row_ss");
  TORCH_CHECK(row_ss.dim() == 2 && row_ss.size(0) == M && row_ss.size(1) > 0, op, ": row_ss must be [M, n]");
}

int64_t esimd_gemv_fp8_add_rms_norm_defer_groups(int64_t N) { return cek_gemv_fp8_add_rms_norm_defer_groups(N); }

int64_t esimd_defer_norm_shift(double max_abs_norm_weight) {
  return cek_defer_norm_shift((float)max_abs_norm_weight);
}

void esimd_gemv_fp8_add_rms_norm_defer(at::Tensor input, at::Tensor weight, at::Tensor weight_scale,
                                       at::Tensor residual, at::Tensor norm_weight, at::Tensor output,
                                       at::Tensor row_ss, int64_t norm_shift) {
  const char* op = "esimd_gemv_fp8_add_rms_norm_defer";
  int64_t M, N, K;
  check_defer_common(input, weight, weight_scale, output, op, M, N, K);
  TORCH_CHECK(output.numel() == M * N, op, ": output must be [M, N]");
  TORCH_CHECK(residual.scalar_type() == input.scalar_type() && norm_weight.scalar_type() == input.scalar_type(), op,
              ": residual and norm_weight must have the input's dtype");
  check_device(residual, input, op, "residual");
  check_device(norm_weight, input, op, "norm_weight");
  check_contig(residual, op, "residual");
  check_contig(norm_weight, op, "norm_weight");
  TORCH_CHECK(residual.numel() == M * N && norm_weight.numel() == N, op,
              ": residual must be [M, N] and norm_weight [N]");
  TORCH_CHECK(N % 16 == 0, op, ": N must be a multiple of 16");
  TORCH_CHECK(row_ss.scalar_type() == at::ScalarType::Float, op, ": row_ss must be fp32");
  check_device(row_ss, input, op, "row_ss");
  check_contig(row_ss, op, "row_ss");
  TORCH_CHECK(row_ss.numel() == M * cek_gemv_fp8_add_rms_norm_defer_groups(N), op,
              ": row_ss must be [M, esimd_gemv_fp8_add_rms_norm_defer_groups(N)]");
  TORCH_CHECK(norm_shift >= -24 && norm_shift <= 24, op, ": norm_shift must be in [-24, 24]");
  const int scale_code = scale_code_of(weight_scale, N, op);
  c10::OptionalDeviceGuard guard(input.device());
  check_rc(cek_gemv_fp8_add_rms_norm_defer(input.data_ptr(), weight.data_ptr(), weight_scale.data_ptr(),
                                           residual.data_ptr(), norm_weight.data_ptr(), output.data_ptr(),
                                           static_cast<float*>(row_ss.data_ptr()), (int)norm_shift, M, N, K,
                                           io_code(input.scalar_type()), fp8_code(weight), scale_code,
                                           current_stream(input)),
           op);
}

void esimd_gemv_fp8_pern_rs(at::Tensor input, at::Tensor weight, at::Tensor weight_scale, at::Tensor output,
                            at::Tensor row_ss, double eps) {
  const char* op = "esimd_gemv_fp8_pern_rs";
  int64_t M, N, K;
  check_defer_common(input, weight, weight_scale, output, op, M, N, K);
  TORCH_CHECK(output.numel() == M * N, op, ": output must be [M, N]");
  check_row_ss(row_ss, input, M, op);
  const int scale_code = scale_code_of(weight_scale, N, op);
  c10::OptionalDeviceGuard guard(input.device());
  check_rc(cek_gemv_fp8_pern_rs(input.data_ptr(), weight.data_ptr(), weight_scale.data_ptr(), output.data_ptr(),
                                static_cast<const float*>(row_ss.data_ptr()), row_ss.size(1), (float)eps, M, N, K,
                                io_code(input.scalar_type()), fp8_code(weight), scale_code, current_stream(input)),
           op);
}

void esimd_gemv_fp8_gelu_and_mul_rs(at::Tensor input, at::Tensor weight, at::Tensor weight_scale, at::Tensor output,
                                    at::Tensor row_ss, double eps) {
  const char* op = "esimd_gemv_fp8_gelu_and_mul_rs";
  int64_t M, N, K;
  check_defer_common(input, weight, weight_scale, output, op, M, N, K);
  TORCH_CHECK(N % 2 == 0 && output.size(-1) == N / 2 && output.numel() == M * (N / 2), op,
              ": weight must be [2d, K] and output [M, d]");
  TORCH_CHECK(weight_scale.numel() == N, op, ": weight_scale must hold 2d elements");
  check_row_ss(row_ss, input, M, op);
  const int scale_code = scale_code_of(weight_scale, N, op);
  c10::OptionalDeviceGuard guard(input.device());
  check_rc(cek_gemv_fp8_gelu_and_mul_rs(input.data_ptr(), weight.data_ptr(), weight_scale.data_ptr(),
                                        output.data_ptr(), static_cast<const float*>(row_ss.data_ptr()),
                                        row_ss.size(1), (float)eps, M, N / 2, K, io_code(input.scalar_type()),
                                        fp8_code(weight), scale_code, current_stream(input)),
           op);
}

void esimd_gemv_fp8_qk_norm_rope_rs(at::Tensor input, at::Tensor weight, at::Tensor weight_scale, at::Tensor output,
                                    at::Tensor q_weight, at::Tensor k_weight, at::Tensor positions, int64_t n_q,
                                    int64_t n_k, double eps, double theta, bool is_neox, at::Tensor counters,
                                    at::Tensor row_ss, double row_eps, c10::optional<at::Tensor> q_out) {
  const char* op = "esimd_gemv_fp8_qk_norm_rope_rs";
  int64_t M, N, K;
  check_defer_common(input, weight, weight_scale, output, op, M, N, K);
  TORCH_CHECK(output.numel() == M * N, op, ": output must be [M, N]");
  for (const auto* t : {&q_weight, &k_weight, &positions}) check_device(*t, input, op, "operand");
  check_contig(q_weight, op, "q_weight");
  check_contig(k_weight, op, "k_weight");
  check_contig(positions, op, "positions");
  TORCH_CHECK(q_weight.scalar_type() == input.scalar_type() && k_weight.scalar_type() == input.scalar_type(), op,
              ": q_weight and k_weight must have the input's dtype");
  TORCH_CHECK(positions.scalar_type() == at::ScalarType::Long && positions.numel() == M, op,
              ": positions must be int64 [M]");
  const int64_t hd = q_weight.numel();
  TORCH_CHECK(k_weight.numel() == hd && hd > 0, op, ": q_weight and k_weight must both have head_dim elements");
  TORCH_CHECK(n_q >= 0 && n_k >= 0 && (n_q + n_k) * hd <= N, op, ": the q and k heads must fit in the output row");
  check_counters(counters, input, 64 * (n_q + n_k), op);
  check_row_ss(row_ss, input, M, op);
  void* qo = check_q_out(q_out, input, M, n_q, hd, op);
  const int scale_code = scale_code_of(weight_scale, N, op);
  c10::OptionalDeviceGuard guard(input.device());
  check_rc(cek_gemv_fp8_qk_norm_rope_rs(
               input.data_ptr(), weight.data_ptr(), weight_scale.data_ptr(), output.data_ptr(), q_weight.data_ptr(),
               k_weight.data_ptr(), static_cast<const int64_t*>(positions.data_ptr()), n_q, n_k, hd, (float)eps,
               (float)theta, is_neox ? 1 : 0, static_cast<int*>(counters.data_ptr()), qo,
               static_cast<const float*>(row_ss.data_ptr()), row_ss.size(1), (float)row_eps, M, N, K,
               io_code(input.scalar_type()), fp8_code(weight), scale_code, current_stream(input)),
           op);
}
