// torch_ops.h -- at::Tensor entry points of the custom_esimd_kernels_vllm ops.
//
// The first four keep the reference's C++ signatures (reference
// include/kernel_ops.h:11-14,17-19,21-23,28-30); the rest are new ops in the
// same namespace.  Each shim validates its tensors, takes the current HIP
// stream of the input's device and calls the C ABI in include/cek.h.
#pragma once

#include <ATen/ATen.h>

#include <vector>

at::Tensor esimd_gemv_fp8_pern(at::Tensor input, at::Tensor weight, at::Tensor weight_scale,
                               at::Tensor output, int64_t N, int64_t K);

at::Tensor esimd_gemv_fp8_pert(at::Tensor input, at::Tensor weight, at::Tensor weight_scale,
                               at::Tensor output);

at::Tensor esimd_fused_add_rms_norm_batched(at::Tensor hidden_states, at::Tensor residual,
                                            at::Tensor weight, double eps);

at::Tensor esimd_gemm_fp8_pert(at::Tensor input, at::Tensor weight, at::Tensor weight_scale,
                               at::Tensor output);

// ---- new ops (no reference op) ----
// Fused GEMVs over several weight matrices sharing `input` (the reference's
// unregistered GEMV_fp8_pern_fused_host / GEMV_fp8_pert_fused_host).
void esimd_gemv_fp8_pern_fused(at::Tensor input, std::vector<at::Tensor> weights,
                               std::vector<at::Tensor> weight_scales, std::vector<at::Tensor> outputs);
void esimd_gemv_fp8_pert_fused(at::Tensor input, std::vector<at::Tensor> weights,
                               std::vector<at::Tensor> weight_scales, std::vector<at::Tensor> outputs);

void esimd_fused_add_rms_norm_quant_fp8(at::Tensor hidden_states, at::Tensor residual,
                                        at::Tensor weight, double eps, at::Tensor out_q,
                                        at::Tensor out_scale);

void esimd_per_token_quant_fp8(at::Tensor input, at::Tensor out_q, at::Tensor out_scale);

void esimd_gelu_and_mul(at::Tensor out, at::Tensor input);

// add+RMSNorm (+ per-token e4m3 quant) fused into the GEMV it feeds.
void esimd_fused_add_rms_norm_gemv_fp8(at::Tensor hidden_states, at::Tensor residual, at::Tensor weight, double eps,
                                       at::Tensor residual_out, at::Tensor w, at::Tensor w_scale, at::Tensor output,
                                       bool gelu_and_mul);
void esimd_fused_add_rms_norm_quant_gemv_fp8(at::Tensor hidden_states, at::Tensor residual, at::Tensor weight,
                                             double eps, at::Tensor residual_out, at::Tensor out_q,
                                             at::Tensor out_scale, at::Tensor b, at::Tensor b_scale,
                                             at::Tensor output, bool gelu_and_mul);

// Gate/up GEMV over a merged [2d, K] weight with gelu_and_mul fused.
void esimd_gemv_fp8_gelu_and_mul(at::Tensor input, at::Tensor weight, at::Tensor weight_scale, at::Tensor output);

void esimd_qk_norm_rope(at::Tensor q, at::Tensor k, at::Tensor q_weight, at::Tensor k_weight,
                        at::Tensor positions, double eps, double theta, bool is_neox);

// The QKV GEMV with QK RMSNorm + RoPE on its q and k columns fused into
// the last workgroup of each head.
void esimd_gemv_fp8_qk_norm_rope(at::Tensor input, at::Tensor weight, at::Tensor weight_scale, at::Tensor output,
                                 at::Tensor q_weight, at::Tensor k_weight, at::Tensor positions, int64_t n_q,
                                 int64_t n_k, double eps, double theta, bool is_neox, at::Tensor counters,
                                 c10::optional<at::Tensor> q_out);

// Deferred RMSNorm between two decode GEMVs: the producer (residual add,
// norm weight, per-tile sums of squares) and the row-scaled consumers.
int64_t esimd_gemv_fp8_add_rms_norm_defer_groups(int64_t N);
int64_t esimd_defer_norm_shift(double max_abs_norm_weight);
void esimd_gemv_fp8_add_rms_norm_defer(at::Tensor input, at::Tensor weight, at::Tensor weight_scale,
                                       at::Tensor residual, at::Tensor norm_weight, at::Tensor output,
                                       at::Tensor row_ss, int64_t norm_shift);
void esimd_gemv_fp8_pern_rs(at::Tensor input, at::Tensor weight, at::Tensor weight_scale, at::Tensor output,
                            at::Tensor row_ss, double eps);
void esimd_gemv_fp8_gelu_and_mul_rs(at::Tensor input, at::Tensor weight, at::Tensor weight_scale, at::Tensor output,
                                    at::Tensor row_ss, double eps);
void esimd_gemv_fp8_qk_norm_rope_rs(at::Tensor input, at::Tensor weight, at::Tensor weight_scale, at::Tensor output,
                                    at::Tensor q_weight, at::Tensor k_weight, at::Tensor positions, int64_t n_q,
                                    int64_t n_k, double eps, double theta, bool is_neox, at::Tensor counters,
                                    at::Tensor row_ss, double row_eps, c10::optional<at::Tensor> q_out);

at::Tensor esimd_gemm_fp8_a8w8(at::Tensor a, at::Tensor a_scale, at::Tensor b, at::Tensor b_scale,
                               at::Tensor output);

// The a8w8 form of esimd_gemv_fp8_gelu_and_mul (e4m3 activations and weights).
void esimd_gemm_fp8_a8w8_gelu_and_mul(at::Tensor a, at::Tensor a_scale, at::Tensor b, at::Tensor b_scale,
                                      at::Tensor output);
