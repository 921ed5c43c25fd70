/*
 * cek.h -- C ABI of the MI355X (gfx950) fp8 decode/prefill op pack.
 *
 * Library: libcek.so (built with hipcc --offload-arch=gfx950).
 * All pointers are HIP device pointers unless stated; sizes are element
 * counts; `stream` is a hipStream_t passed as void* (NULL = legacy default
 * stream).  Every entry point only enqueues work on `stream`: no host
 * synchronisation, no host read of device scales, no allocation.  Entry
 * points are stateless and re-entrant (cek_gemm_fp8_a8w8_noalloc aside: its
 * calls share one static buffer per GPU).  Return value: CEK_OK (0) or a
 * CEK_ERR_* code; cek_error_string() names it.  Nothing throws across the
 * ABI.
 *
 * The reference (Intel-XPU SYCL-ESIMD package custom_esimd_kernels_vllm)
 * has no C ABI: its boundary is torch ops whose host shims extract raw
 * pointers and launch kernels.  Each entry point below names the reference
 * shim / host function it takes over (paths relative to the reference
 * repository root).  Functions marked NEW have no reference counterpart.
 */
#ifndef CEK_H
#define CEK_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types of activation / output tensors */
enum cek_dtype { CEK_F16 = 0, CEK_BF16 = 1, CEK_F32 = 2 };
/* fp8 weight encodings (reference get_fp8_mode, csrc/xpu/esimd_kernel.sycl:14-16) */
enum cek_fp8 { CEK_E4M3 = 0, CEK_E5M2 = 1 };

enum cek_status {
  CEK_OK = 0,
  CEK_ERR_INVALID = 1,      /* bad size, pointer, alignment or enum value */
  CEK_ERR_UNSUPPORTED = 2,  /* valid request this build has no kernel for */
  CEK_ERR_HIP = 3,          /* a HIP runtime call or launch failed */
  CEK_ERR_SCRATCH = 4       /* request needs more than the static scratch buffer holds */
};

const char* cek_error_string(int status);
/* Last HIP error message seen by this thread (empty string if none). */
const char* cek_last_hip_error(void);
/* ABI version: major * 10000 + minor * 100 + patch. */
int cek_version(void);

/*
 * fp8-weight GEMV with per-output-channel scale.
 *   y[m, n] = Out( (sum_k f32(x[m, k]) * dq(w[n, k])) * f32(scale[n]) )
 * x [M, K] io_dtype (F16|BF16), w [N, K] fp8 row-major (K contiguous),
 * scale [N] of scale_dtype (F16|BF16|F32), y [M, N] io_dtype.  M <= 16 runs
 * the decode GEMV kernels; larger M the w8a16 GEMM of cek_gemm_fp8_pert
 * with this scale (the weights are streamed once for all rows).
 * Replaces esimd_gemv_fp8_pern, csrc/xpu/esimd_kernel.sycl:22-53 ->
 * GEMV_fp8_pern_host, csrc/xpu/esimd_kernels/fp8_GEMV_v2.h:127-191 (which
 * computes row 0 only; here every row m < M).
 */
int cek_gemv_fp8_pern(const void* x, const void* w, const void* scale, void* y,
                      int64_t M, int64_t N, int64_t K,
                      int io_dtype, int fp8_fmt, int scale_dtype, void* stream);

/*
 * Same with a per-tensor fp32 scale read on the device (*scale).
 * Replaces esimd_gemv_fp8_pert, csrc/xpu/esimd_kernel.sycl:57-89 ->
 * GEMV_fp8_pert_host, csrc/xpu/esimd_kernels/fp8_GEMV_v2.h:370-434.
 */
int cek_gemv_fp8_pert(const void* x, const void* w, const float* scale, void* y,
                      int64_t M, int64_t N, int64_t K,
                      int io_dtype, int fp8_fmt, void* stream);

/*
 * Several fp8-weight GEMVs that share one activation matrix, in one launch
 * (e.g. Q, K and V, or gate and up projections).  Host arrays of `count`
 * (1..8) device pointers / row counts: w[i] [N[i], K], scale[i] (per-channel
 * of scale_dtype for _pern, fp32 device scalar for _pert), y[i] [M, N[i]].
 * Each y[i] equals what cek_gemv_fp8_pern/pert computes for matrix i.
 * Replaces the reference's GEMV_fp8_pern_fused_host (fp8_GEMV_v2.h:263-316)
 * and GEMV_fp8_pert_fused_host (:506-558), csrc/xpu/esimd_kernels/, which
 * the reference defines but does not register as an op.
 */
int cek_gemv_fp8_pern_multi(const void* x, int count, const void* const* w, const void* const* scale,
                            void* const* y, const int64_t* N, int64_t M, int64_t K,
                            int io_dtype, int fp8_fmt, int scale_dtype, void* stream);
int cek_gemv_fp8_pert_multi(const void* x, int count, const void* const* w, const float* const* scale,
                            void* const* y, const int64_t* N, int64_t M, int64_t K,
                            int io_dtype, int fp8_fmt, void* stream);

/*
 * fp8-weight GEMM, fp16|bf16 activations, per-tensor fp32 scale, any M.
 *   Y[m, n] = Out( (sum_k f32(X[m, k]) * dq(W[n, k])) * (*scale) )
 * M <= 16 uses the GEMV kernels; N <= 16 an activation-streaming MFMA
 * kernel (the reference's tiny-N path); 16 < M <= 32 the LDS-staged GEMV
 * kernel where it has an instantiation; otherwise a tiled w8a16 MFMA GEMM.
 * Replaces esimd_gemm_fp8_pert, csrc/xpu/esimd_kernel_gemm.sycl:23-65 ->
 * GEMM_fp8_pert_dispatch, csrc/xpu/esimd_kernels/fp8_GEMM_pert.h:4017-4062.
 */
int cek_gemm_fp8_pert(const void* x, const void* w, const float* scale, void* y,
                      int64_t M, int64_t N, int64_t K,
                      int io_dtype, int fp8_fmt, void* stream);

/*
 * The same product with a caller-provided workspace, which lets shapes with
 * too few output tiles (e.g. M = 512, K = 14336) split K into parts: fp32
 * partial sums in the workspace, then a second launch that adds them in
 * order and scales (deterministic).  cek_gemm_fp8_pert_workspace_size gives
 * the bytes the plan needs for (M, N, K), 0 when it runs unsplit; with a
 * smaller workspace (or none) the call runs unsplit, like cek_gemm_fp8_pert.
 * The workspace needs no initialisation and must be 4-byte aligned
 * (CEK_ERR_INVALID otherwise).  Extends esimd_gemm_fp8_pert (same
 * reference entry as cek_gemm_fp8_pert): the reference has no split K.
 */
int64_t cek_gemm_fp8_pert_workspace_size(int64_t M, int64_t N, int64_t K);
int cek_gemm_fp8_pert_ws(const void* x, const void* w, const float* scale, void* y,
                         int64_t M, int64_t N, int64_t K, int io_dtype, int fp8_fmt,
                         void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Batched fused residual add + RMSNorm, in place:
 *   residual = f16(hidden + residual);
 *   hidden   = f16(residual * rsqrt(mean((hidden+residual)^2) + eps) * weight)
 * hidden, residual [rows, H] io_dtype; weight [H] io_dtype (Gemma w+1).
 * Replaces esimd_fused_add_rms_norm_batched, csrc/xpu/esimd_kernel.sycl:92-109
 * -> fused_add_rms_norm_batched_host,
 * csrc/xpu/esimd_kernels/fused_add_rms_norm_batched.h:66-76.
 */
int cek_fused_add_rms_norm(void* hidden, void* residual, const void* weight,
                           int64_t rows, int64_t H, float eps, int io_dtype, void* stream);

/*
 * NEW: fused residual add + RMSNorm + per-token e4m3 quantisation.
 * residual is updated as above; hidden is only read.  The normed row is
 * rounded to io_dtype, then
 *   scale[t] = max(amax_t / 448, 1 / (448 * 512))     (fp32)
 *   q[t, i]  = e4m3_rne(clamp(normed[t, i] / scale[t], -448, 448))
 * q [rows, H] bytes; scale [rows] fp32.  Equal, bit for bit, to
 * cek_fused_add_rms_norm followed by cek_per_token_quant_fp8.
 */
int cek_fused_add_rms_norm_quant_fp8(const void* hidden, void* residual, const void* weight,
                                     int64_t rows, int64_t H, float eps, int io_dtype,
                                     uint8_t* q, float* scale, void* stream);

/* NEW: per-token e4m3 quantisation of x [rows, H] (same formula as above). */
int cek_per_token_quant_fp8(const void* x, int64_t rows, int64_t H, int io_dtype,
                            uint8_t* q, float* scale, void* stream);

/*
 * NEW: a8w8 GEMM on fp8 MFMA.
 *   Y[m, n] = Out( sa[m] * sb[n] * sum_k dq(A[m, k]) * dq(B[n, k]) )
 * A [M, K], B [N, K] e4m3 row-major; sa [M], sb [N] fp32; Y [M, N] out_dtype
 * (F16|BF16).  K % 16 == 0.
 */
int cek_gemm_fp8_a8w8(const uint8_t* a, const float* sa, const uint8_t* b, const float* sb,
                      void* y, int64_t M, int64_t N, int64_t K, int out_dtype, void* stream);

/*
 * NEW: the same product with a caller-provided workspace, which lets shapes
 * with too few output tiles to fill the GPU (e.g. M = 512, K = 14336; M = 64) split
 * K into parts: each part's fp32 partial sums go to the workspace, and a
 * second launch adds them in order, scales and converts (deterministic).
 * cek_gemm_fp8_a8w8_workspace_size returns the bytes that plan needs for
 * (M, N, K), 0 when the shape runs unsplit; with a smaller workspace (or
 * none) the call runs unsplit, like cek_gemm_fp8_a8w8.  The workspace is
 * fully written before it is read: it needs no initialisation.  It must be
 * 4-byte aligned (CEK_ERR_INVALID otherwise); 16-byte alignment lets the
 * second launch use 16-byte accesses.
 */
int64_t cek_gemm_fp8_a8w8_workspace_size(int64_t M, int64_t N, int64_t K);
int cek_gemm_fp8_a8w8_ws(const uint8_t* a, const float* sa, const uint8_t* b, const float* sb,
                         void* y, int64_t M, int64_t N, int64_t K, int out_dtype,
                         void* workspace, int64_t workspace_bytes, void* stream);

/*
 * NEW, and with no counterpart in the reference: the a8w8 GEMM for callers
 * that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments and results as
 * cek_gemm_fp8_a8w8_ws given the workspace its plan asks for, but the
 * split-K partial sums go to a static device buffer inside the library
 * (32 MiB, one per GPU, held until the process ends); the call allocates
 * nothing.  Shapes whose plan needs more (cek_gemm_fp8_a8w8_workspace_size
 * above 33554432 bytes) return CEK_ERR_SCRATCH; shapes that run unsplit use
 * no scratch.  The first call on a device looks up the buffer's address on
 * that device (a host query, no allocation); make that call once at set-up,
 * outside any graph capture, after which calls may be captured.  All calls
 * on one GPU share the buffer: calls that overlap in time there (e.g. on two
 * streams, or two replays of graphs holding such calls) race.
 */
int cek_gemm_fp8_a8w8_noalloc(const uint8_t* a, const float* sa, const uint8_t* b, const float* sb,
                              void* y, int64_t M, int64_t N, int64_t K, int out_dtype, void* stream);

/*
 * NEW: out[t, i] = gelu_tanh(x[t, i]) * x[t, d + i], fp32 math.
 * x rows have stride x_stride elements (>= 2d), out rows out_stride (>= d).
 */
int cek_gelu_and_mul(void* out, const void* x, int64_t T, int64_t d,
                     int64_t x_stride, int64_t out_stride, int io_dtype, void* stream);

/*
 * NEW: fused residual add + RMSNorm (+ per-token e4m3 quantisation) feeding
 * the fp8 GEMV, in one launch (no counterpart in the reference: it is
 * esimd_fused_add_rms_norm_batched, csrc/xpu/esimd_kernel.sycl:92-109,
 * followed by esimd_gemv_fp8_pern, :22-53):
 *   residual_out = Out(hidden + residual)                      [M, K]
 *   x            = Out(residual_out * rsqrt(mean((hidden + residual)^2) + eps) * norm_weight)
 *   q_out == NULL: hidden_out = x (if not NULL); y = GEMV(x, W, scale)
 *   q_out != NULL: q_out, q_scale = per-token e4m3 quant of x (the formula
 *                  of cek_fused_add_rms_norm_quant_fp8); y = a8w8 GEMV of
 *                  the codes (W e4m3, scale fp32 [N])
 * with gelu_and_mul != 0: W holds 2d = N rows (gate, then up) and y [M, d]
 * is gelu_tanh(gate) * up, as cek_gemv_fp8_gelu_and_mul.  residual_out,
 * hidden_out, q_out and q_scale equal the unfused ops' bit for bit, and so
 * does y from three rows on and with gelu_and_mul (at one or two rows the
 * unfused GEMV sums in another order: y within the GEMV's tolerance).
 * residual_out and hidden_out must not overlap hidden or residual.  Covers
 * M <= 4 (with q_out: M = 1, where one launch is faster than two), K in
 * {3072, 4096, 5120}, e4m3 weights and 16-byte aligned operands;
 * CEK_ERR_UNSUPPORTED otherwise, for the caller to run the norm and the
 * GEMV as two launches.
 */
int cek_add_rms_norm_gemv_fp8(const void* hidden, const void* residual, const void* norm_weight, float eps,
                              void* residual_out, void* hidden_out, uint8_t* q_out, float* q_scale,
                              const void* w, const void* scale, void* y, int64_t M, int64_t N, int64_t K,
                              int gelu_and_mul, int io_dtype, int fp8_fmt, int scale_dtype, void* stream);

/*
 * NEW: gate/up GEMV with gelu_and_mul fused into its epilogue (no
 * counterpart in the reference: it is esimd_gemv_fp8_pern over a merged
 * [2d, K] gate/up weight, csrc/xpu/esimd_kernel.sycl:22-53, followed by
 * cek_gelu_and_mul, in one launch):
 *   g[m, i] = Out(sum_k x[m, k] * dq(W[i, k]) * s[i])          rows [0, d)
 *   u[m, i] = Out(sum_k x[m, k] * dq(W[d + i, k]) * s[d + i])  rows [d, 2d)
 *   y[m, i] = Out(gelu_tanh(g[m, i]) * u[m, i])                y [M, d]
 * x_scale == NULL: x is io_dtype [M, K], s [2d] of scale_dtype (F16|BF16|F32),
 * W e4m3 or e5m2 (fp8_fmt).  x_scale != NULL: x holds e4m3 codes [M, K] with
 * per-row fp32 scales x_scale [M], W e4m3 and s fp32 (the a8w8 contract; the
 * sums then carry x_scale[m] too).  Covers M <= 16, K in {3072, 4096, 5120}
 * and 16-byte aligned x and W; CEK_ERR_UNSUPPORTED otherwise, for the caller
 * to run the GEMV and cek_gelu_and_mul instead.
 */
int cek_gemv_fp8_gelu_and_mul(const void* x, const float* x_scale, const void* w, const void* scale,
                              void* y, int64_t M, int64_t d, int64_t K, int io_dtype, int fp8_fmt,
                              int scale_dtype, void* stream);

/*
 * NEW: the fused QKV GEMV with the per-head QK RMSNorm + RoPE fused in (no
 * counterpart in the reference: it is esimd_gemv_fp8_pern over the QKV
 * weight, csrc/xpu/esimd_kernel.sycl:22-53, followed by cek_qk_norm_rope on
 * the q and k columns of its output):
 *   y = GEMV(x, w, scale) [M, N]; then, in place, cek_qk_norm_rope on
 *   q = y[:, 0 : n_q hd] and k = y[:, n_q hd : (n_q + n_k) hd] (row stride N)
 * with the same values bit for bit.  For each q / k head the workgroup that
 * finishes the head's rows last does its norm and rotation; `counters`
 * (64 * (n_q + n_k) ints: one counter per head, 256 bytes apart) must be
 * zero before the first call and are left zero -- calls that may overlap in
 * time need their own.  q_out (may be null): [M, n_q hd], also receives the
 * rotated q heads (what a copy of y's q columns gives), written by the same
 * workgroups; it must not overlap y, x or w.  Covers M <= 4,
 * K in {3072, 4096, 5120}, N % 16 == 0, head_dim 128 or 256, e4m3 weights,
 * 16-byte aligned operands; CEK_ERR_UNSUPPORTED otherwise (run the GEMV,
 * then cek_qk_norm_rope).
 */
int cek_gemv_fp8_qk_norm_rope(const void* x, const void* w, const void* scale, void* y, const void* q_weight,
                              const void* k_weight, const int64_t* positions, int64_t n_q, int64_t n_k,
                              int64_t head_dim, float eps, float theta, int is_neox, int* counters, void* q_out,
                              int64_t M, int64_t N, int64_t K, int io_dtype, int fp8_fmt, int scale_dtype,
                              void* stream);

/*
 * NEW: an add + RMSNorm deferred across the GEMV that produces its input
 * and the GEMV that consumes its output (no counterpart in the reference:
 * there it is esimd_gemv_fp8_pern, csrc/xpu/esimd_kernel.sycl:22-53, then
 * esimd_fused_add_rms_norm_batched, :92-120, then the next GEMV).
 *
 * Producer, cek_gemv_fp8_add_rms_norm_defer: o = the GEMV's rounded output
 * [M, N]; s = o + residual (fp32); residual = round(s) in place;
 * y = round(residual * norm_weight[n] * 2^-norm_shift) -- the norm without
 * its 1 / rms -- and ss_out [M][G], G = cek_gemv_fp8_add_rms_norm_defer_groups(N):
 * the sums of (s * 2^-norm_shift)^2 over each of G equal runs of N / G
 * columns (G = N / 16, or N / 12 where 16-column runs would give fewer than
 * 256 workgroups and N is a multiple of 48: N = 3072 -> 256).  Both products
 * are exact in fp32, so the shift only moves y's one rounding.  With
 * 2^norm_shift >= max |norm_weight| (cek_defer_norm_shift) |y| <= |residual|,
 * so y cannot overflow a 16-bit type whatever the residual holds; with
 * norm_shift = 0 an fp16 y overflows once |residual * norm_weight| > 65504.
 * |norm_shift| <= 24 (else CEK_ERR_INVALID).  y, residual and ss_out must
 * not overlap each other, x, w, the weight scale or norm_weight.
 *
 * Consumers (_rs): the named op over x = the producer's y, with each output
 * row m scaled, before rounding (and before gelu_and_mul, QK-norm and RoPE),
 * by inv[m] = rsqrt(sum_j row_ss[m][j] / K + row_eps); n_ss = the producer's
 * G (<= 256, a multiple of 4, row_ss 16-byte aligned), summed in a fixed
 * order.  For the norm's eps pass row_eps = eps * 4^-norm_shift: the scaled
 * sums then give 2^norm_shift / rms, which undoes the producer's shift.
 * The result equals the unfused norm -> GEMV to within the rounding of the
 * moved 1 / rms (not bit for bit).
 *
 * All: M <= 4, K a multiple of 1024 (producer and plain consumer: K / 1024
 * in {2, 3, 4, 5, 14, 24}; gate/up and QKV: 3072, 4096, 5120), N % 16 == 0,
 * e4m3 weights, 16-byte aligned x and w; CEK_ERR_UNSUPPORTED otherwise (no
 * fallback: run the unfused ops).
 */
int64_t cek_gemv_fp8_add_rms_norm_defer_groups(int64_t N);  /* G for N (a multiple of 16), else 0 */
/* The smallest shift E with 2^E >= max_abs_norm_weight (0 for 0, clamped to +-24). */
int cek_defer_norm_shift(float max_abs_norm_weight);
int cek_gemv_fp8_add_rms_norm_defer(const void* x, const void* w, const void* scale, void* residual,
                                    const void* norm_weight, void* y, float* ss_out, int norm_shift, int64_t M,
                                    int64_t N, int64_t K, int io_dtype, int fp8_fmt, int scale_dtype, void* stream);
int cek_gemv_fp8_pern_rs(const void* x, const void* w, const void* scale, void* y, const float* row_ss, int64_t n_ss,
                         float row_eps, int64_t M, int64_t N, int64_t K, int io_dtype, int fp8_fmt, int scale_dtype,
                         void* stream);
int cek_gemv_fp8_gelu_and_mul_rs(const void* x, const void* w, const void* scale, void* y, const float* row_ss,
                                 int64_t n_ss, float row_eps, int64_t M, int64_t d, int64_t K, int io_dtype,
                                 int fp8_fmt, int scale_dtype, void* stream);
int cek_gemv_fp8_qk_norm_rope_rs(const void* x, const void* w, const void* scale, void* y, const void* q_weight,
                                 const void* k_weight, const int64_t* positions, int64_t n_q, int64_t n_k,
                                 int64_t head_dim, float eps, float theta, int is_neox, int* counters, void* q_out,
                                 const float* row_ss, int64_t n_ss, float row_eps, int64_t M, int64_t N, int64_t K,
                                 int io_dtype, int fp8_fmt, int scale_dtype, void* stream);

/*
 * NEW: per-head RMSNorm (weight qw / kw of length head_dim, Gemma w+1) then
 * rotary embedding, in place on q [T, n_q * head_dim] and
 * k [T, n_k * head_dim] (row strides q_stride / k_stride elements, so both
 * may be views into one QKV buffer).  positions [T] int64 on the device.
 * is_neox != 0: rotate-half pairs (i, i + hd/2); else interleaved (2i, 2i+1).
 */
int cek_qk_norm_rope(void* q, void* k, const void* qw, const void* kw, const int64_t* positions,
                     int64_t T, int64_t n_q, int64_t n_k, int64_t head_dim,
                     int64_t q_stride, int64_t k_stride, float eps, float theta,
                     int is_neox, int io_dtype, void* stream);

/*
 * Measurement utility, no counterpart in the reference: reads `bytes` bytes
 * of buf (16-byte aligned, bytes % 16 == 0) once with 16-byte non-temporal
 * loads.  With sink != NULL it writes the XOR of each of its 1024
 * workgroups' 32-bit words into sink[0 .. 1023] (so the XOR of the sink
 * words is the XOR of the buffer's words); with sink == NULL it only reads
 * (the timed mode).  Its duration is the practical ceiling of one pass over
 * the same bytes, which the benchmark quotes the HBM-bound kernels against.
 */
int cek_hbm_read_probe(const void* buf, int64_t bytes, uint32_t* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CEK_H */
