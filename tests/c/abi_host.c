/*
 * A plain C99 host of the C ABI in include/cek.h, compiled and run by
 * tests/test_cabi.py (CPU only: every call below returns before any HIP
 * call).  It shows the header is usable from C and that argument checks and
 * status strings behave as documented.
 */
#include <stdio.h>
#include <string.h>

#include "cek.h"

static int fails = 0;

static void expect(int got, int want, const char* what) {
  if (got != want) {
    printf("FAIL %s: got %d (%s), want %d\n", what, got, cek_error_string(got), want);
    ++fails;
  }
}

int main(void) {
  void* p = (void*)(uintptr_t)256; /* never dereferenced: validation fails first */
  const void* ws[2] = {p, p};
  const void* ss[2] = {p, p};
  void* ys[2] = {p, p};
  int64_t ns[2] = {8, 8};

  expect(cek_version() / 10000, 0, "major version");
  expect(strcmp(cek_error_string(CEK_OK), cek_error_string(CEK_ERR_INVALID)) != 0, 1, "distinct status strings");
  expect(cek_gemv_fp8_pern(p, p, p, p, -1, 8, 64, CEK_F16, CEK_E4M3, CEK_F32, NULL), CEK_ERR_INVALID, "gemv M < 0");
  expect(cek_gemv_fp8_pern(NULL, NULL, NULL, NULL, 0, 8, 64, CEK_F16, CEK_E4M3, CEK_F32, NULL), CEK_OK, "gemv M = 0");
  expect(cek_gemv_fp8_pert(p, p, NULL, p, 1, 8, 0, CEK_BF16, CEK_E5M2, NULL), CEK_ERR_INVALID, "gemv K = 0");
  expect(cek_gemv_fp8_pern_multi(p, 0, ws, ss, ys, ns, 1, 64, CEK_F16, CEK_E4M3, CEK_F32, NULL), CEK_ERR_INVALID,
         "multi count 0");
  expect(cek_gemm_fp8_pert(p, p, NULL, p, 4, 8, 64, CEK_F16, 7, NULL), CEK_ERR_INVALID, "gemm fp8 format");
  expect(cek_gemm_fp8_a8w8(p, NULL, p, NULL, p, 4, 4, 40, CEK_F16, NULL), CEK_ERR_INVALID, "a8w8 K % 16");
  expect(cek_fused_add_rms_norm(p, p, p, 4, 0, 1e-6f, CEK_F16, NULL), CEK_ERR_INVALID, "norm H = 0");
  expect(cek_per_token_quant_fp8(p, -1, 64, CEK_F16, p, NULL, NULL), CEK_ERR_INVALID, "quant rows < 0");
  expect(cek_gelu_and_mul(p, p, 4, 64, 100, 64, CEK_F16, NULL), CEK_ERR_INVALID, "gelu x stride");
  expect(cek_qk_norm_rope(p, p, p, p, NULL, 4, 2, 2, 1024, 2048, 2048, 1e-6f, 1e4f, 1, CEK_F16, NULL),
         CEK_ERR_INVALID, "rope head_dim");
  expect((int)cek_gemv_fp8_add_rms_norm_defer_groups(3072), 256, "defer groups N = 3072 (12-column runs)");
  expect((int)cek_gemv_fp8_add_rms_norm_defer_groups(4096), 256, "defer groups N = 4096 (16-column runs)");
  expect((int)cek_gemv_fp8_add_rms_norm_defer_groups(100), 0, "defer groups N % 16");
  expect(cek_defer_norm_shift(1.36f), 1, "defer shift max|w| 1.36");
  expect(cek_defer_norm_shift(8.0f), 3, "defer shift max|w| 8");
  expect(cek_gemv_fp8_add_rms_norm_defer(p, p, p, p, p, p, NULL, 25, 4, 3072, 4096, CEK_F16, CEK_E4M3, CEK_F32, NULL),
         CEK_ERR_INVALID, "defer shift out of range");
  if (fails == 0) printf("ok\n");
  return fails != 0;
}
