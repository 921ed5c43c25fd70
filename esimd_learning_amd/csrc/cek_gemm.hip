// cek_gemm.hip -- fp8 GEMMs for prefill, gfx950.
//
// * a8w8:  Y[m, n] = Out(sa[m] * sb[n] * sum_k dq(A[m, k]) * dq(B[n, k])) on the
//   gfx950 fp8 MFMA v_mfma_f32_16x16x128_f8f6f4 (OCP e4m3 operands, fp32
//   accumulation).  No reference op (the reference's prefill GEMM takes fp16
//   activations, below).
// * w8a16: Y[m, n] = Out((sum_k X[m, k] * dq(W[n, k])) * scale), the
//   reference's esimd_gemm_fp8_pert for M > 16 (reference dispatcher
//   csrc/xpu/esimd_kernels/fp8_GEMM_pert.h:4017-4062 sends M > 64 to a
//   weight-stationary SIMD kernel, :165-210).  Here: weights decoded to the
//   activation type in registers, then v_mfma_f32_16x16x32_{f16,bf16}.
//
// Both kernels compute C tiles as 16 x 16 MFMA blocks.  A and B operands are
// "K-major" ([rows, K] row-major), so lane l of a wave carries row (l & 15)
// of A and column (l & 15) of B^T; both carry the same K positions in the
// same register slots, so any K ordering the hardware uses inside an
// instruction cancels out.  The accumulator of a 16 x 16 block holds
// D[4 * (l >> 4) + v][l & 15] in element v of lane l.
#include "cek_common.h"

namespace cek {

int launch_gemv(const void* x, const void* w, const void* scale, int skind, void* y,
                int64_t M, int64_t N, int64_t K, int io_dtype, int fp8_fmt, hipStream_t st);
int launch_gemv_generic(const void* x, const void* w, const void* scale, int skind, void* y,
                        int64_t M, int64_t N, int64_t K, int io_dtype, int fp8_fmt, hipStream_t st);

__device__ inline f4 mfma_fp8_16x16x128(const i8& a, const i8& b, f4 c) {
  // cbsz = blgp = 0: both operands OCP e4m3; scale operands unused (0).
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// a8w8, direct-from-global v0: workgroup = 4 waves = 64 x 64 C tile, each wave
// a 32 x 32 quarter (2 x 2 MFMA blocks), K step 128.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void gemm_a8w8_simple_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ sa,
    const uint8_t* __restrict__ B, const float* __restrict__ sb,
    uint16_t* __restrict__ Y, int M, int N, int K) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m0 = blockIdx.y * 64 + (wave >> 1) * 32;
  const int n0 = blockIdx.x * 64 + (wave & 1) * 32;
  const int r16 = lane & 15, g = lane >> 4;
  const uint8_t* ap[2];
  const uint8_t* bp[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    int m = min(m0 + i * 16 + r16, M - 1);
    int n = min(n0 + i * 16 + r16, N - 1);
    ap[i] = A + (size_t)m * K + g * 32;
    bp[i] = B + (size_t)n * K + g * 32;
  }
  f4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  for (int kb = 0; kb < K; kb += 128) {
    const int k0 = kb + g * 32;  // this lane's 32 K positions: [k0, k0 + 32)
    i8 a[2], b[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      u4 a0 = k0 < K ? load_u4(ap[i] + kb) : u4{0, 0, 0, 0};
      u4 a1 = k0 + 16 < K ? load_u4(ap[i] + kb + 16) : u4{0, 0, 0, 0};
      u4 b0 = k0 < K ? load_u4(bp[i] + kb) : u4{0, 0, 0, 0};
      u4 b1 = k0 + 16 < K ? load_u4(bp[i] + kb + 16) : u4{0, 0, 0, 0};
      a[i] = i8{(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3], (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
      b[i] = i8{(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3], (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = mfma_fp8_16x16x128(a[i], b[j], acc[i][j]);
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + j * 16 + r16;
    if (n >= N) continue;
    const float sn = sb[n];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = m0 + i * 16 + g * 4 + v;
        if (m < M) Y[(size_t)m * N + n] = T::from_f32(acc[i][j][v] * sa[m] * sn);
      }
  }
}

// ---------------------------------------------------------------------------
// w8a16, direct-from-global v0: 64 x 64 C tile per workgroup, K step 64.
// ---------------------------------------------------------------------------

template <typename T, int FMT>
__device__ inline void decode16(u4 w, u4& lo, u4& hi) {
  typedef typename T::pair P;
  P p[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    p[2 * j] = fp8x2_to_pair<T, FMT, false>(w[j]);
    p[2 * j + 1] = fp8x2_to_pair<T, FMT, true>(w[j]);
  }
  lo = u4{__builtin_bit_cast(uint32_t, p[0]), __builtin_bit_cast(uint32_t, p[1]),
          __builtin_bit_cast(uint32_t, p[2]), __builtin_bit_cast(uint32_t, p[3])};
  hi = u4{__builtin_bit_cast(uint32_t, p[4]), __builtin_bit_cast(uint32_t, p[5]),
          __builtin_bit_cast(uint32_t, p[6]), __builtin_bit_cast(uint32_t, p[7])};
}

template <typename T, int FMT>
__global__ __launch_bounds__(256) void gemm_w8a16_simple_kernel(
    const uint16_t* __restrict__ X, const uint8_t* __restrict__ W, const float* __restrict__ scale,
    uint16_t* __restrict__ Y, int M, int N, int K) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m0 = blockIdx.y * 64 + (wave >> 1) * 32;
  const int n0 = blockIdx.x * 64 + (wave & 1) * 32;
  const int r16 = lane & 15, g = lane >> 4;
  const uint16_t* xp[2];
  const uint8_t* wp[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    int m = min(m0 + i * 16 + r16, M - 1);
    int n = min(n0 + i * 16 + r16, N - 1);
    xp[i] = X + (size_t)m * K + g * 16;
    wp[i] = W + (size_t)n * K + g * 16;
  }
  f4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
  for (int kb = 0; kb < K; kb += 64) {  // K % 64 == 0 on this path
    u4 xa[2], xb[2], wl[2], wh[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const u4* p = reinterpret_cast<const u4*>(xp[i] + kb);
      xa[i] = p[0];
      xb[i] = p[1];
      decode16<T, FMT>(load_u4(wp[i] + kb), wl[i], wh[i]);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        acc[i][j] = mfma16x16x32<T>(xa[i], wl[j], acc[i][j]);
        acc[i][j] = mfma16x16x32<T>(xb[i], wh[j], acc[i][j]);
      }
  }
  const float sc = *scale;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + j * 16 + r16;
    if (n >= N) continue;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = m0 + i * 16 + g * 4 + v;
        if (m < M) Y[(size_t)m * N + n] = T::from_f32(acc[i][j][v] * sc);
      }
  }
}

}  // namespace cek

using namespace cek;

extern "C" int cek_gemm_fp8_pert(const void* x, const void* w, const float* scale, void* y,
                                 int64_t M, int64_t N, int64_t K,
                                 int io_dtype, int fp8_fmt, void* stream) {
  if (M < 0 || N < 0 || K <= 0 || M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) return CEK_ERR_INVALID;
  if (M == 0 || N == 0) return CEK_OK;
  if (!x || !w || !scale || !y) return CEK_ERR_INVALID;
  if (io_dtype != CEK_F16 && io_dtype != CEK_BF16) return CEK_ERR_INVALID;
  if (fp8_fmt != CEK_E4M3 && fp8_fmt != CEK_E5M2) return CEK_ERR_INVALID;
  hipStream_t st = (hipStream_t)stream;
  if (M <= 16) return launch_gemv(x, w, scale, 3 /* f32 scalar */, y, M, N, K, io_dtype, fp8_fmt, st);
  if (K % 64 != 0 || !aligned(x, 16) || !aligned(w, 16) || M > 65535 * 64)
    return launch_gemv_generic(x, w, scale, 3, y, M, N, K, io_dtype, fp8_fmt, st);
  dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64));
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const uint8_t* wp = static_cast<const uint8_t*>(w);
  uint16_t* yp = static_cast<uint16_t*>(y);
  if (io_dtype == CEK_F16 && fp8_fmt == CEK_E4M3) gemm_w8a16_simple_kernel<F16, CEK_E4M3><<<grid, 256, 0, st>>>(xp, wp, scale, yp, M, N, K);
  else if (io_dtype == CEK_F16) gemm_w8a16_simple_kernel<F16, CEK_E5M2><<<grid, 256, 0, st>>>(xp, wp, scale, yp, M, N, K);
  else if (fp8_fmt == CEK_E4M3) gemm_w8a16_simple_kernel<BF16, CEK_E4M3><<<grid, 256, 0, st>>>(xp, wp, scale, yp, M, N, K);
  else gemm_w8a16_simple_kernel<BF16, CEK_E5M2><<<grid, 256, 0, st>>>(xp, wp, scale, yp, M, N, K);
  return check_launch();
}

extern "C" int cek_gemm_fp8_a8w8(const uint8_t* a, const float* sa, const uint8_t* b, const float* sb,
                                 void* y, int64_t M, int64_t N, int64_t K, int out_dtype, void* stream) {
  if (M < 0 || N < 0 || K <= 0 || K % 16 != 0) return CEK_ERR_INVALID;
  if (M > 65535 * 64 || N > INT32_MAX || K > INT32_MAX) return CEK_ERR_INVALID;
  if (M == 0 || N == 0) return CEK_OK;
  if (!a || !sa || !b || !sb || !y) return CEK_ERR_INVALID;
  if (!aligned(a, 16) || !aligned(b, 16)) return CEK_ERR_INVALID;
  hipStream_t st = (hipStream_t)stream;
  dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64));
  uint16_t* yp = static_cast<uint16_t*>(y);
  if (out_dtype == CEK_F16) gemm_a8w8_simple_kernel<F16><<<grid, 256, 0, st>>>(a, sa, b, sb, yp, M, N, K);
  else if (out_dtype == CEK_BF16) gemm_a8w8_simple_kernel<BF16><<<grid, 256, 0, st>>>(a, sa, b, sb, yp, M, N, K);
  else return CEK_ERR_INVALID;
  return check_launch();
}
