// cek_norm.hip -- fused residual-add + RMSNorm (+ per-token e4m3 quant), and
// standalone per-token e4m3 quantisation, gfx950.
//
// Reference algorithm (csrc/xpu/esimd_kernels/fused_add_rms_norm_batched.h):
//   pass 1 (:30-50)  r' = f16(h + r) stored; sum_sq over the unrounded fp32 sum
//   (:52-53)         inv = rsqrt(sum_sq / H + eps)
//   pass 2 (:55-62)  h  = f16(r' * inv * w)
// The reference runs one work-item per row; here one 256-thread workgroup
// owns a row: each thread keeps UPT 8-element units of the row in registers
// between the passes, so the row is read once and written once.
//
// The quantising variant rounds the normed row to the activation type, takes
// amax over those rounded values, and quantises them exactly as
// per_token_quant_kernel does, with the same launch shape and reduction
// order as the plain norm kernel.  The fused result is therefore bit-identical
// to the unfused pair (norm kernel, then quant kernel).
#include "cek_rowops.h"

namespace cek {

constexpr int NORM_THREADS = 256;

// Workgroup-wide sum / max for NORM_THREADS threads (4 waves).
__device__ inline float block_sum(float v, float* sh) { return wg4_sum(v, sh); }
__device__ inline float block_max(float v, float* sh) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) sh[wave] = v;
  __syncthreads();
  float t = fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]));
  __syncthreads();
  return t;
}


// Vector path: H % 8 == 0, 16-byte aligned rows, H <= 8 * NORM_THREADS * UPT.
template <typename T, int UPT, bool QUANT>
__global__ __launch_bounds__(NORM_THREADS) void add_rmsnorm_kernel(
    uint16_t* __restrict__ hidden, uint16_t* __restrict__ residual,
    const uint16_t* __restrict__ weight, int H, float eps,
    uint8_t* __restrict__ q, float* __restrict__ qscale) {
  __shared__ float sh[4];
  const int row = blockIdx.x;
  const int units = H >> 3;
  uint16_t* hr = hidden + (size_t)row * H;
  uint16_t* rr = residual + (size_t)row * H;

  u4 rv[UPT];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < UPT; ++j) {
    const int u = threadIdx.x + j * NORM_THREADS;
    if (u < units) {
      const u4 o = addnorm_pass1<T>(load_u4(hr + u * 8), load_u4(rr + u * 8), ss);
      rv[j] = o;
      *reinterpret_cast<u4*>(rr + u * 8) = o;
    }
  }
  ss = block_sum(ss, sh);
  const float inv = rsqrtf(ss / (float)H + eps);

  float amax = 0.f;
  u4 nv[UPT];
#pragma unroll
  for (int j = 0; j < UPT; ++j) {
    const int u = threadIdx.x + j * NORM_THREADS;
    if (u < units) {
      const u4 o = addnorm_pass2<T>(rv[j], load_u4(weight + u * 8), inv);
      if (QUANT) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          amax = fmaxf(amax, fmaxf(fabsf(T::to_f32(o[e] & 0xFFFF)), fabsf(T::to_f32(o[e] >> 16))));
        nv[j] = o;
      } else {
        *reinterpret_cast<u4*>(hr + u * 8) = o;
      }
    }
  }
  if (!QUANT) return;

  amax = block_max(amax, sh);
  const float s = quant_scale(amax);
  if (threadIdx.x == 0) qscale[row] = s;
  uint8_t* qr = q + (size_t)row * H;
#pragma unroll
  for (int j = 0; j < UPT; ++j) {
    const int u = threadIdx.x + j * NORM_THREADS;
    if (u < units) {
      uint32_t c[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const uint32_t a = nv[j][2 * e], b = nv[j][2 * e + 1];
        c[e] = f32x4_to_e4m3x4(quant_clamp(T::to_f32(a & 0xFFFF), s), quant_clamp(T::to_f32(a >> 16), s),
                               quant_clamp(T::to_f32(b & 0xFFFF), s), quant_clamp(T::to_f32(b >> 16), s));
      }
      *reinterpret_cast<uint2*>(qr + u * 8) = make_uint2(c[0], c[1]);
    }
  }
}

// Scalar path for any H / alignment: three passes over global memory.
template <typename T, bool QUANT>
__global__ __launch_bounds__(NORM_THREADS) void add_rmsnorm_generic_kernel(
    uint16_t* __restrict__ hidden, uint16_t* __restrict__ residual,
    const uint16_t* __restrict__ weight, int H, float eps,
    uint8_t* __restrict__ q, float* __restrict__ qscale) {
  __shared__ float sh[4];
  const int row = blockIdx.x;
  uint16_t* hr = hidden + (size_t)row * H;
  uint16_t* rr = residual + (size_t)row * H;
  float ss = 0.f;
  for (int i = threadIdx.x; i < H; i += NORM_THREADS) {
    float a = T::to_f32(hr[i]) + T::to_f32(rr[i]);
    ss = fmaf(a, a, ss);
    rr[i] = T::from_f32(a);  // re-read below by this same thread only
  }
  ss = block_sum(ss, sh);
  const float inv = rsqrtf(ss / (float)H + eps);
  float amax = 0.f;
  for (int i = threadIdx.x; i < H; i += NORM_THREADS) {
    uint16_t b = T::from_f32(f32_round(T::to_f32(rr[i]) * inv * T::to_f32(weight[i])));
    if (QUANT) amax = fmaxf(amax, fabsf(T::to_f32(b)));
    else hr[i] = b;
  }
  if (!QUANT) return;
  amax = block_max(amax, sh);
  const float s = quant_scale(amax);
  if (threadIdx.x == 0) qscale[row] = s;
  for (int i = threadIdx.x; i < H; i += NORM_THREADS) {
    uint16_t b = T::from_f32(f32_round(T::to_f32(rr[i]) * inv * T::to_f32(weight[i])));
    q[(size_t)row * H + i] = (uint8_t)f32_to_e4m3(quant_clamp(T::to_f32(b), s));
  }
}

// Per-token quantisation of a [rows, H] activation matrix.
template <typename T>
__global__ __launch_bounds__(NORM_THREADS) void per_token_quant_kernel(
    const uint16_t* __restrict__ x, int H, uint8_t* __restrict__ q, float* __restrict__ qscale, int vec) {
  __shared__ float sh[4];
  const int row = blockIdx.x;
  const uint16_t* xr = x + (size_t)row * H;
  uint8_t* qr = q + (size_t)row * H;
  float amax = 0.f;
  if (vec) {
    for (int u = threadIdx.x; u < (H >> 3); u += NORM_THREADS) {
      u4 v = load_u4(xr + u * 8);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        amax = fmaxf(amax, fmaxf(fabsf(T::to_f32(v[e] & 0xFFFF)), fabsf(T::to_f32(v[e] >> 16))));
    }
  } else {
    for (int i = threadIdx.x; i < H; i += NORM_THREADS) amax = fmaxf(amax, fabsf(T::to_f32(xr[i])));
  }
  amax = block_max(amax, sh);
  const float s = quant_scale(amax);
  if (threadIdx.x == 0) qscale[row] = s;
  if (vec) {
    for (int u = threadIdx.x; u < (H >> 3); u += NORM_THREADS) {
      u4 v = load_u4(xr + u * 8);
      uint32_t c[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const uint32_t a = v[2 * e], b = v[2 * e + 1];
        c[e] = f32x4_to_e4m3x4(quant_clamp(T::to_f32(a & 0xFFFF), s), quant_clamp(T::to_f32(a >> 16), s),
                               quant_clamp(T::to_f32(b & 0xFFFF), s), quant_clamp(T::to_f32(b >> 16), s));
      }
      *reinterpret_cast<uint2*>(qr + u * 8) = make_uint2(c[0], c[1]);
    }
  } else {
    for (int i = threadIdx.x; i < H; i += NORM_THREADS)
      qr[i] = (uint8_t)f32_to_e4m3(quant_clamp(T::to_f32(xr[i]), s));
  }
}

template <typename T, bool QUANT>
static int launch_norm_t(void* hidden, void* residual, const void* weight, int rows, int H, float eps,
                         uint8_t* q, float* qs, hipStream_t st) {
  uint16_t* h = static_cast<uint16_t*>(hidden);
  uint16_t* r = static_cast<uint16_t*>(residual);
  const uint16_t* w = static_cast<const uint16_t*>(weight);
  const int units = H / 8;
  const bool vec = H % 8 == 0 && aligned(hidden, 16) && aligned(residual, 16) && aligned(weight, 16) &&
                   (!QUANT || aligned(q, 8));
  const int upt = (units + NORM_THREADS - 1) / NORM_THREADS;
  dim3 grid(rows);
  if (vec && upt <= 1) add_rmsnorm_kernel<T, 1, QUANT><<<grid, NORM_THREADS, 0, st>>>(h, r, w, H, eps, q, qs);
  else if (vec && upt <= 2) add_rmsnorm_kernel<T, 2, QUANT><<<grid, NORM_THREADS, 0, st>>>(h, r, w, H, eps, q, qs);
  else if (vec && upt <= 3) add_rmsnorm_kernel<T, 3, QUANT><<<grid, NORM_THREADS, 0, st>>>(h, r, w, H, eps, q, qs);
  else if (vec && upt <= 4) add_rmsnorm_kernel<T, 4, QUANT><<<grid, NORM_THREADS, 0, st>>>(h, r, w, H, eps, q, qs);
  else if (vec && upt <= 8) add_rmsnorm_kernel<T, 8, QUANT><<<grid, NORM_THREADS, 0, st>>>(h, r, w, H, eps, q, qs);
  else add_rmsnorm_generic_kernel<T, QUANT><<<grid, NORM_THREADS, 0, st>>>(h, r, w, H, eps, q, qs);
  return check_launch();
}

}  // namespace cek

using namespace cek;

static int norm_args_ok(const void* h, const void* r, const void* w, int64_t rows, int64_t H) {
  if (rows < 0 || H <= 0 || rows > INT32_MAX || H > INT32_MAX / 2) return CEK_ERR_INVALID;
  if (rows > 0 && (!h || !r || !w)) return CEK_ERR_INVALID;
  return CEK_OK;
}

extern "C" int cek_fused_add_rms_norm(void* hidden, void* residual, const void* weight,
                                      int64_t rows, int64_t H, float eps, int io_dtype, void* stream) {
  int rc = norm_args_ok(hidden, residual, weight, rows, H);
  if (rc) return rc;
  if (rows == 0) return CEK_OK;
  hipStream_t st = (hipStream_t)stream;
  if (io_dtype == CEK_F16) return launch_norm_t<F16, false>(hidden, residual, weight, rows, H, eps, nullptr, nullptr, st);
  if (io_dtype == CEK_BF16) return launch_norm_t<BF16, false>(hidden, residual, weight, rows, H, eps, nullptr, nullptr, st);
  return CEK_ERR_INVALID;
}

extern "C" int cek_fused_add_rms_norm_quant_fp8(const void* hidden, void* residual, const void* weight,
                                                int64_t rows, int64_t H, float eps, int io_dtype,
                                                uint8_t* q, float* scale, void* stream) {
  int rc = norm_args_ok(hidden, residual, weight, rows, H);
  if (rc) return rc;
  if (rows == 0) return CEK_OK;
  if (!q || !scale) return CEK_ERR_INVALID;
  hipStream_t st = (hipStream_t)stream;
  // hidden is read-only in the quantising variant (the kernel never stores it).
  void* h = const_cast<void*>(hidden);
  if (io_dtype == CEK_F16) return launch_norm_t<F16, true>(h, residual, weight, rows, H, eps, q, scale, st);
  if (io_dtype == CEK_BF16) return launch_norm_t<BF16, true>(h, residual, weight, rows, H, eps, q, scale, st);
  return CEK_ERR_INVALID;
}

extern "C" int cek_per_token_quant_fp8(const void* x, int64_t rows, int64_t H, int io_dtype,
                                       uint8_t* q, float* scale, void* stream) {
  if (rows < 0 || H <= 0 || rows > INT32_MAX || H > INT32_MAX / 2) return CEK_ERR_INVALID;
  if (rows == 0) return CEK_OK;
  if (!x || !q || !scale) return CEK_ERR_INVALID;
  hipStream_t st = (hipStream_t)stream;
  const int vec = H % 8 == 0 && aligned(x, 16) && aligned(q, 8);
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  if (io_dtype == CEK_F16) per_token_quant_kernel<F16><<<dim3(rows), NORM_THREADS, 0, st>>>(xp, H, q, scale, vec);
  else if (io_dtype == CEK_BF16) per_token_quant_kernel<BF16><<<dim3(rows), NORM_THREADS, 0, st>>>(xp, H, q, scale, vec);
  else return CEK_ERR_INVALID;
  return check_launch();
}
