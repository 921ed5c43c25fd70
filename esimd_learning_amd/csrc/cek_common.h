// cek_common.h -- device/host helpers shared by the gfx950 kernels.
//
// fp8 decode uses the gfx950 OCP conversion instructions
// (v_cvt_scalef32_pk_{f16,bf16}_{fp8,bf8}, v_cvt_pk_f32_fp8): exact OCP
// e4m3fn / e5m2 decoding, subnormals kept, NaN codes decode to NaN.  This is
// the decode of the reference's torch oracle (weight_fp8.to(torch.float16),
// tests/test_gemv_fp8.py:31), not the reference kernels' approximate decode
// (fp8_GEMV_v2.h:15-38 flushes subnormals and maps NaN to +-480).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "cek.h"

namespace cek {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef int i4 __attribute__((ext_vector_type(4)));
typedef int i8 __attribute__((ext_vector_type(8)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

// 16-bit activation element types, stored as raw bits.
struct F16 {
  static constexpr int code = CEK_F16;
  typedef h2 pair;
  __device__ static inline float to_f32(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
  __device__ static inline uint16_t from_f32(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
};
struct BF16 {
  static constexpr int code = CEK_BF16;
  typedef bf2 pair;
  __device__ static inline float to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
  // v_cvt_pk_bf16_f32 on gfx950: round to nearest even, NaN stays NaN.
  __device__ static inline uint16_t from_f32(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
};

// An fp32 value as a register value: the empty asm keeps the compiler from
// folding the multiply that produced v into the 16-bit conversion that
// follows (a mixed-precision fma, v_fma_mix*, that rounds the exact product
// straight to 16 bits).  Whether it folds differs between call sites, so
// kernels that must agree bit for bit (a fused kernel and the ops it fuses)
// round every stored product through here: to fp32, then to the 16-bit type,
// as the source and the torch oracle do.
__device__ inline float f32_round(float v) {
  asm volatile("" : "+v"(v));
  return v;
}

// gelu with the tanh approximation, fp32 math:
// gelu_tanh(u) = 0.5 u (1 + tanh(sqrt(2/pi) (u + 0.044715 u^3))).  One
// definition for gelu_and_mul and the GEMV epilogue that fuses it, each
// operation rounded to fp32 (no contraction into fma), so every call site
// computes the same value.
__device__ inline float gelu_tanh(float u) {
#pragma clang fp contract(off)
  const float k0 = 0.7978845608028654f;  // sqrt(2/pi)
  const float k1 = 0.044715f;
  return 0.5f * u * (1.0f + tanhf(k0 * (u + k1 * u * u * u)));
}

// Decode the two fp8 bytes in the low (HI=false) or high (HI=true) half of
// `w` into a pair of the activation type; FMT is CEK_E4M3 or CEK_E5M2.
template <typename T, int FMT, bool HI>
__device__ inline typename T::pair fp8x2_to_pair(uint32_t w);

template <> __device__ inline h2 fp8x2_to_pair<F16, CEK_E4M3, false>(uint32_t w) { return __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false); }
template <> __device__ inline h2 fp8x2_to_pair<F16, CEK_E4M3, true>(uint32_t w) { return __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true); }
template <> __device__ inline h2 fp8x2_to_pair<F16, CEK_E5M2, false>(uint32_t w) { return __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(w, 1.0f, false); }
template <> __device__ inline h2 fp8x2_to_pair<F16, CEK_E5M2, true>(uint32_t w) { return __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(w, 1.0f, true); }
template <> __device__ inline bf2 fp8x2_to_pair<BF16, CEK_E4M3, false>(uint32_t w) { return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false); }
template <> __device__ inline bf2 fp8x2_to_pair<BF16, CEK_E4M3, true>(uint32_t w) { return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true); }
template <> __device__ inline bf2 fp8x2_to_pair<BF16, CEK_E5M2, false>(uint32_t w) { return __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, 1.0f, false); }
template <> __device__ inline bf2 fp8x2_to_pair<BF16, CEK_E5M2, true>(uint32_t w) { return __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, 1.0f, true); }

// acc + a.x*b.x + a.y*b.y with fp32 accumulation (v_dot2_f32_{f16,bf16}).
__device__ inline float dot2(h2 a, h2 b, float acc) { return __builtin_amdgcn_fdot2(a, b, acc, false); }
__device__ inline float dot2(bf2 a, bf2 b, float acc) { return __builtin_amdgcn_fdot2_f32_bf16(a, b, acc, false); }

// C += A * B^T on one 16 x 16 x 32 MFMA block, 16-bit operands (8 per lane).
template <typename T>
__device__ inline f4 mfma16x16x32(u4 a, u4 b, f4 c);
template <>
__device__ inline f4 mfma16x16x32<F16>(u4 a, u4 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, a), __builtin_bit_cast(h8, b), c, 0, 0, 0);
}
template <>
__device__ inline f4 mfma16x16x32<BF16>(u4 a, u4 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf8, a), __builtin_bit_cast(bf8, b), c, 0, 0, 0);
}

// C += A * B^T on one 16 x 16 x 128 fp8 MFMA block (32 OCP e4m3 bytes per
// lane; cbsz = blgp = 0 select e4m3 for both operands; block scales unused).
__device__ inline f4 mfma_fp8_16x16x128(const i8& a, const i8& b, f4 c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// s_waitcnt vmcnt(N): this wave's vector-memory loads, all but the N most
// recent, are complete (for direct-to-LDS loads: their data is in LDS).
template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier without the vmcnt(0) that a fenced __syncthreads adds
// (which would drain loads still meant to be in flight).  The "memory"
// clobber keeps the compiler from moving memory accesses across it.
__device__ inline void bare_barrier() { asm volatile("s_barrier" ::: "memory"); }

__device__ inline i8 cat_i8(u4 lo, u4 hi) {
  return i8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}

// Decode 16 fp8 bytes into two u4 of activation-typed values (k-slots 0-7, 8-15).
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

// Exact decode of one fp8 byte to fp32 (used by the generic paths).
template <int FMT>
__device__ inline float fp8_to_f32(uint32_t byte) {
  if (FMT == CEK_E4M3) {
    f2 v = __builtin_amdgcn_cvt_pk_f32_fp8(byte, false);
    return v.x;
  } else {
    f2 v = __builtin_amdgcn_cvt_pk_f32_bf8(byte, false);
    return v.x;
  }
}

// fp32 -> e4m3fn byte, round to nearest even.  The input must already be
// clamped to [-448, 448] (v_cvt_pk_fp8_f32 does not saturate otherwise).
__device__ inline uint32_t f32_to_e4m3(float v) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v, 0.0f, 0, false) & 0xFFu;
}
__device__ inline uint32_t f32x4_to_e4m3x4(float a, float b, float c, float d) {
  int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
}

// Per-token e4m3 quantisation: scale = max(amax / 448, 1 / (448 * 512)),
// code = e4m3_rne(clamp(v / scale, -448, 448)).  Shared by the norm kernels
// and the GEMV whose prologue fuses the norm.
constexpr float E4M3_MAX = 448.0f;
constexpr float MIN_SCALE = 1.0f / (448.0f * 512.0f);
__device__ inline float quant_scale(float amax) { return fmaxf(amax / E4M3_MAX, MIN_SCALE); }
__device__ inline float quant_clamp(float v, float s) {
  return fminf(fmaxf(v / s, -E4M3_MAX), E4M3_MAX);  // IEEE divide (no fast math)
}

// Butterfly sum over the 64 lanes of a wave; every lane gets the total.
__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
// 64-lane sum with DPP row permutes (xor 1, xor 2, half-mirror, mirror give
// each 16-lane row its total) plus four readlanes; the result is uniform.
// Cheaper than the ds_bpermute butterfly when a kernel reduces many values.
#define CEK_DPP_F32(v, ctrl) __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), ctrl, 0xF, 0xF, true))
__device__ inline float wave_sum_dpp(float v) {
  v += CEK_DPP_F32(v, 0xB1);   // quad_perm [1,0,3,2]
  v += CEK_DPP_F32(v, 0x4E);   // quad_perm [2,3,0,1]
  v += CEK_DPP_F32(v, 0x141);  // row_half_mirror
  v += CEK_DPP_F32(v, 0x140);  // row_mirror
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)) +
         __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16)) +
         __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32)) +
         __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
}
__device__ inline float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Weight scale kinds of the GEMV / GEMM kernels: per output channel (fp16,
// bf16 or fp32 [N]) or one fp32 value for the whole tensor.
enum ScaleKind { SK_F16 = 0, SK_BF16 = 1, SK_F32 = 2, SK_F32_SCALAR = 3 };

__device__ inline float load_scale(const void* s, int kind, int n) {
  switch (kind) {
    case SK_F16: return F16::to_f32(reinterpret_cast<const uint16_t*>(s)[n]);
    case SK_BF16: return BF16::to_f32(reinterpret_cast<const uint16_t*>(s)[n]);
    case SK_F32: return reinterpret_cast<const float*>(s)[n];
    default: return *reinterpret_cast<const float*>(s);
  }
}

// The same in two halves, for kernels that load the scale long before they
// use it: the load alone (raw bits, no conversion, so nothing waits for it
// until scale_value) and the conversion.
__device__ inline uint32_t load_scale_bits(const void* s, int kind, int n) {
  uint32_t b;
  if (kind == SK_F16 || kind == SK_BF16) b = reinterpret_cast<const uint16_t*>(s)[n];
  else if (kind == SK_F32) b = reinterpret_cast<const uint32_t*>(s)[n];
  else b = *reinterpret_cast<const uint32_t*>(s);
  return b;
}
__device__ inline float scale_value(uint32_t b, int kind) {
  if (kind == SK_F16) return F16::to_f32((uint16_t)b);
  if (kind == SK_BF16) return BF16::to_f32((uint16_t)b);
  return __uint_as_float(b);
}

__device__ inline u4 load_u4(const void* p) { return *reinterpret_cast<const u4*>(p); }
// Streaming (non-temporal) 16-byte load for data read exactly once.
__device__ inline u4 load_u4_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u4*>(p));
}

}  // namespace cek

// ---- host-side helpers ----------------------------------------------------
namespace cek {
int record_hip_error(hipError_t e);  // stores the message, returns CEK_ERR_HIP
inline int check_launch() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? CEK_OK : record_hip_error(e);
}
inline bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }
}  // namespace cek
