// cek_rowops.h -- per-row arithmetic shared by the standalone norm / RoPE
// kernels and the GEMV epilogues that fuse them, so that both compute the
// same values bit for bit.
//
//  * add+RMSNorm of one 8-element unit (the reference's algorithm,
//    csrc/xpu/esimd_kernels/fused_add_rms_norm_batched.h:30-62): pass 1
//    s = h + r in fp32, r' = Out(s), sum of squares over the unrounded s;
//    pass 2 h = Out(r' * inv * w).
//  * QK RMSNorm + rotary embedding of one head row held by L lanes as two
//    16-byte chunks per lane (lane c: elements 8 c .. and hd / 2 + 8 c ..).
#pragma once

#include "cek_common.h"

namespace cek {

// Pass 1 of one unit: returns r' packed, accumulates the squares of the
// unrounded sums into ss (fmaf, element order).
template <typename T>
__device__ inline u4 addnorm_pass1(u4 hv, u4 xv, float& ss) {
  u4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float a0 = T::to_f32(hv[e] & 0xFFFF) + T::to_f32(xv[e] & 0xFFFF);
    const float a1 = T::to_f32(hv[e] >> 16) + T::to_f32(xv[e] >> 16);
    ss = fmaf(a0, a0, ss);
    ss = fmaf(a1, a1, ss);
    o[e] = (uint32_t)T::from_f32(a0) | ((uint32_t)T::from_f32(a1) << 16);
  }
  return o;
}

// Pass 2 of one unit: Out(r' * inv * w), each product rounded to fp32 first.
template <typename T>
__device__ inline u4 addnorm_pass2(u4 rv, u4 wv, float inv) {
  u4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float n0 = f32_round(T::to_f32(rv[e] & 0xFFFF) * inv * T::to_f32(wv[e] & 0xFFFF));
    const float n1 = f32_round(T::to_f32(rv[e] >> 16) * inv * T::to_f32(wv[e] >> 16));
    o[e] = (uint32_t)T::from_f32(n0) | ((uint32_t)T::from_f32(n1) << 16);
  }
  return o;
}

// Sum over the 4 waves of a 256-thread workgroup: wave butterfly, then the
// four wave totals in wave order (sh: 4 floats of LDS).
__device__ inline float wg4_sum(float v, float* sh) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) sh[wave] = v;
  __syncthreads();
  const float t = sh[0] + sh[1] + sh[2] + sh[3];
  __syncthreads();
  return t;
}

// RMSNorm (weights wa / wb, Gemma w + 1) then the rotation of one head row:
// this lane's chunks va (elements 8 c ..) and vb (hd / 2 + 8 c ..) of a head
// of hd = 16 L, L lanes per head in aligned groups; cs / sn hold the row's
// cos / sin of the hd / 2 angles.  Every lane of the wave must call it (the
// head's sum of squares is an xor butterfly over its L lanes).
template <typename T, int L>
__device__ inline void norm_rope_chunks(u4 va, u4 vb, u4 wa, u4 wb, const float* cs, const float* sn, float eps,
                                        bool neox, int c, u4& oa, u4& ob) {
  constexpr int HD = 16 * L;
  float a[8], b[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    a[2 * e] = T::to_f32(va[e] & 0xFFFF);
    a[2 * e + 1] = T::to_f32(va[e] >> 16);
    b[2 * e] = T::to_f32(vb[e] & 0xFFFF);
    b[2 * e + 1] = T::to_f32(vb[e] >> 16);
  }
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    ss = fmaf(a[e], a[e], ss);
    ss = fmaf(b[e], b[e], ss);
  }
#pragma unroll
  for (int off = L / 2; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
  const float inv = rsqrtf(ss / (float)HD + eps);
  // norm, then round to the activation type before the rotation
  float na[8], nb[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    na[2 * e] = T::to_f32(T::from_f32(f32_round(a[2 * e] * inv * T::to_f32(wa[e] & 0xFFFF))));
    na[2 * e + 1] = T::to_f32(T::from_f32(f32_round(a[2 * e + 1] * inv * T::to_f32(wa[e] >> 16))));
    nb[2 * e] = T::to_f32(T::from_f32(f32_round(b[2 * e] * inv * T::to_f32(wb[e] & 0xFFFF))));
    nb[2 * e + 1] = T::to_f32(T::from_f32(f32_round(b[2 * e + 1] * inv * T::to_f32(wb[e] >> 16))));
  }
  if (neox) {
    // pair p = 8 c + e: (na[e], nb[e])
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int p0 = 8 * c + 2 * e, p1 = p0 + 1;
      const float x0 = na[2 * e] * cs[p0] - nb[2 * e] * sn[p0];
      const float x1 = na[2 * e + 1] * cs[p1] - nb[2 * e + 1] * sn[p1];
      const float y0 = nb[2 * e] * cs[p0] + na[2 * e] * sn[p0];
      const float y1 = nb[2 * e + 1] * cs[p1] + na[2 * e + 1] * sn[p1];
      oa[e] = (uint32_t)T::from_f32(x0) | ((uint32_t)T::from_f32(x1) << 16);
      ob[e] = (uint32_t)T::from_f32(y0) | ((uint32_t)T::from_f32(y1) << 16);
    }
  } else {
    // pairs inside each chunk: chunk c holds pairs 4 c + e, chunk c + L pairs 4 (c + L) + e
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int pa = 4 * c + e, pb = 4 * (c + L) + e;
      const float xa = na[2 * e] * cs[pa] - na[2 * e + 1] * sn[pa];
      const float ya = na[2 * e + 1] * cs[pa] + na[2 * e] * sn[pa];
      const float xb = nb[2 * e] * cs[pb] - nb[2 * e + 1] * sn[pb];
      const float yb = nb[2 * e + 1] * cs[pb] + nb[2 * e] * sn[pb];
      oa[e] = (uint32_t)T::from_f32(xa) | ((uint32_t)T::from_f32(ya) << 16);
      ob[e] = (uint32_t)T::from_f32(xb) | ((uint32_t)T::from_f32(yb) << 16);
    }
  }
}

// cos / sin of the rotary angles pos * base^(-2 i / hd), i < hd / 2, in
// double precision, rounded to fp32 (each call site the same expression).
__device__ inline void rope_angle(double pos, int i, int hd, double log2_theta, float& c, float& s) {
  const double inv_freq = exp2(-(double)(2 * i) / (double)hd * log2_theta);
  double sd, cd;
  sincos(pos * inv_freq, &sd, &cd);
  c = (float)cd;
  s = (float)sd;
}

}  // namespace cek
