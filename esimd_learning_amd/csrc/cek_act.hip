// cek_act.hip -- gelu_and_mul and per-head QK RMSNorm + rotary embedding, gfx950.
//
// Neither op exists in the reference package; both are the small
// HBM/latency-bound kernels of a decoder layer that sit between the fp8
// GEMVs.
//
// gelu_and_mul:  out[t, i] = gelu_tanh(x[t, i]) * x[t, d + i], fp32 math,
//   gelu_tanh(u) = 0.5 u (1 + tanh(sqrt(2/pi) (u + 0.044715 u^3))).
//   Grid: (row chunks of 2048 outputs, T); each thread handles 8 outputs with
//   16-byte loads/stores.
//
// qk_norm_rope:  256-thread workgroups over (token, group of heads); with
//   many tokens a group is all of a token's heads, with few (decode) it is
//   four, one per wave, so the work still spreads over many workgroups.  The
//   cos/sin of the token's hd/2 rotary angles are computed in double
//   precision (angle = pos * base^(-2i/hd)) into LDS and shared by the
//   group's heads; each wave owns whole heads of q and k: RMS over the head
//   via a wave butterfly, weight multiply, rounding to the activation type,
//   rotation in fp32, and store in place.
#include "cek_common.h"

namespace cek {

template <typename T>
__global__ __launch_bounds__(256) void gelu_and_mul_kernel(
    uint16_t* __restrict__ out, const uint16_t* __restrict__ x, int d, int64_t xs, int64_t os, int vec) {
  const int t = blockIdx.y;
  const uint16_t* xr = x + (size_t)t * xs;
  uint16_t* orow = out + (size_t)t * os;
  if (vec) {
    const int i = (blockIdx.x * 256 + threadIdx.x) * 8;
    if (i >= d) return;
    u4 a = load_u4(xr + i), b = load_u4(xr + d + i), o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float g0 = f32_round(gelu_tanh(T::to_f32(a[e] & 0xFFFF)) * T::to_f32(b[e] & 0xFFFF));
      float g1 = f32_round(gelu_tanh(T::to_f32(a[e] >> 16)) * T::to_f32(b[e] >> 16));
      o[e] = (uint32_t)T::from_f32(g0) | ((uint32_t)T::from_f32(g1) << 16);
    }
    *reinterpret_cast<u4*>(orow + i) = o;
  } else {
    for (int i = (blockIdx.x * 256 + threadIdx.x) * 8, e = 0; e < 8; ++e, ++i)
      if (i < d) orow[i] = T::from_f32(f32_round(gelu_tanh(T::to_f32(xr[i])) * T::to_f32(xr[d + i])));
  }
}

// PPL = rotary pairs per lane = ceil(hd / 2 / 64), hd <= 512.
template <typename T, int PPL>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(
    uint16_t* __restrict__ q, uint16_t* __restrict__ k,
    const uint16_t* __restrict__ qw, const uint16_t* __restrict__ kw,
    const int64_t* __restrict__ positions, int nq, int nk, int hd,
    int64_t qs, int64_t ks, float eps, float theta, int neox, int heads_per_wg) {
  __shared__ float cs[256], sn[256];
  const int t = blockIdx.x;
  const int half = hd >> 1;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h0 = (int)blockIdx.y * heads_per_wg + wave;
  const int h_end = min(nq + nk, ((int)blockIdx.y + 1) * heads_per_wg);
  auto head = [&](int h) {
    return h < nq ? q + (size_t)t * qs + (size_t)h * hd : k + (size_t)t * ks + (size_t)(h - nq) * hd;
  };
  // This lane's pairs p = lane + 64 j of a head: element indices, raw values
  // and norm weights (0 past the head).
  int ia[PPL], ib[PPL];
  uint16_t ra[PPL], rb[PPL], wa[PPL], wb[PPL];
#pragma unroll
  for (int j = 0; j < PPL; ++j) {
    const int p = lane + 64 * j;
    ia[j] = neox ? p : 2 * p;
    ib[j] = neox ? p + half : 2 * p + 1;
  }
  auto load_head = [&](int h) {
    const uint16_t* v = head(h);
    const uint16_t* w = h < nq ? qw : kw;
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
      const bool in = lane + 64 * j < half;
      ra[j] = in ? v[ia[j]] : 0;
      rb[j] = in ? v[ib[j]] : 0;
      wa[j] = in ? w[ia[j]] : 0;
      wb[j] = in ? w[ib[j]] : 0;
    }
  };
  // The first head's loads are issued before the fp64 cos/sin table, so
  // their latency overlaps its arithmetic (the barrier below waits for both).
  if (h0 < h_end) load_head(h0);
  asm volatile("" ::: "memory");
  const double pos = (double)positions[t];
  const double lt = log2((double)theta);
  for (int i = threadIdx.x; i < half; i += 256) {
    const double inv_freq = exp2(-(double)(2 * i) / (double)hd * lt);
    double s, c;
    sincos(pos * inv_freq, &s, &c);
    cs[i] = (float)c;
    sn[i] = (float)s;
  }
  __syncthreads();

  for (int h = h0; h < h_end; h += 4) {
    if (h != h0) load_head(h);
    uint16_t* v = head(h);
    float a[PPL], b[PPL];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
      a[j] = T::to_f32(ra[j]);
      b[j] = T::to_f32(rb[j]);
      ss = fmaf(a[j], a[j], ss);
      ss = fmaf(b[j], b[j], ss);
    }
    ss = wave_sum(ss);
    const float inv = rsqrtf(ss / (float)hd + eps);
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
      const int p = lane + 64 * j;
      if (p >= half) continue;
      // norm, then round to the activation type before the rotation
      const float na = T::to_f32(T::from_f32(a[j] * inv * T::to_f32(wa[j])));
      const float nb = T::to_f32(T::from_f32(b[j] * inv * T::to_f32(wb[j])));
      const float c = cs[p], s = sn[p];
      v[ia[j]] = T::from_f32(na * c - nb * s);
      v[ib[j]] = T::from_f32(nb * c + na * s);
    }
  }
}

}  // namespace cek

using namespace cek;

extern "C" int cek_gelu_and_mul(void* out, const void* x, int64_t T, int64_t d,
                                int64_t x_stride, int64_t out_stride, int io_dtype, void* stream) {
  if (T < 0 || d <= 0 || T > 65535 || d > INT32_MAX / 2 || x_stride < 2 * d || out_stride < d) return CEK_ERR_INVALID;
  if (T == 0) return CEK_OK;
  if (!out || !x) return CEK_ERR_INVALID;
  hipStream_t st = (hipStream_t)stream;
  const int vec = d % 8 == 0 && x_stride % 8 == 0 && out_stride % 8 == 0 && aligned(x, 16) && aligned(out, 16);
  dim3 grid((unsigned)((d + 2047) / 2048), (unsigned)T);
  uint16_t* o = static_cast<uint16_t*>(out);
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  if (io_dtype == CEK_F16) gelu_and_mul_kernel<F16><<<grid, 256, 0, st>>>(o, xp, (int)d, x_stride, out_stride, vec);
  else if (io_dtype == CEK_BF16) gelu_and_mul_kernel<BF16><<<grid, 256, 0, st>>>(o, xp, (int)d, x_stride, out_stride, vec);
  else return CEK_ERR_INVALID;
  return check_launch();
}

extern "C" int cek_qk_norm_rope(void* q, void* k, const void* qw, const void* kw, const int64_t* positions,
                                int64_t T, int64_t n_q, int64_t n_k, int64_t head_dim,
                                int64_t q_stride, int64_t k_stride, float eps, float theta,
                                int is_neox, int io_dtype, void* stream) {
  if (T < 0 || n_q < 0 || n_k < 0 || head_dim <= 0 || head_dim % 2 || head_dim > 512) return CEK_ERR_INVALID;
  if (T > INT32_MAX || n_q + n_k > 65536) return CEK_ERR_INVALID;
  if (n_q > 0 && q_stride < n_q * head_dim) return CEK_ERR_INVALID;
  if (n_k > 0 && k_stride < n_k * head_dim) return CEK_ERR_INVALID;
  if (!(theta > 0.f)) return CEK_ERR_INVALID;
  if (T == 0 || n_q + n_k == 0) return CEK_OK;
  if (!positions || (n_q > 0 && (!q || !qw)) || (n_k > 0 && (!k || !kw))) return CEK_ERR_INVALID;
  hipStream_t st = (hipStream_t)stream;
  const int ppl = (int)((head_dim / 2 + 63) / 64);
  // Heads per workgroup (a multiple of the 4 waves): all of a token's heads
  // once there are enough tokens to fill the GPU; otherwise one head per wave,
  // so a decode step's few tokens still spread over many workgroups (each
  // rebuilds its token's cos/sin table).
  const int nh = (int)(n_q + n_k);
  const int hpw = T >= 64 ? (nh + 3) / 4 * 4 : 4;
  const dim3 grid((unsigned)T, (unsigned)((nh + hpw - 1) / hpw));
  uint16_t* qp = static_cast<uint16_t*>(q);
  uint16_t* kp = static_cast<uint16_t*>(k);
  const uint16_t* qwp = static_cast<const uint16_t*>(qw);
  const uint16_t* kwp = static_cast<const uint16_t*>(kw);
#define CEK_ROPE_LAUNCH(TY, P)                                                                              \
  qk_norm_rope_kernel<TY, P><<<grid, 256, 0, st>>>(qp, kp, qwp, kwp, positions, (int)n_q, (int)n_k, (int)head_dim, \
                                                   q_stride, k_stride, eps, theta, is_neox, hpw)
  if (io_dtype == CEK_F16) {
    if (ppl == 1) CEK_ROPE_LAUNCH(F16, 1);
    else if (ppl == 2) CEK_ROPE_LAUNCH(F16, 2);
    else CEK_ROPE_LAUNCH(F16, 4);
  } else if (io_dtype == CEK_BF16) {
    if (ppl == 1) CEK_ROPE_LAUNCH(BF16, 1);
    else if (ppl == 2) CEK_ROPE_LAUNCH(BF16, 2);
    else CEK_ROPE_LAUNCH(BF16, 4);
  } else {
    return CEK_ERR_INVALID;
  }
#undef CEK_ROPE_LAUNCH
  return check_launch();
}
