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
#include "cek_rowops.h"

namespace cek {

template <typename T>
__global__ __launch_bounds__(256) void gelu_and_mul_kernel(
    uint16_t* __restrict__ out, const uint16_t* __restrict__ x, int64_t T_rows, int d, int64_t xs, int64_t os,
    int vec) {
  const int i0 = (blockIdx.x * 256 + threadIdx.x) * 8;
  if (i0 >= d) return;
  // rows blockIdx.y, + gridDim.y, ... (the grid's y extent is capped at 65535)
  for (int64_t t = blockIdx.y; t < T_rows; t += gridDim.y) {
    const uint16_t* xr = x + t * xs;
    uint16_t* orow = out + t * os;
    if (vec) {
      u4 a = load_u4(xr + i0), b = load_u4(xr + d + i0), o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float g0 = f32_round(gelu_tanh(T::to_f32(a[e] & 0xFFFF)) * T::to_f32(b[e] & 0xFFFF));
        float g1 = f32_round(gelu_tanh(T::to_f32(a[e] >> 16)) * T::to_f32(b[e] >> 16));
        o[e] = (uint32_t)T::from_f32(g0) | ((uint32_t)T::from_f32(g1) << 16);
      }
      *reinterpret_cast<u4*>(orow + i0) = o;
    } else {
      for (int i = i0, e = 0; e < 8; ++e, ++i)
        if (i < d) orow[i] = T::from_f32(f32_round(gelu_tanh(T::to_f32(xr[i])) * T::to_f32(xr[d + i])));
    }
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

// 16-byte form for hd = 16 L (L = 2 .. 32, a power of two), 16-byte aligned
// rows and weights: L lanes own a head, lane c of them the 16-byte chunks c
// and c + L (elements 8 c .. 8 c + 7 and hd / 2 + 8 c ..).  NeoX pairs are
// then element e of the first chunk with element e of the second; GPT-J
// pairs sit inside each chunk.  A wave holds 64 / L heads at once; the head's
// sum of squares is an xor-butterfly over its L lanes.  Same arithmetic per
// element as qk_norm_rope_kernel (its order of the squares' sum aside).
template <typename T, int L>
__global__ __launch_bounds__(256) void qk_norm_rope_vec_kernel(
    uint16_t* __restrict__ q, uint16_t* __restrict__ k,
    const uint16_t* __restrict__ qw, const uint16_t* __restrict__ kw,
    const int64_t* __restrict__ positions, int nq, int nk,
    int64_t qs, int64_t ks, float eps, float theta, int neox, int heads_per_wg) {
  constexpr int HD = 16 * L, HALF = 8 * L, HPW = 64 / L;  // heads per wave and pass
  __shared__ float cs[HALF], sn[HALF];
  const int t = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane % L;
  const int hbase = (int)blockIdx.y * heads_per_wg;
  const int h_end = min(nq + nk, hbase + heads_per_wg);
  // the pass's head of this lane: its row pointer, two chunks and their weights
  u4 va = u4{0u, 0u, 0u, 0u}, vb = va, wa = va, wb = va;
  const int h_first = hbase + wave * HPW + lane / L;
  // the first pass's loads go out before the fp64 cos/sin table, so their
  // latency overlaps its arithmetic (the barrier below waits for both)
  if (h_first < h_end) {
    const uint16_t* v = h_first < nq ? q + (size_t)t * qs + (size_t)h_first * HD
                                     : k + (size_t)t * ks + (size_t)(h_first - nq) * HD;
    const uint16_t* w = h_first < nq ? qw : kw;
    va = load_u4(v + 8 * c);
    vb = load_u4(v + HALF + 8 * c);
    wa = load_u4(w + 8 * c);
    wb = load_u4(w + HALF + 8 * c);
  }
  asm volatile("" ::: "memory");
  const double pos = (double)positions[t];
  const double lt = log2((double)theta);
  for (int i = threadIdx.x; i < HALF; i += 256) rope_angle(pos, i, HD, lt, cs[i], sn[i]);
  __syncthreads();

  for (int h = h_first; h - lane / L - wave * HPW < h_end; h += 4 * HPW) {
    uint16_t* v = h < nq ? q + (size_t)t * qs + (size_t)h * HD : k + (size_t)t * ks + (size_t)(h - nq) * HD;
    if (h != h_first) {
      if (h < h_end) {
        const uint16_t* w = h < nq ? qw : kw;
        va = load_u4(v + 8 * c);
        vb = load_u4(v + HALF + 8 * c);
        wa = load_u4(w + 8 * c);
        wb = load_u4(w + HALF + 8 * c);
      } else {
        va = vb = wa = wb = u4{0u, 0u, 0u, 0u};
      }
    }
    u4 oa, ob;
    norm_rope_chunks<T, L>(va, vb, wa, wb, cs, sn, eps, neox != 0, c, oa, ob);
    if (h < h_end) {
      *reinterpret_cast<u4*>(v + 8 * c) = oa;
      *reinterpret_cast<u4*>(v + HALF + 8 * c) = ob;
    }
  }
}

}  // namespace cek

using namespace cek;

extern "C" int cek_gelu_and_mul(void* out, const void* x, int64_t T, int64_t d,
                                int64_t x_stride, int64_t out_stride, int io_dtype, void* stream) {
  if (T < 0 || d <= 0 || d > INT32_MAX / 2 || x_stride < 2 * d || out_stride < d) return CEK_ERR_INVALID;
  if (T == 0) return CEK_OK;
  if (!out || !x) return CEK_ERR_INVALID;
  hipStream_t st = (hipStream_t)stream;
  const int vec = d % 8 == 0 && x_stride % 8 == 0 && out_stride % 8 == 0 && aligned(x, 16) && aligned(out, 16);
  // one workgroup row per token up to the grid's y limit; beyond it each
  // workgroup row walks tokens with a stride of 65535
  dim3 grid((unsigned)((d + 2047) / 2048), (unsigned)(T < 65535 ? T : 65535));
  uint16_t* o = static_cast<uint16_t*>(out);
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  if (io_dtype == CEK_F16) gelu_and_mul_kernel<F16><<<grid, 256, 0, st>>>(o, xp, T, (int)d, x_stride, out_stride, vec);
  else if (io_dtype == CEK_BF16) gelu_and_mul_kernel<BF16><<<grid, 256, 0, st>>>(o, xp, T, (int)d, x_stride, out_stride, vec);
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
  const int nh = (int)(n_q + n_k);
  uint16_t* qp = static_cast<uint16_t*>(q);
  uint16_t* kp = static_cast<uint16_t*>(k);
  const uint16_t* qwp = static_cast<const uint16_t*>(qw);
  const uint16_t* kwp = static_cast<const uint16_t*>(kw);
  // 16-byte form: hd = 16 L with L a power of two from 2 to 32, 16-byte
  // aligned row starts (row strides in 8-element units) and weights.
  const int64_t lph = head_dim / 16;
  const bool vec = head_dim % 16 == 0 && lph >= 2 && lph <= 32 && (lph & (lph - 1)) == 0 &&
                   (n_q == 0 || (aligned(q, 16) && q_stride % 8 == 0 && aligned(qw, 16))) &&
                   (n_k == 0 || (aligned(k, 16) && k_stride % 8 == 0 && aligned(kw, 16)));
  if (vec) {
    // Heads per workgroup: a multiple of one pass (4 waves x 64 / L heads);
    // all of a token's heads once there are enough tokens to fill the GPU,
    // else one pass, so a decode step's few tokens spread over workgroups.
    const int pass = 4 * (int)(64 / lph);
    const int hpw = T >= 64 ? (nh + pass - 1) / pass * pass : pass;
    const dim3 grid((unsigned)T, (unsigned)((nh + hpw - 1) / hpw));
#define CEK_ROPE_VEC(TY, LL)                                                                                  \
  qk_norm_rope_vec_kernel<TY, LL><<<grid, 256, 0, st>>>(qp, kp, qwp, kwp, positions, (int)n_q, (int)n_k, q_stride, \
                                                        k_stride, eps, theta, is_neox, hpw)
#define CEK_ROPE_VEC_ALL(TY)                   \
  do {                                         \
    switch (lph) {                             \
      case 2: CEK_ROPE_VEC(TY, 2); break;      \
      case 4: CEK_ROPE_VEC(TY, 4); break;      \
      case 8: CEK_ROPE_VEC(TY, 8); break;      \
      case 16: CEK_ROPE_VEC(TY, 16); break;    \
      default: CEK_ROPE_VEC(TY, 32); break;    \
    }                                          \
  } while (0)
    if (io_dtype == CEK_F16) CEK_ROPE_VEC_ALL(F16);
    else if (io_dtype == CEK_BF16) CEK_ROPE_VEC_ALL(BF16);
    else return CEK_ERR_INVALID;
#undef CEK_ROPE_VEC_ALL
#undef CEK_ROPE_VEC
    return check_launch();
  }
  const int ppl = (int)((head_dim / 2 + 63) / 64);
  // Heads per workgroup (a multiple of the 4 waves): all of a token's heads
  // once there are enough tokens to fill the GPU; otherwise one head per wave,
  // so a decode step's few tokens still spread over many workgroups (each
  // rebuilds its token's cos/sin table).
  const int hpw = T >= 64 ? (nh + 3) / 4 * 4 : 4;
  const dim3 grid((unsigned)T, (unsigned)((nh + hpw - 1) / hpw));
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
