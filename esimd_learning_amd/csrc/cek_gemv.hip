// cek_gemv.hip -- fp8-weight GEMV for decode (M <= 16 activation rows), gfx950.
//
// y[m, n] = Out((sum_k x[m, k] * dq(W[n, k])) * scale[n])   (scale after the
// reduction, as reference fp8_GEMV_v2.h:77 / :355 apply it).
//
// W is [N, K] row-major fp8 and is the only large operand: the kernels are
// HBM-bound and are built to stream W once with 16-byte loads per lane.
//
//  * gemv_dot_kernel (M <= 4): a 256-thread workgroup owns 2 output rows;
//    one load instruction of the workgroup reads 4 KB of contiguous weight
//    bytes of a row (thread t reads bytes [16 t, 16 t + 16) of the chunk),
//    which are decoded with v_cvt_scalef32_pk_{f16,bf16}_fp8 into
//    activation-typed pairs and accumulated with v_dot2_f32_{f16,bf16}
//    (fp32 accumulation).  The activation slice a thread needs is re-read
//    from L1/L2 (x is tiny).  DPP wave sums and an LDS combine end a row.
//  * gemv_mfma_kernel (4 < M <= 16): the 16 x 16 x 32 f16/bf16 MFMA does
//    the M x 16-row dot products; lane l streams row (l & 15) of a 16-row
//    tile at k-offset 16 * (l >> 4) of each 64-byte step, so a tile is read
//    as 16 rows x 64 contiguous bytes per load instruction.  The four waves
//    of a workgroup interleave over the K steps of the same tile (256
//    contiguous bytes per row per round) and reduce through LDS.
//  * gemv_generic_kernel: any K / alignment; byte loads.  Correctness path
//    for shapes the vector kernels do not take.
#include "cek_common.h"

namespace cek {

enum ScaleKind { SK_F16 = 0, SK_BF16 = 1, SK_F32 = 2, SK_F32_SCALAR = 3 };

__device__ inline float load_scale(const void* s, int kind, int n) {
  switch (kind) {
    case SK_F16: return F16::to_f32(reinterpret_cast<const uint16_t*>(s)[n]);
    case SK_BF16: return BF16::to_f32(reinterpret_cast<const uint16_t*>(s)[n]);
    case SK_F32: return reinterpret_cast<const float*>(s)[n];
    default: return *reinterpret_cast<const float*>(s);
  }
}

// ---------------------------------------------------------------------------
// M <= MT (MT in {1, 2, 4}): v_dot2 path.  A 256-thread workgroup owns R
// consecutive output rows; thread t handles the 16-byte weight units
// t, t + 256, ... of every one of them, U units per round, so one load
// instruction of the workgroup covers 4 KB of a row and the R rows x U units
// are in flight together.  Per-wave DPP sums, then an LDS combine of the four
// waves.  Small workgroups dispatched in order keep the rows being read in
// a sliding window of HBM, which streams better than long-lived persistent
// waves each walking its own region.
// ---------------------------------------------------------------------------
template <typename T, int FMT, int MT, int R, int U>
__global__ __launch_bounds__(256) void gemv_dot_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ w,
    const void* __restrict__ scale, int skind, uint16_t* __restrict__ y,
    int M, int N, int K) {
  typedef typename T::pair P;
  __shared__ float red[4][MT * R];
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int row0 = blockIdx.x * R;
  const int K16 = K >> 4;

  const uint8_t* wrow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = row0 + r < N ? row0 + r : N - 1;  // clamped rows are never stored
    wrow[r] = w + (size_t)row * K;
  }
  float acc[MT][R];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = 0.f;

  for (int base = t; base < K16; base += 256 * U) {
    u4 wv[U][R];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int idx = base + u * 256;
#pragma unroll
      for (int r = 0; r < R; ++r)
        wv[u][r] = idx < K16 ? load_u4_stream(wrow[r] + (size_t)idx * 16) : u4{0, 0, 0, 0};
    }
    // All activation loads of the round are issued before any arithmetic
    // (rows m >= M read row M - 1 and are never stored), so their L2 round
    // trips overlap each other and the weight loads.  Pairs are read through
    // a pair-typed pointer: bit-casting elements of a loaded u4 instead is
    // mis-lowered by this hipcc (every element reads element 0).
    P xv[U][MT][8];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int idx = min(base + u * 256, K16 - 1);
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const P* xp = reinterpret_cast<const P*>(x + (size_t)min(m, M - 1) * K + (size_t)idx * 16);
#pragma unroll
        for (int j = 0; j < 8; ++j) xv[u][m][j] = xp[j];
      }
    }
    // Keep the scheduler from sinking the loads into the arithmetic below (it
    // otherwise serialises them through one register quad).
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (base + u * 256 >= K16) break;
      P wp[R][8];
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          wp[r][2 * j] = fp8x2_to_pair<T, FMT, false>(wv[u][r][j]);
          wp[r][2 * j + 1] = fp8x2_to_pair<T, FMT, true>(wv[u][r][j]);
        }
#pragma unroll
      for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[m][r] = dot2(xv[u][m][j], wp[r][j], acc[m][r]);
    }
  }

#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float s = wave_sum_dpp(acc[m][r]);
      if (lane == 0) red[wave][m * R + r] = s;
    }
  __syncthreads();
  if (t < MT * R) {
    const int m = t / R, r = t % R, n = row0 + r;
    if (m < M && n < N) {
      const float s = red[0][t] + red[1][t] + red[2][t] + red[3][t];
      y[(size_t)m * N + n] = T::from_f32(s * load_scale(scale, skind, n));
    }
  }
}

// ---------------------------------------------------------------------------
// 4 < M <= 16: MFMA 16x16x32 path.  Workgroup = 4 waves = one 16*NT-row
// tile; wave w takes the 64-byte K steps s with s % 4 == w.
// ---------------------------------------------------------------------------

template <typename T, int FMT, int NT, int UNROLL>
__global__ __launch_bounds__(256) void gemv_mfma_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ w,
    const void* __restrict__ scale, int skind, uint16_t* __restrict__ y,
    int M, int N, int K) {
  typedef typename T::pair P;
  __shared__ f4 red[3][NT][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * 16 * NT;
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int steps = K >> 6;  // 64-byte K steps (K % 64 == 0 on this path)

  const uint8_t* wrow[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    int row = n0 + t * 16 + r16;
    row = row < N ? row : N - 1;  // clamped rows are never stored
    wrow[t] = w + (size_t)row * K + g * 16;
  }
  const bool xrow_ok = r16 < M;
  const uint16_t* xrow = x + (size_t)(xrow_ok ? r16 : 0) * K + g * 16;

  f4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};

  for (int s0 = wave; s0 < steps; s0 += 4 * UNROLL) {
    u4 wv[UNROLL][NT];
    u4 xa[UNROLL], xb[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int s = s0 + 4 * u;
#pragma unroll
      for (int t = 0; t < NT; ++t)
        wv[u][t] = s < steps ? load_u4_stream(wrow[t] + (size_t)s * 64) : u4{0, 0, 0, 0};
      if (s < steps && xrow_ok) {
        const u4* xp = reinterpret_cast<const u4*>(xrow + (size_t)s * 64);
        xa[u] = xp[0];
        xb[u] = xp[1];
      } else {
        xa[u] = u4{0, 0, 0, 0};
        xb[u] = u4{0, 0, 0, 0};
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // all loads of the round before any arithmetic
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        u4 lo, hi;  // decoded weights for k-slots [0,8) and [8,16) of this lane
        P p0 = fp8x2_to_pair<T, FMT, false>(wv[u][t][0]);
        P p1 = fp8x2_to_pair<T, FMT, true>(wv[u][t][0]);
        P p2 = fp8x2_to_pair<T, FMT, false>(wv[u][t][1]);
        P p3 = fp8x2_to_pair<T, FMT, true>(wv[u][t][1]);
        P p4 = fp8x2_to_pair<T, FMT, false>(wv[u][t][2]);
        P p5 = fp8x2_to_pair<T, FMT, true>(wv[u][t][2]);
        P p6 = fp8x2_to_pair<T, FMT, false>(wv[u][t][3]);
        P p7 = fp8x2_to_pair<T, FMT, true>(wv[u][t][3]);
        lo = u4{__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1),
                __builtin_bit_cast(uint32_t, p2), __builtin_bit_cast(uint32_t, p3)};
        hi = u4{__builtin_bit_cast(uint32_t, p4), __builtin_bit_cast(uint32_t, p5),
                __builtin_bit_cast(uint32_t, p6), __builtin_bit_cast(uint32_t, p7)};
        // A = activations (row r16 = m), B = weights (column r16 = n).
        acc[t] = mfma16x16x32<T>(xa[u], lo, acc[t]);
        acc[t] = mfma16x16x32<T>(xb[u], hi, acc[t]);
      }
    }
  }

  if (wave > 0) {
#pragma unroll
    for (int t = 0; t < NT; ++t) red[wave - 1][t][lane] = acc[t];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    f4 c = acc[t] + red[0][t][lane] + red[1][t][lane] + red[2][t][lane];
    const int n = n0 + t * 16 + r16;  // D column = lane & 15
    if (n >= N) continue;
    const float sc = load_scale(scale, skind, n);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = g * 4 + v;  // D row = 4 * (lane >> 4) + v
      if (m < M) y[(size_t)m * N + n] = T::from_f32(c[v] * sc);
    }
  }
}

// ---------------------------------------------------------------------------
// Generic: any M, K, alignment.  One wave per output row.
// ---------------------------------------------------------------------------
template <typename T, int FMT>
__global__ __launch_bounds__(256) void gemv_generic_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ w,
    const void* __restrict__ scale, int skind, uint16_t* __restrict__ y,
    int M, int N, int K) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const uint8_t* wr = w + (size_t)n * K;
  const float sc = load_scale(scale, skind, n);
  for (int m = 0; m < M; ++m) {
    const uint16_t* xr = x + (size_t)m * K;
    float acc = 0.f;
    for (int k = lane; k < K; k += 64) acc += T::to_f32(xr[k]) * fp8_to_f32<FMT>(wr[k]);
    acc = wave_sum(acc);
    if (lane == 0) y[(size_t)m * N + n] = T::from_f32(acc * sc);
  }
}

// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------
template <typename T, int FMT>
static int launch_gemv_t(const void* x, const void* w, const void* scale, int skind, void* y,
                         int M, int N, int K, hipStream_t st) {
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const uint8_t* wp = static_cast<const uint8_t*>(w);
  uint16_t* yp = static_cast<uint16_t*>(y);
  const bool vec16 = (K % 16 == 0) && aligned(x, 16) && aligned(w, 16);
  if (vec16 && M <= 4) {
    // Rows per workgroup (measured on MI355X, one pass over > 2 GB of
    // rotating weights): 2 for M = 1 up to K = 4096, else 4, which amortises
    // each workgroup's re-read of the M activation rows over more weight
    // rows.  One 16-byte unit per thread and row per round.
    const int K16 = K / 16;
    const bool r2 = M == 1 && K16 <= 256;
#define CEK_DOT(MT, R) gemv_dot_kernel<T, FMT, MT, R, 1><<<dim3((N + R - 1) / R), 256, 0, st>>>(xp, wp, scale, skind, yp, M, N, K)
    if (M == 1) { if (r2) CEK_DOT(1, 2); else CEK_DOT(1, 4); }
    else if (M == 2) CEK_DOT(2, 4);
    else CEK_DOT(4, 4);
#undef CEK_DOT
  } else if (vec16 && K % 64 == 0 && M <= 16) {
    // 16-row tiles per wave (NT) and 64-byte K steps in flight per wave
    // (UNROLL), measured per shape class: wide N amortises the activation
    // reads over more tiles; narrow N needs more workgroups and deeper K.
#define CEK_MF(NT, UN) gemv_mfma_kernel<T, FMT, NT, UN><<<dim3((N + 16 * NT - 1) / (16 * NT)), 256, 0, st>>>(xp, wp, scale, skind, yp, M, N, K)
    if (N >= 16384) CEK_MF(4, 4);
    else if (N >= 8192) { if (M > 8) CEK_MF(4, 2); else if (K <= 3072) CEK_MF(1, 8); else CEK_MF(2, 8); }
    else if (K <= 4096) { if (N >= 6144) CEK_MF(2, 16); else CEK_MF(1, 16); }
    else CEK_MF(1, 4);
#undef CEK_MF
  } else {
    dim3 grid((N + 3) / 4);
    gemv_generic_kernel<T, FMT><<<grid, 256, 0, st>>>(xp, wp, scale, skind, yp, M, N, K);
  }
  return check_launch();
}

int launch_gemv(const void* x, const void* w, const void* scale, int skind, void* y,
                int64_t M, int64_t N, int64_t K, int io_dtype, int fp8_fmt, hipStream_t st) {
  if (M < 0 || N < 0 || K <= 0 || M > 16) return CEK_ERR_INVALID;
  if (N > INT32_MAX || K > INT32_MAX || (int64_t)N * K > ((int64_t)1 << 40)) return CEK_ERR_INVALID;
  if (M == 0 || N == 0) return CEK_OK;
  if (!x || !w || !scale || !y) return CEK_ERR_INVALID;
  if (io_dtype == CEK_F16 && fp8_fmt == CEK_E4M3) return launch_gemv_t<F16, CEK_E4M3>(x, w, scale, skind, y, M, N, K, st);
  if (io_dtype == CEK_F16 && fp8_fmt == CEK_E5M2) return launch_gemv_t<F16, CEK_E5M2>(x, w, scale, skind, y, M, N, K, st);
  if (io_dtype == CEK_BF16 && fp8_fmt == CEK_E4M3) return launch_gemv_t<BF16, CEK_E4M3>(x, w, scale, skind, y, M, N, K, st);
  if (io_dtype == CEK_BF16 && fp8_fmt == CEK_E5M2) return launch_gemv_t<BF16, CEK_E5M2>(x, w, scale, skind, y, M, N, K, st);
  return CEK_ERR_INVALID;
}

// Generic path for any M (used by the GEMM entry point for odd shapes).
int launch_gemv_generic(const void* x, const void* w, const void* scale, int skind, void* y,
                        int64_t M, int64_t N, int64_t K, int io_dtype, int fp8_fmt, hipStream_t st) {
  dim3 grid((unsigned)((N + 3) / 4));
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const uint8_t* wp = static_cast<const uint8_t*>(w);
  uint16_t* yp = static_cast<uint16_t*>(y);
  if (io_dtype == CEK_F16 && fp8_fmt == CEK_E4M3) gemv_generic_kernel<F16, CEK_E4M3><<<grid, 256, 0, st>>>(xp, wp, scale, skind, yp, M, N, K);
  else if (io_dtype == CEK_F16 && fp8_fmt == CEK_E5M2) gemv_generic_kernel<F16, CEK_E5M2><<<grid, 256, 0, st>>>(xp, wp, scale, skind, yp, M, N, K);
  else if (io_dtype == CEK_BF16 && fp8_fmt == CEK_E4M3) gemv_generic_kernel<BF16, CEK_E4M3><<<grid, 256, 0, st>>>(xp, wp, scale, skind, yp, M, N, K);
  else if (io_dtype == CEK_BF16 && fp8_fmt == CEK_E5M2) gemv_generic_kernel<BF16, CEK_E5M2><<<grid, 256, 0, st>>>(xp, wp, scale, skind, yp, M, N, K);
  else return CEK_ERR_INVALID;
  return check_launch();
}

}  // namespace cek

extern "C" int cek_gemv_fp8_pern(const void* x, const void* w, const void* scale, void* y,
                                 int64_t M, int64_t N, int64_t K,
                                 int io_dtype, int fp8_fmt, int scale_dtype, void* stream) {
  int skind;
  if (scale_dtype == CEK_F16) skind = cek::SK_F16;
  else if (scale_dtype == CEK_BF16) skind = cek::SK_BF16;
  else if (scale_dtype == CEK_F32) skind = cek::SK_F32;
  else return CEK_ERR_INVALID;
  return cek::launch_gemv(x, w, scale, skind, y, M, N, K, io_dtype, fp8_fmt, (hipStream_t)stream);
}

extern "C" int cek_gemv_fp8_pert(const void* x, const void* w, const float* scale, void* y,
                                 int64_t M, int64_t N, int64_t K,
                                 int io_dtype, int fp8_fmt, void* stream) {
  return cek::launch_gemv(x, w, scale, cek::SK_F32_SCALAR, y, M, N, K, io_dtype, fp8_fmt, (hipStream_t)stream);
}
