// cek_gemv.hip -- fp8-weight GEMV for decode (M <= 16 activation rows; up
// to 64 for the skinny GEMMs that reuse these kernels), gfx950.
//
// y[m, n] = Out((sum_k x[m, k] * dq(W[n, k])) * scale[n])   (scale after the
// reduction, as reference fp8_GEMV_v2.h:77 / :355 apply it).
//
// W is [N, K] row-major fp8 and is the only large operand: the kernels are
// HBM-bound and are built to stream W once with 16-byte loads per lane.
//
// Every launch covers a table of 1..8 weight matrices ("segments") that share
// the activations x -- one matrix for esimd_gemv_fp8_pern/pert, several for
// the fused variants (QKV or gate/up in one launch, what the reference's
// unregistered GEMV_fp8_pern_fused_kernel / GEMV_fp8_pert_fused_kernel do,
// fp8_GEMV_v2.h:197-316, 440-558).  The table is passed by value in the
// kernel arguments; workgroup b finds its segment from the table's prefix
// sums of workgroups per segment.
//
//  * gemv_dot_kernel (M <= 2, and M <= 4 where the LDS kernel has no
//    instantiation): a 256-thread workgroup owns R output rows; one load
//    instruction of the workgroup reads 4 KB of contiguous weight bytes of a
//    row (thread t reads bytes [16 t, 16 t + 16) of the chunk), which are
//    decoded with v_cvt_scalef32_pk_{f16,bf16}_fp8 into activation-typed
//    pairs and accumulated with v_dot2_f32_{f16,bf16} (fp32 accumulation).
//    The activation slice a thread needs is re-read from L1/L2 (x is tiny).
//    DPP wave sums and an LDS combine end a row.
//  * gemv_lds_kernel (3 <= M <= 64, K in {2, 3, 4, 5, 14, 24} x 1024): MFMA
//    on weights staged through LDS so that every load instruction still
//    reads 1 KB of one row (see the comment at the kernel).  Also the a8w8
//    path (e4m3 activations) for 3 <= M <= 64.
//  * gemv_mfma_kernel (4 < M <= 16, other K % 64 == 0): the 16 x 16 x 32
//    f16/bf16 MFMA does the M x 16-row dot products; lane l streams row
//    (l & 15) of a 16-row tile at k-offset 16 * (l >> 4) of each 64-byte
//    step.  The four waves of a workgroup interleave over the K steps of the
//    same tile and reduce through LDS.
//  * gemv_xres_kernel (9 <= M <= 16, 512 < N / 16 <= 2048, K <= 4096) and
//    gemv_xres8_kernel (e4m3 activations, 17 <= M <= 32): the activations
//    stay in LDS for the whole launch and the weights stream straight into
//    MFMA operand registers (see the comments at the kernels).
//  * gemv_generic_kernel: any K / alignment; byte loads.  Correctness path
//    for shapes the vector kernels do not take.
//
// Launch balance: a weight-streaming workgroup runs at the rate its loads in
// flight allow, so a launch lasts as long as its busiest CU's share.  The
// launchers pick rows per workgroup (tiles per workgroup or slot, 12- or
// 16-row tiles) to even that share out over the 256 CUs, among forms whose
// outputs agree bit for bit.
#include <climits>
#include <type_traits>

#include "cek_rowops.h"

namespace cek {

constexpr int kCUs = 256;  // MI355X compute units, for the launch-balance rules

int launch_w8a16(const void* x, const void* w, const void* scale, int skind, void* y, int64_t M, int64_t N, int64_t K,
                 int io_dtype, int fp8_fmt, float* ws, int64_t ws_bytes, hipStream_t st);  // cek_gemm.hip

constexpr int MAX_SEGS = 8;

// Weight matrices sharing one x; gstart[i] = first workgroup of segment i.
struct GemvSegs {
  const uint8_t* w[MAX_SEGS];
  const void* s[MAX_SEGS];
  uint16_t* y[MAX_SEGS];
  int n[MAX_SEGS];
  int gstart[MAX_SEGS + 1];
  int count;
  const float* xs;  // per-row activation scales [M] when x holds e4m3 codes
};

// Inputs and side outputs of the add+RMSNorm (+ e4m3 quant) that
// gemv_lds_kernel's NORM form computes in its prologue (unused otherwise).
// Epilogue work on the GEMV's output done by the workgroup that finishes
// last (TAIL != TAIL_NONE in gemv_lds_kernel); arrival counters zero before
// the launch, and left zero by it.
enum TailKind { TAIL_NONE = 0, TAIL_ROPE = 2 };
struct TailArgs {
  int* counters;          // ROPE: one per q / k head, TAIL_SLOT ints apart
  const uint16_t* qw;     // ROPE: q head RMSNorm weight [hd]
  const uint16_t* kw;     // ROPE: k head RMSNorm weight [hd]
  const int64_t* pos;     // ROPE: positions [M]
  int nq, nk;             // ROPE: heads q then k at output columns [0, (nq + nk) hd)
  float eps, theta;
  int neox;
  uint16_t* qcopy;        // ROPE: optional [M, nq hd] copy of the rotated q heads
};

struct NormArgs {
  const uint16_t* h;  // hidden [M, K]
  const uint16_t* r;  // residual [M, K] (read)
  const uint16_t* w;  // RMSNorm weight [K] (Gemma w+1 convention); EPI_ADDNORM: [N]
  uint16_t* r_out;    // h + r rounded [M, K], written by workgroup 0; EPI_ADDNORM: the residual [M, N], in place
  uint16_t* h_out;    // normed rows [M, K] (fp16/bf16 form; may be null), workgroup 0
  uint8_t* q_out;     // e4m3 codes [M, K] (quant form), workgroup 0
  float* s_out;       // per-row scales [M] (quant form), workgroup 0
  float eps;
  TailArgs tail;      // epilogue arguments (TAIL forms only)
  float* ss_out;      // EPI_ADDNORM(12): per-tile sums of squares [M][N / tile rows]
  const float* ss_in; // EPI_ROWSCALE: the producer's [M][nss] sums of squares
  int nss;
  float yscale = 1.f; // EPI_ADDNORM(12): 2^-shift, applied to y and (squared) to the sums
};

// Deferred RMSNorm between two GEMVs (EPI in gemv_lds_kernel).
// EPI_ADDNORM (the producer, e.g. o_proj): after the tile's sums, o =
// Out(sum * scale) as usual, then s = o + r (fp32), r = Out(s) in place,
// y = Out(f32(r) * w[n] * 2^-E) -- the norm's weight product without its
// 1 / rms -- and the tile's sum of (s * 2^-E)^2 per row to ss_out[m][tile]
// (E = the caller's shift, yscale = 2^-E: both products are exact in fp32,
// so only the final rounding differs from E = 0, and with 2^E >= max |w|
// no y can exceed |r| <= the largest finite value of Out; the consumer,
// given eps * 4^-E, then computes the same 1 / rms times 2^E).
// EPI_ADDNORM12: the same producer with 12-row tiles, for N whose 16-row
// tiles leave CUs idle (N = 3072: 256 workgroups instead of 192; each
// wave streams 3 rows, lanes 12-15 of the MFMA operand repeat row 11 and
// are dropped in the epilogue).
// EPI_ROWSCALE (the consumer, e.g. gate/up): x holds the producer's y; every
// workgroup's wave 0 sums the nss partials of each row in a fixed order
// (nss <= 256 and a multiple of 4, M <= 4), inv = rsqrt(sum / K + eps), and
// scales its outputs by inv[m].
enum EpiKind { EPI_NONE = 0, EPI_ADDNORM = 1, EPI_ROWSCALE = 2, EPI_ADDNORM12 = 3 };

struct SegRef {
  const uint8_t* w;
  const void* s;
  uint16_t* y;
  int n, group;
};

__device__ inline SegRef find_seg(const GemvSegs& sg, int b) {
  int i = 0;
#pragma unroll
  for (int j = 1; j < MAX_SEGS; ++j)
    if (j < sg.count && b >= sg.gstart[j]) i = j;
  return SegRef{sg.w[i], sg.s[i], sg.y[i], sg.n[i], b - sg.gstart[i]};
}

// ---------------------------------------------------------------------------
// M <= MT (MT in {1, 2, 4}): v_dot2 path.  A 256-thread workgroup owns R
// consecutive output rows of one segment; thread t handles the 16-byte weight
// units t, t + 256, ... of every one of them, U units per round, so one load
// instruction of the workgroup covers 4 KB of a row and the R rows x U units
// are in flight together.  Per-wave DPP sums, then an LDS combine of the four
// waves.  Small workgroups dispatched in order keep the rows being read in a
// sliding window of HBM, which streams better than long-lived persistent
// waves each walking its own region.
// RP > 1 (rows shorter than 4 KB: K = 4096 / RP, RP in {2, 4}): a load
// instruction covers RP consecutive rows of 256 / RP units each, thread t
// taking unit t % (256 / RP) of row t / (256 / RP) of each pass, so no thread
// idles; the workgroup owns R passes (R x RP rows).  A row's units, wave sums
// and the order they are added in are those of RP = 1 without the idle
// threads' zeros, so the outputs do not depend on RP or R.
// ---------------------------------------------------------------------------
// With XF8 the activations are e4m3 codes (x points at bytes) decoded exactly
// into T pairs, and the epilogue multiplies by the row's activation scale.
template <typename T, typename TO, int FMT, bool XF8, int MT, int R, int U, int RP = 1>
__global__ __launch_bounds__(256) void gemv_dot_kernel(const uint16_t* __restrict__ x, GemvSegs sg, int skind,
                                                       int M, int K) {
  static_assert(RP == 1 || RP == 2 || RP == 4, "a row covers whole waves");
  typedef typename T::pair P;
  __shared__ float red[4][MT * R];
  const SegRef sr = find_seg(sg, blockIdx.x);
  const int N = sr.n;
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int row0 = sr.group * R * RP;
  const int K16 = K >> 4;  // 256 / RP when RP > 1
  constexpr int TPR = 256 / RP;  // threads per row of a pass
  const int sub = t / TPR;       // this thread's row within each pass
  const int tu = t % TPR;        // and its first 16-byte unit
  // Output scales are loaded up front: their latency then overlaps the
  // weight loads' instead of following the reduction with the workgroup's
  // slot held and no weight bytes in flight.
  uint32_t sc_bits = 0;
  float sc_m = 1.f;
  if (t < MT * R * RP) {
    const int m = t / (R * RP), n = row0 + t % (R * RP);
    if (m < M && n < N) {
      sc_bits = load_scale_bits(sr.s, skind, n);
      if (XF8) sc_m = sg.xs[m];
    }
  }

  const uint8_t* wrow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = row0 + r * RP + sub < N ? row0 + r * RP + sub : N - 1;  // clamped rows are never stored
    wrow[r] = sr.w + (size_t)row * K;
  }
  float acc[MT][R];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = 0.f;

  for (int base = tu; base < K16; base += 256 * U) {
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
        if (XF8) {
          const u4 c = load_u4(reinterpret_cast<const uint8_t*>(x) + (size_t)min(m, M - 1) * K + (size_t)idx * 16);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            xv[u][m][2 * j] = fp8x2_to_pair<T, CEK_E4M3, false>(c[j]);
            xv[u][m][2 * j + 1] = fp8x2_to_pair<T, CEK_E4M3, true>(c[j]);
          }
        } else {
          const P* xp = reinterpret_cast<const P*>(x + (size_t)min(m, M - 1) * K + (size_t)idx * 16);
#pragma unroll
          for (int j = 0; j < 8; ++j) xv[u][m][j] = xp[j];
        }
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
  if (t < MT * R * RP) {
    // output (m, row row0 + q): pass r = q / RP, row sub = q % RP of it, whose
    // sums sit in waves 4 / RP * sub .. 4 / RP * (sub + 1) - 1
    const int m = t / (R * RP), q = t % (R * RP), n = row0 + q;
    if (m < M && n < N) {
      const int i = m * R + q / RP;
      float s;
      if (RP == 1) s = red[0][i] + red[1][i] + red[2][i] + red[3][i];
      else if (RP == 2) s = red[2 * (q % 2)][i] + red[2 * (q % 2) + 1][i];
      else s = red[q % 4][i];
      if (XF8) s *= sc_m;
      sr.y[(size_t)m * N + n] = TO::from_f32(s * scale_value(sc_bits, skind));
    }
  }
}

// ---------------------------------------------------------------------------
// 4 < M <= 16: MFMA 16x16x32 path.  Workgroup = 4 waves = one 16*NT-row
// tile of one segment; wave w takes the 64-byte K steps s with s % 4 == w.
// ---------------------------------------------------------------------------
template <typename T, typename TO, int FMT, bool XF8, int NT, int UNROLL>
__global__ __launch_bounds__(256) void gemv_mfma_kernel(const uint16_t* __restrict__ x, GemvSegs sg, int skind,
                                                        int M, int K) {
  typedef typename T::pair P;
  __shared__ f4 red[3][NT][64];
  const SegRef sr = find_seg(sg, blockIdx.x);
  const int N = sr.n;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n0 = sr.group * 16 * NT;
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int steps = K >> 6;  // 64-byte K steps (K % 64 == 0 on this path)

  const uint8_t* wrow[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    int row = n0 + t * 16 + r16;
    row = row < N ? row : N - 1;  // clamped rows are never stored
    wrow[t] = sr.w + (size_t)row * K + g * 16;
  }
  const bool xrow_ok = r16 < M;
  const uint16_t* xrow = x + (size_t)(xrow_ok ? r16 : 0) * K + g * 16;
  const uint8_t* xrow8 = reinterpret_cast<const uint8_t*>(x) + (size_t)(xrow_ok ? r16 : 0) * K + g * 16;
  // wave 0's output scales, loaded up front (their latency then overlaps the
  // weight loads')
  uint32_t sc_n[NT];
  float sc_m[4];
#pragma unroll
  for (int t = 0; t < NT; ++t) sc_n[t] = wave == 0 ? load_scale_bits(sr.s, skind, min(n0 + t * 16 + r16, N - 1)) : 0u;
#pragma unroll
  for (int v = 0; v < 4; ++v) sc_m[v] = (XF8 && wave == 0) ? sg.xs[min(g * 4 + v, M - 1)] : 1.f;

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
      if (s < steps && xrow_ok && XF8) {
        decode16<T, CEK_E4M3>(load_u4(xrow8 + (size_t)s * 64), xa[u], xb[u]);
      } else if (s < steps && xrow_ok) {
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
        decode16<T, FMT>(wv[u][t], lo, hi);
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
    const float sc = scale_value(sc_n[t], skind);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = g * 4 + v;  // D row = 4 * (lane >> 4) + v
      if (m < M) sr.y[(size_t)m * N + n] = TO::from_f32(c[v] * (XF8 ? sc * sc_m[v] : sc));
    }
  }
}

// ---------------------------------------------------------------------------
// 4 < M <= 64, K % 1024 == 0: LDS-staged MFMA path.
//
// HBM streams best when every load instruction of a wave reads 1 KB of ONE
// row (measured on MI355X: 6.4 TB/s, against 4.0-5.3 TB/s when an instruction
// gathers 64-512-byte pieces of 16 rows, which is what an MFMA operand needs).
// So the weights go through LDS: stage i holds bytes [1024 i, 1024 i + 1024)
// of the workgroup's 16*NT rows, each row fetched by one 1 KB load instruction
// into registers (16 bytes per lane), D stages ahead, and written to LDS
// (lane j's 16 bytes at row base + 16 j) just before the stage's barrier.
// Lane j fetches 16-byte unit j ^ (row & 15) instead of unit j -- the same
// 1 KB -- so unit v of row r sits at slot v ^ (r & 15), and the sixteen rows
// an MFMA fragment read touches fall in sixteen different bank groups.  Two
// LDS stages alternate; the loads of stage i + D are issued right after the
// barrier that publishes stage i and run under its arithmetic.
//
// The activations (a few hundred KB at most) are read from L2 straight into
// MFMA operand layout, before the next stage's weights so that waiting for
// them leaves those in flight.  Each wave takes a quarter of a stage's K
// units; the four partial sums meet in LDS at the end.
//
//  * gemv_lds_kernel: fp16/bf16 activations; a lane's 16-byte weight unit
//    (16 K values) is decoded to two 8-value operands of
//    v_mfma_f32_16x16x32_{f16,bf16}.
//  * gemv_lds_a8w8_kernel: e4m3 activation codes with per-row scales; two
//    units per lane feed one v_mfma_f32_16x16x128_f8f6f4 (no decode).
// ---------------------------------------------------------------------------
// Wave 0's output scales of the LDS-staged kernels: sc_n[t] (raw bits) for
// column n0 + SH t + (lane & 15) (SH = 16 or 12 rows per MFMA tile; lanes past
// SH repeat the tile's last row), sc_m[b][v] for row 16 b + 4 (lane >> 4) + v
// (xs: per-row activation scales, or null).  Loaded at the start of the
// kernel so that their latency overlaps the weight loads'.
template <int NT, int MB, int SH = 16>
__device__ inline void lds_load_scales(uint32_t (&sc_n)[NT], float (&sc_m)[MB][4], int wave, int lane, int n0, int N,
                                       int M, const SegRef& sr, int skind, const float* xs) {
  const int n16 = lane & 15, g = lane >> 4;
#pragma unroll
  for (int t = 0; t < NT; ++t)
    sc_n[t] = wave == 0 ? load_scale_bits(sr.s, skind, min(n0 + t * SH + min(n16, SH - 1), N - 1)) : 0u;
#pragma unroll
  for (int b = 0; b < MB; ++b)
#pragma unroll
    for (int v = 0; v < 4; ++v) sc_m[b][v] = (xs && wave == 0) ? xs[min(b * 16 + g * 4 + v, M - 1)] : 1.f;
}

// COH: the outputs are stored at device scope (global_store ... sc1: written
// through to the level every XCD sees), for a tail epilogue that another
// workgroup runs on them.  SH: rows per MFMA tile (16, or 12 with operand
// columns 12-15 repeating row 11, which are not stored).
template <int NT, int MB, bool COH = false, int SH = 16>
__device__ inline void lds_reduce_store(f4 (&acc)[NT][MB], uint8_t* smem, int wave, int lane, int n0, int N,
                                        int M, const SegRef& sr, int skind, const uint32_t (&sc_n)[NT],
                                        const float (&sc_m)[MB][4], bool xscaled, bool bf16_out) {
  f4* red = reinterpret_cast<f4*>(smem);  // [3][NT][MB][64]
  __syncthreads();                         // every wave is done with the stages
  if (wave > 0) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int b = 0; b < MB; ++b) red[(((wave - 1) * NT + t) * MB + b) * 64 + lane] = acc[t][b];
  }
  __syncthreads();
  if (wave != 0) return;
  const int n16 = lane & 15, g = lane >> 4;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int n = n0 + t * SH + n16;  // D column = lane & 15
    if (n >= N || n16 >= SH) continue;
    const float sc = scale_value(sc_n[t], skind);
#pragma unroll
    for (int b = 0; b < MB; ++b) {
      f4 c = acc[t][b];
#pragma unroll
      for (int w = 0; w < 3; ++w) c += red[((w * NT + t) * MB + b) * 64 + lane];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = b * 16 + g * 4 + v;  // D row = 4 * (lane >> 4) + v
        if (m >= M) continue;
        const float o = f32_round(c[v] * (xscaled ? sc * sc_m[b][v] : sc));
        const uint16_t ob = bf16_out ? BF16::from_f32(o) : F16::from_f32(o);
        if constexpr (COH) __hip_atomic_store(sr.y + (size_t)m * N + n, ob, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else sr.y[(size_t)m * N + n] = ob;
      }
    }
  }
}

// EPI_ADDNORM(12) epilogue of one tile of ROWS (16 or 12) rows (M <= 16):
// the cross-wave sum, o = Out(sum * scale), then the residual add, the norm
// weight product and the tile's per-row sum of squares (see EpiKind) to
// ss_out[m][n0 / ROWS] of N / ROWS per row; columns past ROWS (and N) add 0.
template <typename T, int ROWS>
__device__ inline void lds_reduce_addnorm(const f4& acc, uint8_t* smem, int wave, int lane, int n0, int N, int M,
                                          const SegRef& sr, int skind, uint32_t sc_bits, const NormArgs& na,
                                          const uint32_t (&pres)[4], uint32_t pnw) {
  f4* red = reinterpret_cast<f4*>(smem);  // [3][64]
  __syncthreads();                         // every wave is done with the stages
  if (wave > 0) red[(wave - 1) * 64 + lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  const int n16 = lane & 15, g = lane >> 4, n = n0 + n16;
  const bool col = n16 < ROWS && n < N;  // a column of this tile
  const float sc = scale_value(sc_bits, skind);
  uint32_t pw = pnw;
  asm volatile("" : "+v"(pw));  // the conversion stays here, after the loads are long in
  const float wn = T::to_f32((uint16_t)pw);
  const float ys = na.yscale, ys2 = ys * ys;  // powers of two: exact products
  f4 c = acc;
#pragma unroll
  for (int w = 0; w < 3; ++w) c += red[w * 64 + lane];
  float s2[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int m = g * 4 + v;
    const float o = T::to_f32(T::from_f32(f32_round(c[v] * sc)));
    const float sv = o + T::to_f32((uint16_t)pres[v]);
    const uint16_t rp = T::from_f32(sv);
    s2[v] = col ? f32_round(sv * sv) * ys2 : 0.f;  // rounded before the sums (no fma contraction)
    if (col && m < M) {
      na.r_out[(size_t)m * N + n] = rp;
      sr.y[(size_t)m * N + n] = T::from_f32(f32_round(f32_round(T::to_f32(rp) * wn) * ys));
    }
  }
  // each D row (one 16-lane DPP row): the tile's 16 lanes, pairwise
  // ((c0 + c1) + (c2 + c3)) + ... through xor 1, xor 2, half mirror, mirror
#pragma unroll
  for (int v = 0; v < 4; ++v) s2[v] += CEK_DPP_F32(s2[v], 0xB1);
#pragma unroll
  for (int v = 0; v < 4; ++v) s2[v] += CEK_DPP_F32(s2[v], 0x4E);
#pragma unroll
  for (int v = 0; v < 4; ++v) s2[v] += CEK_DPP_F32(s2[v], 0x141);
#pragma unroll
  for (int v = 0; v < 4; ++v) s2[v] += CEK_DPP_F32(s2[v], 0x140);
#pragma unroll
  for (int v = 0; v < 4; ++v)
    if (n16 == 0 && g * 4 + v < M) na.ss_out[(size_t)(g * 4 + v) * (N / ROWS) + n0 / ROWS] = s2[v];
}

// LDS writes of this wave done, then a workgroup barrier -- without the
// vmcnt(0) a fenced __syncthreads adds, which would drain the loads of the
// stages in flight.  The "memory" clobber keeps LDS accesses (and the
// activation loads, which are therefore not __restrict__) on their side.
__device__ inline void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// The cross-wave sum of one tile of a multi-tile workgroup, in a reduction
// area of its own (red, 3 x NT x MB x 64 f4), with LDS-only barriers so that
// the next tile's loads stay in flight, and no early return.  The leading
// barrier also orders this tile's reduction writes after wave 0's reads of
// the previous tile's.  Wave 0 then calls emit(t, b, v, o) for every element
// of its fragments: o = the scaled sum of D row 16 b + 4 (lane >> 4) + v,
// column 16 t + (lane & 15) of the tile (rows and columns not yet bounded).
template <int NT, int MB, typename Emit>
__device__ inline void lds_reduce_tile(const f4 (&acc)[NT][MB], uint8_t* redp, int wave, int lane, int skind,
                                       const uint32_t (&sc_n)[NT], const float (&sc_m)[MB][4], bool xscaled,
                                       Emit&& emit) {
  f4* red = reinterpret_cast<f4*>(redp);  // [3][NT][MB][64]
  lds_barrier();
  if (wave > 0) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int b = 0; b < MB; ++b) red[(((wave - 1) * NT + t) * MB + b) * 64 + lane] = acc[t][b];
  }
  lds_barrier();
  if (wave == 0) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const float sc = scale_value(sc_n[t], skind);
#pragma unroll
      for (int b = 0; b < MB; ++b) {
        f4 c = acc[t][b];
#pragma unroll
        for (int w = 0; w < 3; ++w) c += red[((w * NT + t) * MB + b) * 64 + lane];
#pragma unroll
        for (int v = 0; v < 4; ++v) emit(t, b, v, f32_round(c[v] * (xscaled ? sc * sc_m[b][v] : sc)));
      }
    }
  }
}

// lds_reduce_store for one tile of a multi-tile workgroup (n0 = the tile's
// first row).
template <int NT, int MB, int SH = 16>
__device__ inline void lds_reduce_store_tile(const f4 (&acc)[NT][MB], uint8_t* redp, int wave, int lane, int n0, int N,
                                             int M, const SegRef& sr, int skind, const uint32_t (&sc_n)[NT],
                                             const float (&sc_m)[MB][4], bool xscaled, bool bf16_out) {
  const int n16 = lane & 15, g = lane >> 4;
  lds_reduce_tile<NT, MB>(acc, redp, wave, lane, skind, sc_n, sc_m, xscaled, [&](int t, int b, int v, float o) {
    const int n = n0 + t * SH + n16, m = b * 16 + g * 4 + v;  // D column = lane & 15, row = 4 (lane >> 4) + v
    if (n < N && n16 < SH && m < M) sr.y[(size_t)m * N + n] = bf16_out ? BF16::from_f32(o) : F16::from_f32(o);
  });
}

// Tail epilogue of gemv_lds_kernel (one 16-row tile per workgroup, one
// segment, y [M, N] with row stride N).  Every thread of the workgroup calls
// it after the tile's store, which wave 0 made at device scope (sc1 stores,
// lds_reduce_store's COH form): once wave 0 has seen them complete, the
// workgroup counts itself in on its head's counter.  The workgroup that
// completes the count does the work over all of the head's tiles, reading
// the other tiles' outputs with device-scope (sc1) loads, and puts the
// counter back to zero.  Nobody waits, so no workgroup depends on another
// being resident.
//  * TAIL_ROPE (TP = L, head dim 16 L): the hd / 16 tiles of one q or k head
//    h (columns [h hd, (h + 1) hd), h < nq + nk) count on slot h; then
//    qk_norm_rope_vec_kernel's computation on that head for every row m < M,
//    in place.
// Measured on MI355X at the config-5 QKV shape (M = 4, K = 3072, N = 12288,
// 32 q / k heads of 256): 10.9 us per launch against 8.6 us for the GEMV
// alone and 2.7 us for the separate QK-norm+RoPE launch.  What did not pay:
// a plain __threadfence (an L2 write-back) in every workgroup (15.6 us),
// the 32 counters in one 128-byte line (13.8 us), an L2 invalidate and plain
// loads in each head's last workgroup instead of sc1 loads (12.5 us); and
// the same scheme for the add+RMSNorm after the o_proj GEMV (192 workgroups
// into one norm over all outputs): 13.1 us against 5.2 + 2.5 us, since its
// chain of device-scope round trips (stores, the count, the loads) sits on
// the critical path of the launch's last workgroup.
constexpr int TAIL_SLOT = 64;  // ints between counters (256 bytes)

// 16 bytes read at device scope (two 8-byte sc1 loads): another XCD's
// device-scope stores, not a stale line of this XCD's L2.
__device__ inline u4 load_u4_dev(const uint16_t* p) {
  const uint64_t* q = reinterpret_cast<const uint64_t*>(p);
  const uint64_t a = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t b = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return u4{(uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32)};
}

// Counts the workgroup in on counters[slot]; true for the arrival that
// completes `expect` (which then resets the counter).  Uniform per workgroup.
__device__ inline bool tail_arrive(int* counters, int slot, int expect, int* flag) {
  __syncthreads();
  if (threadIdx.x == 0) {
    const bool done = atomicAdd(counters + slot * TAIL_SLOT, 1) == expect - 1;
    if (done) atomicExch(counters + slot * TAIL_SLOT, 0);  // all arrivals are in: ready for the next launch
    *flag = done;
  }
  __syncthreads();
  return *flag != 0;
}

template <typename T, int TAIL, int TP>
__device__ void gemv_tail(const TailArgs& ta, uint16_t* y, int n0, int N, int M, uint8_t* smem, const float (&rcs)[2],
                          const float (&rsn)[2]) {
  static_assert(TAIL == TAIL_ROPE, "tail kinds");
  __shared__ int flag;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (n0 / (16 * TP) >= ta.nq + ta.nk) return;  // v rows: no tail (uniform per workgroup)
  if (wave == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this tile's device-scope stores are done

  {
    constexpr int L = TP, HD = 16 * L, HALF = 8 * L, HPW = 64 / L;  // rows per wave and pass
    const int head = n0 / HD;
    if (!tail_arrive(ta.counters, head, HD / 16, &flag)) return;
    float* cs = reinterpret_cast<float*>(smem);  // [M][HALF]
    float* sn = cs + M * HALF;
    const uint16_t* w = head < ta.nq ? ta.qw : ta.kw;
    const int c = lane % L;
    const u4 wa = load_u4(w + 8 * c), wb = load_u4(w + HALF + 8 * c);
    for (int m0 = 0; m0 < M; m0 += 4 * HPW) {
      const int m = m0 + wave * HPW + lane / L, mc = min(m, M - 1);
      uint16_t* v = y + (size_t)mc * N + (size_t)head * HD;
      // the row's loads first; the cos / sin table (entries tid and tid +
      // 256, M * HALF <= 512 for M <= 4) was computed in the prologue
      const u4 va = load_u4_dev(v + 8 * c), vb = load_u4_dev(v + HALF + 8 * c);
      if (m0 == 0) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int i = tid + 256 * j;
          if (i < M * HALF) {
            cs[i] = rcs[j];
            sn[i] = rsn[j];
          }
        }
      }
      __syncthreads();
      u4 oa, ob;
      norm_rope_chunks<T, L>(va, vb, wa, wb, cs + mc * HALF, sn + mc * HALF, ta.eps, ta.neox != 0, c, oa, ob);
      if (m < M) {
        *reinterpret_cast<u4*>(v + 8 * c) = oa;
        *reinterpret_cast<u4*>(v + HALF + 8 * c) = ob;
        if (ta.qcopy && head < ta.nq) {
          uint16_t* qv = ta.qcopy + (size_t)m * ta.nq * HD + (size_t)head * HD;
          *reinterpret_cast<u4*>(qv + 8 * c) = oa;
          *reinterpret_cast<u4*>(qv + HALF + 8 * c) = ob;
        }
      }
    }
  }
}

// One kernel for both activation kinds.  XF8 = false: x is T (fp16/bf16), a
// lane's 16-byte weight unit (16 K values) is decoded to two 8-value operands
// of v_mfma_f32_16x16x32_{f16,bf16}.  XF8 = true: x holds e4m3 codes with
// per-row scales sg.xs; two units per lane feed one
// v_mfma_f32_16x16x128_f8f6f4 with no decode.
//
// Stage i = bytes [1024 i, 1024 i + 1024) of the workgroup's 16*NT weight
// rows plus the activation operands that go with them.  Loads run D stages
// ahead into registers (a ring of D + 1 slots, so the loop body is unrolled
// D + 1 times); stage i is copied into one of two LDS buffers, then read back
// in MFMA layout.  K = 1024 STEPS.
//
// TPW > 1: a workgroup owns TPW consecutive tiles of 16*NT rows and streams
// them as one run of TPW * STEPS stages; each tile ends with its own
// cross-wave reduction and store while the next tile's stages are already in
// flight.  For short K (few stages per tile) this spreads the pipeline fill
// and the epilogue of a workgroup over several tiles.
//
// R12: tiles of 12 rows instead of 16 (each wave streams 3 rows per stage
// and tile; MFMA operand lanes 12-15 read row 11 again and are not stored),
// so that a launch can spread its rows more evenly over the CUs; NT = 2 then
// gives 24-row workgroups.  Only without ROT: every tile then reads its K
// chunks in the same order, so each output's sum is the 16-row form's bit
// for bit.
//
// GLU (gate/up matrix with gelu_and_mul fused into the epilogue; TPW = 2,
// one segment of N = 2 d rows): the workgroup's two tiles are gate rows
// [n, n + 16) and up rows [d + n, d + n + 16); the gate tile's scaled sums
// are rounded to TO and kept in wave 0's registers, and the up tile's end
// stores y[m, n + c] = TO(gelu_tanh(gate) * up) into the [M, d] output --
// the values gelu_and_mul computes from the rounded GEMV output.
//
// NORM (M <= MX <= 4 rows, one tile row block): the activations are not read
// from x but computed in the prologue from (na.h, na.r, na.w) -- the
// add+RMSNorm of add_rmsnorm_kernel, with its thread layout and reduction
// order, so the values are bit-identical, and with XF8 its per-row e4m3
// quantisation -- for the whole K into LDS, where the stages read them.  The
// loads of h and r are issued before the weight prologue, so the norm runs
// while the first weight stages are in flight.  Workgroup 0 also writes the
// side outputs (na.r_out, na.h_out or na.q_out / na.s_out); the other
// workgroups read na.r meanwhile, so na.r_out must not alias it.
//
// TAIL (with TP, see gemv_tail): after the tile's store, the last workgroup
// to finish (of all, or of one head's tiles) runs a fused epilogue on the
// output: add+RMSNorm with a residual, or QK RMSNorm + RoPE per head.
//
// ROT: tile t (16-row block index t16 of its first row) reads its K chunks
// in the order t16 mod STEPS, t16 mod STEPS + 1, ... (wrapping), so that
// tiles streaming at the same time read different 1 KB columns of their rows
// instead of all the same one (HBM channels then share the load: M = 4,
// K = 3072, N = 12288: 9.2 -> 8.4 us; K = 4096, N = 4096: 6.5 -> 5.8 us).
// It changes the order of the K sums of every tile, so all forms that must
// agree bit for bit (plain, GLU, NORM, TAIL, multi-matrix) take it under the
// same rule: fp16 / bf16 activations and M <= 4 (launch_lds_steps).  The
// runtime chunk offsets cost VALU address arithmetic, which made the
// multi-tile and M > 4 forms 1-5% slower with it.
template <typename T, typename TO, int FMT, bool XF8, int NT, int MB, int D, int STEPS, int MX = 0, int TPW = 1,
          bool GLU = false, bool NORM = false, int TAIL = TAIL_NONE, int TP = 0, bool ROT = false, int EPI = EPI_NONE,
          bool R12 = false>
__global__ __launch_bounds__(256) void gemv_lds_kernel(const void* xv, GemvSegs sg, int skind, int M, NormArgs na) {
  constexpr bool PROD = EPI == EPI_ADDNORM || EPI == EPI_ADDNORM12;  // deferred-norm producer
  static_assert(!PROD || (TPW == 1 && NT == 1 && MB == 1 && !GLU && !NORM && TAIL == TAIL_NONE && !XF8 &&
                                       std::is_same<T, TO>::value),
                "deferred norm producer: one 16- or 12-row tile, fp16 / bf16");
  static_assert(EPI != EPI_ROWSCALE || (MB == 1 && !NORM && !XF8), "deferred norm consumer: fp16 / bf16, M <= 16");
  static_assert(EPI != EPI_ROWSCALE || STEPS >= 2, "deferred norm consumer: row scales at stage 1, before tile 0 ends");
  constexpr int NS = STEPS * TPW;  // stages of the workgroup
  static_assert(D >= 1 && D <= NS, "prefetch depth");
  static_assert(MX == 0 || (MB == 1 && MX <= 16), "activations go through LDS only for M <= 16");
  static_assert(!GLU || (TPW == 2 && NT == 1), "gate/up pairs are two 16-row tiles");
  static_assert(!NORM || (MX >= 1 && MX <= 4 && NT == 1), "fused norm: up to four rows");
  static_assert(TAIL == TAIL_NONE || (TPW == 1 && NT == 1 && MB == 1 && !GLU && !NORM && !XF8 &&
                                      std::is_same<T, TO>::value),
                "tails: one 16-row tile per workgroup, fp16 / bf16 activations");
  static_assert(!R12 || (NT <= 2 && MB == 1 && !GLU && !NORM && TAIL == TAIL_NONE && !ROT && EPI == EPI_NONE),
                "12-row plain tiles: one or two tiles wide, no K rotation (so each output's sum order is the 16-row "
                "form's)");
  constexpr int K = STEPS * 1024;
  constexpr int SH = EPI == EPI_ADDNORM12 || R12 ? 12 : 16;  // rows of one MFMA tile
  constexpr int ROWS = SH * NT, S = D + 1, STAGE = ROWS * 1024;
  constexpr int QN = XF8 ? 2 : 4;  // operand groups per wave and stage
  constexpr int XB = XF8 ? 1 : 2;  // activation bytes per value
  constexpr int LW = ROWS / 4;     // weight rows per wave and stage
  // MX > 0: the stage's activations (MX rows, rows >= M repeating row M - 1)
  // are loaded 16 contiguous bytes per lane and staged in LDS next to the
  // weights, XU units per thread; MX = 0: each lane loads its MFMA operands
  // straight from L2 (all 16 operand rows, the clamped ones included).
  constexpr int XROW = 1024 * XB;                  // activation bytes per row and stage
  constexpr int XU = MX > 0 && !NORM ? MX * XROW / 16 / 256 : 1;
  constexpr int XSTAGE = MX * XROW;
  static_assert(MX == 0 || NORM || XU * 16 * 256 == XSTAGE, "activation units per thread");
  // two weight stage buffers; the activations of two stages (NORM: of all
  // STEPS stages); (TPW > 1) the cross-wave reduction area; (NORM) the
  // norm's per-row partial sums and maxima
  constexpr int XAREA = NORM ? STEPS * XSTAGE : 2 * XSTAGE;
  constexpr int RED = TPW > 1 ? 3 * NT * MB * 64 * 16 : 0;
  constexpr int NSH = NORM ? 2 * 4 * MX * 4 : 0;
  __shared__ __align__(16) uint8_t smem[2 * STAGE + XAREA + RED + NSH];
  const SegRef sr = find_seg(sg, blockIdx.x);
  const int N = sr.n;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n16 = lane & 15, g = lane >> 4;
  const int wn16 = SH < 16 ? min(n16, SH - 1) : n16;  // this lane's weight row of an MFMA tile (operand)
  const int half = GLU ? N >> 1 : 0;                 // GLU: d, the up rows' offset
  const int nw = sr.group * ROWS * (GLU ? 1 : TPW);  // first row of the workgroup
  // first row of tile t
  auto tile_row = [&](int t) { return GLU ? nw + t * half : nw + ROWS * t; };
  // K chunk (1 KB of each row) that stage i reads
  auto kchunk = [&](int i) {
    const int s = i % STEPS;
    if constexpr (!ROT) {
      return s;
    } else {
      const int r = (EPI == EPI_ADDNORM12 ? sr.group : tile_row(i / STEPS) >> 4) % STEPS;
      return s + r >= STEPS ? s + r - STEPS : s + r;
    }
  };
  uint32_t sc_n[NT];
  float sc_m[MB][4];
  lds_load_scales<NT, MB, SH>(sc_n, sc_m, wave, lane, nw, N, M, sr, skind, XF8 && !NORM ? sg.xs : nullptr);
  // this wave loads rows wave + 4 j of every stage of tile t: row
  // tile_row(t) + wave + 4 j, clamped into the tile's matrix (clamped rows are
  // never stored)
  auto wrow = [&](int t, int j) {
    const int r = wave + 4 * j;
    const int row = GLU ? t * half + min(nw + r, half - 1) : min(nw + ROWS * t + r, N - 1);
    return sr.w + (size_t)row * K + 16 * (lane ^ (r & 15));
  };
  const uint8_t* gx[MB];
#pragma unroll
  for (int b = 0; b < MB; ++b)  // rows >= M are never stored
    gx[b] = static_cast<const uint8_t*>(xv) + (size_t)min(16 * b + n16, M - 1) * K * XB;
  // MX > 0: thread t's units t + 256 j of the MX x XROW stage: row, 16-byte chunk
  const uint8_t* gxu[XU];
  int xdst[XU];
#pragma unroll
  for (int j = 0; j < XU; ++j) {
    const int q = threadIdx.x + 256 * j, row = q / (XROW / 16), col = q % (XROW / 16);
    gxu[j] = static_cast<const uint8_t*>(xv) + (size_t)min(row, M - 1) * K * XB + 16 * col;
    xdst[j] = row * XROW + 16 * (col ^ (row & 7));  // chunk c of row r at c ^ (r & 7)
  }

  // Unit (16 K values) of operand group q for this lane: XF8 = false: unit
  // 4 (wave + 4 q) + g; XF8 = true: units 2 (4 (wave + 4 q) + g) and the next.
  auto unit = [&](int q) { return XF8 ? 2 * (4 * (wave + 4 * q) + g) : 4 * (wave + 4 * q) + g; };

  u4 wr[S][LW];
  u4 xr[S][MX > 0 ? XU : QN][MX > 0 ? 1 : MB][MX > 0 ? 1 : 2];
  auto issue = [&](int i, u4 (&ws)[LW], u4 (&xs)[MX > 0 ? XU : QN][MX > 0 ? 1 : MB][MX > 0 ? 1 : 2]) {
    const int k0 = kchunk(i) << 10;
#pragma unroll
    for (int j = 0; j < LW; ++j) ws[j] = load_u4_stream(wrow(i / STEPS, j) + k0);  // 1 KB of one row per instruction
    asm volatile("" ::: "memory");  // same issue order in every step (weights, then activations)
    if constexpr (NORM) {
      (void)xs;  // activations are resident in LDS
    } else if constexpr (MX > 0) {
#pragma unroll
      for (int j = 0; j < XU; ++j) xs[j][0][0] = load_u4(gxu[j] + (size_t)k0 * XB);
    } else {
#pragma unroll
      for (int q = 0; q < QN; ++q)
#pragma unroll
        for (int b = 0; b < MB; ++b) {
          const u4* p = reinterpret_cast<const u4*>(gx[b] + (size_t)(k0 + 16 * unit(q)) * XB);
          xs[q][b][0] = p[0];
          xs[q][b][1] = p[1];
        }
    }
    asm volatile("" ::: "memory");
  };

  f4 acc[NT][MB];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int b = 0; b < MB; ++b) acc[t][b] = f4{0.f, 0.f, 0.f, 0.f};
  [[maybe_unused]] float gate[MB][4];  // GLU: wave 0's rounded gate values (D layout)

  // NORM: thread t's 8-element units t + 256 j of every row (add_rmsnorm_kernel's
  // layout), rows >= M repeating row M - 1 and units past the row repeating
  // the last (both never used), so that every load is unconditional.
  constexpr int NU = NORM ? (K / 8 + 255) / 256 : 1;
  constexpr int NR = NORM ? MX : 1;
  [[maybe_unused]] u4 nh[NR][NU], nr[NR][NU], ng[NU];
  [[maybe_unused]] float rsc[NR];  // NORM + XF8: the rows' quantisation scales
  if constexpr (NORM) {
#pragma unroll
    for (int j = 0; j < NU; ++j) {
      const int u = min((int)threadIdx.x + 256 * j, K / 8 - 1);
#pragma unroll
      for (int m = 0; m < MX; ++m) {
        const size_t o = (size_t)min(m, M - 1) * K + (size_t)u * 8;
        nh[m][j] = load_u4(na.h + o);
        nr[m][j] = load_u4(na.r + o);
      }
      ng[j] = load_u4(na.w + u * 8);
    }
    asm volatile("" ::: "memory");  // before the weight prologue
  }
  // TAIL_ROPE: the positions of the cos / sin table entries this thread
  // fills if its workgroup runs the tail (entries t and t + 256 of the
  // M x hd/2 table), loaded before the weight prologue so that the wait for
  // them does not drain the weight stages
  [[maybe_unused]] int64_t rpos[2] = {0, 0};
  if constexpr (TAIL == TAIL_ROPE) {
    constexpr int HALF = 8 * TP;
#pragma unroll
    for (int j = 0; j < 2; ++j) rpos[j] = na.tail.pos[min((int)threadIdx.x + 256 * j, M * HALF - 1) / HALF];
    asm volatile("" ::: "memory");  // before the weight prologue
  }
  // EPI_ROWSCALE: wave 0 (the only wave that scales outputs) loads the
  // producer's partial sums of rows 0..3, four per lane (nss <= 256, rows
  // 16-byte aligned), before the weight prologue, so that its wait for them
  // leaves the weight stages in flight
  // The loads are unconditional (clamped addresses, dead values dropped at
  // their use) under a wave-uniform branch: a lane-divergent load makes the
  // compiler wait for it at the end of its branch.
  [[maybe_unused]] const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  [[maybe_unused]] f4 rsp[4];
  [[maybe_unused]] float rinv[4] = {1.f, 1.f, 1.f, 1.f};
  if constexpr (EPI == EPI_ROWSCALE) {
    if (wave_u == 0) {
      const int e = min(4 * lane, na.nss - 4);
#pragma unroll
      for (int m = 0; m < 4; ++m)
        rsp[m] = *reinterpret_cast<const f4*>(na.ss_in + (size_t)min(m, M - 1) * na.nss + e);
    }
    asm volatile("" ::: "memory");  // before the weight prologue
  }
  // EPI_ADDNORM: the residual values (rows 4 (lane >> 4) + v, column
  // lane & 15 of the tile) and norm weight that wave 0's epilogue uses, raw,
  // loaded before the weight prologue so that the epilogue does not wait
  // for them
  // (wave 0 only, under a wave-uniform branch, each value zero-extended to
  // 32 bits: 16-bit values merged at the branch's end get packed in pairs,
  // which makes the compiler wait for the loads there)
  [[maybe_unused]] uint32_t pres[4];  // (set in wave 0 only, used there only)
  [[maybe_unused]] uint32_t pnw;
  if constexpr (PROD) {
    if (wave_u == 0) {
      const int n = min(nw + n16, N - 1);
      pnw = na.w[n];
#pragma unroll
      for (int v = 0; v < 4; ++v) pres[v] = na.r_out[(size_t)min(g * 4 + v, M - 1) * N + n];
    }
    asm volatile("" ::: "memory");  // before the weight prologue
  }
  // EPI_ROWSCALE: wave 0's epilogue row scales, sc_m[0][v] = inv of row 4 (lane >> 4) + v
  auto pick_rs = [&]() {
    if constexpr (EPI == EPI_ROWSCALE) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = min(g * 4 + v, 3);
        sc_m[0][v] = m == 0 ? rinv[0] : (m == 1 ? rinv[1] : (m == 2 ? rinv[2] : rinv[3]));
      }
    }
  };
  // NORM + XF8: wave 0's epilogue row scales, sc_m[0][v] for row 4 (lane >> 4) + v
  auto pick_row_scales = [&]() {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = min(g * 4 + v, M - 1);
      float pick = rsc[0];
#pragma unroll
      for (int mm = 1; mm < NR; ++mm) pick = m == mm ? rsc[mm] : pick;
      sc_m[0][v] = pick;
    }
  };

  // Fully unrolled over the NS stages (the host instantiates the K values
  // it supports), so every slot index and every condition is static and the
  // compiler's in-order vmcnt waits are exact: the wait for stage i leaves
  // the loads of the stages after it in flight.
#pragma unroll
  for (int j = 0; j < D; ++j) issue(j, wr[j], xr[j]);

  // TAIL_ROPE: this thread's cos / sin table entries (fp64 angles, the
  // standalone op's rope_angle), computed while the first weight stages are
  // in flight -- in the tail they sat on the launch's critical path.  Every
  // q / k workgroup computes them; only the last of each head uses them.
  [[maybe_unused]] float rcs[2] = {0.f, 0.f}, rsn[2] = {0.f, 0.f};
  if constexpr (TAIL == TAIL_ROPE) {
    constexpr int HALF = 8 * TP, HD = 16 * TP;
    if (nw / HD < na.tail.nq + na.tail.nk) {  // q / k heads (uniform per workgroup)
      const double lt = log2((double)na.tail.theta);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int i = (int)threadIdx.x + 256 * j;
        if (i < M * HALF) rope_angle((double)rpos[j], i % HALF, HD, lt, rcs[j], rsn[j]);
      }
    }
  }

  // EPI_ROWSCALE: the rows' sums in a fixed order -- each lane's four,
  // then the wave's 64 lanes (the DPP steps of wave_sum_dpp, the four rows
  // interleaved) -- and their 1 / rms (v_rsq_f32 of sum / K + eps, the
  // argument >= eps), in wave 0 (no barrier).  Run at the top of the second
  // K stage: the partial sums' loads (issued before stage 0's) are in, and
  // wave 0 would otherwise wait there for stage 1's; before stage 0 it
  // delayed the first stage, in the epilogue it lengthened every
  // workgroup's critical path.
  auto rowscale_sums = [&]() {
    if constexpr (EPI == EPI_ROWSCALE) {
      if (wave_u == 0) {
        const bool in = 4 * lane < na.nss;
        float t[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) t[m] = in && m < M ? (rsp[m][0] + rsp[m][1]) + (rsp[m][2] + rsp[m][3]) : 0.f;
#pragma unroll
        for (int m = 0; m < 4; ++m) t[m] += CEK_DPP_F32(t[m], 0xB1);
#pragma unroll
        for (int m = 0; m < 4; ++m) t[m] += CEK_DPP_F32(t[m], 0x4E);
#pragma unroll
        for (int m = 0; m < 4; ++m) t[m] += CEK_DPP_F32(t[m], 0x141);
#pragma unroll
        for (int m = 0; m < 4; ++m) t[m] += CEK_DPP_F32(t[m], 0x140);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const float sum = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t[m]), 0)) +
                            __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t[m]), 16)) +
                            __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t[m]), 32)) +
                            __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t[m]), 48));
          rinv[m] = __builtin_amdgcn_rsqf(sum * (1.f / (float)K) + na.eps);
        }
        pick_rs();
      }
    }
  };

  if constexpr (NORM) {
    // add_rmsnorm_kernel's arithmetic, row by row: s = h + r in fp32, r' =
    // Out(s) (stored by workgroup 0), sum of s^2 over the unrounded s (fmaf in
    // unit order, wave butterfly, then the four waves in order), inv =
    // rsqrt(sum / K + eps), normed = Out(r' * inv * w).
    typedef typename std::conditional<XF8, TO, T>::type TN;  // the norm's activation type
    constexpr int UNITS = K / 8;
    const int t = threadIdx.x;
    const bool side = blockIdx.x == 0;  // writes the side outputs
    uint8_t* xall = smem + 2 * STAGE;
    float* nsh = reinterpret_cast<float*>(smem + 2 * STAGE + XAREA + RED);  // [2][MX][4]
    float ss[MX];
    u4 rp[MX][NU];
#pragma unroll
    for (int m = 0; m < MX; ++m) {
      ss[m] = 0.f;
#pragma unroll
      for (int j = 0; j < NU; ++j) {
        const int u = t + 256 * j;
        u4 o = u4{0, 0, 0, 0};
        if (u < UNITS) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float a0 = TN::to_f32(nh[m][j][e] & 0xFFFF) + TN::to_f32(nr[m][j][e] & 0xFFFF);
            const float a1 = TN::to_f32(nh[m][j][e] >> 16) + TN::to_f32(nr[m][j][e] >> 16);
            ss[m] = fmaf(a0, a0, ss[m]);
            ss[m] = fmaf(a1, a1, ss[m]);
            o[e] = (uint32_t)TN::from_f32(a0) | ((uint32_t)TN::from_f32(a1) << 16);
          }
          if (side && m < M) *reinterpret_cast<u4*>(na.r_out + (size_t)m * K + u * 8) = o;
        }
        rp[m][j] = o;
      }
      const float v = wave_sum(ss[m]);
      if (lane == 0) nsh[m * 4 + wave] = v;
    }
    lds_barrier();
    float amax[MX];
    u4 nv[MX][NU];
#pragma unroll
    for (int m = 0; m < MX; ++m) {
      const float inv = rsqrtf((nsh[m * 4] + nsh[m * 4 + 1] + nsh[m * 4 + 2] + nsh[m * 4 + 3]) / (float)K + na.eps);
      amax[m] = 0.f;
#pragma unroll
      for (int j = 0; j < NU; ++j) {
        const int u = t + 256 * j;
        if (u >= UNITS) continue;
        u4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float n0 = f32_round(TN::to_f32(rp[m][j][e] & 0xFFFF) * inv * TN::to_f32(ng[j][e] & 0xFFFF));
          const float n1 = f32_round(TN::to_f32(rp[m][j][e] >> 16) * inv * TN::to_f32(ng[j][e] >> 16));
          const uint16_t b0 = TN::from_f32(n0), b1 = TN::from_f32(n1);
          if (XF8) amax[m] = fmaxf(amax[m], fmaxf(fabsf(TN::to_f32(b0)), fabsf(TN::to_f32(b1))));
          o[e] = (uint32_t)b0 | ((uint32_t)b1 << 16);
        }
        if constexpr (XF8) {
          nv[m][j] = o;
        } else {
          // unit u = chunk u % 128 of stage u / 128, rows swizzled as the stages' are
          *reinterpret_cast<u4*>(xall + (u >> 7) * XSTAGE + m * XROW + 16 * ((u & 127) ^ (m & 7))) = o;
          if (side && m < M && na.h_out) *reinterpret_cast<u4*>(na.h_out + (size_t)m * K + u * 8) = o;
        }
      }
    }
    if constexpr (XF8) {
      // per_token_quant_kernel's quantisation of the rounded normed rows
#pragma unroll
      for (int m = 0; m < MX; ++m) {
        const float v = wave_max(amax[m]);
        if (lane == 0) nsh[(MX + m) * 4 + wave] = v;
      }
      lds_barrier();
#pragma unroll
      for (int m = 0; m < MX; ++m) {
        const float* mx = nsh + (MX + m) * 4;
        const float sq = quant_scale(fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3])));
        rsc[m] = sq;
        if (side && m < M && t == 0) na.s_out[m] = sq;
#pragma unroll
        for (int j = 0; j < NU; ++j) {
          const int u = t + 256 * j;
          if (u >= UNITS) continue;
          uint32_t c[2];
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const uint32_t a = nv[m][j][2 * e], b = nv[m][j][2 * e + 1];
            c[e] = f32x4_to_e4m3x4(quant_clamp(TN::to_f32(a & 0xFFFF), sq), quant_clamp(TN::to_f32(a >> 16), sq),
                                   quant_clamp(TN::to_f32(b & 0xFFFF), sq), quant_clamp(TN::to_f32(b >> 16), sq));
          }
          // unit u = half u & 1 of 16-code chunk (u % 128) / 2 of stage u / 128
          *reinterpret_cast<uint2*>(xall + (u >> 7) * XSTAGE + m * XROW + 16 * (((u & 127) >> 1) ^ (m & 7)) +
                                    8 * (u & 1)) = make_uint2(c[0], c[1]);
          if (side && m < M) *reinterpret_cast<uint2*>(na.q_out + (size_t)m * K + u * 8) = make_uint2(c[0], c[1]);
        }
      }
      pick_row_scales();
    }
    // the first stage's barrier orders these LDS writes before any read
  }
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    if (i == 1) rowscale_sums();
    // Stage i into LDS buffer i & 1 (last read at step i - 2, which every
    // wave finished before the barrier of step i - 1).  Lane l's unit lands
    // at slot l, i.e. unit v of row r at slot v ^ (r & 15).
    uint8_t* sw = smem + (i & 1) * STAGE;
    uint8_t* sx = smem + 2 * STAGE + (NORM ? kchunk(i) : i & 1) * XSTAGE;
#pragma unroll
    for (int jj = 0; jj < LW; ++jj) *reinterpret_cast<u4*>(sw + (wave + 4 * jj) * 1024 + 16 * lane) = wr[i % S][jj];
    if constexpr (MX > 0 && !NORM) {
#pragma unroll
      for (int j = 0; j < XU; ++j) *reinterpret_cast<u4*>(sx + xdst[j]) = xr[i % S][j][0][0];
    }
    lds_barrier();
    if (i + D < NS) issue(i + D, wr[(i + D) % S], xr[(i + D) % S]);
    const int xrow = min(n16, M - 1);  // MX > 0: this lane's operand row in LDS
    const uint8_t* sxr = sx + xrow * XROW;
#pragma unroll
    for (int q = 0; q < QN; ++q) {
      const int v = unit(q);
      // this lane's activation operand for group q: 32 bytes of its row
      u4 xa0, xa1;
      if constexpr (MX > 0) {
        const int c0 = XF8 ? v : 2 * v;  // first 16-byte chunk
        xa0 = *reinterpret_cast<const u4*>(sxr + 16 * (c0 ^ (xrow & 7)));
        xa1 = *reinterpret_cast<const u4*>(sxr + 16 * ((c0 + 1) ^ (xrow & 7)));
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int rr = SH * t + wn16;  // the lane's row of MFMA tile t in the stage
        const uint8_t* rw = sw + rr * 1024;  // its unit v sits at slot v ^ (rr & 15)
        if constexpr (XF8) {
          const i8 bf = cat_i8(*reinterpret_cast<const u4*>(rw + 16 * (v ^ (rr & 15))),
                               *reinterpret_cast<const u4*>(rw + 16 * ((v + 1) ^ (rr & 15))));
#pragma unroll
          for (int b = 0; b < MB; ++b) {
            if constexpr (MX > 0) acc[t][b] = mfma_fp8_16x16x128(cat_i8(xa0, xa1), bf, acc[t][b]);
            else acc[t][b] = mfma_fp8_16x16x128(cat_i8(xr[i % S][q][b][0], xr[i % S][q][b][1]), bf, acc[t][b]);
          }
        } else {
          u4 lo, hi;
          decode16<T, FMT>(*reinterpret_cast<const u4*>(rw + 16 * (v ^ (rr & 15))), lo, hi);
#pragma unroll
          for (int b = 0; b < MB; ++b) {
            if constexpr (MX > 0) {
              acc[t][b] = mfma16x16x32<T>(xa0, lo, acc[t][b]);
              acc[t][b] = mfma16x16x32<T>(xa1, hi, acc[t][b]);
            } else {
              acc[t][b] = mfma16x16x32<T>(xr[i % S][q][b][0], lo, acc[t][b]);
              acc[t][b] = mfma16x16x32<T>(xr[i % S][q][b][1], hi, acc[t][b]);
            }
          }
        }
      }
    }
    if constexpr (TPW > 1) {
      if (i % STEPS == STEPS - 1) {  // tile i / STEPS is complete
        uint8_t* redp = smem + 2 * STAGE + XAREA;
        if constexpr (GLU) {
          if (i / STEPS == 0) {  // gate tile: keep the rounded values
            lds_reduce_tile<NT, MB>(acc, redp, wave, lane, skind, sc_n, sc_m, XF8 || EPI == EPI_ROWSCALE,
                                    [&](int, int b, int v, float o) { gate[b][v] = TO::to_f32(TO::from_f32(o)); });
          } else {  // up tile: gelu_and_mul and the store
            lds_reduce_tile<NT, MB>(acc, redp, wave, lane, skind, sc_n, sc_m, XF8 || EPI == EPI_ROWSCALE,
                                    [&](int, int b, int v, float o) {
              const int n = nw + n16, m = b * 16 + g * 4 + v;
              if (n < half && m < M)
                sr.y[(size_t)m * half + n] =
                    TO::from_f32(f32_round(gelu_tanh(gate[b][v]) * TO::to_f32(TO::from_f32(o))));
            });
          }
        } else {
          lds_reduce_store_tile<NT, MB, SH>(acc, redp, wave, lane, tile_row(i / STEPS), N, M, sr, skind, sc_n, sc_m,
                                            XF8 || EPI == EPI_ROWSCALE, std::is_same<TO, BF16>::value);
        }
        if (i + 1 < NS) {
#pragma unroll
          for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int b = 0; b < MB; ++b) acc[t][b] = f4{0.f, 0.f, 0.f, 0.f};
          lds_load_scales<NT, MB, SH>(sc_n, sc_m, wave, lane, tile_row(i / STEPS + 1), N, M, sr, skind,
                                      XF8 && !NORM ? sg.xs : nullptr);
          if constexpr (NORM && XF8) pick_row_scales();
          pick_rs();
        }
      }
    }
  }
  if constexpr (PROD)
    lds_reduce_addnorm<T, ROWS>(acc[0][0], smem, wave, lane, nw, N, M, sr, skind, sc_n[0], na, pres, pnw);
  else if constexpr (TPW == 1)
    lds_reduce_store<NT, MB, TAIL != TAIL_NONE, SH>(acc, smem, wave, lane, nw, N, M, sr, skind, sc_n, sc_m,
                                                    XF8 || EPI == EPI_ROWSCALE, std::is_same<TO, BF16>::value);
  if constexpr (TAIL != TAIL_NONE) gemv_tail<T, TAIL, TP>(na.tail, sr.y, nw, N, M, smem, rcs, rsn);
}

// ---------------------------------------------------------------------------
// 9 <= M <= 16 with wide N: the activations resident in LDS.
//
// gemv_lds_kernel reads, for every 16-row tile, the 16 activation rows of
// each K stage from L2 straight into MFMA operand layout: lane l takes row
// l & 15, so every such load touches 16 cache lines, and at M = 16 the
// texture-address unit stalls on them (its waves wait on outstanding loads
// most of their cycles).  Here a workgroup loads the whole activation matrix
// (16 rows x K values, rows >= M repeating row M - 1: 64-128 KB) into LDS
// once, by direct-to-LDS loads, and streams its weight rows from global
// memory straight into operand registers (no weight staging, no barrier per
// stage).  A workgroup runs TPB tiles of 16 weight rows at a time, each tile
// split over two waves: the wave of half h takes K values [h K / 2,
// (h + 1) K / 2) of the tile's rows, as 64-byte chunks (lane group g = lane
// >> 4 takes bytes 16 g .. 16 g + 15 of a chunk, two 8-value MFMA operands),
// PD chunks in flight; the second half's sum is then added to the first's
// through LDS, scaled and rounded as in gemv_lds_kernel.  The sum order
// differs from gemv_lds_kernel's, so the outputs may differ from it in the
// last bit: the dispatcher picks the kernel per weight matrix (by its own
// row count), so a multi-matrix launch still gives each matrix what it gets
// alone.  Slots of TPB tiles run grid-stride over the tiles of all segments.
//
// LDS: activation chunk lc (16 bytes) of row r sits at (lc & ~15) | ((lc ^ r)
// & 15): the 16 rows that one 16-lane group of a ds_read_b128 reads at the
// same K land in 16 different 16-byte bank groups.  The direct-to-LDS loads
// fill LDS in order, so lane i of load j fetches the logical chunk that
// belongs at physical chunk 64 j + i (the map is its own inverse).
//
// Measured on MI355X against gemv_lds_kernel (weights from HBM, M = 16 unless
// given): K = 4096, N = 14336 17.37 -> 15.25 us, N = 28672 29.99 -> 26.49,
// M = 12, N = 14336 16.44 -> 15.01, M = 9, N = 28672 27.15 -> 26.31;
// K = 3072, N = 12288 12.65 -> 12.29.  Not faster at 512 tiles or fewer
// (N = 6144: 10.34 us against 9.99 for gemv_lds_kernel; N = 8192 equal) nor
// above 2048 (N = 49152: 44.7 against 44.2).  Splitting each tile's K by residues mod 4 over the
// waves instead (which sums in gemv_lds_kernel's order, bit for bit) was
// 0-8% slower than this form where it gained, and 8% slower than
// gemv_lds_kernel at M = 9, N = 28672.
template <typename T, typename TO, int FMT, int K, int TPB, int PD>
__global__ __launch_bounds__(128 * TPB) void gemv_xres_kernel(const uint16_t* __restrict__ x, GemvSegs sg, int skind,
                                                             int M, int tiles) {
  constexpr int NCW = K / 128;  // 64-byte chunks per wave and tile (half of the K values)
  constexpr int XBYTES = 16 * K * 2, CPR = K / 8;
  static_assert(NCW % PD == 0, "whole prefetch groups");
  static_assert(XBYTES % 1024 == 0, "1 KB direct-to-LDS loads");
  __shared__ __attribute__((aligned(1024))) uint8_t sx[XBYTES];
  __shared__ f4 red[TPB * 64];  // the second halves' sums
  static_assert(sizeof(sx) + sizeof(red) <= 160 * 1024, "LDS");
  // wave-uniform indices (so that the segment table is read by scalar loads,
  // which do not count against the weight loads' vmcnt)
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int tw = wave >> 1, kh = wave & 1;
  const int r16 = lane & 15, g = lane >> 4;
  const int nslot = (tiles + TPB - 1) / TPB;
  // this wave's tile of slot s (clamped: a wave past the last tile repeats
  // it and stores nothing) and the first weight byte it reads: its row
  // (clamped into its matrix; rows past it are never stored), K half, lane group
  auto wsrc = [&](int s) {
    const SegRef r = find_seg(sg, min(s * TPB + tw, tiles - 1));
    return r.w + (size_t)min(16 * r.group + r16, r.n - 1) * K + (K / 2) * kh + 16 * g;
  };
  // half 0: the weight scale of this lane's output column of slot s's tile
  auto scale_bits = [&](int s) {
    const SegRef r = find_seg(sg, min(s * TPB + tw, tiles - 1));
    return kh == 0 ? load_scale_bits(r.s, skind, min(16 * r.group + r16, r.n - 1)) : 0u;
  };
  int s = blockIdx.x;
  uint32_t scb = s < nslot ? scale_bits(s) : 0u;
  {
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(x), 0, M * K * 2, 0x00020000);
    for (int j = wave; j < XBYTES / 1024; j += 2 * TPB) {
      const int pc = 64 * j + lane, r = pc / CPR, p = pc % CPR;
      const int lc = (p & ~15) | ((p ^ r) & 15);
#if defined(__HIP_DEVICE_COMPILE__)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr_t)(sx + 1024 * j), 16,
                                               (uint32_t)((min(r, M - 1) * K + 8 * lc) * 2), 0, 0, 0);
#endif
    }
  }
  u4 wb[PD];
  const uint8_t* wr = wsrc(s);
  if (s < nslot) {
#pragma unroll
    for (int i = 0; i < PD; ++i) wb[i] = load_u4(wr + 64 * i);
    wait_vmcnt<PD>();  // this wave's activation loads (older) are in LDS
  } else {
    wait_vmcnt<0>();
  }
  bare_barrier();
  const uint8_t* xr = sx + r16 * (K * 2);
  const int c0 = NCW * kh;  // this wave's first chunk
  for (; s < nslot; s += gridDim.x) {
    const int sn = s + gridDim.x;
    const uint8_t* wn = wsrc(sn);
    f4 acc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
    for (int j0 = 0; j0 < NCW; j0 += PD) {
      // the next PD chunks of this tile, or the first of the next slot's
      // (after the last slot: the PD chunks just read again, still in the
      // caches and never used -- the loads stay unconditional, so every wait
      // count is static)
      const uint8_t* src = j0 + PD < NCW ? wr + 64 * (j0 + PD) : (sn < nslot ? wn : wr + 64 * (NCW - PD));
#pragma unroll
      for (int i = 0; i < PD; ++i) {
        const u4 w = wb[i];
        wb[i] = load_u4(src + 64 * i);
        u4 lo, hi;
        decode16<T, FMT>(w, lo, hi);
        const int lc = 8 * (c0 + j0 + i) + 2 * g;  // chunk c: 16-byte activation pieces 8 c + 2 g, + 1
        const u4 x0 = *reinterpret_cast<const u4*>(xr + 16 * ((lc & ~15) | ((lc ^ r16) & 15)));
        const u4 x1 = *reinterpret_cast<const u4*>(xr + 16 * (((lc + 1) & ~15) | (((lc + 1) ^ r16) & 15)));
        acc = mfma16x16x32<T>(x0, lo, acc);
        acc = mfma16x16x32<T>(x1, hi, acc);
      }
    }
    if (kh == 1) red[tw * 64 + lane] = acc;
    lds_barrier();
    const int tile = s * TPB + tw;
    if (kh == 0 && tile < tiles) {
      const SegRef r = find_seg(sg, tile);
      const f4 c = acc + red[tw * 64 + lane];
      const int n = 16 * r.group + r16;
      const float sc = scale_value(scb, skind);
      if (n < r.n) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int m = 4 * g + v;
          if (m < M) r.y[(size_t)m * r.n + n] = TO::from_f32(f32_round(c[v] * sc));
        }
      }
    }
    if (sn < nslot) scb = scale_bits(sn);
    lds_barrier();  // half 0 has read red before the next slot writes it
    wr = wn;
  }
}

// ---------------------------------------------------------------------------
// The same for e4m3 activations (the a8w8 GEMV, per-row activation scales
// sg.xs, fp32 per-channel weight scales), 17 <= M <= 32: the activation codes
// of MB = 2 blocks of 16 rows (rows >= M repeating row M - 1; 32 K bytes: up
// to 128 KB) resident in LDS, the weights straight into the operands of
// v_mfma_f32_16x16x128_f8f6f4.  A lane's operand for the 128-byte K chunk c
// is bytes 128 c + 16 g .. + 15 and 128 c + 64 + 16 g .. + 15 of its row (two
// 16-byte loads, each of 16 rows x 64 contiguous bytes), the activation
// operand the same bytes of its activation row.  Each tile's K is split in
// KS contiguous parts over KS waves, added in order through LDS; outputs
// Out(sum * (sb[n] * sa[m])) as in gemv_lds_kernel.  Measured on MI355X
// against gemv_lds_kernel (weights from HBM, K = 4096, M = 32 unless given):
// N = 6144 (32 tokens into a 4096-wide QKV) 12.53 -> 10.32 us, N = 14336
// 23.71 -> 16.1, N = 28672 33.97 -> 27.28, M = 24, N = 6144 11.09 -> 10.21,
// M = 17, N = 14336 18.3 -> 15.83; at 256 tiles (N = 4096) no faster
// (8.69-9.74 us against 8.68 for gemv_lds_kernel).  Of 1 x 4, 2 x 2, 2 x 4 and 4 x 2 (tiles per slot x K parts),
// 2 x 4 was the fastest or within 1% of it wherever the kernel gained.
// ONE (the launch runs one slot per workgroup): the later K parts' sums go
// through the activation area, once every wave is done reading it, so that
// 32 rows of K = 5120 (160 KB, all of LDS) fit.
// RT = 12: tiles of 12 weight rows (the segment table counts 12-row groups);
// operand lanes 12-15 load row 11 again (the same cache lines as lane 11's,
// in the same instruction) and are not stored.  A tile's K parts and their
// order do not depend on RT, so neither do the outputs.
template <typename TO, int K, int TPB, int KS, int PD, bool ONE = false, int RT = 16>
__global__ __launch_bounds__(64 * TPB * KS) void gemv_xres8_kernel(const uint8_t* __restrict__ x, GemvSegs sg, int M,
                                                                  int tiles) {
  static_assert(RT == 16 || RT == 12, "tile rows");
  constexpr int MB = 2;
  constexpr int NCW = K / 128 / KS;  // 128-byte K chunks per wave and tile
  constexpr int XBYTES = 16 * MB * K, CPR = K / 16;
  constexpr int REDB = TPB * (KS - 1) * MB * 64 * 16;  // bytes of the later parts' sums
  static_assert(NCW % PD == 0, "whole prefetch groups");
  static_assert(XBYTES % 1024 == 0, "1 KB direct-to-LDS loads");
  static_assert(!ONE || REDB <= XBYTES, "the sums fit the activation area");
  __shared__ __attribute__((aligned(1024))) uint8_t sx[XBYTES + (ONE ? 0 : REDB)];
  static_assert(sizeof(sx) <= 160 * 1024, "LDS");
  f4* red = reinterpret_cast<f4*>(ONE ? sx : sx + XBYTES);
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int tw = wave / KS, kh = wave % KS;
  const int r16 = lane & 15, g = lane >> 4;
  const int nslot = (tiles + TPB - 1) / TPB;
  auto wsrc = [&](int s) {
    const SegRef r = find_seg(sg, min(s * TPB + tw, tiles - 1));
    return r.w + (size_t)min(RT * r.group + min(r16, RT - 1), r.n - 1) * K + (K / KS) * kh + 16 * g;
  };
  auto scale_bits = [&](int s) {
    const SegRef r = find_seg(sg, min(s * TPB + tw, tiles - 1));
    return kh == 0 ? load_scale_bits(r.s, SK_F32, min(RT * r.group + min(r16, RT - 1), r.n - 1)) : 0u;
  };
  float scm[MB][4];  // the activation rows' scales (D row 16 b + 4 g + v)
#pragma unroll
  for (int b = 0; b < MB; ++b)
#pragma unroll
    for (int v = 0; v < 4; ++v) scm[b][v] = sg.xs[min(16 * b + 4 * g + v, M - 1)];
  int s = blockIdx.x;
  uint32_t scb = s < nslot ? scale_bits(s) : 0u;
  {
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(x), 0, M * K, 0x00020000);
    for (int j = wave; j < XBYTES / 1024; j += TPB * KS) {
      const int pc = 64 * j + lane, r = pc / CPR, p = pc % CPR;
      const int lc = (p & ~15) | ((p ^ r) & 15);
#if defined(__HIP_DEVICE_COMPILE__)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr_t)(sx + 1024 * j), 16,
                                               (uint32_t)(min(r, M - 1) * K + 16 * lc), 0, 0, 0);
#endif
    }
  }
  u4 wb[PD][2];
  const uint8_t* wr = wsrc(s);
  if (s < nslot) {
#pragma unroll
    for (int i = 0; i < PD; ++i) {
      wb[i][0] = load_u4(wr + 128 * i);
      wb[i][1] = load_u4(wr + 128 * i + 64);
    }
    wait_vmcnt<2 * PD>();  // this wave's activation loads (older) are in LDS
  } else {
    wait_vmcnt<0>();
  }
  bare_barrier();
  const int c0 = NCW * kh;  // this wave's first chunk
  for (; s < nslot; s += gridDim.x) {
    const int sn = s + gridDim.x;
    const uint8_t* wn = wsrc(sn);
    f4 acc[MB];
#pragma unroll
    for (int b = 0; b < MB; ++b) acc[b] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
    for (int j0 = 0; j0 < NCW; j0 += PD) {
      // the next PD chunks, the next slot's first, or (after the last slot)
      // the ones just read again: unconditional loads, static wait counts
      const uint8_t* src = j0 + PD < NCW ? wr + 128 * (j0 + PD) : (sn < nslot ? wn : wr + 128 * (NCW - PD));
#pragma unroll
      for (int i = 0; i < PD; ++i) {
        const i8 wop = cat_i8(wb[i][0], wb[i][1]);
        wb[i][0] = load_u4(src + 128 * i);
        wb[i][1] = load_u4(src + 128 * i + 64);
        const int lc0 = 8 * (c0 + j0 + i) + g, lc1 = lc0 + 4;  // 16-byte pieces of chunk c
#pragma unroll
        for (int b = 0; b < MB; ++b) {
          const int rr = 16 * b + r16;
          const uint8_t* xr = sx + rr * K;
          const u4 x0 = *reinterpret_cast<const u4*>(xr + 16 * ((lc0 & ~15) | ((lc0 ^ rr) & 15)));
          const u4 x1 = *reinterpret_cast<const u4*>(xr + 16 * ((lc1 & ~15) | ((lc1 ^ rr) & 15)));
          acc[b] = mfma_fp8_16x16x128(cat_i8(x0, x1), wop, acc[b]);
        }
      }
    }
    if constexpr (ONE) lds_barrier();  // every wave is done reading the activations
    if (kh > 0) {
#pragma unroll
      for (int b = 0; b < MB; ++b) red[((tw * (KS - 1) + kh - 1) * MB + b) * 64 + lane] = acc[b];
    }
    lds_barrier();
    const int tile = s * TPB + tw;
    if (kh == 0 && tile < tiles) {
      const SegRef r = find_seg(sg, tile);
      const int n = RT * r.group + r16;
      const float sc = scale_value(scb, SK_F32);
      if (n < r.n && r16 < RT) {
#pragma unroll
        for (int b = 0; b < MB; ++b) {
          f4 c = acc[b];
#pragma unroll
          for (int q = 1; q < KS; ++q) c += red[((tw * (KS - 1) + q - 1) * MB + b) * 64 + lane];
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int m = 16 * b + 4 * g + v;
            if (m < M) r.y[(size_t)m * r.n + n] = TO::from_f32(f32_round(c[v] * (sc * scm[b][v])));
          }
        }
      }
    }
    if (sn < nslot) scb = scale_bits(sn);
    lds_barrier();  // part 0 has read red before the next slot writes it
    wr = wn;
  }
}

// ---------------------------------------------------------------------------
// Generic: any M, K, alignment.  One wave per output row of a segment.
// ---------------------------------------------------------------------------
template <typename T, int FMT>
__global__ __launch_bounds__(256) void gemv_generic_kernel(const uint16_t* __restrict__ x, GemvSegs sg, int skind,
                                                           int M, int K) {
  const SegRef sr = find_seg(sg, blockIdx.x);
  const int lane = threadIdx.x & 63;
  const int n = sr.group * 4 + (threadIdx.x >> 6);
  // the row's weight scale before any branch (a wave past the last row reads
  // the last row's and returns)
  const float sc = load_scale(sr.s, skind, min(n, sr.n - 1));
  if (n >= sr.n) return;
  const uint8_t* wr = sr.w + (size_t)n * K;
  for (int m = 0; m < M; ++m) {
    const uint16_t* xr = x + (size_t)m * K;
    float acc = 0.f;
    for (int k = lane; k < K; k += 64) acc += T::to_f32(xr[k]) * fp8_to_f32<FMT>(wr[k]);
    acc = wave_sum(acc);
    if (lane == 0) sr.y[(size_t)m * sr.n + n] = T::from_f32(acc * sc);
  }
}

// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------
// Fill gstart for `rows_per_wg` output rows per workgroup; returns the grid.
static int seg_grid(GemvSegs& sg, int rows_per_wg) {
  int g = 0;
  for (int i = 0; i < sg.count; ++i) {
    sg.gstart[i] = g;
    g += (sg.n[i] + rows_per_wg - 1) / rows_per_wg;
  }
  for (int i = sg.count; i <= MAX_SEGS; ++i) sg.gstart[i] = g;
  return g;
}

// LDS-staged path: configuration per (rows M, total weight rows N, K stages),
// from sweeps on MI355X over the decode shapes.  Returns false when no
// instantiation covers the shape (K not one of 2, 3, 4, 5, 14 or 24 KiB
// values, or M / N outside the ranges below); the caller then uses another
// kernel.  Requires 16-byte aligned x and weights.
template <typename T, typename TO, int FMT, bool XF8, int S>
static bool launch_lds_steps(const void* x, GemvSegs& sg, int skind, int M, int N, hipStream_t st) {
#define CEK_LDS(NT, MB, D) \
  gemv_lds_kernel<T, TO, FMT, XF8, NT, MB, D, S><<<dim3(seg_grid(sg, 16 * (NT))), 256, 0, st>>>(x, sg, skind, M, NormArgs{})
#define CEK_LDS_T(NT, D, MX, TPW, ROT)                                                                         \
  gemv_lds_kernel<T, TO, FMT, XF8, NT, 1, D, S, MX, TPW, false, false, TAIL_NONE, 0, ROT>                     \
      <<<dim3(seg_grid(sg, 16 * (NT) * (TPW))), 256, 0, st>>>(x, sg, skind, M, NormArgs{})
  constexpr bool SHORT = S >= 3 && S <= 5;
  constexpr bool MULTI = S == 4 || S == 5;  // multi-tile workgroups (K = 4096, 5120)
#define CEK_LDS_T12(D, MX, TPW)                                                                          \
  gemv_lds_kernel<T, TO, FMT, XF8, 1, 1, D, S, MX, TPW, false, false, TAIL_NONE, 0, false, EPI_NONE, true> \
      <<<dim3(seg_grid(sg, 12 * (TPW))), 256, 0, st>>>(x, sg, skind, M, NormArgs{})
#define CEK_LDS_24(D)                                                                                   \
  gemv_lds_kernel<T, TO, FMT, XF8, 2, 1, D, S, 0, 1, false, false, TAIL_NONE, 0, false, EPI_NONE, true> \
      <<<dim3(seg_grid(sg, 24)), 256, 0, st>>>(x, sg, skind, M, NormArgs{})
#define CEK_LDS_TPW(NT, D, MX, ROT)                                  \
  do {                                                               \
    if (!(ROT) && (NT) == 1 && r12) {                                \
      if constexpr (MULTI) {                                         \
        if (tpw12 == 4) CEK_LDS_T12(D, MX, 4);                       \
        else if (tpw12 == 2) CEK_LDS_T12(D, MX, 2);                  \
        else CEK_LDS_T12(D, MX, 1);                                  \
      } else {                                                       \
        CEK_LDS_T12(D, MX, 1);                                       \
      }                                                              \
    } else if constexpr (MULTI) {                                    \
      const int tpw = (ROT) ? tpw_rot : tpw_plain;                   \
      if (tpw == 4) CEK_LDS_T(NT, D, MX, 4, ROT);                    \
      else if (tpw == 2) CEK_LDS_T(NT, D, MX, 2, ROT);               \
      else CEK_LDS_T(NT, D, MX, 1, ROT);                             \
    } else {                                                         \
      CEK_LDS_T(NT, D, MX, 1, ROT);                                  \
    }                                                                \
  } while (0)
  // K = 4096 or 5120 (4-5 stages per 16-row tile): TPW consecutive tiles
  // per workgroup.  A workgroup streams at a rate its stages in flight set,
  // so a launch takes as long as its busiest CU's share: of 4, 2 and 1 tiles
  // per workgroup the count with the least ceil(workgroups / CUs) * (tpw *
  // STEPS + F), F the stages' worth a workgroup loses filling its pipeline
  // (0.5 for the rotated forms -- fp16 / bf16, M <= 4, prefetch depth 3 --
  // and 1.5 for the others), the larger count on a tie.  Measured on MI355X
  // (weights from HBM, us for 4 / 2 / 1 tiles), M = 4: N = 14336 12.78 /
  // 13.36 / 13.19; N = 20480 21.05 / 17.94 / 16.99; N = 24576 21.21 / 19.46
  // / 19.71; N = 28672 22.40 / 23.14 / 21.88; N = 32768 23.01 / 24.12 /
  // 25.66; N = 6144: 2 tiles 7.84, 1 tile 8.21; M = 8: N = 20480 22.84 / - /
  // 20.17, N = 24576 23.53 / 20.99 / -, M = 6, N = 28672 23.36 / - / 25.43.
  // Over 48 shapes (M 3-8, K 4096 / 5120, N 8192-30000) its pick was 1.5%
  // above the fastest of the three on average and 7.6% at worst.  The forms
  // agree bit for bit.  At K = 3072 one tile was fastest.
  auto pick_tpw_fill = [&](int f2) {  // f2 = 2 F
    int best = 1;
    long cost = LONG_MAX;
    for (int c = MULTI ? 4 : 1; c >= 1; c >>= 1) {
      const long wgs = ((N + 15) / 16 + c - 1) / c;
      const long k = ((wgs + kCUs - 1) / kCUs) * (2L * c * S + f2);
      if (k < cost) {
        cost = k;
        best = c;
      }
    }
    return best;
  };
  const int tpw_rot = pick_tpw_fill(1), tpw_plain = pick_tpw_fill(3);
  // 12-row tiles (the forms without the K rotation, one tile wide; MFMA
  // operand lanes 12-15 repeat row 11 and are not stored): each output's
  // sum is the 16-row form's bit for bit, so they are free to pick where
  // they cut the busiest CU's rows by a fifth or more -- N = 6144 (24 rows
  // against 32; measured on MI355X, weights from HBM: fp16 M = 8, K = 4096
  // 8.17 -> 7.75 us, M = 5 7.82 -> 7.35, K = 5120 9.59 -> 9.06; e4m3
  // activations M = 8, K = 4096 7.76 -> 7.10, K = 5120 8.84 -> 8.16, M = 4
  // 7.04 -> 6.66) or N = 3072.  9-16 rows above 256 16-row tiles take
  // two-tile workgroups instead (one 12-row tile per workgroup: M = 16,
  // N = 6144 9.82 -> 11.23 us).
  // least_rows(rt, rows): the tiles per workgroup that give the busiest CU
  // the fewest rows with tiles of rt rows, and that count of rows
  auto least_rows = [&](int rt, int& rows) {
    const int t = (N + rt - 1) / rt;
    int best = 1;
    rows = INT_MAX;
    for (int c = MULTI ? 4 : 1; c >= 1; c >>= 1) {
      const int r = rt * c * (((t + c - 1) / c + kCUs - 1) / kCUs);
      if (r < rows) {
        rows = r;
        best = c;
      }
    }
    return best;
  };
  int rows16, rows12;
  least_rows(16, rows16);
  const int tpw12 = least_rows(12, rows12);
  const bool r12 = 5 * rows12 <= 4 * rows16;
  // two-tile workgroups: 2 x 12 rows where they cut the busiest CU's rows
  // against 2 x 16 by a fifth or more (N = 4112-6144: 24 rows against 32)
  auto busiest = [&](int wrows) { return wrows * (((N + wrows - 1) / wrows + kCUs - 1) / kCUs); };
  const bool n24 = 5 * busiest(24) <= 4 * busiest(32);
  if constexpr (!XF8) {
    // fp16/bf16, M <= 8: activations staged through LDS (contiguous loads
    // of just the M rows); for long K only up to 12288 rows (5-20% faster
    // there, slower for wider matrices), except at one row (M = 1,
    // K = 14336: N = 14336 34.0 against 38.2 us, N = 28672 61.7 against
    // 66.7 us).
    if (M <= 8 && (SHORT || N <= 12288 || M == 1)) {
      if (M <= 4) CEK_LDS_TPW(1, (S >= 3 ? 3 : 2), 4, true);
      else CEK_LDS_TPW(1, 2, 8, false);
      return true;
    }
  }
  if constexpr (!XF8 && S == 14) {
    // K = 14336, 8 < M <= 16, N <= 4096 (the down projection): the 16
    // activation rows staged through LDS (measured on MI355X at M = 16,
    // N = 4096: 18.7 -> 16.2 us; at K = 4096 staging 9-16 rows was 3-33%
    // slower)
    if (M > 8 && M <= 16 && N <= 4096) {
      CEK_LDS_T(1, 2, 16, 1, false);
      return true;
    }
  }
  if (M <= 16) {
    if constexpr (SHORT) {
      // Two 16-row tiles per workgroup halve the activation re-reads; they
      // pay once there are more 16-row tiles than CUs (measured on MI355X,
      // M = 16, K = 4096, weights from HBM: N = 4608 11.02 -> 9.26 us, N =
      // 5120 11.03 -> 9.31, K = 3072, N = 5120 8.94 -> 7.54; M = 12, N = 5120
      // 9.76 -> 8.88; at N = 4096, one tile per CU, 7.67 -> 9.16 slower).
      // Two 12-row tiles (24 rows) where that evens out the CUs (N = 4112 to
      // 6144: every CU one workgroup of 24 rows instead of 3 in 4 CUs one of
      // 32), same outputs: M = 16, K = 4096, N = 6144 9.48 -> 8.90 us, N =
      // 4608 9.29 -> 8.54; M = 9, N = 4608 8.44 -> 7.54; M = 12, N = 6144
      // 9.35 -> 8.52, K = 5120, N = 5120 9.88 -> 9.64; K = 3072, M = 16, N =
      // 6144 7.88 -> 7.65; e4m3 activations M = 12, N = 6144 8.08 -> 7.37,
      // M = 16, K = 5120 9.02 -> 8.84.  At 5-8 rows against the 12-row forms
      // they were within +-3% at N = 6144 and are not used there.
      // (fp16 / bf16 M <= 4 took the staged form above)
      if ((N + 15) / 16 > kCUs && (XF8 ? M > 8 : M >= 8)) {
        if (n24) CEK_LDS_24(2);
        else CEK_LDS(2, 1, 2);
      } else {
        CEK_LDS_TPW(1, 3, 0, false);
      }
    } else if constexpr (XF8 && S >= 3) {
      CEK_LDS(1, 1, 3);
    } else if constexpr (!XF8) {
      if (M <= 4) CEK_LDS_T(1, 2, 0, 1, true);  // fp16 / bf16 M <= 4 rotate in every form
      else CEK_LDS(1, 1, 2);
    } else {
      CEK_LDS(1, 1, 2);
    }
    return true;
  }
  if (M <= 32 && N <= 16384) {  // wider N is served as well by the tiled GEMM
    if constexpr (XF8) CEK_LDS(1, 2, 2);
    else CEK_LDS(1, 2, 1);
    return true;
  }
  if constexpr (XF8) {
    if (M <= 64 && N <= 8192) {
      CEK_LDS(1, 4, 1);
      return true;
    }
  }
  return false;
#undef CEK_LDS
#undef CEK_LDS_T
#undef CEK_LDS_T12
#undef CEK_LDS_24
#undef CEK_LDS_TPW
}

template <typename T, typename TO, int FMT, bool XF8>
static bool launch_lds(const void* x, GemvSegs& sg, int skind, int M, int K, int N, hipStream_t st) {
  if (K % 1024 != 0) return false;
  switch (K >> 10) {
    case 2: return launch_lds_steps<T, TO, FMT, XF8, 2>(x, sg, skind, M, N, st);
    case 3: return launch_lds_steps<T, TO, FMT, XF8, 3>(x, sg, skind, M, N, st);
    case 4: return launch_lds_steps<T, TO, FMT, XF8, 4>(x, sg, skind, M, N, st);
    case 5: return launch_lds_steps<T, TO, FMT, XF8, 5>(x, sg, skind, M, N, st);
    case 14: return launch_lds_steps<T, TO, FMT, XF8, 14>(x, sg, skind, M, N, st);
    case 24: return launch_lds_steps<T, TO, FMT, XF8, 24>(x, sg, skind, M, N, st);
    default: return false;
  }
}

// gemv_xres_kernel takes a weight matrix of 512 < tiles <= 2048 16-row tiles
// (8208 <= N <= 32768) when 9 <= M <= 16, the activations are fp16 / bf16 and
// K is 2, 3 or 4 KiB values (the range where it measured faster).
static bool xres_matrix(int M, int K, int n) {
  const int tiles = (n + 15) / 16;
  return M >= 9 && M <= 16 && (K == 2048 || K == 3072 || K == 4096) && tiles > 512 && tiles <= 2048;
}

// gemv_xres_kernel over every segment of sg (all of them xres_matrix): one
// slot per workgroup (one workgroup per CU) as far as the CUs go, TPB =
// ceil(tiles / CUs) tiles per slot (3 to 8), so that the slots spread evenly
// over the CUs (each tile's sum does not depend on TPB).  Measured on MI355X
// at M = 16 against 4 tiles per slot up to 1024 tiles and 8 above (weights
// from HBM): K = 4096, N = 9000 13.74 -> 12.36 us, N = 16400 23.24 -> 18.55,
// N = 20480 23.86 -> 20.51, N = 24576 25.09 -> 22.50, N = 28672 26.72 ->
// 25.78; K = 3072, N = 12288 12.17 -> 11.83; N = 14336 equal.
template <typename T, typename TO, int FMT>
static void launch_xres(const void* x, GemvSegs& sg, int skind, int M, int K, hipStream_t st) {
  const int tiles = seg_grid(sg, 16);  // gstart: first tile of each segment
  int tpb = (tiles + kCUs - 1) / kCUs;
  tpb = tpb < 3 ? 3 : (tpb > 8 ? 8 : tpb);
  const int nslot = (tiles + tpb - 1) / tpb;
  const dim3 grid((unsigned)(nslot < kCUs ? nslot : kCUs));
  const uint16_t* xp = static_cast<const uint16_t*>(x);
#define CEK_XRES(KK, TT) gemv_xres_kernel<T, TO, FMT, KK, TT, 8><<<grid, 128 * (TT), 0, st>>>(xp, sg, skind, M, tiles)
#define CEK_XRES_K(KK)            \
  do {                            \
    if (tpb == 3) CEK_XRES(KK, 3);      \
    else if (tpb == 4) CEK_XRES(KK, 4); \
    else if (tpb == 5) CEK_XRES(KK, 5); \
    else if (tpb == 6) CEK_XRES(KK, 6); \
    else if (tpb == 7) CEK_XRES(KK, 7); \
    else CEK_XRES(KK, 8);               \
  } while (0)
  if (K == 2048) CEK_XRES_K(2048);
  else if (K == 3072) CEK_XRES_K(3072);
  else CEK_XRES_K(4096);
#undef CEK_XRES_K
#undef CEK_XRES
}

// Gate/up GEMV with gelu_and_mul fused (gemv_lds_kernel's GLU form): one
// segment of 2 d rows, one workgroup per 16 output columns.  The per-M
// configurations are the one-tile ones of launch_lds_steps for these K.
template <typename T, typename TO, int FMT, bool XF8, int S>
static void launch_glu_steps(const void* x, GemvSegs& sg, int skind, int M, int d, const NormArgs* rs,
                             hipStream_t st) {
  const int grid = (d + 15) / 16;
  sg.gstart[0] = 0;
  for (int i = 1; i <= MAX_SEGS; ++i) sg.gstart[i] = grid;
#define CEK_GLU(D, MX, ROT)                                                                   \
  gemv_lds_kernel<T, TO, FMT, XF8, 1, 1, D, S, MX, 2, true, false, TAIL_NONE, 0, ROT><<<dim3(grid), 256, 0, st>>>( \
      x, sg, skind, M, NormArgs{})
  if constexpr (!XF8 && FMT == CEK_E4M3) {
    if (rs) {  // deferred RMSNorm consumer (M <= 4, checked by the caller)
      gemv_lds_kernel<T, TO, FMT, XF8, 1, 1, 3, S, 4, 2, true, false, TAIL_NONE, 0, true, EPI_ROWSCALE>
          <<<dim3(grid), 256, 0, st>>>(x, sg, skind, M, *rs);
      return;
    }
  }
  if constexpr (!XF8) {
    if (M <= 4) {
      CEK_GLU(3, 4, true);
      return;
    }
    if (M <= 8) {
      CEK_GLU(2, 8, false);
      return;
    }
  }
  CEK_GLU(3, 0, false);
#undef CEK_GLU
}

template <typename T, typename TO, int FMT, bool XF8>
static int launch_glu(const void* x, GemvSegs& sg, int skind, int M, int d, int K, hipStream_t st,
                      const NormArgs* rs = nullptr) {
  switch (K >> 10) {
    case 3: launch_glu_steps<T, TO, FMT, XF8, 3>(x, sg, skind, M, d, rs, st); break;
    case 4: launch_glu_steps<T, TO, FMT, XF8, 4>(x, sg, skind, M, d, rs, st); break;
    case 5: launch_glu_steps<T, TO, FMT, XF8, 5>(x, sg, skind, M, d, rs, st); break;
    default: return CEK_ERR_UNSUPPORTED;
  }
  return check_launch();
}

// add+RMSNorm (+ quant) fused into the GEMV (gemv_lds_kernel's NORM form):
// e4m3 weights, prefetch depth 3, MX = 1 or 4 activation rows in LDS; with
// gelu_and_mul also the GLU form (N = 2 d rows).  Two consecutive tiles per
// workgroup from 384 tiles at K = 4096 / 5120, as for the plain GEMV.
template <typename T, typename TO, bool XF8, int S, int MX>
static void launch_norm_steps(GemvSegs& sg, const NormArgs& na, int skind, int M, int N, bool glu, hipStream_t st) {
  if (glu) {
    const int grid = (N / 2 + 15) / 16;
    sg.gstart[0] = 0;
    for (int i = 1; i <= MAX_SEGS; ++i) sg.gstart[i] = grid;
    gemv_lds_kernel<T, TO, CEK_E4M3, XF8, 1, 1, 3, S, MX, 2, true, true, TAIL_NONE, 0, !XF8>
        <<<dim3(grid), 256, 0, st>>>(nullptr, sg, skind, M, na);
    return;
  }
  if constexpr (S == 4 || S == 5) {
    if ((N + 15) / 16 >= 384) {
      gemv_lds_kernel<T, TO, CEK_E4M3, XF8, 1, 1, 3, S, MX, 2, false, true, TAIL_NONE, 0, !XF8>
          <<<dim3(seg_grid(sg, 32)), 256, 0, st>>>(nullptr, sg, skind, M, na);
      return;
    }
  }
  gemv_lds_kernel<T, TO, CEK_E4M3, XF8, 1, 1, 3, S, MX, 1, false, true, TAIL_NONE, 0, !XF8>
      <<<dim3(seg_grid(sg, 16)), 256, 0, st>>>(nullptr, sg, skind, M, na);
}

template <typename T, typename TO, bool XF8>
static void launch_norm_t(GemvSegs& sg, const NormArgs& na, int skind, int M, int N, int K, bool glu, hipStream_t st) {
  // one activation row (M = 1) or up to four (the quantising form: one)
  auto by_rows = [&](auto s) {
    constexpr int S_ = decltype(s)::value;
    if constexpr (XF8) launch_norm_steps<T, TO, XF8, S_, 1>(sg, na, skind, M, N, glu, st);
    else if (M == 1) launch_norm_steps<T, TO, XF8, S_, 1>(sg, na, skind, M, N, glu, st);
    else launch_norm_steps<T, TO, XF8, S_, 4>(sg, na, skind, M, N, glu, st);
  };
  if (K == 3072) by_rows(std::integral_constant<int, 3>{});
  else if (K == 4096) by_rows(std::integral_constant<int, 4>{});
  else by_rows(std::integral_constant<int, 5>{});
}

// Whether [a, a + a_bytes) and [b, b + b_bytes) share a byte (an empty
// range shares none).
static bool overlaps(const void* a, int64_t a_bytes, const void* b, int64_t b_bytes) {
  if (a_bytes <= 0 || b_bytes <= 0 || !a || !b) return false;
  const char* pa = static_cast<const char*>(a);
  const char* pb = static_cast<const char*>(b);
  return pa < pb + b_bytes && pb < pa + a_bytes;
}

// The fused launch covers M <= 4 rows (the quantising form: M = 1), K in
// {3072, 4096, 5120}, e4m3 weights, 16-byte aligned operands and side
// outputs that do not overlap the inputs; CEK_ERR_UNSUPPORTED otherwise (the
// caller runs the norm, then the GEMV).  q_out != null selects the
// quantising form (a8w8 GEMV: fp32 per-channel weight scales).
int launch_norm_gemv(const NormArgs& na, const void* w, const void* scale, int skind, void* y, int64_t M,
                     int64_t N, int64_t K, bool glu, int io_dtype, int fp8_fmt, hipStream_t st) {
  const bool quant = na.q_out != nullptr;
  if (M < 0 || N < 0 || K <= 0 || N > INT32_MAX || K > INT32_MAX) return CEK_ERR_INVALID;
  if (io_dtype != CEK_F16 && io_dtype != CEK_BF16) return CEK_ERR_INVALID;
  if (fp8_fmt != CEK_E4M3 && fp8_fmt != CEK_E5M2) return CEK_ERR_INVALID;
  if (skind < 0 || skind == SK_F32_SCALAR) return CEK_ERR_INVALID;
  if (quant && (fp8_fmt != CEK_E4M3 || skind != SK_F32 || !na.s_out || na.h_out)) return CEK_ERR_INVALID;
  if (glu && N % 2) return CEK_ERR_INVALID;
  if (M == 0) return CEK_OK;
  if (!na.h || !na.r || !na.w || !na.r_out || !w || !scale || !y) return CEK_ERR_INVALID;
  if (N * K > ((int64_t)1 << 40)) return CEK_ERR_INVALID;
  const int64_t rb = M * K * 2;  // bytes of one [M, K] activation matrix
  if (N == 0 || M > 4 || (K != 3072 && K != 4096 && K != 5120) || fp8_fmt != CEK_E4M3) return CEK_ERR_UNSUPPORTED;
  // The quantising form fuses one row only: from two rows on, the prologue
  // that every workgroup runs (the norm and the quantisation of all M rows)
  // made the launch slower than the norm+quant launch and the product
  // (measured on MI355X, weights from HBM, us fused / two launches: M = 2-4,
  // K = 4096, N = 6144 12.6-13.0 / 10.1-10.2; K = 5120 26.0-26.7 /
  // 11.8-12.0; K = 3072, N = 12288 27.4-27.7 / 11.3-12.0; at M = 1 7.9 /
  // 9.4, 9.1 / 11.5 and 9.8 / 11.7).
  if (quant && M > 1) return CEK_ERR_UNSUPPORTED;
  if (!aligned(na.h, 16) || !aligned(na.r, 16) || !aligned(na.w, 16) || !aligned(na.r_out, 16) || !aligned(w, 16) ||
      (na.h_out && !aligned(na.h_out, 16)) || (quant && !aligned(na.q_out, 16)))
    return CEK_ERR_UNSUPPORTED;
  // Every workgroup reads h and r in its prologue while others already write
  // y and workgroup 0 writes the side outputs: no output may share memory
  // with an input.
  const int64_t yb = M * (glu ? N / 2 : N) * 2;
  auto hits_inputs = [&](const void* p, int64_t bytes) {
    return p && (overlaps(p, bytes, na.r, rb) || overlaps(p, bytes, na.h, rb) || overlaps(p, bytes, na.w, K * 2));
  };
  if (hits_inputs(na.r_out, rb) || hits_inputs(na.h_out, rb) || hits_inputs(y, yb) ||
      (quant && (hits_inputs(na.q_out, M * K) || hits_inputs(na.s_out, M * 4))))
    return CEK_ERR_UNSUPPORTED;
  GemvSegs sg{};
  sg.count = 1;
  sg.w[0] = static_cast<const uint8_t*>(w);
  sg.s[0] = scale;
  sg.y[0] = static_cast<uint16_t*>(y);
  sg.n[0] = (int)N;
  const int m = (int)M, n = (int)N, k = (int)K;
  if (quant) {
    if (io_dtype == CEK_F16) launch_norm_t<F16, F16, true>(sg, na, SK_F32, m, n, k, glu, st);
    else launch_norm_t<F16, BF16, true>(sg, na, SK_F32, m, n, k, glu, st);
  } else {
    if (io_dtype == CEK_F16) launch_norm_t<F16, F16, false>(sg, na, skind, m, n, k, glu, st);
    else launch_norm_t<BF16, BF16, false>(sg, na, skind, m, n, k, glu, st);
  }
  return check_launch();
}

template <typename T, typename TO, int FMT, bool XF8>
static int launch_gemv_t(const void* x, GemvSegs sg, int skind, int M, int K, bool vec16, hipStream_t st) {
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  int N = 0;  // launch shape is chosen from the total row count
  for (int i = 0; i < sg.count; ++i) N += sg.n[i];
  // The LDS-staged MFMA kernel from three rows on (measured faster than the
  // v_dot2 kernel there, and than the direct MFMA kernel throughout); from one
  // row on for K >= 14336, whose v_dot2 workgroups re-read long activation
  // rows (M = 1, K = 14336, N = 4096: 11.54 -> 11.06 us).  The choice depends
  // on M and K only, so a multi-matrix launch runs the kernel family that
  // each matrix alone would (the LDS forms it may pick between agree bit for
  // bit).
  const int m_lds = K >= 14336 ? 1 : 3;
  if constexpr (!XF8) {
    // matrices that gemv_xres_kernel serves go to one launch of it, the rest
    // on through the kernels below (its sum order differs from theirs, so the
    // choice is per matrix: a multi-matrix launch gives each matrix what it
    // gets alone)
    if (vec16) {
      GemvSegs sx{}, so{};
      sx.xs = so.xs = sg.xs;
      for (int i = 0; i < sg.count; ++i) {
        GemvSegs& d = xres_matrix(M, K, sg.n[i]) ? sx : so;
        d.w[d.count] = sg.w[i];
        d.s[d.count] = sg.s[i];
        d.y[d.count] = sg.y[i];
        d.n[d.count] = sg.n[i];
        ++d.count;
      }
      if (sx.count > 0) {
        launch_xres<T, TO, FMT>(x, sx, skind, M, K, st);
        if (so.count == 0) return check_launch();
        sg = so;
        N = 0;
        for (int i = 0; i < sg.count; ++i) N += sg.n[i];
      }
    }
  }
  if (vec16 && M >= m_lds && launch_lds<T, TO, FMT, XF8>(x, sg, skind, M, K, N, st)) return check_launch();
  if (M > 16) return CEK_ERR_UNSUPPORTED;
  if (vec16 && M <= 4) {
    // Rows per workgroup (measured on MI355X, one pass over > 2 GB of
    // rotating weights): 2 for M = 1 up to K = 4096, else 4, which amortises
    // each workgroup's re-read of the M activation rows over more weight
    // rows.  One 16-byte unit per thread and row per round.
    const int K16 = K / 16;
    const bool r2 = M == 1 && K16 <= 256;
    // K = 2048 and 1024 (rows of 128 and 64 units): 2 and 4 rows per load
    // instruction (RP), two passes per workgroup, instead of 256-thread
    // workgroups half or three quarters idle (M = 1, K = 1024, N = 16384:
    // 7.67 -> 4.71 us; K = 2048: 8.31 -> 7.04 us; M = 2, K = 2048: 8.73 ->
    // 7.83 us; one pass or three or four measured slower; outputs unchanged).
#define CEK_DOT(MT, R, RP) \
  gemv_dot_kernel<T, TO, FMT, XF8, MT, R, 1, RP><<<dim3(seg_grid(sg, (R) * (RP))), 256, 0, st>>>(xp, sg, skind, M, K)
    if (K16 == 128 || K16 == 64) {
      if (K16 == 128) {
        if (M == 1) CEK_DOT(1, 2, 2);
        else if (M == 2) CEK_DOT(2, 2, 2);
        else CEK_DOT(4, 2, 2);
      } else {
        if (M == 1) CEK_DOT(1, 2, 4);
        else if (M == 2) CEK_DOT(2, 2, 4);
        else CEK_DOT(4, 2, 4);
      }
    } else if (M == 1) {
      if (r2) CEK_DOT(1, 2, 1);
      else CEK_DOT(1, 4, 1);
    } else if (M == 2) CEK_DOT(2, 4, 1);
    else CEK_DOT(4, 4, 1);
#undef CEK_DOT
  } else if (vec16 && K % 64 == 0 && M <= 16) {
    // 16-row tiles per wave (NT) and 64-byte K steps in flight per wave
    // (UNROLL), measured per shape class: wide N amortises the activation
    // reads over more tiles; narrow N needs more workgroups and deeper K.
#define CEK_MF(NT, UN) gemv_mfma_kernel<T, TO, FMT, XF8, NT, UN><<<dim3(seg_grid(sg, 16 * NT)), 256, 0, st>>>(xp, sg, skind, M, K)
    if (N >= 16384) CEK_MF(4, 4);
    else if (N >= 8192) { if (M > 8) CEK_MF(4, 2); else if (K <= 3072) CEK_MF(1, 8); else CEK_MF(2, 8); }
    else if (K <= 4096) { if (N >= 6144) CEK_MF(2, 16); else CEK_MF(1, 16); }
    else CEK_MF(1, 4);
#undef CEK_MF
  } else if (!XF8) {
    gemv_generic_kernel<T, FMT><<<dim3(seg_grid(sg, 4)), 256, 0, st>>>(xp, sg, skind, M, K);
  } else {
    return CEK_ERR_UNSUPPORTED;  // the caller only routes vector-friendly shapes here
  }
  return check_launch();
}

// Validates and launches one GEMV over count (<= MAX_SEGS) weight matrices.
// M <= 16 for the GEMV entry points; the GEMM entry point also sends
// 16 < M <= 32 here (max_m = 32), which only the LDS path takes
// (CEK_ERR_UNSUPPORTED otherwise).
int launch_gemv_segs(const void* x, int count, const void* const* w, const void* const* scale,
                     void* const* y, const int64_t* Ns, int64_t M, int64_t K, int skind, int io_dtype,
                     int fp8_fmt, hipStream_t st, int max_m = 16) {
  if (count < 1 || count > MAX_SEGS || !w || !scale || !y || !Ns) return CEK_ERR_INVALID;
  if (M < 0 || K <= 0 || K > INT32_MAX) return CEK_ERR_INVALID;
  if (io_dtype != CEK_F16 && io_dtype != CEK_BF16) return CEK_ERR_INVALID;
  if (fp8_fmt != CEK_E4M3 && fp8_fmt != CEK_E5M2) return CEK_ERR_INVALID;
  GemvSegs sg{};
  int64_t total = 0;
  bool vec16 = K % 16 == 0 && aligned(x, 16);
  for (int i = 0; i < count; ++i) {
    if (Ns[i] < 0 || Ns[i] > INT32_MAX || Ns[i] * K > ((int64_t)1 << 40)) return CEK_ERR_INVALID;
    total += Ns[i];
    sg.w[sg.count] = static_cast<const uint8_t*>(w[i]);
    sg.s[sg.count] = scale[i];
    sg.y[sg.count] = static_cast<uint16_t*>(y[i]);
    sg.n[sg.count] = (int)Ns[i];
    if (Ns[i] == 0) continue;  // empty matrices take no workgroups
    if (!w[i] || !scale[i] || !y[i]) return CEK_ERR_INVALID;
    vec16 = vec16 && aligned(w[i], 16);
    ++sg.count;
  }
  if (total > INT32_MAX) return CEK_ERR_INVALID;
  if (M == 0 || sg.count == 0) return CEK_OK;
  if (M > max_m) return CEK_ERR_INVALID;
  if (!x) return CEK_ERR_INVALID;
  if (io_dtype == CEK_F16 && fp8_fmt == CEK_E4M3) return launch_gemv_t<F16, F16, CEK_E4M3, false>(x, sg, skind, M, K, vec16, st);
  if (io_dtype == CEK_F16 && fp8_fmt == CEK_E5M2) return launch_gemv_t<F16, F16, CEK_E5M2, false>(x, sg, skind, M, K, vec16, st);
  if (fp8_fmt == CEK_E4M3) return launch_gemv_t<BF16, BF16, CEK_E4M3, false>(x, sg, skind, M, K, vec16, st);
  return launch_gemv_t<BF16, BF16, CEK_E5M2, false>(x, sg, skind, M, K, vec16, st);
}

// a8w8 for skinny A (M <= 64): x [M, K] e4m3 codes with per-row scales
// xs [M], e4m3 weights with per-channel fp32 scales; fp16 or bf16 output.
// Requires 16-byte aligned x and w and K % 16 == 0 (the caller checks).
// Returns CEK_ERR_UNSUPPORTED for shapes it leaves to the tiled GEMM.
int launch_gemv_a8w8(const uint8_t* x, const float* xs, const uint8_t* w, const float* ws, void* y,
                     int64_t M, int64_t N, int64_t K, int out_dtype, hipStream_t st) {
  if (M < 1 || M > 64 || N < 1 || N > INT32_MAX || K > INT32_MAX) return CEK_ERR_UNSUPPORTED;
  GemvSegs sg{};
  sg.count = 1;
  sg.w[0] = w;
  sg.s[0] = ws;
  sg.y[0] = static_cast<uint16_t*>(y);
  sg.n[0] = (int)N;
  sg.xs = xs;
  // 17 <= M <= 32 with K of 2, 3 or 4 KiB values and at least 384 16-row
  // tiles: gemv_xres8_kernel, 2 tiles x 4 K parts per workgroup, one slot per
  // workgroup as far as 256 workgroups go; K = 5120 (160 KB of activations)
  // only where one round of slots covers the tiles (384 to 512 tiles).  Where
  // a workgroup has one slot (up to 512 tiles) only from 24 rows on: its
  // activation load is not amortised, and below that the other kernel's
  // repeated rows cost little (K = 5120, N = 8000: M = 17 12.04 -> 13.23 us,
  // M = 24, N = 6144 13.37 -> 12.28, M = 32 15.12 -> 12.38).
  const int tiles16 = (int)((N + 15) / 16);
  const int m_min = tiles16 <= 512 ? 24 : 17;
  // 12-row tiles (RT = 12) where they cut the busiest CU's rows by a fifth
  // or more (N ~ 6144: 256 slots of 2 x 12 rows against 192 of 2 x 16; the
  // outputs do not change).  Measured on MI355X, weights from HBM: M = 32,
  // N = 6144, K = 4096 10.29 -> 9.89 us, K = 5120 12.36 -> 11.87 us; M = 24
  // 10.17 -> 9.78 and 12.20 -> 11.69 us.
  auto busiest_rows = [&](int rt) {
    const int ns = ((int)((N + rt - 1) / rt) + 1) / 2;
    return 2 * rt * ((ns + kCUs - 1) / kCUs);
  };
  const bool x12 = 5 * busiest_rows(12) <= 4 * busiest_rows(16);
  // With 12-row tiles the kernel also takes N from 384 12-row tiles (4608)
  // up: M = 32, K = 4096, N = 4608 / 5120 / 6100 12.13 / 12.25 / 12.53 ->
  // 8.92 / 9.20 / 9.91 us against the LDS kernel; K = 5120 14.81 / 14.87 /
  // 15.05 -> 10.56 / 10.85 / 11.80 us; M = 24, N = 5120 10.77 -> 9.21 us.
  const int tiles12 = (int)((N + 11) / 12);
  const bool wide = tiles16 >= 384 || (x12 && tiles12 >= 384);
  if (M >= m_min && M <= 32 && K == 5120 && wide && (tiles16 <= 512 || (x12 && tiles12 <= 512))) {
    // (RT = 12 only where one round of slots still covers its tiles)
    const bool r12 = x12 && (((int)((N + 11) / 12) + 1) / 2 <= kCUs);
    const int tiles = seg_grid(sg, r12 ? 12 : 16);
    const int nslot = (tiles + 1) / 2;
    const int m = (int)M;
#define CEK_X8ONE(TY, RTT) gemv_xres8_kernel<TY, 5120, 2, 4, 5, true, RTT><<<nslot, 512, 0, st>>>(x, sg, m, tiles)
    if (out_dtype == CEK_F16) {
      if (r12) CEK_X8ONE(F16, 12);
      else CEK_X8ONE(F16, 16);
    } else {
      if (r12) CEK_X8ONE(BF16, 12);
      else CEK_X8ONE(BF16, 16);
    }
#undef CEK_X8ONE
    return check_launch();
  }
  if (M >= m_min && M <= 32 && (K == 2048 || K == 3072 || K == 4096) && wide) {
    const int tiles = seg_grid(sg, x12 ? 12 : 16);
    const int nslot = (tiles + 1) / 2;
    const dim3 grid((unsigned)(nslot < kCUs ? nslot : kCUs));
    const int m = (int)M;
#define CEK_X8R(KK, PP, RTT)                                                                                         \
  do {                                                                                                               \
    if (out_dtype == CEK_F16) gemv_xres8_kernel<F16, KK, 2, 4, PP, false, RTT><<<grid, 512, 0, st>>>(x, sg, m, tiles); \
    else gemv_xres8_kernel<BF16, KK, 2, 4, PP, false, RTT><<<grid, 512, 0, st>>>(x, sg, m, tiles);                     \
  } while (0)
#define CEK_X8(KK, PP)               \
  do {                               \
    if (x12) CEK_X8R(KK, PP, 12);    \
    else CEK_X8R(KK, PP, 16);        \
  } while (0)
    if (K == 2048) CEK_X8(2048, 4);
    else if (K == 3072) CEK_X8(3072, 6);
    else CEK_X8(4096, 4);
#undef CEK_X8
#undef CEK_X8R
    return check_launch();
  }
  if (M > 16) {  // only the LDS path takes these
    const bool ok = out_dtype == CEK_F16 ? launch_lds<F16, F16, CEK_E4M3, true>(x, sg, SK_F32, (int)M, (int)K, (int)N, st)
                                         : launch_lds<F16, BF16, CEK_E4M3, true>(x, sg, SK_F32, (int)M, (int)K, (int)N, st);
    return ok ? check_launch() : CEK_ERR_UNSUPPORTED;
  }
  if (out_dtype == CEK_F16) return launch_gemv_t<F16, F16, CEK_E4M3, true>(x, sg, SK_F32, (int)M, (int)K, true, st);
  return launch_gemv_t<F16, BF16, CEK_E4M3, true>(x, sg, SK_F32, (int)M, (int)K, true, st);
}

int launch_gemv(const void* x, const void* w, const void* scale, int skind, void* y,
                int64_t M, int64_t N, int64_t K, int io_dtype, int fp8_fmt, hipStream_t st) {
  if (N < 0) return CEK_ERR_INVALID;
  if (M < 0 || M > 16) return CEK_ERR_INVALID;
  if (M == 0 || N == 0) return K > 0 ? CEK_OK : CEK_ERR_INVALID;
  return launch_gemv_segs(x, 1, &w, &scale, &y, &N, M, K, skind, io_dtype, fp8_fmt, st);
}

// 16 < M <= 32 (GEMM entry point): the LDS path when it covers the shape.
int launch_gemv_wide(const void* x, const void* w, const void* scale, int skind, void* y,
                     int64_t M, int64_t N, int64_t K, int io_dtype, int fp8_fmt, hipStream_t st) {
  if (M <= 16 || M > 32 || N <= 0) return CEK_ERR_UNSUPPORTED;
  return launch_gemv_segs(x, 1, &w, &scale, &y, &N, M, K, skind, io_dtype, fp8_fmt, st, 32);
}

// Generic path for any M (used by the GEMM entry point for odd shapes).
int launch_gemv_generic(const void* x, const void* w, const void* scale, int skind, void* y,
                        int64_t M, int64_t N, int64_t K, int io_dtype, int fp8_fmt, hipStream_t st) {
  GemvSegs sg{};
  sg.count = 1;
  sg.w[0] = static_cast<const uint8_t*>(w);
  sg.s[0] = scale;
  sg.y[0] = static_cast<uint16_t*>(y);
  sg.n[0] = (int)N;
  dim3 grid((unsigned)seg_grid(sg, 4));
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  if (io_dtype == CEK_F16 && fp8_fmt == CEK_E4M3) gemv_generic_kernel<F16, CEK_E4M3><<<grid, 256, 0, st>>>(xp, sg, skind, M, K);
  else if (io_dtype == CEK_F16 && fp8_fmt == CEK_E5M2) gemv_generic_kernel<F16, CEK_E5M2><<<grid, 256, 0, st>>>(xp, sg, skind, M, K);
  else if (io_dtype == CEK_BF16 && fp8_fmt == CEK_E4M3) gemv_generic_kernel<BF16, CEK_E4M3><<<grid, 256, 0, st>>>(xp, sg, skind, M, K);
  else if (io_dtype == CEK_BF16 && fp8_fmt == CEK_E5M2) gemv_generic_kernel<BF16, CEK_E5M2><<<grid, 256, 0, st>>>(xp, sg, skind, M, K);
  else return CEK_ERR_INVALID;
  return check_launch();
}

static int scale_kind(int scale_dtype) {
  if (scale_dtype == CEK_F16) return SK_F16;
  if (scale_dtype == CEK_BF16) return SK_BF16;
  if (scale_dtype == CEK_F32) return SK_F32;
  return -1;
}

// y[m, i] = gelu_tanh(g[m, i]) * u[m, i] with g = GEMV over weight rows
// [0, d), u over rows [d, 2 d), both rounded to the output type first.
// xs == null: x is io_dtype [M, K]; else x holds e4m3 codes [M, K] with
// per-row fp32 scales xs (the a8w8 contract: e4m3 weights, fp32 scales).
int launch_gemv_glu(const void* x, const float* xs, const void* w, const void* scale, int skind, void* y,
                    int64_t M, int64_t d, int64_t K, int io_dtype, int fp8_fmt, hipStream_t st,
                    const NormArgs* rs = nullptr) {
  if (M < 0 || d < 0 || K <= 0 || d > INT32_MAX / 2 || K > INT32_MAX) return CEK_ERR_INVALID;
  if (io_dtype != CEK_F16 && io_dtype != CEK_BF16) return CEK_ERR_INVALID;
  if (fp8_fmt != CEK_E4M3 && fp8_fmt != CEK_E5M2) return CEK_ERR_INVALID;
  if (skind < 0 || skind == SK_F32_SCALAR) return CEK_ERR_INVALID;
  if (xs && (fp8_fmt != CEK_E4M3 || skind != SK_F32)) return CEK_ERR_INVALID;
  if (M == 0 || d == 0) return CEK_OK;
  if (!x || !w || !scale || !y) return CEK_ERR_INVALID;
  if (2 * d * K > ((int64_t)1 << 40)) return CEK_ERR_INVALID;
  // The fused kernel: up to 16 rows, K of 3, 4 or 5 KiB values, 16-byte
  // aligned operands; other requests are left to GEMV + gelu_and_mul.
  if (M > 16 || K % 1024 != 0 || K < 3072 || K > 5120 || !aligned(x, 16) || !aligned(w, 16))
    return CEK_ERR_UNSUPPORTED;
  if (rs && (xs || M > 4 || fp8_fmt != CEK_E4M3)) return CEK_ERR_UNSUPPORTED;
  GemvSegs sg{};
  sg.count = 1;
  sg.w[0] = static_cast<const uint8_t*>(w);
  sg.s[0] = scale;
  sg.y[0] = static_cast<uint16_t*>(y);
  sg.n[0] = (int)(2 * d);
  sg.xs = xs;
  const int m = (int)M, dd = (int)d, k = (int)K;
  if (rs) {
    if (io_dtype == CEK_F16) return launch_glu<F16, F16, CEK_E4M3, false>(x, sg, skind, m, dd, k, st, rs);
    return launch_glu<BF16, BF16, CEK_E4M3, false>(x, sg, skind, m, dd, k, st, rs);
  }
  if (xs) {
    if (io_dtype == CEK_F16) return launch_glu<F16, F16, CEK_E4M3, true>(x, sg, SK_F32, m, dd, k, st);
    return launch_glu<F16, BF16, CEK_E4M3, true>(x, sg, SK_F32, m, dd, k, st);
  }
  if (io_dtype == CEK_F16 && fp8_fmt == CEK_E4M3) return launch_glu<F16, F16, CEK_E4M3, false>(x, sg, skind, m, dd, k, st);
  if (io_dtype == CEK_F16) return launch_glu<F16, F16, CEK_E5M2, false>(x, sg, skind, m, dd, k, st);
  if (fp8_fmt == CEK_E4M3) return launch_glu<BF16, BF16, CEK_E4M3, false>(x, sg, skind, m, dd, k, st);
  return launch_glu<BF16, BF16, CEK_E5M2, false>(x, sg, skind, m, dd, k, st);
}

// GEMV with a fused epilogue (gemv_lds_kernel's TAIL forms): one 16-row
// tile per workgroup, activations staged through LDS (M <= 4), prefetch
// depth 3, e4m3 weights, K in {3, 4, 5} KiB values; tp = L (ROPE, head dim
// 128 or 256).  CEK_ERR_UNSUPPORTED for
// other shapes (the caller runs the GEMV, then the op).
template <typename T, int TAIL, int TP, int EPI = EPI_NONE>
static void launch_tail_t(const void* x, GemvSegs& sg, int skind, int M, int K, const NormArgs& na, hipStream_t st) {
  const dim3 grid((unsigned)seg_grid(sg, 16));
#define CEK_TAIL(S)                                                                                       \
  gemv_lds_kernel<T, T, CEK_E4M3, false, 1, 1, 3, S, 4, 1, false, false, TAIL, TP, true, EPI><<<grid, 256, 0, st>>>( \
      x, sg, skind, M, na)
  if (K == 3072) CEK_TAIL(3);
  else if (K == 4096) CEK_TAIL(4);
  else CEK_TAIL(5);
#undef CEK_TAIL
}

int launch_gemv_tail(const void* x, const void* w, const void* scale, int skind, void* y, int64_t M, int64_t N,
                     int64_t K, int io_dtype, int fp8_fmt, int tail, int tp, const NormArgs& na, hipStream_t st) {
  if (M < 0 || N < 0 || K <= 0 || N > INT32_MAX || K > INT32_MAX) return CEK_ERR_INVALID;
  if (io_dtype != CEK_F16 && io_dtype != CEK_BF16) return CEK_ERR_INVALID;
  if (fp8_fmt != CEK_E4M3 && fp8_fmt != CEK_E5M2) return CEK_ERR_INVALID;
  if (skind < 0 || skind == SK_F32_SCALAR) return CEK_ERR_INVALID;
  if (M == 0 || N == 0) return CEK_OK;
  if (!x || !w || !scale || !y || !na.tail.counters) return CEK_ERR_INVALID;
  if (N * K > ((int64_t)1 << 40)) return CEK_ERR_INVALID;
  if (M > 4 || (K != 3072 && K != 4096 && K != 5120) || fp8_fmt != CEK_E4M3 || N % 16 != 0) return CEK_ERR_UNSUPPORTED;
  if (!aligned(x, 16) || !aligned(w, 16) || !aligned(y, 16)) return CEK_ERR_UNSUPPORTED;
  // the output is re-read by the tail: it must not share memory with the
  // inputs, nor with the q copy that other heads' tails write meanwhile;
  // every workgroup reads the weight scale, the q / k norm weights, the
  // positions and (deferred norm) the partial sums while others write the
  // output and the q copy
  {
    const int64_t hd = 16 * (int64_t)tp;
    const int64_t scb = N * (skind == SK_F32 ? 4 : 2);
    const int64_t qb = na.tail.qcopy ? M * na.tail.nq * hd * 2 : 0;
    const std::pair<const void*, int64_t> ins[] = {
        {x, M * K * 2}, {w, N * K}, {scale, scb}, {na.tail.qw, na.tail.nq > 0 ? hd * 2 : 0},
        {na.tail.kw, na.tail.nk > 0 ? hd * 2 : 0}, {na.tail.pos, M * 8}, {na.ss_in, na.ss_in ? M * na.nss * 4 : 0}};
    for (const auto& [p, b] : ins)
      if (overlaps(y, M * N * 2, p, b) || (qb && overlaps(na.tail.qcopy, qb, p, b))) return CEK_ERR_UNSUPPORTED;
    if (qb && overlaps(na.tail.qcopy, qb, y, M * N * 2)) return CEK_ERR_UNSUPPORTED;
  }
  GemvSegs sg{};
  sg.count = 1;
  sg.w[0] = static_cast<const uint8_t*>(w);
  sg.s[0] = scale;
  sg.y[0] = static_cast<uint16_t*>(y);
  sg.n[0] = (int)N;
  const int m = (int)M, k = (int)K;
  const bool f16 = io_dtype == CEK_F16;
  (void)tail;
  if (na.ss_in) {  // deferred RMSNorm consumer
    if (tp == 8) {
      if (f16) launch_tail_t<F16, TAIL_ROPE, 8, EPI_ROWSCALE>(x, sg, skind, m, k, na, st);
      else launch_tail_t<BF16, TAIL_ROPE, 8, EPI_ROWSCALE>(x, sg, skind, m, k, na, st);
    } else {
      if (f16) launch_tail_t<F16, TAIL_ROPE, 16, EPI_ROWSCALE>(x, sg, skind, m, k, na, st);
      else launch_tail_t<BF16, TAIL_ROPE, 16, EPI_ROWSCALE>(x, sg, skind, m, k, na, st);
    }
    return check_launch();
  }
  if (tp == 8) { if (f16) launch_tail_t<F16, TAIL_ROPE, 8>(x, sg, skind, m, k, na, st); else launch_tail_t<BF16, TAIL_ROPE, 8>(x, sg, skind, m, k, na, st); }
  else { if (f16) launch_tail_t<F16, TAIL_ROPE, 16>(x, sg, skind, m, k, na, st); else launch_tail_t<BF16, TAIL_ROPE, 16>(x, sg, skind, m, k, na, st); }
  return check_launch();
}

// Deferred RMSNorm producer (EPI_ADDNORM, EPI_ADDNORM12) and plain consumer
// (EPI_ROWSCALE): M <= 4 rows staged through LDS, one 16-row (12-row) tile
// per workgroup, rotated K order, e4m3 weights, K in {2, 3, 4, 5, 14, 24}
// KiB values.
template <typename T, int EPI, int S>
static void launch_defer_t(const void* x, GemvSegs& sg, int skind, int M, const NormArgs& na, hipStream_t st) {
  gemv_lds_kernel<T, T, CEK_E4M3, false, 1, 1, (S >= 3 ? 3 : 2), S, 4, 1, false, false, TAIL_NONE, 0, true, EPI>
      <<<dim3(seg_grid(sg, EPI == EPI_ADDNORM12 ? 12 : 16)), 256, 0, st>>>(x, sg, skind, M, na);
}

// Rows per producer tile for N (a multiple of 16): 12 where the 16-row tiles
// would leave CUs idle (fewer than 256 of them) and N / 12 is a valid
// partial-sum count for the consumers (a multiple of 4, at most 256), else
// 16.  M = 4, K = 24576, N = 3072: 16.5 us with 192 16-row tiles, against
// 18.4 us for 256 tiles at N = 4096 (a third more bytes).
static int defer_rows(int64_t N) { return N % 48 == 0 && N / 16 < 256 && N / 12 <= 256 ? 12 : 16; }

template <typename T, int EPI>
static bool launch_defer_k(const void* x, GemvSegs& sg, int skind, int M, int K, const NormArgs& na, hipStream_t st) {
  switch (K >> 10) {
    case 2: launch_defer_t<T, EPI, 2>(x, sg, skind, M, na, st); return true;
    case 3: launch_defer_t<T, EPI, 3>(x, sg, skind, M, na, st); return true;
    case 4: launch_defer_t<T, EPI, 4>(x, sg, skind, M, na, st); return true;
    case 5: launch_defer_t<T, EPI, 5>(x, sg, skind, M, na, st); return true;
    case 14: launch_defer_t<T, EPI, 14>(x, sg, skind, M, na, st); return true;
    case 24: launch_defer_t<T, EPI, 24>(x, sg, skind, M, na, st); return true;
    default: return false;
  }
}

// Common checks of the deferred-norm launches; CEK_OK to go on, else the status.
static int defer_checks(const void* x, const void* w, const void* scale, int skind, void* y, int64_t M, int64_t N,
                        int64_t K, int io_dtype, int fp8_fmt) {
  if (M < 0 || N < 0 || K <= 0 || N > INT32_MAX || K > INT32_MAX) return CEK_ERR_INVALID;
  if (io_dtype != CEK_F16 && io_dtype != CEK_BF16) return CEK_ERR_INVALID;
  if (fp8_fmt != CEK_E4M3 && fp8_fmt != CEK_E5M2) return CEK_ERR_INVALID;
  if (skind < 0) return CEK_ERR_INVALID;
  if (M == 0 || N == 0) return CEK_OK;
  if (!x || !w || !scale || !y) return CEK_ERR_INVALID;
  if (N * K > ((int64_t)1 << 40)) return CEK_ERR_INVALID;
  if (M > 4 || K % 1024 != 0 || fp8_fmt != CEK_E4M3 || N % 16 != 0 || !aligned(x, 16) || !aligned(w, 16))
    return CEK_ERR_UNSUPPORTED;
  return CEK_OK;
}

int launch_gemv_addnorm(const void* x, const void* w, const void* scale, int skind, void* residual,
                        const void* norm_weight, void* y, float* ss_out, int norm_shift, int64_t M, int64_t N,
                        int64_t K, int io_dtype, int fp8_fmt, hipStream_t st) {
  if (norm_shift < -24 || norm_shift > 24) return CEK_ERR_INVALID;
  const int rc = defer_checks(x, w, scale, skind, y, M, N, K, io_dtype, fp8_fmt);
  if (rc != CEK_OK || M == 0 || N == 0) return rc;
  if (!residual || !norm_weight || !ss_out) return CEK_ERR_INVALID;
  // other workgroups still read x, w, the weight scale and the norm weight
  // while one writes y, the residual and the partial sums
  const int rows = defer_rows(N);
  const int64_t yb = M * N * 2, sb = M * (N / rows) * 4;
  const int64_t scb = skind == SK_F32_SCALAR ? 4 : N * (skind == SK_F32 ? 4 : 2);
  for (const auto& [p, b] : {std::pair<const void*, int64_t>{y, yb}, {residual, yb}, {ss_out, sb}})
    if (overlaps(p, b, x, M * K * 2) || overlaps(p, b, w, N * K) || overlaps(p, b, scale, scb) ||
        overlaps(p, b, norm_weight, N * 2))
      return CEK_ERR_UNSUPPORTED;
  if (overlaps(y, yb, residual, yb) || overlaps(ss_out, sb, y, yb) || overlaps(ss_out, sb, residual, yb))
    return CEK_ERR_UNSUPPORTED;
  GemvSegs sg{};
  sg.count = 1;
  sg.w[0] = static_cast<const uint8_t*>(w);
  sg.s[0] = scale;
  sg.y[0] = static_cast<uint16_t*>(y);
  sg.n[0] = (int)N;
  NormArgs na{};
  na.r_out = static_cast<uint16_t*>(residual);
  na.w = static_cast<const uint16_t*>(norm_weight);
  na.ss_out = ss_out;
  na.yscale = ldexpf(1.f, -norm_shift);
  const bool f16 = io_dtype == CEK_F16;
  const bool ok = rows == 12 ? (f16 ? launch_defer_k<F16, EPI_ADDNORM12>(x, sg, skind, (int)M, (int)K, na, st)
                                    : launch_defer_k<BF16, EPI_ADDNORM12>(x, sg, skind, (int)M, (int)K, na, st))
                             : (f16 ? launch_defer_k<F16, EPI_ADDNORM>(x, sg, skind, (int)M, (int)K, na, st)
                                    : launch_defer_k<BF16, EPI_ADDNORM>(x, sg, skind, (int)M, (int)K, na, st));
  return ok ? check_launch() : CEK_ERR_UNSUPPORTED;
}

int64_t defer_groups(int64_t N) { return N > 0 && N % 16 == 0 ? N / defer_rows(N) : 0; }

// The row-scale arguments of the deferred-norm consumers; CEK_OK or the status.
static int rowscale_args(const float* row_ss, int64_t n_ss, float row_eps, int64_t M, NormArgs& na) {
  if (M == 0) return CEK_OK;
  if (!row_ss || n_ss < 1) return CEK_ERR_INVALID;
  if (n_ss > 256 || n_ss % 4 != 0 || !aligned(row_ss, 16)) return CEK_ERR_UNSUPPORTED;
  na.ss_in = row_ss;
  na.nss = (int)n_ss;
  na.eps = row_eps;
  return CEK_OK;
}

int launch_gemv_rowscale(const void* x, const void* w, const void* scale, int skind, void* y, const float* row_ss,
                         int64_t n_ss, float row_eps, int64_t M, int64_t N, int64_t K, int io_dtype, int fp8_fmt,
                         hipStream_t st) {
  const int rc = defer_checks(x, w, scale, skind, y, M, N, K, io_dtype, fp8_fmt);
  if (rc != CEK_OK || M == 0 || N == 0) return rc;
  NormArgs na{};
  const int rc2 = rowscale_args(row_ss, n_ss, row_eps, M, na);
  if (rc2 != CEK_OK) return rc2;
  GemvSegs sg{};
  sg.count = 1;
  sg.w[0] = static_cast<const uint8_t*>(w);
  sg.s[0] = scale;
  sg.y[0] = static_cast<uint16_t*>(y);
  sg.n[0] = (int)N;
  const bool ok = io_dtype == CEK_F16 ? launch_defer_k<F16, EPI_ROWSCALE>(x, sg, skind, (int)M, (int)K, na, st)
                                      : launch_defer_k<BF16, EPI_ROWSCALE>(x, sg, skind, (int)M, (int)K, na, st);
  return ok ? check_launch() : CEK_ERR_UNSUPPORTED;
}

}  // namespace cek

extern "C" int64_t cek_gemv_fp8_add_rms_norm_defer_groups(int64_t N) { return cek::defer_groups(N); }

extern "C" int cek_defer_norm_shift(float max_abs_norm_weight) {
  const float m = fabsf(max_abs_norm_weight);
  if (!(m > 0.f)) return 0;  // zero or NaN
  if (m > 0x1p24f) return 24;
  int e;
  const float f = frexpf(m, &e);  // m = f 2^e, f in [0.5, 1): 2^e > m >= 2^(e-1)
  const int s = f == 0.5f ? e - 1 : e;
  return s < -24 ? -24 : s;
}

extern "C" int cek_gemv_fp8_add_rms_norm_defer(const void* x, const void* w, const void* scale, void* residual,
                                               const void* norm_weight, void* y, float* ss_out, int norm_shift,
                                               int64_t M, int64_t N, int64_t K, int io_dtype, int fp8_fmt,
                                               int scale_dtype, void* stream) {
  return cek::launch_gemv_addnorm(x, w, scale, cek::scale_kind(scale_dtype), residual, norm_weight, y, ss_out,
                                  norm_shift, M, N, K, io_dtype, fp8_fmt, (hipStream_t)stream);
}

extern "C" int cek_gemv_fp8_pern_rs(const void* x, const void* w, const void* scale, void* y, const float* row_ss,
                                    int64_t n_ss, float row_eps, int64_t M, int64_t N, int64_t K, int io_dtype,
                                    int fp8_fmt, int scale_dtype, void* stream) {
  return cek::launch_gemv_rowscale(x, w, scale, cek::scale_kind(scale_dtype), y, row_ss, n_ss, row_eps, M, N, K,
                                   io_dtype, fp8_fmt, (hipStream_t)stream);
}

extern "C" int cek_gemv_fp8_gelu_and_mul_rs(const void* x, const void* w, const void* scale, void* y,
                                            const float* row_ss, int64_t n_ss, float row_eps, int64_t M, int64_t d,
                                            int64_t K, int io_dtype, int fp8_fmt, int scale_dtype, void* stream) {
  cek::NormArgs na{};
  const int rc = cek::rowscale_args(row_ss, n_ss, row_eps, M, na);
  if (rc != CEK_OK) return rc;
  if (M > 4) return CEK_ERR_UNSUPPORTED;
  return cek::launch_gemv_glu(x, nullptr, w, scale, cek::scale_kind(scale_dtype), y, M, d, K, io_dtype, fp8_fmt,
                              (hipStream_t)stream, M == 0 ? nullptr : &na);
}

namespace cek {
// The checks and tail arguments shared by the two QKV + q/k-norm + rope entry
// points; CEK_OK when the launch may go ahead with na.
static int qk_rope_args(const void* q_weight, const void* k_weight, const int64_t* positions, int64_t n_q,
                        int64_t n_k, int64_t head_dim, float eps, float theta, int is_neox, int* counters,
                        void* q_out, int64_t M, int64_t N, NormArgs& na) {
  if (M < 0 || N < 0 || n_q < 0 || n_k < 0 || head_dim <= 0 || !(theta > 0.f)) return CEK_ERR_INVALID;
  if ((n_q + n_k) * head_dim > N) return CEK_ERR_INVALID;
  if (M > 0 && N > 0 && (!positions || (n_q > 0 && !q_weight) || (n_k > 0 && !k_weight))) return CEK_ERR_INVALID;
  if (head_dim != 128 && head_dim != 256) return M == 0 || N == 0 ? CEK_OK : CEK_ERR_UNSUPPORTED;
  if (N % 8 != 0 || (n_q > 0 && !aligned(q_weight, 16)) || (n_k > 0 && !aligned(k_weight, 16)))
    return M == 0 || N == 0 ? CEK_OK : CEK_ERR_UNSUPPORTED;
  na.tail.counters = counters;
  na.tail.qw = static_cast<const uint16_t*>(q_weight);
  na.tail.kw = static_cast<const uint16_t*>(k_weight);
  na.tail.pos = positions;
  na.tail.nq = (int)n_q;
  na.tail.nk = (int)n_k;
  na.tail.eps = eps;
  na.tail.theta = theta;
  na.tail.neox = is_neox != 0;
  if (q_out && n_q > 0 && M > 0) {
    if (!aligned(q_out, 16)) return CEK_ERR_UNSUPPORTED;
    na.tail.qcopy = static_cast<uint16_t*>(q_out);
  }
  return CEK_OK;
}
}  // namespace cek

extern "C" int cek_gemv_fp8_qk_norm_rope(const void* x, const void* w, const void* scale, void* y,
                                         const void* q_weight, const void* k_weight, const int64_t* positions,
                                         int64_t n_q, int64_t n_k, int64_t head_dim, float eps, float theta,
                                         int is_neox, int* counters, void* q_out, int64_t M, int64_t N, int64_t K,
                                         int io_dtype, int fp8_fmt, int scale_dtype, void* stream) {
  cek::NormArgs na{};
  const int rc = cek::qk_rope_args(q_weight, k_weight, positions, n_q, n_k, head_dim, eps, theta, is_neox, counters,
                                   q_out, M, N, na);
  if (rc != CEK_OK || (head_dim != 128 && head_dim != 256)) return rc;
  return cek::launch_gemv_tail(x, w, scale, cek::scale_kind(scale_dtype), y, M, N, K, io_dtype, fp8_fmt,
                               cek::TAIL_ROPE, (int)(head_dim / 16), na, (hipStream_t)stream);
}

extern "C" int cek_gemv_fp8_qk_norm_rope_rs(const void* x, const void* w, const void* scale, void* y,
                                            const void* q_weight, const void* k_weight, const int64_t* positions,
                                            int64_t n_q, int64_t n_k, int64_t head_dim, float eps, float theta,
                                            int is_neox, int* counters, void* q_out, const float* row_ss,
                                            int64_t n_ss, float row_eps, int64_t M, int64_t N, int64_t K,
                                            int io_dtype, int fp8_fmt, int scale_dtype, void* stream) {
  cek::NormArgs na{};
  int rc = cek::qk_rope_args(q_weight, k_weight, positions, n_q, n_k, head_dim, eps, theta, is_neox, counters, q_out,
                             M, N, na);
  if (rc != CEK_OK || (head_dim != 128 && head_dim != 256)) return rc;
  if (M == 0 || N == 0) return CEK_OK;
  rc = cek::rowscale_args(row_ss, n_ss, row_eps, M, na);
  if (rc != CEK_OK) return rc;
  return cek::launch_gemv_tail(x, w, scale, cek::scale_kind(scale_dtype), y, M, N, K, io_dtype, fp8_fmt,
                               cek::TAIL_ROPE, (int)(head_dim / 16), na, (hipStream_t)stream);
}

extern "C" int cek_add_rms_norm_gemv_fp8(const void* hidden, const void* residual, const void* norm_weight, float eps,
                                         void* residual_out, void* hidden_out, uint8_t* q_out, float* q_scale,
                                         const void* w, const void* scale, void* y, int64_t M, int64_t N, int64_t K,
                                         int gelu_and_mul, int io_dtype, int fp8_fmt, int scale_dtype, void* stream) {
  cek::NormArgs na{static_cast<const uint16_t*>(hidden), static_cast<const uint16_t*>(residual),
                   static_cast<const uint16_t*>(norm_weight), static_cast<uint16_t*>(residual_out),
                   static_cast<uint16_t*>(hidden_out), q_out, q_scale, eps};
  return cek::launch_norm_gemv(na, w, scale, cek::scale_kind(scale_dtype), y, M, N, K, gelu_and_mul != 0, io_dtype,
                               fp8_fmt, (hipStream_t)stream);
}

extern "C" int cek_gemv_fp8_gelu_and_mul(const void* x, const float* x_scale, const void* w, const void* scale,
                                         void* y, int64_t M, int64_t d, int64_t K, int io_dtype, int fp8_fmt,
                                         int scale_dtype, void* stream) {
  return cek::launch_gemv_glu(x, x_scale, w, scale, cek::scale_kind(scale_dtype), y, M, d, K, io_dtype, fp8_fmt,
                              (hipStream_t)stream);
}

// More than 16 rows: the w8a16 GEMM dispatch (cek_gemm.hip), which streams
// the weights once for all rows instead of once per 16-row slab.
extern "C" int cek_gemv_fp8_pern(const void* x, const void* w, const void* scale, void* y,
                                 int64_t M, int64_t N, int64_t K,
                                 int io_dtype, int fp8_fmt, int scale_dtype, void* stream) {
  const int skind = cek::scale_kind(scale_dtype);
  if (skind < 0) return CEK_ERR_INVALID;
  if (M > 16) return cek::launch_w8a16(x, w, scale, skind, y, M, N, K, io_dtype, fp8_fmt, nullptr, 0, (hipStream_t)stream);
  return cek::launch_gemv(x, w, scale, skind, y, M, N, K, io_dtype, fp8_fmt, (hipStream_t)stream);
}

extern "C" int cek_gemv_fp8_pert(const void* x, const void* w, const float* scale, void* y,
                                 int64_t M, int64_t N, int64_t K,
                                 int io_dtype, int fp8_fmt, void* stream) {
  if (M > 16)
    return cek::launch_w8a16(x, w, scale, cek::SK_F32_SCALAR, y, M, N, K, io_dtype, fp8_fmt, nullptr, 0,
                             (hipStream_t)stream);
  return cek::launch_gemv(x, w, scale, cek::SK_F32_SCALAR, y, M, N, K, io_dtype, fp8_fmt, (hipStream_t)stream);
}

extern "C" int cek_gemv_fp8_pern_multi(const void* x, int count, const void* const* w,
                                       const void* const* scale, void* const* y, const int64_t* N,
                                       int64_t M, int64_t K, int io_dtype, int fp8_fmt, int scale_dtype,
                                       void* stream) {
  const int skind = cek::scale_kind(scale_dtype);
  if (skind < 0) return CEK_ERR_INVALID;
  return cek::launch_gemv_segs(x, count, w, scale, y, N, M, K, skind, io_dtype, fp8_fmt, (hipStream_t)stream);
}

extern "C" int cek_gemv_fp8_pert_multi(const void* x, int count, const void* const* w,
                                       const float* const* scale, void* const* y, const int64_t* N,
                                       int64_t M, int64_t K, int io_dtype, int fp8_fmt, void* stream) {
  return cek::launch_gemv_segs(x, count, w, reinterpret_cast<const void* const*>(scale), y, N, M, K,
                               cek::SK_F32_SCALAR, io_dtype, fp8_fmt, (hipStream_t)stream);
}
