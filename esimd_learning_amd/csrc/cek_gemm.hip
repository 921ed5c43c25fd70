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
#include <atomic>
#include <mutex>

#include "cek_common.h"

namespace cek {

int launch_gemv(const void* x, const void* w, const void* scale, int skind, void* y,
                int64_t M, int64_t N, int64_t K, int io_dtype, int fp8_fmt, hipStream_t st);
int launch_gemv_generic(const void* x, const void* w, const void* scale, int skind, void* y,
                        int64_t M, int64_t N, int64_t K, int io_dtype, int fp8_fmt, hipStream_t st);
int launch_gemv_a8w8(const uint8_t* x, const float* xs, const uint8_t* w, const float* ws, void* y,
                     int64_t M, int64_t N, int64_t K, int out_dtype, hipStream_t st);
int launch_gemv_wide(const void* x, const void* w, const void* scale, int skind, void* y,
                     int64_t M, int64_t N, int64_t K, int io_dtype, int fp8_fmt, hipStream_t st);

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
// a8w8, LDS-tiled: block tile BM x BN, K step 128, four waves in a WM x WN
// grid (wave tile (BM/WM) x (BN/WN), i.e. FM x FN MFMA blocks of 16 x 16).
//
// The A and B K-slices are staged row-major in LDS (128 bytes per row, eight
// 16-byte chunks), double-buffered, by direct-to-LDS loads
// (global_load_lds_dwordx4: one instruction moves 1 KB = 8 full rows; lane
// i's 16 bytes land at LDS + 16 i).  Chunk c of row r is stored at position
// c ^ s(r).  An operand fragment gives lane l row (l & 15) and two chunks
// (LAYOUT 0: 2g and 2g+1; LAYOUT 1: g and g+4; g = l >> 4) -- the same K
// positions for A and B, so any assignment sums the right products.  The
// swizzles s(r) = (r ^ ((r >> 3) & 1)) & 7 (LAYOUT 0) and r & 7 (LAYOUT 1) make
// each 16-lane group of such a ds_read_b128 hit distinct banks (measured
// with SQ_LDS_BANK_CONFLICT on MI355X).
// The stage written during step k+1 was last read in step k-1; the barrier
// at the top of each step (which also drains this wave's outstanding loads)
// separates the two.  Tiles are numbered so that consecutive workgroups on
// one XCD (workgroup i runs on XCD i % 8) share A rows and B columns in that
// XCD's L2.  Requires K % 128 == 0 and 16-byte aligned A and B.
// ---------------------------------------------------------------------------
template <int LAYOUT>
__device__ inline int swz(int row) { return LAYOUT == 0 ? ((row ^ ((row >> 3) & 1)) & 7) : (row & 7); }

template <int BM, int BN, int GROUP_M>
__device__ inline void tile_of(int b, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int T = tiles_m * tiles_n;
  int t = b;
  if ((T & 7) == 0) t = (b & 7) * (T >> 3) + (b >> 3);  // XCD-contiguous numbering
  const int per_group = GROUP_M * tiles_n;
  const int group = t / per_group;
  const int first_m = group * GROUP_M;
  const int gsize = min(tiles_m - first_m, GROUP_M);
  const int tin = t - group * per_group;
  tm = first_m + tin % gsize;
  tn = tin / gsize;
}

// Direct-to-LDS loads of one K step (128 bytes) of the A and B slices into a
// stage: this wave's 1 KB writer chunks j = wave + 4 i (rows 8 j .. 8 j + 7).
template <int BM, int BN, int ACH, int BCH, int NW = 4>
__device__ inline void a8w8_issue(uint8_t* smem, int stage, int kb, int wave,
                                  const uint8_t* const (&ga)[ACH], const uint8_t* const (&gb)[BCH]) {
#if defined(__HIP_DEVICE_COMPILE__)  // device-only builtin; the host pass only needs the kernel's stub
  uint8_t* sA = smem + stage * (BM + BN) * 128;
  uint8_t* sB = sA + BM * 128;
#pragma unroll
  for (int i = 0; i < ACH; ++i)
    __builtin_amdgcn_global_load_lds(ga[i] + kb, (lds_ptr_t)(sA + (wave + NW * i) * 1024), 16, 0, 0);
#pragma unroll
  for (int i = 0; i < BCH; ++i)
    __builtin_amdgcn_global_load_lds(gb[i] + kb, (lds_ptr_t)(sB + (wave + NW * i) * 1024), 16, 0, 0);
#endif
}

__device__ inline i8 lds_frag(const uint8_t* row, int p0, int p1) {
  const u4 lo = *reinterpret_cast<const u4*>(row + p0 * 16);
  const u4 hi = *reinterpret_cast<const u4*>(row + p1 * 16);
  return i8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}

// Epilogue of the tiled GEMMs.  The accumulators are scaled (row scale rs[m]
// if given, column scale cs[n] if given, times s0), converted, and staged as
// the BM x BN output tile in LDS; then every thread writes 16-byte pieces of
// output rows with non-temporal stores (1-2 us less than default stores at
// 2048 x 6144).  Writing straight from the MFMA layout instead stores 2 bytes
// per lane, four rows per instruction, and took 20-40% of a K = 4096 GEMM.
// In LDS, the 16-byte column chunk k of tile row r sits at k ^ 2 ((r >> 2) & 3),
// so the four row groups of an accumulator write land in distinct banks;
// where a tile row is not a multiple of 8 chunks (BN = 96) the rows are
// instead BN * 2 + 16 bytes apart (rows 4 apart then start 16 banks apart).
// smem must hold out_tile_bytes(BM, BN) bytes; every wave must be done with
// it (the leading barrier).
// With SL (scales in LDS), rs and cs point at LDS copies of the tile's BM row
// and BN column scales (loaded by the kernel's prologue, outside smem's first
// out_tile_bytes(BM, BN) bytes) instead of the global vectors.
// With wskind >= 0 the column scale is the weight scale ws of that kind
// (ScaleKind: per channel fp16 / bf16 / fp32, or one fp32 value), in place
// of cs * s0.
constexpr int out_tile_bytes(int BM, int BN) { return BM * ((BN / 8) % 8 == 0 ? BN * 2 : BN * 2 + 16); }

template <typename T, int BM, int BN, int WM, int WN, int NT = 256, bool SL = false>
__device__ inline void store_tile(const f4 (&acc)[BM / WM / 16][BN / WN / 16], uint8_t* smem, int wm, int wn,
                                  int lane, int m0, int n0, int M, int N, const float* rs, const float* cs,
                                  float s0, uint16_t* Y, int mlo = 0,
                                  int nlo = 0, const void* ws = nullptr, int wskind = -1) {
  constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 16, FN = TN / 16;
  constexpr int CPR = BN / 8;  // 16-byte chunks per tile row
  constexpr bool XS = CPR % 8 == 0;          // chunk swizzle (inside aligned groups of 8), else padded rows
  constexpr int RS = XS ? BN * 2 : BN * 2 + 16;  // LDS bytes per tile row
  auto cpos = [](int r, int k) { return XS ? k ^ (2 * ((r >> 2) & 3)) : k; };
  const int r16 = lane & 15, g = lane >> 4;
  float rsv[FM][4];
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    if (SL) {
      const f4 v4 = *reinterpret_cast<const f4*>(rs + wm * TM + i * 16 + 4 * g);
#pragma unroll
      for (int v = 0; v < 4; ++v) rsv[i][v] = v4[v];
    } else {
#pragma unroll
      for (int v = 0; v < 4; ++v) rsv[i][v] = rs ? rs[min(m0 + wm * TM + i * 16 + 4 * g + v, M - 1)] : 1.f;
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int c = wn * TN + j * 16 + r16;
    const float cv = wskind >= 0 ? load_scale(ws, wskind, min(n0 + c, N - 1))
                                 : (SL ? cs[c] : (cs ? cs[min(n0 + c, N - 1)] : 1.f)) * s0;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int r = wm * TM + i * 16 + 4 * g + v;  // D row = 4 * (lane >> 4) + v
        *reinterpret_cast<uint16_t*>(smem + r * RS + cpos(r, c >> 3) * 16 + (c & 7) * 2) =
            T::from_f32(acc[i][j][v] * rsv[i][v] * cv);
      }
  }
  __syncthreads();
  const bool vec = (N & 7) == 0 && (reinterpret_cast<uintptr_t>(Y) & 15) == 0;
  for (int q = threadIdx.x; q < BM * CPR; q += NT) {
    const int r = q / CPR, k = q % CPR;
    const int m = m0 + r, n = n0 + 8 * k;
    if (m >= M || n >= N || m < mlo) continue;
    const uint8_t* src = smem + r * RS + cpos(r, k) * 16;
    uint16_t* dst = Y + (size_t)m * N + n;
    if (vec && n >= nlo) {
      __builtin_nontemporal_store(*reinterpret_cast<const u4*>(src), reinterpret_cast<u4*>(dst));
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (n + e < N && n + e >= nlo) dst[e] = reinterpret_cast<const uint16_t*>(src)[e];
    }
  }
}

template <typename T, int BM, int BN, int WM, int WN, int LAYOUT, int OCC>
__global__ __launch_bounds__(64 * WM * WN, OCC) void gemm_a8w8_lds_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ sa,
    const uint8_t* __restrict__ B, const float* __restrict__ sb,
    uint16_t* __restrict__ Y, int M, int N, int K, int tiles_m, int tiles_n) {
  constexpr int BK = 128;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 16, FN = TN / 16;
  constexpr int STAGE = (BM + BN) * BK;
  constexpr int NW = WM * WN;                         // waves per workgroup
  constexpr int ACH = BM / 8 / NW, BCH = BN / 8 / NW;  // 1 KB writer chunks per wave per stage
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * STAGE];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  int tm, tn;
  tile_of<BM, BN, 8>(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;

  // writer chunk j: lane i fills row 8 j + (i >> 3), position i & 7, i.e.
  // logical chunk (i & 7) ^ s(row)
  const uint8_t* ga[ACH];
  const uint8_t* gb[BCH];
#pragma unroll
  for (int i = 0; i < ACH; ++i) {
    const int row = (wave + NW * i) * 8 + (lane >> 3);
    ga[i] = A + (size_t)min(m0 + row, M - 1) * K + ((lane & 7) ^ swz<LAYOUT>(row)) * 16;
  }
#pragma unroll
  for (int i = 0; i < BCH; ++i) {
    const int row = (wave + NW * i) * 8 + (lane >> 3);
    gb[i] = B + (size_t)min(n0 + row, N - 1) * K + ((lane & 7) ^ swz<LAYOUT>(row)) * 16;
  }

  // reader: row (lane & 15) of each 16-row block; both swizzles depend only
  // on row & 15, and blocks start at multiples of 16, so s(row) = s(lane & 15)
  const int r16 = lane & 15, g = lane >> 4;
  const int c0 = LAYOUT == 0 ? 2 * g : g;
  const int c1 = LAYOUT == 0 ? 2 * g + 1 : g + 4;
  const int p0 = c0 ^ swz<LAYOUT>(r16), p1 = c1 ^ swz<LAYOUT>(r16);

  f4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  const int KT = K / BK;
  a8w8_issue<BM, BN, ACH, BCH, NW>(smem, 0, 0, wave, ga, gb);
  for (int kt = 0; kt < KT; ++kt) {
    __syncthreads();  // this step's stage has landed; the other stage is free
    if (kt + 1 < KT) a8w8_issue<BM, BN, ACH, BCH, NW>(smem, (kt + 1) & 1, (kt + 1) * BK, wave, ga, gb);
    const uint8_t* sA = smem + (kt & 1) * STAGE + (wm * TM + r16) * BK;
    const uint8_t* sB = smem + (kt & 1) * STAGE + (BM + wn * TN + r16) * BK;
    i8 bf[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) bf[j] = lds_frag(sB + j * 16 * BK, p0, p1);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const i8 af = lds_frag(sA + i * 16 * BK, p0, p1);
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = mfma_fp8_16x16x128(af, bf[j], acc[i][j]);
    }
  }

  static_assert(sizeof(smem) >= out_tile_bytes(BM, BN), "output tile must fit the stages");
  store_tile<T, BM, BN, WM, WN, 64 * NW>(acc, smem, wm, wn, lane, m0, n0, M, N, sa, sb, 1.f, Y);
}

// ---------------------------------------------------------------------------
// a8w8, LDS-tiled with register-pipelined fragment reads and loader waves.
// Same K slices, row layout, swizzle and direct-to-LDS loads as
// gemm_a8w8_lds_kernel, two-slot rings for A and B; the difference is the
// order of work inside a K step and which waves load.
// * A wave's step is FM groups of FN MFMAs (group i: A fragment i against the
//   FN B fragments).  The A fragment of group i + 1 is read from LDS while
//   group i's MFMAs run (two A register sets), and the step's one barrier
//   sits before the last group: after it the loaders issue the direct-to-LDS
//   loads of step k + 2's B and A rows into the slots step k used, and every
//   wave reads step k + 1's B fragments and first A fragment (two B register
//   sets) behind the last group's MFMAs.
// * Only LW of the NW waves load (waves 0 .. LW-1; with LW = NW / 2 one wave
//   per SIMD).  The load path accepts a 1 KB direct-to-LDS load about every
//   16 cycles per CU, so a wave that issues its loads stalls until the path
//   takes them; a cycle-counter trace of the 8-wave 256 x 192 kernel on
//   MI355X put 530-840 of a step's ~2500 cycles there, with both waves of a
//   SIMD stalled at once.  With loader waves the SIMD's other wave keeps the
//   MFMA pipe busy meanwhile (M = 2048: 5-14% faster than all waves loading).
// * The loads are MUBUF buffer loads with the LDS bit (buffer resources over
//   A and B), not global_load_lds: the compiler counts a global_load_lds as
//   an outstanding LDS event as well, so every fragment read behind one waited
//   for lgkmcnt(0); with buffer loads it waits only for its own fragment.
// * With NCH > 1 (8-wave tiles) a loader issues only the first of NCH chunks
//   of its loads after the barrier and the others in the next step's first
//   NCH - 1 MFMA groups, so that it is not stalled behind the load path for
//   the whole batch (M = 2048, weights from HBM: 3-5% faster, NCH = 3 best).
// The barrier orders, for all waves: step k + 1's rows have landed (the
// loaders' only outstanding loads), every read of step k's slots is done
// (lgkmcnt(0)), so they may be overwritten.
// Requires K % 128 == 0, FM even, M >= BM, N >= BN, 16-byte aligned A and B,
// each below 4 GB (the buffer resources' 32-bit byte range).
// ---------------------------------------------------------------------------
template <int BM, int BN, int WM, int WN>
struct PipeCfg {
  static constexpr int BK = 128;
  static constexpr int TM = BM / WM, TN = BN / WN;
  static constexpr int FM = TM / 16, FN = TN / 16;
  static constexpr int ASLOT = BM * BK, BSLOT = BN * BK;
  static constexpr int NW = WM * WN;
  static_assert(TM * WM == BM && TN * WN == BN && TM % 16 == 0 && TN % 16 == 0, "wave tiles cover the tile");
  static_assert(FM % 2 == 0, "A fragments alternate between two register sets");
};

// 1 KB loads per loader wave and slot with LW loader waves
template <int BM, int BN, int LW>
struct LoadSplit {
  static constexpr int AL = BM / 8 / LW, BL = BN / 8 / LW;
  static_assert(AL * 8 * LW == BM && BL * 8 * LW == BN, "loader chunks cover the tile");
};

// s_waitcnt vmcnt(N) lgkmcnt(0) + s_barrier: every one of this wave's loads
// but its N most recent is complete and its LDS reads are done, then all
// waves meet.
template <int N>
__device__ inline void barrier_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// The same leaving min(steps, MAXS) later steps' loads in flight (PER loads
// per step and wave, issued in step order): the count is an immediate, so a
// uniform branch picks it.  Waves with fewer loads out pass at once.
template <int MAXS, int PER>
__device__ inline void barrier_upto(int steps) {
  static_assert(MAXS <= 3 && MAXS * PER <= 63, "vmcnt immediate");
  if constexpr (MAXS >= 3) {
    if (steps >= 3) { barrier_vmcnt<3 * PER>(); return; }
  }
  if constexpr (MAXS >= 2) {
    if (steps >= 2) { barrier_vmcnt<2 * PER>(); return; }
  }
  if constexpr (MAXS >= 1) {
    if (steps >= 1) { barrier_vmcnt<PER>(); return; }
  }
  barrier_vmcnt<0>();
}

// Buffer resource over n bytes at p (raw, stride 0); loads beyond n return 0.
__device__ inline __amdgpu_buffer_rsrc_t buf_rsrc(const void* p, uint32_t n) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)n, 0x00020000);
}

// Direct-to-LDS loads of chunk ch (of NCH) of one K step (128 bytes of each
// row) by loader w: its BL B loads, then its AL A loads, cut into NCH runs of
// ceil((AL + BL) / NCH).  Load i of a kind moves rows 8 j .. 8 j + 7, j = w +
// LW i, into 1 KB piece j of the slot; the lane's byte offset (ga / gb, one
// VGPR) plus kb addresses chunk 0's row and i * LW * 8 * K (a uniform
// SGPR offset, unsigned 32-bit like the whole offset) the row of load i.
template <int AL, int BL, int LW, int NCH>
__device__ __forceinline__ void a8w8_issue_chunk(int ch, uint8_t* sB, uint8_t* sA, int kb, int w, __amdgpu_buffer_rsrc_t rA,
                                                 __amdgpu_buffer_rsrc_t rB, int K, uint32_t ga, uint32_t gb) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int T = AL + BL, CS = (T + NCH - 1) / NCH;
#pragma unroll
  for (int i = 0; i < T; ++i) {
    if (i < ch * CS || i >= ch * CS + CS) continue;
    if (i < BL)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, (lds_ptr_t)(sB + (w + LW * i) * 1024), 16, gb + (uint32_t)kb,
                                               (int)((uint32_t)(i * LW * 8) * (uint32_t)K), 0, 0);
    else
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, (lds_ptr_t)(sA + (w + LW * (i - BL)) * 1024), 16, ga + (uint32_t)kb,
                                               (int)((uint32_t)((i - BL) * LW * 8) * (uint32_t)K), 0, 0);
  }
#endif
}

// The epilogue's scales (the tile's BM row scales from sa, then its BN column
// scales from sb) go to LDS at sc first, by 4-byte direct-to-LDS loads (one
// instruction per wave for 64 of them), so that the prologue's wait covers
// their latency; register loads mixed with the direct-to-LDS ones would make
// the compiler drain every load before using them.  Waves 0 .. BM / 64 - 1
// load row scales, the rest column scales.  Each wave issues at most one
// load, before any of its operand loads.
template <int BM, int BN, int NW>
__device__ __forceinline__ void stage_tile_scales(float* sc, const float* sa, const float* sb, int M, int N, int m0,
                                                  int n0, int wave, int lane) {
  static_assert(BM % 64 == 0, "a wave's scales come from one of sa, sb");
  static_assert(BM + BN <= 64 * NW, "one scale per thread");
  if (64 * wave < BM + BN) {
    const int t = min(64 * wave + lane, BM + BN - 1);
    const bool rows = 64 * wave < BM;
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(buf_rsrc(rows ? sa : sb, (uint32_t)(rows ? M : N) * 4u),
                                             (lds_ptr_t)(sc + 64 * wave), 4,
                                             (uint32_t)(rows ? m0 + t : n0 + t - BM) * 4u, 0, 0, 0);
#endif
  }
}

// One K step kt from ring slot c (the next step's slot cn).  Its barrier
// (before the last MFMA group) waits for step kt + 1's loads, leaves up to
// RING - 2 later steps' in flight, and is followed by chunk 0 of step
// kt + RING into slot c (fully read by then); chunks 1 .. NCH - 1 of step
// kt + RING - 1 (whose chunk 0 went out after the previous step's barrier)
// go out in groups 0 .. NCH - 2.  Steps 0 .. RING - 1 are loaded whole by the
// prologue, hence kt >= 1 for the chunks.
template <int BM, int BN, int WM, int WN, int LW, int RING, int NCH>
__device__ __forceinline__ void a8w8_pipe_step(int kt, int KT, int c, int cn, uint8_t* sAr, uint8_t* sBr, bool loader, int wave,
                                               int wm, int wn, int r16, int p0, int p1, __amdgpu_buffer_rsrc_t rA,
                                               __amdgpu_buffer_rsrc_t rB, int K, uint32_t ga, uint32_t gb,
                                               f4 (&acc)[PipeCfg<BM, BN, WM, WN>::FM][PipeCfg<BM, BN, WM, WN>::FN],
                                               i8 (&a)[2], const i8 (&bc)[PipeCfg<BM, BN, WM, WN>::FN],
                                               i8 (&bn)[PipeCfg<BM, BN, WM, WN>::FN]) {
  using C = PipeCfg<BM, BN, WM, WN>;
  using L = LoadSplit<BM, BN, LW>;
  constexpr int BK = C::BK, TM = C::TM, TN = C::TN, FM = C::FM, FN = C::FN;
  static_assert(NCH >= 1 && NCH <= FM, "chunks 1 .. NCH - 1 go out in the groups before the barrier");
  const uint8_t* sA = sAr + c * C::ASLOT + (wm * TM + r16) * BK;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    if (i + 1 < FM) {
      a[(i + 1) & 1] = lds_frag(sA + (i + 1) * 16 * BK, p0, p1);
      if (i < NCH - 1 && loader && kt >= 1 && kt + RING - 1 < KT) {
        const int cl = c == 0 ? RING - 1 : c - 1;  // slot of step kt + RING - 1
        a8w8_issue_chunk<L::AL, L::BL, LW, NCH>(i + 1, sBr + cl * C::BSLOT, sAr + cl * C::ASLOT, (kt + RING - 1) * BK,
                                                wave, rA, rB, K, ga, gb);
      }
    } else if (kt + 1 < KT) {
      barrier_upto<RING - 2, L::AL + L::BL>(KT - 2 - kt);
      if (loader && kt + RING < KT)
        a8w8_issue_chunk<L::AL, L::BL, LW, NCH>(0, sBr + c * C::BSLOT, sAr + c * C::ASLOT, (kt + RING) * BK, wave, rA, rB,
                                                K, ga, gb);
      const uint8_t* nA = sAr + cn * C::ASLOT + (wm * TM + r16) * BK;
      const uint8_t* nB = sBr + cn * C::BSLOT + (wn * TN + r16) * BK;
#pragma unroll
      for (int j = 0; j < FN; ++j) bn[j] = lds_frag(nB + j * 16 * BK, p0, p1);
      a[0] = lds_frag(nA, p0, p1);
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = mfma_fp8_16x16x128(a[i & 1], bc[j], acc[i][j]);
    __builtin_amdgcn_sched_barrier(0);
  }
}

//
// SPLIT > 1 (split K, for shapes with too few tiles to fill the GPU):
// workgroup b computes tile b / SPLIT over the K range of part b % SPLIT
// ((K / SPLIT) % 128 == 0) and stores its unscaled fp32 sums to part
// P[b % SPLIT] of the [SPLIT][M][N] workspace P; gemm_splitk_finalize then
// adds the parts in order, scales and converts.
// RING: slots of the A and B rings (loads run RING - 1 steps ahead).  NCH:
// chunks a loader's loads of a step are issued in (a8w8_pipe_step).
template <typename T, int BM, int BN, int WM, int WN, int OCC, int LW, int SPLIT = 1, int RING = 2, int NCH = 1>
__global__ __launch_bounds__(64 * WM * WN, OCC) void gemm_a8w8_pipe_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ sa,
    const uint8_t* __restrict__ B, const float* __restrict__ sb,
    uint16_t* __restrict__ Y, float* __restrict__ P, int M, int N, int K, int tiles_m, int tiles_n) {
  using C = PipeCfg<BM, BN, WM, WN>;
  using L = LoadSplit<BM, BN, LW>;
  constexpr int BK = C::BK, TM = C::TM, TN = C::TN, FM = C::FM, FN = C::FN, NW = C::NW;
  constexpr int AL = L::AL, BL = L::BL;
  static_assert(LW >= 1 && LW <= NW, "loader waves");
  static_assert(RING >= 2 && RING <= 4, "ring slots");
  constexpr int RINGS = RING * (C::ASLOT + C::BSLOT);
  constexpr int SMEM = RINGS > out_tile_bytes(BM, BN) ? RINGS : out_tile_bytes(BM, BN);
  // the A ring and the B ring (or the output tile), then the tile's row and
  // column scales
  __shared__ __attribute__((aligned(1024))) uint8_t smem[SMEM + (BM + BN) * 4];
  uint8_t* sAr = smem;
  uint8_t* sBr = smem + RING * C::ASLOT;
  float* sc = reinterpret_cast<float*>(smem + SMEM);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const bool loader = wave < LW;
  const int part = SPLIT > 1 ? (int)blockIdx.x % SPLIT : 0;
  int tm, tn;
  tile_of<BM, BN, 8>(SPLIT > 1 ? blockIdx.x / SPLIT : blockIdx.x, tiles_m, tiles_n, tm, tn);
  // A last tile that would cross M (N) is moved back to end there (M >= BM,
  // N >= BN): every row it loads exists, so no load needs a clamp, and it
  // stores only from its own first row (column) mlo (nlo) on -- the rows
  // before are the previous tile's, which computes the same values.
  const int mlo = tm * BM, nlo = tn * BN;
  const int m0 = min(mlo, M - BM), n0 = min(nlo, N - BN);
  const __amdgpu_buffer_rsrc_t rA = buf_rsrc(A, (uint32_t)((size_t)M * K));
  const __amdgpu_buffer_rsrc_t rB = buf_rsrc(B, (uint32_t)((size_t)N * K));
  stage_tile_scales<BM, BN, NW>(sc, sa, sb, M, N, m0, n0, wave, lane);

  // loader chunk j = wave + LW i: lane l fills row 8 j + (l >> 3), position
  // l & 7, i.e. logical chunk (l & 7) ^ s(row) (s(row) = row & 7 = (l >> 3)
  // & 7 for every chunk).  Byte offsets into A and B of this lane's chunk 0
  // rows; chunk i is LW * 8 rows further (a uniform stride).
  const uint32_t cofs = (uint32_t)(((lane & 7) ^ swz<1>(lane >> 3)) * 16);
  const uint32_t kpart = (uint32_t)(part * (K / SPLIT));  // first K value of this part
  const uint32_t ga = (uint32_t)(m0 + wave * 8 + (lane >> 3)) * (uint32_t)K + cofs + kpart;
  const uint32_t gb = (uint32_t)(n0 + wave * 8 + (lane >> 3)) * (uint32_t)K + cofs + kpart;
  const int r16 = lane & 15, g = lane >> 4;
  const int p0 = g ^ swz<1>(r16), p1 = (g + 4) ^ swz<1>(r16);

  f4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  const int KT = K / BK / SPLIT;
  // Prologue: steps 0 .. RING - 1 into their slots, then wait for step 0 (a
  // loader's later steps, issued after it, may fly; a non-loader has at most
  // its older scale load out).
  if (loader) {
#pragma unroll
    for (int s = 0; s < RING; ++s)
      if (s == 0 || s < KT) {
        a8w8_issue_chunk<AL, BL, LW, 1>(0, sBr + s * C::BSLOT, sAr + s * C::ASLOT, s * BK, wave, rA, rB, K, ga, gb);
      }
  }
  barrier_upto<RING - 1, AL + BL>(KT - 1);
  i8 a[2], b0[FN], b1[FN];
  {
    const uint8_t* sA = sAr + (wm * TM + r16) * BK;
    const uint8_t* sB = sBr + (wn * TN + r16) * BK;
#pragma unroll
    for (int j = 0; j < FN; ++j) b0[j] = lds_frag(sB + j * 16 * BK, p0, p1);
    a[0] = lds_frag(sA, p0, p1);
  }
  int kt = 0, c = 0;
  auto nxt = [](int v) { return v + 1 == RING ? 0 : v + 1; };
  for (; kt + 1 < KT; kt += 2) {
    const int c1 = RING == 2 ? 1 : nxt(c), c2 = RING == 2 ? 0 : nxt(c1);
    a8w8_pipe_step<BM, BN, WM, WN, LW, RING, NCH>(kt, KT, RING == 2 ? 0 : c, c1, sAr, sBr, loader, wave, wm, wn, r16,
                                                  p0, p1, rA, rB, K, ga, gb, acc, a, b0, b1);
    a8w8_pipe_step<BM, BN, WM, WN, LW, RING, NCH>(kt + 1, KT, c1, c2, sAr, sBr, loader, wave, wm, wn, r16, p0, p1, rA,
                                                  rB, K, ga, gb, acc, a, b1, b0);
    c = c2;
  }
  if (kt < KT)
    a8w8_pipe_step<BM, BN, WM, WN, LW, RING, NCH>(kt, KT, RING == 2 ? 0 : c, RING == 2 ? 1 : nxt(c), sAr, sBr, loader,
                                                  wave, wm, wn, r16, p0, p1, rA, rB, K, ga, gb, acc, a, b0, b1);
  // every wave's loads (a non-loader's scale load included) are complete
  // here: step KT - 2's barrier (the last) waited for vmcnt(0), and with
  // KT == 1 the prologue's did
  static_assert(SMEM >= out_tile_bytes(BM, BN), "output tile must fit");
  if constexpr (SPLIT > 1) {
    // fp32 partial sums in D layout: lane l holds column l & 15, rows
    // 4 (l >> 4) + v of each 16 x 16 block (rows before mlo / columns before
    // nlo belong to the previous tile)
    float* Pp = P + (size_t)part * M * N;
    const int r16 = lane & 15, g4 = (lane >> 4) * 4;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int n = n0 + wn * TN + j * 16 + r16;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int m = m0 + wm * TM + i * 16 + g4 + v;
          if (m >= mlo && n >= nlo) Pp[(size_t)m * N + n] = acc[i][j][v];
        }
      }
  } else {
    store_tile<T, BM, BN, WM, WN, 64 * NW, true>(acc, smem, wm, wn, lane, m0, n0, M, N, sc, sc + BM, 1.f, Y, mlo, nlo);
  }
}

// ---------------------------------------------------------------------------
// gemm_a8w8_pipe_kernel with a deeper B ring: A in 2 slots, B in 3, so the
// B (weight) loads run two K steps ahead instead of one and an HBM miss has
// two steps to land (M = 2048, K = 4096, N = 6144 with weights from HBM:
// 45.0 -> 41.2 us; cache-resident 39.6 -> 40.1 us; 256 x 192 needs
// 2 x 32 + 3 x 24 KB of LDS, a joint third slot 168 KB).  Unsplit only.
//
// Load group G(k), issued from the barrier of step k on (chunk 0 there,
// chunks 1 .. NCH - 1 in the next step's first MFMA groups), is A(k + 2) into
// A slot k % 2 and B(k + 3) into B slot k % 3 -- the slots step k has just
// given up -- A loads first.  The barrier of step k needs A(k + 1) (in
// G(k - 1)) and B(k + 1) (in G(k - 2)); the only loads issued after A(k + 1)
// are G(k - 1)'s B loads, so the wait leaves those BL in flight
// (vmcnt(BL) while B(k + 2) exists, vmcnt(0) after).  The prologue loads
// A(0) B(0), A(1) B(1) and B(2).
// ---------------------------------------------------------------------------

// Chunk ch (of NCH) of a load group: A step ka's AL loads into sA (if ha),
// then B step kb's BL loads into sB (if hb); rows and offsets as in
// a8w8_issue_chunk.
template <int AL, int BL, int LW, int NCH>
__device__ __forceinline__ void a8w8_issue_chunk_ab(int ch, uint8_t* sA, uint8_t* sB, int ka, int kb, bool ha, bool hb,
                                                    int w, __amdgpu_buffer_rsrc_t rA, __amdgpu_buffer_rsrc_t rB, int K,
                                                    uint32_t ga, uint32_t gb) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int T = AL + BL, CS = (T + NCH - 1) / NCH;
#pragma unroll
  for (int i = 0; i < T; ++i) {
    if (i < ch * CS || i >= ch * CS + CS) continue;
    if (i < AL) {
      if (ha)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, (lds_ptr_t)(sA + (w + LW * i) * 1024), 16, ga + (uint32_t)ka,
                                                 (int)((uint32_t)(i * LW * 8) * (uint32_t)K), 0, 0);
    } else {
      if (hb)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, (lds_ptr_t)(sB + (w + LW * (i - AL)) * 1024), 16,
                                                 gb + (uint32_t)kb, (int)((uint32_t)((i - AL) * LW * 8) * (uint32_t)K),
                                                 0, 0);
    }
  }
#endif
}

// One K step kt: A slot CA = kt % 2, B slot cb = kt % 3.
template <int BM, int BN, int WM, int WN, int LW, int NCH, int CA>
__device__ __forceinline__ void a8w8_b3_step(int kt, int KT, int cb, uint8_t* sAr, uint8_t* sBr, bool loader,
                                             int wave, int wm, int wn, int r16, int p0, int p1,
                                             __amdgpu_buffer_rsrc_t rA, __amdgpu_buffer_rsrc_t rB, int K, uint32_t ga,
                                             uint32_t gb,
                                             f4 (&acc)[PipeCfg<BM, BN, WM, WN>::FM][PipeCfg<BM, BN, WM, WN>::FN],
                                             i8 (&a)[2], const i8 (&bc)[PipeCfg<BM, BN, WM, WN>::FN],
                                             i8 (&bn)[PipeCfg<BM, BN, WM, WN>::FN]) {
  using C = PipeCfg<BM, BN, WM, WN>;
  using L = LoadSplit<BM, BN, LW>;
  constexpr int BK = C::BK, TM = C::TM, TN = C::TN, FM = C::FM, FN = C::FN;
  static_assert(NCH >= 1 && NCH <= FM, "chunks 1 .. NCH - 1 go out in the groups before the barrier");
  const uint8_t* sA = sAr + CA * C::ASLOT + (wm * TM + r16) * BK;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    if (i + 1 < FM) {
      a[(i + 1) & 1] = lds_frag(sA + (i + 1) * 16 * BK, p0, p1);
      if (i < NCH - 1 && loader && kt >= 1) {  // chunk i + 1 of G(kt - 1)
        const int cbp = cb == 0 ? 2 : cb - 1;  // B slot (kt - 1) % 3 = (kt + 2) % 3
        a8w8_issue_chunk_ab<L::AL, L::BL, LW, NCH>(i + 1, sAr + (1 - CA) * C::ASLOT, sBr + cbp * C::BSLOT,
                                                   (kt + 1) * BK, (kt + 2) * BK, kt + 1 < KT, kt + 2 < KT, wave, rA,
                                                   rB, K, ga, gb);
      }
    } else if (kt + 1 < KT) {
      if (kt + 2 < KT) barrier_vmcnt<L::BL>();
      else barrier_vmcnt<0>();
      if (loader)  // chunk 0 of G(kt)
        a8w8_issue_chunk_ab<L::AL, L::BL, LW, NCH>(0, sAr + CA * C::ASLOT, sBr + cb * C::BSLOT, (kt + 2) * BK,
                                                   (kt + 3) * BK, kt + 2 < KT, kt + 3 < KT, wave, rA, rB, K, ga, gb);
      const int cbn = cb == 2 ? 0 : cb + 1;
      const uint8_t* nA = sAr + (1 - CA) * C::ASLOT + (wm * TM + r16) * BK;
      const uint8_t* nB = sBr + cbn * C::BSLOT + (wn * TN + r16) * BK;
#pragma unroll
      for (int j = 0; j < FN; ++j) bn[j] = lds_frag(nB + j * 16 * BK, p0, p1);
      a[0] = lds_frag(nA, p0, p1);
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = mfma_fp8_16x16x128(a[i & 1], bc[j], acc[i][j]);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Tile order: groups of 4 tile rows (the XCD's 32 tiles of a 2048 x 6144
// output are then 4 x 8 tiles, 10 MB of A and B, against 11 MB for 8 x 4:
// 1-3% faster with weights from HBM).
template <typename T, int BM, int BN, int WM, int WN, int LW, int NCH>
__global__ __launch_bounds__(64 * WM * WN, 1) void gemm_a8w8_pipe_b3_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ sa,
    const uint8_t* __restrict__ B, const float* __restrict__ sb,
    uint16_t* __restrict__ Y, int M, int N, int K, int tiles_m, int tiles_n) {
  using C = PipeCfg<BM, BN, WM, WN>;
  using L = LoadSplit<BM, BN, LW>;
  constexpr int BK = C::BK, TM = C::TM, TN = C::TN, FM = C::FM, FN = C::FN, NW = C::NW;
  constexpr int AL = L::AL, BL = L::BL;
  static_assert(LW >= 1 && LW <= NW, "loader waves");
  static_assert(AL + 2 * BL <= 63, "vmcnt immediate");
  constexpr int RINGS = 2 * C::ASLOT + 3 * C::BSLOT;
  constexpr int SMEM = RINGS > out_tile_bytes(BM, BN) ? RINGS : out_tile_bytes(BM, BN);
  __shared__ __attribute__((aligned(1024))) uint8_t smem[SMEM + (BM + BN) * 4];
  static_assert(sizeof(smem) <= 160 * 1024, "LDS");
  uint8_t* sAr = smem;
  uint8_t* sBr = smem + 2 * C::ASLOT;
  float* sc = reinterpret_cast<float*>(smem + SMEM);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const bool loader = wave < LW;
  int tm, tn;
  tile_of<BM, BN, 4>(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int mlo = tm * BM, nlo = tn * BN;  // edge tiles moved back inside, as in gemm_a8w8_pipe_kernel
  const int m0 = min(mlo, M - BM), n0 = min(nlo, N - BN);
  const __amdgpu_buffer_rsrc_t rA = buf_rsrc(A, (uint32_t)((size_t)M * K));
  const __amdgpu_buffer_rsrc_t rB = buf_rsrc(B, (uint32_t)((size_t)N * K));
  stage_tile_scales<BM, BN, NW>(sc, sa, sb, M, N, m0, n0, wave, lane);
  const uint32_t cofs = (uint32_t)(((lane & 7) ^ swz<1>(lane >> 3)) * 16);
  const uint32_t ga = (uint32_t)(m0 + wave * 8 + (lane >> 3)) * (uint32_t)K + cofs;
  const uint32_t gb = (uint32_t)(n0 + wave * 8 + (lane >> 3)) * (uint32_t)K + cofs;
  const int r16 = lane & 15, g = lane >> 4;
  const int p0 = g ^ swz<1>(r16), p1 = (g + 4) ^ swz<1>(r16);

  f4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  const int KT = K / BK;
  if (loader) {
    a8w8_issue_chunk_ab<AL, BL, LW, 1>(0, sAr, sBr, 0, 0, true, true, wave, rA, rB, K, ga, gb);
    a8w8_issue_chunk_ab<AL, BL, LW, 1>(0, sAr + C::ASLOT, sBr + C::BSLOT, BK, BK, KT > 1, KT > 1, wave, rA, rB, K, ga,
                                       gb);
    a8w8_issue_chunk_ab<AL, BL, LW, 1>(0, sAr, sBr + 2 * C::BSLOT, 0, 2 * BK, false, KT > 2, wave, rA, rB, K, ga, gb);
  }
  // step 0 in (a non-loader has at most its older scale load out)
  if (KT > 2) barrier_vmcnt<AL + 2 * BL>();
  else if (KT > 1) barrier_vmcnt<AL + BL>();
  else barrier_vmcnt<0>();
  i8 a[2], b0[FN], b1[FN];
  {
    const uint8_t* sA = sAr + (wm * TM + r16) * BK;
    const uint8_t* sB = sBr + (wn * TN + r16) * BK;
#pragma unroll
    for (int j = 0; j < FN; ++j) b0[j] = lds_frag(sB + j * 16 * BK, p0, p1);
    a[0] = lds_frag(sA, p0, p1);
  }
  int kt = 0, cb = 0;
  for (; kt + 1 < KT; kt += 2) {
    a8w8_b3_step<BM, BN, WM, WN, LW, NCH, 0>(kt, KT, cb, sAr, sBr, loader, wave, wm, wn, r16, p0, p1, rA, rB, K, ga,
                                             gb, acc, a, b0, b1);
    cb = cb == 2 ? 0 : cb + 1;
    a8w8_b3_step<BM, BN, WM, WN, LW, NCH, 1>(kt + 1, KT, cb, sAr, sBr, loader, wave, wm, wn, r16, p0, p1, rA, rB, K,
                                             ga, gb, acc, a, b1, b0);
    cb = cb == 2 ? 0 : cb + 1;
  }
  if (kt < KT)
    a8w8_b3_step<BM, BN, WM, WN, LW, NCH, 0>(kt, KT, cb, sAr, sBr, loader, wave, wm, wn, r16, p0, p1, rA, rB, K, ga,
                                             gb, acc, a, b0, b1);
  // every load is complete: the last barrier (step KT - 2's, or the
  // prologue's with KT == 1) waited for vmcnt(0)
  store_tile<T, BM, BN, WM, WN, 64 * NW, true>(acc, smem, wm, wn, lane, m0, n0, M, N, sc, sc + BM, 1.f, Y, mlo, nlo);
}

// Y[m, n] = Out(sa[m] * sb[n] * (P[0][m, n] + P[1][m, n] + ...)), the parts
// added in order (so the result does not depend on which part finished
// first).  Grid (ceil(N / 1024), rows): four consecutive outputs of one row
// per thread, read as a 16-byte piece of every part and stored as one 8-byte
// piece when N % 4 == 0 (P, Y and sb 16-byte aligned), element by element
// otherwise; rows past gridDim.y are taken grid-stride.  (Eight outputs per
// thread, half the workgroups, measured 0-4% slower: M = 64, K = 4096, N =
// 14336 20.00 against 20.48 us.)
template <typename T, int SPLIT>
__global__ __launch_bounds__(256) void gemm_splitk_finalize(const float* __restrict__ P, const float* __restrict__ sa,
                                                            const float* __restrict__ sb, uint16_t* __restrict__ Y,
                                                            int M, int N) {
  const size_t total = (size_t)M * N;
  const int n = ((int)blockIdx.x * 256 + (int)threadIdx.x) * 4;
  if (n >= N) return;
  const bool vec = (N & 3) == 0 && ((reinterpret_cast<uintptr_t>(P) | reinterpret_cast<uintptr_t>(Y) | reinterpret_cast<uintptr_t>(sb)) & 15) == 0;
  for (int m = blockIdx.y; m < M; m += gridDim.y) {
    const size_t i = (size_t)m * N + n;
    const float rs = sa[m];
    if (vec) {
      f4 s0 = *reinterpret_cast<const f4*>(P + i);
#pragma unroll
      for (int q = 1; q < SPLIT; ++q) {
        const f4 p0 = *reinterpret_cast<const f4*>(P + q * total + i);
#pragma unroll
        for (int e = 0; e < 4; ++e) s0[e] += p0[e];
      }
      const f4 c0 = *reinterpret_cast<const f4*>(sb + n);
      uint2 o;
      o.x = (uint32_t)T::from_f32(f32_round(s0[0] * rs * c0[0])) | ((uint32_t)T::from_f32(f32_round(s0[1] * rs * c0[1])) << 16);
      o.y = (uint32_t)T::from_f32(f32_round(s0[2] * rs * c0[2])) | ((uint32_t)T::from_f32(f32_round(s0[3] * rs * c0[3])) << 16);
      *reinterpret_cast<uint2*>(Y + i) = o;
    } else {
      for (int e = 0; e < 4 && n + e < N; ++e) {
        float s = P[i + e];
#pragma unroll
        for (int q = 1; q < SPLIT; ++q) s += P[q * total + i + e];
        Y[i + e] = T::from_f32(f32_round(s * rs * sb[n + e]));
      }
    }
  }
}

// The same for the w8a16 split K: Y[m, n] = Out(w_scale[n] * (P[0][m, n] +
// P[1][m, n] + ...)), the weight scale of kind skind (ScaleKind; per channel
// or one value), the parts added in order.
template <typename T, int SPLIT>
__global__ __launch_bounds__(256) void gemm_splitk_finalize_w(const float* __restrict__ P, const void* __restrict__ ws,
                                                              int skind, uint16_t* __restrict__ Y, int M, int N) {
  const size_t total = (size_t)M * N;
  const int n = ((int)blockIdx.x * 256 + (int)threadIdx.x) * 8;
  if (n >= N) return;
  const bool vec = (N & 7) == 0 && ((reinterpret_cast<uintptr_t>(P) | reinterpret_cast<uintptr_t>(Y)) & 15) == 0;
  float cs[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) cs[e] = load_scale(ws, skind, min(n + e, N - 1));
  for (int m = blockIdx.y; m < M; m += gridDim.y) {
    const size_t i = (size_t)m * N + n;
    if (vec) {
      f4 s0 = *reinterpret_cast<const f4*>(P + i), s1 = *reinterpret_cast<const f4*>(P + i + 4);
#pragma unroll
      for (int q = 1; q < SPLIT; ++q) {
        const f4 p0 = *reinterpret_cast<const f4*>(P + q * total + i);
        const f4 p1 = *reinterpret_cast<const f4*>(P + q * total + i + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          s0[e] += p0[e];
          s1[e] += p1[e];
        }
      }
      u4 o;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const uint32_t lo0 = T::from_f32(f32_round(s0[2 * e] * cs[2 * e]));
        const uint32_t hi0 = T::from_f32(f32_round(s0[2 * e + 1] * cs[2 * e + 1]));
        const uint32_t lo1 = T::from_f32(f32_round(s1[2 * e] * cs[4 + 2 * e]));
        const uint32_t hi1 = T::from_f32(f32_round(s1[2 * e + 1] * cs[4 + 2 * e + 1]));
        o[e] = lo0 | (hi0 << 16);
        o[2 + e] = lo1 | (hi1 << 16);
      }
      *reinterpret_cast<u4*>(Y + i) = o;
    } else {
      for (int e = 0; e < 8 && n + e < N; ++e) {
        float s = P[i + e];
#pragma unroll
        for (int q = 1; q < SPLIT; ++q) s += P[q * total + i + e];
        Y[i + e] = T::from_f32(f32_round(s * cs[e]));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// w8a16, LDS-tiled: block tile BM x BN, K step 64, four waves 2 x 2.
// LDS stage: A as BM rows of 128 bytes (64 activations, eight 16-byte chunks,
// chunk c of row r at c ^ sA(r)), B as BN rows of 64 bytes (64 fp8 codes,
// four chunks, chunk c of row r at c ^ sB(r)); both filled by direct-to-LDS
// loads (one instruction: 8 A rows or 16 B rows).  Lane l of a wave takes
// row (l & 15) of a 16-row block and K positions 16 g .. 16 g + 15, g = l >> 4:
// 32 bytes of A (two chunks) and 16 bytes of B (one chunk), decoded to the
// activation type in registers; two 16 x 16 x 32 MFMAs consume them.
// ---------------------------------------------------------------------------
__device__ inline int swzA(int row) { return (row ^ ((row >> 3) & 1)) & 7; }
__device__ inline int swzB(int row) { return (row >> 2) & 3; }

template <int BM, int BN, int ACH, int BCH, int NW = 4>
__device__ inline void w8a16_issue(uint8_t* smem, int stage, int kb, int wave,
                                   const uint8_t* const (&ga)[ACH], const uint8_t* const (&gb)[BCH]) {
#if defined(__HIP_DEVICE_COMPILE__)  // device-only builtin; the host pass only needs the kernel's stub
  uint8_t* sA = smem + stage * (BM * 128 + BN * 64);
  uint8_t* sB = sA + BM * 128;
#pragma unroll
  for (int i = 0; i < ACH; ++i)
    __builtin_amdgcn_global_load_lds(ga[i] + 2 * kb, (lds_ptr_t)(sA + (wave + NW * i) * 1024), 16, 0, 0);
#pragma unroll
  for (int i = 0; i < BCH; ++i)
    __builtin_amdgcn_global_load_lds(gb[i] + kb, (lds_ptr_t)(sB + (wave + NW * i) * 1024), 16, 0, 0);
#endif
}

// Same loads from 32-bit byte offsets (one VGPR per load instead of a 64-bit
// pointer; the caller checks that both matrices are below 4 GB) as buffer
// loads over resources rX, rW, chunk ch of NCH: the loader's ACH A loads,
// then its BCH B loads, cut into NCH runs of ceil((ACH + BCH) / NCH).
template <int BM, int BN, int ACH, int BCH, int STRIDE, int NCH>
__device__ __forceinline__ void w8a16_issue_chunk(int ch, uint8_t* smem, int stage, int kb, int wave,
                                                  __amdgpu_buffer_rsrc_t rX, __amdgpu_buffer_rsrc_t rW,
                                                  const uint32_t (&oa)[ACH], const uint32_t (&ob)[BCH]) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int T = ACH + BCH, CS = (T + NCH - 1) / NCH;
  uint8_t* sA = smem + stage * (BM * 128 + BN * 64);
  uint8_t* sB = sA + BM * 128;
#pragma unroll
  for (int i = 0; i < T; ++i) {
    if (i < ch * CS || i >= ch * CS + CS) continue;
    if (i < ACH)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rX, (lds_ptr_t)(sA + (wave + STRIDE * i) * 1024), 16,
                                               oa[i] + 2u * (uint32_t)kb, 0, 0, 0);
    else
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rW, (lds_ptr_t)(sB + (wave + STRIDE * (i - ACH)) * 1024), 16,
                                               ob[i - ACH] + (uint32_t)kb, 0, 0, 0);
  }
#endif
}

template <typename T, int FMT, int BM, int BN, int OCC, int WM = 2, int WN = 2>
__global__ __launch_bounds__(64 * WM * WN, OCC) void gemm_w8a16_lds_kernel(
    const uint16_t* __restrict__ X, const uint8_t* __restrict__ W, const void* __restrict__ scale, int skind,
    uint16_t* __restrict__ Y, int M, int N, int K, int tiles_m, int tiles_n) {
  constexpr int BK = 64;
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 16, FN = TN / 16;
  constexpr int STAGE = BM * 128 + BN * 64;
  constexpr int ACH = BM / 8 / NW, BCH = BN / 16 / NW;   // 1 KB writer chunks per wave per stage
  static_assert(ACH * 8 * NW == BM && BCH * 16 * NW == BN, "writer chunks");
  // two stages, or the output tile of the epilogue if that is larger
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * STAGE > BM * BN * 2 ? 2 * STAGE : BM * BN * 2];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  int tm, tn;
  tile_of<BM, BN, 8>(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const uint8_t* Xb = reinterpret_cast<const uint8_t*>(X);

  // A writer chunk j: lane i -> row 8 j + (i >> 3), position i & 7
  // B writer chunk j: lane i -> row 16 j + (i >> 2), position i & 3
  const uint8_t* ga[ACH];
  const uint8_t* gb[BCH];
#pragma unroll
  for (int i = 0; i < ACH; ++i) {
    const int row = (wave + NW * i) * 8 + (lane >> 3);
    ga[i] = Xb + ((size_t)min(m0 + row, M - 1) * K) * 2 + ((lane & 7) ^ swzA(row)) * 16;
  }
#pragma unroll
  for (int i = 0; i < BCH; ++i) {
    const int row = (wave + NW * i) * 16 + (lane >> 2);
    gb[i] = W + (size_t)min(n0 + row, N - 1) * K + ((lane & 3) ^ swzB(row)) * 16;
  }

  const int r16 = lane & 15, g = lane >> 4;
  const int pa0 = (2 * g) ^ swzA(r16), pa1 = (2 * g + 1) ^ swzA(r16), pb = g ^ swzB(r16);

  f4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  const int KT = K / BK;
  w8a16_issue<BM, BN, ACH, BCH, NW>(smem, 0, 0, wave, ga, gb);
  for (int kt = 0; kt < KT; ++kt) {
    __syncthreads();  // this step's stage has landed; the other stage is free
    if (kt + 1 < KT) w8a16_issue<BM, BN, ACH, BCH, NW>(smem, (kt + 1) & 1, (kt + 1) * BK, wave, ga, gb);
    const uint8_t* sA = smem + (kt & 1) * STAGE + (wm * TM + r16) * 128;
    const uint8_t* sB = smem + (kt & 1) * STAGE + BM * 128 + (wn * TN + r16) * 64;
    u4 blo[FN], bhi[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) decode16<T, FMT>(*reinterpret_cast<const u4*>(sB + j * 16 * 64 + pb * 16), blo[j], bhi[j]);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const u4 alo = *reinterpret_cast<const u4*>(sA + i * 16 * 128 + pa0 * 16);
      const u4 ahi = *reinterpret_cast<const u4*>(sA + i * 16 * 128 + pa1 * 16);
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        acc[i][j] = mfma16x16x32<T>(alo, blo[j], acc[i][j]);
        acc[i][j] = mfma16x16x32<T>(ahi, bhi[j], acc[i][j]);
      }
    }
  }

  static_assert(sizeof(smem) >= out_tile_bytes(BM, BN), "output tile must fit the stages");
  store_tile<T, BM, BN, WM, WN, 64 * NW>(acc, smem, wm, wn, lane, m0, n0, M, N, nullptr, nullptr, 1.f, Y, 0, 0, scale,
                                         skind);
}

// ---------------------------------------------------------------------------
// w8a16, LDS-tiled with register-pipelined fragment reads: the stage layout,
// swizzles and direct-to-LDS loads of gemm_w8a16_lds_kernel, with the order
// of work of gemm_a8w8_pipe_kernel.  A wave's K step (64 values) is FM groups
// of FN MFMA block updates (two 16 x 16 x 32 MFMAs each); group i + 1's A
// fragment is read while group i's MFMAs run, and the step's one barrier
// sits before the last group, after which the loader waves (the first LW)
// issue the loads of step k + RING into the stage step k used and every wave
// reads and decodes step k + 1's B fragments and first A fragment behind the
// last group's MFMAs.  Loader waves, ring slots (RING stages, loads RING - 1
// steps ahead) and buffer loads as in gemm_a8w8_pipe_kernel.  NCH > 1 (the
// loads in chunks over the MFMA groups) measured 1-4% slower here than all
// of a step's loads after the barrier, so the launches use NCH = 1.
// Requires K % 64 == 0, FM even, 16-byte aligned X and W.
// ---------------------------------------------------------------------------
template <typename T, int FMT, int BM, int BN, int WM, int WN, int LW, int RING = 2, int NCH = 1>
struct W8Pipe {
  static constexpr int BK = 64;
  static constexpr int NW = WM * WN;
  static constexpr int TM = BM / WM, TN = BN / WN;
  static constexpr int FM = TM / 16, FN = TN / 16;
  static constexpr int STAGE = BM * 128 + BN * 64;
  static constexpr int ACH = BM / 8 / LW, BCH = BN / 16 / LW;  // 1 KB loads per loader wave and stage
  static_assert(LW >= 1 && LW <= NW, "loader waves");
  static_assert(ACH * 8 * LW == BM && BCH * 16 * LW == BN, "writer chunks");
  static_assert(FM % 2 == 0, "A fragments alternate between two register sets");

  // A fragment (rows r16 of a 16-row block, K values 16 g .. 16 g + 15)
  __device__ static inline void read_a(const uint8_t* row, int pa0, int pa1, u4 (&a)[2]) {
    a[0] = *reinterpret_cast<const u4*>(row + pa0 * 16);
    a[1] = *reinterpret_cast<const u4*>(row + pa1 * 16);
  }
  // B fragments of a step, decoded to the activation type
  __device__ static inline void read_b(const uint8_t* sB, int pb, u4 (&b)[FN][2]) {
#pragma unroll
    for (int j = 0; j < FN; ++j) decode16<T, FMT>(*reinterpret_cast<const u4*>(sB + j * 16 * 64 + pb * 16), b[j][0], b[j][1]);
  }

  // step kt from ring slot c (the next step's slot cn); the loads are issued
  // in NCH chunks as in a8w8_pipe_step
  __device__ static __forceinline__ void step(int kt, int KT, int c, int cn, uint8_t* smem, bool loader, int wave, int wm,
                                              int wn, int r16, int pa0, int pa1, int pb, __amdgpu_buffer_rsrc_t rX,
                                              __amdgpu_buffer_rsrc_t rW, const uint32_t (&ga)[ACH],
                                              const uint32_t (&gb)[BCH], f4 (&acc)[FM][FN], u4 (&a)[2][2],
                                              const u4 (&bc)[FN][2], u4 (&bn)[FN][2]) {
    static_assert(NCH >= 1 && NCH <= FM, "chunks 1 .. NCH - 1 go out in the groups before the barrier");
    const uint8_t* sA = smem + c * STAGE + (wm * TM + r16) * 128;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      if (i + 1 < FM) {
        read_a(sA + (i + 1) * 16 * 128, pa0, pa1, a[(i + 1) & 1]);
        if (i < NCH - 1 && loader && kt >= 1 && kt + RING - 1 < KT)
          w8a16_issue_chunk<BM, BN, ACH, BCH, LW, NCH>(i + 1, smem, c == 0 ? RING - 1 : c - 1, (kt + RING - 1) * BK, wave,
                                                       rX, rW, ga, gb);
      } else if (kt + 1 < KT) {
        // step k + 1 has landed (later steps' loads may fly); slot c is free
        barrier_upto<RING - 2, ACH + BCH>(KT - 2 - kt);
        if (loader && kt + RING < KT)
          w8a16_issue_chunk<BM, BN, ACH, BCH, LW, NCH>(0, smem, c, (kt + RING) * BK, wave, rX, rW, ga, gb);
        const uint8_t* nxt = smem + cn * STAGE;
        read_b(nxt + BM * 128 + (wn * TN + r16) * 64, pb, bn);
        read_a(nxt + (wm * TM + r16) * 128, pa0, pa1, a[0]);
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        acc[i][j] = mfma16x16x32<T>(a[i & 1][0], bc[j][0], acc[i][j]);
        acc[i][j] = mfma16x16x32<T>(a[i & 1][1], bc[j][1], acc[i][j]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
};

// SPLIT > 1 (split K): workgroup b computes tile b / SPLIT over the K range
// of part b % SPLIT ((K / SPLIT) % 64 == 0) and stores its unscaled fp32
// sums to part P[b % SPLIT] of the [SPLIT][M][N] workspace P;
// gemm_splitk_finalize_w then adds the parts in order and scales.
template <typename T, int FMT, int BM, int BN, int OCC, int WM, int WN, int LW, int SPLIT = 1, int RING = 2, int NCH = 1>
__global__ __launch_bounds__(64 * WM * WN, OCC) void gemm_w8a16_pipe_kernel(
    const uint16_t* __restrict__ X, const uint8_t* __restrict__ W, const void* __restrict__ scale, int skind,
    uint16_t* __restrict__ Y, float* __restrict__ Pw, int M, int N, int K, int tiles_m, int tiles_n) {
  using P = W8Pipe<T, FMT, BM, BN, WM, WN, LW, RING, NCH>;
  constexpr int BK = P::BK, NW = P::NW, TM = P::TM, TN = P::TN, FM = P::FM, FN = P::FN, STAGE = P::STAGE;
  constexpr int ACH = P::ACH, BCH = P::BCH;
  static_assert(RING >= 2 && RING <= 4, "ring slots");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[RING * STAGE > BM * BN * 2 ? RING * STAGE : BM * BN * 2];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const bool loader = wave < LW;
  const int part = SPLIT > 1 ? (int)blockIdx.x % SPLIT : 0;
  const uint32_t kpart = (uint32_t)(part * (K / SPLIT));  // first K value of this part
  int tm, tn;
  tile_of<BM, BN, 8>(SPLIT > 1 ? blockIdx.x / SPLIT : blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const __amdgpu_buffer_rsrc_t rX = buf_rsrc(X, (uint32_t)((size_t)M * K * 2));
  const __amdgpu_buffer_rsrc_t rW = buf_rsrc(W, (uint32_t)((size_t)N * K));

  // A writer chunk j = wave + LW i: lane l -> row 8 j + (l >> 3), position l & 7
  // B writer chunk j = wave + LW i: lane l -> row 16 j + (l >> 2), position l & 3
  // (non-loaders set up clamped pointers they never use)
  uint32_t ga[ACH], gb[BCH];
#pragma unroll
  for (int i = 0; i < ACH; ++i) {
    const int row = (wave + LW * i) * 8 + (lane >> 3);
    ga[i] = (uint32_t)min(m0 + row, M - 1) * (uint32_t)K * 2u + 2u * kpart + (uint32_t)(((lane & 7) ^ swzA(row)) * 16);
  }
#pragma unroll
  for (int i = 0; i < BCH; ++i) {
    const int row = (wave + LW * i) * 16 + (lane >> 2);
    gb[i] = (uint32_t)min(n0 + row, N - 1) * (uint32_t)K + kpart + (uint32_t)(((lane & 3) ^ swzB(row)) * 16);
  }
  const int r16 = lane & 15, g = lane >> 4;
  const int pa0 = (2 * g) ^ swzA(r16), pa1 = (2 * g + 1) ^ swzA(r16), pb = g ^ swzB(r16);

  f4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  const int KT = K / BK / SPLIT;
  // prologue: steps 0 .. RING - 1 into their slots, then wait for step 0
  if (loader) {
#pragma unroll
    for (int s = 0; s < RING; ++s)
      if (s == 0 || s < KT) w8a16_issue_chunk<BM, BN, ACH, BCH, LW, 1>(0, smem, s, s * BK, wave, rX, rW, ga, gb);
  }
  barrier_upto<RING - 1, ACH + BCH>(KT - 1);
  u4 a[2][2], b0[FN][2], b1[FN][2];
  P::read_b(smem + BM * 128 + (wn * TN + r16) * 64, pb, b0);
  P::read_a(smem + (wm * TM + r16) * 128, pa0, pa1, a[0]);
  int kt = 0, c = 0;
  auto nxt = [](int v) { return v + 1 == RING ? 0 : v + 1; };
  for (; kt + 1 < KT; kt += 2) {
    const int c1 = RING == 2 ? 1 : nxt(c), c2 = RING == 2 ? 0 : nxt(c1);
    P::step(kt, KT, RING == 2 ? 0 : c, c1, smem, loader, wave, wm, wn, r16, pa0, pa1, pb, rX, rW, ga, gb, acc, a, b0,
            b1);
    P::step(kt + 1, KT, c1, c2, smem, loader, wave, wm, wn, r16, pa0, pa1, pb, rX, rW, ga, gb, acc, a, b1, b0);
    c = c2;
  }
  if (kt < KT)
    P::step(kt, KT, RING == 2 ? 0 : c, RING == 2 ? 1 : nxt(c), smem, loader, wave, wm, wn, r16, pa0, pa1, pb, rX, rW,
            ga, gb, acc, a, b0, b1);

  static_assert(sizeof(smem) >= out_tile_bytes(BM, BN), "output tile must fit the stages");
  if constexpr (SPLIT > 1) {
    // fp32 partial sums in D layout: lane l holds column l & 15, rows
    // 4 (l >> 4) + v of each 16 x 16 block (rows and columns past the
    // matrix are clamped copies, not stored)
    float* Pp = Pw + (size_t)part * M * N;
    const int g4 = (lane >> 4) * 4;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int n = n0 + wn * TN + j * 16 + r16;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int m = m0 + wm * TM + i * 16 + g4 + v;
          if (m < M && n < N) Pp[(size_t)m * N + n] = acc[i][j][v];
        }
      }
  } else {
    store_tile<T, BM, BN, WM, WN, 64 * NW>(acc, smem, wm, wn, lane, m0, n0, M, N, nullptr, nullptr, 1.f, Y, 0, 0,
                                           scale, skind);
  }
}

// ---------------------------------------------------------------------------
// w8a16 with N <= 16 and M > 16 (the reference's tiny-N M-parallel path,
// fp8_GEMM_pert.h:3913-3994 via the dispatcher at :4030-4046): here the
// activations are the large operand, so the roles flip.  A workgroup owns 16
// activation rows and streams them once; the N (<= 16) weight rows, a few KB
// that stay in L2, are decoded into the MFMA B operand (rows >= N read row
// N - 1 and are never stored).  Lane l takes row l & 15 and the 16 K values
// 16 (l >> 4) .. + 15 of each 64-value step (32 bytes of x, 16 of w); the
// four waves take the steps s with s % 4 == wave, U in flight, and meet in
// LDS.  Requires K % 64 == 0 and 16-byte aligned x and w.
// ---------------------------------------------------------------------------
template <typename T, int FMT, int U>
__global__ __launch_bounds__(256) void gemm_w8a16_tinyn_kernel(const uint16_t* __restrict__ X,
                                                               const uint8_t* __restrict__ W,
                                                               const void* __restrict__ scale, int skind,
                                                               uint16_t* __restrict__ Y, int M, int N, int K) {
  __shared__ f4 red[3][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  const int m0 = blockIdx.x * 16;
  const uint16_t* xrow = X + (size_t)min(m0 + r16, M - 1) * K + g * 16;  // rows >= M are never stored
  const uint8_t* wrow = W + (size_t)min(r16, N - 1) * K + g * 16;
  const int steps = K >> 6;
  f4 acc = f4{0.f, 0.f, 0.f, 0.f};
  for (int s0 = wave; s0 < steps; s0 += 4 * U) {
    u4 xa[U], xb[U], wv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = s0 + 4 * u;
      if (s < steps) {
        const u4* xp = reinterpret_cast<const u4*>(xrow + (size_t)s * 64);
        xa[u] = load_u4_stream(xp);
        xb[u] = load_u4_stream(xp + 1);
        wv[u] = load_u4(wrow + (size_t)s * 64);
      } else {
        xa[u] = xb[u] = wv[u] = u4{0, 0, 0, 0};
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // every load of the round before any arithmetic
#pragma unroll
    for (int u = 0; u < U; ++u) {
      u4 lo, hi;
      decode16<T, FMT>(wv[u], lo, hi);
      acc = mfma16x16x32<T>(xa[u], lo, acc);
      acc = mfma16x16x32<T>(xb[u], hi, acc);
    }
  }
  if (wave > 0) red[wave - 1][lane] = acc;
  // the column's weight scale, loaded by every lane before the branches
  // below (columns >= N read column N - 1 and are never stored)
  const float sc = load_scale(scale, skind, min(r16, N - 1));
  __syncthreads();
  if (wave != 0) return;
  const f4 c = acc + red[0][lane] + red[1][lane] + red[2][lane];
  const int n = r16;  // D column = lane & 15
  if (n >= N) return;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int m = m0 + 4 * g + v;  // D row = 4 * (lane >> 4) + v
    if (m < M) Y[(size_t)m * N + n] = T::from_f32(c[v] * sc);
  }
}

// ---------------------------------------------------------------------------
// w8a16, direct-from-global v0: 64 x 64 C tile per workgroup, K step 64.
// ---------------------------------------------------------------------------


template <typename T, int FMT>
__global__ __launch_bounds__(256) void gemm_w8a16_simple_kernel(
    const uint16_t* __restrict__ X, const uint8_t* __restrict__ W, const void* __restrict__ scale, int skind,
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
  float sc[2];  // the columns' weight scales, loaded before any branch (column N - 1 past N)
#pragma unroll
  for (int j = 0; j < 2; ++j) sc[j] = load_scale(scale, skind, min(n0 + j * 16 + r16, N - 1));
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + j * 16 + r16;
    if (n >= N) continue;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = m0 + i * 16 + g * 4 + v;
        if (m < M) Y[(size_t)m * N + n] = T::from_f32(acc[i][j][v] * sc[j]);
      }
  }
}

}  // namespace cek

using namespace cek;

namespace cek {

// loader waves of the score-picked w8a16 pipelined launches (one per SIMD),
// and the row layout of gemm_a8w8_lds_kernel's launches
constexpr int kW8a16Loaders = 4;
constexpr int kA8w8LdsLayout = 1;

// w8a16 product for any M with a weight scale of kind skind (ScaleKind):
// M <= 16 the GEMV kernels, N <= 16 the activation-streaming kernel,
// 16 < M <= 32 the LDS-staged GEMV where it has an instantiation, else the
// tiled MFMA GEMM (or the generic kernels for unaligned shapes).
// Tiled w8a16 configurations of the round model (M, N >= 128, matrices
// below 4 GB): the 8-wave register-pipelined kernel (2 x 4 waves, four
// loader waves) with its ring slots, and t0 / step of the round model (us
// per round: t0 + step per 64-deep K step of one workgroup), fitted to the
// nine config-4 shapes with operands streamed from HBM (MI355X):
//  0  256 x 128, 3 slots;   1  256 x 192, 3 slots;   2  256 x 256, 2 slots;
//  3  128 x 256, 3 slots;   4  128 x 128, 3 slots (split K only);
//  5  128 x 96 (4 x 2 waves, two loader waves), 3 slots, unsplit, only as one
//     round of 192 .. 256 tiles with K <= 8192 (fitted at M = 512, N = 6144).
// Unsplit: 0-3 and 5; split in 2, 4 or 8 parts (K values per part >= 1024): 0
// and 3, and 4 in 4 or 8 parts.  On the nine config-4 shapes (HBM and
// cache-resident) and ten others (M = 128 .. 3000) the plan's pick measured
// within 7% of the fastest of sixteen forms (M = 512, K = 14336: 171 -> 68 us
// split in 4; M = 512, K = 4096, N = 6144: 52 -> 36 us).
struct W8Opt { int bm, bn; double t0, step; };
constexpr int kW8Cfgs = 6;
constexpr W8Opt kW8Opts[kW8Cfgs] = {{256, 128, 0.49, 0.972}, {256, 192, 6.84, 1.166}, {256, 256, 0.0, 1.595},
                                    {128, 256, 2.05, 0.904}, {128, 128, 0.0, 0.491},  {128, 96, 4.30, 0.447}};
struct W8Plan { int cfg, split; };

static bool w8_off32(int64_t M, int64_t N, int64_t K) {
  return (uint64_t)M * (uint64_t)K * 2 < (1ull << 32) && (uint64_t)N * (uint64_t)K < (1ull << 32);
}

// cfg -1: the shape is outside the round model (the score-based choice of
// launch_w8a16 applies)
static W8Plan plan_w8a16(int64_t M, int64_t N, int64_t K, bool allow_split) {
  W8Plan best{-1, 1};
  if (M < 128 || N < 128 || K % 64 != 0 || !w8_off32(M, N, K)) return best;
  double tbest = -1.0;
  for (int c = 0; c < kW8Cfgs; ++c) {
    const W8Opt& o = kW8Opts[c];
    if (M < o.bm || N < o.bn) continue;
    for (int sp : {1, 2, 4, 8}) {
      const bool ok = sp == 1 ? c != 4 : (allow_split && (c == 0 || c == 3 || (c == 4 && sp >= 4)));
      if (!ok || (K / 64) % sp || (sp > 1 && K / sp < 1024)) continue;
      const int64_t units = ((M + o.bm - 1) / o.bm) * ((N + o.bn - 1) / o.bn) * sp;
      // 128 x 96 only as one nearly full round of at most 8192 K values, where
      // it was measured (M = 384 / 512, N = 6144, K = 1024 .. 8192; with a
      // quarter or more of the CUs idle, or two rounds, it lost)
      if (c == 5 && (units > 256 || units < 192 || K > 8192)) continue;
      const int64_t full = units / 256;
      const double f = (double)(units - full * 256) / 256.0;
      const double rounds = (double)full + (f > 0.0 ? 0.6 + 0.4 * f : 0.0);
      double t = rounds * (o.t0 + (double)(K / 64 / sp) * o.step);
      if (sp > 1) t += ((double)sp * M * N * 4.0 + (double)M * N * 2.0) / 5.0e6 + 1.5;
      if (tbest < 0 || t < tbest) {
        tbest = t;
        best = W8Plan{c, sp};
      }
    }
  }
  return best;
}

// Bytes of fp32 partials the w8a16 split-K plan needs for (M, N, K) (0: unsplit).
static int64_t w8a16_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 32 || N <= 16 || M > 65535 * 64 || N > INT32_MAX || K > INT32_MAX || K <= 0) return 0;
  const W8Plan p = plan_w8a16(M, N, K, true);
  return p.split > 1 ? (int64_t)p.split * M * N * 4 : 0;
}

int launch_w8a16(const void* x, const void* w, const void* scale, int skind, void* y, int64_t M, int64_t N, int64_t K,
                 int io_dtype, int fp8_fmt, float* ws, int64_t ws_bytes, hipStream_t st) {
  if (M < 0 || N < 0 || K <= 0 || M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) return CEK_ERR_INVALID;
  if (M == 0 || N == 0) return CEK_OK;
  if (!x || !w || !scale || !y) return CEK_ERR_INVALID;
  if (io_dtype != CEK_F16 && io_dtype != CEK_BF16) return CEK_ERR_INVALID;
  if (fp8_fmt != CEK_E4M3 && fp8_fmt != CEK_E5M2) return CEK_ERR_INVALID;
  if (skind < SK_F16 || skind > SK_F32_SCALAR) return CEK_ERR_INVALID;
  if (M <= 16) return launch_gemv(x, w, scale, skind, y, M, N, K, io_dtype, fp8_fmt, st);
  if (N <= 16 && K % 64 == 0 && aligned(x, 16) && aligned(w, 16) && M <= (int64_t)INT32_MAX - 16) {
    const dim3 grid((unsigned)((M + 15) / 16));
    const uint16_t* xp = static_cast<const uint16_t*>(x);
    const uint8_t* wp = static_cast<const uint8_t*>(w);
    uint16_t* yp = static_cast<uint16_t*>(y);
#define CEK_TINYN(TY, F) gemm_w8a16_tinyn_kernel<TY, F, 4><<<grid, 256, 0, st>>>(xp, wp, scale, skind, yp, (int)M, (int)N, (int)K)
    if (io_dtype == CEK_F16 && fp8_fmt == CEK_E4M3) CEK_TINYN(F16, CEK_E4M3);
    else if (io_dtype == CEK_F16) CEK_TINYN(F16, CEK_E5M2);
    else if (fp8_fmt == CEK_E4M3) CEK_TINYN(BF16, CEK_E4M3);
    else CEK_TINYN(BF16, CEK_E5M2);
#undef CEK_TINYN
    return check_launch();
  }
  if (M <= 32 && aligned(x, 16) && aligned(w, 16)) {
    const int rc = launch_gemv_wide(x, w, scale, skind, y, M, N, K, io_dtype, fp8_fmt, st);
    if (rc != CEK_ERR_UNSUPPORTED) return rc;
  }
  if (K % 64 != 0 || !aligned(x, 16) || !aligned(w, 16) || M > 65535 * 64)
    return launch_gemv_generic(x, w, scale, skind, y, M, N, K, io_dtype, fp8_fmt, st);
  {
    const int64_t need = w8a16_workspace_bytes(M, N, K);
    const W8Plan plan = plan_w8a16(M, N, K, need > 0 && ws && ws_bytes >= need);
    if (plan.cfg >= 0) {
      const uint16_t* xp = static_cast<const uint16_t*>(x);
      const uint8_t* wp = static_cast<const uint8_t*>(w);
      uint16_t* yp = static_cast<uint16_t*>(y);
#define CEK_W8P(TY, F, BM, BN, SP, RING)                                                                         \
  do {                                                                                                          \
    const int tm = (int)((M + BM - 1) / BM), tn = (int)((N + BN - 1) / BN);                                     \
    gemm_w8a16_pipe_kernel<TY, F, BM, BN, 1, 2, 4, 4, SP, RING>                                                 \
        <<<dim3((unsigned)(tm * tn * SP)), 512, 0, st>>>(xp, wp, scale, skind, yp, ws, M, N, K, tm, tn);         \
    if (SP > 1)                                                                                                 \
      gemm_splitk_finalize_w<TY, SP><<<dim3((unsigned)((N + 2047) / 2048), (unsigned)(M < 65535 ? M : 65535)),  \
                                        256, 0, st>>>(ws, scale, skind, yp, (int)M, (int)N);                     \
  } while (0)
// 128 x 96: waves 4 x 2 (32 x 48 wave tiles), two loader waves (the 16-row
// B load chunks of 96 rows split evenly over 2), 3 slots
#define CEK_W8P96(TY, F)                                                                                         \
  do {                                                                                                          \
    const int tm = (int)((M + 127) / 128), tn = (int)((N + 95) / 96);                                           \
    gemm_w8a16_pipe_kernel<TY, F, 128, 96, 1, 4, 2, 2, 1, 3>                                                    \
        <<<dim3((unsigned)(tm * tn)), 512, 0, st>>>(xp, wp, scale, skind, yp, ws, M, N, K, tm, tn);             \
  } while (0)
#define CEK_W8P_SPLITS(TY, F, BM, BN)                        \
  do {                                                       \
    if (plan.split == 2) CEK_W8P(TY, F, BM, BN, 2, 3);       \
    else if (plan.split == 4) CEK_W8P(TY, F, BM, BN, 4, 3);  \
    else CEK_W8P(TY, F, BM, BN, 8, 3);                       \
  } while (0)
#define CEK_W8P_ALL(TY, F)                                                 \
  do {                                                                     \
    if (plan.split > 1) {                                                  \
      if (plan.cfg == 0) CEK_W8P_SPLITS(TY, F, 256, 128);                  \
      else if (plan.cfg == 3) CEK_W8P_SPLITS(TY, F, 128, 256);             \
      else if (plan.split == 4) CEK_W8P(TY, F, 128, 128, 4, 3);            \
      else CEK_W8P(TY, F, 128, 128, 8, 3);                                 \
    } else if (plan.cfg == 0) {                                            \
      CEK_W8P(TY, F, 256, 128, 1, 3);                                      \
    } else if (plan.cfg == 1) {                                            \
      CEK_W8P(TY, F, 256, 192, 1, 3);                                      \
    } else if (plan.cfg == 2) {                                            \
      CEK_W8P(TY, F, 256, 256, 1, 2);                                      \
    } else if (plan.cfg == 5) {                                            \
      CEK_W8P96(TY, F);                                                    \
    } else {                                                               \
      CEK_W8P(TY, F, 128, 256, 1, 3);                                      \
    }                                                                      \
  } while (0)
      if (io_dtype == CEK_F16 && fp8_fmt == CEK_E4M3) CEK_W8P_ALL(F16, CEK_E4M3);
      else if (io_dtype == CEK_F16) CEK_W8P_ALL(F16, CEK_E5M2);
      else if (fp8_fmt == CEK_E4M3) CEK_W8P_ALL(BF16, CEK_E4M3);
      else CEK_W8P_ALL(BF16, CEK_E5M2);
#undef CEK_W8P_ALL
#undef CEK_W8P96
#undef CEK_W8P_SPLITS
#undef CEK_W8P
      return check_launch();
    }
  }
  {
    // Tiles: 128 x 128 with 4 waves and two workgroups per CU, or the
    // register-pipelined 8-wave kernel (2 x 4 waves, four loader waves) at
    // 256 x 128, 256 x 192 or 256 x 256 -- each configuration's measured rate
    // (MI355X, config-4 shapes with fp16 activations, TFLOP/s at full
    // occupancy) times the fill of its last round over 256 CUs, best score
    // wins.  (256 x 128: 205 us at M = 2048, K = 14336, N = 4096, against
    // 217 us for 128 x 128.)
    auto score = [&](int bm, int bn, double rate, int slots) {
      const int64_t tiles = ((M + bm - 1) / bm) * ((N + bn - 1) / bn);
      const int64_t rounds = (tiles + slots - 1) / slots;
      // useful share of the tile area the rounds could cover
      return rate * (double)(M * N) / ((double)(rounds * slots) * bm * bn);
    };
    // the pipelined kernel addresses X and W by 32-bit byte offsets
    const bool off32 = w8_off32(M, N, K);
    const double s128 = score(128, 128, 1150, 512);
    const double s192 = off32 ? score(256, 192, 1250, 256) : -1.0;
    const double s256 = off32 ? score(256, 256, 1400, 256) : -1.0;
    // 256 x 128 only from one full round of tiles (at M = 512 it measured
    // 24-28% slower than 128 x 128, whose fill the score rates the same)
    const bool full256n128 = ((M + 255) / 256) * ((N + 127) / 128) >= 256;
    const double s256n128 = off32 && full256n128 ? score(256, 128, 1170, 256) : -1.0;
    const double best = std::max(std::max(s128, s192), std::max(s256, s256n128));
    const int tile = best == s256 ? 2 : (best == s192 ? 1 : (best == s256n128 ? 3 : 0));
    const uint16_t* xp = static_cast<const uint16_t*>(x);
    const uint8_t* wp = static_cast<const uint8_t*>(w);
    uint16_t* yp = static_cast<uint16_t*>(y);
#define CEK_W8A16_TILE(TY, F, BM, BN, OCC, WM, WN)                                                                 \
  do {                                                                                                         \
    const int tm = (int)((M + BM - 1) / BM), tn = (int)((N + BN - 1) / BN);                                    \
    gemm_w8a16_lds_kernel<TY, F, BM, BN, OCC, WM, WN>                                                          \
        <<<dim3((unsigned)(tm * tn)), 64 * WM * WN, 0, st>>>(xp, wp, scale, skind, yp, M, N, K, tm, tn);       \
  } while (0)
#define CEK_W8A16_PIPE(TY, F, BM, BN, OCC, WM, WN)                                                                 \
  do {                                                                                                         \
    const int tm = (int)((M + BM - 1) / BM), tn = (int)((N + BN - 1) / BN);                                    \
    gemm_w8a16_pipe_kernel<TY, F, BM, BN, OCC, WM, WN, kW8a16Loaders>                                                        \
        <<<dim3((unsigned)(tm * tn)), 64 * WM * WN, 0, st>>>(xp, wp, scale, skind, yp, nullptr, M, N, K, tm, tn); \
  } while (0)
#define CEK_W8A16(TY, F)                                          \
  do {                                                            \
    if (tile == 2) CEK_W8A16_PIPE(TY, F, 256, 256, 1, 2, 4);      \
    else if (tile == 1) CEK_W8A16_PIPE(TY, F, 256, 192, 1, 2, 4); \
    else if (tile == 3) CEK_W8A16_PIPE(TY, F, 256, 128, 1, 2, 4); \
    else CEK_W8A16_TILE(TY, F, 128, 128, 2, 2, 2);                \
  } while (0)
    if (io_dtype == CEK_F16 && fp8_fmt == CEK_E4M3) CEK_W8A16(F16, CEK_E4M3);
    else if (io_dtype == CEK_F16) CEK_W8A16(F16, CEK_E5M2);
    else if (fp8_fmt == CEK_E4M3) CEK_W8A16(BF16, CEK_E4M3);
    else CEK_W8A16(BF16, CEK_E5M2);
#undef CEK_W8A16
#undef CEK_W8A16_TILE
#undef CEK_W8A16_PIPE
    return check_launch();
  }
  dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64));
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const uint8_t* wp = static_cast<const uint8_t*>(w);
  uint16_t* yp = static_cast<uint16_t*>(y);
  if (io_dtype == CEK_F16 && fp8_fmt == CEK_E4M3) gemm_w8a16_simple_kernel<F16, CEK_E4M3><<<grid, 256, 0, st>>>(xp, wp, scale, skind, yp, M, N, K);
  else if (io_dtype == CEK_F16) gemm_w8a16_simple_kernel<F16, CEK_E5M2><<<grid, 256, 0, st>>>(xp, wp, scale, skind, yp, M, N, K);
  else if (fp8_fmt == CEK_E4M3) gemm_w8a16_simple_kernel<BF16, CEK_E4M3><<<grid, 256, 0, st>>>(xp, wp, scale, skind, yp, M, N, K);
  else gemm_w8a16_simple_kernel<BF16, CEK_E5M2><<<grid, 256, 0, st>>>(xp, wp, scale, skind, yp, M, N, K);
  return check_launch();
}

}  // namespace cek

extern "C" int cek_gemm_fp8_pert(const void* x, const void* w, const float* scale, void* y,
                                 int64_t M, int64_t N, int64_t K,
                                 int io_dtype, int fp8_fmt, void* stream) {
  return cek::launch_w8a16(x, w, scale, cek::SK_F32_SCALAR, y, M, N, K, io_dtype, fp8_fmt, nullptr, 0,
                           (hipStream_t)stream);
}

extern "C" int64_t cek_gemm_fp8_pert_workspace_size(int64_t M, int64_t N, int64_t K) {
  return cek::w8a16_workspace_bytes(M, N, K);
}

extern "C" int cek_gemm_fp8_pert_ws(const void* x, const void* w, const float* scale, void* y, int64_t M, int64_t N,
                                    int64_t K, int io_dtype, int fp8_fmt, void* workspace, int64_t workspace_bytes,
                                    void* stream) {
  if (workspace_bytes < 0 || (workspace_bytes > 0 && (!workspace || !cek::aligned(workspace, 4)))) return CEK_ERR_INVALID;
  return cek::launch_w8a16(x, w, scale, cek::SK_F32_SCALAR, y, M, N, K, io_dtype, fp8_fmt,
                           static_cast<float*>(workspace), workspace_bytes, (hipStream_t)stream);
}

namespace cek {

// Tiled a8w8 configurations.  Rate: measured TFLOP/s at full occupancy
// (cache-resident operands; the model for M < 128 and matrices above 4 GB).
// Slots: workgroups over 256 CUs at once.  t0 / step: the round model fitted
// to the nine config-4 shapes with operands streamed from HBM (us per round:
// t0 + step per 128-deep K step of one workgroup; every launch below timed
// on MI355X).
//  0  64 x 128, 4 waves (2 x 2), two workgroups per CU, 2 ring slots;
//  1  128 x 128, 4 waves, two per CU (one's MFMAs cover the other's LDS
//     reads and barrier waits), 2 slots;
//  2  256 x 192, 8 waves (2 x 4, four loader waves), 2 slots;
//  3  256 x 256, 8 waves (wave tile 128 x 64, two waves per SIMD): the least
//     load and LDS traffic per MFMA, 2 slots (128 KB of LDS);
//  4  128 x 128, 8 waves (2 x 4, four loader waves), 3 slots: loads two
//     steps ahead, one workgroup per CU;
//  5  128 x 256, 8 waves, 3 slots;
//  6  256 x 128, 8 waves, 3 slots;
//  7  128 x 96, 8 waves (4 x 2, wave tile 32 x 48, four loader waves), 3
//     slots: 256 tiles at M = 512, N = 6144 (K = 4096 from HBM 21.2 -> 19.2
//     us against 4; t0 / step fitted against 4's model at K = 1024 .. 8192).
// The 3-slot tiles are for weights streamed from HBM, whose latency one step
// of lead does not cover on a small tile (M = 512, K = 4096, N = 6144: 64 x
// 128 in 2 slots 32.0 us, 128 x 128 8-wave in 3 slots 21.5 us).
struct A8w8Opt { int bm, bn; double rate; int slots; double t0, step; };
constexpr int kA8w8Cfgs = 8;
constexpr A8w8Opt kA8w8Opts[kA8w8Cfgs] = {
    {64, 128, 1750, 512, 0.0, 0.686},   {128, 128, 2250, 512, 1.56, 1.085}, {256, 192, 2480, 256, 0.0, 1.461},
    {256, 256, 2650, 256, 0.0, 1.760},  {128, 128, 0, 256, 2.87, 0.560},    {128, 256, 0, 256, 3.65, 0.914},
    {256, 128, 0, 256, 2.99, 0.957},    {128, 96, 0, 256, 2.40, 0.453}};
constexpr bool a8w8_splits(int c) { return c == 1 || c == 5 || c == 6; }

struct A8w8Plan { int cfg, split; };

// Round model (us) of configuration c with K in sp parts: U workgroups over
// S slots run floor(U / S) full rounds and, for a last round of fill f,
// 0.6 + 0.4 f of one (its workgroups share HBM and L2 with fewer others); a
// round takes t0 + step per K step of a part.  Split adds the finalize: the
// parts read and the output written at ~5 TB/s, plus a launch.
static double a8w8_round_us(const A8w8Opt& o, int64_t M, int64_t N, int64_t K, int sp) {
  const int64_t units = ((M + o.bm - 1) / o.bm) * ((N + o.bn - 1) / o.bn) * sp;
  const int64_t full = units / o.slots;
  const double f = (double)(units - full * o.slots) / (double)o.slots;
  const double rounds = (double)full + (f > 0.0 ? 0.6 + 0.4 * f : 0.0);
  double t = rounds * (o.t0 + (double)(K / 128 / sp) * o.step);
  if (sp > 1) t += ((double)sp * M * N * 4.0 + (double)M * N * 2.0) / 5.0e6 + 1.5;
  return t;
}

// M >= 128 on the pipelined path: the fastest configuration by the round
// model, split in 2, 4 or 8 parts (at least 1024 K values each) where
// allowed.  Fitted on the nine config-4 shapes (weights from HBM), it picks
// the measured fastest on all nine, with cache-resident operands too; on
// twelve other shapes (M = 128 .. 3000, K = 2048 .. 14336, ragged N) within
// 6% of the fastest of thirteen measured forms.
static A8w8Plan plan_a8w8_rounds(int64_t M, int64_t N, int64_t K, bool allow_split) {
  A8w8Plan best{1, 1};
  double tbest = -1.0;
  for (int c = 0; c < kA8w8Cfgs; ++c) {
    const A8w8Opt& o = kA8w8Opts[c];
    if (M < o.bm || N < o.bn) continue;
    for (int sp : {1, 2, 4, 8}) {
      if (sp > 1 && (!allow_split || !a8w8_splits(c) || (K / 128) % sp || K / sp < 1024)) continue;
      const double t = a8w8_round_us(o, M, N, K, sp);
      if (tbest < 0 || t < tbest) {
        tbest = t;
        best = A8w8Plan{c, sp};
      }
    }
  }
  return best;
}

// Below 128 rows or columns (only the 64 x 128 tile fits), or with matrices
// above 4 GB (the clamped-load kernel, configurations 0-3): each configuration's
// rounds of workgroups at its full-occupancy rate (a partial round costs a
// full one), the 64 x 128 tile also split in 2, 4 or 8 parts plus the fp32
// partials' traffic and the finalize launch; split only when allowed, on the
// pipelined path, and 10% faster than the best unsplit plan.  At M = 64
// (config 3's prefill-sized decode) the split plans measured 1.2-1.8x faster
// than the weight-streaming kernels, and 8 parts of 512 K values slower than
// 4 (M = 64, K = 4096: 13.8 against 11.2 us).  The split 64 x 128 launches
// run a 3-slot ring (72 KB per workgroup, two per CU): M = 64, N = 6144,
// weights from HBM, K = 4096 15.3 -> 13.2 us, K = 5120 16.0 -> 13.2 us; M = 96
// 17.4 -> 16.4 us.
static A8w8Plan plan_a8w8(int64_t M, int64_t N, int64_t K, bool pipe_ok, bool allow_split) {
  if (pipe_ok && M >= 128 && N >= 128) return plan_a8w8_rounds(M, N, K, allow_split);
  A8w8Plan best{0, 1};
  double tbest = -1.0;
  for (int c = 0; c < 4; ++c) {
    const A8w8Opt& o = kA8w8Opts[c];
    const int64_t tiles = ((M + o.bm - 1) / o.bm) * ((N + o.bn - 1) / o.bn);
    const int64_t rounds = (tiles + o.slots - 1) / o.slots;
    const double t = (double)(rounds * o.slots) * 2.0 * o.bm * o.bn * (double)K / (o.rate * 1e12);
    if (tbest < 0 || t < tbest) {
      tbest = t;
      best = A8w8Plan{c, 1};
    }
  }
  if (!allow_split) return best;
  const double tplain = tbest;
  for (int c = 0; c < 2; ++c) {
    const A8w8Opt& o = kA8w8Opts[c];
    if (!pipe_ok || M < o.bm || N < o.bn) continue;
    for (int sp : {2, 4, 8}) {
      if ((K / 128) % sp || K / sp < 1024) continue;
      const int64_t units = ((M + o.bm - 1) / o.bm) * ((N + o.bn - 1) / o.bn) * sp;
      const int64_t rounds = (units + o.slots - 1) / o.slots;
      const double tg = (double)(rounds * o.slots) * 2.0 * o.bm * o.bn * (double)(K / sp) / (o.rate * 1e12);
      // partials written and read back (mostly from the Infinity Cache), the output, a launch
      const double tx = ((double)sp * M * N * 4.0 * 2.0 + (double)M * N * 2.0) / 8e12 + 2e-6;
      if (tg + tx < 0.9 * tplain && tg + tx < tbest) {
        tbest = tg + tx;
        best = A8w8Plan{c, sp};
      }
    }
  }
  return best;
}

static bool a8w8_off32(int64_t M, int64_t N, int64_t K) {
  return (uint64_t)M * (uint64_t)K < (1ull << 32) && (uint64_t)N * (uint64_t)K < (1ull << 32);
}

// Bytes of fp32 partials the split-K plan for this shape needs (0: unsplit).
static int64_t a8w8_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M < 64 || K % 128 != 0 || M > 65535 * 64 || N > INT32_MAX || K > INT32_MAX || M <= 0 || N <= 0) return 0;
  const A8w8Plan p = plan_a8w8(M, N, K, a8w8_off32(M, N, K), true);
  return p.split > 1 ? (int64_t)p.split * M * N * 4 : 0;
}

static int launch_a8w8(const uint8_t* a, const float* sa, const uint8_t* b, const float* sb, void* y, int64_t M,
                       int64_t N, int64_t K, int out_dtype, float* ws, int64_t ws_bytes, hipStream_t st);

}  // namespace cek

extern "C" int64_t cek_gemm_fp8_a8w8_workspace_size(int64_t M, int64_t N, int64_t K) {
  return cek::a8w8_workspace_bytes(M, N, K);
}

extern "C" int cek_gemm_fp8_a8w8_ws(const uint8_t* a, const float* sa, const uint8_t* b, const float* sb, void* y,
                                    int64_t M, int64_t N, int64_t K, int out_dtype, void* workspace,
                                    int64_t workspace_bytes, void* stream) {
  if (workspace_bytes < 0 || (workspace_bytes > 0 && (!workspace || !cek::aligned(workspace, 4)))) return CEK_ERR_INVALID;
  return cek::launch_a8w8(a, sa, b, sb, y, M, N, K, out_dtype, static_cast<float*>(workspace), workspace_bytes,
                          (hipStream_t)stream);
}

extern "C" int cek_gemm_fp8_a8w8(const uint8_t* a, const float* sa, const uint8_t* b, const float* sb,
                                 void* y, int64_t M, int64_t N, int64_t K, int out_dtype, void* stream) {
  return cek::launch_a8w8(a, sa, b, sb, y, M, N, K, out_dtype, nullptr, 0, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
// Split-K scratch of cek_gemm_fp8_a8w8_noalloc: a file-scope device array,
// one copy per GPU the library runs on, held until the process ends.  Host
// code never passes the array's name to a kernel (on the host it is only a
// handle of the symbol): each device's address comes from
// hipGetSymbolAddress, taken once per device with that device current, and
// only that address is used.  The split-K kernels write every partial sum
// they later read, so the buffer needs no clearing between calls; calls that
// overlap on one GPU (e.g. on two streams) share it and race.
// ---------------------------------------------------------------------------
namespace cek {

constexpr int64_t kScratchBytes = (int64_t)32 << 20;  // 32 MiB: every BASELINE split-K plan fits
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxScratchDevices = 64;
static std::atomic<void*> g_scratch_addr[kMaxScratchDevices];
static std::mutex g_scratch_mu;

// Device address of `scratch` on the device `st` runs on (taken once per
// device); CEK_OK or an error status.
static int scratch_address(hipStream_t st, void** out) {
  int dev = -1;
  hipError_t e = st ? hipStreamGetDevice(st, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return record_hip_error(e);
  if (dev < 0 || dev >= kMaxScratchDevices) return CEK_ERR_UNSUPPORTED;
  void* p = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_addr[dev].load(std::memory_order_relaxed);
    if (!p) {
      int cur = -1;
      e = hipGetDevice(&cur);
      if (e != hipSuccess) return record_hip_error(e);
      if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return record_hip_error(e);
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      const hipError_t e2 = cur != dev ? hipSetDevice(cur) : hipSuccess;
      if (e != hipSuccess) return record_hip_error(e);
      if (e2 != hipSuccess) return record_hip_error(e2);
      if (!p) return CEK_ERR_HIP;
      g_scratch_addr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return CEK_OK;
}

}  // namespace cek

extern "C" int cek_gemm_fp8_a8w8_noalloc(const uint8_t* a, const float* sa, const uint8_t* b, const float* sb,
                                         void* y, int64_t M, int64_t N, int64_t K, int out_dtype, void* stream) {
  hipStream_t st = (hipStream_t)stream;
  const int64_t need = cek::a8w8_workspace_bytes(M, N, K);
  if (need > cek::kScratchBytes) return CEK_ERR_SCRATCH;
  if (need == 0) return cek::launch_a8w8(a, sa, b, sb, y, M, N, K, out_dtype, nullptr, 0, st);
  void* ws = nullptr;
  const int rc = cek::scratch_address(st, &ws);
  if (rc != CEK_OK) return rc;
  return cek::launch_a8w8(a, sa, b, sb, y, M, N, K, out_dtype, static_cast<float*>(ws), cek::kScratchBytes, st);
}

namespace cek {

static int launch_a8w8(const uint8_t* a, const float* sa, const uint8_t* b, const float* sb, void* y, int64_t M,
                       int64_t N, int64_t K, int out_dtype, float* ws, int64_t ws_bytes, hipStream_t st) {
  if (M < 0 || N < 0 || K <= 0 || K % 16 != 0) return CEK_ERR_INVALID;
  if (M > 65535 * 64 || N > INT32_MAX || K > INT32_MAX) return CEK_ERR_INVALID;
  if (M == 0 || N == 0) return CEK_OK;
  if (!a || !sa || !b || !sb || !y) return CEK_ERR_INVALID;
  if (!aligned(a, 16) || !aligned(b, 16)) return CEK_ERR_INVALID;
  uint16_t* yp = static_cast<uint16_t*>(y);
  if (out_dtype != CEK_F16 && out_dtype != CEK_BF16) return CEK_ERR_INVALID;
  // Skinny A: stream the weights once with the GEMV kernels rather than tile
  // a mostly empty GEMM (they decline the shapes the tiles serve better).
  // At M = 64 (the 64-row tile's smallest M), given the workspace the
  // split-K plan asks for, the tiled GEMM in K parts is 1.2-1.8x faster
  // (measured on MI355X, K = 4096..14336, N = 4096..28672).
  if (M <= 64) {
    const int64_t need64 = M == 64 ? a8w8_workspace_bytes(M, N, K) : 0;
    if (!(need64 > 0 && ws && ws_bytes >= need64)) {
      const int rc = launch_gemv_a8w8(a, sa, b, sb, y, M, N, K, out_dtype, st);
      if (rc != CEK_ERR_UNSUPPORTED) return rc;
    }
  }
  if (K % 128 == 0) {
    // Tile (and split-K) choice: plan_a8w8.  Every configuration runs
    // gemm_a8w8_pipe_kernel (register-pipelined fragment reads,
    // single-offset addressing; configuration 2, 256 x 192, its 3-slot B
    // ring form gemm_a8w8_pipe_b3_kernel) when the matrices are below 4 GB
    // and hold at least one tile in each dimension; otherwise configurations
    // 0-3 run gemm_a8w8_lds_kernel with the same tile (its loads clamp rows),
    // and the plan only picks 4-7 where the pipelined kernel applies.  Split K
    // needs a workspace of a8w8_workspace_bytes; without one the unsplit
    // plan runs.
    const bool off32 = a8w8_off32(M, N, K);
    const int64_t need = a8w8_workspace_bytes(M, N, K);
    const A8w8Plan plan = plan_a8w8(M, N, K, off32, need > 0 && ws && ws_bytes >= need);
    const int cfg = plan.cfg;
    // The split 64 x 128 plan with fewer parts than CUs runs 64 x 96 tiles
    // instead where those still make one part per CU at most: the outputs are
    // the same (a part's K order and the parts' order do not depend on the
    // tile), and the CUs are evenly loaded (measured on MI355X, weights from
    // HBM: M = 64, N = 6144, K = 4096 13.11 -> 12.64 us, K = 5120 13.20 ->
    // 12.59 us, 192 -> 256 workgroups; where 64 x 128 already fills the CUs,
    // 64 x 96 was slower, e.g. K = 14336, N = 4096 17.83 -> 21.46 us).
    constexpr int64_t kCUs = 256;  // MI355X compute units
    auto parts = [&](int64_t bm, int64_t bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn) * plan.split; };
    const bool n96 = cfg == 0 && plan.split > 1 && parts(64, 128) < kCUs && parts(64, 96) <= kCUs;
    const bool pipe = off32 && M >= kA8w8Opts[cfg].bm && N >= kA8w8Opts[cfg].bn;
#define CEK_A8W8(TY, BM, BN, WM, WN, OCC)                                                               \
  do {                                                                                                \
    const int tm = (int)((M + BM - 1) / BM), tn = (int)((N + BN - 1) / BN);                           \
    gemm_a8w8_lds_kernel<TY, BM, BN, WM, WN, kA8w8LdsLayout, OCC>                                     \
        <<<dim3((unsigned)(tm * tn)), 64 * WM * WN, 0, st>>>(a, sa, b, sb, yp, M, N, K, tm, tn);      \
  } while (0)
#define CEK_A8W8_PIPE(TY, BM, BN, WM, WN, OCC, LW, RING)                                                \
  do {                                                                                                \
    const int tm = (int)((M + BM - 1) / BM), tn = (int)((N + BN - 1) / BN);                           \
    gemm_a8w8_pipe_kernel<TY, BM, BN, WM, WN, OCC, LW, 1, RING, WM * WN == 8 ? (BM / WM >= 48 ? 3 : 2) : 1> \
        <<<dim3((unsigned)(tm * tn)), 64 * WM * WN, 0, st>>>(a, sa, b, sb, yp, nullptr, M, N, K, tm, tn); \
  } while (0)
#define CEK_A8W8_PIPE_B3(TY, BM, BN, WM, WN, LW, NCH)                                                  \
  do {                                                                                                \
    const int tm = (int)((M + BM - 1) / BM), tn = (int)((N + BN - 1) / BN);                           \
    gemm_a8w8_pipe_b3_kernel<TY, BM, BN, WM, WN, LW, NCH>                                             \
        <<<dim3((unsigned)(tm * tn)), 64 * WM * WN, 0, st>>>(a, sa, b, sb, yp, M, N, K, tm, tn);      \
  } while (0)
#define CEK_A8W8_SPLIT(TY, BM, BN, WM, WN, OCC, LW, SP, RING)                                          \
  do {                                                                                                \
    const int tm = (int)((M + BM - 1) / BM), tn = (int)((N + BN - 1) / BN);                           \
    gemm_a8w8_pipe_kernel<TY, BM, BN, WM, WN, OCC, LW, SP, RING, WM * WN == 8 ? 3 : 1>                \
        <<<dim3((unsigned)(tm * tn * SP)), 64 * WM * WN, 0, st>>>(a, sa, b, sb, yp, ws, M, N, K, tm, tn); \
    gemm_splitk_finalize<TY, SP><<<dim3((unsigned)((N + 1023) / 1024), (unsigned)(M < 65535 ? M : 65535)), \
                                   256, 0, st>>>(ws, sa, sb, yp, (int)M, (int)N);                       \
  } while (0)
#define CEK_A8W8_SPLITS(TY, BM, BN, WM, WN, OCC, LW, RING)                                             \
  do {                                                                                                \
    if (plan.split == 2) CEK_A8W8_SPLIT(TY, BM, BN, WM, WN, OCC, LW, 2, RING);                        \
    else if (plan.split == 4) CEK_A8W8_SPLIT(TY, BM, BN, WM, WN, OCC, LW, 4, RING);                   \
    else CEK_A8W8_SPLIT(TY, BM, BN, WM, WN, OCC, LW, 8, RING);                                        \
  } while (0)
#define CEK_A8W8_ALL(TY)                                                               \
  do {                                                                                 \
    if (plan.split > 1) {                                                              \
      if (cfg == 6) CEK_A8W8_SPLITS(TY, 256, 128, 2, 4, 1, 4, 3);                      \
      else if (cfg == 5) CEK_A8W8_SPLITS(TY, 128, 256, 2, 4, 1, 4, 3);                 \
      else if (cfg == 1) CEK_A8W8_SPLITS(TY, 128, 128, 2, 2, 2, 4, 2);                 \
      else if (n96) CEK_A8W8_SPLITS(TY, 64, 96, 2, 2, 2, 2, 3);                        \
      else CEK_A8W8_SPLITS(TY, 64, 128, 2, 2, 2, 2, 3);                                \
    } else if (cfg == 7) {                                                             \
      CEK_A8W8_PIPE(TY, 128, 96, 4, 2, 1, 4, 3);                                       \
    } else if (cfg == 6) {                                                             \
      CEK_A8W8_PIPE(TY, 256, 128, 2, 4, 1, 4, 3);                                      \
    } else if (cfg == 5) {                                                             \
      CEK_A8W8_PIPE(TY, 128, 256, 2, 4, 1, 4, 3);                                      \
    } else if (cfg == 4) {                                                             \
      CEK_A8W8_PIPE(TY, 128, 128, 2, 4, 1, 4, 3);                                      \
    } else if (cfg == 3) {                                                             \
      if (pipe) CEK_A8W8_PIPE(TY, 256, 256, 2, 4, 1, 4, 2);                            \
      else CEK_A8W8(TY, 256, 256, 4, 2, 1);                                            \
    } else if (cfg == 2) {                                                             \
      if (pipe) CEK_A8W8_PIPE_B3(TY, 256, 192, 2, 4, 4, 3);                           \
      else CEK_A8W8(TY, 256, 192, 2, 4, 1);                                            \
    } else if (cfg == 1) {                                                             \
      if (pipe) CEK_A8W8_PIPE(TY, 128, 128, 2, 2, 2, 4, 2);                            \
      else CEK_A8W8(TY, 128, 128, 2, 2, 2);                                            \
    } else {                                                                           \
      if (pipe) CEK_A8W8_PIPE(TY, 64, 128, 2, 2, 2, 2, 2);                             \
      else CEK_A8W8(TY, 64, 128, 2, 2, 2);                                             \
    }                                                                                  \
  } while (0)
    if (out_dtype == CEK_F16) CEK_A8W8_ALL(F16);
    else CEK_A8W8_ALL(BF16);
#undef CEK_A8W8
#undef CEK_A8W8_PIPE
#undef CEK_A8W8_PIPE_B3
#undef CEK_A8W8_SPLIT
#undef CEK_A8W8_SPLITS
#undef CEK_A8W8_ALL
    return check_launch();
  }
  dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64));
  if (out_dtype == CEK_F16) gemm_a8w8_simple_kernel<F16><<<grid, 256, 0, st>>>(a, sa, b, sb, yp, M, N, K);
  else if (out_dtype == CEK_BF16) gemm_a8w8_simple_kernel<BF16><<<grid, 256, 0, st>>>(a, sa, b, sb, yp, M, N, K);
  else return CEK_ERR_INVALID;
  return check_launch();
}

}  // namespace cek
