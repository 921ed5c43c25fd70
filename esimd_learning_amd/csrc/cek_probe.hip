// cek_probe.hip -- HBM read-rate probe (measurement utility, gfx950).
//
// Reads a buffer once with 16-byte non-temporal loads.  With a sink it folds
// the bytes into one 32-bit XOR per workgroup (the checkable mode); without
// one it ends right after the loads (the timed mode: the same load loop,
// without the cross-wave reduction that would otherwise add a few hundred
// cycles to the end of the kernel).  It is the practical ceiling a single pass over
// the same bytes can reach (launch ramp-up and drain included), which the
// benchmark quotes the HBM-bound kernels against beside the spec peak.
// Layout: a grid-stride loop of PROBE_WG workgroups x 512 threads with four
// loads in flight per thread (the fastest of the one-pass read shapes
// measured on MI355X over 58.7 MB: per-row workgroups of 1, 2 or 4 rows and
// grid strides of 1024-4096 workgroups were 0.1-0.5 us slower).
#include "cek_common.h"

namespace cek {

constexpr int PROBE_WG = 1024, PROBE_T = 512, PROBE_U = 4;

__global__ __launch_bounds__(PROBE_T) void hbm_read_probe_kernel(const u4* __restrict__ p, size_t n16,
                                                                 uint32_t* __restrict__ sink) {
  __shared__ uint32_t red[PROBE_T / 64];
  u4 acc = u4{0, 0, 0, 0};
  const size_t stride = (size_t)PROBE_WG * PROBE_T * PROBE_U;
  for (size_t i = (size_t)blockIdx.x * PROBE_T * PROBE_U + threadIdx.x; i < n16; i += stride) {
    u4 v[PROBE_U];
#pragma unroll
    for (int u = 0; u < PROBE_U; ++u)
      v[u] = i + (size_t)u * PROBE_T < n16 ? __builtin_nontemporal_load(p + i + (size_t)u * PROBE_T) : u4{0, 0, 0, 0};
#pragma unroll
    for (int u = 0; u < PROBE_U; ++u) acc ^= v[u];
  }
  uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  asm volatile("" ::"v"(x));  // the loads stay live in both modes
  if (sink == nullptr) return;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x ^= __shfl_xor(x, off, 64);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t s = 0;
#pragma unroll
    for (int w = 0; w < PROBE_T / 64; ++w) s ^= red[w];
    sink[blockIdx.x] = s;
  }
}

}  // namespace cek

extern "C" int cek_hbm_read_probe(const void* buf, int64_t bytes, uint32_t* sink, void* stream) {
  using namespace cek;
  if (bytes <= 0 || bytes % 16 != 0 || !buf || !aligned(buf, 16)) return CEK_ERR_INVALID;
  hbm_read_probe_kernel<<<dim3(PROBE_WG), PROBE_T, 0, (hipStream_t)stream>>>(static_cast<const u4*>(buf),
                                                                            (size_t)bytes / 16, sink);
  return check_launch();
}
