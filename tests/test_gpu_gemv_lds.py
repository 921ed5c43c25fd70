"""GPU parity of the LDS-staged GEMV kernel across its dispatch branches.

The kernel is instantiated per K (2, 3, 4, 5, 14 and 24 KiB values) and per
configuration (one or two 16-row weight tiles per workgroup, one to four
16-row activation blocks, prefetch depth); these cases reach each of them
through the public ops:

* esimd_gemv_fp8_pern / _pert, 3 <= M <= 16, fp16/bf16 x e4m3/e5m2;
* esimd_gemm_fp8_pert with 16 < M <= 32 (the GEMM entry's skinny route);
* esimd_gemm_fp8_a8w8 with 3 <= M <= 64 (e4m3 activations and weights);
* the fused multi-matrix GEMV (segment table), whose segments share a launch;
* K = 4096 or 5120 with many rows, where a workgroup streams two or four
  consecutive 16-row tiles (ragged last workgroup);
* 12-row tiles, one or two per workgroup, where they balance the CUs better
  than 16-row ones.

N values include ones that are not multiples of the 16- and 32-row tiles.
Reference: the CPU oracle; tolerance |out - ref| <= 1e-2 max|ref| + 2e-2 |ref|.
"""

import sys

import pytest
import torch

from conftest import assert_close_fp
from esimd_learning_amd import synthetic
from oracle import gemm as ogemm
from oracle import gemv as ogemv
from oracle import norm as onorm

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


# (K, N): every instantiated K, with N on both sides of the switch to
# two-tile workgroups for 9-16 rows (more 16-row tiles than CUs: N = 4112 and
# up): 24 rows (two 12-row tiles) up to N = 6144, 32 rows above
SHAPES = [(2048, 1000), (3072, 6200), (4096, 6144), (4096, 2050), (5120, 6150), (14336, 1030), (24576, 520),
          (4096, 4610), (4096, 7000)]


@pytest.mark.parametrize("K,N", SHAPES)
@pytest.mark.parametrize("M", [3, 5, 8, 13, 16])
def test_gemv_pern_lds(ops, dev, K, N, M):
    _say(f"lds gemv pern M={M} K={K} N={N}")
    W8, s = synthetic.weight_fp8(N, K, seed=K + M)
    x = synthetic.activations(M, K, seed=N + M)
    y = torch.zeros(M, N, dtype=torch.float16, device=dev)
    ops.esimd_gemv_fp8_pern(x.to(dev), W8.to(dev), s.to(dev), y, N, K)
    torch.cuda.synchronize()
    assert_close_fp(y.cpu(), ogemv.gemv_fp8_pern(x, W8, s), f"pern M={M} K={K} N={N}")


@pytest.mark.parametrize("io", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("fmt", [torch.float8_e4m3fn, torch.float8_e5m2])
@pytest.mark.parametrize("K,N,M", [(4096, 6150, 9), (3072, 700, 4), (14336, 260, 16)])
def test_gemv_pert_lds_types(ops, dev, io, fmt, K, N, M):
    _say(f"lds gemv pert M={M} K={K} N={N} {io} {fmt}")
    g = torch.Generator().manual_seed(K + N)
    W8 = (torch.randn(N, K, generator=g).half() * 0.1).to(fmt)
    sv = torch.tensor(0.07)
    x = (torch.randn(M, K, generator=g) * 0.5).to(io)
    y = torch.zeros(M, N, dtype=io, device=dev)
    ops.esimd_gemv_fp8_pert(x.to(dev), W8.to(dev), sv.to(dev), y)
    torch.cuda.synchronize()
    assert_close_fp(y.cpu(), ogemv.gemv_fp8_pert(x, W8, sv), f"pert {io} {fmt}")


@pytest.mark.parametrize("M,K,N", [(17, 2048, 3000), (24, 4096, 6144), (32, 5120, 1100), (32, 4096, 20000)])
def test_gemm_pert_skinny(ops, dev, M, K, N):
    """16 < M <= 32 through esimd_gemm_fp8_pert (N = 20000 takes the tiles)."""
    _say(f"lds gemm pert M={M} K={K} N={N}")
    W8, _ = synthetic.weight_fp8(N, K, seed=M + K)
    x = synthetic.activations(M, K, seed=M)
    sv = torch.tensor(0.02)
    y = torch.zeros(M, N, dtype=torch.float16, device=dev)
    ops.esimd_gemm_fp8_pert(x.to(dev), W8.to(dev), sv.to(dev), y)
    torch.cuda.synchronize()
    assert_close_fp(y.cpu(), ogemv.gemm_fp8_pert(x, W8, sv), f"gemm pert M={M}")


@pytest.mark.parametrize("M,K,N", [(3, 3072, 1000), (7, 24576, 300), (12, 4096, 6160), (16, 5120, 6144),
                                   (20, 4096, 3000), (32, 14336, 1024), (33, 4096, 2000), (64, 2048, 8192),
                                   (48, 4096, 9000), (12, 4096, 4610), (16, 5120, 5000)])
def test_a8w8_skinny(ops, dev, M, K, N):
    """a8w8 M <= 64: LDS kernel with 1, 2 and 4 activation blocks (and the
    tiled GEMM for M > 32, N > 8192).  The torch op gives the split-K plan
    its workspace, which at M = 64 (64 x 128 tiles in K parts) replaces the
    weight-streaming kernel; the C-ABI call without a workspace
    (cek_gemm_fp8_a8w8) keeps the 4-block LDS kernel there, so both are run."""
    from esimd_learning_amd import cabi
    _say(f"lds a8w8 M={M} K={K} N={N}")
    lib = cabi.load()
    x = synthetic.activations(M, K, seed=M + 5)
    q, sa = onorm.per_token_quant(x)
    W8, sb = synthetic.weight_fp8(N, K, seed=K + 3)
    ref = ogemm.gemm_a8w8(q, sa, W8.view(torch.uint8), sb)
    qd, sad, Wd, sbd = q.to(dev), sa.to(dev), W8.view(torch.uint8).to(dev), sb.to(dev)
    st = cabi.stream_ptr(torch.cuda.current_stream())
    for code, out_dt in ((0, torch.float16), (1, torch.bfloat16)):
        y = torch.zeros(M, N, dtype=out_dt, device=dev)
        ops.esimd_gemm_fp8_a8w8(qd, sad, Wd, sbd, y)
        y_nows = torch.zeros(M, N, dtype=out_dt, device=dev)
        assert lib.cek_gemm_fp8_a8w8(qd.data_ptr(), sad.data_ptr(), Wd.data_ptr(), sbd.data_ptr(), y_nows.data_ptr(),
                                     M, N, K, code, st) == 0
        torch.cuda.synchronize()
        assert_close_fp(y.cpu(), ref, f"a8w8 M={M} K={K} N={N} {out_dt}")
        assert_close_fp(y_nows.cpu(), ref, f"a8w8 no workspace M={M} K={K} N={N} {out_dt}")


def test_fused_segments_lds(ops, dev):
    """Three matrices of different heights in one launch at M = 8."""
    M, K = 8, 4096
    x = synthetic.activations(M, K, seed=9)
    Ns = [4096, 1030, 2000]
    Ws, Ss = zip(*[synthetic.weight_fp8(n, K, seed=n) for n in Ns])
    ys = [torch.zeros(M, n, dtype=torch.float16, device=dev) for n in Ns]
    ops.esimd_gemv_fp8_pern_fused(x.to(dev), [w.to(dev) for w in Ws], [s.to(dev) for s in Ss], ys)
    torch.cuda.synchronize()
    for w, s, y in zip(Ws, Ss, ys):
        assert_close_fp(y.cpu(), ogemv.gemv_fp8_pern(x, w, s), f"fused N={w.shape[0]}")


@pytest.mark.parametrize("M,K,N", [(4, 4096, 14336), (3, 4096, 14350), (8, 4096, 28700), (6, 5120, 14400),
                                   (4, 3072, 12300), (2, 4096, 14336),
                                   (4, 4096, 20470), (3, 5120, 24570), (8, 4096, 24570), (8, 4096, 20470)])
def test_gemv_multi_tile(ops, dev, M, K, N):
    """Workgroups that own 2 or 4 consecutive tiles (the last one partly
    past N), fp16 and bf16 activations; at 1280 and 1536 tiles the
    launch-balance rule picks 1 or 2 tiles per workgroup for the rotated
    (M <= 4) and the other forms."""
    _say(f"lds gemv multi-tile M={M} K={K} N={N}")
    W8, s = synthetic.weight_fp8(N, K, seed=N + K)
    x = synthetic.activations(M, K, seed=M + 11)
    for io in (torch.float16, torch.bfloat16):
        xi = x.to(io)
        y = torch.zeros(M, N, dtype=io, device=dev)
        ops.esimd_gemv_fp8_pern(xi.to(dev), W8.to(dev), s.to(dev), y, N, K)
        torch.cuda.synchronize()
        assert_close_fp(y.cpu(), ogemv.gemv_fp8_pern(xi, W8, s), f"multi-tile M={M} K={K} N={N} {io}")


@pytest.mark.parametrize("M,K,N", [(4, 4096, 14350), (8, 5120, 7000), (1, 4096, 28672)])
def test_a8w8_multi_tile(ops, dev, M, K, N):
    """The a8w8 skinny path with multi-tile workgroups (e4m3 activations)."""
    _say(f"lds a8w8 multi-tile M={M} K={K} N={N}")
    x = synthetic.activations(M, K, seed=M + 7)
    q, sa = onorm.per_token_quant(x)
    W8, sb = synthetic.weight_fp8(N, K, seed=K + 9)
    ref = ogemm.gemm_a8w8(q, sa, W8.view(torch.uint8), sb)
    y = torch.zeros(M, N, dtype=torch.float16, device=dev)
    ops.esimd_gemm_fp8_a8w8(q.to(dev), sa.to(dev), W8.view(torch.uint8).to(dev), sb.to(dev), y)
    torch.cuda.synchronize()
    assert_close_fp(y.cpu(), ref, f"a8w8 multi-tile M={M} K={K} N={N}")


def test_fused_segments_multi_tile(ops, dev):
    """Segments of a launch whose total row count selects 4-tile workgroups."""
    M, K = 4, 4096
    x = synthetic.activations(M, K, seed=19)
    Ns = [9000, 1030, 6150]
    Ws, Ss = zip(*[synthetic.weight_fp8(n, K, seed=n + 1) for n in Ns])
    ys = [torch.zeros(M, n, dtype=torch.float16, device=dev) for n in Ns]
    ops.esimd_gemv_fp8_pern_fused(x.to(dev), [w.to(dev) for w in Ws], [s.to(dev) for s in Ss], ys)
    torch.cuda.synchronize()
    for w, s, y in zip(Ws, Ss, ys):
        assert_close_fp(y.cpu(), ogemv.gemv_fp8_pern(x, w, s), f"fused multi-tile N={w.shape[0]}")


# 12-row tiles: the forms without the K rotation (5-8 fp16 / bf16 rows, e4m3
# activations up to 8 rows, 9-16 rows below N = 6144) take them where they cut
# the busiest CU's rows by a fifth (N = 6000-6150: 24 rows against 32; N =
# 3000-3072: 12 against 16), ragged N ending inside a 12-row tile and inside a
# two-tile workgroup.
@pytest.mark.parametrize("M,K,N", [(5, 4096, 6144), (8, 4096, 6100), (7, 3072, 6000), (6, 5120, 6143), (12, 4096, 3000),
                                   (16, 3072, 3072)])
def test_gemv_12row_tiles(ops, dev, M, K, N):
    _say(f"lds gemv 12-row tiles M={M} K={K} N={N}")
    for io, fmt in [(torch.float16, torch.float8_e4m3fn), (torch.bfloat16, torch.float8_e5m2)]:
        W8, s = synthetic.weight_fp8(N, K, seed=N + K + 1, fmt=fmt)
        x = synthetic.activations(M, K, seed=M + 13, dtype=io)
        y = torch.full((M, N), float("nan"), dtype=io, device=dev)
        ops.esimd_gemv_fp8_pern(x.to(dev), W8.to(dev), s.to(dev), y, N, K)
        torch.cuda.synchronize()
        assert_close_fp(y.cpu(), ogemv.gemv_fp8_pern(x, W8, s), f"12-row M={M} K={K} N={N} {io}")


@pytest.mark.parametrize("M,K,N", [(4, 4096, 6144), (8, 5120, 6101), (8, 4096, 6144)])
def test_a8w8_12row_tiles(ops, dev, M, K, N):
    _say(f"lds a8w8 12-row tiles M={M} K={K} N={N}")
    x = synthetic.activations(M, K, seed=M + 17)
    q, sa = onorm.per_token_quant(x)
    W8, sb = synthetic.weight_fp8(N, K, seed=K + 21)
    ref = ogemm.gemm_a8w8(q, sa, W8.view(torch.uint8), sb)
    for out_dt in (torch.float16, torch.bfloat16):
        y = torch.full((M, N), float("nan"), dtype=out_dt, device=dev)
        ops.esimd_gemm_fp8_a8w8(q.to(dev), sa.to(dev), W8.view(torch.uint8).to(dev), sb.to(dev), y)
        torch.cuda.synchronize()
        assert_close_fp(y.cpu(), ref, f"a8w8 12-row M={M} K={K} N={N} {out_dt}")


# Two 12-row tiles per workgroup (24 rows): 9-16 rows (e4m3 activations: 9-16)
# where there are more 16-row tiles than CUs and 24-row workgroups cut the
# busiest CU's rows against 32-row ones by a fifth (N = 4112-6144); ragged N
# ending inside either tile of the last workgroup.
@pytest.mark.parametrize("M,K,N", [(16, 4096, 6144), (9, 4096, 4112), (12, 5120, 5000), (16, 3072, 4610),
                                   (13, 4096, 6133)])
def test_gemv_24row_tiles(ops, dev, M, K, N):
    _say(f"lds gemv 24-row tiles M={M} K={K} N={N}")
    for io, fmt in [(torch.float16, torch.float8_e4m3fn), (torch.bfloat16, torch.float8_e5m2)]:
        W8, s = synthetic.weight_fp8(N, K, seed=N + K + 5, fmt=fmt)
        x = synthetic.activations(M, K, seed=M + 19, dtype=io)
        y = torch.full((M, N), float("nan"), dtype=io, device=dev)
        ops.esimd_gemv_fp8_pern(x.to(dev), W8.to(dev), s.to(dev), y, N, K)
        torch.cuda.synchronize()
        assert_close_fp(y.cpu(), ogemv.gemv_fp8_pern(x, W8, s), f"24-row M={M} K={K} N={N} {io}")
    W8, _ = synthetic.weight_fp8(N, K, seed=N + 41)
    sv = torch.tensor(0.029)
    x = synthetic.activations(M, K, seed=M + 43)
    y = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
    ops.esimd_gemv_fp8_pert(x.to(dev), W8.to(dev), sv.to(dev), y)
    torch.cuda.synchronize()
    assert_close_fp(y.cpu(), ogemv.gemv_fp8_pert(x, W8, sv), f"pert 24-row M={M} K={K} N={N}")


@pytest.mark.parametrize("M,K,N", [(12, 4096, 6144), (16, 5120, 4700), (9, 3072, 6100)])
def test_a8w8_24row_tiles(ops, dev, M, K, N):
    _say(f"lds a8w8 24-row tiles M={M} K={K} N={N}")
    x = synthetic.activations(M, K, seed=M + 47)
    q, sa = onorm.per_token_quant(x)
    W8, sb = synthetic.weight_fp8(N, K, seed=K + 53)
    ref = ogemm.gemm_a8w8(q, sa, W8.view(torch.uint8), sb)
    for out_dt in (torch.float16, torch.bfloat16):
        y = torch.full((M, N), float("nan"), dtype=out_dt, device=dev)
        ops.esimd_gemm_fp8_a8w8(q.to(dev), sa.to(dev), W8.view(torch.uint8).to(dev), sb.to(dev), y)
        torch.cuda.synchronize()
        assert_close_fp(y.cpu(), ref, f"a8w8 24-row M={M} K={K} N={N} {out_dt}")


# A matrix alone takes 12-row tiles; in a fused launch whose total row count
# picks 16-row tiles (M = 8: 20480 rows, one tile per workgroup), 24-row
# workgroups (M = 12: 6144 rows; M = 16: 6001 rows over two ragged matrices,
# 6008 with an 8-row one inside a single workgroup)
# or 32-row ones (M = 12: 7168 rows) it must still get the same outputs bit
# for bit (the tile heights add each output's K chunks in the same order).
@pytest.mark.parametrize("M,K,Ns", [(8, 4096, (6144, 14336)), (12, 3072, (3072, 3072)), (16, 4096, (3000, 3001)),
                                    (12, 4096, (3072, 4096)), (16, 4096, (6000, 8))])
def test_12row_fused_equals_single(ops, dev, M, K, Ns):
    _say(f"lds 12-row fused == single M={M} K={K} Ns={Ns}")
    x = synthetic.activations(M, K, seed=23)
    Ws, Ss = zip(*[synthetic.weight_fp8(n, K, seed=n + 3) for n in Ns])
    xd = x.to(dev)
    Wd = [w.to(dev) for w in Ws]
    Sd = [s.to(dev) for s in Ss]
    ys = [torch.full((M, n), float("nan"), dtype=torch.float16, device=dev) for n in Ns]
    ops.esimd_gemv_fp8_pern_fused(xd, Wd, Sd, ys)
    for i, n in enumerate(Ns):
        y1 = torch.full((M, n), float("nan"), dtype=torch.float16, device=dev)
        ops.esimd_gemv_fp8_pern(xd, Wd[i], Sd[i], y1, n, K)
        torch.cuda.synchronize()
        assert torch.equal(ys[i], y1), f"matrix {i} (N={n})"
        assert_close_fp(y1.cpu(), ogemv.gemv_fp8_pern(x, Ws[i], Ss[i]), f"matrix {i}")


@pytest.mark.parametrize("M,K,N", [(8, 4096, 6144), (12, 3072, 3070)])
def test_gemv_pert_12row_tiles(ops, dev, M, K, N):
    """The per-tensor-scale op on 12-row tiles (fp16 and bf16)."""
    _say(f"lds gemv pert 12-row tiles M={M} K={K} N={N}")
    W8, _ = synthetic.weight_fp8(N, K, seed=N + 31)
    sv = torch.tensor(0.031)
    for io in (torch.float16, torch.bfloat16):
        x = synthetic.activations(M, K, seed=M + 37, dtype=io)
        y = torch.full((M, N), float("nan"), dtype=io, device=dev)
        ops.esimd_gemv_fp8_pert(x.to(dev), W8.to(dev), sv.to(dev), y)
        torch.cuda.synchronize()
        assert_close_fp(y.cpu(), ogemv.gemv_fp8_pert(x, W8, sv), f"pert 12-row M={M} K={K} N={N} {io}")
