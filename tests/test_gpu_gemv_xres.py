"""The wide batched GEMV: 9 <= M <= 16, K of 2, 3 or 4 KiB values and
512 < N / 16 <= 2048 row tiles per weight matrix run gemv_xres_kernel
(activations resident in LDS, weights streamed into MFMA operands, each
tile's K in two halves).  Checked against the CPU oracle (tolerance as in
the other GEMV tests) over 3 to 8 tiles per workgroup slot, ragged N, both
fp8 formats, both activation types and every scale kind; and, since its sum
order differs from the other GEMV kernels', the multi-matrix op must still
give each matrix, bit for bit, what the single op gives it -- with matrices
on either side of the kernel choice in one call, and with more slots than
workgroups (grid-stride slots).
"""

import sys

import pytest
import torch

from conftest import assert_close_fp
from esimd_learning_amd import synthetic
from oracle import gemv as ogemv

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _pern(ops, xd, Wd, sd, io):
    M, K = xd.shape
    N = Wd.shape[0]
    y = torch.full((M, N), float("nan"), dtype=io, device=xd.device)
    ops.esimd_gemv_fp8_pern(xd, Wd, sd, y, N, K)
    return y


# (K, N): tiles per slot ceil(tiles / 256): 563 tiles (3 per slot, ragged N),
# 768 (3), 896 (4), 1025 (5, ragged), 1536 (6), 1792 (7), 2048 (8)
SHAPES = [(4096, 9000), (3072, 12288), (4096, 14336), (4096, 16400), (4096, 24576), (2048, 28672), (2048, 32768)]


@pytest.mark.parametrize("M", [9, 12, 16])
@pytest.mark.parametrize("K,N", SHAPES)
def test_xres_vs_oracle(ops, dev, M, K, N):
    _say(f"gemv xres M={M} K={K} N={N}")
    W8, s = synthetic.weight_fp8(N, K, seed=N + K)
    x = synthetic.activations(M, K, seed=M + 3)
    xd, Wd, sd = x.to(dev), W8.to(dev), s.to(dev)
    y = _pern(ops, xd, Wd, sd, torch.float16)
    y2 = _pern(ops, xd, Wd, sd, torch.float16)
    torch.cuda.synchronize()
    assert torch.equal(y, y2), "not deterministic"
    assert_close_fp(y.cpu(), ogemv.gemv_fp8_pern(x, W8, s), f"xres M={M} K={K} N={N}")


@pytest.mark.parametrize("io,fmt,sdt", [(torch.bfloat16, torch.float8_e4m3fn, torch.bfloat16),
                                        (torch.float16, torch.float8_e5m2, torch.float16),
                                        (torch.bfloat16, torch.float8_e5m2, torch.float32)])
def test_xres_dtypes(ops, dev, io, fmt, sdt):
    M, K, N = 16, 4096, 14336
    _say(f"gemv xres dtypes io={io} fmt={fmt} scale={sdt}")
    W8, s = synthetic.weight_fp8(N, K, seed=11, fmt=fmt)
    s = s.to(sdt)
    x = synthetic.activations(M, K, seed=12, dtype=io)
    y = _pern(ops, x.to(dev), W8.to(dev), s.to(dev), io)
    torch.cuda.synchronize()
    assert y.dtype == io
    assert_close_fp(y.cpu(), ogemv.gemv_fp8_pern(x, W8, s), f"xres io={io} fmt={fmt} scale={sdt}")


def test_xres_per_tensor_scale(ops, dev):
    M, K, N = 10, 3072, 12288
    _say("gemv xres per-tensor scale")
    W8, _ = synthetic.weight_fp8(N, K, seed=13)
    s = torch.tensor([0.0123], dtype=torch.float32)
    x = synthetic.activations(M, K, seed=14)
    y = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
    ops.esimd_gemv_fp8_pert(x.to(dev), W8.to(dev), s.to(dev), y)
    torch.cuda.synchronize()
    assert_close_fp(y.cpu(), ogemv.gemv_fp8_pert(x, W8, s), "xres pert")


@pytest.mark.parametrize("Ns,K", [((14336, 4096, 1024, 9000), 4096),  # xres and LDS-kernel matrices in one call
                                  ((32768, 32768), 2048),              # 4096 tiles: two slots per workgroup
                                  ((12288, 6144), 3072)])
@pytest.mark.parametrize("M", [9, 16])
def test_xres_multi_matrix_equals_single(ops, dev, M, Ns, K):
    _say(f"gemv xres multi M={M} Ns={Ns} K={K}")
    Ws, Ss = zip(*[synthetic.weight_fp8(n, K, seed=n + 7 * i) for i, n in enumerate(Ns)])
    x = synthetic.activations(M, K, seed=21)
    xd = x.to(dev)
    Wd = [w.to(dev) for w in Ws]
    Sd = [s.to(dev) for s in Ss]
    ys = [torch.full((M, n), float("nan"), dtype=torch.float16, device=dev) for n in Ns]
    ops.esimd_gemv_fp8_pern_fused(xd, Wd, Sd, ys)
    for i, n in enumerate(Ns):
        y1 = _pern(ops, xd, Wd[i], Sd[i], torch.float16)
        torch.cuda.synchronize()
        assert torch.equal(ys[i], y1), f"matrix {i} (N={n})"
        assert_close_fp(ys[i].cpu(), ogemv.gemv_fp8_pern(x, Ws[i], Ss[i]), f"matrix {i}")


# The e4m3-activation form (gemv_xres8_kernel): the a8w8 GEMM op sends M <= 64
# (without a split-K workspace) to the GEMV kernels; 17 <= M <= 32 with at
# least 384 row tiles and K of 2, 3 or 4 KiB values takes this one (up to 512
# tiles from 24 rows on).  N = 28672 gives 896 slots of 2 tiles: 3-4 slots per
# workgroup.  K = 5120 (the 32 activation rows fill all of LDS; the K parts'
# sums reuse it) up to 512 tiles; N = 14336 at K = 5120 and M = 17 at up to
# 512 tiles stay on the other kernel.  N ~ 6144 runs 12-row tiles (256 slots),
# N = 6140 and 6130 with a ragged last one; 12-row tiles also take N from 384
# of them (4608) up, from 24 rows (N = 4608, 5000, 5120).
@pytest.mark.parametrize("M", [17, 24, 32])
@pytest.mark.parametrize("K,N", [(4096, 6144), (4096, 6140), (3072, 12288), (2048, 8200), (4096, 28672), (5120, 6144),
                                 (5120, 6130), (5120, 8190), (5120, 14336), (4096, 4608), (4096, 5000), (5120, 5120)])
def test_xres8_a8w8_vs_oracle(ops, dev, M, K, N):
    from oracle import gemm as ogemm
    from oracle import norm as onorm
    _say(f"a8w8 gemv xres8 M={M} K={K} N={N}")
    x = synthetic.activations(M, K, seed=M + K)
    q, sa = onorm.per_token_quant(x)
    W8, sb = synthetic.weight_fp8(N, K, seed=N + 5)
    W8 = W8.view(torch.uint8)
    qd, sad, Wd, sbd = q.to(dev), sa.to(dev), W8.to(dev), sb.to(dev)
    ref = ogemm.gemm_a8w8(q, sa, W8, sb)
    for out_dt in (torch.float16, torch.bfloat16):
        y = torch.full((M, N), float("nan"), dtype=out_dt, device=dev)
        ops.esimd_gemm_fp8_a8w8(qd, sad, Wd, sbd, y)
        y2 = torch.full((M, N), float("nan"), dtype=out_dt, device=dev)
        ops.esimd_gemm_fp8_a8w8(qd, sad, Wd, sbd, y2)
        torch.cuda.synchronize()
        assert torch.equal(y, y2), "not deterministic"
        assert_close_fp(y.cpu(), ref, f"a8w8 xres8 M={M} K={K} N={N} {out_dt}")
