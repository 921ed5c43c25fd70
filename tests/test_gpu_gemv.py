"""GPU parity of the fp8 GEMV ops against the CPU oracle.

Shapes: BASELINE config 2 (decode M in {1,2,4,8,16} x the Llama-style
projections) and the reference's own GEMV test shapes
(reference tests/test_gemv_fp8.py:21-22,48,337,367,398,427), with the
reference's input recipe for the latter (randn * 0.1 fp16 -> e4m3, fp16
scale randn * 0.1).  Tolerance: |out - ref| <= 1e-2 max|ref| + 2e-2 |ref|.
"""

import sys

import numpy as np
import pytest
import torch

from conftest import assert_close_fp
from esimd_learning_amd import synthetic
from oracle import fp8 as ofp8
from oracle import gemv as ogemv

pytestmark = pytest.mark.gpu

CONFIG2 = [(4096, 6144), (4096, 4096), (4096, 28672), (14336, 4096), (4096, 14336)]


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _run_pern(ops, x, W8, s, dev):
    M, K = x.shape
    N = W8.shape[0]
    y = torch.zeros(M, N, dtype=x.dtype, device=dev)
    ops.esimd_gemv_fp8_pern(x.to(dev), W8.to(dev), s.to(dev), y, N, K)
    torch.cuda.synchronize()
    return y.cpu()


@pytest.mark.parametrize("K,N", CONFIG2)
@pytest.mark.parametrize("M", [1, 2, 4, 8, 16])
def test_gemv_config2_fp32_scale(ops, dev, M, K, N):
    _say(f"gemv pern M={M} K={K} N={N}")
    W8, s = synthetic.weight_fp8(N, K, seed=K + N)
    x = synthetic.activations(M, K, seed=M)
    y = _run_pern(ops, x, W8, s, dev)
    assert_close_fp(y, ogemv.gemv_fp8_pern(x, W8, s), f"M={M} K={K} N={N}")


@pytest.mark.parametrize("io", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("sdt", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M", [1, 3, 5, 16])
def test_gemv_dtypes(ops, dev, io, sdt, M):
    K, N = 2048, 1000        # N not a multiple of the row tiles
    _say(f"gemv dtypes io={io} scale={sdt} M={M}")
    W8, s = synthetic.weight_fp8(N, K, seed=7)
    x = synthetic.activations(M, K, seed=8, dtype=io)
    s = s.to(sdt)
    y = _run_pern(ops, x, W8, s, dev)
    assert y.dtype == io
    assert_close_fp(y, ogemv.gemv_fp8_pern(x, W8, s), f"io={io} sdt={sdt} M={M}")


REF_SHAPES_BASIC = [(3072, 2560), (2560, 2048), (20480, 2560), (2560, 10240), (256, 2560), (2048, 128),
                    (3072, 2048), (16, 2048)]
REF_SHAPES_SCALE = [(3072, 2560), (2560, 2048), (20480, 2560), (2560, 10240), (128, 2048), (2560, 10752)]


def _ref_inputs(N, K, seed, fmt=torch.float8_e4m3fn):
    g = torch.Generator().manual_seed(seed)
    W8 = (torch.randn(N, K, generator=g).half() * 0.1).to(fmt)
    s = torch.randn(N, generator=g).half() * 0.1
    x = torch.randn(1, K, generator=g).half() * 0.1
    return x, W8, s


@pytest.mark.parametrize("N,K", sorted(set(REF_SHAPES_BASIC + REF_SHAPES_SCALE)))
@pytest.mark.parametrize("fmt", [torch.float8_e4m3fn, torch.float8_e5m2])
def test_gemv_reference_shapes(ops, dev, N, K, fmt):
    _say(f"gemv reference-shape N={N} K={K} fmt={fmt}")
    x, W8, s = _ref_inputs(N, K, N * 7 + K, fmt)
    y = _run_pern(ops, x, W8, s, dev)
    assert_close_fp(y, ogemv.gemv_fp8_pern(x, W8, s), f"N={N} K={K}")


@pytest.mark.parametrize("N,K", [(1024, 1024), (2560, 2048), (512, 2048), (3072, 2048), (128, 2048),
                                 (16, 2048), (2048, 512)])
def test_gemv_pert(ops, dev, N, K):
    _say(f"gemv pert N={N} K={K}")
    x, W8, _ = _ref_inputs(N, K, N + K)
    sv = torch.tensor(0.0731, dtype=torch.float32)
    y = torch.zeros(1, N, dtype=torch.float16, device=dev)
    ops.esimd_gemv_fp8_pert(x.to(dev), W8.to(dev), sv.to(dev), y)
    torch.cuda.synchronize()
    assert_close_fp(y.cpu(), ogemv.gemv_fp8_pert(x, W8, sv), f"pert N={N} K={K}")


def test_pert_equals_pern_uniform(ops, dev):
    # reference tests/test_gemv_fp8.py:361-388 (there within 1 % because its
    # per-N scale is fp16); with an fp32 per-N scale the two are bit-identical.
    N, K = 2560, 2048
    _say("pert == pern (uniform fp32 scale)")
    x, W8, _ = _ref_inputs(N, K, 5)
    xd, wd = x.to(dev), W8.to(dev)
    a = torch.zeros(1, N, dtype=torch.float16, device=dev)
    b = torch.zeros(1, N, dtype=torch.float16, device=dev)
    ops.esimd_gemv_fp8_pert(xd, wd, torch.tensor(0.073, device=dev), a)
    ops.esimd_gemv_fp8_pern(xd, wd, torch.full((N,), 0.073, device=dev), b, N, K)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("io", [torch.float16, torch.bfloat16])
def test_gemm_m1_equals_gemv(ops, dev, io):
    # reference tests/test_gemm_fp8.py:65-93
    _say(f"gemm(M=1) == gemv io={io}")
    for N, K in [(2560, 2048), (512, 2048), (128, 2048), (2048, 512)]:
        x, W8, _ = _ref_inputs(N, K, N)
        xd, wd = x.to(io).to(dev), W8.to(dev)
        sc = torch.tensor(0.073, device=dev)
        a = torch.zeros(1, N, dtype=io, device=dev)
        b = torch.zeros(1, N, dtype=io, device=dev)
        ops.esimd_gemv_fp8_pert(xd, wd, sc, a)
        ops.esimd_gemm_fp8_pert(xd, wd, sc, b)
        torch.cuda.synchronize()
        assert torch.equal(a, b)


@pytest.mark.parametrize("M,K", [(1, 100), (3, 100), (2, 4100), (20, 72)])
def test_gemv_generic_path(ops, dev, M, K):
    # K not a multiple of 16 -> the byte-load kernel
    N = 77
    _say(f"gemv generic M={M} K={K}")
    W8, s = synthetic.weight_fp8(N, K, seed=3)
    x = synthetic.activations(M, K, seed=4)
    y = _run_pern(ops, x, W8, s, dev)
    assert_close_fp(y, ogemv.gemv_fp8_pern(x, W8, s), f"generic M={M} K={K}")


# K = 2048 and 1024 with one or two rows: the v_dot2 kernel puts 2 and 4 rows
# into each load instruction (two passes per workgroup, 4 and 8 rows).  N not
# a multiple of the rows per workgroup ends a workgroup inside a pass or
# before its second pass; N = 1 and 3 leave most of the only workgroup's rows
# clamped.  Both fp8 formats, both activation types, and the e4m3-activation
# form (the a8w8 op's GEMV route for one or two rows).
@pytest.mark.parametrize("K,N", [(2048, 1001), (2048, 8192), (1024, 999), (1024, 16384), (1024, 3), (2048, 1)])
@pytest.mark.parametrize("M", [1, 2])
def test_gemv_rows_per_pass(ops, dev, M, K, N):
    _say(f"gemv rows-per-pass M={M} K={K} N={N}")
    for io, fmt in [(torch.float16, torch.float8_e4m3fn), (torch.bfloat16, torch.float8_e5m2)]:
        W8, s = synthetic.weight_fp8(N, K, seed=K + N + M, fmt=fmt)
        x = synthetic.activations(M, K, seed=M + 40, dtype=io)
        y = _run_pern(ops, x, W8, s, dev)
        assert y.dtype == io
        assert_close_fp(y, ogemv.gemv_fp8_pern(x, W8, s), f"rows-per-pass M={M} K={K} N={N} io={io}")
    from oracle import gemm as ogemm
    from oracle import norm as onorm
    x = synthetic.activations(M, K, seed=M + 41)
    q, sa = onorm.per_token_quant(x)
    W8, sb = synthetic.weight_fp8(N, K, seed=N + 9)
    W8 = W8.view(torch.uint8)
    y = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
    ops.esimd_gemm_fp8_a8w8(q.to(dev), sa.to(dev), W8.to(dev), sb.to(dev), y)
    torch.cuda.synchronize()
    assert_close_fp(y.cpu(), ogemm.gemm_a8w8(q, sa, W8, sb), f"a8w8 rows-per-pass M={M} K={K} N={N}")


def test_gemv_misaligned_input(ops, dev):
    # an input view starting 2 bytes into its buffer -> generic path
    N, K = 64, 256
    _say("gemv misaligned input")
    W8, s = synthetic.weight_fp8(N, K, seed=9)
    buf = synthetic.activations(1, K + 1, seed=10)
    x = buf[:, 1:].contiguous()
    xd = buf.to(dev)[:, 1:]
    y = torch.zeros(1, N, dtype=torch.float16, device=dev)
    ops.esimd_gemv_fp8_pern(xd.contiguous() if not xd.is_contiguous() else xd, W8.to(dev), s.to(dev), y, N, K)
    torch.cuda.synchronize()
    assert_close_fp(y.cpu(), ogemv.gemv_fp8_pern(x, W8, s), "misaligned")


@pytest.mark.parametrize("sdt", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("io", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,K,N", [(17, 2048, 3000), (37, 1024, 512), (64, 4096, 4096), (300, 2048, 6000),
                                   (100, 640, 100), (40, 1000, 72), (50, 2048, 12)])
def test_gemv_many_rows(ops, dev, M, K, N, io, sdt):
    """M > 16 through the GEMV ops: the w8a16 GEMM dispatch with the
    per-channel scale (LDS GEMV up to 32 rows, tiled MFMA GEMM, tiny-N kernel
    for N <= 16, generic kernel for K % 64 != 0), weights streamed once; also
    the per-tensor op."""
    _say(f"gemv many rows M={M} K={K} N={N} {io} scale {sdt}")
    W8, s = synthetic.weight_fp8(N, K, seed=M + N)
    s = s.to(sdt)
    x = synthetic.activations(M, K, seed=M, dtype=io)
    y = torch.full((M, N), float("nan"), dtype=io, device=dev)
    ops.esimd_gemv_fp8_pern(x.to(dev), W8.to(dev), s.to(dev), y, N, K)
    sv = torch.tensor(0.013)
    yt = torch.full((M, N), float("nan"), dtype=io, device=dev)
    ops.esimd_gemv_fp8_pert(x.to(dev), W8.to(dev), sv.to(dev), yt)
    torch.cuda.synchronize()
    assert_close_fp(y.cpu(), ogemv.gemv_fp8_pern(x, W8, s), f"pern M={M}")
    assert_close_fp(yt.cpu(), ogemv.gemv_fp8_pert(x, W8, sv), f"pert M={M}")


def test_gemv_reference_row0_semantics(ops, dev):
    # output holding one row: only row 0 is computed, as the reference does
    N, K = 256, 512
    W8, s = synthetic.weight_fp8(N, K, seed=13)
    x = synthetic.activations(4, K, seed=14)
    y = torch.zeros(1, N, dtype=torch.float16, device=dev)
    ops.esimd_gemv_fp8_pern(x.to(dev), W8.to(dev), s.to(dev), y, N, K)
    torch.cuda.synchronize()
    assert_close_fp(y.cpu(), ogemv.gemv_fp8_pern(x[:1], W8, s), "row0")


@pytest.mark.parametrize("fmt", [torch.float8_e4m3fn, torch.float8_e5m2])
@pytest.mark.parametrize("M", [4, 16])
def test_fp8_decode_all_codes(ops, dev, fmt, M):
    """Known-answer test of the hardware decode: every finite code.

    x = identity rows, W[0, k] = code k  =>  y[m, 0] = dq(code m) exactly.
    M = 4 exercises the dot2 kernel, M = 16 the MFMA kernel.
    """
    _say(f"decode KAT fmt={fmt} M={M}")
    table = ofp8.E5M2_TABLE if fmt == torch.float8_e5m2 else ofp8.E4M3_TABLE
    codes = np.arange(256, dtype=np.uint8)
    finite = np.isfinite(table)
    row = np.where(finite, codes, 0).astype(np.uint8)
    W = torch.from_numpy(np.stack([row, row[::-1].copy()])).view(fmt).to(dev)   # N = 2
    one = torch.ones(1, dtype=torch.float32, device=dev)
    got = np.zeros(256, dtype=np.float32)
    for m0 in range(0, 256, M):
        x = torch.zeros(M, 256, dtype=torch.float32)
        for i in range(M):
            x[i, m0 + i] = 1.0
        y = torch.zeros(M, 2, dtype=torch.float32, device=dev).half()
        # e5m2 max 57344 overflows fp16 output only if > 65504: it does not.
        ops.esimd_gemv_fp8_pert(x.half().to(dev), W, one, y)
        torch.cuda.synchronize()
        got[m0:m0 + M] = y[:, 0].float().cpu().numpy()
    want = np.where(finite, table, 0.0).astype(np.float16).astype(np.float32)
    assert np.array_equal(got, want)


def test_fp8_nan_code_propagates(ops, dev):
    N, K = 2, 256
    W = torch.full((N, K), 0x38, dtype=torch.uint8)
    W[1, 5] = 0x7F
    x = torch.ones(1, K, dtype=torch.float16)
    y = torch.zeros(1, N, dtype=torch.float16, device=dev)
    ops.esimd_gemv_fp8_pert(x.to(dev), W.view(torch.float8_e4m3fn).to(dev), torch.ones(1, device=dev), y)
    torch.cuda.synchronize()
    ref = ogemv.gemv_fp8_pert(x, W.view(torch.float8_e4m3fn), torch.ones(1))
    assert y[0, 0].item() == ref[0, 0].item() == 256.0
    assert torch.isnan(y[0, 1]).item() and torch.isnan(ref[0, 1]).item()


def test_gemv_rejects_bad_input(ops, dev):
    W8 = torch.zeros(8, 64, dtype=torch.float8_e4m3fn, device=dev)
    x = torch.zeros(1, 64, dtype=torch.float32, device=dev)
    y = torch.zeros(1, 8, dtype=torch.float16, device=dev)
    with pytest.raises(RuntimeError, match="input must be fp16 or bf16"):
        ops.esimd_gemv_fp8_pern(x, W8, torch.ones(8, device=dev), y, 8, 64)
    with pytest.raises(RuntimeError, match="same dtype"):
        ops.esimd_gemv_fp8_pern(x.half(), W8, torch.ones(8, device=dev), y.bfloat16(), 8, 64)
    with pytest.raises(RuntimeError, match="weight holds"):
        ops.esimd_gemv_fp8_pern(x.half(), W8, torch.ones(8, device=dev), y, 8, 128)
    with pytest.raises(RuntimeError, match="fp32 scalar"):
        ops.esimd_gemv_fp8_pert(x.half(), W8, torch.ones(1, device=dev).half(), y)
