"""GPU parity of the gate/up GEMV with gelu_and_mul fused into its epilogue.

esimd_gemv_fp8_gelu_and_mul(input [M, K], weight [2d, K], weight_scale [2d],
output [M, d]) and esimd_gemm_fp8_a8w8_gelu_and_mul (e4m3 activations with
per-token scales, e4m3 weights with fp32 per-channel scales).

Two references:

* the CPU oracle composition -- the GEMV (oracle/gemv.py, oracle/gemm.py)
  rounded to the activation dtype, then gelu_and_mul in float64
  (oracle/act.py) -- to the op pack's tolerance;
* the same device ops unfused (the GEMV into [M, 2d], then
  esimd_gelu_and_mul): bit-identical wherever the unfused GEMV runs the same
  LDS-staged MFMA kernel (M >= 3 here), since the fused epilogue rounds g and
  u to the output type and applies the same gelu code -- except, with fp16 /
  bf16 activations at M <= 4 (where each 16-row tile reads its K chunks in a
  rotated order), for d not a multiple of 16: the fused kernel's up tiles
  then straddle two of the unfused GEMV's tiles, whose K sums run in
  different orders.

The shapes reach every fused configuration (M <= 4, <= 8, <= 16; K = 3, 4
and 5 KiB values), d a multiple of 16 and not, M > 16 (the w8a16 GEMM, then
gelu_and_mul), and the unfused path the ops take for K outside the fused
set.
"""

import sys

import pytest
import torch

from conftest import assert_close_fp
from esimd_learning_amd import synthetic
from oracle import act as oact
from oracle import gemm as ogemm
from oracle import gemv as ogemv
from oracle import norm as onorm

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _ref_glu(gu_f32, dtype):
    """Oracle: round the GEMV output to the activation dtype, then gelu_and_mul."""
    gu = gu_f32.to(dtype)
    return torch.from_numpy(oact.gelu_and_mul(gu.float().numpy()))


def _unfused(ops, x, W8, s, dtype, dev):
    M, K = x.shape
    d = W8.shape[0] // 2
    gu = torch.empty(M, 2 * d, dtype=dtype, device=dev)
    ops.esimd_gemv_fp8_pern(x, W8, s, gu, 2 * d, K)
    out = torch.empty(M, d, dtype=dtype, device=dev)
    ops.esimd_gelu_and_mul(out, gu)
    return out


@pytest.mark.parametrize("K,d", [(3072, 1000), (4096, 2056), (5120, 520), (3072, 8), (3072, 1024), (4096, 3072)])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 6, 8, 11, 16, 21])
def test_glu_fp16(ops, dev, M, K, d):
    _say(f"glu fp16 M={M} K={K} d={d}")
    W8, s = synthetic.weight_fp8(2 * d, K, seed=K + d)
    x = synthetic.activations(M, K, seed=M + d)
    xd, Wd, sd = x.to(dev), W8.to(dev), s.to(dev)
    out = torch.full((M, d), float("nan"), dtype=torch.float16, device=dev)
    ops.esimd_gemv_fp8_gelu_and_mul(xd, Wd, sd, out)
    ref_dev = _unfused(ops, xd, Wd, sd, torch.float16, dev)
    torch.cuda.synchronize()
    assert_close_fp(out.cpu(), _ref_glu(ogemv.gemv_fp8_pern(x, W8, s), torch.float16), f"glu M={M} K={K} d={d}")
    if M >= 3 and (d % 16 == 0 or M > 4):
        assert torch.equal(out.cpu(), ref_dev.cpu()), "fused and unfused device results differ"


@pytest.mark.parametrize("io", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("fmt", [torch.float8_e4m3fn, torch.float8_e5m2])
@pytest.mark.parametrize("sdt", [torch.float16, torch.bfloat16, torch.float32])
def test_glu_types(ops, dev, io, fmt, sdt):
    M, K, d = 5, 4096, 700
    _say(f"glu types {io} {fmt} scale {sdt}")
    g = torch.Generator().manual_seed(7)
    W8 = (torch.randn(2 * d, K, generator=g) * 0.1).to(fmt)
    s = (torch.rand(2 * d, generator=g) * 0.05 + 0.01).to(sdt)
    x = (torch.randn(M, K, generator=g) * 0.5).to(io)
    xd, Wd, sd = x.to(dev), W8.to(dev), s.to(dev)
    out = torch.zeros(M, d, dtype=io, device=dev)
    ops.esimd_gemv_fp8_gelu_and_mul(xd, Wd, sd, out)
    ref_dev = _unfused(ops, xd, Wd, sd, io, dev)
    torch.cuda.synchronize()
    assert_close_fp(out.cpu(), _ref_glu(ogemv.gemv_fp8_pern(x, W8, s), io), f"glu {io} {fmt} {sdt}")
    assert torch.equal(out.cpu(), ref_dev.cpu())


@pytest.mark.parametrize("K", [2048, 14336])
def test_glu_unfused_path(ops, dev, K):
    """K outside the fused kernel's set: the op runs the GEMV, then gelu_and_mul."""
    M, d = 4, 264
    _say(f"glu unfused path K={K}")
    W8, s = synthetic.weight_fp8(2 * d, K, seed=K)
    x = synthetic.activations(M, K, seed=3)
    out = torch.zeros(M, d, dtype=torch.float16, device=dev)
    ops.esimd_gemv_fp8_gelu_and_mul(x.to(dev), W8.to(dev), s.to(dev), out)
    torch.cuda.synchronize()
    assert_close_fp(out.cpu(), _ref_glu(ogemv.gemv_fp8_pern(x, W8, s), torch.float16), f"glu K={K}")


def test_glu_rejects_bad_shapes(ops, dev):
    x = torch.zeros(2, 4096, dtype=torch.float16, device=dev)
    W8 = torch.zeros(63, 4096, dtype=torch.float8_e4m3fn, device=dev)
    s = torch.ones(63, dtype=torch.float32, device=dev)
    out = torch.zeros(2, 31, dtype=torch.float16, device=dev)
    with pytest.raises(RuntimeError, match="2d"):
        ops.esimd_gemv_fp8_gelu_and_mul(x, W8, s, out)
    W8 = torch.zeros(64, 4096, dtype=torch.float8_e4m3fn, device=dev)
    s = torch.ones(64, dtype=torch.float32, device=dev)
    with pytest.raises(RuntimeError, match=r"\[M, d\]"):
        ops.esimd_gemv_fp8_gelu_and_mul(x, W8, s, out)


@pytest.mark.parametrize("K,d", [(3072, 1000), (4096, 6144), (5120, 24)])
@pytest.mark.parametrize("M", [1, 4, 9, 16, 20])
def test_glu_a8w8(ops, dev, M, K, d):
    """e4m3 activations from the per-token quant; M = 20 runs the tiled GEMM + gelu."""
    _say(f"glu a8w8 M={M} K={K} d={d}")
    W8, s = synthetic.weight_fp8(2 * d, K, seed=K + M)
    x = synthetic.activations(M, K, seed=d)
    q, qs = onorm.per_token_quant(x)
    qd, qsd = q.view(torch.uint8).to(dev), qs.to(dev)
    b8, sb = W8.view(torch.uint8).to(dev), s.float().to(dev)
    out = torch.full((M, d), float("nan"), dtype=torch.float16, device=dev)
    ops.esimd_gemm_fp8_a8w8_gelu_and_mul(qd, qsd, b8, sb, out)
    gu = torch.empty(M, 2 * d, dtype=torch.float16, device=dev)
    ops.esimd_gemm_fp8_a8w8(qd, qsd, b8, sb, gu)
    ref_dev = torch.empty(M, d, dtype=torch.float16, device=dev)
    ops.esimd_gelu_and_mul(ref_dev, gu)
    torch.cuda.synchronize()
    ref = _ref_glu(ogemm.gemm_a8w8(q, qs, W8.view(torch.uint8), s.float()), torch.float16)
    assert_close_fp(out.cpu(), ref, f"glu a8w8 M={M} K={K} d={d}")
    if 3 <= M <= 16:
        assert torch.equal(out.cpu(), ref_dev.cpu()), "fused and unfused device results differ"


def test_glu_a8w8_bf16_out(ops, dev):
    M, K, d = 8, 3072, 520
    W8, s = synthetic.weight_fp8(2 * d, K, seed=11)
    x = synthetic.activations(M, K, seed=12)
    q, qs = onorm.per_token_quant(x)
    out = torch.zeros(M, d, dtype=torch.bfloat16, device=dev)
    ops.esimd_gemm_fp8_a8w8_gelu_and_mul(q.view(torch.uint8).to(dev), qs.to(dev), W8.view(torch.uint8).to(dev),
                                         s.float().to(dev), out)
    torch.cuda.synchronize()
    ref = _ref_glu(ogemm.gemm_a8w8(q, qs, W8.view(torch.uint8), s.float()), torch.bfloat16)
    assert_close_fp(out.cpu(), ref, "glu a8w8 bf16")
