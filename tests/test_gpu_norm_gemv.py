"""GPU parity of add+RMSNorm (+ per-token e4m3 quant) fused into the GEMV.

esimd_fused_add_rms_norm_gemv_fp8 / esimd_fused_add_rms_norm_quant_gemv_fp8:
residual_out = hidden + residual, and the GEMV (or the gate/up GEMV with
gelu_and_mul) of the normed rows -- or of their e4m3 codes, which are also
written out with their scales.

Two references:

* the CPU oracle composition (oracle/norm.py, then oracle/gemv.py or
  oracle/gemm.py, then oracle/act.py for gelu_and_mul), to the op pack's
  tolerance; residual_out bit-exact, codes within one e4m3 step (the
  oracle's sum of squares runs in another order);
* the same device ops unfused (the norm op on copies, then the GEMV op):
  residual_out, codes and scales bit-identical always, and the product
  bit-identical wherever the unfused GEMV runs the LDS-staged kernel (three
  rows and more, or the gate/up form at any M) -- the fused prologue
  reproduces the norm kernel's thread layout and reduction order.

Shapes: every fused configuration (1 or up to 4 rows, the quantising form
1 row; K = 3, 4, 5 KiB values; one or two tiles per workgroup; the gate/up
form), N not a multiple of 16, and the two-launch path the ops take for
more rows (the quantising form: from two rows), other K, or a residual_out
that aliases residual.
"""

import sys

import numpy as np
import pytest
import torch

from conftest import assert_close_fp
from esimd_learning_amd import synthetic
from oracle import act as oact
from oracle import gemm as ogemm
from oracle import gemv as ogemv
from oracle import norm as onorm

pytestmark = pytest.mark.gpu
EPS = 1e-6


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _inputs(M, K, N, dtype, seed):
    h = synthetic.activations(M, K, seed=seed, dtype=dtype)
    r = synthetic.activations(M, K, seed=seed + 1, dtype=dtype)
    g = synthetic.norm_weight(K, seed=seed + 2, dtype=dtype)
    W8, s = synthetic.weight_fp8(N, K, seed=seed + 3)
    return h, r, g, W8, s


def _codes_near_oracle(q, qs, q_ref, s_ref, ulp):
    """The oracle sums the squares in another order, so a normed value can
    round one step apart: scales within one rounding step of the activation
    type, codes within one e4m3 step (exactness given the same normed values
    is checked against the device norm op)."""
    assert np.allclose(qs.numpy(), s_ref.numpy(), rtol=ulp, atol=0)
    mag = lambda c: np.where(c & 0x80, -(c & 0x7F), c & 0x7F)  # noqa: E731
    diff = np.abs(mag(q.numpy().astype(np.int64)) - mag(q_ref.numpy().astype(np.int64)))
    assert diff.max() <= 1


def _glu_ref(gu_f32, dtype):
    return torch.from_numpy(oact.gelu_and_mul(gu_f32.to(dtype).float().numpy()))


@pytest.mark.parametrize("glu", [False, True])
@pytest.mark.parametrize("K,N", [(3072, 6144), (4096, 6160), (5120, 1000), (4096, 16)])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 6])
def test_norm_gemv(ops, dev, M, K, N, glu):
    _say(f"norm+gemv M={M} K={K} N={N} glu={glu}")
    dt = torch.float16
    h, r, g, W8, s = _inputs(M, K, N, dt, seed=M + K + N)
    hd, rd, gd, Wd, sd = h.to(dev), r.to(dev), g.to(dev), W8.to(dev), s.to(dev)
    nout = N // 2 if glu else N
    r_out = torch.full((M, K), float("nan"), dtype=dt, device=dev)
    y = torch.full((M, nout), float("nan"), dtype=dt, device=dev)
    ops.esimd_fused_add_rms_norm_gemv_fp8(hd, rd, gd, EPS, r_out, Wd, sd, y, glu)
    # unfused device ops on copies
    h2, r2 = hd.clone(), rd.clone()
    ops.esimd_fused_add_rms_norm_batched(h2, r2, gd, EPS)
    y2 = torch.empty(M, nout, dtype=dt, device=dev)
    if glu:
        ops.esimd_gemv_fp8_gelu_and_mul(h2, Wd, sd, y2)
    else:
        ops.esimd_gemv_fp8_pern(h2, Wd, sd, y2, N, K)
    torch.cuda.synchronize()
    assert torch.equal(hd.cpu(), h) and torch.equal(rd.cpu(), r), "inputs must be left unchanged"
    assert torch.equal(r_out.cpu(), r2.cpu())
    r_ref, normed = onorm.fused_add_rms_norm(h, r, g, EPS)
    assert torch.equal(r_out.cpu(), r_ref)
    gu = ogemv.gemv_fp8_pern(normed.to(dt), W8, s)
    ref = _glu_ref(gu, dt) if glu else gu
    assert_close_fp(y.cpu(), ref, f"norm+gemv M={M} K={K} N={N} glu={glu}")
    if M >= 3 or glu:
        assert torch.equal(y.cpu(), y2.cpu()), "fused and unfused device results differ"


@pytest.mark.parametrize("glu", [False, True])
@pytest.mark.parametrize("K,N", [(3072, 12288), (4096, 6144), (5120, 520)])
@pytest.mark.parametrize("M", [1, 3, 4, 9])
def test_norm_quant_gemv(ops, dev, M, K, N, glu):
    _say(f"norm+quant+gemv M={M} K={K} N={N} glu={glu}")
    dt = torch.float16
    h, r, g, W8, s = _inputs(M, K, N, dt, seed=2 * M + K + N)
    hd, rd, gd = h.to(dev), r.to(dev), g.to(dev)
    b8, sb = W8.view(torch.uint8).to(dev), s.float().to(dev)
    nout = N // 2 if glu else N
    r_out = torch.full((M, K), float("nan"), dtype=dt, device=dev)
    q = torch.zeros(M, K, dtype=torch.uint8, device=dev)
    qs = torch.zeros(M, dtype=torch.float32, device=dev)
    y = torch.full((M, nout), float("nan"), dtype=dt, device=dev)
    ops.esimd_fused_add_rms_norm_quant_gemv_fp8(hd, rd, gd, EPS, r_out, q, qs, b8, sb, y, glu)
    # unfused device ops
    r2 = rd.clone()
    q2 = torch.empty(M, K, dtype=torch.uint8, device=dev)
    qs2 = torch.empty(M, dtype=torch.float32, device=dev)
    ops.esimd_fused_add_rms_norm_quant_fp8(hd, r2, gd, EPS, q2, qs2)
    y2 = torch.empty(M, nout, dtype=dt, device=dev)
    if glu:
        ops.esimd_gemm_fp8_a8w8_gelu_and_mul(q2, qs2, b8, sb, y2)
    else:
        ops.esimd_gemm_fp8_a8w8(q2, qs2, b8, sb, y2)
    torch.cuda.synchronize()
    assert torch.equal(rd.cpu(), r), "residual must be left unchanged"
    assert torch.equal(r_out.cpu(), r2.cpu())
    assert torch.equal(q.cpu(), q2.cpu()) and torch.equal(qs.cpu(), qs2.cpu())
    r_ref, q_ref, s_ref, _ = onorm.fused_add_rms_norm_quant(h, r, g, EPS)
    assert torch.equal(r_out.cpu(), r_ref)
    _codes_near_oracle(q.cpu(), qs.cpu(), q_ref, s_ref, 2.0 ** -10)
    gu = ogemm.gemm_a8w8(q_ref, s_ref, W8.view(torch.uint8), s.float())
    ref = _glu_ref(gu, dt) if glu else gu
    assert_close_fp(y.cpu(), ref, f"norm+quant+gemv M={M} K={K} N={N} glu={glu}")
    if 3 <= M <= 16 or (glu and M <= 16):
        assert torch.equal(y.cpu(), y2.cpu()), "fused and unfused device results differ"


@pytest.mark.parametrize("quant", [False, True])
def test_norm_gemv_bf16(ops, dev, quant):
    M, K, N = 4, 4096, 2000
    dt = torch.bfloat16
    _say(f"norm+gemv bf16 quant={quant}")
    h, r, g, W8, s = _inputs(M, K, N, dt, seed=77)
    hd, rd, gd = h.to(dev), r.to(dev), g.to(dev)
    r_out = torch.zeros(M, K, dtype=dt, device=dev)
    y = torch.zeros(M, N, dtype=dt, device=dev)
    if quant:
        q = torch.zeros(M, K, dtype=torch.uint8, device=dev)
        qs = torch.zeros(M, dtype=torch.float32, device=dev)
        ops.esimd_fused_add_rms_norm_quant_gemv_fp8(hd, rd, gd, EPS, r_out, q, qs, W8.view(torch.uint8).to(dev),
                                                    s.float().to(dev), y)
        r_ref, q_ref, s_ref, _ = onorm.fused_add_rms_norm_quant(h, r, g, EPS)
        ref = ogemm.gemm_a8w8(q_ref, s_ref, W8.view(torch.uint8), s.float())
    else:
        ops.esimd_fused_add_rms_norm_gemv_fp8(hd, rd, gd, EPS, r_out, W8.to(dev), s.to(dev), y)
        r_ref, normed = onorm.fused_add_rms_norm(h, r, g, EPS)
        ref = ogemv.gemv_fp8_pern(normed.to(dt), W8, s)
    torch.cuda.synchronize()
    assert torch.equal(r_out.cpu(), r_ref)
    if quant:
        _codes_near_oracle(q.cpu(), qs.cpu(), q_ref, s_ref, 2.0 ** -7)
    assert_close_fp(y.cpu(), ref, f"norm+gemv bf16 quant={quant}")


@pytest.mark.parametrize("K", [2048, 14336])
def test_norm_gemv_two_launch_shapes(ops, dev, K):
    """K outside the fused set: the op runs the norm on copies, then the GEMV."""
    M, N = 4, 520
    dt = torch.float16
    _say(f"norm+gemv two-launch K={K}")
    h, r, g, W8, s = _inputs(M, K, N, dt, seed=K)
    r_out = torch.zeros(M, K, dtype=dt, device=dev)
    y = torch.zeros(M, N, dtype=dt, device=dev)
    ops.esimd_fused_add_rms_norm_gemv_fp8(h.to(dev), r.to(dev), g.to(dev), EPS, r_out, W8.to(dev), s.to(dev), y)
    torch.cuda.synchronize()
    r_ref, normed = onorm.fused_add_rms_norm(h, r, g, EPS)
    assert torch.equal(r_out.cpu(), r_ref)
    assert_close_fp(y.cpu(), ogemv.gemv_fp8_pern(normed.to(dt), W8, s), f"two-launch K={K}")


@pytest.mark.parametrize("quant", [False, True])
def test_norm_gemv_residual_in_place(ops, dev, quant):
    """residual_out aliasing residual takes the two-launch path (a fused launch
    would race: workgroup 0 writes while the others still read)."""
    M, K, N = 4, 3072, 1024
    dt = torch.float16
    h, r, g, W8, s = _inputs(M, K, N, dt, seed=5)
    rd = r.to(dev)
    y = torch.zeros(M, N, dtype=dt, device=dev)
    if quant:
        q = torch.zeros(M, K, dtype=torch.uint8, device=dev)
        qs = torch.zeros(M, dtype=torch.float32, device=dev)
        ops.esimd_fused_add_rms_norm_quant_gemv_fp8(h.to(dev), rd, g.to(dev), EPS, rd, q, qs,
                                                    W8.view(torch.uint8).to(dev), s.float().to(dev), y)
        r_ref, q_ref, s_ref, _ = onorm.fused_add_rms_norm_quant(h, r, g, EPS)
        ref = ogemm.gemm_a8w8(q_ref, s_ref, W8.view(torch.uint8), s.float())
    else:
        ops.esimd_fused_add_rms_norm_gemv_fp8(h.to(dev), rd, g.to(dev), EPS, rd, W8.to(dev), s.to(dev), y)
        r_ref, normed = onorm.fused_add_rms_norm(h, r, g, EPS)
        ref = ogemv.gemv_fp8_pern(normed.to(dt), W8, s)
    torch.cuda.synchronize()
    assert torch.equal(rd.cpu(), r_ref)
    assert_close_fp(y.cpu(), ref, f"in-place residual quant={quant}")


@pytest.mark.parametrize("quant", [False, True])
@pytest.mark.parametrize("M,K", [(4, 3072), (6, 4096), (2, 2048)])
def test_norm_gemv_residual_out_is_hidden(ops, dev, quant, M, K):
    """residual_out aliasing hidden_states: the two-launch path seeds
    residual_out with residual, so it must read hidden from a copy first
    (M = 4 would be a fused shape, M = 6 and K = 2048 are two-launch shapes
    by size)."""
    N = 1040
    dt = torch.float16
    _say(f"norm+gemv residual_out=hidden M={M} K={K} quant={quant}")
    h, r, g, W8, s = _inputs(M, K, N, dt, seed=9 + M + K)
    hd = h.to(dev)
    y = torch.zeros(M, N, dtype=dt, device=dev)
    if quant:
        q = torch.zeros(M, K, dtype=torch.uint8, device=dev)
        qs = torch.zeros(M, dtype=torch.float32, device=dev)
        ops.esimd_fused_add_rms_norm_quant_gemv_fp8(hd, r.to(dev), g.to(dev), EPS, hd, q, qs,
                                                    W8.view(torch.uint8).to(dev), s.float().to(dev), y)
        r_ref, q_ref, s_ref, _ = onorm.fused_add_rms_norm_quant(h, r, g, EPS)
        ref = ogemm.gemm_a8w8(q_ref, s_ref, W8.view(torch.uint8), s.float())
    else:
        ops.esimd_fused_add_rms_norm_gemv_fp8(hd, r.to(dev), g.to(dev), EPS, hd, W8.to(dev), s.to(dev), y)
        r_ref, normed = onorm.fused_add_rms_norm(h, r, g, EPS)
        ref = ogemv.gemv_fp8_pern(normed.to(dt), W8, s)
    torch.cuda.synchronize()
    assert torch.equal(hd.cpu(), r_ref)
    if quant:
        _codes_near_oracle(q.cpu(), qs.cpu(), q_ref, s_ref, 2.0 ** -10)
    assert_close_fp(y.cpu(), ref, f"residual_out=hidden M={M} K={K} quant={quant}")


@pytest.mark.parametrize("quant", [False, True])
def test_norm_gemv_output_aliasing_input_falls_back(ops, dev, quant):
    """An output that shares memory with an input (here y over the tail of
    residual) would race in the fused launch: the op takes the two-launch
    path and the values stay those of the unaliased call."""
    M, K, N = 2, 4096, 2048
    dt = torch.float16
    _say(f"norm+gemv y aliasing residual quant={quant}")
    h, r, g, W8, s = _inputs(M, K, N, dt, seed=21)
    # residual [M, K] followed by y [M, N] in one buffer, y starting inside residual's last row
    buf = torch.zeros(M * K + M * N, dtype=dt, device=dev)
    rv = buf[: M * K].view(M, K)
    rv.copy_(r.to(dev))
    off = M * K - 1024
    yv = buf[off: off + M * N].view(M, N)
    r_out = torch.zeros(M, K, dtype=dt, device=dev)
    if quant:
        q = torch.zeros(M, K, dtype=torch.uint8, device=dev)
        qs = torch.zeros(M, dtype=torch.float32, device=dev)
        ops.esimd_fused_add_rms_norm_quant_gemv_fp8(h.to(dev), rv, g.to(dev), EPS, r_out, q, qs,
                                                    W8.view(torch.uint8).to(dev), s.float().to(dev), yv)
        r_ref, q_ref, s_ref, _ = onorm.fused_add_rms_norm_quant(h, r, g, EPS)
        ref = ogemm.gemm_a8w8(q_ref, s_ref, W8.view(torch.uint8), s.float())
    else:
        ops.esimd_fused_add_rms_norm_gemv_fp8(h.to(dev), rv, g.to(dev), EPS, r_out, W8.to(dev), s.to(dev), yv)
        r_ref, normed = onorm.fused_add_rms_norm(h, r, g, EPS)
        ref = ogemv.gemv_fp8_pern(normed.to(dt), W8, s)
    torch.cuda.synchronize()
    assert torch.equal(r_out.cpu(), r_ref)
    assert_close_fp(yv.cpu(), ref, f"y aliasing residual quant={quant}")
