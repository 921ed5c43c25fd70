"""GPU parity of the deferred add + RMSNorm between two decode GEMVs.

Producer esimd_gemv_fp8_add_rms_norm_defer (o = GEMV(x); s = o + residual;
residual = round(s); output = round(residual * w); row_ss = per-16-column
sums of s^2) and the row-scaled consumers esimd_gemv_fp8_pern_rs,
esimd_gemv_fp8_gelu_and_mul_rs, esimd_gemv_fp8_qk_norm_rope_rs.

* The producer's GEMV part is checked against the oracle GEMV through a
  call with a zero residual (then residual_out = o exactly); its residual,
  output and sums are then checked bit for bit against the same fp32
  arithmetic done on the host from o (the sums' butterfly order included,
  over 16-column runs or, N = 1536 and 3072, 12-column runs padded to 16
  with zeros).
* The plain consumer is checked against the oracle composition: the norm
  of the reference (x * w / rms, oracle/norm.py) then the oracle GEMV,
  to the op pack's tolerance -- the moved 1 / rms changes the rounding, so
  not bit for bit.
* The gate/up and QKV consumers equal the plain consumer followed by the
  device gelu_and_mul / QK-norm + RoPE ops, bit for bit (same kernel
  family, same K order, same row scales).
* A decode forward over two layers with the norms deferred matches the
  oracle's two decoder steps, and its graph replays equal the eager run.
"""

import sys

import numpy as np
import pytest
import torch

from conftest import assert_close_fp
from esimd_learning_amd import synthetic
from esimd_learning_amd.layer import GemmaDecodeLayer, capture_forward, forward
from oracle import gemv as ogemv
from oracle import layer as olayer

pytestmark = pytest.mark.gpu

CONFIG5 = dict(hidden=3072, n_q=16, n_kv=16, head_dim=256, mlp=24576)
EPS = 1e-6


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _butterfly16(sq, groups):
    """The producer's per-tile sum of the fp32 squares of N / groups columns
    (16 or 12; 12 padded with four zeros to the 16 lanes), pairwise:
    ((c0 + c1) + (c2 + c3)) + ((c4 + c5) + (c6 + c7)), then the two halves
    (xor-partner adds over offsets 1, 2, 4, 8).  sq: float32 [M, N]."""
    M, N = sq.shape
    rows = N // groups
    assert rows in (12, 16) and rows * groups == N
    a = np.zeros((M, groups, 16), dtype=np.float32)
    a[..., :rows] = sq.reshape(M, groups, rows)
    idx = np.arange(16)
    for off in (1, 2, 4, 8):
        a = (a + a[..., idx ^ off]).astype(np.float32)
    return a[..., 0]


def _producer(ops, x, W, s, r, w, dtype, dev):
    M, N = x.shape[0], W.shape[0]
    rd = r.to(dev).clone()
    y = torch.full((M, N), float("nan"), dtype=dtype, device=dev)
    ss = torch.full((M, ops.esimd_gemv_fp8_add_rms_norm_defer_groups(N)), float("nan"), dtype=torch.float32,
                    device=dev)
    ops.esimd_gemv_fp8_add_rms_norm_defer(x.to(dev), W.to(dev), s.to(dev), rd, w.to(dev), y, ss)
    torch.cuda.synchronize()
    return rd.cpu(), y.cpu(), ss.cpu()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("K,N", [(4096, 3072), (2048, 512), (24576, 3072), (5120, 4096), (3072, 1536)])
@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_producer(ops, dev, M, K, N, dtype):
    _say(f"defer producer M={M} K={K} N={N} {dtype}")
    W, s = synthetic.weight_fp8(N, K, seed=K + N)
    x = synthetic.activations(M, K, seed=M + 3, dtype=dtype)
    r = synthetic.activations(M, N, seed=M + 4, dtype=dtype)
    w = synthetic.norm_weight(N, seed=5).to(dtype)
    # zero residual: residual_out is the GEMV's rounded output
    o, y0, ss0 = _producer(ops, x, W, s, torch.zeros(M, N, dtype=dtype), w, dtype, dev)
    assert_close_fp(o.float(), ogemv.gemv_fp8_pern(x, W, s).to(dtype).float(), f"GEMV part M={M} K={K}")
    of = o.float().numpy()
    wf = w.float().numpy()
    assert torch.equal(y0, torch.from_numpy(of * wf).to(dtype))
    G = ss0.shape[1]
    assert G == (N // 12 if N in (1536, 3072) else N // 16)
    assert torch.equal(ss0, torch.from_numpy(_butterfly16(of * of, G)))
    # with the residual: the same o, then the host's fp32 arithmetic
    r1, y1, ss1 = _producer(ops, x, W, s, r, w, dtype, dev)
    sv = (of + r.float().numpy()).astype(np.float32)
    r_ref = torch.from_numpy(sv).to(dtype)
    assert torch.equal(r1, r_ref)
    assert torch.equal(y1, torch.from_numpy(r_ref.float().numpy() * wf).to(dtype))
    assert torch.equal(ss1, torch.from_numpy(_butterfly16(sv * sv, G)))


def _ss_of(v, nss):
    """Partial sums of squares [M, nss] of v [M, K] over K / nss columns each (float32)."""
    M = v.shape[0]
    return torch.from_numpy((v.float().numpy() ** 2).reshape(M, nss, -1).sum(-1).astype(np.float32))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("K,N", [(3072, 4096), (4096, 3072), (24576, 3072), (2048, 1040)])
@pytest.mark.parametrize("M", [1, 2, 4])
def test_rowscale_vs_oracle(ops, dev, M, K, N, dtype):
    """pern_rs(round(v * w), ss(v)) against the reference's norm -> GEMV:
    GEMV(round(v * w / rms(v))), rms from the same sums."""
    _say(f"defer consumer M={M} K={K} N={N} {dtype}")
    W, s = synthetic.weight_fp8(N, K, seed=K + 2 * N)
    v = synthetic.activations(M, K, seed=M + 7, dtype=dtype)
    w = synthetic.norm_weight(K, seed=8).to(dtype)
    nss = min(K // 16, 256)              # the consumers take up to 256 partial sums per row
    ss = _ss_of(v, nss)
    xp = (v.float() * w.float()).to(dtype)
    y = torch.full((M, N), float("nan"), dtype=dtype, device=dev)
    ops.esimd_gemv_fp8_pern_rs(xp.to(dev), W.to(dev), s.to(dev), y, ss.to(dev), EPS)
    torch.cuda.synchronize()
    inv = torch.rsqrt(ss.double().sum(-1, keepdim=True) / K + EPS)
    normed = (v.double() * inv * w.double()).to(dtype)            # the reference's norm output
    ref = ogemv.gemv_fp8_pern(normed, W, s).to(dtype)
    assert_close_fp(y.cpu().float(), ref.float(), f"pern_rs M={M} K={K} N={N}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("K", [3072, 4096, 5120])
@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_glu_rs_equals_unfused(ops, dev, M, K, dtype):
    d = 1024
    _say(f"defer glu M={M} K={K} {dtype}")
    W, s = synthetic.weight_fp8(2 * d, K, seed=K + 11)
    v = synthetic.activations(M, K, seed=M + 12, dtype=dtype).to(dev)
    ss = _ss_of(v.cpu(), min(K // 16, 256)).to(dev)
    Wd, sd = W.to(dev), s.to(dev)
    out = torch.full((M, d), float("nan"), dtype=dtype, device=dev)
    ops.esimd_gemv_fp8_gelu_and_mul_rs(v, Wd, sd, out, ss, EPS)
    gu = torch.empty(M, 2 * d, dtype=dtype, device=dev)
    ops.esimd_gemv_fp8_pern_rs(v, Wd, sd, gu, ss, EPS)
    ref = torch.empty(M, d, dtype=dtype, device=dev)
    ops.esimd_gelu_and_mul(ref, gu)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hd,nq,nk", [(256, 16, 16), (128, 8, 2)])
@pytest.mark.parametrize("M", [1, 4])
def test_qk_rope_rs_equals_unfused(ops, dev, M, hd, nq, nk, dtype):
    K = 3072
    N = (nq + 2 * nk) * hd
    _say(f"defer qkv M={M} hd={hd}")
    W, s = synthetic.weight_fp8(N, K, seed=N + 13)
    v = synthetic.activations(M, K, seed=M + 14, dtype=dtype).to(dev)
    ss = _ss_of(v.cpu(), 96).to(dev)
    qw = synthetic.norm_weight(hd, seed=15).to(dtype).to(dev)
    kw = synthetic.norm_weight(hd, seed=16).to(dtype).to(dev)
    pos = synthetic.positions(M, seed=17).to(dev)
    cnt = ops.gemv_tail_counters(nq, nk, dev)
    Wd, sd = W.to(dev), s.to(dev)
    out = torch.full((M, N), float("nan"), dtype=dtype, device=dev)
    q_out = torch.full((M, nq * hd), float("nan"), dtype=dtype, device=dev)
    ops.esimd_gemv_fp8_qk_norm_rope_rs(v, Wd, sd, out, qw, kw, pos, nq, nk, EPS, 10000.0, True, cnt, ss, EPS, q_out)
    ref = torch.empty(M, N, dtype=dtype, device=dev)
    ops.esimd_gemv_fp8_pern_rs(v, Wd, sd, ref, ss, EPS)
    ops.esimd_qk_norm_rope(ref[:, : nq * hd], ref[:, nq * hd:(nq + nk) * hd], qw, kw, pos, EPS, 10000.0, True)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    assert torch.equal(q_out, ref[:, : nq * hd])
    assert int(cnt.abs().sum()) == 0, "arrival counters must be left zero"


def test_empty_batch_is_a_no_op(ops, dev):
    """M = 0: every deferred-norm op returns without touching its outputs."""
    K, N, d = 4096, 3072, 1024
    W, s = synthetic.weight_fp8(N, K, seed=3)
    Wg, sg = synthetic.weight_fp8(2 * d, 3072, seed=4)
    Wd, sd, Wgd, sgd = W.to(dev), s.to(dev), Wg.to(dev), sg.to(dev)
    x = torch.empty(0, K, dtype=torch.float16, device=dev)
    res = torch.empty(0, N, dtype=torch.float16, device=dev)
    y = torch.empty(0, N, dtype=torch.float16, device=dev)
    ss = torch.empty(0, ops.esimd_gemv_fp8_add_rms_norm_defer_groups(N), dtype=torch.float32, device=dev)
    nw = synthetic.norm_weight(N, seed=5).to(dev)
    ops.esimd_gemv_fp8_add_rms_norm_defer(x, Wd, sd, res, nw, y, ss)
    ops.esimd_gemv_fp8_pern_rs(x, Wd, sd, y, ss, EPS)
    xg = torch.empty(0, 3072, dtype=torch.float16, device=dev)
    out = torch.empty(0, d, dtype=torch.float16, device=dev)
    ops.esimd_gemv_fp8_gelu_and_mul_rs(xg, Wgd, sgd, out, torch.empty(0, 192, device=dev), EPS)
    torch.cuda.synchronize()


def test_producer_refuses_aliased_outputs(ops, dev):
    """The producer's output must not share memory with the residual it
    updates (other workgroups still read it), and row_ss must hold this N's
    partial-sum count: the op raises."""
    M, K, N = 2, 4096, 3072
    W, s = synthetic.weight_fp8(N, K, seed=6)
    x = synthetic.activations(M, K, seed=7).to(dev)
    res = synthetic.activations(M, N, seed=8).to(dev)
    nw = synthetic.norm_weight(N, seed=9).to(dev)
    ss = torch.empty(M, ops.esimd_gemv_fp8_add_rms_norm_defer_groups(N), dtype=torch.float32, device=dev)
    with pytest.raises(RuntimeError):
        ops.esimd_gemv_fp8_add_rms_norm_defer(x, W.to(dev), s.to(dev), res, nw, res, ss)
    with pytest.raises(RuntimeError):   # row_ss of the 16-column runs: not this N's G
        ops.esimd_gemv_fp8_add_rms_norm_defer(x, W.to(dev), s.to(dev), res, nw,
                                              torch.empty(M, N, dtype=torch.float16, device=dev),
                                              torch.empty(M, N // 16, dtype=torch.float32, device=dev))


def test_unsupported_shapes_raise(ops, dev):
    W, s = synthetic.weight_fp8(512, 1000, seed=1)
    x = torch.zeros(2, 1000, dtype=torch.float16, device=dev)
    y = torch.empty(2, 512, dtype=torch.float16, device=dev)
    ss = torch.ones(2, 8, dtype=torch.float32, device=dev)
    with pytest.raises(RuntimeError):
        ops.esimd_gemv_fp8_pern_rs(x, W.to(dev), s.to(dev), y, ss, EPS)   # K not a multiple of 1024
    W, s = synthetic.weight_fp8(512, 4096, seed=1)
    x = torch.zeros(5, 4096, dtype=torch.float16, device=dev)
    y = torch.empty(5, 512, dtype=torch.float16, device=dev)
    with pytest.raises(RuntimeError):
        ops.esimd_gemv_fp8_pern_rs(x, W.to(dev), s.to(dev), y, torch.ones(5, 8, device=dev), EPS)  # M > 4
    with pytest.raises(RuntimeError):
        ops.esimd_gemv_fp8_pern_rs(x[:2], W.to(dev), s.to(dev), y[:2], torch.ones(2, 260, device=dev), EPS)
    with pytest.raises(RuntimeError):   # n_ss not a multiple of 4
        ops.esimd_gemv_fp8_pern_rs(x[:2], W.to(dev), s.to(dev), y[:2], torch.ones(2, 6, device=dev), EPS)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_forward_deferred_vs_oracle(ops, dev, dtype):
    """Two config-5 layers with the default step -- the norms deferred in
    fp16; in bf16, where the moved rounding exceeds the tolerance over two
    layers, the norm launches kept: the output and residual match the
    oracle's two decoder steps; graph replays equal the eager run."""
    M, dims = 4, CONFIG5
    ps = [synthetic.gemma_layer(seed=sd, **dims) for sd in (70, 71)]
    for p in ps:   # the norm weights in the activation dtype, as the layer holds them
        for k in ("w_in", "w_post", "qw", "kw"):
            p[k] = p[k].to(dtype)
    stack = [GemmaDecodeLayer(p, M, dev, dtype=dtype) for p in ps]
    assert all(layer.defer_norm == (dtype == torch.float16) for layer in stack)
    h = synthetic.activations(M, dims["hidden"], seed=72, dtype=dtype)
    r = synthetic.activations(M, dims["hidden"], seed=73, dtype=dtype)
    pos = synthetic.positions(M, seed=74)
    hd, rd, posd = h.to(dev), r.to(dev), pos.to(dev)
    out = forward(stack, hd.clone(), rd, posd).clone()
    ref_r = rd.clone()
    torch.cuda.synchronize()
    o1, r1, _ = olayer.decoder_step(ps[0], h, r, pos)
    o2, r2, _ = olayer.decoder_step(ps[1], o1.to(h.dtype), r1, pos)
    assert_close_fp(rd.cpu().float(), r2.float(), "residual after two layers")
    assert_close_fp(out.cpu().float(), o2.float(), "output of two layers")
    hb, rb = hd.clone(), r.to(dev)
    g = capture_forward(stack, hb, rb, posd)
    for _ in range(3):
        hb.copy_(hd)
        rb.copy_(r.to(dev))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(stack[1].out, out)
        assert torch.equal(rb, ref_r)
        torch.randn(1000, device=dev).sum().item()   # unrelated eager work between replays
