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


def _producer(ops, x, W, s, r, w, dtype, dev, shift=0):
    M, N = x.shape[0], W.shape[0]
    rd = r.to(dev).clone()
    y = torch.full((M, N), float("nan"), dtype=dtype, device=dev)
    ss = torch.full((M, ops.esimd_gemv_fp8_add_rms_norm_defer_groups(N)), float("nan"), dtype=torch.float32,
                    device=dev)
    ops.esimd_gemv_fp8_add_rms_norm_defer(x.to(dev), W.to(dev), s.to(dev), rd, w.to(dev), y, ss, shift)
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


def test_defer_norm_shift_values(ops):
    """The shift is the smallest E with 2^E >= max|w| (host function)."""
    for m, e in ((1.0, 0), (1.36, 1), (2.0, 1), (8.0, 3), (8.31, 4), (0.3, -1), (0.5, -1), (0.0, 0), (65504.0, 16)):
        assert ops.esimd_defer_norm_shift(torch.tensor([m, -m / 2])) == e, m


@pytest.mark.parametrize("N", [3072, 4096])
def test_producer_shift_large_residual(ops, dev, N):
    """|residual| up to 3e4 and a norm weight up to ~8: residual * w
    reaches ~2.4e5, past fp16's 65504.  With the shift from
    esimd_defer_norm_shift (3 or 4), output = round(residual * w * 2^-shift) and the
    sums (times 4^-shift) equal the host's fp32 arithmetic bit for bit and are
    finite; with shift 0 the output overflows to inf (the documented limit
    of an unshifted hand-off)."""
    M, K, dtype = 4, 4096, torch.float16
    _say(f"defer producer shift N={N}")
    W, s = synthetic.weight_fp8(N, K, seed=N + 21)
    x = synthetic.activations(M, K, seed=22)
    r = (synthetic.activations(M, N, seed=23).float() * 1e4).clamp(-3e4, 3e4).half()
    w = (synthetic.norm_weight(N, seed=24).float() * 6.0).half()
    shift = ops.esimd_defer_norm_shift(w.to(dev))
    m = w.float().abs().max().item()
    assert 2.0 ** shift >= m > 2.0 ** (shift - 1) and shift >= 3
    o, _, _ = _producer(ops, x, W, s, torch.zeros(M, N, dtype=dtype), w, dtype, dev)  # the GEMV's rounded output
    of = o.float().numpy()
    r1, y1, ss1 = _producer(ops, x, W, s, r, w, dtype, dev, shift)
    sv = (of + r.float().numpy()).astype(np.float32)
    r_ref = torch.from_numpy(sv).to(dtype)
    assert torch.equal(r1, r_ref)
    ys = np.float32(2.0 ** -shift)
    y_ref = torch.from_numpy((r_ref.float().numpy() * w.float().numpy()).astype(np.float32) * ys).to(dtype)
    assert torch.isfinite(y1.float()).all()
    assert torch.equal(y1, y_ref)
    G = ss1.shape[1]
    assert torch.equal(ss1, torch.from_numpy(_butterfly16((sv * sv).astype(np.float32) * (ys * ys), G)))
    _, y0, _ = _producer(ops, x, W, s, r, w, dtype, dev, 0)
    assert not torch.isfinite(y0.float()).all()


@pytest.mark.parametrize("consumer", ["pern", "glu"])
def test_defer_extreme_rows_vs_oracle(ops, dev, consumer):
    """Producer (K = 4096 -> N = 3072, config 5's hidden size) then a
    consumer (the plain GEMV to 4096, or gate/up + gelu_and_mul to d = 1024)
    against the oracle's unfused chain (GEMV, add+RMSNorm, GEMV / gate-up +
    gelu_and_mul), row by row, on rows whose residual rms is 1e4 (|r|
    clipped to 3e4), 1, 1e-4 and 1e-5 (the tiny rows with a zero GEMV input,
    so that their sums are the residual's alone), with a norm weight up to
    ~8 (shift 3 or 4).  Below rms ~1e-5 the fp16 residual
    itself holds fewer than 8 significant bits and the moved rounding leaves
    the tolerance (a CPU model of the arithmetic: 3.5-4% of max|out| at
    rms 1e-6, 0.3-0.5% at 1e-5)."""
    from oracle import act as oact
    from oracle import norm as onorm
    M, K, H, d, dtype = 4, 4096, 3072, 1024, torch.float16
    _say(f"defer extreme rows {consumer}")
    Wo, so = synthetic.weight_fp8(H, K, seed=31)
    rows = torch.tensor([1e4, 1.0, 1e-4, 1e-5])[:, None]
    x = (synthetic.activations(M, K, seed=32).float() * torch.tensor([1.0, 1.0, 0.0, 0.0])[:, None]).half()
    r = (synthetic.activations(M, H, seed=33).float() * rows).clamp(-3e4, 3e4).half()
    w = (synthetic.norm_weight(H, seed=34).float() * 6.0).half()
    N2 = 2 * d if consumer == "glu" else 4096
    W2, s2 = synthetic.weight_fp8(N2, H, seed=35)
    shift = ops.esimd_defer_norm_shift(w)
    assert shift >= 3
    rd = r.to(dev).clone()
    y = torch.empty(M, H, dtype=dtype, device=dev)
    ss = torch.empty(M, ops.esimd_gemv_fp8_add_rms_norm_defer_groups(H), dtype=torch.float32, device=dev)
    ops.esimd_gemv_fp8_add_rms_norm_defer(x.to(dev), Wo.to(dev), so.to(dev), rd, w.to(dev), y, ss, shift)
    out = torch.full((M, d if consumer == "glu" else N2), float("nan"), dtype=dtype, device=dev)
    eps_s = EPS * 4.0 ** -shift
    if consumer == "glu":
        ops.esimd_gemv_fp8_gelu_and_mul_rs(y, W2.to(dev), s2.to(dev), out, ss, eps_s)
    else:
        ops.esimd_gemv_fp8_pern_rs(y, W2.to(dev), s2.to(dev), out, ss, eps_s)
    torch.cuda.synchronize()
    o = ogemv.gemv_fp8_pern(x, Wo, so).to(dtype)
    r_new, normed = onorm.fused_add_rms_norm(o, r, w, EPS)
    ref = ogemv.gemv_fp8_pern(normed.to(dtype), W2, s2)
    if consumer == "glu":
        ref = torch.from_numpy(oact.gelu_and_mul(ref.to(dtype).float().numpy())).to(dtype)
    else:
        ref = ref.to(dtype)
    assert_close_fp(rd.cpu().float(), r_new.float(), "residual")
    for m in range(M):
        err, mx = assert_close_fp(out.cpu()[m].float(), ref[m].float(), f"{consumer} row {m} (rms {rows[m, 0]:g})")
        print(f"  row {m} rms {rows[m, 0]:g}: max err / max|ref| = {err / mx:.2e}")


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


def test_forward_deferred_large_residual_vs_oracle(ops, dev):
    """Two config-5 layers (fp16, norms deferred) on a residual stream of
    |r| up to 3e4 (N(0, 1e4) clipped) with the add+RMSNorm weights scaled
    to ~8 (so residual * w reaches ~2.5e5, past fp16): the producers' shift
    keeps the hand-off finite; output and residual against the oracle's two
    decoder steps."""
    M, dims = 4, CONFIG5
    _say("defer forward, large residual")
    ps = [synthetic.gemma_layer(seed=sd, **dims) for sd in (80, 81)]
    for p in ps:
        for k in ("w_in", "w_post"):
            p[k] = (p[k].float() * 6.0).half()
    stack = [GemmaDecodeLayer(p, M, dev) for p in ps]
    assert all(layer.defer_norm and layer.shift_in >= 3 and layer.shift_post >= 3 for layer in stack)
    h = synthetic.activations(M, dims["hidden"], seed=82)
    r = (synthetic.activations(M, dims["hidden"], seed=83).float() * 1e4).clamp(-3e4, 3e4).half()
    pos = synthetic.positions(M, seed=84)
    rd = r.to(dev)
    out = forward(stack, h.to(dev), rd, pos.to(dev)).clone()
    torch.cuda.synchronize()
    o1, r1, _ = olayer.decoder_step(ps[0], h, r, pos)
    o2, r2, _ = olayer.decoder_step(ps[1], o1.to(h.dtype), r1, pos)
    assert_close_fp(rd.cpu().float(), r2.float(), "residual after two layers")
    err, mx = assert_close_fp(out.cpu().float(), o2.float(), "output of two layers")
    print(f"  output max err / max|ref| = {err / mx:.2e}")


def test_forward_eight_layers_as_benched(ops, dev):
    """The decode forward the benchmark times (bench_layer): eight chained
    config-5 layers sharing one weight set (seed 10; the bench gives each
    layer its own copy of the same values), M = 4, fp16, the default step
    (both add+RMSNorms deferred across the GEMVs around them, QK-norm+RoPE
    in the QKV GEMV's tail, gate/up with gelu_and_mul), hidden, residual and
    positions from seeds 20, 21 and 22; run once eagerly, and its graph
    replayed.  Output and residual against eight oracle decoder steps, to
    the op pack's tolerance; the errors are printed as max-abs / max|ref|."""
    M, L = 4, 8
    _say("defer forward, eight layers")
    p = synthetic.gemma_layer(seed=10)
    pd = {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in p.items()}
    stack = [GemmaDecodeLayer(pd, M, dev) for _ in range(L)]
    assert all(layer.defer_norm and layer.fuse_tails and layer.fuse_glu for layer in stack)
    h = synthetic.activations(M, p["hidden"], seed=20)
    r = synthetic.activations(M, p["hidden"], seed=21)
    pos = synthetic.positions(M, seed=22)
    hd, rd, posd = h.to(dev), r.to(dev), pos.to(dev)
    out = forward(stack, hd.clone(), rd, posd).clone()
    torch.cuda.synchronize()
    ho, ro = h, r
    for _ in range(L):
        o, ro, _ = olayer.decoder_step(p, ho, ro, pos)
        ho = o.to(h.dtype)
    err_r, mr = assert_close_fp(rd.cpu().float(), ro.float(), "residual after eight layers")
    err_o, mo = assert_close_fp(out.cpu().float(), o.float(), "output after eight layers")
    print(f"  eight layers: output max err / max|ref| = {err_o / mo:.2e}, residual {err_r / mr:.2e}")
    # the captured forward (what the bench replays) gives the same values
    hb, rb = hd.clone(), r.to(dev)
    g = capture_forward(stack, hb, rb, posd)
    for _ in range(2):
        hb.copy_(hd)
        rb.copy_(r.to(dev))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(stack[-1].out, out)
        assert torch.equal(rb, rd)
