"""Pins of the GEMV / GEMM / norm / activation / RoPE oracles (CPU).

Each oracle is checked against something other than its own formula: a
float64 loop or brute force on tiny shapes, a library routine computing the
same function (torch.nn.functional.gelu, rms_norm), a different formulation
(complex rotation for RoPE), or invariants a wrong index or sign breaks.
"""

import math

import numpy as np
import pytest
import torch

from esimd_learning_amd import synthetic
from oracle import act, fp8, gemm, gemv, norm


def _tiny_gemv(M=2, N=8, K=64, seed=0):
    W8, s = synthetic.weight_fp8(N, K, seed=seed)
    x = synthetic.activations(M, K, seed=seed + 1)
    return x, W8, s


# ---------------------------------------------------------------- GEMV / GEMM
def test_gemv_vs_bruteforce_f64():
    x, W8, s = _tiny_gemv()
    y = gemv.gemv_fp8_pern(x, W8, s).double().numpy()
    yb = gemv.gemv_bruteforce_f64(x, W8, s)
    assert np.allclose(y, yb, rtol=1e-5, atol=1e-6 * np.abs(yb).max())


def test_gemv_e5m2_vs_bruteforce_f64():
    W = torch.randn(8, 64, generator=torch.Generator().manual_seed(3)) * 0.1
    W8 = W.to(torch.float8_e5m2)
    x = synthetic.activations(3, 64, seed=4)
    s = torch.rand(8, generator=torch.Generator().manual_seed(5)).half()
    y = gemv.gemv_fp8_pern(x, W8, s).double().numpy()
    yb = gemv.gemv_bruteforce_f64(x, W8, s)
    assert np.allclose(y, yb, rtol=1e-5, atol=1e-6 * np.abs(yb).max())


def test_gemv_decode_uses_table():
    # decoding through the oracle's own table gives the same weights as torch
    _, W8, _ = _tiny_gemv(N=32, K=128)
    wf = gemv.dequant_weight(W8).numpy()
    assert np.array_equal(wf, fp8.decode_e4m3(W8.view(torch.uint8).numpy()))


def test_gemv_linear_in_scale_and_zero_weight():
    x, W8, s = _tiny_gemv(M=3, N=16, K=128)
    y1 = gemv.gemv_fp8_pern(x, W8, s)
    y2 = gemv.gemv_fp8_pern(x, W8, s * 2)
    assert torch.equal(y2, y1 * 2)
    z = gemv.gemv_fp8_pern(x, torch.zeros_like(W8.view(torch.uint8)).view(torch.float8_e4m3fn), s)
    assert torch.count_nonzero(z) == 0


def test_pert_equals_pern_uniform_scale():
    x, W8, _ = _tiny_gemv(M=1, N=16, K=128)
    sv = torch.tensor(0.073, dtype=torch.float32)
    a = gemv.gemv_fp8_pert(x, W8, sv)
    b = gemv.gemv_fp8_pern(x, W8, torch.full((16,), 0.073, dtype=torch.float32))
    assert torch.equal(a, b)


def test_gemm_m1_equals_gemv():
    x, W8, _ = _tiny_gemv(M=1, N=16, K=128)
    sv = torch.tensor(0.05)
    assert torch.equal(gemv.gemm_fp8_pert(x, W8, sv), gemv.gemv_fp8_pert(x, W8, sv))


def test_a8w8_vs_bruteforce_and_bilinear():
    rng = np.random.default_rng(7)
    M, N, K = 3, 5, 48
    a8 = torch.from_numpy(rng.integers(0, 256, (M, K), dtype=np.uint8))
    b8 = torch.from_numpy(rng.integers(0, 256, (N, K), dtype=np.uint8))
    a8[a8 & 0x7F == 0x7F] = 0x38    # no NaN codes
    b8[b8 & 0x7F == 0x7F] = 0x30
    sa = torch.rand(M) + 0.5
    sb = torch.rand(N) + 0.5
    y = gemm.gemm_a8w8(a8, sa, b8, sb).double().numpy()
    A, B = fp8.decode_e4m3(a8.numpy()).astype(np.float64), fp8.decode_e4m3(b8.numpy()).astype(np.float64)
    yb = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            yb[m, n] = sum(A[m, k] * B[n, k] for k in range(K)) * float(sa[m]) * float(sb[n])
    assert np.allclose(y, yb, rtol=1e-5, atol=1e-5 * np.abs(yb).max())
    y2 = gemm.gemm_a8w8(a8, sa * 2, b8, sb * 4).double().numpy()
    assert np.allclose(y2, 8 * y, rtol=1e-6)


def test_a8w8_matches_fp16_gemm_oracle():
    # A's e4m3 codes are exactly representable in fp16, so a8w8 with sa = 1
    # equals the fp16-activation GEMM oracle fed those values.
    x, W8, s = _tiny_gemv(M=4, N=8, K=64)
    q, sa = norm.per_token_quant(x)
    xa = q.view(torch.float8_e4m3fn).to(torch.float16)
    ref = gemv.gemv_fp8_pern(xa, W8, s)
    got = gemm.gemm_a8w8(q, torch.ones(4), W8.view(torch.uint8), s)
    assert torch.allclose(got, ref, rtol=1e-6, atol=1e-6)


# ---------------------------------------------------------------- norm
def test_norm_residual_is_f16_sum():
    h = synthetic.activations(4, 256, seed=11)
    r = synthetic.activations(4, 256, seed=12)
    w = synthetic.norm_weight(256)
    r_new, _ = norm.fused_add_rms_norm(h, r, w, 1e-6)
    ref = (h.numpy().astype(np.float32) + r.numpy().astype(np.float32)).astype(np.float16)
    assert np.array_equal(r_new.numpy(), ref)


def test_norm_vs_f64_loop_and_library():
    h = synthetic.activations(3, 128, seed=13)
    r = synthetic.activations(3, 128, seed=14)
    w = synthetic.norm_weight(128)
    r_new, normed = norm.fused_add_rms_norm(h, r, w, 1e-6)
    # statistics from the unrounded sum, scaling of the stored (rounded) sum
    added = h.double().numpy() + r.double().numpy()
    ref64 = norm.rms_norm_f64(r_new.float().numpy(), w.float().numpy(), 1e-6, stat=added)
    assert np.allclose(normed.numpy(), ref64, rtol=1e-5, atol=1e-6)
    # with a zero residual the sum is exact, so the library routine applies directly
    _, n0 = norm.fused_add_rms_norm(h, torch.zeros_like(r), w, 1e-6)
    lib = torch.nn.functional.rms_norm(h.float(), (128,), w.float(), eps=1e-6)
    assert torch.allclose(n0, lib, rtol=1e-5, atol=1e-6)
    # the reference test's formula (unrounded sum in pass 2) agrees within fp16 rounding
    _, tf = norm.fused_add_rms_norm_testformula(h, r, w, 1e-6)
    assert torch.allclose(normed, tf, rtol=2e-3, atol=2e-3)


def test_norm_scale_invariance():
    h = synthetic.activations(2, 256, seed=15)
    z = torch.zeros_like(h)
    w = synthetic.norm_weight(256)
    _, n1 = norm.fused_add_rms_norm(h, z, w, 0.0)
    _, n2 = norm.fused_add_rms_norm((h.float() * 4).half(), z, w, 0.0)
    assert torch.allclose(n1, n2, rtol=1e-6, atol=1e-6)


def test_norm_quant_codes_bruteforce():
    h = synthetic.activations(2, 64, seed=16)
    r = synthetic.activations(2, 64, seed=17)
    w = synthetic.norm_weight(64)
    _, q, s, nlp = norm.fused_add_rms_norm_quant(h, r, w, 1e-6)
    v = (nlp.float().numpy() / s.numpy()[:, None]).astype(np.float32)
    v = np.clip(v, -448, 448).astype(np.float32)
    assert np.array_equal(q.numpy().reshape(-1), fp8.encode_e4m3_bruteforce(v.reshape(-1)))


# ---------------------------------------------------------------- gelu / rope
def test_gelu_matches_torch_and_limits():
    u = np.linspace(-8, 8, 1001)
    ref = torch.nn.functional.gelu(torch.from_numpy(u), approximate="tanh").numpy()
    assert np.allclose(act.gelu_tanh_f64(u), ref, rtol=1e-12, atol=1e-12)
    assert act.gelu_tanh_f64(0.0) == 0.0
    assert abs(act.gelu_tanh_f64(20.0) - 20.0) < 1e-12 and abs(act.gelu_tanh_f64(-20.0)) < 1e-12
    x = np.random.default_rng(0).standard_normal((3, 16))
    out = act.gelu_and_mul(x)
    assert np.allclose(out, act.gelu_tanh_f64(x[:, :8]) * x[:, 8:])
    # the second half multiplies, the first half is activated (swap breaks it)
    assert not np.allclose(out, act.gelu_tanh_f64(x[:, 8:]) * x[:, :8])


def _rope_complex(v, pos, theta, neox):
    T, H, hd = v.shape
    half = hd // 2
    inv = theta ** (-np.arange(half) * 2.0 / hd)
    rot = np.exp(1j * np.asarray(pos, dtype=np.float64)[:, None, None] * inv[None, None, :])
    if neox:
        z = (v[..., :half] + 1j * v[..., half:]) * rot
        return np.concatenate([z.real, z.imag], axis=-1)
    z = (v[..., 0::2] + 1j * v[..., 1::2]) * rot
    out = np.empty_like(v)
    out[..., 0::2], out[..., 1::2] = z.real, z.imag
    return out


@pytest.mark.parametrize("neox", [True, False])
def test_rope_vs_complex_rotation(neox):
    rng = np.random.default_rng(1)
    v = rng.standard_normal((4, 3, 64))
    pos = [0, 1, 77, 8191]
    got = act.rope_f64(v, pos, 10000.0, neox)
    assert np.allclose(got, _rope_complex(v, pos, 10000.0, neox), atol=1e-12)
    assert np.allclose(got[0], v[0])                     # position 0 is the identity
    if neox:
        n = lambda a: a[..., :32] ** 2 + a[..., 32:] ** 2
    else:
        n = lambda a: a[..., 0::2] ** 2 + a[..., 1::2] ** 2
    assert np.allclose(n(got), n(v))                     # each pair keeps its norm


def test_rope_relative_position():
    # q(p+d) . k(p) depends only on d
    rng = np.random.default_rng(2)
    q = rng.standard_normal((1, 1, 32)).repeat(3, 0)
    k = rng.standard_normal((1, 1, 32)).repeat(3, 0)
    qs = act.rope_f64(q, [10, 110, 5010], 10000.0, True)
    ks = act.rope_f64(k, [3, 103, 5003], 10000.0, True)
    dots = (qs * ks).sum(-1).ravel()
    assert np.allclose(dots, dots[0], rtol=1e-9)


def test_head_norm_vs_library():
    rng = np.random.default_rng(3)
    v = rng.standard_normal((2, 4, 64))
    w = 1 + 0.1 * rng.standard_normal(64)
    lib = torch.nn.functional.rms_norm(torch.from_numpy(v), (64,), torch.from_numpy(w), eps=1e-6).numpy()
    assert np.allclose(act.head_rms_norm_f64(v, w, 1e-6), lib, rtol=1e-10)


def test_qk_norm_rope_composition():
    rng = np.random.default_rng(4)
    T, nq, nk, hd = 2, 2, 1, 32
    q = rng.standard_normal((T, nq * hd)).astype(np.float16).astype(np.float64)
    k = rng.standard_normal((T, nk * hd)).astype(np.float16).astype(np.float64)
    w = np.ones(hd)
    qo, ko = act.qk_norm_rope(q, k, w, w, [5, 9], 1e-6, 10000.0, True, hd)
    # rotation preserves the per-head norm: sqrt(hd) after RMSNorm with w = 1
    for o, n in ((qo, nq), (ko, nk)):
        norms = np.linalg.norm(o.reshape(T, n, hd), axis=-1)
        assert np.allclose(norms, math.sqrt(hd), rtol=2e-3)
