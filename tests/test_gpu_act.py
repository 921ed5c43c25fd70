"""GPU parity of gelu_and_mul and QK-norm + RoPE against float64 closed forms."""

import sys

import numpy as np
import pytest
import torch

from conftest import assert_close_fp
from esimd_learning_amd import synthetic
from oracle import act as oact

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("T,d", [(4, 24576), (1, 14336), (64, 4096), (3, 100), (7, 8)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_gelu_and_mul(ops, dev, T, d, dtype):
    _say(f"gelu_and_mul T={T} d={d} {dtype}")
    x = synthetic.activations(T, 2 * d, seed=T + d, dtype=dtype, std=2.0)
    out = torch.zeros(T, d, dtype=dtype, device=dev)
    ops.esimd_gelu_and_mul(out, x.to(dev))
    torch.cuda.synchronize()
    ref = oact.gelu_and_mul(x.float().numpy())
    assert_close_fp(out.cpu(), torch.from_numpy(ref), f"gelu T={T} d={d}")


@pytest.mark.parametrize("d", [8, 12])
def test_gelu_and_mul_many_rows(ops, dev, d):
    """More rows than the grid's y extent (65535): workgroup rows walk the
    tokens with that stride (vector and element-wise forms)."""
    T = 65535 + 70
    _say(f"gelu_and_mul T={T} d={d}")
    x = synthetic.activations(T, 2 * d, seed=d, dtype=torch.float16, std=2.0)
    out = torch.zeros(T, d, dtype=torch.float16, device=dev)
    ops.esimd_gelu_and_mul(out, x.to(dev))
    torch.cuda.synchronize()
    assert_close_fp(out.cpu(), torch.from_numpy(oact.gelu_and_mul(x.float().numpy())), f"gelu T={T} d={d}")


def test_gelu_and_mul_strided_rows(ops, dev):
    # input rows are a view into a wider buffer (e.g. a fused gate/up output)
    T, d = 4, 512
    buf = synthetic.activations(T, 3 * d, seed=5)
    x = buf[:, : 2 * d]
    out = torch.zeros(T, d, dtype=torch.float16, device=dev)
    ops.esimd_gelu_and_mul(out, buf.to(dev)[:, : 2 * d])
    torch.cuda.synchronize()
    assert_close_fp(out.cpu(), torch.from_numpy(oact.gelu_and_mul(x.float().numpy())), "strided")


def _qkv(T, nq, nk, hd, dtype, seed):
    return synthetic.activations(T, (nq + 2 * nk) * hd, seed=seed, dtype=dtype)


@pytest.mark.parametrize("T,nq,nk,hd", [(4, 16, 16, 256), (1, 32, 8, 128), (9, 8, 2, 64), (2, 2, 1, 96),
                                        (3, 4, 2, 512), (5, 8, 8, 32), (70, 16, 16, 256), (65, 3, 1, 128)])
@pytest.mark.parametrize("neox", [True, False])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_qk_norm_rope(ops, dev, T, nq, nk, hd, neox, dtype):
    _say(f"qk_norm_rope T={T} nq={nq} nk={nk} hd={hd} neox={neox} {dtype}")
    qkv = _qkv(T, nq, nk, hd, dtype, seed=T + nq + hd)
    qw = synthetic.norm_weight(hd, seed=1, dtype=dtype)
    kw = synthetic.norm_weight(hd, seed=2, dtype=dtype)
    pos = synthetic.positions(T, seed=T)
    d = qkv.to(dev)
    q = d[:, : nq * hd]
    k = d[:, nq * hd:(nq + nk) * hd]
    ops.esimd_qk_norm_rope(q, k, qw.to(dev), kw.to(dev), pos.to(dev), 1e-6, 10000.0, neox)
    torch.cuda.synchronize()
    out = d.cpu()
    qo, ko = oact.qk_norm_rope(qkv[:, : nq * hd].float().numpy(), qkv[:, nq * hd:(nq + nk) * hd].float().numpy(),
                               qw.float().numpy(), kw.float().numpy(), pos.numpy(), 1e-6, 10000.0, neox, hd)
    assert_close_fp(out[:, : nq * hd], torch.from_numpy(qo), "q")
    assert_close_fp(out[:, nq * hd:(nq + nk) * hd], torch.from_numpy(ko), "k")
    # the v slice is untouched
    assert torch.equal(out[:, (nq + nk) * hd:], qkv[:, (nq + nk) * hd:])


def test_qk_norm_rope_3d_views(ops, dev):
    T, nq, nk, hd = 3, 4, 2, 128
    qkv = _qkv(T, nq, nk, hd, torch.float16, seed=3)
    qw, kw = synthetic.norm_weight(hd, 1), synthetic.norm_weight(hd, 2)
    pos = torch.tensor([0, 4095, 8191])
    d = qkv.to(dev)
    q = d[:, : nq * hd].view(T, nq, hd)
    k = d[:, nq * hd:(nq + nk) * hd].view(T, nk, hd)
    ops.esimd_qk_norm_rope(q, k, qw.to(dev), kw.to(dev), pos.to(dev), 1e-6, 10000.0, True)
    torch.cuda.synchronize()
    qo, ko = oact.qk_norm_rope(qkv[:, : nq * hd].float().numpy(), qkv[:, nq * hd:(nq + nk) * hd].float().numpy(),
                               qw.float().numpy(), kw.float().numpy(), pos.numpy(), 1e-6, 10000.0, True, hd)
    assert_close_fp(d.cpu()[:, : nq * hd], torch.from_numpy(qo), "q3d")
    assert_close_fp(d.cpu()[:, nq * hd:(nq + nk) * hd], torch.from_numpy(ko), "k3d")


@pytest.mark.parametrize("neox", [True, False])
def test_qk_norm_rope_unaligned_rows(ops, dev, neox):
    """Row strides that are not a multiple of 8 elements take the element-wise
    kernel (the 16-byte form needs aligned row starts)."""
    T, nq, nk, hd = 5, 4, 2, 128
    width = (nq + 2 * nk) * hd + 4
    _say(f"qk_norm_rope unaligned rows neox={neox}")
    qkv = synthetic.activations(T, width, seed=17, dtype=torch.float16)
    qw, kw = synthetic.norm_weight(hd, 1), synthetic.norm_weight(hd, 2)
    pos = synthetic.positions(T, seed=4)
    d = qkv.to(dev)
    q = d[:, : nq * hd]
    k = d[:, nq * hd:(nq + nk) * hd]
    ops.esimd_qk_norm_rope(q, k, qw.to(dev), kw.to(dev), pos.to(dev), 1e-6, 10000.0, neox)
    torch.cuda.synchronize()
    qo, ko = oact.qk_norm_rope(qkv[:, : nq * hd].float().numpy(), qkv[:, nq * hd:(nq + nk) * hd].float().numpy(),
                               qw.float().numpy(), kw.float().numpy(), pos.numpy(), 1e-6, 10000.0, neox, hd)
    out = d.cpu()
    assert_close_fp(out[:, : nq * hd], torch.from_numpy(qo), "q unaligned")
    assert_close_fp(out[:, nq * hd:(nq + nk) * hd], torch.from_numpy(ko), "k unaligned")
    assert torch.equal(out[:, (nq + nk) * hd:], qkv[:, (nq + nk) * hd:])
