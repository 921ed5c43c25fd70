"""Committed fixtures (tests/golden/golden.npz, written by make_golden.py).

CPU: the fixtures are reproduced exactly by the input recipe and the oracle
(a regression pin for both, and a check that this torch build draws the same
seeded tensors), and the fp8 tables equal the format's hand-derived values.
GPU: the kernels reproduce the fixtures within tolerance (codes and residual
bit-exact).
"""

import hashlib
from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import assert_close_fp

G = np.load(Path(__file__).resolve().parent / "golden" / "golden.npz", allow_pickle=False)


def f16(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.float16)


def test_tables_fixture():
    from oracle import fp8
    assert np.array_equal(G["e4m3_bits"], fp8.E4M3_TABLE.view(np.uint32))
    t = G["e4m3_bits"].view(np.float32)
    assert t[0x38] == 1.0 and t[0x7E] == 448.0 and t[0x01] == 2.0 ** -9 and np.isnan(t[0x7F])


def test_fixtures_reproduced_by_oracle():
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_golden", Path(__file__).parent / "golden" / "make_golden.py")
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    d = mg.build()
    for k, v in d.items():
        assert np.array_equal(G[k], v, equal_nan=v.dtype.kind == "f"), k


def _cfg1_weight():
    from esimd_learning_amd import synthetic
    W8, s = synthetic.weight_fp8(4096, 4096, seed=0)
    sha = hashlib.sha256(W8.view(torch.uint8).numpy().tobytes()).hexdigest()
    assert sha == G["cfg1_w_sha256"].tobytes().decode(), "config-1 weights differ from the fixture's"
    return W8, s


def test_cfg1_weights_reproducible():
    _, s = _cfg1_weight()
    assert np.array_equal(s.numpy(), G["cfg1_s"])


@pytest.mark.gpu
def test_gpu_cfg1_gemv(ops, dev):
    W8, s = _cfg1_weight()
    x = f16(G["cfg1_x"])
    y = torch.zeros(1, 4096, dtype=torch.float16, device=dev)
    ops.esimd_gemv_fp8_pern(x.to(dev), W8.to(dev), s.to(dev), y, 4096, 4096)
    torch.cuda.synchronize()
    assert_close_fp(y.cpu(), torch.from_numpy(G["cfg1_y"]), "config 1")


@pytest.mark.gpu
def test_gpu_small_fixtures(ops, dev):
    # gemv
    y = torch.zeros(2, 16, dtype=torch.float16, device=dev)
    ops.esimd_gemv_fp8_pern(f16(G["gemv_x"]).to(dev), torch.from_numpy(G["gemv_w"]).view(torch.float8_e4m3fn).to(dev),
                            torch.from_numpy(G["gemv_s"]).to(dev), y, 16, 256)
    # norm
    h, r = f16(G["norm_h"]).to(dev), f16(G["norm_r"]).to(dev)
    ops.esimd_fused_add_rms_norm_batched(h, r, f16(G["norm_w"]).to(dev), 1e-6)
    # quant
    q = torch.empty(4, 256, dtype=torch.uint8, device=dev)
    qs = torch.empty(4, dtype=torch.float32, device=dev)
    ops.esimd_per_token_quant_fp8(f16(G["quant_x"]).to(dev), q, qs)
    # gelu
    go = torch.empty(2, 64, dtype=torch.float16, device=dev)
    ops.esimd_gelu_and_mul(go, f16(G["gelu_x"]).to(dev))
    # rope
    qkv = f16(G["rope_qkv"]).to(dev)
    ops.esimd_qk_norm_rope(qkv[:, :128], qkv[:, 128:192], f16(G["rope_qw"]).to(dev), f16(G["rope_kw"]).to(dev),
                           torch.from_numpy(G["rope_pos"]).to(dev), 1e-6, 10000.0, True)
    # a8w8
    ya = torch.empty(8, 32, dtype=torch.float16, device=dev)
    ops.esimd_gemm_fp8_a8w8(torch.from_numpy(G["a8w8_a"]).to(dev), torch.from_numpy(G["a8w8_sa"]).to(dev),
                            torch.from_numpy(G["a8w8_b"]).to(dev), torch.from_numpy(G["a8w8_sb"]).to(dev), ya)
    torch.cuda.synchronize()
    assert_close_fp(y.cpu(), torch.from_numpy(G["gemv_y"]), "gemv fixture")
    assert torch.equal(r.cpu(), f16(G["norm_rout"]))
    assert_close_fp(h.cpu(), torch.from_numpy(G["norm_normed"]), "norm fixture")
    assert np.array_equal(q.cpu().numpy(), G["quant_q"]) and np.array_equal(qs.cpu().numpy(), G["quant_s"])
    assert_close_fp(go.cpu(), torch.from_numpy(G["gelu_out"]), "gelu fixture")
    assert_close_fp(qkv.cpu()[:, :128], torch.from_numpy(G["rope_q"]), "rope q fixture")
    assert_close_fp(qkv.cpu()[:, 128:192], torch.from_numpy(G["rope_k"]), "rope k fixture")
    assert_close_fp(ya.cpu(), torch.from_numpy(G["a8w8_y"]), "a8w8 fixture")
