"""GPU parity of the decode pipeline: fused add+RMSNorm+per-token fp8 quant,
then the fp8 x fp8 GEMV/GEMM to N = 6144 (the QKV projection).

Stage one's codes and scales are checked against the oracle (codes may
differ by one step only where the oracle's fp16-rounded normed value and the
kernel's differ at a rounding tie, which test_gpu_norm counts); stage two is
checked against the oracle's a8w8 product of the GPU's own codes and scales,
to the fp16 tolerance.  T <= 16 runs the weight-streaming GEMV kernels,
T = 32 and 64 the tiled fp8 MFMA GEMM.
"""

import sys

import numpy as np
import pytest
import torch

from conftest import assert_close_fp
from esimd_learning_amd import synthetic
from oracle import gemm as ogemm
from oracle import norm as onorm

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T", [1, 8, 32, 64])
@pytest.mark.parametrize("H", [4096, 5120])
def test_norm_quant_then_gemv(ops, dev, T, H):
    N = 6144
    print(f"pipeline T={T} H={H} N={N}", flush=True)
    sys.stdout.flush()
    h = synthetic.activations(T, H, seed=T + H)
    r = synthetic.activations(T, H, seed=T + H + 1)
    w = synthetic.norm_weight(H, seed=H)
    W8, sb = synthetic.weight_fp8(N, H, seed=H + 7)

    hd, rd, wd = h.to(dev), r.to(dev), w.to(dev)
    q = torch.empty(T, H, dtype=torch.float8_e4m3fn, device=dev)
    s = torch.empty(T, dtype=torch.float32, device=dev)
    ops.esimd_fused_add_rms_norm_quant_fp8(hd, rd, wd, 1e-6, q, s)
    y = torch.zeros(T, N, dtype=torch.float16, device=dev)
    ops.esimd_gemm_fp8_a8w8(q.view(torch.uint8), s, W8.view(torch.uint8).to(dev), sb.to(dev), y)
    torch.cuda.synchronize()

    r_ref, q_ref, s_ref, _ = onorm.fused_add_rms_norm_quant(h, r, w, 1e-6)
    assert torch.equal(rd.cpu(), r_ref)
    # scale within one fp16 rounding step of the oracle's; codes one step at
    # most where the normed value rounds differently (sum-of-squares order)
    assert np.allclose(s.cpu().numpy(), s_ref.numpy(), rtol=2.0 ** -10, atol=0)
    qg = q.view(torch.uint8).cpu()
    mag = lambda c: np.where(c & 0x80, -(c & 0x7F), c & 0x7F)   # monotone code order  # noqa: E731
    diff = np.abs(mag(qg.numpy().astype(np.int64)) - mag(q_ref.numpy().astype(np.int64)))
    assert diff.max() <= 1 and int((diff > 0).sum()) <= max(4, T * H // 1000)

    ref = ogemm.gemm_a8w8(qg, s.cpu(), W8.view(torch.uint8), sb)
    assert_close_fp(y.cpu(), ref, f"pipeline T={T} H={H}")
