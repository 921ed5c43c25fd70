"""fp8-weight GEMV / GEMM (fp16|bf16 activations) -- CPU restatement.

Test infrastructure only (see ``oracle/__init__.py``).

Follows the reference's own dequantise-then-matmul oracle in fp32:
  pern: ``ref = (x.float() @ W8.to(fp16).float().T) * scale.float()``
        (reference ``tests/test_gemv_fp8.py:31-32,58-59``)
  pert: ``... * scale_val`` (``tests/test_gemv_fp8.py:349-350``)
  gemm: ``(x.float() @ W8.to(fp16).float().T) * scale_val``
        (``tests/test_gemm_fp8.py:35-36``)
with the scale applied after the K reduction, as the kernels do
(``csrc/xpu/esimd_kernels/fp8_GEMV_v2.h:77,355``).  All M rows are computed;
the reference kernels compute row 0 only (``fp8_GEMV_v2.h:62-75``) and the
build treats all rows (a superset).

Pins (tests/test_oracle_ops.py): float64 brute-force triple loop on tiny
shapes; y is linear in the scale; zero weights give zero; pert == pern with a
uniform scale; GEMM at M=1 == GEMV; decoding through ``oracle.fp8`` tables
equals decoding through torch.
"""

import torch


def dequant_weight(w8):
    """fp8 [N,K] (float8_e4m3fn / float8_e5m2 / uint8 e4m3 bytes) -> fp32."""
    if w8.dtype == torch.uint8:
        w8 = w8.view(torch.float8_e4m3fn)
    return w8.to(torch.float16).float()


def gemv_fp8_pern(x, w8, scale):
    """x [M,K] fp16/bf16, w8 [N,K] fp8, scale [N] (any float dtype) -> fp32 [M,N]."""
    wf = dequant_weight(w8.cpu())
    return (x.cpu().float() @ wf.T) * scale.cpu().float().reshape(1, -1)


def gemv_fp8_pert(x, w8, scale):
    """Per-tensor scale variant: ``scale`` is a 0-d/1-element fp32 tensor."""
    wf = dequant_weight(w8.cpu())
    return (x.cpu().float() @ wf.T) * float(scale.reshape(-1)[0])


gemm_fp8_pert = gemv_fp8_pert


def gemv_bruteforce_f64(x, w8, scale):
    """Independent float64 triple loop, for tiny shapes only."""
    import numpy as np
    from .fp8 import E4M3_TABLE, E5M2_TABLE
    if w8.dtype == torch.float8_e5m2:
        table = E5M2_TABLE
    else:
        table = E4M3_TABLE
    codes = w8.cpu().view(torch.uint8).numpy()
    xs = x.cpu().float().numpy().astype(np.float64)
    sc = scale.cpu().float().reshape(-1).numpy().astype(np.float64)
    M, K = xs.shape
    N = codes.shape[0]
    y = np.zeros((M, N), dtype=np.float64)
    for m in range(M):
        for n in range(N):
            acc = 0.0
            for k in range(K):
                acc += xs[m, k] * float(table[codes[n, k]])
            y[m, n] = acc * (sc[n] if sc.size > 1 else sc[0])
    return y
