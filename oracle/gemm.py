"""a8w8 fp8 GEMM (per-token A scale, per-channel B scale) -- CPU restatement.

Test infrastructure only (see ``oracle/__init__.py``).

The reference has no a8w8 op.  Definition, fp32 accumulate:
    Y[m, n] = f16(sa[m] * sb[n] * sum_k dq(A[m, k]) * dq(B[n, k]))
computed here as the fp32 dequantise-then-matmul of the codes, the same
style as the reference's GEMM oracle (``tests/test_gemm_fp8.py:35-36``).

Pins (tests/test_oracle_ops.py): float64 brute force on tiny shapes;
a8w8 with sa == 1 equals the fp16-activation GEMM oracle of
``oracle.gemv`` when A's codes are fed as fp16 activations; bilinearity in
(sa, sb).
"""

import torch


def _f32(codes):
    if codes.dtype == torch.uint8:
        codes = codes.view(torch.float8_e4m3fn)
    return codes.to(torch.float16).float()


def gemm_a8w8(a8, sa, b8, sb):
    """a8 [M,K], b8 [N,K] e4m3; sa [M], sb [N] fp32 -> fp32 [M,N]."""
    acc = _f32(a8.cpu()) @ _f32(b8.cpu()).T
    return acc * sa.cpu().float().reshape(-1, 1) * sb.cpu().float().reshape(1, -1)
