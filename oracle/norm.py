"""Fused residual-add + RMSNorm (+ per-token fp8 quant) -- CPU restatement.

Test infrastructure only (see ``oracle/__init__.py``).

Reference algorithm (``csrc/xpu/esimd_kernels/fused_add_rms_norm_batched.h``):
  pass 1 (:30-50): r' = f16(f32(h) + f32(r)) is stored; sum_sq accumulates the
                   *unrounded* fp32 sum (h + r)^2;
  (:52-53)         inv = rsqrt(sum_sq / K + eps);
  pass 2 (:55-62): h = f16(f32(r') * inv * f32(w)), reading the stored r'.
The weight is Gemma-style, already shifted to w + 1 by the caller
(``python/custom_esimd_kernels_vllm/ops.py:44``).
The reference test's formula (``tests/test_fused_add_rms_norm_batched_fp8.py:7-27``)
uses the unrounded sum in pass 2; ``fused_add_rms_norm_testformula`` restates
it and the oracle tests check both agree within the op tolerance.

The fp8 extension (the reference has no op for it): quantise the fp16-rounded
normed row per token with ``oracle.fp8.per_token_quant``.

Pins (tests/test_oracle_ops.py): r' is f16(h+r) elementwise (checked
against numpy float16 addition), the normed output against a float64 loop and
against ``torch.nn.functional.rms_norm``, scale invariance of the normed
output, and the quant codes against ``oracle.fp8`` brute force.
"""

import numpy as np
import torch

from . import fp8


def fused_add_rms_norm(h, r, w, eps):
    """Returns (residual_out fp16/bf16 [T,H], normed fp32 [T,H])."""
    hf, rf = h.cpu().float(), r.cpu().float()
    added = hf + rf
    r_new = added.to(h.dtype)
    ss = (added * added).sum(-1, keepdim=True)
    inv = torch.rsqrt(ss / h.shape[-1] + eps)
    normed = r_new.float() * inv * w.cpu().float()
    return r_new, normed


def fused_add_rms_norm_testformula(h, r, w, eps):
    """The reference test's formula (unrounded residual in pass 2)."""
    hf, rf = h.cpu().float(), r.cpu().float()
    updated = hf + rf
    var = updated.pow(2).mean(dim=-1, keepdim=True)
    return updated, updated * torch.rsqrt(var + eps) * w.cpu().float()


def fused_add_rms_norm_quant(h, r, w, eps):
    """Returns (residual_out, codes uint8 [T,H], scale fp32 [T], normed_f16)."""
    r_new, normed = fused_add_rms_norm(h, r, w, eps)
    normed_lp = normed.to(h.dtype)
    q, s = fp8.per_token_quant(normed_lp.float().numpy())
    return r_new, torch.from_numpy(q), torch.from_numpy(s), normed_lp


def per_token_quant(x):
    """x [T,H] fp16/bf16 -> (codes uint8 [T,H], scale fp32 [T]), per-token e4m3."""
    q, s = fp8.per_token_quant(x.cpu().float().numpy())
    return torch.from_numpy(q), torch.from_numpy(s)


def rms_norm_f64(v, w, eps, stat=None):
    """float64 loop restatement for tiny shapes (pin only).

    The mean square comes from ``stat`` when given (the kernel takes it from
    the unrounded h + r while scaling the rounded residual), else from v.
    """
    v = np.asarray(v, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    st = v if stat is None else np.asarray(stat, dtype=np.float64)
    out = np.empty_like(v)
    for t in range(v.shape[0]):
        ms = sum(float(a) * float(a) for a in st[t]) / v.shape[1]
        inv = 1.0 / np.sqrt(ms + eps)
        out[t] = v[t] * inv * w
    return out
