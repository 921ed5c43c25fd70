"""Writes tests/golden/golden.npz: small seeded fixtures for the op pack.

The reference ships no golden vectors or known-answer tables for this path
(its tests compare against torch formulas on freshly drawn inputs), so the
fixtures here are generated from the seeded quantisation recipe
(esimd_learning_amd.synthetic) and the CPU oracle:

  e4m3_bits / e5m2_bits   float32 bit patterns of all 256 decoded codes
  gemv_*                  M=2, K=256, N=16 GEMV (fp32 per-channel scale)
  cfg1_*                  BASELINE config 1: x [1,4096] fp16 (seed 1),
                          W [4096,4096] recipe seed 0 (stored as its SHA-256,
                          16 MB is regenerated from the seed), s, y
  norm_*                  T=4, H=512 add+RMSNorm (+ quant)
  quant_*                 T=4, H=256 per-token quant incl. a zero row
  gelu_*, rope_*          small gelu_and_mul / QK-norm+RoPE cases (float64)
  a8w8_*                  M=8, K=256, N=32 a8w8 GEMM

Run:  python tests/golden/make_golden.py   (rewrites golden.npz)
"""

import hashlib
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from esimd_learning_amd import synthetic  # noqa: E402
from oracle import act, fp8, gemm, gemv, norm  # noqa: E402

OUT = Path(__file__).resolve().parent / "golden.npz"


def f16_bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def sha256(t):
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def cfg1():
    W8, s = synthetic.weight_fp8(4096, 4096, seed=0)
    x = synthetic.activations(1, 4096, seed=1)
    y = gemv.gemv_fp8_pern(x, W8, s)
    return W8, s, x, y


def build():
    d = {}
    tab = fp8.E4M3_TABLE.copy()
    d["e4m3_bits"] = tab.view(np.uint32)
    d["e5m2_bits"] = fp8.E5M2_TABLE.copy().view(np.uint32)

    W8, s = synthetic.weight_fp8(16, 256, seed=100)
    x = synthetic.activations(2, 256, seed=101)
    d["gemv_x"] = f16_bits(x)
    d["gemv_w"] = W8.view(torch.uint8).numpy()
    d["gemv_s"] = s.numpy()
    d["gemv_y"] = gemv.gemv_fp8_pern(x, W8, s).numpy()

    W8, s, x, y = cfg1()
    d["cfg1_x"] = f16_bits(x)
    d["cfg1_s"] = s.numpy()
    d["cfg1_y"] = y.numpy()
    d["cfg1_w_sha256"] = np.frombuffer(sha256(W8).encode(), dtype=np.uint8)

    h = synthetic.activations(4, 512, seed=200)
    r = synthetic.activations(4, 512, seed=201)
    w = synthetic.norm_weight(512, seed=202)
    r_new, q, qs, nlp = norm.fused_add_rms_norm_quant(h, r, w, 1e-6)
    _, normed = norm.fused_add_rms_norm(h, r, w, 1e-6)
    d.update(norm_h=f16_bits(h), norm_r=f16_bits(r), norm_w=f16_bits(w), norm_rout=f16_bits(r_new),
             norm_normed=normed.numpy(), norm_q=q.numpy(), norm_qs=qs.numpy())

    xq = synthetic.activations(4, 256, seed=300)
    xq[2] = 0
    q, qs = norm.per_token_quant(xq)
    d.update(quant_x=f16_bits(xq), quant_q=q.numpy(), quant_s=qs.numpy())

    xg = synthetic.activations(2, 128, seed=400, std=2.0)
    d.update(gelu_x=f16_bits(xg), gelu_out=act.gelu_and_mul(xg.float().numpy()))

    T, nq, nk, hd = 2, 2, 1, 64
    qkv = synthetic.activations(T, (nq + 2 * nk) * hd, seed=500)
    qw, kw = synthetic.norm_weight(hd, seed=501), synthetic.norm_weight(hd, seed=502)
    pos = torch.tensor([3, 8000])
    qo, ko = act.qk_norm_rope(qkv[:, :nq * hd].float().numpy(), qkv[:, nq * hd:(nq + nk) * hd].float().numpy(),
                              qw.float().numpy(), kw.float().numpy(), pos.numpy(), 1e-6, 10000.0, True, hd)
    d.update(rope_qkv=f16_bits(qkv), rope_qw=f16_bits(qw), rope_kw=f16_bits(kw), rope_pos=pos.numpy(),
             rope_q=qo, rope_k=ko)

    xa = synthetic.activations(8, 256, seed=600)
    qa, sa = norm.per_token_quant(xa)
    Wb, sb = synthetic.weight_fp8(32, 256, seed=601)
    d.update(a8w8_a=qa.numpy(), a8w8_sa=sa.numpy(), a8w8_b=Wb.view(torch.uint8).numpy(), a8w8_sb=sb.numpy(),
             a8w8_y=gemm.gemm_a8w8(qa, sa, Wb.view(torch.uint8), sb).numpy())
    return d


if __name__ == "__main__":
    np.savez_compressed(OUT, **build())
    print("wrote", OUT, OUT.stat().st_size, "bytes")
