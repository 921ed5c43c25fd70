"""One Gemma-style decoder-layer decode step composed from the oracle ops.

Test infrastructure only (see ``oracle/__init__.py``).

Composition (no single reference function -- the steps
are the reference's ops plus the new ops, each rounded to the activation
dtype between steps exactly as the device pipeline hands fp16 tensors on):

  h1, r1 = add_rmsnorm(hidden, residual, w_in)            (a5)
  qkv    = gemv(h1, Wqkv, sqkv)                            (a1)
  q, k   = qk_norm_rope(qkv[:, :nq*hd], qkv[:, nq*hd:(nq+nk)*hd])  (a11)
  o      = gemv(q, Wo, so)   # q stands in for the attention output
  h2, r2 = add_rmsnorm(o, r1, w_post)                      (a5)
  gu     = gemv(h2, Wgu, sgu)                              (a1)
  a      = gelu_and_mul(gu)                                (a10)
  out    = gemv(a, Wd, sd)                                 (a1)

With act_fp8 the two add_rmsnorm -> gemv hand-offs go through the per-token
e4m3 quant (a6) and the a8w8 product (a9) instead.

Pins: each step is pinned in its own module; this file only composes them.
"""

import torch

from . import act, gemm, gemv, norm


def _norm_then_gemv(x, r, w, eps, W8, s, act_fp8):
    """add_rmsnorm then the projection; returns (residual_out, y fp32)."""
    if act_fp8:
        r_new, q, qs, _ = norm.fused_add_rms_norm_quant(x, r, w, eps)
        return r_new, gemm.gemm_a8w8(q, qs, W8.view(torch.uint8), s.float())
    r_new, h = norm.fused_add_rms_norm(x, r, w, eps)
    return r_new, gemv.gemv_fp8_pern(h.to(x.dtype), W8, s)


def decoder_step(p, hidden, residual, positions, act_fp8=False):
    """p: dict of CPU tensors (see esimd_learning_amd.synthetic.gemma_layer)."""
    dt = hidden.dtype
    hd, nq, nk = p["head_dim"], p["n_q"], p["n_kv"]
    r1, qkv = _norm_then_gemv(hidden, residual, p["w_in"], p["eps"], p["Wqkv"], p["sqkv"], act_fp8)
    qkv = qkv.to(dt)
    q = qkv[:, : nq * hd].float().numpy()
    k = qkv[:, nq * hd:(nq + nk) * hd].float().numpy()
    qo, ko = act.qk_norm_rope(q, k, p["qw"].float().numpy(), p["kw"].float().numpy(),
                              positions.numpy(), p["eps"], p["theta"], True, hd)
    qkv[:, : nq * hd] = torch.from_numpy(qo).to(dt)
    qkv[:, nq * hd:(nq + nk) * hd] = torch.from_numpy(ko).to(dt)
    o = gemv.gemv_fp8_pern(qkv[:, : nq * hd], p["Wo"], p["so"]).to(dt)
    r2, gu = _norm_then_gemv(o, r1, p["w_post"], p["eps"], p["Wgu"], p["sgu"], act_fp8)
    gu = gu.to(dt)
    a = torch.from_numpy(act.gelu_and_mul(gu.float().numpy())).to(dt)
    out = gemv.gemv_fp8_pern(a, p["Wd"], p["sd"])
    return out, r2, qkv
