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

Pins: each step is pinned in its own module; this file only composes them.
"""

import torch

from . import act, gemv, norm


def decoder_step(p, hidden, residual, positions):
    """p: dict of CPU tensors (see esimd_learning_amd.synthetic.gemma_layer)."""
    dt = hidden.dtype
    hd, nq, nk = p["head_dim"], p["n_q"], p["n_kv"]
    r1, h1 = norm.fused_add_rms_norm(hidden, residual, p["w_in"], p["eps"])
    h1 = h1.to(dt)
    qkv = gemv.gemv_fp8_pern(h1, p["Wqkv"], p["sqkv"]).to(dt)
    q = qkv[:, : nq * hd].float().numpy()
    k = qkv[:, nq * hd:(nq + nk) * hd].float().numpy()
    qo, ko = act.qk_norm_rope(q, k, p["qw"].float().numpy(), p["kw"].float().numpy(),
                              positions.numpy(), p["eps"], p["theta"], True, hd)
    qkv[:, : nq * hd] = torch.from_numpy(qo).to(dt)
    qkv[:, nq * hd:(nq + nk) * hd] = torch.from_numpy(ko).to(dt)
    o = gemv.gemv_fp8_pern(qkv[:, : nq * hd], p["Wo"], p["so"]).to(dt)
    r2, h2 = norm.fused_add_rms_norm(o, r1, p["w_post"], p["eps"])
    h2 = h2.to(dt)
    gu = gemv.gemv_fp8_pern(h2, p["Wgu"], p["sgu"]).to(dt)
    a = torch.from_numpy(act.gelu_and_mul(gu.float().numpy())).to(dt)
    out = gemv.gemv_fp8_pern(a, p["Wd"], p["sd"])
    return out, r2, qkv
