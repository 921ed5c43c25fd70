"""Seeded synthetic inputs for the benchmark configurations.

Everything is drawn on the CPU with ``torch.Generator().manual_seed(seed)``
so any machine with the same torch build reproduces the tensors bit for bit;
callers move them to the GPU.

Weight recipe (per output row n):
    W ~ N(0, 0.02) fp32;  s[n] = amax_k |W[n, k]| / 448 (fp32);
    W8 = e4m3(clamp(W / s[:, None], -448, 448))        (RNE)
Activations are fp16 N(0, 1); RMSNorm weights 1 + N(0, 0.1) in fp16 (already
in the Gemma w + 1 convention); eps 1e-6; RoPE theta 10000 and positions drawn
from [0, 8192).
"""

import torch

E4M3_MAX = 448.0
E5M2_MAX = 57344.0


def gen(seed):
    return torch.Generator().manual_seed(seed)


def quantize_rows(W, fmt=torch.float8_e4m3fn):
    """Per-row fp8 quantisation of an fp32 [N, K] matrix -> (W8, s fp32 [N])."""
    fmax = E5M2_MAX if fmt == torch.float8_e5m2 else E4M3_MAX
    s = W.abs().amax(dim=1) / fmax
    W8 = (W / s[:, None]).clamp(-fmax, fmax).to(fmt)
    return W8, s.float()


def weight_fp8(N, K, seed=0, std=0.02, fmt=torch.float8_e4m3fn):
    W = torch.randn(N, K, generator=gen(seed)) * std
    return quantize_rows(W, fmt)


def activations(M, K, seed=1, dtype=torch.float16, std=1.0):
    return (torch.randn(M, K, generator=gen(seed)) * std).to(dtype)


def norm_weight(H, seed=2, dtype=torch.float16):
    return (1.0 + 0.1 * torch.randn(H, generator=gen(seed))).to(dtype)


def positions(T, seed=3, max_pos=8192):
    return torch.randint(0, max_pos, (T,), generator=gen(seed), dtype=torch.int64)


def gemma_layer(seed=10, hidden=3072, n_q=16, n_kv=16, head_dim=256, mlp=24576,
                fmt=torch.float8_e4m3fn):
    """Random-init fp8 weights of one Gemma-style decoder layer (config 5)."""
    qkv_n = (n_q + 2 * n_kv) * head_dim
    p = {"hidden": hidden, "n_q": n_q, "n_kv": n_kv, "head_dim": head_dim, "mlp": mlp,
         "eps": 1e-6, "theta": 10000.0}
    p["Wqkv"], p["sqkv"] = weight_fp8(qkv_n, hidden, seed, fmt=fmt)
    p["Wo"], p["so"] = weight_fp8(hidden, n_q * head_dim, seed + 1, fmt=fmt)
    p["Wgu"], p["sgu"] = weight_fp8(2 * mlp, hidden, seed + 2, fmt=fmt)
    p["Wd"], p["sd"] = weight_fp8(hidden, mlp, seed + 3, fmt=fmt)
    p["w_in"] = norm_weight(hidden, seed + 4)
    p["w_post"] = norm_weight(hidden, seed + 5)
    p["qw"] = norm_weight(head_dim, seed + 6)
    p["kw"] = norm_weight(head_dim, seed + 7)
    return p


def layer_weight_bytes(p):
    return sum(p[k].numel() for k in ("Wqkv", "Wo", "Wgu", "Wd"))
