"""gelu_and_mul and QK-norm + RoPE -- closed forms in float64.

Test infrastructure only (see ``oracle/__init__.py``).

Neither op exists in the reference (a search of its .py/.h/.cc/.sycl files
for gelu, rope, rotary or qk_norm finds nothing), so these are the closed
forms that the op definitions name:

gelu_and_mul (vLLM ``gelu_tanh_and_mul(out, x)`` convention):
    out[t, i] = gelu_tanh(x[t, i]) * x[t, d + i]
    gelu_tanh(u) = 0.5 u (1 + tanh(sqrt(2/pi) (u + 0.044715 u^3)))

qk_norm_rope, per head of q and of k (head size hd):
    v  = f16(rmsnorm(v) * w)         (w Gemma-shifted by the caller, as in
                                      reference ``ops.py:44``)
    NeoX rotate-half:  theta_i = pos * base^(-2i/hd), i < hd/2,
        [a_i, b_i] = [v_i, v_{i+hd/2}] -> [a cos - b sin, b cos + a sin]
    GPT-J interleaved: the pair is (v_{2i}, v_{2i+1}).

Pins (tests/test_oracle_ops.py): gelu against
``torch.nn.functional.gelu(approximate='tanh')`` and its limits; RoPE
against complex multiplication by exp(i*theta) (a different formulation),
norm preservation per pair, identity at position 0, and relative-position
invariance of q.k; the head norm against ``torch.nn.functional.rms_norm``.
"""

import math

import numpy as np


def gelu_tanh_f64(u):
    u = np.asarray(u, dtype=np.float64)
    return 0.5 * u * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (u + 0.044715 * u ** 3)))


def gelu_and_mul(x):
    """x [T, 2d] -> float64 [T, d]."""
    x = np.asarray(x, dtype=np.float64)
    d = x.shape[-1] // 2
    return gelu_tanh_f64(x[..., :d]) * x[..., d:]


def rope_f64(v, pos, theta, is_neox):
    """v [T, heads, hd] float64, pos [T] ints -> rotated float64."""
    v = np.asarray(v, dtype=np.float64)
    T, H, hd = v.shape
    half = hd // 2
    inv_freq = float(theta) ** (-np.arange(half, dtype=np.float64) * 2.0 / hd)
    ang = np.asarray(pos, dtype=np.float64)[:, None] * inv_freq[None, :]   # [T, half]
    c = np.cos(ang)[:, None, :]
    s = np.sin(ang)[:, None, :]
    out = np.empty_like(v)
    if is_neox:
        a, b = v[..., :half], v[..., half:]
        out[..., :half] = a * c - b * s
        out[..., half:] = b * c + a * s
    else:
        a, b = v[..., 0::2], v[..., 1::2]
        out[..., 0::2] = a * c - b * s
        out[..., 1::2] = b * c + a * s
    return out


def head_rms_norm_f64(v, w, eps):
    """v [T, heads, hd], w [hd] -> float64 normed."""
    v = np.asarray(v, dtype=np.float64)
    ms = np.mean(v * v, axis=-1, keepdims=True)
    return v / np.sqrt(ms + eps) * np.asarray(w, dtype=np.float64)


def qk_norm_rope(q, k, qw, kw, pos, eps, theta, is_neox, hd):
    """q [T, nq*hd], k [T, nk*hd] (float arrays of the fp16 inputs).

    Returns float64 (q_out, k_out) with the fp16 rounding between norm and
    rotation that the op definition specifies.
    """
    outs = []
    for x, w in ((q, qw), (k, kw)):
        x = np.asarray(x, dtype=np.float64)
        T = x.shape[0]
        v = x.reshape(T, -1, hd)
        n = head_rms_norm_f64(v, w, eps).astype(np.float16).astype(np.float64)
        outs.append(rope_f64(n, pos, theta, is_neox).reshape(T, -1))
    return outs[0], outs[1]
