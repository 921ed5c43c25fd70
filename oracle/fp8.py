"""OCP fp8 codec restated from the format definition (numpy, bit-exact).

Test infrastructure only (see ``oracle/__init__.py``).

The reference's own oracle decodes weights with torch's
``weight_fp8.to(torch.float16)`` (reference ``tests/test_gemv_fp8.py:31``,
``tests/test_gemm_fp8.py:35``), i.e. exact OCP e4m3fn / e5m2 decoding that
keeps subnormals.  Its kernels instead flush e4m3 subnormals to zero and map
the NaN code to +-480 (reference ``csrc/xpu/esimd_kernels/fp8_GEMV_v2.h:15-38``);
the parity target is the oracle, so this module follows the exact decode.

Quantisation (values -> codes) follows torch's CPU ``.to(float8_e4m3fn)``:
round-to-nearest-even on the e4m3 grid, *not* saturating (|v| > 464 -> NaN,
|v| == 464 ties to 448).  Callers that quantise clamp to +-448 first, as the
quantisation recipe does.

Pins (tests/test_oracle_fp8.py):
  * ``decode_e4m3``/``decode_e5m2`` == torch's library decode for all 256
    codes, and hand-derived values (0x01 = 2^-9, 0x08 = 2^-6, 0x38 = 1,
    0x7E = 448, 0x7F = NaN, e5m2 0x7B = 57344, 0x7C = inf).
  * ``encode_e4m3`` == an independent brute-force nearest-value search over
    the 256-code table (ties -> even code) on every fp16 value, every
    midpoint between adjacent codes and random fp32 values, and == torch's
    library encode on the same values.
"""

import numpy as np

E4M3_MAX = 448.0
# Smallest per-token scale: keeps x / s finite when a row is all zeros.
MIN_SCALE = np.float32(1.0 / (448.0 * 512.0))


def decode_e4m3(codes):
    """e4m3fn code bytes -> float32 values (exact; 0x7F/0xFF -> NaN)."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    s = np.where((c >> 7) & 1, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    mag = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e.astype(np.float64) - 7.0))
    mag = np.where((e == 15) & (m == 7), np.nan, mag)
    return (s * mag).astype(np.float32)


def decode_e5m2(codes):
    """e5m2 code bytes -> float32 values (exact; e=31 -> inf/NaN)."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    s = np.where((c >> 7) & 1, -1.0, 1.0)
    e = (c >> 2) & 0x1F
    m = c & 0x3
    mag = np.where(e == 0, m * 2.0 ** -16, (1.0 + m / 4.0) * np.exp2(e.astype(np.float64) - 15.0))
    mag = np.where(e == 31, np.where(m == 0, np.inf, np.nan), mag)
    return (s * mag).astype(np.float32)


E4M3_TABLE = decode_e4m3(np.arange(256, dtype=np.uint8))
E5M2_TABLE = decode_e5m2(np.arange(256, dtype=np.uint8))


def encode_e4m3(x):
    """float32 values -> e4m3fn codes, RNE, torch semantics (see module doc)."""
    x = np.asarray(x, dtype=np.float32)
    bits = x.view(np.uint32).astype(np.int64)
    sign = ((bits >> 31) & 1) << 7
    a = np.abs(x.astype(np.float64))
    finite = np.isfinite(a)
    a = np.where(finite, a, 0.0)

    # subnormal range |x| < 2^-6: units of 2^-9, RNE (np.rint ties to even)
    q_sub = np.rint(np.minimum(a, 1.0) * 512.0).astype(np.int64)   # 0..8; 8 == 2^-6 code
    # normal range: round the 23-bit mantissa to 3 bits, RNE
    abits = bits & 0x7FFFFFFF
    e = (abits >> 23) - 127
    m23 = abits & 0x7FFFFF
    q = m23 >> 20
    rem = m23 & 0xFFFFF
    up = (rem > 0x80000) | ((rem == 0x80000) & ((q & 1) == 1))
    q = q + up
    carry = q == 8
    q = np.where(carry, 0, q)
    e = e + carry
    code_n = ((e + 7) << 3) | q
    overflow = (e > 8) | ((e == 8) & (q == 7))
    code_n = np.where(overflow, 0x7F, code_n)

    normal = a >= 2.0 ** -6
    out = np.where(normal, code_n, q_sub)
    out = np.where(np.isnan(x) | np.isinf(x), 0x7F, out)
    return (out | sign).astype(np.uint8)


def e4m3_is_tie(x):
    """True where x lies exactly half-way between two adjacent e4m3 values."""
    x = np.asarray(x, dtype=np.float32)
    a = np.abs(x.astype(np.float64))
    sub_tie = (a < 2.0 ** -6) & (np.abs(a * 512.0 - np.floor(a * 512.0) - 0.5) == 0.0)
    m23 = x.view(np.uint32).astype(np.int64) & 0x7FFFFF
    norm_tie = (a >= 2.0 ** -6) & ((m23 & 0xFFFFF) == 0x80000)
    return sub_tie | norm_tie


def encode_e4m3_bruteforce(x):
    """Independent encoder: nearest finite code, ties to the even code.

    The virtual value 480 (code 0x7F, NaN in e4m3fn) is a candidate so that
    values nearer to 480 than to 448 overflow to NaN as torch does.
    """
    x = np.asarray(x, dtype=np.float32).reshape(-1)
    vals = E4M3_TABLE[:128].astype(np.float64).copy()
    vals[0x7F] = 480.0
    out = np.empty(x.shape, dtype=np.uint8)
    for i, v in enumerate(x.astype(np.float64)):
        if np.isnan(v):
            out[i] = 0x7F
            continue
        if np.isinf(v):
            out[i] = 0x7F | (0x80 if v < 0 else 0)
            continue
        d = np.abs(vals - abs(v))
        best = np.flatnonzero(d == d.min())
        c = int(best[0]) if len(best) == 1 else int(best[best % 2 == 0][0])
        out[i] = c | (0x80 if np.signbit(v) else 0)
    return out


def per_token_quant(xf):
    """Per-row e4m3 quantisation of float32 rows (the per-token activation quant).

    s_t = max(amax_t / 448, MIN_SCALE) in fp32,
    q   = e4m3(RNE(clamp(x / s_t, -448, 448))) with an IEEE fp32 divide.
    Returns (codes uint8 [T,H], scale float32 [T]).
    """
    xf = np.asarray(xf, dtype=np.float32)
    amax = np.max(np.abs(xf), axis=-1)
    s = np.maximum((amax / np.float32(E4M3_MAX)).astype(np.float32), MIN_SCALE)
    v = (xf / s[..., None]).astype(np.float32)
    v = np.clip(v, np.float32(-E4M3_MAX), np.float32(E4M3_MAX))
    return encode_e4m3(v), s.astype(np.float32)


def quantize_weight_per_row(wf):
    """Weight recipe: s[n] = amax_k|W[n,k]| / 448, codes = e4m3(clamp(W/s)).

    Same arithmetic as ``per_token_quant`` without the scale floor (weights
    drawn from N(0, 0.02) never have an all-zero row at the sizes used).
    """
    wf = np.asarray(wf, dtype=np.float32)
    amax = np.max(np.abs(wf), axis=-1)
    s = (amax / np.float32(E4M3_MAX)).astype(np.float32)
    v = np.clip((wf / s[:, None]).astype(np.float32), -E4M3_MAX, E4M3_MAX).astype(np.float32)
    return encode_e4m3(v), s
