"""Pins of the fp8 codec oracle (CPU).

The decode is checked against hand-derived values of the OCP e4m3fn / e5m2
formats and against torch's library decode of all 256 codes; the encoder
against an independent brute-force nearest-code search and against torch's
library encode, over every fp16 value, every midpoint between adjacent
codes, and random fp32 values.
"""

import numpy as np
import torch

from oracle import fp8


def test_decode_known_values():
    t = fp8.E4M3_TABLE
    assert t[0x00] == 0.0 and np.signbit(t[0x80])
    assert t[0x01] == 2.0 ** -9          # smallest subnormal
    assert t[0x07] == 7 * 2.0 ** -9      # largest subnormal
    assert t[0x08] == 2.0 ** -6          # smallest normal
    assert t[0x38] == 1.0
    assert t[0x7E] == 448.0 and t[0xFE] == -448.0
    assert np.isnan(t[0x7F]) and np.isnan(t[0xFF])
    assert np.isnan(t).sum() == 2
    e5 = fp8.E5M2_TABLE
    assert e5[0x7B] == 57344.0 and np.isinf(e5[0x7C]) and np.isnan(e5[0x7D])
    assert e5[0x01] == 2.0 ** -16 and e5[0x3C] == 1.0


def test_decode_matches_torch_all_codes():
    codes = torch.arange(256, dtype=torch.uint8)
    for table, dt in ((fp8.E4M3_TABLE, torch.float8_e4m3fn), (fp8.E5M2_TABLE, torch.float8_e5m2)):
        ref = codes.view(dt).float().numpy()
        same = (ref == table) | (np.isnan(ref) & np.isnan(table))
        assert same.all()
        # bit patterns too (signed zeros)
        fin = ~np.isnan(ref)
        assert (ref[fin].view(np.uint32) == table[fin].view(np.uint32)).all()


def _probe_values():
    rng = np.random.default_rng(0)
    all_f16 = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    fin = fp8.E4M3_TABLE[np.isfinite(fp8.E4M3_TABLE)]
    pos = np.unique(np.abs(fin)).astype(np.float64)
    mids = ((pos[1:] + pos[:-1]) / 2).astype(np.float32)      # exact ties
    near = np.concatenate([np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(0))])
    extra = np.array([464.0, 470.0, 479.9, 480.0, 1e9, np.inf, -np.inf, np.nan, 2.0 ** -10,
                      3 * 2.0 ** -11, 2.0 ** -20], dtype=np.float32)
    rnd = (rng.standard_normal(20000) * rng.choice([1e-3, 1e-1, 1, 10, 300], 20000)).astype(np.float32)
    v = np.concatenate([all_f16, mids, near, extra, rnd])
    return np.concatenate([v, -v]).astype(np.float32)


def _same_codes(a, b):
    # all NaN encodings are the 0x7F/0xFF pattern; compare exactly
    return np.array_equal(a, b)


def test_encode_matches_torch():
    v = _probe_values()
    ours = fp8.encode_e4m3(v)
    ref = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    # torch may produce either NaN sign for NaN inputs; compare on non-NaN inputs
    ok = ~np.isnan(v)
    assert _same_codes(ours[ok], ref[ok])
    assert (ours[~ok] & 0x7F == 0x7F).all()


def test_encode_matches_bruteforce():
    v = _probe_values()
    rng = np.random.default_rng(1)
    sub = np.concatenate([v[65536:], rng.choice(v[:65536], 4000)])   # all ties + a sample of fp16
    sub = sub[~np.isnan(sub)]
    assert _same_codes(fp8.encode_e4m3(sub), fp8.encode_e4m3_bruteforce(sub))


def test_tie_detector():
    fin = fp8.E4M3_TABLE[np.isfinite(fp8.E4M3_TABLE)]
    pos = np.unique(np.abs(fin)).astype(np.float64)
    mids = ((pos[1:] + pos[:-1]) / 2).astype(np.float32)
    assert fp8.e4m3_is_tie(mids).all()
    assert not fp8.e4m3_is_tie(pos.astype(np.float32)).any()
    assert not fp8.e4m3_is_tie(np.nextafter(mids, np.float32(np.inf))).any()


def test_round_trip_codes():
    codes = np.arange(256, dtype=np.uint8)
    vals = fp8.E4M3_TABLE
    fin = np.isfinite(vals)
    back = fp8.encode_e4m3(vals[fin])
    # -0 and +0 keep their sign bit
    assert np.array_equal(back, codes[fin])


def test_per_token_quant_properties():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((16, 512)).astype(np.float16).astype(np.float32)
    x[3] = 0.0                                   # all-zero row -> floor scale, zero codes
    q, s = fp8.per_token_quant(x)
    assert s.dtype == np.float32 and s[3] == fp8.MIN_SCALE and (q[3] & 0x7F == 0).all()
    amax = np.abs(x).max(axis=1)
    nz = amax > 0
    assert np.array_equal(s[nz], (amax[nz] / np.float32(448)).astype(np.float32))
    deq = fp8.decode_e4m3(q) * s[:, None]
    # the max-magnitude element of each row maps to +-448 exactly
    assert np.all(np.abs(fp8.decode_e4m3(q[nz])).max(axis=1) == 448.0)
    # relative error of e4m3 RNE is at most 2^-4 for normal codes
    big = np.abs(x) > 2.0 ** -6 * s[:, None] * 2
    assert np.all(np.abs(deq - x)[big] <= np.abs(x)[big] * 2.0 ** -4 + 1e-12)


def test_weight_recipe_matches_torch_recipe():
    from esimd_learning_amd import synthetic
    W8, s = synthetic.weight_fp8(64, 256, seed=5)
    Wf = (torch.randn(64, 256, generator=torch.Generator().manual_seed(5)) * 0.02).numpy()
    q, s2 = fp8.quantize_weight_per_row(Wf)
    assert np.array_equal(s.numpy(), s2)
    assert np.array_equal(W8.view(torch.uint8).numpy(), q)
