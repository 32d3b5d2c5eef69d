"""Pins the oracle's formats: f16 conversions, the 6-bit scale unpack, dequantization and
Q8_K quantization. Reference: quant.rs:876-899, 1504-1660; q4k_gemv.rs:70-85;
quant_q8k.rs:84-121 (and its property test :342-362)."""
import json
import os

import numpy as np
import pytest

from oracle import ffi
from tests import refdata as R

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def test_f16_to_f32_exhaustive():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([ffi.lib.or_f16_to_f32(int(v)) for v in h], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_round_to_nearest_even():
    rng = np.random.default_rng(5)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32),
        (rng.standard_normal(20000) * 1e-5).astype(np.float32),   # subnormal halfs
        (rng.standard_normal(5000) * 3e4).astype(np.float32),     # near overflow
        np.array([0.0, -0.0, 65504.0, 65520.0, 65519.996, 2 ** -25, 2 ** -24, 3 * 2 ** -26, np.inf, -np.inf], np.float32),
    ])
    # midpoints between adjacent halfs round to even
    hs = np.arange(0, 0x7BFF, 7, dtype=np.uint16)
    a = hs.view(np.float16).astype(np.float64)
    b = (hs + 1).view(np.float16).astype(np.float64)
    vals = np.concatenate([vals, ((a + b) / 2).astype(np.float32)])
    want = vals.astype(np.float16).view(np.uint16)
    got = np.array([ffi.lib.or_f32_to_f16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, want)


def _q4k_block(d, dmin, scales, rule):
    qs = [eval(rule, {"i": i}) for i in range(128)]
    return np.frombuffer(int(d).to_bytes(2, "little") + int(dmin).to_bytes(2, "little") + bytes(scales) + bytes(qs), np.uint8).copy()


@pytest.mark.parametrize("case", range(2))
def test_q4k_known_answer_block(case):
    g = json.load(open(os.path.join(GOLD, "known_blocks.json")))["q4k"][case]
    blk = _q4k_block(g["d"], g["dmin"], g["scales"], g["qs_rule"])
    s = np.empty(8, np.uint8)
    m = np.empty(8, np.uint8)
    ffi.lib.or_unpack_q4k_scales(ffi.ptr(blk[4:16].copy()), ffi.ptr(s), ffi.ptr(m))
    assert s.tolist() == g["sc"] and m.tolist() == g["mn"]
    y = ffi.dequant_row(ffi.Q4K, blk, 256)
    for e, v in g["elements"].items():
        assert y[int(e)] == np.float32(v), (e, y[int(e)], v)


def test_q6k_known_answer_block():
    g = json.load(open(os.path.join(GOLD, "known_blocks.json")))["q6k"]
    ql = bytes((i * 37 + 11) & 255 for i in range(128))
    qh = bytes((i * 53 + 7) & 255 for i in range(64))
    sc = bytes((i * 9 - 70) & 255 for i in range(16))
    blk = np.frombuffer(ql + qh + sc + int(g["d"]).to_bytes(2, "little"), np.uint8).copy()
    y = ffi.dequant_row(ffi.Q6K, blk, 256)
    for e, v in g["elements"].items():
        assert y[int(e)] == np.float32(v), (e, y[int(e)], v)


def test_q5_0_and_q8_0_known_answer():
    g = json.load(open(os.path.join(GOLD, "known_blocks.json")))["q5_0"]
    blk = np.frombuffer(int(g["d"]).to_bytes(2, "little") + int(g["qh"]).to_bytes(4, "little") +
                        bytes((j * 17) & 255 for j in range(16)), np.uint8).copy()
    y = ffi.dequant_row(ffi.Q5_0, blk, 32)
    for e, v in g["elements"].items():
        assert y[int(e)] == np.float32(v)
    codes = np.arange(-128, 128, 8, dtype=np.int8)
    blk = np.frombuffer((0x3800).to_bytes(2, "little") + codes.tobytes(), np.uint8).copy()
    assert np.array_equal(ffi.dequant_row(ffi.Q8_0, blk, 32), codes.astype(np.float32) * 0.5)


def test_q8k_quantize_reference_property():
    """quant_q8k.rs:342-362 (same seed), plus the closed form d = amax/127, q = rint(x*127/amax)."""
    rng = R.Rng(11)
    x = rng.floats(768, -3.0, 3.0)
    d, qs, bs = ffi.q8k_quantize(x)
    for b in range(3):
        chunk = x[b * 256:(b + 1) * 256]
        amax = np.float32(np.abs(chunk).max())
        back = d[b] * qs[b * 256:(b + 1) * 256].astype(np.float32)
        assert np.all(np.abs(back - chunk) <= amax / np.float32(127.0) * np.float32(0.5) + np.float32(1e-6))
        assert d[b] == amax / np.float32(127.0)
        iscale = np.float32(127.0) / amax
        assert np.array_equal(qs[b * 256:(b + 1) * 256], np.rint(chunk * iscale).astype(np.int8))
    assert np.array_equal(bs.astype(np.int32), qs.astype(np.int32).reshape(-1, 16).sum(1))
    d, qs, bs = ffi.q8k_quantize(np.zeros(256, np.float32))
    assert d[0] == 0 and not qs.any() and not bs.any()


def test_q8k_quantize_nonfinite_block_is_zero():
    x = np.ones(512, np.float32)
    x[300] = np.inf
    d, qs, bs = ffi.q8k_quantize(x)
    assert d[1] == 0 and not qs[256:].any() and not bs[16:].any()
    assert d[0] == np.float32(1.0) / np.float32(127.0) and np.all(qs[:256] == 127)


def _nan_block(big=100.0):
    """Lane l of quantize_avx2's running max sees x[8i + l]; values chosen so that each lane's
    maximum names the lane: |x| = l + 1 everywhere, one big value in lane 0 at group 0."""
    x = np.tile(np.arange(1, 9, dtype=np.float32), 32) * np.float32(0.5)
    x[0] = big
    return x


@pytest.mark.parametrize("case", ["reset", "last_lane7", "last_lane6", "last_lane3", "inf_after_reset"])
def test_q8k_quantize_nan_follows_maxps_order(case):
    """_mm256_max_ps / _mm_max_ps / _mm_max_ss return the second operand when either is NaN
    (quant_q8k.rs:89-98), so the block maximum depends on where the NaN sits; derived by hand:
    - reset: NaN at x[8] (lane 0, group 1) makes lane 0 restart, dropping x[0] = 100 -> amax 4.0
    - last_lane7: NaN at x[255] survives max_ps(am3, am7), (v1, v3) and (v0, v1) -> zero block
    - last_lane6: NaN at x[254] makes v2 and then v0 NaN, which max_ss drops -> amax = v1 =
      the odd lanes' maximum 4.0 (lane 0's 100 is lost with v0)
    - last_lane3: NaN at x[251] is max_ps's first operand against lane 7 -> dropped, amax 100
    - inf_after_reset: +inf at x[0] then NaN at x[8]: amax 4.0 and the inf codes as cvtps'
      out-of-range INT_MIN saturated to -128; a NaN element codes as -128 too."""
    x = _nan_block()
    if case == "reset":
        x[8] = np.nan
        want = 4.0
    elif case == "last_lane7":
        x[255] = np.nan
        want = None
    elif case == "last_lane6":
        x[254] = np.nan
        want = 4.0
    elif case == "last_lane3":
        x[251] = np.nan
        want = 100.0
    else:
        x[0] = np.inf
        x[8] = np.nan
        want = 4.0
    d, qs, bs = ffi.q8k_quantize(x)
    if want is None:
        assert d[0] == 0 and not qs.any() and not bs.any()
        return
    want = np.float32(want)
    assert d[0] == want / np.float32(127.0)
    iscale = np.float32(127.0) / want
    nan = np.isnan(x)
    ok = ~nan & np.isfinite(x)
    assert np.array_equal(qs[ok], np.clip(np.rint(x[ok] * iscale), -128, 127).astype(np.int8))
    assert np.all(qs[nan] == -128) and np.all(qs[np.isinf(x)] == -128)
    if case == "reset":
        assert qs[0] == 127  # 100 * 127/4 saturates
    assert np.array_equal(bs.astype(np.int32), qs.astype(np.int32).reshape(-1, 16).sum(1))


def test_q5k_dequant_pinned_by_q4k_and_the_high_bit_rule():
    """Q5_K (quant.rs:1122-1137, dequant :1612-1640) shares Q4_K's header and code nibbles:
    with every high bit clear a Q5_K block dequantizes exactly like the Q4_K block with the
    same d, dmin, scales and codes (Q4_K is pinned by the known-answer blocks above); setting
    bit 2c+h of qh[t] raises exactly element 64c + 32h + t, by 16 * d * sc_(2c+h) in code units
    (the value is recomputed from the code, so compare through the dequant of code + 16)."""
    rng = np.random.default_rng(3)
    hdr = bytearray(rng.integers(0, 256, 16, dtype=np.uint8).tobytes())
    hdr[0:2] = np.float16(0.03).tobytes()
    hdr[2:4] = np.float16(0.01).tobytes()
    qs = rng.integers(0, 256, 128, dtype=np.uint8).tobytes()
    q4 = np.frombuffer(bytes(hdr) + qs, np.uint8).copy()
    q5 = np.frombuffer(bytes(hdr) + bytes(32) + qs, np.uint8).copy()
    base = ffi.dequant_row(ffi.Q4K, q4, 256)
    assert np.array_equal(ffi.dequant_row(ffi.Q5K, q5, 256), base)
    d = float(np.frombuffer(bytes(hdr[0:2]), np.float16)[0])
    dmin = float(np.frombuffer(bytes(hdr[2:4]), np.float16)[0])
    s12 = hdr[4:16]
    def scale_min(j):  # unpack_q4k_scales (q4k_gemv.rs:70-85)
        if j < 4:
            return s12[j] & 63, s12[j + 4] & 63
        return (s12[j + 4] & 0xF) | ((s12[j - 4] >> 6) << 4), (s12[j + 4] >> 4) | ((s12[j] >> 6) << 4)
    for t, c, h in [(0, 0, 0), (5, 1, 1), (31, 3, 0), (17, 2, 1), (8, 3, 1)]:
        blk = bytearray(q5.tobytes())
        blk[16 + t] |= 1 << (2 * c + h)
        y = ffi.dequant_row(ffi.Q5K, np.frombuffer(bytes(blk), np.uint8).copy(), 256)
        e = 64 * c + 32 * h + t
        changed = np.nonzero(y != base)[0]
        assert changed.tolist() == [e], (t, c, h, changed)
        sc, mn = scale_min(2 * c + h)
        code = (qs[32 * c + t] >> 4) if h else (qs[32 * c + t] & 0xF)
        want = np.float32(np.float32(d * sc) * np.float32(code + 16)) - np.float32(np.float32(dmin) * np.float32(mn))
        assert y[e] == want, (t, c, h, y[e], want)
