"""Seeded test data exactly as the reference's own tests generate it.

Rng is the xorshift64 of quant.rs:1666-1677 (also quant_q8k.rs:302-313, quant_multi.rs).
The f16 helpers and matrix builders restate the reference's test helpers, including their
quirks (the truncating f16 of quant_q8k.rs:315-321, the subnormal flush of quant.rs:1680-1690),
so the same seeds give the same bytes as the reference's test runs.
"""
import numpy as np

MASK = (1 << 64) - 1
F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q4K, Q5K, Q6K, BF16 = 0, 1, 2, 3, 6, 7, 8, 12, 13, 14, 30
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), Q4_1: (32, 20), Q5_0: (32, 22),
         Q5_1: (32, 24), Q8_0: (32, 34), Q4K: (256, 144), Q5K: (256, 176), Q6K: (256, 210)}


def row_bytes(dtype, n):
    b, s = BLOCK[dtype]
    assert n % b == 0
    return n // b * s


class Rng:
    def __init__(self, seed):
        self.s = seed & MASK

    def next(self):
        s = self.s
        s ^= (s << 13) & MASK
        s ^= s >> 7
        s ^= (s << 17) & MASK
        self.s = s
        return s

    def f(self, lo, hi):
        lo, hi = np.float32(lo), np.float32(hi)
        t = np.float32(self.next() >> 40) / np.float32(1 << 24)
        return np.float32(lo + np.float32((hi - lo) * t))

    def bytes(self, n):
        out = bytearray(n)
        s = self.s
        for i in range(n):
            s ^= (s << 13) & MASK
            s ^= s >> 7
            s ^= (s << 17) & MASK
            out[i] = s & 0xFF
        self.s = s
        return out

    def floats(self, n, lo, hi):
        return np.array([self.f(lo, hi) for _ in range(n)], np.float32)


def f16_trunc(v):
    """quant_q8k.rs:315-321 / quant_multi.rs f16(): truncating, no subnormal handling."""
    b = int(np.float32(v).view(np.uint32))
    sign = (b >> 16) & 0x8000
    exp = (((b >> 23) & 0xFF) - 127 + 15) & 0xFFFF
    mant = (b >> 13) & 0x3FF
    return ((sign | (exp << 10) | mant) & 0xFFFF).to_bytes(2, "little")


def f16_flush(v):
    """quant.rs:1680-1690 f16(): flushes values below the smallest normal half."""
    b = int(np.float32(v).view(np.uint32))
    sign = (b >> 16) & 0x8000
    if abs(float(v)) < 6.1035156e-05:
        return sign.to_bytes(2, "little")
    exp = (((b >> 23) & 0xFF) - 127 + 15) & 0xFFFF
    mant = (b >> 13) & 0x3FF
    return ((sign | (exp << 10) | mant) & 0xFFFF).to_bytes(2, "little")


def random_matrix(dtype, n, rows, rng):
    """quant_q8k.rs:323-336 and quant_multi.rs random_matrix."""
    rb = row_bytes(dtype, n)
    m = rng.bytes(rb * rows)
    if dtype == F32:
        for i in range(0, len(m), 4):
            m[i:i + 4] = rng.f(-1.0, 1.0).tobytes()
        return np.frombuffer(bytes(m), np.uint8).copy()
    bb, offs = {Q8_0: (34, [0]), Q4K: (144, [0, 2]), Q6K: (210, [208])}[dtype]
    for b0 in range(0, len(m), bb):
        for o in offs:
            m[b0 + o:b0 + o + 2] = f16_trunc(rng.f(0.001, 0.05))
    return np.frombuffer(bytes(m), np.uint8).copy()


def random_row(dtype, n, rng):
    """quant.rs:1693-1725 random_row."""
    ln = row_bytes(dtype, n)
    row = rng.bytes(ln)
    if dtype == BF16:
        for i in range(0, ln, 2):
            row[i:i + 2] = (int(rng.f(-1.0, 1.0).view(np.uint32)) >> 16).to_bytes(2, "little")
        return row
    if dtype == F32:
        for i in range(0, ln, 4):
            row[i:i + 4] = rng.f(-1.0, 1.0).tobytes()
        return row
    if dtype in (Q8_0, Q4_0, Q5_0):
        bb, offs = row_bytes(dtype, 32), [0]
    elif dtype in (Q4_1, Q5_1):
        bb, offs = row_bytes(dtype, 32), [0, 2]
    elif dtype in (Q4K, Q5K):
        bb, offs = row_bytes(dtype, 256), [0, 2]
    elif dtype == Q6K:
        bb, offs = 210, [208]
    else:  # F16
        bb, offs = 2, [0]
    for b0 in range(0, ln, bb):
        for o in offs:
            v = rng.f(-1.0, 1.0) if dtype == F16 else rng.f(0.001, 0.05)
            row[b0 + o:b0 + o + 2] = f16_flush(v)
    return row
