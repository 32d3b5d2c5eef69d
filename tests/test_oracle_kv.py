"""Pins the oracle's KV window (or_shift_kv / or_ensure_kv_room, smollm_chat.rs:2924-2971):
the eviction policy by hand-worked numbers, and the re-rotated keys against keys rotated at the
new positions from scratch (RoPE rotations compose, :1393-1396), per pair layout."""
import ctypes as C

import numpy as np
import pytest

from oracle import ffi
from oracle.model import OracleModel
from spindle_amd import model as M


def _model(max_seq=100):
    cfg = M.TINY["tiny-qwen3"].replace(max_seq=max_seq)
    return OracleModel(cfg, M.synth_model(cfg, seed=2))


@pytest.mark.parametrize("keep,cur,needed,want", [(10, 50, 10, 50), (10, 95, 10, 53), (10, 100, 1, 55), (0, 100, 60, 40),
                                                  (98, 100, 5, 98), (10, 91, 9, 91)])
def test_ensure_room_policy(keep, cur, needed, want):
    """Fits: unchanged. Else discard max(overflow, (cur - keep) / 2), at most cur - keep:
    95 + 10 - 100 = 5 < 85 / 2 = 42 -> 53; 1 < 45 -> 55; 60 > 50 -> 40; keep 98 leaves 2 -> 98;
    91 + 9 = 100 fits."""
    om = _model()
    assert ffi.lib.or_ensure_kv_room(C.byref(om.m), keep, cur, needed) == want


def _rot(x, inv, pos, neox):
    """Rope::rotate of one head at position pos (float32 arithmetic as the reference)."""
    half = x.size // 2
    y = x.copy()
    for i in range(half):
        a, b = (i, i + half) if neox else (2 * i, 2 * i + 1)
        ang = np.float32(pos) * inv[i]
        s, c = np.float32(np.sin(np.float64(ang))), np.float32(np.cos(np.float64(ang)))
        y[a] = x[a] * c - x[b] * s
        y[b] = x[a] * s + x[b] * c
    return y


@pytest.mark.parametrize("neox", [0, 1])
def test_shift_moves_v_and_rerotates_k(neox):
    L, S, hd, nkv = 2, 64, 16, 2
    kvd = hd * nkv
    rng = np.random.default_rng(neox)
    inv = np.array([1.0 / np.float32(10000.0) ** (np.float32(2 * i) / hd) for i in range(hd // 2)], np.float32)
    raw = rng.standard_normal((L, S, kvd)).astype(np.float32)
    k = np.empty((L, S, kvd), np.float16)
    for l in range(L):
        for p in range(S):
            for h in range(nkv):
                k[l, p, h * hd:(h + 1) * hd] = _rot(raw[l, p, h * hd:(h + 1) * hd], inv, p, neox).astype(np.float16)
    v = rng.standard_normal((L, S, kvd)).astype(np.float16)
    k16, v16 = k.view(np.uint16).copy(), v.view(np.uint16).copy()
    keep, disc, cur = 5, 12, 50
    new = ffi.shift_kv(k16, v16, L, S, kvd, hd, neox, 10000.0, keep, disc, cur)
    assert new == cur - disc
    kk, vv = k16.view(np.float16), v16.view(np.float16)
    assert np.array_equal(v16[:, :keep], v.view(np.uint16)[:, :keep]) and np.array_equal(k16[:, :keep], k.view(np.uint16)[:, :keep])
    assert np.array_equal(v16[:, keep:new], v.view(np.uint16)[:, keep + disc:cur])  # V moves bit for bit
    for l in range(L):
        for p in range(keep, new):  # the moved key now encodes position p (within f16 rounding twice)
            for h in range(nkv):
                fresh = _rot(raw[l, p + disc, h * hd:(h + 1) * hd], inv, p, neox)
                got = kk[l, p, h * hd:(h + 1) * hd].astype(np.float32)
                assert np.all(np.abs(got - fresh) <= 2e-3 * np.abs(fresh).max() + 1e-3), (l, p, h)
    # discard clamped to the unpinned context
    k16b, v16b = k.view(np.uint16).copy(), v.view(np.uint16).copy()
    assert ffi.shift_kv(k16b, v16b, L, S, kvd, hd, neox, 10000.0, keep, 100, cur) == keep
