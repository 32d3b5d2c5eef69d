"""Pins the oracle's small operators, MoE layer and speculation helpers (CPU only).

Each check is independent of the oracle's own code: the reference's textbook / loop
references restated in numpy (float64), hand-built corpora with expected drafts worked out by
hand, and the reference's deterministic SpecModel test."""
import ctypes as C

import numpy as np
import pytest

from oracle import ffi

# a handle of its own: the typed signatures below must not change ffi.lib's, which other
# modules call with void pointers
lib = C.CDLL(ffi.LIB_PATH)
P = C.c_void_p
fp = C.POINTER(C.c_float)
ip = C.POINTER(C.c_int)


def _f(name, res, *args):
    f = getattr(lib, name)
    f.restype, f.argtypes = res, list(args)
    return f


rope_inv_freq = _f("or_rope_inv_freq", None, C.c_size_t, C.c_float, fp)
rope_rotate = _f("or_rope_rotate", None, fp, C.c_int, fp, C.c_size_t, C.c_size_t, C.c_float)
rmsnorm = _f("or_rmsnorm", None, fp, fp, fp, C.c_size_t, C.c_float)
moe_forward = _f("or_moe_forward", C.c_int, C.POINTER(ffi.Config), C.POINTER(ffi.Layer), C.c_int,
                 C.POINTER(fp), C.POINTER(fp), ip, ip)
argmax = _f("or_argmax", C.c_int, fp, C.c_int, C.c_float)
lookup_draft = _f("or_lookup_draft", C.c_int, ip, C.c_int, C.c_int, ip, C.c_int, C.c_int, C.c_int, ip, ip)
spec_init = _f("or_spec_init", None, C.POINTER(ffi.SpecModel), C.c_int)
spec_best_len = _f("or_spec_best_len", C.c_int, C.POINTER(ffi.SpecModel), C.c_int, C.c_int)
spec_reset = _f("or_spec_reset_rates", None, C.POINTER(ffi.SpecModel))
spec_draft = _f("or_spec_record_draft", None, C.POINTER(ffi.SpecModel), C.c_int, C.c_int, C.c_int)
spec_step = _f("or_spec_record_step", None, C.POINTER(ffi.SpecModel), C.c_uint64)
spec_verify = _f("or_spec_record_verify", None, C.POINTER(ffi.SpecModel), C.c_int, C.c_uint64)


def _p(a, t=fp):
    return a.ctypes.data_as(t)


def _rope_textbook(v, head_dim, pos, theta, neox):
    """rope_reference (smollm_chat.rs:4852-4865) in float64."""
    out = v.astype(np.float64).copy()
    half = head_dim // 2
    for h in range(v.size // head_dim):
        for i in range(half):
            ang = pos * theta ** (-(2.0 * i) / head_dim)
            a, b = (h * head_dim + i, h * head_dim + i + half) if neox else (h * head_dim + 2 * i, h * head_dim + 2 * i + 1)
            out[a] = v[a] * np.cos(ang) - v[b] * np.sin(ang)
            out[b] = v[a] * np.sin(ang) + v[b] * np.cos(ang)
    return out


@pytest.mark.parametrize("neox", [0, 1])
def test_rope_matches_textbook_and_composes(neox):
    """rope_matches_reference_and_composes (smollm_chat.rs:4867-4886)."""
    hd, theta = 64, 100000.0
    v = np.array([((i * 37 % 101) / 50.0) - 1.0 for i in range(3 * hd)], np.float32)
    inv = np.zeros(hd // 2, np.float32)
    rope_inv_freq(hd, theta, _p(inv))
    a = v.copy()
    rope_rotate(_p(inv), neox, _p(a), a.size, hd, 17.0)
    assert np.max(np.abs(a - _rope_textbook(v, hd, 17.0, theta, neox))) < 1e-4
    rope_rotate(_p(inv), neox, _p(a), a.size, hd, -5.0)
    b = v.copy()
    rope_rotate(_p(inv), neox, _p(b), b.size, hd, 12.0)
    assert np.max(np.abs(a - b)) < 1e-4
    # a planted mistake (the pair layout of the other RoPE style) fails the textbook check
    c = v.copy()
    rope_rotate(_p(inv), 1 - neox, _p(c), c.size, hd, 17.0)
    assert np.max(np.abs(c - _rope_textbook(v, hd, 17.0, theta, neox))) > 1e-2


def test_rmsnorm_matches_float64():
    rng = np.random.default_rng(3)
    for n in (576, 1024, 2048):
        x = rng.standard_normal(n).astype(np.float32) * 3
        w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        out = np.zeros(n, np.float32)
        rmsnorm(_p(x), _p(w), _p(out), n, 1e-5)
        x64 = x.astype(np.float64)
        want = x64 / np.sqrt(np.mean(x64 * x64) + 1e-5) * w
        assert np.max(np.abs(out - want)) <= 1e-5 * np.max(np.abs(want))


def test_rmsnorm_sums_in_sequence():
    """rmsnorm (smollm_chat.rs:569-575) sums x*x with Iterator::sum, one f32 add at a time in
    index order: the oracle's result equals that sequence bit for bit."""
    rng = np.random.default_rng(4)
    for n in (576, 2048):
        x = (rng.standard_normal(n) * np.exp(rng.uniform(-3, 3, n))).astype(np.float32)
        w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        ss = np.float32(0.0)
        for v in x:
            ss = np.float32(ss + np.float32(v * v))
        inv = np.float32(1.0) / np.sqrt(np.float32(ss / np.float32(n) + np.float32(1e-5)))
        want = (x * inv).astype(np.float32) * w
        out = np.zeros(n, np.float32)
        rmsnorm(_p(x), _p(w), _p(out), n, 1e-5)
        assert np.array_equal(out.view(np.uint32), want.astype(np.float32).view(np.uint32)), n


def _fma32(a, b, c):
    from fractions import Fraction
    return np.float32(float(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))))


def test_norm_order_knob_is_the_gpu_tree():
    """The sensitivity knob (ffi.set_norm_order): per 256-value block the four-value fma chain
    of each group, a pairwise tree over the 64 groups in index order, the blocks in order; off
    again, the reference's sequence."""
    from oracle import ffi
    rng = np.random.default_rng(5)
    n = 512
    x = (rng.standard_normal(n) * np.exp(rng.uniform(-4, 4, n))).astype(np.float32)
    w = np.ones(n, np.float32)
    S = np.float32(0.0)
    for b in range(n // 256):
        p = []
        for j in range(64):
            v = x[256 * b + 4 * j: 256 * b + 4 * j + 4]
            t = np.float32(v[0] * v[0])
            for k in (1, 2, 3):
                t = _fma32(v[k], v[k], t)
            p.append(t)
        while len(p) > 1:
            p = [np.float32(p[i] + p[i + 1]) for i in range(0, len(p), 2)]
        S = np.float32(S + p[0])
    inv = np.float32(1.0) / np.sqrt(np.float32(S / np.float32(n) + np.float32(1e-5)))
    want = ((x * inv).astype(np.float32) * w).astype(np.float32)
    out = np.zeros(n, np.float32)
    ffi.set_norm_order(True)
    try:
        rmsnorm(_p(x), _p(w), _p(out), n, 1e-5)
    finally:
        ffi.set_norm_order(False)
    assert np.array_equal(out.view(np.uint32), want.view(np.uint32))
    seq = np.zeros(n, np.float32)
    rmsnorm(_p(x), _p(w), _p(seq), n, 1e-5)
    assert np.max(np.abs(seq - out)) <= 1e-5 * np.max(np.abs(out))  # the two orders: last bits only


def _xorshift_floats(seed, n):
    """The reference tests' generator (smollm_chat.rs:4894-4903): xorshift64, (s>>40)/2^24 - 0.5."""
    out = np.empty(n, np.float32)
    s = seed
    m = (1 << 64) - 1
    for i in range(n):
        s ^= (s << 13) & m
        s ^= s >> 7
        s ^= (s << 17) & m
        out[i] = np.float32((s >> 40) / float(1 << 24) - 0.5)
    return out, s


@pytest.mark.parametrize("norm", [1, 0])
def test_moe_forward_matches_loop_reference(norm):
    """moe_forward_matches_reference (smollm_chat.rs:4888-4973), F32 experts, no shared expert."""
    dim, ff, ne, k = 32, 24, 6, 2
    flat, _ = _xorshift_floats(12345, dim * ne + 3 * dim * ff * ne)
    o = 0
    router = flat[o:o + dim * ne].reshape(ne, dim); o += dim * ne
    gate = flat[o:o + dim * ff * ne].reshape(ne, ff, dim); o += dim * ff * ne
    up = flat[o:o + dim * ff * ne].reshape(ne, ff, dim); o += dim * ff * ne
    down = flat[o:o + ff * dim * ne].reshape(ne, dim, ff)
    x = np.sin(np.arange(dim) * 0.37).astype(np.float32)
    cfg = ffi.Config(dim=dim, n_expert=ne, n_expert_used=k, expert_norm=norm, moe_prune=0.0)
    ly = ffi.Layer()
    ly.is_moe = 1
    keep = [np.ascontiguousarray(a) for a in (router, gate, up, down)]
    ly.router = ffi.Mat(ffi.F32, dim, ne, keep[0].ctypes.data)
    ly.gate = ffi.Mat(ffi.F32, dim, ff, keep[1].ctypes.data)
    ly.up = ffi.Mat(ffi.F32, dim, ff, keep[2].ctypes.data)
    ly.down = ffi.Mat(ffi.F32, ff, dim, keep[3].ctypes.data)
    out = np.zeros(dim, np.float32)
    xs = (fp * 1)(_p(x))
    outs = (fp * 1)(_p(out))
    chosen = np.zeros(32, np.int32)
    nkeep = np.zeros(1, np.int32)
    assert moe_forward(C.byref(cfg), C.byref(ly), 1, xs, outs, _p(chosen, ip), _p(nkeep, ip)) == 0
    # loop reference in float64
    x64 = x.astype(np.float64)
    logits = router.astype(np.float64) @ x64
    ex = np.exp(logits - logits.max())
    probs = ex / ex.sum()
    top = np.argsort(-probs, kind="stable")[:k]
    want = np.zeros(dim)
    for e in top:
        g = gate[e].astype(np.float64) @ x64
        u = up[e].astype(np.float64) @ x64
        h = g / (1 + np.exp(-g)) * u
        wt = probs[e] / probs[top].sum() if norm else probs[e]
        want += wt * (down[e].astype(np.float64) @ h)
    assert sorted(chosen[:k].tolist()) == sorted(top.tolist())
    assert np.max(np.abs(out - want)) < 1e-4


def _draft(corpus, k, stop=(), min_ng=2, max_ng=4):
    c = np.array(corpus, np.int32)
    s = np.array(list(stop) or [0], np.int32)
    d = np.zeros(max(k, 1), np.int32)
    ng = C.c_int(0)
    n = lookup_draft(_p(c, ip), c.size, k, _p(s, ip), len(stop), min_ng, max_ng, _p(d, ip), C.byref(ng))
    return d[:n].tolist(), ng.value


def test_lookup_draft_hand_built_corpora():
    """lookup_draft (smollm_chat.rs:2982-3015), expectations worked out by hand."""
    # the last 4 tokens 1 2 3 4 occur at 0..3; the next tokens there are 5 6 7 ...
    assert _draft([1, 2, 3, 4, 5, 6, 7, 8, 1, 2, 3, 4], 3) == ([5, 6, 7], 4)
    # only a 3-gram match (9 2 3 4 does not occur earlier)
    assert _draft([1, 2, 3, 4, 5, 6, 7, 9, 2, 3, 4], 5) == ([5, 6, 7, 9, 2], 3)
    # the latest earlier occurrence wins: 3 4 is followed by 5 at 2..3 and by 8 at 5..6
    assert _draft([3, 4, 5, 0, 0, 3, 4, 8, 3, 4], 4) == ([8, 3], 2)
    # a 2-gram match proposes at most 2 tokens
    assert _draft([7, 8, 1, 2, 3, 4, 9, 7, 8], 6) == ([1, 2], 2)
    # drafts stop at a stop id
    assert _draft([1, 2, 3, 4, 5, 99, 6, 1, 2, 3, 4], 5, stop=[99]) == ([5], 4)
    # the proposal ends at the corpus end
    assert _draft([5, 6, 7, 5, 6, 7], 8) == ([5, 6, 7], 3)
    # no match
    assert _draft([1, 2, 3, 4, 5], 3) == ([], 0)


def test_spec_model_reference_case():
    """spec_model_skips_drafts_that_do_not_pay (smollm_chat.rs:4667-4694)."""
    m = ffi.SpecModel()
    spec_init(C.byref(m), 0)
    spec_step(C.byref(m), 100_000)
    spec_verify(C.byref(m), 5, 260_000)
    for _ in range(40):
        spec_draft(C.byref(m), 0, 2, 0)
    assert spec_best_len(C.byref(m), 0, 2) == 0
    for _ in range(40):
        spec_draft(C.byref(m), 2, 6, 6)
    assert spec_best_len(C.byref(m), 2, 6) == 6
    m2 = ffi.SpecModel.from_buffer_copy(m)
    spec_reset(C.byref(m2))
    for _ in range(60):
        spec_draft(C.byref(m2), 1, 3, 1)
    assert spec_best_len(C.byref(m2), 1, 6) <= 2
    f = ffi.SpecModel()
    spec_init(C.byref(f), 1)
    assert spec_best_len(C.byref(f), 0, 4) == 4


def _route_case(logits, n_used, prune, norm=1):
    """or_moe_forward on x = e_0 against an F32 router whose column 0 holds `logits` (so the
    router's output is exactly `logits`) and small F32 experts; returns the kept experts in
    choice order."""
    ne, dim, ff = len(logits), 32, 16
    router = np.zeros((ne, dim), np.float32)
    router[:, 0] = logits
    rng = np.random.default_rng(1)
    gate = (rng.standard_normal((ne, ff, dim)) * 0.1).astype(np.float32)
    up = (rng.standard_normal((ne, ff, dim)) * 0.1).astype(np.float32)
    down = (rng.standard_normal((ne, dim, ff)) * 0.1).astype(np.float32)
    x = np.zeros(dim, np.float32)
    x[0] = 1.0
    cfg = ffi.Config(dim=dim, n_expert=ne, n_expert_used=n_used, expert_norm=norm, moe_prune=prune)
    ly = ffi.Layer()
    ly.is_moe = 1
    keep = [np.ascontiguousarray(a) for a in (router, gate, up, down)]
    ly.router = ffi.Mat(ffi.F32, dim, ne, keep[0].ctypes.data)
    ly.gate = ffi.Mat(ffi.F32, dim, ff, keep[1].ctypes.data)
    ly.up = ffi.Mat(ffi.F32, dim, ff, keep[2].ctypes.data)
    ly.down = ffi.Mat(ffi.F32, ff, dim, keep[3].ctypes.data)
    out = np.zeros(dim, np.float32)
    chosen = np.zeros(32, np.int32)
    nkeep = np.zeros(1, np.int32)
    assert moe_forward(C.byref(cfg), C.byref(ly), 1, (fp * 1)(_p(x)), (fp * 1)(_p(out)), _p(chosen, ip), _p(nkeep, ip)) == 0
    return chosen[:nkeep[0]].tolist()


# probabilities of ten experts, assigned to a shuffled expert order so that choice order matters
_PROBS = [0.40, 0.20, 0.15, 0.10, 0.05, 0.04, 0.03, 0.02, 0.005, 0.005]
_PERM = [7, 2, 9, 0, 4, 8, 1, 5, 3, 6]  # expert holding the i-th largest probability


def _prune_logits():
    lg = np.zeros(10, np.float32)
    for i, e in enumerate(_PERM):
        lg[e] = np.log(_PROBS[i])
    return lg


@pytest.mark.parametrize("prune,keep", [(0.0, 8), (4.0, 4), (2.0, 4), (6.0, 6), (9.0, 8)])
def test_prune_count_rule_by_hand(prune, keep):
    """moe_prune >= 1 (smollm_chat.rs:1224-1226): keep clamp(prune, max(2, n_used/2), n_used) of
    the top n_used = 8 by probability; here min_keep = 4. Expected counts worked out by hand."""
    assert _route_case(_prune_logits(), 8, prune) == _PERM[:keep]


@pytest.mark.parametrize("prune,keep", [(0.5, 4), (0.1, 5), (0.03, 7)])
def test_prune_mass_rule_by_hand(prune, keep):
    """moe_prune < 1 (:1227-1235): keep the fewest top choices (at least min_keep = 4) whose mass
    reaches (1 - prune) of the top-8 mass 0.99. 0.5: target 0.495, the first four already hold
    0.85, so the cut falls exactly at min_keep; 0.1: target 0.891, 0.85 + 0.05 reaches it at 5;
    0.03: target 0.9603, the cumulative 0.94 (6) then 0.97 (7)."""
    assert _route_case(_prune_logits(), 8, prune) == _PERM[:keep]


def test_route_ties_go_to_the_lower_index():
    """Exactly equal probabilities: the lower expert index is chosen first (the reference's
    select_nth_unstable_by leaves tie order unspecified; this build fixes it)."""
    lg = np.array([0.0, 1.0, 0.0, 2.0, 0.0, 0.0, 1.0, 0.0], np.float32)
    assert _route_case(lg, 4, 0.0) == [3, 1, 6, 0]


def test_argmax_total_order_last_max():
    """sample_from_logits' greedy pick (:3661-3671): logits / logit_scale, then
    max_by(total_cmp) over the logits in index order, which keeps the last of equal maxima;
    -0.0 orders below +0.0 and a positive NaN above +inf."""
    def am(v, scale=1.0):
        a = np.array(v, np.float32)
        return argmax(_p(a), a.size, scale)
    assert am([1.0, 3.0, 3.0, 2.0]) == 2
    assert am([1.0, 3.0, 3.0, 2.0], 6.0) == 2
    assert am([5.0, 5.0, 5.0]) == 2
    assert am([-0.0, 0.0]) == 1 and am([0.0, -0.0]) == 0
    assert am([1.0, np.nan, np.inf, 2.0]) == 1
    assert am([-np.inf, -np.inf]) == 1
    assert am([-3.0, -1.0, -2.0]) == 1
