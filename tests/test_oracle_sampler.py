"""Pins the oracle's sampler (or_sample, SplitMix64) against hand-derived cases and the
distributions the reference's sample_from_logits (smollm_chat.rs:3624-3726) fixes. CPU only.

Tie order: the reference orders candidates with select_nth_unstable / sort_unstable, which
leave logits equal under total order in an unspecified order; the oracle and the GPU order
them by ascending token id (parity holds wherever the kept candidates have distinct logits)."""
import ctypes as C
import math

import numpy as np
import pytest

from oracle import ffi


def test_splitmix64_published_vectors():
    """SplitMix64 (Steele, Lea & Flood 2014; Vigna's splitmix64.c) from state 0: the commonly
    published first outputs."""
    x = C.c_uint64(0)
    got = [ffi.lib.or_splitmix_next(C.byref(x)) for _ in range(3)]
    assert got == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    x = C.c_uint64(0)
    assert ffi.lib.or_splitmix_f32(C.byref(x)) == np.float32(0xE220A8 / 2 ** 24)  # top 24 bits / 2^24


def greedy(**kw):
    return ffi.OracleSampler(temperature=0.0, **kw)


def test_repeat_penalty_divides_positive_multiplies_negative_once():
    lg = np.array([2.0, 0.9, -1.0, -1.5], np.float32)
    s = greedy(repeat_penalty=2.0)
    assert s.sample(lg) == 0
    assert s.sample(lg, recent=[0]) == 0           # 2 / 2 = 1.0 > 0.9
    assert s.sample(lg, recent=[0, 0, 0]) == 0     # a repeated token is penalised once (else 0.25)
    neg = np.array([-1.0, -1.5], np.float32)
    assert s.sample(neg, recent=[0]) == 1          # -1 * 2 = -2 < -1.5 (dividing would give -0.5)
    assert s.sample(lg, recent=[7, -3, 4]) == 0    # ids outside the vocabulary are skipped
    lg2 = np.array([1.0, 0.9], np.float32)
    assert greedy(repeat_penalty=1.2).sample(lg2, recent=[0]) == 1


def test_forbid_stop_and_think_mask_to_minus_infinity():
    lg = np.array([5.0, 1.0, 3.0], np.float32)
    s = greedy(stop_ids=[0], think_open=2)
    assert s.sample(lg) == 0
    assert s.sample(lg, forbid_stop=True) == 2
    assert s.sample(lg, forbid_stop=True, forbid_think=True) == 1
    t = ffi.OracleSampler(temperature=1.0, top_k=0, stop_ids=[0, 2], seed=5)
    assert all(t.sample(lg, forbid_stop=True) == 1 for _ in range(20))  # masked ids never drawn


def test_greedy_is_last_maximum_under_total_order():
    s = greedy()
    assert s.sample(np.array([1, 3, 3, 2], np.float32)) == 2
    assert s.sample(np.array([np.inf, np.nan, 1], np.float32)) == 1  # +NaN above +inf
    assert s.sample(np.array([0.0, -0.0], np.float32)) == 0           # -0 < +0
    assert s.sample(np.array([-np.inf, -np.inf], np.float32)) == 1


def test_no_finite_candidate_falls_back_to_argmax_without_a_draw():
    s = ffi.OracleSampler(temperature=1.0, seed=0)
    assert s.sample(np.array([-np.inf, np.nan, np.inf], np.float32)) == 1
    assert s.s.rng == 0  # no draw consumed
    s.sample(np.array([0.0, 1.0], np.float32))
    assert s.s.rng == 0x9E3779B97F4A7C15  # one draw


def test_first_draw_of_seed_zero():
    """probs [0.75, 0.25] (logits ln 3 and 0 at T = 1); the first draw 0.8833 of seed 0 lands
    past 0.75, on the second candidate (token 0)."""
    lg = np.array([0.0, math.log(3.0)], np.float32)
    s = ffi.OracleSampler(temperature=1.0, top_k=40, top_p=1.0, min_p=0.0, repeat_penalty=1.0, seed=0)
    assert s.sample(lg) == 0
    s = ffi.OracleSampler(temperature=1.0, top_k=1, top_p=1.0, min_p=0.0, repeat_penalty=1.0, seed=0)
    assert s.sample(lg) == 1  # top-k 1: the best whatever the draw


def _freq(sampler, lg, n=20000):
    c = np.bincount([sampler.sample(lg) for _ in range(n)], minlength=lg.size)
    return c / n


def _close(f, p, n=20000):
    sd = np.sqrt(np.maximum(p * (1 - p), 1e-12) / n)
    return np.all(np.abs(f - p) <= 5 * sd + 1e-9)


@pytest.mark.parametrize("case", ["plain", "temperature", "min_p", "top_p", "top_k"])
def test_distributions(case):
    p = np.array([0.5, 0.3, 0.2], np.float64)
    lg = np.log(p).astype(np.float32)[[2, 0, 1]]  # token ids shuffled: token 1 is the best
    perm = np.array([1, 2, 0])  # want[token] from p[rank]
    kw = dict(temperature=1.0, top_k=40, top_p=1.0, min_p=0.0, repeat_penalty=1.0, seed=11)
    if case == "temperature":
        kw["temperature"] = 0.5
        q = p ** 2 / (p ** 2).sum()
    elif case == "min_p":
        kw["min_p"] = 0.5  # floor 0.25 drops the 0.2 token
        q = np.array([0.5, 0.3, 0.0]) / 0.8
    elif case == "top_p":
        kw["top_p"] = 0.7  # 0.5 < 0.7 <= 0.8: two survive
        q = np.array([0.5, 0.3, 0.0]) / 0.8
    elif case == "top_k":
        kw["top_k"] = 2
        q = np.array([0.5, 0.3, 0.0]) / 0.8
    else:
        q = p
    want = np.zeros(3)
    want[perm] = q
    assert _close(_freq(ffi.OracleSampler(**kw), lg), want), case


def test_equal_logits_order_by_token_id():
    s = ffi.OracleSampler(temperature=1.0, top_k=1, seed=3)
    assert s.sample(np.array([0.0, 1.0, 1.0, 1.0], np.float32)) == 1


def test_sampled_generation_same_with_and_without_speculation():
    """The reference's design (:4207-4212): verify rows are sampled with the same sampler and
    the same draws as plain decoding, so a seeded reply is the same tokens either way; a stop
    id ends it before being emitted."""
    from oracle.model import OracleModel
    from spindle_amd import model as M
    c = M.TINY["tiny-llama"].replace(sigma=0.06)
    w = M.synth_model(c, seed=31)
    om = OracleModel(c, w)
    rng = np.random.default_rng(5)
    base = rng.integers(0, c.vocab, 12)
    prompt = np.concatenate([base, base, base[:6]]).astype(np.int32)
    for kw in (dict(temperature=0.6, top_k=40, top_p=0.9, min_p=0.05, repeat_penalty=1.1),
               dict(temperature=0.0, repeat_penalty=1.3)):
        plain, _ = om.generate(prompt, 30, speculate=False, sampler=ffi.OracleSampler(seed=9, **kw))
        spec, st = om.generate(prompt, 30, draft_len=4, min_ngram=1, fixed=True, speculate=True,
                               sampler=ffi.OracleSampler(seed=9, **kw))
        assert np.array_equal(plain, spec) and st["verifies"] > 0, st
        stop = [int(plain[5]), int(plain[9])]
        p2, _ = om.generate(prompt, 30, speculate=False, sampler=ffi.OracleSampler(seed=9, stop_ids=stop, **kw))
        s2, _ = om.generate(prompt, 30, draft_len=4, min_ngram=1, fixed=True, speculate=True,
                            sampler=ffi.OracleSampler(seed=9, stop_ids=stop, **kw))
        assert np.array_equal(p2, s2)
        assert not np.isin(p2[2:], stop).any()  # a drawn stop id ends the reply unemitted
