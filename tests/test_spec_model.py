"""The product's draft-length model (spindle_amd/csrc/spec.h, the object spx_engine_generate
drives) through its C entry points, against the reference's own case
spec_model_skips_drafts_that_do_not_pay (smollm_chat.rs:4667-4694) and against the oracle's
restatement on a long random sequence of events. Host code only: no GPU."""
import ctypes as C

import numpy as np
import pytest

from oracle import ffi


@pytest.fixture(scope="module")
def lib():
    from spindle_amd import _lib
    return _lib.load()


class Spec:
    def __init__(self, lib, fixed=False, handle=None):
        self.lib = lib
        self.h = handle if handle is not None else lib.spx_spec_create(int(fixed))
        assert self.h

    def clone(self):
        return Spec(self.lib, handle=self.lib.spx_spec_clone(self.h))

    def __getattr__(self, name):
        f = getattr(self.lib, "spx_spec_" + name)
        return lambda *a: f(self.h, *a)

    def __del__(self):
        self.lib.spx_spec_destroy(self.h)


def test_reference_case(lib):
    """smollm_chat.rs:4667-4694, step for step."""
    m = Spec(lib)
    m.record_step(100_000)
    m.record_verify(5, 260_000)  # an extra verify row costs 40% of a step
    for _ in range(40):
        assert m.record_draft(0, 2, 0) == 0
    assert m.best_len(0, 2) == 0  # rarely accepted 2-gram drafts: not worth a verify
    for _ in range(40):
        m.record_draft(2, 6, 6)
    assert m.best_len(2, 6) == 6  # long, usually accepted 4+-gram drafts: all of them
    m2 = m.clone()
    m2.reset_rates()
    for _ in range(60):
        m2.record_draft(1, 3, 1)
    assert m2.best_len(1, 6) <= 2  # a middling rate picks a short draft
    f = Spec(lib, fixed=True)
    assert f.best_len(0, 4) == 4  # fixed mode takes the whole draft


def test_class_map(lib):
    """SpecModel::class (:1710-1717)."""
    assert [lib.spx_spec_class(n) for n in range(7)] == [3, 0, 0, 1, 2, 2, 2]


def test_closed_forms(lib):
    """Values the formulas fix: rate = acc / (acc + fail) with unit pseudo-counts, the 0.97
    decay and its 0.5 floor, the verify-cost clamp at 1.5 t1, and best_len's comparison
    gain(k) / (t1 + extra k) against 1 / t1 at p = 0.5."""
    m = Spec(lib)
    assert m.accept_rate(0) == 0.5
    m.record_draft(1, 4, 2)
    assert m.accept_rate(1) == (0.97 + 2) / (0.97 + 2 + 0.97 + 1)
    assert m.accept_rate(0) == 0.5  # other classes decay both counts alike
    for _ in range(60):
        m.record_draft(3, 1, 1)
    assert m.accept_rate(0) == 0.5  # both at the 0.5 floor
    m = Spec(lib)
    m.record_step(1000)
    m.record_verify(3, 10_000)  # (10000 - 1000) / 2 = 4500 > 1.5 t1 -> 1500
    # p = 0.5, t1 = 1000, extra = 1500: gain(1)/cost(2) = 1.5/2500 < 1/1000 -> 0; retry at the 24th
    got = [m.best_len(0, 5) for _ in range(24)]
    assert got == [0] * 23 + [2]
    m = Spec(lib)
    m.record_step(1000)
    m.record_verify(2, 1100)  # extra = 100: gain(k)/(1000 + 100 k), p = 0.5
    gains = np.cumsum([0.5 ** k for k in range(8)])
    rates = [gains[k] / (1000 + 100 * k) for k in range(8)]
    assert m.best_len(0, 7) == int(np.argmax(rates))


def test_invalid_arguments(lib):
    m = Spec(lib)
    assert m.best_len(4, 3) == -1 and m.best_len(-1, 3) == -1 and m.best_len(0, -1) == -1
    assert m.record_draft(0, 2, 3) == -1
    assert lib.spx_spec_best_len(None, 0, 2) == -1
    assert m.accept_rate(7) == -1.0


def test_matches_oracle_on_random_events(lib):
    """A long random mix of steps, verifies, drafts and queries: the product's model and the
    oracle's restatement answer alike at every query (same doubles, same lengths)."""
    rng = np.random.default_rng(3)
    for fixed in (0, 1):
        m = Spec(lib, fixed=bool(fixed))
        o = ffi.SpecModel()
        ffi.lib.or_spec_init(C.byref(o), fixed)
        for _ in range(5000):
            ev = rng.integers(0, 5)
            if ev == 0:
                us = int(rng.integers(0, 300_000))
                m.record_step(us)
                ffi.lib.or_spec_record_step(C.byref(o), us)
            elif ev == 1:
                b, us = int(rng.integers(0, 9)), int(rng.integers(0, 900_000))
                m.record_verify(b, us)
                ffi.lib.or_spec_record_verify(C.byref(o), b, us)
            elif ev == 2:
                c, d = int(rng.integers(0, 4)), int(rng.integers(1, 9))
                a = int(rng.integers(0, d + 1))
                m.record_draft(c, d, a)
                ffi.lib.or_spec_record_draft(C.byref(o), c, d, a)
            elif ev == 3:
                c, av = int(rng.integers(0, 4)), int(rng.integers(0, 9))
                assert m.best_len(c, av) == ffi.lib.or_spec_best_len(C.byref(o), c, av)
            else:
                m.reset_rates()
                ffi.lib.or_spec_reset_rates(C.byref(o))
            c = int(rng.integers(0, 4))
            assert m.accept_rate(c) == ffi.lib.or_spec_accept_rate(C.byref(o), c)
