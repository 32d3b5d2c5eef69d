"""GPU sampler (spx_sample, spx_sample_verify, the engine's sampled generate) against the
oracle's sample_from_logits (smollm_chat.rs:3624-3726) on the same logits and seed: identical
token sequences draw for draw (so the SplitMix64 states stay in step), across the reference's
defaults, greedy with penalty, top-k 1 / 1024 / 0 (all finite), extreme temperatures,
logit_scale, non-finite logits and the stop / think masks."""
import numpy as np
import pytest

from oracle import ffi
from oracle.model import OracleModel

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ctx():
    from spindle_amd import ops
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    c = ops.Context(0)
    yield c
    c.close()


CONFIGS = {
    "reference-default": dict(temperature=0.6, top_k=40, top_p=0.9, min_p=0.05, repeat_penalty=1.1),
    "greedy-penalty": dict(temperature=0.0, repeat_penalty=1.1),
    "top1": dict(temperature=1.0, top_k=1, top_p=1.0, min_p=0.0, repeat_penalty=1.3),
    "top1024-hot": dict(temperature=1.7, top_k=1024, top_p=1.0, min_p=0.0, repeat_penalty=0.9),
    "all-finite": dict(temperature=0.8, top_k=0, top_p=0.95, min_p=0.0, repeat_penalty=1.1),
    "cold-minp": dict(temperature=0.05, top_k=200, top_p=0.5, min_p=0.3, repeat_penalty=1.05),
}


def _logits(rng, V, rows, kind):
    x = (rng.standard_normal((rows, V)) * (3.0 if kind != "flat" else 0.05)).astype(np.float32)
    if kind == "special":
        for r in range(rows):
            x[r, rng.integers(0, V, 50)] = x[r].max() if rng.random() < 0.5 else x[r, 0]  # exact ties
            x[r, rng.integers(0, V, 5)] = np.inf
            x[r, rng.integers(0, V, 5)] = -np.inf
            x[r, rng.integers(0, V, 3)] = np.nan
    return x


@pytest.mark.parametrize("V", [1000, 151936])
@pytest.mark.parametrize("cfg", list(CONFIGS))
def test_sample_matches_oracle(ctx, cfg, V):
    from spindle_amd import ops
    rng = np.random.default_rng(V + len(cfg))
    stop = [int(v) for v in rng.integers(0, V, 3)]
    kw = dict(CONFIGS[cfg], seed=12345, stop_ids=stop, think_open=int(rng.integers(0, V)))
    gs = ops.Sampler(ctx, V, **kw)
    os_ = ffi.OracleSampler(**kw)
    n = 60 if V > 10000 else 200
    for kind in ("normal", "special", "flat"):
        x = _logits(rng, V, 4, kind)
        xd = torch.from_numpy(x).cuda()
        for i in range(n // 3):
            r = i % 4
            recent = rng.integers(0, V, int(rng.integers(0, 40))).tolist()
            recent += [int(x[r].argmax())] * int(rng.integers(0, 2))  # penalise the favourite now and then
            fs, ft = bool(rng.random() < 0.5), bool(rng.random() < 0.3)
            lsc = float(rng.choice([1.0, 1.0, 2.5]))
            g = gs.sample(xd[r], recent, fs, ft, lsc)
            o = os_.sample(x[r], recent, fs, ft, lsc)
            assert g == o, (cfg, V, kind, i, g, o)
    assert gs.sample(xd[0]) == os_.sample(x[0])  # still in step
    gs.close()


@pytest.mark.parametrize("cfg", ["reference-default", "greedy-penalty", "all-finite"])
def test_sample_verify_matches_oracle(ctx, cfg):
    """Rows sampled in order with the window growing by each accepted draft, stop ids masked
    while generated + i < 2, the first mismatch (or the bonus row) ending the pass, and
    max_accept ending it without a further draw."""
    from spindle_amd import ops
    V = 4096
    rng = np.random.default_rng(9)
    stop = [7, 11]
    kw = dict(CONFIGS[cfg], seed=77, stop_ids=stop)
    gs = ops.Sampler(ctx, V, **kw)
    os_ = ffi.OracleSampler(**kw)
    for trial in range(60):
        nd = int(rng.integers(0, 9))
        x = (rng.standard_normal((nd + 1, V)) * 2.0).astype(np.float32)
        x[:, 7] = 9.0  # a stop id would win where it is not masked
        recent = rng.integers(0, V, int(rng.integers(0, 30))).tolist()
        gen = int(rng.integers(0, 4))
        max_accept = int(rng.integers(1, 10))
        # drafts: the oracle's own picks for a random prefix (copied RNG state), then noise
        probe = ffi.OracleSampler(**kw)
        probe.s.rng = os_.s.rng
        draft, win = [], list(recent)
        n_good = int(rng.integers(0, nd + 1))
        for i in range(nd):
            t = probe.sample(x[i], win, gen + i < 2) if i < n_good else int(rng.integers(0, V))
            draft.append(t)
            win.append(t)
        got = gs.sample_verify(torch.from_numpy(x).cuda(), recent, draft, gen, max_accept)
        want, win = [], list(recent)
        for i in range(nd + 1):
            t = os_.sample(x[i], win, gen + i < 2)
            want.append(t)
            if i == nd or t != draft[i] or len(want) >= max_accept:
                break
            win.append(t)
        assert got.tolist() == want, (cfg, trial, nd, n_good, max_accept, got, want)
    gs.close()


def _replay(eng, prompt, n_max, sampler, stop):
    """generate_reply's token sequence rebuilt from the engine's own logits with the oracle's
    sampler: the prompt fed in 16-row chunks as generate does, then one token at a time, each
    drawn over the reply so far with stop ids forbidden while fewer than 2 are out, ending
    before a stop id. Speculation draws the same tokens with the same draws (:4207-4212)."""
    lg = None
    for s in range(0, len(prompt), 16):
        _, _, lg = eng.forward(prompt[s:s + 16], s, logits=True)
    row, pos, out = lg[-1], len(prompt), []
    while True:
        t = sampler.sample(row, out, len(out) < 2, False, eng.cfg.logit_scale)
        if t in stop:
            return out
        out.append(t)
        if len(out) >= n_max:
            return out
        _, _, lg = eng.forward([t], pos, logits=True)
        row, pos = lg[0], pos + 1


@pytest.mark.parametrize("name", ["tiny-llama", "tiny-qwen3moe"])
@pytest.mark.parametrize("cfg", ["reference-default", "greedy-penalty"])
def test_generate_sampled_matches_replay(ctx, name, cfg):
    """spx_engine_generate with a sampler: the tokens the oracle's sampler draws from the
    engine's own logits, one reply after another with the SplitMix64 state carried, with
    speculation on and off; a stop id among the likely tokens ends replies early. (Against the
    oracle's logits the streams part where a last-bit difference in a re-quantized activation
    moves a logit by ~1e-2 and a draw lands between the two cumulative sums.)"""
    from spindle_amd import model as M
    c = M.TINY[name].replace(sigma=0.06)
    w = M.synth_model(c, seed=31)
    rng = np.random.default_rng(5)
    base = rng.integers(0, c.vocab, 12)
    prompt = np.concatenate([base, base, base[:6]]).astype(np.int32)
    eng = M.Engine(ctx, c, w)
    eng.set_mfma(False)  # verify rows bit-identical to one-row passes
    _, _, lg = eng.forward(prompt[:16], 0, logits=True)
    stop = [int(np.argsort(lg[-1])[-3]), int(rng.integers(0, c.vocab))]  # a plausible token stops
    kw = dict(CONFIGS[cfg], seed=2024, stop_ids=stop)
    for spec in (False, True):
        eng.set_sampler(**kw)
        os_ = ffi.OracleSampler(**kw)
        lens = []
        for reply in range(3):
            g, gst = eng.generate(prompt, 40, draft_len=4, min_ngram=2, max_ngram=4, speculate=spec)
            want = _replay(eng, prompt, 40, os_, stop)
            assert g.tolist() == want, (name, cfg, spec, reply, g, want)
            lens.append(len(g))
        print(name, cfg, "spec" if spec else "plain", "reply lengths", lens)
    eng.set_sampler()
    eng.close()
