"""Prefill passes of 17..128 rows (forward_batch_slice at M up to 128, the prompt chunks of feed,
smollm_chat.rs:3090-3101) on the prefill kernels: the matvecs in 16-vector groups, the
attention rows prepared once, MoE jobs of at most 16 users staged job by job.

A row's matvec arithmetic in these kernels is the reference's: each wavefront contracts the
reference's lane classes on the int8 matrix cores and runs their fp32 chains (the same bits as
the per-lane dot kernels and as one-row passes). Attention is the one stage with several forms:
by default position slices with online softmaxes merged in LDS and bits of their own (k_attn_fs,
SPX_PF_ATTN=4), the chunk loop with split partials (k_attn_fl, 3), or the multi-tile kernels
whose per-chunk partials and merges give a row the bits it gets in a verify or decode pass
(SPX_PF_ATTN=2). With the latter the bar is bitwise: hidden states, logits, greedy picks and the
KV cache of a 128-row pass equal those of the same tokens in passes of at most 16 rows on the
lane kernels. The others are held to the oracle row by row on the GPU's own KV cache (the bars
of test_gpu_engine.py), at contexts of several chunks, and their attention stage directly
against the oracle's attention of the same raw rows."""
import numpy as np
import pytest

from spindle_amd import model as M
from oracle.model import OracleModel
from tests import layer_pins as LP

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

KQ = dict(t_embd=M.Q4K, t_q=M.Q4K, t_k=M.Q4K, t_v=M.Q6K, t_o=M.Q4K, t_gate=M.Q4K, t_up=M.Q4K, t_down=M.Q6K, t_out=M.Q6K)
CASES = {
    "moe": M.TINY["tiny-qwen3moe"].replace(sigma=0.05),
    "moe-prune-mass": M.TINY["tiny-qwen3moe"].replace(sigma=0.05, moe_prune=0.3),
    "dense-kquant": M.TINY["tiny-qwen3"].replace(sigma=0.05, **KQ),
    "a3b": M.TINY["tiny-a3b"].replace(sigma=0.05),
    "a3b-prune4": M.TINY["tiny-a3b"].replace(sigma=0.05, moe_prune=4.0),
    # interleaved RoPE pairs (2i, 2i + 1), no q/k norms, Granite's scales
    "granite-kquant": M.TINY["tiny-granite"].replace(sigma=0.05, n_ff=256, **KQ),
}
# pass sizes: a full chunk and ragged ones (a last vector group of 1, 8 and 2 rows), 252 positions
SIZES = (128, 17, 40, 1, 50, 16)


@pytest.fixture(scope="module")
def ctx():
    from spindle_amd import ops
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    c = ops.Context(0)
    yield c
    c.close()


def _same(a, b):
    return np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))


def _split16(n):
    """Pass sizes of at most 16 rows for n rows (a ragged last pass of 1..15 rows included)."""
    return [16] * (n // 16) + ([n % 16] if n % 16 else [])


def _in16(eng, ids, pos):
    """The same rows in passes of at most 16 rows: (argmax, hidden, logits) concatenated."""
    outs, s = [], 0
    for n in _split16(len(ids)):
        outs.append(eng.forward(ids[s:s + n], pos + s, hidden=True, logits=True))
        s += n
    return tuple(np.concatenate([o[i] for o in outs]) for i in range(3))


@pytest.fixture
def shared_bits(monkeypatch):
    """Prefill attention on the multi-tile kernels: a prefill row gets its verify row's bits."""
    monkeypatch.setenv("SPX_PF_ATTN", "2")


@pytest.mark.parametrize("case", list(CASES))
def test_prefill_pass_equals_16_row_passes(ctx, case, shared_bits):
    cfg = CASES[case]
    w = M.synth_model(cfg, seed=41)
    a, b = M.Engine(ctx, cfg, w), M.Engine(ctx, cfg, w)
    assert a.decode_pipeline()
    b.set_mfma(False)  # the reference: passes of at most 16 rows on the lane-exact kernels
    ids = np.random.default_rng(9).integers(0, cfg.vocab, sum(SIZES))
    pos = 0
    for m in SIZES:
        print(f"{case}: pass of {m} rows at {pos}", flush=True)
        am0, h0, l0 = a.forward(ids[pos:pos + m], pos, hidden=True, logits=True)
        am1, h1, l1 = _in16(b, ids[pos:pos + m], pos)
        assert _same(h0, h1), (case, m, pos, "hidden")
        assert _same(l0, l1), (case, m, pos, "logits")
        assert np.array_equal(am0, am1), (case, m, pos)
        pos += m
    ka, va = a.kv_cache()
    kb, vb = b.kv_cache()
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    if cfg.moe:  # the last pass's experts with users per layer (distinct experts, not jobs)
        assert all(0 < n <= cfg.n_expert for n in a.last_experts())
    a.close()
    b.close()


@pytest.mark.parametrize("case", ["a3b", "moe"])
def test_prefill_long_context(ctx, case, shared_bits):
    """128-row passes past 1024 positions (17+ attention chunks, two merge levels; 128 rows x 8
    query heads = 64 query tiles a kv head) against lane-exact 16-row passes, bitwise."""
    cfg = CASES[case].replace(max_seq=1280)
    w = M.synth_model(cfg, seed=42)
    a, b = M.Engine(ctx, cfg, w), M.Engine(ctx, cfg, w)
    b.set_mfma(False)
    ids = np.random.default_rng(10).integers(0, cfg.vocab, 1240)
    for s0 in range(0, 1240, 128):
        n = min(128, 1240 - s0)
        print(f"{case}: pass of {n} rows at {s0}", flush=True)
        am0, h0, l0 = a.forward(ids[s0:s0 + n], s0, hidden=True, logits=True)
        am1, h1, l1 = _in16(b, ids[s0:s0 + n], s0)
        assert _same(h0, h1) and _same(l0, l1) and np.array_equal(am0, am1), (case, s0)
    ka, va = a.kv_cache()
    kb, vb = b.kv_cache()
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    a.close()
    b.close()


def _norm_err(x, y):
    return float(np.max(np.abs(x.astype(np.float64) - y.astype(np.float64))) / max(1.0, float(np.max(np.abs(y)))))


PF_ATTN = {"slices": "4", "loop": "3", "shared": "2"}


@pytest.mark.parametrize("case", ["moe", "dense-kquant", "a3b", "granite-kquant"])
@pytest.mark.parametrize("attn", list(PF_ATTN))
def test_prefill_pass_at_context_matches_oracle(ctx, case, attn, monkeypatch):
    """A 128-row pass at positions 256..383 (each of the chunk loop's four splits holds one or two
    of its six chunks) against the oracle row by row on the GPU's own KV cache, as below:
    logits median <= 1e-5, in every attention form."""
    monkeypatch.setenv("SPX_PF_ATTN", PF_ATTN[attn])
    cfg = CASES[case].replace(max_seq=512)
    w = M.synth_model(cfg, seed=43)
    eng = M.Engine(ctx, cfg, w)
    om = OracleModel(cfg, w)
    ids = np.random.default_rng(11).integers(0, cfg.vocab, 384)
    for s0 in (0, 128):
        eng.forward(ids[s0:s0 + 128], s0)
    _, _, lg = eng.forward(ids[256:384], 256, logits=True)
    k, v = eng.kv_cache()
    errs = []
    for p in range(256, 384, 4):
        om.k_cache[:] = k
        om.v_cache[:] = v
        lo = om.logits(om.forward(ids[p:p + 1], p))[0]
        errs.append(_norm_err(lg[p - 256], lo))
    errs = np.array(errs)
    print(f"{case} ({attn}): logits err median {np.median(errs):.1e} max {errs.max():.1e}, rows above 1e-3: {(errs > 1e-3).sum()}")
    assert np.median(errs) <= 1e-5
    eng.close()


@pytest.mark.parametrize("case,attn,m", [(c, a, 128) for c in ("a3b", "dense-kquant", "moe", "granite-kquant") for a in PF_ATTN]
                         + [(c, "slices", r) for c in ("a3b", "moe") for r in (17, 50, 97)])
def test_prefill_attention_matches_oracle(ctx, case, attn, m, monkeypatch):
    """The attention stage of an m-row pass at positions 384.. (eight chunks at 128 rows: four
    steps of each half's walk, two chunks of each split, sixteen 32-position slices; ragged
    passes leave a part-filled last query block) against the oracle's attention of the same raw
    q / k / v rows on the GPU's own KV cache (the last layer's buffers after the pass): every
    row within 1e-4 (max-abs normalised, the layer pins' attention bar), in every attention form."""
    monkeypatch.setenv("SPX_PF_ATTN", PF_ATTN[attn])
    cfg = CASES[case].replace(max_seq=512)
    w = M.synth_model(cfg, seed=47)
    eng = M.Engine(ctx, cfg, w)
    om = OracleModel(cfg, w)
    ids = np.random.default_rng(13).integers(0, cfg.vocab, 512)
    for s0 in (0, 128, 256):
        eng.forward(ids[s0:s0 + 128], s0)
    eng.forward(ids[384:384 + m], 384)
    L = cfg.n_layers - 1
    q = eng.debug_buf("q", m * cfg.q_dim).reshape(m, cfg.q_dim)
    k = eng.debug_buf("k", m * cfg.kv_dim).reshape(m, cfg.kv_dim)
    v = eng.debug_buf("v", m * cfg.kv_dim).reshape(m, cfg.kv_dim)
    att = eng.debug_buf("att", m * cfg.q_dim).reshape(m, cfg.q_dim)
    kc, vc = eng.kv_cache()
    om.k_cache[:] = kc
    om.v_cache[:] = vc
    ref = om.attn_rows(L, q, k, v, 384)
    errs = np.array([LP._nerr(att[b], ref[b]) for b in range(m)])
    print(f"{case} ({attn}, {m} rows): attention err median {np.median(errs):.1e} max {errs.max():.1e}")
    assert np.isfinite(att).all()
    assert errs.max() <= 1e-4
    eng.close()


@pytest.mark.parametrize("case", ["moe", "dense-kquant", "a3b"])
def test_prefill_matches_oracle(ctx, case):
    """A 128-row pass against the oracle, row by row on the pass's own context: after the GPU
    pass the oracle gets the GPU's KV cache and computes row p alone at position p (positions
    below p from the GPU's cache), so a Q8_K rounding step in one row does not carry into the
    rows after it through attention. Logits median <= 1e-5; a row above 1e-3 is traced layer by
    layer (the pass's rows are one-row passes' bits): every stage pinned, every moved Q8_K code
    a single step."""
    cfg = CASES[case]
    w = M.synth_model(cfg, seed=43)
    eng = M.Engine(ctx, cfg, w)
    om = OracleModel(cfg, w)
    ids = np.random.default_rng(11).integers(0, cfg.vocab, 128)
    _, _, lg = eng.forward(ids, 0, logits=True)
    k, v = eng.kv_cache()
    errs = []
    for p in range(128):
        om.k_cache[:] = k
        om.v_cache[:] = v
        lo = om.logits(om.forward(ids[p:p + 1], p))[0]
        errs.append(_norm_err(lg[p], lo))
    errs = np.array(errs)
    print(f"{case}: logits err median {np.median(errs):.1e} max {errs.max():.1e}, rows above 1e-3: {(errs > 1e-3).sum()}")
    assert np.median(errs) <= 1e-5

    def sync():
        kk, vv = eng.kv_cache()
        om.k_cache[:] = kk
        om.v_cache[:] = vv
    for p in np.nonzero(errs > 1e-3)[0]:
        LP.report(case, f"row {p} ({errs[p]:.1e})", LP.layer_pins(eng, om, cfg, ids[p:p + 1], int(p), sync, case))
    eng.close()


@pytest.mark.parametrize("name", ["tiny-llama", "tiny-granite"])
def test_prefill_without_prefill_kernels(ctx, name):
    """Models outside the K-quant pipeline (and K-quant models with the matrix cores off) run a
    pass of more than 16 rows as passes of at most 16: the same bits."""
    cfg = M.TINY[name].replace(sigma=0.05)
    w = M.synth_model(cfg, seed=44)
    a, b = M.Engine(ctx, cfg, w), M.Engine(ctx, cfg, w)
    ids = np.random.default_rng(12).integers(0, cfg.vocab, 60)
    am0, h0, l0 = a.forward(ids, 0, hidden=True, logits=True)
    am1, h1, l1 = _in16(b, ids, 0)
    assert _same(h0, h1) and _same(l0, l1) and np.array_equal(am0, am1)
    a.close()
    b.close()
    cfg = CASES["moe"]
    w = M.synth_model(cfg, seed=45)
    a, b = M.Engine(ctx, cfg, w), M.Engine(ctx, cfg, w)
    a.set_mfma(False)
    b.set_mfma(False)
    am0, h0, l0 = a.forward(ids[:40], 0, hidden=True, logits=True)
    am1, h1, l1 = _in16(b, ids[:40], 0)
    assert _same(h0, h1) and _same(l0, l1) and np.array_equal(am0, am1)
    a.close()
    b.close()


@pytest.mark.parametrize("case", ["moe", "a3b"])
def test_generate_with_128_row_prompt_chunks(ctx, case, shared_bits):
    """generate with feed's 128-row prompt chunks gives the stream and counts of 16-row chunks
    (the prompt's KV cache is the same bits), and the default chunk is 128."""
    cfg = CASES[case]
    w = M.synth_model(cfg, seed=46)
    rng = np.random.default_rng(13)
    head = rng.integers(0, cfg.vocab, 150)
    prompt = np.concatenate([head, head[40:110]]).astype(np.int32)
    eng = M.Engine(ctx, cfg, w)
    t16, s16 = eng.generate(prompt, 24, draft_len=8, min_ngram=2, max_ngram=4, fixed=True, prefill_chunk=16)
    t128, s128 = eng.generate(prompt, 24, draft_len=8, min_ngram=2, max_ngram=4, fixed=True, prefill_chunk=128)
    t0, s0 = eng.generate(prompt, 24, draft_len=8, min_ngram=2, max_ngram=4, fixed=True, prefill_chunk=0)
    assert np.array_equal(t16, t128) and np.array_equal(t16, t0)
    for k in ("accepted", "drafted", "verifies", "steps"):
        assert s16[k] == s128[k] == s0[k], k
    eng.close()


@pytest.mark.parametrize("case", ["a3b", "dense-kquant", "tiny-llama", "tiny-granite"])
def test_feed_equals_forward_last_row(ctx, case):
    """spx_engine_feed (feed :3044-3104: prompt chunks of up to 128 rows, the LM head for the last
    row only) gives the last row's hidden state of spx_engine_forward over the same chunks and
    the same KV cache, bitwise; prompts ending in a 44-row, a one-row and a full chunk. Its
    logits come from the one-row LM head, as the reference computes them from feed's last
    hidden: for K-quant models the bits of the multi-row pass's last row; for the float formats
    (whose 2..16-row LM head sums in its own order) within the matvec bar 1e-4 of it, and the
    same pick unless the top two logits are within that bar."""
    cfg = (CASES[case] if case in CASES else M.TINY[case].replace(sigma=0.05)).replace(max_seq=320)
    w = M.synth_model(cfg, seed=47)
    rng = np.random.default_rng(14)
    for n in (300, 257, 128):
        a, b = M.Engine(ctx, cfg, w), M.Engine(ctx, cfg, w)
        ids = rng.integers(0, cfg.vocab, n)
        print(f"{case}: feed of {n} rows", flush=True)
        am0, h0, l0 = a.feed(ids, 0, hidden=True, logits=True)
        for s0 in range(0, n, 128):
            am1, h1, l1 = b.forward(ids[s0:s0 + 128], s0, hidden=True, logits=True)
        assert _same(h0, h1[-1]), (case, n)
        if case in CASES:
            assert _same(l0, l1[-1]) and am0 == am1[-1], (case, n)
        else:
            bar = 1e-4 * np.abs(l1[-1]).max()
            assert np.abs(l0 - l1[-1]).max() <= bar, (case, n)
            top2 = np.sort(l1[-1])[-2:]
            assert am0 == am1[-1] or top2[1] - top2[0] <= 2 * bar, (case, n)
        ka, va = a.kv_cache()
        kb, vb = b.kv_cache()
        assert np.array_equal(ka, kb) and np.array_equal(va, vb), (case, n)
        a.close()
        b.close()
