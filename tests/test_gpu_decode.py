"""The one-row decode pipeline (decode.hip) against the fused pass kernels (fused.hip).

Both compute forward_slice (smollm_chat.rs:3364-3552) with the same operations in the same
order, so every one-token pass must give the same bits on both: final hidden state, logits,
greedy pick, KV cache rows and MoE routing statistics. The fused kernels are themselves
held to the CPU oracle by test_gpu_engine.py; the pipeline is also checked against the oracle
directly here (teacher-forced, same bars as there)."""
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
    "moe-prune2": M.TINY["tiny-qwen3moe"].replace(sigma=0.05, moe_prune=2.0),
    "moe-prune-mass": M.TINY["tiny-qwen3moe"].replace(sigma=0.05, moe_prune=0.3),
    "dense-kquant": M.TINY["tiny-qwen3"].replace(sigma=0.05, **KQ),
    # Qwen3-30B-A3B's kernel shapes: head_dim 128, hpk 8, 128 experts top-8, moe_prune off / top-4 / mass
    "a3b": M.TINY["tiny-a3b"].replace(sigma=0.05),
    "a3b-prune4": M.TINY["tiny-a3b"].replace(sigma=0.05, moe_prune=4.0),
    "a3b-prune-mass": M.TINY["tiny-a3b"].replace(sigma=0.05, moe_prune=0.1),
}
LONG = ("moe", "a3b")  # contexts past 16 chunks (two-level merge) and past position 1024


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


def test_pipeline_applies_to_kquant_models_only(ctx):
    for name, want in (("tiny-qwen3moe", True), ("tiny-llama", False), ("tiny-qwen3", False), ("tiny-granite", False)):
        cfg = M.TINY[name]
        eng = M.Engine(ctx, cfg, M.synth_model(cfg, seed=3))
        assert eng.decode_pipeline() == want, name
        eng.set_decode(False)
        assert not eng.decode_pipeline()
        eng.close()


@pytest.mark.parametrize("case", list(CASES))
def test_decode_pipeline_bitwise(ctx, case):
    """One-token passes at contexts of one chunk, several 64-position chunks and (for the MoE
    case) more than 16 chunks, where the merge runs in two levels."""
    cfg = CASES[case]
    long_ctx = case in LONG
    if long_ctx:
        cfg = cfg.replace(max_seq=1280)
    w = M.synth_model(cfg, seed=31)
    a, b = M.Engine(ctx, cfg, w), M.Engine(ctx, cfg, w)
    assert a.decode_pipeline()
    a.set_mfma(False)  # multi-row prefill passes on the lane-exact kernels: the same KV bits
    b.set_decode(False)
    assert not b.decode_pipeline()
    rng = np.random.default_rng(5)
    n_pre = 1100 if long_ctx else 150
    ids = rng.integers(0, cfg.vocab, n_pre + 40)
    checkpoints = [16, 70, 140] + ([1090] if long_ctx else [])
    pos = 0
    for cp in checkpoints:
        while pos < cp:  # prefill up to the checkpoint
            m = min(16, cp - pos)
            a.forward(ids[pos:pos + m], pos)
            b.forward(ids[pos:pos + m], pos)
            pos += m
        for _ in range(3):
            am0, h0, l0 = a.forward(ids[pos:pos + 1], pos, hidden=True, logits=True)
            am1, h1, l1 = b.forward(ids[pos:pos + 1], pos, hidden=True, logits=True)
            assert _same(h0, h1), (case, pos, "hidden")
            assert _same(l0, l1), (case, pos, "logits")
            assert np.array_equal(am0, am1), (case, pos)
            pos += 1
    ka, va = a.kv_cache()
    kb, vb = b.kv_cache()
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    if cfg.moe:
        assert np.array_equal(a.last_experts(), b.last_experts())
    a.close()
    b.close()


def test_back_to_back_decode_on_pipeline(ctx):
    """spx_engine_decode's one-row graph (the pick advances the step record on the device)
    on the pipeline picks what separate passes on the fused kernels pick."""
    cfg = CASES["moe"]
    w = M.synth_model(cfg, seed=32)
    a, b = M.Engine(ctx, cfg, w), M.Engine(ctx, cfg, w)
    a.set_mfma(False)
    b.set_decode(False)
    ids = np.arange(20) * 13 % cfg.vocab
    a.forward(ids[:16], 0)
    b.forward(ids[:16], 0)
    got = a.decode(int(ids[16]), 16, 40)
    tok, want = int(ids[16]), []
    for i in range(40):
        am, _, _ = b.forward([tok], 16 + i)
        tok = int(am[0])
        want.append(tok)
    assert got.tolist() == want
    ka, va = a.kv_cache()
    kb, vb = b.kv_cache()
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    a.close()
    b.close()


def test_toggle_recaptures_graphs(ctx):
    """Switching pipelines drops the captured one-row graphs; both directions keep the bits."""
    cfg = CASES["moe"]
    w = M.synth_model(cfg, seed=33)
    eng = M.Engine(ctx, cfg, w)
    ids = np.arange(24) * 3 % cfg.vocab
    eng.forward(ids[:16], 0)
    outs = []
    for on in (True, False, True):
        eng.set_decode(on)
        _, h, l = eng.forward(ids[16:17], 16, hidden=True, logits=True)
        outs.append((h, l))
    assert all(_same(outs[0][0], o[0]) and _same(outs[0][1], o[1]) for o in outs[1:])
    eng.close()


@pytest.mark.parametrize("case", list(CASES))
def test_decode_pipeline_matches_oracle(ctx, case):
    """Teacher-forced: the oracle gets the GPU's KV cache before each one-token pass (for the
    headline-shaped family also at positions past 1024, 17+ attention chunks)."""
    cfg = CASES[case]
    w = M.synth_model(cfg, seed=34)
    eng = M.Engine(ctx, cfg, w)
    assert eng.decode_pipeline()
    om = OracleModel(cfg, w)
    n_pre = 1100 if case in LONG and cfg.max_seq >= 1280 else 16
    ids = np.random.default_rng(6).integers(0, cfg.vocab, n_pre + 32)
    for s0 in range(0, n_pre, 16):
        eng.forward(ids[s0:min(s0 + 16, n_pre)], s0)
    errs, flips = [], 0
    for pos in range(n_pre, len(ids)):
        k, v = eng.kv_cache()
        om.k_cache[:] = k
        om.v_cache[:] = v
        _, _, lg = eng.forward(ids[pos:pos + 1], pos, logits=True)
        want = om.logits(om.forward(ids[pos:pos + 1], pos))[0].astype(np.float64)
        e = float(np.max(np.abs(lg[0] - want)) / max(1.0, float(np.max(np.abs(want)))))
        errs.append(e)
        if e > 1e-3:  # traced layer by layer: every stage pinned, every moved Q8_K code one step
            LP.report(case, f"step at {pos} ({e:.1e})", LP.layer_pins(eng, om, cfg, ids[pos:pos + 1], pos, lambda: _sync(eng, om), case))
            flips += 1
    print(f"{case}: logits err median {np.median(errs):.1e} max {max(errs):.1e}, steps traced to Q8_K steps {flips}")
    assert np.median(errs) <= 1e-5
    eng.close()


def _sync(eng, om):
    k, v = eng.kv_cache()
    om.k_cache[:] = k
    om.v_cache[:] = v


@pytest.mark.parametrize("case", list(CASES))
def test_multi_row_passes_bitwise(ctx, case):
    """Passes of 2..16 rows on the pipeline's lane-exact multi-row kernels (norm once per layer,
    grouped expert jobs) against the fused pass kernels: the same bits for every row."""
    cfg = CASES[case]
    w = M.synth_model(cfg, seed=35)
    a, b = M.Engine(ctx, cfg, w), M.Engine(ctx, cfg, w)
    a.set_mfma(False)
    b.set_decode(False)
    ids = np.random.default_rng(7).integers(0, cfg.vocab, 120)
    pos = 0
    for m in (16, 5, 2, 9, 16, 3, 1, 12, 16, 7):
        am0, h0, l0 = a.forward(ids[pos:pos + m], pos, hidden=True, logits=True)
        am1, h1, l1 = b.forward(ids[pos:pos + m], pos, hidden=True, logits=True)
        assert _same(h0, h1), (case, m, pos, "hidden")
        assert _same(l0, l1), (case, m, pos, "logits")
        assert np.array_equal(am0, am1), (case, m, pos)
        if cfg.moe:
            assert np.array_equal(a.last_experts(), b.last_experts()), (case, m, pos)
        pos += m
    ka, va = a.kv_cache()
    kb, vb = b.kv_cache()
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    a.close()
    b.close()


def _rel(a, b):
    return float(np.max(np.abs(a.astype(np.float64) - b.astype(np.float64))) / max(1e-30, float(np.max(np.abs(b)))))


def _margin(logits):
    top = np.sort(logits.astype(np.float64))[-2:]
    return top[1] - top[0]


@pytest.mark.parametrize("case", list(CASES))
def test_multi_row_passes_mfma(ctx, case, monkeypatch):
    """Passes of 2..16 rows on the int8 matrix cores (the reference's eight lane classes kept apart,
    each with its fp32 chain; SPX_MQ_ROWS=2,...: every projection on the matrix cores from two
    rows, where the default takes them from a few rows more) against the lane-exact kernels: the
    same bits for every row (hidden state, logits, picks, routing statistics, KV cache),
    128-expert cases included; and so the same bits as one-row passes (the reference's batch
    invariance, quant_q8k.rs:413-442)."""
    cfg = CASES[case]
    w = M.synth_model(cfg, seed=35)
    monkeypatch.setenv("SPX_MQ_ROWS", "2,2,2,2,2")
    a = M.Engine(ctx, cfg, w)
    monkeypatch.delenv("SPX_MQ_ROWS")
    b = M.Engine(ctx, cfg, w)
    a.set_mfma(True)
    b.set_mfma(False)
    ids = np.random.default_rng(7).integers(0, cfg.vocab, 120)
    pos = 0
    for m in (16, 5, 2, 9, 16, 3, 12, 16, 7, 4, 11):
        am0, h0, l0 = a.forward(ids[pos:pos + m], pos, hidden=True, logits=True)
        am1, h1, l1 = b.forward(ids[pos:pos + m], pos, hidden=True, logits=True)
        assert _same(h0, h1), (case, m, pos, "hidden", _rel(h0, h1))
        assert _same(l0, l1), (case, m, pos, "logits", _rel(l0, l1))
        assert np.array_equal(am0, am1), (case, m, pos)
        if cfg.moe:
            assert np.array_equal(a.last_experts(), b.last_experts()), (case, m, pos)
        pos += m
    ka, va = a.kv_cache()
    kb, vb = b.kv_cache()
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    a.close()
    b.close()


@pytest.mark.parametrize("case", list(CASES))
def test_persistent_pass_bitwise(ctx, case):
    """One-row passes with their layers as cooperative launches (persist.hip) against the decode
    pipeline's kernel sequence: the same bits for hidden state, logits, pick, KV cache rows and
    routing statistics, at contexts of one chunk, several, and (long cases) past 16 chunks."""
    cfg = CASES[case]
    long_ctx = case in LONG
    if long_ctx:
        cfg = cfg.replace(max_seq=1280)
    w = M.synth_model(cfg, seed=36)
    a, b = M.Engine(ctx, cfg, w), M.Engine(ctx, cfg, w)
    a.set_mfma(False)
    b.set_mfma(False)
    a.set_persist(True)
    assert a.persist_active(), case
    b.set_persist(False)
    assert not b.persist_active() and b.decode_pipeline()
    rng = np.random.default_rng(8)
    n_pre = 1100 if long_ctx else 150
    ids = rng.integers(0, cfg.vocab, n_pre + 40)
    checkpoints = [16, 70, 140] + ([1090] if long_ctx else [])
    pos = 0
    for cp in checkpoints:
        while pos < cp:
            m = min(16, cp - pos)
            a.forward(ids[pos:pos + m], pos)
            b.forward(ids[pos:pos + m], pos)
            pos += m
        for _ in range(3):
            am0, h0, l0 = a.forward(ids[pos:pos + 1], pos, hidden=True, logits=True)
            am1, h1, l1 = b.forward(ids[pos:pos + 1], pos, hidden=True, logits=True)
            assert _same(h0, h1), (case, pos, "hidden")
            assert _same(l0, l1), (case, pos, "logits")
            assert np.array_equal(am0, am1), (case, pos)
            if cfg.moe:
                assert np.array_equal(a.last_experts(), b.last_experts()), (case, pos)
            pos += 1
    # back-to-back decoding (the pick feeds the next pass on the device)
    got = a.decode(int(ids[pos]), pos, 12)
    want = b.decode(int(ids[pos]), pos, 12)
    assert got.tolist() == want.tolist(), case
    ka, va = a.kv_cache()
    kb, vb = b.kv_cache()
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    a.close()
    b.close()
