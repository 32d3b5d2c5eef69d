"""Multi-tile attention (launch_attention_mt: one workgroup per (64-position chunk, kv head) with a
wavefront per 16-query tile, then a merge launch a workgroup per 256 att values) against the
tile-per-workgroup kernel with its in-kernel merges (SPX_ATT_MT=0). Per (chunk, query) the
operations and their order are the same (the scores computed as K Q^T, the reductions as the
same butterflies), so the bar is bitwise: hidden states, logits, picks and the KV cache of
passes of 1..16 rows, on head_dim 64 and 128, NEOX and pairwise rotation, with and without
QK-norm, one and two merge levels (contexts past 16 chunks); and prefill passes of 17..128 rows
(SPX_PF_ATTN=2: the same kernels, a workgroup per 128 queries of a (chunk, kv head)) against
the prepared-rows prefill kernels (k_rows_prep + k_attn_pf)."""
import os

import numpy as np
import pytest

from spindle_amd import model as M

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

CASES = {
    "llama": M.TINY["tiny-llama"].replace(sigma=0.05),          # hd 64, 3 q heads / kv head, pairs, no QK-norm
    "granite": M.TINY["tiny-granite"].replace(sigma=0.05),      # hd 64, 2 / kv head, pairs, attention scale
    "qwen3": M.TINY["tiny-qwen3"].replace(sigma=0.05),          # hd 64, NEOX, QK-norm
    "qwen3moe": M.TINY["tiny-qwen3moe"].replace(sigma=0.05),    # hd 64, 4 / kv head, K-quant multi-row pipeline
    "a3b": M.TINY["tiny-a3b"].replace(sigma=0.05),              # hd 128, 8 / kv head, K-quant multi-row pipeline
}
SIZES = (9, 16, 2, 5, 1, 13, 3, 16, 8, 7, 11, 4, 16, 12, 6, 10, 15, 14, 1, 9)


@pytest.fixture(scope="module")
def ctx():
    from spindle_amd import ops
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    c = ops.Context(0)
    yield c
    c.close()


def _engine(ctx, cfg, w, mt, pf=None):
    env = {"SPX_ATT_MT": "1" if mt else "0"}  # read when the engine is created
    if pf is not None:
        env["SPX_PF_ATTN"] = str(pf)
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        return M.Engine(ctx, cfg, w)
    finally:
        for k, v in old.items():
            if v is None:
                del os.environ[k]
            else:
                os.environ[k] = v


def _same(a, b):
    return np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))


def _run(ctx, case, cfg, start, seed):
    w = M.synth_model(cfg, seed=seed)
    a, b = _engine(ctx, cfg, w, True), _engine(ctx, cfg, w, False)
    rng = np.random.default_rng(seed)
    pos = 0
    if start:  # a prompt in 128-row passes (the same prefill kernels in both engines)
        ids = rng.integers(0, cfg.vocab, start)
        for s0 in range(0, start, 128):
            n = min(128, start - s0)
            a.forward(ids[s0:s0 + n], s0)
            b.forward(ids[s0:s0 + n], s0)
        pos = start
    for m in SIZES:
        if pos + m > cfg.max_seq:
            break
        ids = rng.integers(0, cfg.vocab, m)
        print(f"{case}: pass of {m} rows at {pos}", flush=True)
        am0, h0, l0 = a.forward(ids, pos, hidden=True, logits=True)
        am1, h1, l1 = b.forward(ids, pos, hidden=True, logits=True)
        assert _same(h0, h1), (case, m, pos, "hidden")
        assert _same(l0, l1), (case, m, pos, "logits")
        assert np.array_equal(am0, am1), (case, m, pos)
        pos += m
    ka, va = a.kv_cache()
    kb, vb = b.kv_cache()
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    a.close()
    b.close()


@pytest.mark.parametrize("case", list(CASES))
def test_multi_tile_attention_bitwise(ctx, case):
    _run(ctx, case, CASES[case], 0, 61)


@pytest.mark.parametrize("case", ["a3b", "qwen3moe"])
def test_multi_tile_attention_two_merge_levels(ctx, case):
    """Passes after a prompt of more than 16 chunks (groups of 16 chunks, then the groups)."""
    _run(ctx, case, CASES[case].replace(max_seq=1280), 1070, 62)


def test_multi_tile_attention_lane_exact_verify(ctx):
    """On the lane-exact kernels a verify pass equals one-row decode passes bit for bit; with the
    multi-tile attention it still does (its partials are the one-row kernel's)."""
    cfg = CASES["a3b"]
    w = M.synth_model(cfg, seed=63)
    a = _engine(ctx, cfg, w, True)
    b = M.Engine(ctx, cfg, w)
    a.set_mfma(False)
    b.set_mfma(False)
    ids = np.random.default_rng(64).integers(0, cfg.vocab, 40)
    _, h0, l0 = a.forward(ids[:31], 0, hidden=True, logits=True)  # 16 + 15 rows
    hs, ls = [], []
    for p in range(31):
        _, h, l = b.forward(ids[p:p + 1], p, hidden=True, logits=True)
        hs.append(h)
        ls.append(l)
    assert _same(h0, np.concatenate(hs)) and _same(l0, np.concatenate(ls))
    a.close()
    b.close()


PF_CASES = ["a3b", "qwen3moe", "qwen3", "granite"]


@pytest.mark.parametrize("case", PF_CASES)
def test_multi_tile_prefill_bitwise(ctx, case):
    """Prefill passes on the multi-tile kernels against the prepared-rows prefill kernels (the
    K-quant pipelines) or 16-row passes (the fused path), bitwise, past 16 chunks."""
    cfg = CASES[case].replace(max_seq=1280)
    w = M.synth_model(cfg, seed=65)
    a, b = _engine(ctx, cfg, w, True, pf=2), _engine(ctx, cfg, w, True, pf=1)
    rng = np.random.default_rng(66)
    ids = rng.integers(0, cfg.vocab, 1200)
    pos = 0
    for m in (128, 17, 40, 128, 100, 128, 33, 128, 64, 128, 128, 90, 128):
        if pos + m > 1200:
            break
        print(f"{case}: prefill pass of {m} rows at {pos}", flush=True)
        am0, h0, l0 = a.forward(ids[pos:pos + m], pos, hidden=True, logits=True)
        am1, h1, l1 = b.forward(ids[pos:pos + m], pos, hidden=True, logits=True)
        assert _same(h0, h1), (case, m, pos, "hidden")
        assert _same(l0, l1), (case, m, pos, "logits")
        assert np.array_equal(am0, am1), (case, m, pos)
        pos += m
    ka, va = a.kv_cache()
    kb, vb = b.kv_cache()
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    a.close()
    b.close()


def test_multi_tile_attention_nine_groups(ctx):
    """Past 8192 positions (129+ chunks, nine chunk groups: the merge's slices take a second
    group each): verify passes and prefill passes against the earlier kernels, bitwise."""
    cfg = CASES["a3b"].replace(max_seq=8448)
    w = M.synth_model(cfg, seed=67)
    a, b = _engine(ctx, cfg, w, True, pf=2), _engine(ctx, cfg, w, False, pf=1)
    rng = np.random.default_rng(68)
    ids = rng.integers(0, cfg.vocab, 8300)
    for s0 in range(0, 8192, 128):
        a.forward(ids[s0:s0 + 128], s0)
        b.forward(ids[s0:s0 + 128], s0)
    pos = 8192
    for m in (9, 16, 2, 1, 128):
        print(f"pass of {m} rows at {pos}", flush=True)
        am0, h0, l0 = a.forward(ids[pos:pos + m], pos, hidden=True, logits=True)
        am1, h1, l1 = b.forward(ids[pos:pos + m], pos, hidden=True, logits=True)
        assert _same(h0, h1) and _same(l0, l1) and np.array_equal(am0, am1), (m, pos)
        pos += m
    a.close()
    b.close()
