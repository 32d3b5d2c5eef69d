"""The KV window on the GPU (spx_engine_shift_kv / spx_engine_ensure_kv_room, shift_kv and
ensure_kv_room smollm_chat.rs:2924-2971): the slid caches bit for bit against the oracle's
shift of the same caches, and generation through a window smaller than the reply."""
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


@pytest.mark.parametrize("name", ["tiny-llama", "tiny-qwen3", "tiny-a3b"])
@pytest.mark.parametrize("keep,disc", [(0, 40), (7, 30), (7, 200)])
def test_shift_matches_oracle(ctx, name, keep, disc):
    from spindle_amd import model as M
    cfg = M.TINY[name].replace(max_seq=160)
    eng = M.Engine(ctx, cfg, M.synth_model(cfg, seed=4))
    ids = np.random.default_rng(1).integers(0, cfg.vocab, 112).astype(np.int32)
    for s in range(0, 112, 16):
        eng.forward(ids[s:s + 16], s)
    k0, v0 = eng.kv_download()
    new = eng.shift_kv(keep, disc, 112)
    k1, v1 = eng.kv_download()
    kw, vw = k0.copy(), v0.copy()
    want = ffi.shift_kv(kw, vw, cfg.n_layers, cfg.max_seq, cfg.kv_dim, cfg.head_dim, cfg.rope_neox, cfg.rope_theta, keep, disc, 112)
    assert new == want == 112 - min(disc, 112 - keep)
    assert np.array_equal(k1, kw) and np.array_equal(v1, vw)
    eng.close()


def _manual(eng, prompt, max_new, keep):
    """generate's plain greedy loop rebuilt from forward / ensure_kv_room calls."""
    pos = 0
    for s in range(0, len(prompt), 16):
        pos = eng.ensure_kv_room(keep, pos, len(prompt[s:s + 16]))
        am, _, _ = eng.forward(prompt[s:s + 16], pos)
        pos += len(prompt[s:s + 16])
    out, tok = [], int(am[-1])
    while True:
        out.append(tok)
        if len(out) >= max_new:
            return out
        pos = eng.ensure_kv_room(keep, pos, 1)
        tok = int(eng.forward([tok], pos)[0][0])
        pos += 1


@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-qwen3moe"])
def test_generate_through_a_sliding_window(ctx, name):
    """A reply longer than the window: spx_engine_generate slides where ensure_kv_room says
    (prefill chunks, then every step), token for token as the same loop over forward and
    ensure_kv_room; with speculation the reply stays within the window rules too."""
    from spindle_amd import model as M
    cfg = M.TINY[name].replace(max_seq=96)
    w = M.synth_model(cfg, seed=6)
    eng = M.Engine(ctx, cfg, w)
    eng.set_mfma(False)
    rng = np.random.default_rng(2)
    base = rng.integers(0, cfg.vocab, 20)
    prompt = np.concatenate([base, base, base[:14]]).astype(np.int32)
    g, st = eng.generate(prompt, 120, speculate=False, kv_keep=8)
    assert g.tolist() == _manual(eng, prompt, 120, 8)
    gs, st2 = eng.generate(prompt, 120, draft_len=4, speculate=True, kv_keep=8)
    assert len(gs) == 120 and st2["verifies"] > 0
    if name == "tiny-qwen3":  # float activations: logits ~1e-6 from the oracle's
        o, _ = OracleModel(cfg, w).generate(prompt, 120, speculate=False, kv_keep=8)
        n = int(np.argmax(g != o)) if not np.array_equal(g, o) else len(g)
        assert n >= 60, (n, g[:n + 2], o[:n + 2])  # the same stream through two slides at least
    eng.close()
