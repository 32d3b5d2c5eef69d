"""Model-level properties of the oracle (CPU): the reference's own invariants.

- qwen3_moe_batch_is_bitwise (smollm_chat.rs:4696-4736): on an all-K-quant MoE model the
  batched forward equals one-token steps bit for bit.
- batched_forward_matches_sequential (:4772-4796): relative L1 < 2e-3 on float-kernel models.
- prompt_lookup_speculation_is_exact (:4798-4825): spec on and off give the same reply.
"""
import numpy as np
import pytest

from spindle_amd import model as M
from oracle.model import OracleModel


def _seq(om, ids, start=0):
    return np.stack([om.forward([t], start + i)[0] for i, t in enumerate(ids)])


def test_moe_batch_is_bitwise():
    cfg = M.TINY["tiny-qwen3moe"]
    w = M.synth_model(cfg, seed=3)
    a, b = OracleModel(cfg, w), OracleModel(cfg, w)
    ids = [5, 77, 400, 12, 999, 3, 64]
    seq = _seq(a, ids)
    bat = b.forward(ids, 0)
    assert np.array_equal(seq.view(np.uint32), bat.view(np.uint32))


@pytest.mark.parametrize("name", ["tiny-llama", "tiny-qwen3", "tiny-granite"])
def test_batched_forward_matches_sequential(name):
    cfg = M.TINY[name]
    w = M.synth_model(cfg, seed=4)
    a, b = OracleModel(cfg, w), OracleModel(cfg, w)
    ids = [1, 2, 3, 50, 60, 70, 80, 90, 100, 110, 120, 130]
    seq = _seq(a, ids)
    bat = b.forward(ids, 0)
    for i in range(len(ids)):
        rel = np.abs(seq[i] - bat[i]).sum() / max(1e-6, np.abs(seq[i]).sum())
        assert rel < 2e-3, (i, rel)


@pytest.mark.parametrize("name", ["tiny-qwen3moe", "tiny-granite"])
def test_speculation_is_exact(name):
    cfg = M.TINY[name].replace(sigma=0.06)
    w = M.synth_model(cfg, seed=5)
    rng = np.random.default_rng(0)
    head = rng.integers(0, cfg.vocab, 24)
    prompt = np.concatenate([head, head[4:20], head[:12]])
    off, _ = OracleModel(cfg, w).generate(prompt, 40, speculate=False)
    on, st = OracleModel(cfg, w).generate(prompt, 40, draft_len=4, speculate=True)
    assert st["verifies"] > 0
    if name == "tiny-qwen3moe":   # integer kernels: verify rows are bitwise decode rows
        assert np.array_equal(off, on)


def test_draft_model_speculation():
    """generate_reply with a draft engine (:4244-4269): verification keeps the target's own
    greedy stream whatever the draft proposes; a draft identical to the target has every
    proposal accepted; a different draft model fewer."""
    cfg = M.TINY["tiny-qwen3"].replace(sigma=0.06)
    w = M.synth_model(cfg, seed=21)
    rng = np.random.default_rng(2)
    base = rng.integers(0, cfg.vocab, 20)
    prompt = np.concatenate([base, base]).astype(np.int32)
    plain, _ = OracleModel(cfg, w).generate(prompt, 40, speculate=False)
    same, st = OracleModel(cfg, w).generate(prompt, 40, draft_len=4, draft=OracleModel(cfg, w))
    assert np.array_equal(plain, same) and st["drafted"] > 0 and st["accepted"] == st["drafted"] and st["steps"] == 0
    other = OracleModel(cfg, M.synth_model(cfg, seed=22))
    diff, st2 = OracleModel(cfg, w).generate(prompt, 40, draft_len=4, draft=other)
    assert np.array_equal(plain, diff) and st2["accepted"] < st2["drafted"]


def test_layer_stages_compose_to_the_forward():
    """The per-layer entry points the layer-by-layer GPU tests feed with the GPU's own values:
    embedding + layer_forward over the layers + output_norm gives forward()'s hidden state bit for
    bit, and writes forward()'s KV rows (a 5-row batch); moe_row's SwiGLU rows through
    down_combine give moe_row's output (within 1e-5: the routing weights are recomputed here in
    numpy, not by the oracle's route())."""
    from oracle import ffi
    cfg = M.TINY["tiny-qwen3moe"]
    w = M.synth_model(cfg, seed=8)
    a, b = OracleModel(cfg, w), OracleModel(cfg, w)
    ids = np.array([5, 77, 400, 12, 999], np.int32)
    want = a.forward(ids, 3)
    emb, _ = w["token_embd.weight"]
    x = np.stack([ffi.dequant_row(emb.dtype, w["token_embd.weight"][1][t * ffi.row_bytes(emb.dtype, cfg.dim):(t + 1) * ffi.row_bytes(emb.dtype, cfg.dim)], cfg.dim)
                  for t in ids]) * np.float32(cfg.embedding_scale)
    for l in range(cfg.n_layers):
        x = b.layer_forward(l, x, 3)
    assert np.array_equal(a.k_cache, b.k_cache) and np.array_equal(a.v_cache, b.v_cache)
    onorm = w["output_norm.weight"][1]
    for r in range(len(ids)):
        h = np.empty(cfg.dim, np.float32)
        ffi.lib.or_rmsnorm(ffi.ptr(np.ascontiguousarray(x[r])), onorm.ctypes.data, ffi.ptr(h), cfg.dim, cfg.rms_eps)
        assert np.array_equal(h.view(np.uint32), want[r].view(np.uint32)), r
    xn = b.norm(0, "ffn", x[0])
    y, ch, hr = b.moe_row(0, xn)
    assert len(ch) == cfg.n_expert_used and np.isfinite(hr).all()
    # the routing weights as route() forms them: softmax over the router logits, renormalised
    rl = ffi.matvec(b.mat(0, "router"), xn).astype(np.float32)
    p = np.exp(rl - rl.max()).astype(np.float32)
    p = p / p.sum(dtype=np.float32)
    wts = (p[ch] / p[ch].sum(dtype=np.float32)) if cfg.expert_norm else p[ch]
    y2 = b.down_combine(0, ch, wts.astype(np.float32), hr)
    assert np.allclose(y2, y, rtol=1e-5, atol=1e-6 * float(np.abs(y).max()))
