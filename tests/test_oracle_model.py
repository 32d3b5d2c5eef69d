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
