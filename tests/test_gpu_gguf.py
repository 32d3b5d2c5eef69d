"""The engine loaded from a GGUF file (spx_engine_load_gguf, SmolLm2Engine::load
smollm_chat.rs:1887-2154) against the engine built from the same tensors in memory: the same
logits bit for bit, and load_with_index_sharded's refusals."""
import numpy as np
import pytest

from spindle_amd import gguf as G
from spindle_amd import model as M
from spindle_amd._lib import SpxError

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


@pytest.mark.parametrize("name", ["tiny-llama", "tiny-granite", "tiny-qwen3moe"])
def test_gguf_engine_matches_in_memory_engine(ctx, tmp_path, name):
    cfg = M.TINY[name]
    w = M.synth_model(cfg, seed=8)
    path = str(tmp_path / "m.gguf")
    G.write_model(path, cfg, w, eos=3, alignment=64)
    ref = M.Engine(ctx, cfg, w)
    with G.GgufFile(path) as g:
        eng = G.load_engine(ctx, g, cfg=cfg)
        assert g.stop_ids() == [3]
    rng = np.random.default_rng(1)
    ids = rng.integers(0, cfg.vocab, 24).astype(np.int32)
    for s, n in [(0, 16), (16, 8)]:
        a0, _, l0 = ref.forward(ids[s:s + n], s, logits=True)
        a1, _, l1 = eng.forward(ids[s:s + n], s, logits=True)
        assert np.array_equal(a0, a1) and np.array_equal(l0.view(np.uint32), l1.view(np.uint32)), (name, s)
    t0, _ = ref.generate(ids[:20], 12)
    t1, _ = eng.generate(ids[:20], 12)
    assert np.array_equal(t0, t1)
    eng.close()
    ref.close()


@pytest.mark.parametrize("case,msg", [("shared", "shared experts"), ("mixtral", "Mixtral"),
                                      ("missing", "missing tensor"), ("no_counts", "expert_count")])
def test_gguf_refusals(ctx, tmp_path, case, msg):
    cfg = M.TINY["tiny-qwen3moe"]
    w = dict(M.synth_model(cfg, seed=8))
    spec, data = w["blk.1.ffn_gate_exps.weight"]
    if case == "shared":
        w["blk.1.ffn_gate_shexp.weight"] = (M.TensorSpec("blk.1.ffn_gate_shexp.weight", spec.dtype, spec.cols, spec.rows), data[:spec.nbytes // spec.n_expert])
    elif case == "mixtral":
        for k in ("blk.1.ffn_gate_inp.weight", "blk.1.ffn_gate_exps.weight", "blk.1.ffn_up_exps.weight", "blk.1.ffn_down_exps.weight"):
            del w[k]
        w["blk.1.ffn_gate.0.weight"] = (M.TensorSpec("blk.1.ffn_gate.0.weight", spec.dtype, spec.cols, spec.rows), data[:spec.nbytes // spec.n_expert])
    elif case == "missing":
        del w["blk.2.attn_v.weight"]
    path = str(tmp_path / "m.gguf")
    c = cfg.replace(n_expert=0, n_expert_used=0) if case == "no_counts" else cfg
    G.write_model(path, c, w)
    with G.GgufFile(path) as g:
        with pytest.raises(SpxError, match=msg):
            G.load_engine(ctx, g, cfg=cfg)
