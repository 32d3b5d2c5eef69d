"""spx_engine_attention (the attention block of forward_batch_slice smollm_chat.rs:3226-3300 /
forward_slice :3432-3470) against the engine's own passes (bit for bit: the same q / k / v
give the same att and cache rows) and against a float64 evaluation over the f16 cache."""
import numpy as np
import pytest

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


def _read(eng, what, shape):
    import ctypes as C
    from spindle_amd._lib import check, lib
    a = np.empty(shape, np.float32)
    check(lib.spx_engine_debug_read(eng.h, what.encode(), a.ctypes.data_as(C.c_void_p), a.nbytes))
    return a


@pytest.mark.parametrize("name", ["tiny-llama", "tiny-qwen3", "tiny-a3b"])
@pytest.mark.parametrize("m", [1, 5, 16])
def test_attention_matches_pass(ctx, name, m):
    from spindle_amd import model as M
    cfg = M.TINY[name]
    eng = M.Engine(ctx, cfg, M.synth_model(cfg, seed=5))
    ids = np.random.default_rng(m).integers(0, cfg.vocab, 80 + m).astype(np.int32)
    for s in range(0, 80, 16):
        eng.forward(ids[s:s + 16], s)
    eng.forward(ids[80:80 + m], 80)
    last = cfg.n_layers - 1
    q, k, v = (_read(eng, w, (m, d)) for w, d in (("q", cfg.q_dim), ("k", cfg.kv_dim), ("v", cfg.kv_dim)))
    att = _read(eng, "att", (m, cfg.q_dim))
    kc0, vc0 = eng.kv_download()
    got = eng.attention(last, *(torch.from_numpy(a).cuda() for a in (q, k, v)), 80).cpu().numpy()
    kc1, vc1 = eng.kv_download()
    assert np.array_equal(got.view(np.uint32), att.view(np.uint32))
    assert np.array_equal(kc0, kc1) and np.array_equal(vc0, vc1)
    eng.close()


def test_attention_float64(ctx):
    """tiny-llama (no biases or Q/K norms, pair RoPE): each head's softmax(q.K / sqrt(hd)) V over
    positions <= its row's, in float64 from the f16 cache the call leaves."""
    from spindle_amd import model as M
    cfg = M.TINY["tiny-llama"]
    eng = M.Engine(ctx, cfg, M.synth_model(cfg, seed=6))
    rng = np.random.default_rng(3)
    ids = rng.integers(0, cfg.vocab, 48).astype(np.int32)
    for s in range(0, 48, 16):
        eng.forward(ids[s:s + 16], s)
    m, start, hd = 6, 48, cfg.head_dim
    q = rng.standard_normal((m, cfg.q_dim)).astype(np.float32)
    k = rng.standard_normal((m, cfg.kv_dim)).astype(np.float32)
    v = rng.standard_normal((m, cfg.kv_dim)).astype(np.float32)
    got = eng.attention(0, *(torch.from_numpy(a).cuda() for a in (q, k, v)), start).cpu().numpy().astype(np.float64)
    kc, vc = eng.kv_download()
    K = kc[0].view(np.float16).astype(np.float64)
    V = vc[0].view(np.float16).astype(np.float64)
    inv = 1.0 / 10000.0 ** (np.arange(hd // 2) * 2.0 / hd)
    g = cfg.n_heads // cfg.n_kv_heads
    for b in range(m):
        pos = start + b
        ang = pos * inv
        for h in range(cfg.n_heads):
            x = q[b, h * hd:(h + 1) * hd].astype(np.float64)
            qr = x.copy()
            qr[0::2] = x[0::2] * np.cos(ang) - x[1::2] * np.sin(ang)
            qr[1::2] = x[0::2] * np.sin(ang) + x[1::2] * np.cos(ang)
            kh = h // g
            sc = K[:pos + 1, kh * hd:(kh + 1) * hd] @ qr / np.sqrt(hd)
            p = np.exp(sc - sc.max())
            want = p @ V[:pos + 1, kh * hd:(kh + 1) * hd] / p.sum()
            assert np.abs(got[b, h * hd:(h + 1) * hd] - want).max() <= 2e-4 * max(1.0, np.abs(want).max()), (b, h)
    eng.close()
