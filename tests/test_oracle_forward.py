"""The oracle's whole forward pass pinned by an independent float64 restatement.

`Ref` below recomputes forward_slice (smollm_chat.rs:3364-3552) in numpy float64 straight from
the formulas, sharing nothing with oracle.c but the dequantized weights (or_dequant_row, pinned
by the known-answer blocks in test_oracle_formats.py): RMSNorm (:569-575), per-head q/k norm
(:577-584), RoPE in both pair layouts (Rope::rotate :1404-1419; NEOX for qwen archs :75-79),
grouped-query attention over an f16 KV cache with kv head h / (n_heads / n_kv) (:3456-3495),
plain softmax (the reference's online softmax is the same sum), the Granite scales (embedding,
residual, attention :3385-3387, :3518-3540), MoE routing (softmax, top-k with ties to the lower
index, both pruning rules, weight normalisation :1199-1239), SwiGLU (:586-588) and the weighted
combine. Matrices on the integer path (Q4_K / Q6_K) take their input through an 8-bit Q8_K
round trip restated here (quant_q8k.rs:84-121: d = amax/127, codes = rint(x * 127/amax)).

Bars: float-activation models (Q8_0) within 1e-3 of the oracle's logits (max-abs, normalised by
max |logit|; the north star's logits bar) — typically ~1e-7, except where a K or V value sits at
an f16 rounding boundary, so that the float32 and float64 rows are cached one f16 step apart
(2^-11 relative) and that element carries ~1e-4 into every later step; K-quant models within
2e-2 (the same for the 8-bit Q8_K codes of every integer-path input). A planted mistake in the
reference forward (kv head h % n_kv instead of h / hpk) must exceed the bar tenfold, so the
comparison does catch a wrong head mapping.
"""
import numpy as np
import pytest

from oracle import ffi
from oracle.model import OracleModel
from spindle_amd import model as M

Q4K, Q6K, Q8_0 = M.Q4K, M.Q6K, M.Q8_0


def _deq(spec, data):
    rows = spec.rows * spec.n_expert
    m = ffi.dequant(spec.dtype, data, rows, spec.cols).astype(np.float64)
    return m.reshape(spec.n_expert, spec.rows, spec.cols) if spec.n_expert > 1 else m


def _q8k_roundtrip(x):
    """Q8_K quantize + dequantize of a float vector (per 256 values)."""
    x32 = x.astype(np.float32).reshape(-1, 256)
    out = np.zeros_like(x32, dtype=np.float64)
    for b in range(x32.shape[0]):
        amax = np.float32(np.max(np.abs(x32[b])))
        if amax == 0 or not np.isfinite(amax):
            continue
        iscale = np.float32(127.0) / amax
        q = np.clip(np.rint(x32[b] * iscale), -128, 127)
        out[b] = q.astype(np.float64) * np.float64(np.float32(amax / np.float32(127.0)))
    return out.reshape(-1)


class Ref:
    """float64 forward of a synthetic model; kv_head(h) maps a query head to its kv head."""

    def __init__(self, cfg, w, kv_head=None):
        self.cfg = cfg
        self.W = {n: _deq(s, d) for n, (s, d) in w.items()}
        self.dt = {n: s.dtype for n, (s, d) in w.items()}
        hpk = cfg.n_heads // cfg.n_kv_heads
        self.kv_head = kv_head or (lambda h: h // hpk)
        self.K = np.zeros((cfg.n_layers, cfg.max_seq, cfg.kv_dim))
        self.V = np.zeros((cfg.n_layers, cfg.max_seq, cfg.kv_dim))
        hd = cfg.head_dim
        self.inv_freq = 1.0 / cfg.rope_theta ** (2.0 * np.arange(hd // 2) / hd)

    def mv(self, name, x, expert=None):
        W = self.W[name] if expert is None else self.W[name][expert]
        if self.dt[name] in (Q4K, Q6K):
            x = _q8k_roundtrip(x)
        return W @ x

    def norm(self, x, w):
        return x / np.sqrt(np.sum(x * x) / x.size + self.cfg.rms_eps) * w

    def rope(self, v, pos):
        hd, half = self.cfg.head_dim, self.cfg.head_dim // 2
        v = v.reshape(-1, hd).copy()
        ang = pos * self.inv_freq
        c, s = np.cos(ang), np.sin(ang)
        a = np.arange(half) if self.cfg.rope_neox else 2 * np.arange(half)
        b = a + half if self.cfg.rope_neox else a + 1
        x0, x1 = v[:, a].copy(), v[:, b].copy()
        v[:, a] = x0 * c - x1 * s
        v[:, b] = x0 * s + x1 * c
        return v.reshape(-1)

    def moe(self, l, xn):
        c = self.cfg
        p = f"blk.{l}."
        logits = self.W[p + "ffn_gate_inp.weight"] @ xn
        pr = np.exp(logits - logits.max())
        pr /= pr.sum()
        order = sorted(range(c.n_expert), key=lambda e: (-pr[e], e))[:c.n_expert_used]
        keep = c.n_expert_used
        if c.moe_prune > 0 and c.n_expert_used > 2:
            min_keep = max(2, c.n_expert_used // 2)
            if c.moe_prune >= 1:
                keep = min(max(int(c.moe_prune), min_keep), c.n_expert_used)
            else:
                target = sum(pr[e] for e in order) * (1 - c.moe_prune)
                k, cum = 0, 0.0
                while k < c.n_expert_used and (k < min_keep or cum < target):
                    cum += pr[order[k]]
                    k += 1
                keep = k
        chosen = order[:keep]
        wsum = sum(pr[e] for e in chosen)
        out = np.zeros(c.dim)
        for e in chosen:
            g = self.mv(p + "ffn_gate_exps.weight", xn, e)
            u = self.mv(p + "ffn_up_exps.weight", xn, e)
            h = g / (1 + np.exp(-g)) * u
            wt = pr[e] / wsum if c.expert_norm else pr[e]
            out += wt * self.mv(p + "ffn_down_exps.weight", h, e)
        return out

    def forward(self, tok, pos):
        c = self.cfg
        hd = c.head_dim
        x = self.W["token_embd.weight"][tok] * c.embedding_scale
        scale = c.attn_scale if c.attn_scale > 0 else 1.0 / np.sqrt(hd)
        for l in range(c.n_layers):
            p = f"blk.{l}."
            xn = self.norm(x, self.W[p + "attn_norm.weight"][0])
            q, k, v = (self.mv(p + n, xn) for n in ("attn_q.weight", "attn_k.weight", "attn_v.weight"))
            if c.qk_norm:
                q = np.concatenate([self.norm(h, self.W[p + "attn_q_norm.weight"][0]) for h in q.reshape(-1, hd)])
                k = np.concatenate([self.norm(h, self.W[p + "attn_k_norm.weight"][0]) for h in k.reshape(-1, hd)])
            q, k = self.rope(q, pos), self.rope(k, pos)
            self.K[l, pos] = k.astype(np.float16).astype(np.float64)  # the f16 cache (RNE)
            self.V[l, pos] = v.astype(np.float16).astype(np.float64)
            att = np.zeros(c.q_dim)
            for h in range(c.n_heads):
                kv = self.kv_head(h)
                Kh = self.K[l, :pos + 1, kv * hd:(kv + 1) * hd]
                Vh = self.V[l, :pos + 1, kv * hd:(kv + 1) * hd]
                s = Kh @ q[h * hd:(h + 1) * hd] * scale
                pr = np.exp(s - s.max())
                att[h * hd:(h + 1) * hd] = (pr / pr.sum()) @ Vh
            x = x + c.residual_scale * self.mv(p + "attn_output.weight", att)
            xn = self.norm(x, self.W[p + "ffn_norm.weight"][0])
            if c.moe:
                f = self.moe(l, xn)
            else:
                g = self.mv(p + "ffn_gate.weight", xn)
                u = self.mv(p + "ffn_up.weight", xn)
                f = self.mv(p + "ffn_down.weight", g / (1 + np.exp(-g)) * u)
            x = x + c.residual_scale * f
        return self.norm(x, self.W["output_norm.weight"][0])

    def logits(self, hidden):
        head = "output.weight" if "output.weight" in self.W else "token_embd.weight"
        return self.mv(head, hidden)


KQ = dict(t_embd=Q4K, t_q=Q4K, t_k=Q4K, t_v=Q6K, t_o=Q4K, t_gate=Q4K, t_up=Q4K, t_down=Q6K, t_out=Q6K)
MODELS = {
    # hd 64, hpk 3, pair RoPE
    "llama-hpk3": M.ModelConfig("llama-hpk3", "llama", 256, 2, 6, 2, 64, 512, 300, max_seq=64),
    # hd 128, hpk 8, NEOX RoPE, QK-norm
    "qwen3-hd128-hpk8": M.ModelConfig("qwen3-hd128-hpk8", "qwen3", 256, 2, 16, 2, 128, 512, 300, max_seq=64,
                                      rope_theta=1e6, rms_eps=1e-6, qk_norm=True),
    # hd 64, hpk 1, Granite scales, MoE 8 experts top-4 (no pruning / top-2 / mass rule)
    "granite-hpk1": M.ModelConfig("granite-hpk1", "granitemoe", 256, 2, 4, 4, 64, 128, 300, max_seq=64, rms_eps=1e-6,
                                  n_expert=8, n_expert_used=4, embedding_scale=12.0, residual_scale=0.22,
                                  logit_scale=6.0, attn_scale=0.03),
    "granite-prune2": M.ModelConfig("granite-prune2", "granitemoe", 256, 2, 4, 4, 64, 128, 300, max_seq=64, rms_eps=1e-6,
                                    n_expert=8, n_expert_used=4, moe_prune=2.0, embedding_scale=12.0,
                                    residual_scale=0.22, logit_scale=6.0, attn_scale=0.03),
    "granite-prune-mass": M.ModelConfig("granite-prune-mass", "granitemoe", 256, 2, 4, 4, 64, 128, 300, max_seq=64,
                                        rms_eps=1e-6, n_expert=8, n_expert_used=4, moe_prune=0.4, embedding_scale=12.0,
                                        residual_scale=0.22, logit_scale=6.0, attn_scale=0.03),
    # the integer path: hd 128, hpk 8, 16 experts top-4, Q4_K_M formats
    "qwen3moe-kquant": M.ModelConfig("qwen3moe-kquant", "qwen3moe", 512, 2, 16, 2, 128, 256, 300, max_seq=64,
                                     rope_theta=1e6, rms_eps=1e-6, qk_norm=True, n_expert=16, n_expert_used=4,
                                     tied=False, **KQ),
}


def _err(a, b):
    return float(np.max(np.abs(a - b)) / max(1e-30, float(np.max(np.abs(b)))))


def _bar(cfg):
    return 2e-2 if cfg.t_q in (Q4K, Q6K) else 1e-3


def _run(cfg, w, steps, kv_head=None):
    ref = Ref(cfg, w, kv_head)
    om = OracleModel(cfg, w)
    ids = np.random.default_rng(3).integers(0, cfg.vocab, steps)
    errs = []
    for pos, t in enumerate(ids):
        lo = om.logits(om.forward([t], pos))[0].astype(np.float64)
        lr = ref.logits(ref.forward(int(t), pos))
        errs.append(_err(lo, lr))
    return errs, ids


@pytest.mark.parametrize("name", list(MODELS))
def test_oracle_forward_matches_float64(name):
    cfg = MODELS[name].replace(sigma=0.05)
    w = M.synth_model(cfg, seed=17)
    errs, _ = _run(cfg, w, 12)
    print(f"{name}: logits err vs float64 median {np.median(errs):.1e} max {max(errs):.1e}")
    assert max(errs) <= _bar(cfg), errs


@pytest.mark.parametrize("name", ["llama-hpk3", "qwen3-hd128-hpk8", "qwen3moe-kquant"])
def test_planted_head_mapping_mistake_is_caught(name):
    """kv head h % n_kv instead of h / hpk: the comparison fails by far more than its bar."""
    cfg = MODELS[name].replace(sigma=0.05)
    w = M.synth_model(cfg, seed=17)
    errs, _ = _run(cfg, w, 8, kv_head=lambda h: h % cfg.n_kv_heads)
    assert max(errs) > 10 * _bar(cfg), errs


def test_batched_pass_matches_float64():
    """forward_batch_slice (:3142-3362): rows of one pass see their own and earlier positions
    only; the oracle's batched pass against the float64 forward run row by row."""
    cfg = MODELS["qwen3-hd128-hpk8"].replace(sigma=0.05)
    w = M.synth_model(cfg, seed=18)
    ref = Ref(cfg, w)
    om = OracleModel(cfg, w)
    ids = np.random.default_rng(4).integers(0, cfg.vocab, 14)
    om.forward(ids[:5], 0)
    for p in range(5):
        ref.forward(int(ids[p]), p)
    lo = om.logits(om.forward(ids[5:14], 5)).astype(np.float64)
    for i in range(9):
        lr = ref.logits(ref.forward(int(ids[5 + i]), 5 + i))
        assert _err(lo[i], lr) <= _bar(cfg), i
