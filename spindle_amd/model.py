"""Model configurations, seeded synthetic weights and the engine wrapper.

`Engine` mirrors the reference engine's hot API (SmolLm2Engine, smollm_chat.rs:1574-1668):
forward_slice / forward_batch_slice (:3364, :3142) return final hidden states, `logits`
and `argmax` the LM head output and greedy pick (:3560-3671), `generate` the speculative
greedy loop of generate_reply (:4205-4348). Compute runs in libspx.so on the GPU.

Synthetic models follow BASELINE.json's configs: random-init weights in GGUF block layout
with the dtypes of a Q4_K_M / Q8_0 file, generated from a seed by spx_synth_tensor.
"""
import ctypes as C
import dataclasses
import zlib

import numpy as np

from ._lib import P, check, lib, load

F32, F16, Q5_0, Q8_0, Q4K, Q5K, Q6K = 0, 1, 6, 8, 12, 13, 14
BLOCK = {F32: (1, 4), F16: (1, 2), Q5_0: (32, 22), Q8_0: (32, 34), Q4K: (256, 144), Q5K: (256, 176), Q6K: (256, 210)}


def row_bytes(dtype, cols):
    b, s = BLOCK[dtype]
    assert cols % b == 0, (dtype, cols)
    return cols // b * s


@dataclasses.dataclass
class ModelConfig:
    """ModelConfig (smollm_chat.rs:38-120) plus the tensor dtypes of the synthetic file."""
    name: str
    arch: str
    dim: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    n_ff: int
    vocab: int
    max_seq: int = 4096
    rope_theta: float = 10000.0
    rms_eps: float = 1e-5
    qk_norm: bool = False
    n_expert: int = 0
    n_expert_used: int = 0
    expert_norm: bool = True
    moe_prune: float = 0.0
    embedding_scale: float = 1.0
    residual_scale: float = 1.0
    logit_scale: float = 1.0
    attn_scale: float = 0.0
    tied: bool = True
    # dtypes
    t_embd: int = Q8_0
    t_q: int = Q8_0
    t_k: int = Q8_0
    t_v: int = Q8_0
    t_o: int = Q8_0
    t_gate: int = Q8_0
    t_up: int = Q8_0
    t_down: int = Q8_0
    t_out: int = Q8_0
    sigma: float = 0.02

    @property
    def rope_neox(self):
        return self.arch in ("qwen2", "qwen2moe", "qwen3", "qwen3moe", "olmoe")

    @property
    def q_dim(self):
        return self.n_heads * self.head_dim

    @property
    def kv_dim(self):
        return self.n_kv_heads * self.head_dim

    @property
    def moe(self):
        return self.n_expert > 0

    def replace(self, **kw):
        return dataclasses.replace(self, **kw)


# BASELINE.json configs (random-init weights; shapes as stated there). D4 of the survey:
# SmolLM2's 576-column tensors cannot be K-quants, so llama.cpp's Q5_0 / Q8_0 fallback applies.
CONFIGS = {
    "smollm2-135m": ModelConfig("smollm2-135m", "llama", 576, 30, 9, 3, 64, 1536, 49152, max_seq=4096,
                                t_embd=Q8_0, t_q=Q5_0, t_k=Q5_0, t_v=Q5_0, t_o=Q5_0, t_gate=Q5_0, t_up=Q5_0,
                                t_down=Q6K, t_out=Q8_0),
    "qwen3-0.6b": ModelConfig("qwen3-0.6b", "qwen3", 1024, 28, 16, 8, 128, 3072, 151936, max_seq=4096,
                              rope_theta=1e6, rms_eps=1e-6, qk_norm=True),
    "granite-1b-a400m": ModelConfig("granite-1b-a400m", "granitemoe", 1024, 24, 16, 8, 64, 512, 49155, max_seq=4096,
                                    rms_eps=1e-6, n_expert=32, n_expert_used=8, embedding_scale=12.0,
                                    residual_scale=0.22, logit_scale=6.0, attn_scale=0.015625),
    "qwen3-30b-a3b": ModelConfig("qwen3-30b-a3b", "qwen3moe", 2048, 48, 32, 4, 128, 768, 151936, max_seq=8448,
                                 rope_theta=1e6, rms_eps=1e-6, qk_norm=True, n_expert=128, n_expert_used=8,
                                 tied=False, t_embd=Q4K, t_q=Q4K, t_k=Q4K, t_v=Q6K, t_o=Q4K, t_gate=Q4K, t_up=Q4K,
                                 t_down=Q6K, t_out=Q6K),
}

# Small models of the same families for parity tests against the CPU oracle.
TINY = {
    "tiny-llama": ModelConfig("tiny-llama", "llama", 192, 2, 3, 1, 64, 512, 512, max_seq=256,
                              t_embd=Q8_0, t_q=Q5_0, t_k=Q5_0, t_v=Q5_0, t_o=Q5_0, t_gate=Q5_0, t_up=Q5_0,
                              t_down=Q6K, t_out=Q8_0),
    "tiny-qwen3": ModelConfig("tiny-qwen3", "qwen3", 256, 2, 4, 2, 64, 768, 1000, max_seq=256, rope_theta=1e6,
                              rms_eps=1e-6, qk_norm=True),
    "tiny-granite": ModelConfig("tiny-granite", "granitemoe", 256, 2, 4, 2, 64, 128, 777, max_seq=256, rms_eps=1e-6,
                                n_expert=8, n_expert_used=4, embedding_scale=12.0, residual_scale=0.22,
                                logit_scale=6.0, attn_scale=0.03),
    "tiny-q5k": ModelConfig("tiny-q5k", "qwen3", 256, 2, 4, 2, 64, 768, 1000, max_seq=256, rope_theta=1e6, rms_eps=1e-6,
                            qk_norm=True, t_embd=Q5K, t_q=Q5K, t_k=Q5K, t_v=Q5K, t_o=Q5K, t_gate=Q5K, t_up=Q5K, t_down=Q5K,
                            t_out=Q5K),
    "tiny-qwen3moe": ModelConfig("tiny-qwen3moe", "qwen3moe", 512, 3, 8, 2, 64, 256, 1000, max_seq=320,
                                 rope_theta=1e6, rms_eps=1e-6, qk_norm=True, n_expert=16, n_expert_used=4,
                                 tied=False, t_embd=Q4K, t_q=Q4K, t_k=Q4K, t_v=Q6K, t_o=Q4K, t_gate=Q4K,
                                 t_up=Q4K, t_down=Q6K, t_out=Q6K),
    # the headline kernels' shapes at small width: head_dim 128, 8 query heads a kv head, 128
    # experts top-8 (Qwen3-30B-A3B's attention tiles and routing), a context past 16 chunks
    "tiny-a3b": ModelConfig("tiny-a3b", "qwen3moe", 512, 2, 16, 2, 128, 256, 1000, max_seq=1280,
                            rope_theta=1e6, rms_eps=1e-6, qk_norm=True, n_expert=128, n_expert_used=8,
                            tied=False, t_embd=Q4K, t_q=Q4K, t_k=Q4K, t_v=Q6K, t_o=Q4K, t_gate=Q4K,
                            t_up=Q4K, t_down=Q6K, t_out=Q6K),
}


def get_config(name):
    return CONFIGS.get(name) or TINY[name]


@dataclasses.dataclass
class TensorSpec:
    name: str
    dtype: int
    cols: int
    rows: int
    n_expert: int = 1
    kind: int = 0       # 0 quantized weight, 1 F32 uniform, 2 F32 norm (1 + noise)
    sigma: float = 0.02

    @property
    def nbytes(self):
        return row_bytes(self.dtype, self.cols) * self.rows * self.n_expert


def tensor_specs(cfg):
    """GGUF tensor names and shapes of resolve_layers (smollm_chat.rs:214-284)."""
    s = []
    s.append(TensorSpec("token_embd.weight", cfg.t_embd, cfg.dim, cfg.vocab, sigma=cfg.sigma))
    if not cfg.tied:
        s.append(TensorSpec("output.weight", cfg.t_out, cfg.dim, cfg.vocab, sigma=cfg.sigma))
    s.append(TensorSpec("output_norm.weight", F32, cfg.dim, 1, kind=2, sigma=0.1))
    for l in range(cfg.n_layers):
        p = f"blk.{l}."
        s.append(TensorSpec(p + "attn_norm.weight", F32, cfg.dim, 1, kind=2, sigma=0.1))
        s.append(TensorSpec(p + "attn_q.weight", cfg.t_q, cfg.dim, cfg.q_dim, sigma=cfg.sigma))
        s.append(TensorSpec(p + "attn_k.weight", cfg.t_k, cfg.dim, cfg.kv_dim, sigma=cfg.sigma))
        s.append(TensorSpec(p + "attn_v.weight", cfg.t_v, cfg.dim, cfg.kv_dim, sigma=cfg.sigma))
        s.append(TensorSpec(p + "attn_output.weight", cfg.t_o, cfg.q_dim, cfg.dim, sigma=cfg.sigma))
        if cfg.qk_norm:
            s.append(TensorSpec(p + "attn_q_norm.weight", F32, cfg.head_dim, 1, kind=2, sigma=0.1))
            s.append(TensorSpec(p + "attn_k_norm.weight", F32, cfg.head_dim, 1, kind=2, sigma=0.1))
        s.append(TensorSpec(p + "ffn_norm.weight", F32, cfg.dim, 1, kind=2, sigma=0.1))
        if cfg.moe:
            s.append(TensorSpec(p + "ffn_gate_inp.weight", F32, cfg.dim, cfg.n_expert, kind=1, sigma=float(1.0 / np.sqrt(cfg.dim))))
            s.append(TensorSpec(p + "ffn_gate_exps.weight", cfg.t_gate, cfg.dim, cfg.n_ff, cfg.n_expert, sigma=cfg.sigma))
            s.append(TensorSpec(p + "ffn_up_exps.weight", cfg.t_up, cfg.dim, cfg.n_ff, cfg.n_expert, sigma=cfg.sigma))
            s.append(TensorSpec(p + "ffn_down_exps.weight", cfg.t_down, cfg.n_ff, cfg.dim, cfg.n_expert, sigma=cfg.sigma))
        else:
            s.append(TensorSpec(p + "ffn_gate.weight", cfg.t_gate, cfg.dim, cfg.n_ff, sigma=cfg.sigma))
            s.append(TensorSpec(p + "ffn_up.weight", cfg.t_up, cfg.dim, cfg.n_ff, sigma=cfg.sigma))
            s.append(TensorSpec(p + "ffn_down.weight", cfg.t_down, cfg.n_ff, cfg.dim, sigma=cfg.sigma))
    return s


def tensor_seed(seed, name):
    return (seed * 1000003 + zlib.crc32(name.encode())) & ((1 << 64) - 1)


def synth_tensor(spec, seed):
    out = np.empty(spec.nbytes, np.uint8)
    check(load().spx_synth_tensor(spec.dtype, spec.cols, spec.rows, spec.n_expert, tensor_seed(seed, spec.name),
                                  C.c_float(spec.sigma), spec.kind, out.ctypes.data_as(P)))
    return out


def synth_model(cfg, seed=1):
    """{name: (spec, uint8 array)} for every tensor of the synthetic model."""
    return {s.name: (s, synth_tensor(s, seed)) for s in tensor_specs(cfg)}


class ModelConfigC(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("dim", "n_heads", "n_kv_heads", "head_dim", "n_layers", "vocab", "max_seq")] + \
        [("rope_theta", C.c_float), ("rms_eps", C.c_float), ("rope_neox", C.c_int),
         ("n_expert", C.c_int), ("n_expert_used", C.c_int), ("expert_norm", C.c_int), ("moe_prune", C.c_float),
         ("embedding_scale", C.c_float), ("residual_scale", C.c_float), ("logit_scale", C.c_float),
         ("attn_scale", C.c_float)]


class GenParams(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("draft_len", "min_ngram", "max_ngram", "fixed", "speculate", "adaptive_k", "prefill_chunk", "n_cached",
                                       "kv_keep")]


class GenStats(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("accepted", "drafted", "verifies", "steps")] + \
        [(n, C.c_double) for n in ("prefill_us", "step_us", "verify_us")]


def config_c(cfg):
    return ModelConfigC(cfg.dim, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.n_layers, cfg.vocab, cfg.max_seq,
                        cfg.rope_theta, cfg.rms_eps, int(cfg.rope_neox), cfg.n_expert, cfg.n_expert_used,
                        int(cfg.expert_norm), cfg.moe_prune, cfg.embedding_scale, cfg.residual_scale,
                        cfg.logit_scale, cfg.attn_scale)


class Engine:
    """The GPU engine for one model (spx_engine)."""

    def __init__(self, ctx, cfg, tensors, graphs=True):
        self.ctx, self.cfg = ctx, cfg
        h = P()
        cc = config_c(cfg)
        check(lib.spx_engine_create(ctx.h, C.byref(cc), C.byref(h)))
        self.h = h
        for name, (spec, data) in tensors.items():
            check(lib.spx_engine_set_tensor(h, name.encode(), spec.dtype, spec.cols, spec.rows, spec.n_expert,
                                            data.ctypes.data_as(P)))
        check(lib.spx_engine_prepare(h))
        check(lib.spx_engine_set_graphs(h, int(graphs)))
        ctx.adopt(self)

    def set_decode(self, on):
        """One-token passes on the decode pipeline (True, the default) or the fused pass kernels."""
        check(lib.spx_engine_set_decode(self.h, int(on)))

    def set_mfma(self, on):
        """Passes of 2..16 rows on the int8 matrix cores (True, the default; block totals exact,
        fp32 sums to rounding) or on the lane-exact dot chains (False: the same bits as one-row
        passes)."""
        check(lib.spx_engine_set_mfma(self.h, int(on)))

    def set_persist(self, on):
        """One-row passes with each layer as one cooperative launch (True; where the model fits
        it) or as the decode pipeline's kernel sequence (False, the default); the same bits."""
        check(lib.spx_engine_set_persist(self.h, int(on)))

    def persist_active(self):
        """True when one-row passes run as the persistent pass."""
        v = C.c_int()
        check(lib.spx_engine_persist_active(self.h, C.byref(v)))
        return bool(v.value)

    def decode_pipeline(self):
        """True when one-token passes run on the decode pipeline."""
        v = C.c_int()
        check(lib.spx_engine_decode_pipeline(self.h, C.byref(v)))
        return bool(v.value)

    def forward(self, ids, start_pos, hidden=False, logits=False):
        """One pass; returns (argmax [m], hidden [m, dim] or None, logits [m, vocab] or None)."""
        ids = np.ascontiguousarray(ids, np.int32)
        m = ids.size
        am = np.empty(m, np.int32)
        hid = np.empty((m, self.cfg.dim), np.float32) if hidden else None
        lg = np.empty((m, self.cfg.vocab), np.float32) if logits else None
        check(lib.spx_engine_forward(self.h, ids.ctypes.data_as(P), m, start_pos,
                                     hid.ctypes.data_as(P) if hidden else None,
                                     lg.ctypes.data_as(P) if logits else None, am.ctypes.data_as(P)))
        return am, hid, lg

    def feed(self, ids, start_pos, hidden=False, logits=False):
        """feed (spx_engine_feed): the prompt in passes of up to 128 rows, logits for the last
        row only; returns (argmax of the last row, hidden [dim] or None, logits [vocab] or None)."""
        ids = np.ascontiguousarray(ids, np.int32)
        am = np.empty(1, np.int32)
        hid = np.empty(self.cfg.dim, np.float32) if hidden else None
        lg = np.empty(self.cfg.vocab, np.float32) if logits else None
        check(lib.spx_engine_feed(self.h, ids.ctypes.data_as(P), ids.size, start_pos,
                                  hid.ctypes.data_as(P) if hidden else None,
                                  lg.ctypes.data_as(P) if logits else None, am.ctypes.data_as(P)))
        return int(am[0]), hid, lg

    def forward_slice(self, token, pos):
        return self.forward([token], pos, hidden=True)[1][0]

    def forward_batch_slice(self, ids, start_pos):
        return self.forward(ids, start_pos, hidden=True)[1]

    def generate(self, prompt, max_new, draft_len=8, min_ngram=2, max_ngram=4, fixed=False, speculate=True,
                 adaptive_k=True, prefill_chunk=16, n_cached=0, kv_keep=0):
        prompt = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(max_new, np.int32)
        gp = GenParams(draft_len, min_ngram, max_ngram, int(fixed), int(speculate), int(adaptive_k), prefill_chunk, n_cached,
                       kv_keep)
        st = GenStats()
        n = lib.spx_engine_generate(self.h, prompt.ctypes.data_as(P), prompt.size, max_new, C.byref(gp),
                                    out.ctypes.data_as(P), C.byref(st))
        if n < 0:
            check(n)
        return out[:n], {k: getattr(st, k) for k, _ in GenStats._fields_}

    def attention(self, layer, q, k, v, start_pos):
        """The attention block for rows of projections q [m, q_dim], k / v [m, kv_dim] (float32
        cuda tensors) at start_pos..; writes their K / V to the cache; returns att [m, q_dim]."""
        import torch
        m = q.shape[0]
        att = torch.empty((m, self.cfg.q_dim), dtype=torch.float32, device=q.device)
        for t in (q, k, v):
            assert t.is_cuda and t.dtype == torch.float32 and t.is_contiguous()
        torch.cuda.synchronize()  # inputs written on torch's stream; the engine runs on its context's
        check(lib.spx_engine_attention(self.h, layer, P(q.data_ptr()), P(k.data_ptr()), P(v.data_ptr()), m, start_pos,
                                       P(att.data_ptr())))
        return att

    def shift_kv(self, n_keep, n_discard, cur_pos):
        """shift_kv: returns the next position."""
        v = C.c_int()
        check(lib.spx_engine_shift_kv(self.h, n_keep, n_discard, cur_pos, C.byref(v)))
        return v.value

    def ensure_kv_room(self, n_keep, cur_pos, needed):
        """ensure_kv_room: returns the next position."""
        v = C.c_int()
        check(lib.spx_engine_ensure_kv_room(self.h, n_keep, cur_pos, needed, C.byref(v)))
        return v.value

    def kv_download(self):
        """The f16 K and V caches as uint16 arrays [n_layers][max_seq][kv_dim]."""
        c = self.cfg
        k = np.empty((c.n_layers, c.max_seq, c.kv_dim), np.uint16)
        v = np.empty_like(k)
        check(lib.spx_engine_kv_download(self.h, k.ctypes.data_as(P), v.ctypes.data_as(P)))
        return k, v

    def set_draft(self, draft):
        """A draft-model Engine for generate() (None: prompt lookup)."""
        self._draft = draft  # kept alive while in use
        check(lib.spx_engine_set_draft(self.h, draft.h if draft is not None else None))

    def set_sampler(self, **kw):
        """The sampler generate() draws with (ops.sampler_params keywords: temperature, top_k,
        top_p, min_p, repeat_penalty, seed, stop_ids, think_open); no keywords: plain greedy."""
        from .ops import sampler_params
        if not kw:
            check(lib.spx_engine_set_sampler(self.h, None))
            return
        params, keep = sampler_params(**kw)
        check(lib.spx_engine_set_sampler(self.h, C.byref(params)))

    def decode(self, token, start_pos, n):
        """n greedy one-token passes starting with `token` at start_pos; returns the n picks."""
        out = np.empty(n, np.int32)
        check(lib.spx_engine_decode(self.h, int(token), start_pos, n, out.ctypes.data_as(P)))
        return out

    def profile(self, on):
        check(lib.spx_engine_profile(self.h, int(on)))

    def profile_read(self):
        """{kernel class: (launches, total_us, algorithmic bytes)} accumulated while profiling."""
        res = {}
        for cls in range(64):
            name = C.c_char_p()
            n = C.c_int64()
            us = C.c_double()
            by = C.c_double()
            if lib.spx_engine_profile_read(self.h, cls, C.byref(name), C.byref(n), C.byref(us), C.byref(by)) != 0:
                break
            res[name.value.decode()] = (n.value, us.value, by.value)
        return res

    LAYER_FIELDS = ("x_in", "q", "k", "v", "att", "proj", "x_mid", "rlog", "h", "chosen", "weights", "nkeep")

    def debug_layers(self, on):
        """Layer snapshots on (passes run eagerly and record each layer's values) or off."""
        check(lib.spx_engine_debug_layers(self.h, int(on)))

    def read_layers(self, m):
        """The last pass's layer snapshots (m rows): {field: array [n_layers + 1, m, len]}; x_in of
        layer n_layers is the final residual; chosen / nkeep as int32."""
        off = np.zeros(13, np.int64)
        check(lib.spx_engine_debug_layout(self.h, off.ctypes.data_as(P)))
        R, L = int(off[12]), self.cfg.n_layers + 1
        buf = np.empty(L * 16 * R, np.float32)
        check(lib.spx_engine_debug_read(self.h, b"layers", buf.ctypes.data_as(P), buf.nbytes))
        buf = buf.reshape(L, 16, R)[:, :m]
        out = {}
        for f, name in enumerate(self.LAYER_FIELDS):
            a = buf[:, :, off[f]:off[f + 1]]
            out[name] = a.view(np.int32).copy() if name in ("chosen", "nkeep") else a.copy()
        return out

    def debug_buf(self, name, n):
        """n float32 values of an engine work buffer after the last pass (synchronised): 'q', 'k',
        'v' (the last layer's raw projections [m, q_dim | kv_dim]), 'att' (its attention rows),
        'x', 'xn', 'proj', ..."""
        buf = np.empty(n, np.float32)
        check(lib.spx_engine_debug_read(self.h, name.encode(), buf.ctypes.data_as(P), buf.nbytes))
        return buf

    def last_experts(self):
        out = np.empty(self.cfg.n_layers, np.int32)
        check(lib.spx_engine_last_experts(self.h, out.ctypes.data_as(P)))
        return out

    def kv_cache(self):
        n = self.cfg.n_layers * self.cfg.max_seq * self.cfg.kv_dim
        k = np.empty(n, np.uint16)
        v = np.empty(n, np.uint16)
        check(lib.spx_engine_kv_download(self.h, k.ctypes.data_as(P), v.ctypes.data_as(P)))
        return k, v

    def close(self):
        if self.h and self.ctx.h:
            lib.spx_engine_destroy(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def lookup_draft(corpus, k, min_ngram=2, max_ngram=4, stop_ids=()):
    """lookup_draft (smollm_chat.rs:2982-3015) through the C ABI (host-only)."""
    c = np.ascontiguousarray(corpus, np.int32)
    st = np.ascontiguousarray(stop_ids, np.int32)
    d = np.empty(max(k, 1), np.int32)
    ng = C.c_int()
    n = load().spx_lookup_draft(c.ctypes.data_as(P), c.size, k, st.ctypes.data_as(P) if st.size else None, st.size,
                                min_ngram, max_ngram, d.ctypes.data_as(P), C.byref(ng))
    return d[:n].tolist(), ng.value
