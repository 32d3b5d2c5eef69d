"""Builds the oracle's CPU model (or_model) from the same tensors the GPU engine gets.

TEST INFRASTRUCTURE ONLY (tests/, smoke() and bench.py's cpu_baseline leg)."""
import ctypes as C

import numpy as np

from . import ffi


class OracleModel:
    def __init__(self, cfg, tensors):
        self.cfg = cfg
        self.keep = []
        self.tensors = tensors
        oc = ffi.Config(cfg.dim, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.n_layers, cfg.vocab, cfg.max_seq,
                        cfg.rope_theta, cfg.rms_eps, int(cfg.rope_neox), cfg.n_expert, cfg.n_expert_used,
                        int(cfg.expert_norm), cfg.moe_prune, cfg.embedding_scale, cfg.residual_scale,
                        cfg.logit_scale, cfg.attn_scale)
        layers = (ffi.Layer * cfg.n_layers)()
        for l in range(cfg.n_layers):
            p = f"blk.{l}."
            ly = layers[l]
            ly.attn_norm = self._vec(p + "attn_norm.weight")
            ly.ffn_norm = self._vec(p + "ffn_norm.weight")
            ly.wq, ly.wk, ly.wv, ly.wo = (self._mat(p + n) for n in ("attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_output.weight"))
            ly.q_norm = self._vec(p + "attn_q_norm.weight")
            ly.k_norm = self._vec(p + "attn_k_norm.weight")
            ly.q_bias = self._vec(p + "attn_q.bias")
            ly.k_bias = self._vec(p + "attn_k.bias")
            ly.v_bias = self._vec(p + "attn_v.bias")
            if (p + "ffn_gate_inp.weight") in tensors:
                ly.is_moe = 1
                ly.router = self._mat(p + "ffn_gate_inp.weight")
                ly.gate, ly.up, ly.down = (self._mat(p + n) for n in ("ffn_gate_exps.weight", "ffn_up_exps.weight", "ffn_down_exps.weight"))
            else:
                ly.gate, ly.up, ly.down = (self._mat(p + n) for n in ("ffn_gate.weight", "ffn_up.weight", "ffn_down.weight"))
        self.layers = layers
        n = cfg.n_layers * cfg.max_seq * cfg.kv_dim
        self.k_cache = np.zeros(n, np.uint16)
        self.v_cache = np.zeros(n, np.uint16)
        m = ffi.Model()
        m.c = oc
        m.layers = C.cast(layers, C.POINTER(ffi.Layer))
        m.embed = self._mat("token_embd.weight")
        m.lm_head = self._mat("output.weight") if "output.weight" in tensors else m.embed
        m.output_norm = self._vec("output_norm.weight")
        m.k_cache = self.k_cache.ctypes.data
        m.v_cache = self.v_cache.ctypes.data
        self.m = m
        ffi.lib.or_model_init(C.byref(m))

    def _vec(self, name):
        if name not in self.tensors:
            return None
        return self.tensors[name][1].ctypes.data

    def _mat(self, name):
        spec, data = self.tensors[name]
        return ffi.Mat(spec.dtype, spec.cols, spec.rows, data.ctypes.data)

    def forward(self, ids, start_pos):
        ids = np.ascontiguousarray(ids, np.int32)
        h = np.empty((ids.size, self.cfg.dim), np.float32)
        rc = ffi.lib.or_forward_batch(C.byref(self.m), ids.ctypes.data_as(C.c_void_p), ids.size, start_pos, h.ctypes.data_as(C.c_void_p))
        assert rc == 0
        return h

    def logits(self, hidden):
        hidden = np.ascontiguousarray(hidden, np.float32)
        out = np.empty((hidden.shape[0], self.cfg.vocab), np.float32)
        assert ffi.lib.or_logits(C.byref(self.m), hidden.ctypes.data_as(C.c_void_p), hidden.shape[0], out.ctypes.data_as(C.c_void_p)) == 0
        return out

    def argmax(self, logits):
        lg = np.ascontiguousarray(logits, np.float32)
        return ffi.lib.or_argmax(lg.ctypes.data_as(C.c_void_p), lg.size, self.cfg.logit_scale)

    def generate(self, prompt, max_new, draft_len=8, min_ngram=2, max_ngram=4, fixed=False, speculate=True,
                 adaptive_k=True, prefill_chunk=16, n_cached=0, sampler=None, kv_keep=0, draft=None):
        """sampler: an ffi.OracleSampler (its SplitMix64 state advances), or None for greedy;
        draft: an OracleModel drafting instead of the prompt lookup."""
        prompt = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(max_new, np.int32)
        gp = ffi.GenParams(draft_len, min_ngram, max_ngram, int(fixed), int(speculate), int(adaptive_k), prefill_chunk, n_cached,
                           kv_keep)
        st = ffi.GenStats()
        if draft is not None:
            n = ffi.lib.or_generate_full(C.byref(self.m), C.byref(draft.m), prompt.ctypes.data_as(C.c_void_p), prompt.size, max_new,
                                         C.byref(gp), C.byref(sampler.s) if sampler is not None else None,
                                         out.ctypes.data_as(C.c_void_p), C.byref(st))
        elif sampler is not None:
            n = ffi.lib.or_generate_sampled(C.byref(self.m), prompt.ctypes.data_as(C.c_void_p), prompt.size, max_new,
                                            C.byref(gp), C.byref(sampler.s), out.ctypes.data_as(C.c_void_p), C.byref(st))
        else:
            n = ffi.lib.or_generate(C.byref(self.m), prompt.ctypes.data_as(C.c_void_p), prompt.size, max_new, C.byref(gp),
                                    out.ctypes.data_as(C.c_void_p), C.byref(st))
        assert n >= 0
        return out[:n], {k: getattr(st, k) for k, _ in ffi.GenStats._fields_}

    # ---- per-layer stages (the layer-by-layer parity tests feed these the GPU's own inputs)
    def layer_forward(self, layer, x, start):
        """One layer on x [n, dim] (a copy) at positions start..start+n-1: forward_slice's layer
        for n == 1, forward_batch_slice's for n > 1; writes the rows' K/V into the oracle's cache."""
        x = np.array(x, np.float32, copy=True, order="C")
        assert ffi.lib.or_layer_forward(C.byref(self.m), layer, x.shape[0], start, ffi.ptr(x)) == 0
        return x

    def attn_rows(self, layer, q, k, v, start):
        """qkv_post + attention of n rows from the raw projections (copies); returns att [n, q_dim]."""
        q, k, v = (np.array(a, np.float32, copy=True, order="C") for a in (q, k, v))
        att = np.empty_like(q)
        assert ffi.lib.or_attn_rows(C.byref(self.m), layer, q.shape[0], start, ffi.ptr(q), ffi.ptr(k), ffi.ptr(v), ffi.ptr(att)) == 0
        return att

    def norm(self, layer, which, x):
        """attn_norm ('attn') or ffn_norm ('ffn') of layer on one row x; 'out': output_norm."""
        if which == "out":
            w = self.m.output_norm
        else:
            ly = self.layers[layer]
            w = ly.attn_norm if which == "attn" else ly.ffn_norm
        out = np.empty(self.cfg.dim, np.float32)
        x = np.ascontiguousarray(x, np.float32)
        ffi.lib.or_rmsnorm(ffi.ptr(x), w, ffi.ptr(out), self.cfg.dim, self.cfg.rms_eps)
        return out

    def mat(self, layer, name):
        """The layer's matrix descriptor: wq, wk, wv, wo, gate, up, down, router."""
        return getattr(self.layers[layer], name)

    def moe_row(self, layer, xn):
        """moe_forward of one ffn-normed row (router, routing, ffns_fused): (out, chosen, h) with
        h the chosen experts' SwiGLU rows [keep, n_ff] in chosen order."""
        cfg = self.cfg
        ly = self.layers[layer]
        nff = ly.gate.rows
        h = np.full((cfg.n_expert_used, nff), np.nan, np.float32)
        out = np.empty(cfg.dim, np.float32)
        chosen = np.full(32, -1, np.int32)
        nkeep = np.zeros(1, np.int32)
        xn = np.ascontiguousarray(xn, np.float32)
        xs = (C.c_void_p * 1)(xn.ctypes.data)
        os_ = (C.c_void_p * 1)(out.ctypes.data)
        ffi.lib.or_set_dbg_h(ffi.ptr(h))
        try:
            assert ffi.lib.or_moe_forward(C.byref(self.m.c), C.byref(ly), 1, xs, os_, ffi.ptr(chosen), ffi.ptr(nkeep)) == 0
        finally:
            ffi.lib.or_set_dbg_h(None)
        k = int(nkeep[0])
        return out, chosen[:k].copy(), h[:k].copy()

    def down_combine(self, layer, chosen, weights, h):
        """The routed experts' down projections of the given SwiGLU rows h [k, n_ff] (Q8_K-quantized
        for an integer down) combined with the weights in chosen order, from zero."""
        ly = self.layers[layer]
        k = len(chosen)
        chosen = np.ascontiguousarray(chosen, np.int32)
        weights = np.ascontiguousarray(weights, np.float32)
        h = np.ascontiguousarray(h, np.float32)
        out = np.zeros(self.cfg.dim, np.float32)
        assert ffi.lib.or_down_combine(C.byref(ly.down), k, ffi.ptr(chosen), ffi.ptr(weights), ffi.ptr(h), ffi.ptr(out)) == 0
        return out

    def dense_row(self, layer, xn):
        """ffn_forward of one ffn-normed row (the fused job with k = 1, w = 1): (out, h) with h the
        SwiGLU row [1, n_ff]."""
        ly = self.layers[layer]
        h = np.full((1, ly.gate.rows), np.nan, np.float32)
        out = np.zeros(self.cfg.dim, np.float32)
        e0 = np.zeros(1, np.int32)
        w1 = np.ones(1, np.float32)
        xn = np.ascontiguousarray(xn, np.float32)
        ffi.lib.or_set_dbg_h(ffi.ptr(h))
        try:
            assert ffi.lib.or_ffns_fused(C.byref(ly.gate), C.byref(ly.up), C.byref(ly.down), 1, ffi.ptr(e0), ffi.ptr(w1),
                                         ffi.ptr(xn), ffi.ptr(out)) == 0
        finally:
            ffi.lib.or_set_dbg_h(None)
        return out, h
