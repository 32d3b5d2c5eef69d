"""ctypes binding of the CPU oracle (oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker or the timed CPU baseline. The product (spindle_amd/)
never imports it.
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "liboracle.so")

F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q4K, Q5K, Q6K, BF16 = 0, 1, 2, 3, 6, 7, 8, 12, 13, 14, 30
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), Q4_1: (32, 20), Q5_0: (32, 22),
         Q5_1: (32, 24), Q8_0: (32, 34), Q4K: (256, 144), Q5K: (256, 176), Q6K: (256, 210)}


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def _load():
    if not os.path.exists(LIB_PATH):
        build()
    return C.CDLL(LIB_PATH)


lib = _load()
P = C.c_void_p
fp = C.POINTER(C.c_float)


class Mat(C.Structure):
    _fields_ = [("dtype", C.c_int), ("cols", C.c_size_t), ("rows", C.c_size_t), ("data", P)]


class Config(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("dim", "n_heads", "n_kv_heads", "head_dim", "n_layers", "vocab", "max_seq")] + \
        [("rope_theta", C.c_float), ("rms_eps", C.c_float), ("rope_neox", C.c_int),
         ("n_expert", C.c_int), ("n_expert_used", C.c_int), ("expert_norm", C.c_int), ("moe_prune", C.c_float),
         ("embedding_scale", C.c_float), ("residual_scale", C.c_float), ("logit_scale", C.c_float),
         ("attn_scale", C.c_float)]


class Layer(C.Structure):
    _fields_ = [("attn_norm", P), ("ffn_norm", P), ("wq", Mat), ("wk", Mat), ("wv", Mat), ("wo", Mat),
                ("q_bias", P), ("k_bias", P), ("v_bias", P), ("q_norm", P), ("k_norm", P),
                ("qk_norm_full", C.c_int), ("is_moe", C.c_int),
                ("gate", Mat), ("up", Mat), ("down", Mat), ("router", Mat)]


class Model(C.Structure):
    _fields_ = [("c", Config), ("layers", C.POINTER(Layer)), ("embed", Mat), ("lm_head", Mat),
                ("output_norm", P), ("k_cache", P), ("v_cache", P), ("inv_freq", P),
                ("last_chosen", C.c_int * (16 * 32)),
                ("dbg_q", P), ("dbg_att", P), ("dbg_proj", P), ("dbg_ffn", P)]


class SpecModel(C.Structure):
    _fields_ = [("acc", C.c_double * 4), ("fail", C.c_double * 4), ("t1_us", C.c_double), ("extra_us", C.c_double),
                ("have_t1", C.c_int), ("have_extra", C.c_int), ("since_try", C.c_int), ("fixed", C.c_int)]


class GenParams(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("draft_len", "min_ngram", "max_ngram", "fixed", "speculate", "adaptive_k", "prefill_chunk", "n_cached",
                                       "kv_keep")]


class SamplerParams(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int), ("top_p", C.c_float), ("min_p", C.c_float),
                ("repeat_penalty", C.c_float), ("seed", C.c_uint64), ("stop_ids", C.POINTER(C.c_int)),
                ("n_stop", C.c_int), ("think_open", C.c_int)]


class Sampler(C.Structure):
    _fields_ = [("p", SamplerParams), ("rng", C.c_uint64)]


class GenStats(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("accepted", "drafted", "verifies", "steps")]


def _sig(name, res, *args):
    f = getattr(lib, name)
    f.restype = res
    f.argtypes = list(args)
    return f


_sig("or_row_bytes", C.c_size_t, C.c_int, C.c_size_t)
_sig("or_f16_to_f32", C.c_float, C.c_uint16)
_sig("or_f32_to_f16", C.c_uint16, C.c_float)
_sig("or_unpack_q4k_scales", None, P, P, P)
_sig("or_dequant_row", C.c_int, C.c_int, P, C.c_size_t, P)
_sig("or_q8k_quantize", None, P, C.c_size_t, P, P, P)
_sig("or_q8k_matmul_rows", None, P, C.c_int, C.c_size_t, C.c_int, P, P, P, P, C.c_size_t, C.c_size_t)
_sig("or_q8k_block_sums", None, P, C.c_int, C.c_size_t, P, P, P, P, P)
_sig("or_matvec_rows", C.c_int, P, C.c_int, C.c_size_t, P, P, C.c_size_t, C.c_size_t)
_sig("or_matmul_rows_multi", C.c_int, P, C.c_int, C.c_size_t, C.c_int, P, P, C.c_size_t, C.c_size_t)
_sig("or_matvec", C.c_int, C.POINTER(Mat), P, P)
_sig("or_matvec_multi", C.c_int, C.POINTER(Mat), C.c_int, P, P)
_sig("or_rmsnorm", None, P, P, P, C.c_size_t, C.c_float)
_sig("or_rmsnorm_heads", None, P, P, C.c_size_t, C.c_size_t, C.c_float)
_sig("or_silu", C.c_float, C.c_float)
_sig("or_rope_inv_freq", None, C.c_size_t, C.c_float, P)
_sig("or_rope_rotate", None, P, C.c_int, P, C.c_size_t, C.c_size_t, C.c_float)
_sig("or_model_init", None, C.POINTER(Model))
_sig("or_forward_slice", C.c_int, C.POINTER(Model), C.c_int, C.c_int, P)
_sig("or_forward_batch", C.c_int, C.POINTER(Model), P, C.c_int, C.c_int, P)
_sig("or_attn_rows", C.c_int, C.POINTER(Model), C.c_int, C.c_int, C.c_int, P, P, P, P)
_sig("or_layer_forward", C.c_int, C.POINTER(Model), C.c_int, C.c_int, C.c_int, P)
_sig("or_down_combine", C.c_int, C.POINTER(Mat), C.c_int, P, P, P, P)
_sig("or_set_dbg_h", None, P)
_sig("or_logits", C.c_int, C.POINTER(Model), P, C.c_int, P)
_sig("or_argmax", C.c_int, P, C.c_int, C.c_float)
_sig("or_moe_forward", C.c_int, C.POINTER(Config), C.POINTER(Layer), C.c_int, P, P, P, P)
_sig("or_ffns_fused", C.c_int, C.POINTER(Mat), C.POINTER(Mat), C.POINTER(Mat), C.c_int, P, P, P, P)
_sig("or_lookup_draft", C.c_int, P, C.c_int, C.c_int, P, C.c_int, C.c_int, C.c_int, P, P)
_sig("or_spec_init", None, C.POINTER(SpecModel), C.c_int)
_sig("or_spec_class", C.c_int, C.c_int)
_sig("or_spec_accept_rate", C.c_double, C.POINTER(SpecModel), C.c_int)
_sig("or_spec_best_len", C.c_int, C.POINTER(SpecModel), C.c_int, C.c_int)
_sig("or_spec_reset_rates", None, C.POINTER(SpecModel))
_sig("or_spec_record_draft", None, C.POINTER(SpecModel), C.c_int, C.c_int, C.c_int)
_sig("or_spec_record_step", None, C.POINTER(SpecModel), C.c_uint64)
_sig("or_spec_record_verify", None, C.POINTER(SpecModel), C.c_int, C.c_uint64)
_sig("or_generate", C.c_int, C.POINTER(Model), P, C.c_int, C.c_int, C.POINTER(GenParams), P, C.POINTER(GenStats))
_sig("or_generate_sampled", C.c_int, C.POINTER(Model), P, C.c_int, C.c_int, C.POINTER(GenParams), C.POINTER(Sampler), P, C.POINTER(GenStats))
_sig("or_generate_full", C.c_int, C.POINTER(Model), C.POINTER(Model), P, C.c_int, C.c_int, C.POINTER(GenParams), C.POINTER(Sampler), P,
     C.POINTER(GenStats))
_sig("or_sampler_init", None, C.POINTER(Sampler), C.POINTER(SamplerParams))
_sig("or_splitmix_next", C.c_uint64, C.POINTER(C.c_uint64))
_sig("or_splitmix_f32", C.c_float, C.POINTER(C.c_uint64))
_sig("or_sample", C.c_int, C.POINTER(Sampler), P, C.c_int, C.c_float, P, C.c_int, C.c_int, C.c_int)
_sig("or_shift_kv", C.c_int, P, P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, P, C.c_int, C.c_int, C.c_int)
_sig("or_ensure_kv_room", C.c_int, C.POINTER(Model), C.c_int, C.c_int, C.c_int)
_sig("or_set_threads", None, C.c_int)
_sig("or_set_simd", None, C.c_int)
_sig("or_set_norm_order", None, C.c_int)
_sig("or_get_threads", C.c_int)


def ptr(a):
    return a.ctypes.data_as(P) if a is not None else None


def row_bytes(dtype, cols):
    return lib.or_row_bytes(dtype, cols)


def dequant_row(dtype, row, cols):
    out = np.empty(cols, np.float32)
    assert lib.or_dequant_row(dtype, ptr(row), cols, ptr(out)) == 0
    return out


def dequant(dtype, data, rows, cols):
    rb = row_bytes(dtype, cols)
    return np.stack([dequant_row(dtype, data[r * rb:(r + 1) * rb], cols) for r in range(rows)])


def q8k_quantize(x):
    x = np.ascontiguousarray(x, np.float32)
    n = x.size
    d = np.empty(n // 256, np.float32)
    qs = np.empty(n, np.int8)
    bs = np.empty(n // 16, np.int16)
    lib.or_q8k_quantize(ptr(x), n, ptr(d), ptr(qs), ptr(bs))
    return d, qs, bs


def _parr(arrs):
    return (P * len(arrs))(*[a.ctypes.data for a in arrs])


def q8k_matmul_rows(data, dtype, cols, qs_list, rows, r0=0, r1=None, outs=None):
    r1 = rows if r1 is None else r1
    if outs is None:
        outs = [np.full(rows, np.nan, np.float32) for _ in qs_list]
    lib.or_q8k_matmul_rows(ptr(data), dtype, cols, len(qs_list), _parr([q[0] for q in qs_list]),
                           _parr([q[1] for q in qs_list]), _parr([q[2] for q in qs_list]), _parr(outs), r0, r1)
    return outs


def q8k_block_sums(row, dtype, cols, q):
    nb = cols // 256
    s = np.empty(nb, np.int32)
    c = np.empty(nb, np.int32)
    lanes = np.empty(nb * 8, np.int32)
    lib.or_q8k_block_sums(ptr(row), dtype, cols, ptr(q[1]), ptr(q[2]), ptr(s), ptr(c), ptr(lanes))
    return s, c, lanes.reshape(nb, 8)


def matvec_rows(data, dtype, cols, x, r0, nrows):
    out = np.empty(nrows, np.float32)
    assert lib.or_matvec_rows(ptr(data), dtype, cols, ptr(x), ptr(out), r0, nrows) == 0
    return out


def matmul_rows_multi(data, dtype, cols, xs, rows, r0=0, r1=None, outs=None):
    r1 = rows if r1 is None else r1
    if outs is None:
        outs = [np.full(rows, np.nan, np.float32) for _ in xs]
    assert lib.or_matmul_rows_multi(ptr(data), dtype, cols, len(xs), _parr(xs), _parr(outs), r0, r1) == 0
    return outs


def mat(dtype, data, rows, cols):
    return Mat(dtype, cols, rows, data.ctypes.data)


def matvec(m, x):
    out = np.empty(m.rows, np.float32)
    assert lib.or_matvec(C.byref(m), ptr(x), ptr(out)) == 0
    return out


def matvec_multi(m, xs):
    outs = [np.empty(m.rows, np.float32) for _ in xs]
    assert lib.or_matvec_multi(C.byref(m), len(xs), _parr(xs), _parr(outs)) == 0
    return outs


class OracleSampler:
    """sample_from_logits with its SplitMix64 state (or_sample); keeps the stop-id array alive."""

    def __init__(self, temperature=0.6, top_k=40, top_p=0.9, min_p=0.05, repeat_penalty=1.1, seed=1,
                 stop_ids=(), think_open=-1):
        self._stop = (C.c_int * max(1, len(stop_ids)))(*stop_ids)
        self.params = SamplerParams(temperature, top_k, top_p, min_p, repeat_penalty, seed,
                                    C.cast(self._stop, C.POINTER(C.c_int)), len(stop_ids), think_open)
        self.s = Sampler()
        lib.or_sampler_init(C.byref(self.s), C.byref(self.params))

    def sample(self, logits, recent=(), forbid_stop=False, forbid_think=False, logit_scale=1.0):
        lg = np.ascontiguousarray(logits, np.float32)
        rc = np.ascontiguousarray(np.asarray(recent, np.int32).reshape(-1))
        return lib.or_sample(C.byref(self.s), ptr(lg), lg.size, logit_scale, ptr(rc) if rc.size else None, rc.size,
                             int(forbid_stop), int(forbid_think))


def shift_kv(k16, v16, n_layers, max_seq, kv_dim, head_dim, neox, theta, n_keep, n_discard, cur_pos):
    """shift_kv on uint16 (f16-bit) caches [n_layers][max_seq][kv_dim], in place; returns the new cur_pos."""
    inv = np.empty(head_dim // 2 + 1, np.float32)
    lib.or_rope_inv_freq(head_dim, theta, ptr(inv))
    return lib.or_shift_kv(ptr(k16), ptr(v16), n_layers, max_seq, kv_dim, head_dim, int(neox), ptr(inv), n_keep, n_discard, cur_pos)


def set_simd(on):
    """The AVX2 kernels (True, default) or the scalar restatement (False): the same bits."""
    lib.or_set_simd(int(bool(on)))


def set_threads(n):
    lib.or_set_threads(n)


def set_norm_order(gpu_order):
    """Test knob: RMSNorm sums in the GPU kernels' order (True) or the reference's (False)."""
    lib.or_set_norm_order(int(bool(gpu_order)))
