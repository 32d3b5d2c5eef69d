"""GGUF v3 files: a writer for synthetic models and a reader over the C ABI.

`write_gguf` lays out a file the way llama.cpp does and the reference reads it
(GgufModelIndex::parse_file, gguf_loader.rs:142-247): header, metadata, tensor table, the data
section at the header's end rounded up to general.alignment (32 when absent), each tensor's
data at an offset aligned the same way. `write_model` writes a synthetic model with the
metadata ModelConfig::from_gguf reads (smollm_chat.rs:69-120) and resolve_layers' tensor names.
`GgufFile` opens a file with the C reader (spx_gguf_*), and `load_engine` builds the GPU engine
from it (spx_engine_load_gguf)."""
import ctypes as C
import struct

import numpy as np

from ._lib import P, check, lib

MAGIC = 0x46554747
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q", I64: "<q",
           F64: "<d"}


def _str(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(vtype, v):
    if vtype == STR:
        return _str(v)
    if vtype == ARR:
        elem, items = v
        out = struct.pack("<IQ", elem, len(items))
        if elem == STR:
            return out + b"".join(_str(x) for x in items)
        return out + b"".join(struct.pack(_SCALAR[elem], x) for x in items)
    return struct.pack(_SCALAR[vtype], v)


def write_gguf(path, metadata, tensors, alignment=None, version=3, alignment_type=U32):
    """metadata: [(key, type, value)] (arrays: (ARR, (elem_type, items))); tensors: [(name,
    ggml_type, dims, bytes)] with dims in GGUF order (dims[0] = columns). alignment: written as
    general.alignment (of alignment_type) when given. Returns the data section's offset."""
    meta = list(metadata)
    if alignment is not None:
        meta.append(("general.alignment", alignment_type, alignment))
    align = max(alignment, 32) if alignment is not None else 32
    head = struct.pack("<IIQQ", MAGIC, version, len(tensors), len(meta))
    head += b"".join(_str(k) + struct.pack("<I", t) + _value(t, v) for k, t, v in meta)
    offs, off = [], 0
    for _, _, _, data in tensors:
        offs.append(off)
        off = (off + len(data) + align - 1) // align * align
    for (name, dtype, dims, _), o in zip(tensors, offs):
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", dtype, o)
    data_off = (len(head) + align - 1) // align * align
    with open(path, "wb") as f:
        f.write(head + b"\0" * (data_off - len(head)))
        for (_, _, _, data), o in zip(tensors, offs):
            f.seek(data_off + o)
            f.write(np.ascontiguousarray(data).tobytes())
    return data_off


def model_metadata(cfg, vocab_tokens=None, eos=None):
    """The hyperparameter keys of Appendix-B files for a spindle_amd.model.ModelConfig."""
    a = cfg.arch
    m = [("general.architecture", STR, a), ("general.name", STR, cfg.name),
         (f"{a}.embedding_length", U32, cfg.dim), (f"{a}.block_count", U32, cfg.n_layers),
         (f"{a}.attention.head_count", U32, cfg.n_heads), (f"{a}.attention.head_count_kv", U32, cfg.n_kv_heads),
         (f"{a}.context_length", U32, cfg.max_seq), (f"{a}.rope.freq_base", F32, cfg.rope_theta),
         (f"{a}.attention.layer_norm_rms_epsilon", F32, cfg.rms_eps)]
    if cfg.head_dim != cfg.dim // cfg.n_heads:
        m.append((f"{a}.attention.key_length", U32, cfg.head_dim))
    if cfg.n_expert:
        m += [(f"{a}.expert_count", U32, cfg.n_expert), (f"{a}.expert_used_count", U32, cfg.n_expert_used),
              (f"{a}.expert_weights_norm", BOOL, bool(cfg.expert_norm))]
    if cfg.embedding_scale != 1.0:
        m.append((f"{a}.embedding_scale", F32, cfg.embedding_scale))
    if cfg.residual_scale != 1.0:
        m.append((f"{a}.residual_scale", F32, cfg.residual_scale))
    if cfg.logit_scale != 1.0:
        m.append((f"{a}.logit_scale", F32, cfg.logit_scale))
    if cfg.attn_scale:
        m.append((f"{a}.attention.scale", F32, cfg.attn_scale))
    tokens = vocab_tokens if vocab_tokens is not None else [f"<t{i}>" for i in range(cfg.vocab)]
    m.append(("tokenizer.ggml.tokens", ARR, (STR, tokens)))
    if eos is not None:
        m.append(("tokenizer.ggml.eos_token_id", U32, eos))
    return m


def write_model(path, cfg, weights, vocab_tokens=None, eos=None, alignment=None):
    """A synthetic model (spindle_amd.model.synth_model's {name: (spec, bytes)}) as a GGUF file."""
    tensors = []
    for name, (spec, data) in weights.items():
        dims = [spec.cols] if spec.rows == 1 and spec.n_expert == 1 and spec.dtype == F32 and name.endswith(("norm.weight", ".bias")) \
            else [spec.cols, spec.rows] + ([spec.n_expert] if spec.n_expert > 1 else [])
        tensors.append((name, spec.dtype, dims, data))
    return write_gguf(path, model_metadata(cfg, vocab_tokens, eos), tensors, alignment)


class GgufFile:
    """A GGUF file opened by the C reader (spx_gguf_open); needs no GPU."""

    def __init__(self, path):
        h = P()
        check(lib.spx_gguf_open(path.encode(), C.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            lib.spx_gguf_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def info(self):
        v, al, do, nt, nm = C.c_uint32(), C.c_uint64(), C.c_uint64(), C.c_int64(), C.c_int64()
        check(lib.spx_gguf_info(self.h, C.byref(v), C.byref(al), C.byref(do), C.byref(nt), C.byref(nm)))
        return dict(version=v.value, alignment=al.value, data_offset=do.value, n_tensors=nt.value, n_meta=nm.value)

    def tensor(self, i):
        name, dt, nd, off = C.c_char_p(), C.c_int(), C.c_int(), C.c_uint64()
        dims = (C.c_uint64 * 4)()
        check(lib.spx_gguf_tensor(self.h, i, C.byref(name), C.byref(dt), C.byref(nd), dims, C.byref(off)))
        return name.value.decode(), dt.value, list(dims[:nd.value]), off.value

    def find(self, name):
        return lib.spx_gguf_find(self.h, name.encode())

    def meta_type(self, key):
        return lib.spx_gguf_meta_type(self.h, key.encode())

    def meta(self, key):
        """A metadata value by its type: int, float, bool, str, or (elem_type, count) for arrays."""
        t, k = self.meta_type(key), key.encode()
        if t < 0:
            return None
        if t in (F32, F64):
            v = C.c_float()
            check(lib.spx_gguf_meta_f32(self.h, k, C.byref(v)))
            return v.value
        if t == BOOL:
            v = C.c_int()
            check(lib.spx_gguf_meta_bool(self.h, k, C.byref(v)))
            return bool(v.value)
        if t == STR:
            v = C.c_char_p()
            check(lib.spx_gguf_meta_str(self.h, k, C.byref(v)))
            return v.value.decode()
        if t == ARR:
            e, n = C.c_int(), C.c_uint64()
            check(lib.spx_gguf_meta_array(self.h, k, C.byref(e), C.byref(n)))
            return (e.value, n.value)
        v = C.c_uint64()
        if lib.spx_gguf_meta_index(self.h, k, C.byref(v)) != 0:
            return "negative"
        return v.value

    def vocab_size(self):
        return lib.spx_gguf_vocab_size(self.h)

    def token(self, i):
        s = lib.spx_gguf_token(self.h, i)
        return None if s is None else s.decode()

    def config(self):
        from .model import ModelConfigC
        c = ModelConfigC()
        check(lib.spx_gguf_config(self.h, C.byref(c)))
        return {n: getattr(c, n) for n, _ in ModelConfigC._fields_}

    def stop_ids(self):
        ids, n = (C.c_int32 * 16)(), C.c_int()
        check(lib.spx_gguf_stop_ids(self.h, ids, 16, C.byref(n)))
        return list(ids[:min(16, n.value)])

    def think_ids(self):
        a, b = C.c_int32(), C.c_int32()
        check(lib.spx_gguf_think_ids(self.h, C.byref(a), C.byref(b)))
        return a.value, b.value

    def check(self):
        check(lib.spx_gguf_check(self.h))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def load_engine(ctx, gguf, max_seq=0, moe_prune=0.0, cfg=None):
    """SmolLm2Engine::load onto the GPU: a spindle_amd.model.Engine over spx_engine_load_gguf.
    cfg: the spindle_amd.model.ModelConfig to attach (for its shapes); from the file if None."""
    from . import model as M
    h = P()
    check(lib.spx_engine_load_gguf(ctx.h, gguf.h, max_seq, C.c_float(moe_prune), C.byref(h)))
    eng = M.Engine.__new__(M.Engine)
    eng.ctx, eng.h = ctx, h
    if cfg is None:
        c = gguf.config()
        cfg = M.ModelConfig(name="gguf", arch="gguf", dim=c["dim"], n_layers=c["n_layers"], n_heads=c["n_heads"],
                            n_kv_heads=c["n_kv_heads"], head_dim=c["head_dim"], n_ff=0, vocab=c["vocab"],
                            max_seq=max_seq or c["max_seq"], logit_scale=c["logit_scale"])
    eng.cfg = cfg
    ctx.adopt(eng)
    return eng
