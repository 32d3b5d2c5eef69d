"""GGUF files through the C reader (spx_gguf_*), against the reference's parse_file
(gguf_loader.rs:142-247) and ModelConfig::from_gguf (smollm_chat.rs:69-120) rules. Host only:
files written by spindle_amd.gguf's writer and by hand, read back without a GPU.

Pinning: hand-built headers with offsets worked out by hand (24-byte header -> data at 32;
alignment rounded up to 32), every value type read back, the from_gguf defaults and refusals
case by case, and the writer's bytes found again at the reader's tensor offsets."""
import os
import struct

import numpy as np
import pytest

from spindle_amd import gguf as G
from spindle_amd._lib import SpxError


@pytest.fixture
def path(tmp_path):
    return str(tmp_path / "f.gguf")


def test_empty_file_layout_by_hand(path):
    with open(path, "wb") as f:  # magic, version 3, 0 tensors, 0 keys: 24 bytes -> data at 32
        f.write(struct.pack("<IIQQ", G.MAGIC, 3, 0, 0))
    with G.GgufFile(path) as g:
        assert g.info() == dict(version=3, alignment=32, data_offset=32, n_tensors=0, n_meta=0)
    with open(path, "wb") as f:  # + general.alignment U32 64: 24 + 8 + 17 + 4 + 4 = 57 -> 64
        f.write(struct.pack("<IIQQ", G.MAGIC, 2, 0, 1) + struct.pack("<Q", 17) + b"general.alignment" + struct.pack("<II", 4, 64))
    with G.GgufFile(path) as g:
        assert g.info() == dict(version=2, alignment=64, data_offset=64, n_tensors=0, n_meta=1)


@pytest.mark.parametrize("align,atype,want", [(None, G.U32, 32), (64, G.U32, 64), (16, G.U32, 32), (4096, G.U64, 4096),
                                              (256, G.I32, 32)])
def test_alignment_rule(path, align, atype, want):
    """general.alignment as U32 or U64, at least 32 (:186-190); other types are ignored."""
    data = np.arange(96, dtype=np.uint8)
    meta = [("general.alignment", atype, align)] if align is not None else []
    tensors = [("a", 0, [8], data[:32]), ("b", 0, [4, 4], data[32:96])]
    G.write_gguf(path, meta, tensors, alignment=None)
    with G.GgufFile(path) as g:
        inf = g.info()
        assert inf["alignment"] == want and inf["data_offset"] % want == 0
        n, dt, dims, off = g.tensor(1)
        assert (n, dt, dims) == ("b", 0, [4, 4]) and off == inf["data_offset"] + 32


def test_value_types(path):
    meta = [("u8", G.U8, 200), ("i8", G.I8, -5), ("u16", G.U16, 60000), ("i16", G.I16, 7), ("u32", G.U32, 4000000000),
            ("i32", G.I32, -1), ("f32", G.F32, 0.5), ("bool", G.BOOL, True), ("str", G.STR, "qwen3moe"),
            ("u64", G.U64, 1 << 40), ("i64", G.I64, 12), ("f64", G.F64, 0.25),
            ("arr_u32", G.ARR, (G.U32, [1, 2, 3])), ("arr_f64", G.ARR, (G.F64, [1.0])),
            ("arr_str", G.ARR, (G.STR, ["a", "bb"])), ("tokenizer.ggml.tokens", G.ARR, (G.STR, ["x", "<think>", "yz"]))]
    G.write_gguf(path, meta, [])
    with G.GgufFile(path) as g:
        assert [g.meta_type(k) for k, _, _ in meta] == [t for _, t, _ in meta]
        assert g.meta("u8") == 200 and g.meta("u16") == 60000 and g.meta("u32") == 4000000000 and g.meta("u64") == 1 << 40
        assert g.meta("i16") == 7 and g.meta("i64") == 12
        assert g.meta("i8") == "negative" and g.meta("i32") == "negative"  # as_usize: None for negatives
        assert g.meta("f32") == 0.5 and g.meta("f64") == 0.25 and g.meta("bool") is True and g.meta("str") == "qwen3moe"
        assert g.meta("arr_u32") == (G.U32, 3) and g.meta("arr_f64") == (G.F64, 1) and g.meta("arr_str") == (G.STR, 2)
        assert g.meta("missing") is None
        assert g.vocab_size() == 3 and [g.token(i) for i in range(4)] == ["x", "<think>", "yz", None]


def _cfg_file(path, arch, extra=(), tokens=10, tensors=()):
    meta = [("general.architecture", G.STR, arch)] + [(f"{arch}.{k}", t, v) for k, t, v in extra]
    if tokens:
        meta.append(("tokenizer.ggml.tokens", G.ARR, (G.STR, [f"t{i}" for i in range(tokens)])))
    G.write_gguf(path, meta, list(tensors))
    return G.GgufFile(path)


BASE = [("embedding_length", G.U32, 64), ("attention.head_count", G.U32, 4), ("block_count", G.U32, 2)]


def test_config_defaults(path):
    c = _cfg_file(path, "llama", BASE).config()
    assert (c["dim"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["n_layers"], c["vocab"]) == (64, 4, 4, 16, 2, 10)
    assert (c["max_seq"], c["rope_neox"], c["n_expert"], c["n_expert_used"], c["expert_norm"]) == (2048, 0, 0, 0, 1)
    assert c["rope_theta"] == 10000.0 and c["rms_eps"] == np.float32(1e-5) and c["attn_scale"] == 0.0
    assert c["embedding_scale"] == c["residual_scale"] == c["logit_scale"] == 1.0


@pytest.mark.parametrize("arch,neox,norm", [("llama", 0, 1), ("granite", 0, 1), ("granitemoe", 0, 1), ("qwen2", 1, 1),
                                            ("qwen2moe", 1, 0), ("qwen3", 1, 1), ("qwen3moe", 1, 1), ("olmoe", 1, 0)])
def test_config_per_architecture(path, arch, neox, norm):
    extra = BASE + [("attention.head_count_kv", G.U32, 2), ("attention.key_length", G.U32, 32),
                    ("context_length", G.U64, 40960), ("rope.freq_base", G.F32, 1e6),
                    ("attention.layer_norm_rms_epsilon", G.F32, 1e-6), ("expert_count", G.U32, 8),
                    ("expert_used_count", G.U32, 10)]
    c = _cfg_file(path, arch, extra).config()
    assert (c["rope_neox"], c["expert_norm"], c["n_kv_heads"], c["head_dim"], c["max_seq"]) == (neox, norm, 2, 32, 40960)
    assert c["n_expert"] == 8 and c["n_expert_used"] == 8  # used count capped at the expert count
    assert c["rope_theta"] == 1e6 and c["rms_eps"] == np.float32(1e-6)
    c = _cfg_file(path, arch, extra + [("expert_weights_norm", G.BOOL, not norm)]).config()
    assert c["expert_norm"] == (not norm)


def test_config_granite_scales(path):
    extra = BASE + [("embedding_scale", G.F32, 12.0), ("residual_scale", G.F32, 0.22), ("logit_scale", G.F32, 6.0),
                    ("attention.scale", G.F32, 0.015625), ("expert_gating_func", G.U32, 1)]
    c = _cfg_file(path, "granitemoe", extra).config()
    assert (c["embedding_scale"], c["logit_scale"], c["attn_scale"]) == (12.0, 6.0, 0.015625)
    assert c["residual_scale"] == np.float32(0.22)


@pytest.mark.parametrize("arch,extra,msg", [
    ("mamba", BASE, "unsupported architecture"),
    ("qwen3moe", BASE + [("expert_gating_func", G.U32, 2)], "softmax expert gating"),
    ("llama", BASE[1:], "embedding_length"),
    ("llama", BASE + [("attention.key_length", G.U32, 12)], "head layout"),
    ("llama", BASE + [("attention.head_count_kv", G.U32, 3)], "head layout"),
])
def test_config_refusals(path, arch, extra, msg):
    with pytest.raises(SpxError, match=msg):
        _cfg_file(path, arch, extra).config()


def test_vocab_without_tokenizer_is_the_embedding_rows(path):
    t = [("token_embd.weight", 0, [64, 123], np.zeros(64 * 123 * 4, np.uint8))]
    assert _cfg_file(path, "llama", BASE, tokens=0, tensors=t).config()["vocab"] == 123


def test_stop_and_think_ids(path):
    toks = ["a", "<think>", "</think>", "<|endoftext|>", "b", "<|im_end|>", "<|end_of_text|>"]
    G.write_gguf(path, [("tokenizer.ggml.tokens", G.ARR, (G.STR, toks)), ("tokenizer.ggml.eos_token_id", G.U32, 5)], [])
    with G.GgufFile(path) as g:
        assert g.stop_ids() == [5, 3, 6]  # eos first, then the named tokens, no repeats
        assert g.think_ids() == (1, 2)
    G.write_gguf(path, [("tokenizer.ggml.tokens", G.ARR, (G.STR, ["<think>", "x"]))], [])
    with G.GgufFile(path) as g:
        assert g.stop_ids() == [] and g.think_ids() == (-1, -1)


@pytest.mark.parametrize("case", ["magic", "truncated", "value_type", "nested_array", "long_string"])
def test_malformed_files(path, case):
    head = struct.pack("<IIQQ", G.MAGIC, 3, 0, 1) + struct.pack("<Q", 1) + b"k"
    body = {"magic": struct.pack("<IIQQ", 0x12345678, 3, 0, 0),
            "truncated": head + struct.pack("<I", 4) + b"\x01",
            "value_type": head + struct.pack("<I", 13) + b"\0" * 8,
            "nested_array": head + struct.pack("<IIQ", 9, 9, 1) + b"\0" * 16,
            "long_string": head + struct.pack("<IQ", 8, (16 << 20) + 1)}[case]
    with open(path, "wb") as f:
        f.write(body)
    with pytest.raises(SpxError, match={"magic": "not a GGUF", "truncated": "truncated", "value_type": "unknown GGUF value type",
                                        "nested_array": "array elem", "long_string": "16 MiB"}[case]):
        G.GgufFile(path)


def test_written_model_round_trip_and_cut_off_file(path):
    """Every tensor of a synthetic model is found at the reader's offset with its bytes, dtype and
    dims; a file cut short fails the completeness check (:1944-1963)."""
    from spindle_amd import model as M
    cfg = M.TINY["tiny-qwen3moe"]
    w = M.synth_model(cfg, seed=3)
    G.write_model(path, cfg, w, eos=7)
    raw = np.fromfile(path, np.uint8)
    with G.GgufFile(path) as g:
        assert g.info()["n_tensors"] == len(w)
        for name, (spec, data) in w.items():
            i = g.find(name)
            n, dt, dims, off = g.tensor(i)
            assert n == name and dt == spec.dtype and dims[0] == spec.cols
            assert np.array_equal(raw[off:off + data.size], data), name
        c = g.config()
        assert (c["dim"], c["n_layers"], c["n_expert"], c["vocab"], c["max_seq"]) == (cfg.dim, cfg.n_layers, cfg.n_expert, cfg.vocab, cfg.max_seq)
        g.check()
    with open(path, "r+b") as f:
        f.truncate(os.path.getsize(path) - 1000)
    with G.GgufFile(path) as g:
        with pytest.raises(SpxError, match="incomplete"):
            g.check()


def _one_tensor_file(path, dims, rel=0, dtype=0, alignment=None):
    """A GGUF v3 file by hand: optional general.alignment (U64), one tensor with the given dims and
    data offset, then 64 data bytes."""
    meta = b""
    n_kv = 0
    if alignment is not None:
        meta = struct.pack("<Q", 17) + b"general.alignment" + struct.pack("<IQ", G.U64, alignment)
        n_kv = 1
    t = struct.pack("<Q", 1) + b"w" + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
    t += struct.pack("<IQ", dtype, rel)
    body = struct.pack("<IIQQ", G.MAGIC, 3, 1, n_kv) + meta + t
    body += b"\0" * ((-len(body)) % 32) + bytes(64)
    with open(path, "wb") as f:
        f.write(body)


@pytest.mark.parametrize("case", ["rows_wrap", "bytes_wrap", "offset_wrap", "offset_past_end", "cols_huge"])
def test_sizes_that_wrap_are_refused(path, case):
    """Dims whose product, byte count or offset wraps 64 bits (and offsets past the end) fail the
    completeness check instead of passing it with a wrapped sum: the bounds the reference's slice
    indexing enforces (gguf_loader.rs, :1944-1963)."""
    dims, rel = {"rows_wrap": ([32, 1 << 40, 1 << 40], 0),          # rows overflow int64
                 "bytes_wrap": ([32, (1 << 62) // 4], 0),            # F32: 128 B a row x 2^60 rows
                 "offset_wrap": ([8], (1 << 64) - 16),               # data_offset + rel wraps
                 "offset_past_end": ([8], 1 << 40),
                 "cols_huge": ([1 << 63, 1], 0)}[case]
    _one_tensor_file(path, dims, rel)
    if case == "offset_wrap":
        with pytest.raises(SpxError, match="overflows"):
            G.GgufFile(path)
        return
    with G.GgufFile(path) as g:
        with pytest.raises(SpxError, match="incomplete|out of range"):
            g.check()


@pytest.mark.parametrize("align", [0, 48, 1 << 31])
def test_alignment_not_a_power_of_two_is_refused(path, align):
    _one_tensor_file(path, [8], alignment=align)
    with pytest.raises(SpxError, match="power of two"):
        G.GgufFile(path)
