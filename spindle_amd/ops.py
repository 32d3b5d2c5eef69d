"""Operator-level mirror of the reference's kernel interface over the C ABI.

Names follow the reference: `matvec` / `matvec_multi` (smollm_chat.rs:309, 447),
`q8k_quantize` (Q8K::quantize, quant_q8k.rs:73), `matmul_rows_q8k` (quant_q8k::matmul_rows,
:255). Device memory comes from torch (cuda == HIP on ROCm); torch is plumbing only.
"""
import ctypes as C
import weakref

import numpy as np

from ._lib import P, check, lib

try:  # device buffers of the operator functions below are torch tensors; a context needs no torch
    import torch
except ImportError:  # pragma: no cover - torch is part of this image
    torch = None

F32, F16, Q5_0, Q8_0, Q4K, Q6K = 0, 1, 6, 8, 12, 14


class Context:
    """A device + HIP stream (replaces the reference's WorkerPool as the execution resource)."""

    def __init__(self, device=0):
        self.device = device
        if torch is not None and torch.cuda.is_available():
            torch.cuda.set_device(device)  # torch's buffers on the same device
        h = P()
        check(lib.spx_create(device, C.byref(h)))  # fails (SpxError) without a visible GPU
        self.h = h
        self._children = weakref.WeakSet()   # engines / tensors to release before the context

    def adopt(self, obj):
        self._children.add(obj)

    def sync(self):
        check(lib.spx_sync(self.h))

    def close(self):
        if self.h:
            for ch in list(self._children):
                ch.close()
            lib.spx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Tensor:
    """An uploaded weight tensor: n_expert slabs of rows x cols in GGUF block layout (Mat)."""

    def __init__(self, ctx, dtype, cols, rows, ggml_bytes, n_expert=1):
        self.ctx, self.dtype, self.cols, self.rows, self.n_expert = ctx, dtype, cols, rows, n_expert
        data = np.ascontiguousarray(ggml_bytes, dtype=np.uint8)
        rb = lib.spx_row_bytes(dtype, cols)
        if rb <= 0 or data.size != rb * rows * n_expert:
            raise ValueError(f"expected {rb * rows * n_expert} bytes for dtype {dtype} {rows}x{cols}x{n_expert}, got {data.size}")
        h = P()
        check(lib.spx_tensor_upload(ctx.h, dtype, cols, rows, n_expert, data.ctypes.data_as(P), C.byref(h)))
        self.h = h
        self.nbytes = data.size
        ctx.adopt(self)

    def download(self):
        out = np.empty(self.nbytes, np.uint8)
        check(lib.spx_tensor_download(self.ctx.h, self.h, out.ctypes.data_as(P)))
        return out

    def free(self):
        if self.h and self.ctx.h:
            lib.spx_tensor_free(self.ctx.h, self.h)
        self.h = None

    close = free

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _p(t):
    return C.c_void_p(t.data_ptr())


def q8k_quantize(ctx, x):
    """x: [m, n] float32 cuda tensor -> (d [m, n/256] f32, qs [m, n] i8, bsums [m, n/16] i16)."""
    x = x.contiguous()
    m, n = x.shape
    d = torch.empty((m, n // 256), dtype=torch.float32, device=x.device)
    qs = torch.empty((m, n), dtype=torch.int8, device=x.device)
    bs = torch.empty((m, n // 16), dtype=torch.int16, device=x.device)
    torch.cuda.synchronize()
    check(lib.spx_q8k_quantize(ctx.h, _p(x), n, n, m, _p(d), _p(qs), _p(bs)))
    ctx.sync()
    return d, qs, bs


def matmul_rows_q8k(ctx, w, q, expert=0, r0=0, r1=None, out=None):
    d, qs, bs = q
    m = qs.shape[0]
    r1 = w.rows if r1 is None else r1
    if out is None:
        out = torch.full((m, w.rows), float("nan"), dtype=torch.float32, device=qs.device)
    torch.cuda.synchronize()
    check(lib.spx_matmul_rows_q8k(ctx.h, w.h, expert, _p(d), _p(qs), _p(bs), m, _p(out), out.shape[1], r0, r1))
    ctx.sync()
    return out


def block_sums_q8k(ctx, w, row, q, expert=0):
    d, qs, bs = q
    nb = w.cols // 256
    out = torch.empty((nb, 2), dtype=torch.int32, device=qs.device)
    torch.cuda.synchronize()
    check(lib.spx_block_sums_q8k(ctx.h, w.h, expert, row, _p(qs), _p(bs), _p(out)))
    ctx.sync()
    return out


def matvec(ctx, w, x, expert=0):
    """x: [m, cols] float32 cuda (m <= 16) -> [m, rows] (matvec for m == 1, matvec_multi above)."""
    x = x.contiguous()
    m = x.shape[0]
    out = torch.empty((m, w.rows), dtype=torch.float32, device=x.device)
    torch.cuda.synchronize()
    check(lib.spx_matvec(ctx.h, w.h, expert, _p(x), x.shape[1], m, _p(out), w.rows))
    ctx.sync()
    return out


def matvec_noalloc(ctx, w, x, expert=0):
    """matvec through spx_matvec_noalloc: the K-quant activations' Q8_K staged in the library's
    fixed per-device scratch array instead of an allocated workspace (same results)."""
    x = x.contiguous()
    m = x.shape[0]
    out = torch.empty((m, w.rows), dtype=torch.float32, device=x.device)
    torch.cuda.synchronize()
    check(lib.spx_matvec_noalloc(ctx.h, w.h, expert, _p(x), x.shape[1], m, _p(out), w.rows))
    ctx.sync()
    return out


matvec_multi = matvec


def moe(ctx, gate, up, down, x, chosen, weights):
    """ffns_fused / moe_batch_fused with the combine: x [m, dim] float32 cuda; chosen, weights
    [m, k] host arrays (each row's experts distinct). Returns y [m, dim]."""
    assert x.is_cuda and x.dtype == torch.float32 and x.dim() == 2
    ch = np.ascontiguousarray(chosen, np.int32)
    wt = np.ascontiguousarray(weights, np.float32)
    m, k = ch.shape
    y = torch.empty((m, down.rows), dtype=torch.float32, device=x.device)
    torch.cuda.synchronize()  # x is written on torch's stream, the library runs on the context's
    check(lib.spx_moe(ctx.h, gate.h, up.h, down.h, _p(x), x.stride(0), m, k, ch.ctypes.data_as(P), wt.ctypes.data_as(P),
                      _p(y), y.stride(0)))
    ctx.sync()
    return y


def moe_dev(ctx, gate, up, down, x, chosen, weights):
    """moe with the routing in device memory (spx_moe_dev): chosen [m, k] int32 and weights
    [m, k] float32 cuda tensors, as a router on the GPU leaves them; K-quant experts. A row whose
    ids are out of range or repeated comes back NaN. Returns y [m, dim]."""
    assert x.is_cuda and x.dtype == torch.float32 and x.dim() == 2
    assert chosen.is_cuda and chosen.dtype == torch.int32 and weights.is_cuda and weights.dtype == torch.float32
    chosen, weights = chosen.contiguous(), weights.contiguous()
    m, k = chosen.shape
    y = torch.empty((m, down.rows), dtype=torch.float32, device=x.device)
    torch.cuda.synchronize()  # inputs written on torch's stream, the library runs on the context's
    check(lib.spx_moe_dev(ctx.h, gate.h, up.h, down.h, _p(x), x.stride(0), m, k, _p(chosen), _p(weights), _p(y), y.stride(0)))
    ctx.sync()
    return y


class SamplerParams(C.Structure):
    """spx_sampler_params (SamplerConfig, smollm_chat.rs:1523-1555)."""
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int), ("top_p", C.c_float), ("min_p", C.c_float),
                ("repeat_penalty", C.c_float), ("seed", C.c_uint64), ("stop_ids", C.POINTER(C.c_int32)),
                ("n_stop", C.c_int), ("think_open", C.c_int)]


def sampler_params(temperature=0.6, top_k=40, top_p=0.9, min_p=0.05, repeat_penalty=1.1, seed=1, stop_ids=(),
                   think_open=-1):
    """The reference's defaults (a fixed seed instead of the clock); returns (params, keep-alive)."""
    stop = (C.c_int32 * max(1, len(stop_ids)))(*stop_ids)
    return SamplerParams(temperature, top_k, top_p, min_p, repeat_penalty, seed,
                         C.cast(stop, C.POINTER(C.c_int32)), len(stop_ids), think_open), stop


class Sampler:
    """sample_from_logits over device logits with its own SplitMix64 state (spx_sampler)."""

    def __init__(self, ctx, vocab, **kw):
        self.ctx, self.vocab = ctx, vocab
        params, keep = sampler_params(**kw)
        h = P()
        check(lib.spx_sampler_create(ctx.h, C.byref(params), vocab, C.byref(h)))
        self.h = h
        ctx.adopt(self)

    def reseed(self, seed):
        check(lib.spx_sampler_reseed(self.h, seed))

    def sample(self, logits, recent=(), forbid_stop=False, forbid_think=False, logit_scale=1.0):
        """One token from one row of device logits [vocab] (a float32 cuda tensor)."""
        assert logits.is_cuda and logits.dtype == torch.float32 and logits.numel() == self.vocab and logits.is_contiguous()
        rc = np.ascontiguousarray(np.asarray(recent, np.int32).reshape(-1))
        tok = C.c_int32()
        torch.cuda.synchronize()
        check(lib.spx_sample(self.h, _p(logits), logit_scale, rc.ctypes.data_as(P) if rc.size else None, rc.size,
                             int(forbid_stop), int(forbid_think), C.byref(tok)))
        return tok.value

    def sample_verify(self, logits, recent, draft, generated, max_accept, forbid_think=False, logit_scale=1.0):
        """The verify loop's sampling over rows 0..len(draft) of logits [>= len(draft)+1, vocab]."""
        assert logits.is_cuda and logits.dtype == torch.float32 and logits.shape[-1] == self.vocab
        rc = np.ascontiguousarray(np.asarray(recent, np.int32).reshape(-1))
        dr = np.ascontiguousarray(np.asarray(draft, np.int32).reshape(-1))
        toks = np.empty(dr.size + 1, np.int32)
        n = C.c_int()
        torch.cuda.synchronize()
        check(lib.spx_sample_verify(self.h, _p(logits), logits.stride(0), dr.size, logit_scale,
                                    rc.ctypes.data_as(P) if rc.size else None, rc.size,
                                    dr.ctypes.data_as(P) if dr.size else None, generated, max_accept,
                                    int(forbid_think), toks.ctypes.data_as(P), C.byref(n)))
        return toks[:n.value]

    def close(self):
        if self.h:
            lib.spx_sampler_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
