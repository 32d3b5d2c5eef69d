"""The reference's own kernel tests, replayed against the oracle with the same seeds and
tolerances (quant_q8k.rs:364-442, quant.rs:1727-1771, quant_multi.rs:369-417), plus an exact
integer identity that pins the per-block int32 sums."""
import numpy as np
import pytest

from oracle import ffi
from tests import refdata as R


def _dq8k(q):
    d, qs, _ = q
    return (np.repeat(d, 256) * qs.astype(np.float32)).astype(np.float32)


def test_int_kernel_matches_reference():
    """quant_q8k.rs:364-411: every batch size 1..11, rows split [0,3)+[3,37)."""
    rng = R.Rng(0x51ED)
    for dtype in (R.Q4K, R.Q6K):
        for n in (256, 768, 2048):
            rows = 37
            mat = R.random_matrix(dtype, n, rows, rng)
            w = ffi.dequant(dtype, mat, rows, n).astype(np.float64)
            for bsz in range(1, 12):
                xs = [rng.floats(n, -2.0, 2.0) for _ in range(bsz)]
                qs = [ffi.q8k_quantize(x) for x in xs]
                outs = [np.full(rows, np.nan, np.float32) for _ in range(bsz)]
                ffi.q8k_matmul_rows(mat, dtype, n, qs, rows, 0, 3, outs)
                ffi.q8k_matmul_rows(mat, dtype, n, qs, rows, 3, rows, outs)
                for b in range(bsz):
                    xq = _dq8k(qs[b]).astype(np.float64)
                    want = w @ xq
                    scale = np.abs(w * xq).sum(1)
                    got = outs[b].astype(np.float64)
                    assert np.all(np.abs(got - want) <= 1e-4 * scale + 1e-6), (dtype, n, bsz, b)
                    exact = w @ xs[b].astype(np.float64)
                    assert np.all(np.abs(got - exact) <= 0.02 * scale + 1e-4)


def test_int_kernel_batch_is_bitwise():
    """quant_q8k.rs:413-442."""
    rng = R.Rng(77)
    for dtype in (R.Q4K, R.Q6K):
        n, rows = 768, 37
        mat = R.random_matrix(dtype, n, rows, rng)
        qs = [ffi.q8k_quantize(rng.floats(n, -2.0, 2.0)) for _ in range(11)]
        batch = ffi.q8k_matmul_rows(mat, dtype, n, qs, rows)
        for b, q in enumerate(qs):
            one = ffi.q8k_matmul_rows(mat, dtype, n, [q], rows)[0]
            assert np.array_equal(one.view(np.uint32), batch[b].view(np.uint32))


@pytest.mark.parametrize("dtype", [R.Q4K, R.Q6K])
def test_block_sums_exact_integer_identity(dtype):
    """With d = 1 and dmin in {0, 1} the dequantized weights are small integers, so the f64 dot
    of dequant_row (pinned by the known-answer blocks) with the integer Q8_K codes is exact and
    must equal sumi - corr bit for bit, block by block."""
    rng = np.random.default_rng(3)
    n = 1024
    for dmin in (0x0000, 0x3C00):
        for trial in range(20):
            raw = rng.integers(0, 256, R.row_bytes(dtype, n), dtype=np.uint8)
            bb = 144 if dtype == R.Q4K else 210
            for b0 in range(0, raw.size, bb):
                if dtype == R.Q4K:
                    raw[b0:b0 + 2] = [0x00, 0x3C]
                    raw[b0 + 2:b0 + 4] = [dmin & 255, dmin >> 8]
                else:
                    raw[b0 + 208:b0 + 210] = [0x00, 0x3C]
            x = rng.standard_normal(n).astype(np.float32) * (trial + 1)
            q = ffi.q8k_quantize(x)
            sumi, corr, lanes = ffi.q8k_block_sums(raw, dtype, n, q)
            assert np.array_equal(lanes.sum(1), sumi)
            w = ffi.dequant_row(dtype, raw, n).astype(np.float64)
            y = q[1].astype(np.float64)
            for i in range(n // 256):
                exact = float(w[i * 256:(i + 1) * 256] @ y[i * 256:(i + 1) * 256])
                if dtype == R.Q4K and dmin == 0:
                    assert exact == sumi[i]
                else:
                    assert exact == float(sumi[i]) - float(corr[i])


def test_int_lane_partition():
    """Lane l of the AVX2 accumulator holds elements with (e % 32) // 4 == l (quant_q8k.rs:235-242):
    isolate one element at a time and check which lane it lands in."""
    rng = np.random.default_rng(9)
    raw = rng.integers(0, 256, 144, dtype=np.uint8)
    raw[0:2] = [0x00, 0x3C]
    for e in [0, 3, 4, 31, 32, 77, 128, 255]:
        x = np.zeros(256, np.float32)
        x[e] = 1.0
        q = ffi.q8k_quantize(x)
        _, _, lanes = ffi.q8k_block_sums(raw, R.Q4K, 256, q)
        nz = np.nonzero(lanes[0])[0]
        assert nz.size <= 1
        if nz.size:
            assert nz[0] == (e % 32) // 4


SIMD_TYPES = [R.F32, R.F16, R.BF16, R.Q4_0, R.Q4_1, R.Q5_0, R.Q5_1, R.Q8_0, R.Q4K, R.Q5K, R.Q6K]
ORACLE_FLOAT = {R.F32, R.F16, R.Q5_0, R.Q8_0, R.Q5K}


def test_float_kernels_match_scalar_reference():
    """quant.rs:1727-1771 with the same seed; the oracle restates the float kernels the
    decode path uses (F32, F16, Q5_0, Q8_0, Q5_K), the other types only consume the stream."""
    rng = R.Rng(0x2545F4914F6CDD1D)
    for dtype in SIMD_TYPES:
        for n in (256, 768, 2048):
            for rows in (2, 3, 4, 5, 6, 8, 10):
                mat = bytearray()
                for _ in range(rows):
                    mat += R.random_row(dtype, n, rng)
                x = rng.floats(n, -1.0, 1.0)
                if dtype not in ORACLE_FLOAT:
                    continue
                mat = np.frombuffer(bytes(mat), np.uint8).copy()
                out = ffi.matvec_rows(mat, dtype, n, x, 1, rows - 1)
                w = ffi.dequant(dtype, mat, rows, n).astype(np.float64)
                want = w[1:] @ x.astype(np.float64)
                scale = np.abs(w[1:] * x.astype(np.float64)).sum(1)
                assert np.all(np.abs(out - want) <= 1e-4 * scale + 1e-6), (dtype, n, rows)


def test_multi_matvec_matches_scalar_reference():
    """quant_multi.rs:369-417 with the same seed (Q8_0 and F32 restated; K-quants take the
    integer path in the engine, so their float multi kernels only consume the stream)."""
    rng = R.Rng(0x9E3779B97F4A7C15)
    for dtype in (R.Q4K, R.Q6K, R.Q8_0, R.F32, R.Q5K):
        for n in (256, 768, 2048):
            rows = 7
            if dtype == R.Q5K:
                rb = R.row_bytes(dtype, n)
                m = rng.bytes(rb * rows)
                for b0 in range(0, len(m), 176):
                    m[b0:b0 + 2] = R.f16_trunc(rng.f(0.001, 0.05))
                    m[b0 + 2:b0 + 4] = R.f16_trunc(rng.f(0.001, 0.05))
                mat = np.frombuffer(bytes(m), np.uint8).copy()
            else:
                mat = R.random_matrix(dtype, n, rows, rng)
            check = dtype in (R.Q8_0, R.F32)
            w = ffi.dequant(dtype, mat, rows, n).astype(np.float64) if check else None
            for bsz in range(1, 12):
                xs = [rng.floats(n, -1.0, 1.0) for _ in range(bsz)]
                if not check:
                    continue
                outs = [np.full(rows, np.nan, np.float32) for _ in range(bsz)]
                ffi.matmul_rows_multi(mat, dtype, n, xs, rows, 0, 3, outs)
                ffi.matmul_rows_multi(mat, dtype, n, xs, rows, 3, rows, outs)
                for b in range(bsz):
                    want = w @ xs[b].astype(np.float64)
                    scale = np.abs(w * xs[b].astype(np.float64)).sum(1)
                    assert np.all(np.abs(outs[b] - want) <= 1e-4 * scale + 1e-6), (dtype, n, bsz)


def test_q8_0_single_and_multi_orders_differ_but_agree():
    """The reference's M=1 (quant.rs:48-107) and M>1 (quant_multi.rs:168-190) Q8_0 kernels sum in
    different orders; both must sit within 1e-4 of the f64 dot, and they are not bitwise equal
    in general (which is why the reference's verify is not bitwise equal to decode on Q8_0)."""
    rng = np.random.default_rng(1)
    n, rows = 1024, 64
    mat = rng.integers(0, 256, R.row_bytes(R.Q8_0, n) * rows, dtype=np.uint8)
    for b0 in range(0, mat.size, 34):
        mat[b0:b0 + 2] = np.frombuffer(np.float16(rng.uniform(0.001, 0.05)).tobytes(), np.uint8)
    x = rng.standard_normal(n).astype(np.float32)
    one = ffi.matvec_rows(mat, R.Q8_0, n, x, 0, rows)
    multi = ffi.matmul_rows_multi(mat, R.Q8_0, n, [x, x], rows)[0]
    w = ffi.dequant(R.Q8_0, mat, rows, n).astype(np.float64)
    want = w @ x.astype(np.float64)
    scale = np.abs(w * x.astype(np.float64)).sum(1)
    for o in (one, multi):
        assert np.all(np.abs(o - want) <= 1e-4 * scale)
    assert not np.array_equal(one, multi)


def test_pool_shrink_keeps_results():
    """Lowering the oracle's thread count after a larger one leaves the extra workers idle: the
    row split changes, the results (rows are independent) do not."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal(1024).astype(np.float32)
    raw = rng.integers(0, 256, 34 * 32 * 300).astype(np.uint8)
    raw.reshape(-1, 34)[:, 1] = 0x1C  # finite f16 scales
    m = ffi.mat(ffi.Q8_0, raw, 300, 1024)
    outs = []
    for t in (8, 2, 5, 1):
        ffi.set_threads(t)
        outs.append(ffi.matvec(m, x))
    assert all(np.array_equal(outs[0].view(np.uint32), o.view(np.uint32)) for o in outs[1:])


@pytest.mark.parametrize("dtype", [R.Q4K, R.Q6K])
def test_avx2_rows_kernel_equals_scalar(dtype):
    """The oracle's AVX2 rows kernel (the reference's maddubs / madd lanes, each block decoded
    once for all vectors) gives the scalar restatement's bits for every vector count."""
    rng = R.Rng(7 + dtype)
    n, rows = 1024, 23
    mat = R.random_matrix(dtype, n, rows, rng)
    xs = [rng.floats(n, -2.0, 2.0) for _ in range(20)]
    qs = [ffi.q8k_quantize(x) for x in xs]
    try:
        for nv in (1, 3, 16, 20):
            ffi.set_simd(False)
            a = ffi.q8k_matmul_rows(mat, dtype, n, qs[:nv], rows)
            ffi.set_simd(True)
            b = ffi.q8k_matmul_rows(mat, dtype, n, qs[:nv], rows)
            for v in range(nv):
                assert np.array_equal(a[v].view(np.uint32), b[v].view(np.uint32)), (nv, v)
    finally:
        ffi.set_simd(True)


def test_avx2_attention_equals_scalar():
    """A whole forward (attention included) with the AVX2 kernels equals the scalar one bit for bit."""
    from oracle.model import OracleModel
    from spindle_amd import model as M
    cfg = M.TINY["tiny-qwen3moe"]
    w = M.synth_model(cfg, seed=5)
    ids = np.random.default_rng(2).integers(0, cfg.vocab, 40).astype(np.int32)
    out = []
    try:
        for simd in (False, True):
            ffi.set_simd(simd)
            om = OracleModel(cfg, w)
            h = np.concatenate([om.forward(ids[s:s + 8], s) for s in range(0, 40, 8)])
            out.append(h)
    finally:
        ffi.set_simd(True)
    assert np.array_equal(out[0].view(np.uint32), out[1].view(np.uint32))
