"""GPU parity of the matvec kernels against the oracle (same inputs, through the C ABI).

Bars: Q8_K quantization, per-block int32 sums and the integer path's fp32 outputs bit-exact
against the oracle (the reference's arithmetic, including its 8-lane fp32 epilogue); the
fp32-activation path (Q8_0/Q5_0/F32) within 1e-4 max-abs-normalised of the oracle and within
the reference's own per-row tolerance 1e-4*sum|w*x| + 1e-6 of the f64 dot; a vector's output
bitwise identical alone and inside any batch."""
import numpy as np
import pytest

from oracle import ffi
from tests import refdata as R

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


@pytest.fixture(params=["auto", "tiles", "rows"])
def mv_mode(request, monkeypatch):
    """Integer matvec launch shape: the default (row-parallel lanes at one row, the int8 matrix
    cores from two), or forced eight-row lane tiles, or forced row-parallel lanes; every shape
    must give the reference's bits."""
    if request.param == "auto":
        monkeypatch.delenv("SPX_MV_MODE", raising=False)
    else:
        monkeypatch.setenv("SPX_MV_MODE", "0" if request.param == "tiles" else "1")
    return request.param


def _cuda(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _rand_kquant(dtype, n, rows, rng, n_expert=1):
    """Random K-quant bytes with sane f16 scales (d ~ U(0.001, 0.05) like the reference tests)."""
    bb = 144 if dtype == R.Q4K else 210
    raw = rng.integers(0, 256, R.row_bytes(dtype, n) * rows * n_expert, dtype=np.uint8)
    sc = np.float16(rng.uniform(0.001, 0.05, raw.size // bb * 2)).view(np.uint8).reshape(-1, 4)
    blk = raw.reshape(-1, bb)
    if dtype == R.Q4K:
        blk[:, 0:4] = sc
    else:
        blk[:, 208:210] = sc[:, 0:2]
    return raw


def _norm_err(got, want):
    return float(np.max(np.abs(got.astype(np.float64) - want.astype(np.float64))) / max(1e-30, np.max(np.abs(want))))


def test_q8k_quantize_bitwise(ctx):
    from spindle_amd import ops
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((5, 2048)) * rng.uniform(0.01, 10, (5, 1))).astype(np.float32)
    x[1, 256:512] = 0.0           # all-zero block
    x[2, 0:256] *= 1e-30          # tiny but finite
    x[3, 1000] = np.inf           # non-finite block
    x[4, :] = np.round(x[4, :] * 4) / 4  # many exact halves -> round-half-even cases
    d, qs, bs = ops.q8k_quantize(ctx, _cuda(x))
    for v in range(5):
        od, oq, ob = ffi.q8k_quantize(x[v])
        assert np.array_equal(d[v].cpu().numpy().view(np.uint32), od.view(np.uint32)), v
        assert np.array_equal(qs[v].cpu().numpy(), oq), v
        assert np.array_equal(bs[v].cpu().numpy(), ob), v


def _nan_rows(rng, rows, n):
    """Blocks with NaN at random places, often in the last group of eight (where the
    reference's max order lets one survive or drops it by lane), and some +-inf."""
    x = (rng.standard_normal((rows, n)) * 3).astype(np.float32)
    for r in range(rows):
        for b in range(n // 256):
            pos = rng.integers(0, 256, rng.integers(0, 4))
            if rng.random() < 0.5:
                pos = np.append(pos, 248 + rng.integers(0, 8))
            x[r, b * 256 + pos] = np.nan
            if rng.random() < 0.25:
                x[r, b * 256 + rng.integers(0, 256)] = np.inf * rng.choice([-1.0, 1.0])
    return x


def test_q8k_quantize_nan_bitwise(ctx):
    """NaN/inf blocks: the block maximum in quantize_avx2's max_ps order, bit for bit, through
    the plain quantizer and through the matvec's own (permuted) one."""
    from spindle_amd import ops
    rng = np.random.default_rng(5)
    n = 2048
    x = _nan_rows(rng, 24, n)
    for lane in range(8):  # one NaN in each lane of the last group, alone in its block
        x[lane, 248 + lane] = np.nan
        x[lane, 256:512] = rng.standard_normal(256)
        x[lane, 256 + 248 + lane] = np.nan
    d, qs, bs = ops.q8k_quantize(ctx, _cuda(x))
    zeroed = 0
    for v in range(x.shape[0]):
        od, oq, ob = ffi.q8k_quantize(x[v])
        zeroed += int((od == 0).sum())
        assert np.array_equal(d[v].cpu().numpy().view(np.uint32), od.view(np.uint32)), v
        assert np.array_equal(qs[v].cpu().numpy(), oq), v
        assert np.array_equal(bs[v].cpu().numpy(), ob), v
    assert zeroed > 0  # some NaN survived to zero its block, as x[255] does
    raw = _rand_kquant(R.Q4K, n, 96, rng)
    w = ops.Tensor(ctx, R.Q4K, n, 96, raw)
    got = ops.matvec(ctx, w, _cuda(x[:6])).cpu().numpy()
    m = ffi.mat(R.Q4K, raw, 96, n)
    for v in range(6):
        want = ffi.matvec(m, x[v])
        assert np.array_equal(got[v].view(np.uint32), want.view(np.uint32)), v


@pytest.mark.parametrize("dtype", [R.Q4K, R.Q6K])
@pytest.mark.parametrize("n", [256, 768, 2048, 4096])
def test_block_sums_bitwise(ctx, dtype, n):
    from spindle_amd import ops
    rng = np.random.default_rng(n + dtype)
    rows = 5
    raw = _rand_kquant(dtype, n, rows, rng)
    w = ops.Tensor(ctx, dtype, n, rows, raw)
    x = rng.standard_normal(n).astype(np.float32)
    q = ffi.q8k_quantize(x)
    qg = tuple(_cuda(a[None]) for a in q)
    rb = R.row_bytes(dtype, n)
    for r in range(rows):
        got = ops.block_sums_q8k(ctx, w, r, qg).cpu().numpy()
        sumi, corr, _ = ffi.q8k_block_sums(raw[r * rb:(r + 1) * rb], dtype, n, q)
        assert np.array_equal(got[:, 0], sumi) and np.array_equal(got[:, 1], corr), (r,)


def test_int_kernel_reference_seed(ctx, mv_mode):
    """The data of quant_q8k.rs:364-411 (seed 0x51ED): GPU vs oracle and vs the f64 dot."""
    from spindle_amd import ops
    rng = R.Rng(0x51ED)
    for dtype in (R.Q4K, R.Q6K):
        for n in (256, 512, 768, 1024, 1536, 2048):
            rows = 37
            mat = R.random_matrix(dtype, n, rows, rng)
            w = ops.Tensor(ctx, dtype, n, rows, mat)
            wd = ffi.dequant(dtype, mat, rows, n).astype(np.float64)
            for bsz in range(1, 12):
                xs = [rng.floats(n, -2.0, 2.0) for _ in range(bsz)]
                qs = [ffi.q8k_quantize(x) for x in xs]
                want = ffi.q8k_matmul_rows(mat, dtype, n, qs, rows)
                qg = tuple(_cuda(np.stack([q[k] for q in qs])) for k in range(3))
                out = torch.full((bsz, rows), float("nan"), device="cuda")
                ops.matmul_rows_q8k(ctx, w, qg, 0, 0, 3, out)
                ops.matmul_rows_q8k(ctx, w, qg, 0, 3, rows, out)
                got = out.cpu().numpy()
                for b in range(bsz):
                    assert np.array_equal(got[b].view(np.uint32), want[b].view(np.uint32)), (dtype, n, bsz, b)
                    xq = (np.repeat(qs[b][0], 256) * qs[b][1]).astype(np.float64)
                    scale = np.abs(wd * xq).sum(1)
                    assert np.all(np.abs(got[b] - wd @ xq) <= 1e-4 * scale + 1e-6)


@pytest.mark.parametrize("dtype", [R.Q4K, R.Q6K])
def test_int_kernel_batch_bitwise(ctx, dtype, mv_mode):
    from spindle_amd import ops
    rng = np.random.default_rng(7)
    n, rows = 2048, 300
    w = ops.Tensor(ctx, dtype, n, rows, _rand_kquant(dtype, n, rows, rng))
    x = _cuda(rng.standard_normal((16, n)).astype(np.float32))
    full = ops.matvec(ctx, w, x).cpu().numpy()
    for m in (1, 2, 3, 5, 8, 9, 13):
        part = ops.matvec(ctx, w, x[:m]).cpu().numpy()
        assert np.array_equal(part.view(np.uint32), full[:m].view(np.uint32)), m
    one = ops.matvec(ctx, w, x[11:12]).cpu().numpy()
    assert np.array_equal(one.view(np.uint32), full[11:12].view(np.uint32))


@pytest.mark.parametrize("dtype,n,rows,ne", [(R.Q4K, 2048, 768, 8), (R.Q6K, 768, 2048, 8), (R.Q4K, 4096, 2048, 1),
                                              (R.Q6K, 2048, 151936, 1)])
def test_int_matvec_real_shapes(ctx, dtype, n, rows, ne, mv_mode):
    """Qwen3-30B-A3B shapes: expert gate/up, expert down, attn_output, LM head, at 1, 2 and 9
    vectors (the default launch: row-parallel lanes, then the int8 matrix cores)."""
    from spindle_amd import ops
    rng = np.random.default_rng(rows)
    raw = _rand_kquant(dtype, n, rows, rng, ne)
    w = ops.Tensor(ctx, dtype, n, rows, raw, ne)
    ffi.set_threads(8)
    for e in sorted({0, ne - 1}):
        m = ffi.mat(dtype, raw[e * rows * R.row_bytes(dtype, n):], rows, n)
        for nv in (1, 2, 9):
            x = rng.standard_normal((nv, n)).astype(np.float32)
            got = ops.matvec(ctx, w, _cuda(x), expert=e).cpu().numpy()
            for v in range(nv):
                want = ffi.matvec(m, x[v])
                assert np.array_equal(got[v].view(np.uint32), want.view(np.uint32)), (e, nv, v)


@pytest.mark.parametrize("n,rows", [(1024, 2048), (2048, 1024), (1024, 3072), (3072, 1024)])
def test_q8_0_multi_config2_shapes(ctx, n, rows):
    """Qwen3-0.6B's Q8_0 projections (q, attn_output, gate/up, down) at 2, 9 and 16 vectors:
    the fp32 matrix-core kernel (k_mv_fq) against the reference's multi-row kernel
    (quant_multi.rs, the oracle's or_matmul_rows_multi) within 1e-4 of the largest output, and
    within the reference's per-row tolerance 1e-4 * sum|w x| + 1e-6 of the f64 dot; a vector's
    bits the same in any batch of two or more."""
    from spindle_amd import ops
    rng = np.random.default_rng(n + rows)
    raw = rng.integers(0, 256, R.row_bytes(R.Q8_0, n) * rows, dtype=np.uint8)
    raw.reshape(-1, 34)[:, 0:2] = np.float16(rng.uniform(0.001, 0.05, raw.size // 34)).view(np.uint8).reshape(-1, 2)
    w = ops.Tensor(ctx, R.Q8_0, n, rows, raw)
    wd = ffi.dequant(R.Q8_0, raw, rows, n).astype(np.float64)
    ffi.set_threads(8)
    x = rng.standard_normal((16, n)).astype(np.float32)
    full = ops.matvec(ctx, w, _cuda(x)).cpu().numpy()
    want = ffi.matmul_rows_multi(raw, R.Q8_0, n, list(x), rows)
    for v in range(16):
        assert _norm_err(full[v], want[v]) <= 1e-4, v
        scale = np.abs(wd * x[v].astype(np.float64)).sum(1)
        assert np.all(np.abs(full[v] - wd @ x[v].astype(np.float64)) <= 1e-4 * scale + 1e-6), v
    for nv, v0 in ((2, 5), (9, 7)):
        part = ops.matvec(ctx, w, _cuda(x[v0:v0 + nv])).cpu().numpy()
        assert np.array_equal(part.view(np.uint32), full[v0:v0 + nv].view(np.uint32)), nv


@pytest.mark.parametrize("dtype", [R.Q8_0, R.Q5_0, R.Q5K, R.F32])
def test_float_matvec(ctx, dtype):
    from spindle_amd import ops
    rng = np.random.default_rng(dtype)
    for n, rows in [(1024, 100), (576, 64), (3072, 65)]:
        if dtype == R.Q5K and n % 256:
            n = 768
        if dtype == R.F32:
            raw = rng.uniform(-1, 1, n * rows).astype(np.float32).view(np.uint8)
        else:
            bb = {R.Q8_0: 34, R.Q5_0: 22, R.Q5K: 176}[dtype]
            raw = rng.integers(0, 256, R.row_bytes(dtype, n) * rows, dtype=np.uint8)
            raw.reshape(-1, bb)[:, 0:2] = np.float16(rng.uniform(0.001, 0.05, raw.size // bb)).view(np.uint8).reshape(-1, 2)
            if dtype == R.Q5K:  # dmin
                raw.reshape(-1, bb)[:, 2:4] = np.float16(rng.uniform(0.001, 0.05, raw.size // bb)).view(np.uint8).reshape(-1, 2)
        w = ops.Tensor(ctx, dtype, n, rows, raw)
        x = rng.standard_normal((9, n)).astype(np.float32)
        got = ops.matvec(ctx, w, _cuda(x)).cpu().numpy()
        wd = ffi.dequant(dtype, raw, rows, n).astype(np.float64)
        m1 = ffi.mat(dtype, raw, rows, n)
        multi = ffi.matmul_rows_multi(raw, dtype, n, list(x), rows)  # the reference's multi-row kernel
        for v in range(9):
            want = ffi.matvec(m1, x[v])              # the reference's M=1 kernel
            assert _norm_err(got[v], want) <= 1e-4
            assert _norm_err(got[v], multi[v]) <= 1e-4
            if dtype == R.Q5K:  # the GPU walker follows the reference's lanes: the same bits
                assert np.array_equal(got[v].view(np.uint32), want.view(np.uint32)), v
            scale = np.abs(wd * x[v].astype(np.float64)).sum(1)
            assert np.all(np.abs(got[v] - wd @ x[v].astype(np.float64)) <= 1e-4 * scale + 1e-6)
        one = ops.matvec(ctx, w, _cuda(x[4:5])).cpu().numpy()
        assert _norm_err(one[0], got[4]) <= 1e-4
        if dtype != R.Q8_0:  # the same walk at any batch size (Q8_0 takes the matrix cores from two rows)
            assert np.array_equal(one.view(np.uint32), got[4:5].view(np.uint32))
        pair = ops.matvec(ctx, w, _cuda(x[4:6])).cpu().numpy()
        assert np.array_equal(pair.view(np.uint32), got[4:6].view(np.uint32))


@pytest.mark.parametrize("dtype,n", [(R.Q4K, 2048), (R.Q6K, 768), (R.Q8_0, 1024), (R.Q5_0, 576), (R.Q5K, 512), (R.F32, 64)])
def test_tensor_round_trip(ctx, dtype, n):
    from spindle_amd import ops
    rng = np.random.default_rng(1)
    raw = rng.integers(0, 256, R.row_bytes(dtype, n) * 7 * 3, dtype=np.uint8)
    w = ops.Tensor(ctx, dtype, n, 7, raw, 3)
    assert np.array_equal(w.download(), raw)
