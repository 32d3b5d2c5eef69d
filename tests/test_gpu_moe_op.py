"""spx_moe (ffns_fused smollm_chat.rs:379-442 / moe_batch_fused :650-760 with the combine
:1133-1140, routing given) against the oracle's ffns_fused row by row, and a row's result the
same bits whatever the other rows; bad routing refused.

Bars: the integer path (Q4_K gate/up, Q6_K down) within 1e-5 of the largest output: the
integer dots are the reference's bits, but SiLU's exp on the GPU can round an h value one ulp
away from the C library's, which may move a Q8_K code of h; the fp32 path (Q8_0) within its
1e-4 bar."""
import ctypes as C

import numpy as np
import pytest

from oracle import ffi
from spindle_amd._lib import SpxError
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


def _experts(ctx, tg, td, dim, nff, ne, seed):
    from spindle_amd import model as M, ops
    out = {}
    for name, dt, cols, rows in [("gate", tg, dim, nff), ("up", tg, dim, nff), ("down", td, nff, dim)]:
        spec = M.TensorSpec(name, dt, cols, rows, ne, sigma=0.05)
        raw = M.synth_tensor(spec, seed)
        out[name] = (raw, ops.Tensor(ctx, dt, cols, rows, raw, ne), ffi.mat(dt, raw, rows, cols))
    return out


def _oracle_row(ex, x, chosen, weights):
    o = np.zeros(ex["down"][1].rows, np.float32)
    ch = np.ascontiguousarray(chosen, np.int32)
    wt = np.ascontiguousarray(weights, np.float32)
    assert ffi.lib.or_ffns_fused(C.byref(ex["gate"][2]), C.byref(ex["up"][2]), C.byref(ex["down"][2]), ch.size,
                                 ffi.ptr(ch), ffi.ptr(wt), ffi.ptr(np.ascontiguousarray(x, np.float32)), ffi.ptr(o)) == 0
    return o


@pytest.mark.parametrize("fmt", ["kquant", "q8_0"])
@pytest.mark.parametrize("m,k", [(1, 8), (3, 4), (9, 8), (16, 8)])
def test_moe_matches_oracle(ctx, fmt, m, k):
    from spindle_amd import ops
    dim, nff, ne = (512, 256, 16) if fmt == "kquant" else (256, 128, 8)
    k = min(k, ne)
    tg, td = (R.Q4K, R.Q6K) if fmt == "kquant" else (R.Q8_0, R.Q8_0)
    ex = _experts(ctx, tg, td, dim, nff, ne, seed=m * 10 + k)
    rng = np.random.default_rng(m + k)
    x = rng.standard_normal((m, dim)).astype(np.float32)
    chosen = np.stack([rng.permutation(ne)[:k] for _ in range(m)]).astype(np.int32)
    weights = rng.dirichlet(np.ones(k), m).astype(np.float32)
    y = ops.moe(ctx, ex["gate"][1], ex["up"][1], ex["down"][1], torch.from_numpy(x).cuda(), chosen, weights).cpu().numpy()
    for b in range(m):
        want = _oracle_row(ex, x[b], chosen[b], weights[b])
        bar = 1e-5 if fmt == "kquant" else 1e-4
        assert np.abs(y[b] - want).max() <= bar * np.abs(want).max(), b
        alone = ops.moe(ctx, ex["gate"][1], ex["up"][1], ex["down"][1], torch.from_numpy(x[b:b + 1]).cuda(), chosen[b:b + 1],
                        weights[b:b + 1]).cpu().numpy()
        assert np.array_equal(alone[0].view(np.uint32), y[b].view(np.uint32)), b


def test_moe_refuses_bad_routing(ctx):
    from spindle_amd import ops
    ex = _experts(ctx, R.Q4K, R.Q6K, 512, 256, 16, seed=1)
    x = torch.zeros((1, 512), device="cuda")
    with pytest.raises(SpxError, match="twice"):
        ops.moe(ctx, ex["gate"][1], ex["up"][1], ex["down"][1], x, [[3, 3]], [[0.5, 0.5]])
    with pytest.raises(SpxError, match="out of range"):
        ops.moe(ctx, ex["gate"][1], ex["up"][1], ex["down"][1], x, [[3, 16]], [[0.5, 0.5]])


@pytest.mark.parametrize("fmt", [(R.Q4K, R.Q6K), (R.Q6K, R.Q4K)], ids=["q4k-q6k", "q6k-q4k"])
@pytest.mark.parametrize("m,k", [(1, 8), (9, 8), (16, 8), (64, 8)])
def test_moe_dev_matches_oracle(ctx, fmt, m, k):
    """spx_moe_dev (routing in device memory, the prefill pass's matrix-core kernels): each row
    within the integer path's 1e-5 bar of the oracle, and the same bits as spx_moe (host
    routing, the lane-exact kernels) wherever spx_moe takes the batch (m * k <= 256)."""
    from spindle_amd import ops
    dim, nff, ne = 512, 256, 16
    ex = _experts(ctx, fmt[0], fmt[1], dim, nff, ne, seed=m * 7 + k)
    rng = np.random.default_rng(100 + m)
    x = rng.standard_normal((m, dim)).astype(np.float32)
    chosen = np.stack([rng.permutation(ne)[:k] for _ in range(m)]).astype(np.int32)
    weights = rng.dirichlet(np.ones(k), m).astype(np.float32)
    xd = torch.from_numpy(x).cuda()
    y = ops.moe_dev(ctx, ex["gate"][1], ex["up"][1], ex["down"][1], xd, torch.from_numpy(chosen).cuda(),
                    torch.from_numpy(weights).cuda()).cpu().numpy()
    rows = range(m) if m <= 16 else [0, 1, m // 2, m - 1]
    for b in rows:
        want = _oracle_row(ex, x[b], chosen[b], weights[b])
        assert np.abs(y[b] - want).max() <= 1e-5 * np.abs(want).max(), b
    if m * k <= 256:
        host = ops.moe(ctx, ex["gate"][1], ex["up"][1], ex["down"][1], xd, chosen, weights).cpu().numpy()
        assert np.array_equal(host.view(np.uint32), y.view(np.uint32))


def test_moe_dev_bad_rows_nan(ctx):
    """A row whose ids repeat or leave the expert range comes back NaN; the other rows keep
    their bits (spx_moe refuses such a call on the host; on the device no error can be raised
    without a wait)."""
    from spindle_amd import ops
    ex = _experts(ctx, R.Q4K, R.Q6K, 512, 256, 16, seed=3)
    rng = np.random.default_rng(5)
    x = torch.from_numpy(rng.standard_normal((4, 512)).astype(np.float32)).cuda()
    chosen = np.array([[1, 2], [3, 3], [4, 16], [5, 6]], np.int32)
    weights = np.full((4, 2), 0.5, np.float32)
    y = ops.moe_dev(ctx, ex["gate"][1], ex["up"][1], ex["down"][1], x, torch.from_numpy(chosen).cuda(),
                    torch.from_numpy(weights).cuda()).cpu().numpy()
    assert np.isnan(y[1]).all() and np.isnan(y[2]).all()
    good = ops.moe_dev(ctx, ex["gate"][1], ex["up"][1], ex["down"][1], x[[0, 3]], torch.from_numpy(chosen[[0, 3]]).cuda(),
                       torch.from_numpy(weights[[0, 3]]).cuda()).cpu().numpy()
    assert np.array_equal(good.view(np.uint32), y[[0, 3]].view(np.uint32))
