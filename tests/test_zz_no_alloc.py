"""spx_matvec_noalloc (Q8_K staging in the library's fixed per-device scratch array, no
allocation) against spx_matvec, through the C ABI: bit for bit, on two calls in a row whose
second input is smaller (the array keeps the first call's contents), and a request beyond the
array's size is refused with an error before anything is launched."""
import numpy as np
import pytest

from spindle_amd import model as M

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


def _tensor(ctx, dtype, cols, rows, seed):
    from spindle_amd import ops
    spec = M.TensorSpec(f"t{seed}", dtype, cols, rows)
    return ops.Tensor(ctx, dtype, cols, rows, M.synth_tensor(spec, seed), 1)


@pytest.mark.parametrize("dtype", [M.Q4K, M.Q6K])
def test_noalloc_matches_matvec(ctx, dtype):
    from spindle_amd import ops
    rng = np.random.default_rng(dtype)
    # first call: 16 vectors of 8192 columns; second: 3 vectors of 2048 (a smaller image over the
    # first call's leftovers)
    for i, (cols, rows, m) in enumerate([(8192, 300, 16), (2048, 200, 3)]):
        w = _tensor(ctx, dtype, cols, rows, 100 + i)
        x = torch.from_numpy(rng.standard_normal((m, cols)).astype(np.float32)).cuda()
        want = ops.matvec(ctx, w, x).cpu().numpy()
        got = ops.matvec_noalloc(ctx, w, x).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (dtype, cols, m)
        w.close()


def test_noalloc_refuses_beyond_scratch(ctx):
    from spindle_amd import ops
    from spindle_amd._lib import SpxError
    w = _tensor(ctx, M.Q4K, 65536, 8, 7)
    x = torch.zeros((16, 65536), dtype=torch.float32, device="cuda")
    with pytest.raises(SpxError, match="fixed scratch"):
        ops.matvec_noalloc(ctx, w, x)
    w.close()


def test_noalloc_two_contexts_take_turns(ctx):
    """Two contexts (two streams) call spx_matvec_noalloc back to back with no synchronisation in
    between, several rounds: the second call waits for the first call's kernels through the
    per-device event, so neither overwrites the other's staging (both equal spx_matvec)."""
    from spindle_amd import ops
    from spindle_amd._lib import check, lib
    from spindle_amd.ops import _p
    ctx2 = ops.Context(0)
    try:
        rng = np.random.default_rng(11)
        w = _tensor(ctx, M.Q4K, 8192, 2048, 21)
        xs = [torch.from_numpy(rng.standard_normal((16, 8192)).astype(np.float32)).cuda() for _ in range(2)]
        want = [ops.matvec(ctx, w, x).cpu().numpy() for x in xs]
        for _ in range(4):
            outs = [torch.empty((16, w.rows), dtype=torch.float32, device="cuda") for _ in range(2)]
            torch.cuda.synchronize()
            for c, x, o in zip((ctx, ctx2), xs, outs):
                check(lib.spx_matvec_noalloc(c.h, w.h, 0, _p(x), 8192, 16, _p(o), w.rows))
            ctx.sync()
            ctx2.sync()
            for o, wv in zip(outs, want):
                assert np.array_equal(o.cpu().numpy().view(np.uint32), wv.view(np.uint32))
        w.close()
    finally:
        ctx2.close()
