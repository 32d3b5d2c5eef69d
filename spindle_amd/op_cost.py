"""Cost per call of the operator entry points at Qwen3-30B-A3B shapes.

spx_matvec on attn_output (Q4_K, 4096 -> 2048) and the LM head (Q6_K, 2048 -> 151936) at 1, 9
and 16 vectors; spx_moe (routing on the host) and spx_moe_dev (routing in device memory) on the
128 experts of a layer (Q4_K gate / up 2048 -> 768, Q6_K down 768 -> 2048) with k = 8 at 1, 9
and 16 rows, random distinct choices a row. Each call is timed two ways: back to back on the
context's stream (wall time / calls after a final wait) and followed by a wait each time.
spx_moe_dev's output is compared bit for bit with spx_moe's.

    python3 -m spindle_amd.op_cost
"""
import ctypes as C
import os
import sys
import time

import numpy as np


def _rand_kq(R, dtype, n, rows, ne, rng):
    """Random K-quant blocks with fp16 scales in 0.001..0.05."""
    bb = 144 if dtype == R.Q4K else 210
    raw = rng.integers(0, 256, R.row_bytes(dtype, n) * rows * ne, dtype=np.uint8)
    blk = raw.reshape(-1, bb)
    sc = np.float16(rng.uniform(0.001, 0.05, blk.shape[0] * 2)).view(np.uint8).reshape(-1, 4)
    if dtype == R.Q4K:
        blk[:, 0:4] = sc
    else:
        blk[:, 208:210] = sc[:, 0:2]
    return raw


def main():
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    if root not in sys.path:
        sys.path.insert(0, root)
    import torch
    from spindle_amd import ops
    from spindle_amd import model as R
    from spindle_amd._lib import check, lib

    def p(t):
        return C.c_void_p(t.data_ptr())

    ctx = ops.Context(0)
    rng = np.random.default_rng(1)

    def timeit(fn, n=50):
        fn()
        ctx.sync()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        ctx.sync()
        tb = (time.perf_counter() - t0) / n * 1e6
        t0 = time.perf_counter()
        for _ in range(10):
            fn()
            ctx.sync()
        return tb, (time.perf_counter() - t0) / 10 * 1e6

    for name, dt, n, rows in [("attn_output Q4_K 4096->2048", R.Q4K, 4096, 2048), ("LM head Q6_K 2048->151936", R.Q6K, 2048, 151936)]:
        w = ops.Tensor(ctx, dt, n, rows, _rand_kq(R, dt, n, rows, 1, rng))
        for m in (1, 9, 16):
            x = torch.randn(m, n, device="cuda")
            y = torch.empty(m, rows, device="cuda")
            torch.cuda.synchronize()
            tb, tl = timeit(lambda: check(lib.spx_matvec(ctx.h, w.h, 0, p(x), n, m, p(y), rows)))
            print(f"spx_matvec {name} m={m}: {tb:.1f} us back to back, {tl:.1f} us with a wait; "
                  f"{w.nbytes / 1e6:.1f} MB of weights -> {w.nbytes / tb / 1e3:.0f} GB/s", flush=True)
        w.free()
    ne, dim, nff, k = 128, 2048, 768, 8
    g = ops.Tensor(ctx, R.Q4K, dim, nff, _rand_kq(R, R.Q4K, dim, nff, ne, rng), ne)
    u = ops.Tensor(ctx, R.Q4K, dim, nff, _rand_kq(R, R.Q4K, dim, nff, ne, rng), ne)
    d = ops.Tensor(ctx, R.Q6K, nff, dim, _rand_kq(R, R.Q6K, nff, dim, ne, rng), ne)
    for m in (1, 9, 16):
        x = torch.randn(m, dim, device="cuda")
        y = torch.empty(m, dim, device="cuda")
        ch = np.stack([rng.permutation(ne)[:k] for _ in range(m)]).astype(np.int32)
        wt = rng.dirichlet(np.ones(k), m).astype(np.float32)
        chd, wtd = torch.from_numpy(ch).cuda(), torch.from_numpy(wt).cuda()
        torch.cuda.synchronize()
        used = len(set(ch.ravel().tolist()))
        mb = used * (g.nbytes + u.nbytes + d.nbytes) / ne / 1e6
        tb, tl = timeit(lambda: check(lib.spx_moe(ctx.h, g.h, u.h, d.h, p(x), dim, m, k, ch.ctypes.data_as(C.c_void_p),
                                                  wt.ctypes.data_as(C.c_void_p), p(y), dim)))
        print(f"spx_moe m={m} ({used} experts, {mb:.1f} MB): {tb:.1f} us back to back, {tl:.1f} us with a wait", flush=True)
        y1 = y.clone()
        tb, tl = timeit(lambda: check(lib.spx_moe_dev(ctx.h, g.h, u.h, d.h, p(x), dim, m, k, p(chd), p(wtd), p(y), dim)))
        print(f"spx_moe_dev m={m}: {tb:.1f} us back to back, {tl:.1f} us with a wait; same bits as spx_moe: "
              f"{bool(torch.equal(y, y1))}", flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
