"""Per-phase times of the persistent one-row pass against the kernel pipeline.

The persistent pass (csrc/persist.hip) runs each layer as one cooperative launch whose phases
(q|k|v, attention partials, merge, attn_output, router, gate/up, down) meet at device-wide
barriers. With SPX_PERSIST_TSTAMP set at engine preparation, workgroup 0 records the real-time
counter (100 MHz) when a layer's launch starts and when it arrives at and leaves each barrier;
this tool reads those stamps back after a few decode steps and prints, per phase, the median
over the layers of workgroup 0's work before the barrier and its wait at the barrier (the wait
is the time until the slowest workgroup arrives, plus the hand-off). The last phase (down)
runs to the next layer's launch, so it includes the launch boundary.

    python3 -m spindle_amd.phase_probe [--config qwen3-30b-a3b] [--prompt 4096] [--steps 10]
"""
import argparse
import ctypes
import os
import sys
import time

import numpy as np

PHASES = ("q|k|v", "attention", "merge", "attn_output", "router", "gate/up", "down")


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--config", default="qwen3-30b-a3b")
    ap.add_argument("--prompt", type=int, default=4096)
    ap.add_argument("--steps", type=int, default=10)
    args = ap.parse_args(argv)
    os.environ["SPX_PERSIST_TSTAMP"] = "1"
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    if root not in sys.path:
        sys.path.insert(0, root)
    from spindle_amd import model as M, ops
    from spindle_amd._lib import check, lib
    import bench as B

    cfg = M.CONFIGS[args.config]
    if not cfg.moe:
        sys.exit("phase_probe: the stamps follow a MoE layer's seven phases")
    ctx = ops.Context(0)
    eng = M.Engine(ctx, cfg, M.synth_model(cfg, 1))
    prompt = B.spec_prompt(cfg.vocab, args.prompt, 1)
    tok, _ = B.prefill(eng, prompt)
    pos = len(prompt)
    for mode in (False, True):
        eng.set_persist(mode)
        out = eng.decode(tok, pos, 4)
        ctx.sync()
        pos, tok = pos + 4, int(out[-1])
        t0 = time.perf_counter()
        out = eng.decode(tok, pos, args.steps)
        ctx.sync()
        dt = time.perf_counter() - t0
        pos, tok = pos + args.steps, int(out[-1])
        print(f"{'persistent pass' if mode else 'kernel pipeline'}: {dt / args.steps * 1e3:.3f} ms/token ({args.steps / dt:.1f} tok/s)")
    buf = np.zeros(4096, np.uint64)
    check(lib.spx_engine_debug_read(eng.h, b"tstamp", buf.ctypes.data_as(ctypes.c_void_p), buf.nbytes))
    L = cfg.n_layers
    start = buf[1024:1024 + 2 * L:2].astype(np.int64)
    work = np.zeros((L - 1, 7))
    wait = np.zeros((L - 1, 6))
    for li in range(L - 1):  # the last layer's down phase has no next launch to end it
        prev = int(start[li])
        for k in range(6):
            arrive, leave = int(buf[2 * (6 * li + k)]), int(buf[2 * (6 * li + k) + 1])
            work[li, k] = (arrive - prev) / 100.0
            wait[li, k] = (leave - arrive) / 100.0
            prev = leave
        work[li, 6] = (int(start[li + 1]) - prev) / 100.0
    w, b = np.median(work, axis=0), np.median(wait, axis=0)
    print(f"per layer, median over layers 0..{L - 2} (us): phase work of workgroup 0 | wait at the barrier after it")
    for k, name in enumerate(PHASES):
        print(f"  {name:12s} {w[k]:7.2f} | " + (f"{b[k]:6.2f}" if k < 6 else "   (to the next layer's launch)"))
    print(f"  work {w.sum():.1f} + barriers {b.sum():.1f} = layer {np.median(np.diff(start)) / 100.0:.1f} us")
    eng.close()
    ctx.close()


if __name__ == "__main__":
    main()
