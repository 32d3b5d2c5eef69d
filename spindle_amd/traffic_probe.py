"""Workload for rocprofv3 hardware-counter runs (HBM traffic per kernel launch).

Builds the first --layers layers of a model config with synthetic weights, prefills --prompt
tokens in passes of --pf-rows rows (16 by default), runs --decode greedy one-row passes (back
to back, as bench.py's timed decode does) and --verify nine-row passes (a token and a k=8
draft, on the int8 matrix cores) at --verify-pos (1024 by default; the K/V rows there are
rewritten in place), then copies 512 MiB device-to-device and fills 512 MiB: kernels of known traffic to
calibrate the counters against. Run under

  rocprofv3 --pmc FETCH_SIZE -d <dir> -o run --output-format csv -- python3 -m spindle_amd.traffic_probe
  rocprofv3 --pmc WRITE_SIZE -d <dir> -o run --output-format csv -- python3 -m spindle_amd.traffic_probe

and compare each kernel's counter per dispatch with the copy's (a 512 MiB copy reads and
writes 512 MiB). `--summarize <run_counter_collection.csv>` prints the mean counter value per
dispatch of every (kernel, grid size, counter) triple (values in the counter's own unit; the
traffic counters count KiB); --after / --before KERNEL keep one phase of the run (the dispatches
after the last, or before the first, dispatch of that kernel).
"""
import argparse
import os
import sys

import numpy as np


def summarize(path, after=None, before=None):
    """Mean counter value per dispatch of every (kernel, counter, grid size); with `after`, only
    the dispatches after the last one whose kernel name contains it; with `before`, only those
    before the first such dispatch (in dispatch order)."""
    import collections
    import csv
    with open(path) as f:
        rows = list(csv.DictReader(f))
    key = "Dispatch_Id" if rows and "Dispatch_Id" in rows[0] else "Correlation_Id"
    rows.sort(key=lambda r: int(r[key]))
    if after:
        last = max((int(r[key]) for r in rows if after in r["Kernel_Name"]), default=-1)
        rows = [r for r in rows if int(r[key]) > last]
    if before:
        first = min((int(r[key]) for r in rows if before in r["Kernel_Name"]), default=1 << 62)
        rows = [r for r in rows if int(r[key]) < first]
    by = collections.defaultdict(list)
    for r in rows:
        by[(r["Kernel_Name"].split("(")[0], r.get("Counter_Name", ""), r["Grid_Size"])].append(float(r["Counter_Value"]))
    for (n, c, g), v in sorted(by.items(), key=lambda kv: -sum(kv[1])):
        print(f"{n[:48]:48s} {c:26s} grid {g:>9s} n={len(v):6d} mean {sum(v) / len(v):14.1f}")


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--config", default="qwen3-30b-a3b")
    ap.add_argument("--layers", type=int, default=4)
    ap.add_argument("--prompt", type=int, default=4096)
    ap.add_argument("--decode", type=int, default=40)
    ap.add_argument("--verify", type=int, default=0, help="nine-row passes after the decode passes")
    ap.add_argument("--verify-pos", type=int, default=1024, help="position of the nine-row passes")
    ap.add_argument("--pf-rows", type=int, default=16, help="rows per prefill pass (1..128)")
    ap.add_argument("--summarize", metavar="CSV", help="summarise a counter_collection.csv instead")
    ap.add_argument("--after", metavar="KERNEL", help="--summarize: dispatches after the last of KERNEL")
    ap.add_argument("--before", metavar="KERNEL", help="--summarize: dispatches before the first of KERNEL")
    args = ap.parse_args()
    if args.summarize:
        summarize(args.summarize, args.after, args.before)
        return
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import torch
    from spindle_amd import model as M, ops
    cfg = M.get_config(args.config)
    cfg = cfg.replace(n_layers=min(args.layers, cfg.n_layers), max_seq=args.prompt + args.decode + 64)
    assert args.verify == 0 or 0 <= args.verify_pos <= args.prompt + args.decode + 64 - 9, "--verify-pos"
    assert 1 <= args.pf_rows <= 128, "--pf-rows"
    w = M.synth_model(cfg, 1)
    ctx = ops.Context(0)
    eng = M.Engine(ctx, cfg, w)
    ids = np.random.default_rng(0).integers(0, cfg.vocab, args.prompt)
    am = None
    r = args.pf_rows
    for s in range(0, args.prompt, r):
        am, _, _ = eng.forward(ids[s:s + r], s)
        if s // 1024 != (s + r) // 1024:
            print(f"prefill {min(s + r, args.prompt)}/{args.prompt}", flush=True)
    eng.decode(int(am[-1]), args.prompt, args.decode)
    ctx.sync()
    print(f"decode {args.decode} passes done", flush=True)
    for _ in range(args.verify):  # rows 100..108 of the prompt (K/V rows at --verify-pos rewritten in place)
        eng.forward(ids[100:109], args.verify_pos)
    ctx.sync()
    if args.verify:
        print(f"verify {args.verify} nine-row passes done", flush=True)
    x = torch.empty(128 * 1024 * 1024, dtype=torch.float32, device="cuda")
    x.fill_(1.0)
    y = x.clone()
    torch.cuda.synchronize()
    print("calibration: 512 MiB fill and 512 MiB copy done", flush=True)
    eng.close()


if __name__ == "__main__":
    main()
