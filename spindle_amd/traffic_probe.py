"""Workload for rocprofv3 hardware-counter runs (HBM traffic per kernel launch).

Builds the first --layers layers of a model config with synthetic weights, prefills --prompt
tokens in 16-row passes, runs --decode greedy one-row passes (back to back, as bench.py's
timed decode does) and --verify nine-row passes (a token and a k=8 draft, on the int8 matrix
cores), then copies 512 MiB device-to-device and fills 512 MiB: kernels of known traffic to
calibrate the counters against. Run under

  rocprofv3 --pmc FETCH_SIZE -d <dir> -o run --output-format csv -- python3 -m spindle_amd.traffic_probe
  rocprofv3 --pmc WRITE_SIZE -d <dir> -o run --output-format csv -- python3 -m spindle_amd.traffic_probe

and compare each kernel's counter per dispatch with the copy's (a 512 MiB copy reads and
writes 512 MiB). `--summarize <run_counter_collection.csv>` prints the mean counter value per
dispatch of every (kernel, grid size, counter) triple (values in the counter's own unit; the
traffic counters count KiB).
"""
import argparse
import os
import sys

import numpy as np


def summarize(path):
    import collections
    import csv
    by = collections.defaultdict(list)
    with open(path) as f:
        for r in csv.DictReader(f):
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
    ap.add_argument("--summarize", metavar="CSV", help="summarise a counter_collection.csv instead")
    args = ap.parse_args()
    if args.summarize:
        summarize(args.summarize)
        return
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import torch
    from spindle_amd import model as M, ops
    cfg = M.get_config(args.config)
    cfg = cfg.replace(n_layers=min(args.layers, cfg.n_layers), max_seq=args.prompt + args.decode + 64)
    assert args.verify == 0 or args.prompt >= 1024 + 9, "--verify passes run at position 1024"
    w = M.synth_model(cfg, 1)
    ctx = ops.Context(0)
    eng = M.Engine(ctx, cfg, w)
    ids = np.random.default_rng(0).integers(0, cfg.vocab, args.prompt)
    am = None
    for s in range(0, args.prompt, 16):
        am, _, _ = eng.forward(ids[s:s + 16], s)
        if s % 1024 == 0:
            print(f"prefill {s + 16}/{args.prompt}", flush=True)
    eng.decode(int(am[-1]), args.prompt, args.decode)
    ctx.sync()
    print(f"decode {args.decode} passes done", flush=True)
    for _ in range(args.verify):  # rows 100..108 of the prompt at position 1024 (K/V rows rewritten in place)
        eng.forward(ids[100:109], 1024)
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
