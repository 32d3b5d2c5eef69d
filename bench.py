#!/usr/bin/env python3
"""Benchmark of the decode / verify hot path on one MI355X (BASELINE.json's metric).

Workload: Qwen3-30B-A3B-shaped Q4_K_M model (random-init, GGUF block layout, ~17 GiB,
resident in HBM), a 4096-token repeated-span synthetic prompt, then
  * decode: K greedy one-token passes (M=1) at context ~4.1K -> value = decode tok/s;
  * verify: greedy generation with prompt-lookup drafts (n-gram 3, k=8, fixed length), M=9
    verify passes -> verify-pass us, mean accepted tokens per pass, end-to-end tok/s;
  * kernel profile: HIP events around every launch of a few eager decode passes; the kernel
    class with the most time is the roofline line (algorithmic bytes per launch / average
    launch time vs the 8 TB/s HBM peak);
  * cpu_baseline: the C oracle (the reference's AVX2 arithmetic restated in C, pthreads over
    rows like the reference's worker pool) decoding a few tokens from the same KV state.
Prints ONE JSON line on stdout; progress goes to stderr.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0

# HBM bytes per M=1 decode launch at context ~4.1K, measured with rocprofv3 hardware counters
# (FETCH_SIZE x 2.0 + WRITE_SIZE x 1.0, factors from a 512 MiB copy measured the same way) by
# spindle_amd.traffic_probe; profiles/decode_qwen3_30b_a3b_hbm_traffic.txt holds the runs. The
# attention class is the split-K kernel plus its merge. Counters cannot be read inside a timed
# run, so the bench reports this measurement.
MEASURED_TRAFFIC = {
    "attention": 11_692_237, "qkv_matvec": 6_446_080, "attn_output_matvec": 4_982_784,
    "router_route": 1_236_992, "gate_up_swiglu": 14_435_021, "down_combine": 10_970_112,
    "lm_head_matvec": 256_769_434,
}


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def spec_prompt(vocab, n, seed):
    """BASELINE.json config 3's construction at length n: n/2 random tokens, then copied spans
    of 16..64 tokens from the first half, each token replaced by a random one with p = 0.1."""
    rng = np.random.default_rng(seed)
    half = n // 2
    head = rng.integers(0, vocab, half)
    tail = []
    while len(tail) < n - half:
        ln = int(rng.integers(16, 65))
        s = int(rng.integers(0, half - 16))
        for t in head[s:s + ln]:
            tail.append(int(rng.integers(0, vocab)) if rng.random() < 0.1 else int(t))
    return np.concatenate([head, np.array(tail[:n - half])]).astype(np.int32)


def decode_bytes(cfg, specs, pos, experts_per_layer):
    """Algorithmic HBM bytes of one decode pass at position pos (weights read once, the
    experts actually selected, K and V of positions 0..pos)."""
    from spindle_amd.model import row_bytes
    by = 0.0
    for s in specs:
        b = row_bytes(s.dtype, s.cols) * s.rows
        if s.name == "token_embd.weight":
            by += row_bytes(s.dtype, s.cols) if not cfg.tied else b  # one row, or the tied LM head
        elif "_exps" in s.name:
            layer = int(s.name.split(".")[1])
            by += b * experts_per_layer[layer]
        else:
            by += b * s.n_expert
    by += cfg.n_layers * (pos + 1) * cfg.kv_dim * 2 * 2
    return by


def cpu_info(threads):
    """Model name, sockets, physical cores of the host (and of the cores this process may use),
    from /proc/cpuinfo and the sysfs topology."""
    info = {"model": None, "sockets": None, "physical_cores": None, "threads_used": threads}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    info["model"] = line.split(":", 1)[1].strip()
                    break
        pkgs, cores = set(), set()
        for c in sorted(os.sched_getaffinity(0)):
            base = f"/sys/devices/system/cpu/cpu{c}/topology/"
            pk = open(base + "physical_package_id").read().strip()
            co = open(base + "core_id").read().strip()
            pkgs.add(pk)
            cores.add((pk, co))
        info["sockets"] = len(pkgs)
        info["physical_cores"] = len(cores)
    except OSError:
        pass
    return info


def cpu_baseline(cfg, w, eng, tok, pos, seconds, threads):
    from oracle import ffi
    from oracle.model import OracleModel
    ffi.set_threads(threads)
    om = OracleModel(cfg, w)
    k, v = eng.kv_cache()
    om.k_cache[:] = k
    om.v_cache[:] = v
    n, t0 = 0, time.perf_counter()
    while True:
        h = om.forward([tok], pos + n)
        tok = om.argmax(om.logits(h)[0])
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds or n >= 64:
            break
    return n / el, n, el


# the reference's one-thread kernel bench shapes (bench_int_vs_float, src/quant_q8k.rs:450-455)
BENCH_INT_SHAPES = (("Q4_K expert gate/up (2048 cols)", "Q4K", 2048, 768 * 16),
                    ("Q6_K expert down (768 cols)", "Q6K", 768, 2048 * 16),
                    ("Q4_K expert down (768 cols)", "Q4K", 768, 2048 * 16),
                    ("Q6_K LM-head slice (2048 cols)", "Q6K", 2048, 16384))


def cpu_microbench(seed, seconds=0.3):
    """One thread: the C oracle's AVX2 integer rows kernel (the reference's rows<B, T> and its
    Q8_K activations) on the reference's bench_int_vs_float shapes, 1 and 8 vectors: us per call
    and GB/s of weight bytes, comparable with the reference's own single-thread figures."""
    from oracle import ffi
    from spindle_amd import model as M
    ffi.set_threads(1)
    rng = np.random.default_rng(seed)
    res = []
    for name, dt, cols, rows in BENCH_INT_SHAPES:
        dtype = getattr(M, dt)
        data = M.synth_tensor(M.TensorSpec(name, dtype, cols, rows), seed)
        for b in (1, 8):
            qs = [ffi.q8k_quantize(rng.uniform(-1.0, 1.0, cols).astype(np.float32)) for _ in range(b)]
            outs = [np.empty(rows, np.float32) for _ in range(b)]
            ffi.q8k_matmul_rows(data, dtype, cols, qs, rows, outs=outs)
            n, t0 = 0, time.perf_counter()
            while True:
                ffi.q8k_matmul_rows(data, dtype, cols, qs, rows, outs=outs)
                n += 1
                el = time.perf_counter() - t0
                if el >= seconds:
                    break
            us = el / n * 1e6
            res.append({"shape": name, "rows": rows, "cols": cols, "vectors": b, "us": round(us, 1),
                        "weight_gb_s": round(data.size / us / 1e3, 2)})
    return res


def time_pass(eng, ids, pos, reps=20):
    """Median wall time (us) of one pass of len(ids) rows at pos (graph replay, ids in and picks
    out, synchronised), over reps passes after three warm ones."""
    for _ in range(3):
        eng.forward(ids, pos)
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        eng.forward(ids, pos)
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts)) * 1e6


PREFILL_CHUNK = 128  # feed's prompt chunks (smollm_chat.rs:3090)


def prefill(eng, prompt, verbose=False):
    """feed (spx_engine_feed): 128-row passes, logits for the last prompt row only."""
    t0 = time.perf_counter()
    am, _, _ = eng.feed(prompt, 0)
    if verbose:
        log(f"prefill {len(prompt)} rows")
    return int(am), time.perf_counter() - t0


def timed_decode(ctx, eng, tok, pos, warmup, steps):
    out = eng.decode(tok, pos, warmup)
    tok, pos = int(out[-1]), pos + warmup
    ctx.sync()
    t0 = time.perf_counter()
    out = eng.decode(tok, pos, steps)
    ctx.sync()
    return steps / (time.perf_counter() - t0), int(out[-1]), pos + steps


def small_config_leg(ctx, name, seed, prompt_len, spans, steps):
    """decode tok/s at the config's context, one M=9 pass, and for the
    repeated-span prompts the speculative generation (n-gram 3, k=8, fixed)."""
    from spindle_amd import model as M
    cfg = M.CONFIGS[name]
    w = M.synth_model(cfg, seed)
    eng = M.Engine(ctx, cfg, w)
    prompt = spec_prompt(cfg.vocab, prompt_len, seed) if spans else \
        np.random.default_rng(seed).integers(0, cfg.vocab, prompt_len).astype(np.int32)
    tok, _ = prefill(eng, prompt)
    tok_s, tok, pos = timed_decode(ctx, eng, tok, len(prompt), 4, steps)
    by = decode_bytes(cfg, M.tensor_specs(cfg), pos - steps // 2,
                      eng.last_experts() if cfg.moe else [0] * cfg.n_layers)
    r = {"decode_tok_s": round(tok_s, 1), "decode_gb_per_pass": round(by / 1e9, 4),
         "decode_roofline_frac": round(by * tok_s / 1e9 / HBM_PEAK_GBS, 4), "context": pos}
    m9 = time_pass(eng, prompt[-9:], pos)
    r["verify_m9_pass_us"] = round(m9, 1)
    if spans:
        toks, st = eng.generate(prompt, 128, draft_len=8, min_ngram=3, max_ngram=3, fixed=True,
                                adaptive_k=False, n_cached=len(prompt) - 1)
        r["spec_tok_s"] = round(len(toks) / ((st["verify_us"] + st["step_us"]) / 1e6), 1)
        r["verify_pass_us"] = round(st["verify_us"] / max(1, st["verifies"]), 1)
        r["accepted_per_pass"] = round(st["accepted"] / max(1, st["verifies"]), 3)
    log(f"config {name}: {r}")
    eng.close()
    return r


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128, help="timed decode passes")
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--config", default="qwen3-30b-a3b")
    ap.add_argument("--prompt-len", type=int, default=4096)
    ap.add_argument("--spec-tokens", type=int, default=256)
    ap.add_argument("--profile-passes", type=int, default=4)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--cpu-threads", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-legs", action="store_true", help="skip the prune / diverse-routing / configs 1-4 legs")
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--prefill-only", action="store_true",
                    help="build the model, prefill the prompt in 128-row passes, report prompt tok/s and exit (no JSON line)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the whole model fits in one MI355X's HBM and this build "
              "has no multi-GPU path (the expert slabs would shard by expert over the GPUs, with one "
              "all-to-all of the routed rows each way a layer). Use --gpus 1.", file=sys.stderr)
        sys.exit(2)

    from spindle_amd import model as M
    from spindle_amd import ops

    cfg = M.get_config(args.config)
    need = args.prompt_len + args.warmup + args.steps + 3 * args.profile_passes + 64
    if cfg.max_seq < need:
        cfg = cfg.replace(max_seq=need)
    specs = M.tensor_specs(cfg)
    t0 = time.perf_counter()
    w = M.synth_model(cfg, args.seed)
    gib = sum(d.size for _, d in w.values()) / 2**30
    log(f"synthetic {cfg.name}: {gib:.2f} GiB in {time.perf_counter() - t0:.1f}s")
    ctx = ops.Context(0)
    t0 = time.perf_counter()
    eng = M.Engine(ctx, cfg, w)
    log(f"uploaded in {time.perf_counter() - t0:.1f}s")

    prompt = spec_prompt(cfg.vocab, args.prompt_len, args.seed)
    tok, prefill_s = prefill(eng, prompt, verbose=True)
    pos = len(prompt)
    log(f"prefill {len(prompt)} tokens in {prefill_s:.2f}s ({len(prompt) / prefill_s:.0f} tok/s, {PREFILL_CHUNK}-row passes)")
    if args.prefill_only:
        return

    # CPU baseline from the KV state the GPU's timed decode starts from (read-only on the GPU)
    cpu = None
    if not args.no_cpu_baseline:
        threads = min(args.cpu_threads, len(os.sched_getaffinity(0)))
        cpu_tok_s, n_cpu, el = cpu_baseline(cfg, w, eng, tok, pos, args.cpu_seconds, threads)
        ci = cpu_info(threads)
        log(f"cpu baseline (oracle, {threads} threads on {ci}): {n_cpu} tokens in {el:.1f}s = {cpu_tok_s:.3f} tok/s")
        cpu = {"value": round(cpu_tok_s, 4), "unit": "tok/s", "cores": threads, "kind": "port",
               "sample": f"{n_cpu} greedy decode passes at positions {pos}..{pos + n_cpu - 1} from the KV state the GPU "
                         f"decode starts from (same weights, C restatement of the reference's AVX2 kernels, {threads} threads)",
               "cpu": ci}
        cpu["microbench_1thread"] = cpu_microbench(args.seed)
        for r in cpu["microbench_1thread"]:
            log(f"cpu 1-thread {r['shape']}, {r['vectors']} vector(s): {r['us']:.0f} us, {r['weight_gb_s']:.2f} GB/s")

    # warmup, then the timed decode passes (back-to-back graph replays, picks fed forward on the device)
    tok_s, tok, pos = timed_decode(ctx, eng, tok, pos, args.warmup, args.steps)
    experts = eng.last_experts()
    dec_bytes = decode_bytes(cfg, specs, pos - args.steps // 2, experts)
    log(f"decode: {args.steps} passes = {tok_s:.1f} tok/s, "
        f"{dec_bytes / 1e9:.3f} GB/pass -> {dec_bytes * tok_s / 1e9:.0f} GB/s end to end")

    # per-kernel profile of eager decode passes (HIP events on the engine's stream): three rounds
    # of profile_passes, each class's figures from its fastest round (a one-off stall of the host
    # or the box inside one class's events would otherwise decide the roofline kernel)
    prof = {}
    for _ in range(3):
        eng.profile(True)
        out = eng.decode(tok, pos, args.profile_passes)
        eng.profile(False)
        for k, v in eng.profile_read().items():
            if k not in prof or (v[0] and v[1] < prof[k][1]):
                prof[k] = v
        tok, pos = int(out[-1]), pos + args.profile_passes
    tot = sum(v[1] for v in prof.values())
    for name, (n, us, by) in sorted(prof.items(), key=lambda kv: -kv[1][1]):
        if n:
            log(f"  {name:22s} {n:6d} launches {us / args.profile_passes:9.1f} us/pass ({100 * us / tot:4.1f}%)"
                + (f"  {by / us / 1e3:8.1f} GB/s" if by > 0 else ""))
    dom = max((k for k in prof if prof[k][2] > 0), key=lambda k: prof[k][1])
    n, us, by = prof[dom]
    achieved = by / us / 1e3
    roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": MEASURED_TRAFFIC.get(dom), "kernel": dom,
            "bytes_per_launch": round(by / n), "avg_launch_us": round(us / n, 3)}

    # one M=9 verify pass at the decode context (past every position written so far): the
    # prompt-lookup draft of the generated stream, on the int8 matrix cores and lane-exact
    ids = np.concatenate([[tok], out[-8:]]).astype(np.int32) if len(out) >= 8 else prompt[-9:]
    m9_pos = pos
    m9_us = time_pass(eng, ids, m9_pos)
    ver_experts = eng.last_experts()
    ver_bytes = decode_bytes(cfg, specs, m9_pos + 8, ver_experts)
    eng.set_mfma(False)
    m9_exact_us = time_pass(eng, ids, m9_pos)
    eng.set_mfma(True)
    log(f"M=9 pass at position {m9_pos}: {m9_us:.0f} us on the matrix cores ({ver_bytes / m9_us / 1e3:.0f} GB/s, "
        f"{np.mean(ver_experts):.1f} unique experts a layer), {m9_exact_us:.0f} us lane-exact")

    # speculative generation, benchmark mode (n-gram 3, k = 8, fixed length), from the prefilled prompt
    toks, st = eng.generate(prompt, args.spec_tokens, draft_len=8, min_ngram=3, max_ngram=3, fixed=True,
                            adaptive_k=False, prefill_chunk=16, n_cached=len(prompt) - 1)
    ver_us = st["verify_us"] / max(1, st["verifies"])
    acc = st["accepted"] / max(1, st["verifies"])
    spec_tok_s = len(toks) / ((st["verify_us"] + st["step_us"]) / 1e6)
    rows = 1 + st["drafted"] / max(1, st["verifies"])  # a random-init model falls into short loops: short drafts
    log(f"verify: {st['verifies']} passes of M<=9 (mean {rows:.2f} rows), {ver_us:.0f} us/pass, {acc:.2f} accepted/pass, "
        f"{st['steps']} plain steps, {spec_tok_s:.1f} tok/s end to end")
    eng.close()

    legs = {}
    if not args.no_legs and args.config == "qwen3-30b-a3b":
        # moe_prune top-4 (the reference's optional variant, smollm_chat.rs:1221-1237)
        e4 = M.Engine(ctx, cfg.replace(moe_prune=4.0), w)
        tk, _ = prefill(e4, prompt)
        p4_tok_s, tk, p4 = timed_decode(ctx, e4, tk, len(prompt), 4, 64)
        b4 = decode_bytes(cfg, specs, p4 - 32, e4.last_experts())
        m9p = time_pass(e4, prompt[-9:], p4)
        legs["moe_prune_top4"] = {"decode_tok_s": round(p4_tok_s, 1), "decode_gb_per_pass": round(b4 / 1e9, 4),
                                  "decode_roofline_frac": round(b4 * p4_tok_s / 1e9 / HBM_PEAK_GBS, 4),
                                  "verify_m9_pass_us": round(m9p, 1)}
        log(f"moe_prune top-4: {legs['moe_prune_top4']}")
        e4.close()
        # diverse routing: token embeddings scaled up so that each row's residual stream is its
        # own and the 9 rows of a pass choose experts nearly independently (a random-init model
        # otherwise drifts to a common hidden direction over a long context)
        # (at the headline context: the whole prompt prefilled first)
        ed = M.Engine(ctx, cfg.replace(embedding_scale=40.0), w)
        tk, _ = prefill(ed, prompt)
        ids9 = np.random.default_rng(args.seed).integers(0, cfg.vocab, 9).astype(np.int32)
        dv_us = time_pass(ed, ids9, len(prompt))
        dv_exp = ed.last_experts()
        dv_bytes = decode_bytes(cfg, specs, len(prompt) + 8, dv_exp)
        legs["verify_m9_diverse_routing"] = {"pass_us": round(dv_us, 1), "unique_experts_per_layer": round(float(np.mean(dv_exp)), 1),
                                             "gb_per_pass": round(dv_bytes / 1e9, 4), "hbm_gbs": round(dv_bytes / dv_us / 1e3, 1),
                                             "roofline_frac": round(dv_bytes / dv_us / 1e3 / HBM_PEAK_GBS, 4),
                                             "context": len(prompt) + 9}
        log(f"M=9 diverse routing: {legs['verify_m9_diverse_routing']}")
        ed.close()
        del w
        for name, plen, spans in (("smollm2-135m", 32, False), ("qwen3-0.6b", 512, False),
                                  ("granite-1b-a400m", 256, False)):
            legs[name] = small_config_leg(ctx, name, args.seed, plen, spans, 64)
        legs["qwen3-0.6b-spec"] = small_config_leg(ctx, "qwen3-0.6b", args.seed, 2048, True, 32)

    res = {
        "metric": "decode tok/s (Qwen3-30B-A3B Q4_K_M-shaped, 1 GPU); k=8 verify-pass us; HBM GB/s",
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(1e3 / tok_s, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "i8 dot (int32) + f32", "data": "synthetic (random-init weights, seed %d)" % args.seed,
        "config": {"workload": f"{cfg.name} greedy decode, M=1, context {args.prompt_len}+ of {cfg.max_seq}",
                   "prompt_tokens": args.prompt_len, "weights_gib": round(gib, 2)},
        "decode_gb_per_pass": round(dec_bytes / 1e9, 4), "decode_hbm_gbs": round(dec_bytes * tok_s / 1e9, 1),
        "decode_roofline_frac": round(dec_bytes * tok_s / 1e9 / HBM_PEAK_GBS, 4),
        "verify_m9_pass_us": round(m9_us, 1), "verify_m9_position": m9_pos,
        "verify_m9_pass_us_lane_exact": round(m9_exact_us, 1), "verify_m9_hbm_gbs": round(ver_bytes / m9_us / 1e3, 1),
        "verify_gb_per_pass": round(ver_bytes / 1e9, 4), "verify_unique_experts_per_layer": round(float(np.mean(ver_experts)), 1),
        "spec_verify_pass_us": round(ver_us, 1), "spec_verify_mean_rows": round(rows, 2),
        "accepted_per_pass": round(acc, 3), "spec_tok_s": round(spec_tok_s, 2), "prefill_tok_s": round(len(prompt) / prefill_s, 1),
        "legs": legs, "roofline": roof, "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
