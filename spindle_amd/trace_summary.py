"""Summarises a rocprofv3 kernel trace of the engine per forward pass.

A pass is the kernels from k_embed to k_argmax_final (or to the next k_embed: a prompt chunk of
spx_engine_feed runs no LM head); passes are grouped by kernel count, their
first matrix kernel (k_mvr<M> / k_mvt<M> / k_mv_f<M>: M = the pass's row bucket; kd_mv / kd_mm /
kd_mq: the decode, lane-exact multi-row and int8-MFMA multi-row kernels) and their row count
(k_embed's grid: 256 threads a row). For each group: pass span vs busy time, and (groups of at
least 10 passes) the median per-pass time of every kernel.

  python3 -m spindle_amd.trace_summary <run_kernel_trace.csv> <summary.txt>
"""
import csv, sys, collections, statistics as S
if len(sys.argv) != 3:
    sys.exit(__doc__)
path, out = sys.argv[1], sys.argv[2]
rows = []
with open(path) as f:
    for r in csv.DictReader(f):
        rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"], int(r.get("Grid_Size_X", r.get("Grid_Size", 0)) or 0), int(r.get("Workgroup_Size_X", 0) or 0)))
rows.sort()
def short(n):
    n = n.split("(")[0]
    return n.replace("void ", "").replace("spx::", "")[:60]
passes, cur = [], None
for r in rows:
    nm = short(r[2])
    if nm.startswith("k_embed"):
        if cur is not None:
            passes.append(cur)
        cur = [r]
    elif cur is not None:
        cur.append(r)
        if nm.startswith("k_argmax"):
            passes.append(cur); cur = None
lines = []
lines.append(f"kernels in trace: {len(rows)}; forward passes found: {len(passes)}")
# classify by kernel count
groups = collections.defaultdict(list)
for p in passes:
    sig = next((short(r[2]) for r in p if short(r[2]).startswith(("k_mvr", "k_mvt", "k_mv_f", "kd_mv", "kd_mm", "kd_mq"))), "none")
    groups[(len(p), sig, "rows %d" % (p[0][3] // 256))].append(p)
for n, ps in sorted(groups.items()):
    spans = [(p[-1][1] - p[0][0]) / 1e3 for p in ps]
    busy = [sum(r[1] - r[0] for r in p) / 1e3 for p in ps]
    lines.append(f"passes {n}: {len(ps)}; span median {S.median(spans):.1f} us, busy median {S.median(busy):.1f} us, gap median {(S.median(spans)-S.median(busy)):.1f} us")
# per-kernel breakdown in the most common pass type(s): take the last 20 passes of each group
for n, ps in sorted(groups.items(), key=lambda kv: -len(kv[1])):
    if len(ps) < 10:
        continue
    sel = ps[-20:]
    agg = collections.defaultdict(list)
    for p in sel:
        per = collections.defaultdict(float); cnt = collections.Counter()
        for r in p:
            k = short(r[2])
            if k.startswith(("kd_mq", "kd_mm", "kd_mv")) and r[4]:
                k += " [%d wg]" % (r[3] // r[4])  # the launches of one matrix kernel, told apart by grid
            per[k] += (r[1] - r[0]) / 1e3; cnt[k] += 1
        for k in per: agg[k].append((per[k], cnt[k]))
    lines.append(f"-- per-pass kernel time, passes {n} (median over {len(sel)} passes)")
    tot = 0
    for k, v in sorted(agg.items(), key=lambda kv: -S.median([x[0] for x in kv[1]])):
        t = S.median([x[0] for x in v]); c = v[0][1]; tot += t
        lines.append(f"  {t:9.1f} us  {c:5d} launches  {t / c:7.2f} us/launch  {k}")
    lines.append(f"  {tot:9.1f} us  total")
open(out, "w").write("\n".join(lines) + "\n")
print("\n".join(lines))
