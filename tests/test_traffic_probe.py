"""The hardware-counter summary of spindle_amd/traffic_probe.py on a small counter CSV of the
shape rocprofv3 --pmc writes: means per (kernel, counter, grid), and the --after / --before
phase filters, which select by dispatch order (not by the order of the CSV's rows)."""
import csv
import re

from spindle_amd import traffic_probe as tp

COLS = ["Correlation_Id", "Dispatch_Id", "Grid_Size", "Kernel_Name", "Counter_Name", "Counter_Value"]
# dispatch order: prefill (A, B), decode (D, LM), verify (A, B), calibration copy
ROWS = [
    (1, 1, 256, "spx::A(args)", "FETCH_SIZE", 10.0),
    (2, 2, 512, "void spx::B<1>(args)", "FETCH_SIZE", 20.0),
    (3, 3, 64, "spx::D(args)", "FETCH_SIZE", 1.0),
    (4, 4, 128, "void spx::LM<14, 1, 4>(args)", "FETCH_SIZE", 100.0),
    (5, 5, 256, "spx::A(args)", "FETCH_SIZE", 30.0),
    (6, 6, 512, "void spx::B<1>(args)", "FETCH_SIZE", 40.0),
    (7, 7, 131072, "__amd_rocclr_copyBuffer", "FETCH_SIZE", 262144.0),
]


def _csv(tmp_path, rows):
    p = tmp_path / "run_counter_collection.csv"
    with open(p, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(COLS)
        for r in rows:
            w.writerow(r)
    return str(p)


def _parse(out):
    res = {}
    for line in out.strip().splitlines():
        m = re.fullmatch(r"(.{48}) (\S+)\s+grid\s+(\d+) n=\s*(\d+) mean\s+(\S+)", line)
        assert m, line
        res[(m.group(1).strip(), int(m.group(3)))] = (int(m.group(4)), float(m.group(5)))
    return res


def test_summary_means_and_phases(tmp_path, capsys):
    path = _csv(tmp_path, list(reversed(ROWS)))  # rows out of dispatch order
    tp.summarize(path)
    allp = _parse(capsys.readouterr().out)
    assert allp[("spx::A", 256)] == (2, 20.0)
    assert allp[("void spx::B<1>", 512)] == (2, 30.0)
    tp.summarize(path, after="LM<14, 1, 4>")
    ver = _parse(capsys.readouterr().out)
    assert ver[("spx::A", 256)] == (1, 30.0) and ver[("void spx::B<1>", 512)] == (1, 40.0)
    assert ("spx::D", 64) not in ver and ("__amd_rocclr_copyBuffer", 131072) in ver
    tp.summarize(path, before="spx::D")
    pre = _parse(capsys.readouterr().out)
    assert set(pre) == {("spx::A", 256), ("void spx::B<1>", 512)}
    assert pre[("spx::A", 256)] == (1, 10.0)
