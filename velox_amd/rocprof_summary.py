"""Summaries of rocprofv3 result databases (ROCm 7.x writes SQLite).

    python -m velox_amd.rocprof_summary trace RESULTS.db|run_kernel_trace.csv [--top N]
        per (kernel, grid) dispatch count and duration statistics
    python -m velox_amd.rocprof_summary verify RESULTS.db [--rounds R] [--pmc FILE.db ...]
        the verify int4 GEMMs of the spec bench's timed rounds: every packed
        GEMM dispatch (qmm_f16_dma_kernel / qmm_f16_k2_kernel) with three
        32-row tiles (<3, ...>, the 80 verify rows) and a one-row grid (prefill
        uses many row blocks), plus the SwiGLU finish (qmm_reduce_kernel) that
        follows a gate|up dispatch; per-round sums
        and the average per GEMM op, and with --pmc the FETCH_SIZE / WRITE_SIZE
        sums of the same dispatches scaled by the calibration copy
    python -m velox_amd.rocprof_summary calib RESULTS.db --bytes B
        FETCH_SIZE or WRITE_SIZE (KiB) read for the largest
        __amd_rocclr_copyBuffer dispatch, and the byte factor B / (KiB * 1024)
    python -m velox_amd.rocprof_summary pmc RESULTS.db|counter_collection.csv --kernel REGEX [--skip N]
        mean per dispatch of every counter over the dispatches whose kernel
        name matches REGEX (the first N of them skipped as warm-up)

The kernel-trace duration of a dispatch is end - start (ns).
"""
from __future__ import annotations

import argparse
import collections
import re
import sqlite3


def _short(name: str) -> str:
    n = name.replace("void ", "").replace("vx::", "").replace("(anonymous namespace)::", "")
    return n.split("(")[0] if not n.startswith("(") else n


def dispatches(db: str):
    """[(short name, start, end, workgroups along x, grid_y, dispatch_id)] in start order
    (rocprofv3 records grid_x in work-items).  db is a results database, or
    the run_kernel_trace.csv of `--output-format csv`."""
    if db.endswith(".csv"):
        import csv

        rows = sorted(csv.DictReader(open(db)), key=lambda r: int(r["Start_Timestamp"]))
        return [(_short(r["Kernel_Name"]), int(r["Start_Timestamp"]), int(r["End_Timestamp"]),
                 int(r["Grid_Size_X"]) // max(1, int(r["Workgroup_Size_X"])), int(r["Grid_Size_Y"]),
                 int(r["Dispatch_Id"])) for r in rows]
    c = sqlite3.connect(db)
    rows = c.execute("select name, start, end, grid_x, grid_y, dispatch_id, workgroup_x from kernels "
                     "order by start").fetchall()
    return [(_short(n), s, e, gx // max(1, wx), gy, d) for n, s, e, gx, gy, d, wx in rows]


def counters(db: str):
    """{dispatch_id: {counter: value}} from a --pmc run (results database or
    the counter_collection.csv of `--output-format csv`)."""
    if db.endswith(".csv"):
        import csv

        out = collections.defaultdict(dict)
        for r in csv.DictReader(open(db)):
            out[int(r["Dispatch_Id"])][r["Counter_Name"]] = float(r["Counter_Value"])
        return out
    c = sqlite3.connect(db)
    cols = [r[1] for r in c.execute("pragma table_info('counters_collection')")]
    out = collections.defaultdict(dict)
    for r in c.execute("select * from counters_collection"):
        rec = dict(zip(cols, r))
        out[rec["dispatch_id"]][rec["counter_name"]] = rec["value"]
    return out


def cmd_trace(args):
    ds = dispatches(args.db)
    st = collections.defaultdict(list)
    for n, s, e, gx, gy, _ in ds:
        st[(n, gx, gy)].append(e - s)
    total = sum(e - s for _, s, e, *_ in ds)
    print(f"total kernel time {total / 1e3:.1f} us over {len(ds)} dispatches")
    print(f"{'kernel':64s} {'grid (wg x, y)':>14s} {'n':>6s} {'total us':>10s} {'avg us':>8s} {'med us':>8s} {'min us':>8s}")
    for (n, gx, gy), v in sorted(st.items(), key=lambda kv: -sum(kv[1]))[: args.top]:
        v.sort()
        print(f"{n[:64]:64s} {f'{gx}x{gy}':>14s} {len(v):6d} {sum(v) / 1e3:10.1f} {sum(v) / len(v) / 1e3:8.2f} "
              f"{v[len(v) // 2] / 1e3:8.2f} {v[0] / 1e3:8.2f}")


def _verify_ops(ds, rounds):
    """Group the verify GEMM dispatches of the last `rounds` rounds into ops."""
    ops = []
    prev_gate_up = False
    for n, s, e, gx, gy, d in ds:
        m = re.match(r"qmm_f16_(?:dma|k2)_kernel<(\d+), (\d+), (\d+)(?:, \d+)?>", n)
        if m and m.group(1) == "3" and gy == 1:
            ops.append([(n, s, e, d)])
            prev_gate_up = True
            continue
        if n.startswith("qmm_reduce_kernel") and prev_gate_up and ops:
            ops[-1].append((n, s, e, d))
        prev_gate_up = False
    return ops


def cmd_verify(args):
    ds = dispatches(args.db)
    ops = _verify_ops(ds, args.rounds)
    per_round = len(ops) // max(1, args.total_rounds)
    sel = ops[-per_round * args.rounds:] if per_round else ops
    dur = [sum(e - s for _, s, e, _ in op) for op in sel]
    print(f"verify GEMM ops found: {len(ops)} ({per_round} per round over {args.total_rounds} rounds); "
          f"summarised: last {args.rounds} rounds = {len(sel)} ops")
    print(f"sum per round {sum(dur) / args.rounds / 1e3:.1f} us; average per op {sum(dur) / len(dur) / 1e3:.2f} us")
    for path in args.pmc or []:
        pm = counters(path)
        pds = dispatches(path)
        pops = _verify_ops(pds, args.rounds)
        psel = pops[-per_round * args.rounds:] if per_round else pops
        tot = collections.Counter()
        for op in psel:
            for _, _, _, d in op:
                for k, v in pm.get(d, {}).items():
                    tot[k] += v
        for k, v in tot.items():
            print(f"{path}: {k} summed over {len(psel)} ops = {v:.0f} KiB; per op {v / len(psel):.1f} KiB")


def cmd_calib(args):
    pm = counters(args.db)
    ds = [d for d in dispatches(args.db) if d[0].startswith("__amd_rocclr_copyBuffer")]
    best = None
    for n, s, e, gx, gy, d in ds:
        for k, v in pm.get(d, {}).items():
            if best is None or v > best[1]:
                best = (k, v, d)
    if best is None:
        print("no copy dispatch with counters found")
        return
    k, v, d = best
    print(f"{k} of the calibration copy (dispatch {d}): {v:.0f} KiB for {args.bytes} bytes; "
          f"factor = {args.bytes / (v * 1024):.4f}")


def cmd_pmc(args):
    """Mean counter values per dispatch of one kernel."""
    pm = counters(args.db)
    if args.db.endswith(".csv"):
        import csv

        names = {}
        for r in csv.DictReader(open(args.db)):
            names[int(r["Dispatch_Id"])] = _short(r["Kernel_Name"])
    else:
        names = {d: n for n, _, _, _, _, d in dispatches(args.db)}
    sel = sorted(d for d, n in names.items() if re.search(args.kernel, n))[args.skip:]
    if not sel:
        print("no matching dispatches")
        return
    tot = collections.Counter()
    for d in sel:
        for k, v in pm.get(d, {}).items():
            tot[k] += v
    print(f"{len(sel)} dispatches of {names[sel[0]]} (first {args.skip} matching skipped)")
    for k in sorted(tot):
        print(f"  {k:28s} {tot[k] / len(sel):16.1f}")


def main():
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    a = sub.add_parser("trace")
    a.add_argument("db")
    a.add_argument("--top", type=int, default=40)
    b = sub.add_parser("verify")
    b.add_argument("db")
    b.add_argument("--rounds", type=int, default=4)
    b.add_argument("--total-rounds", type=int, default=6)
    b.add_argument("--pmc", nargs="*")
    d = sub.add_parser("pmc")
    d.add_argument("db")
    d.add_argument("--kernel", required=True)
    d.add_argument("--skip", type=int, default=0)
    c = sub.add_parser("calib")
    c.add_argument("db")
    c.add_argument("--bytes", type=float, required=True)
    args = ap.parse_args()
    {"trace": cmd_trace, "verify": cmd_verify, "calib": cmd_calib, "pmc": cmd_pmc}[args.cmd](args)


if __name__ == "__main__":
    main()
