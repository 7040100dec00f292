"""Short text summaries of rocprofv3 output for profiles/.

    python prof_summary.py trace   --dir D --out FILE --cmd "..."
        kernel-trace --stats run (csv output): per-kernel calls and durations.
    python prof_summary.py traffic --fetch D1 --write D2 --kernel NAME --out FILE --cmd "..."
        two --pmc runs of `bench.py --pmc` (FETCH_SIZE, WRITE_SIZE): HBM bytes per
        launch of the kernel whose name contains NAME, each counter scaled by what it
        reads for lg_buf_copy (kernel k_copy16) of a known size.
    python prof_summary.py counters --dirs D1 [D2 ...] --kernel NAME --weights W --out FILE --cmd "..."
        --pmc runs of `bench.py --pmc` with SQ_* counters: each counter's average per
        dispatch of the kernel whose name contains NAME, and per wavefront and per
        weight (W weights per launch).
"""
import argparse
import csv
import glob
import os

CAL_BYTES = 64 << 20


def _rows(d, pattern):
    files = glob.glob(os.path.join(d, "**", pattern), recursive=True)
    if not files:
        raise SystemExit(f"no {pattern} under {d}")
    return list(csv.DictReader(open(files[0])))


def _avg(rows, counter, name):
    v = [float(r["Counter_Value"]) for r in rows if r["Counter_Name"] == counter and name in r["Kernel_Name"]]
    if not v:
        raise SystemExit(f"no {counter} samples for {name}")
    return sum(v) / len(v), len(v)


def trace(args):
    rows = _rows(args.dir, "*kernel_stats.csv")
    out = [f"# rocprofv3 kernel trace summary", "", f"command: {args.cmd}", "",
           "| kernel | calls | avg us | min us | max us | share % |", "|---|---|---|---|---|---|"]
    for r in rows:
        name = r["Name"].replace("(anonymous namespace)::", "")
        name = name[5:] if name.startswith("void ") else name
        name = name.split("(")[0]
        out.append(f"| {name} | {r['Calls']} | {float(r['AverageNs']) / 1e3:.3f} | {float(r['MinNs']) / 1e3:.3f} | "
                   f"{float(r['MaxNs']) / 1e3:.3f} | {float(r['Percentage']):.1f} |")
    open(args.out, "w").write("\n".join(out) + "\n")
    print("\n".join(out))


def traffic(args):
    f = _rows(args.fetch, "*counter_collection.csv")
    w = _rows(args.write, "*counter_collection.csv")
    fc, _ = _avg(f, "FETCH_SIZE", "k_copy16")
    wc, _ = _avg(w, "WRITE_SIZE", "k_copy16")
    ff = (CAL_BYTES / 1024) / fc  # KiB actually moved per KiB counted
    wf = (CAL_BYTES / 1024) / wc
    fk, nf = _avg(f, "FETCH_SIZE", args.kernel)
    wk, nw = _avg(w, "WRITE_SIZE", args.kernel)
    traffic = (fk * ff + wk * wf) * 1024
    out = ["# HBM traffic per launch (rocprofv3 --pmc)", "", f"command (FETCH_SIZE run): {args.cmd}",
           "command (WRITE_SIZE run): the same with --pmc WRITE_SIZE", "",
           f"calibration: lg_buf_copy of {CAL_BYTES} bytes reads FETCH_SIZE {fc:.1f} KiB and WRITE_SIZE "
           f"{wc:.1f} KiB, so fetch factor {ff:.4f}, write factor {wf:.4f}",
           f"kernel {args.kernel}: FETCH_SIZE {fk:.1f} KiB ({nf} dispatches), WRITE_SIZE {wk:.1f} KiB ({nw})",
           f"traffic_bytes_per_launch: {traffic:.0f}"]
    open(args.out, "w").write("\n".join(out) + "\n")
    print("\n".join(out))


def counters(args):
    vals = {}
    for d in args.dirs:
        for r in _rows(d, "*counter_collection.csv"):
            if args.kernel in r["Kernel_Name"] and "k_copy16" not in r["Kernel_Name"]:
                vals.setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    if not vals:
        raise SystemExit(f"no counter samples for {args.kernel}")
    avg = {k: sum(v) / len(v) for k, v in vals.items()}
    out = ["# Counters per launch (rocprofv3 --pmc)", "", f"command: {args.cmd}", "",
           f"kernel: names containing `{args.kernel}`; {args.weights} weights per launch", "",
           "| counter | per launch | per wavefront | per 1000 weights | dispatches |", "|---|---|---|---|---|"]
    waves = avg.get("SQ_WAVES")
    for k in sorted(avg):
        pw = f"{avg[k] / waves:.1f}" if waves else "-"
        out.append(f"| {k} | {avg[k]:.0f} | {pw} | {1000.0 * avg[k] / args.weights:.3f} | {len(vals[k])} |")
    open(args.out, "w").write("\n".join(out) + "\n")
    print("\n".join(out))


def main():
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="mode", required=True)
    t = sub.add_parser("trace")
    t.add_argument("--dir", required=True)
    t.add_argument("--out", required=True)
    t.add_argument("--cmd", required=True)
    p = sub.add_parser("traffic")
    p.add_argument("--fetch", required=True)
    p.add_argument("--write", required=True)
    p.add_argument("--kernel", required=True)
    p.add_argument("--out", required=True)
    p.add_argument("--cmd", required=True)
    c = sub.add_parser("counters")
    c.add_argument("--dirs", nargs="+", required=True)
    c.add_argument("--kernel", required=True)
    c.add_argument("--weights", type=float, required=True)
    c.add_argument("--out", required=True)
    c.add_argument("--cmd", required=True)
    args = ap.parse_args()
    {"trace": trace, "traffic": traffic, "counters": counters}[args.mode](args)


if __name__ == "__main__":
    main()
