#!/usr/bin/env python
"""Short text summaries of rocprofv3 results (SQLite *_results.db, ROCm 7).

    prof_summary.py stats   DB_OR_DIR --cmd "<command that made it>" [--bench-json FILE] [--plain-json FILE] [--top N]
    prof_summary.py traffic FETCH_DB WRITE_DB --bench-json FILE [--calib-bytes N]
    prof_summary.py sweep   BENCH_JSON --cmd "<command that made it>"
    prof_summary.py steps   DB_OR_DIR --cmd "<command that made it>" [--rows 4] [--title T]

stats   : per-kernel calls / total / average duration of a --kernel-trace run,
          and, given the benchmark's JSON line, the average duration of the
          roofline kernel over exactly the dispatches the benchmark's events
          bracketed (roofline.dispatches: ordinal of the first one among that
          kernel's dispatches, and their count), next to the benchmark's own
          event-timed figure, in the traced run and (--plain-json) in a run of
          the same command without the tracer.
traffic : HBM bytes per launch of the roofline kernel from two --pmc runs
          (FETCH_SIZE, WRITE_SIZE; KiB per dispatch), each scaled by what the
          same counter reads for the k_copy kernel of known size (the
          benchmark's --copy-calib: 5 copies of 256 MiB).  Prints JSON.
sweep   : the table of a `bench.py --mode sweep` line (formats x shapes x B).
steps   : per-kernel time of one verify step of a --kernel-trace run of the model
          benchmark.  The trace is cut after every k_argmax_final; a verify step
          is a piece that ends in the argmax of --rows rows (drafts and decode
          steps end in a one-row argmax).  Durations are averaged over all verify
          steps of the run (the timed spec cycles, forced acceptance and the
          step timings).
"""
import argparse
import glob
import json
import os
import sqlite3
import statistics
import sys


def find_db(p):
    if os.path.isdir(p):
        dbs = sorted(glob.glob(os.path.join(p, "**", "*_results.db"), recursive=True))
        if not dbs:
            sys.exit(f"no *_results.db under {p}")
        return dbs[-1]
    return p


def short(name):
    n = name[5:] if name.startswith("void ") else name
    i = n.find("(")
    return n[:i] if i > 0 else n


def bench_line(path):
    with open(path) as f:
        for ln in f:
            ln = ln.strip()
            if ln.startswith("{") and '"metric"' in ln:
                return json.loads(ln)
    sys.exit(f"no benchmark JSON line in {path}")


def kernel_rows(db):
    c = sqlite3.connect(find_db(db))
    return c.execute("select name, dispatch_id, duration, grid_x, workgroup_x from kernels "
                     "order by dispatch_id").fetchall()


def cmd_stats(a):
    rows = kernel_rows(a.db)
    agg = {}
    for name, _, dur, _, _ in rows:
        s = agg.setdefault(short(name), [0, 0.0, float("inf"), 0.0])
        s[0] += 1
        s[1] += dur
        s[2] = min(s[2], dur)
        s[3] = max(s[3], dur)
    total = sum(v[1] for v in agg.values()) or 1.0
    out = [f"# rocprofv3 kernel trace: {a.title or os.path.basename(find_db(a.db))}", "",
           "Command (`/root/repo` is the repository root):", "", "```", a.cmd, "```", "",
           f"{len(rows)} kernel dispatches, {total / 1e6:.3f} ms of kernel time.", "",
           "| kernel | calls | total ms | avg us | min us | max us | % |", "|---|---:|---:|---:|---:|---:|---:|"]
    for name, (n, t, lo, hi) in sorted(agg.items(), key=lambda kv: -kv[1][1])[:a.top]:
        out.append(f"| `{name}` | {n} | {t / 1e6:.3f} | {t / n / 1e3:.3f} | {lo / 1e3:.3f} | {hi / 1e3:.3f} | "
                   f"{100 * t / total:.1f} |")
    if a.bench_json:
        b = bench_line(a.bench_json)
        r = b["roofline"]
        durs = [d for name, _, d, _, _ in rows if short(name) == r["kernel"]]
        first, count = r["dispatches"]["first"], r["dispatches"]["count"]
        sel = durs[first:first + count]
        if len(sel) == count:
            avg = statistics.fmean(sel) / 1e3
            out += ["", f"## Roofline kernel `{r['kernel']}` ({r.get('workload', '')})", "",
                    f"Dispatches {first}..{first + count - 1} of this kernel (the ones the benchmark's events "
                    f"bracket): average {avg:.3f} us, median {statistics.median(sel) / 1e3:.3f} us.",
                    f"Benchmark's event-timed average over the same launches in the traced run: {r['kernel_us']:.3f} us "
                    f"(ratio {r['kernel_us'] / avg:.3f}; the tracer's per-dispatch cost is inside this figure when the "
                    f"launches are graph replays)."]
            if a.plain_json:
                rp = bench_line(a.plain_json)["roofline"]
                out += [f"Same command without the tracer: event-timed average {rp['kernel_us']:.3f} us "
                        f"(ratio {rp['kernel_us'] / avg:.3f} to the traced kernel durations)."]
            out += [
                    f"Algorithmic bytes per launch {r['algo_bytes']:,} -> {r['algo_bytes'] / avg / 1e3:.1f} GB/s "
                    f"= {r['algo_bytes'] / avg / 1e3 / r['peak']:.3f} of {r['peak']:.0f} GB/s."]
        else:
            out += ["", f"roofline kernel {r['kernel']}: only {len(durs)} dispatches in the trace"]
        keys = [k for k in ("value", "unit", "ms_per_step", "verify_ms", "decode_ms", "draft_ms",
                            "verify_over_decode", "verify_hbm_gbs", "forced_accept_tok_s") if k in b]
        out += ["", "Benchmark line of the traced run: " + ", ".join(f"{k} = {b[k]}" for k in keys) + "."]
        if a.plain_json:
            bp = bench_line(a.plain_json)
            out += ["", "Benchmark line without the tracer: " + ", ".join(f"{k} = {bp[k]}" for k in keys if k in bp) + "."]
    print("\n".join(out))


def counter_values(db, counter, kernel):
    c = sqlite3.connect(find_db(db))
    rows = c.execute("select kernel_name, dispatch_id, value from counters_collection where counter_name = ? "
                     "order by dispatch_id", (counter,)).fetchall()
    per = {}
    for name, did, v in rows:
        per.setdefault(short(name), {}).setdefault(did, 0.0)
        per[short(name)][did] += v
    return [per.get(kernel, {})[d] for d in sorted(per.get(kernel, {}))]


def cmd_traffic(a):
    b = bench_line(a.bench_json)
    r = b["roofline"]
    first, count = r["dispatches"]["first"], r["dispatches"]["count"]
    res = {}
    for counter, db in (("FETCH_SIZE", a.fetch_db), ("WRITE_SIZE", a.write_db)):
        vals = counter_values(db, counter, r["kernel"])[first:first + count]
        cal = counter_values(db, counter, "k_copy")
        if len(vals) != count or not cal:
            sys.exit(f"{counter}: {len(vals)} roofline dispatches, {len(cal)} calibration copies")
        factor = a.calib_bytes / (statistics.median(cal) * 1024.0)
        res[counter] = {"kib_per_launch": statistics.fmean(vals), "copy_kib": statistics.median(cal),
                        "scale": factor, "bytes_per_launch": statistics.fmean(vals) * 1024.0 * factor}
    traffic = res["FETCH_SIZE"]["bytes_per_launch"] + res["WRITE_SIZE"]["bytes_per_launch"]
    print(json.dumps({r["kernel"].split("<")[0]: {
        "kernel": r["kernel"], "workload": r.get("workload"), "bytes_per_launch": round(traffic),
        "algo_bytes": r["algo_bytes"], "traffic_over_algo": round(traffic / r["algo_bytes"], 4),
        "counters": res, "calibration": f"k_copy of {a.calib_bytes} bytes (reads and writes that many)"}},
        indent=1))


def cmd_sweep(a):
    b = bench_line(a.bench_json)
    rows = b["sweep"]
    out = ["# gemv_batch sweep over formats, shapes and batch (config 2)", "",
           "Command (`/root/repo` is the repository root):", "", "```", a.cmd, "```", "",
           "Each point: warm-up calls, then 40 `qgpu_gemv_batch` calls (activation preparation + GEMV) captured in a",
           "HIP graph, replayed once untimed and once between HIP events on the library stream; weights rotate over",
           "enough device copies to exceed the 256 MB MALL.  GB/s = (weight bytes + B x (in + out) x 4) / time;",
           "% = of 8 TB/s.  Every format runs the int8-MFMA digit GEMV on packed 16-row tile records",
           "(`k_gemv_mfma<format, ...>`).", ""]
    bs = sorted({r["B"] for r in rows})
    out.append("| format | rows x cols | weight MB | " + " | ".join(f"B={B} us | B={B} GB/s" for B in bs) + " |")
    out.append("|---|---|---:|" + "---:|---:|" * len(bs))
    seen = []
    for r in rows:
        key = (r["format"], r["rows"], r["cols"])
        if key not in seen:
            seen.append(key)
    for f, nr, nc in seen:
        pts = {r["B"]: r for r in rows if (r["format"], r["rows"], r["cols"]) == (f, nr, nc)}
        wmb = next(iter(pts.values()))["weight_bytes"] / 1e6
        cells = []
        for B in bs:
            p = pts.get(B)
            cells.append(f"{p['us']:.1f} | {p['gbs']:.0f} ({100 * p['frac']:.0f}%)" if p else " | ")
        out.append(f"| {f} | {nr} x {nc} | {wmb:.1f} | " + " | ".join(cells) + " |")
    print("\n".join(out))


def cmd_steps(a):
    rows = kernel_rows(a.db)
    segs, cur = [], []
    for r in rows:
        cur.append(r)
        if short(r[0]).startswith("k_argmax_final"):
            segs.append(cur)
            cur = []
    steps = [g for g in segs if g[-1][3] // max(g[-1][4], 1) == a.rows]
    if not steps:
        sys.exit(f"no step ending in a {a.rows}-row argmax")
    agg = {}
    for g in steps:
        for name, _, dur, gx, wx in g:
            key = (short(name), gx // max(wx, 1), wx)
            c = agg.setdefault(key, [0, 0])
            c[0] += 1
            c[1] += dur
    n = len(steps)
    busy = sum(c[1] for c in agg.values()) / n
    out = [f"# rocprofv3 kernel trace: one verify step (B = {a.rows}){' -- ' + a.title if a.title else ''}", "",
           "Command (`/root/repo` is the repository root):", "", "```", a.cmd, "```", "",
           f"{n} verify steps in the trace; {statistics.median(len(g) for g in steps):.0f} dispatches and "
           f"{busy / 1e3:.1f} us of kernel time per step (sum of kernel durations).", "",
           "| kernel | grid x block | launches per step | avg us | us per step | % |",
           "|---|---|---:|---:|---:|---:|"]
    for (name, gb, wx), (cnt, tot) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
        if tot / n / 1e3 < a.min_us:
            continue
        out.append(f"| `{name}` | {gb} x {wx} | {cnt / n:.1f} | {tot / cnt / 1e3:.2f} | {tot / n / 1e3:.1f} | "
                   f"{100 * tot / n / busy:.1f} |")
    print("\n".join(out))


def main():
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd_name", required=True)
    s = sub.add_parser("stats")
    s.add_argument("db")
    s.add_argument("--cmd", required=True)
    s.add_argument("--title", default=None)
    s.add_argument("--bench-json", default=None)
    s.add_argument("--plain-json", default=None, help="bench line of the same command run without the tracer")
    s.add_argument("--top", type=int, default=25)
    t = sub.add_parser("traffic")
    t.add_argument("fetch_db")
    t.add_argument("write_db")
    t.add_argument("--bench-json", required=True)
    t.add_argument("--calib-bytes", type=int, default=256 << 20)
    w = sub.add_parser("sweep")
    w.add_argument("bench_json")
    w.add_argument("--cmd", required=True)
    st = sub.add_parser("steps")
    st.add_argument("db")
    st.add_argument("--cmd", required=True)
    st.add_argument("--rows", type=int, default=4)
    st.add_argument("--title", default=None)
    st.add_argument("--min-us", type=float, default=1.0, help="omit kernels below this many us per step")
    a = ap.parse_args()
    {"stats": cmd_stats, "traffic": cmd_traffic, "sweep": cmd_sweep, "steps": cmd_steps}[a.cmd_name](a)


if __name__ == "__main__":
    main()
