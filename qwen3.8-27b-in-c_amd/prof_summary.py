#!/usr/bin/env python
"""Short text summaries of rocprofv3 results (SQLite *_results.db, ROCm 7).

    prof_summary.py stats   DB_OR_DIR --cmd "<command that made it>" [--bench-json FILE] [--plain-json FILE] [--top N]
    prof_summary.py traffic FETCH_DB WRITE_DB --bench-json FILE [--calib-bytes N]
    prof_summary.py sweep   BENCH_JSON --cmd "<command that made it>"
    prof_summary.py steps   DB_OR_DIR --cmd "<command that made it>" [--rows 4] [--title T]
    prof_summary.py counters DB [DB ...] --bench-json FILE --cmd "<commands that made them>"
    prof_summary.py kcounters DB [DB ...] --bench-json FILE [--kernel k_attn_span] --cmd "<commands>"

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
counters: every PMC counter of one or more --pmc runs of `bench.py --mode gemv`,
          averaged per launch over the roofline kernel's bracketed dispatches
          and over the plain-read kernel (k_checksum) of the read floor, side
          by side: the GEMV's instruction mix and vector-memory path against a
          kernel that only reads the same bytes.
kcounters: every PMC counter of --pmc runs of `bench.py --mode attn --eager` for one kernel
          (name prefix), averaged per dispatch for each of the benchmark's attention cases,
          with per-wave and per-tile instruction counts.
steps   : per-kernel time of one verify step of a --kernel-trace run of the model
          benchmark.  The trace is cut after every k_argmax_final; a verify step
          is a piece that ends in the argmax of --rows rows (drafts and decode
          steps end in a one-row argmax).  Durations are averaged over all verify
          steps of the run (the timed spec cycles, forced acceptance and the
          step timings).  A second table gives each kernel's role in the step
          (from its place in the launch order), its algorithmic HBM bytes per
          launch (27B hybrid dimensions, --pos KV positions) and the achieved
          fraction of 8 TB/s.
"""
import argparse
import glob
import json
import os
import re
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


def counter_table(db):
    """{counter: {kernel: [per-dispatch value in dispatch order]}} of one --pmc run"""
    c = sqlite3.connect(find_db(db))
    rows = c.execute("select kernel_name, dispatch_id, counter_name, value from counters_collection "
                     "order by dispatch_id").fetchall()
    acc = {}
    for name, did, cn, v in rows:
        acc.setdefault(cn, {}).setdefault(short(name), {}).setdefault(did, 0.0)
        acc[cn][short(name)][did] += v
    return {cn: {k: [d[i] for i in sorted(d)] for k, d in per.items()} for cn, per in acc.items()}


def cmd_counters(a):
    b = bench_line(a.bench_json)
    r = b["roofline"]
    first, count = r["dispatches"]["first"], r["dispatches"]["count"]
    out = ["# PMC counters: the roofline GEMV against a plain read of the same bytes", "",
           "Commands (`/root/repo` is the repository root; one rocprofv3 --pmc pass per line):", "", "```",
           *a.cmd.split(" ;; "), "```", "",
           f"Per launch, averaged over the {count} bracketed dispatches of `{r['kernel']}` ({r.get('workload', '')}, "
           f"{r['algo_bytes']:,} algorithmic bytes) and over the last {count} dispatches of `k_checksum` (the read "
           f"floor: the same {r['algo_bytes'] - 4 * (5120 + 17408) * 4:,} weight bytes, XOR-reduced).  Values are summed over the "
           "counter's instances (XCDs, SEs, channels) of one dispatch.", "",
           "| counter | GEMV per launch | read kernel per launch | GEMV / read |", "|---|---:|---:|---:|"]
    seen = {}
    for db in a.dbs:
        for cn, per in counter_table(db).items():
            g = per.get(r["kernel"], [])[first:first + count]
            rd = per.get("k_checksum", [])[-count:]
            if len(g) == count and rd:
                seen[cn] = (statistics.fmean(g), statistics.fmean(rd))
    for cn in sorted(seen):
        gv, rv = seen[cn]
        out.append(f"| {cn} | {gv:,.0f} | {rv:,.0f} | {gv / rv:.2f} |" if rv else f"| {cn} | {gv:,.0f} | {rv:,.0f} | - |")
    if "TCP_TCC_READ_REQ_sum" in seen:
        gv, rv = seen["TCP_TCC_READ_REQ_sum"]
        out += ["", f"L2 read requests from the CUs (TCP_TCC_READ_REQ): GEMV {gv:,.0f} per launch, read kernel "
                    f"{rv:,.0f} ({gv / rv:.2f}x) for the same weight bytes; the excess is the activation digit "
                    "tiles every row tile reads again from L2."]
    print("\n".join(out))


def span_tiles(pos, B, nspan=64, mintps=2, tp=16):
    """(tiles per span, spans) of the attention span kernel for a call at pos with B new positions"""
    ntl = (pos + B + tp - 1) // tp
    ns = min(ntl, nspan)
    tps = max(-(-ntl // ns), mintps)
    return tps, -(-ntl // tps)


def cmd_kcounters(a):
    b = bench_line(a.bench_json)
    cases = b["attn"]
    out = [f"# PMC counters: `{a.kernel}` per attention call (bench.py --mode attn --eager)", "",
           "Commands (`/root/repo` is the repository root; one rocprofv3 --pmc pass per line):", "", "```",
           *a.cmd.split(" ;; "), "```", "",
           f"The benchmark runs the cases in order with the same number of calls each, so the kernel's dispatches "
           f"split into {len(cases)} equal consecutive groups; each value is the average over the second half of its "
           "group (after the warm-up calls), summed over the counter's instances of one dispatch.  Per-wave "
           "figures divide by SQ_WAVES; per-tile figures also by the tiles each block streams.", ""]
    vals = {}
    for db in a.dbs:
        c = sqlite3.connect(find_db(db))
        acc = {}
        for name, did, cn, v in c.execute("select kernel_name, dispatch_id, counter_name, value from "
                                          "counters_collection order by dispatch_id").fetchall():
            if short(name).startswith(a.kernel):
                acc.setdefault(cn, {}).setdefault(did, 0.0)
                acc[cn][did] += v
        for cn, per in acc.items():
            seq = [per[d] for d in sorted(per)]         # every instance of the kernel, in dispatch order
            if not seq or len(seq) % len(cases):
                continue
            n = len(seq) // len(cases)
            vals[cn] = [statistics.fmean(seq[i * n + n // 2:(i + 1) * n]) for i in range(len(cases))]
    hdr = [f"{c['pos']} / B={c['B']}" for c in cases]
    out += ["| counter | " + " | ".join(hdr) + " |", "|---|" + "---:|" * len(cases)]
    for cn in sorted(vals):
        out.append(f"| {cn} | " + " | ".join(f"{v:,.0f}" for v in vals[cn]) + " |")
    if "SQ_WAVES" in vals:
        tiles = [span_tiles(c["pos"], c["B"]) for c in cases]
        out += ["", "| per wave | " + " | ".join(hdr) + " |", "|---|" + "---:|" * len(cases)]
        out.append("| tiles per span, spans | " + " | ".join(f"{t}, {s}" for t, s in tiles) + " |")
        for cn in ("SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_INSTS_LDS", "SQ_INSTS_SALU", "SQ_INSTS_VMEM_RD"):
            if cn in vals:
                out.append(f"| {cn} per wave | " + " | ".join(
                    f"{v / w:,.0f}" for v, w in zip(vals[cn], vals["SQ_WAVES"])) + " |")
                out.append(f"| {cn} per wave per tile | " + " | ".join(
                    f"{v / w / t[0]:,.1f}" for v, w, t in zip(vals[cn], vals["SQ_WAVES"], tiles)) + " |")
    if "SQ_LDS_BANK_CONFLICT" in vals and "SQ_ACTIVE_INST_LDS" in vals:
        out.append("| LDS bank-conflict cycles / LDS active cycles | " + " | ".join(
            f"{c / l:.3f}" if l else "-" for c, l in zip(vals["SQ_LDS_BANK_CONFLICT"], vals["SQ_ACTIVE_INST_LDS"])) + " |")
    print("\n".join(out))


def cmd_sweep(a):
    b = bench_line(a.bench_json)
    rows = b["sweep"]
    out = ["# gemv_batch sweep over formats, shapes and batch (config 2)", "",
           "Command (`/root/repo` is the repository root):", "", "```", a.cmd, "```", "",
           "Each point: warm-up calls, then 40 `qgpu_gemv_batch` calls (activation preparation + GEMV) captured in a",
           "HIP graph, replayed once untimed and once between HIP events on the library stream (each shape first",
           "runs one discarded B = 1 graph of its own: the first replay after the copies are made ran 10-15% slow);",
           "weights rotate over enough device copies to exceed the 256 MB MALL.  GB/s = (weight bytes + B x",
           "(in + out) x 4) / time;",
           "% = of 8 TB/s.  Every format runs the int8-MFMA digit GEMV on packed 16-row tile records",
           "(`k_gemv_mfma<format, ...>`; the 248320-row lm_head at B = 4 and 8 through `k_gemv_wide`, its",
           "activations in LDS, where that measured faster).", ""]
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


# The 27B hybrid's dimensions (hidden 5120, FFN 17408, vocab 248320; GDN: 16 key heads and
# 48 value heads of 128, conv kernel 4; attention: 24 query / 4 KV heads of 256, q||gate)
D27 = dict(E=5120, F=17408, V=248320, KD=2048, VD=6144, VH=48, HS=128, CONV=10240, QD=6144, KV=1024)
IQ4_ROW = lambda cols: cols // 256 * 136        # bytes of one IQ4_XS row
DIGITS = 3                                      # activation digit bytes per element (int8 x 3)


def prep_kind(k):
    """(transform kind, partial planes or None) of a preparation kernel name: k_prep_tok<KIND, NP>
    (one token per block) or the older k_prep_act<KIND>; kinds 2 SiLU x up, 3 gated norm, 4 RMSNorm,
    5 RMSNorm on gathered embedding rows"""
    m = re.match(r"k_prep_(tok|act)<(\d+)(?:, (\d+))?>", k)
    if not m:
        return None, None
    return int(m.group(2)), (int(m.group(3)) if m.group(3) is not None else None)


def gemv_tiles(k, grid, ncu=256):
    """row tiles of a k_gemv_mfma launch of grid blocks: a pair-split launch (mode bit 4) runs its last
    r = tiles mod ncu tiles as two blocks each (r <= ncu / 2), so grid = tiles + r"""
    m = re.match(r"k_gemv_mfma<\d+, \d+, \d+, (\d+)>", k)
    if not m or not int(m.group(1)) & 4:
        return grid
    for t in range(grid // 2, grid + 1):
        r = t % ncu
        if t > ncu and 0 < r <= ncu // 2 and t + r == grid:
            return t
    return grid


def step_roles(step, B, P):
    """(role, bytes) of each dispatch of one verify step, by kernel name, grid and what came before"""
    d, f4 = D27, 4
    out, prev, n_part = [], "", 0
    gdn_in = d["CONV"] + d["VD"] + 2 * d["VH"]          # rows of the GDN input projection
    for name, _, dur, gx, wx in step:
        k, grid = short(name), gx // max(wx, 1)
        kind, planes = prep_kind(k)
        prev_kind, _ = prep_kind(prev)
        mm = re.match(r"k_gemv_mfma<\d+, \d+, \d+, (\d+)>", k)
        split = bool(mm) and bool(int(mm.group(1)) & 2)          # mode bit 2: K-split partial planes
        if k.startswith("k_dequant_rows"):
            role, by = "embedding rows (dequant)", B * IQ4_ROW(d["E"]) + B * d["E"] * f4
        elif kind == 5:   # the first RMSNorm of a forward on embedding rows it gathers itself
            role = "RMSNorm prep (embedding rows gathered)"
            by = B * IQ4_ROW(d["E"]) + d["E"] * f4 + B * d["E"] * (2 * f4 + DIGITS)
        elif kind == 4:
            np_ = n_part if planes is None else planes
            role = "RMSNorm prep (+ residual partials)"
            by = (1 + np_) * B * d["E"] * f4 + d["E"] * f4 + B * d["E"] * (2 * f4 + DIGITS)
        elif kind == 3:
            role, by = "gated-norm prep (GDN out)", 2 * B * d["VD"] * f4 + B * d["VD"] * (f4 + DIGITS)
        elif kind == 2:
            role, by = "SiLU x up prep", 2 * B * d["F"] * f4 + B * d["F"] * (f4 + DIGITS)
        elif split and grid > 1024 and grid < 1280 and prev_kind in (4, 5):
            # the GDN input projection with beta and alpha cut into one K range per super-block
            kba = (grid - (d["CONV"] + d["VD"]) // 16) // (2 * d["VH"] // 16)
            role = "GEMV GDN in (qkv, z; beta, alpha K-split)"
            by = gdn_in * IQ4_ROW(d["E"]) + B * d["E"] * DIGITS + B * (d["CONV"] + d["VD"]) * f4 + \
                kba * B * 2 * d["VH"] * f4
            n_part = 0
        elif split:
            ks = max(1, grid // (d["E"] // 16))
            cols = {3: d["VD"], 2: d["F"]}.get(prev_kind, d["QD"] if prev == "k_attn_combine_act" else 0)
            role = {3: "GEMV ssm_out (K-split)", 2: "GEMV ffn_down (K-split)"}.get(
                prev_kind, "GEMV attn_output (K-split)" if prev == "k_attn_combine_act" else "GEMV K-split (?)")
            by = d["E"] * IQ4_ROW(cols) + B * cols * DIGITS + ks * B * d["E"] * f4
            n_part = ks
        elif k.startswith("k_gemv_mfma"):
            grid = gemv_tiles(k, grid)
            rows = {1030: gdn_in, 896: 2 * d["QD"] + 2 * d["KV"], 2176: 2 * d["F"],
                    15520: d["V"]}.get(grid, grid * 16)
            role = {1030: "GEMV GDN in (qkv, z, beta, alpha)", 896: "GEMV attention q||gate, k, v",
                    2176: "GEMV ffn_gate + ffn_up", 15520: "GEMV lm_head"}.get(grid, f"GEMV {rows} rows")
            by = rows * IQ4_ROW(d["E"]) + B * d["E"] * DIGITS + B * rows * f4
            if grid != 15520:
                n_part = 0
        elif k.startswith("k_gemv_wide"):      # the lm_head with its activations in LDS
            role = "GEMV lm_head"
            by = d["V"] * IQ4_ROW(d["E"]) + B * d["E"] * DIGITS + B * d["V"] * f4
        elif k == "k_gdn_fused":
            state = d["VH"] * d["HS"] * d["HS"] * f4
            io = (1 + B) * d["CONV"] * 3 * f4 + B * (d["CONV"] + d["VD"] + 2 * d["VH"]) * f4
            if B >= 5:      # rank-1 factor form (the model's default from 5 tokens): one state in, one out
                ftok = (d["VD"] + d["KD"] + d["VH"]) * f4
                role = "GDN conv + recurrence (factor form)"
                by = 2 * state + 2 * B * ftok + io
            else:
                role = "GDN conv + recurrence + snapshots"
                by = (1 + B) * state + io
        elif k.startswith("k_attn_span"):
            role = "attention spans (KV read)"
            by = P * 2 * d["KV"] * f4 + B * (2 * d["QD"] + 2 * d["KV"]) * f4
        elif k == "k_attn_combine_act":
            role, by = "attention combine + o-proj prep", B * d["QD"] * (2 * f4 + DIGITS)
        elif k == "k_copy":
            role, by = "hidden-state copy (h_save)", 2 * B * d["E"] * f4
        elif k.startswith("k_argmax"):
            role, by = "argmax", B * d["V"] * f4 if k == "k_argmax_part" else 0
        else:
            role, by = k, 0
        out.append((role, k, grid, wx, dur, by))
        prev = k
    return out


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
    roles = {}
    for g in steps:
        for role, k, gb, wx, dur, by in step_roles(g, a.rows, a.pos):
            r = roles.setdefault((role, k), [0, 0.0, 0.0])
            r[0] += 1
            r[1] += dur
            r[2] += by
    tot_by = sum(r[2] for r in roles.values()) / n
    out += ["", f"## HBM fraction per kernel role (B = {a.rows}, {a.pos} KV positions)", "",
            "Algorithmic bytes per launch: the weights a GEMV streams (IQ4_XS rows of the 27B matrices) plus its",
            "activation digits in and fp32 outputs (or K-split partial planes) out; a preparation's fp32 rows in",
            "(residual + partial planes, gate and up, ...) and its fp32 rows and digit planes out; GDN: the state",
            "read, B state snapshots written, conv state and inputs/outputs; attention: the K and V rows of every",
            "position.  GB/s = bytes / average duration; fraction of 8000 GB/s.",
            "", "| role | kernel | launches per step | avg us | MB per launch | GB/s | fraction | % of step time |",
            "|---|---|---:|---:|---:|---:|---:|---:|"]
    for (role, k), (cnt, dur, by) in sorted(roles.items(), key=lambda kv: -kv[1][1]):
        if dur / n / 1e3 < a.min_us:
            continue
        gbs = by / dur if dur else 0.0          # bytes / ns = GB/s
        out.append(f"| {role} | `{k}` | {cnt / n:.1f} | {dur / cnt / 1e3:.2f} | {by / cnt / 1e6:.2f} | {gbs:.0f} | "
                   f"{gbs / 8000:.3f} | {100 * dur / n / busy:.1f} |")
    out += ["", f"Whole step: {tot_by / 1e9:.2f} GB algorithmic in {busy / 1e3:.1f} us of kernel time = "
                f"{tot_by / busy:.0f} GB/s ({tot_by / busy / 8000:.3f} of 8 TB/s)."]
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
    st.add_argument("--pos", type=int, default=640, help="KV positions of the verify steps (bytes of attention)")
    cn = sub.add_parser("counters")
    cn.add_argument("dbs", nargs="+")
    cn.add_argument("--bench-json", required=True)
    cn.add_argument("--cmd", required=True, help="the commands, separated by ' ;; '")
    kc = sub.add_parser("kcounters")
    kc.add_argument("dbs", nargs="+")
    kc.add_argument("--bench-json", required=True)
    kc.add_argument("--kernel", default="k_attn_span")
    kc.add_argument("--cmd", required=True, help="the commands, separated by ' ;; '")
    a = ap.parse_args()
    {"stats": cmd_stats, "traffic": cmd_traffic, "sweep": cmd_sweep, "steps": cmd_steps,
     "counters": cmd_counters, "kcounters": cmd_kcounters}[a.cmd_name](a)


if __name__ == "__main__":
    main()
