"""Summaries of rocprofv3 output for the committed profiles (kernel traces and HBM traffic).

rocprofv3 writes one row per dispatch (`--kernel-trace`: `*_kernel_trace.csv`; `--pmc`:
`*_counter_collection.csv`, one row per dispatch and counter). The library GEMMs of the draft step
share one kernel name between shapes (the teacher table and the head dgrad GEMM run the same
solution), so dispatches are grouped by (kernel name, grid size), and a region of the bench maps to
one such group.

    python -m aspec_amd.profiling trace <kernel_trace.csv> [--md OUT] [--gaps NAME ...]
    python -m aspec_amd.profiling traffic --fetch <csv> --write <csv> --copy-fetch <csv>
                                          --copy-write <csv> --copy-mib MIB [--json OUT]
    python -m aspec_amd.profiling counters <counter_collection.csv> ... [--match NAME ...] [--md OUT]

`trace` prints per-group launch statistics and, for each `--gaps` pattern, the GPU-idle time
before each matching dispatch (its start minus the latest end of every earlier dispatch).
`traffic` turns FETCH_SIZE / WRITE_SIZE (KiB per dispatch) into bytes per launch, each scaled by
what the same counter reads for a plain device copy of known size (`bench.py --copy-calibration`).
`counters` averages SQ / GRBM counters per (kernel, grid) over one or more passes and derives:
MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (SIMDs x GRBM_GUI_ACTIVE / XCDs), the share of the kernel's
cycles an average SIMD's MFMA pipe is busy; VALU, SALU and LDS instructions per MFMA
(SQ_INSTS_VALU counts the MFMAs too); the LDS bank-conflict rate; and the shares of the waves'
resident cycles spent waiting for an LDS result or for anything.
"""

from __future__ import annotations

import argparse
import csv
import json
import re
import statistics
from collections import defaultdict

# The bench's regions and the dispatch group each times: (kernel-name pattern, grid size or None).
# The head GEMMs are the solutions recorded in aspec_amd/tuning/head_gemms_gfx950.csv; the grid
# sizes are those solutions' launch grids at config 2.
REGION_GROUPS = {
    "attn_fwd": ("attn_fwd_kernel<4>", None),
    "attn_bwd_prepare": ("attn_bwd_pre_kernel", None),
    "attn_bwd_dq": ("attn_bwd_dq_kernel<4>", None),
    "attn_bwd_dkdv": ("attn_bwd_dkdv_kernel<4>", None),
    "attn_bwd_finalize": ("attn_bwd_acc_kernel", None),
    "loss_fused": ("loss_fwd_persistent<8, false, true, true>", None),
    "loss_fwd": ("loss_fwd_persistent<8, false, true>", None),
    "loss_bwd": ("loss_bwd_rows_kernel", None),
    "head_gemm_fwd": ("Cijk_Alik_Bljk_BBS_BH_MT256x256x64_MI16x16x1_UserArgs_shortname0", 1024000),
    "head_gemm_dgrad": ("Cijk_Alik_Bljk_BBS_BH_MT256x256x64_MI16x16x1_UserArgs_shortname1", 131072),
    "teacher_gemm": ("Cijk_Alik_Bljk_BBS_BH_MT256x256x64_MI16x16x1_UserArgs_shortname1", 512000),
    "qk_norm_rope_fwd": ("qk_norm_rope_fwd_kernel<false>", None),
    "qk_norm_rope_bwd": ("qk_norm_rope_bwd_kernel<false>", None),
    "pack_copy": ("pack_copy_kernel", None),
}


def short_name(name: str) -> str:
    """The kernel's name without namespaces, return type and argument list (templates kept)."""
    name = name.strip().replace("(anonymous namespace)::", "")
    if name.startswith("void "):
        name = name[5:]
    depth, cut = 0, len(name)
    for i, ch in enumerate(name):  # the argument list starts at the first '(' outside templates
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            cut = i
            break
    name = name[:cut]
    return re.sub(r"^(?:[A-Za-z_][A-Za-z0-9_]*::)+(?=[A-Za-z_~])", "", name)


def _grid(row) -> int:
    if "Grid_Size_X" in row:
        return int(row["Grid_Size_X"]) * int(row["Grid_Size_Y"]) * int(row["Grid_Size_Z"])
    return int(row["Grid_Size"])


def load_dispatches(path):
    """Kernel-trace rows as dicts (name, grid, start_ns, end_ns), in start order."""
    out = []
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            if r.get("Kind", "KERNEL_DISPATCH") != "KERNEL_DISPATCH":
                continue
            out.append({"name": short_name(r["Kernel_Name"]), "grid": _grid(r),
                        "start": int(r["Start_Timestamp"]), "end": int(r["End_Timestamp"])})
    out.sort(key=lambda d: d["start"])
    return out


def group_key(name: str, grid: int) -> str:
    return f"{name} [grid {grid}]"


def kernel_stats(dispatches):
    """{group: {calls, avg_us, min_us, max_us, total_us}} over (name, grid) groups."""
    groups = defaultdict(list)
    for d in dispatches:
        groups[group_key(d["name"], d["grid"])].append((d["end"] - d["start"]) / 1e3)
    return {k: {"calls": len(v), "avg_us": sum(v) / len(v), "min_us": min(v), "max_us": max(v),
                "total_us": sum(v)} for k, v in groups.items()}


def region_matches(region: str, name: str, grid: int) -> bool:
    pattern, want_grid = REGION_GROUPS[region]
    return pattern in name and (want_grid is None or grid == want_grid)


def region_stats(dispatches, phases=None):
    """Per bench region: launches and mean/median duration (us) of the dispatches it times. With
    `phases` [(label, count), ...] (a region launches once per step, so its k-th dispatch belongs
    to step k), the same figures per consecutive phase of steps, e.g. the bench's warmup, timed
    steps, and its per-kernel timing pass."""
    out = {}
    for region in REGION_GROUPS:
        ds = [(d["end"] - d["start"]) / 1e3 for d in dispatches if region_matches(region, d["name"], d["grid"])]
        if not ds:
            continue
        out[region] = {"calls": len(ds), "avg_us": sum(ds) / len(ds), "median_us": statistics.median(ds)}
        if phases:
            at, split = 0, {}
            for label, count in phases:
                part = ds[at:at + count]
                at += count
                if part:
                    split[label] = {"calls": len(part), "avg_us": sum(part) / len(part)}
            out[region]["phases"] = split
    return out


def idle_gaps(dispatches, pattern: str, grid: int | None = None):
    """GPU-idle microseconds before each dispatch whose name contains `pattern` (and of `grid`):
    its start minus the latest end among all earlier dispatches."""
    latest, gaps = None, []
    for d in dispatches:
        if pattern in d["name"] and (grid is None or d["grid"] == grid) and latest is not None:
            gaps.append(max(0.0, (d["start"] - latest) / 1e3))
        latest = d["end"] if latest is None else max(latest, d["end"])
    return gaps


def step_timeline(dispatches, marker: str, grid: int | None = None):
    """Split the trace into steps at each dispatch matching `marker` (and `grid`) and report, per
    step, the span from one marker dispatch to the next, the time at least one kernel ran (the
    union of the dispatch intervals, so overlapping streams count once), the idle rest and the
    three largest idle gaps with the kernel that followed each."""
    starts = [i for i, d in enumerate(dispatches) if marker in d["name"] and (grid is None or d["grid"] == grid)]
    steps = []
    for a, b in zip(starts, starts[1:]):
        seg = dispatches[a:b]
        t0, t1 = seg[0]["start"], dispatches[b]["start"]
        busy, cur_s, cur_e, gaps = 0, None, None, []
        for d in sorted(seg, key=lambda x: x["start"]):
            s0, e0 = d["start"], min(d["end"], t1)
            if cur_e is None or s0 > cur_e:
                if cur_e is not None:
                    busy += cur_e - cur_s
                    gaps.append(((s0 - cur_e) / 1e3, d["name"]))
                cur_s, cur_e = s0, e0
            else:
                cur_e = max(cur_e, e0)
        busy += cur_e - cur_s
        if t1 > cur_e:
            gaps.append(((t1 - cur_e) / 1e3, dispatches[b]["name"]))
        gaps.sort(key=lambda g: -g[0])
        steps.append({"span_us": (t1 - t0) / 1e3, "busy_us": busy / 1e3, "idle_us": (t1 - t0 - busy) / 1e3,
                      "largest_gaps": [(round(g, 1), n[:48]) for g, n in gaps[:3]]})
    return steps


def counter_per_dispatch(path, counter: str):
    """{(name, grid): [value per dispatch]} of one counter from a counter_collection.csv."""
    out = defaultdict(list)
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] == counter:
                out[(short_name(r["Kernel_Name"]), _grid(r))].append(float(r["Counter_Value"]))
    return out


def copy_factor(path, counter: str, mib: int) -> float:
    """Bytes per counter unit: a plain device copy of `mib` MiB reads and writes mib MiB; its
    largest dispatch's reading of the counter (KiB) gives the scale."""
    values = counter_per_dispatch(path, counter)
    best = max(max(v) for v in values.values())
    return mib * 2**20 / (best * 1024.0)


def traffic(fetch_csv, write_csv, copy_fetch_csv, copy_write_csv, copy_mib):
    """{group: {read_bytes, write_bytes}} per launch, calibrated by the copy kernel."""
    ff = copy_factor(copy_fetch_csv, "FETCH_SIZE", copy_mib)
    wf = copy_factor(copy_write_csv, "WRITE_SIZE", copy_mib)
    fetch = counter_per_dispatch(fetch_csv, "FETCH_SIZE")
    write = counter_per_dispatch(write_csv, "WRITE_SIZE")
    kernels = {}
    for key in sorted(set(fetch) | set(write)):
        r = fetch.get(key, [])
        w = write.get(key, [])
        kernels[group_key(*key)] = {
            "calls": max(len(r), len(w)),
            "read_bytes": (sum(r) / len(r)) * 1024.0 * ff if r else None,
            "write_bytes": (sum(w) / len(w)) * 1024.0 * wf if w else None,
        }
    regions = {}
    for region in REGION_GROUPS:
        for (name, grid) in set(fetch) | set(write):
            if region_matches(region, name, grid):
                k = kernels[group_key(name, grid)]
                regions[region] = {"group": group_key(name, grid), "read_bytes": k["read_bytes"],
                                   "write_bytes": k["write_bytes"]}
    return {"calibration": {"fetch_factor": ff, "write_factor": wf, "copy_mib": copy_mib},
            "regions": regions, "kernels": kernels}


MI355X_SIMDS, MI355X_XCDS = 1024, 8


def counter_summary(paths, match=()):
    """{group: {counter: mean per dispatch}} over counter_collection CSVs (several passes of the
    same program), restricted to kernels whose name contains one of `match` (all when empty)."""
    sums = defaultdict(lambda: defaultdict(list))
    for path in paths:
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                name = short_name(r["Kernel_Name"])
                if match and not any(m in name for m in match):
                    continue
                sums[group_key(name, _grid(r))][r["Counter_Name"]].append(float(r["Counter_Value"]))
    return {k: {c: sum(v) / len(v) for c, v in d.items()} for k, d in sums.items()}


def counters_markdown(summary):
    def ratio(d, a, b, scale=1.0):
        return d[a] / (d[b] * scale) if a in d and b in d and d[b] else float("nan")

    lines = ["| kernel [grid] | GRBM cycles/XCD | MFMA busy | VALU per MFMA | SALU per MFMA | "
             "LDS per MFMA | LDS bank conflicts | LDS wait share | any-wait share |",
             "|---|---:|---:|---:|---:|---:|---:|---:|---:|"]
    for k, d in sorted(summary.items(), key=lambda kv: -kv[1].get("GRBM_GUI_ACTIVE", 0)):
        gui = d.get("GRBM_GUI_ACTIVE", float("nan"))
        busy = d["SQ_VALU_MFMA_BUSY_CYCLES"] / (MI355X_SIMDS * gui / MI355X_XCDS) if "SQ_VALU_MFMA_BUSY_CYCLES" in d else float("nan")
        lines.append(f"| `{k[:80]}` | {gui / MI355X_XCDS:.0f} | {busy:.3f} | {ratio(d, 'SQ_INSTS_VALU', 'SQ_INSTS_MFMA'):.2f} | "
                     f"{ratio(d, 'SQ_INSTS_SALU', 'SQ_INSTS_MFMA'):.2f} | {ratio(d, 'SQ_INSTS_LDS', 'SQ_INSTS_MFMA'):.2f} | "
                     f"{ratio(d, 'SQ_LDS_BANK_CONFLICT', 'SQ_LDS_IDX_ACTIVE'):.4f} | "
                     f"{ratio(d, 'SQ_WAIT_INST_LDS', 'SQ_WAVE_CYCLES'):.3f} | {ratio(d, 'SQ_WAIT_ANY', 'SQ_WAVE_CYCLES'):.3f} |")
    lines += ["", "Raw means per dispatch:", ""]
    for k, d in sorted(summary.items()):
        lines.append(f"- `{k[:80]}`: " + ", ".join(f"{c} {v:.4g}" for c, v in sorted(d.items())))
    return "\n".join(lines)


def traffic_markdown(out, top=20):
    cal = out["calibration"]
    lines = [f"Calibration: a {cal['copy_mib']} MiB device copy gives {cal['fetch_factor']:.4f} bytes per FETCH_SIZE "
             f"byte-unit and {cal['write_factor']:.4f} per WRITE_SIZE byte-unit (KiB counters x 1024 x factor).", "",
             "| bench region | dispatch group | HBM read MB | HBM write MB |", "|---|---|---:|---:|"]
    for region, r in out["regions"].items():
        rd = "" if r["read_bytes"] is None else f"{r['read_bytes'] / 1e6:.1f}"
        wr = "" if r["write_bytes"] is None else f"{r['write_bytes'] / 1e6:.1f}"
        lines.append(f"| {region} | `{r['group'][:80]}` | {rd} | {wr} |")
    lines += ["", f"All dispatch groups, largest traffic first (top {top}):", "",
              "| dispatch group | launches | HBM read MB | HBM write MB |", "|---|---:|---:|---:|"]
    rows = sorted(out["kernels"].items(), key=lambda kv: -((kv[1]["read_bytes"] or 0) + (kv[1]["write_bytes"] or 0)))
    for k, r in rows[:top]:
        rd = "" if r["read_bytes"] is None else f"{r['read_bytes'] / 1e6:.1f}"
        wr = "" if r["write_bytes"] is None else f"{r['write_bytes'] / 1e6:.1f}"
        lines.append(f"| `{k[:90]}` | {r['calls']} | {rd} | {wr} |")
    return "\n".join(lines)


def trace_markdown(dispatches, gap_patterns=(), phases=None):
    stats = kernel_stats(dispatches)
    total = sum(s["total_us"] for s in stats.values())
    lines = ["| kernel [grid] | calls | avg us | min us | max us | % of GPU time |",
             "|---|---:|---:|---:|---:|---:|"]
    for k, s in sorted(stats.items(), key=lambda kv: -kv[1]["total_us"]):
        lines.append(f"| `{k[:90]}` | {s['calls']} | {s['avg_us']:.1f} | {s['min_us']:.1f} | "
                     f"{s['max_us']:.1f} | {100 * s['total_us'] / total:.2f} |")
    labels = [label for label, _ in phases or ()]
    lines += ["", "Per bench region (dispatch groups of `aspec_amd.profiling.REGION_GROUPS`)"
              + (f"; avg us per phase of steps ({', '.join(f'{l}: {c}' for l, c in phases)})" if phases else "")
              + ":", "",
              "| region | calls | avg us | median us |" + "".join(f" {l} avg us |" for l in labels),
              "|---|---:|---:|---:|" + "---:|" * len(labels)]
    for region, s in region_stats(dispatches, phases).items():
        cells = "".join(f" {s['phases'][l]['avg_us']:.1f} |" if l in s.get("phases", {}) else " |" for l in labels)
        lines.append(f"| {region} | {s['calls']} | {s['avg_us']:.1f} | {s['median_us']:.1f} |" + cells)
    for spec in gap_patterns:
        pattern, _, grid = spec.partition("@")
        gaps = idle_gaps(dispatches, pattern, int(grid) if grid else None)
        if gaps:
            lines += ["", f"GPU idle before `{spec}` ({len(gaps)} dispatches): median "
                          f"{statistics.median(gaps):.1f} us, max {max(gaps):.1f} us, "
                          f"{sum(g > 10 for g in gaps)} above 10 us"]
    return "\n".join(lines)


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = p.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("trace")
    t.add_argument("csv")
    t.add_argument("--md")
    t.add_argument("--gaps", nargs="*", default=[],
                   help="kernel-name patterns (optionally NAME@GRID) whose preceding idle time is reported")
    t.add_argument("--steps-at", default="",
                   help="NAME[@GRID] of a kernel launched once per step: per-step span, busy and idle time")
    t.add_argument("--phases", default="",
                   help="consecutive phases of steps as LABEL:COUNT,... (bench.py --serial --steps S "
                        "--warmup W: warmup:W,timed:S,timing-warmup:1,timing:S)")
    q = sub.add_parser("counters")
    q.add_argument("csv", nargs="+")
    q.add_argument("--match", nargs="*", default=[])
    q.add_argument("--md")
    c = sub.add_parser("traffic")
    for name in ("fetch", "write", "copy-fetch", "copy-write"):
        c.add_argument(f"--{name}", required=True)
    c.add_argument("--copy-mib", type=int, required=True)
    c.add_argument("--json")
    c.add_argument("--md")
    args = p.parse_args(argv)
    if args.cmd == "trace":
        phases = [(p.split(":")[0], int(p.split(":")[1])) for p in args.phases.split(",") if p]
        dispatches = load_dispatches(args.csv)
        text = trace_markdown(dispatches, args.gaps, phases or None)
        if args.steps_at:
            name, _, grid = args.steps_at.partition("@")
            steps = step_timeline(dispatches, name, int(grid) if grid else None)
            text += ("\n\nPer step (from one `" + args.steps_at + "` dispatch to the next):\n\n"
                     "| step | span us | busy us | idle us | largest idle gaps (us, next kernel) |\n"
                     "|---:|---:|---:|---:|---|\n")
            for i, st in enumerate(steps):
                gaps = "; ".join(f"{g} before `{n}`" for g, n in st["largest_gaps"])
                text += f"| {i} | {st['span_us']:.1f} | {st['busy_us']:.1f} | {st['idle_us']:.1f} | {gaps} |\n"
        if args.md:
            with open(args.md, "w") as f:
                f.write(text + "\n")
        print(text)
    elif args.cmd == "counters":
        text = counters_markdown(counter_summary(args.csv, args.match))
        if args.md:
            with open(args.md, "w") as f:
                f.write(text + "\n")
        print(text)
    else:
        out = traffic(args.fetch, args.write, args.copy_fetch, args.copy_write, args.copy_mib)
        text = json.dumps(out, indent=1)
        if args.json:
            with open(args.json, "w") as f:
                f.write(text + "\n")
        if args.md:
            with open(args.md, "w") as f:
                f.write(traffic_markdown(out) + "\n")
        print(text if not args.md else traffic_markdown(out))


if __name__ == "__main__":
    main()
