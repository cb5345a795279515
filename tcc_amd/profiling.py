"""Reduce rocprofv3 output of bench.py runs to the summaries kept under
profiles/ (kernel-time tables and the counter-measured HBM traffic that
bench.py's roofline reports).

    python -m tcc_amd.profiling stats --csv <kernel_stats.csv> --title T --command C [--kernels REGEX]
        [--trace <kernel_trace.csv> --anchor REGEX] --out profiles/<name>.md
    python -m tcc_amd.profiling counters --csv <counter csv> --kernels REGEX --title T --command C
        --out profiles/<name>.md
    python -m tcc_amd.profiling traffic --config N --fetch <FETCH_SIZE counter csv> --write <WRITE_SIZE csv>
        [--hits <TCC_HIT_sum TCC_MISS_sum csv>] --stats <kernel_stats.csv> --kernels REGEX --launches L
        --command C --out profiles/traffic_configN.json

The counter runs profile `bench.py --profile-step --copy-calibration-mib
1024`: only the timed step's kernels run L = warmup + steps times, and one
1 GiB device copy gives the factors that turn FETCH_SIZE / WRITE_SIZE (KiB
per dispatch) into bytes (calibration_copy_kernel: known bytes read and
written, unlike the runtime's blit copies, whose counters vary with what the
process copied before).
"""
from __future__ import annotations

import argparse
import collections
import csv
import hashlib
import json
import os
import re
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KIB = 1024
COPY_KERNEL = "calibration_copy_kernel"


def kernel_key(name: str) -> str:
    """A kernel's name without its argument list and namespaces
    ("gather_kernel<4, Packed, values>")."""
    name = name.replace("(anonymous namespace)::", "").replace("tcc::", "")
    name = re.sub(r"^void ", "", name)
    depth, out = 0, []
    for ch in name:  # drop the parenthesised argument list, keep template arguments
        if ch == "(" and depth == 0 and out and out[-1] not in "<,":
            break
        out.append(ch)
        depth += ch == "<"
        depth -= ch == ">"
    return "".join(out).strip()


def read_counters(path: str) -> dict:
    """{kernel key: {counter: [value per dispatch]}} from a counter-collection csv."""
    per = collections.defaultdict(lambda: collections.defaultdict(list))
    with open(path) as f:
        for r in csv.DictReader(f):
            per[kernel_key(r["Kernel_Name"])][r["Counter_Name"]].append(float(r["Counter_Value"]))
    return per


def read_stats(path: str) -> list[dict]:
    with open(path) as f:
        rows = list(csv.DictReader(f))
    out = [{"kernel": kernel_key(r["Name"]), "calls": int(r["Calls"]), "avg_ms": float(r["AverageNs"]) / 1e6,
            "total_ms": float(r["TotalDurationNs"]) / 1e6, "pct": float(r["Percentage"])} for r in rows]
    return sorted(out, key=lambda r: -r["total_ms"])


def _sha(rel: str) -> str:
    with open(os.path.join(ROOT, rel), "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()[:16]


def kernel_sources(kernels) -> list[str]:
    """The source files that define the given kernels (by the base name of
    each key, as a __global__ function of tcc_amd/csrc/*.hip or *.hpp), with
    every file they include from this repository, transitively."""
    csrc = os.path.join(ROOT, "tcc_amd", "csrc")
    texts = {f"tcc_amd/csrc/{n}": open(os.path.join(csrc, n)).read()
             for n in sorted(os.listdir(csrc)) if n.endswith((".hip", ".hpp", ".cpp"))}
    found = set()
    for k in kernels:
        base = re.split(r"[<(]", k, maxsplit=1)[0].strip()
        pat = re.compile(r"__global__[^;{]*?\b" + re.escape(base) + r"\s*\(", re.S)
        found |= {rel for rel, text in texts.items() if pat.search(text)}
    todo, seen = sorted(found), set()
    while todo:
        rel = todo.pop()
        if rel in seen:
            continue
        seen.add(rel)
        text = texts.get(rel) or open(os.path.join(ROOT, rel)).read()
        for inc in re.findall(r'#include\s+"([^"]+)"', text):
            dep = os.path.normpath(os.path.join(os.path.dirname(rel), inc))
            if os.path.exists(os.path.join(ROOT, dep)) and dep not in seen:
                todo.append(dep)
    return sorted(seen)


def sources_sha(kernels=None) -> dict:
    """sha256[:16] of the sources a traffic file depends on (the files that
    define its kernels and what they include; every kernel source when
    `kernels` is None): the file holds only while they are unchanged."""
    if kernels is not None:
        return {rel: _sha(rel) for rel in kernel_sources(kernels)}
    out = {}
    for d in ("tcc_amd/csrc", "include"):
        for name in sorted(os.listdir(os.path.join(ROOT, d))):
            if name.endswith((".hip", ".hpp", ".h", ".cpp")):
                out[f"{d}/{name}"] = _sha(f"{d}/{name}")
    return out


def step_periods(trace_csv: str, anchor: str) -> list[float]:
    """Milliseconds from each dispatch of the step's anchor kernel (a kernel
    that runs once per step; regex over kernel keys) to the next one's, from
    a rocprofv3 kernel-trace csv: the step's wall time on the GPU, gaps and
    kernels that overlap on other streams included."""
    pat = re.compile(anchor)
    starts = []
    with open(trace_csv) as f:
        for r in csv.DictReader(f):
            if pat.search(kernel_key(r["Kernel_Name"])):
                starts.append(int(r["Start_Timestamp"]))
    starts.sort()
    return [(b - a) / 1e6 for a, b in zip(starts, starts[1:])]


def _short(name: str, width: int = 72) -> str:
    return name if len(name) <= width else name[: width - 3] + "..."


def stats_md(args) -> str:
    rows = read_stats(args.csv)
    total = sum(r["total_ms"] for r in rows)
    lines = [f"# {args.title}", "", "Command (from the repository root on the GPU box, TMPDIR=/tmp):", "", "```",
             args.command, "```", ""]
    d = re.search(r"rocprofv3 --kernel-trace --stats\b.*? -d (\S+) -o run\b", args.command)
    if d:
        # the tables' own command, over the files the profiling run wrote
        t = [f"python -m tcc_amd.profiling stats --csv {d.group(1)}/run_kernel_stats.csv"]
        if args.launches:
            t.append(f"--launches {args.launches}")
        if args.kernels:
            t.append(f"--kernels '{args.kernels}'")
        if args.trace:
            t.append(f"--trace {d.group(1)}/run_kernel_trace.csv --anchor '{args.anchor}'")
        t.append(f"--out {os.path.relpath(args.out, ROOT) if os.path.isabs(args.out) else args.out}")
        lines += [f"Tables: `{' '.join(t)}` (plus `--title` / `--command`).", ""]
    if args.kernels:
        pat = re.compile(args.kernels)
        step = [r for r in rows if pat.search(r["kernel"])]
        if args.launches:
            L = args.launches
            lines += [f"Step kernels (`{args.kernels}`), {L} steps:", "", "| kernel | calls | avg ms | ms per step |",
                      "|---|---:|---:|---:|"]
            lines += [f"| `{r['kernel']}` | {r['calls']} | {r['avg_ms']:.4f} | {r['total_ms'] / L:.4f} |" for r in step]
            lines += [f"| **per step** | | | **{sum(r['total_ms'] for r in step) / L:.4f}** |", ""]
        else:
            lines += [f"Step kernels (`{args.kernels}`):", "", "| kernel | calls | avg ms |", "|---|---:|---:|"]
            lines += [f"| `{r['kernel']}` | {r['calls']} | {r['avg_ms']:.4f} |" for r in step]
            lines += [f"| **sum of averages** | | **{sum(r['avg_ms'] for r in step):.4f}** |", ""]
    if args.trace:
        per = sorted(step_periods(args.trace, args.anchor))
        if per:
            med = per[len(per) // 2] if len(per) % 2 else 0.5 * (per[len(per) // 2 - 1] + per[len(per) // 2])
            lines += [f"Step period from the kernel trace (one dispatch of `{args.anchor}` to the next, "
                      f"{len(per)} periods): median **{med:.4f} ms**, min {per[0]:.4f}, max {per[-1]:.4f}.", ""]
    lines += ["All kernels, by total time:", "",
              "| kernel | calls | avg ms | total ms | % of GPU time |", "|---|---:|---:|---:|---:|"]
    for r in rows[: args.top]:
        lines.append(f"| `{_short(r['kernel'])}` | {r['calls']} | {r['avg_ms']:.4f} | {r['total_ms']:.2f} | "
                     f"{100 * r['total_ms'] / total:.1f} |")
    if args.note:
        lines += ["", args.note]
    return "\n".join(lines) + "\n"


XCDS, SIMDS = 8, 1024  # MI355X: GRBM_GUI_ACTIVE is summed over the XCDs; 256 CUs x 4 SIMDs


def counters_md(args) -> str:
    """Per-kernel means of one counter pass, with the MFMA-busy fraction
    SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / XCDs x SIMDs) and the
    dependency-wait fraction SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES when present."""
    per = read_counters(args.csv)
    pat = re.compile(args.kernels)
    names = sorted({c for k, cs in per.items() if pat.search(k) for c in cs})
    lines = [f"# {args.title}", "", "Command (from the repository root on the GPU box, TMPDIR=/tmp):", "", "```",
             args.command, "```", "", "Means per dispatch:", ""]
    extra = []
    if "SQ_VALU_MFMA_BUSY_CYCLES" in names and "GRBM_GUI_ACTIVE" in names:
        extra.append("MFMA busy")
    if "SQ_WAIT_INST_ANY" in names and "SQ_WAVE_CYCLES" in names:
        extra.append("wait / wave cycles")
    lines.append("| kernel | dispatches | " + " | ".join(names + extra) + " |")
    lines.append("|---|---:|" + "---:|" * (len(names) + len(extra)))
    for k in sorted(per):
        if not pat.search(k):
            continue
        c = per[k]
        mean = {n: sum(c[n]) / len(c[n]) for n in names if c.get(n)}
        cells = [f"{mean[n]:,.0f}" if n in mean else "" for n in names]
        if "MFMA busy" in extra:
            gui = mean.get("GRBM_GUI_ACTIVE", 0)
            cells.append(f"{mean.get('SQ_VALU_MFMA_BUSY_CYCLES', 0) / (gui / XCDS * SIMDS):.3f}" if gui else "")
        if "wait / wave cycles" in extra:
            wc = mean.get("SQ_WAVE_CYCLES", 0)
            cells.append(f"{mean.get('SQ_WAIT_INST_ANY', 0) / wc:.3f}" if wc else "")
        n_disp = max(len(v) for v in c.values())
        lines.append(f"| `{_short(k)}` | {n_disp} | " + " | ".join(cells) + " |")
    if args.note:
        lines += ["", args.note]
    return "\n".join(lines) + "\n"


def traffic_json(args) -> dict:
    fetch, write = read_counters(args.fetch), read_counters(args.write)
    hits = read_counters(args.hits) if args.hits else {}
    stats = {r["kernel"]: r for r in read_stats(args.stats)}
    copy_f = [v for k, c in fetch.items() if COPY_KERNEL in k for v in c.get("FETCH_SIZE", [])]
    copy_w = [v for k, c in write.items() if COPY_KERNEL in k for v in c.get("WRITE_SIZE", [])]
    if not copy_f or not copy_w:
        raise SystemExit("no calibration_copy_kernel dispatch in the counter files (run bench.py with "
                         "--copy-calibration-mib)")
    gib_kib = (1 << 30) / KIB
    ff, fw = gib_kib / max(copy_f), gib_kib / max(copy_w)
    pat = re.compile(args.kernels)
    per, total = {}, 0.0
    for k in sorted(set(fetch) | set(write)):
        if not pat.search(k) or COPY_KERNEL in k:
            continue
        f = fetch.get(k, {}).get("FETCH_SIZE", [])
        w = write.get(k, {}).get("WRITE_SIZE", [])
        b = (sum(f) * ff + sum(w) * fw) * KIB / args.launches
        total += b
        e = {"dispatches": len(f), "fetch_kib_raw_sum": round(sum(f)), "write_kib_raw_sum": round(sum(w)),
             "hbm_bytes_per_step": round(b)}
        h = hits.get(k, {})
        if h.get("TCC_HIT_sum") and h.get("TCC_MISS_sum"):
            hs, ms = sum(h["TCC_HIT_sum"]), sum(h["TCC_MISS_sum"])
            e["l2_hit_rate"] = round(hs / (hs + ms), 4)
        if k in stats:
            e["avg_ms_rocprof"] = round(stats[k]["avg_ms"], 6)
            e["calls_rocprof"] = stats[k]["calls"]
        per[k] = e
    # the stats may come from another run: average launch time x dispatches per step
    step_ms = sum(stats[k]["avg_ms"] * per[k]["dispatches"] / args.launches for k in per if k in stats) or None
    out = {"config": args.config, "kernels": args.kernels, "launches": args.launches,
           "hbm_bytes_per_launch": round(total), "per_kernel": per,
           "copy_calibration": {"bytes": 1 << 30, "fetch_kib": round(max(copy_f)), "write_kib": round(max(copy_w)),
                                "fetch_scale": round(ff, 4), "write_scale": round(fw, 4)},
           "step_kernel_ms_rocprof": None if step_ms is None else round(step_ms, 6),
           "command": args.command, "sources": sources_sha(list(per))}
    if step_ms:
        out["dram_side_GBps"] = round(total / (step_ms * 1e-3) / 1e9, 1)
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stats")
    s.add_argument("--csv", required=True)
    s.add_argument("--title", required=True)
    s.add_argument("--command", required=True)
    s.add_argument("--note", default="")
    s.add_argument("--kernels", default="", help="regex over kernel names: the step's kernels, listed first")
    s.add_argument("--launches", type=int, default=0, help="steps in the run: report each kernel's time per step")
    s.add_argument("--top", type=int, default=15)
    s.add_argument("--trace", help="kernel-trace csv of the same run: report the step period")
    s.add_argument("--anchor", default="", help="regex of a kernel that runs once per step (with --trace)")
    s.add_argument("--out", required=True)
    c = sub.add_parser("counters")
    c.add_argument("--csv", required=True)
    c.add_argument("--kernels", required=True)
    c.add_argument("--title", required=True)
    c.add_argument("--command", required=True)
    c.add_argument("--note", default="")
    c.add_argument("--out", required=True)
    t = sub.add_parser("traffic")
    t.add_argument("--config", type=int, required=True)
    t.add_argument("--fetch", required=True)
    t.add_argument("--write", required=True)
    t.add_argument("--hits")
    t.add_argument("--stats", required=True)
    t.add_argument("--kernels", required=True, help="regex over kernel names: the step's kernels")
    t.add_argument("--launches", type=int, required=True, help="step executions in the profiled run")
    t.add_argument("--command", required=True)
    t.add_argument("--out", required=True)
    args = ap.parse_args(argv)
    if args.cmd == "stats":
        text = stats_md(args)
    elif args.cmd == "counters":
        text = counters_md(args)
    else:
        text = json.dumps(traffic_json(args), indent=1) + "\n"
    with open(args.out, "w") as f:
        f.write(text)
    sys.stdout.write(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
