"""HBM traffic per launch of the decoder step's kernels from rocprofv3 PMC runs.

``python -m cruise_amd.pmcsummary FETCH_DIR WRITE_DIR COPY_FETCH_DIR
COPY_WRITE_DIR --trace TRACE.json [--out NAME]`` reads four
``run_counter_collection.csv`` files written by

    rocprofv3 --pmc FETCH_SIZE -f csv -d FETCH_DIR -o run -- python3 -m cruise_amd.opbench --iters 5
    rocprofv3 --pmc WRITE_SIZE -f csv -d WRITE_DIR -o run -- python3 -m cruise_amd.opbench --iters 5
    rocprofv3 --pmc FETCH_SIZE -f csv -d COPY_FETCH_DIR -o run -- python3 -m cruise_amd.opbench --copy-bytes 1073741824 --iters 3
    rocprofv3 --pmc WRITE_SIZE -f csv -d COPY_WRITE_DIR -o run -- python3 -m cruise_amd.opbench --copy-bytes 1073741824 --iters 3

Each counter is scaled by what it reads for the plain 1 GiB device copy
(``__amd_rocclr_copyBuffer``: true bytes / counter KiB).  The traffic of a
kernel is the median calibrated FETCH_SIZE + WRITE_SIZE over its dispatches;
it is set against the launch's algorithmic bytes (``opbench``'s formula at the
opbench workload: B=4, context 128) and, with the mean in-graph duration from
a kernel-trace summary of ``bench.py`` (``profsummary --out``'s JSON), gives
the achieved algorithmic GB/s and the fraction of the 8 TB/s peak.
"""
from __future__ import annotations

import argparse
import csv
import json
import statistics
from pathlib import Path

from .opbench import algorithmic_bytes
from .profsummary import short_name

HBM_PEAK_GBS = 8000.0
COPY_KERNEL = "__amd_rocclr_copyBuffer"
COPY_BYTES = 1 << 30
# Qwen2.5-7B shape at the opbench workload
SHAPE = dict(B=4, H=3584, I=18944, V=152064, qkv_rows=4608, kv_dim=512, ctx=128)
# decoder-step kernels (short names) -> opbench op
OPS = {
    "k_qkv_ksplit<9>": "qkv",
    "k_attn<unsigned short, 128, true>": "attention",
    "k_resid<unsigned short, 4, 7>": "o_proj",
    "k_proj<unsigned short, 4, 4, 1, true>": "gate_up",
    "k_down_whole": "down",
    "k_proj<unsigned short, 4, 4, 2, true>": "lm_head",
}


def counters(directory: Path) -> dict[str, list[float]]:
    """Counter values (KiB) per kernel short name."""
    out: dict[str, list[float]] = {}
    with open(directory / "run_counter_collection.csv") as f:
        for row in csv.DictReader(f):
            out.setdefault(short_name(row["Kernel_Name"]), []).append(float(row["Counter_Value"]))
    return out


def summarize(fetch: Path, write: Path, copy_fetch: Path, copy_write: Path, trace: Path | None) -> dict:
    f, w = counters(fetch), counters(write)
    cf = statistics.median(counters(copy_fetch)[COPY_KERNEL])
    cw = statistics.median(counters(copy_write)[COPY_KERNEL])
    f_factor, w_factor = COPY_BYTES / (cf * 1024), COPY_BYTES / (cw * 1024)
    durations = {}
    if trace is not None:
        durations = {k["kernel"]: k["mean_us"] for k in json.loads(trace.read_text())["kernels"]}
    rows = []
    for kernel, op in OPS.items():
        if kernel not in f or kernel not in w:
            continue
        fetch_b = statistics.median(f[kernel]) * 1024 * f_factor
        write_b = statistics.median(w[kernel]) * 1024 * w_factor
        algo = algorithmic_bytes(op, **SHAPE)
        us = durations.get(kernel)
        rows.append({
            "kernel": kernel, "op": op, "dispatches": len(f[kernel]),
            "fetch_bytes": round(fetch_b), "write_bytes": round(write_b), "traffic_bytes": round(fetch_b + write_b),
            "algorithmic_bytes": algo, "traffic_over_algorithmic": round((fetch_b + write_b) / algo, 4),
            "in_graph_mean_us": round(us, 2) if us else None,
            "achieved_gbs": round(algo / (us * 1e-6) / 1e9, 1) if us else None,
            "hbm_frac": round(algo / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4) if us else None,
        })
    return {"copy_calibration": {"bytes": COPY_BYTES, "fetch_kib": cf, "write_kib": cw,
                                 "fetch_factor": f_factor, "write_factor": w_factor}, "kernels": rows}


def markdown(s: dict, commands: list[str]) -> str:
    c = s["copy_calibration"]
    lines = ["Commands (repository root, one MI355X):", "", "```", *commands, "```", "",
             f"Calibration: a 1 GiB device copy reads FETCH_SIZE {c['fetch_kib']:.1f} KiB (x{c['fetch_factor']:.3f} "
             f"to true bytes) and WRITE_SIZE {c['write_kib']:.1f} KiB (x{c['write_factor']:.3f}).", "",
             "| kernel | op | traffic B/launch | algorithmic B/launch | traffic / algorithmic | in-graph mean us | "
             "algorithmic GB/s | HBM frac |", "|---|---|---:|---:|---:|---:|---:|---:|"]
    for r in s["kernels"]:
        us = f"{r['in_graph_mean_us']:.2f}" if r["in_graph_mean_us"] else "-"
        gbs = f"{r['achieved_gbs']:.0f}" if r["achieved_gbs"] else "-"
        frac = f"{r['hbm_frac']:.3f}" if r["hbm_frac"] else "-"
        lines.append(f"| `{r['kernel']}` | {r['op']} | {r['traffic_bytes']:,} | {r['algorithmic_bytes']:,} | "
                     f"{r['traffic_over_algorithmic']:.3f} | {us} | {gbs} | {frac} |")
    return "\n".join(lines) + "\n"


def main() -> int:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("fetch", type=Path)
    p.add_argument("write", type=Path)
    p.add_argument("copy_fetch", type=Path)
    p.add_argument("copy_write", type=Path)
    p.add_argument("--trace", type=Path, help="profsummary JSON of a bench.py kernel trace (in-graph durations)")
    p.add_argument("--command", action="append", default=[], help="a command that produced the inputs")
    p.add_argument("--out", type=Path)
    args = p.parse_args()
    s = summarize(args.fetch, args.write, args.copy_fetch, args.copy_write, args.trace)
    text = markdown(s, args.command)
    print(text)
    if args.out:
        args.out.with_suffix(".md").write_text(text)
        args.out.with_suffix(".json").write_text(json.dumps(s, indent=1) + "\n")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
