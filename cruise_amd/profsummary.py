"""Summaries of rocprofv3 kernel traces of the resident epoch.

``python -m cruise_amd.profsummary RESULTS.db [--out NAME]`` reads the SQLite
database rocprofv3 writes with ``--kernel-trace`` (its ``kernels`` view) and
prints, per kernel, the dispatch count and the mean, minimum and maximum
duration, plus the epoch structure the trace shows: for every epoch (one
``k_ctrl_init`` ... ``k_ctrl_finish`` run) the number of copy dispatches
(``__amd_rocclr_copyBuffer``: HIP runs a captured memory copy as such a
dispatch) between it and the previous epoch, the decoder steps it ran and its
device time.  ``--out NAME`` also writes NAME.md and NAME.json.
"""
from __future__ import annotations

import argparse
import json
import sqlite3
import statistics
from pathlib import Path

COPY_KERNEL = "__amd_rocclr_copyBuffer"


def short_name(name: str) -> str:
    """Kernel name without the namespace and argument list."""
    base = name.replace("(anonymous namespace)::", "")
    base = base.split("(")[0]
    for prefix in ("void ", "re::"):
        base = base.replace(prefix, "")
    return base.strip()


def load_dispatches(db: Path) -> list[tuple[str, int, int]]:
    con = sqlite3.connect(str(db))
    try:
        rows = con.execute("select name, start, end from kernels order by start").fetchall()
    finally:
        con.close()
    return [(short_name(n), int(s), int(e)) for n, s, e in rows]


def kernel_table(dispatches) -> list[dict]:
    by: dict[str, list[float]] = {}
    for name, start, end in dispatches:
        by.setdefault(name, []).append((end - start) / 1000.0)
    table = [
        {"kernel": k, "count": len(v), "mean_us": statistics.mean(v), "min_us": min(v), "max_us": max(v),
         "total_us": sum(v)}
        for k, v in by.items()
    ]
    return sorted(table, key=lambda r: -r["total_us"])


def epochs(dispatches) -> list[dict]:
    """One record per epoch: copy dispatches since the previous epoch's
    finish (the previous fetch and this feed), steps (k_ctrl_step
    dispatches) and the device time from init to finish."""
    out = []
    copies = 0
    current = None
    for name, start, end in dispatches:
        if name == COPY_KERNEL:
            copies += 1
        elif name == "k_ctrl_init":
            current = {"copies_before": copies, "steps": 0, "start": start}
            copies = 0
        elif name == "k_ctrl_step" and current is not None:
            current["steps"] += 1
        elif name == "k_ctrl_finish" and current is not None:
            current["device_us"] = (end - current.pop("start")) / 1000.0
            out.append(current)
            current = None
    return out


def summarize(db: Path) -> dict:
    d = load_dispatches(db)
    eps = epochs(d)
    # every epoch after the first: the previous epoch's fetch and this feed
    between = [e["copies_before"] for e in eps[1:]]
    return {
        "kernels": kernel_table(d),
        "epochs": len(eps),
        "copy_dispatches_between_epochs": sorted(set(between)),
        "steps_per_epoch": sorted({e["steps"] for e in eps}),
        "epoch_device_us_median": statistics.median([e["device_us"] for e in eps]) if eps else None,
    }


def markdown(s: dict, command: str | None) -> str:
    lines = []
    if command:
        lines += ["Command:", "", "```", command, "```", ""]
    lines += [f"Epochs in the trace: {s['epochs']}; decoder steps per epoch: {s['steps_per_epoch']}; "
              f"median device time per epoch (k_ctrl_init start to k_ctrl_finish end): "
              f"{s['epoch_device_us_median']:.1f} us" if s["epoch_device_us_median"] is not None else "No epochs.",
              "",
              f"Copy dispatches between consecutive epochs: {s['copy_dispatches_between_epochs']} "
              "(the previous epoch's fetch and the next epoch's feed).", "",
              "| kernel | dispatches | mean us | min us | max us | total us |", "|---|---:|---:|---:|---:|---:|"]
    for r in s["kernels"]:
        lines.append(f"| `{r['kernel']}` | {r['count']} | {r['mean_us']:.2f} | {r['min_us']:.2f} | {r['max_us']:.2f} | "
                     f"{r['total_us']:.1f} |")
    return "\n".join(lines) + "\n"


def main() -> int:
    p = argparse.ArgumentParser()
    p.add_argument("db", type=Path)
    p.add_argument("--out", type=Path)
    p.add_argument("--command", help="the command that produced the trace, recorded in the summary")
    args = p.parse_args()
    s = summarize(args.db)
    text = markdown(s, args.command)
    print(text)
    if args.out:
        args.out.with_suffix(".md").write_text(text)
        args.out.with_suffix(".json").write_text(json.dumps(s, indent=1) + "\n")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
