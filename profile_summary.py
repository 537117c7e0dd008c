"""Summaries of rocprofv3 output (kernel-trace stats and --pmc counters) as
markdown, for the text files kept under profiles/.

  python profile_summary.py stats <rocprof_dir>
  python profile_summary.py pmc <rocprof_dir> [kernel-substring]
  python profile_summary.py loop <rocprof_dir> <after-substring> <kernel-substring> <count>

"loop": mean tracer durations of the first <count> dispatches matching
<kernel-substring> that follow the first dispatch matching <after-substring>,
and of the dispatch right after each (e.g. a split kernel and its merge).
"""
from __future__ import annotations

import collections
import csv
import glob
import re
import sys


def _short(name: str) -> str:
    name = name.replace("(anonymous namespace)::", "")
    name = re.sub(r"\(.*", "", name)
    name = name.replace("void ", "").replace("rth::", "")
    return name[:90]


def stats(root: str) -> str:
    rows = []
    for f in glob.glob(f"{root}/**/*kernel_stats.csv", recursive=True):
        rows += list(csv.DictReader(open(f)))
    lines = ["| kernel | calls | avg us | min us | max us | % time |", "|---|---|---|---|---|---|"]
    for r in sorted(rows, key=lambda r: -float(r["TotalDurationNs"])):
        lines.append(f"| {_short(r['Name'])} | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                     f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | "
                     f"{float(r['Percentage']):.1f} |")
    return "\n".join(lines)


def pmc(root: str, pattern: str = "") -> dict[str, dict[str, float]]:
    """Mean counter value per dispatch, per kernel (names shortened)."""
    acc: dict[str, dict[str, list[float]]] = collections.defaultdict(lambda: collections.defaultdict(list))
    for f in glob.glob(f"{root}/**/*counter_collection.csv", recursive=True):
        for r in csv.DictReader(open(f)):
            if pattern in r["Kernel_Name"]:
                acc[_short(r["Kernel_Name"])][r["Counter_Name"]].append(float(r["Counter_Value"]))
    return {k: {c: sum(v) / len(v) for c, v in cs.items()} for k, cs in acc.items()}


def loop(root: str, after: str, kernel: str, count: int) -> str:
    rows = []
    for f in glob.glob(f"{root}/**/*kernel_trace.csv", recursive=True):
        rows += list(csv.DictReader(open(f)))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    dur = [int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in rows]
    start = min((i for i, r in enumerate(rows) if after in r["Kernel_Name"]), default=-1) + 1
    first, second, names = [], [], None
    i = start
    while len(first) < count and i + 1 < len(rows):
        if kernel in rows[i]["Kernel_Name"]:
            first.append(dur[i])
            second.append(dur[i + 1])
            names = (_short(rows[i]["Kernel_Name"]), _short(rows[i + 1]["Kernel_Name"]))
            i += 2
        else:
            i += 1
    if not first:
        return "no matching dispatches"
    mean = lambda v: sum(v) / len(v) / 1e3
    return (f"| dispatches | {names[0]} avg us | {names[1]} avg us | sum us |\n|---|---|---|---|\n"
            f"| {len(first)} | {mean(first):.2f} | {mean(second):.2f} | "
            f"{mean(first) + mean(second):.2f} |")


def main(argv: list[str]) -> int:
    if len(argv) >= 2 and argv[0] == "stats":
        print(stats(argv[1]))
        return 0
    if len(argv) >= 2 and argv[0] == "pmc":
        res = pmc(argv[1], argv[2] if len(argv) > 2 else "")
        print("| kernel | counter | mean per dispatch |\n|---|---|---|")
        for k, cs in res.items():
            for c, v in sorted(cs.items()):
                print(f"| {k} | {c} | {v:.6g} |")
        return 0
    if len(argv) >= 5 and argv[0] == "loop":
        print(loop(argv[1], argv[2], argv[3], int(argv[4])))
        return 0
    print(__doc__)
    return 2


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
