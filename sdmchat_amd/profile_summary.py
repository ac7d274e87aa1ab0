"""Summaries of rocprofv3 output for the profiles/ folder.

    python -m sdmchat_amd.profile_summary counters <dir> [<dir> ...]   # --pmc runs: per kernel, mean per dispatch
    python -m sdmchat_amd.profile_summary stats <dir>                   # --kernel-trace --stats runs

``counters`` reads every ``*counter_collection.csv`` under the given folders (one rocprofv3 --pmc pass each) and
prints, per kernel name, the mean value of each counter per dispatch and the number of dispatches, plus derived
ratios when their counters are present: LDS bank-conflict rate (SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE), the
fraction of wave time spent waiting (SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES), and MFMA busy (SQ_VALU_MFMA_BUSY_CYCLES /
(SQ_BUSY_CU_CYCLES * 4 SIMDs)).  ``stats`` prints the kernel_stats.csv table (calls, average and total duration).
"""
import csv
import glob
import os
import sys
from collections import defaultdict


def _short(name, width=60):
    name = name.replace("(anonymous namespace)::", "").replace("void ", "", 1)
    depth, cut = 0, len(name)
    for i, ch in enumerate(name):   # drop the argument list: the first '(' outside template brackets
        depth += ch == "<"
        depth -= ch == ">"
        if ch == "(" and depth == 0:
            cut = i
            break
    name = name[:cut]
    return name if len(name) <= width else name[:width - 3] + "..."


def counters(dirs):
    vals = defaultdict(lambda: defaultdict(list))
    for d in dirs:
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            with open(f) as fh:
                for r in csv.DictReader(fh):
                    vals[r["Kernel_Name"]][r["Counter_Name"]].append(float(r["Counter_Value"]))
    for k in sorted(vals):
        c = vals[k]
        n = max(len(v) for v in c.values())
        print(f"{_short(k)}  ({n} dispatches)")
        mean = {name: sum(v) / len(v) for name, v in c.items()}
        for name in sorted(mean):
            print(f"    {name:32s} {mean[name]:16.1f}")
        if mean.get("SQ_LDS_IDX_ACTIVE"):
            if "SQ_LDS_BANK_CONFLICT" in mean:
                print(f"    {'lds bank-conflict rate':32s} {mean['SQ_LDS_BANK_CONFLICT'] / mean['SQ_LDS_IDX_ACTIVE']:16.3f}")
        if mean.get("SQ_WAVE_CYCLES") and "SQ_WAIT_INST_ANY" in mean:
            print(f"    {'wave time waiting (fraction)':32s} {mean['SQ_WAIT_INST_ANY'] / mean['SQ_WAVE_CYCLES']:16.3f}")
        if mean.get("SQ_BUSY_CU_CYCLES") and "SQ_VALU_MFMA_BUSY_CYCLES" in mean:
            print(f"    {'mfma busy (fraction of SIMD time)':32s} "
                  f"{mean['SQ_VALU_MFMA_BUSY_CYCLES'] / (4 * mean['SQ_BUSY_CU_CYCLES']):16.3f}")


def stats(d):
    for f in glob.glob(os.path.join(d, "**", "*kernel_stats.csv"), recursive=True):
        with open(f) as fh:
            rows = list(csv.DictReader(fh))
        print(f"{'kernel':62s} {'calls':>6s} {'avg us':>10s} {'total us':>12s} {'%':>6s}")
        for r in rows:
            print(f"{_short(r['Name']):62s} {int(r['Calls']):6d} {float(r['AverageNs']) / 1e3:10.2f} "
                  f"{float(r['TotalDurationNs']) / 1e3:12.1f} {float(r['Percentage']):6.2f}")


if __name__ == "__main__":
    if len(sys.argv) < 3 or sys.argv[1] not in ("counters", "stats"):
        sys.exit(__doc__)
    counters(sys.argv[2:]) if sys.argv[1] == "counters" else stats(sys.argv[2])
