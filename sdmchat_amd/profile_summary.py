"""Summaries of rocprofv3 output for the profiles/ folder.

    python -m sdmchat_amd.profile_summary counters <dir> [<dir> ...]   # --pmc runs: per kernel, mean per dispatch
    python -m sdmchat_amd.profile_summary stats <dir>                   # --kernel-trace --stats runs
    python -m sdmchat_amd.profile_summary traffic <fetch dir> <write dir> <algorithmic bytes> <kernel prefix> ...

``counters`` reads every ``*counter_collection.csv`` under the given folders (one rocprofv3 --pmc pass each) and
prints, per kernel name, the mean value of each counter per dispatch and the number of dispatches, plus derived
ratios when their counters are present: LDS bank-conflict rate (SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE), the
fraction of wave time spent waiting (SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES), and MFMA busy (SQ_VALU_MFMA_BUSY_CYCLES /
(SQ_BUSY_CU_CYCLES * 4 SIMDs)).  ``stats`` prints the kernel_stats.csv table (calls, average and total duration).
``traffic`` reads a FETCH_SIZE pass and a WRITE_SIZE pass (run with bench.py --copy-probe) and prints, per kernel
whose short name starts with one of the prefixes, the mean KiB per dispatch, calibrated by what the same counters
read for the 256 MiB device copy (262,144 KiB each way), the total HBM bytes per call of those kernels
(``traffic_bytes_per_call``, which bench.py reads) and its ratio to the algorithmic bytes.
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


def _pmc(d, counter):
    per, copy = defaultdict(list), []
    for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
        with open(f) as fh:
            for r in csv.DictReader(fh):
                if r["Counter_Name"] != counter:
                    continue
                name = _short(r["Kernel_Name"], 1000)
                v = float(r["Counter_Value"])
                if name.startswith("__amd_rocclr_copyBuffer") and int(r["Grid_Size"]) == 131072:
                    copy.append(v)
                per[name].append(v)
    return per, copy


def traffic(fetch_dir, write_dir, alg, prefixes):
    F, cf = _pmc(fetch_dir, "FETCH_SIZE")
    W, cw = _pmc(write_dir, "WRITE_SIZE")
    if not cf or not cw:
        sys.exit("no 256 MiB copy in the runs (run bench.py with --copy-probe)")
    ff, fw = 262144.0 / max(cf), 262144.0 / max(cw)
    ks = [k for p in prefixes for k in sorted(F) if k.split("<")[0].split("::")[-1].startswith(p)]
    print("calibration: the 256 MiB device copy (__amd_rocclr_copyBuffer, grid 131072) moves 262144 KiB each way;")
    print(f"  FETCH_SIZE read {max(cf):.1f} KiB -> factor {ff:.4f}")
    print(f"  WRITE_SIZE read {max(cw):.1f} KiB -> factor {fw:.4f}")
    print()
    print(f"{'kernel':60s} {'dispatches':>10s} {'FETCH KiB':>11s} {'WRITE KiB':>11s} {'calibrated MB':>14s}")
    tf = tw = 0.0
    for k in ks:
        f = sum(F[k]) / len(F[k])
        w = sum(W[k]) / len(W[k]) if W.get(k) else 0.0
        tf += f
        tw += w
        print(f"{_short(k):60s} {len(F[k]):10d} {f:11.1f} {w:11.1f} {(f * ff + w * fw) * 1024 / 1e6:14.2f}")
    total = (tf * ff + tw * fw) * 1024
    print()
    print(f"total: FETCH {tf:.1f} KiB x {ff:.4f} + WRITE {tw:.1f} KiB x {fw:.4f}")
    print(f"traffic_bytes_per_call: {total:.0f}")
    print(f"algorithmic_bytes_per_call: {alg}   (ratio {total / alg:.2f})")


if __name__ == "__main__":
    if len(sys.argv) < 3 or sys.argv[1] not in ("counters", "stats", "traffic"):
        sys.exit(__doc__)
    if sys.argv[1] == "counters":
        counters(sys.argv[2:])
    elif sys.argv[1] == "stats":
        stats(sys.argv[2])
    else:
        traffic(sys.argv[2], sys.argv[3], int(sys.argv[4]), sys.argv[5:])
