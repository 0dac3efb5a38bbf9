"""Averages one rocprofv3 --pmc counter per kernel from its CSV output (counter_collection.csv).

    python runeforgeai-project-aesir_amd/pmc_summary.py <run_counter_collection.csv> <COUNTER>

Prints a markdown table: kernel, dispatches, average counter value per dispatch.
"""
import csv
import sys
from collections import defaultdict


def per_kernel(path: str, counter: str) -> dict:
    sums, counts = defaultdict(float), defaultdict(int)
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            if row.get("Counter_Name") != counter:
                continue
            name = row.get("Kernel_Name", "?")
            sums[name] += float(row["Counter_Value"])
            counts[name] += 1
    return {k: (counts[k], sums[k] / counts[k]) for k in sums}


def main():
    path, counter = sys.argv[1], sys.argv[2]
    rows = sorted(per_kernel(path, counter).items(), key=lambda kv: -kv[1][1] * kv[1][0])
    print(f"| kernel | dispatches | avg {counter} per dispatch |")
    print("|---|---:|---:|")
    for name, (n, avg) in rows:
        short = name if len(name) < 100 else name[:97] + "..."
        print(f"| `{short}` | {n} | {avg:.1f} |")


if __name__ == "__main__":
    main()
