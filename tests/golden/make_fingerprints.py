"""Extract per-instance generator fingerprints from the reference's CSVs.

Run in a container where the reference repository is mounted (it reads only
data files, never code):

    python tests/golden/make_fingerprints.py /root/reference > tests/golden/fingerprints.json

The reference benchmark prints, per run, ``useful_gflops`` = flops /
(gpu_median_ms * 1e6) with flops = 2 * rhs * S and S = sum over blocks of h*w
(bench/benchmark.cpp:197-207, 215-225), and prints ``gpu_median_ms`` rounded to
5 decimals.  Each CSV row therefore bounds S to an interval:

    S_row = useful_gflops * gpu_median_ms * 1e6 / (2 * rhs)
    |S - S_row| <= S_row * (0.5e-5 / gpu_median_ms + 0.5e-5 / useful_gflops)

``generate`` ignores rhs (src/format/generator.cpp:7-88), so all methods and
RHS widths of one (rows, degree, distribution, locality, seed) instance bound
the same S.  The fixture keeps the intersection of those intervals.
"""

import csv
import glob
import json
import os
import sys


def rows_of(path):
    with open(path, newline="") as handle:
        yield from csv.DictReader(handle)


def main(reference_root):
    files = sorted(glob.glob(os.path.join(reference_root, "data", "publication", "regime_map_seed*.csv")))
    files += sorted(glob.glob(os.path.join(reference_root, "data", "regime_map*.csv")))
    bounds = {}
    for path in files:
        for row in rows_of(path):
            key = (int(row["block_rows"]), int(row["degree"]), row["distribution"], row["locality"],
                   int(row["seed"]))
            rhs = int(row["rhs"])
            median_ms = float(row["gpu_median_ms"])
            gflops = float(row["useful_gflops"])
            estimate = gflops * median_ms * 1e6 / (2.0 * rhs)
            slack = estimate * (0.5e-5 / median_ms + 0.5e-5 / gflops)
            low, high = estimate - slack, estimate + slack
            old = bounds.get(key)
            if old is None:
                bounds[key] = [low, high, 1, [os.path.relpath(path, reference_root)]]
            else:
                old[0] = max(old[0], low)
                old[1] = min(old[1], high)
                old[2] += 1
                rel = os.path.relpath(path, reference_root)
                if rel not in old[3]:
                    old[3].append(rel)
    instances = []
    for (block_rows, degree, distribution, locality, seed), (low, high, count, sources) in sorted(bounds.items()):
        if low > high:
            raise SystemExit(f"inconsistent rows for {block_rows},{degree},{distribution},{locality},{seed}")
        instances.append({
            "block_rows": block_rows, "block_cols": block_rows, "degree": degree,
            "distribution": distribution, "locality": locality, "seed": seed,
            "sum_hw_low": low, "sum_hw_high": high, "csv_rows": count, "sources": sources,
        })
    json.dump({
        "description": "Bounds on S = sum(h*w) per generated instance, implied by the reference's "
                       "published benchmark CSVs (see make_fingerprints.py).",
        "instances": instances,
    }, sys.stdout, indent=1)
    sys.stdout.write("\n")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
