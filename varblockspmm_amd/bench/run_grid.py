"""Regime sweep over vbsr_benchmark: the counterpart of the reference's
scripts/run_grid.sh (one benchmark run per case, one CSV with the header
written once, run_grid.sh:11-22).

Grids:

  config5    the 128-case regime sweep of the benchmark configurations:
             4096 block rows; distribution {tied8to64 (sizes uniform over
             8..64), low, high, bimodal8or64} x locality {clamped (local
             +-degree), random} x degree {1, 4, 8, 16} x rhs {8, 16, 32, 64},
             nested in that order (the reference's loop order), with
             seed = case index 0..127.
  reference  the reference's publication grid (run_grid.sh:11-14) with the
             reference generator's own distributions and cyclic local
             columns: distribution {uniform, low, high, bimodal} x locality
             {local, random} x degree {2, 4, 8, 16} x rhs {8, 16, 32, 64},
             one seed for every case (--seed), so its rows line up with the
             reference's data/publication/regime_map_seed<seed>.csv.

Usage:
  python varblockspmm_amd/bench/run_grid.py --grid config5 --out regime_map.csv
"""

import argparse
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
EXECUTABLE = os.path.join(HERE, "vbsr_benchmark")
RHS = (8, 16, 32, 64)


def cases(grid, seed=1):
    """The grid's cases in run order, as dicts of vbsr_benchmark arguments."""
    if grid == "config5":
        distributions = ("tied8to64", "low", "high", "bimodal8or64")
        localities = ("clamped", "random")
        degrees = (1, 4, 8, 16)
    elif grid == "reference":
        distributions = ("uniform", "low", "high", "bimodal")
        localities = ("local", "random")
        degrees = (2, 4, 8, 16)
    else:
        raise ValueError(f"unknown grid: {grid}")
    out = []
    for distribution in distributions:
        for locality in localities:
            for degree in degrees:
                for rhs in RHS:
                    case_seed = len(out) if grid == "config5" else seed
                    out.append({"distribution": distribution, "locality": locality, "degree": degree,
                                "rhs": rhs, "seed": case_seed})
    return out


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--grid", choices=["config5", "reference"], default="config5")
    p.add_argument("--out", default="regime_map.csv")
    p.add_argument("--rows", type=int, default=4096)
    p.add_argument("--reps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--seed", type=int, default=1, help="seed of every case of the reference grid")
    p.add_argument("--input", choices=["constant", "random"], default="constant")
    p.add_argument("--no-cold", action="store_true", help="skip the cold-cache repetitions")
    p.add_argument("--limit", type=int, default=0, help="run only the first N cases")
    p.add_argument("--kernel", choices=["auto", "row_owned", "split_row"], default="auto",
                   help="the plan's kernel selection (auto, the default, is the row-owned kernel as in the "
                        "reference; split_row rows are reported under the method name split_row)")
    p.add_argument("--exe", default=EXECUTABLE)
    args = p.parse_args(argv)
    if not os.path.exists(args.exe):
        sys.exit(f"{args.exe} is not built (make -C varblockspmm_amd/bench)")

    todo = cases(args.grid, args.seed)
    if args.limit:
        todo = todo[:args.limit]
    with open(args.out, "w") as out:
        for index, case in enumerate(todo):
            command = [args.exe, "--rows", str(args.rows), "--degree", str(case["degree"]), "--rhs", str(case["rhs"]),
                       "--distribution", case["distribution"], "--locality", case["locality"],
                       "--reps", str(args.reps), "--warmup", str(args.warmup), "--seed", str(case["seed"]),
                       "--input", args.input, "--kernel", args.kernel]
            if args.no_cold:
                command.append("--no-cold")
            if index > 0:
                command.append("--no-header")
            print(f"[run_grid] case {index + 1}/{len(todo)}: {case}", file=sys.stderr, flush=True)
            result = subprocess.run(command, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)
            if result.returncode != 0:
                sys.exit(f"case {index}: {' '.join(command)} failed ({result.returncode}): {result.stderr.strip()}")
            out.write(result.stdout)
            out.flush()
    print(f"Wrote {args.out}", file=sys.stderr)


if __name__ == "__main__":
    main()
