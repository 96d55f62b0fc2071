"""Run every feasible kernel variant of a family at its BASELINE shape, and summarize counters.

The solver ranks each family's compiled variants by predicted time (the candidate lines of its
SOLVE log, each naming its variant). This module runs them one at a time through uk_run with the
same seeded inputs, self-verification and settled timing as the solver's own pick, and prints
the prediction beside the measurement. Run under rocprofv3, it attributes counters to each
variant's kernel; `--summarize` turns a `--pmc GRBM_GUI_ACTIVE SQ_VALU_MFMA_BUSY_CYCLES
SQ_BUSY_CU_CYCLES` run into a table of matrix-core busy fraction and shader clock per kernel.

    python3 -m unikern_amd.sweep [gemm_f16] [conv] [gemm_f32] [q8_0] [q8_narrow] [q8_longk] [rows] [offgrid] [--iters N]
    python3 -m unikern_amd.sweep --summarize PMC_DIR

Counter arithmetic (gfx950, 8 XCDs of 32 CUs, 4 SIMDs per CU): GRBM_GUI_ACTIVE is summed over
the XCDs, so its eighth is the active window in shader cycles; SQ_VALU_MFMA_BUSY_CYCLES sums the
cycles each SIMD's matrix pipe is busy, so over (window cycles x 1024 SIMDs) it is the matrix
cores' busy fraction (the MfmaUtil metric, per XCD), and SQ_BUSY_CU_CYCLES over (window cycles x
256 CUs) the CUs' busy fraction. Under counter collection the window also spans some
microseconds around each dispatch, so both read low for short kernels; compare variants of one
family at one shape.
"""
from __future__ import annotations

import argparse
import csv
import ctypes as C
import re
import statistics
import sys
from collections import defaultdict
from pathlib import Path

SHAPES = {
    "gemm_f16": [("gemm", [4096, 4096, 4096], dict(dtype="fp16", layout="TN"))],
    "gemm_f32": [("gemm", [1024, 1024, 1024], dict(dtype="fp32", layout="NT"))],
    "conv": [("conv", [56, 56, 64, 3, 3, 64], dict(layout="NCHW", batch=8, pad=1, epilogue="channelscale"))],
    "q8_0": [("gemm", [m, n, 4096], dict(dtype="q8_0", layout="TN")) for n in (4096, 11008) for m in (1, 8, 16)],
    "rows": [(op, [4096, 4096], {}) for op in ("reduce", "rmsnorm", "softmax")],
    # Grids narrower than the chip (an eighth of the LLaMA-7B projections' rows, as one GPU of an
    # 8-way row split holds) and the down projection's long K: the Q8_0 ranking off its grid.
    "q8_narrow": [("gemm", [m, n, k], dict(dtype="q8_0", layout="TN"))
                  for n, k in ((512, 4096), (1376, 4096), (4096, 11008)) for m in (1, 16)],
    # One activation row at K beyond the one-row-per-wavefront kernel's 4096 (the tile kernels'
    # partial last rounds).
    "q8_longk": [("gemm", [1, n, k], dict(dtype="q8_0", layout="TN"))
                 for n, k in ((4096, 4608), (4096, 6144), (4096, 8192), (11008, 8192), (14336, 5120))],
    # Shapes none of the variant efficiencies was fitted at: the solver's ranking off its grid.
    "offgrid": [("gemm", [2048, 2048, 2048], dict(dtype="fp16", layout="TN")),
                ("gemm", [8192, 4096, 4096], dict(dtype="fp16", layout="TN")),
                ("conv", [28, 28, 128, 3, 3, 128], dict(layout="NCHW", batch=8, pad=1, epilogue="channelscale"))]
               + [("gemm", [m, 14336, 4096], dict(dtype="q8_0", layout="TN")) for m in (1, 8, 16)]
               + [(op, [8192, 2048], {}) for op in ("reduce", "rmsnorm", "softmax")],
}
_CAND = re.compile(r"candidate (\S+) family=(\d+) variant=(\d+) predicted_us=([0-9.eE+-]+)")
XCDS, SIMDS = 8, 1024


def sweep(families, iters: int = 50, out=sys.stdout):
    import unikern_amd as uk

    for fam in families:
        for op, dims, kw in SHAPES[fam]:
            d = uk.make_desc(op, dims, **kw)
            sol = uk.solve(d)
            print(f"{fam} {op} {dims}: solver pick {sol.key} (predicted {sol.predicted_us:.2f} us)", file=out, flush=True)
            # One untimed run of the pick first: the first candidate timed after a change of shape
            # read up to 1.8x its time at a 2.2 MB Q8_0 shape (and matched it when re-timed).
            uk.run(d, iters=iters)
            for m in _CAND.finditer(sol.log):
                key, family, variant, pred = m.group(1), int(m.group(2)), int(m.group(3)), float(m.group(4))
                p = uk.Plan()
                C.memmove(C.byref(p), C.byref(sol.plan), C.sizeof(p))
                p.family, p.variant = family, variant
                p.key = key.encode()[:63]
                r = uk.run(d, iters=iters, plan=p)
                status = "PASS" if r.verified else f"FAIL(rc={r.exit_code})"
                print(f"  {key:44s} variant={variant:2d} predicted {pred:8.2f} us  measured {r.kernel_ms * 1e3:8.2f} us  "
                      f"{r.achieved:9.1f} {'TFLOP/s' if r.bound == 'mfma' else 'GB/s'} frac={r.frac:.3f} {status}",
                      file=out, flush=True)


def summarize(pmc_dir: Path) -> str:
    files = list(Path(pmc_dir).rglob("*counter_collection.csv"))
    if not files:
        raise SystemExit(f"no counter_collection.csv under {pmc_dir}")
    disp = defaultdict(dict)  # (kernel, dispatch) -> counters, duration
    for f in files:
        for row in csv.DictReader(open(f)):
            k = (row["Kernel_Name"], row["Dispatch_Id"], f.name)
            disp[k][row["Counter_Name"]] = float(row["Counter_Value"])
            disp[k]["ns"] = float(row["End_Timestamp"]) - float(row["Start_Timestamp"])
    per = defaultdict(list)
    for (name, _, _), c in disp.items():
        if {"GRBM_GUI_ACTIVE", "SQ_VALU_MFMA_BUSY_CYCLES"} <= c.keys() and c["ns"] > 0:
            cyc = c["GRBM_GUI_ACTIVE"] / XCDS
            per[name].append((c["ns"] / 1e3, c["SQ_VALU_MFMA_BUSY_CYCLES"] / (cyc * SIMDS),
                              c.get("SQ_BUSY_CU_CYCLES", 0.0) / (cyc * SIMDS / 4)))
    lines = ["| kernel | dispatches | median us | matrix cores busy | CUs busy |", "|---|---:|---:|---:|---:|"]
    for name, v in sorted(per.items(), key=lambda kv: statistics.median(x[0] for x in kv[1])):
        if statistics.median(x[1] for x in v) <= 0:
            continue
        short = name.split("(")[0].replace("void ", "")
        lines.append(f"| `{short}` | {len(v)} | {statistics.median(x[0] for x in v):.2f} | "
                     f"{statistics.median(x[1] for x in v):.3f} | {statistics.median(x[2] for x in v):.3f} |")
    return "\n".join(lines) + "\n"


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("families", nargs="*", default=[], help=f"any of {', '.join(SHAPES)}")
    ap.add_argument("--iters", type=int, default=50)
    ap.add_argument("--summarize", type=Path, help="rocprofv3 --pmc output directory")
    a = ap.parse_args(argv)
    if a.summarize:
        sys.stdout.write(summarize(a.summarize))
        return 0
    bad = [f for f in a.families if f not in SHAPES]
    if bad or not a.families:
        ap.error(f"families: choose from {', '.join(SHAPES)}")
    sweep(a.families, a.iters)
    return 0


if __name__ == "__main__":
    sys.exit(main())
