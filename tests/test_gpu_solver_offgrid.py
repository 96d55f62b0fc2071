"""The solver's ranking at shapes its variant efficiencies were not fitted at (the reference's
solver contract, src/solver.cpp:141-186: the argmin over feasible candidates; here checked against
the measured times of the compiled candidates).

For each shape, the solver's pick and the next-best candidates of its own ranking run through
uk_run (same seeded inputs, self-verified, settled kernel-only median). The numbers are printed;
the timing assertion (the pick within 15% of the fastest candidate measured) is a performance
bound, not correctness, so the module carries the perf marker and stays out of -m gpu.
profiles/solver_offgrid.md holds a full sweep of every candidate at these shapes.
"""
import ctypes as C
import re

import pytest

pytestmark = pytest.mark.perf

_CAND = re.compile(r"candidate (\S+) family=(\d+) variant=(\d+) predicted_us=([0-9.eE+-]+)")

SHAPES = [
    ("gemm", [2048, 2048, 2048], dict(dtype="fp16", layout="TN")),
    ("gemm", [1, 14336, 4096], dict(dtype="q8_0", layout="TN")),
    ("gemm", [16, 14336, 4096], dict(dtype="q8_0", layout="TN")),
    ("conv", [28, 28, 128, 3, 3, 128], dict(layout="NCHW", batch=8, pad=1, epilogue="channelscale")),
    ("rmsnorm", [8192, 2048], {}),
    ("softmax", [8192, 2048], {}),
]


@pytest.mark.parametrize("op,dims,kw", SHAPES, ids=[f"{o}-{'x'.join(map(str, d))}" for o, d, _ in SHAPES])
def test_pick_near_fastest_candidate(gpu, op, dims, kw):
    d = gpu.make_desc(op, dims, **kw)
    sol = gpu.solve(d)
    cands = [(m.group(1), int(m.group(2)), int(m.group(3)), float(m.group(4))) for m in _CAND.finditer(sol.log)]
    assert cands and cands[0][0] == sol.key  # the ranking's head is the pick
    times = {}
    for key, family, variant, pred in cands[:4]:
        p = gpu.Plan()
        C.memmove(C.byref(p), C.byref(sol.plan), C.sizeof(p))
        p.family, p.variant = family, variant
        p.key = key.encode()[:63]
        r = gpu.run(d, iters=20, plan=p)
        assert r.exit_code == 0 and r.verified, r.log
        times[key] = r.kernel_ms * 1e3
        print(f"{op} {dims} {key}: predicted {pred:.2f} us, measured {times[key]:.2f} us")
    best = min(times.values())
    assert times[sol.key] <= 1.15 * best, (sol.key, times)
