"""Solver contract (reference src/solver.cpp:141-186 and its tests, tests/acceptance.cpp:467-581):
a pure function of (hcs, tree) — bitwise-repeatable, deterministic argmin with a canonical-key
tie-break, predicates that filter candidates with violation records, infeasible termination when
nothing is left, and HCS constants that flow into the cost. The candidate set and the cost model
are CDNA4's (compiled kernel variants, LDS/AGPR/wave-quantisation predicates), so the reference's
RDNA tile picks are not expected here; these tests port the properties.
"""
from __future__ import annotations

import json
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
BASE = json.loads((ROOT / "samples" / "hcs_mi355x.json").read_text())


def hcs(**kw) -> str:
    h = json.loads(json.dumps(BASE))
    for k, v in kw.items():
        if k == "vram":
            h["tiers"][0]["bytes"] = v
        else:
            h[k] = v
    return json.dumps(h)


def configs(uk):
    return [uk.kml_load(p) for p in sorted((ROOT / "samples").glob("kml_*.json"))]


def test_solve_is_bitwise_repeatable(uk):
    for d in configs(uk):
        first = uk.solve(d)
        for _ in range(300):
            s = uk.solve(d)
            assert (s.key, s.predicted_us, s.feasible, s.family) == (first.key, first.predicted_us, first.feasible,
                                                                     first.family)


def test_every_baseline_config_has_a_plan(uk):
    fams = {}
    for d in configs(uk):
        s = uk.solve(d)
        assert s.feasible >= 1 and s.predicted_us > 0
        fams[uk.op_signature(d)] = s.family
    assert fams["gemm:fp16:4096x4096x4096:TN"] == "gemm_f16_mfma"
    assert fams["conv:fp32:56x56x64x3x3x64:NCHW:n8:p1:s1:cs"] == "conv_igemm_mfma"
    conv = uk.make_desc("conv", [56, 56, 64, 3, 3, 64], layout="NCHW", batch=8, pad=1, epilogue="channelscale")
    assert uk.solve(conv).key == "conv_lds16:g7x64,cb16"
    assert fams["rmsnorm:fp32:4096x4096"] == "rows"
    assert all(f == "q8_0_gemm" for k, f in fams.items() if ":q8_0:" in k)


def test_capacity_predicate_terminates_infeasible(uk):
    # R4.4: an empty candidate set ends infeasible with the violation record. Resident-only ops
    # (everything but the MFMA GEMMs) need their whole working set in the device tier.
    d = uk.make_desc("rmsnorm", [4096, 4096])
    with pytest.raises(uk.UnikernError) as e:
        uk.solve(d, hcs(vram=100_000_000))
    msg = str(e.value)
    assert e.value.code == uk.UK_INFEASIBLE
    assert "working_set<=device_capacity" in msg and "need=134234112" in msg and "cap=100000000" in msg
    assert uk.solve(d, hcs(vram=134234112)).feasible >= 1  # exactly fitting is feasible
    # A GEMM streams instead (scenario B) and is infeasible only when B and two one-tile shard
    # pairs exceed 0.85 of the tier: 4096^3 f16 needs 33,554,432 + 2 * 256 * 16,384 B.
    g = uk.make_desc("gemm", [4096, 4096, 4096], dtype="fp16", layout="TN")
    with pytest.raises(uk.UnikernError) as e:
        uk.solve(g, hcs(vram=1 << 20))
    assert e.value.code == uk.UK_INFEASIBLE and "stream_working_set<=0.85*device_capacity" in str(e.value)
    assert "need=41943040" in str(e.value)


def test_streaming_plan_for_a_gemm_beyond_the_device_tier(uk):
    # Scenario B (reference src/solver.cpp:14-44, src/codegen_hip.cpp:1480-1708): a GEMM whose
    # payload exceeds 0.85 of the device tier keeps B resident and streams A and C in M-shards.
    g = uk.make_desc("gemm", [4096, 4096, 4096], dtype="fp16", layout="TN")
    resident = uk.solve(g)
    assert resident.plan.shard_rows == 0 and not resident.key.endswith("+stream")
    cap = 96 << 20
    sol = uk.solve(g, hcs(vram=cap))
    sr = sol.plan.shard_rows
    assert sol.key == resident.key + "+stream" and sol.family == "gemm_f16_mfma"
    assert sr > 0 and sr % sol.plan.tile_m == 0 and sr <= 4096
    b_bytes, row_bytes = 4096 * 4096 * 2, (4096 + 4096) * 2
    assert b_bytes + 2 * sr * row_bytes <= 0.85 * cap < b_bytes + 2 * (sr + sol.plan.tile_m) * row_bytes
    assert "scenario B" in sol.log and sol.predicted_us > resident.predicted_us
    # The link time of every byte (100,663,296 B at link_bw_gbps 64) bounds the prediction.
    assert sol.predicted_us >= 100_663_296 / (64 * 1e3)
    # f32 on the tiled kernel streams in 64-row multiples; payloads under 0.85 stay resident.
    f = uk.make_desc("gemm", [1024, 1024, 1024])
    assert uk.solve(f, hcs(vram=12 << 20)).plan.shard_rows % 64 == 0
    assert uk.solve(f, hcs(vram=16 << 20)).plan.shard_rows == 0
    # Q8_0 and the row family never stream: they are resident-only, as the reference's programs.
    q = uk.make_desc("gemm", [16, 11008, 4096], dtype="q8_0", layout="TN")
    assert uk.solve(q, hcs(vram=56 << 20)).plan.shard_rows == 0


def test_stream_data_paths_are_costed_candidates(uk):
    # Scenario B's two paths for A (reference src/solver.cpp:14-44, :52-66, :96-121; its tests,
    # tests/acceptance.cpp:1040-1090): pinned copies, and A read by the kernel from host-mapped
    # staging paged in from storage. Without an nvme tier the mapped candidate is infeasible by a
    # named predicate; with one it is costed and dominated (its copy term adds the nvme page-in
    # and the link reads of every consuming workgroup column), so pinned is chosen by the cost
    # model, even against an absurdly fast nvme tier.
    g = uk.make_desc("gemm", [4096, 4096, 4096], dtype="fp16", layout="TN")
    h = json.loads(hcs(vram=96 << 20))
    plain = uk.solve(g, json.dumps(h))
    assert plain.plan.stream_path == 1 and plain.key.endswith("+stream")
    assert "violates mmap_stream_requires_nvme_tier_bw>0" in plain.log
    assert "stream_path=mmap" not in plain.log
    h["tiers"].append({"name": "nvme", "bytes": 2 << 40, "bw_gbps": 7, "confidence": "predicted"})
    both = uk.solve(g, json.dumps(h))
    assert both.plan.stream_path == 1 and both.key == plain.key
    assert both.feasible == 2 * plain.feasible  # every kernel candidate with each path
    cands = {ln.split()[1]: float(ln.split("predicted_us=")[1]) for ln in both.log.splitlines()
             if ln.startswith("  candidate ") and "stream_path=" in ln}
    pinned, mapped = cands[plain.key], cands[plain.key + "_mmap"]
    assert mapped > pinned and pinned == pytest.approx(both.predicted_us, rel=1e-5)  # log prints 6 digits
    # A at 7 GB/s once, and over the 64 GB/s link once per 256-column workgroup (16 of them),
    # bound the mapped prediction from below.
    a_bytes = 4096 * 4096 * 2
    assert mapped >= a_bytes / 7e3 + a_bytes * 16 / 64e3
    for t in h["tiers"]:
        if t["name"] == "nvme":
            t["bw_gbps"] = 100000
    assert uk.solve(g, json.dumps(h)).plan.stream_path == 1
    # Resident plans carry no data path.
    assert uk.solve(g).plan.stream_path == 0


def test_lds_predicate_filters_and_records(uk):
    small = hcs(lds_bytes_per_block=16384, lds_bytes_per_cu=16384)
    g = uk.solve(uk.make_desc("gemm", [4096, 4096, 4096], dtype="fp16", layout="TN"), small)
    assert g.family == "gemm_generic_mfma" and "violates LDS" in g.log
    with pytest.raises(uk.UnikernError) as e:
        uk.solve(uk.make_desc("conv", [56, 56, 64, 3, 3, 64], layout="NCHW", batch=8, pad=1,
                              epilogue="channelscale"), small)
    assert e.value.code == uk.UK_INFEASIBLE and "violates LDS per workgroup" in str(e.value)


def test_conv16_index_limit(uk):
    # The 16-pixel conv divides its pixel indices through an f32 reciprocal, exact below 2^21
    # (tests/test_conv_l16_quotient.py): a plane of 40000 x 56 pixels (2.24e6) is refused and the
    # solver falls back to another conv kernel; a plane just under the limit still takes it.
    big = uk.solve(uk.make_desc("conv", [40000, 56, 16, 3, 3, 64], layout="NCHW", batch=1, pad=1))
    assert not big.key.startswith("conv_lds16") and "index quotients below 2^21" in big.log
    ok = uk.solve(uk.make_desc("conv", [36000, 56, 16, 3, 3, 64], layout="NCHW", batch=1, pad=1))
    assert "conv_lds16" in ok.log and "index quotients below 2^21" not in ok.log


def test_divisibility_predicate(uk):
    s = uk.solve(uk.make_desc("gemm", [4096, 4000, 4096], dtype="fp16", layout="TN"))
    assert s.family == "gemm_generic_mfma" and "violates M%bm==0" in s.log
    r = uk.solve(uk.make_desc("softmax", [64, 70001]))
    assert r.family == "rows_stream"


def test_hcs_constants_flow_into_cost(uk):
    # R3.3: an HBM-bound op's predicted time scales with the declared bandwidth
    d = uk.make_desc("reduce", [4096, 4096])
    a = uk.solve(d, hcs(hbm_bw_gbps=8000))
    b = uk.solve(d, hcs(hbm_bw_gbps=4000))
    launch = BASE["launch_overhead_us"]
    assert 1.9 < (b.predicted_us - launch) / (a.predicted_us - launch) < 2.1
    # MFMA-bound work is priced at CUs x SIMDs x FLOP per cycle of the MFMA table x clock_mhz:
    # half the clock, twice the time (the epilogue store and launch are not clock-bound).
    g = uk.make_desc("gemm", [4096, 4096, 4096], dtype="fp16", layout="TN")
    fast = uk.solve(g, hcs(clock_mhz=2400))
    slow = uk.solve(g, hcs(clock_mhz=1200))
    assert slow.predicted_us > 1.8 * (fast.predicted_us - launch)
    c = uk.make_desc("conv", [56, 56, 64, 3, 3, 64], layout="NCHW", batch=8, pad=1, epilogue="channelscale")
    assert uk.solve(c, hcs(clock_mhz=1200)).predicted_us > 1.8 * (uk.solve(c, hcs()).predicted_us - launch)
    # Without an MFMA table (a reference-format description) the declared peak sets the rate.
    fast = uk.solve(g, hcs(mfma=[], peak_f16_mfma_tflops=2516.5824))
    slow = uk.solve(g, hcs(mfma=[], peak_f16_mfma_tflops=1258.2912))
    assert slow.predicted_us > 1.8 * (fast.predicted_us - launch)
    assert fast.predicted_us == uk.solve(g, hcs()).predicted_us  # the table agrees with the peak at 2.4 GHz
    assert uk.solve(d, hcs(constants_version=2)).key == a.key


def test_argmin_is_deterministic_under_candidate_ties(uk):
    # Two HCS that differ only in fields the cost does not read give the same pick, and the
    # pick of a tie group is the smallest canonical key: rows variants with identical predicted
    # cost (bandwidth-capped) resolve by key, not by table order.
    d = uk.make_desc("rmsnorm", [4096, 4096])
    a = uk.solve(d, hcs(device="renamed"))
    b = uk.solve(d)
    assert (a.key, a.predicted_us) == (b.key, b.predicted_us)
    # At C = 256 only the uncalibrated 64-thread variants hold a row, both one row per wavefront
    # in 256-thread workgroups: under a 100 GB/s cap they price identically.
    d = uk.make_desc("rmsnorm", [4096, 256])
    keys = _feasible_rows_keys(d)
    assert keys == ["rows:tpr=64,nv=1", "rows:tpr=64,nv=2"]
    capped = hcs(hbm_bw_gbps=100)
    s = uk.solve(d, capped)
    assert s.key == min(keys)
    assert s.plan.variant == 0


def test_calibrated_rows_picks(uk):
    # The per-op efficiencies measured at 4096 x 4096 decide: the non-temporal 512-thread variant
    # for row-sum, one wavefront per row with grouped stores for RMSNorm and softmax.
    picks = {op: uk.solve(uk.make_desc(op, [4096, 4096])).key for op in ("reduce", "rmsnorm", "softmax")}
    assert picks == {"reduce": "rows:tpr=512,nv=2,nt", "rmsnorm": "rows:tpr=64,nv=16,nt,grp",
                     "softmax": "rows:tpr=64,nv=16,nt,grp"}


def _feasible_rows_keys(d):
    out = []
    for tpr, nv, nt, rpb, grp in [(64, 1, 0, 1, 0), (64, 2, 0, 1, 0), (64, 4, 0, 1, 0), (64, 8, 0, 1, 0),
                                  (64, 16, 0, 1, 0), (128, 4, 0, 1, 0), (128, 8, 0, 1, 0), (256, 1, 0, 1, 0),
                                  (256, 2, 0, 1, 0), (256, 4, 0, 1, 0), (256, 8, 0, 1, 0), (512, 2, 0, 1, 0),
                                  (512, 4, 0, 1, 0), (1024, 1, 0, 1, 0), (1024, 2, 0, 1, 0), (1024, 4, 0, 1, 0),
                                  (256, 4, 1, 1, 0), (512, 2, 1, 1, 0), (1024, 1, 1, 1, 0), (512, 4, 1, 1, 0),
                                  (1024, 2, 1, 1, 0), (128, 8, 1, 1, 0), (256, 4, 1, 2, 0), (512, 2, 1, 2, 0),
                                  (64, 16, 1, 1, 1)]:
        cap = tpr * nv * 4
        C = d.dims[1]
        if C % 4 == 0 and C <= cap and not (cap >= 4 * C and cap > 256) and not (grp and cap >= 2 * C):
            out.append(f"rows:tpr={tpr},nv={nv}" + (",nt" if nt else "") + (f",rpb={rpb}" if rpb > 1 else "")
                       + (",grp" if grp else ""))
    return out


def test_calibrated_gemm_pick(uk):
    # the variant measured fastest at 4096^3 (four wavefronts of 128x128 on 16x16x32 MFMAs,
    # 64-deep k-tiles) is the pick
    s = uk.solve(uk.make_desc("gemm", [4096, 4096, 4096], dtype="fp16", layout="TN"))
    assert s.key == "gemm_f16:256x256x64,w2x2,s2,z1,w4k16"
    assert s.plan.tile_m == 256 and s.plan.tile_k == 64 and s.plan.threads == 256


@pytest.mark.parametrize("op,dims,kw", [("gemm", [4096, 4096, 4096], dict(dtype="fp16", layout="TN")),
                                        ("conv", [56, 56, 64, 3, 3, 64],
                                         dict(layout="NCHW", batch=8, pad=1, epilogue="channelscale")),
                                        ("gemm", [8, 11008, 4096], dict(dtype="q8_0", layout="TN"))])
def test_candidate_log_names_family_and_variant(uk, op, dims, kw):
    # every feasible candidate is listed once, cheapest first, with the family and variant that
    # run it: the first line is the pick itself
    from unikern_amd.sweep import _CAND
    s = uk.solve(uk.make_desc(op, dims, **kw))
    c = _CAND.findall(s.log)
    assert len(c) == s.feasible == len({(f, v) for _, f, v, _ in c})
    assert c[0][0] == s.key and int(c[0][1]) == s.plan.family and int(c[0][2]) == s.plan.variant
    assert [float(x[3]) for x in c] == sorted(float(x[3]) for x in c)
