"""The CDNA4 hardware description (samples/hcs_mi355x.json) against the device it describes, read
through the C ABI (uk_device_props: hipGetDeviceProperties). The reference reads the same facts
from the device at run time (src/codegen_hip.cpp:451-571: multiProcessorCount for the conv plan)
and imports its description from a JSON file (src/hcs.cpp:52-101); here the solver prices with the
description, so what it claims about the part is checked on the part."""
import json
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

HCS = json.loads((Path(__file__).resolve().parent.parent / "samples" / "hcs_mi355x.json").read_text())


def test_description_matches_device(gpu):
    p = gpu.device_props()
    print(p)
    assert p["compute_units"] == HCS["compute_units"] == 256
    assert p["lds_per_block"] == HCS["lds_bytes_per_block"] == 163840
    vram = next(t["bytes"] for t in HCS["tiers"] if t["name"] == "vram")
    # 288 GiB of HBM3E; the runtime reports the whole device memory (never more than the tier)
    assert vram == 288 * 2**30
    assert 0.97 * vram <= p["total_bytes"] <= vram
    # the description's clock is the part's peak engine clock (kHz)
    assert p["clock_khz"] == HCS["clock_mhz"] * 1000
