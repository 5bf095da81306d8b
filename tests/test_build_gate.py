"""The build's resource gate (r4dx_amd/build.py, after the reference's third_party/check_trellis_isa.cmake:1-40):
hipcc's kernel-resource-usage remarks are parsed per kernel, and any scratch use, spill or occupancy below a kernel
family's floor fails the build. Checked on a synthetic report, and on the report of the library as built here."""
import json
import os

import pytest

from r4dx_amd import build as B

REPORT = """x.hip:1:1: remark: Function Name: _Z14tq_gemv_kernelILi4ELi1ELi1ELi4ELb1ELi0ELb0EEvv [-Rpass-analysis=kernel-resource-usage]
x.hip:1:1: remark:     VGPRs: 76 [-Rpass-analysis=kernel-resource-usage]
x.hip:1:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:1:1: remark:     Occupancy [waves/SIMD]: 5 [-Rpass-analysis=kernel-resource-usage]
x.hip:1:1: remark:     SGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:1:1: remark:     VGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:2:1: remark: Function Name: _Z14tq_m256_kernelILi4ELi8ELb0EEvv [-Rpass-analysis=kernel-resource-usage]
x.hip:2:1: remark:     VGPRs: 254 [-Rpass-analysis=kernel-resource-usage]
x.hip:2:1: remark:     ScratchSize [bytes/lane]: 336 [-Rpass-analysis=kernel-resource-usage]
x.hip:2:1: remark:     Occupancy [waves/SIMD]: 2 [-Rpass-analysis=kernel-resource-usage]
x.hip:2:1: remark:     SGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:2:1: remark:     VGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]
"""


def test_gate_parses_and_flags():
    recs = B.parse_resources(REPORT)
    assert [r["name"] for r in recs] == ["tq_gemv_kernel<4, 1, 1, 4, true, 0, false>()", "tq_m256_kernel<4, 8, false>()"]
    assert recs[0]["VGPRs"] == 76 and recs[1]["ScratchSize"] == 336
    bad = B.gate(recs)
    assert len(bad) == 1 and "tq_m256_kernel" in bad[0] and "scratch 336" in bad[0]
    recs[0]["Occupancy"] = 4            # the decode GEMV's floor is 5
    assert any("occupancy 4" in b for b in B.gate(recs))


def test_built_library_passes_the_gate():
    path = os.path.join(B.PKG, "_build", "resources.json")
    if not os.path.exists(path):
        pytest.skip("no build report here (python -m r4dx_amd.build writes it)")
    recs = json.load(open(path))
    assert len(recs) > 100 and B.gate(recs) == []
