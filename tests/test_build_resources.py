"""The build's kernel resource guard (longctx100m_amd/build.py): the compiler's
resource remarks are parsed per kernel, and a hot kernel over its scratch
limit fails the build."""

import pytest

from longctx100m_amd import build

SAMPLE = """\
x.hip:73:1: remark: Function Name: _ZN2lc12_GLOBAL__N_112dq128_kernelENS0_10Bwd128ArgsE [-Rpass-analysis=kernel-resource-usage]
x.hip:73:1: remark:     VGPRs: 238 [-Rpass-analysis=kernel-resource-usage]
x.hip:73:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:73:1: remark:     Occupancy [waves/SIMD]: 2 [-Rpass-analysis=kernel-resource-usage]
x.hip:274:1: remark: Function Name: _ZN2lc12_GLOBAL__N_114dkdv128_kernelENS0_10Bwd128ArgsE [-Rpass-analysis=kernel-resource-usage]
x.hip:274:1: remark:     VGPRs: 256 [-Rpass-analysis=kernel-resource-usage]
x.hip:274:1: remark:     ScratchSize [bytes/lane]: 28 [-Rpass-analysis=kernel-resource-usage]
x.hip:1:1: warning: something unrelated
"""


def test_parse_resource_remarks():
    u = build._resource_usage(SAMPLE)
    dq = u["_ZN2lc12_GLOBAL__N_112dq128_kernelENS0_10Bwd128ArgsE"]
    assert dq == {"VGPRs": "238", "ScratchSize": "0", "Occupancy": "2"}
    assert u["_ZN2lc12_GLOBAL__N_114dkdv128_kernelENS0_10Bwd128ArgsE"]["ScratchSize"] == "28"


def test_scratch_limit_enforced(tmp_path, monkeypatch):
    monkeypatch.setattr(build, "BUILD", tmp_path)
    usage = {f"k_{name}": {"ScratchSize": "0"} for name in build.SCRATCH_LIMITS}
    build._check_resources(usage)  # within limits
    assert (tmp_path / "resource_usage.txt").exists()
    usage["k_fwd128_kernel"]["ScratchSize"] = "16"
    with pytest.raises(RuntimeError, match="scratch"):
        build._check_resources(usage)
    del usage["k_fwd128_kernel"]
    with pytest.raises(RuntimeError, match="no kernel matching"):
        build._check_resources(usage)
