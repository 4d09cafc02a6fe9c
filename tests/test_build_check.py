"""The build's scratch guard (katali-lab_amd/build.py): it reads the
compiler's per-kernel resource remarks and refuses a library in which any
kernel uses private (scratch) memory. Pinned here on remark text of the form
hipcc prints, so the guard cannot silently stop matching."""
import build

REMARKS = """\
kq_moe.hip:1687:1: remark: Function Name: _ZN2kq9k_moe_xcdILi8E [-Rpass-analysis=kernel-resource-usage]
kq_moe.hip:1687:1: remark:     VGPRs: 58 [-Rpass-analysis=kernel-resource-usage]
kq_moe.hip:1687:1: remark:     ScratchSize [bytes/lane]: 392 [-Rpass-analysis=kernel-resource-usage]
kq_moe.hip:807:1: remark: Function Name: _ZN2kq8k_moe_guILi8E [-Rpass-analysis=kernel-resource-usage]
kq_moe.hip:807:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
kq_gemv.hip:40:1: remark: Function Name: _ZN2kq6k_gemvE [-Rpass-analysis=kernel-resource-usage]
kq_gemv.hip:40:1: remark:     ScratchSize [bytes/lane]: 40 [-Rpass-analysis=kernel-resource-usage]
"""


def test_scratch_kernels_lists_only_kernels_with_scratch():
    assert build.scratch_kernels(REMARKS) == [("_ZN2kq9k_moe_xcdILi8E", 392), ("_ZN2kq6k_gemvE", 40)]


def test_scratch_kernels_empty_when_none():
    clean = "\n".join(l for l in REMARKS.splitlines() if "ScratchSize" not in l or ": 0 " in l)
    assert build.scratch_kernels(clean) == []
    assert build.scratch_kernels("") == []
