"""The host-side rule that decides whether a layer may run as one of the
launches whose workgroups wait for each other (the XCD-sliced layer and its
stack): every one of its 256 workgroups must be resident at once, one per CU
of a 256-CU device, with the occupancy API reporting at least one block of
the kernel per CU (katali-lab_amd/csrc/kq_plan.h, used by launch_moe_xcd and
launch_moe_stack). Compiled with the host compiler and run here; no device."""
import os
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(REPO, "katali-lab_amd", "csrc")

DRIVER = r"""
#include <stdio.h>
#include "kq_plan.h"
int main() {
    struct { int cus, bpc; unsigned grid; } c[] = {
        {256, 1, 256}, {256, 2, 256}, {256, 0, 256}, {304, 1, 256}, {128, 2, 256}, {0, 4, 256}, {-1, 1, 256},
        {80, 1, 80}, {256, 1, 512}};
    for (unsigned i = 0; i < sizeof c / sizeof c[0]; i++) printf("%d\n", kq::xcd_coresident(c[i].cus, c[i].bpc, c[i].grid) ? 1 : 0);
    return 0;
}
"""


def test_coresident_rule(tmp_path):
    src = tmp_path / "plan.cpp"
    src.write_text(DRIVER)
    exe = tmp_path / "plan"
    r = subprocess.run(["g++", "-std=c++17", "-O1", "-I", CSRC, str(src), "-o", str(exe)], capture_output=True,
                       text=True)
    if r.returncode:
        pytest.fail(r.stderr)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()
    # one per CU on exactly 256 CUs: yes; a kernel that fits no CU, another
    # CU count (the slot-to-XCD mapping needs 256), a grid above the CUs: no
    assert out == ["1", "1", "0", "0", "0", "0", "0", "1", "0"]
