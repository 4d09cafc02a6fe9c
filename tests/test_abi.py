"""The C-ABI library loads and exports exactly what include/katali_hip.h
declares (CPU only: no compute calls)."""
import ctypes
import os
import re
import subprocess

import pytest

import katali_hip as K

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "katali_hip.h")


def declared(header: str) -> set[str]:
    src = open(header).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return set(re.findall(r"\b(katali_hip_\w+)\s*\(", src))


def test_library_built():
    assert os.path.exists(K.DEFAULT_SO), "run python katali-lab_amd/build.py"


def test_every_declared_symbol_is_exported_and_bound():
    names = declared(HEADER)
    assert len(names) >= 30
    lib = ctypes.CDLL(K.DEFAULT_SO)
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing
    assert names == set(K.SIGNATURES), (names ^ set(K.SIGNATURES))
    out = subprocess.run(["nm", "-D", "--defined-only", K.DEFAULT_SO], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (katali_hip_\w+)", out))
    assert exported == names, exported ^ names


def test_loads_and_reports_status():
    hip = K.KataliHip()
    assert hip.lib.katali_hip_abi_version() == 1
    ok = hip.probe()
    status = hip.status()
    assert status and status != "not probed"
    if not ok:
        # no GPU here: every entry point must refuse cleanly, not crash
        rc = hip.lib.katali_hip_matvec(12, None, 1, 256, None, None)
        assert rc == -2
        assert "no usable device" in hip.lib.katali_hip_last_error().decode()
        p = ctypes.c_void_p()
        assert hip.lib.katali_hip_malloc(ctypes.byref(p), 16) == -2


def test_struct_layouts_match_header():
    # field order and sizes of the descriptors (checked against a C compile)
    src = """
#include <stdio.h>
#include <stddef.h>
#include "katali_hip.h"
int main(void) {
  printf("%zu %zu %zu %zu %zu %zu %zu %zu %zu\\n", sizeof(KataliHipMoe), offsetof(KataliHipMoe, gate_exps),
         offsetof(KataliHipMoe, down_shexp), sizeof(KataliHipMoeRoute),
         offsetof(KataliHipMoeRoute, logits_stride), offsetof(KataliHipMoeRoute, weights_out),
         sizeof(KataliHipMoeBatch), offsetof(KataliHipMoeBatch, ids), offsetof(KataliHipMoeBatch, weights));
  return 0;
}
"""
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "t.c")
        open(c, "w").write(src)
        exe = os.path.join(d, "t")
        subprocess.run(["gcc", "-I" + os.path.join(REPO, "include"), c, "-o", exe], check=True)
        vals = [int(v) for v in subprocess.run([exe], capture_output=True, text=True).stdout.split()]
    M, R, B = K.KataliHipMoe, K.KataliHipMoeRoute, K.KataliHipMoeBatch
    assert vals == [ctypes.sizeof(M), M.gate_exps.offset, M.down_shexp.offset, ctypes.sizeof(R),
                    R.logits_stride.offset, R.weights_out.offset, ctypes.sizeof(B), B.ids.offset,
                    B.weights.offset]


@pytest.mark.parametrize("t,ok", [(12, 1), (14, 1), (0, 1), (2, 0), (13, 0)])
def test_supports_type(t, ok):
    assert K.KataliHip().lib.katali_hip_supports_type(t) == ok


def test_loader_exports_its_headers():
    """libkatali_hip_loader.so (the engine-side loader, dense shim and GGUF
    module) exports every function include/katali_hip_loader.h,
    include/katali_dense_hip.h and include/katali_hip_gguf.h declare."""
    so = os.path.join(REPO, "katali-lab_amd", "libkatali_hip_loader.so")
    assert os.path.exists(so), "run python katali-lab_amd/build.py"
    names = set()
    for h, prefix in (("katali_hip_loader.h", "katali_gpu_"), ("katali_dense_hip.h", "katali_dense_hip_"),
                      ("katali_hip_gguf.h", "katali_hip_(?:gguf|weights|tier|ggml)_")):
        src = re.sub(r"/\*.*?\*/", "", open(os.path.join(REPO, "include", h)).read(), flags=re.S)
        names |= set(re.findall(r"\b(" + prefix + r"\w+)\s*\(", src))
    assert "katali_gpu_moe_batch" in names and "katali_dense_hip_matvec" in names and "katali_hip_tier_layer" in names
    out = subprocess.run(["nm", "-D", "--defined-only", so], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (katali_(?:gpu|dense_hip|hip_gguf|hip_weights|hip_tier|hip_ggml)_\w+)", out))
    assert names <= exported, names - exported
