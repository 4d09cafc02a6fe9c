"""The engine-side binding compiles against the engine's own headers.

INTEGRATION.md gives the maintainer a forwarding katali_dense_cuda.c (the
engine's katali_dense_cuda_* entry points over katali_dense_hip.c). This test
takes that code block verbatim, compiles it against the reference's
include/katali_dense_cuda.h and include/katali_gguf.h (read from the reference
tree in the build container; skipped where it is absent) with the shim and
the loader, and drives the fallback contract the engine relies on
(vendor/katali_gguf_dense/src/katali_dense_cuda.c:14-22; gguf_model.c:500-504,
533-541): without the opt-in, with the library missing, and with the library
present but no usable device, every call returns -1 so the engine computes on
the CPU. CPU only.
"""
import os
import re
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_INC = "/root/reference/vendor/katali_gguf_dense/include"
HOST = os.path.join(REPO, "katali-lab_amd", "host")
LIB = os.path.join(REPO, "katali-lab_amd", "libkatali_hip.so")

DRIVER = r'''
#include "katali_dense_cuda.h"
#include <stdio.h>
#include <string.h>

int main(void) {
    static unsigned char w[2 * 144];
    float x[256], y0[2], y1[2];
    memset(x, 0, sizeof x);
    KataliGgufTensor t;
    memset(&t, 0, sizeof t);
    t.n_dims = 2;
    t.dims[0] = 256;            /* cols */
    t.dims[1] = 2;              /* rows */
    t.type = 12;                /* Q4_K */
    t.data = w;
    t.nbytes = sizeof w;
    t.n_elements = 512;
    const KataliGgufTensor *ts[2] = {&t, &t};
    float *ys[2] = {y0, y1};
    const int en = katali_dense_cuda_enabled();
    const int one = katali_dense_cuda_matvec(&t, x, y0);
    const int multi = katali_dense_cuda_matvec_multi(ts, ys, 2, x);
    const int null_t = katali_dense_cuda_matvec(NULL, x, y0);
    katali_dense_cuda_shutdown();
    printf("%d %d %d %d\n", en, one, multi, null_t);
    return 0;
}
'''


def forwarding_source() -> str:
    text = open(os.path.join(REPO, "INTEGRATION.md")).read()
    blocks = re.findall(r"```c\n(.*?)```", text, flags=re.S)
    fwd = [b for b in blocks if "katali_dense_cuda_matvec_multi" in b and "katali_dense_hip" in b]
    assert len(fwd) == 1, "INTEGRATION.md must hold exactly one forwarding katali_dense_cuda.c block"
    return fwd[0]


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    if not os.path.exists(os.path.join(REF_INC, "katali_dense_cuda.h")):
        pytest.skip("the engine's headers are not present here")
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    d = tmp_path_factory.mktemp("engine_binding")
    (d / "katali_dense_cuda.c").write_text(forwarding_source())
    (d / "main.c").write_text(DRIVER)
    exe = d / "drv"
    cmd = [cc, "-std=c11", "-O1", "-Wall", "-Werror=implicit-function-declaration",
           "-Werror=incompatible-pointer-types", "-Werror=int-conversion", "-Werror=return-type",
           "-I", REF_INC, "-I", os.path.join(REPO, "include"),
           str(d / "katali_dense_cuda.c"), str(d / "main.c"),
           os.path.join(HOST, "katali_dense_hip.c"), os.path.join(HOST, "katali_hip_loader.c"),
           "-o", str(exe), "-ldl"]
    out = subprocess.run(cmd, capture_output=True, text=True)
    assert out.returncode == 0, out.stderr
    fwd_warnings = [ln for ln in out.stderr.splitlines() if "katali_dense_cuda.c" in ln and "warning" in ln]
    assert not fwd_warnings, fwd_warnings
    return str(exe)


def run(exe, env_extra):
    env = {k: v for k, v in os.environ.items() if k not in ("KATALI_HIP", "KATALI_CUDA", "KATALI_HIP_DLL")}
    env.update(env_extra)
    out = subprocess.run([exe], env=env, capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    return [int(v) for v in out.stdout.split()], out.stderr


def test_no_opt_in_keeps_the_cpu_path(driver):
    vals, err = run(driver, {})
    assert vals == [0, -1, -1, -1]
    assert "phase: dense hip OFF" in err


def test_missing_library_keeps_the_cpu_path(driver):
    vals, err = run(driver, {"KATALI_CUDA": "1", "KATALI_HIP_DLL": "/nonexistent/libkatali_hip.so"})
    assert vals == [0, -1, -1, -1]
    assert "OFF" in err and "/nonexistent/libkatali_hip.so" in err


def test_library_without_device_keeps_the_cpu_path(driver):
    if not os.path.exists(LIB):
        pytest.skip("libkatali_hip.so not built")
    vals, err = run(driver, {"KATALI_HIP": "1", "KATALI_HIP_DLL": LIB})
    if vals[0] == 1:
        pytest.skip("a usable device is present: the fallback is not reachable here")
    assert vals == [0, -1, -1, -1]
    assert "OFF" in err
