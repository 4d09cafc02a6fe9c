"""Build recipe for libkatali_hip.so (gfx950) and the C host side.

    python katali-lab_amd/build.py          # builds everything in-tree

Outputs (all next to this file, git-ignored, shipped with the tree):
    libkatali_hip.so        the HIP backend (C ABI: include/katali_hip.h)
    libkatali_hip_loader.so the engine-side loader (dlopen, CPU fallback)
    katali-hip              the CLI harness (hip-check, hip-bench, ...)

    python katali-lab_amd/build.py --stamps   # the measurement build only
    libkatali_hip_stamps.so the same library with the one-launch layers'
                            phase stamps (KQ_STAMPS), for profile_bench.py --phases
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import re
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
HOST = os.path.join(PKG, "host")
BUILD = os.path.join(PKG, "_build")
INCLUDE = os.path.join(REPO, "include")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CC = os.environ.get("CC", "gcc")

# -ffp-contract=off: the only fused multiply-adds are explicit fmaf() calls, so
#   the q8_1 quantizer and SiLU round exactly like the CPU oracle.
# -packed-fp32-ops: never emit v_pk_{add,mul,fma}_f32.
# -amdgpu-mfma-vgpr-form: MFMA results land in VGPRs (the AGPR form costs a
#   v_accvgpr_read per result element before the fp32 scale arithmetic).
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-Wall", "-Wno-unused-function", "-I" + INCLUDE,
]
HIP_SOURCES = ["kq_moe.hip", "kq_gemv.hip", "kq_moe_batch.hip", "kq_sample.hip", "kq_norm.hip", "kq_gemv_f32.hip",
               "kq_floor.hip", "katali_hip.cpp"]
C_FLAGS = ["-std=c11", "-O2", "-fPIC", "-Wall", "-Wextra", "-I" + INCLUDE, "-D_POSIX_C_SOURCE=200809L"]


def _run(cmd: list[str]) -> str:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + r.stdout + r.stderr)
        raise RuntimeError(f"build step failed: {cmd[0]} ... {cmd[-1]}")
    if r.stderr.strip():
        # keep real warnings visible, drop the host-pass note about the
        # device-only target feature, the resource remarks (read below) and
        # the source lines they quote
        lines = [l for l in r.stderr.splitlines()
                 if "packed-fp32-ops" not in l and "kernel-resource-usage" not in l and l.strip()
                 and not re.match(r"\s*\d*\s*\|", l)]
        if lines:
            sys.stderr.write("\n".join(lines) + "\n")
    return r.stderr


def scratch_kernels(remarks: str) -> list[tuple[str, int]]:
    """(kernel, bytes per lane) for every kernel whose resource remark shows
    private (scratch) memory: a stack frame or spills, which turn every wave's
    launch into a scratch allocation and cost the MoE layer several times
    its time (a pointer conditional once copied the argument block there)."""
    out, name = [], None
    for line in remarks.splitlines():
        if "Function Name:" in line:
            name = line.split("Function Name:", 1)[1].split("[")[0].strip()
        elif "ScratchSize [bytes/lane]:" in line and name:
            n = int(line.split("ScratchSize [bytes/lane]:", 1)[1].split("[")[0])
            if n:
                out.append((name, n))
    return out


def _hip_object(src: str, build: str = BUILD, defines: tuple[str, ...] = ()) -> str:
    obj = os.path.join(build, os.path.basename(src) + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else ["-x", "hip"]
    remarks = _run([HIPCC, *HIP_FLAGS, *[f"-D{d}" for d in defines], "-Rpass-analysis=kernel-resource-usage",
                    *lang, "-c", os.path.join(CSRC, src), "-o", obj])
    bad = scratch_kernels(remarks)
    if bad:
        raise RuntimeError(f"{src}: kernels with scratch memory (bytes per lane): " +
                           ", ".join(f"{n} ({b})" for n, b in bad[:8]))
    return obj


def build_hip(jobs: int = 3, stamps: bool = False) -> str:
    """The library; stamps: the measurement build (KQ_STAMPS: the one-launch
    layers record phase stamps), libkatali_hip_stamps.so, off by default."""
    build = BUILD + ("_stamps" if stamps else "")
    defines = ("KQ_STAMPS",) if stamps else ()
    os.makedirs(build, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda src: _hip_object(src, build, defines), HIP_SOURCES))
    out = os.path.join(PKG, "libkatali_hip_stamps.so" if stamps else "libkatali_hip.so")
    tmp = out + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, out)
    return out


def build_host() -> list[str]:
    outs = []
    if not os.path.isdir(HOST):
        return outs
    loader = os.path.join(HOST, "katali_hip_loader.c")
    dense = os.path.join(HOST, "katali_dense_hip.c")
    gguf = os.path.join(HOST, "katali_hip_gguf.c")
    cli = os.path.join(HOST, "katali_hip_cli.c")
    if os.path.exists(loader):
        so = os.path.join(PKG, "libkatali_hip_loader.so")
        srcs = [loader] + [p for p in (dense, gguf) if os.path.exists(p)]
        _run([CC, *C_FLAGS, "-shared", *srcs, "-o", so, "-ldl"])
        outs.append(so)
        if os.path.exists(cli):
            exe = os.path.join(PKG, "katali-hip")
            # the harness's CPU side (GPU-versus-CPU checks) links into the CLI only
            _run([CC, *C_FLAGS, cli, os.path.join(HOST, "katali_hip_cpu.c"), *srcs, "-o", exe, "-ldl", "-lm"])
            outs.append(exe)
    return outs


def build_all(verbose: bool = True) -> list[str]:
    if shutil.which(HIPCC) is None and not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    outs = [build_hip()] + build_host()
    if verbose:
        for o in outs:
            print("built", os.path.relpath(o, REPO))
    return outs


if __name__ == "__main__":
    if "--stamps" in sys.argv[1:]:
        print("built", os.path.relpath(build_hip(stamps=True), REPO))
    else:
        build_all()
