"""The harness's CPU side (katali-lab_amd/host/katali_hip_cpu.c), which
`katali-hip check` / `check-moe` compare the GPU against, checked against the
oracle: f16 conversions on every code, dequantization and q8_1 quantization
bit for bit, the q8_1-path Q4_K dot and SiLU bit for bit. CPU only (the file
is compiled here into a throwaway shared object)."""
import ctypes as C
import os
import shutil
import subprocess

import numpy as np
import pytest

import kq_synth as S
from oracle import Q4_K, Q6_K, Q8_1

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(REPO, "katali-lab_amd", "host", "katali_hip_cpu.c")


@pytest.fixture(scope="module")
def cpu(tmp_path_factory):
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    so = tmp_path_factory.mktemp("harness_cpu") / "libkh_cpu.so"
    out = subprocess.run([cc, "-std=c11", "-O2", "-fPIC", "-shared", "-Wall", "-Wextra", "-Werror", SRC, "-o", str(so),
                          "-lm"], capture_output=True, text=True)
    assert out.returncode == 0, out.stderr
    lib = C.CDLL(str(so))
    lib.kh_cpu_half_to_float.restype = C.c_float
    lib.kh_cpu_half_to_float.argtypes = [C.c_uint16]
    lib.kh_cpu_float_to_half.restype = C.c_uint16
    lib.kh_cpu_float_to_half.argtypes = [C.c_float]
    lib.kh_cpu_dequant.argtypes = [C.c_uint32, C.c_void_p, C.c_uint64, C.c_void_p]
    lib.kh_cpu_quantize_q8_1.argtypes = [C.c_void_p, C.c_uint64, C.c_void_p]
    lib.kh_cpu_dot_q4k_q8.restype = C.c_float
    lib.kh_cpu_dot_q4k_q8.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64]
    lib.kh_cpu_silu_mul.restype = C.c_float
    lib.kh_cpu_silu_mul.argtypes = [C.c_float, C.c_float]
    lib.kh_cpu_matvec.argtypes = [C.c_uint32, C.c_void_p, C.c_uint64, C.c_uint64, C.c_void_p, C.c_void_p]
    return lib


def test_half_conversions(cpu, oracle):
    codes = np.arange(65536, dtype=np.uint16)
    got = np.array([cpu.kh_cpu_half_to_float(int(h)) for h in codes], np.float32)
    want = codes.view(np.float16).astype(np.float32)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all()
    # float -> half: every half value, the midpoints between neighbours (ties
    # to even) and random floats, against numpy's conversion
    rng = np.random.default_rng(1)
    fin = want[np.isfinite(want)]
    mids = ((fin[:-1].astype(np.float64) + fin[1:]) / 2).astype(np.float32)
    vals = np.concatenate([fin, mids, rng.standard_normal(20000).astype(np.float32) * 1000,
                           np.array([65519.0, 65520.0, 1e-8, -1e-8, 6e-8, np.inf, -np.inf], np.float32)])
    got = np.array([cpu.kh_cpu_float_to_half(float(v)) for v in vals], np.uint16)
    with np.errstate(over="ignore"):
        want16 = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want16)


@pytest.mark.parametrize("t,nb", [(Q4_K, 64), (Q6_K, 64)])
def test_dequant_matches_oracle(cpu, oracle, t, nb):
    rng = np.random.default_rng(2 + t)
    w = S.matrix(rng, t, nb, 256)
    got = np.empty(nb * 256, np.float32)
    assert cpu.kh_cpu_dequant(t, w.ctypes.data, nb * 256, got.ctypes.data) == 0
    assert np.array_equal(got.view(np.uint32), oracle.dequant(t, w, nb * 256).view(np.uint32))


def test_q8_1_quantize_and_dequant_match_oracle(cpu, oracle):
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(4096).astype(np.float32), np.zeros(32, np.float32),
                        S.representable_activation(rng, 256)])
    got = np.empty(len(x) // 32 * 36, np.uint8)
    cpu.kh_cpu_quantize_q8_1(x.ctypes.data, len(x), got.ctypes.data)
    want = oracle.quantize_q8_1(x)
    assert np.array_equal(got, want)
    deq = np.empty(len(x), np.float32)
    assert cpu.kh_cpu_dequant(Q8_1, got.ctypes.data, len(x), deq.ctypes.data) == 0
    assert np.array_equal(deq.view(np.uint32), oracle.dequant(Q8_1, want, len(x)).view(np.uint32))


@pytest.mark.parametrize("cols", [256, 768, 2048, 4096])
def test_q4k_q8_dot_and_silu_match_oracle(cpu, oracle, cols):
    rng = np.random.default_rng(4 + cols)
    rows = 32
    w = S.matrix(rng, Q4_K, rows, cols)
    q8 = oracle.quantize_q8_1(S.activation(rng, cols))
    rb = cols // 256 * 144
    got = np.array([cpu.kh_cpu_dot_q4k_q8(w[r * rb:].ctypes.data, q8.ctypes.data, cols // 256) for r in range(rows)],
                   np.float32)
    want = np.array([oracle.dot_q4K_q8(w[r * rb:(r + 1) * rb], q8) for r in range(rows)], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    g = rng.standard_normal(4096).astype(np.float32) * 6
    u = rng.standard_normal(4096).astype(np.float32)
    s = np.array([cpu.kh_cpu_silu_mul(float(a), float(b)) for a, b in zip(g, u)], np.float32)
    assert np.array_equal(s.view(np.uint32), oracle.silu_mul(g, u).view(np.uint32))


def test_matvec_is_the_double_dot_of_dequantized_rows(cpu, oracle):
    rng = np.random.default_rng(5)
    for t, rows, cols in ((Q4_K, 16, 512), (Q6_K, 16, 768)):
        w = S.matrix(rng, t, rows, cols)
        x = S.activation(rng, cols)
        y = np.empty(rows, np.float64)
        assert cpu.kh_cpu_matvec(t, w.ctypes.data, rows, cols, x.ctypes.data, y.ctypes.data) == 0
        want = oracle.dequant(t, w, rows * cols).reshape(rows, cols).astype(np.float64) @ x.astype(np.float64)
        assert np.allclose(y, want, rtol=1e-12, atol=1e-12)
