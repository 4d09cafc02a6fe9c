"""Engine-side loader and dense shim (katali_dense_hip.c), in fresh processes.

The CPU cases pin the fallback contract of the engine's CUDA shim
(vendor/katali_gguf_dense/src/katali_dense_cuda.c:14-22,46-56): no opt-in,
a missing library or no usable device all give -1 so the engine computes on
the CPU. The GPU case checks the shim's GEMV against the oracle and its
per-host-pointer weight cache."""
import os
import subprocess
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LOADER = os.path.join(REPO, "katali-lab_amd", "libkatali_hip_loader.so")

PROBE = r'''
import ctypes as C, sys
lib = C.CDLL(sys.argv[1])
lib.katali_gpu_status.restype = C.c_char_p
lib.katali_dense_hip_matvec.argtypes = [C.c_uint32, C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64, C.c_void_p, C.c_void_p]
w = (C.c_uint8 * 144)(); x = (C.c_float * 256)(); y = (C.c_float * 1)()
rc = lib.katali_dense_hip_matvec(12, C.addressof(w), 144, 1, 256, C.addressof(x), C.addressof(y))
print(lib.katali_dense_hip_enabled(), rc, lib.katali_gpu_status().decode())
'''


def run_probe(env_extra, drop=("KATALI_HIP", "KATALI_CUDA", "KATALI_HIP_DLL")):
    env = {k: v for k, v in os.environ.items() if k not in drop}
    env.update(env_extra)
    out = subprocess.run([sys.executable, "-c", PROBE, LOADER], env=env, capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    en, rc, status = out.stdout.strip().split(" ", 2)
    return int(en), int(rc), status, out.stderr


def have_loader():
    return os.path.exists(LOADER)


@pytest.mark.skipif(not have_loader(), reason="host library not built")
def test_shim_off_without_opt_in():
    en, rc, status, err = run_probe({})
    assert en == 0 and rc == -1
    assert "phase: dense hip OFF" in err


@pytest.mark.skipif(not have_loader(), reason="host library not built")
def test_shim_missing_library_falls_back():
    en, rc, status, err = run_probe({"KATALI_HIP": "1", "KATALI_HIP_DLL": "/nonexistent/libkatali_hip.so"})
    assert en == 0 and rc == -1
    assert "not loaded" in status and "/nonexistent/libkatali_hip.so" in status


@pytest.mark.skipif(not have_loader(), reason="host library not built")
def test_shim_accepts_engine_switch():
    """KATALI_CUDA=1 (the engine's existing switch) opts in as well."""
    en, rc, status, err = run_probe({"KATALI_CUDA": "y", "KATALI_HIP_DLL": "/nonexistent/libkatali_hip.so"})
    assert "/nonexistent/libkatali_hip.so" in status   # it tried to load, so the switch was honoured
    assert rc == -1


@pytest.mark.gpu
def test_shim_matvec_on_gpu(oracle):
    import ctypes as C
    import kq_synth as S
    from oracle import Q4_K, Q6_K
    os.environ["KATALI_HIP"] = "1"
    lib = C.CDLL(LOADER)
    lib.katali_dense_hip_matvec.argtypes = [C.c_uint32, C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64, C.c_void_p,
                                            C.c_void_p]
    lib.katali_dense_hip_matvec_multi.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                                  C.c_uint64, C.c_void_p, C.c_void_p]
    assert lib.katali_dense_hip_enabled() == 1
    rng = np.random.default_rng(3)
    cols = 2048
    mats = [(Q4_K, 512), (Q4_K, 128), (Q6_K, 256)]
    ws = [S.matrix(rng, t, r, cols) for t, r in mats]
    x = S.activation(rng, cols)
    n0 = lib.katali_dense_hip_cached()
    singles = []
    for (t, r), w in zip(mats, ws):
        y = np.empty(r, np.float32)
        singles.append(y)
        for _ in range(2):   # second call reuses the cached device copy
            assert lib.katali_dense_hip_matvec(t, w.ctypes.data, w.nbytes, r, cols, x.ctypes.data, y.ctypes.data) == 0
        want = oracle.matvec_f32x(t, w, r, cols, x, 1)
        assert np.all(np.abs(y - want) <= 1e-4 + 1e-3 * np.abs(want))
    assert lib.katali_dense_hip_cached() == n0 + len(mats)
    ys = [np.empty(r, np.float32) for _, r in mats]
    types = (C.c_uint32 * 3)(*[t for t, _ in mats])
    ptrs = (C.c_void_p * 3)(*[w.ctypes.data for w in ws])
    sizes = (C.c_uint64 * 3)(*[w.nbytes for w in ws])
    rows = (C.c_uint64 * 3)(*[r for _, r in mats])
    outs = (C.c_void_p * 3)(*[y.ctypes.data for y in ys])
    assert lib.katali_dense_hip_matvec_multi(3, types, ptrs, sizes, rows, cols, x.ctypes.data, outs) == 0
    for (t, r), w, y, y1 in zip(mats, ws, ys, singles):
        want = oracle.matvec_f32x(t, w, r, cols, x, 1)
        assert np.all(np.abs(y - want) <= 1e-4 + 1e-3 * np.abs(want))
        assert np.array_equal(y.view(np.uint32), y1.view(np.uint32))   # one launch, same bits
    assert lib.katali_dense_hip_cached() == n0 + len(mats)
    lib.katali_dense_hip_shutdown()
    assert lib.katali_dense_hip_cached() == 0


def test_moe_structs_keep_their_buffers_alive():
    """The MoE descriptor and route hold raw device pointers; the structs
    must keep the buffers behind them alive, or a temporary buffer passed
    straight into moe_desc / moe_route is freed before the layer runs."""
    import gc
    import weakref
    from katali_hip import KataliHip

    class Buf:   # stands in for DeviceBuffer (no device needed)
        def __init__(self, ptr):
            self.ptr = ptr

    refs = []

    def buf(p):
        b = Buf(p)
        refs.append(weakref.ref(b))
        return b

    d = KataliHip.moe_desc(256, 256, 4, buf(0x1000), buf(0x2000), buf(0x3000), shared=(buf(1), buf(2), buf(3)))
    r = KataliHip.moe_route(2, logits=buf(0x4000), ids_out=buf(0x5000))
    gc.collect()
    assert all(ref() is not None for ref in refs)
    assert d.gate_exps == 0x1000 and d.down_shexp == 3 and r.logits == 0x4000
    del d, r
    gc.collect()
    assert all(ref() is None for ref in refs)
