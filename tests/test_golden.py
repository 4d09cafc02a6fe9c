"""The oracle against the reference's recorded outputs (tests/golden/, written by
tests/golden/make_golden.py from the reference compiled from its own sources).
Bit-exact for the fp32 paths the oracle restates; runs without the reference."""
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden as MG  # noqa: E402

from oracle import Q4_K  # noqa: E402

FIX = np.load(os.path.join(HERE, "golden", "ref_cpu_vectors.npz"))


@pytest.mark.parametrize("case", MG.MATVEC_CASES, ids=[c[0] for c in MG.MATVEC_CASES])
def test_matvec_fixtures(oracle, case):
    name, t, rows, cols, seed, fixed = case
    w, x = MG.case_inputs(t, rows, cols, seed, fixed)
    assert MG.sha(w, x) == str(FIX[f"{name}/input_sha256"]), "input generator changed"
    fast = oracle.matvec_f32x(t, w, rows, cols, x)
    assert np.array_equal(fast.view(np.uint32), FIX[f"{name}/matvec"])
    # row-parallel form (the CPU-baseline port) is bit-identical too
    assert np.array_equal(oracle.matvec_f32x(t, w, rows, cols, x, threads=3).view(np.uint32), FIX[f"{name}/matvec"])
    ref = oracle.vec_dot_ref_rows(t, w, rows, cols, x)
    assert np.array_equal(ref.view(np.uint32), FIX[f"{name}/vec_dot_ref"])
    if t == Q4_K:
        import ctypes
        rb = cols // 256 * 144
        sc = np.array([oracle.lib.kqo_dot_q4_K_scalar(ctypes.c_void_p(w.ctypes.data + r * rb),
                                                      x.ctypes.data_as(ctypes.c_void_p), cols // 256)
                       for r in range(rows)], np.float32)
        assert np.array_equal(sc.view(np.uint32), FIX[f"{name}/vec_dot_scalar"])
    assert MG.sha(oracle.dequant(t, w, rows * cols)) == str(FIX[f"{name}/dequant_sha256"])
    # the reference's own tolerance between its fast and double paths (gguf_dtype.c:1206)
    assert np.all(np.abs(fast - ref) <= 1e-4 + 1e-3 * np.abs(ref))


def test_silu_fixture(oracle):
    rng = np.random.default_rng(201)
    g = (rng.standard_normal(768) * 4).astype(np.float32)
    u = rng.standard_normal(768).astype(np.float32)
    assert MG.sha(g, u) == str(FIX["silu/input_sha256"])
    assert np.array_equal(oracle.silu_mul_ref(g, u).view(np.uint32), FIX["silu/out"])


def test_softmax_fixture_pins_router_weights(oracle):
    """The reference softmax, renormalised over the top 8, agrees with the
    oracle router weights (which never form the full softmax)."""
    rng = np.random.default_rng(202)
    logits = rng.standard_normal(128).astype(np.float32)
    assert MG.sha(logits) == str(FIX["softmax/input_sha256"])
    p = FIX["softmax/out"].view(np.float32).astype(np.float64)
    ids, w = oracle.router_topk(logits, 8)
    assert ids.tolist() == list(np.argsort(-p, kind="stable")[:8])
    assert np.allclose(w, p[ids] / p[ids].sum(), rtol=1e-5, atol=0)
