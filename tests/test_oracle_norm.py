"""The oracle's RMSNorm and residual step, pinned three ways: bit-exact
against the compiled reference (katali_gguf_rmsnorm, katali_gguf_add_inplace,
V/src/gguf_kernels.c:13-18,319-321), the reference's own known answer
(gguf_kernels.c:348-358) and invariants the definition fixes (a constant
vector, exact power-of-two scaling at eps = 0)."""
import numpy as np
import pytest

SIZES = [1, 4, 257, 2048, 4096, 5120, 12288]


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("eps", [0.0, 1e-6, 1e-5])
def test_rmsnorm_bit_exact_vs_reference(oracle, refcpu, n, eps):
    rng = np.random.default_rng(n * 7 + int(eps * 1e7))
    x = (rng.standard_normal(n) * rng.uniform(0.1, 30)).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    assert np.array_equal(oracle.rmsnorm(x, w, eps).view(np.uint32), refcpu.rmsnorm(x, w, eps).view(np.uint32))


@pytest.mark.parametrize("scale", [1.0, 0.5, 1.7])
def test_add_rmsnorm_vs_reference_sequence(oracle, refcpu, scale):
    rng = np.random.default_rng(11)
    n, eps = 4096, 1e-6
    x, d, w = (rng.standard_normal(n).astype(np.float32) for _ in range(3))
    xs, out = oracle.add_rmsnorm(x, d, scale, w, eps)
    if scale == 1.0:
        want_x = refcpu.add_inplace(x, d)                   # gguf_model.c:677
    else:
        want_x = x + np.float32(scale) * d                  # gguf_model.c:678, float32 ops, no contraction
    assert np.array_equal(xs.view(np.uint32), want_x.view(np.uint32))
    assert np.array_equal(out.view(np.uint32), refcpu.rmsnorm(want_x, w, eps).view(np.uint32))


def test_rmsnorm_reference_known_answer(oracle):
    x = np.array([3.0, -3.0, 3.0, -3.0], np.float32)        # gguf_kernels.c:350-357
    out = oracle.rmsnorm(x, np.ones(4, np.float32), 0.0)
    assert np.all(np.abs(out - x / 3.0) <= 1e-5)


@pytest.mark.parametrize("c,eps", [(2.0, 0.0), (-0.5, 1e-5), (3.0, 16.0)])
def test_rmsnorm_constant_vector(oracle, c, eps):
    n = 1000
    out = oracle.rmsnorm(np.full(n, c, np.float32), np.ones(n, np.float32), eps)
    want = c / np.sqrt(c * c + eps)                          # mean of squares = c^2
    assert np.allclose(out, want, rtol=2e-7, atol=0)


def test_rmsnorm_power_of_two_scaling_is_exact(oracle):
    rng = np.random.default_rng(5)
    x = rng.standard_normal(3000).astype(np.float32)
    w = rng.standard_normal(3000).astype(np.float32)
    a = oracle.rmsnorm(x, w, 0.0)
    b = oracle.rmsnorm(x * np.float32(4.0), w, 0.0)         # sumsq * 16, sqrt * 4, inv / 4
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
