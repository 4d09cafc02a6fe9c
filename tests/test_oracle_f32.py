"""The oracle's F32 matvec (the MoE router's logits), pinned bit-exact against
the compiled reference's katali_ggml_matvec on F32 rows (AVX2 path,
V/src/gguf_simd_x86.c:111-122, 674-682), and against what the arithmetic
fixes: exact integer dots, and the engine's 16-chain order (a sequential sum
differs on a crafted row)."""
import numpy as np
import pytest

SHAPES = [(128, 2048), (256, 7168), (3, 4100), (5, 12), (1, 16), (7, 2060), (2, 4), (64, 32768)]


@pytest.mark.parametrize("rows,cols", SHAPES)
def test_f32_matvec_bit_exact_vs_reference(oracle, refcpu, rows, cols):
    if not refcpu.simd():
        pytest.skip("the compiled reference takes its scalar path on this CPU")
    rng = np.random.default_rng(rows * 131 + cols)
    w = rng.standard_normal((rows, cols)).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    got = oracle.matvec_f32x(0, w, rows, cols, x)
    want = refcpu.matvec(0, w, rows, cols, x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_f32_matvec_exact_on_integers(oracle):
    rng = np.random.default_rng(2)
    rows, cols = 9, 2052
    w = rng.integers(-8, 9, (rows, cols)).astype(np.float32)
    x = rng.integers(-8, 9, cols).astype(np.float32)
    want = (w.astype(np.int64) @ x.astype(np.int64)).astype(np.float32)   # |sums| < 2^24: exact
    assert np.array_equal(oracle.matvec_f32x(0, w, rows, cols, x), want)


def test_f32_matvec_follows_the_sixteen_chain_order(oracle):
    # Columns 0 and 16 share chain 0, column 1 is chain 1: 2^25 + 1 - 2^25 in
    # chain order loses the 1 only if the 1 meets 2^25 first.
    cols = 32
    x = np.ones(cols, np.float32)
    w = np.zeros((1, cols), np.float32)
    w[0, 0], w[0, 1], w[0, 16] = 2.0 ** 25, 1.0, -(2.0 ** 25)
    seq = np.float32(0)
    for v in w[0]:
        seq = np.float32(seq + v)              # a sequential float sum gives 0
    assert seq == 0.0
    assert oracle.matvec_f32x(0, w, 1, cols, x)[0] == 1.0   # chains: (2^25 - 2^25) + 1


def test_f32_matvec_close_to_float64(oracle):
    rng = np.random.default_rng(4)
    w = rng.standard_normal((32, 4096)).astype(np.float32)
    x = rng.standard_normal(4096).astype(np.float32)
    ref = w.astype(np.float64) @ x.astype(np.float64)
    got = oracle.matvec_f32x(0, w, 32, 4096, x).astype(np.float64)
    assert np.max(np.abs(got - ref) / (np.abs(w) @ np.abs(x))) < 4096 * 2.0 ** -24
