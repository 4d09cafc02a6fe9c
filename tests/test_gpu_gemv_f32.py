"""GPU parity: F32 matvec (the MoE router's logits) through the C ABI,
bit-identical to the oracle's restatement of the engine's AVX2 F32 dot (itself
bit-exact against the compiled reference)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SHAPES = [(128, 2048), (256, 7168), (3, 4100), (5, 12), (1, 16), (7, 2060), (300, 2048), (1100, 512),
          (64, 32768), (40, 4), (513, 2052)]


@pytest.mark.parametrize("rows,cols", SHAPES)
def test_f32_matvec_bit_identical(hip, oracle, rows, cols):
    print(f"[matvec-f32] rows={rows} cols={cols}", flush=True)
    rng = np.random.default_rng(rows * 7 + cols)
    w = rng.standard_normal((rows, cols)).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    wd, xd, yd = hip.to_device(w), hip.to_device(x), hip.alloc(rows * 4)
    hip.matvec(0, wd, rows, cols, xd, yd)
    got = yd.download(np.uint32, rows)
    assert np.array_equal(got, oracle.matvec_f32x(0, w, rows, cols, x).view(np.uint32))


def test_f32_matvec_signed_zero_and_integers(hip, oracle):
    """A row of -0 products gives +0 (acc + 0.0f, as the engine); integer
    inputs give the exact dot."""
    rows, cols = 3, 48
    w = np.zeros((rows, cols), np.float32)
    w[0] = -0.0
    w[1] = np.arange(cols) - 20
    w[2, 5] = -1.0
    x = np.ones(cols, np.float32)
    x[5] = 0.0
    wd, xd, yd = hip.to_device(w), hip.to_device(x), hip.alloc(rows * 4)
    hip.matvec(0, wd, rows, cols, xd, yd)
    got = yd.download(np.float32, rows)
    assert np.array_equal(got.view(np.uint32), oracle.matvec_f32x(0, w, rows, cols, x).view(np.uint32))
    assert got[1] == float(np.sum((np.arange(cols) - 20) * (np.arange(cols) != 5))) and not np.signbit(got[2]) and not np.signbit(got[0])


def test_f32_matvec_rejects_bad_arguments(hip):
    from katali_hip import HipError
    w, x, y = hip.alloc(4096), hip.alloc(4096), hip.alloc(4096)
    with pytest.raises(HipError):
        hip.matvec(0, w, 2, 6, x, y)                      # cols % 4
    with pytest.raises(HipError):
        hip.check(hip.lib.katali_hip_matvec(0, w.ptr + 4, 2, 8, x.ptr, y.ptr))   # w not 16-byte aligned
    with pytest.raises(HipError):
        hip.matvec_q8(0, w, 2, 256, x, y)                 # F32 is matvec only
    with pytest.raises(HipError):
        hip.matvec_multi([0], [w], [2], 256, x, [y])
