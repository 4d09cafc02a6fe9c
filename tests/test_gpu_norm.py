"""GPU parity: RMSNorm and the residual step before it, through the C ABI,
against the oracle (itself bit-exact to the reference's katali_gguf_rmsnorm).
Bar: bit-identical (the device sums squares in double in another order; its
rounding to float differs only on a float rounding boundary)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SIZES = [1, 4, 1000, 2048, 4096, 5120, 12288, 70000]


@pytest.mark.parametrize("n", SIZES)
def test_rmsnorm_bit_identical(hip, oracle, n):
    print(f"[rmsnorm] n={n}", flush=True)
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * 3).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    xd, wd, out = hip.to_device(x), hip.to_device(w), hip.alloc(n * 4)
    for eps in (1e-5, 1e-6):
        hip.rmsnorm(xd, wd, n, eps, out)
        assert np.array_equal(out.download(np.uint32, n), oracle.rmsnorm(x, w, eps).view(np.uint32))
    hip.rmsnorm(xd, wd, n, 1e-6, xd)   # in place (katali_gguf_rmsnorm_inplace)
    assert np.array_equal(xd.download(np.uint32, n), oracle.rmsnorm(x, w, 1e-6).view(np.uint32))


@pytest.mark.parametrize("scale", [1.0, 0.25])
@pytest.mark.parametrize("n", [4096, 12288, 3001])
def test_add_rmsnorm_bit_identical(hip, oracle, n, scale):
    print(f"[add_rmsnorm] n={n} scale={scale}", flush=True)
    rng = np.random.default_rng(n + int(scale * 8))
    x, d, w = (rng.standard_normal(n).astype(np.float32) for _ in range(3))
    xd, dd, wd, out = hip.to_device(x), hip.to_device(d), hip.to_device(w), hip.alloc(n * 4)
    want_x, want = oracle.add_rmsnorm(x, d, scale, w, 1e-6)
    hip.add_rmsnorm(xd, dd, scale, wd, n, 1e-6, out)
    assert np.array_equal(xd.download(np.uint32, n), want_x.view(np.uint32))   # residual in place
    assert np.array_equal(out.download(np.uint32, n), want.view(np.uint32))


def test_add_rmsnorm_graph_replays(hip, oracle):
    """Captured once, replayed: each replay adds the residual again."""
    n = 4096
    rng = np.random.default_rng(3)
    x, d, w = (rng.standard_normal(n).astype(np.float32) for _ in range(3))
    xd, dd, wd, out = hip.to_device(x), hip.to_device(d), hip.to_device(w), hip.alloc(n * 4)
    hip.graph_begin()
    hip.add_rmsnorm(xd, dd, 1.0, wd, n, 1e-5, out)
    g = hip.graph_end()
    try:
        cur = x
        for i in range(3):
            hip.graph_launch(g)
            hip.sync()
            cur, want = oracle.add_rmsnorm(cur, d, 1.0, w, 1e-5)
            assert np.array_equal(xd.download(np.uint32, n), cur.view(np.uint32)), i
            assert np.array_equal(out.download(np.uint32, n), want.view(np.uint32)), i
    finally:
        hip.graph_destroy(g)


def test_norm_rejects_bad_arguments(hip):
    from katali_hip import HipError
    x = hip.alloc(64)
    for n in (0, (1 << 20) + 1):
        with pytest.raises(HipError):
            hip.rmsnorm(x, x, n, 1e-6, x)
    assert hip.lib.katali_hip_add_rmsnorm(x.ptr, None, 1.0, x.ptr, 4, 1e-6, x.ptr) == -1


NR_CASES = [
    # n, rows, residual scale (None: no residual step)
    (2048, 128, 1.0), (2048, 128, None), (4096, 256, 0.5), (7168, 300, 1.0), (8192, 1030, None),
    (1000, 64, 1.0), (12, 1, 1.0), (3072, 513, 0.25),
]


@pytest.mark.parametrize("n,rows,scale", NR_CASES)
def test_norm_router_bit_identical(hip, oracle, n, rows, scale):
    """Residual step + RMSNorm + F32 router logits in one launch: each output
    bit-identical to the oracle's separate steps."""
    print(f"[norm-router] n={n} rows={rows} scale={scale}", flush=True)
    rng = np.random.default_rng(n + rows)
    x, d, nw = (rng.standard_normal(n).astype(np.float32) for _ in range(3))
    w = (rng.standard_normal((rows, n)) * 0.05).astype(np.float32)
    xd, dd, nwd, wd = hip.to_device(x), hip.to_device(d), hip.to_device(nw), hip.to_device(w)
    xo, xn, y = hip.alloc(n * 4), hip.alloc(n * 4), hip.alloc(rows * 4)
    if scale is None:
        hip.rmsnorm_matvec_f32(xd, None, 1.0, None, nwd, n, 1e-6, xn, wd, rows, y)
        want_x, want_xn = x, oracle.rmsnorm(x, nw, 1e-6)
    else:
        hip.rmsnorm_matvec_f32(xd, dd, scale, xo, nwd, n, 1e-6, xn, wd, rows, y)
        want_x, want_xn = oracle.add_rmsnorm(x, d, scale, nw, 1e-6)
        assert np.array_equal(xo.download(np.uint32, n), want_x.view(np.uint32))
    assert np.array_equal(xd.download(np.uint32, n), x.view(np.uint32))          # x untouched
    assert np.array_equal(xn.download(np.uint32, n), want_xn.view(np.uint32))
    want_y = oracle.matvec_f32x(0, w, rows, n, want_xn)
    assert np.array_equal(y.download(np.uint32, rows), want_y.view(np.uint32))


def test_norm_router_rejects_bad_arguments(hip):
    from katali_hip import HipError
    n, rows = 256, 8
    a, b, c, xn, w, y = (hip.alloc(n * rows * 4) for _ in range(6))
    bad = [
        (a, b, 1.0, None, c, n, 1e-6, xn, w, rows, y),      # residual without x_out
        (a, b, 1.0, a, c, n, 1e-6, xn, w, rows, y),         # x_out is x
        (a, None, 1.0, None, c, n, 1e-6, a, w, rows, y),    # xn is x
        (a, None, 1.0, None, c, n, 1e-6, xn, w, rows, w),   # y inside W
        (a, None, 1.0, None, c, 8196, 1e-6, xn, w, 1, y),   # n above 8192
        (a, None, 1.0, None, c, 6, 1e-6, xn, w, rows, y),   # n % 4
        (a, None, 1.0, None, c, n, 1e-6, xn, w, 0, y),      # no rows
    ]
    for args in bad:
        with pytest.raises(HipError):
            hip.rmsnorm_matvec_f32(*args)
