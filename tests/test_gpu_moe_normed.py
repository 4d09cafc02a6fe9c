"""katali_hip_moe_layer_normed through the C ABI: the residual step, RMSNorm,
F32 router and MoE layer in two launches, against the same steps as separate
calls (katali_hip_rmsnorm_matvec_f32 then katali_hip_moe_layer routed from its
logits), which the norm and MoE tests pin to the oracle. Every output must be
bit-identical: the new residual, xn, the logits, the routing and y. Shapes
cover the merged path (router rows spread over kernel A's workgroups, one or
several rows each) and the fallback (more than four rows per workgroup), with
and without the residual step and the shared expert; queued layers, graph
replays with eager work between them, and bad arguments. The tests run the
layer as kernels A and B (KATALI_HIP_XCD=0) unless they name the XCD mode:
eight-slot layers then run as the XCD-sliced layer with the steps before it
in its prologue (one launch), against the same steps as separate calls whose
layer is the XCD-sliced one too."""
import copy

import numpy as np
import pytest

from katali_hip import HipError
from oracle import Q4_K, Q6_K

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("two_launch_layer")]

CASES = [
    # hidden, ffn, n_expert, n_sel, shared, down, residual scale (None: no residual step)
    (2048, 768, 128, 8, False, Q6_K, 1.0),     # the decode layer: one router row per workgroup
    (2048, 768, 128, 8, False, Q6_K, None),
    (2048, 512, 256, 8, True, Q6_K, 0.5),      # 144 workgroups, two rows each
    (4096, 256, 64, 4, False, Q6_K, 1.0),      # wide hidden (512-thread workgroups, 4 float4 per norm thread)
    (256, 512, 64, 4, True, Q4_K, 1.0),        # narrow hidden, Q4_K down
    (1024, 256, 512, 2, False, Q6_K, 1.0),     # 16 workgroups for 512 rows: the two-step fallback
    (512, 256, 60, 3, False, Q6_K, 0.25),      # rows not a multiple of the workgroups
]


XCD_CASES = [
    # eight slots: hidden 1024 or 2048, ffn <= 1024, <= 256 experts
    (2048, 768, 128, 8, False, Q6_K, 1.0),     # the decode layer
    (2048, 768, 128, 8, False, Q6_K, None),
    (2048, 512, 256, 7, True, Q6_K, 0.5),      # seven routed and the shared expert; one router row per workgroup
    (1024, 1024, 64, 8, False, Q4_K, 1.0),     # narrow hidden, the widest ffn, Q4_K down
    (1024, 256, 200, 8, False, Q6_K, 0.25),    # rows not a multiple of 64
    # up to 128 experts each XCD forms every logit itself, rows w / 8 + 32 v:
    # expert counts that leave the last row group partly empty
    (1024, 256, 100, 8, False, Q6_K, 1.0),
    (2048, 256, 40, 8, False, Q6_K, None),
]


def set_mode(monkeypatch, mode):
    monkeypatch.setenv("KATALI_HIP_XCD", "1" if mode == "xcd" else "0")


def case_id(c):
    return (f"h{c[0]}_f{c[1]}_e{c[2]}_k{c[3]}{'_sh' if c[4] else ''}"
            f"{'_q4down' if c[5] == Q4_K else ''}_s{c[6]}")


class Layer:
    def __init__(self, hip, hidden, ffn, n_expert, shared, down, seed):
        self.hidden, self.ffn, self.n_expert = hidden, ffn, n_expert
        nb_gu, nb_d = n_expert * ffn * hidden // 256, n_expert * hidden * ffn // 256
        bb = {Q4_K: 144, Q6_K: 210}
        self.bufs = [hip.alloc(nb_gu * 144), hip.alloc(nb_gu * 144), hip.alloc(nb_d * bb[down])]
        for i, (t, b, n) in enumerate(((Q4_K, self.bufs[0], nb_gu), (Q4_K, self.bufs[1], nb_gu),
                                       (down, self.bufs[2], nb_d))):
            hip.synth_fill(t, b, n, seed=seed + i)
        sh = None
        if shared:
            n1 = ffn * hidden // 256
            sh = (hip.alloc(n1 * 144), hip.alloc(n1 * 144), hip.alloc(n1 * bb[down]))
            for i, (t, b) in enumerate(((Q4_K, sh[0]), (Q4_K, sh[1]), (down, sh[2]))):
                hip.synth_fill(t, b, n1, seed=seed + 10 + i)
        self.desc = hip.moe_desc(hidden, ffn, n_expert, *self.bufs, down_type=down, shared=sh)
        rng = np.random.default_rng(seed)
        self.router = hip.to_device((rng.standard_normal((n_expert, hidden)) * 0.05).astype(np.float32))
        self.norm_w = hip.to_device(rng.standard_normal(hidden).astype(np.float32))


def separate(hip, L, n_sel, x, delta, scale):
    """The reference path: norm/router launch, then the layer from its logits."""
    H, E = L.hidden, L.n_expert
    xo, xn, lg, y = hip.alloc(H * 4), hip.alloc(H * 4), hip.alloc(E * 4), hip.alloc(H * 4)
    ids, w = hip.alloc(64), hip.alloc(64)
    hip.rmsnorm_matvec_f32(x, delta, scale, xo if delta else None, L.norm_w, H, 1e-6, xn, L.router, E, lg)
    hip.moe_layer(L.desc, hip.moe_route(n_sel, logits=lg, ids_out=ids, weights_out=w), y, x=xn)
    return xo, xn, lg, ids, w, y


def normed(hip, L, n_sel, x, delta, scale, outputs=True):
    H, E = L.hidden, L.n_expert
    xo, xn, lg, y = hip.alloc(H * 4), hip.alloc(H * 4), hip.alloc(E * 4), hip.alloc(H * 4)
    ids, w = hip.alloc(64), hip.alloc(64)
    hip.moe_layer_normed(L.desc, n_sel, x, L.norm_w, L.router, y, delta=delta, scale=scale,
                         x_out=xo if delta else None, xn_out=xn if outputs else None,
                         logits_out=lg if outputs else None, ids_out=ids, weights_out=w)
    return xo, xn, lg, ids, w, y


def same(a, b, n, dtype=np.uint32):
    return np.array_equal(a.download(dtype, n), b.download(dtype, n))


@pytest.fixture(scope="module")
def layers(hip):
    cache = {}

    def get(hidden, ffn, n_expert, shared, down):
        key = (hidden, ffn, n_expert, shared, down)
        if key not in cache:
            cache.clear()
            cache[key] = Layer(hip, hidden, ffn, n_expert, shared, down, seed=hash(key) & 0xFFFF)
        return cache[key]
    return get


@pytest.mark.parametrize("case", [("two_launch", c) for c in CASES] + [("xcd", c) for c in XCD_CASES],
                         ids=[f"two_launch-{case_id(c)}" for c in CASES] + [f"xcd-{case_id(c)}" for c in XCD_CASES])
def test_normed_layer_matches_separate_steps(hip, layers, case, monkeypatch):
    mode, (hidden, ffn, n_expert, n_sel, shared, down, scale) = case
    set_mode(monkeypatch, mode)
    print(f"[moe-normed] mode={mode} case={case[1]}", flush=True)
    L = layers(hidden, ffn, n_expert, shared, down)
    rng = np.random.default_rng(hidden + n_expert + n_sel)
    x = hip.to_device(rng.standard_normal(hidden).astype(np.float32))
    delta = hip.to_device(rng.standard_normal(hidden).astype(np.float32)) if scale is not None else None
    sc = 1.0 if scale is None else scale
    want = separate(hip, L, n_sel, x, delta, sc)
    for outputs in (True, False):
        got = normed(hip, L, n_sel, x, delta, sc, outputs)
        hip.sync()
        if delta is not None:
            assert same(got[0], want[0], hidden), "x_out"
        if outputs:
            assert same(got[1], want[1], hidden), "xn"
            assert same(got[2], want[2], n_expert), "logits"
        assert same(got[3], want[3], n_sel, np.int32), "ids"
        assert same(got[4], want[4], n_sel), "weights"
        y = got[5].download(np.uint32, hidden)
        assert np.array_equal(y, want[5].download(np.uint32, hidden)), int(np.sum(y != want[5].download(np.uint32, hidden)))
        assert np.any(y != 0)


@pytest.mark.parametrize("mode", ["two_launch", "xcd"])
def test_normed_layers_queued_back_to_back(hip, layers, mode, monkeypatch):
    """24 normed layers queued without a wait (each call's exchange a new
    generation): every one equals its separate-steps run."""
    set_mode(monkeypatch, mode)
    print(f"[moe-normed] queued mode={mode}", flush=True)
    hidden, ffn, n_expert, n_sel = 2048, 768, 128, 8
    L = layers(hidden, ffn, n_expert, False, Q6_K)
    rng = np.random.default_rng(9)
    n = 24
    xs = [hip.to_device(rng.standard_normal(hidden).astype(np.float32)) for _ in range(n)]
    ds = [hip.to_device(rng.standard_normal(hidden).astype(np.float32)) for _ in range(n)]
    outs = [normed(hip, L, n_sel, xs[i], ds[i], 1.0) for i in range(n)]
    hip.sync()
    for i in (0, 1, 11, n - 1):
        want = separate(hip, L, n_sel, xs[i], ds[i], 1.0)
        hip.sync()
        for k, name in ((0, "x_out"), (1, "xn"), (5, "y")):
            assert same(outs[i][k], want[k], hidden), (i, name)


@pytest.mark.parametrize("mode,n_sel", [("two_launch", 8), ("xcd", 7)])
def test_normed_layer_graph_replays(hip, layers, mode, n_sel, monkeypatch):
    """Two chained normed layers (the second's residual step adds the first's
    y) captured once and replayed with eager work between the replays: every
    replay equals the eager run."""
    set_mode(monkeypatch, mode)
    hidden, ffn, n_expert = 2048, 512, 256
    L = layers(hidden, ffn, n_expert, True, Q6_K)
    rng = np.random.default_rng(10)
    x0 = hip.to_device(rng.standard_normal(hidden).astype(np.float32))
    x1, y0, y1 = hip.alloc(hidden * 4), hip.alloc(hidden * 4), hip.alloc(hidden * 4)

    def token():
        hip.moe_layer_normed(L.desc, n_sel, x0, L.norm_w, L.router, y0)
        hip.moe_layer_normed(L.desc, n_sel, x0, L.norm_w, L.router, y1, delta=y0, scale=1.0, x_out=x1)

    token()
    hip.sync()
    want = (y0.download(np.uint32), y1.download(np.uint32), x1.download(np.uint32))
    hip.graph_begin()
    token()
    g = hip.graph_end()
    try:
        for i in range(4):
            for b in (y0, y1, x1):
                hip.memset(b, 0, hidden * 4)
            print(f"[moe-normed] replay {i}", flush=True)
            hip.graph_launch(g)
            hip.sync()
            assert np.array_equal(y0.download(np.uint32), want[0]), i
            assert np.array_equal(y1.download(np.uint32), want[1]), i
            assert np.array_equal(x1.download(np.uint32), want[2]), i
            token()   # eager work between replays
            hip.sync()
            assert np.array_equal(y1.download(np.uint32), want[1]), i
    finally:
        hip.graph_destroy(g)


@pytest.mark.parametrize("n_expert", [128, 256])
def test_normed_xcd_routing_ties_match_oracle(hip, oracle, layers, n_expert, monkeypatch):
    """Twelve equal router rows whose logits rise above the rest, so the
    logits tie across the first eight ranks: the one-launch normed layer's
    routing (the workgroup's ranking, then each wave's ranking once it sees
    the tie) selects what the oracle router selects from the same logits
    (the lower index first), and every output equals the separate steps'."""
    set_mode(monkeypatch, "xcd")
    hidden, ffn, n_sel = 1024, 256, 8
    print(f"[moe-normed] ties n_expert={n_expert}", flush=True)
    L = copy.copy(layers(hidden, ffn, n_expert, False, Q6_K))
    rng = np.random.default_rng(n_expert)
    xh = rng.standard_normal(hidden).astype(np.float32)
    dh = rng.standard_normal(hidden).astype(np.float32)
    nw = L.norm_w.download(np.float32, hidden).astype(np.float64)
    r = xh.astype(np.float64) + dh
    xn = r / np.sqrt(np.mean(r * r) + 1e-6) * nw
    router = (rng.standard_normal((n_expert, hidden)) * 0.05).astype(np.float32)
    tied = rng.permutation(n_expert)[:12]
    router[tied] = (0.1 * np.sign(xn)).astype(np.float32)
    L.router = hip.to_device(router)
    x, delta = hip.to_device(xh), hip.to_device(dh)
    want = separate(hip, L, n_sel, x, delta, 1.0)
    got = normed(hip, L, n_sel, x, delta, 1.0)
    hip.sync()
    lg = got[2].download(np.float32, n_expert)
    rest = np.delete(lg, tied)
    assert np.all(lg[tied] == lg[tied[0]]) and lg[tied[0]] > rest.max(), "the twelve logits tie at the top"
    assert same(got[2], want[2], n_expert), "logits"
    ids, w = oracle.router_topk(lg, n_sel)
    assert ids.tolist() == sorted(tied.tolist())[:n_sel]
    for path, o in (("normed", got), ("separate", want)):
        assert o[3].download(np.int32, n_sel).tolist() == ids.tolist(), path
        assert np.array_equal(o[4].download(np.uint32, n_sel), w.view(np.uint32)), path
    assert same(got[5], want[5], hidden), "y"


def test_normed_layer_rejects_bad_arguments(hip, layers):
    L = layers(512, 256, 60, False, Q6_K)
    x, y = hip.alloc(512 * 4), hip.alloc(512 * 4)
    with pytest.raises(HipError):
        hip.moe_layer_normed(L.desc, 0, x, L.norm_w, L.router, y)              # must route
    with pytest.raises(HipError):
        hip.moe_layer_normed(L.desc, 61, x, L.norm_w, L.router, y)             # n_sel > n_expert
    with pytest.raises(HipError):
        hip.moe_layer_normed(L.desc, 2, x, L.norm_w, L.router, y, delta=y)     # delta without x_out
    with pytest.raises(HipError):
        hip.moe_layer_normed(L.desc, 2, x, L.norm_w, L.router, x)              # y overlaps x
    hip.sync()
