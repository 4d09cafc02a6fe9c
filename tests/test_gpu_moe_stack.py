"""katali_hip_moe_stack_* through the C ABI: n layers in one launch, each
layer waiting for the previous layer's output.

Plain stack: every layer's y, ids and weights bit-identical to
katali_hip_moe_layer called layer by layer on the same inputs (each layer's
own x, or x_l = y_{l-1}: without a norm such a chain grows quadratically
from layer to layer, so chained cases are two layers long and every compared
output is checked finite);
normed stack: every layer's y, residual, normalized vector, logits, ids and
weights bit-identical to katali_hip_moe_layer_normed called layer by layer
(x_l = x_{l-1} + y_{l-1}). Those single-layer entry points are pinned to the
oracle by test_gpu_moe.py / test_gpu_moe_normed.py; here the stack's first
two layers are also checked against the oracle's q8 path directly. Also:
the layer-by-layer path the stack takes for other shapes or with
KATALI_HIP_XCD=0, graph replays with eager work between them, and bad
arguments refused.
"""
import numpy as np
import pytest

import kq_synth as S
from katali_hip import HipError
from oracle import Q4_K, Q6_K

pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


class Stack:
    """n_layers layers of distinct synthetic weights on the device."""

    def __init__(self, hip, hidden, ffn, n_expert, n_sel, shared, down, n_layers, seed, normed=False,
                 chained=False):
        # a chain x_1 = y_0 keeps finite, non-zero values (h's q8_1 scale is
        # f16) only where y_0 is of x_0's order: small block scales then
        sg, sd = (1e-3, 4e-7) if chained else (0.02, 0.02)
        self.hidden, self.ffn, self.n_expert, self.n_sel = hidden, ffn, n_expert, n_sel
        self.n_layers, self.normed = n_layers, normed
        nb_gu, nb_d = n_expert * ffn * hidden // 256, n_expert * hidden * ffn // 256
        bb = {Q4_K: 144, Q6_K: 210}
        rng = np.random.default_rng(seed)
        self.layers = []
        for li in range(n_layers):
            g, u, d = hip.alloc(nb_gu * 144), hip.alloc(nb_gu * 144), hip.alloc(nb_d * bb[down])
            for i, (t, b, n, sc) in enumerate(((Q4_K, g, nb_gu, sg), (Q4_K, u, nb_gu, sg), (down, d, nb_d, sd))):
                hip.synth_fill(t, b, n, seed=seed + 16 * li + i, d_sigma=sc)
            sh = None
            if shared:
                n1 = ffn * hidden // 256
                sh = (hip.alloc(n1 * 144), hip.alloc(n1 * 144), hip.alloc(n1 * bb[down]))
                for i, (t, b, sc) in enumerate(((Q4_K, sh[0], sg), (Q4_K, sh[1], sg), (down, sh[2], sd))):
                    hip.synth_fill(t, b, n1, seed=seed + 16 * li + 8 + i, d_sigma=sc)
            L = {"gate": g, "up": u, "down": d, "shared": sh,
                 "desc": hip.moe_desc(hidden, ffn, n_expert, g, u, d, down_type=down, shared=sh)}
            if normed:
                L["norm_w"] = hip.to_device(rng.standard_normal(hidden).astype(np.float32))
                L["router"] = hip.to_device((rng.standard_normal((n_expert, hidden)) * 0.05).astype(np.float32))
            else:
                L["logits"] = hip.to_device(rng.standard_normal(n_expert).astype(np.float32))
                if li and not chained:   # the layer's own input
                    L["x"] = hip.to_device(rng.standard_normal(hidden).astype(np.float32))
            self.layers.append(L)
        self.desc = self.layers[0]["desc"]
        self.x = hip.to_device(rng.standard_normal(hidden).astype(np.float32))
        self.delta = hip.to_device(rng.standard_normal(hidden).astype(np.float32))

    def outputs(self, hip):
        """Fresh per-layer output buffers."""
        H, E = self.hidden, self.n_expert
        return [{"y": hip.alloc(H * 4), "ids": hip.alloc(64), "w": hip.alloc(64), "x_out": hip.alloc(H * 4),
                 "xn": hip.alloc(H * 4), "lg": hip.alloc(E * 4)} for _ in range(self.n_layers)]

    def make(self, hip, outs):
        entries = []
        for L, o in zip(self.layers, outs):
            e = {"gate": L["gate"], "up": L["up"], "down": L["down"], "shared": L["shared"], "y": o["y"]}
            if self.normed:
                e.update(norm_w=L["norm_w"], router=L["router"], x_out=o["x_out"], xn_out=o["xn"],
                         logits_out=o["lg"], route=hip.moe_route(self.n_sel, ids_out=o["ids"], weights_out=o["w"]))
            else:
                e["route"] = hip.moe_route(self.n_sel, logits=L["logits"], ids_out=o["ids"], weights_out=o["w"])
                e["x"] = L.get("x")
            entries.append(e)
        return hip.moe_stack(self.desc, self.n_sel, entries, normed=self.normed)

    def layer_by_layer(self, hip, outs, scale=None):
        """The single-layer entry points on the same chain."""
        cur = self.x
        for li, (L, o) in enumerate(zip(self.layers, outs)):
            if self.normed:
                delta = (self.delta if scale is not None else None) if li == 0 else outs[li - 1]["y"]
                sc = (scale if scale is not None else 1.0) if li == 0 else 1.0
                hip.moe_layer_normed(L["desc"], self.n_sel, cur, L["norm_w"], L["router"], o["y"], delta=delta,
                                     scale=sc, x_out=o["x_out"] if delta is not None else None, xn_out=o["xn"],
                                     logits_out=o["lg"], ids_out=o["ids"], weights_out=o["w"])
                if delta is not None:
                    cur = o["x_out"]
            else:
                route = hip.moe_route(self.n_sel, logits=L["logits"], ids_out=o["ids"], weights_out=o["w"])
                hip.moe_layer(L["desc"], route, o["y"], x=L.get("x", cur) if li else cur)
                cur = o["y"]


def words(buf, n):
    return buf.download(np.uint32, n)


def compare(st, a, b, with_residual=True):
    H, E, k = st.hidden, st.n_expert, st.n_sel
    for li in range(st.n_layers):
        yv = a[li]["y"].download(np.float32, H)
        assert np.isfinite(yv).all() and np.abs(yv).max() > 0, f"layer {li}: y not finite, or all zero"
        assert np.array_equal(words(a[li]["y"], H), words(b[li]["y"], H)), f"layer {li}: y"
        assert np.array_equal(a[li]["ids"].download(np.int32, k), b[li]["ids"].download(np.int32, k)), f"layer {li}: ids"
        assert np.array_equal(words(a[li]["w"], k), words(b[li]["w"], k)), f"layer {li}: weights"
        if st.normed:
            assert np.array_equal(words(a[li]["xn"], H), words(b[li]["xn"], H)), f"layer {li}: xn"
            assert np.array_equal(words(a[li]["lg"], E), words(b[li]["lg"], E)), f"layer {li}: logits"
            if with_residual and li > 0:
                assert np.array_equal(words(a[li]["x_out"], H), words(b[li]["x_out"], H)), f"layer {li}: residual"


PLAIN = [
    # hidden, ffn, n_expert, n_sel, shared, down, layers (each layer its own x)
    (2048, 768, 128, 8, False, Q6_K, 5),    # the decode layer's shape
    (2048, 512, 256, 8, True, Q6_K, 4),     # top-8 of 256 plus the shared expert (spread over every workgroup)
    (2048, 512, 256, 7, True, Q6_K, 3),     # seven routed plus the shared expert
    (1024, 1024, 64, 8, False, Q4_K, 4),    # narrow hidden, the widest ffn, Q4_K down
    (1024, 256, 200, 8, False, Q6_K, 3),
]
NORMED = [
    (2048, 768, 128, 8, False, Q6_K, 5),
    (1024, 1024, 64, 8, False, Q4_K, 3),
    (1024, 256, 200, 8, False, Q6_K, 3),
]
# shapes the one-launch stack does not take: layer by layer
OTHER = [
    (2048, 768, 128, 4, False, Q6_K, 3, False),
    (512, 256, 16, 4, True, Q4_K, 3, True),
]


def cid(c):
    return f"h{c[0]}_f{c[1]}_e{c[2]}_k{c[3]}{'_sh' if c[4] else ''}{'_q4down' if c[5] == Q4_K else ''}_L{c[6]}"


@pytest.fixture(autouse=True)
def one_launch(monkeypatch):
    for k in ("KATALI_HIP_XCD", "KATALI_HIP_XCD_SHARED", "KATALI_HIP_FUSED"):
        monkeypatch.delenv(k, raising=False)


@pytest.mark.parametrize("chained", [False, True], ids=["own_x", "chained"])
@pytest.mark.parametrize("case", PLAIN, ids=[cid(c) for c in PLAIN])
def test_plain_stack_matches_layer_by_layer(hip, case, chained):
    hidden, ffn, n_expert, n_sel, shared, down, n = case
    if chained:
        n = 2   # x_1 = y_0; a third layer would overflow fp32 without a norm
    print(f"[moe-stack] plain {case} chained={chained}", flush=True)
    st = Stack(hip, hidden, ffn, n_expert, n_sel, shared, down, n, seed=hidden + ffn + n_expert, chained=chained)
    a, b = st.outputs(hip), st.outputs(hip)
    s = st.make(hip, a)
    s.run(st.x)
    st.layer_by_layer(hip, b)
    hip.sync()
    compare(st, a, b)
    # a second run on the same table gives the same bits (tags advance by n)
    s.run(st.x)
    hip.sync()
    compare(st, a, b)
    s.destroy()


@pytest.mark.parametrize("scale", [None, 0.5], ids=["no_delta", "delta"])
@pytest.mark.parametrize("case", NORMED, ids=[cid(c) for c in NORMED])
def test_normed_stack_matches_layer_by_layer(hip, case, scale):
    hidden, ffn, n_expert, n_sel, shared, down, n = case
    print(f"[moe-stack] normed {case} scale={scale}", flush=True)
    st = Stack(hip, hidden, ffn, n_expert, n_sel, shared, down, n, seed=7 + hidden + ffn, normed=True)
    a, b = st.outputs(hip), st.outputs(hip)
    s = st.make(hip, a)
    s.run(st.x, delta=st.delta if scale is not None else None, scale=scale if scale is not None else 1.0)
    st.layer_by_layer(hip, b, scale=scale)
    hip.sync()
    compare(st, a, b)
    # layer 0's x_out: the residual entering its norm (x, or x + scale * delta)
    H = hidden
    x = st.x.download(np.float32, H)
    want = x if scale is None else (x + np.float32(scale) * st.delta.download(np.float32, H)).astype(np.float32)
    got = a[0]["x_out"].download(np.float32, H)
    if scale is None:
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    else:
        assert np.array_equal(got.view(np.uint32), b[0]["x_out"].download(np.uint32, H))
    s.destroy()


@pytest.mark.parametrize("case", OTHER, ids=[cid(c) + ("_normed" if c[7] else "") for c in OTHER])
def test_stack_layer_by_layer_shapes(hip, case):
    hidden, ffn, n_expert, n_sel, shared, down, n, normed = case
    print(f"[moe-stack] other {case}", flush=True)
    st = Stack(hip, hidden, ffn, n_expert, n_sel, shared, down, n, seed=11 + hidden, normed=normed)
    a, b = st.outputs(hip), st.outputs(hip)
    s = st.make(hip, a)
    s.run(st.x)
    st.layer_by_layer(hip, b)
    hip.sync()
    compare(st, a, b)
    s.destroy()


def test_stack_with_one_launch_layers_off(hip, monkeypatch):
    """KATALI_HIP_XCD=0: the stack runs kernels A and B layer by layer,
    bit-identical to the single-layer calls under the same switch."""
    monkeypatch.setenv("KATALI_HIP_XCD", "0")
    st = Stack(hip, 2048, 768, 128, 8, False, Q6_K, 3, seed=5, normed=True)
    a, b = st.outputs(hip), st.outputs(hip)
    s = st.make(hip, a)
    s.run(st.x)
    st.layer_by_layer(hip, b)
    hip.sync()
    compare(st, a, b)
    s.destroy()


def test_stack_first_layers_against_oracle(hip, oracle):
    """Layers 0 and 1 of a plain stack against the oracle's q8 path, layer 1
    on the GPU's y of layer 0 (the chain's input)."""
    hidden, ffn, n_expert, n_sel = 1024, 256, 64, 8
    rng = np.random.default_rng(3)
    mats, devs, lgs = [], [], []
    for li in range(2):   # block scales that keep y_0 of x_0's order (h's q8_1 scale is f16)
        g = S.matrix(rng, Q4_K, n_expert * ffn, hidden, 1e-3)
        u = S.matrix(rng, Q4_K, n_expert * ffn, hidden, 1e-3)
        d = S.matrix(rng, Q6_K, n_expert * hidden, ffn, 4e-7)
        mats.append(oracle.moe_desc(hidden, ffn, n_expert, g, u, d))
        devs.append((hip.to_device(g), hip.to_device(u), hip.to_device(d)))
        lgs.append(rng.standard_normal(n_expert).astype(np.float32))
    x = S.activation(rng, hidden)
    desc = hip.moe_desc(hidden, ffn, n_expert, *devs[0])
    ys = [hip.alloc(hidden * 4) for _ in range(2)]
    dl = [hip.to_device(v) for v in lgs]
    entries = [{"gate": devs[i][0], "up": devs[i][1], "down": devs[i][2], "y": ys[i],
                "route": hip.moe_route(n_sel, logits=dl[i])} for i in range(2)]
    s = hip.moe_stack(desc, n_sel, entries)
    s.run(hip.to_device(x))
    hip.sync()
    y0, y1 = ys[0].download(np.float32), ys[1].download(np.float32)
    ids0, w0 = oracle.router_topk(lgs[0], n_sel)
    ids1, w1 = oracle.router_topk(lgs[1], n_sel)
    assert np.isfinite(y0).all() and np.isfinite(y1).all() and np.abs(y1).max() > 0
    r0 = rel_l2(y0, oracle.moe_layer_q8(mats[0], x, ids0, w0))
    r1 = rel_l2(y1, oracle.moe_layer_q8(mats[1], y0, ids1, w1))
    print(f"rel_L2 vs oracle q8: layer 0 {r0:.2e}, layer 1 {r1:.2e}")
    assert r0 <= 1e-5 and r1 <= 1e-5
    s.destroy()


def test_stack_graph_replays(hip):
    """A captured stack replays bit-equal to its eager run, with eager work
    (single-layer calls on the same scratch) between the replays."""
    st = Stack(hip, 2048, 768, 128, 8, False, Q6_K, 4, seed=9, normed=True)
    a, b = st.outputs(hip), st.outputs(hip)
    s = st.make(hip, a)
    s.run(st.x)
    hip.sync()
    want = [words(o["y"], st.hidden) for o in a]
    hip.graph_begin()
    s.run(st.x)
    g = hip.graph_end()
    try:
        for rep in range(4):
            for o in a:
                hip.memset(o["y"], 0, st.hidden * 4)
            hip.graph_launch(g)
            st.layer_by_layer(hip, b)
            hip.sync()
            for li, o in enumerate(a):
                assert np.array_equal(words(o["y"], st.hidden), want[li]), f"replay {rep} layer {li}"
            compare(st, a, b)
    finally:
        hip.graph_destroy(g)
        s.destroy()


def test_stack_bad_arguments(hip):
    st = Stack(hip, 1024, 256, 64, 8, False, Q6_K, 2, seed=13)
    a = st.outputs(hip)
    with pytest.raises(HipError):   # n_sel of a route not the stack's
        e = [{"gate": L["gate"], "up": L["up"], "down": L["down"], "y": o["y"],
              "route": hip.moe_route(4, logits=L["logits"])} for L, o in zip(st.layers, a)]
        hip.moe_stack(st.desc, 8, e)
    with pytest.raises(HipError):   # layer 1's y is layer 0's
        e = [{"gate": L["gate"], "up": L["up"], "down": L["down"], "y": a[0]["y"],
              "route": hip.moe_route(8, logits=L["logits"])} for L in st.layers]
        hip.moe_stack(st.desc, 8, e)
    with pytest.raises(HipError):   # the normed stack needs norm weights and a router
        e = [{"gate": L["gate"], "up": L["up"], "down": L["down"], "y": o["y"]} for L, o in zip(st.layers, a)]
        hip.moe_stack(st.desc, 8, e, normed=True)
    s = st.make(hip, a)
    with pytest.raises(HipError):   # the plain stack takes no delta
        s.run(st.x, delta=st.delta)
    with pytest.raises(HipError):   # layer 0's output is its input
        s.run(a[0]["y"])
    s.destroy()
