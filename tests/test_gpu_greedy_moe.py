"""Greedy decode of a routed MoE model, token by token, GPU against the
oracle's q8_1 CPU path.

Model: embedding -> 4 x (residual add, RMSNorm, F32 router, top-8 of 128
experts, gate/up 2048 -> 768 Q4_K, down Q6_K) -> residual add, output RMSNorm
-> Q6_K LM head (vocab 8192) -> greedy argmax; 32 decode steps, each arm
feeding its own previous token. The GPU runs the chain on the device in the
engine's order (katali_hip_rmsnorm_matvec_f32, katali_hip_moe_layer routed
from those logits, katali_hip_add_rmsnorm, the q8_1 head, katali_hip_argmax)
and, as a second arm, as the normed stack (katali_hip_moe_stack_run, one
launch for the four layers), which must give the same logits bit for bit.
Against the oracle: the GPU and the oracle follow the same q8_1 path but sum
the down projection in another fp32 order, and from the second layer on
that difference can flip a q8_1 rounding (or a block's f16 scale) of x or
h, a jump of one step. So while the histories agree, every head logit and
every router logit must lie within an a-priori bound built from the q8_1
step sizes alone (routed_bounds: every rounding counted as a possible
error of its step's variance, 8 standard deviations, as test_gpu_sample's
fp32_logit_bound for dense layers, extended to the routed slots and the
routing weights' sensitivity to the router logits), and the routing must be
identical unless the oracle's router-logit margin at the top-8 cut is
within that bound. Tokens must be identical, unless the oracle's top-2
head-logit margin is within the bound of the two logits; the first such
step is reported and the arms then follow different tokens."""
import numpy as np
import pytest

import kq_synth as S
from oracle import Q4_K, Q6_K

pytestmark = pytest.mark.gpu

EPS = 1e-6
L, H, F, E, K, V = 4, 2048, 768, 128, 8, 8192
STEPS = 32


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


class Model:
    def __init__(self, hip, oracle, seed):
        rng = np.random.default_rng(seed)
        self.emb = (rng.standard_normal((V, H)) * 2).astype(np.float32)
        self.layers, self.host = [], []
        for _ in range(L):
            g = S.matrix(rng, Q4_K, E * F, H)
            u = S.matrix(rng, Q4_K, E * F, H)
            d = S.matrix(rng, Q6_K, E * H, F)
            self.host.append((g, u, d))
            dev = [hip.to_device(g), hip.to_device(u), hip.to_device(d)]
            router = (rng.standard_normal((E, H)) * 0.05).astype(np.float32)
            norm_w = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
            self.layers.append(dict(
                dev=dev, router=router, norm_w=norm_w, d_router=hip.to_device(router),
                d_norm_w=hip.to_device(norm_w), desc=hip.moe_desc(H, F, E, *dev),
                odesc=oracle.moe_desc(H, F, E, g, u, d), xn=hip.alloc(H * 4), logits=hip.alloc(E * 4),
                y=hip.alloc(H * 4), x_out=hip.alloc(H * 4), ids=hip.alloc(64), wts=hip.alloc(64)))
        self.out_norm_w = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
        self.head = S.matrix(rng, Q6_K, V, H)
        self.d_out_norm_w, self.d_head = hip.to_device(self.out_norm_w), hip.to_device(self.head)


class GpuArm:
    """The chain on the device; stacked: the four layers as the normed stack."""

    def __init__(self, hip, m, stacked):
        self.hip, self.m, self.stacked = hip, m, stacked
        self.x = hip.alloc(H * 4)
        self.xpp = [hip.alloc(H * 4), hip.alloc(H * 4)]
        self.xn_out, self.logits, self.tok = hip.alloc(H * 4), hip.alloc(V * 4), hip.alloc(4)
        self.stack = None
        if stacked:
            self.ys = [hip.alloc(H * 4) for _ in range(L)]
            self.stack = hip.moe_stack(m.layers[0]["desc"], K, [
                {"gate": ly["dev"][0], "up": ly["dev"][1], "down": ly["dev"][2], "y": self.ys[i],
                 "norm_w": ly["d_norm_w"], "router": ly["d_router"], "x_out": ly["x_out"], "xn_out": ly["xn"],
                 "logits_out": ly["logits"],
                 "route": hip.moe_route(K, ids_out=ly["ids"], weights_out=ly["wts"])}
                for i, ly in enumerate(m.layers)], normed=True, eps=EPS)

    def step(self, tok):
        hip, m = self.hip, self.m
        self.x.upload(m.emb[tok])
        if self.stacked:
            self.stack.run(self.x)
            last, y_last = m.layers[L - 1]["x_out"], self.ys[L - 1]
        else:
            cur = self.x
            for i, ly in enumerate(m.layers):
                nxt = self.xpp[i % 2] if i else None
                hip.rmsnorm_matvec_f32(cur, m.layers[i - 1]["y"] if i else None, 1.0, nxt, ly["d_norm_w"], H, EPS,
                                       ly["xn"], ly["d_router"], E, ly["logits"])
                hip.moe_layer(ly["desc"], hip.moe_route(K, logits=ly["logits"], ids_out=ly["ids"],
                                                        weights_out=ly["wts"]), ly["y"], x=ly["xn"])
                if i:
                    cur = nxt
            last, y_last = cur, m.layers[L - 1]["y"]
        hip.add_rmsnorm(last, y_last, 1.0, m.d_out_norm_w, H, EPS, self.xn_out)
        hip.matvec_dp4a(Q6_K, m.d_head, V, H, self.xn_out, self.logits)
        hip.argmax(self.logits, V, self.tok)
        hip.sync()
        ids = [ly["ids"].download(np.int32, K) for ly in m.layers]
        return int(self.tok.download(np.int32)[0]), self.logits.download(np.float32), ids

    def close(self):
        if self.stack:
            self.stack.destroy()


def oracle_step(oracle, m, tok):
    """The q8_1 CPU path; also each layer's router-logit margin at the cut."""
    x = m.emb[tok].copy()
    ids_all, cut = [], []
    for i, ly in enumerate(m.layers):
        if i == 0:
            xn = oracle.rmsnorm(x, ly["norm_w"], EPS)
        else:
            x, xn = oracle.add_rmsnorm(x, y, 1.0, ly["norm_w"], EPS)
        lg = oracle.matvec_f32x(0, ly["router"], E, H, xn)
        ids, w = oracle.router_topk(lg, K)
        srt = np.sort(lg)[::-1]
        cut.append((float(srt[K - 1] - srt[K]), float(np.max(np.abs(lg)))))
        ids_all.append(ids)
        y = oracle.moe_layer_q8(ly["odesc"], xn, ids, w)
    x, xn = oracle.add_rmsnorm(x, y, 1.0, m.out_norm_w, EPS)
    head = oracle.matvec_q8(Q6_K, m.head, V, H, oracle.quantize_q8_1(xn))
    return oracle.argmax_greedy(head), head, ids_all, cut


SIGMAS = 8.0
FP32_SUM = 2.0 * 2.0 ** -48


def q8_var(v):
    """Variance of the q8_1 rounding error of each value of v (step d^2 / 12
    plus the f16 of d, (2^-11 |v|)^2 / 3)."""
    v = np.abs(np.asarray(v, np.float64))
    d = np.repeat(v.reshape(-1, 32).max(axis=1) / 127.0, 32)
    return d * d / 12.0 + (2.0 ** -11 * v) ** 2 / 3.0


class Dequant:
    """float64 rows of the experts a step touches, and the head."""

    def __init__(self, oracle, m):
        self.oracle, self.m, self.cache = oracle, m, {}
        self.W = oracle.dequant(Q6_K, m.head, V * H).astype(np.float64).reshape(V, H)
        self.R = [ly["router"].astype(np.float64) for ly in m.layers]

    def expert(self, li, e):
        key = (li, e)
        if key not in self.cache:
            g, u, d = self.m.host[li]
            rg, rd = H // 256 * 144, F // 256 * 210
            de = lambda t, a, rows, cols, rb: self.oracle.dequant(  # noqa: E731
                t, a[e * rows * rb:(e + 1) * rows * rb], rows * cols).astype(np.float64).reshape(rows, cols)
            self.cache[key] = (de(Q4_K, g, F, H, rg), de(Q4_K, u, F, H, rg), de(Q6_K, d, H, F, rd))
        return self.cache[key]


def routed_bounds(oracle, m, A, tok):
    """For one step of token tok: the bound on each head logit and on each
    layer's router logits, as the module docstring states. The oracle's own
    q8_1 path gives the values and scales."""
    x = m.emb[tok].copy()
    vx = np.zeros(H)
    rb = []
    for li, ly in enumerate(m.layers):
        if li == 0:
            xn = oracle.rmsnorm(x, ly["norm_w"], EPS)
        else:
            x, xn = oracle.add_rmsnorm(x, y, 1.0, ly["norm_w"], EPS)
        r = np.sqrt(np.mean(x.astype(np.float64) ** 2) + EPS)
        vxn = vx * (ly["norm_w"].astype(np.float64) / r) ** 2
        R2 = A.R[li] ** 2
        x2 = xn.astype(np.float64) ** 2
        vl = R2 @ vxn + FP32_SUM * H * (R2 @ x2)   # router logits
        rb.append(SIGMAS * np.sqrt(vl))
        lg = oracle.matvec_f32x(0, ly["router"], E, H, xn)
        ids, w = oracle.router_topk(lg, K)
        y, g, u, hq = oracle.moe_layer_q8(ly["odesc"], xn, ids, w, with_stages=True)
        vin = vxn + q8_var(xn)
        w64 = w.astype(np.float64)
        vw = np.array([sum((w64[s] * ((s == j) - w64[j])) ** 2 * vl[ids[j]] for j in range(K)) for s in range(K)])
        vy = np.zeros(H)
        for s, e in enumerate(ids):
            G, U, D = A.expert(li, int(e))
            gs, us = g[s].astype(np.float64), u[s].astype(np.float64)
            sig = 0.5 * (1.0 + np.tanh(0.5 * gs))
            sg = gs * sig
            a = sig * (1.0 + gs * (1.0 - sig)) * us
            G2, U2, D2 = G * G, U * U, D * D
            vg = G2 @ vin + FP32_SUM * H * (G2 @ x2)
            vu = U2 @ vin + FP32_SUM * H * (U2 @ x2)
            h = sg * us
            vh = a * a * vg + sg * sg * vu + 2.0 * a * sg * ((G * U) @ vin) + (1e-6 * h) ** 2 + q8_var(h)
            ys = D @ h
            vy += w64[s] ** 2 * (D2 @ vh + FP32_SUM * F * (D2 @ (h * h))) + vw[s] * ys * ys
        vx = vx + vy
    x, xn = oracle.add_rmsnorm(x, y, 1.0, m.out_norm_w, EPS)
    r = np.sqrt(np.mean(x.astype(np.float64) ** 2) + EPS)
    vin = vx * (m.out_norm_w.astype(np.float64) / r) ** 2 + q8_var(xn)
    W2 = A.W ** 2
    return SIGMAS * np.sqrt(W2 @ vin + FP32_SUM * H * (W2 @ xn.astype(np.float64) ** 2)), rb


def margin(lg):
    top2 = np.sort(lg)[-2:]
    return float(top2[1] - top2[0])


def test_routed_greedy_decode_token_identical(hip, oracle):
    m = Model(hip, oracle, seed=2026)
    A = Dequant(oracle, m)
    arms = [GpuArm(hip, m, stacked=False), GpuArm(hip, m, stacked=True)]
    try:
        gtok = ctok = 7
        gseq, cseq = [], []
        diverged = None
        for s in range(STEPS):
            print(f"[greedy-moe] step {s}", flush=True)
            (gt, gl, gids), (st, sl, sids) = arms[0].step(gtok), arms[1].step(gtok)
            # the stacked arm: the same computation, bit for bit
            assert st == gt and np.array_equal(sl.view(np.uint32), gl.view(np.uint32)), f"step {s}: stack"
            assert all(np.array_equal(a, b) for a, b in zip(sids, gids)), f"step {s}: stack routing"
            ct, cl, cids, cut = oracle_step(oracle, m, ctok)
            gseq.append(gt)
            cseq.append(ct)
            if diverged is None:
                # same history: every logit within the a-priori bound, routing
                # identical unless within that bound at the cut
                hb, rbs = routed_bounds(oracle, m, A, ctok)
                for i in range(L):
                    if not np.array_equal(gids[i], cids[i]):
                        print(f"step {s} layer {i}: routing {gids[i].tolist()} vs {cids[i].tolist()}, router "
                              f"margin at the cut {cut[i][0]:.3e}, bound {2 * rbs[i].max():.3e}")
                        assert cut[i][0] <= 2 * rbs[i].max(), f"step {s} layer {i}: routing differs beyond the bound"
                        diverged = s
                        break
                if diverged is None:
                    d = np.abs(gl.astype(np.float64) - cl)
                    worst = int(np.argmax(d / hb))
                    print(f"step {s}: token {gt} / {ct}, head rel_L2 {rel_l2(gl, cl):.2e}, max |gpu - q8| / bound "
                          f"{d[worst] / hb[worst]:.3f}, top-2 margin {margin(cl):.3e}")
                    assert np.all(d <= hb), f"step {s}: logit {worst} off by {d[worst]:.3e}, bound {hb[worst]:.3e}"
                    if gt != ct:
                        allowed = float(hb[gt] + hb[ct])
                        print(f"step {s}: first divergence, GPU {gt} vs q8 path {ct}: margin {margin(cl):.3e}, "
                              f"bound of the two logits {allowed:.3e}")
                        assert margin(cl) <= allowed, f"step {s}: tokens differ beyond the bound"
                        diverged = s
            gtok, ctok = gt, ct
        print(f"GPU tokens : {gseq}")
        print(f"q8 CPU path: {cseq}")
        print(f"first divergence: {'none' if diverged is None else diverged}")
        assert len(set(gseq)) > 1, "degenerate decode (one token repeated)"
        if diverged is None:
            assert gseq == cseq
    finally:
        for a in arms:
            a.close()
