"""GPU parity: one decode token of a MoE model's FFN chain, all on the device,
eager and as one captured graph (attention is outside the path):

  x0 -> RMSNorm -> router logits (F32 matvec) -> MoE layer (routing on device)
     -> residual + RMSNorm -> ... (L layers) -> residual + output RMSNorm
     -> Q6_K LM head -> greedy argmax

The engine's order of these steps is gguf_model.c:677-701 (residual add,
norm, FFN; final norm, LM head, sampler). Each stage is checked on the GPU's
own input to it: norms, residuals and router logits bit-identical to the
oracle, routing ids and weights bit-identical, MoE outputs within the
layer's q8 bar, the LM head within rel_L2 1e-5 (fp32 dots in another
order), the token equal to the
oracle's argmax of the GPU's logits. Graph replays reproduce the eager bits.
Run twice: with separate norm and router launches, and with the fused
residual + norm + router launch (residual stream in two buffers).
"""
import numpy as np
import pytest

import kq_synth as S
from oracle import Q4_K, Q6_K

pytestmark = pytest.mark.gpu

EPS = 1e-6


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


class Chain:
    def __init__(self, hip, oracle, L, hidden, ffn, n_expert, n_sel, shared, vocab, seed, fused=False):
        rng = np.random.default_rng(seed)
        self.L, self.hidden, self.n_expert, self.n_sel, self.vocab = L, hidden, n_expert, n_sel, vocab
        self.layers = []
        for _ in range(L):
            g = S.matrix(rng, Q4_K, n_expert * ffn, hidden)
            u = S.matrix(rng, Q4_K, n_expert * ffn, hidden)
            d = S.matrix(rng, Q6_K, n_expert * hidden, ffn)
            sh = dsh = None
            if shared:
                sh = (ffn, S.matrix(rng, Q4_K, ffn, hidden), S.matrix(rng, Q4_K, ffn, hidden),
                      S.matrix(rng, Q6_K, hidden, ffn))
                dsh = tuple(hip.to_device(a) for a in sh[1:])
            dev = [hip.to_device(g), hip.to_device(u), hip.to_device(d)]
            router = (rng.standard_normal((n_expert, hidden)) * 0.05).astype(np.float32)
            norm_w = (1.0 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)
            self.layers.append(dict(
                host=(g, u, d, sh), dev=dev, dsh=dsh, router=router, norm_w=norm_w,
                desc=hip.moe_desc(hidden, ffn, n_expert, *dev, shared=dsh),
                odesc=oracle.moe_desc(hidden, ffn, n_expert, g, u, d, shared=sh),
                d_router=hip.to_device(router), d_norm_w=hip.to_device(norm_w),
                xn=hip.alloc(hidden * 4), logits=hip.alloc(n_expert * 4), y=hip.alloc(hidden * 4),
                ids=hip.alloc(64 * 4), wts=hip.alloc(64 * 4)))
        self.out_norm_w = (1.0 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)
        self.head = S.matrix(rng, Q6_K, vocab, hidden)
        self.d_out_norm_w, self.d_head = hip.to_device(self.out_norm_w), hip.to_device(self.head)
        self.fused = fused
        self.x = hip.alloc(hidden * 4)
        self.xpp = [hip.alloc(hidden * 4), hip.alloc(hidden * 4)]   # residual ping-pong (fused)
        self.xn_out = hip.alloc(hidden * 4)
        self.head_logits = hip.alloc(vocab * 4)
        self.tok = hip.alloc(4)
        self.x0 = (rng.standard_normal(hidden) * 2).astype(np.float32)

    def enqueue(self, hip):
        """The token's launches, in order, on the library stream."""
        if self.fused:
            return self.enqueue_fused(hip)
        h = self.hidden
        for i, ly in enumerate(self.layers):
            if i == 0:
                hip.rmsnorm(self.x, ly["d_norm_w"], h, EPS, ly["xn"])
            else:
                hip.add_rmsnorm(self.x, self.layers[i - 1]["y"], 1.0, ly["d_norm_w"], h, EPS, ly["xn"])
            hip.matvec(0, ly["d_router"], self.n_expert, h, ly["xn"], ly["logits"])
            route = hip.moe_route(self.n_sel, logits=ly["logits"], ids_out=ly["ids"], weights_out=ly["wts"])
            hip.moe_layer(ly["desc"], route, ly["y"], x=ly["xn"])
        hip.add_rmsnorm(self.x, self.layers[-1]["y"], 1.0, self.d_out_norm_w, h, EPS, self.xn_out)
        hip.matvec(Q6_K, self.d_head, self.vocab, h, self.xn_out, self.head_logits)
        hip.argmax(self.head_logits, self.vocab, self.tok)

    def enqueue_fused(self, hip):
        """Residual step, norm and router logits in one launch per layer; the
        residual stream moves between two buffers (x stays the token input)."""
        h, cur = self.hidden, self.x
        for i, ly in enumerate(self.layers):
            if i == 0:
                hip.rmsnorm_matvec_f32(cur, None, 1.0, None, ly["d_norm_w"], h, EPS, ly["xn"], ly["d_router"],
                                       self.n_expert, ly["logits"])
            else:
                nxt = self.xpp[i % 2]
                hip.rmsnorm_matvec_f32(cur, self.layers[i - 1]["y"], 1.0, nxt, ly["d_norm_w"], h, EPS, ly["xn"],
                                       ly["d_router"], self.n_expert, ly["logits"])
                cur = nxt
            route = hip.moe_route(self.n_sel, logits=ly["logits"], ids_out=ly["ids"], weights_out=ly["wts"])
            hip.moe_layer(ly["desc"], route, ly["y"], x=ly["xn"])
        hip.add_rmsnorm(cur, self.layers[-1]["y"], 1.0, self.d_out_norm_w, h, EPS, self.xn_out)
        hip.matvec(Q6_K, self.d_head, self.vocab, h, self.xn_out, self.head_logits)
        hip.argmax(self.head_logits, self.vocab, self.tok)
        self.x_final = cur

    def snapshot(self):
        xf = self.x_final if self.fused else self.x
        out = {"x": xf.download(np.float32), "xn_out": self.xn_out.download(np.float32),
               "head": self.head_logits.download(np.float32), "tok": int(self.tok.download(np.int32)[0])}
        for i, ly in enumerate(self.layers):
            for k in ("xn", "logits", "y", "ids", "wts"):
                dt = np.int32 if k == "ids" else np.float32
                out[f"{k}{i}"] = ly[k].download(dt)
        return out


def check_against_oracle(c, oracle, s):
    x = c.x0
    for i, ly in enumerate(c.layers):
        if i == 0:
            xn = oracle.rmsnorm(x, ly["norm_w"], EPS)
        else:
            x, xn = oracle.add_rmsnorm(x, s[f"y{i - 1}"], 1.0, ly["norm_w"], EPS)
        assert np.array_equal(s[f"xn{i}"].view(np.uint32), xn.view(np.uint32)), f"norm, layer {i}"
        logits = oracle.matvec_f32x(0, ly["router"], c.n_expert, c.hidden, s[f"xn{i}"])
        assert np.array_equal(s[f"logits{i}"].view(np.uint32), logits.view(np.uint32)), f"router, layer {i}"
        ids, w = oracle.router_topk(s[f"logits{i}"], c.n_sel)
        assert s[f"ids{i}"][:c.n_sel].tolist() == ids.tolist(), f"routing, layer {i}"
        assert np.array_equal(s[f"wts{i}"][:c.n_sel].view(np.uint32), w.view(np.uint32)), f"weights, layer {i}"
        y = oracle.moe_layer_q8(ly["odesc"], s[f"xn{i}"], ids, w)
        r = rel_l2(s[f"y{i}"], y)
        print(f"layer {i}: experts {ids.tolist()} rel_L2(y) = {r:.2e}", flush=True)
        # h bit-identical (the q8_1 path's gate/up order); down in its own fp32 order
        assert r <= 1e-5, f"moe, layer {i}"
    x, xn = oracle.add_rmsnorm(x, s[f"y{c.L - 1}"], 1.0, c.out_norm_w, EPS)
    assert np.array_equal(s["x"].view(np.uint32), x.view(np.uint32)), "residual stream"
    assert np.array_equal(s["xn_out"].view(np.uint32), xn.view(np.uint32)), "output norm"
    head = oracle.matvec_f32x(Q6_K, c.head, c.vocab, c.hidden, s["xn_out"])
    # fp32 dots in another order over 2048 terms of up to ~1e3: rel_L2 bar
    r = rel_l2(s["head"], head)
    print(f"LM head rel_L2 = {r:.2e}, max |diff| = {np.max(np.abs(s['head'] - head)):.3g}", flush=True)
    assert r <= 1e-5, "LM head"
    assert s["tok"] == oracle.argmax_greedy(s["head"]), "argmax"


CASES = [
    # L, hidden, ffn, n_expert, n_sel, shared, vocab
    (3, 2048, 768, 16, 8, False, 4096),
    (2, 1024, 512, 32, 3, True, 3000),
]


@pytest.mark.parametrize("fused", [False, True], ids=["separate", "norm_router"])
@pytest.mark.parametrize("case", CASES, ids=["h2048_e16_k8", "h1024_e32_k3_sh"])
def test_decode_chain_eager_and_graph(hip, oracle, case, fused):
    print(f"[decode-chain] case={case} fused={fused}", flush=True)
    c = Chain(hip, oracle, *case, seed=sum(case[:5]), fused=fused)
    c.x.upload(c.x0)
    c.enqueue(hip)
    hip.sync()
    eager = c.snapshot()
    check_against_oracle(c, oracle, eager)

    hip.graph_begin()
    c.enqueue(hip)
    g = hip.graph_end()
    try:
        for rep in range(3):
            c.x.upload(c.x0)            # the residual stream starts over each token
            hip.graph_launch(g)
            hip.sync()
            s = c.snapshot()
            for k, v in eager.items():
                if k == "tok":
                    assert s[k] == v, (rep, k)
                else:
                    assert np.array_equal(np.asarray(s[k]).view(np.uint32), np.asarray(v).view(np.uint32)), (rep, k)
    finally:
        hip.graph_destroy(g)
