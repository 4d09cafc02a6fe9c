"""GPU: a MoE model's tensors from a GGUF file onto the device and through
the fused path. A synthetic qwen3moe-named GGUF (expert stacks Q4_K/Q6_K in
GGUF layout, F32 routers and norms, a shared expert on one layer, Q6_K LM
head) is opened by the library's reader; the weight cache uploads each tensor
once; the MoE layers assembled from the tensor names run the whole decode
token on the device and match the oracle on the same tensors as written.
The expert VRAM tier (per-expert slots, least recently used out) gives the
same bits as the fully resident layer and the hits and misses of an LRU model.
"""
import numpy as np
import pytest

import kq_synth as S
from gguf_models import build_gguf
from katali_hip_gguf import ExpertTier, Gguf, GgufError, Weights
from oracle import Q4_K, Q6_K

pytestmark = pytest.mark.gpu

EPS = 1e-6


class View:
    def __init__(self, ptr):
        self.ptr = ptr


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    p = tmp_path_factory.mktemp("gguf") / "moe.gguf"
    return str(p), build_gguf(str(p))


def test_gguf_decode_token_matches_oracle(hip, oracle, model):
    path, H = model
    print(f"[gguf] decode token from {path}", flush=True)
    L, h, E, k, vocab = H["L"], H["hidden"], H["E"], H["n_sel"], H["vocab"]
    g = Gguf(path)
    wts = Weights(g)
    try:
        layers = [wts.moe_layer(li) for li in range(L)]
        assert wts.moe_layer(0)[0].gate_exps == layers[0][0].gate_exps      # cached, not uploaded twice
        head, onw = wts.get("output.weight"), wts.get("output_norm.weight")
        want_bytes = sum(t["nbytes"] for t in g.tensors())
        assert wts.resident == want_bytes
        assert layers[1][0].gate_shexp and not layers[0][0].gate_shexp
        x0 = (np.random.default_rng(9).standard_normal(h) * 2).astype(np.float32)
        x, xpp = hip.to_device(x0), [hip.alloc(h * 4), hip.alloc(h * 4)]
        xn = [hip.alloc(h * 4) for _ in range(L)]
        logits = [hip.alloc(E * 4) for _ in range(L)]
        ys = [hip.alloc(h * 4) for _ in range(L)]
        ids = [hip.alloc(64 * 4) for _ in range(L)]
        xo, hl, tok = hip.alloc(h * 4), hip.alloc(vocab * 4), hip.alloc(4)
        cur = x
        for li, (m, router, norm) in enumerate(layers):
            if li == 0:
                hip.rmsnorm_matvec_f32(cur, None, 1.0, None, View(norm), h, EPS, xn[li], View(router), E, logits[li])
            else:
                hip.rmsnorm_matvec_f32(cur, ys[li - 1], 1.0, xpp[li % 2], View(norm), h, EPS, xn[li], View(router),
                                       E, logits[li])
                cur = xpp[li % 2]
            hip.moe_layer(m, hip.moe_route(k, logits=logits[li], ids_out=ids[li]), ys[li], x=xn[li])
        hip.add_rmsnorm(cur, ys[L - 1], 1.0, View(onw), h, EPS, xo)
        hip.matvec(Q6_K, View(head), vocab, h, xo, hl)
        hip.argmax(hl, vocab, tok)
        hip.sync()

        xr = x0
        for li, ly in enumerate(H["layers"]):
            if li == 0:
                want_xn = oracle.rmsnorm(xr, ly["norm"], EPS)
            else:
                xr, want_xn = oracle.add_rmsnorm(xr, ys[li - 1].download(np.float32), 1.0, ly["norm"], EPS)
            got_xn = xn[li].download(np.float32)
            assert np.array_equal(got_xn.view(np.uint32), want_xn.view(np.uint32)), li
            lg = logits[li].download(np.float32)
            assert np.array_equal(lg.view(np.uint32), oracle.matvec_f32x(0, ly["router"], E, h, got_xn).view(np.uint32))
            sel, wsel = oracle.router_topk(lg, k)
            assert ids[li].download(np.int32)[:k].tolist() == sel.tolist()
            od = oracle.moe_desc(h, H["ffn"], E, ly["g"], ly["u"], ly["d"], shared=ly["sh"])
            r = rel_l2(ys[li].download(np.float32), oracle.moe_layer_q8(od, got_xn, sel, wsel))
            print(f"layer {li}: experts {sel.tolist()} rel_L2 {r:.2e}", flush=True)
            assert r <= 1e-5
        xr, want_o = oracle.add_rmsnorm(xr, ys[L - 1].download(np.float32), 1.0, H["out_norm"], EPS)
        assert np.array_equal(xo.download(np.uint32, h), want_o.view(np.uint32))
        lh = hl.download(np.float32)
        assert rel_l2(lh, oracle.matvec_f32x(Q6_K, H["head"], vocab, h, want_o)) <= 1e-5
        assert int(tok.download(np.int32)[0]) == oracle.argmax_greedy(lh)
    finally:
        wts.destroy()
        g.close()


def test_gguf_weight_budget_refuses(hip, model):
    path, H = model
    g = Gguf(path)
    wts = Weights(g, budget=1 << 20)   # 1 MiB: not even one expert stack
    try:
        with pytest.raises(GgufError, match="budget"):
            wts.moe_layer(0)
        assert wts.resident == 0
        assert wts.get("blk.0.ffn_norm.weight")     # a small tensor still fits
    finally:
        wts.destroy()
        g.close()


def lru_model(n_slots, calls, picks=None):
    """Hits and misses of the tier's rule (least recently used slot not asked
    for in the same call, the lowest slot among equals); picks, when given,
    gets each call's slot numbers."""
    slots = [(-1, 0)] * n_slots
    hits = misses = 0
    for tick, (layer, ids) in enumerate(calls, 1):
        got = []
        for e in ids:
            key = layer * 65536 + e
            s = next((i for i, (kk, _) in enumerate(slots) if kk == key), None)
            if s is not None:
                hits += 1
            else:
                misses += 1
                cand = [i for i, (_, u) in enumerate(slots) if u != tick]
                s = min(cand, key=lambda i: (slots[i][1], i))
            slots[s] = (key, tick)
            got.append(s)
        if picks is not None:
            picks.append(got)
    return hits, misses


def test_expert_tier_matches_resident_layer(hip, oracle, model):
    path, H = model
    L, h, ffn, E, k = H["L"], H["hidden"], H["ffn"], H["E"], H["n_sel"]
    g = Gguf(path)
    wts = Weights(g)
    per = ffn * (h // 256 * 144) * 2 + h * (ffn // 256 * 210)
    tier = ExpertTier(g, 0, budget=6 * per + per // 2, max_slots=64)
    try:
        assert tier.stats()["n_slots"] == 6
        rng = np.random.default_rng(4)
        x = hip.to_device(S.activation(rng, h))
        y_res, y_tier = hip.alloc(h * 4), hip.alloc(h * 4)
        calls = []
        for t in range(12):
            for li in range(L):
                sel = rng.choice(E, k, replace=False).astype(np.int32)
                wsel = rng.dirichlet(np.ones(k)).astype(np.float32)
                print(f"[tier] token {t} layer {li} experts {sel.tolist()}", flush=True)
                calls.append((li, sel.tolist()))
                m_res = wts.moe_layer(li)[0]
                m_res.gate_shexp = m_res.up_shexp = m_res.down_shexp = None   # routed experts only
                m_tier, slots = tier.layer(li, sel.tolist())
                assert sorted(set(slots)) == sorted(slots) and max(slots) < 6
                dw = hip.to_device(wsel)
                hip.moe_layer(m_res, hip.moe_route(k, ids=hip.to_device(sel), weights=dw), y_res, x=x)
                hip.moe_layer(m_tier, hip.moe_route(k, ids=hip.to_device(np.array(slots, np.int32)), weights=dw),
                              y_tier, x=x)
                hip.sync()
                assert np.array_equal(y_res.download(np.uint32, h), y_tier.download(np.uint32, h)), (t, li)
        st = tier.stats()
        hits, misses = lru_model(6, calls)
        assert (st["hits"], st["misses"]) == (hits, misses)
        assert st["uploaded_bytes"] == misses * per
        with pytest.raises(GgufError):
            tier.layer(0, list(range(7)))      # more experts than slots
        with pytest.raises(GgufError):
            tier.layer(0, [E])                 # id outside the layer
    finally:
        tier.destroy()
        wts.destroy()
        g.close()


@pytest.mark.parametrize("chunk", [64 << 10, 4 << 20])
def test_expert_tier_pipelined_matches_resident_layer(hip, oracle, model, chunk):
    """Pipelined uploads with as many slots as experts per call, so every
    call's misses refill slots the kernel queued just before still reads:
    no host synchronisation between calls (ids, weights and slot numbers are
    on the device beforehand, the slot numbers from the LRU model), each
    upload must wait for that kernel on the device, and the layer after it
    for the upload. Every call's output equals the resident layer's, bit for
    bit. Some calls repeat the previous call's experts (all hits, no
    uploads), so the next misses must also wait for the kernels of calls
    that took no mark. 64 KiB chunks wrap the three-chunk ring inside one
    expert (and are copied by the calling thread alone); 4 MiB chunks are
    copied by the worker threads too."""
    path, H = model
    L, h, ffn, E, k = H["L"], H["hidden"], H["ffn"], H["E"], H["n_sel"]
    g = Gguf(path)
    wts = Weights(g)
    per = ffn * (h // 256 * 144) * 2 + h * (ffn // 256 * 210)
    tier = ExpertTier(g, 0, budget=k * per + per // 2, max_slots=64)
    try:
        assert tier.stats()["n_slots"] == k
        tier.pipeline(chunk_bytes=chunk, n_chunks=3)
        rng = np.random.default_rng(5)
        calls, wsel = [], []
        for t in range(6):
            for li in range(L):
                calls.append((li, rng.choice(E, k, replace=False).astype(np.int32).tolist()))
                wsel.append(rng.dirichlet(np.ones(k)).astype(np.float32))
                if t % 2 == 0:   # the same experts again: all hits, a call that takes no mark
                    calls.append(calls[-1])
                    wsel.append(rng.dirichlet(np.ones(k)).astype(np.float32))
        picks = []
        hits, misses = lru_model(k, calls, picks)
        x = hip.to_device(S.activation(rng, h))
        sdev = [hip.to_device(np.array(p, np.int32)) for p in picks]
        wdev = [hip.to_device(w) for w in wsel]
        ys = [hip.alloc(h * 4) for _ in calls]
        hip.sync()
        print(f"[tier pipelined] chunk {chunk}: {len(calls)} calls, {misses} misses, no sync between them", flush=True)
        for i, (li, sel) in enumerate(calls):
            m_tier, slots = tier.layer(li, sel)
            assert slots == picks[i], i
            hip.moe_layer(m_tier, hip.moe_route(k, ids=sdev[i], weights=wdev[i]), ys[i], x=x)
        hip.sync()
        st = tier.stats()
        assert (st["hits"], st["misses"]) == (hits, misses)
        y_res = hip.alloc(h * 4)
        for i, (li, sel) in enumerate(calls):
            m_res = wts.moe_layer(li)[0]
            m_res.gate_shexp = m_res.up_shexp = m_res.down_shexp = None   # routed experts only
            hip.moe_layer(m_res, hip.moe_route(k, ids=hip.to_device(np.array(sel, np.int32)), weights=wdev[i]),
                          y_res, x=x)
            hip.sync()
            assert np.array_equal(y_res.download(np.uint32, h), ys[i].download(np.uint32, h)), (i, li, sel)
    finally:
        tier.destroy()
        wts.destroy()
        g.close()
