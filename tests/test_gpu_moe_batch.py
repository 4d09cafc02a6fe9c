"""GPU parity of the batched MoE layer (ragged token batches, Zipf routing).

Every token's output is checked against the oracle's single-token q8_1 layer
with that token's experts and weights. Each case runs three ways: the
default grouped-GEMM threshold (experts with >= 16 pairs on int8 MFMA), every
expert on MFMA, and every expert on the v_dot4 GEMV kernels. All three form
gate/up in the q8_1 path's order (per-sub-block terms, pairwise), so every
pair's h is bit-identical to the oracle's and every token's output is within
rel_L2 1e-5 of it (the down projections sum in fp32 in their own orders);
the MFMA and GEMV paths agree token by token to the same bar. The cases
include the sweep's own points: 128 experts of the 2048 -> 768 -> 2048 shape
at n_sel 2, 4, 8 and 16, 33, 64 tokens.
"""
import concurrent.futures as cf

import numpy as np
import pytest

import kq_synth as S
from oracle import Q4_K, Q6_K

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("two_launch_layer")]


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def zipf_routes(rng, T, n_expert, n_sel, s=1.1):
    """Per-token experts drawn without replacement from a Zipf(s) popularity
    over a random expert order; weights renormalised over the selection and
    listed largest first."""
    pop = 1.0 / np.arange(1, n_expert + 1) ** s
    pop /= pop.sum()
    order = rng.permutation(n_expert)
    ids = np.empty((T, n_sel), np.int32)
    w = np.empty((T, n_sel), np.float32)
    for t in range(T):
        pick = order[rng.choice(n_expert, n_sel, replace=False, p=pop)]
        lw = rng.standard_normal(n_sel).astype(np.float32)
        ww = np.exp(lw - lw.max())
        ww /= ww.sum()
        o = np.argsort(-ww, kind="stable")
        ids[t], w[t] = pick[o], ww[o].astype(np.float32)
    return ids, w


CASES = [
    # hidden, ffn, n_expert, n_sel, T, shared, down_type
    (2048, 768, 32, 8, 64, False, Q6_K),     # config-1 expert shape, 512 pairs on 32 experts
    (2048, 512, 64, 8, 48, True, Q6_K),      # shared expert: 48 pairs, always grouped
    (1024, 512, 16, 4, 33, True, Q4_K),      # Q4_K down
    (2048, 768, 128, 1, 64, False, Q6_K),    # n_sel 1
    (512, 256, 16, 2, 5, False, Q6_K),       # a short batch: every expert small
    (256, 512, 4, 2, 40, False, Q6_K),       # hidden of one block: one-block gate/up slices
    (4096, 256, 8, 2, 20, False, Q6_K),      # wide hidden
    (1024, 2304, 8, 2, 12, True, Q6_K),      # 9 down blocks: h staged 8 blocks at a time
    (512, 2304, 4, 2, 9, False, Q4_K),       # the same with a Q4_K down
    (512, 6656, 8, 2, 12, False, Q4_K),      # Q4_K down of 26 blocks: the grouped down's block loop
] + [(2048, 768, 128, k, t, False, Q6_K) for k in (2, 4, 8) for t in (16, 33, 64)]   # the sweep's points


@pytest.fixture(scope="module")
def built(hip, oracle):
    cache = {}

    def get(case):
        hidden, ffn, n_expert, n_sel, T, shared, down_type = case
        key = (hidden, ffn, n_expert, shared, down_type)
        if key not in cache:
            rng = np.random.default_rng(hidden + 7 * ffn + n_expert)
            g = S.matrix(rng, Q4_K, n_expert * ffn, hidden)
            u = S.matrix(rng, Q4_K, n_expert * ffn, hidden)
            d = S.matrix(rng, down_type, n_expert * hidden, ffn)
            sh = None
            dsh = None
            if shared:
                sh = (ffn, S.matrix(rng, Q4_K, ffn, hidden), S.matrix(rng, Q4_K, ffn, hidden),
                      S.matrix(rng, down_type, hidden, ffn))
                dsh = tuple(hip.to_device(a) for a in sh[1:])
            dev = [hip.to_device(a) for a in (g, u, d)]
            desc = hip.moe_desc(hidden, ffn, n_expert, *dev, down_type=down_type, shared=dsh)
            odesc = oracle.moe_desc(hidden, ffn, n_expert, g, u, d, down_type=down_type, shared=sh)
            cache[key] = (desc, odesc, dev, dsh, (g, u, d, sh))   # the oracle descriptor points into g, u, d
        return cache[key]
    return get


@pytest.mark.parametrize("case", CASES, ids=[f"h{c[0]}_f{c[1]}_e{c[2]}_k{c[3]}_t{c[4]}{'_sh' if c[5] else ''}"
                                             f"{'_q4down' if c[6] == Q4_K else ''}" for c in CASES])
def test_moe_batch_parity(hip, oracle, built, case):
    hidden, ffn, n_expert, n_sel, T, shared, down_type = case
    print(f"[moe-batch] case={case}", flush=True)
    desc, odesc = built(case)[:2]
    rng = np.random.default_rng(T * 131 + n_sel)
    ids, w = zipf_routes(rng, T, n_expert, n_sel)
    x = rng.standard_normal((T, hidden)).astype(np.float32)
    counts = np.bincount(ids.reshape(-1), minlength=n_expert)
    print(f"pairs per expert: max {counts.max()}, experts with >= 16: {int((counts >= 16).sum())}")
    with cf.ThreadPoolExecutor(8) as ex:   # the oracle's C calls release the GIL
        want = np.stack(list(ex.map(lambda t: oracle.moe_layer_q8(odesc, x[t], ids[t], w[t]), range(T))))
    dids, dw, dx = hip.to_device(ids), hip.to_device(w), hip.to_device(x)
    outs = {}
    for name, thr in (("default", 0), ("all-mfma", 1), ("all-gemv", 1000)):
        y = hip.alloc(T * hidden * 4)
        hip.moe_batch(desc, T, n_sel, dids, dw, dx, y, mfma_min_tokens=thr)
        hip.sync()
        got = y.download(np.float32).reshape(T, hidden)
        tok = [rel_l2(got[t], want[t]) for t in range(T)]
        print(f"{name}: batch rel_L2 {rel_l2(got, want):.2e}, median token {np.median(tok):.2e}, "
              f"worst token {max(tok):.2e}")
        assert max(tok) <= 1e-5
        outs[name] = got
    assert max(rel_l2(outs["all-mfma"][t], outs["all-gemv"][t]) for t in range(T)) <= 1e-5


def test_moe_batch_single_token_matches_layer(hip, oracle, built):
    """T = 1 through the batch entry equals the single-token layer with the
    same explicit experts (both on the GEMV kernels: bit-identical)."""
    case = CASES[0]
    hidden, ffn, n_expert, n_sel = case[:4]
    desc, odesc = built(case)[:2]
    rng = np.random.default_rng(77)
    ids, w = zipf_routes(rng, 1, n_expert, n_sel)
    x = rng.standard_normal((1, hidden)).astype(np.float32)
    dx = hip.to_device(x)
    y1, y2 = hip.alloc(hidden * 4), hip.alloc(hidden * 4)
    hip.moe_batch(desc, 1, n_sel, hip.to_device(ids), hip.to_device(w), dx, y1)
    hip.moe_layer(desc, hip.moe_route(n_sel, ids=hip.to_device(ids[0]), weights=hip.to_device(w[0])), y2, x=dx)
    hip.sync()
    assert np.array_equal(y1.download(np.uint32), y2.download(np.uint32))


def test_moe_batch_rejects_bad_arguments(hip, built):
    from katali_hip import HipError
    case = CASES[4]
    desc = built(case)[0]
    hidden = case[0]
    x, y = hip.alloc(65 * hidden * 4), hip.alloc(65 * hidden * 4)
    ids = hip.to_device(np.zeros((65, 2), np.int32))
    w = hip.to_device(np.ones((65, 2), np.float32))
    for T in (0, 65):
        with pytest.raises(HipError):
            hip.moe_batch(desc, T, 2, ids, w, x, y)
    with pytest.raises(HipError):
        hip.moe_batch(desc, 4, 17, ids, w, x, y)


@pytest.mark.parametrize("T,thr", [(64, 0), (64, 1), (5, 0)], ids=["fork", "fork_all_mfma", "one_stream"])
def test_moe_batch_graph_replays_match_eager(hip, oracle, built, T, thr):
    """One batched layer captured in a graph (two stream branches from 96
    pairs on) replays to the eager call's bits, with eager work between the
    replays."""
    case = CASES[0]
    hidden, ffn, n_expert, n_sel = case[:4]
    print(f"[moe-batch-graph] T={T} thr={thr}", flush=True)
    desc = built(case)[0]
    rng = np.random.default_rng(900 + T + thr)
    ids, w = zipf_routes(rng, T, n_expert, n_sel)
    x = rng.standard_normal((T, hidden)).astype(np.float32)
    dids, dw, dx = hip.to_device(ids), hip.to_device(w), hip.to_device(x)
    want, got = hip.alloc(T * hidden * 4), hip.alloc(T * hidden * 4)
    hip.moe_batch(desc, T, n_sel, dids, dw, dx, want, mfma_min_tokens=thr)
    hip.sync()
    ref = want.download(np.uint32)
    hip.graph_begin()
    hip.moe_batch(desc, T, n_sel, dids, dw, dx, got, mfma_min_tokens=thr)
    g = hip.graph_end()
    other = hip.alloc(T * hidden * 4)
    try:
        for i in range(3):
            hip.memset(got, 0, T * hidden * 4)
            hip.graph_launch(g)
            hip.sync()
            assert np.array_equal(got.download(np.uint32), ref), i
            # eager work between replays, on the same scratch
            hip.moe_batch(desc, T, n_sel, dids, dw, dx, other, mfma_min_tokens=thr)
            hip.sync()
            assert np.array_equal(other.download(np.uint32), ref), i
    finally:
        hip.graph_destroy(g)


def batch_logits(rng, T, E, kind):
    if kind == "ties":
        return rng.integers(-2, 3, (T, E)).astype(np.float32)
    v = rng.standard_normal((T, E)).astype(np.float32)
    if kind == "special":   # NaN ranks as -inf, -0 equals +0
        v[:, ::7] = np.nan
        v[:, 1::11] = -np.inf
        v[:, 2::13] = -0.0
        v[:, 3::13] = 0.0
    return v


ROUTE_BATCH = [(37, 128, 8, "normal"), (64, 256, 8, "ties"), (5, 512, 16, "normal"), (20, 200, 5, "special"),
               (9, 16, 16, "normal"), (3, 64, 1, "special")]


@pytest.mark.parametrize("T,E,k,kind", ROUTE_BATCH, ids=[f"t{c[0]}_e{c[1]}_k{c[2]}_{c[3]}" for c in ROUTE_BATCH])
def test_route_batch_matches_oracle(hip, oracle, T, E, k, kind):
    """Device routing of a prompt's logits: every token's experts and weights
    bit-identical to the oracle router (the single-token layer's routing)."""
    print(f"[route-batch] T={T} E={E} k={k} {kind}", flush=True)
    rng = np.random.default_rng(T * 1000 + E + k)
    logits = batch_logits(rng, T, E, kind)
    ids, w = hip.alloc(T * k * 4), hip.alloc(T * k * 4)
    hip.moe_route_batch(hip.to_device(logits), T, E, k, ids, w)
    got_i = ids.download(np.int32).reshape(T, k)
    got_w = w.download(np.float32).reshape(T, k)
    for t in range(T):
        oi, ow = oracle.router_topk(logits[t], k)
        assert got_i[t].tolist() == oi.tolist(), t
        assert np.array_equal(got_w[t].view(np.uint32), ow.view(np.uint32)), t


def test_prefill_with_device_routing(hip, oracle, built):
    """Prefill on the device end to end: logits -> katali_hip_moe_route_batch
    -> katali_hip_moe_batch gives the bits of the same batch with the
    oracle's routing uploaded."""
    case = CASES[2]
    hidden, ffn, n_expert, n_sel, T = case[:5]
    desc = built(case)[0]
    rng = np.random.default_rng(5)
    logits = rng.standard_normal((T, n_expert)).astype(np.float32)
    x = rng.standard_normal((T, hidden)).astype(np.float32)
    dx = hip.to_device(x)
    ids, w = hip.alloc(T * n_sel * 4), hip.alloc(T * n_sel * 4)
    hip.moe_route_batch(hip.to_device(logits), T, n_expert, n_sel, ids, w)
    y1, y2 = hip.alloc(T * hidden * 4), hip.alloc(T * hidden * 4)
    hip.moe_batch(desc, T, n_sel, ids, w, dx, y1)
    routes = [oracle.router_topk(logits[t], n_sel) for t in range(T)]
    oi = np.stack([r[0] for r in routes]).astype(np.int32)
    ow = np.stack([r[1] for r in routes]).astype(np.float32)
    di, dw = hip.to_device(oi), hip.to_device(ow)
    hip.moe_batch(desc, T, n_sel, di, dw, dx, y2)
    hip.sync()
    assert np.array_equal(y1.download(np.uint32), y2.download(np.uint32))


def test_route_batch_rejects_bad_arguments(hip):
    from katali_hip import HipError
    b = hip.alloc(4096)
    for T, E, k in ((0, 8, 2), (4, 513, 2), (4, 8, 0), (4, 8, 17), (4, 8, 9)):
        with pytest.raises(HipError):
            hip.moe_route_batch(b, T, E, k, b, b)
