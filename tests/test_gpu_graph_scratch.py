"""Captured graphs and the library's scratch, through the C ABI.

The library allocates its MoE scratch once at its largest size and never
moves it, so a graph captured around a small call stays valid after larger
calls (wider layers, a 64-token batch). Calls that would end a capture
(sync, memset, upload, download, malloc) are refused while one is open, and
a buffer freed during a capture lives as long as the graph made from it;
every replay is checked against an eager run.
"""
import numpy as np
import pytest

import kq_synth as S
from katali_hip import HipError
from oracle import Q4_K, Q6_K

pytestmark = pytest.mark.gpu


def _layer(hip, hidden, ffn, n_expert, shared, seed):
    nb_gu, nb_d = n_expert * ffn * hidden // 256, n_expert * hidden * ffn // 256
    bufs = [hip.alloc(nb_gu * 144), hip.alloc(nb_gu * 144), hip.alloc(nb_d * 210)]
    for i, (t, b, n) in enumerate(((Q4_K, bufs[0], nb_gu), (Q4_K, bufs[1], nb_gu), (Q6_K, bufs[2], nb_d))):
        hip.synth_fill(t, b, n, seed=seed + i)
    sh = None
    if shared:
        n1 = ffn * hidden // 256
        sh = (hip.alloc(n1 * 144), hip.alloc(n1 * 144), hip.alloc(n1 * 210))
        for i, (t, b) in enumerate(((Q4_K, sh[0]), (Q4_K, sh[1]), (Q6_K, sh[2]))):
            hip.synth_fill(t, b, n1, seed=seed + 10 + i)
    return hip.moe_desc(hidden, ffn, n_expert, *bufs, shared=sh)


def test_graph_stays_valid_after_larger_calls(hip):
    rng = np.random.default_rng(31)
    small = _layer(hip, 1024, 512, 32, False, seed=100)
    hidden, n_expert, n_sel = 1024, 32, 4
    x = hip.to_device(S.activation(rng, hidden))
    route = hip.moe_route(n_sel, logits=hip.to_device(rng.standard_normal(n_expert).astype(np.float32)))
    y_eager, y_graph = hip.alloc(hidden * 4), hip.alloc(hidden * 4)
    print("[graph-scratch] eager small layer", flush=True)
    hip.moe_layer(small, route, y_eager, x=x)
    hip.sync()
    want = y_eager.download(np.uint32)
    hip.graph_begin()
    hip.moe_layer(small, route, y_graph, x=x)
    g = hip.graph_end()
    try:
        hip.graph_launch(g)
        hip.sync()
        assert np.array_equal(y_graph.download(np.uint32), want)
        # larger calls after the capture: a 17-slot layer with 12x the h, and
        # the batched layer at its 64-token maximum
        big = _layer(hip, 2048, 6144, 16, True, seed=200)
        hb = 2048
        xb = hip.to_device(S.activation(rng, hb))
        yb = hip.alloc(hb * 4)
        print("[graph-scratch] eager 17-slot layer, ffn 6144", flush=True)
        hip.moe_layer(big, hip.moe_route(16, logits=hip.to_device(rng.standard_normal(16).astype(np.float32))),
                      yb, x=xb)
        T = 64
        ids = hip.to_device(np.stack([rng.permutation(16)[:16] for _ in range(T)]).astype(np.int32))
        w = hip.to_device(np.full((T, 16), 1.0 / 16, np.float32))
        xt = hip.to_device(rng.standard_normal((T, hb)).astype(np.float32))
        yt = hip.alloc(T * hb * 4)
        print("[graph-scratch] eager 64-token batch, 17 slots", flush=True)
        hip.moe_batch(big, T, 16, ids, w, xt, yt)
        hip.sync()
        assert np.any(yt.download(np.uint32) != 0)
        for i in range(3):
            hip.memset(y_graph, 0, hidden * 4)
            print(f"[graph-scratch] replay {i}", flush=True)
            hip.graph_launch(g)
            hip.sync()
            assert np.array_equal(y_graph.download(np.uint32), want), i
            hip.moe_batch(big, T, 16, ids, w, xt, yt)   # eager work between replays
            hip.sync()
    finally:
        hip.graph_destroy(g)


def test_calls_that_would_end_a_capture_are_refused(hip):
    rng = np.random.default_rng(32)
    m = _layer(hip, 512, 256, 16, False, seed=300)
    x = hip.to_device(S.activation(rng, 512))
    route = hip.moe_route(2, logits=hip.to_device(rng.standard_normal(16).astype(np.float32)))
    y0, y1 = hip.alloc(512 * 4), hip.alloc(512 * 4)
    hip.moe_layer(m, route, y0, x=x)
    hip.sync()
    doomed = hip.alloc(4096)
    host = np.zeros(16, np.float32)
    hip.graph_begin()
    try:
        hip.moe_layer(m, route, y1, x=x)
        for call in (hip.sync, lambda: hip.memset(y1, 0, 16), lambda: y1.upload(host),
                     lambda: y1.download(np.float32, 4), lambda: hip.alloc(64)):
            with pytest.raises(HipError, match="capture"):
                call()
        doomed.free()                     # released with the graph
    finally:
        g = hip.graph_end()
    try:
        hip.graph_launch(g)
        hip.sync()
        assert np.array_equal(y1.download(np.uint32), y0.download(np.uint32))
    finally:
        hip.graph_destroy(g)


def test_buffer_freed_during_capture_lives_with_the_graph(hip):
    """A buffer the captured work reads, freed inside the capture, stays
    allocated as long as the graph: replays keep reading it, while new
    allocations of its size (filled with other data) are made between them;
    katali_hip_graph_destroy releases it."""
    rng = np.random.default_rng(33)
    m = _layer(hip, 512, 256, 16, False, seed=301)
    xv = S.activation(rng, 512)
    route = hip.moe_route(2, logits=hip.to_device(rng.standard_normal(16).astype(np.float32)))
    y0, y1 = hip.alloc(512 * 4), hip.alloc(512 * 4)
    hip.moe_layer(m, route, y0, x=hip.to_device(xv))
    hip.sync()
    want = y0.download(np.uint32)
    x = hip.to_device(xv)
    hip.graph_begin()
    try:
        hip.moe_layer(m, route, y1, x=x)
        x.free()                          # the graph reads x: it lives on with the graph
    finally:
        g = hip.graph_end()
    others = []
    try:
        for i in range(3):
            junk = hip.to_device(rng.standard_normal(512).astype(np.float32) * 1e3)
            others.append(junk)
            hip.memset(y1, 0, 512 * 4)
            hip.graph_launch(g)
            hip.sync()
            assert np.array_equal(y1.download(np.uint32), want), i
    finally:
        hip.graph_destroy(g)
