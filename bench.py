"""Benchmark of the quantized expert-GEMV path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload moe48|moe40cold|gemv6144|qwen8b|moebatch|tier48|...]

Workloads:
  moe48     (default) one decode token through 48 fused MoE layers,
hidden 2048, 128 experts, top-8, gate/up 2048->768 Q4_K, down 768->2048 Q6_K,
random weights (independent seed per layer), N(0,1) activations and router
logits. Every token draws new router logits (a ring of 64 positions), so each
token touches a different 1.17 GB of the 18.8 GB expert pool: a cold working
set far beyond L2 and the 256 MB MALL. Each ring position's 48 layers are
captured in one hipGraph, reading that position's logits from fixed addresses
(as a decode loop reads its router's output buffer); a step is one token, one
replay, and consecutive steps replay consecutive positions.
  moe40cold 40 MoE layers x 256 experts, gate/up 2048->512 Q4_K, down 512->2048
            Q6_K, top-8 plus an always-on shared expert, 64-position logit ring.
  gemv6144  dense Q4_K 6144x2048 GEMV, batch 1, fp32 x quantized to q8_1
            inside the kernel; 144 distinct weight copies (1.02 GB) are cycled
            so every GEMV reads cold weights; a step is one pass over them.
  qwen8b    dense Qwen3-8B-shaped decode GEMV chain, 36 layers, hidden 4096,
            q/o 4096x4096 and k 1024x4096 Q4_K, v 1024x4096 Q6_K, SwiGLU
            12288 (gate/up Q4_K, down Q6_K); per layer q,k,v = W x (one launch), o = Wo q
            (q stands in for the attention output, which is not a GEMV),
            FFN(o) through the MoE kernels with the shared expert only; every
            layer reads its own N(0,1) x; a step is one token (one replay).
  moe48duty the moe48 layers submitted one by one with a host busy interval
            (0, 20, 200, 1000 us) before each, as an engine running attention
            on the CPU between GPU layers: GPU time per layer at each duty
            cycle (event-timed, synchronous submission) against back to back,
            and tok/s of synchronous vs asynchronous submission; the JSON
            value is the layer's GB/s at 200 us per layer.
  moebatch  the config-1 MoE layer over ragged token batches (1..64 tokens,
            per-token experts from a Zipf(1.1) popularity), swept over
            n_sel in {1, 2, 4, 8}; experts that gather >= 16 tokens run as an
            int8 MFMA grouped GEMM, the rest on the GEMV kernels; 16 layers
            of distinct weights per pass; the JSON value is the n_sel = 8,
            64-token point, the whole sweep is in "sweep".
  floor48   one moe48 layer's 24.5 MB of weights streamed with no arithmetic
            in the layer's launch shape (katali_hip_stream_floor): one read,
            two launches, and one launch with the layer's two in-kernel waits;
            then the exchange probe (katali_hip_exchange_probe): the time of
            one word handed from one workgroup to a waiting one inside an XCD
            group (through its L2, or written through) and across XCDs, in
            "exchanges"; the JSON value is the one-launch read.
  tier48    48 host-routed layers of the moe48 expert shape whose experts
            come through the expert VRAM tier (64 slots) from a GGUF file
            written on the box, m in {0, 1, 2, 4} misses per layer call,
            synchronous vs pipelined uploads (pinned ring + copy stream), in
            the engine flow (y downloaded per layer) and the queued flow (one
            wait per token); the JSON value is tok/s at one miss per layer,
            pipelined, engine flow; roofline: the upload rate against PCIe 5.0
            x16.

Printed: ONE JSON line. value = algorithmic HBM GB/s of the whole token
(selected expert weights + q8_1 activation + fp32 output, per layer) with
everything resident in HBM; tok_s = tokens per second of the 48-layer chain;
roofline = the dominant kernel work: one MoE layer (its two launches) or
one GEMV, algorithmic bytes over the timed-region time per unit, with HBM
traffic from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE profile when one
exists for the workload (profiles/traffic_<workload>.txt);
cpu_baseline = the reference's own CPU path (compiled from its sources into
oracle/_ref) on a bounded sample of the same workload on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "katali-lab_amd"))

import katali_hip as K  # noqa: E402

HBM_PEAK_GBS = 8000.0
Q4_K, Q6_K = K.Q4_K, K.Q6_K


def row_bytes(t, cols):
    return cols // 256 * K.BLOCK_BYTES[t]


# ---------------------------------------------------------------------------
# MoE decode chain
# ---------------------------------------------------------------------------
MOE_WORKLOADS = {
    # name: layers, hidden, ffn, n_expert, n_sel, shared
    "moe48": (48, 2048, 768, 128, 8, False),
    "moe40cold": (40, 2048, 512, 256, 8, True),
}


# Whole decode tokens of a MoE workload, attention aside: the token's
# residual stream, per layer RMSNorm (residual add from the second layer on),
# F32 router logits and the MoE layer routed from them on the device, then the
# output norm, the Q6_K LM head and the greedy argmax, all in one hipGraph.
TOKEN_WORKLOADS = {
    # name: MoE workload, vocabulary
    "moe48tok": ("moe48", 151936),
}


def xcd_layer(hip, hidden, ffn, n_expert, n_slots, shared=False):
    """Whether the library runs this layer shape as the XCD-sliced one-launch
    layer (k_moe_xcd) rather than kernels A and B: the rule launch_moe
    applies (eight slots, or eight routed experts plus the shared expert with
    ffn 256 or 512 unless KATALI_HIP_XCD_SHARED=0; hidden 1024 or 2048,
    ffn <= 1024, <= 256 experts, a 256-CU device, KATALI_HIP_XCD not 0)."""
    if os.environ.get("KATALI_HIP_XCD", "1")[:1] in ("0", "n", "N"):
        return False
    spread = (n_slots == 9 and shared and ffn in (256, 512)
              and os.environ.get("KATALI_HIP_XCD_SHARED", "1")[:1] not in ("0", "n", "N"))
    return ((n_slots == 8 or spread) and hidden in (1024, 2048) and ffn <= 1024 and n_expert <= 256
            and " 256 CUs" in hip.status())


def layer_kernels(hip, hidden, ffn, n_expert, n_slots, shared=False):
    return ("k_moe_xcd (one launch per layer)" if xcd_layer(hip, hidden, ffn, n_expert, n_slots, shared)
            else "k_moe_gu + k_moe_down (two launches per layer)")


def moe_bytes_per_layer(hidden, ffn, n_sel, shared):
    per_expert = 2 * ffn * row_bytes(Q4_K, hidden) + hidden * row_bytes(Q6_K, ffn)
    slots = n_sel + (1 if shared else 0)
    return slots * per_expert + hidden // 32 * 36 + hidden * 4, slots * per_expert


class View:  # a device pointer inside a larger buffer
    def __init__(self, ptr):
        self.ptr = ptr


def moe_setup(hip, name, ring=64):
    """A MoE workload's device state: per layer distinct random expert stacks
    (and shared expert), one x and one y slot per layer, and a ring of router
    logits (position t, layer l at (t * L + l) * n_expert) with a route per
    (position, layer) reading its logits from a fixed address."""
    L, hidden, ffn, n_expert, n_sel, shared = MOE_WORKLOADS[name]
    rb_g, rb_d = row_bytes(Q4_K, hidden), row_bytes(Q6_K, ffn)
    layers = []
    seed = 1000
    for li in range(L):
        g = hip.alloc(n_expert * ffn * rb_g)
        u = hip.alloc(n_expert * ffn * rb_g)
        d = hip.alloc(n_expert * hidden * rb_d)
        for buf, t, nb in ((g, Q4_K, n_expert * ffn * hidden // 256), (u, Q4_K, n_expert * ffn * hidden // 256),
                           (d, Q6_K, n_expert * hidden * ffn // 256)):
            hip.synth_fill(t, buf, nb, seed)
            seed += 1
        sh = None
        if shared:
            sh = [hip.alloc(ffn * rb_g), hip.alloc(ffn * rb_g), hip.alloc(hidden * rb_d)]
            for buf, t, nb in ((sh[0], Q4_K, ffn * hidden // 256), (sh[1], Q4_K, ffn * hidden // 256),
                               (sh[2], Q6_K, hidden * ffn // 256)):
                hip.synth_fill(t, buf, nb, seed)
                seed += 1
        layers.append((g, u, d, sh))
    x = hip.alloc(L * hidden * 4)
    hip.synth_normal(x, L * hidden, 77)
    y = hip.alloc(L * hidden * 4)
    # router logits of ring position t, layer l at (t * L + l) * n_expert: each
    # token reads its own logits from a fixed address, as a decode loop reads
    # the router's output buffer
    logits = hip.alloc(ring * L * n_expert * 4)
    hip.synth_normal(logits, ring * L * n_expert, 78)
    descs = [hip.moe_desc(hidden, ffn, n_expert, g, u, d, shared=sh) for (g, u, d, sh) in layers]
    routes = []
    for t in range(ring):
        rt = []
        for li in range(L):
            r = hip.moe_route(n_sel)
            r.logits = logits.ptr + (t * L + li) * n_expert * 4
            rt.append(r)
        routes.append(rt)

    xs = [View(x.ptr + li * hidden * 4) for li in range(L)]
    ys = [View(y.ptr + li * hidden * 4) for li in range(L)]
    return layers, descs, routes, (x, y, logits), xs, ys, seed


def moe_free(layers, bufs):
    for g, u, d, sh in layers:
        for b in (g, u, d) + tuple(sh or ()):
            b.free()
    for b in bufs:
        b.free()


def host_routes(hip, logits, ring, L, n_expert, n_sel):
    """Routes with the selection given, as the engine's CPU router hands it
    to the reference's layer call: per ring position and layer, the top
    n_sel experts of the same logits (larger logit first, lower index on
    ties) and their weights exp(l - l_0) / sum over the selection, computed
    on the host and uploaded once. Returns the routes and the two buffers."""
    lg = logits.download(np.float32).reshape(ring, L, n_expert).astype(np.float64)
    ids = np.zeros((ring, L, n_sel), np.int32)
    wts = np.zeros((ring, L, n_sel), np.float32)
    for t in range(ring):
        for li in range(L):
            o = np.lexsort((np.arange(n_expert), -lg[t, li]))[:n_sel]
            e = np.exp(lg[t, li][o] - lg[t, li][o[0]])
            ids[t, li], wts[t, li] = o, e / e.sum()
    dids, dwts = hip.to_device(ids), hip.to_device(wts)
    routes = [[hip.moe_route(n_sel, ids=View(dids.ptr + 4 * n_sel * (t * L + li)),
                             weights=View(dwts.ptr + 4 * n_sel * (t * L + li))) for li in range(L)]
              for t in range(ring)]
    return routes, (dids, dwts)


def bench_moe(hip, name, steps, warmup, ring=64, vocab=0, normed=False, stacked=False, stamps=None,
              given=False):
    """One hipGraph per ring position, replayed per token. vocab == 0: the
    MoE layers only (router logits from a ring). vocab > 0: the whole token
    chain (TOKEN_WORKLOADS), routing from the device router's logits.
    stacked: the token's L layers as one stacked launch
    (katali_hip_moe_stack_*): each layer on its own x, its weight loads held
    until the previous layer's y is complete (with vocab: the normed stack,
    x_l = x_{l-1} + y_{l-1}), instead of one call per layer. stamps: a dict
    that gets the measurement build's phase stamps of the timed replays.
    given: each layer call gets its selection (host_routes) instead of
    ranking the logits on the device."""
    L, hidden, ffn, n_expert, n_sel, shared = MOE_WORKLOADS[name]
    rb_g, rb_d = row_bytes(Q4_K, hidden), row_bytes(Q6_K, ffn)
    layers, descs, routes, bufs, xs, ys, seed = moe_setup(hip, name, ring)
    given_bufs = ()
    if given:
        routes, given_bufs = host_routes(hip, bufs[2], ring, L, n_expert, n_sel)
    stacks = []

    def token(t):
        for li in range(L):
            hip.moe_layer(descs[li], routes[t][li], ys[li], x=xs[li])

    if stacked and not vocab:
        # one stack per ring position: its layer table names that position's logits
        for t in range(ring):
            stacks.append(hip.moe_stack(descs[0], n_sel, [
                {"gate": layers[li][0], "up": layers[li][1], "down": layers[li][2], "shared": layers[li][3],
                 "y": ys[li], "route": routes[t][li], "x": xs[li] if li else None} for li in range(L)]))

        def token(t):  # noqa: F811
            stacks[t].run(xs[0])

    chain_bufs = []
    if vocab:
        rb_h = row_bytes(Q6_K, hidden)
        router = hip.alloc(L * n_expert * hidden * 4)
        hip.synth_normal(router, L * n_expert * hidden, 79, 0.05)
        norm_w = hip.alloc((L + 1) * hidden * 4)
        hip.synth_normal(norm_w, (L + 1) * hidden, 80, 1.0)
        x0 = hip.alloc(ring * hidden * 4)          # the ring's token inputs
        hip.synth_normal(x0, ring * hidden, 81, 1.0)
        xpp, xn_out = [hip.alloc(hidden * 4), hip.alloc(hidden * 4)], hip.alloc(hidden * 4)
        clog = hip.alloc(L * n_expert * 4)
        head = hip.alloc(vocab * rb_h)
        hip.synth_fill(Q6_K, head, vocab * hidden // 256, seed)
        head_logits, tok = hip.alloc(vocab * 4), hip.alloc(256)
        chain_bufs = [router, norm_w, x0, *xpp, xn_out, clog, head, head_logits, tok]
        routers = [View(router.ptr + li * n_expert * hidden * 4) for li in range(L + 1)]
        nws = [View(norm_w.ptr + li * hidden * 4) for li in range(L + 1)]
        cls = [View(clog.ptr + li * n_expert * 4) for li in range(L)]
        croutes = [hip.moe_route(n_sel, logits=cls[li]) for li in range(L)]

        if stacked:
            # the token's layers as the normed stack (one launch); then the
            # output norm adds the last layer's y to the residual entering it
            xo_last = hip.alloc(L * hidden * 4)
            chain_bufs.append(xo_last)
            xol = [View(xo_last.ptr + li * hidden * 4) for li in range(L)]
            stk = hip.moe_stack(descs[0], n_sel, [
                {"gate": layers[li][0], "up": layers[li][1], "down": layers[li][2], "shared": layers[li][3],
                 "y": ys[li], "norm_w": nws[li], "router": routers[li], "x_out": xol[li]} for li in range(L)],
                normed=True)
            stacks.append(stk)

        def token(t):  # noqa: F811
            if stacked:
                stacks[0].run(View(x0.ptr + t * hidden * 4))
                hip.add_rmsnorm(xol[L - 1], ys[L - 1], 1.0, nws[L], hidden, 1e-6, xn_out)
                hip.matvec_dp4a(Q6_K, head, vocab, hidden, xn_out, head_logits)
                hip.argmax(head_logits, vocab, tok)
                return
            # per layer the residual step, the norm, the router logits and the
            # MoE layer: three launches (katali_hip_rmsnorm_matvec_f32, then
            # the layer), or two with normed (katali_hip_moe_layer_normed);
            # the residual stream alternates between two buffers
            cur = View(x0.ptr + t * hidden * 4)
            for li in range(L):
                delta = ys[li - 1] if li else None
                nxt = xpp[li % 2] if li else None
                if normed:
                    hip.moe_layer_normed(descs[li], n_sel, cur, nws[li], routers[li], ys[li], delta=delta,
                                         scale=1.0, x_out=nxt)
                else:
                    hip.rmsnorm_matvec_f32(cur, delta, 1.0, nxt, nws[li], hidden, 1e-6, xs[li], routers[li],
                                           n_expert, cls[li])
                    hip.moe_layer(descs[li], croutes[li], ys[li], x=xs[li])
                if li:
                    cur = nxt
            hip.add_rmsnorm(cur, ys[L - 1], 1.0, nws[L], hidden, 1e-6, xn_out)
            hip.matvec_dp4a(Q6_K, head, vocab, hidden, xn_out, head_logits)
            hip.argmax(head_logits, vocab, tok)

    # eager pass sizes the scratch, then one graph per ring position
    token(0)
    hip.sync()
    graphs = []
    for t in range(ring):
        hip.graph_begin()
        token(t)
        graphs.append(hip.graph_end())

    for i in range(warmup):
        hip.graph_launch(graphs[i % ring])
    hip.sync()
    e0, e1 = hip.event(), hip.event()
    hip.sync()
    t0 = time.perf_counter()
    hip.record(e0)
    for i in range(steps):
        hip.graph_launch(graphs[(warmup + i) % ring])
    hip.record(e1)
    ms = hip.elapsed_ms(e0, e1)
    wall = time.perf_counter() - t0
    hip.sync()
    if stamps is not None:   # the last 64 layers of the timed replays
        stamps["stamps"] = hip.phase_stamps()

    # per-launch kernel time: an event pair around each layer (or, stacked,
    # each stack launch, per layer), eager
    ev = [hip.event() for _ in range(2 * L)]
    per = []
    for t in range(0 if vocab else 3):   # (the token chain reports the graph only)
        if stacked:
            hip.record(ev[0])
            stacks[t].run(xs[0])
            hip.record(ev[1])
            hip.sync()
            per.append(hip.elapsed_ms(ev[0], ev[1]) / L)
            continue
        for li in range(L):
            hip.record(ev[2 * li])
            hip.moe_layer(descs[li], croutes[li] if vocab else routes[t][li], ys[li], x=xs[li])
            hip.record(ev[2 * li + 1])
        hip.sync()
        per += [hip.elapsed_ms(ev[2 * li], ev[2 * li + 1]) for li in range(L)]
    for e in ev + [e0, e1]:
        hip.event_destroy(e)
    for gr in graphs:
        hip.graph_destroy(gr)
    for stk in stacks:
        stk.destroy()

    layer_bytes, weight_bytes = moe_bytes_per_layer(hidden, ffn, n_sel, shared)
    tok_bytes = L * layer_bytes
    if vocab:
        # + per layer: router weights and logits out; the norm's x, delta, w
        # in and x_out, xn written (20 B per element); + the output norm, the
        # LM head (weights, logits out) and the argmax read
        tok_bytes += L * (n_expert * hidden * 4 + n_expert * 4 + 20 * hidden)
        tok_bytes += 16 * hidden + vocab * row_bytes(Q6_K, hidden) + vocab * 4 + vocab * 4
        for b in chain_bufs:
            b.free()
    s_per_tok = ms / 1e3 / steps
    kernel_ms = float(np.mean(per)) if per else float("nan")
    res = {
        "ms_per_step": ms / steps,
        "wall_ms_per_step": wall * 1e3 / steps,
        "value": tok_bytes / s_per_tok / 1e9,
        "tok_s": 1.0 / s_per_tok,
        "bytes_per_token": tok_bytes,
        "kernel_ms_mean": kernel_ms,
        "kernel_ms_median": float(np.median(per)) if per else float("nan"),
        "kernel_gbs": layer_bytes / (kernel_ms / 1e3) / 1e9,
        "layer_bytes": layer_bytes,
        "pool_gb": L * (n_expert * (2 * ffn * rb_g + hidden * rb_d)) / 1e9,
    }
    moe_free(layers, bufs + tuple(given_bufs))
    return res, (L, hidden, ffn, n_expert, n_sel, shared)


# ---------------------------------------------------------------------------
# Streaming floors: a MoE layer's bytes with no arithmetic
# ---------------------------------------------------------------------------
FLOOR_KINDS = {0: "one launch reading the layer's bytes",
               1: "gate/up bytes, then down bytes, in two launches",
               2: "gate/up then down bytes in one launch with the XCD-sliced layer's two in-kernel waits"}


def bench_floor(hip, base, steps, warmup, kinds=None):
    """Each of the three floors (katali_hip_stream_floor) over L units of one
    layer's weight bytes (distinct per unit, like the layers), one graph per
    pass of L units; per unit time and GB/s."""
    L, hidden, ffn, n_expert, n_sel, shared = MOE_WORKLOADS[base]
    slots = n_sel + (1 if shared else 0)
    a_bytes = slots * 2 * ffn * row_bytes(Q4_K, hidden)
    b_bytes = slots * hidden * row_bytes(Q6_K, ffn)
    unit = a_bytes + b_bytes
    pool = hip.alloc(L * unit)
    hip.memset(pool, 1, L * unit)
    sync = hip.alloc(4096)
    hip.memset(sync, 0, 4096)
    hip.sync()
    out = {}
    for kind in (kinds or FLOOR_KINDS):
        def units():
            for u in range(L):
                a = View(pool.ptr + u * unit)
                b = View(pool.ptr + u * unit + a_bytes)
                if kind == 0:
                    hip.stream_floor(0, a, unit, None, 0, sync)
                else:
                    hip.stream_floor(kind, a, a_bytes, b, b_bytes, sync)
        units()
        hip.sync()
        hip.graph_begin()
        units()
        g = hip.graph_end()
        for _ in range(warmup):
            hip.graph_launch(g)
        e0, e1 = hip.event(), hip.event()
        hip.sync()
        hip.record(e0)
        for _ in range(steps):
            hip.graph_launch(g)
        hip.record(e1)
        ms = hip.elapsed_ms(e0, e1)
        hip.sync()
        hip.graph_destroy(g)
        hip.event_destroy(e0)
        hip.event_destroy(e1)
        us = ms * 1e3 / steps / L
        out[kind] = {"what": FLOOR_KINDS[kind], "us_per_unit": round(us, 3), "gbs": round(unit / us / 1e3, 1)}
        print(f"[bench] floor {kind}: {us:.2f} us per unit, {unit / us / 1e3:.0f} GB/s", file=sys.stderr, flush=True)
    pool.free()
    sync.free()
    return out, (L, a_bytes, b_bytes)


XCHG_KINDS = {0: "inside one XCD group, through its L2", 1: "inside one XCD group, written through",
              2: "across two XCDs, written through"}


def bench_xchg(hip, rounds=2000, reps=5):
    """The exchange probe (katali_hip_exchange_probe): per kind, the median
    over reps calls of the time per one-way hand-off (a call makes
    2 * rounds of them), with the XCC ids the pairs ran on."""
    words = hip.alloc(4 * 1025)
    hip.memset(words, 0, 4 * 1025)
    hip.sync()
    out = {}
    for kind, what in XCHG_KINDS.items():
        hip.exchange_probe(kind, 64, words)   # warm-up
        hip.sync()
        us = []
        for _ in range(reps):
            e0, e1 = hip.event(), hip.event()
            hip.record(e0)
            hip.exchange_probe(kind, rounds, words)
            hip.record(e1)
            hip.sync()
            us.append(hip.elapsed_ms(e0, e1) * 1e3 / (2 * rounds))
            hip.event_destroy(e0)
            hip.event_destroy(e1)
        w = words.download(np.uint32, 1025)
        ids, err = w[768:1024], int(w[1024])
        part = np.arange(256) ^ (1 if kind == 2 else 8)
        same = int(np.sum(ids == ids[part]))
        out[kind] = {"what": what, "us_one_way": round(float(np.median(us)), 3),
                     "us_range": [round(min(us), 3), round(max(us), 3)], "rounds": rounds,
                     "pairs_on_one_xcd": f"{same // 2} of 128", "wait_expired": bool(err & 1)}
        print(f"[bench] exchange {kind} ({what}): {np.median(us):.3f} us one way, "
              f"{same // 2} of 128 pairs on one XCD", file=sys.stderr, flush=True)
    words.free()
    return out


# ---------------------------------------------------------------------------
# Duty cycle: host work between MoE layer submissions
# ---------------------------------------------------------------------------
DUTY_INTERVALS_US = (0, 20, 200, 1000)   # host time per layer (200: the engine's ~6 % GPU duty cycle)


def spin_us(us):
    """Busy the calling host thread for `us` microseconds (it stands in for
    the engine's CPU attention of one layer)."""
    if us <= 0:
        return
    end = time.perf_counter() + us * 1e-6
    while time.perf_counter() < end:
        pass


def bench_duty(hip, name, steps, warmup, intervals=DUTY_INTERVALS_US):
    """The moe48 layers submitted one by one (no graph) with a host busy
    interval before each layer, as an engine that runs attention on the CPU
    between GPU MoE layers does. Per interval:
      sync:  interval, submit the layer, wait for it (the synchronous engine);
             HIP events around each layer give its GPU time at this duty cycle;
      async: interval, submit, no wait; one wait per token (the host work of
             the next layer overlaps the GPU's layer).
    Reported per interval: GPU us per layer (event-timed, sync mode), tok/s of
    both modes and the GPU duty cycle of the sync mode. Interval 0 is the
    back-to-back case."""
    L, hidden, ffn, n_expert, n_sel, shared = MOE_WORKLOADS[name]
    layers, descs, routes, bufs, xs, ys, _ = moe_setup(hip, name)
    ring = len(routes)
    ev = [hip.event() for _ in range(2 * L)]
    points = []
    tok = 0
    for us in intervals:
        for mode in ("sync", "async"):
            per, walls = [], []
            for i in range(warmup + steps):
                t = routes[tok % ring]
                tok += 1
                t0 = time.perf_counter()
                for li in range(L):
                    spin_us(us)
                    if mode == "sync":
                        hip.record(ev[2 * li])
                    hip.moe_layer(descs[li], t[li], ys[li], x=xs[li])
                    if mode == "sync":
                        hip.record(ev[2 * li + 1])
                        hip.sync()
                hip.sync()
                if i >= warmup:
                    walls.append(time.perf_counter() - t0)
                    if mode == "sync":
                        per += [hip.elapsed_ms(ev[2 * li], ev[2 * li + 1]) for li in range(L)]
            wall = float(np.mean(walls))
            pt = {"host_us_per_layer": us, "mode": mode, "tok_s": round(1.0 / wall, 2),
                  "ms_per_token": round(wall * 1e3, 4)}
            if mode == "sync":
                pt["gpu_us_per_layer"] = round(float(np.mean(per)) * 1e3, 3)
                pt["gpu_us_per_layer_median"] = round(float(np.median(per)) * 1e3, 3)
                pt["duty_cycle"] = round(float(np.sum(per)) / 1e3 / steps / wall, 4)
            points.append(pt)
            print(f"[bench] duty {us:5d} us/layer {mode:5s}: {pt['tok_s']:8.2f} tok/s"
                  + (f", GPU {pt['gpu_us_per_layer']:.2f} us/layer, duty {pt['duty_cycle']:.3f}" if mode == "sync" else ""),
                  file=sys.stderr, flush=True)
    for e in ev:
        hip.event_destroy(e)
    moe_free(layers, bufs)
    layer_bytes, _ = moe_bytes_per_layer(hidden, ffn, n_sel, shared)
    base = next(p for p in points if p["mode"] == "sync" and p["host_us_per_layer"] == 0)
    head = next(p for p in points if p["mode"] == "sync" and p["host_us_per_layer"] == 200)
    res = {
        "points": points,
        "layer_bytes": layer_bytes,
        # the headline: GPU GB/s of a layer at the engine's duty cycle (host
        # 200 us per layer, synchronous), from its event-timed GPU time
        "value": layer_bytes / (head["gpu_us_per_layer"] * 1e-6) / 1e9,
        "ms_per_step": head["ms_per_token"],
        "unit_ms": head["gpu_us_per_layer"] / 1e3,
        "back_to_back_unit_ms": base["gpu_us_per_layer"] / 1e3,
    }
    return res, (L, hidden, ffn, n_expert, n_sel, shared)


# ---------------------------------------------------------------------------
# Expert VRAM tier: host-routed layers whose experts come from a GGUF file
# ---------------------------------------------------------------------------
TIER_SHAPE = (2048, 768, 128, 8)   # hidden, ffn, experts, top-k: the moe48 expert shape
TIER_MISSES = (0, 1, 2, 4)         # misses per layer call (of 8 experts)
PCIE5_X16_GBS = 64.0               # published PCIe 5.0 x16 rate per direction


def host_blocks(rng, t, nblocks):
    """Random Q4_K / Q6_K blocks on the host with d (and dmin) ~ |N(0, 0.02)|."""
    bb = 144 if t == Q4_K else 210
    b = rng.integers(0, 256, (nblocks, bb), dtype=np.uint8)
    d = np.abs(rng.standard_normal((nblocks, 2)) * 0.02).astype(np.float16).view(np.uint8).reshape(nblocks, 4)
    if t == Q4_K:
        b[:, 0:4] = d
    else:
        b[:, 208:210] = d[:, 0:2]
    return b


def tier_file(path, file_layers, seed=900):
    import gguf_writer as W
    hidden, ffn, E, k = TIER_SHAPE
    rng = np.random.default_rng(seed)
    w = W.GgufWriter(alignment=32)
    w.kv("general.architecture", W.STR, "qwen3moe").kv("qwen3moe.block_count", W.U32, file_layers)
    w.kv("qwen3moe.embedding_length", W.U32, hidden).kv("qwen3moe.expert_count", W.U32, E)
    w.kv("qwen3moe.expert_used_count", W.U32, k)
    for li in range(file_layers):
        w.tensor(f"blk.{li}.ffn_gate_exps.weight", [hidden, ffn, E], Q4_K, host_blocks(rng, Q4_K, E * ffn * hidden // 256))
        w.tensor(f"blk.{li}.ffn_up_exps.weight", [hidden, ffn, E], Q4_K, host_blocks(rng, Q4_K, E * ffn * hidden // 256))
        w.tensor(f"blk.{li}.ffn_down_exps.weight", [ffn, hidden, E], Q6_K, host_blocks(rng, Q6_K, E * hidden * ffn // 256))
    w.write(path)


def tier_calls(m, layers, file_layers, n_calls, seed=901):
    """n_calls layer calls of top-8 experts with exactly m misses each once
    warm: per file layer a fixed hot set of 8 - m experts (asked for at every
    call of that layer, so never the least recently used) and m experts from
    a rotation over the other 120, which come back only after every other
    cold expert of the layer has been asked for (long after the slots
    evicted them)."""
    hidden, ffn, E, k = TIER_SHAPE
    rng = np.random.default_rng(seed)
    perm = [rng.permutation(E) for _ in range(file_layers)]
    hot = [p[:k - m].tolist() for p in perm]
    cold = [p[k - m:].tolist() for p in perm]
    ptr = [0] * file_layers
    calls = []
    for c in range(n_calls):
        fl = (c % layers) % file_layers
        ids = hot[fl] + [cold[fl][(ptr[fl] + j) % len(cold[fl])] for j in range(m)]
        ptr[fl] += m
        calls.append((fl, ids))
    return calls


def tier_slots(n_slots, calls):
    """The tier's slot numbers for each call (its rule: the least recently
    used slot not asked for in the same call, the lowest among equals)."""
    slots = [(-1, 0)] * n_slots
    out = []
    for tick, (layer, ids) in enumerate(calls, 1):
        got = []
        for e in ids:
            key = layer * 65536 + e
            s = next((i for i, (kk, _) in enumerate(slots) if kk == key), None)
            if s is None:
                s = min((i for i, (_, u) in enumerate(slots) if u != tick), key=lambda i: (slots[i][1], i))
            slots[s] = (key, tick)
            got.append(s)
        out.append(got)
    return out


class _View:
    """A device address inside a buffer the caller keeps alive."""

    def __init__(self, ptr):
        self.ptr = ptr


def bench_tier(hip, steps, warmup, misses=TIER_MISSES, layers=48, file_layers=2, n_slots=64):
    """Decode tokens of `layers` host-routed MoE layers (the moe48 expert
    shape) whose experts come through the expert VRAM tier (n_slots slots)
    from a GGUF file of file_layers layers (layer l uses file layer
    l % file_layers), at m misses per layer call. Per m, uploads synchronous
    (each miss copied from the mapped file and waited for) or pipelined
    (pinned ring + copy stream), in two submission flows:
      engine: per layer the tier call, the slot ids uploaded, the layer, and
              y downloaded (the host router of the next layer needs it);
      queued: the expert ids of the whole token known up front (slot ids
              uploaded once per token from the tier's rule), no wait between
              layers, one per token: uploads overlap the kernels queued
              before them.
    tok/s per (m, mode, flow) and the upload rate of the pipelined queued flow."""
    import tempfile

    from katali_hip_gguf import ExpertTier, Gguf
    hidden, ffn, E, k = TIER_SHAPE
    path = os.path.join(tempfile.gettempdir(), f"katali_tier_{os.getpid()}.gguf")
    print(f"[bench] tier: writing {file_layers} layers of {E} experts to {path}", file=sys.stderr, flush=True)
    tier_file(path, file_layers)
    g = Gguf(path)
    x = hip.alloc(hidden * 4)
    hip.synth_normal(x, hidden, 77)
    y = hip.alloc(hidden * 4)
    wts = hip.to_device(np.full(k, 1.0 / k, np.float32))
    sbuf, ebuf = hip.alloc(layers * k * 4), hip.alloc(k * 4)
    per_expert = None
    points = []
    try:
        for m in misses:
            n_calls = (warmup + steps) * layers
            calls = tier_calls(m, layers, file_layers, n_calls)
            for mode in ("sync", "pipelined"):
                for flow in ("engine", "queued"):
                    tier = ExpertTier(g, 0, budget=0, max_slots=n_slots)
                    if mode == "pipelined":
                        tier.pipeline()
                    # warm the hot sets (and the file's pages) outside the timing
                    for c in calls[:file_layers]:
                        tier.layer(*c)
                    hip.sync()
                    pred = tier_slots(n_slots, calls[:file_layers] + calls)[file_layers:]
                    walls = []
                    st0 = None
                    for tok in range(warmup + steps):
                        if tok == warmup:
                            st0 = tier.stats()
                        t0 = time.perf_counter()
                        batch = calls[tok * layers:(tok + 1) * layers]
                        if flow == "queued":
                            sbuf.upload(np.array(pred[tok * layers:(tok + 1) * layers], np.int32).ravel())
                        for li, c in enumerate(batch):
                            m_tier, slots = tier.layer(*c)
                            if flow == "queued":
                                assert slots == pred[tok * layers + li], "tier slots differ from its rule"
                                ids = _View(sbuf.ptr + li * k * 4)
                            else:
                                ids = ebuf.upload(np.array(slots, np.int32))
                            hip.moe_layer(m_tier, hip.moe_route(k, ids=ids, weights=wts), y, x=x)
                            if flow == "engine":
                                y.download(np.float32, hidden)
                        hip.sync()
                        if tok >= warmup:
                            walls.append(time.perf_counter() - t0)
                    st = tier.stats()
                    per_expert = st["uploaded_bytes"] // max(st["misses"], 1) if st["misses"] else per_expert
                    tier.destroy()
                    wall = float(np.mean(walls))
                    up = (st["uploaded_bytes"] - st0["uploaded_bytes"]) / steps
                    pt = {"misses_per_layer": m, "mode": mode, "flow": flow, "tok_s": round(1.0 / wall, 2),
                          "ms_per_token": round(wall * 1e3, 3), "upload_mb_per_token": round(up / 1e6, 2),
                          "upload_gbs": round(up / wall / 1e9, 2),
                          "misses_measured": (st["misses"] - st0["misses"]) / (steps * layers)}
                    points.append(pt)
                    print(f"[bench] tier m={m} {mode:9s} {flow:6s}: {pt['tok_s']:8.2f} tok/s, "
                          f"{pt['upload_mb_per_token']:.1f} MB/token uploaded at {pt['upload_gbs']:.2f} GB/s",
                          file=sys.stderr, flush=True)
    finally:
        g.close()
        os.unlink(path)
    return points, per_expert, (layers, file_layers, n_slots)


# ---------------------------------------------------------------------------
# Dense decode chain (Qwen3-8B shapes)
# ---------------------------------------------------------------------------
DENSE_WORKLOADS = {
    # name: layers, hidden, q_rows, kv_rows, ffn
    "qwen8b": (36, 4096, 4096, 1024, 12288),
}


def dense_layer_bytes(hidden, q_rows, kv_rows, ffn):
    rb4, rb6 = row_bytes(Q4_K, hidden), row_bytes(Q6_K, hidden)
    w = (q_rows + kv_rows) * rb4 + kv_rows * rb6 + hidden * row_bytes(Q4_K, q_rows) \
        + 2 * ffn * rb4 + hidden * row_bytes(Q6_K, ffn)
    act = 4 * (hidden * 4 + 2 * hidden)   # x, q, o, y reads/writes (fp32) plus k, v outputs
    return w + act, w


def bench_dense(hip, name, steps, warmup):
    L, hidden, q_rows, kv_rows, ffn = DENSE_WORKLOADS[name]
    seed = 500
    layers = []

    def filled(t, rows, cols):
        nonlocal seed
        b = hip.alloc(rows * row_bytes(t, cols))
        hip.synth_fill(t, b, rows * cols // 256, seed)
        seed += 1
        return b

    for _ in range(L):
        wq, wk, wv = filled(Q4_K, q_rows, hidden), filled(Q4_K, kv_rows, hidden), filled(Q6_K, kv_rows, hidden)
        wo = filled(Q4_K, hidden, q_rows)
        g, u, d = filled(Q4_K, ffn, hidden), filled(Q4_K, ffn, hidden), filled(Q6_K, hidden, ffn)
        layers.append((wq, wk, wv, wo, g, u, d))
    x = hip.alloc(L * hidden * 4)
    hip.synth_normal(x, L * hidden, 91)
    q, k, v, o, y = (hip.alloc(L * n * 4) for n in (q_rows, kv_rows, kv_rows, hidden, hidden))

    class View:
        def __init__(self, ptr):
            self.ptr = ptr

    def at(buf, li, n):
        return View(buf.ptr + li * n * 4)

    descs = [hip.moe_desc(hidden, ffn, 0, None, None, None, shared=(g, u, d)) for (_, _, _, _, g, u, d) in layers]
    route = hip.moe_route(0)

    def token():
        for li, (wq, wk, wv, wo, g, u, d) in enumerate(layers):
            xl = at(x, li, hidden)
            # q, k and v share x: one launch (the engine's matvec_multi)
            hip.matvec_multi([Q4_K, Q4_K, Q6_K], [wq, wk, wv], [q_rows, kv_rows, kv_rows], hidden, xl,
                             [at(q, li, q_rows), at(k, li, kv_rows), at(v, li, kv_rows)], dp4a=True)
            hip.matvec_dp4a(Q4_K, wo, hidden, q_rows, at(q, li, q_rows), at(o, li, hidden))
            hip.moe_layer(descs[li], route, at(y, li, hidden), x=at(o, li, hidden))

    token()
    hip.sync()
    hip.graph_begin()
    token()
    graph = hip.graph_end()
    for _ in range(warmup):
        hip.graph_launch(graph)
    hip.sync()
    e0, e1 = hip.event(), hip.event()
    t0 = time.perf_counter()
    hip.record(e0)
    for _ in range(steps):
        hip.graph_launch(graph)
    hip.record(e1)
    ms = hip.elapsed_ms(e0, e1)
    wall = time.perf_counter() - t0
    hip.sync()
    for e in (e0, e1):
        hip.event_destroy(e)
    hip.graph_destroy(graph)
    layer_bytes, weight_bytes = dense_layer_bytes(hidden, q_rows, kv_rows, ffn)
    s_per_tok = ms / 1e3 / steps
    res = {
        "ms_per_step": ms / steps,
        "wall_ms_per_step": wall * 1e3 / steps,
        "value": L * layer_bytes / s_per_tok / 1e9,
        "tok_s": 1.0 / s_per_tok,
        "layer_bytes": layer_bytes,
        "bytes_per_token": L * layer_bytes,
        "weights_gb": L * weight_bytes / 1e9,
    }
    for bufs in layers:
        for b in bufs:
            b.free()
    for b in (x, q, k, v, o, y):
        b.free()
    return res, (L, hidden, q_rows, kv_rows, ffn)


# ---------------------------------------------------------------------------
# Batched MoE (prefill) sweep
# ---------------------------------------------------------------------------
BATCH_SHAPE = (16, 2048, 768, 128)   # layers per pass, hidden, ffn, experts
BATCH_POINTS = [(n, t) for n in (1, 2, 4, 8) for t in (1, 7, 16, 33, 64)]


def zipf_routes(rng, T, n_expert, n_sel, s=1.1):
    pop = 1.0 / np.arange(1, n_expert + 1) ** s
    pop /= pop.sum()
    order = rng.permutation(n_expert)
    ids = np.empty((T, n_sel), np.int32)
    w = np.empty((T, n_sel), np.float32)
    for t in range(T):
        pick = order[rng.choice(n_expert, n_sel, replace=False, p=pop)]
        lw = rng.standard_normal(n_sel)
        ww = np.exp(lw - lw.max())
        ww /= ww.sum()
        o = np.argsort(-ww, kind="stable")
        ids[t], w[t] = pick[o], ww[o].astype(np.float32)
    return ids, w


def bench_moe_batch(hip, steps, warmup, only=None):
    L, hidden, ffn, n_expert = BATCH_SHAPE
    rb_g, rb_d = row_bytes(Q4_K, hidden), row_bytes(Q6_K, ffn)
    expert_bytes = 2 * ffn * rb_g + hidden * rb_d
    seed = 3000
    layers = []
    for _ in range(L):
        bufs = []
        for t, rows, cols in ((Q4_K, n_expert * ffn, hidden), (Q4_K, n_expert * ffn, hidden),
                              (Q6_K, n_expert * hidden, ffn)):
            b = hip.alloc(rows * row_bytes(t, cols))
            hip.synth_fill(t, b, rows * cols // 256, seed)
            seed += 1
            bufs.append(b)
        layers.append(bufs)
    descs = [hip.moe_desc(hidden, ffn, n_expert, g, u, d) for g, u, d in layers]
    rng = np.random.default_rng(2024)
    x = hip.alloc(64 * hidden * 4)
    y = hip.alloc(L * 64 * hidden * 4)
    hip.synth_normal(x, 64 * hidden, 55)

    class View:
        def __init__(self, ptr):
            self.ptr = ptr

    points = []
    for n_sel, T in (only or BATCH_POINTS):
        routes = [zipf_routes(rng, T, n_expert, n_sel) for _ in range(L)]
        dev = [(hip.to_device(i), hip.to_device(w)) for i, w in routes]
        distinct = sum(len(np.unique(i)) for i, _ in routes)
        big = sum(int((np.bincount(i.reshape(-1), minlength=n_expert) >= 16).sum()) for i, _ in routes)

        def run():
            for li in range(L):
                hip.moe_batch(descs[li], T, n_sel, dev[li][0], dev[li][1], x, View(y.ptr + li * 64 * hidden * 4))

        run()
        hip.sync()
        hip.graph_begin()
        run()
        graph = hip.graph_end()
        for _ in range(warmup):
            hip.graph_launch(graph)
        hip.sync()
        e0, e1 = hip.event(), hip.event()
        hip.record(e0)
        for _ in range(steps):
            hip.graph_launch(graph)
        hip.record(e1)
        ms = hip.elapsed_ms(e0, e1)
        hip.sync()
        for e in (e0, e1):
            hip.event_destroy(e)
        hip.graph_destroy(graph)
        for a, b in dev:
            a.free()
            b.free()
        layer_ms = ms / steps / L
        bytes_per_layer = distinct / L * expert_bytes + T * (hidden // 32 * 36 + hidden * 4)
        ops = T * n_sel * 2 * (2 * ffn * hidden + hidden * ffn)
        points.append({
            "n_sel": n_sel, "tokens": T, "layer_us": round(layer_ms * 1e3, 2),
            "gbs": round(bytes_per_layer / (layer_ms / 1e3) / 1e9, 1),
            "tok_s": round(T / (layer_ms / 1e3), 1),
            "tops": round(ops / (layer_ms / 1e3) / 1e12, 2),
            "experts_per_layer": round(distinct / L, 1), "grouped_gemm_experts_per_layer": round(big / L, 2),
        })
        print(f"[bench] moebatch n_sel={n_sel} T={T}: {points[-1]}", file=sys.stderr, flush=True)
    for bufs in layers:
        for b in bufs:
            b.free()
    for b in (x, y):
        b.free()
    head = next((p for p in points if p["n_sel"] == 8 and p["tokens"] == 64), points[-1])
    res = {"points": points, "head": head, "ms_per_step": head["layer_us"] * L / 1e3,
           "value": head["gbs"], "pool_gb": L * n_expert * expert_bytes / 1e9}
    return res, BATCH_SHAPE


# ---------------------------------------------------------------------------
# Dense GEMV over a cold rotating pool
# ---------------------------------------------------------------------------
GEMV_WORKLOADS = {
    # name: type, rows, cols, copies
    "gemv6144": (Q4_K, 6144, 2048, 144),
}


def gemv_bytes(t, rows, cols):
    return rows * row_bytes(t, cols) + cols // 32 * 36 + rows * 4


def bench_gemv(hip, name, steps, warmup):
    t, rows, cols, copies = GEMV_WORKLOADS[name]
    rb = row_bytes(t, cols)
    pool = hip.alloc(copies * rows * rb)
    hip.synth_fill(t, pool, copies * rows * cols // 256, 4242)
    x = hip.alloc(cols * 4)
    hip.synth_normal(x, cols, 77)
    y = hip.alloc(copies * rows * 4)

    class View:
        def __init__(self, ptr):
            self.ptr = ptr

    ws = [View(pool.ptr + i * rows * rb) for i in range(copies)]
    ys = [View(y.ptr + i * rows * 4) for i in range(copies)]

    def step():
        for i in range(copies):
            hip.matvec_dp4a(t, ws[i], rows, cols, x, ys[i])

    step()
    hip.sync()
    hip.graph_begin()
    step()
    graph = hip.graph_end()
    for _ in range(warmup):
        hip.graph_launch(graph)
    hip.sync()
    e0, e1 = hip.event(), hip.event()
    t0 = time.perf_counter()
    hip.record(e0)
    for _ in range(steps):
        hip.graph_launch(graph)
    hip.record(e1)
    ms = hip.elapsed_ms(e0, e1)
    wall = time.perf_counter() - t0
    hip.sync()
    for e in (e0, e1):
        hip.event_destroy(e)
    hip.graph_destroy(graph)
    unit_bytes = gemv_bytes(t, rows, cols)
    per_gemv_ms = ms / steps / copies
    res = {
        "ms_per_step": ms / steps,
        "wall_ms_per_step": wall * 1e3 / steps,
        "value": unit_bytes / (per_gemv_ms / 1e3) / 1e9,
        "unit_bytes": unit_bytes,
        "unit_ms": per_gemv_ms,
        "units_per_step": copies,
        "pool_gb": copies * rows * rb / 1e9,
    }
    for b in (pool, x, y):
        b.free()
    return res, (t, rows, cols, copies)


def cpu_baseline_gemv(shape, threads, budget_s=8.0):
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    from oracle import RefCPU, ref_available, Oracle
    t, rows, cols, _ = shape
    rng = np.random.default_rng(9)
    bb = K.BLOCK_BYTES[t]
    n = rows * cols // 256
    w = np.frombuffer(rng.bytes(n * bb), np.uint8).reshape(n, bb).copy()
    w[:, 0:4] = np.abs(rng.normal(0, 0.02, (n, 2))).astype(np.float16).view(np.uint8).reshape(n, 4)
    w = w.reshape(-1)
    x = rng.standard_normal(cols).astype(np.float32)
    y = np.empty(rows, np.float32)
    if ref_available():
        ref = RefCPU()
        kind = "reference"

        def call():
            ref.lib.katali_ggml_matvec(t, w.ctypes.data, rows, cols, x.ctypes.data, y.ctypes.data, threads, None, None, 0)
    else:
        o = Oracle()
        kind = "port"

        def call():
            o.matvec_f32x(t, w, rows, cols, x, threads)
    call()
    t0 = time.perf_counter()
    calls = 0
    while time.perf_counter() - t0 < budget_s and calls < 20000:
        call()
        calls += 1
    dt = time.perf_counter() - t0
    ub = gemv_bytes(t, rows, cols)
    return {
        "value": calls * ub / dt / 1e9,
        "unit": "GB/s",
        "cores": threads,
        "kind": kind,
        "sample": f"{calls} calls of the {rows}x{cols} {'Q4_K' if t == Q4_K else 'Q6_K'} GEMV (one weight matrix, "
                  f"cache-resident as in the reference's own probe), "
                  f"{'reference katali_ggml_matvec' if kind == 'reference' else 'oracle port of the reference AVX2 row loop'}, "
                  f"{threads} threads",
    }


def cpu_baseline_dense(shape, threads, budget_s=8.0):
    """The reference CPU path on the same per-layer GEMV chain (fused q/k/v,
    o, fused gate/up, SiLU-GLU, down), distinct weights per layer."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    from oracle import MatvecJob, RefCPU, ref_available
    if not ref_available():
        return None
    L, hidden, q_rows, kv_rows, ffn = shape
    rng = np.random.default_rng(13)
    n_layers = 4   # distinct weights for 4 layers (0.49 GB), cycled

    def blocks(t, rows, cols):
        bb = K.BLOCK_BYTES[t]
        n = rows * cols // 256
        b = np.frombuffer(rng.bytes(n * bb), np.uint8).reshape(n, bb).copy()
        d = np.abs(rng.normal(0, 0.02, (n, 2))).astype(np.float16).view(np.uint8)
        if t == Q4_K:
            b[:, 0:4] = d.reshape(n, 4)
        else:
            b[:, 208:210] = d[:, :2]
        return b.reshape(-1)

    ws = [(blocks(Q4_K, q_rows, hidden), blocks(Q4_K, kv_rows, hidden), blocks(Q6_K, kv_rows, hidden),
           blocks(Q4_K, hidden, q_rows), blocks(Q4_K, ffn, hidden), blocks(Q4_K, ffn, hidden),
           blocks(Q6_K, hidden, ffn)) for _ in range(n_layers)]
    ref = RefCPU()
    x = rng.standard_normal(hidden).astype(np.float32)
    q, k, v = np.empty(q_rows, np.float32), np.empty(kv_rows, np.float32), np.empty(kv_rows, np.float32)
    o, y = np.empty(hidden, np.float32), np.empty(hidden, np.float32)
    g, u = np.empty(ffn, np.float32), np.empty(ffn, np.float32)
    sums = np.empty(max(hidden, q_rows) // 256 * 64, np.float32)

    def layer(li):
        wq, wk, wv, wo, wg, wu, wd = ws[li % n_layers]
        ref.matvec_fused([MatvecJob(Q4_K, wq.ctypes.data, q_rows, q.ctypes.data, 0),
                          MatvecJob(Q4_K, wk.ctypes.data, kv_rows, k.ctypes.data, 1),
                          MatvecJob(Q6_K, wv.ctypes.data, kv_rows, v.ctypes.data, 2)], hidden, x, threads, sums)
        ref.lib.katali_ggml_matvec(Q4_K, wo.ctypes.data, hidden, q_rows, q.ctypes.data, o.ctypes.data, threads,
                                   None, None, 0)
        ref.matvec_fused([MatvecJob(Q4_K, wg.ctypes.data, ffn, g.ctypes.data, 6),
                          MatvecJob(Q4_K, wu.ctypes.data, ffn, u.ctypes.data, 7)], hidden, o, threads, sums)
        h = ref.silu_mul(g, u)
        ref.lib.katali_ggml_matvec(Q6_K, wd.ctypes.data, hidden, ffn, h.ctypes.data, y.ctypes.data, threads,
                                   None, None, 0)

    layer(0)
    t0 = time.perf_counter()
    n = 0
    while time.perf_counter() - t0 < budget_s and n < 50 * L:
        layer(n)
        n += 1
    dt = time.perf_counter() - t0
    lb, _ = dense_layer_bytes(hidden, q_rows, kv_rows, ffn)
    return {
        "value": n * lb / dt / 1e9,
        "unit": "GB/s",
        "cores": threads,
        "kind": "reference",
        "tok_s": (n / L) / dt,
        "sample": f"{n} layers ({n / L:.2f} tokens) of the same GEMV chain, 4 layers of distinct weights cycled "
                  f"(0.49 GB, DRAM-cold), reference katali_ggml_matvec_fused + silu_mul_avx2 + katali_ggml_matvec, "
                  f"{threads} threads",
    }


def read_traffic(workload):
    """HBM bytes per unit from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE
    profile of this workload, if there is one."""
    path = os.path.join(REPO, "profiles", f"traffic_{workload}.txt")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith("traffic_bytes_per_unit:"):
                return int(float(line.split(":", 1)[1]))
    return None


# ---------------------------------------------------------------------------
# CPU baseline: the reference's own CPU path on a bounded sample
# ---------------------------------------------------------------------------
def cpu_baseline_moe(shape, threads, budget_s=8.0):
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    from oracle import MatvecJob, RefCPU, ref_available, Oracle
    L, hidden, ffn, n_expert, n_sel, shared = shape
    rng = np.random.default_rng(5)
    slots = n_sel + (1 if shared else 0)
    rb_g, rb_d = row_bytes(Q4_K, hidden), row_bytes(Q6_K, ffn)

    def blocks(t, n):
        bb = K.BLOCK_BYTES[t]
        b = np.frombuffer(rng.bytes(n * bb), np.uint8).reshape(n, bb).copy()
        d = np.abs(rng.normal(0, 0.02, (n, 2))).astype(np.float16).view(np.uint8)
        if t == Q4_K:
            b[:, 0:4] = d.reshape(n, 4)
        else:
            b[:, 208:210] = d[:, :2]
        return b.reshape(-1)

    # distinct weights for every (layer, slot): nothing stays cache-resident
    experts = [[(blocks(Q4_K, ffn * hidden // 256), blocks(Q4_K, ffn * hidden // 256),
                 blocks(Q6_K, hidden * ffn // 256)) for _ in range(slots)] for _ in range(L)]
    x = rng.standard_normal(hidden).astype(np.float32)
    w = np.full(slots, 1.0 / slots, np.float32)
    g = np.empty(ffn, np.float32)
    u = np.empty(ffn, np.float32)
    yd = np.empty(hidden, np.float32)
    sums = np.empty(hidden // 256 * 64, np.float32)
    if ref_available():
        ref = RefCPU()
        kind = "reference"

        def layer(li):
            y = np.zeros(hidden, np.float32)
            for s in range(slots):
                G, U, D = experts[li][s]
                jobs = [MatvecJob(Q4_K, G.ctypes.data, ffn, g.ctypes.data, 6),
                        MatvecJob(Q4_K, U.ctypes.data, ffn, u.ctypes.data, 7)]
                ref.matvec_fused(jobs, hidden, x, threads, sums)
                h = ref.silu_mul(g, u)
                ref.lib.katali_ggml_matvec(Q6_K, D.ctypes.data, hidden, ffn, h.ctypes.data, yd.ctypes.data,
                                           threads, None, None, 0)
                y += w[s] * yd
            return y
    else:
        o = Oracle()
        kind = "port"

        def layer(li):
            y = np.zeros(hidden, np.float32)
            for s in range(slots):
                G, U, D = experts[li][s]
                gg = o.matvec_f32x(Q4_K, G, ffn, hidden, x, threads)
                uu = o.matvec_f32x(Q4_K, U, ffn, hidden, x, threads)
                y += w[s] * o.matvec_f32x(Q6_K, D, hidden, ffn, o.silu_mul_ref(gg, uu), threads)
            return y

    layer(0)  # pool start-up
    t0 = time.perf_counter()
    tokens = 0
    while True:
        for li in range(L):
            layer(li)
        tokens += 1
        if time.perf_counter() - t0 >= budget_s or tokens >= 50:
            break
    dt = time.perf_counter() - t0
    layer_bytes, _ = moe_bytes_per_layer(hidden, ffn, n_sel, shared)
    return {
        "value": tokens * L * layer_bytes / dt / 1e9,
        "unit": "GB/s",
        "cores": threads,
        "kind": kind,
        "tok_s": tokens / dt,
        "sample": f"{tokens} token(s) x {L} layers x {slots} experts, distinct expert weights per (layer, slot) "
                  f"({L * slots * 2 * (ffn * rb_g) / 1e9 + L * slots * hidden * rb_d / 1e9:.2f} GB), "
                  f"{'reference katali_ggml_matvec_fused + silu_mul_avx2 + katali_ggml_matvec' if kind == 'reference' else 'oracle port of the reference AVX2 row loop'}, "
                  f"{threads} threads",
    }


# The box a GPU job runs on grants it a share of the host's cores; the CPU
# baseline uses at most this many threads whatever the host has.
CPU_SHARE = 16


def host_cpu():
    """The host CPU as lscpu reports it, and the CPUs this process may run on
    (with the socket of each)."""
    info = {"nproc": os.cpu_count()}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        kv = {}
        for ln in out.splitlines():
            if ":" in ln:
                k, v = ln.split(":", 1)
                kv[k.strip()] = v.strip()
        info["model"] = kv.get("Model name")
        for key, name in (("Socket(s)", "sockets"), ("Core(s) per socket", "cores_per_socket"),
                          ("Thread(s) per core", "threads_per_core"), ("NUMA node(s)", "numa_nodes")):
            if kv.get(key, "").isdigit():
                info[name] = int(kv[key])
        if "sockets" in info and "cores_per_socket" in info:
            info["physical_cores"] = info["sockets"] * info["cores_per_socket"]
        info["numa"] = {k.split()[1]: v for k, v in kv.items() if k.startswith("NUMA node") and "CPU(s)" in k}
    except (OSError, subprocess.SubprocessError):
        info["model"] = None
    allowed = sorted(os.sched_getaffinity(0))
    sockets = {}
    for c in allowed:
        try:
            with open(f"/sys/devices/system/cpu/cpu{c}/topology/physical_package_id") as f:
                sockets.setdefault(int(f.read()), []).append(c)
        except OSError:
            sockets.setdefault(0, []).append(c)
    info["allowed_cpus"] = len(allowed)
    info["allowed_by_socket"] = {str(k): len(v) for k, v in sorted(sockets.items())}
    return info, sockets


def cpu_sample(kind, shape, threads, pin=None):
    """One CPU baseline sample in a child process (so a pinned run starts its
    thread pool under the pinning); it never touches the GPU."""
    spec = json.dumps({"kind": kind, "shape": list(shape), "threads": threads, "pin": pin})
    out = subprocess.run([sys.executable, os.path.abspath(__file__), "--cpu-sample", spec], capture_output=True,
                         text=True, timeout=600)
    if out.returncode != 0:
        print(f"[bench] cpu sample failed: {out.stderr[-2000:]}", file=sys.stderr, flush=True)
        return None
    return json.loads(out.stdout.strip().splitlines()[-1])


def run_cpu_sample(spec):
    s = json.loads(spec)
    if s["pin"]:
        os.sched_setaffinity(0, s["pin"])
    fn = {"moe": cpu_baseline_moe, "dense": cpu_baseline_dense, "gemv": cpu_baseline_gemv}[s["kind"]]
    print(json.dumps(fn(tuple(s["shape"]), s["threads"])), flush=True)


def cpu_baseline(kind, shape):
    """The reference CPU path timed twice: on every CPU this job may use (at
    most CPU_SHARE threads) and pinned to one socket's share of them."""
    info, sockets = host_cpu()
    threads = int(os.environ.get("KATALI_BENCH_CPU_THREADS", min(CPU_SHARE, info["allowed_cpus"])))
    res = cpu_sample(kind, shape, threads)
    if res is None:
        return None
    sock, cpus = max(sockets.items(), key=lambda kv: len(kv[1]))
    pinned_cpus = cpus[:threads]
    pinned = cpu_sample(kind, shape, len(pinned_cpus), pin=pinned_cpus)
    res["host"] = info
    phys = info.get("physical_cores")
    if phys is not None and threads >= phys:
        res["threads_note"] = f"{threads} threads: all {phys} physical cores"
    else:
        res["threads_note"] = (f"{threads} threads: the CPUs this job may use ({info['allowed_cpus']}), capped at the "
                               f"{CPU_SHARE}-thread share a one-GPU job gets on this host, of its {phys} physical "
                               f"cores")
    if pinned is not None:
        res["pinned_one_socket"] = {"value": pinned["value"], "unit": pinned["unit"], "threads": len(pinned_cpus),
                                    "socket": sock, "cpus": pinned_cpus}
    return res


def main():
    if len(sys.argv) > 2 and sys.argv[1] == "--cpu-sample":
        run_cpu_sample(sys.argv[2])
        return
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--workload", default="moe48",
                    choices=sorted(MOE_WORKLOADS) + sorted(TOKEN_WORKLOADS) + sorted(GEMV_WORKLOADS) + sorted(DENSE_WORKLOADS) + ["moebatch", "moe48duty", "floor48", "tier48"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--normed-layer", action="store_true",
                    help="moe48tok: katali_hip_moe_layer_normed, the residual add, norm and router in the layer's "
                         "own launch (the default; kept for older command lines)")
    ap.add_argument("--separate-norm", action="store_true",
                    help="moe48tok: a k_norm_router launch (residual add, norm, router) before each layer instead")
    ap.add_argument("--given-routing", action="store_true",
                    help="moe48 / moe40cold: each layer call gets its experts and weights (ranked on the host from "
                         "the same logit ring, as the reference's layer call takes them) instead of ranking "
                         "the logits on the device")
    ap.add_argument("--stacked", action="store_true",
                    help="moe48 / moe40cold / moe48tok: the token's layers as one stacked launch "
                         "(katali_hip_moe_stack_run), each layer's input the previous layer's output")
    ap.add_argument("--dump-stamps", default="", metavar="NPY",
                    help="moe48 / moe40cold / moe48tok with the measurement build (KATALI_HIP_DLL="
                         "libkatali_hip_stamps.so): save the phase stamps of the timed replays' last 64 layers")
    ap.add_argument("--floor-kind", type=int, action="append", choices=sorted(FLOOR_KINDS),
                    help="floor48: only this floor (repeatable; profiling)")
    ap.add_argument("--batch-points", default="", metavar="NxT,...",
                    help="moebatch: only these (n_sel x tokens) points, e.g. 8x64,2x64 (profiling)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="run one plain copy kernel of MIB MiB before the workload (untimed), as the "
                         "known-size reference for HBM counter profiles")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the expert-parallel "
              "layout for several GPUs is a design note, not a measured path).", file=sys.stderr)
        sys.exit(2)

    # the CPU baseline first, in child processes started before this process
    # initialises the GPU
    cpu = None
    if not args.no_cpu_baseline:
        if args.workload in MOE_WORKLOADS:
            cpu = cpu_baseline("moe", MOE_WORKLOADS[args.workload])
        elif args.workload in DENSE_WORKLOADS:
            cpu = cpu_baseline("dense", DENSE_WORKLOADS[args.workload])
        elif args.workload in GEMV_WORKLOADS:
            cpu = cpu_baseline("gemv", GEMV_WORKLOADS[args.workload])
        # moebatch and the whole-token workloads: no CPU counterpart of that
        # exact workload is timed here
        if cpu:
            print(f"[bench] cpu baseline: {cpu['value']:.2f} GB/s ({cpu['kind']}, {cpu['cores']} threads)",
                  file=sys.stderr, flush=True)

    hip = K.KataliHip()
    if not hip.probe():
        print(f"no usable gfx950 device: {hip.status()}", file=sys.stderr)
        sys.exit(1)
    print(f"[bench] device: {hip.status()}; workload {args.workload}", file=sys.stderr, flush=True)
    if args.calibrate_copy > 0:
        n = args.calibrate_copy << 20
        a, b = hip.alloc(n), hip.alloc(n)
        hip.memset(a, 1, n)
        hip.copy(b, a, n)
        hip.sync()
        a.free()
        b.free()
        print(f"[bench] calibration copy: {n} bytes read + {n} bytes written", file=sys.stderr, flush=True)

    if args.workload == "tier48":
        points, per_expert, (L, file_layers, n_slots) = bench_tier(hip, args.steps, args.warmup)
        hidden, ffn, E, k = TIER_SHAPE
        head = next(p for p in points if p["misses_per_layer"] == 1 and p["mode"] == "pipelined"
                    and p["flow"] == "engine")
        top = max((p for p in points if p["mode"] == "pipelined" and p["flow"] == "queued"),
                  key=lambda p: p["misses_per_layer"])
        line = {
            "metric": "expert-tier decode tok/s at 1 miss per layer (pipelined uploads, host-routed engine flow)",
            "value": head["tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": head["ms_per_token"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "q4_k/q6_k weights x q8_1 activations (int8 dot4, fp32 scales)",
            "data": "synthetic (random Q4_K/Q6_K blocks in a GGUF file written on the box)",
            "config": {
                "workload": f"tier48: {L} host-routed MoE layers (hidden {hidden}, {E} experts, top-{k}, gate/up "
                            f"{hidden}->{ffn} Q4_K, down Q6_K) whose experts come through the expert VRAM tier "
                            f"({n_slots} slots) from a {file_layers}-layer GGUF file; m of the 8 experts of every "
                            f"layer call miss (m in {list(TIER_MISSES)}); synchronous vs pipelined uploads; engine "
                            f"flow (y downloaded per layer) and queued flow (one wait per token)",
                "layers": L, "n_slots": n_slots, "expert_bytes": per_expert, "parallelism": "single GPU",
            },
            "tier_points": points,
            "roofline": {
                "bound": "pcie", "achieved": top["upload_gbs"], "peak": PCIE5_X16_GBS, "unit": "GB/s",
                "frac": round(top["upload_gbs"] / PCIE5_X16_GBS, 4), "traffic": None,
                "kernel": f"host-to-device expert uploads, pipelined queued flow at {top['misses_per_layer']} "
                          f"misses per layer",
                "bytes_per_unit": per_expert, "unit_ms": None,
            },
            "cpu_baseline": None,
        }
        print(json.dumps(line), flush=True)
        return

    traffic = read_traffic(args.workload)
    if args.workload in MOE_WORKLOADS:
        st = {} if args.dump_stamps else None
        res, shape = bench_moe(hip, args.workload, args.steps, args.warmup, stacked=args.stacked, stamps=st,
                               given=args.given_routing)
        if st:
            np.save(args.dump_stamps, st["stamps"])
        L, hidden, ffn, n_expert, n_sel, shared = shape
        unit_ms = res["ms_per_step"] / L
        unit_bytes = res["layer_bytes"]
        metric = "fused MoE layer HBM GB/s (% of ~8 TB/s peak) + decode tok/s, top-8 Q4_K"
        how = (f"the {L} layers as one stacked launch per token (katali_hip_moe_stack_run; each layer on its own "
               f"x, and no layer loads a weight before the previous layer's y is complete, a decode chain's order)"
               if args.stacked else "one katali_hip_moe_layer call per layer on its own x")
        if args.given_routing:
            how += (", each call given its selection (ids and weights of the same logits, ranked on the host "
                    "once, as the engine's CPU router hands them to the reference's layer call)")
        config = {
            "workload": f"{args.workload}: {L}-layer MoE decode, 1 token, hidden {hidden}, {n_expert} experts, "
                        f"top-{n_sel}{' + shared expert' if shared else ''}, gate/up {hidden}->{ffn} Q4_K, "
                        f"down {ffn}->{hidden} Q6_K, fp32 x quantized to q8_1 in the layer, new routing every "
                        f"token from a 64-position logit ring (fixed logits addresses per position), {how}, "
                        f"hipGraph per token",
            "layers": L, "hidden": hidden, "ffn": ffn, "n_expert": n_expert, "n_sel": n_sel,
            "shared_expert": shared, "expert_pool_gb": round(res["pool_gb"], 2),
            "bytes_per_token": res["bytes_per_token"], "parallelism": "single GPU",
        }
        kernel = "MoE layer: " + layer_kernels(hip, hidden, ffn, n_expert, n_sel + (1 if shared else 0), shared)
        if args.stacked:
            kernel = (f"MoE layer in the stacked launch k_moe_stack ({L} layers per launch; unit = one layer, "
                      f"launch time / {L})" if kernel.startswith("MoE layer: k_moe_xcd") else
                      kernel + ", layer by layer under katali_hip_moe_stack_run")
        extra = {"tok_s": round(res["tok_s"], 2),
                 "eager_layer_ms_mean": round(res["kernel_ms_mean"], 5)}
    elif args.workload in TOKEN_WORKLOADS:
        base, vocab = TOKEN_WORKLOADS[args.workload]
        st = {} if args.dump_stamps else None
        normed = not args.separate_norm
        res, shape = bench_moe(hip, base, args.steps, args.warmup, vocab=vocab, normed=normed,
                               stacked=args.stacked, stamps=st)
        if st:
            np.save(args.dump_stamps, st["stamps"])
        L, hidden, ffn, n_expert, n_sel, shared = shape
        unit_ms = res["ms_per_step"]
        unit_bytes = res["bytes_per_token"]
        metric = "decode token HBM GB/s (% of ~8 TB/s peak) + tok/s: MoE FFN chain, LM head and argmax on device"
        layer = layer_kernels(hip, hidden, ffn, n_expert, n_sel + (1 if shared else 0), shared)
        one = layer.startswith("k_moe_xcd")
        steps_desc = ("the normed stack (katali_hip_moe_stack_run, one launch for all layers): per layer the "
                      "residual add of the previous layer's y, RMSNorm, F32 router rows and the MoE layer, the "
                      "logits exchanged on the device" if args.stacked else
                      "one launch for residual add + RMSNorm + F32 router, then the MoE layer"
                      if not normed else
                      "katali_hip_moe_layer_normed: the residual add, RMSNorm and F32 router rows in the layer's "
                      "own prologue, the logits exchanged on the device" +
                      (" (k_moe_xcd: one launch)" if one else " (kernel A, then kernel B)"))
        config = {
            "workload": f"{args.workload}: whole decode tokens of {base} with attention aside: per layer "
                        f"{steps_desc}; router {n_expert}x{hidden} F32, the MoE layer routed on the "
                        f"device from those logits (top-{n_sel}, gate/up {hidden}->{ffn} Q4_K, down Q6_K); output "
                        f"RMSNorm, Q6_K LM head {vocab}x{hidden} (v_dot4), greedy argmax; one hipGraph per token "
                        f"(64 input vectors in a ring)",
            "layers": L, "hidden": hidden, "ffn": ffn, "n_expert": n_expert, "n_sel": n_sel, "vocab": vocab,
            "bytes_per_token": res["bytes_per_token"], "parallelism": "single GPU",
        }
        kernel = ("whole token graph (k_moe_stack: every layer's norm, router and MoE layer in one launch; then "
                  "output norm, head, argmax)" if args.stacked else
                  f"whole token graph (per layer k_norm_router + the MoE layer, {layer}; then 3 launches: output "
                  "norm, head, argmax)" if not normed else
                  "whole token graph (per layer " +
                  ("k_moe_xcd with the norm and router in its prologue, one launch" if one else
                   "k_moe_gu with the norm and router, k_moe_down") + "; output norm, head, argmax)")
        extra = {"tok_s": round(res["tok_s"], 2)}
    elif args.workload == "floor48":
        floors, (L, a_bytes, b_bytes) = bench_floor(hip, "moe48", args.steps, args.warmup, args.floor_kind)
        head = floors[min(floors)]
        unit_bytes = a_bytes + b_bytes
        unit_ms = head["us_per_unit"] / 1e3
        res = {"value": head["gbs"], "ms_per_step": unit_ms * L}
        metric = "HBM read floor for one MoE layer's weight bytes (top-8 of 128, 2048 -> 768 -> 2048): GB/s"
        config = {
            "workload": f"floor48: {L} units of one moe48 layer's weight bytes ({a_bytes} B of gate/up, {b_bytes} B "
                        f"of down), distinct per unit, streamed with no arithmetic by 256 workgroups of 1024 "
                        f"threads (katali_hip_stream_floor), one graph per pass; value: the one-launch read",
            "layers": L, "parallelism": "single GPU",
        }
        kernel = "k_floor_read (one launch per unit)"
        extra = {"floors": floors}
        if not args.floor_kind:   # (profiling runs name their floors)
            extra["exchanges"] = bench_xchg(hip)
    elif args.workload == "moe48duty":
        res, shape = bench_duty(hip, "moe48", args.steps, args.warmup)
        L, hidden, ffn, n_expert, n_sel, shared = shape
        unit_ms = res["unit_ms"]
        unit_bytes = res["layer_bytes"]
        metric = ("fused MoE layer HBM GB/s at the engine's duty cycle (200 us of host work before each layer, "
                  "synchronous submission) + tok/s synchronous vs asynchronous")
        config = {
            "workload": f"moe48duty: the moe48 layers (hidden {hidden}, {n_expert} experts, top-{n_sel}, gate/up "
                        f"{hidden}->{ffn} Q4_K, down Q6_K) submitted one by one without a graph, with a host busy "
                        f"interval before each layer standing in for the engine's CPU attention; intervals "
                        f"{list(DUTY_INTERVALS_US)} us; sync = wait after every layer, async = one wait per token",
            "layers": L, "hidden": hidden, "ffn": ffn, "n_expert": n_expert, "n_sel": n_sel,
            "parallelism": "single GPU",
        }
        kernel = "MoE layer at the duty cycle: " + layer_kernels(hip, hidden, ffn, n_expert, n_sel) + \
            ", event-timed per layer"
        extra = {"duty_points": res["points"],
                 "back_to_back_gpu_us_per_layer": round(res["back_to_back_unit_ms"] * 1e3, 3)}
    elif args.workload == "moebatch":
        only = [tuple(int(v) for v in pt.split("x")) for pt in args.batch_points.split(",") if pt] or None
        res, shape = bench_moe_batch(hip, args.steps, args.warmup, only)
        L, hidden, ffn, n_expert = shape
        head = res["head"]
        unit_ms = head["layer_us"] / 1e3
        unit_bytes = head["gbs"] * 1e9 * unit_ms / 1e3
        metric = "batched MoE layer HBM GB/s (% of ~8 TB/s peak), ragged Zipf-routed token batches"
        config = {
            "workload": f"moebatch: MoE layer over ragged token batches (1..64 tokens), hidden {hidden}, {n_expert} "
                        f"experts, gate/up {hidden}->{ffn} Q4_K, down {ffn}->{hidden} Q6_K, per-token experts from a "
                        f"Zipf(1.1) popularity, n_sel in {{1,2,4,8}}; experts with >= 16 tokens on the int8 MFMA "
                        f"grouped GEMM; {L} layers of distinct weights per pass; headline point n_sel 8, 64 tokens",
            "layers": L, "hidden": hidden, "ffn": ffn, "n_expert": n_expert, "parallelism": "single GPU",
        }
        kernel = "batched MoE layer (grouping, grouped v_dot4 GEMV for experts < 16 tokens, int8 MFMA grouped GEMM, combine)"
        extra = {"tok_s": head["tok_s"], "mfma_frac_of_int8_peak": round(head["tops"] / 5000.0, 4),
                 "sweep": res["points"]}
    elif args.workload in DENSE_WORKLOADS:
        res, shape = bench_dense(hip, args.workload, args.steps, args.warmup)
        L, hidden, q_rows, kv_rows, ffn = shape
        unit_ms = res["ms_per_step"] / L
        unit_bytes = res["layer_bytes"]
        metric = "dense decode GEMV chain HBM GB/s (% of ~8 TB/s peak) + decode tok/s, batch 1"
        config = {
            "workload": f"{args.workload}: {L}-layer Qwen3-8B-shaped decode GEMV chain, hidden {hidden}, "
                        f"q/o {q_rows}x{hidden} and k {kv_rows}x{hidden} Q4_K, v {kv_rows}x{hidden} Q6_K, "
                        f"SwiGLU {ffn} (gate/up Q4_K, down Q6_K), q8_1 activations quantized in-kernel, "
                        f"6 launches per layer, hipGraph per token (attention math not included; LM head not included)",
            "layers": L, "hidden": hidden, "ffn": ffn, "weights_gb": round(res["weights_gb"], 2),
            "bytes_per_token": res["bytes_per_token"], "parallelism": "single GPU",
        }
        kernel = "decode layer: k_gemv_multi (q, k, v) + k_gemv (o) + k_moe_gu + k_moe_down (shared expert only)"
        extra = {"tok_s": round(res["tok_s"], 2)}
    else:
        res, shape = bench_gemv(hip, args.workload, args.steps, args.warmup)
        t, rows, cols, copies = shape
        unit_ms = res["unit_ms"]
        unit_bytes = res["unit_bytes"]
        metric = "dense Q4_K GEMV HBM GB/s (% of ~8 TB/s peak), batch 1"
        config = {
            "workload": f"{args.workload}: {'Q4_K' if t == Q4_K else 'Q6_K'} {rows}x{cols} GEMV, batch 1, fp32 x "
                        f"quantized to q8_1 inside the kernel, {copies} distinct weight copies "
                        f"({res['pool_gb']:.2f} GB) cycled in one hipGraph",
            "rows": rows, "cols": cols, "copies": copies, "parallelism": "single GPU",
        }
        kernel = "k_gemv (q8_1 activation quantized in the workgroup)"
        extra = {}
    print(f"[bench] gpu done: {res['value']:.1f} GB/s", file=sys.stderr, flush=True)
    achieved = unit_bytes / (unit_ms / 1e3) / 1e9
    line = {
        "metric": metric,
        "value": round(res["value"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k/q6_k weights x q8_1 activations (int8 dot4, fp32 scales)",
        "data": "synthetic (random Q4_K/Q6_K blocks with d,dmin ~ |N(0,0.02)|; N(0,1) activations and router logits)",
        "config": config,
        **extra,
        "hbm_frac": round(res["value"] / HBM_PEAK_GBS, 4),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "kernel": kernel,
            "bytes_per_unit": unit_bytes,
            "unit_ms": round(unit_ms, 5),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
