"""katali_hip_stream_floor through the C ABI: every floor kind runs (also in
a captured graph, replayed), bad arguments are refused."""
import numpy as np
import pytest

from katali_hip import HipError

pytestmark = pytest.mark.gpu


def test_floor_kinds_run(hip):
    n = 1 << 20
    a, b = hip.alloc(n), hip.alloc(n)
    hip.memset(a, 3, n)
    hip.memset(b, 5, n)
    sync = hip.alloc(4096)
    hip.memset(sync, 0, 4096)
    hip.sync()
    for kind in (0, 1, 2):
        print(f"[floor] kind {kind}", flush=True)
        hip.stream_floor(kind, a, n, b if kind else None, n if kind else 0, sync)
        hip.sync()
    hip.graph_begin()
    hip.stream_floor(2, a, n, b, n, sync)
    g = hip.graph_end()
    try:
        for _ in range(3):
            hip.graph_launch(g)
            hip.sync()
    finally:
        hip.graph_destroy(g)
    # each workgroup's generation word advanced once per kind-2 launch (4)
    gen = sync.download(np.uint32, 256)
    assert (gen == 4).all(), gen[:8]
    for bad in ((3, n), (0, 17)):
        with pytest.raises(HipError):
            hip.stream_floor(bad[0], a, bad[1], None, 0, sync)


def test_exchange_probe_pairs_and_latency(hip):
    """Each kind of the exchange probe runs its rounds without a wait running
    out, with the pairs where the kind puts them (b and b ^ 8 on one XCD,
    b and b ^ 1 on two), and one hand-off takes between 0.05 and 20 us."""
    words = hip.alloc(4 * 1025)
    hip.memset(words, 0, 4 * 1025)
    try:
        for kind in (0, 1, 2):
            print(f"[xchg] kind={kind}", flush=True)
            for rounds in (1, 300):   # tags run on from call to call
                e0, e1 = hip.event(), hip.event()
                hip.record(e0)
                hip.exchange_probe(kind, rounds, words)
                hip.record(e1)
                hip.sync()
                ms = hip.elapsed_ms(e0, e1)
                hip.event_destroy(e0)
                hip.event_destroy(e1)
            w = words.download(np.uint32, 1025)
            assert int(w[1024]) & 1 == 0, "a wait ran out of polls"
            ids = w[768:1024]
            part = np.arange(256) ^ (1 if kind == 2 else 8)
            if kind < 2:
                assert np.array_equal(ids, ids[part])
            else:
                assert not np.any(ids == ids[part])
            us = ms * 1e3 / (2 * 300)
            assert 0.05 < us < 20.0, us
        with pytest.raises(HipError):
            hip.exchange_probe(3, 10, words)
        with pytest.raises(HipError):
            hip.exchange_probe(0, 0, words)
    finally:
        words.free()
