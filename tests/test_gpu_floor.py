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
