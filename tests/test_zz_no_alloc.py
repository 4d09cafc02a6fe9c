"""katali_hip_moe_layer_noalloc against katali_hip_moe_layer through the C ABI.

The allocation-free entry point chooses the same kernels as the allocating
one (the one-launch XCD-sliced layer where that takes it, with its exchange
words in the static scratch; kernels A and B elsewhere or with
KATALI_HIP_XCD=0) on a static device scratch, so its output must be
bit-identical to the allocating entry point's, in both modes. Two calls in a
row, the second with a smaller problem (fewer slots, narrower rows); the
largest layer shape the LDS admits; a shape beyond it refused before any
launch.
"""
import numpy as np
import pytest

import kq_synth as S
from katali_hip import HipError
from oracle import Q4_K, Q6_K

pytestmark = pytest.mark.gpu


def _problem(hip, rng, hidden, ffn, n_expert, shared):
    g = S.matrix(rng, Q4_K, n_expert * ffn, hidden)
    u = S.matrix(rng, Q4_K, n_expert * ffn, hidden)
    d = S.matrix(rng, Q6_K, n_expert * hidden, ffn)
    dev = [hip.to_device(a) for a in (g, u, d)]
    dsh = None
    if shared:
        dsh = tuple(hip.to_device(S.matrix(rng, t, r, c)) for t, r, c in
                    ((Q4_K, ffn, hidden), (Q4_K, ffn, hidden), (Q6_K, hidden, ffn)))
    return hip.moe_desc(hidden, ffn, n_expert, *dev, shared=dsh), dev, dsh


@pytest.mark.parametrize("mode", ["default", "two_launch"])
def test_noalloc_layer_matches_allocating_layer(hip, mode, monkeypatch):
    """default: the top-8 of 128 layer (2048 -> 768) and the top-8 of 256 plus
    shared expert layer run as the one-launch layer in both entry points;
    two_launch (KATALI_HIP_XCD=0): kernels A and B in both."""
    for k in ("KATALI_HIP_XCD", "KATALI_HIP_XCD_SHARED", "KATALI_HIP_FUSED"):
        monkeypatch.delenv(k, raising=False)
    if mode == "two_launch":
        monkeypatch.setenv("KATALI_HIP_XCD", "0")
    rng = np.random.default_rng(2024)
    # the larger calls first, then a smaller one
    for hidden, ffn, n_expert, n_sel, shared in ((2048, 768, 128, 8, False), (2048, 512, 256, 8, True),
                                                 (1024, 512, 32, 3, True)):
        print(f"[noalloc] mode={mode} hidden={hidden} ffn={ffn} n_expert={n_expert} n_sel={n_sel} shared={shared}",
              flush=True)
        desc, keep, keep_sh = _problem(hip, rng, hidden, ffn, n_expert, shared)
        x = hip.to_device(S.activation(rng, hidden))
        logits = hip.to_device(rng.standard_normal(n_expert).astype(np.float32))
        route = hip.moe_route(n_sel, logits=logits)
        y_ref, y_na = hip.alloc(hidden * 4), hip.alloc(hidden * 4)
        hip.moe_layer(desc, route, y_ref, x=x)
        hip.moe_layer_noalloc(desc, route, y_na, x=x)
        hip.sync()
        a, b = y_ref.download(np.uint32), y_na.download(np.uint32)
        assert np.array_equal(a, b), int(np.sum(a != b))
        assert np.any(a != 0)


def test_noalloc_layer_at_the_largest_shape(hip, two_launch_layer):
    """17 slots (16 routed + shared) at ffn 6912: the widest h any layer shape
    takes (17 * 216 * 36 = 132192 bytes, the LDS bound's maximum), inside the
    135168-byte scratch; device-filled weights, bit-identical outputs."""
    hidden, ffn, n_expert, n_sel = 1024, 6912, 16, 16
    print(f"[noalloc] largest: hidden={hidden} ffn={ffn} n_expert={n_expert} n_sel={n_sel} shared", flush=True)
    nb_gu, nb_d = n_expert * ffn * hidden // 256, n_expert * hidden * ffn // 256
    g, u = hip.alloc(nb_gu * 144), hip.alloc(nb_gu * 144)
    d = hip.alloc(nb_d * 210)
    sh = (hip.alloc(ffn * hidden // 256 * 144), hip.alloc(ffn * hidden // 256 * 144), hip.alloc(hidden * ffn // 256 * 210))
    for i, (t, b, n) in enumerate(((Q4_K, g, nb_gu), (Q4_K, u, nb_gu), (Q6_K, d, nb_d), (Q4_K, sh[0], ffn * hidden // 256),
                                   (Q4_K, sh[1], ffn * hidden // 256), (Q6_K, sh[2], hidden * ffn // 256))):
        hip.synth_fill(t, b, n, seed=77 + i)
    desc = hip.moe_desc(hidden, ffn, n_expert, g, u, d, shared=sh)
    hip.moe_check(desc, n_sel)
    rng = np.random.default_rng(5)
    x = hip.to_device(S.activation(rng, hidden))
    route = hip.moe_route(n_sel, logits=hip.to_device(rng.standard_normal(n_expert).astype(np.float32)))
    y_ref, y_na = hip.alloc(hidden * 4), hip.alloc(hidden * 4)
    hip.moe_layer(desc, route, y_ref, x=x)
    hip.moe_layer_noalloc(desc, route, y_na, x=x)
    hip.sync()
    a, b = y_ref.download(np.uint32), y_na.download(np.uint32)
    assert np.array_equal(a, b), int(np.sum(a != b))
    assert np.any(a != 0)


def test_noalloc_layer_refuses_oversized_shape(hip):
    # 16 routed experts + a shared expert at ffn 16384: kernel B would stage
    # 17 * 16384 * 11/8 bytes of h in LDS (and 313,344 bytes of h exceed the
    # scratch); refused before any launch
    hidden, ffn, n_expert = 2048, 16384, 16
    tiny = hip.alloc(256)
    desc = hip.moe_desc(hidden, ffn, n_expert, tiny, tiny, tiny, shared=(tiny, tiny, tiny))
    route = hip.moe_route(16, logits=tiny)
    y = hip.alloc(hidden * 4)
    with pytest.raises(HipError, match="LDS") as e:
        hip.moe_layer_noalloc(desc, route, y, x=tiny)
    assert e.value.rc == -4
    hip.sync()
