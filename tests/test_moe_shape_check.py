"""katali_hip_moe_check: the MoE shape rules, LDS bound included, answered
without a device (CPU only: the library's host arithmetic, no GPU call).

The boundary cases are worked out by hand from the kernels' LDS layouts:
kernel B stages every slot's q8_1 h as ffn + ffn/8 + ffn/4 bytes and keeps at
most 512 + 17 partial sums, so a layer fits gfx950's 163840 bytes of LDS while
n_slots * ffn * 11/8 + 2116 <= 163840; the batched layer's grouped down kernel
stages 8 pairs' h, 8 * ffn * 11/8 <= 163840. Kernel A's largest layout
(hidden 4096: 5632 + 65536 + 256 = 71424 bytes) always fits.
"""
import ctypes as C

import pytest

import katali_hip as K

OK, E_INVALID, E_UNSUPPORTED = 0, -1, -4
FAKE = 0x1000   # descriptors are read for their shape only; no pointer is touched


@pytest.fixture(scope="module")
def lib():
    return K.load_library()


def desc(hidden, ffn, n_expert=16, shared=False, down=K.Q6_K, gate=K.Q4_K):
    d = K.KataliHipMoe(C.sizeof(K.KataliHipMoe), gate, gate, down, hidden, ffn, n_expert, FAKE, FAKE, FAKE,
                       None, None, None)
    if shared:
        d.gate_shexp = d.up_shexp = d.down_shexp = FAKE
    return d


def check(lib, d, n_sel, n_tokens=0):
    rc = lib.katali_hip_moe_check(C.byref(d), n_sel, n_tokens)
    return rc, lib.katali_hip_last_error().decode()


@pytest.mark.parametrize("slots,ffn_ok,ffn_bad", [
    (17, 6912, 7168),      # 17 * 6912 * 11/8 + 2116 = 163684; 7168 -> 169668
    (16, 7168, 7424),      # 159812 / 165444
    (9, 13056, 13312),     # 163684 / 166852
    (8, 14592, 14848),     # 162628 / 165444
])
def test_layer_lds_boundary(lib, slots, ffn_ok, ffn_bad):
    shared = slots == 17 or slots == 9
    n_sel = slots - (1 if shared else 0)
    for hidden in (256, 2048, 4096):
        assert check(lib, desc(hidden, ffn_ok, shared=shared), n_sel)[0] == OK
        rc, msg = check(lib, desc(hidden, ffn_bad, shared=shared), n_sel)
        assert rc == E_UNSUPPORTED and "LDS" in msg and "163840" in msg, msg


def test_layer_up_to_seven_slots_takes_every_ffn(lib):
    # 7 * 16384 * 11/8 + 2116 = 159812
    for down in (K.Q4_K, K.Q6_K):
        assert check(lib, desc(4096, 16384, down=down), 7)[0] == OK
        assert check(lib, desc(4096, 16384, down=down, shared=True), 7)[0] == E_UNSUPPORTED


def test_advised_shapes_are_refused(lib):
    # 17 slots x ffn 8192 (191 KB of kernel B LDS), 8 slots x ffn 16384 (180 KB)
    assert check(lib, desc(2048, 8192, shared=True), 16)[0] == E_UNSUPPORTED
    assert check(lib, desc(2048, 16384), 8)[0] == E_UNSUPPORTED


def test_batch_lds_boundary(lib):
    # grouped down: 8 * 14848 * 11/8 = 163328 fits, 8 * 15104 * 11/8 = 166144 does not
    for t in (1, 16, 64):
        assert check(lib, desc(2048, 14848), 8, t)[0] == OK
        rc, msg = check(lib, desc(2048, 15104), 8, t)
        assert rc == E_UNSUPPORTED and "batch" in msg, msg
    # the batch bound does not depend on the slot count
    assert check(lib, desc(4096, 14848, shared=True), 16, 64)[0] == OK


def test_shape_and_selection_rules(lib):
    assert check(lib, desc(2048, 768, n_expert=128), 8)[0] == OK
    assert check(lib, desc(2048, 768), 17)[0] == E_INVALID
    assert check(lib, desc(2048, 768), -1)[0] == E_INVALID
    assert check(lib, desc(2048, 768), 0)[0] == E_INVALID               # no shared expert
    assert check(lib, desc(2048, 768, shared=True), 0)[0] == OK         # the shared expert alone
    assert check(lib, desc(2048, 768, n_expert=4), 5)[0] == E_INVALID   # n_sel > n_expert
    assert check(lib, desc(2048, 768, n_expert=513), 8)[0] == E_INVALID
    assert check(lib, desc(3072, 768), 8)[0] == E_UNSUPPORTED            # hidden not in the set
    assert check(lib, desc(2048, 700), 8)[0] == E_UNSUPPORTED            # ffn % 256
    assert check(lib, desc(2048, 16640), 1)[0] == E_UNSUPPORTED          # ffn above 16384
    assert check(lib, desc(2048, 768, gate=K.Q6_K), 8)[0] == E_UNSUPPORTED
    assert check(lib, desc(2048, 768), 8, 65)[0] == E_INVALID
    d = desc(2048, 768)
    d.gate_shexp = FAKE                                                 # half a shared expert
    assert check(lib, d, 8)[0] == E_INVALID
    d = desc(2048, 768)
    d.struct_size = 8
    assert check(lib, d, 8)[0] == E_INVALID
    assert lib.katali_hip_moe_check(None, 8, 0) == E_INVALID
