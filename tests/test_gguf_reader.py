"""The GGUF reader (katali-lab_amd/host/katali_hip_gguf.c) against the
engine's own reader compiled from its sources (katali_gguf_open,
V/src/gguf_reader.c:351-543): on every file below both accept or both refuse,
and an accepted file gives the same header and tensor table. The files follow
the reference's own reader tests (V/tests/test_core.c:146-280: a valid file
with string/int/float/bool/array metadata; bad magic, bad version, truncated,
out-of-range offset, unknown tensor type, nested array) and widen them."""
import struct

import numpy as np
import pytest

import gguf_writer as W
from katali_hip_gguf import Gguf, GgufError, load


@pytest.fixture(scope="module")
def lib():
    return load()


def ours(lib, path):
    try:
        g = Gguf(str(path), lib)
    except GgufError:
        return None
    try:
        return (g.version, g.alignment, g.data_offset), g.tensors()
    finally:
        g.close()


def minimal(version=3, t_type=0, offset=None, align=None):
    """The reference test's minimal file: 7 metadata entries, one F32 4x2."""
    w = W.GgufWriter(version=version)
    w.kv("general.architecture", W.STR, "qwen3").kv("qwen3.block_count", W.U32, 1)
    w.kv("qwen3.rope.freq_base", W.F32, 10000.0).kv("general.flag", W.BOOL, 1)
    w.kv_array("tokenizer.ggml.tokens", W.STR, ["a", "b", "c", "Ġ"])
    w.kv_array("tokenizer.ggml.token_type", W.I32, [1, 1, 1, 1]).kv_array("test.nums", W.I32, [10, 20, 30])
    if align is not None:
        w.kv(*align)
    w.tensor("t0", [4, 2], t_type, np.arange(1, 9, dtype=np.float32), offset)
    return w


def moe_file():
    """Several tensor types and ranks, a 3-D expert stack, 64-byte alignment."""
    rng = np.random.default_rng(0)
    w = W.GgufWriter(alignment=64)
    w.kv("general.architecture", W.STR, "qwen3moe").kv("general.alignment", W.U32, 64)
    w.kv("qwen3moe.expert_count", W.U32, 4).kv("qwen3moe.attention.layer_norm_rms_epsilon", W.F32, 1e-6)
    w.kv("qwen3moe.block_count", W.U64, 2).kv("x.neg", W.I32, -5).kv("x.f64", W.F64, 2.5)
    w.tensor("blk.0.ffn_gate_exps.weight", [256, 2, 4], 12, rng.integers(0, 255, 4 * 2 * 144, dtype=np.uint8))
    w.tensor("blk.0.ffn_down_exps.weight", [256, 256, 4], 14, rng.integers(0, 255, 4 * 256 * 210, dtype=np.uint8))
    w.tensor("blk.0.ffn_gate_inp.weight", [256, 4], 0, rng.standard_normal(1024).astype(np.float32))
    w.tensor("f16", [7], 1, np.zeros(7, np.float16))
    w.tensor("odd", [3, 5], 200, np.zeros(8, np.uint8))        # unknown type: no data
    w.tensor("i32", [3], 26, np.array([1, 2, 3], np.int32))
    return w


def malformed():
    cases = {}
    b = bytearray(minimal().build()); b[0] = ord("X"); cases["bad_magic"] = bytes(b)
    for v in (0, 4, 99):
        cases[f"version_{v}"] = minimal(version=v).build()
    cases["truncated_8"] = minimal().build(truncate=8)
    cases["truncated_header"] = minimal().build()[:20]
    cases["offset_far"] = minimal(offset=1 << 40).build()
    w = minimal(); w.tensors[0] = ("t0", [4, 2], 0, np.zeros(2, np.float32).tobytes(), 16)   # 8 of 32 bytes
    cases["tensor_truncated"] = w.build()
    for nd in (0, 5):
        w = minimal(); w.tensors[0] = ("t0", [1] * nd, 0, b"", 0); cases[f"rank_{nd}"] = w.build()
    w = minimal(); w.tensors[0] = ("t0", [4, 0], 0, b"", 0); cases["zero_dim"] = w.build()
    w = minimal(); w.tensors[0] = ("t0", [1 << 40, 1 << 40], 0, b"", 0); cases["dims_overflow"] = w.build()
    w = minimal(); w.kv_raw(W.gstr("bad") + struct.pack("<IIQ", W.ARR, W.ARR, 1)); cases["nested_array"] = w.build()
    w = minimal(); w.kv_raw(W.gstr("big") + struct.pack("<IIQ", W.ARR, W.U8, 1 << 40)); cases["array_count"] = w.build()
    w = minimal(); w.kv_raw(W.gstr("big") + struct.pack("<IIQ", W.ARR, W.U64, 200)); cases["array_payload"] = w.build()
    w = minimal(); w.kv_raw(W.gstr("s") + struct.pack("<IQ", W.STR, 1 << 40)); cases["string_len"] = w.build()
    w = minimal(); w.kv_raw(W.gstr("t") + struct.pack("<I", 13) + b"\0" * 8); cases["kv_type_13"] = w.build()
    w = minimal(); w.kv_raw(W.gstr("t") + struct.pack("<IIQ", W.ARR, 13, 1) + b"\0" * 8); cases["array_type_13"] = w.build()
    w = minimal(); w.n_kv = 1 << 40; cases["kv_count"] = w.build()
    w = minimal(); w.n_tensors = 2; cases["tensor_count_short"] = w.build()
    w = W.GgufWriter(alignment=1 << 20); w.kv("general.alignment", W.U32, 1 << 20)
    w.tensor("t", [3], 200, b"")
    cases["data_offset_past_end"] = w.build()[: 200]
    cases["empty"] = b""
    return cases


def valid():
    files = {"minimal": minimal().build(), "moe": moe_file().build()}
    for v in (1, 2):
        files[f"version_{v}"] = minimal(version=v).build()
    files["unknown_type"] = minimal(t_type=200).build()
    files["align_4_ignored"] = minimal(align=("general.alignment", W.U32, 4)).build()
    files["align_str_ignored"] = minimal(align=("general.alignment", W.STR, "64")).build()
    w = minimal(align=("general.alignment", W.U32, 128)); w.alignment = 128; files["align_128"] = w.build()
    w = minimal(align=("general.alignment", W.I32, 256)); w.alignment = 256; files["align_i32"] = w.build()
    w = W.GgufWriter(); w.kv("k", W.STR, "v"); files["no_tensors"] = w.build()
    return files


@pytest.mark.parametrize("name", sorted(valid()))
def test_reader_accepts_like_reference(lib, refcpu, tmp_path, name):
    p = tmp_path / f"{name}.gguf"
    p.write_bytes(valid()[name])
    want = refcpu.gguf_table(str(p))
    got = ours(lib, p)
    assert want is not None, "the reference refuses this file"
    assert got == want


@pytest.mark.parametrize("name", sorted(malformed()))
def test_reader_refuses_like_reference(lib, refcpu, tmp_path, name):
    p = tmp_path / f"{name}.gguf"
    p.write_bytes(malformed()[name])
    assert refcpu.gguf_table(str(p)) is None, "the reference accepts this file"
    assert ours(lib, p) is None


def test_reader_metadata_and_table(lib, tmp_path):
    """Values as written (independent of the reference)."""
    p = tmp_path / "moe.gguf"
    p.write_bytes(moe_file().build())
    g = Gguf(str(p), lib)
    try:
        assert g.version == 3 and g.alignment == 64 and g.data_offset % 64 == 0
        assert g.get_str("general.architecture") == "qwen3moe"
        assert g.get_int("qwen3moe.expert_count") == 4 and g.get_int("qwen3moe.block_count") == 2
        assert g.get_int("x.neg") == -5 and g.get_float("x.f64") == 2.5
        assert abs(g.get_float("qwen3moe.attention.layer_norm_rms_epsilon") - 1e-6) < 1e-12
        assert g.get_int("missing", 7) == 7 and g.get_str("missing") is None
        t = {e["name"]: e for e in g.tensors()}
        assert t["blk.0.ffn_gate_exps.weight"]["nbytes"] == 4 * 2 * 144
        assert t["blk.0.ffn_down_exps.weight"]["nbytes"] == 4 * 256 * 210
        assert t["blk.0.ffn_gate_inp.weight"]["nbytes"] == 4096 and t["f16"]["nbytes"] == 14
        assert t["odd"]["nbytes"] == 0 and t["odd"]["data_pos"] == -1
        raw = p.read_bytes()
        e = t["blk.0.ffn_gate_inp.weight"]
        assert raw[e["data_pos"]:e["data_pos"] + 16] == moe_file().tensors[2][3][:16]
    finally:
        g.close()


@pytest.mark.parametrize("t,n,want", [(0, 7, 28), (1, 3, 6), (12, 512, 288), (14, 256, 210), (8, 64, 68),
                                      (12, 100, 0), (200, 256, 0), (30, 5, 10)])
def test_row_bytes(lib, t, n, want):
    assert lib.katali_hip_ggml_row_bytes(t, n) == want


def test_reader_matches_reference_at_every_truncation(lib, refcpu, tmp_path):
    """The minimal file cut at every length (and the multi-tensor file at
    every 7th): same verdict and table as the reference reader."""
    for name, raw, step in (("minimal", minimal().build(), 1), ("moe", moe_file().build(), 7)):
        for n in range(0, len(raw) + 1, step):
            p = tmp_path / f"{name}_{n}.gguf"
            p.write_bytes(raw[:n])
            assert ours(lib, p) == refcpu.gguf_table(str(p)), (name, n)
            p.unlink()


def test_reader_matches_reference_on_corrupted_bytes(lib, refcpu, tmp_path):
    """Random single-byte corruptions of the header and directory: same
    verdict and table as the reference reader."""
    raw = bytearray(minimal().build())
    head = len(raw) - 32          # header, metadata and tensor directory
    rng = np.random.default_rng(11)
    for i in range(300):
        b = bytearray(raw)
        pos = int(rng.integers(0, head))
        b[pos] = int(rng.integers(0, 256))
        p = tmp_path / f"c{i}.gguf"
        p.write_bytes(bytes(b))
        assert ours(lib, p) == refcpu.gguf_table(str(p)), (pos, b[pos])
        p.unlink()
