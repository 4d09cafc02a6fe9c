"""ctypes bindings for the oracle (libkq_oracle.so) and for the reference CPU path
compiled from its own sources (oracle/_ref/libkatali_ref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product path.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "libkq_oracle.so")
REF_SO = os.path.join(HERE, "_ref", "libkatali_ref.so")

F32, Q8_1, Q4_K, Q6_K = 0, 9, 12, 14
BLOCK = {Q4_K: (256, 144), Q6_K: (256, 210), Q8_1: (32, 36), F32: (1, 4)}

_vp, _u64, _u32, _i32, _f32 = C.c_void_p, C.c_uint64, C.c_uint32, C.c_int, C.c_float


def row_bytes(t: int, n: int) -> int:
    bs, bb = BLOCK[t]
    assert n % bs == 0
    return n // bs * bb


def _ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_vp)


class KqoMoe(C.Structure):
    _fields_ = [("gate_type", _u32), ("up_type", _u32), ("down_type", _u32),
                ("hidden", _u64), ("ffn", _u64), ("n_expert", _u32),
                ("gate_exps", _vp), ("up_exps", _vp), ("down_exps", _vp),
                ("shared_ffn", _u64), ("gate_sh", _vp), ("up_sh", _vp), ("down_sh", _vp)]


class Oracle:
    """Thin numpy front end over libkq_oracle.so."""

    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        L = self.lib = C.CDLL(path)
        sig = {
            "kqo_f16_to_f32": (_f32, [C.c_uint16]),
            "kqo_f32_to_f16_ref": (C.c_uint16, [_f32]),
            "kqo_f32_to_f16_rne": (C.c_uint16, [_f32]),
            "kqo_dequant": (_i32, [_u32, _vp, _u64, _vp]),
            "kqo_vec_dot_ref": (_f32, [_u32, _vp, _vp, _u64]),
            "kqo_dot_q4_K_scalar": (_f32, [_vp, _vp, _u64]),
            "kqo_dot_q4_K_avx2order": (_f32, [_vp, _vp, _u64]),
            "kqo_dot_q6_K_avx2order": (_f32, [_vp, _vp, _u64]),
            "kqo_matvec_f32x": (_i32, [_u32, _vp, _u64, _u64, _vp, _vp]),
            "kqo_matvec_f32x_mt": (_i32, [_u32, _vp, _u64, _u64, _vp, _vp, _i32]),
            "kqo_quantize_q8_1": (_i32, [_vp, _u64, _vp]),
            "kqo_q4K_q8_isums": (_i32, [_vp, _vp, _u64, _vp]),
            "kqo_q6K_q8_isums": (_i32, [_vp, _vp, _u64, _vp]),
            "kqo_dot_q4K_q8": (_f32, [_vp, _vp, _u64]),
            "kqo_dot_q4K_q8_f64": (_f32, [_vp, _vp, _u64]),
            "kqo_q4K_q8_term": (_f32, [_vp, _i32, _vp]),
            "kqo_dot_q6K_q8": (_f32, [_vp, _vp, _u64]),
            "kqo_matvec_q8": (_i32, [_u32, _vp, _u64, _u64, _vp, _vp]),
            "kqo_expf": (_f32, [_f32]),
            "kqo_silu_mul": (_f32, [_f32, _f32]),
            "kqo_exp_ref_poly": (_f32, [_f32]),
            "kqo_silu_mul_ref": (None, [_vp, _vp, _u64]),
            "kqo_router_topk": (_i32, [_vp, _i32, _i32, _vp, _vp]),
            "kqo_argmax_greedy": (_i32, [_vp, _i32]),
            "kqo_rmsnorm": (None, [_vp, _vp, _u64, _f32, _vp]),
            "kqo_add_rmsnorm": (None, [_vp, _vp, _f32, _vp, _u64, _f32, _vp]),
            "kqo_moe_layer_q8": (_i32, [C.POINTER(KqoMoe), _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp]),
            "kqo_moe_down_q8": (_i32, [C.POINTER(KqoMoe), _i32, _vp, _vp, _vp, _vp]),
            "kqo_moe_layer_f32": (_i32, [C.POINTER(KqoMoe), _vp, _i32, _vp, _vp, _vp]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args

    # -- formats ----------------------------------------------------------
    def f16_to_f32(self, h: int) -> float:
        return self.lib.kqo_f16_to_f32(h)

    def dequant(self, t: int, data: np.ndarray, n: int) -> np.ndarray:
        out = np.empty(n, np.float32)
        assert self.lib.kqo_dequant(t, _ptr(data), n, _ptr(out)) == 0
        return out

    def quantize_q8_1(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(x.size // 32 * 36, np.uint8)
        assert self.lib.kqo_quantize_q8_1(_ptr(x), x.size, _ptr(out)) == 0
        return out

    # -- dots -------------------------------------------------------------
    def matvec_f32x(self, t: int, w: np.ndarray, rows: int, cols: int, x: np.ndarray,
                    threads: int = 1) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty(rows, np.float32)
        if threads > 1:
            rc = self.lib.kqo_matvec_f32x_mt(t, _ptr(w), rows, cols, _ptr(x), _ptr(y), threads)
        else:
            rc = self.lib.kqo_matvec_f32x(t, _ptr(w), rows, cols, _ptr(x), _ptr(y))
        assert rc == 0
        return y

    def matvec_q8(self, t: int, w: np.ndarray, rows: int, cols: int, q8: np.ndarray) -> np.ndarray:
        y = np.empty(rows, np.float32)
        assert self.lib.kqo_matvec_q8(t, _ptr(w), rows, cols, _ptr(q8), _ptr(y)) == 0
        return y

    def dot_q4K_q8(self, row: np.ndarray, q8: np.ndarray, f64: bool = False) -> float:
        """One Q4_K row against q8_1 blocks: the q8 path's pairwise fp32 dot,
        or (f64=True) the same terms' closed form in double."""
        nb = row.size // 144
        fn = self.lib.kqo_dot_q4K_q8_f64 if f64 else self.lib.kqo_dot_q4K_q8
        return float(np.float32(fn(_ptr(row), _ptr(q8), nb)))

    def q4K_q8_term(self, blk: np.ndarray, j: int, q8blk: np.ndarray) -> float:
        return float(np.float32(self.lib.kqo_q4K_q8_term(_ptr(blk), j, _ptr(q8blk))))

    def vec_dot_ref_rows(self, t: int, w: np.ndarray, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
        rb = row_bytes(t, cols)
        x = np.ascontiguousarray(x, np.float32)
        base = w.ctypes.data
        return np.array([self.lib.kqo_vec_dot_ref(t, _vp(base + r * rb), _ptr(x), cols)
                         for r in range(rows)], np.float32)

    def isums(self, t: int, w: np.ndarray, rows: int, cols: int, q8: np.ndarray) -> np.ndarray:
        """Per-row integer block sums: Q4_K -> [rows, cols/32], Q6_K -> [rows, cols/16]."""
        rb, nb = row_bytes(t, cols), cols // 256
        per = 8 if t == Q4_K else 16
        out = np.empty((rows, nb * per), np.int32)
        fn = self.lib.kqo_q4K_q8_isums if t == Q4_K else self.lib.kqo_q6K_q8_isums
        base, obase = w.ctypes.data, out.ctypes.data
        for r in range(rows):
            fn(_vp(base + r * rb), _ptr(q8), nb, _vp(obase + r * nb * per * 4))
        return out

    # -- activation / router -----------------------------------------------
    def expf(self, x: float) -> float:
        return self.lib.kqo_expf(x)

    def silu_mul(self, g: np.ndarray, u: np.ndarray) -> np.ndarray:
        return np.array([self.lib.kqo_silu_mul(float(a), float(b)) for a, b in zip(g, u)], np.float32)

    def silu_mul_ref(self, g: np.ndarray, u: np.ndarray) -> np.ndarray:
        g = np.array(g, np.float32, copy=True)
        u = np.ascontiguousarray(u, np.float32)
        self.lib.kqo_silu_mul_ref(_ptr(g), _ptr(u), g.size)
        return g

    def router_topk(self, logits: np.ndarray, k: int):
        logits = np.ascontiguousarray(logits, np.float32)
        ids = np.empty(k, np.int32)
        w = np.empty(k, np.float32)
        assert self.lib.kqo_router_topk(_ptr(logits), logits.size, k, _ptr(ids), _ptr(w)) == 0
        return ids, w

    def rmsnorm(self, x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        out = np.empty_like(x)
        self.lib.kqo_rmsnorm(_ptr(x), _ptr(w), x.size, eps, _ptr(out))
        return out

    def add_rmsnorm(self, x: np.ndarray, delta: np.ndarray, scale: float, w: np.ndarray, eps: float):
        """(x + scale*delta, its RMSNorm * w); x is not modified."""
        x = np.array(x, np.float32, copy=True)
        delta = np.ascontiguousarray(delta, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        out = np.empty_like(x)
        self.lib.kqo_add_rmsnorm(_ptr(x), _ptr(delta), scale, _ptr(w), x.size, eps, _ptr(out))
        return x, out

    def argmax_greedy(self, logits: np.ndarray) -> int:
        logits = np.ascontiguousarray(logits, np.float32)
        return int(self.lib.kqo_argmax_greedy(_ptr(logits), logits.size))

    # -- MoE ---------------------------------------------------------------
    @staticmethod
    def moe_desc(hidden, ffn, n_expert, gate, up, down, gate_type=Q4_K, up_type=Q4_K,
                 down_type=Q6_K, shared=None) -> KqoMoe:
        d = KqoMoe(gate_type, up_type, down_type, hidden, ffn, n_expert,
                   _ptr(gate), _ptr(up), _ptr(down), 0, None, None, None)
        if shared is not None:
            sffn, sg, su, sd = shared
            d.shared_ffn, d.gate_sh, d.up_sh, d.down_sh = sffn, _ptr(sg), _ptr(su), _ptr(sd)
        # the struct holds raw pointers: keep the arrays alive with it
        d._keep = (gate, up, down, shared)
        return d

    def moe_layer_q8(self, desc: KqoMoe, x, ids, w, with_stages=False):
        x = np.ascontiguousarray(x, np.float32)
        ids = np.ascontiguousarray(ids, np.int32)
        w = np.ascontiguousarray(w, np.float32)
        y = np.empty(desc.hidden, np.float32)
        n_slots = ids.size + (1 if desc.shared_ffn else 0)
        g = u = hq = None
        if with_stages:
            g = np.zeros((n_slots, desc.ffn), np.float32)
            u = np.zeros((n_slots, desc.ffn), np.float32)
            hq = np.zeros((n_slots, desc.ffn // 32 * 36), np.uint8)
        rc = self.lib.kqo_moe_layer_q8(C.byref(desc), _ptr(x), ids.size, _ptr(ids), _ptr(w),
                                       _ptr(y), _ptr(g), _ptr(u), _ptr(hq))
        assert rc == 0
        return (y, g, u, hq) if with_stages else y

    def moe_down_q8(self, desc: KqoMoe, ids, w, hq8):
        ids = np.ascontiguousarray(ids, np.int32)
        w = np.ascontiguousarray(w, np.float32)
        hq8 = np.ascontiguousarray(hq8, np.uint8)
        y = np.empty(desc.hidden, np.float32)
        assert self.lib.kqo_moe_down_q8(C.byref(desc), ids.size, _ptr(ids), _ptr(w), _ptr(hq8), _ptr(y)) == 0
        return y

    def moe_layer_f32(self, desc: KqoMoe, x, ids, w):
        x = np.ascontiguousarray(x, np.float32)
        ids = np.ascontiguousarray(ids, np.int32)
        w = np.ascontiguousarray(w, np.float32)
        y = np.empty(desc.hidden, np.float32)
        assert self.lib.kqo_moe_layer_f32(C.byref(desc), _ptr(x), ids.size, _ptr(ids), _ptr(w), _ptr(y)) == 0
        return y


class MatvecJob(C.Structure):
    """KataliMatvecJob (V/include/katali_gguf_dtype.h:166-172)."""
    _fields_ = [("type", _u32), ("w", _vp), ("rows", _u64), ("y", _vp), ("role", _i32)]


class RefCPU:
    """The reference's own CPU path, compiled from its sources into oracle/_ref."""

    def __init__(self, path: str = REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        L = self.lib = C.CDLL(path)
        L.katali_ggml_vec_dot.restype = _f32
        L.katali_ggml_vec_dot.argtypes = [_u32, _vp, _vp, _u64]
        L.katali_ggml_vec_dot_ref.restype = _f32
        L.katali_ggml_vec_dot_ref.argtypes = [_u32, _vp, _vp, _u64]
        L.katali_ggml_vec_dot_scalar.restype = _f32
        L.katali_ggml_vec_dot_scalar.argtypes = [_u32, _vp, _vp, _u64]
        L.katali_ggml_matvec.restype = None
        L.katali_ggml_matvec.argtypes = [_u32, _vp, _u64, _u64, _vp, _vp, _i32, _vp, _vp, _u64]
        L.katali_ggml_matvec_fused.restype = None
        L.katali_ggml_matvec_fused.argtypes = [C.POINTER(MatvecJob), _i32, _u64, _vp, _i32, _vp, _vp, _u64]
        L.katali_ggml_dequant_ref.restype = _i32
        L.katali_ggml_dequant_ref.argtypes = [_u32, _vp, _u64, _vp]
        L.katali_ggml_silu_mul_avx2.restype = _i32
        L.katali_ggml_silu_mul_avx2.argtypes = [_vp, _vp, C.c_size_t]
        L.katali_gguf_softmax.restype = None
        L.katali_gguf_softmax.argtypes = [_vp, C.c_size_t]
        L.katali_gguf_rmsnorm.restype = None
        L.katali_gguf_rmsnorm.argtypes = [_vp, _vp, C.c_size_t, _f32, _vp]
        L.katali_gguf_add_inplace.restype = None
        L.katali_gguf_add_inplace.argtypes = [_vp, _vp, C.c_size_t]
        L.katali_ggml_simd_available.restype = _i32
        L.katali_gguf_set_threads.argtypes = [_i32]
        L.katali_gguf_threads_shutdown.restype = None
        L.kref_f32_to_f16.restype = C.c_uint16
        L.kref_f32_to_f16.argtypes = [_f32]
        L.kref_f16_to_f32.restype = _f32
        L.kref_f16_to_f32.argtypes = [C.c_uint16]
        L.kref_sample_greedy.restype = _i32
        L.kref_sample_greedy.argtypes = [_vp, _i32]

    def gguf_table(self, path: str, cap: int = 64):
        """The reference reader's verdict on a GGUF file: None when it refuses
        it, else (header (version, alignment, data_offset), tensor table)."""
        L = self.lib
        if not hasattr(self, "_gguf_sig"):
            L.kref_gguf_table.restype = C.c_int64
            L.kref_gguf_table.argtypes = [C.c_char_p, C.c_int64] + [_vp] * 8
            self._gguf_sig = True
        names = C.create_string_buffer(64 * cap)
        nd = np.zeros(cap, np.uint32)
        dims = np.zeros((cap, 4), np.uint64)
        types = np.zeros(cap, np.uint32)
        offs = np.zeros(cap, np.uint64)
        nbytes = np.zeros(cap, np.uint64)
        pos = np.zeros(cap, np.int64)
        hdr = np.zeros(3, np.uint64)
        n = L.kref_gguf_table(path.encode(), cap, names, _ptr(nd), _ptr(dims), _ptr(types), _ptr(offs), _ptr(nbytes),
                              _ptr(pos), _ptr(hdr))
        if n < 0:
            return None
        raw = names.raw
        table = [{"name": raw[64 * i:64 * i + 64].split(b"\0")[0].decode(), "n_dims": int(nd[i]),
                  "dims": [int(v) for v in dims[i]], "type": int(types[i]), "offset": int(offs[i]),
                  "nbytes": int(nbytes[i]), "data_pos": int(pos[i])} for i in range(min(n, cap))]
        return (int(hdr[0]), int(hdr[1]), int(hdr[2])), table

    def simd(self) -> bool:
        return bool(self.lib.katali_ggml_simd_available())

    def sample_greedy(self, logits: np.ndarray) -> int:
        """katali_gguf_sample with temperature 0 (gguf_sampler.c:62-66)."""
        logits = np.ascontiguousarray(logits, np.float32)
        return int(self.lib.kref_sample_greedy(_ptr(logits), logits.size))

    def dequant(self, t, data, n):
        out = np.empty(n, np.float32)
        assert self.lib.katali_ggml_dequant_ref(t, _ptr(data), n, _ptr(out)) == 0
        return out

    def matvec(self, t, w, rows, cols, x, threads=1, sums=True):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty(rows, np.float32)
        scratch = np.empty(max(cols // 256 * 64, 1), np.float32) if sums else None
        self.lib.katali_ggml_matvec(t, _ptr(w), rows, cols, _ptr(x), _ptr(y), threads, None,
                                    _ptr(scratch), 0 if scratch is None else scratch.size)
        return y

    def matvec_fused(self, jobs, cols, x, threads, sums_buf):
        arr = (MatvecJob * len(jobs))(*jobs)
        self.lib.katali_ggml_matvec_fused(arr, len(jobs), cols, _ptr(x), threads, None,
                                          _ptr(sums_buf), sums_buf.size)

    def vec_dot_rows(self, t, w, rows, cols, x, which="fast"):
        rb = row_bytes(t, cols)
        fn = {"fast": self.lib.katali_ggml_vec_dot, "ref": self.lib.katali_ggml_vec_dot_ref,
              "scalar": self.lib.katali_ggml_vec_dot_scalar}[which]
        x = np.ascontiguousarray(x, np.float32)
        base = w.ctypes.data
        return np.array([fn(t, _vp(base + r * rb), _ptr(x), cols) for r in range(rows)], np.float32)

    def silu_mul(self, g, u):
        g = np.array(g, np.float32, copy=True)
        u = np.ascontiguousarray(u, np.float32)
        assert self.lib.katali_ggml_silu_mul_avx2(_ptr(g), _ptr(u), g.size) == 0
        return g

    def softmax(self, x):
        x = np.array(x, np.float32, copy=True)
        self.lib.katali_gguf_softmax(_ptr(x), x.size)
        return x

    def rmsnorm(self, x, w, eps):
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        out = np.empty_like(x)
        self.lib.katali_gguf_rmsnorm(_ptr(x), _ptr(w), x.size, eps, _ptr(out))
        return out

    def add_inplace(self, a, b):
        a = np.array(a, np.float32, copy=True)
        self.lib.katali_gguf_add_inplace(_ptr(a), _ptr(np.ascontiguousarray(b, np.float32)), a.size)
        return a


def ref_available() -> bool:
    return os.path.exists(REF_SO)
