"""ctypes binding of libkatali_hip (include/katali_hip.h) for Python callers.

This is the binding a Python maintainer would add for the library, and what
the tests and bench.py drive. It loads the in-tree build (or KATALI_HIP_DLL)
and raises if the library is missing: there is no CPU fallback here.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
DEFAULT_SO = os.path.join(PKG, "libkatali_hip.so")

Q4_K, Q6_K = 12, 14
BLOCK_BYTES = {Q4_K: 144, Q6_K: 210}

_vp, _u64, _u32, _i32, _i64, _f32, _sz = (C.c_void_p, C.c_uint64, C.c_uint32, C.c_int32, C.c_int64,
                                          C.c_float, C.c_size_t)

# Every exported symbol with (restype, argtypes); include/katali_hip.h is the
# source of truth and tests check the two agree.
SIGNATURES = {
    "katali_hip_abi_version": (C.c_int, []),
    "katali_hip_last_error": (C.c_char_p, []),
    "katali_hip_probe": (C.c_int, []),
    "katali_hip_status": (C.c_char_p, []),
    "katali_hip_malloc": (C.c_int, [C.POINTER(_vp), _sz]),
    "katali_hip_free": (C.c_int, [_vp]),
    "katali_hip_upload": (C.c_int, [_vp, _vp, _sz]),
    "katali_hip_download": (C.c_int, [_vp, _vp, _sz]),
    "katali_hip_supports_type": (C.c_int, [_u32]),
    "katali_hip_matvec": (C.c_int, [_u32, _vp, _u64, _u64, _vp, _vp]),
    "katali_hip_sync": (C.c_int, []),
    "katali_hip_memset": (C.c_int, [_vp, C.c_int, _sz]),
    "katali_hip_set_stream": (C.c_int, [_vp]),
    "katali_hip_quantize_q8_1": (C.c_int, [_vp, _u64, _vp]),
    "katali_hip_matvec_q8": (C.c_int, [_u32, _vp, _u64, _u64, _vp, _vp]),
    "katali_hip_matvec_dp4a": (C.c_int, [_u32, _vp, _u64, _u64, _vp, _vp]),
    "katali_hip_block_isums": (C.c_int, [_u32, _vp, _u64, _u64, _vp, _vp]),
    "katali_hip_moe_layer": (C.c_int, [_vp, _vp, _vp, _vp, _vp]),
    "katali_hip_moe_layer_debug": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "katali_hip_moe_layer_noalloc": (C.c_int, [_vp, _vp, _vp, _vp, _vp]),
    "katali_hip_moe_check": (C.c_int, [_vp, _i32, _u32]),
    "katali_hip_moe_layer_normed": (C.c_int, [_vp, _vp, _i32, _vp, _vp, _vp]),
    "katali_hip_step_advance": (C.c_int, [_vp, _i32]),
    "katali_hip_graph_begin": (C.c_int, []),
    "katali_hip_graph_end": (C.c_int, [C.POINTER(_vp)]),
    "katali_hip_graph_launch": (C.c_int, [_vp]),
    "katali_hip_graph_destroy": (C.c_int, [_vp]),
    "katali_hip_event_create": (C.c_int, [C.POINTER(_vp)]),
    "katali_hip_event_record": (C.c_int, [_vp]),
    "katali_hip_event_elapsed": (C.c_int, [_vp, _vp, C.POINTER(_f32)]),
    "katali_hip_event_destroy": (C.c_int, [_vp]),
    "katali_hip_selftest": (C.c_int, [C.c_char_p, _sz]),
    "katali_hip_synth_fill": (C.c_int, [_u32, _vp, _u64, _u64, _f32]),
    "katali_hip_synth_normal": (C.c_int, [_vp, _u64, _u64, _f32]),
    "katali_hip_copy": (C.c_int, [_vp, _vp, _sz]),
    "katali_hip_argmax": (C.c_int, [_vp, _u64, _vp]),
    "katali_hip_moe_batch": (C.c_int, [_vp, _vp, _vp, _vp]),
    "katali_hip_matvec_multi": (C.c_int, [C.c_int, _vp, _vp, _vp, _u64, _vp, _vp]),
    "katali_hip_matvec_multi_dp4a": (C.c_int, [C.c_int, _vp, _vp, _vp, _u64, _vp, _vp]),
    "katali_hip_rmsnorm": (C.c_int, [_vp, _vp, _u64, _f32, _vp]),
    "katali_hip_add_rmsnorm": (C.c_int, [_vp, _vp, _f32, _vp, _u64, _f32, _vp]),
    "katali_hip_moe_route_batch": (C.c_int, [_vp, _u32, _u32, _i32, _vp, _vp]),
    "katali_hip_rmsnorm_matvec_f32": (C.c_int, [_vp, _vp, _f32, _vp, _vp, _u64, _f32, _vp, _vp, _u64, _vp]),
    "katali_hip_moe_stack_create": (C.c_int, [_vp, _i32, _i32, _f32, _vp, _i32, C.POINTER(_vp)]),
    "katali_hip_moe_stack_run": (C.c_int, [_vp, _vp, _vp, _f32]),
    "katali_hip_moe_stack_destroy": (C.c_int, [_vp]),
    "katali_hip_one_launch": (C.c_int, [_i32]),
    "katali_hip_xcd_handoff": (C.c_int, [_i32]),
    "katali_hip_phase_stamps": (C.c_int, [_vp, _sz]),
    "katali_hip_stream_floor": (C.c_int, [_i32, _vp, _sz, _vp, _sz, _vp]),
    "katali_hip_exchange_probe": (C.c_int, [_i32, C.c_uint32, _vp]),
    "katali_hip_stager_create": (C.c_int, [_u64, _u32, C.POINTER(_vp)]),
    "katali_hip_stager_destroy": (C.c_int, [_vp]),
    "katali_hip_stager_mark": (C.c_int, [_vp, C.POINTER(_u64)]),
    "katali_hip_stager_upload": (C.c_int, [_vp, _vp, _vp, _u64, _u64]),
    "katali_hip_stager_fence": (C.c_int, [_vp]),
}


class KataliHipMoe(C.Structure):
    _fields_ = [("struct_size", _u32), ("gate_type", _u32), ("up_type", _u32), ("down_type", _u32),
                ("hidden", _u32), ("ffn", _u32), ("n_expert", _u32),
                ("gate_exps", _vp), ("up_exps", _vp), ("down_exps", _vp),
                ("gate_shexp", _vp), ("up_shexp", _vp), ("down_shexp", _vp)]


class KataliHipMoeRoute(C.Structure):
    _fields_ = [("struct_size", _u32), ("n_sel", _i32), ("logits", _vp), ("step", _vp),
                ("logits_stride", _u64), ("ids", _vp), ("weights", _vp),
                ("ids_out", _vp), ("weights_out", _vp)]


class KataliHipMoeNorm(C.Structure):
    _fields_ = [("struct_size", _u32), ("x", _vp), ("delta", _vp), ("scale", _f32), ("x_out", _vp),
                ("norm_w", _vp), ("eps", _f32), ("xn_out", _vp), ("router", _vp), ("logits_out", _vp)]


class KataliHipMoeStackLayer(C.Structure):
    _fields_ = [("struct_size", _u32), ("x", _vp), ("gate_exps", _vp), ("up_exps", _vp), ("down_exps", _vp),
                ("gate_shexp", _vp), ("up_shexp", _vp), ("down_shexp", _vp), ("route", KataliHipMoeRoute),
                ("norm_w", _vp), ("router", _vp), ("y", _vp), ("x_out", _vp), ("xn_out", _vp),
                ("logits_out", _vp)]


# error codes of include/katali_hip.h
E_INVALID, E_NODEVICE, E_RUNTIME, E_UNSUPPORTED, E_NOMEM, E_TIMEOUT = -1, -2, -3, -4, -5, -6


class HipError(RuntimeError):
    def __init__(self, rc: int, msg: str):
        super().__init__(f"katali_hip error {rc}: {msg}")
        self.rc = rc


def library_path() -> str:
    return os.environ.get("KATALI_HIP_DLL") or DEFAULT_SO


def load_library(path: str | None = None) -> C.CDLL:
    path = path or library_path()
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} not built: run `python katali-lab_amd/build.py` "
                                "(there is no CPU fallback in this binding)")
    lib = C.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


class KataliHipMoeBatch(C.Structure):
    _fields_ = [("struct_size", _u32), ("n_tokens", _u32), ("n_sel", _i32), ("mfma_min_tokens", _u32),
                ("ids", _vp), ("weights", _vp)]


class DeviceBuffer:
    """A device allocation from katali_hip_malloc."""

    def __init__(self, hip: "KataliHip", nbytes: int):
        self.hip, self.nbytes = hip, int(nbytes)
        p = _vp()
        hip.check(hip.lib.katali_hip_malloc(C.byref(p), self.nbytes))
        self.ptr = p.value

    def upload(self, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes, (arr.nbytes, self.nbytes)
        self.hip.check(self.hip.lib.katali_hip_upload(self.ptr, arr.ctypes.data, arr.nbytes))
        return self

    def download(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        count = (self.nbytes - offset) // dtype.itemsize if count is None else count
        out = np.empty(count, dtype)
        self.hip.check(self.hip.lib.katali_hip_download(out.ctypes.data, self.ptr + offset, out.nbytes))
        return out

    def free(self):
        if self.ptr:
            self.hip.lib.katali_hip_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class MoeStack:
    """A handle from katali_hip_moe_stack_create; holds the buffers its table
    points at until it is destroyed."""

    def __init__(self, hip: "KataliHip", handle: int, keep):
        self.hip, self.handle, self._keep = hip, handle, keep

    def run(self, x, delta=None, scale=1.0) -> None:
        self.hip.check(self.hip.lib.katali_hip_moe_stack_run(self.handle, x.ptr, None if delta is None else delta.ptr,
                                                             scale))

    def destroy(self) -> None:
        if self.handle:
            self.hip.check(self.hip.lib.katali_hip_moe_stack_destroy(self.handle))
            self.handle = None


class KataliHip:
    """Numpy front end over the C ABI."""

    def __init__(self, path: str | None = None):
        self.lib = load_library(path)

    # -- plumbing ---------------------------------------------------------
    def check(self, rc: int) -> None:
        if rc != 0:
            raise HipError(rc, self.lib.katali_hip_last_error().decode(errors="replace"))

    def probe(self) -> bool:
        return bool(self.lib.katali_hip_probe())

    def status(self) -> str:
        return self.lib.katali_hip_status().decode(errors="replace")

    def alloc(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    def to_device(self, arr: np.ndarray) -> DeviceBuffer:
        arr = np.ascontiguousarray(arr)
        return DeviceBuffer(self, max(arr.nbytes, 1)).upload(arr)

    def sync(self) -> None:
        self.check(self.lib.katali_hip_sync())

    def memset(self, buf: DeviceBuffer, value: int, nbytes: int) -> None:
        self.check(self.lib.katali_hip_memset(buf.ptr, value, nbytes))

    # -- compute ----------------------------------------------------------
    def quantize_q8_1(self, x: DeviceBuffer, n: int, out: DeviceBuffer) -> None:
        self.check(self.lib.katali_hip_quantize_q8_1(x.ptr, n, out.ptr))

    def matvec(self, t, w, rows, cols, x, y) -> None:
        self.check(self.lib.katali_hip_matvec(t, w.ptr, rows, cols, x.ptr, y.ptr))

    def matvec_q8(self, t, w, rows, cols, xq, y) -> None:
        self.check(self.lib.katali_hip_matvec_q8(t, w.ptr, rows, cols, xq.ptr, y.ptr))

    def matvec_dp4a(self, t, w, rows, cols, x, y) -> None:
        self.check(self.lib.katali_hip_matvec_dp4a(t, w.ptr, rows, cols, x.ptr, y.ptr))

    def matvec_multi(self, types, ws, rows, cols, x, ys, dp4a: bool = False) -> None:
        """ys[i] = W_i . x for up to four matrices in one launch."""
        n = len(types)
        args = ((_u32 * n)(*types), (_vp * n)(*[w.ptr for w in ws]), (_u64 * n)(*rows), cols, x.ptr,
                (_vp * n)(*[y.ptr for y in ys]))
        fn = self.lib.katali_hip_matvec_multi_dp4a if dp4a else self.lib.katali_hip_matvec_multi
        self.check(fn(n, *args))

    def rmsnorm(self, x, w, n, eps, out) -> None:
        self.check(self.lib.katali_hip_rmsnorm(x.ptr, w.ptr, n, eps, out.ptr))

    def add_rmsnorm(self, x, delta, scale, w, n, eps, out) -> None:
        self.check(self.lib.katali_hip_add_rmsnorm(x.ptr, delta.ptr, scale, w.ptr, n, eps, out.ptr))

    def rmsnorm_matvec_f32(self, x, delta, scale, x_out, norm_w, n, eps, xn, w, rows, y) -> None:
        """x_out = x + scale*delta (delta not None); xn = RMSNorm(.)*norm_w; y = W . xn."""
        p = lambda b: None if b is None else b.ptr  # noqa: E731
        self.check(self.lib.katali_hip_rmsnorm_matvec_f32(x.ptr, p(delta), scale, p(x_out), norm_w.ptr, n, eps,
                                                          xn.ptr, w.ptr, rows, y.ptr))

    def moe_route_batch(self, logits, n_tokens, n_expert, n_sel, ids, weights) -> None:
        self.check(self.lib.katali_hip_moe_route_batch(logits.ptr, n_tokens, n_expert, n_sel, ids.ptr, weights.ptr))

    def block_isums(self, t, w, rows, cols, xq, out) -> None:
        self.check(self.lib.katali_hip_block_isums(t, w.ptr, rows, cols, xq.ptr, out.ptr))

    @staticmethod
    def moe_desc(hidden, ffn, n_expert, gate, up, down, gate_type=Q4_K, down_type=Q6_K,
                 shared=None) -> KataliHipMoe:
        p = lambda b: None if b is None else b.ptr  # noqa: E731
        d = KataliHipMoe(C.sizeof(KataliHipMoe), gate_type, gate_type, down_type, hidden, ffn, n_expert,
                         p(gate), p(up), p(down), None, None, None)
        if shared is not None:
            d.gate_shexp, d.up_shexp, d.down_shexp = shared[0].ptr, shared[1].ptr, shared[2].ptr
        # the struct holds raw device pointers: keep their buffers alive with it
        # (a temporary DeviceBuffer would otherwise be freed before a layer runs)
        d._keep = (gate, up, down, shared)
        return d

    @staticmethod
    def moe_route(n_sel, logits=None, ids=None, weights=None, step=None, logits_stride=0,
                  ids_out=None, weights_out=None) -> KataliHipMoeRoute:
        p = lambda b: None if b is None else b.ptr  # noqa: E731
        r = KataliHipMoeRoute(C.sizeof(KataliHipMoeRoute), n_sel, p(logits), p(step), logits_stride,
                              p(ids), p(weights), p(ids_out), p(weights_out))
        r._keep = (logits, ids, weights, step, ids_out, weights_out)   # as in moe_desc
        return r

    def moe_layer(self, desc, route, y, x=None, xq=None) -> None:
        self.check(self.lib.katali_hip_moe_layer(C.byref(desc), C.byref(route),
                                                 None if x is None else x.ptr,
                                                 None if xq is None else xq.ptr, y.ptr))

    def moe_layer_normed(self, desc, n_sel, x, norm_w, router, y, delta=None, scale=1.0, x_out=None, eps=1e-6,
                         xn_out=None, logits_out=None, ids_out=None, weights_out=None) -> None:
        p = lambda b: None if b is None else b.ptr  # noqa: E731
        nrm = KataliHipMoeNorm(C.sizeof(KataliHipMoeNorm), p(x), p(delta), scale, p(x_out), p(norm_w), eps,
                               p(xn_out), p(router), p(logits_out))
        self.check(self.lib.katali_hip_moe_layer_normed(C.byref(desc), C.byref(nrm), n_sel, p(ids_out),
                                                        p(weights_out), y.ptr))

    def phase_stamps(self) -> np.ndarray:
        """The measurement build's phase stamps, [64 layer slots][256
        workgroups][16 phases] s_memrealtime ticks (100 MHz)."""
        out = np.zeros((64, 256, 16), np.uint64)
        self.check(self.lib.katali_hip_phase_stamps(out.ctypes.data, out.nbytes))
        return out

    def exchange_probe(self, kind: int, rounds: int, words) -> None:
        """The exchange probe (katali_hip_exchange_probe)."""
        self.check(self.lib.katali_hip_exchange_probe(kind, rounds, words.ptr))

    def stream_floor(self, kind: int, a, a_bytes: int, b, b_bytes: int, sync) -> None:
        """The streaming floors (katali_hip_stream_floor)."""
        self.check(self.lib.katali_hip_stream_floor(kind, a.ptr, a_bytes, None if b is None else b.ptr, b_bytes,
                                                     sync.ptr))

    def one_launch(self, mode: int = -1) -> bool:
        """The one-launch layers on (1) or off (0), or only asked (-1);
        returns whether they were on before the call."""
        return bool(self.lib.katali_hip_one_launch(mode))

    def xcd_handoff(self, mode: int = -1) -> bool:
        """The one-launch layers' h hand-off inside the XCD (1) or written
        through (0), or only asked (-1); returns the state before the call."""
        return bool(self.lib.katali_hip_xcd_handoff(mode))

    def moe_check(self, desc, n_sel, n_tokens=0) -> None:
        """Raises HipError when a layer (n_tokens 0) or a batch of n_tokens of
        this shape would be refused; needs no device."""
        self.check(self.lib.katali_hip_moe_check(C.byref(desc), n_sel, n_tokens))

    def moe_layer_noalloc(self, desc, route, y, x=None, xq=None) -> None:
        self.check(self.lib.katali_hip_moe_layer_noalloc(C.byref(desc), C.byref(route),
                                                         None if x is None else x.ptr,
                                                         None if xq is None else xq.ptr, y.ptr))

    def moe_layer_debug(self, desc, route, y, gu, hq8, x=None, xq=None) -> None:
        self.check(self.lib.katali_hip_moe_layer_debug(C.byref(desc), C.byref(route),
                                                       None if x is None else x.ptr,
                                                       None if xq is None else xq.ptr, y.ptr, gu.ptr, hq8.ptr))

    def moe_stack(self, desc, n_sel, layers, normed=False, eps=1e-6) -> "MoeStack":
        """A stack of layers of desc's shape (its weight pointers unused).
        layers: dicts with keys gate, up, down, y and optionally shared (3
        buffers), x (plain stack: a layer's own input; absent: the previous
        layer's y), route (a moe_route), norm_w, router, x_out, xn_out,
        logits_out."""
        p = lambda b: None if b is None else b.ptr  # noqa: E731
        arr = (KataliHipMoeStackLayer * len(layers))()
        keep = [desc]
        for i, L in enumerate(layers):
            sh = L.get("shared")
            e = arr[i]
            e.struct_size = C.sizeof(KataliHipMoeStackLayer)
            e.gate_exps, e.up_exps, e.down_exps = p(L["gate"]), p(L["up"]), p(L["down"])
            if sh is not None:
                e.gate_shexp, e.up_shexp, e.down_shexp = sh[0].ptr, sh[1].ptr, sh[2].ptr
            if L.get("route") is not None:
                e.route = L["route"]
            for k in ("x", "norm_w", "router", "y", "x_out", "xn_out", "logits_out"):
                setattr(e, k, p(L.get(k)))
            keep.append(L)
        h = _vp()
        self.check(self.lib.katali_hip_moe_stack_create(C.byref(desc), n_sel, 1 if normed else 0, eps, arr,
                                                        len(layers), C.byref(h)))
        return MoeStack(self, h.value, keep)

    def moe_batch(self, desc, n_tokens, n_sel, ids, weights, x, y, mfma_min_tokens=0) -> None:
        b = KataliHipMoeBatch(C.sizeof(KataliHipMoeBatch), n_tokens, n_sel, mfma_min_tokens,
                              None if ids is None else ids.ptr, None if weights is None else weights.ptr)
        self.check(self.lib.katali_hip_moe_batch(C.byref(desc), C.byref(b), x.ptr, y.ptr))

    def argmax(self, logits: DeviceBuffer, n: int, out: DeviceBuffer) -> None:
        self.check(self.lib.katali_hip_argmax(logits.ptr, n, out.ptr))

    def step_advance(self, step: DeviceBuffer, n_steps: int) -> None:
        self.check(self.lib.katali_hip_step_advance(step.ptr, n_steps))

    # -- graphs and timing ---------------------------------------------------
    def graph_begin(self) -> None:
        self.check(self.lib.katali_hip_graph_begin())

    def graph_end(self) -> int:
        g = _vp()
        self.check(self.lib.katali_hip_graph_end(C.byref(g)))
        return g.value

    def graph_launch(self, g: int) -> None:
        self.check(self.lib.katali_hip_graph_launch(g))

    def graph_destroy(self, g: int) -> None:
        self.check(self.lib.katali_hip_graph_destroy(g))

    def event(self) -> int:
        e = _vp()
        self.check(self.lib.katali_hip_event_create(C.byref(e)))
        return e.value

    def record(self, e: int) -> None:
        self.check(self.lib.katali_hip_event_record(e))

    def elapsed_ms(self, a: int, b: int) -> float:
        ms = _f32()
        self.check(self.lib.katali_hip_event_elapsed(a, b, C.byref(ms)))
        return float(ms.value)

    def event_destroy(self, e: int) -> None:
        self.check(self.lib.katali_hip_event_destroy(e))

    # -- harness helpers ---------------------------------------------------------
    def selftest(self) -> tuple[int, str]:
        buf = C.create_string_buffer(4096)
        rc = self.lib.katali_hip_selftest(buf, 4096)
        return rc, buf.value.decode()

    def synth_fill(self, t, buf: DeviceBuffer, nblocks: int, seed: int, d_sigma: float = 0.02) -> None:
        self.check(self.lib.katali_hip_synth_fill(t, buf.ptr, nblocks, seed, d_sigma))

    def synth_normal(self, buf: DeviceBuffer, n: int, seed: int, sigma: float = 1.0) -> None:
        self.check(self.lib.katali_hip_synth_normal(buf.ptr, n, seed, sigma))

    def copy(self, dst: DeviceBuffer, src: DeviceBuffer, nbytes: int) -> None:
        self.check(self.lib.katali_hip_copy(dst.ptr, src.ptr, nbytes))
