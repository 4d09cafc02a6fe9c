"""ctypes front end of the GGUF module of libkatali_hip_loader.so
(include/katali_hip_gguf.h): the reader, the device weight cache, MoE layer
assembly and the expert VRAM tier."""
import ctypes as C
import os

from katali_hip import KataliHipMoe

_vp, _u32, _u64, _i32, _i64 = C.c_void_p, C.c_uint32, C.c_uint64, C.c_int32, C.c_int64
LOADER = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libkatali_hip_loader.so")


class GgufTensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("n_dims", _u32), ("dims", _u64 * 4), ("type", _u32), ("offset", _u64),
                ("nbytes", _u64), ("data", _vp)]


class TierStats(C.Structure):
    _fields_ = [("hits", _u64), ("misses", _u64), ("uploaded_bytes", _u64), ("n_slots", _u32)]


_SIG = {
    "katali_hip_gguf_open": (C.c_int, [C.c_char_p, C.POINTER(_vp), C.c_char_p, C.c_size_t]),
    "katali_hip_gguf_close": (None, [_vp]),
    "katali_hip_gguf_last_error": (C.c_char_p, []),
    "katali_hip_gguf_version": (_u32, [_vp]),
    "katali_hip_gguf_tensor_count": (_u64, [_vp]),
    "katali_hip_gguf_alignment": (_u64, [_vp]),
    "katali_hip_gguf_data_offset": (_u64, [_vp]),
    "katali_hip_gguf_base": (_vp, [_vp]),
    "katali_hip_gguf_tensor": (C.c_int, [_vp, _u64, C.POINTER(GgufTensor)]),
    "katali_hip_gguf_find": (C.c_int, [_vp, C.c_char_p, C.POINTER(GgufTensor)]),
    "katali_hip_gguf_get_int": (_i64, [_vp, C.c_char_p, _i64]),
    "katali_hip_gguf_get_float": (C.c_double, [_vp, C.c_char_p, C.c_double]),
    "katali_hip_gguf_get_str": (_vp, [_vp, C.c_char_p, C.POINTER(C.c_size_t)]),
    "katali_hip_ggml_row_bytes": (_u64, [_u32, _u64]),
    "katali_hip_weights_create": (C.c_int, [_vp, _u64, C.POINTER(_vp)]),
    "katali_hip_weights_destroy": (None, [_vp]),
    "katali_hip_weights_get": (_vp, [_vp, C.c_char_p]),
    "katali_hip_weights_resident_bytes": (_u64, [_vp]),
    "katali_hip_gguf_moe_layer": (C.c_int, [_vp, _u32, C.POINTER(KataliHipMoe), C.POINTER(_vp), C.POINTER(_vp)]),
    "katali_hip_tier_create": (C.c_int, [_vp, _u32, _u64, _u32, C.POINTER(_vp)]),
    "katali_hip_tier_destroy": (None, [_vp]),
    "katali_hip_tier_layer": (C.c_int, [_vp, _u32, C.POINTER(_i32), C.c_int, C.POINTER(_i32),
                                        C.POINTER(KataliHipMoe)]),
    "katali_hip_tier_stats": (None, [_vp, C.POINTER(TierStats)]),
    "katali_hip_tier_pipeline": (C.c_int, [_vp, _u64, _u32]),
}


def load(path: str = LOADER) -> C.CDLL:
    lib = C.CDLL(path)
    for name, (res, args) in _SIG.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    return lib


class GgufError(RuntimeError):
    pass


class Gguf:
    """An open GGUF file (read-only map)."""

    def __init__(self, path: str, lib: C.CDLL | None = None):
        self.lib = lib or load()
        self.h = _vp()
        err = C.create_string_buffer(256)
        if self.lib.katali_hip_gguf_open(path.encode(), C.byref(self.h), err, 256) != 0:
            raise GgufError(err.value.decode(errors="replace"))

    def close(self):
        if self.h:
            self.lib.katali_hip_gguf_close(self.h)
            self.h = _vp()

    def __del__(self):
        self.close()

    @property
    def version(self):
        return self.lib.katali_hip_gguf_version(self.h)

    @property
    def alignment(self):
        return self.lib.katali_hip_gguf_alignment(self.h)

    @property
    def data_offset(self):
        return self.lib.katali_hip_gguf_data_offset(self.h)

    def tensors(self):
        base = self.lib.katali_hip_gguf_base(self.h)
        out = []
        for i in range(self.lib.katali_hip_gguf_tensor_count(self.h)):
            t = GgufTensor()
            assert self.lib.katali_hip_gguf_tensor(self.h, i, C.byref(t)) == 0
            out.append({"name": t.name.decode(), "n_dims": t.n_dims, "dims": list(t.dims), "type": t.type,
                        "offset": t.offset, "nbytes": t.nbytes, "data_pos": (t.data - base) if t.data else -1})
        return out

    def get_int(self, key, default=-1):
        return self.lib.katali_hip_gguf_get_int(self.h, key.encode(), default)

    def get_float(self, key, default=float("nan")):
        return self.lib.katali_hip_gguf_get_float(self.h, key.encode(), default)

    def get_str(self, key):
        n = C.c_size_t()
        p = self.lib.katali_hip_gguf_get_str(self.h, key.encode(), C.byref(n))
        return None if not p else C.string_at(p, n.value).decode(errors="replace")


class Weights:
    """Device weight cache keyed by tensor name."""

    def __init__(self, g: Gguf, budget: int = 0):
        self.g, self.lib, self.h = g, g.lib, _vp()
        if self.lib.katali_hip_weights_create(g.h, budget, C.byref(self.h)) != 0:
            raise GgufError(self.lib.katali_hip_gguf_last_error().decode())

    def destroy(self):
        if self.h:
            self.lib.katali_hip_weights_destroy(self.h)
            self.h = _vp()

    def get(self, name):
        p = self.lib.katali_hip_weights_get(self.h, name.encode())
        if not p:
            raise GgufError(self.lib.katali_hip_gguf_last_error().decode())
        return p

    @property
    def resident(self):
        return self.lib.katali_hip_weights_resident_bytes(self.h)

    def moe_layer(self, layer):
        """(KataliHipMoe, router device pointer, ffn_norm device pointer)."""
        m, r, n = KataliHipMoe(), _vp(), _vp()
        if self.lib.katali_hip_gguf_moe_layer(self.h, layer, C.byref(m), C.byref(r), C.byref(n)) != 0:
            raise GgufError(self.lib.katali_hip_gguf_last_error().decode())
        return m, r.value, n.value


class ExpertTier:
    def __init__(self, g: Gguf, layer_for_shape=0, budget=0, max_slots=64):
        self.g, self.lib, self.h = g, g.lib, _vp()
        if self.lib.katali_hip_tier_create(g.h, layer_for_shape, budget, max_slots, C.byref(self.h)) != 0:
            raise GgufError(self.lib.katali_hip_gguf_last_error().decode())

    def destroy(self):
        if self.h:
            self.lib.katali_hip_tier_destroy(self.h)
            self.h = _vp()

    def layer(self, layer, ids):
        n = len(ids)
        a, s, m = (_i32 * max(n, 1))(*ids), (_i32 * max(n, 1))(), KataliHipMoe()
        if self.lib.katali_hip_tier_layer(self.h, layer, a, n, s, C.byref(m)) != 0:
            raise GgufError(self.lib.katali_hip_gguf_last_error().decode())
        return m, list(s)[:n]

    def pipeline(self, chunk_bytes=0, n_chunks=0):
        """Pipelined uploads from here on (a pinned ring and a copy stream)."""
        if self.lib.katali_hip_tier_pipeline(self.h, chunk_bytes, n_chunks) != 0:
            raise GgufError(self.lib.katali_hip_gguf_last_error().decode())

    def stats(self):
        st = TierStats()
        self.lib.katali_hip_tier_stats(self.h, C.byref(st))
        return {"hits": st.hits, "misses": st.misses, "uploaded_bytes": st.uploaded_bytes, "n_slots": st.n_slots}
