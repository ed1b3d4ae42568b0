"""ctypes binding of libjasmine_hip.so (include/jasmine_hip.h)."""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libjasmine_hip.so")

if not os.path.exists(LIB_PATH):
    raise ImportError(f"{LIB_PATH} is missing: build it with `python jasmine_amd/build.py` "
                      "(there is no CPU fallback)")

lib = C.CDLL(LIB_PATH)

VP = C.c_void_p
FP = C.POINTER(C.c_float)
IP = C.POINTER(C.c_int32)
L = C.c_long
I = C.c_int

JAS_F32, JAS_F64, JAS_I32, JAS_BF16 = 0, 1, 2, 3
ERR_NAMES = {1: "invalid argument", 2: "runtime error", 3: "HIP error", 4: "out of memory", 5: "out of range"}


class JasError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"{ERR_NAMES.get(code, code)}: {msg}")
        self.code = code


class Leaf(C.Structure):
    _fields_ = [("d_data", VP), ("dtype", C.c_int32), ("rows", C.c_int32), ("cols", C.c_int32),
                ("row_first", C.c_int32), ("roff", C.c_int32), ("coff", C.c_int32),
                ("transposed", C.c_int32), ("vrows", C.c_int32), ("vcols", C.c_int32)]


class Ins(C.Structure):
    _fields_ = [("op", C.c_int32), ("dtype", C.c_int32), ("arg", C.c_int32), ("pad", C.c_int32),
                ("imm", C.c_double)]


class LmConfig(C.Structure):
    _fields_ = [("kind", C.c_int32), ("n_layer", C.c_int32), ("d_model", C.c_int32), ("n_head", C.c_int32),
                ("d_ff", C.c_int32), ("vocab", C.c_int32), ("max_ctx", C.c_int32), ("max_batch", C.c_int32),
                ("eps", C.c_float), ("rope_theta", C.c_float), ("weight_bf16", C.c_int32), ("kv_bf16", C.c_int32)]


_sigs = {
    "jas_init": [I], "jas_malloc": [C.POINTER(VP), C.c_size_t], "jas_free": [VP],
    "jas_memset": [VP, I, C.c_size_t, VP], "jas_memcpy_h2d": [VP, VP, C.c_size_t, VP],
    "jas_memcpy_d2h": [VP, VP, C.c_size_t, VP], "jas_memcpy_d2d": [VP, VP, C.c_size_t, VP],
    "jas_synchronize": [VP],
    "jas_pool_alloc": [C.POINTER(VP), C.c_size_t], "jas_pool_free": [VP], "jas_pool_trim": [C.POINTER(C.c_size_t)],
    "jas_ew_eval": [C.POINTER(Ins), I, C.POINTER(Leaf), I, VP, C.c_int32, I, I, VP],
    "jas_reduce": [C.POINTER(Leaf), I, I, VP, C.c_int32, VP],
    "jas_softmax": [VP, VP, I, I, L, L, L, VP],
    "jas_softmax_global": [VP, VP, L, VP],
    "jas_causal_mask": [VP, I, I, L, C.c_float, VP],
    "jas_causal_mask_f64": [VP, I, I, L, C.c_double, VP],
    "jas_leaf_assign": [VP, C.c_int32, I, I, C.POINTER(Leaf), VP],
    "jas_layernorm": [VP, VP, I, I, L, L, L, C.c_float, VP, VP, VP],
    "jas_rmsnorm": [VP, VP, I, I, L, L, L, C.c_float, VP, VP],
    "jas_gemm": [I, I, I, VP, L, L, VP, L, L, VP, L, L, VP, I, I, I, I, L, L, L, L, VP],
    "jas_gemm_residual": [I, I, I, VP, L, L, VP, L, L, VP, L, L, VP, I, I, VP, L, L, VP],
    "jas_gemm_f64": [I, I, I, VP, L, L, VP, L, L, VP, L, L, VP, I, VP],
    "jas_attn_prefill": [VP, VP, VP, VP, I, I, I, I, I, L, L, L, L, L, L, L, L, L, C.c_float, I, I, VP],
    "jas_attn_decode": [VP, VP, VP, VP, VP, I, I, I, I, L, L, C.c_float, VP, VP],
    "jas_attn_decode_noalloc": [VP, VP, VP, VP, VP, I, I, I, I, L, L, C.c_float, VP],
    "jas_rope_jasmine": [VP, VP, I, I, VP],
    "jas_rope_jasmine_f64": [VP, VP, I, I, VP],
    "jas_rope_llama": [VP, VP, I, I, I, L, C.c_float, VP],
    "jas_embed": [VP, VP, VP, VP, VP, I, I, VP],
    "jas_argmax": [VP, I, I, L, VP, VP],
    "jas_fill_normal": [VP, C.c_size_t, C.c_uint64, C.c_uint64, C.c_float, C.c_float, VP],
    "jas_lm_create": [C.POINTER(LmConfig), C.POINTER(VP)],
    "jas_lm_destroy": [VP],
    "jas_lm_init_random": [VP, C.c_uint64, C.c_float],
    "jas_lm_weight_shape": [VP, C.c_char_p, C.POINTER(I), C.POINTER(I), C.POINTER(I)],
    "jas_lm_get_weight": [VP, C.c_char_p, FP, C.c_size_t],
    "jas_lm_set_weight": [VP, C.c_char_p, FP, C.c_size_t],
    "jas_lm_prefill": [VP, I, I, IP, IP, FP],
    "jas_lm_decode": [VP, IP, IP, FP],
    "jas_lm_generate": [VP, I, IP],
    "jas_lm_profile": [VP, I, C.POINTER(C.c_double), C.POINTER(C.c_long)],
    "jas_lm_use_graph": [VP, I],
    "jas_lm_save": [VP, C.c_char_p], "jas_lm_load": [VP, C.c_char_p],
    "jas_lm_read_config": [C.c_char_p, C.POINTER(LmConfig)],
    "jas_lm_project": [VP, C.c_char_p, I, I, VP, VP, VP],
    "jas_lm_proj_geometry": [VP, C.c_char_p, IP],
    "jas_stream_release_scratch": [VP],
    "jas_hbm_read_probe": [VP, C.c_size_t, I, I, I, VP, VP],
}
for _n, _a in _sigs.items():
    getattr(lib, _n).argtypes = _a
    getattr(lib, _n).restype = C.c_int
lib.jas_last_error.restype = C.c_char_p
lib.jas_version.restype = C.c_char_p
lib.jas_default_stream.restype = VP
lib.jas_ew_jit_mode.restype = C.c_int
lib.jas_ew_jit_mode.argtypes = [C.c_int]
lib.jas_attn_decode_workspace.restype = C.c_size_t
lib.jas_attn_decode_workspace.argtypes = [I, I, I, I]
lib.jas_attn_decode_scratch_max.restype = C.c_size_t
lib.jas_attn_decode_scratch_max.argtypes = []
lib.jas_lm_position.restype = I
lib.jas_lm_position.argtypes = [VP]
lib.jas_lm_attn_splits.restype = I
lib.jas_lm_attn_splits.argtypes = [VP, I]
lib.jas_lm_stream.restype = VP
lib.jas_lm_stream.argtypes = [VP]

# every symbol the C header declares (checked by the CPU test that the library exports them)
EXPORTED = sorted(list(_sigs) + ["jas_last_error", "jas_version", "jas_default_stream",
                                 "jas_attn_decode_workspace", "jas_attn_decode_scratch_max", "jas_ew_jit_mode", "jas_lm_position", "jas_lm_stream",
                                 "jas_lm_attn_splits"])


def check(code):
    if code != 0:
        raise JasError(code, lib.jas_last_error().decode(errors="replace"))


# uint16 device arrays hold bf16 bit patterns
_DT = {np.dtype(np.float32): JAS_F32, np.dtype(np.float64): JAS_F64, np.dtype(np.int32): JAS_I32,
       np.dtype(np.uint16): JAS_BF16}


class DeviceArray:
    """Owning device buffer with a numpy-like shape/dtype (row-major)."""

    def __init__(self, shape, dtype=np.float32):
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        p = VP()
        check(lib.jas_malloc(C.byref(p), max(self.nbytes, 1)))
        self.ptr = p.value

    def __del__(self):
        if getattr(self, "ptr", None):
            lib.jas_free(VP(self.ptr))
            self.ptr = None

    @property
    def p(self):
        return VP(self.ptr)

    def upload(self, a):
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes, (a.shape, self.shape)
        check(lib.jas_memcpy_h2d(self.p, a.ctypes.data_as(VP), self.nbytes, None))
        return self

    def numpy(self):
        out = np.empty(self.shape, self.dtype)
        check(lib.jas_synchronize(None))
        check(lib.jas_memcpy_d2h(out.ctypes.data_as(VP), self.p, self.nbytes, None))
        return out

    def zero(self):
        check(lib.jas_memset(self.p, 0, self.nbytes, None))
        return self


def to_device(a, dtype=None):
    a = np.asarray(a) if dtype is None else np.asarray(a, dtype=dtype)
    return DeviceArray(a.shape, a.dtype).upload(a)


def leaf(arr, rows=None, cols=None, row_first=1, roff=0, coff=0, transposed=0, vrows=None, vcols=None):
    """jas_leaf for a DeviceArray holding a [rows, cols] matrix (row_first storage)."""
    r = rows if rows is not None else arr.shape[0]
    c = cols if cols is not None else (arr.shape[1] if len(arr.shape) > 1 else 1)
    vr = vrows if vrows is not None else (c - coff if transposed else r - roff)
    vc = vcols if vcols is not None else (r - roff if transposed else c - coff)
    return Leaf(arr.ptr, _DT[arr.dtype], r, c, row_first, roff, coff, transposed, vr, vc)


class Lm:
    """Owning handle of a jas_lm decoder runner."""

    def __init__(self, cfg: LmConfig):
        self.cfg = cfg
        h = VP()
        check(lib.jas_lm_create(C.byref(cfg), C.byref(h)))
        self.h = h

    def close(self):
        if getattr(self, "h", None) is not None and self.h.value:
            lib.jas_lm_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def init_random(self, seed, std=0.02):
        check(lib.jas_lm_init_random(self.h, seed, std))

    def weight_shape(self, name):
        l, r, c = I(), I(), I()
        check(lib.jas_lm_weight_shape(self.h, name.encode(), C.byref(l), C.byref(r), C.byref(c)))
        return l.value, r.value, c.value

    def weight(self, name):
        """Host copy of a weight tensor, flat in logical [layers][rows][cols] order (None if absent)."""
        l, r, c = self.weight_shape(name)
        if l == 0:
            return None
        out = np.empty(l * r * c, np.float32)
        check(lib.jas_lm_get_weight(self.h, name.encode(), out.ctypes.data_as(FP), out.size))
        return out

    def set_weight(self, name, a):
        l, r, c = self.weight_shape(name)
        a = np.ascontiguousarray(a, np.float32).ravel()
        assert l and a.size == l * r * c, (name, a.size, (l, r, c))
        check(lib.jas_lm_set_weight(self.h, name.encode(), a.ctypes.data_as(FP), a.size))

    def save(self, path):
        """Write every weight to a safetensors file (jas_lm_save)."""
        check(lib.jas_lm_save(self.h, os.fsencode(path)))

    def load(self, path):
        """Read every weight from a safetensors file (jas_lm_load)."""
        check(lib.jas_lm_load(self.h, os.fsencode(path)))

    @property
    def stream(self):
        return VP(lib.jas_lm_stream(self.h))

    def prefill(self, ids, want_logits=False):
        ids = np.ascontiguousarray(ids, np.int32)
        B, P = ids.shape
        nxt = np.empty(B, np.int32)
        lg = np.empty((B, self.cfg.vocab), np.float32) if want_logits else None
        check(lib.jas_lm_prefill(self.h, B, P, ids.ctypes.data_as(IP), nxt.ctypes.data_as(IP),
                                 lg.ctypes.data_as(FP) if lg is not None else None))
        return nxt, lg

    def decode(self, ids=None, B=None, want_logits=False):
        B = B if B is not None else (len(ids) if ids is not None else None)
        nxt = np.empty(B, np.int32)
        lg = np.empty((B, self.cfg.vocab), np.float32) if want_logits else None
        a = np.ascontiguousarray(ids, np.int32) if ids is not None else None
        check(lib.jas_lm_decode(self.h, a.ctypes.data_as(IP) if a is not None else None,
                                nxt.ctypes.data_as(IP), lg.ctypes.data_as(FP) if lg is not None else None))
        return nxt, lg

    def generate(self, steps, B):
        out = np.empty((steps, B), np.int32)
        check(lib.jas_lm_generate(self.h, steps, out.ctypes.data_as(IP)))
        return out

    @property
    def position(self):
        return lib.jas_lm_position(self.h)

    def project(self, name, layer, x_dev, y_dev, B, stream=None):
        """y[B][M] = W . x with the decode GEMM on the stored weights (device arrays)."""
        check(lib.jas_lm_project(self.h, name.encode(), int(layer), int(B), x_dev.p, y_dev.p, stream))

    def proj_geometry(self, name):
        """(tiles per workgroup, waves, chunks in flight, K splits) of one decode projection."""
        geo = (C.c_int * 4)()
        check(lib.jas_lm_proj_geometry(self.h, name.encode(), geo))
        return tuple(geo)

    def attn_splits(self, B):
        """Key splits the decode attention takes at batch B (1: one pass, no merge)."""
        return lib.jas_lm_attn_splits(self.h, int(B))

    def use_graph(self, enable):
        check(lib.jas_lm_use_graph(self.h, int(enable)))

    def profile(self, enable):
        ms = (C.c_double * 3)()
        cnt = (C.c_long * 3)()
        check(lib.jas_lm_profile(self.h, int(enable), ms, cnt))
        return list(ms), list(cnt)


def read_lm_config(path):
    """The runner config stored in a weight file's metadata (host only)."""
    cfg = LmConfig()
    check(lib.jas_lm_read_config(os.fsencode(path), C.byref(cfg)))
    return cfg
