"""gadeon_amd -- MI355X (gfx950) implementation of Gadeon's Q2_0 + Gated DeltaNet hot path.

The product is the C-ABI shared library ``libgadeon_hip.so`` (declared in
include/gadeon_hip.h).  This package holds its HIP sources (csrc/), the build
script (build.py) and a thin ctypes binding used by tests and bench.py.  It
has no CPU fallback: loading fails loudly when the library is missing.
"""
from __future__ import annotations

import ctypes as C
import os
import weakref
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libgadeon_hip.so"

GD_OK, GD_EINVAL, GD_ENODEV, GD_ENOMEM, GD_ELAUNCH, GD_EHIP, GD_ESTOPPED = 0, -1, -2, -3, -4, -5, -6
F32, F16 = 0, 1

_vp, _i, _i64, _u64, _f, _sz = C.c_void_p, C.c_int, C.c_int64, C.c_uint64, C.c_float, C.c_size_t
_fp = C.POINTER(C.c_float)


class Q2W(C.Structure):
    """Device Q2_0 matrix: codes[R][K/4] + f16 scales[R][K/128] (gd_q2w)."""
    _fields_ = [("codes", _vp), ("scales", _vp), ("K", _i64), ("R", _i64)]


class StackConfig(C.Structure):
    _fields_ = [(n, _i) for n in ("n_layer", "n_embd", "n_ff", "n_head", "n_head_kv", "head_dim",
                                  "n_rot")] + [("rope_base", _f), ("eps", _f)] + \
               [(n, _i) for n in ("n_vocab", "attn_interval", "d_state", "n_k_head", "n_v_head",
                                  "d_conv", "kv_block", "max_ctx", "max_batch", "dense")]


_Q2WP = C.POINTER(Q2W)

# name -> (restype, argtypes)
_PROTOS = {
    "gd_device_count": (_i, [C.POINTER(_i)]),
    "gd_ctx_create": (_i, [_i, C.POINTER(_vp)]),
    "gd_ctx_destroy": (None, [_vp]),
    "gd_last_error": (C.c_char_p, [_vp]),
    "gd_alloc": (_i, [_vp, _sz, C.POINTER(_vp)]),
    "gd_free": (_i, [_vp, _vp]),
    "gd_upload": (_i, [_vp, _vp, _vp, _sz]),
    "gd_download": (_i, [_vp, _vp, _vp, _sz]),
    "gd_copy": (_i, [_vp, _vp, _vp, _sz]),
    "gd_fill_u32": (_i, [_vp, _vp, C.c_uint32, _sz]),
    "gd_cast": (_i, [_vp, _vp, _i, _vp, _i, _sz]),
    "gd_graph_begin": (_i, [_vp]),
    "gd_graph_end": (_i, [_vp, C.POINTER(_vp)]),
    "gd_graph_launch": (_i, [_vp, _vp]),
    "gd_graph_destroy": (None, [_vp]),
    "gd_sync": (_i, [_vp]),
    "gd_timer_start": (_i, [_vp]),
    "gd_timer_stop": (_i, [_vp, _fp]),
    "gd_q2_0_pack": (_i, [_vp, _vp, _sz, _vp]),
    "gd_q2_0_unpack": (_i, [_vp, _sz, _vp, _vp]),
    "gd_q2w_alloc": (_i, [_vp, _i64, _i64, _Q2WP]),
    "gd_q2w_free": (_i, [_vp, _Q2WP]),
    "gd_q2_0_repack": (_i, [_vp, _vp, _u64, _Q2WP]),
    "gd_q2_0_upload": (_i, [_vp, _vp, _i64, _i64, _Q2WP]),
    "gd_q2_0_export": (_i, [_vp, _Q2WP, _vp]),
    "gd_q2_0_export_rows": (_i, [_vp, _Q2WP, _i64, _i64, _vp]),
    "gd_q2_0_gemv": (_i, [_vp, _Q2WP, _vp, _i, _vp]),
    "gd_q2_0_gemv_split": (_i, [_vp, _Q2WP, _vp, _i, _vp, _i, _vp]),
    "gd_q2_0_gemv_gated": (_i, [_vp, _Q2WP, _vp, _vp, _vp, _f, _vp, _vp]),
    "gd_q2_0_gemv_norm": (_i, [_vp, _Q2WP, _vp, _vp, _i, _i64, _vp, _f, _vp, _vp, _vp]),
    "gd_q2_0_gemm_swiglu": (_i, [_vp, _Q2WP, _i64, _vp, _vp]),
    "gd_q2_0_gemm_swiglu_plan": (_i, [_vp, _Q2WP, _i64, _vp, _vp, _i]),
    "gd_q2_0_gemm": (_i, [_vp, _Q2WP, _i64, _vp, _i, _vp, _i]),
    "gd_q2_0_gemm_plan": (_i, [_vp, _Q2WP, _i64, _vp, _i, _vp, _i, _i, _i, _i, _i]),
    "gd_q2_0_gemm_plan17": (_i, [_vp, _Q2WP, _i64, _vp, _i, _vp, _i, _i]),
    "gd_q2_0_gemm_plan_tail": (_i, [_vp, _Q2WP, _i64, _vp, _vp, _i, _i, _i, _i, _vp, _vp, _vp]),
    "gd_q2_0_dequant_rows": (_i, [_vp, _Q2WP, _vp, _i64, _vp]),
    "gd_split_q_gate": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i64]),
    "gd_rope": (_i, [_vp, _vp, _i, _i, _i, _f, _i, _i64]),
    "gd_kv_append": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i64]),
    "gd_attn_paged": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _f,
                           _i, _i]),
    "gd_attn_batch": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _i, _i64,
                           _i, _i]),
    "gd_gdn_gate": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i64]),
    "gd_gdn_conv": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i64]),
    "gd_l2norm_rows": (_i, [_vp, _vp, _i, _i, _i64, _i64, _f]),
    "gd_rmsnorm_rows": (_i, [_vp, _vp, _i, _i64, _vp, _f]),
    "gd_rmsnorm": (_i, [_vp, _vp, _vp, _vp, _i, _i64, _i64, _f]),
    "gd_silu_mul": (_i, [_vp, _vp, _vp, _i64]),
    "gd_mul_silu": (_i, [_vp, _vp, _vp, _i64]),
    "gd_add": (_i, [_vp, _vp, _vp, _i64]),
    "gd_gdn_scan": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _f]),
    "gd_gdn_scan_batch": (_i, [_vp, _vp, _i, _i, _i, _vp, _vp, _vp, _vp, _i, _i, _i, _f, _i64]),
    "gd_gdn_decode": (_i, [_vp, _i, _i, _i, _i, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp,
                           _vp, _f, _f]),
    "gd_gdn_prefill": (_i, [_vp, _i64, _i, _i, _i, _i, _vp, _i64, _vp, _i64, _vp, _i64, _i,
                            _vp, _vp, _vp, _vp, _i64, _i, _f, _i]),
    "gd_gdn_prefill_noalloc": (_i, [_vp, _i64, _i, _i, _i, _i, _vp, _i64, _vp, _i64, _vp, _i64, _i,
                            _vp, _vp, _vp, _vp, _i64, _i, _f, _i]),
    "gd_rand_uniform": (_i, [_vp, _vp, _sz, _u64, _f, _f]),
    "gd_rand_normal": (_i, [_vp, _vp, _i, _sz, _u64, _f, _f]),
    "gd_rand_q2w": (_i, [_vp, _Q2WP, _u64, _f, _f]),
    "gd_stack_create": (_i, [_vp, C.POINTER(StackConfig), _u64, C.POINTER(_vp)]),
    "gd_stack_destroy": (None, [_vp]),
    "gd_stack_reset": (_i, [_vp]),
    "gd_stack_prefill": (_i, [_vp, _vp, _i, C.POINTER(C.c_int32), _vp]),
    "gd_stack_decode": (_i, [_vp, C.c_int32, C.POINTER(C.c_int32), _vp]),
    "gd_stack_request_stop": (_i, [_vp]),
    "gd_stack_set_eager": (_i, [_vp, _i]),
    "gd_stack_should_stop": (_i, [_vp, C.POINTER(_i)]),
    "gd_stack_tensor": (_i, [_vp, _i, C.c_char_p, _Q2WP, C.POINTER(_i64), C.POINTER(_fp),
                         C.POINTER(_i64)]),
    "gd_stack_position": (_i, [_vp, C.POINTER(_i64)]),
    "gd_stack_kv_pages": (_i, [_vp, C.POINTER(_i64), C.POINTER(_i64), C.POINTER(_i64)]),
    "gd_stack_generate": (_i, [_vp, _i, _vp]),
    "gd_q2_0_repack_rows": (_i, [_vp, _vp, _u64, _i64, _i64, _Q2WP]),
    "gd_stack_bookmark": (_i, [_vp, C.POINTER(_vp)]),
    "gd_stack_restore": (_i, [_vp, _vp]),
    "gd_bookmark_free": (None, [_vp]),
    "gd_stack_serialize": (_i, [_vp, _vp, _vp, _sz, C.POINTER(_sz)]),
    "gd_stack_deserialize": (_i, [_vp, _vp, _sz, C.POINTER(_vp)]),
    "gd_stack_serialize_gdns": (_i, [_vp, _vp, _vp, _sz, C.POINTER(_sz)]),
    "gd_stack_deserialize_gdns": (_i, [_vp, _vp, _sz, C.POINTER(_vp)]),
    "gd_gguf_open": (_i, [C.c_char_p, C.POINTER(_vp)]),
    "gd_gguf_close": (None, [_vp]),
    "gd_gguf_info": (_i, [_vp, C.POINTER(_i64), C.POINTER(_i64), C.POINTER(_i)]),
    "gd_gguf_tensor": (_i, [_vp, C.c_char_p, C.POINTER(_i), C.POINTER(_i64), C.POINTER(_i),
                        C.POINTER(_vp), C.POINTER(_sz)]),
    "gd_gguf_get_int": (_i, [_vp, C.c_char_p, C.POINTER(_i64)]),
    "gd_gguf_get_float": (_i, [_vp, C.c_char_p, C.POINTER(C.c_double)]),
    "gd_gguf_get_bool": (_i, [_vp, C.c_char_p, C.POINTER(_i)]),
    "gd_gguf_get_string": (_i, [_vp, C.c_char_p, C.POINTER(C.c_char_p)]),
    "gd_gguf_get_floats": (_i, [_vp, C.c_char_p, C.POINTER(C.POINTER(C.c_double)),
                            C.POINTER(_i64)]),
    "gd_gguf_get_ints": (_i, [_vp, C.c_char_p, C.POINTER(C.POINTER(_i64)), C.POINTER(_i64)]),
    "gd_gguf_stack_config": (_i, [_vp, C.POINTER(StackConfig)]),
    "gd_stack_create_from_gguf": (_i, [_vp, _vp, _i, _i, _i, C.POINTER(_vp)]),
}

_lib = None


def load(path: os.PathLike | str | None = None) -> C.CDLL:
    """Load libgadeon_hip.so and declare every prototype.  Raises if it is absent."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise RuntimeError(f"{p} is not built; run `python -m gadeon_amd.build` first")
    lib = C.CDLL(str(p))
    for name, (res, args) in _PROTOS.items():
        fn = getattr(lib, name)          # AttributeError = a declared symbol is missing
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def exported_names() -> list[str]:
    return list(_PROTOS)


class GDError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"gadeon_hip error {code}: {msg}")
        self.code = code


class Context:
    """A gd_ctx on one device, with helpers to move numpy arrays in and out."""

    def __init__(self, device: int = 0):
        self.lib = load()
        h = _vp()
        rc = self.lib.gd_ctx_create(device, C.byref(h))
        if rc != GD_OK:
            raise GDError(rc, self.lib.gd_last_error(None).decode())
        self.h = h
        self._bufs: list[int] = []

    # -- error plumbing
    def check(self, rc: int) -> None:
        if rc != GD_OK:
            raise GDError(rc, self.lib.gd_last_error(self.h).decode())

    def __getattr__(self, name):
        """ctx.gd_xxx(args...) calls gd_xxx(ctx, args...) and raises on error."""
        if name.startswith("gd_"):
            fn = getattr(self.lib, name)

            def call(*args):
                rc = fn(self.h, *args)
                if fn.restype is _i:
                    self.check(rc)
                return rc
            return call
        raise AttributeError(name)

    # -- memory
    def alloc(self, nbytes: int) -> int:
        p = _vp()
        self.check(self.lib.gd_alloc(self.h, nbytes, C.byref(p)))
        self._bufs.append(p.value)
        return p.value

    def free(self, ptr: int) -> None:
        if ptr in self._bufs:
            self._bufs.remove(ptr)
        self.check(self.lib.gd_free(self.h, ptr))

    def put(self, a: np.ndarray) -> int:
        a = np.ascontiguousarray(a)
        p = self.alloc(max(a.nbytes, 1))
        if a.nbytes:
            self.check(self.lib.gd_upload(self.h, p, a.ctypes.data, a.nbytes))
        return p

    def get(self, ptr: int, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        if out.nbytes:
            self.check(self.lib.gd_download(self.h, out.ctypes.data, ptr, out.nbytes))
        return out

    def set(self, ptr: int, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        self.check(self.lib.gd_upload(self.h, ptr, a.ctypes.data, a.nbytes))

    def sync(self) -> None:
        self.check(self.lib.gd_sync(self.h))

    def close(self) -> None:
        if getattr(self, "h", None):
            for p in list(self._bufs):
                self.lib.gd_free(self.h, p)
            self._bufs.clear()
            self.lib.gd_ctx_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class GGUF:
    """A GGUF file opened by the library's host reader (gd_gguf_*, no device
    needed).  Tensors come back as read-only numpy views of the mapping; the
    mapping stays in place until close() has been called AND every view (and
    every array derived from one) is gone, so a view never outlives it."""

    def __init__(self, path: os.PathLike | str):
        self.lib = load()
        h = _vp()
        rc = self.lib.gd_gguf_open(os.fsencode(path), C.byref(h))
        if rc != GD_OK:
            raise GDError(rc, self.lib.gd_last_error(None).decode())
        self.h = h
        self._views = 0            # live tensor views of the mapping
        self._closing = False      # close() called; unmap when the last view goes

    def _handle(self):
        if self._closing or not self.mapped:
            raise GDError(GD_EINVAL, "GGUF file is closed")
        return self.h

    def _check(self, rc: int) -> None:
        if rc != GD_OK:
            raise GDError(rc, self.lib.gd_last_error(None).decode())

    def info(self) -> tuple[int, int, int]:
        nt, nkv, ver = _i64(), _i64(), _i()
        self._check(self.lib.gd_gguf_info(self._handle(), C.byref(nt), C.byref(nkv), C.byref(ver)))
        return nt.value, nkv.value, ver.value

    def tensor(self, name: str) -> tuple[tuple[int, ...], int, np.ndarray]:
        """(dims with ne0 first, ggml type, raw bytes as a uint8 array)."""
        nd, ty, data, nb = _i(), _i(), _vp(), _sz()
        dims = (_i64 * 4)()
        self._check(self.lib.gd_gguf_tensor(self._handle(), name.encode(), C.byref(nd), dims,
                                            C.byref(ty), C.byref(data), C.byref(nb)))
        buf = (C.c_uint8 * nb.value).from_address(data.value)
        # The array (and anything sliced from it) holds buf; buf's finalizer
        # holds this object, so the mapping outlives every view.
        self._views += 1
        weakref.finalize(buf, self._release_view)
        arr = np.frombuffer(buf, np.uint8)
        arr.flags.writeable = False
        return tuple(dims[:nd.value]), ty.value, arr

    def _release_view(self) -> None:
        self._views -= 1
        if self._closing and self._views == 0:
            self._unmap()

    def _unmap(self) -> None:
        if getattr(self, "h", None):
            self.lib.gd_gguf_close(self.h)
            self.h = None

    @property
    def mapped(self) -> bool:
        """True while the file mapping is in place."""
        return bool(getattr(self, "h", None))

    def int(self, key: str) -> int:
        v = _i64()
        self._check(self.lib.gd_gguf_get_int(self._handle(), key.encode(), C.byref(v)))
        return v.value

    def float(self, key: str) -> float:
        v = C.c_double()
        self._check(self.lib.gd_gguf_get_float(self._handle(), key.encode(), C.byref(v)))
        return v.value

    def bool(self, key: str) -> bool:
        v = _i()
        self._check(self.lib.gd_gguf_get_bool(self._handle(), key.encode(), C.byref(v)))
        return bool(v.value)

    def floats(self, key: str) -> list[float]:
        v, n = C.POINTER(C.c_double)(), _i64()
        self._check(self.lib.gd_gguf_get_floats(self._handle(), key.encode(), C.byref(v), C.byref(n)))
        return [v[i] for i in range(n.value)]

    def string(self, key: str) -> str:
        v = C.c_char_p()
        self._check(self.lib.gd_gguf_get_string(self._handle(), key.encode(), C.byref(v)))
        return v.value.decode()

    def ints(self, key: str) -> list[int]:
        v, n = C.POINTER(_i64)(), _i64()
        self._check(self.lib.gd_gguf_get_ints(self._handle(), key.encode(), C.byref(v), C.byref(n)))
        return [v[i] for i in range(n.value)]

    def stack_config(self) -> StackConfig:
        c = StackConfig()
        self._check(self.lib.gd_gguf_stack_config(self._handle(), C.byref(c)))
        return c

    def close(self) -> None:
        """No further reads; the mapping goes when the last view does."""
        self._closing = True
        if self._views == 0:
            self._unmap()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def device_count() -> int:
    """Visible HIP devices, via the library (0 when none or when not built)."""
    try:
        lib = load()
    except RuntimeError:
        return 0
    n = _i(0)
    lib.gd_device_count(C.byref(n))
    return n.value
