"""ctypes binding of the CPU oracle (oracle/_build/libgd_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/ as the parity checker and by
bench.py's cpu_baseline leg.  The product library never loads it.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libgd_oracle.so"

_vp, _i, _i64, _u64, _f, _d, _sz = (C.c_void_p, C.c_int, C.c_int64, C.c_uint64, C.c_float,
                                    C.c_double, C.c_size_t)

_PROTOS = {
    "or_lcg_uniform": (None, [_vp, _sz, _u64, _f, _f]),
    "or_lcg_normal": (None, [_vp, _sz, _u64, _f, _f]),
    "or_lcg_normal_f16": (None, [_vp, _sz, _u64, _f, _f]),
    "or_lcg_q2_0": (None, [_vp, _i64, _i64, _u64, _f, _f]),
    "or_h2f": (_f, [C.c_uint16]),
    "or_f2h": (C.c_uint16, [_f]),
    "or_q2_0_dequant": (None, [_vp, _sz, _vp]),
    "or_q2_0_matvec": (None, [_vp, _i64, _i64, _vp, _vp, _i]),
    "or_q2_0_matvec_f64": (None, [_vp, _i64, _i64, _vp, _vp]),
    "or_silu": (_f, [_f]),
    "or_sigmoid": (_f, [_f]),
    "or_softplus": (_f, [_f]),
    "or_rmsnorm": (None, [_vp, _vp, _vp, _i64, _f]),
    "or_rmsnorm_rows": (None, [_vp, _i, _i64, _vp, _f]),
    "or_l2norm_rows": (None, [_vp, _i, _i64, _f]),
    "or_softmax": (None, [_vp, _i]),
    "or_rope_neox": (None, [_vp, _i, _i, _i, _f, _i]),
    "or_gdn_gate": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i64]),
    "or_gdn_conv": (None, [_vp, _vp, _vp, _vp, _i, _i]),
    "or_gdn_scan": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _f]),
    "or_gdn_scan_f64": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _d]),
    "or_gdn_chunked_f64": (None, [_i64, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _d,
                                  _i]),
    "or_mtp_state_after": (None, [_i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp]),
    "or_gdn_decode_batch": (None, [_i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _f, _f,
                                   _i]),
}

_lib = None


def build() -> Path:
    """Compile the oracle with its Makefile (gcc -O2, no -ffast-math)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _PROTOS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def P(a: np.ndarray) -> int:
    """Data pointer of a C-contiguous array."""
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ---- convenience wrappers used by the tests ---------------------------------

def lcg_uniform(n: int, seed: int, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().or_lcg_uniform(P(out), n, seed, lo, hi)
    return out


def lcg_normal(n: int, seed: int, mean: float = 0.0, sd: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().or_lcg_normal(P(out), n, seed, mean, sd)
    return out


def lcg_normal_f16(n: int, seed: int, mean: float = 0.0, sd: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.uint16)
    lib().or_lcg_normal_f16(P(out), n, seed, mean, sd)
    return out.view(np.float16)


def lcg_q2_0(K: int, R: int, seed: int, lo: float = 0.01, hi: float = 0.05) -> np.ndarray:
    out = np.empty(R * (K // 128) * 34, np.uint8)
    lib().or_lcg_q2_0(P(out), K, R, seed, lo, hi)
    return out


def q2_0_dequant(blocks: np.ndarray, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().or_q2_0_dequant(P(blocks), n, P(out))
    return out


def q2_0_matvec(blocks: np.ndarray, K: int, M: int, x: np.ndarray, threads: int = 1) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(M, np.float32)
    lib().or_q2_0_matvec(P(blocks), K, M, P(x), P(out), threads)
    return out


def q2_0_matvec_f64(blocks: np.ndarray, K: int, M: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float64)
    out = np.empty(M, np.float64)
    lib().or_q2_0_matvec_f64(P(blocks), K, M, P(x), P(out))
    return out


def gdn_scan(q, k, v, g, beta, S, nV, nK, dS, qScale):
    """One token of GDN.step's scan in f32; S updated in place; returns o."""
    o = np.empty(nV * dS, np.float32)
    lib().or_gdn_scan(P(q), P(k), P(v), P(g), P(beta), P(S), P(o), nV, nK, dS, qScale)
    return o


def gdn_scan_f64(q, k, v, g, beta, S, nV, nK, dS, qScale):
    o = np.empty(nV * dS, np.float64)
    lib().or_gdn_scan_f64(P(q), P(k), P(v), P(g), P(beta), P(S), P(o), nV, nK, dS, qScale)
    return o


def gdn_chunked_f64(q, k, v, g, beta, S, T, nV, nK, dk, dv, qScale, C_):
    o = np.empty((T, nV, dv), np.float64)
    lib().or_gdn_chunked_f64(T, nV, nK, dk, dv, P(q), P(k), P(v), P(g), P(beta), P(S), P(o),
                             qScale, C_)
    return o


def gdn_sequential(q, k, v, g, beta, S, qScale, f64=False):
    """Token-serial GDN.step scans over T tokens: q,k [T][nK][dS], v [T][nV][dS],
    g,beta [T][nV], S [nV][dS][dS] (updated in place).  Returns o [T][nV][dS]."""
    T, nK, dS = q.shape
    nV = v.shape[1]
    dt = np.float64 if f64 else np.float32
    fn = gdn_scan_f64 if f64 else gdn_scan
    o = np.empty((T, nV, dS), dt)
    for t in range(T):
        o[t] = fn(np.ascontiguousarray(q[t], dt), np.ascontiguousarray(k[t], dt),
                  np.ascontiguousarray(v[t], dt), np.ascontiguousarray(g[t], dt),
                  np.ascontiguousarray(beta[t], dt), S, nV, nK, dS, qScale).reshape(nV, dS)
    return o


def l2norm_rows(x: np.ndarray, d: int, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).copy()
    lib().or_l2norm_rows(P(x), d, x.size // d, eps)
    return x


def rmsnorm_rows(x: np.ndarray, d: int, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).copy()
    lib().or_rmsnorm_rows(P(x), d, x.size // d, P(np.ascontiguousarray(w, np.float32)), eps)
    return x


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    n = x.shape[-1]
    w = np.ascontiguousarray(w, np.float32)
    for r in range(x.size // n):
        lib().or_rmsnorm(P(x) + 4 * r * n, P(w), P(y) + 4 * r * n, n, eps)
    return y


def gdn_gate(bPre, aPre, dt, aNeg, nV):
    bPre = np.ascontiguousarray(bPre, np.float32)
    aPre = np.ascontiguousarray(aPre, np.float32)
    beta = np.empty_like(bPre)
    g = np.empty_like(bPre)
    lib().or_gdn_gate(P(bPre), P(aPre), P(np.ascontiguousarray(dt, np.float32)),
                      P(np.ascontiguousarray(aNeg, np.float32)), P(beta), P(g), nV, bPre.size)
    return beta, g


def gdn_conv(x: np.ndarray, ring: np.ndarray, cw: np.ndarray, convDim: int, dConv: int):
    """Token-serial conv over x [N][convDim]; ring updated in place; returns out."""
    out = np.empty_like(x)
    for n in range(x.shape[0]):
        xn = np.ascontiguousarray(x[n])
        on = np.empty(convDim, np.float32)
        lib().or_gdn_conv(P(xn), P(ring), P(cw), P(on), convDim, dConv)
        out[n] = on
    return out


def mtp_state_after(m, H, DK, DV, C_, s0, delta, k, gcum):
    out = np.empty(H * DK * DV, np.float32)
    arrs = [np.ascontiguousarray(a, np.float32) for a in (s0, delta, k, gcum)]
    lib().or_mtp_state_after(m, H, DK, DV, C_, *[P(a) for a in arrs], P(out))
    return out
