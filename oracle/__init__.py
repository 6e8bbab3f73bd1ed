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
    "or_q2_0_matmat": (None, [_vp, _i64, _i64, _i64, _vp, _vp, _i]),
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

_lib = None  # noqa


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


def q2_0_matmat(blocks: np.ndarray, K: int, M: int, X: np.ndarray, threads: int = 1) -> np.ndarray:
    """X [T][K] -> [T][M]: T mat-vecs, each bit-identical to q2_0_matvec."""
    X = np.ascontiguousarray(X, np.float32)
    T = X.shape[0]
    out = np.empty((T, M), np.float32)
    lib().or_q2_0_matmat(P(blocks), K, M, T, P(X), P(out), threads)
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
    w = np.ascontiguousarray(w, np.float32)
    lib().or_rmsnorm_rows(P(x), d, x.size // d, P(w), eps)
    return x


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    n = x.shape[-1]
    w = np.ascontiguousarray(w, np.float32)
    for r in range(x.size // n):
        lib().or_rmsnorm(P(x) + 4 * r * n, P(w), P(y) + 4 * r * n, n, eps)
    return y


def softmax(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).copy()
    lib().or_softmax(P(x), x.size)
    return x


def rope_neox(x: np.ndarray, head_dim: int, n_rot: int, base: float, pos: int) -> np.ndarray:
    """x [nHead * head_dim] (heads contiguous), rotated in a copy."""
    x = np.ascontiguousarray(x, np.float32).copy()
    lib().or_rope_neox(P(x), head_dim, x.size // head_dim, n_rot, base, pos)
    return x


def gdn_gate(bPre, aPre, dt, aNeg, nV):
    bPre = np.ascontiguousarray(bPre, np.float32)
    aPre = np.ascontiguousarray(aPre, np.float32)
    beta = np.empty_like(bPre)
    g = np.empty_like(bPre)
    dt = np.ascontiguousarray(dt, np.float32)       # keep the converted arrays alive
    aNeg = np.ascontiguousarray(aNeg, np.float32)
    lib().or_gdn_gate(P(bPre), P(aPre), P(dt), P(aNeg), P(beta), P(g), nV, bPre.size)
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


# ---- hybrid stack -------------------------------------------------------------

class OrStackLayer(C.Structure):
    _fields_ = [("rec", _i)] + [(n, _vp) for n in (
        "attn_norm", "post_norm", "wqkv", "wgate", "wbeta", "walpha", "ssm_out", "conv_w", "dt",
        "a_neg", "ssm_norm", "wq", "wk", "wv", "wo", "q_norm", "k_norm", "ffn_gate", "ffn_up",
        "ffn_down", "conv_state", "rec_state", "kcache", "vcache")]


class OrStack(C.Structure):
    _fields_ = [(n, _i) for n in ("n_layer", "n_embd", "n_ff", "n_head", "n_head_kv", "head_dim",
                                  "n_rot")] + [("rope_base", _f), ("eps", _f)] + \
               [(n, _i) for n in ("n_vocab", "d_state", "n_k_head", "n_v_head", "d_conv",
                                  "max_ctx", "stage_f16", "threads", "dense")] + \
               [("layers", C.POINTER(OrStackLayer)), ("embd", _vp), ("out_norm", _vp),
                ("head", _vp), ("rope_shift", _i)]


_PROTOS["or_stack_token"] = (None, [C.POINTER(OrStack), _i, _i, _vp, _vp])
_PROTOS["or_stack_prefill"] = (None, [C.POINTER(OrStack), _vp, _i, _i, _vp, _vp])

STAGE_MV, STAGE_KV, STAGE_MVO = 1, 2, 4       # OR_STAGE_* of gd_oracle.h


class Stack:
    """CPU restatement of BonsaiEngine over given weights.

    `tensors(layer, name)` must return a GGUF-block uint8 array for Q2_0
    tensors and an f32 array otherwise (layer -1: global tensors).

    With stage_f16, `prefill` rounds every mat-vec input to f16 (the reference
    GPU prefill GEMM stages half tiles, Kernels.metal:428) and `token` does not
    (its decode GEMV reads f32 x, Kernels.metal:32-40) unless decode_f16 says
    so: True rounds every decode mat-vec input, "outputs" only those of the
    output projections (ssm_out, attn_output, ffn_down: this build's decode,
    whose norm-fed GEMVs read their input at f32 precision); cached K/V are
    always rounded (half KV pages).  With untied the
    lm_head is tensors(-1, "output"), else the token embedding (Model.swift:145).
    cfg["dense"] (default 0) selects the dense qwen3 lineage: every layer
    attention, plain q, ungated output, the pre-FFN norm named ffn_norm
    (Model.swift:23-25, 103-106)."""

    Q2 = {"rec": ("attn_qkv", "attn_gate", "ssm_beta", "ssm_alpha", "ssm_out"),
          "att": ("attn_q", "attn_k", "attn_v", "attn_output")}

    def __init__(self, cfg: dict, tensors, stage_f16: bool = True, threads: int = 8,
                 decode_f16: bool | str = False, untied: bool = False):
        self.cfg = cfg
        self.stage_prefill = (STAGE_MV | STAGE_KV) if stage_f16 else 0
        if decode_f16 not in (False, True, "outputs"):
            raise ValueError(f"decode_f16: {decode_f16!r}")
        dec = STAGE_MVO if decode_f16 == "outputs" else STAGE_MV if decode_f16 else 0
        self.stage_decode = (STAGE_KV | dec) if stage_f16 else 0
        self.keep = []
        n = cfg["n_layer"]
        self.layers = (OrStackLayer * n)()
        hd, nkv = cfg["head_dim"], cfg["n_head_kv"]
        convDim = (2 * cfg["n_k_head"] + cfg["n_v_head"]) * cfg["d_state"]

        def ptr(a):
            a = np.ascontiguousarray(a)
            self.keep.append(a)
            return a.ctypes.data

        for il in range(n):
            L = self.layers[il]
            L.rec = 1 if (il + 1) % cfg["attn_interval"] != 0 else 0
            get = lambda name: ptr(tensors(il, name))
            L.attn_norm = get("attn_norm")
            L.post_norm = get("ffn_norm" if cfg.get("dense") else "post_attention_norm")
            L.ffn_gate, L.ffn_up, L.ffn_down = get("ffn_gate"), get("ffn_up"), get("ffn_down")
            if L.rec:
                L.wqkv, L.wgate, L.wbeta, L.walpha, L.ssm_out = (get(x) for x in self.Q2["rec"])
                L.conv_w, L.dt, L.a_neg, L.ssm_norm = (get(x) for x in
                                                      ("ssm_conv1d", "ssm_dt", "ssm_a", "ssm_norm"))
                L.conv_state = ptr(np.zeros((cfg["d_conv"] - 1) * convDim, np.float32))
                L.rec_state = ptr(np.zeros(cfg["n_v_head"] * cfg["d_state"] ** 2, np.float32))
            else:
                L.wq, L.wk, L.wv, L.wo = (get(x) for x in self.Q2["att"])
                L.q_norm, L.k_norm = get("attn_q_norm"), get("attn_k_norm")
                L.kcache = ptr(np.zeros(cfg["max_ctx"] * nkv * hd, np.float32))
                L.vcache = ptr(np.zeros(cfg["max_ctx"] * nkv * hd, np.float32))
        st = OrStack()
        for k in ("n_layer", "n_embd", "n_ff", "n_head", "n_head_kv", "head_dim", "n_rot",
                  "rope_base", "eps", "n_vocab", "d_state", "n_k_head", "n_v_head", "d_conv",
                  "max_ctx"):
            setattr(st, k, cfg[k])
        st.stage_f16 = self.stage_decode
        st.threads = threads
        st.dense = 1 if cfg.get("dense") else 0
        st.layers = self.layers
        st.embd = ptr(tensors(-1, "token_embd"))
        st.out_norm = ptr(tensors(-1, "output_norm"))
        st.head = ptr(tensors(-1, "output")) if untied else None
        self.st = st
        self.pos = 0

    @property
    def rope_shift(self) -> int:
        """Rope position = position + rope_shift (MetalEngine.ropeShift)."""
        return self.st.rope_shift

    @rope_shift.setter
    def rope_shift(self, v: int):
        self.st.rope_shift = v

    def token(self, tok: int):
        """Advance one token (decode); returns (hidden, logits)."""
        h = np.empty(self.cfg["n_embd"], np.float32)
        lg = np.empty(self.cfg["n_vocab"], np.float32)
        self.st.stage_f16 = self.stage_decode
        lib().or_stack_token(C.byref(self.st), tok, self.pos, P(h), P(lg))
        self.pos += 1
        return h, lg

    def prefill(self, ids):
        """Advance over a prompt chunk (the same per-token arithmetic as
        `token` per id, with prefill staging); returns the last token's
        (hidden, logits)."""
        ids = np.ascontiguousarray(ids, np.int32)
        h = np.empty(self.cfg["n_embd"], np.float32)
        lg = np.empty(self.cfg["n_vocab"], np.float32)
        self.st.stage_f16 = self.stage_prefill
        lib().or_stack_prefill(C.byref(self.st), P(ids), ids.size, self.pos, P(h), P(lg))
        self.pos += ids.size
        return h, lg

    def layer_state(self, il: int, name: str) -> np.ndarray:
        L = self.layers[il]
        cfg = self.cfg
        if name == "ssm_state":
            n = cfg["n_v_head"] * cfg["d_state"] ** 2
            return np.ctypeslib.as_array(C.cast(L.rec_state, C.POINTER(C.c_float)), (n,)).copy()
        if name == "ssm_conv_state":
            n = (cfg["d_conv"] - 1) * (2 * cfg["n_k_head"] + cfg["n_v_head"]) * cfg["d_state"]
            return np.ctypeslib.as_array(C.cast(L.conv_state, C.POINTER(C.c_float)), (n,)).copy()
        if name in ("k_cache", "v_cache"):
            # Positions [0, pos) of an attention layer's cache, [pos][n_head_kv * head_dim].
            n = self.pos * cfg["n_head_kv"] * cfg["head_dim"]
            ptr = L.kcache if name == "k_cache" else L.vcache
            return np.ctypeslib.as_array(C.cast(ptr, C.POINTER(C.c_float)), (max(n, 1),))[:n].copy()
        raise KeyError(name)
