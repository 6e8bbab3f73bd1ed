"""gd_gdn_prefill_noalloc (the chunked GDN prefill over a fixed device scratch
array, for callers that cannot allocate) against gd_gdn_prefill (the same
kernels over the context workspace): bit-identical o and S on two calls in a
row, the second smaller and run over the first one's leftover scratch; shapes
beyond the scratch are rejected."""
import ctypes as C

import numpy as np
import pytest

import gadeon_amd as ga
import oracle as O
from conftest import rel_diff

pytestmark = pytest.mark.gpu


def inputs(T, nV, nK, dS, seed, io):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((T, nK, dS))
    k = rng.standard_normal((T, nK, dS))
    q = q / np.linalg.norm(q, axis=-1, keepdims=True)
    k = k / np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((T, nV, dS))
    dt = np.float16 if io == ga.F16 else np.float32
    beta = (1 / (1 + np.exp(-rng.standard_normal((T, nV))))).astype(np.float32)
    g = (-np.logaddexp(0, rng.standard_normal((T, nV)))).astype(np.float32)
    S = (rng.standard_normal((nV, dS, dS)) * 0.02).astype(np.float32)
    return q.astype(dt), k.astype(dt), v.astype(dt), g, beta, S


def run(ctx, fn, T, nV, nK, chunk, io, data):
    dS = 128
    q, k, v, g, beta, S = data
    raw = (lambda a: a.view(np.uint16)) if io == ga.F16 else (lambda a: a)
    dq, dk, dv = ctx.put(raw(q)), ctx.put(raw(k)), ctx.put(raw(v))
    dg, db, dS_ = ctx.put(g), ctx.put(beta), ctx.put(S)
    do = ctx.alloc(T * nV * dS * (2 if io == ga.F16 else 4))
    rc = getattr(ctx.lib, fn)(ctx.h, T, nV, nK, dS, dS, dq, nK * dS, dk, nK * dS, dv, nV * dS, io,
                              dg, db, dS_, do, nV * dS, io, C.c_float(1 / np.sqrt(dS)), chunk)
    ctx.check(rc)
    o = ctx.get(do, T * nV * dS, np.uint16 if io == ga.F16 else np.float32)
    Sn = ctx.get(dS_, S.size, np.float32)
    for p in (dq, dk, dv, dg, db, dS_, do):
        ctx.free(p)
    return o, Sn


def test_noalloc_prefill_equals_prefill_twice(ctx):
    cases = [(512, 16, 16, 64, ga.F16), (100, 4, 2, 32, ga.F32)]     # config 2, then smaller
    for i, (T, nV, nK, chunk, io) in enumerate(cases):
        data = inputs(T, nV, nK, 128, 70 + i, io)
        o_ws, S_ws = run(ctx, "gd_gdn_prefill", T, nV, nK, chunk, io, data)
        o_na, S_na = run(ctx, "gd_gdn_prefill_noalloc", T, nV, nK, chunk, io, data)
        assert np.array_equal(o_na, o_ws), (T, nV)
        assert np.array_equal(S_na, S_ws), (T, nV)
        # and both against the sequential scan (the prefill tests' bar)
        q, k, v, g, beta, S = data
        S_ref = S.copy()
        o_ref = O.gdn_sequential(q.astype(np.float32), k.astype(np.float32),
                                 v.astype(np.float32), g, beta, S_ref, np.float32(1 / np.sqrt(128)))
        o_got = o_na.view(np.float16).astype(np.float32) if io == ga.F16 else o_na
        assert rel_diff(o_got.reshape(o_ref.shape), o_ref) < 2e-3
        assert rel_diff(S_na, S_ref) < 2e-3


def test_noalloc_prefill_rejects_beyond_scratch(ctx):
    T, nV, dS = 4096, 16, 128                 # 16 x 64 chunks x 98,560 B > 32 MiB
    d = ctx.alloc(16)
    rc = ctx.lib.gd_gdn_prefill_noalloc(ctx.h, T, nV, nV, dS, dS, d, nV * dS, d, nV * dS, d,
                                        nV * dS, ga.F16, d, d, d, d, nV * dS, ga.F16,
                                        C.c_float(0.1), 64)
    assert rc == ga.GD_EINVAL
    assert b"scratch" in ctx.lib.gd_last_error(ctx.h)
    ctx.free(d)
