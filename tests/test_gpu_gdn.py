"""GPU parity of the Gated DeltaNet path against the CPU oracle (GDN.swift,
Kernels.swift restated).  Tolerance for the recurrence (outputs and states):
norm-wise relative error < 2e-3 (north star), max|a-b|/max|b| as
MetalSelfTest.swift:437-448 defines it.  Elementwise glue: 1e-5 relative."""
import numpy as np
import pytest

import gadeon_amd as ga
import oracle as O
from conftest import rel_diff

pytestmark = pytest.mark.gpu

EPS = 1e-6


def sigmoid(x):
    return 1 / (1 + np.exp(-x))


def softplus(x):
    return np.logaddexp(0, x)


# ------------------------------------------------------------------ glue

def test_gate(ctx):
    nV, N = 16, 37
    bPre = O.lcg_normal(N * nV, 1)
    aPre = O.lcg_normal(N * nV, 2)
    dt = O.lcg_normal(nV, 3, 0, 0.5)
    aNeg = -np.exp(O.lcg_normal(nV, 4, 0, 0.5))
    d = [ctx.put(a) for a in (bPre, aPre, dt, aNeg)]
    db, dg = ctx.alloc(N * nV * 4), ctx.alloc(N * nV * 4)
    ctx.gd_gdn_gate(*d, db, dg, nV, N * nV)
    wb, wg = O.gdn_gate(bPre, aPre, dt, aNeg, nV)
    assert rel_diff(ctx.get(db, N * nV, np.float32), wb) < 1e-5
    assert rel_diff(ctx.get(dg, N * nV, np.float32), wg) < 1e-5


@pytest.mark.parametrize("N", [1, 7])
def test_conv(ctx, N):
    convDim, kc = 6144, 4
    x = O.lcg_normal(N * convDim, 11).reshape(N, convDim)
    ring = O.lcg_normal((kc - 1) * convDim, 12)
    cw = O.lcg_uniform(convDim * kc, 13, -0.5, 0.5)
    dx, dr, dw = ctx.put(x), ctx.put(ring), ctx.put(cw)
    do = ctx.alloc(x.nbytes)
    ctx.gd_gdn_conv(dx, dr, dw, do, convDim, kc, N)
    ring_ref = ring.copy()
    want = O.gdn_conv(x, ring_ref, cw, convDim, kc)
    assert rel_diff(ctx.get(do, (N, convDim), np.float32), want) < 1e-5
    assert rel_diff(ctx.get(dr, ring.size, np.float32), ring_ref) < 1e-6


def test_norms_and_elementwise(ctx):
    N, nK, d, convDim = 9, 16, 128, 6144
    x = O.lcg_normal(N * convDim, 21).reshape(N, convDim)
    dx = ctx.put(x)
    ctx.gd_l2norm_rows(dx, d, 2 * nK, convDim, N, EPS)       # q|k of every token
    got = ctx.get(dx, (N, convDim), np.float32)
    want = x.copy()
    want[:, :2 * nK * d] = O.l2norm_rows(x[:, :2 * nK * d], d, EPS).reshape(N, -1)
    assert rel_diff(got, want) < 1e-5
    w = O.lcg_uniform(d, 22, 0.5, 1.5)
    o = O.lcg_normal(N * 16 * d, 23)
    do, dw = ctx.put(o), ctx.put(w)
    ctx.gd_rmsnorm_rows(do, d, N * 16, dw, EPS)
    assert rel_diff(ctx.get(do, o.size, np.float32), O.rmsnorm_rows(o, d, w, EPS)) < 1e-5
    n = 5120
    h = O.lcg_normal(3 * n, 24).reshape(3, n)
    wn = O.lcg_uniform(n, 25, 0.5, 1.5)
    dh, dwn = ctx.put(h), ctx.put(wn)
    dy = ctx.alloc(h.nbytes)
    ctx.gd_rmsnorm(dh, dwn, dy, ga.F32, n, 3, EPS)
    want = O.rmsnorm(h, wn, EPS)
    assert rel_diff(ctx.get(dy, (3, n), np.float32), want) < 1e-5
    ctx.gd_rmsnorm(dh, dwn, dy, ga.F16, n, 3, EPS)
    assert np.array_equal(ctx.get(dy, (3, n), np.float16), want.astype(np.float16)) or \
        rel_diff(ctx.get(dy, (3, n), np.float16), want) < 1e-3
    a, b = O.lcg_normal(1000, 26), O.lcg_normal(1000, 27)
    for fn, ref in ((ctx.gd_silu_mul, a / (1 + np.exp(-a)) * b),
                    (ctx.gd_mul_silu, a * (b / (1 + np.exp(-b)))),
                    (ctx.gd_add, a + b)):
        da, db = ctx.put(a), ctx.put(b)
        fn(da, db, a.size)
        assert rel_diff(ctx.get(da, a.size, np.float32), ref) < 1e-5


# ------------------------------------------------------------------ scan

@pytest.mark.parametrize("nV,nK,dS", [(16, 16, 128), (16, 4, 128), (6, 3, 64)])
def test_scan_single_token(ctx, nV, nK, dS):
    q = O.l2norm_rows(O.lcg_normal(nK * dS, 31), dS, EPS)
    k = O.l2norm_rows(O.lcg_normal(nK * dS, 32), dS, EPS)
    v = O.lcg_normal(nV * dS, 33)
    g = -softplus(O.lcg_normal(nV, 34)).astype(np.float32)
    beta = sigmoid(O.lcg_normal(nV, 35)).astype(np.float32)
    S = O.lcg_normal(nV * dS * dS, 36, 0, 0.02)
    d = [ctx.put(a) for a in (q, k, v, g, beta, S)]
    do = ctx.alloc(nV * dS * 4)
    ctx.gd_gdn_scan(*d, do, nV, nK, dS, 1 / np.sqrt(dS))
    S_ref = S.copy()
    o_ref = O.gdn_scan(q, k, v, g, beta, S_ref, nV, nK, dS, np.float32(1 / np.sqrt(dS)))
    assert rel_diff(ctx.get(do, nV * dS, np.float32), o_ref) < 2e-3
    assert rel_diff(ctx.get(d[5], S.size, np.float32), S_ref) < 2e-3


def decode_inputs(B, nV, nK, dS, step, gate):
    s = 1000 * step
    q = O.lcg_normal_f16(B * nK * dS, s + 1)
    k = O.lcg_normal_f16(B * nK * dS, s + 2)
    v = O.lcg_normal_f16(B * nV * dS, s + 3)
    a = O.lcg_normal(B * nV, s + 4)
    b = O.lcg_normal(B * nV, s + 5)
    if gate:
        return q, k, v, a, b
    return q, k, v, (-softplus(a)).astype(np.float32), sigmoid(b).astype(np.float32)


@pytest.mark.parametrize("B,steps,gate", [(1, 128, False), (32, 128, False), (4, 16, True)])
def test_decode_fused_vs_oracle(ctx, B, steps, gate):
    """B independent sequences, 16 heads, 128x128 f32
    state ~ N(0, 0.02), raw f16 q/k (normalized in-kernel), 128 steps."""
    nV = nK = 16
    dS = 128
    S = O.lcg_normal(B * nV * dS * dS, 7, 0, 0.02)
    dt = O.lcg_normal(nV, 8, 0, 0.5)
    aNeg = -np.exp(O.lcg_normal(nV, 9, 0, 0.3))
    dS_ = ctx.put(S)
    ddt, daN = (ctx.put(dt), ctx.put(aNeg)) if gate else (None, None)
    S_ref = S.copy()
    qs = np.float32(1 / np.sqrt(dS))
    for step in range(steps):
        q, k, v, gi, bi = decode_inputs(B, nV, nK, dS, step, gate)
        dq, dk, dv = ctx.put(q.view(np.uint16)), ctx.put(k.view(np.uint16)), ctx.put(v.view(np.uint16))
        dg, db = ctx.put(gi), ctx.put(bi)
        do = ctx.alloc(B * nV * dS * 2)
        ctx.gd_gdn_decode(B, nV, nK, dS, dq, dk, dv, ga.F16, dg, db, ddt, daN, dS_, do, qs, EPS)
        if gate:
            beta_r, g_r = O.gdn_gate(bi, gi, dt, aNeg, nV)
        else:
            g_r, beta_r = gi, bi
        q32, k32, v32 = q.astype(np.float32), k.astype(np.float32), v.astype(np.float32)
        g_r, beta_r = np.ascontiguousarray(g_r, np.float32), np.ascontiguousarray(beta_r, np.float32)
        o_ref = np.empty(B * nV * dS, np.float32)
        O.lib().or_gdn_decode_batch(B, nV, nK, dS, O.P(q32), O.P(k32),
                                    O.P(v32), O.P(g_r), O.P(beta_r),
                                    O.P(S_ref), O.P(o_ref), qs, EPS, 16)
        o = ctx.get(do, B * nV * dS, np.float16)
        assert rel_diff(o, o_ref) < 2e-3, step
        for p in (dq, dk, dv, dg, db, do):
            ctx.free(p)
    assert rel_diff(ctx.get(dS_, S.size, np.float32), S_ref) < 2e-3


# ---------------------------------------------------------------- prefill

def prefill_inputs(T, nV, nK, dS, seed, s0_scale=0.0):
    q = O.lcg_normal(T * nK * dS, seed).reshape(T, nK, dS)
    k = O.lcg_normal(T * nK * dS, seed + 1).reshape(T, nK, dS)
    q = (q / np.linalg.norm(q, axis=-1, keepdims=True)).astype(np.float16)
    k = (k / np.linalg.norm(k, axis=-1, keepdims=True)).astype(np.float16)
    v = O.lcg_normal_f16(T * nV * dS, seed + 2).reshape(T, nV, dS)
    beta = sigmoid(O.lcg_normal(T * nV, seed + 3)).astype(np.float32).reshape(T, nV)
    g = (-softplus(O.lcg_normal(T * nV, seed + 4))).astype(np.float32).reshape(T, nV)
    S = O.lcg_normal(nV * dS * dS, seed + 5, 0, s0_scale).reshape(nV, dS, dS) if s0_scale \
        else np.zeros((nV, dS, dS), np.float32)
    return q, k, v, g, beta, S


@pytest.mark.parametrize("T,nV,nK,C,io,s0", [
    (512, 16, 16, 64, ga.F16, 0.0),
    (100, 16, 4, 32, ga.F32, 0.02),      # ragged last chunk, GQA heads, f32 io
    (37, 4, 4, 16, ga.F16, 0.02),
    (1, 2, 2, 64, ga.F32, 0.02),
    (64, 3, 1, 64, ga.F16, 0.0),
])
def test_prefill_chunked_vs_sequential(ctx, T, nV, nK, C, io, s0):
    dS = 128
    q, k, v, g, beta, S = prefill_inputs(T, nV, nK, dS, 50 + T, s0)
    cv = (lambda a: a.view(np.uint16)) if io == ga.F16 else (lambda a: a.astype(np.float32))
    dq, dk, dv = ctx.put(cv(q)), ctx.put(cv(k)), ctx.put(cv(v))
    dg, db, dS_ = ctx.put(g), ctx.put(beta), ctx.put(S)
    do = ctx.alloc(T * nV * dS * (2 if io == ga.F16 else 4))
    ctx.gd_gdn_prefill(T, nV, nK, dS, dS, dq, nK * dS, dk, nK * dS, dv, nV * dS, io, dg, db,
                       dS_, do, nV * dS, io, 1 / np.sqrt(dS), C)
    S_ref = S.astype(np.float32).copy()
    o_ref = O.gdn_sequential(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32),
                             g, beta, S_ref, np.float32(1 / np.sqrt(dS)))
    o = ctx.get(do, (T, nV, dS), np.float16 if io == ga.F16 else np.float32)
    assert rel_diff(o, o_ref) < 2e-3
    assert rel_diff(ctx.get(dS_, S.size, np.float32), S_ref) < 2e-3


@pytest.mark.parametrize("dS", [128, 64, 96, 256, 48])
def test_scan_batch_conv_layout(ctx, dS):
    """MetalEnc.gdnScanBatch's packed convOut[N][q|k|v] layout (MetalEnc.swift:741-778),
    for the state sizes the reference serves: 128 on the chunked prefill, the
    others (dS % 32 == 0 up to 256 in gdn_scan_batch2, anything else in
    gdn_scan_batch) on the token-serial scan."""
    N, nK, nV = 70, 4, 8
    keyDim, valueDim = nK * dS, nV * dS
    convDim = 2 * keyDim + valueDim
    conv = O.lcg_normal(N * convDim, 61).reshape(N, convDim)
    conv[:, :2 * keyDim] = O.l2norm_rows(conv[:, :2 * keyDim], dS, EPS).reshape(N, -1)
    g = (-softplus(O.lcg_normal(N * nV, 62))).astype(np.float32)
    beta = sigmoid(O.lcg_normal(N * nV, 63)).astype(np.float32)
    S = O.lcg_normal(nV * dS * dS, 64, 0, 0.02)
    dc, dg, db, dS_ = ctx.put(conv), ctx.put(g), ctx.put(beta), ctx.put(S)
    do = ctx.alloc(N * valueDim * 4)
    ctx.gd_gdn_scan_batch(dc, keyDim, valueDim, convDim, dg, db, dS_, do, nV, nK, dS,
                          1 / np.sqrt(dS), N)
    S_ref = S.copy()
    qk = conv[:, :2 * keyDim]
    o_ref = O.gdn_sequential(qk[:, :keyDim].reshape(N, nK, dS).copy(),
                             qk[:, keyDim:].reshape(N, nK, dS).copy(),
                             conv[:, 2 * keyDim:].reshape(N, nV, dS).copy(),
                             g.reshape(N, nV), beta.reshape(N, nV), S_ref,
                             np.float32(1 / np.sqrt(dS)))
    assert rel_diff(ctx.get(do, (N, nV, dS), np.float32), o_ref) < 2e-3
    assert rel_diff(ctx.get(dS_, S.size, np.float32), S_ref) < 2e-3


def test_decode_chain_equals_prefill(ctx):
    """Decoding T tokens one at a time equals one chunked prefill of T tokens."""
    T, nV, nK, dS = 48, 4, 4, 128
    q, k, v, g, beta, S = prefill_inputs(T, nV, nK, dS, 80, 0.02)
    dS_a, dS_b = ctx.put(S), ctx.put(S)
    dq, dk, dv = ctx.put(q.view(np.uint16)), ctx.put(k.view(np.uint16)), ctx.put(v.view(np.uint16))
    dg, db = ctx.put(g), ctx.put(beta)
    do = ctx.alloc(T * nV * dS * 4)
    ctx.gd_gdn_prefill(T, nV, nK, dS, dS, dq, nK * dS, dk, nK * dS, dv, nV * dS, ga.F16, dg, db,
                       dS_a, do, nV * dS, ga.F32, 1 / np.sqrt(dS), 64)
    o_pre = ctx.get(do, (T, nV, dS), np.float32)
    do1 = ctx.alloc(nV * dS * 4)
    for t in range(T):
        ctx.gd_gdn_decode(1, nV, nK, dS, dq + t * nK * dS * 2, dk + t * nK * dS * 2,
                          dv + t * nV * dS * 2, ga.F16, dg + t * nV * 4, db + t * nV * 4, None,
                          None, dS_b, do1, 1 / np.sqrt(dS), EPS)
        assert rel_diff(ctx.get(do1, (nV, dS), np.float16), o_pre[t]) < 2e-3, t
    assert rel_diff(ctx.get(dS_b, S.size, np.float32), ctx.get(dS_a, S.size, np.float32)) < 2e-3


@pytest.mark.parametrize("T,nV,nK,C", [(130, 4, 2, 64), (45, 2, 2, 32)])
def test_prefill_f32_inputs_keep_f32_precision(ctx, T, nV, nK, C):
    """f32 q, k, v that f16 cannot hold exactly (the stack's conv outputs):
    the chunked prefill carries them as hi + lo f16 pairs, so o and S follow
    the f64 sequential scan to ~1e-5 (o, whose P delta term sums many
    products, to < 1e-4) -- well inside what rounding q, k, v to f16 would
    cost (a few 1e-4, the reference's prefill scan being f32,
    Kernels.metal:1574-1625)."""
    dS = 128
    rng = np.random.default_rng(T)
    q = rng.standard_normal((T, nK, dS))
    k = rng.standard_normal((T, nK, dS))
    q = (q / np.linalg.norm(q, axis=-1, keepdims=True)).astype(np.float32)
    k = (k / np.linalg.norm(k, axis=-1, keepdims=True)).astype(np.float32)
    v = rng.standard_normal((T, nV, dS)).astype(np.float32)
    beta = sigmoid(rng.standard_normal((T, nV))).astype(np.float32)
    g = (-softplus(rng.standard_normal((T, nV)))).astype(np.float32)
    S = (rng.standard_normal((nV, dS, dS)) * 0.02).astype(np.float32)
    dq, dk, dv = ctx.put(q), ctx.put(k), ctx.put(v)
    dg, db, dS_ = ctx.put(g), ctx.put(beta), ctx.put(S)
    do = ctx.alloc(T * nV * dS * 4)
    ctx.gd_gdn_prefill(T, nV, nK, dS, dS, dq, nK * dS, dk, nK * dS, dv, nV * dS, ga.F32, dg, db,
                       dS_, do, nV * dS, ga.F32, 1 / np.sqrt(dS), C)
    S_ref = S.astype(np.float64).copy()
    o_ref = O.gdn_sequential(q, k, v, g, beta, S_ref, 1 / np.sqrt(dS), f64=True)
    ro = rel_diff(ctx.get(do, (T, nV, dS), np.float32), o_ref)
    rs = rel_diff(ctx.get(dS_, S.size, np.float32), S_ref)
    print(f"f32 io T={T}: o relDiff {ro:.2e}, S relDiff {rs:.2e}")
    assert ro < 1e-4 and rs < 1e-5
