"""GPU parity of the Q2_0 kernels on weights that use all four codes.

The format's code 3 (weight +2d, Quant.swift:56-68) is valid but the
ternary generators never draw it, so every other test sees codes 0..2 only.
Here the code bytes are uniformly random (codes 0..3 equally likely) and the
scales uniform in [0.01, 0.05] (f16), and each kernel form is compared with
the oracle's Q2_0.matvec restatement at the tolerances of the ternary tests:
the GEMV (f16 and f32 x, the fp4 body and, past ~30K, the f16 body), the
fused add + norm GEMV (plain and SwiGLU output), the GEMM on every tile and a
K split, the 17-fragment tile, and the SwiGLU GEMM on both of its tilings.
"""
import ctypes as C

import numpy as np
import pytest

import gadeon_amd as ga
import oracle as O
from conftest import rel_diff

pytestmark = pytest.mark.gpu


def blocks4(K: int, R: int, seed: int) -> np.ndarray:
    """R rows of K/128 Q2_0 blocks with uniformly random code bytes."""
    rng = np.random.default_rng(seed)
    nb = R * (K // 128)
    b = np.empty((nb, 34), np.uint8)
    d = rng.uniform(0.01, 0.05, nb).astype(np.float16)
    b[:, :2] = d.view(np.uint8).reshape(nb, 2)
    b[:, 2:] = rng.integers(0, 256, (nb, 32), dtype=np.uint8)
    return b.ravel()


def upload(ctx, blocks, K, R):
    w = ga.Q2W()
    ctx.gd_q2_0_upload(blocks.ctypes.data, K, R, C.byref(w))
    return w


def test_generator_uses_every_code():
    b = blocks4(1024, 16, 1).reshape(-1, 34)[:, 2:]
    codes = np.stack([(b >> s) & 3 for s in (0, 2, 4, 6)])
    counts = np.bincount(codes.ravel(), minlength=4)
    assert counts.min() > 0.2 * codes.size


@pytest.mark.parametrize("K,R", [(1024, 3072), (5120, 777), (384, 37), (32768, 64)])
@pytest.mark.parametrize("xt", [ga.F16, ga.F32])
def test_gemv_code3(ctx, K, R, xt):
    blocks = blocks4(K, R, K + R + xt)
    w = upload(ctx, blocks, K, R)
    if xt == ga.F16:
        xh = O.lcg_normal_f16(K, 6)
        x_ref, dx = xh.astype(np.float32), ctx.put(xh.view(np.uint16))
    else:
        x_ref = O.lcg_normal(K, 6)
        dx = ctx.put(x_ref)
    dy = ctx.alloc(R * 4)
    ctx.gd_q2_0_gemv(C.byref(w), dx, xt, dy)
    want = O.q2_0_matvec(blocks, K, R, x_ref, threads=8)
    assert rel_diff(ctx.get(dy, R, np.float32), want) < 1e-4
    ctx.free(dx)
    ctx.free(dy)
    ctx.gd_q2w_free(C.byref(w))


@pytest.mark.parametrize("K,R,glu", [(5120, 777, False), (5120, 34816, False), (5120, 1024, True)])
def test_gemv_norm_code3(ctx, K, R, glu):
    eps = 1e-6
    blocks = blocks4(K, R, 7 * K + R)
    w = upload(ctx, blocks, K, R)
    h = O.lcg_normal(K, 91, 0.0, 3.0)
    d = O.lcg_normal(K, 92, 0.0, 1.0)
    wn = O.lcg_normal(K, 93, 1.0, 0.2)
    dh, dd, dwn, dho = ctx.put(h), ctx.put(d), ctx.put(wn), ctx.alloc(K * 4)
    x = O.rmsnorm((h + d).astype(np.float32)[None], wn, eps)[0]
    y = O.q2_0_matvec(blocks, K, R, x, threads=8)
    if glu:
        ff = R // 2
        dO = ctx.alloc(ff * 2)
        ctx.gd_q2_0_gemv_norm(C.byref(w), dh, dd, 1, 0, dwn, eps, dho, None, dO)
        want = (y[:ff] / (1 + np.exp(-y[:ff])) * y[ff:]).astype(np.float16).astype(np.float32)
        got = ctx.get(dO, ff, np.float16).astype(np.float32)
        assert rel_diff(got, want) < 2e-3
        ctx.free(dO)
    else:
        dy = ctx.alloc(R * 4)
        ctx.gd_q2_0_gemv_norm(C.byref(w), dh, dd, 1, 0, dwn, eps, dho, dy, None)
        assert rel_diff(ctx.get(dy, R, np.float32), y) < 1e-4
        ctx.free(dy)
    for p in (dh, dd, dwn, dho):
        ctx.free(p)
    ctx.gd_q2w_free(C.byref(w))


PLANS = [(1, 1, 4), (2, 1, 4), (4, 1, 4), (2, 2, 4), (4, 2, 4), (8, 1, 4),
         (2, 1, 8), (4, 1, 8), (2, 2, 8), (4, 2, 8)]


@pytest.mark.parametrize("mt,nt,nw", PLANS)
@pytest.mark.parametrize("split,yt", [(1, ga.F32), (3, ga.F16)])
def test_gemm_every_plan_code3(ctx, mt, nt, nw, split, yt):
    T, K, R = 150, 2688, 500
    blocks = blocks4(K, R, 13 * mt + 5 * nt + nw)
    w = upload(ctx, blocks, K, R)
    Xh = O.lcg_normal_f16(T * K, 80).reshape(T, K)
    dX = ctx.put(Xh.view(np.uint16))
    dY = ctx.alloc(T * R * (4 if yt == ga.F32 else 2))
    ctx.gd_q2_0_gemm_plan(C.byref(w), T, dX, ga.F16, dY, yt, mt, nt, split, nw)
    Y = ctx.get(dY, (T, R), np.float32 if yt == ga.F32 else np.float16).astype(np.float32)
    want = np.asarray(O.q2_0_matmat(blocks, K, R, Xh.astype(np.float32), 8)).reshape(T, R)
    assert rel_diff(Y, want) < (2e-3 if yt == ga.F16 else 1e-4)
    ctx.free(dX)
    ctx.free(dY)
    ctx.gd_q2w_free(C.byref(w))


@pytest.mark.parametrize("T,K,R,split,yt", [(200, 2688, 1100, 1, ga.F32),
                                            (130, 1024, 1100, 3, ga.F16)])
def test_gemm_plan17_code3(ctx, T, K, R, split, yt):
    blocks = blocks4(K, R, 3 * R + split)
    w = upload(ctx, blocks, K, R)
    Xh = O.lcg_normal_f16(T * K, 84).reshape(T, K)
    dX = ctx.put(Xh.view(np.uint16))
    dY = ctx.alloc(T * R * (4 if yt == ga.F32 else 2))
    ctx.gd_q2_0_gemm_plan17(C.byref(w), T, dX, ga.F16, dY, yt, split)
    Y = ctx.get(dY, (T, R), np.float32 if yt == ga.F32 else np.float16).astype(np.float32)
    want = np.asarray(O.q2_0_matmat(blocks, K, R, Xh.astype(np.float32), 8)).reshape(T, R)
    tol = 2e-3 if yt == ga.F16 else 1e-4
    assert rel_diff(Y, want) < tol
    extra = np.concatenate([np.arange(c, min(c + 32, R)) for c in range(512, R, 544)])
    assert rel_diff(Y[:, extra], want[:, extra]) < tol
    ctx.free(dX)
    ctx.free(dY)
    ctx.gd_q2w_free(C.byref(w))


def test_gemm_plan17_f16_ragged_output_runs_plain_tile(ctx):
    """f16 Y with a K split on an output whose T x R is not a multiple of 4:
    the split is dropped (partials are summed 4 at a time) and, the
    17-fragment tile writing f32 only, the plain tile runs instead."""
    T, K, R = 7, 1024, 545
    assert T * R % 4
    blocks = blocks4(K, R, 99)
    w = upload(ctx, blocks, K, R)
    Xh = O.lcg_normal_f16(T * K, 85).reshape(T, K)
    dX, dY = ctx.put(Xh.view(np.uint16)), ctx.alloc(T * R * 2)
    ctx.gd_q2_0_gemm_plan17(C.byref(w), T, dX, ga.F16, dY, ga.F16, 2)
    Y = ctx.get(dY, (T, R), np.float16).astype(np.float32)
    want = np.asarray(O.q2_0_matmat(blocks, K, R, Xh.astype(np.float32), 8)).reshape(T, R)
    assert rel_diff(Y, want) < 2e-3
    ctx.free(dX)
    ctx.free(dY)
    ctx.gd_q2w_free(C.byref(w))


@pytest.mark.parametrize("T,K,ff", [(512, 1024, 17408), (77, 512, 4352)])
@pytest.mark.parametrize("tile17", [1, 0])
def test_gemm_swiglu_code3(ctx, T, K, ff, tile17):
    R = 2 * ff
    blocks = blocks4(K, R, K + ff + tile17)
    w = upload(ctx, blocks, K, R)
    Xh = O.lcg_normal_f16(T * K, 86).reshape(T, K)
    dX, dO = ctx.put(Xh.view(np.uint16)), ctx.alloc(T * ff * 2)
    ctx.gd_q2_0_gemm_swiglu_plan(C.byref(w), T, dX, dO, tile17)
    out = ctx.get(dO, (T, ff), np.float16).astype(np.float32)
    blk = blocks.reshape(R, -1)
    g, u = np.ascontiguousarray(blk[:ff]), np.ascontiguousarray(blk[ff:])
    for t in sorted({0, 31, 32, 127, 128, 255, 256, T - 1} & set(range(T))):
        x = Xh[t].astype(np.float32)
        gv = O.q2_0_matvec(g, K, ff, x, threads=8)
        uv = O.q2_0_matvec(u, K, ff, x, threads=8)
        want = (gv / (1 + np.exp(-gv)) * uv).astype(np.float16).astype(np.float32)
        assert rel_diff(out[t], want) < 2e-3, t
    ctx.free(dX)
    ctx.free(dO)
    ctx.gd_q2w_free(C.byref(w))
