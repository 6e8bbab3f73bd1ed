"""GPU parity of the Q2_0 path against the CPU oracle (Quant.swift restated).

Tolerances (norm-wise relative error max|a-b|/max|b|, MetalSelfTest.swift:437-448):
  * codec, repack, dequant, synthetic codes/scales: bit-exact;
  * GEMV: 1e-4 (the oracle sees the same f16 x values; only summation order
    differs) -- inside the north-star bound of 1e-2;
  * GEMM: 2e-3 for f32 out (the reference's own GEMM gate, MetalSelfTest.swift:487),
    the oracle receiving X rounded to f16 exactly as both GEMMs stage it.
"""
import ctypes as C

import numpy as np
import pytest

import gadeon_amd as ga
import oracle as O
from conftest import rel_diff

pytestmark = pytest.mark.gpu


def upload_w(ctx, blocks, K, R):
    w = ga.Q2W()
    ctx.gd_q2_0_upload(blocks.ctypes.data, K, R, C.byref(w))
    return w


def free_w(ctx, w):
    ctx.gd_q2w_free(C.byref(w))


def export_w(ctx, w):
    n = w.R * (w.K // 128) * 34
    d = ctx.alloc(n)
    ctx.gd_q2_0_export(C.byref(w), d)
    out = ctx.get(d, n, np.uint8)
    ctx.free(d)
    return out


@pytest.mark.parametrize("K,R", [(128, 1), (1024, 3072), (384, 37), (5120, 64)])
def test_repack_export_round_trip(ctx, K, R):
    blocks = O.lcg_q2_0(K, R, 100 + K)
    w = upload_w(ctx, blocks, K, R)
    assert np.array_equal(export_w(ctx, w), blocks)
    free_w(ctx, w)


def test_device_generators_match_sequential_lcg(ctx):
    K, R = 1024, 300
    w = ga.Q2W()
    ctx.gd_q2w_alloc(K, R, C.byref(w))
    ctx.gd_rand_q2w(C.byref(w), 42, 0.01, 0.05)
    assert np.array_equal(export_w(ctx, w), O.lcg_q2_0(K, R, 42))
    free_w(ctx, w)
    n = 100_003
    d = ctx.alloc(n * 4)
    ctx.gd_rand_uniform(d, n, 9, -2.0, 3.0)
    assert np.array_equal(ctx.get(d, n, np.float32), O.lcg_uniform(n, 9, -2.0, 3.0))
    ctx.gd_rand_normal(d, ga.F32, n, 10, 0.5, 2.0)
    z = ctx.get(d, n, np.float32)
    assert rel_diff(z, O.lcg_normal(n, 10, 0.5, 2.0)) < 1e-5
    ctx.free(d)


def test_dequant_rows_exact(ctx):
    K, R = 5120, 50
    blocks = O.lcg_q2_0(K, R, 7)
    w = upload_w(ctx, blocks, K, R)
    ids = np.array([3, 0, 49, 17, 3, 60, -1], np.int32)    # last two out of range -> 0
    dids = ctx.put(ids)
    dout = ctx.alloc(ids.size * K * 4)
    ctx.gd_q2_0_dequant_rows(C.byref(w), dids, ids.size, dout)
    got = ctx.get(dout, (ids.size, K), np.float32)
    full = O.q2_0_dequant(blocks, K * R).reshape(R, K)
    for n, i in enumerate(ids):
        want = full[i] if 0 <= i < R else np.zeros(K, np.float32)
        assert np.array_equal(got[n], want), (n, i)
    free_w(ctx, w)


# (640, 50001) and (5120, 20500) hold more row sets than the GPU keeps
# resident, so workgroups take several sets and sets are cut between waves;
# K = 7552 is the longest x staged 8 elements a thread (f32 x: one pass of
# the workgroup's 1024 threads), 7680 the shortest staged 16 a thread.
GEMV_SHAPES = [(1024, 3072), (128, 5), (384, 37), (2048, 1000), (5120, 777), (17408, 130),
               (6144, 64), (640, 50001), (5120, 20500), (7552, 300), (7680, 300)]


@pytest.mark.parametrize("K,R", GEMV_SHAPES)
@pytest.mark.parametrize("xt", [ga.F16, ga.F32])
def test_gemv_vs_oracle(ctx, K, R, xt):
    blocks = O.lcg_q2_0(K, R, K + R)
    w = upload_w(ctx, blocks, K, R)
    if xt == ga.F16:
        xh = O.lcg_normal_f16(K, 5)
        x_ref = xh.astype(np.float32)
        dx = ctx.put(xh.view(np.uint16))
    else:
        x_ref = O.lcg_normal(K, 5)
        dx = ctx.put(x_ref)
    dy = ctx.alloc(R * 4)
    ctx.gd_q2_0_gemv(C.byref(w), dx, xt, dy)
    y = ctx.get(dy, R, np.float32)
    want = O.q2_0_matvec(blocks, K, R, x_ref, threads=8)
    assert rel_diff(y, want) < 1e-4
    # The reference's own absolute gate for the gemv self-test (MetalSelfTest.swift:504)
    # holds at these magnitudes too.
    assert np.max(np.abs(y - want)) < 1e-3 * max(1.0, np.max(np.abs(want)) / 10)
    free_w(ctx, w)
    ctx.free(dx)
    ctx.free(dy)


@pytest.mark.parametrize("K,R,with_delta", [(5120, 777, True), (5120, 34816, True),
                                            (1024, 300, False), (15744, 64, True),
                                            (7552, 200, True), (7680, 200, True)])
def test_gemv_norm_vs_oracle_and_unfused(ctx, K, R, with_delta):
    """gd_q2_0_gemv_norm == add + rmsnorm (f32 out) + f32-x GEMV: against the
    oracle, against the three device calls it replaces, and h' exactly."""
    eps = 1e-6
    blocks = O.lcg_q2_0(K, R, K + 7 * R)
    w = upload_w(ctx, blocks, K, R)
    h = O.lcg_normal(K, 91, 0.0, 3.0)
    d = O.lcg_normal(K, 92, 0.0, 1.0) if with_delta else np.zeros(K, np.float32)
    wn = O.lcg_normal(K, 93, 1.0, 0.2)
    dh, dd, dwn = ctx.put(h), ctx.put(d), ctx.put(wn)
    dho, dy = ctx.alloc(K * 4), ctx.alloc(R * 4)
    ctx.gd_q2_0_gemv_norm(C.byref(w), dh, dd if with_delta else None, 1, 0, dwn, eps, dho, dy,
                          None)
    y = ctx.get(dy, R, np.float32)
    hp = (h + d).astype(np.float32)
    assert np.array_equal(ctx.get(dho, K, np.float32), hp)
    x = O.rmsnorm(hp[None], wn, eps)[0]
    want = O.q2_0_matvec(blocks, K, R, x, threads=8)
    assert rel_diff(y, want) < 1e-4
    # the unfused device chain
    dh2, dx32, dy2 = ctx.put(h), ctx.alloc(K * 4), ctx.alloc(R * 4)
    if with_delta:
        ctx.gd_add(dh2, dd, K)
    ctx.gd_rmsnorm(dh2, dwn, dx32, ga.F32, K, 1, eps)
    ctx.gd_q2_0_gemv(C.byref(w), dx32, ga.F32, dy2)
    assert rel_diff(y, ctx.get(dy2, R, np.float32)) < 1e-4
    for p in (dh, dd, dwn, dho, dy, dh2, dx32, dy2):
        ctx.free(p)
    free_w(ctx, w)


@pytest.mark.parametrize("K,R,with_bias", [(2048, 5120, True), (2048, 300, False), (6144, 777, True),
                                           (128, 40, False)])
def test_gemv_gated_head_norm(ctx, K, R, with_bias):
    """gd_q2_0_gemv_gated == f16(rmsnorm of each 128-block of o * w * silu(z))
    into the f16-x GEMV: against the oracle's norm and matvec, and against
    the device chain it replaces (rmsnorm_rows, mul_silu, f16, GEMV).  x is
    rounded to f16 on both sides, from norm scales formed in another order,
    so an element may land one f16 step apart: 1e-3."""
    eps = 1e-6
    blocks = O.lcg_q2_0(K, R, 3 * K + R)
    w = upload_w(ctx, blocks, K, R)
    o = O.lcg_normal(K, 61, 0.0, 0.7)
    z = O.lcg_normal(K, 62, 0.0, 2.0)
    wn = O.lcg_normal(128, 63, 1.0, 0.2)
    bias = O.lcg_normal(R, 64, 0.0, 1.0) if with_bias else None
    do, dz, dwn, dy = ctx.put(o), ctx.put(z), ctx.put(wn), ctx.alloc(R * 4)
    db = ctx.put(bias) if with_bias else None
    ctx.gd_q2_0_gemv_gated(C.byref(w), do, dz, dwn, 1e-6, db, dy)
    y = ctx.get(dy, R, np.float32)
    a = O.rmsnorm_rows(o, 128, wn, eps)
    x16 = (a * (z / (1.0 + np.exp(-z)))).astype(np.float16)
    want = O.q2_0_matvec(blocks, K, R, x16.astype(np.float32), threads=8)
    if with_bias:
        want = want + bias
    assert rel_diff(y, want) < 1e-3
    # the device chain: norm rows in place, a * silu(z), f16, f16-x GEMV
    da = ctx.put(o)
    ctx.gd_rmsnorm_rows(da, 128, K // 128, dwn, eps)
    ctx.gd_mul_silu(da, dz, K)
    dx16 = ctx.put(ctx.get(da, K, np.float32).astype(np.float16).view(np.uint16))
    dy2 = ctx.alloc(R * 4)
    ctx.gd_q2_0_gemv(C.byref(w), dx16, ga.F16, dy2)
    y2 = ctx.get(dy2, R, np.float32) + (bias if with_bias else 0.0)
    assert rel_diff(y, y2) < 1e-3
    for p in (do, dz, dwn, dy, da, dx16, dy2) + ((db,) if with_bias else ()):
        ctx.free(p)
    free_w(ctx, w)


@pytest.mark.parametrize("K,R,ksplit", [(17408, 5120, 4), (2048, 5120, 2), (5120, 777, 3),
                                        (512, 100, 4), (17408, 130, 2)])
def test_gemv_split_partials_sum_to_gemv(ctx, K, R, ksplit):
    """The K-split partials add up to the oracle's y, and feed the fused
    norm GEMV as nd deltas exactly as their sum would."""
    blocks = O.lcg_q2_0(K, R, 5 * K + R)
    w = upload_w(ctx, blocks, K, R)
    x = O.lcg_normal_f16(K, 95)
    dx, dy = ctx.put(x.view(np.uint16)), ctx.alloc(4 * R * 4)
    ns = C.c_int()
    ctx.gd_q2_0_gemv_split(C.byref(w), dx, ga.F16, dy, ksplit, C.byref(ns))
    steps = (K // 128 + 3) // 4
    ks = -(-steps // ksplit)
    assert ns.value == -(-steps // ks)
    parts = ctx.get(dy, ns.value * R, np.float32).reshape(ns.value, R)
    want = O.q2_0_matvec(blocks, K, R, x.astype(np.float32), threads=8)
    assert rel_diff(parts.sum(0), want) < 1e-4
    if 128 <= R <= 15744 and R % 4 == 0:      # partial stride R must be 16-byte aligned
        # the partials as the residual delta of a fused-norm GEMV (K' = R)
        K2, R2 = R - R % 128, 64
        b2 = O.lcg_q2_0(K2, R2, 17)
        w2 = upload_w(ctx, b2, K2, R2)
        h = O.lcg_normal(K2, 96, 0.0, 2.0)
        wn = O.lcg_normal(K2, 97, 1.0, 0.1)
        dh, dwn, dho, dy2 = ctx.put(h), ctx.put(wn), ctx.alloc(K2 * 4), ctx.alloc(R2 * 4)
        ctx.gd_q2_0_gemv_norm(C.byref(w2), dh, dy, ns.value, R, dwn, 1e-6, dho, dy2, None)
        hp = h + parts[:, :K2].sum(0, dtype=np.float32)
        assert np.allclose(ctx.get(dho, K2, np.float32), hp, rtol=1e-6, atol=1e-5)
        x2 = O.rmsnorm(hp[None], wn, 1e-6)[0]
        want2 = O.q2_0_matvec(b2, K2, R2, x2, threads=8)
        assert rel_diff(ctx.get(dy2, R2, np.float32), want2) < 1e-4
        for p in (dh, dwn, dho, dy2):
            ctx.free(p)
        free_w(ctx, w2)
    ctx.free(dx)
    ctx.free(dy)
    free_w(ctx, w)


def test_gemv_norm_rejects_alias_and_long_k(ctx):
    w = ga.Q2W()
    ctx.gd_q2w_alloc(256, 16, C.byref(w))
    dh, dy = ctx.alloc(256 * 4), ctx.alloc(16 * 4)
    with pytest.raises(RuntimeError, match="alias"):
        ctx.gd_q2_0_gemv_norm(C.byref(w), dh, None, 0, 0, dh, 1e-6, dh, dy, None)
    ctx.gd_q2w_free(C.byref(w))
    ctx.gd_q2w_alloc(15872, 16, C.byref(w))
    with pytest.raises(RuntimeError, match="15744"):
        ctx.gd_q2_0_gemv_norm(C.byref(w), dh, None, 0, 0, dh, 1e-6, None, dy, None)
    ctx.gd_q2w_free(C.byref(w))
    ctx.free(dh)
    ctx.free(dy)


def test_gemv_zero_and_single_weight(ctx):
    K, R = 1024, 8
    codes = np.ones(K * R, np.uint8)
    codes[3 * K + 999] = 3                     # +2d at row 3, k 999
    scales = np.full(K * R // 128, 0.03, np.float16).view(np.uint16)
    blocks = np.empty(K * R // 128 * 34, np.uint8)
    ga.load().gd_q2_0_pack(codes.ctypes.data, scales.ctypes.data, K * R, blocks.ctypes.data)
    w = upload_w(ctx, blocks, K, R)
    x = O.lcg_normal(K, 3)
    dx = ctx.put(x)
    dy = ctx.alloc(R * 4)
    ctx.gd_q2_0_gemv(C.byref(w), dx, ga.F32, dy)
    y = ctx.get(dy, R, np.float32)
    want = np.zeros(R, np.float32)
    want[3] = 2 * np.float32(np.float16(0.03)) * x[999]
    # sum(code*x) and sum(x) are formed in different orders, so the all-zero
    # rows carry f32 roundoff of the size of d * sum|x| * 2^-24.
    atol = 1e-6 * 0.03 * np.abs(x).sum()
    assert np.allclose(y, want, rtol=1e-5, atol=atol)
    free_w(ctx, w)


def _gemm(ctx, w, X, xt, yt, T, R):
    dX = ctx.put(X)
    dY = ctx.alloc(T * R * (4 if yt == ga.F32 else 2))
    ctx.gd_q2_0_gemm(C.byref(w), T, dX, xt, dY, yt)
    Y = ctx.get(dY, (T, R), np.float32 if yt == ga.F32 else np.float16)
    ctx.free(dX)
    ctx.free(dY)
    return Y.astype(np.float32)


@pytest.mark.parametrize("T,K,R", [(5, 1024, 300), (33, 5120, 200), (128, 2048, 256),
                                   (200, 17408, 96), (1, 128, 1)])
@pytest.mark.parametrize("xt,yt", [(ga.F16, ga.F32), (ga.F32, ga.F32), (ga.F16, ga.F16)])
def test_gemm_vs_oracle(ctx, T, K, R, xt, yt):
    blocks = O.lcg_q2_0(K, R, 3 * K + R)
    w = upload_w(ctx, blocks, K, R)
    Xh = O.lcg_normal_f16(T * K, 77).reshape(T, K)
    X = Xh.view(np.uint16) if xt == ga.F16 else Xh.astype(np.float32)
    Y = _gemm(ctx, w, X, xt, yt, T, R)
    Xr = Xh.astype(np.float32)                 # f16 staging, as both GEMMs stage X
    want = np.stack([O.q2_0_matvec(blocks, K, R, Xr[t], threads=8) for t in range(T)])
    assert rel_diff(Y, want) < (2e-3 if yt == ga.F16 else 1e-4)
    free_w(ctx, w)


# (mt, nt, waves per workgroup): every kernel the planner can pick.
PLANS_F16 = [(1, 1, 4), (2, 1, 4), (4, 1, 4), (2, 2, 4), (4, 2, 4), (8, 1, 4),
             (2, 1, 8), (4, 1, 8), (2, 2, 8), (4, 2, 8)]
PLANS_F32 = PLANS_F16                   # f32 X is rounded to f16 once, then any tile


@pytest.mark.parametrize("xt,yt,mt,nt,nw", [(ga.F16, yt, mt, nt, nw) for mt, nt, nw in PLANS_F16
                                            for yt in (ga.F32, ga.F16)] +
                         [(ga.F32, ga.F32, mt, nt, nw) for mt, nt, nw in PLANS_F32])
@pytest.mark.parametrize("split", [1, 3])
def test_gemm_every_plan(ctx, xt, yt, mt, nt, nw, split):
    """Every tile shape and a K split against the oracle, on a ragged shape:
    T and R are not multiples of any tile and K/64 = 42 slices do not divide
    evenly into 3 splits of an even slice count."""
    T, K, R = 200, 2688, 700
    blocks = O.lcg_q2_0(K, R, 11 * mt + nt)
    w = upload_w(ctx, blocks, K, R)
    Xh = O.lcg_normal_f16(T * K, 78).reshape(T, K)
    X = Xh.view(np.uint16) if xt == ga.F16 else Xh.astype(np.float32)
    dX = ctx.put(X)
    dY = ctx.alloc(T * R * (4 if yt == ga.F32 else 2))
    ctx.gd_q2_0_gemm_plan(C.byref(w), T, dX, xt, dY, yt, mt, nt, split, nw)
    Y = ctx.get(dY, (T, R), np.float32 if yt == ga.F32 else np.float16).astype(np.float32)
    want = np.stack([O.q2_0_matvec(blocks, K, R, Xh[t].astype(np.float32), threads=8)
                     for t in range(T)])
    assert rel_diff(Y, want) < (2e-3 if yt == ga.F16 else 1e-4)
    ctx.free(dX)
    ctx.free(dY)
    free_w(ctx, w)


@pytest.mark.parametrize("T,K,R,split,yt", [(200, 2688, 700, 1, ga.F32), (200, 2688, 1100, 3, ga.F16),
                                            (77, 384, 600, 2, ga.F32), (512, 5120, 8224, 4, ga.F32)])
def test_gemm_plan17_vs_oracle(ctx, T, K, R, split, yt):
    """The 4 x 2 x 8 tile with a seventeenth 32-row fragment (544 rows a
    workgroup: the waves share the extra fragment's MFMAs by token tile and
    K-step parity and add their halves at the end), against the oracle:
    ragged T and R (the last workgroup's rows past R are dropped), K splits,
    and the GDN in_proj shape the planner gives it (R = 8224, four splits), on
    sampled tokens there.  Every row of the extra fragments is also checked
    on its own."""
    blocks = O.lcg_q2_0(K, R, 7 * K + R)
    w = upload_w(ctx, blocks, K, R)
    Xh = O.lcg_normal_f16(T * K, 83).reshape(T, K)
    dX = ctx.put(Xh.view(np.uint16))
    dY = ctx.alloc(T * R * (4 if yt == ga.F32 else 2))
    ctx.gd_q2_0_gemm_plan17(C.byref(w), T, dX, ga.F16, dY, yt, split)
    Y = ctx.get(dY, (T, R), np.float32 if yt == ga.F32 else np.float16).astype(np.float32)
    toks = range(T) if T <= 200 else (0, 31, 127, 128, 300, 383, 384, T - 1)
    extra = np.concatenate([np.arange(c, min(c + 32, R)) for c in range(512, R, 544)])
    for t in toks:
        want = O.q2_0_matvec(blocks, K, R, Xh[t].astype(np.float32), threads=8)
        tol = 2e-3 if yt == ga.F16 else 1e-4
        assert rel_diff(Y[t], want) < tol, t
        if len(extra):
            assert rel_diff(Y[t, extra], want[extra]) < tol, t
    ctx.free(dX)
    ctx.free(dY)
    free_w(ctx, w)


@pytest.mark.parametrize("T,K,R,mt,nt,nw,split", [(512, 5120, 8224, 2, 1, 4, 8), (77, 2688, 700, 2, 1, 4, 3),
                                                   (200, 384, 100, 4, 1, 8, 2), (33, 1024, 544, 4, 2, 8, 5)])
def test_gemm_tail_vs_oracle(ctx, T, K, R, mt, nt, nw, split):
    """An unsplit tile over the whole row tiles, the rows past them (R is not a
    whole number of tiles) run as K-split partial units of the same launch, as
    the stack runs its GDN in_proj (R = 8224 on 128-row tiles, its 32 gate rows
    in 8 splits), against the oracle: Y below the tail, and the tail as the sum
    of its partials in split order; Y's tail rows are left as they were.  Also
    a tile wider than R (every row in the tail) and a 512-row tile."""
    blocks = O.lcg_q2_0(K, R, 5 * K + R)
    w = upload_w(ctx, blocks, K, R)
    Xh = O.lcg_normal_f16(T * K, 85).reshape(T, K)
    dX = ctx.put(Xh.view(np.uint16))
    dY = ctx.put(np.full((T, R), 7.0, np.float32))
    dP = ctx.alloc(split * T * R * 4)
    nz, r0 = C.c_int(), C.c_int()
    ctx.gd_q2_0_gemm_plan_tail(C.byref(w), T, dX, dY, mt, nt, nw, split, dP, C.byref(nz), C.byref(r0))
    rows = nw * nt * 32
    assert r0.value == R // rows * rows and 1 <= nz.value <= split
    r0 = r0.value
    Y = ctx.get(dY, (T, R), np.float32)
    P = ctx.get(dP, (nz.value, T, R - r0), np.float32)
    tail = P[0].copy()
    for z in range(1, nz.value):
        tail += P[z]
    toks = range(T) if T <= 200 else (0, 63, 64, 255, 256, 300, T - 1)
    for t in toks:
        want = O.q2_0_matvec(blocks, K, R, Xh[t].astype(np.float32), threads=8)
        if r0:
            assert rel_diff(Y[t, :r0], want[:r0]) < 1e-4, t
        assert rel_diff(tail[t], want[r0:]) < 1e-4, t
    assert np.all(Y[:, r0:] == 7.0)
    ctx.free(dX)
    ctx.free(dY)
    ctx.free(dP)
    free_w(ctx, w)


def silu(v):
    return v / (1.0 + np.exp(-v))


@pytest.mark.parametrize("T,K,ff", [(512, 5120, 17408), (512, 256, 17408), (37, 1024, 208),
                                    (1, 256, 16)])
def test_gemm_swiglu_vs_oracle(ctx, T, K, ff):
    """SwiGLU epilogue: f16(silu(X gate^T) * (X up^T)) against the oracle
    GEMV rows (ragged T and ff = 208, 13 groups of 16, exercise partial
    tiles).  At T=512, ff=17408 the columns run as two launches (16384
    columns of 256-column tiles, then 1024 of another tile, K-split at
    K=5120): every column is checked, on ten tokens around the token-tile
    boundaries when T is large."""
    R = 2 * ff
    blocks = O.lcg_q2_0(K, R, K + ff)
    w = upload_w(ctx, blocks, K, R)
    Xh = O.lcg_normal_f16(T * K, 79).reshape(T, K)
    dX, dO = ctx.put(Xh.view(np.uint16)), ctx.alloc(T * ff * 2)
    ctx.gd_q2_0_gemm_swiglu(C.byref(w), T, dX, dO)
    out = ctx.get(dO, (T, ff), np.float16).astype(np.float32)
    rows = np.arange(ff)
    blk = blocks.reshape(R, -1)
    g = np.ascontiguousarray(blk[rows]); u = np.ascontiguousarray(blk[rows + ff])
    toks = range(T) if T <= 64 else (0, 1, 63, 64, 127, 128, 200, 255, 256, T - 1)
    for t in toks:
        x = Xh[t].astype(np.float32)
        gv = O.q2_0_matvec(g, K, len(rows), x, threads=8)
        uv = O.q2_0_matvec(u, K, len(rows), x, threads=8)
        want = (silu(gv) * uv).astype(np.float16).astype(np.float32)
        assert rel_diff(out[t, rows], want) < 2e-3, t
        # The last 1024 columns on their own (the second launch at ff=17408),
        # so that an error there is not diluted by the rest of the row.
        tail = slice(max(0, ff - 1024), ff)
        assert rel_diff(out[t, tail], want[tail]) < 2e-3, t
    ctx.free(dX)
    ctx.free(dO)
    free_w(ctx, w)


@pytest.mark.parametrize("T,K,ff", [(512, 1024, 17408), (300, 1024, 17344), (77, 512, 4352),
                                    (130, 384, 560)])
@pytest.mark.parametrize("tile17", [1, 0])
def test_gemm_swiglu_tile17_vs_oracle(ctx, T, K, ff, tile17):
    """The 17-fragment tile (272 columns a workgroup: its eight waves share
    the seventeenth fragment's MFMAs by token tile and K-step parity and add
    their halves at the end) and the planner's other tiles, on the same
    inputs: every column against the oracle on tokens of each token tile,
    with ragged T, ff not a multiple of 272 (the last workgroup's fragments
    past ff are dropped) and a single partial workgroup (ff = 560)."""
    R = 2 * ff
    blocks = O.lcg_q2_0(K, R, 3 * K + ff)
    w = upload_w(ctx, blocks, K, R)
    Xh = O.lcg_normal_f16(T * K, 81).reshape(T, K)
    dX, dO = ctx.put(Xh.view(np.uint16)), ctx.alloc(T * ff * 2)
    ctx.gd_q2_0_gemm_swiglu_plan(C.byref(w), T, dX, dO, tile17)
    out = ctx.get(dO, (T, ff), np.float16).astype(np.float32)
    blk = blocks.reshape(R, -1)
    g = np.ascontiguousarray(blk[:ff]); u = np.ascontiguousarray(blk[ff:])
    toks = sorted({0, 31, 32, 127, 128, 200, 255, 256, 300 % T, T - 1} & set(range(T)))
    for t in toks:
        x = Xh[t].astype(np.float32)
        gv = O.q2_0_matvec(g, K, ff, x, threads=8)
        uv = O.q2_0_matvec(u, K, ff, x, threads=8)
        want = (silu(gv) * uv).astype(np.float16).astype(np.float32)
        assert rel_diff(out[t], want) < 2e-3, t
        # The seventeenth fragment of every workgroup on its own.
        extra = np.concatenate([np.arange(c, min(c + 16, ff)) for c in range(256, ff, 272)])
        if len(extra):
            assert rel_diff(out[t, extra], want[extra]) < 2e-3, t
    ctx.free(dX)
    ctx.free(dO)
    free_w(ctx, w)


@pytest.mark.parametrize("K,ff", [(5120, 17408), (1024, 208)])
def test_gemv_norm_swiglu_vs_oracle(ctx, K, ff):
    """The decode feed-forward input: fused add + norm, [gate; up] GEMV and
    SwiGLU in one launch, against the oracle."""
    R, eps = 2 * ff, 1e-6
    blocks = O.lcg_q2_0(K, R, 3 * K + ff)
    w = upload_w(ctx, blocks, K, R)
    h = O.lcg_normal(K, 98, 0.0, 2.0)
    d = O.lcg_normal(K, 99, 0.0, 1.0)
    wn = O.lcg_normal(K, 100, 1.0, 0.1)
    dh, dd, dwn, dho, dO = ctx.put(h), ctx.put(d), ctx.put(wn), ctx.alloc(K * 4), ctx.alloc(ff * 2)
    ctx.gd_q2_0_gemv_norm(C.byref(w), dh, dd, 1, 0, dwn, eps, dho, None, dO)
    out = ctx.get(dO, ff, np.float16).astype(np.float32)
    x = O.rmsnorm((h + d)[None], wn, eps)[0]
    y = O.q2_0_matvec(blocks, K, R, x, threads=8)
    want = (silu(y[:ff]) * y[ff:]).astype(np.float16).astype(np.float32)
    assert rel_diff(out, want) < 2e-3
    for p in (dh, dd, dwn, dho, dO):
        ctx.free(p)
    free_w(ctx, w)


def test_gemm_plan_rejects_unknown_tile(ctx):
    w = ga.Q2W()
    ctx.gd_q2w_alloc(256, 64, C.byref(w))
    dX = ctx.alloc(4 * 256 * 4)
    dY = ctx.alloc(4 * 64 * 4)
    for xt in (ga.F16, ga.F32):
        with pytest.raises(RuntimeError, match="no kernel"):
            ctx.gd_q2_0_gemm_plan(C.byref(w), 4, dX, xt, dY, ga.F32, 3, 1, 1, 4)
    for mt, nt, split, nw in ((4, 2, 0, 4), (8, 1, 1, 8), (1, 1, 1, 8), (4, 1, 1, 6)):
        with pytest.raises(RuntimeError, match="no kernel"):
            ctx.gd_q2_0_gemm_plan(C.byref(w), 4, dX, ga.F16, dY, ga.F32, mt, nt, split, nw)
    ctx.free(dX)
    ctx.free(dY)
    ctx.gd_q2w_free(C.byref(w))


def test_gemm_swiglu_rejects_4gib_code_span(ctx):
    """ff = 17408 with K = 985088: one wave's code resource (gate rows from its
    own on, then the up rows) would span 4 GiB of codes, past what its 32-bit
    byte range holds.  The matrix is real (8.6 GB of zero codes), so had the
    shape been taken, the launch would only have read zeros."""
    K, R = 985088, 2 * 17408
    w = ga.Q2W()
    ctx.gd_q2w_alloc(K, R, C.byref(w))
    dX = ctx.alloc(K * 2)
    dO = ctx.alloc(R // 2 * 2)
    try:
        with pytest.raises(RuntimeError, match="4 GiB"):
            ctx.gd_q2_0_gemm_swiglu(C.byref(w), 1, dX, dO)
    finally:
        ctx.free(dX)
        ctx.free(dO)
        ctx.gd_q2w_free(C.byref(w))


def test_gemm_full_size_sampled_rows(ctx):
    """BASELINE config 1 shapes at full size: every output row against the GPU
    GEMV of the same weights (independent kernel), and 48 sampled rows x all
    512 tokens against the oracle."""
    T = 512
    for K, R in ((5120, 17408), (17408, 5120)):
        w = ga.Q2W()
        ctx.gd_q2w_alloc(K, R, C.byref(w))
        ctx.gd_rand_q2w(C.byref(w), K + 1, 0.01, 0.05)
        dX = ctx.alloc(T * K * 2)
        ctx.gd_rand_normal(dX, ga.F16, T * K, 55, 0.0, 1.0)
        dY = ctx.alloc(T * R * 2)
        ctx.gd_q2_0_gemm(C.byref(w), T, dX, ga.F16, dY, ga.F16)
        Y = ctx.get(dY, (T, R), np.float16).astype(np.float32)
        X = ctx.get(dX, (T, K), np.float16)
        # GEMV on a few tokens (all rows)
        dy = ctx.alloc(R * 4)
        for t in (0, 1, 255, 511):
            ctx.gd_q2_0_gemv(C.byref(w), dX + t * K * 2, ga.F16, dy)
            assert rel_diff(Y[t], ctx.get(dy, R, np.float32)) < 2e-3, t
        # Oracle on sampled rows
        blocks = export_w(ctx, w).reshape(R, -1)
        rows = np.random.default_rng(K).choice(R, 48, replace=False)
        sub = np.ascontiguousarray(blocks[rows])
        Xr = X.astype(np.float32)
        want = np.stack([O.q2_0_matvec(sub, K, 48, Xr[t], threads=8) for t in range(T)])
        assert rel_diff(Y[:, rows], want) < 2e-3
        for p in (dX, dY, dy):
            ctx.free(p)
        free_w(ctx, w)


def test_invalid_shapes_are_errors(ctx):
    w = ga.Q2W()
    lib = ga.load()
    assert lib.gd_q2w_alloc(ctx.h, 100, 4, C.byref(w)) == ga.GD_EINVAL
    assert b"multiple of 128" in lib.gd_last_error(ctx.h)
    bad = ga.Q2W(None, None, 128, 1)
    assert lib.gd_q2_0_gemv(ctx.h, C.byref(bad), None, ga.F16, None) == ga.GD_EINVAL


def big_blocks(x, blocks_idx, lo, hi, seed):
    """x with the 128-element blocks `blocks_idx` rescaled so their max |x|
    lies in [lo, hi] (the GEMV stages such blocks with an extra power-of-two
    scale, since x * 16 would overflow f16)."""
    rng = np.random.default_rng(seed)
    x = x.copy()
    for b in blocks_idx:
        seg = x[b * 128:(b + 1) * 128]
        target = rng.uniform(lo, hi)
        x[b * 128:(b + 1) * 128] = seg / np.abs(seg).max() * target
    return x


@pytest.mark.parametrize("xt", [ga.F16, ga.F32])
@pytest.mark.parametrize("K,R,ksplit", [(5120, 777, 1), (17408, 5120, 3), (1024, 3072, 1)])
def test_gemv_large_x_blocks(ctx, xt, K, R, ksplit):
    """Blocks of x with max |x| in [3e3, 3e4] (SwiGLU outputs feeding
    ffn_down, or large norm weights, reach them): the per-block rescale path,
    in f16 and f32 x and in K-split partials, against the oracle at the plain
    GEMV's tolerance."""
    blocks = O.lcg_q2_0(K, R, K + 3 * R)
    w = upload_w(ctx, blocks, K, R)
    nb = K // 128
    big = sorted({0, 1, nb // 2, nb - 1, 5 % nb})
    x = big_blocks(O.lcg_normal(K, 17), big, 3e3, 3e4, K)
    if xt == ga.F16:
        xh = x.astype(np.float16)
        x_ref = xh.astype(np.float32)
        dx = ctx.put(xh.view(np.uint16))
    else:
        x_ref = x.astype(np.float32)
        dx = ctx.put(x_ref)
    dy = ctx.alloc(ksplit * R * 4)
    ns = C.c_int()
    ctx.gd_q2_0_gemv_split(C.byref(w), dx, xt, dy, ksplit, C.byref(ns))
    y = ctx.get(dy, (ns.value, R), np.float32).sum(0)
    want = O.q2_0_matvec(blocks, K, R, x_ref, threads=8)
    assert rel_diff(y, want) < 1e-4
    free_w(ctx, w)
    ctx.free(dx)
    ctx.free(dy)


@pytest.mark.parametrize("xt", [ga.F16, ga.F32])
@pytest.mark.parametrize("K,R", [(5120, 777), (17408, 130), (30720, 48)])
def test_gemv_sparse_outliers(ctx, xt, K, R):
    """Every 97th element of x 3000 times larger than the rest (outlier
    channels).  The fp4 body's matrix cores add products in groups of 8
    aligned to the largest, so small x beside an outlier lose low bits: the
    bound is 1e-3 here (measured about 1.7e-4), against the 1e-2 the
    GEMV contract allows."""
    blocks = O.lcg_q2_0(K, R, 3 * K + R)
    w = upload_w(ctx, blocks, K, R)
    x = O.lcg_normal(K, 23) * np.where(np.arange(K) % 97 == 0, 3000.0, 1.0).astype(np.float32)
    if xt == ga.F16:
        xh = x.astype(np.float16)
        x_ref = xh.astype(np.float32)
        dx = ctx.put(xh.view(np.uint16))
    else:
        x_ref = x.astype(np.float32)
        dx = ctx.put(x_ref)
    dy = ctx.alloc(R * 4)
    ctx.gd_q2_0_gemv(C.byref(w), dx, xt, dy)
    want = O.q2_0_matvec(blocks, K, R, x_ref, threads=8)
    assert rel_diff(ctx.get(dy, R, np.float32), want) < 1e-3
    free_w(ctx, w)
    ctx.free(dx)
    ctx.free(dy)


@pytest.mark.parametrize("xt,K,R", [(ga.F16, 32768, 100), (ga.F16, 65536, 40), (ga.F32, 32768, 100)])
def test_gemv_long_k(ctx, xt, K, R):
    """K past what the fp4 body stages in LDS (about 30K) runs the f16 body,
    with plain and sparse-outlier x, at the plain GEMV's tolerance; and as
    three K-split partials (each workgroup staging only its K range of x),
    whose sum holds the same bound."""
    blocks = O.lcg_q2_0(K, R, K + 11 * R)
    w = upload_w(ctx, blocks, K, R)
    for scale in (1.0, 3000.0):
        x = O.lcg_normal(K, 29) * np.where(np.arange(K) % 97 == 0, scale, 1.0).astype(np.float32)
        if xt == ga.F16:
            xh = x.astype(np.float16)
            x_ref = xh.astype(np.float32)
            dx = ctx.put(xh.view(np.uint16))
        else:
            x_ref = x.astype(np.float32)
            dx = ctx.put(x_ref)
        dy = ctx.alloc(R * 4)
        ctx.gd_q2_0_gemv(C.byref(w), dx, xt, dy)
        want = O.q2_0_matvec(blocks, K, R, x_ref, threads=8)
        assert rel_diff(ctx.get(dy, R, np.float32), want) < 1e-4
        dys, ns = ctx.alloc(3 * R * 4), C.c_int()
        ctx.gd_q2_0_gemv_split(C.byref(w), dx, xt, dys, 3, C.byref(ns))
        assert ns.value == 3
        parts = ctx.get(dys, 3 * R, np.float32).reshape(3, R)
        assert rel_diff(parts.sum(0), want) < 1e-4
        ctx.free(dx)
        ctx.free(dy)
        ctx.free(dys)
    free_w(ctx, w)


def test_gemv_norm_large_norm_weight(ctx):
    """Fused add + RMSNorm input whose norm weight is large on some blocks,
    so the staged x reaches |x| in the thousands there."""
    K, R, eps = 5120, 999, 1e-6
    blocks = O.lcg_q2_0(K, R, 4242)
    w = upload_w(ctx, blocks, K, R)
    h = O.lcg_normal(K, 3, 0.0, 2.0)
    wn = big_blocks(np.ones(K, np.float32) * 0.9, [2, 17, 39], 4e3, 1.5e4, 9).astype(np.float32)
    dh, dwn, dy = ctx.put(h), ctx.put(wn), ctx.alloc(R * 4)
    ctx.gd_q2_0_gemv_norm(C.byref(w), dh, None, 0, 0, dwn, eps, None, dy, None)
    x = O.rmsnorm(h[None], wn, eps)[0]
    assert np.abs(x).max() > 2048
    want = O.q2_0_matvec(blocks, K, R, x, threads=8)
    assert rel_diff(ctx.get(dy, R, np.float32), want) < 1e-4
    for p in (dh, dwn, dy):
        ctx.free(p)
    free_w(ctx, w)


def test_graph_replays_recorded_calls(ctx):
    """gd_graph_begin/end record GEMVs on three distinct matrices and a cast;
    each replay, with eager work and synchronizations in between, gives the
    eager results again."""
    K, R = 1024, 3072
    mats = [O.lcg_q2_0(K, R, 300 + i) for i in range(3)]
    ws = [upload_w(ctx, b, K, R) for b in mats]
    xh = O.lcg_normal_f16(K, 8)
    dx = ctx.put(xh.view(np.uint16))
    dys = [ctx.alloc(R * 4) for _ in ws]
    d16 = ctx.alloc(R * 2)

    def record():
        for w, dy in zip(ws, dys):
            ctx.gd_q2_0_gemv(C.byref(w), dx, ga.F16, dy)
        ctx.gd_cast(dys[0], ga.F32, d16, ga.F16, R)

    record()
    eager = [ctx.get(dy, R, np.float32) for dy in dys]
    eager16 = ctx.get(d16, R, np.uint16)
    for i, b in enumerate(mats):
        assert rel_diff(eager[i], O.q2_0_matvec(b, K, R, xh.astype(np.float32), 8)) < 1e-4
    ctx.check(ctx.lib.gd_graph_begin(ctx.h))
    record()
    g = C.c_void_p()
    ctx.check(ctx.lib.gd_graph_end(ctx.h, C.byref(g)))
    try:
        for rep in range(3):
            for dy in dys:
                ctx.gd_fill_u32(dy, 0x7fc00000, R)        # NaN, so a skipped write shows
            ctx.gd_fill_u32(d16, 0, R // 2)
            ctx.sync()
            ctx.check(ctx.lib.gd_graph_launch(ctx.h, g))
            ctx.sync()
            for i, dy in enumerate(dys):
                assert np.array_equal(ctx.get(dy, R, np.float32), eager[i]), (rep, i)
            assert np.array_equal(ctx.get(d16, R, np.uint16), eager16), rep
    finally:
        ctx.lib.gd_graph_destroy(g)
    for p in dys + [dx, d16]:
        ctx.free(p)
    for w in ws:
        free_w(ctx, w)
