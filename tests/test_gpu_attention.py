"""The attention entries of the C ABI (gd_split_q_gate, gd_rope, gd_kv_append,
gd_attn_paged, gd_attn_batch; MetalEnc.swift:656-706, 780-847, 966-1025)
against an f64 restatement of Attn.step's attention (Attention.swift:79-134):
q and k RMS-normalized and rotated by the oracle's Kern.ropeNeox, K and V
rounded to f16 as the cache holds them, softmax((q . k) / sqrt(hd)) . v, times
sigmoid(gate).  Head dims 128 and 256 with the GQA groups of BASELINE config 4
(40 / 8) and of the reference's 27B (24 / 4), over ragged page sizes.  Norm-wise
relative error < 2e-3 (the f16 cache and the hi/lo f16 MFMA operands are the
error sources); rope and the q|gate split against the oracle / exactly; the
cache append bit-exact (RNE f16).  Prompts up to 600 keys (many query
blocks, dispatched longest first): rows of every query block are checked, and
a second launch of the same call is bit-identical."""
import ctypes as C

import numpy as np
import pytest

import gadeon_amd as ga
import oracle as O
from conftest import rel_diff

pytestmark = pytest.mark.gpu
TOL = 2e-3


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def make_cache(ctx, T, kv_dim, page, seed):
    """A pool of pages in shuffled order (the table maps positions to pages)."""
    npages = (T + page - 1) // page + 2
    rng = np.random.default_rng(seed)
    table = rng.permutation(npages).astype(np.int32)
    kc = ctx.alloc(npages * page * kv_dim * 2)
    vc = ctx.alloc(npages * page * kv_dim * 2)
    ctx.gd_fill_u32(kc, 0x7e007e00, npages * page * kv_dim // 2)     # f16 NaN: unread
    ctx.gd_fill_u32(vc, 0x7e007e00, npages * page * kv_dim // 2)
    return kc, vc, ctx.put(table), table, npages


def ref_attention(q, K, V, gate, nkv, t_end):
    """q [nh][hd] at the keys 0 .. t_end-1 of K, V [T][nkv][hd] (f64)."""
    nh, hd = q.shape
    grp = nh // nkv
    out = np.empty((nh, hd))
    for h in range(nh):
        k = K[:t_end, h // grp].astype(np.float64)
        v = V[:t_end, h // grp].astype(np.float64)
        s = k @ q[h].astype(np.float64) / np.sqrt(hd)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ v * sigmoid(gate[h].astype(np.float64))
    return out


@pytest.mark.parametrize("hd,nh,nkv,page,T", [(128, 40, 8, 16, 77), (256, 24, 4, 16, 130),
                                              (256, 24, 4, 7, 45), (128, 4, 2, 5, 300),
                                              (128, 40, 8, 16, 600), (256, 24, 4, 16, 520)])
def test_decode_and_batch_attention(ctx, hd, nh, nkv, page, T):
    rng = np.random.default_rng(hd + T)
    kv_dim = hd * nkv
    n_rot, base, eps = 64, 1e7, 1e-6
    # Projections as the engine makes them: per head q | gate, then norms, rope.
    qfull = rng.standard_normal((T, nh, 2 * hd)).astype(np.float32)
    k = rng.standard_normal((T, nkv, hd)).astype(np.float32)
    v = rng.standard_normal((T, nkv, hd)).astype(np.float32)
    qn = rng.uniform(0.8, 1.2, hd).astype(np.float32)
    kn = rng.uniform(0.8, 1.2, hd).astype(np.float32)
    # device: split, norm, rope, append
    dqf = ctx.put(qfull)
    dq, dg = ctx.alloc(T * nh * hd * 4), ctx.alloc(T * nh * hd * 4)
    ctx.gd_split_q_gate(dqf, dq, dg, hd, nh, T)
    q_dev = ctx.get(dq, (T, nh, hd), np.float32)
    assert np.array_equal(q_dev, qfull[:, :, :hd]) and \
        np.array_equal(ctx.get(dg, (T, nh, hd), np.float32), qfull[:, :, hd:])
    dqn, dkn = ctx.put(qn), ctx.put(kn)
    dk, dv = ctx.put(k), ctx.put(v)
    ctx.gd_rmsnorm_rows(dq, hd, T * nh, dqn, eps)
    ctx.gd_rmsnorm_rows(dk, hd, T * nkv, dkn, eps)
    ctx.gd_rope(dq, hd, nh, n_rot, base, 0, T)
    ctx.gd_rope(dk, hd, nkv, n_rot, base, 0, T)
    # oracle: the same preparation per token (Attention.swift:94-107)
    q_ref = np.stack([O.rope_neox(O.rmsnorm_rows(qfull[t, :, :hd].ravel(), hd, qn, eps), hd, n_rot,
                                  base, t) for t in range(T)]).reshape(T, nh, hd)
    k_ref = np.stack([O.rope_neox(O.rmsnorm_rows(k[t].ravel(), hd, kn, eps), hd, n_rot, base, t)
                      for t in range(T)]).reshape(T, nkv, hd)
    # The rotation angle pos * theta carries f32 rounding that grows with the
    # position (about 600 * 2^-24 rad at T = 600): the bound follows it.
    rtol = 1e-5 if T <= 300 else 1e-4
    assert rel_diff(ctx.get(dq, (T, nh, hd), np.float32), q_ref) < rtol
    assert rel_diff(ctx.get(dk, (T, nkv, hd), np.float32), k_ref) < rtol
    kc, vc, dtab, table, npages = make_cache(ctx, T, kv_dim, page, hd)
    # append in two calls (a prefix, then the rest)
    cut = T // 3
    ctx.gd_kv_append(dk, dv, kc, vc, dtab, kv_dim, 0, page, cut)
    ctx.gd_kv_append(dk + cut * kv_dim * 4, dv + cut * kv_dim * 4, kc, vc, dtab, kv_dim, cut, page,
                     T - cut)
    kpool = ctx.get(kc, (npages, page, kv_dim), np.float16)
    vpool = ctx.get(vc, (npages, page, kv_dim), np.float16)
    pos = np.arange(T)
    K16 = kpool[table[pos // page], pos % page].reshape(T, nkv, hd)
    V16 = vpool[table[pos // page], pos % page].reshape(T, nkv, hd)
    k_dev = ctx.get(dk, (T, nkv, hd), np.float32)
    assert np.array_equal(K16, k_dev.astype(np.float16))
    assert np.array_equal(V16, v.astype(np.float16))
    gate = qfull[:, :, hd:]
    # batch (prefill) attention of every token, in two chunks
    dout = ctx.alloc(T * nh * hd * 4)
    scale = 1 / np.sqrt(hd)
    for lo, hi in ((0, cut), (cut, T)):
        ctx.gd_attn_batch(dq + lo * nh * hd * 4, kc, vc, dtab, dg + lo * nh * hd * 4,
                          dout + lo * nh * hd * 4, hd, nh, nkv, kv_dim, page, C.c_float(scale), lo,
                          hi - lo, 1, 0)
    got = ctx.get(dout, (T, nh, hd), np.float32)
    q_used = ctx.get(dq, (T, nh, hd), np.float32)
    for t in sorted({0, 1, cut - 1, cut, T // 2, T - 1, *range(5, T, 61)}):
        want = ref_attention(q_used[t], K16, V16, gate[t], nkv, t + 1)
        assert rel_diff(got[t], want) < TOL, t
    # The same launch again: bit-identical.
    ctx.gd_attn_batch(dq + cut * nh * hd * 4, kc, vc, dtab, dg + cut * nh * hd * 4,
                      dout + cut * nh * hd * 4, hd, nh, nkv, kv_dim, page, C.c_float(scale), cut,
                      T - cut, 1, 0)
    assert np.array_equal(ctx.get(dout, (T, nh, hd), np.float32), got)
    # decode attention of the last token over all T cached keys, gated and not
    part = ctx.alloc(nh * 16 * (hd + 2) * 4)
    dq1 = dq + (T - 1) * nh * hd * 4
    dg1 = dg + (T - 1) * nh * hd * 4
    do1 = ctx.alloc(nh * hd * 4)
    for gated in (1, 0):
        ctx.gd_attn_paged(dq1, kc, vc, dtab, dg1 if gated else None, do1, part, hd, nh, nkv, T,
                          kv_dim, page, C.c_float(scale), gated, 0)
        g1 = gate[T - 1] if gated else np.full((nh, hd), 1e9, np.float32)
        want = ref_attention(q_used[T - 1], K16, V16, g1, nkv, T)
        r = rel_diff(ctx.get(do1, (nh, hd), np.float32), want)
        assert r < TOL, (gated, r)
    # and it equals the batch path's last row
    ctx.gd_attn_paged(dq1, kc, vc, dtab, dg1, do1, part, hd, nh, nkv, T, kv_dim, page,
                      C.c_float(scale), 1, 0)
    assert rel_diff(ctx.get(do1, (nh, hd), np.float32), got[T - 1]) < TOL
    for p in (dqf, dq, dg, dqn, dkn, dk, dv, kc, vc, dtab, dout, part, do1):
        ctx.free(p)


def test_attention_rejects_bad_shapes(ctx):
    d = ctx.alloc(64)
    lib = ctx.lib
    assert lib.gd_attn_paged(ctx.h, d, d, d, d, d, d, d, 64, 4, 2, 8, 128, 16, C.c_float(0.1), 1,
                             0) == ga.GD_EINVAL
    assert b"head_dim" in lib.gd_last_error(ctx.h)
    assert lib.gd_attn_paged(ctx.h, d, d, d, d, d, d, d, 128, 5, 2, 8, 256, 16, C.c_float(0.1), 1,
                             0) == ga.GD_EINVAL
    assert lib.gd_attn_batch(ctx.h, d, d, d, d, d, d, 128, 4, 2, 256, 16, C.c_float(0.1), 0, 4, 1,
                             8) == ga.GD_EINVAL
    assert b"window" in lib.gd_last_error(ctx.h)
    assert lib.gd_rope(ctx.h, d, 128, 2, 130, C.c_float(1e4), 0, 1) == ga.GD_EINVAL
    ctx.free(d)
