"""Pins for the CPU oracle (oracle/gd_oracle.c) before it is trusted as the
checker: the reference's own known-answer vectors, closed forms and
invariants of the recurrence, and f64 brute force.  CPU only."""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle as O
from conftest import rel_diff

GOLD = Path(__file__).resolve().parent / "golden"


# ---------------------------------------------------------------- LCG inputs

def test_lcg_stream_matches_definition():
    # The LCG of MetalSelfTest.swift:12-21 with Python integers (u64
    # wraparound); its 31 output bits scaled by 2^-31 into [0, 1).
    seed, n = 7, 1000
    s = (seed + 0x9E3779B97F4A7C15) % 2**64
    want = []
    for _ in range(n):
        s = (s * 6364136223846793005 + 1442695040888963407) % 2**64
        u = np.float32(np.float32(s >> 33) * np.float32(2.0 ** -31))
        want.append(np.float32(-1) + np.float32(2) * u)
    got = O.lcg_uniform(n, seed)
    assert np.array_equal(got, np.array(want, np.float32))
    assert got.min() >= -1 and got.max() < 1
    big = O.lcg_uniform(100_000, seed, 0.0, 1.0)
    assert abs(big.mean() - 0.5) < 0.01 and big.max() > 0.99


def test_lcg_normal_moments():
    z = O.lcg_normal(200_000, 3)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01


def test_lcg_q2_0_ternary_and_scales():
    K, R = 1024, 64
    blocks = O.lcg_q2_0(K, R, 11)
    codes = np.empty(K * R, np.uint8)
    scales = np.empty(K * R // 128, np.uint16)
    import gadeon_amd as ga
    lib = ga.load()
    assert lib.gd_q2_0_unpack(blocks.ctypes.data, K * R, codes.ctypes.data, scales.ctypes.data) == 0
    counts = np.bincount(codes, minlength=4)
    assert counts[3] == 0                         # code 11 never drawn
    assert np.all(np.abs(counts[:3] / codes.size - 1 / 3) < 0.01)
    d = scales.view(np.float16).astype(np.float32)
    assert d.min() >= 0.0099 and d.max() <= 0.0501


# ------------------------------------------------------------------ f16 RNE

def test_f16_round_trip_and_rne():
    for h in range(0, 0x10000, 7):
        if (h & 0x7c00) == 0x7c00:
            continue
        assert O.lib().or_f2h(O.lib().or_h2f(h)) == h
    x = np.random.default_rng(0).standard_normal(20000).astype(np.float32) * 100
    x = np.concatenate([x, np.float32([65504, 65519.9, 65520, 1e-8, 3e-8, 6e-5, -0.0])])
    want = x.astype(np.float16).view(np.uint16)
    got = np.array([O.lib().or_f2h(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, want)


# --------------------------------------------------------------------- Q2_0

def _blocks_from(codes, scales):
    import gadeon_amd as ga
    n = codes.size
    out = np.empty(n // 128 * 34, np.uint8)
    assert ga.load().gd_q2_0_pack(codes.ctypes.data, scales.ctypes.data, n, out.ctypes.data) == 0
    return out


def test_dequant_is_exact():
    blocks = O.lcg_q2_0(512, 8, 5)
    got = O.q2_0_dequant(blocks, 512 * 8)
    b = blocks.reshape(-1, 34)
    d = b[:, :2].copy().view(np.float16).astype(np.float64).ravel()
    codes = np.stack([(b[:, 2:] >> (2 * j)) & 3 for j in range(4)], -1).reshape(-1, 128)
    want = (codes.astype(np.float64) - 1) * d[:, None]
    assert np.array_equal(got.astype(np.float64), want.ravel())


def test_matvec_special_cases():
    K, M = 256, 4
    codes = np.ones(K * M, np.uint8)                  # every weight 0
    scales = np.full(K * M // 128, 0.03, np.float16).view(np.uint16)
    x = O.lcg_normal(K, 1)
    assert np.all(O.q2_0_matvec(_blocks_from(codes, scales), K, M, x) == 0)
    for code, mult in ((0, -1.0), (2, 1.0), (3, 2.0)):
        c = np.ones(K * M, np.uint8)
        c[1 * K + 77] = code                          # one weight in row 1
        y = O.q2_0_matvec(_blocks_from(c, scales), K, M, x)
        want = np.zeros(M, np.float32)
        want[1] = np.float32(mult) * np.float32(np.float16(0.03)) * x[77]
        assert np.allclose(y, want, rtol=1e-6, atol=1e-7)


def test_matvec_f32_vs_f64_bruteforce():
    K, M = 5120, 96
    blocks = O.lcg_q2_0(K, M, 21)
    x = O.lcg_normal(K, 22)
    got = O.q2_0_matvec(blocks, K, M, x, threads=4)
    want = O.q2_0_matvec_f64(blocks, K, M, x.astype(np.float64))
    assert rel_diff(got, want) < 1e-5
    # The threaded split does not change any row's arithmetic.
    assert np.array_equal(got, O.q2_0_matvec(blocks, K, M, x, threads=1))


def test_matvec_linearity():
    K, M = 1024, 64
    blocks = O.lcg_q2_0(K, M, 31)
    x1, x2 = O.lcg_normal(K, 32), O.lcg_normal(K, 33)
    y = O.q2_0_matvec(blocks, K, M, x1 + x2)
    assert rel_diff(y, O.q2_0_matvec(blocks, K, M, x1) + O.q2_0_matvec(blocks, K, M, x2)) < 1e-5


# -------------------------------------------------------------- closed form

def test_mtp_rollback_known_answers():
    data = json.loads((GOLD / "mtp_rollback_kats.json").read_text())
    for c in data["cases"]:
        got = O.mtp_state_after(c["m"], c["H"], c["DK"], c["DV"], c["C"], c["s0"], c["delta"],
                                c["k"], c["gcum"])
        assert np.allclose(got, c["want"], atol=data["tolerance_abs"], rtol=0), c["name"]


def _gdn_inputs(T, nV, nK, dS, seed, S_scale=0.0):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((T, nK, dS))
    k = rng.standard_normal((T, nK, dS))
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((T, nV, dS))
    beta = 1 / (1 + np.exp(-rng.standard_normal((T, nV))))
    g = -np.log1p(np.exp(rng.standard_normal((T, nV))))
    S = rng.standard_normal((nV, dS, dS)) * S_scale
    return q, k, v, g, beta, S


def test_scan_delta_rule_invariants():
    """beta=1, |k|=1: after the step S^T k = v for any decay (pins decay BEFORE
    S^T k and the sign of the delta); with q = k the readout is qScale*v
    (pins readout AFTER the update).  beta=0: pure decay."""
    nV = nK = 2
    dS = 16
    q, k, v, g, beta, S = _gdn_inputs(1, nV, nK, dS, 4, S_scale=0.5)
    S64 = S.copy()
    o = O.gdn_scan_f64(k[0].ravel(), k[0].ravel(), v[0].ravel(), g[0], np.ones(nV), S64,
                       nV, nK, dS, 0.25)
    for h in range(nV):
        assert np.allclose(S64[h].T @ k[0, h], v[0, h], atol=1e-12)
        assert np.allclose(o.reshape(nV, dS)[h], 0.25 * v[0, h], atol=1e-12)
    S32 = S.astype(np.float32)
    o32 = O.gdn_scan(k[0].astype(np.float32).ravel(), k[0].astype(np.float32).ravel(),
                     v[0].astype(np.float32).ravel(), g[0].astype(np.float32),
                     np.ones(nV, np.float32), S32, nV, nK, dS, 0.25)
    for h in range(nV):
        assert np.allclose(S32[h].T @ k[0, h], v[0, h], atol=1e-4)
    S0 = S.copy()
    O.gdn_scan_f64(q[0].ravel(), k[0].ravel(), v[0].ravel(), g[0], np.zeros(nV), S0, nV, nK,
                   dS, 0.25)
    assert np.allclose(S0, np.exp(g[0])[:, None, None] * S, atol=1e-14)


def test_scan_f32_order_vs_f64():
    T, nV, nK, dS = 40, 4, 2, 32
    q, k, v, g, beta, S = _gdn_inputs(T, nV, nK, dS, 5, S_scale=0.02)
    S64, S32 = S.copy(), S.astype(np.float32)
    o64 = O.gdn_sequential(q, k, v, g, beta, S64, 0.125, f64=True)
    o32 = O.gdn_sequential(q, k, v, g, beta, S32, 0.125, f64=False)
    assert rel_diff(o32, o64) < 1e-5 and rel_diff(S32, S64) < 1e-5


def test_sequential_state_is_closed_form():
    """Run the token-serial scan, recover each token's rank-1 update delta_t
    from consecutive states, and check the MtpRollback closed form rebuilds
    every intermediate state (MtpRollback.swift:3-12)."""
    T, dS = 9, 8
    q, k, v, g, beta, S = _gdn_inputs(T, 1, 1, dS, 6, S_scale=0.3)
    S0 = S.copy()
    states, deltas = [], []
    Sc = S.copy()
    for t in range(T):
        prev = Sc.copy()
        O.gdn_scan_f64(q[t].ravel(), k[t].ravel(), v[t].ravel(), g[t], beta[t], Sc, 1, 1, dS, 1.0)
        dU = Sc[0] - np.exp(g[t, 0]) * prev[0]                 # = k_t delta_t^T
        deltas.append(k[t, 0] @ dU)                             # |k_t| = 1
        assert np.allclose(np.outer(k[t, 0], deltas[-1]), dU, atol=1e-12)
        states.append(Sc[0].copy())
    gcum = np.cumsum(g[:, 0])
    for m in range(1, T + 1):
        got = O.mtp_state_after(m, 1, dS, dS, T, S0[0].ravel(), np.array(deltas).ravel(),
                                k[:, 0].ravel(), gcum)
        assert np.allclose(got, states[m - 1].ravel(), atol=2e-5), m


@pytest.mark.parametrize("T,C,nV,nK", [(64, 64, 2, 2), (100, 32, 2, 1), (37, 16, 3, 3),
                                       (130, 64, 4, 2)])
def test_chunked_equals_sequential(T, C, nV, nK):
    dS = 32
    q, k, v, g, beta, S = _gdn_inputs(T, nV, nK, dS, 7 + T, S_scale=0.05)
    Sseq, Sch = S.copy(), S.copy()
    oseq = O.gdn_sequential(q, k, v, g, beta, Sseq, 0.17, f64=True)
    och = O.gdn_chunked_f64(q, k, v, g, beta, Sch, T, nV, nK, dS, dS, 0.17, C)
    assert rel_diff(och, oseq) < 1e-10 and rel_diff(Sch, Sseq) < 1e-10


def test_gate_and_softplus():
    x = np.linspace(-30, 30, 601).astype(np.float32)
    sp = np.array([O.lib().or_softplus(float(t)) for t in x], np.float32)
    assert np.allclose(sp, np.logaddexp(0, x.astype(np.float64)), rtol=1e-6, atol=1e-7)
    beta, g = O.gdn_gate(x[:8], x[8:16], np.zeros(4), -np.ones(4), 4)
    assert np.all(g <= 0) and np.all((beta > 0) & (beta < 1))


def test_conv_is_causal_fir():
    convDim, kc, N = 5, 4, 9
    rng = np.random.default_rng(8)
    x = rng.standard_normal((N, convDim)).astype(np.float32)
    cw = rng.standard_normal((convDim, kc)).astype(np.float32)
    ring = np.zeros((kc - 1) * convDim, np.float32)
    out = O.gdn_conv(x, ring, cw, convDim, kc)
    xp = np.concatenate([np.zeros((kc - 1, convDim)), x.astype(np.float64)])
    pre = np.stack([sum(xp[n + j] * cw[:, j] for j in range(kc)) for n in range(N)])
    assert np.allclose(out, pre / (1 + np.exp(-pre)), atol=1e-5)
    assert np.array_equal(ring.reshape(kc - 1, convDim), x[-(kc - 1):])


@pytest.mark.parametrize("d,scale", [(128, 1.0), (128, 1e-4), (64, 30.0)])
def test_l2norm_rows_pins(d, scale):
    """Kern.l2normRows (Kernels.swift:41-52): x / sqrt(sum(x^2) + eps), with
    the SUM of squares (not the mean, Kernels.swift:39-40) and eps inside the
    root.  Rows of scale 1e-4 have sum(x^2) ~ d*1e-8, comparable to eps, so
    eps placement shows; any row's result times its own norm gives x back."""
    eps = 1e-6
    rng = np.random.default_rng(d)
    x = (rng.standard_normal((5, d)) * scale).astype(np.float32)
    y = O.l2norm_rows(x.ravel(), d, eps).reshape(5, d)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 ** 2).sum(1, keepdims=True) + eps)
    assert np.allclose(y, want, rtol=2e-6, atol=1e-9)
    # a mean-based norm would differ by sqrt(d); without eps, by the eps term
    mean_based = x64 / np.sqrt((x64 ** 2).mean(1, keepdims=True) + eps)
    assert not np.allclose(y, mean_based, rtol=1e-2)
    if scale == 1.0:
        assert np.allclose((y.astype(np.float64) ** 2).sum(1), 1.0, atol=1e-5)
    if scale == 1e-4:
        no_eps = x64 / np.sqrt((x64 ** 2).sum(1, keepdims=True))
        assert not np.allclose(y, no_eps, rtol=1e-3)


def test_gate_per_head_indexing():
    """GDN.swift:39-42 over several tokens: element i belongs to value head
    h = i % nV and takes dt[h] and aNeg[h]; beta = sigmoid(b),
    g = softplus(a + dt[h]) * aNeg[h], against logaddexp in f64."""
    nV, T = 5, 7
    rng = np.random.default_rng(17)
    b = rng.normal(0, 2, T * nV).astype(np.float32)
    a = rng.normal(0, 2, T * nV).astype(np.float32)
    dt = np.linspace(-1.5, 2.0, nV).astype(np.float32)            # distinct per head
    aNeg = -np.exp(np.linspace(-1.0, 1.0, nV)).astype(np.float32)
    beta, g = O.gdn_gate(b, a, dt, aNeg, nV)
    h = np.arange(T * nV) % nV
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    want_b = 1.0 / (1.0 + np.exp(-b64))
    want_g = np.logaddexp(0.0, a64 + dt[h].astype(np.float64)) * aNeg[h].astype(np.float64)
    assert np.allclose(beta, want_b, rtol=1e-6, atol=1e-7)
    assert np.allclose(g, want_g, rtol=2e-6, atol=1e-7)
    # a transposed head map (i // T) would not pass
    h2 = np.arange(T * nV) // T
    wrong = np.logaddexp(0.0, a64 + dt[h2].astype(np.float64)) * aNeg[h2].astype(np.float64)
    assert not np.allclose(g, wrong, rtol=1e-3)
