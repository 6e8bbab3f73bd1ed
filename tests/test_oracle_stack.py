"""CPU pins of the pieces of the stack restatement (oracle/gd_oracle_stack.c)
that the Q2_0 and GDN tests do not cover: softmax, partial NEOX RoPE and
RMSNorm (Kernels.swift:15-84) by invariants and known answers, and the wiring
of BonsaiEngine.forward / Attn.step (BonsaiEngine.swift:155-178,
Attention.swift:72-139) by identities whose right-hand side is built from the
already-pinned mat-vec and norms."""
import numpy as np
import pytest

import oracle as O


def test_softmax_invariants():
    rng = np.random.default_rng(1)
    x = rng.normal(0, 3, 257).astype(np.float32)
    p = O.softmax(x)
    assert abs(p.sum() - 1) < 1e-6 and (p > 0).all()
    # shift invariance and exact ratios e^(xi - xj)
    assert np.allclose(O.softmax(x + 40.0), p, rtol=1e-5, atol=1e-9)
    i, j = int(np.argmax(x)), int(np.argmin(x))
    assert np.isclose(p[j] / p[i], np.exp(np.float64(x[j] - x[i])), rtol=1e-5)
    # large logits must not overflow (max-subtracted)
    big = np.array([1000.0, 999.0, -1000.0], np.float32)
    q = O.softmax(big)
    assert np.isfinite(q).all() and np.isclose(q[0] / q[1], np.e, rtol=1e-5)
    assert np.allclose(O.softmax(np.zeros(5, np.float32)), 0.2)


@pytest.mark.parametrize("hd,n_rot", [(128, 64), (256, 64), (128, 128)])
def test_rope_neox_invariants(hd, n_rot):
    rng = np.random.default_rng(hd + n_rot)
    nh, base, half = 3, 1e7, n_rot // 2
    x = rng.normal(size=nh * hd).astype(np.float32)
    # position 0 is the identity
    assert np.array_equal(O.rope_neox(x, hd, n_rot, base, 0), x)
    y = O.rope_neox(x, hd, n_rot, base, 1234)
    xs, ys = x.reshape(nh, hd), y.reshape(nh, hd)
    # dimensions past n_rot are untouched
    assert np.array_equal(ys[:, n_rot:], xs[:, n_rot:])
    # NEOX pairing: element i rotates with element i + n_rot/2 (norm of each pair kept)
    pn = lambda a: np.hypot(a[:, :half], a[:, half:n_rot])
    assert np.allclose(pn(ys), pn(xs), rtol=2e-5)
    e = np.zeros(hd, np.float32)
    e[3] = 1.0
    r = O.rope_neox(e, hd, n_rot, base, 7)
    nz = set(np.nonzero(np.abs(r) > 1e-7)[0])
    assert nz <= {3, 3 + half}
    # pair 0 turns by exactly `pos` radians (frequency base^0 = 1)
    e0 = np.zeros(hd, np.float32)
    e0[0] = 1.0
    r0 = O.rope_neox(e0, hd, n_rot, base, 5)
    assert np.isclose(r0[0], np.cos(5.0), atol=1e-6) and np.isclose(r0[half], np.sin(5.0), atol=1e-6)
    # last pair's frequency is base^(-(n_rot-2)/n_rot)
    el = np.zeros(hd, np.float32)
    el[half - 1] = 1.0
    rl = O.rope_neox(el, hd, n_rot, base, 1000)
    ang = 1000.0 * base ** (-(n_rot - 2) / n_rot)
    assert np.isclose(rl[half - 1], np.cos(ang), atol=2e-5)
    assert np.isclose(rl[n_rot - 1], np.sin(ang), atol=2e-5)
    # relative-position property: <R_m q, R_n k> depends only on m - n
    q = rng.normal(size=hd).astype(np.float32)
    k = rng.normal(size=hd).astype(np.float32)
    d1 = float(np.dot(O.rope_neox(q, hd, n_rot, base, 10), O.rope_neox(k, hd, n_rot, base, 3)))
    d2 = float(np.dot(O.rope_neox(q, hd, n_rot, base, 107), O.rope_neox(k, hd, n_rot, base, 100)))
    assert abs(d1 - d2) < 1e-3 * max(1.0, abs(d1))


def test_rmsnorm_invariants():
    rng = np.random.default_rng(3)
    x = rng.normal(0, 5, 5120).astype(np.float32)
    w = np.ones(5120, np.float32)
    y = O.rmsnorm(x, w, 0.0)
    assert abs(np.sqrt(np.mean(y.astype(np.float64) ** 2)) - 1) < 1e-5     # unit RMS
    assert np.allclose(O.rmsnorm(7.5 * x, w, 0.0), y, rtol=1e-5, atol=1e-6)  # scale invariant
    w2 = rng.uniform(0.5, 1.5, 5120).astype(np.float32)
    assert np.allclose(O.rmsnorm(x, w2, 0.0), y * w2, rtol=1e-5, atol=1e-6)  # weight is w, not 1+w
    rows = O.rmsnorm_rows(np.tile(x[:128], 4), 128, w[:128], 1e-6)
    assert np.allclose(rows.reshape(4, 128), O.rmsnorm(x[:128], w[:128], 1e-6), rtol=1e-6)


# ---- stack wiring -------------------------------------------------------------

CFG = dict(n_layer=1, n_embd=256, n_ff=256, n_head=4, n_head_kv=2, head_dim=128, n_rot=64,
           rope_base=1e7, eps=1e-6, n_vocab=64, attn_interval=1, d_state=128, n_k_head=2,
           n_v_head=2, d_conv=4, max_ctx=8)


def q2_blocks(K, R, seed, zero=False):
    b = O.lcg_q2_0(K, R, seed)
    if zero:                                  # every code 01 -> weight 0 (Quant.swift:4-7)
        b = b.reshape(-1, 34).copy()
        b[:, 2:] = 0x55
        b = b.reshape(-1)
    return b


def make_tensors(cfg, zero=()):
    E, FF, hd, nh, nkv = cfg["n_embd"], cfg["n_ff"], cfg["head_dim"], cfg["n_head"], cfg["n_head_kv"]
    rng = np.random.default_rng(5)
    T = {}
    shapes = {"attn_q": (E, 2 * nh * hd), "attn_k": (E, nkv * hd), "attn_v": (E, nkv * hd),
              "attn_output": (nh * hd, E), "ffn_gate": (E, FF), "ffn_up": (E, FF), "ffn_down": (FF, E)}
    for i, (name, (K, R)) in enumerate(shapes.items()):
        T[name] = q2_blocks(K, R, 100 + i, name in zero)
    T["token_embd"] = q2_blocks(E, cfg["n_vocab"], 99)
    for name, n in (("attn_norm", E), ("post_attention_norm", E), ("output_norm", E),
                    ("attn_q_norm", hd), ("attn_k_norm", hd)):
        T[name] = rng.uniform(0.8, 1.2, n).astype(np.float32)
    return T


def stack_of(cfg, T):
    return O.Stack(cfg, lambda layer, name: T[name], stage_f16=False, threads=2)


def mv(T, name, K, R, x):
    return O.q2_0_matvec(T[name], K, R, np.ascontiguousarray(x, np.float32), 2)


def test_stack_with_zero_projections_is_embedding_then_head():
    """wo = ffn_down = 0: the residual stream stays the token embedding, so
    hidden = rmsnorm(embd[t]) * out_norm and logits = embd . hidden (tied)."""
    cfg = dict(CFG)
    T = make_tensors(cfg, zero=("attn_output", "ffn_down"))
    st = stack_of(cfg, T)
    E = cfg["n_embd"]
    for pos, tok in enumerate((7, 31, 7)):
        h, lg = st.token(tok)
        e = O.q2_0_dequant(T["token_embd"][tok * E // 128 * 34:(tok + 1) * E // 128 * 34], E)
        want_h = O.rmsnorm(e, T["output_norm"], cfg["eps"])
        assert np.allclose(h, want_h, rtol=1e-6, atol=1e-6), pos
        assert np.allclose(lg, mv(T, "token_embd", E, cfg["n_vocab"], want_h), rtol=1e-5, atol=1e-5)


def test_attention_first_position_is_gated_value():
    """At position 0 the softmax has one entry, so Attn.step returns
    sigmoid(gate) * v of each head's kv head (q, k, RoPE and the norms of q/k
    drop out); with ffn_down = 0 the hidden state is x + wo . that."""
    cfg = dict(CFG)
    T = make_tensors(cfg, zero=("ffn_down",))
    st = stack_of(cfg, T)
    E, hd, nh, nkv = cfg["n_embd"], cfg["head_dim"], cfg["n_head"], cfg["n_head_kv"]
    tok = 11
    h, _ = st.token(tok)
    x = O.q2_0_dequant(T["token_embd"][tok * E // 128 * 34:(tok + 1) * E // 128 * 34], E)
    n = O.rmsnorm(x, T["attn_norm"], cfg["eps"])
    qfull = mv(T, "attn_q", E, 2 * nh * hd, n).reshape(nh, 2, hd)     # per head [q | gate]
    gate = qfull[:, 1, :]
    v = mv(T, "attn_v", E, nkv * hd, n).reshape(nkv, hd)
    ao = (1.0 / (1.0 + np.exp(-gate.astype(np.float64)))) * v[np.arange(nh) // (nh // nkv)]
    a = mv(T, "attn_output", nh * hd, E, ao.reshape(-1))
    want = O.rmsnorm((x + a).astype(np.float32), T["output_norm"], cfg["eps"])
    assert np.allclose(h, want, rtol=2e-5, atol=2e-5)
