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


DCFG = dict(CFG, dense=1, n_rot=128, rope_base=1e6, d_state=0, n_k_head=0, n_v_head=0,
            d_conv=0)


def make_dense_tensors(cfg, zero=("ffn_down",)):
    """The dense lineage's layer: q without a gate (wq [E, nh hd]) and the
    pre-FFN norm named ffn_norm (Model.swift:100-130)."""
    T = make_tensors(cfg, zero)
    E, hd, nh = cfg["n_embd"], cfg["head_dim"], cfg["n_head"]
    T["attn_q"] = q2_blocks(E, nh * hd, 150)
    T["ffn_norm"] = T.pop("post_attention_norm")
    return T


def test_dense_attention_is_ungated_softmax_attention():
    """The dense branch of Attn.step (Attention.swift:81-83, 132-134) over two
    positions, against a direct numpy statement: plain q from wq, q/k RMS
    norms, full-head NEOX rope at each position, softmax over the cached keys
    and no output gate; with ffn_down = 0 the hidden state is x + wo . ao.
    At position 0 the attention output is the value itself."""
    cfg = dict(DCFG)
    T = make_dense_tensors(cfg)
    st = stack_of(cfg, T)
    E, hd, nh, nkv = cfg["n_embd"], cfg["head_dim"], cfg["n_head"], cfg["n_head_kv"]
    eps, rot, base = cfg["eps"], cfg["n_rot"], cfg["rope_base"]
    keys, vals = [], []
    for pos, tok in enumerate((11, 40)):
        h, _ = st.token(tok)
        x = O.q2_0_dequant(T["token_embd"][tok * E // 128 * 34:(tok + 1) * E // 128 * 34], E)
        n = O.rmsnorm(x, T["attn_norm"], eps)
        q = mv(T, "attn_q", E, nh * hd, n).reshape(nh, hd).astype(np.float64)
        k = mv(T, "attn_k", E, nkv * hd, n).reshape(nkv, hd).astype(np.float64)
        v = mv(T, "attn_v", E, nkv * hd, n).reshape(nkv, hd).astype(np.float64)
        rms = lambda a, w: a / np.sqrt((a * a).mean(axis=1, keepdims=True) + eps) * w
        q, k = rms(q, T["attn_q_norm"]), rms(k, T["attn_k_norm"])
        q = O.rope_neox(q.astype(np.float32).reshape(-1), hd, rot, base, pos).reshape(nh, hd)
        k = O.rope_neox(k.astype(np.float32).reshape(-1), hd, rot, base, pos).reshape(nkv, hd)
        keys.append(k.astype(np.float64))
        vals.append(v)
        ao = np.empty((nh, hd))
        for hh in range(nh):
            g = hh // (nh // nkv)
            s = np.array([q[hh] @ kk[g] for kk in keys]) / np.sqrt(hd)
            p = np.exp(s - s.max())
            p /= p.sum()
            ao[hh] = sum(pi * vv[g] for pi, vv in zip(p, vals))
        if pos == 0:
            assert np.allclose(ao, v[np.arange(nh) // (nh // nkv)])
        a = mv(T, "attn_output", nh * hd, E, ao.reshape(-1))
        want = O.rmsnorm((x + a).astype(np.float32), T["output_norm"], eps)
        assert np.allclose(h, want, rtol=5e-5, atol=5e-5), pos


def test_rope_shift_rotates_at_position_plus_shift():
    """MetalEngine.ropeShift (MetalEngine.swift:432-435): a token at position p
    is rotated at p + shift while its K/V are cached at p and causality stays
    on positions.  Three dense-attention tokens, the shift changed from 0 to 5
    before the third, against a direct numpy statement (cached keys keep the
    rotation they were made with).  And RoPE is relative: the same shift on
    every token from the first changes nothing beyond f32 rounding."""
    cfg = dict(DCFG)
    T = make_dense_tensors(cfg)
    E, hd, nh, nkv = cfg["n_embd"], cfg["head_dim"], cfg["n_head"], cfg["n_head_kv"]
    eps, rot, base = cfg["eps"], cfg["n_rot"], cfg["rope_base"]
    toks, shifts = (11, 40, 23), (0, 0, 5)
    st = stack_of(cfg, T)
    keys, vals = [], []
    for pos, (tok, sh) in enumerate(zip(toks, shifts)):
        st.rope_shift = sh
        h, _ = st.token(tok)
        x = O.q2_0_dequant(T["token_embd"][tok * E // 128 * 34:(tok + 1) * E // 128 * 34], E)
        n = O.rmsnorm(x, T["attn_norm"], eps)
        q = mv(T, "attn_q", E, nh * hd, n).reshape(nh, hd).astype(np.float64)
        k = mv(T, "attn_k", E, nkv * hd, n).reshape(nkv, hd).astype(np.float64)
        v = mv(T, "attn_v", E, nkv * hd, n).reshape(nkv, hd).astype(np.float64)
        rms = lambda a, w: a / np.sqrt((a * a).mean(axis=1, keepdims=True) + eps) * w
        q, k = rms(q, T["attn_q_norm"]), rms(k, T["attn_k_norm"])
        q = O.rope_neox(q.astype(np.float32).reshape(-1), hd, rot, base, pos + sh).reshape(nh, hd)
        k = O.rope_neox(k.astype(np.float32).reshape(-1), hd, rot, base, pos + sh).reshape(nkv, hd)
        keys.append(k.astype(np.float64))
        vals.append(v)
        ao = np.empty((nh, hd))
        for hh in range(nh):
            g = hh // (nh // nkv)
            s = np.array([q[hh] @ kk[g] for kk in keys]) / np.sqrt(hd)
            p = np.exp(s - s.max())
            p /= p.sum()
            ao[hh] = sum(pi * vv[g] for pi, vv in zip(p, vals))
        a = mv(T, "attn_output", nh * hd, E, ao.reshape(-1))
        want = O.rmsnorm((x + a).astype(np.float32), T["output_norm"], eps)
        assert np.allclose(h, want, rtol=5e-5, atol=5e-5), pos
    # The shift of the third token mattered: without it the output differs.
    ref = stack_of(cfg, T)
    hs = [ref.token(t)[0] for t in toks]
    assert np.abs(hs[2] - h).max() > 1e-3
    # One shift for every token: relative positions, hence outputs, unchanged.
    sh = stack_of(cfg, T)
    sh.rope_shift = 37
    for tok, want in zip(toks, hs):
        assert np.allclose(sh.token(tok)[0], want, rtol=2e-4, atol=2e-4)


GCFG = dict(n_layer=1, n_embd=256, n_ff=256, n_head=4, n_head_kv=2, head_dim=128, n_rot=64,
            rope_base=1e7, eps=1e-6, n_vocab=64, attn_interval=9, d_state=128, n_k_head=1,
            n_v_head=2, d_conv=4, max_ctx=8)


def make_gdn_tensors(cfg, zero=("ffn_down",)):
    E, FF, dS = cfg["n_embd"], cfg["n_ff"], cfg["d_state"]
    nK, nV = cfg["n_k_head"], cfg["n_v_head"]
    convDim, valDim = (2 * nK + nV) * dS, nV * dS
    rng = np.random.default_rng(6)
    T = {}
    shapes = {"attn_qkv": (E, convDim), "attn_gate": (E, valDim), "ssm_beta": (E, nV),
              "ssm_alpha": (E, nV), "ssm_out": (valDim, E), "ffn_gate": (E, FF), "ffn_up": (E, FF),
              "ffn_down": (FF, E)}
    for i, (name, (K, R)) in enumerate(shapes.items()):
        T[name] = q2_blocks(K, R, 200 + i, name in zero)
    T["token_embd"] = q2_blocks(E, cfg["n_vocab"], 98)
    for name, n in (("attn_norm", E), ("post_attention_norm", E), ("output_norm", E),
                    ("ssm_norm", dS)):
        T[name] = rng.uniform(0.8, 1.2, n).astype(np.float32)
    T["ssm_conv1d"] = rng.uniform(-0.5, 0.5, convDim * cfg["d_conv"]).astype(np.float32)
    T["ssm_dt"] = rng.uniform(-0.5, 0.5, nV).astype(np.float32)
    T["ssm_a"] = -rng.uniform(0.3, 2.0, nV).astype(np.float32)
    return T


def test_stack_gdn_layer_matches_its_definition():
    """The stack oracle's GDN layer (GDN.step, GDN.swift:20-120, inside
    BonsaiEngine.forward) against an independent f64 build of the same layer
    from numpy formulas and the pinned f64 scan: projections (f64 brute-force
    mat-vec), gates, causal conv + silu with the ring carried across tokens,
    L2 norm of q and k, the delta-rule scan, per-head RMSNorm times ssm_norm,
    times silu(z), then ssm_out.  ffn_down = 0, so hidden = rmsnorm(x + layer
    output).  Three tokens, so the conv ring and the state carry over; one key
    head shared by two value heads (hk = hv % nK)."""
    cfg = dict(GCFG)
    T = make_gdn_tensors(cfg)
    st = O.Stack(cfg, lambda layer, name: T[name], stage_f16=False, threads=2)
    E, dS, nK, nV, eps = cfg["n_embd"], cfg["d_state"], cfg["n_k_head"], cfg["n_v_head"], cfg["eps"]
    keyDim, valDim = nK * dS, nV * dS
    convDim = 2 * keyDim + valDim
    mv64 = lambda name, K, R, x: O.q2_0_matvec_f64(T[name], K, R, np.asarray(x, np.float64))
    rms = lambda x, w: x / np.sqrt(np.mean(x ** 2) + eps) * w
    silu = lambda x: x / (1 + np.exp(-x))
    cw = T["ssm_conv1d"].astype(np.float64).reshape(convDim, 4)
    hist = np.zeros((3, convDim))                       # previous three conv inputs
    S = np.zeros(nV * dS * dS)
    for pos, tok in enumerate((9, 40, 9)):
        h, _ = st.token(tok)
        x = O.q2_0_dequant(T["token_embd"][tok * E // 128 * 34:(tok + 1) * E // 128 * 34],
                           E).astype(np.float64)
        n = rms(x, T["attn_norm"].astype(np.float64))
        qkv, z = mv64("attn_qkv", E, convDim, n), mv64("attn_gate", E, valDim, n)
        bp, ap = mv64("ssm_beta", E, nV, n), mv64("ssm_alpha", E, nV, n)
        beta = 1 / (1 + np.exp(-bp))
        g = np.logaddexp(0, ap + T["ssm_dt"]) * T["ssm_a"]
        win = np.vstack([hist, qkv])                    # tokens t-3 .. t
        conv = silu((win.T * cw).sum(1))
        hist = win[1:]
        q = conv[:keyDim].reshape(nK, dS)
        k = conv[keyDim:2 * keyDim].reshape(nK, dS)
        q = q / np.sqrt((q ** 2).sum(1, keepdims=True) + eps)
        k = k / np.sqrt((k ** 2).sum(1, keepdims=True) + eps)
        v = conv[2 * keyDim:]
        o = O.gdn_scan_f64(q.ravel(), k.ravel(), v, g, beta, S, nV, nK, dS, 1 / np.sqrt(dS))
        o = o.reshape(nV, dS)
        o = o / np.sqrt(np.mean(o ** 2, 1, keepdims=True) + eps) * T["ssm_norm"]
        o = o.ravel() * silu(z)
        a = mv64("ssm_out", valDim, E, o)
        want = rms(x + a, T["output_norm"].astype(np.float64))
        assert np.allclose(h, want, rtol=1e-4, atol=1e-4 * np.abs(want).max()), pos
        assert np.allclose(st.layer_state(0, "ssm_state"), S, rtol=1e-4,
                           atol=1e-4 * np.abs(S).max()), pos


def test_prefill_is_token_serial():
    """or_stack_prefill (layer by layer, batched mat-vecs) equals token-by-token
    or_stack_token bit for bit: hidden, logits and every state, on a hybrid
    geometry (GDN layers with nK < nV and a gated attention layer), with and
    without f16 staging, over two chunks."""
    cfg = dict(n_layer=4, n_embd=256, n_ff=384, n_head=4, n_head_kv=2, head_dim=128, n_rot=64,
               rope_base=1e7, eps=1e-6, n_vocab=300, attn_interval=2, d_state=128, n_k_head=1,
               n_v_head=2, d_conv=4, max_ctx=40)
    Tg = make_gdn_tensors(cfg, zero=())
    Ta = make_tensors(dict(cfg, n_vocab=cfg["n_vocab"]))
    tensors = lambda layer, name: Tg[name] if name in Tg else Ta[name]
    ids = (np.arange(29) * 13 % cfg["n_vocab"]).astype(np.int32)
    for stage in (False, True):
        a = O.Stack(cfg, tensors, stage_f16=stage, threads=3, decode_f16=True)
        b = O.Stack(cfg, tensors, stage_f16=stage, threads=2, decode_f16=True)
        ha, la = a.prefill(ids[:17])
        ha, la = a.prefill(ids[17:])
        for t in ids:
            hb, lb = b.token(int(t))
        assert np.array_equal(ha, hb) and np.array_equal(la, lb)
        for il in (0, 2):
            assert np.array_equal(a.layer_state(il, "ssm_state"), b.layer_state(il, "ssm_state"))
        # one more decode token from both
        assert np.array_equal(a.token(5)[1], b.token(5)[1])


def test_decode_staging_outputs_mode():
    """decode_f16="outputs" rounds only the inputs of the output projections
    (ssm_out, attn_output, ffn_down) to f16.  With those three weights zero,
    their outputs are zero whatever their inputs, so the mode must give the
    f32 decode's logits bit for bit, while rounding every mat-vec input
    (decode_f16=True) must not; with them nonzero it must differ from both."""
    cfg = dict(n_layer=4, n_embd=256, n_ff=384, n_head=4, n_head_kv=2, head_dim=128, n_rot=64,
               rope_base=1e7, eps=1e-6, n_vocab=300, attn_interval=2, d_state=128, n_k_head=1,
               n_v_head=2, d_conv=4, max_ctx=40)
    ids = (np.arange(9) * 13 % cfg["n_vocab"]).astype(np.int32)
    for zero in (("ssm_out", "attn_output", "ffn_down"), ()):
        Tg = make_gdn_tensors(cfg, zero=tuple(z for z in zero if z != "attn_output"))
        Ta = make_tensors(dict(cfg, n_vocab=cfg["n_vocab"]), zero=zero)
        tensors = lambda layer, name: Tg[name] if name in Tg else Ta[name]
        out = {}
        for mode in (False, True, "outputs"):
            s = O.Stack(cfg, tensors, stage_f16=True, threads=2, decode_f16=mode)
            s.prefill(ids)
            out[mode] = np.concatenate([s.token(int(t))[1] for t in (3, 7, 11)])
        if zero:
            assert np.array_equal(out["outputs"], out[False])
            assert not np.array_equal(out[True], out[False])
        else:
            assert not np.array_equal(out["outputs"], out[False])
            assert not np.array_equal(out["outputs"], out[True])
    with pytest.raises(ValueError):
        O.Stack(cfg, tensors, decode_f16="inputs")
