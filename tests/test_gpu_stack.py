"""GPU parity of the hybrid stack (BASELINE config 4's engine) against the CPU
restatement of BonsaiEngine / GDN.step / Attn.step (oracle/gd_oracle_stack.c).

Geometries:
  * small: 4 layers (3 GDN + 1 gated attention), hidden 256, GQA on both the
    GDN heads (4 value / 2 key) and the attention heads (4 q / 2 kv); prompts
    over one or two prefill chunks, crossing KV pages of 16;
  * past 64: the same small geometry with a 100-token single-chunk prompt (two
    64-query blocks of the prefill attention) and 40 decode / generate steps
    past position 64, where every decode attention split holds several keys;
  * config 4: BASELINE config 4's per-layer geometry at full width -- hidden
    5120, FFN 17408, 40 q / 8 kv heads of 128, 16/16 GDN heads, vocab 151936,
    kv pages of 16 -- with 4 layers (3 GDN + 1 attention), one 512-token
    prefill chunk (the T=512 GEMM plans, split-K partials, two-launch SwiGLU),
    then decode and generate steps;
  * dense: the qwen3 lineage (Model.swift:1-69; every layer plain ungated
    attention with the whole head rotated), small and at the reference 1.7B's
    per-layer geometry (hidden 2048, FFN 6144, 16 q / 8 kv heads of 128,
    vocab 151936) with 4 of its 28 layers.

The oracle's prefill rounds every mat-vec input to f16, as the reference
GPU prefill GEMM stages half tiles (Kernels.metal:428); this build does the
same.  In decode the reference GEMV reads f32 x (Kernels.metal:32-40), while
this build's decode GEMVs take f16 x (the north star's fp16-in GEMV), so
decode is checked against two oracles that share the prefill:
  * `ref16` stages decode mat-vec inputs as this build does: logits < 5e-3,
    GDN recurrent state and conv ring < 2e-3 (the north star's GDN bound);
  * `ref` keeps the reference's f32 decode inputs: logits < 5e-3 and states
    < 5e-3 -- the measured deviation of f16 decode inputs, printed.
K/V are cached as f16 on all sides.  After prefill the states are held to
2e-3 against the (single) prefill oracle.  Errors are norm-wise relative,
max|a-b| / max|b| (MetalSelfTest.swift:437-448); greedy tokens must agree
wherever the oracle's top-2 margin is clear.
Measured values are printed (pytest -s)."""
import ctypes as C
import os

import numpy as np
import pytest

import gadeon_amd as ga
import oracle as O
from conftest import rel_diff

pytestmark = pytest.mark.gpu

CFG = dict(n_layer=4, n_embd=256, n_ff=512, n_head=4, n_head_kv=2, head_dim=128, n_rot=64,
           rope_base=1e7, eps=1e-6, n_vocab=1000, attn_interval=4, d_state=128, n_k_head=2,
           n_v_head=4, d_conv=4, kv_block=16, max_ctx=128, max_batch=32)
CONFIG4 = dict(n_layer=4, n_embd=5120, n_ff=17408, n_head=40, n_head_kv=8, head_dim=128,
               n_rot=64, rope_base=1e7, eps=1e-6, n_vocab=151936, attn_interval=4, d_state=128,
               n_k_head=16, n_v_head=16, d_conv=4, kv_block=16, max_ctx=544, max_batch=512)
# The dense qwen3 lineage: no GDN geometry, attention in every layer, the
# whole head rotated.
DENSE = dict(dense=1, attn_interval=1, d_state=0, n_k_head=0, n_v_head=0, d_conv=0, n_rot=128,
             rope_base=1e6)
DENSE_1P7B = dict(DENSE, n_layer=4, n_embd=2048, n_ff=6144, n_head=16, n_head_kv=8,
                  head_dim=128, n_vocab=151936, kv_block=16, max_ctx=256, max_batch=128)
TOL = 5e-3          # logits
TOL_STATE = 2e-3    # GDN recurrent state and conv ring (the last three in_proj rows)
TOL_STATE_F32 = 5e-3  # the same against f32 decode inputs (this build decodes in f16)
THREADS = max(1, min(16, os.cpu_count() or 1))


def make_stack(ctx, seed=7, **over):
    cfg = dict(CFG, **over)
    sc = ga.StackConfig(**cfg)
    h = C.c_void_p()
    ctx.check(ctx.lib.gd_stack_create(ctx.h, C.byref(sc), seed, C.byref(h)))
    return cfg, h


def tensor_reader(ctx, st):
    cache = {}

    def read(layer, name):
        if (layer, name) in cache and name not in ("ssm_state", "ssm_conv_state"):
            return cache[layer, name]
        w = ga.Q2W()
        f = C.POINTER(C.c_float)()
        r0 = C.c_int64()
        n = C.c_int64()
        ctx.check(ctx.lib.gd_stack_tensor(st, layer, name.encode(), C.byref(w), C.byref(r0),
                                          C.byref(f), C.byref(n)))
        if f:
            out = ctx.get(C.cast(f, C.c_void_p).value, n.value, np.float32)
        else:
            nbytes = n.value * (w.K // 128) * 34
            d = ctx.alloc(nbytes)
            ctx.gd_q2_0_export_rows(C.byref(w), r0.value, n.value, d)
            out = ctx.get(d, nbytes, np.uint8)
            ctx.free(d)
        cache[layer, name] = out
        return out
    return read


def margin_ok(logits):
    top = np.sort(logits)[-2:]
    return top[1] - top[0] > 1e-2 * max(1.0, np.abs(logits).max())


def check_states(cfg, read, ref, what, tol=TOL_STATE):
    for il in range(cfg["n_layer"]):
        if (il + 1) % cfg["attn_interval"] == 0:
            continue
        rs = rel_diff(read(il, "ssm_state"), ref.layer_state(il, "ssm_state"))
        rc = rel_diff(read(il, "ssm_conv_state"), ref.layer_state(il, "ssm_conv_state"))
        print(f"  {what} layer {il}: state relDiff {rs:.2e}, conv ring {rc:.2e}")
        assert rs < tol, (what, il, rs)
        assert rc < tol, (what, il, rc)


def run_parity(ctx, cfg, st, ids, n_decode, n_gen, chain=True):
    """Prefill `ids`, then n_decode decode steps fed with the oracle's greedy
    picks, then n_gen graph-replayed generate steps; logits, states and picks
    against the oracles at every step."""
    lib = ctx.lib
    read = tensor_reader(ctx, st)
    ref = O.Stack(cfg, read, stage_f16=True, threads=THREADS)
    # This build's decode numerics: the output projections read f16 inputs,
    # the norm-fed GEMVs theirs at f32 precision.
    ref16 = O.Stack(cfg, read, stage_f16=True, threads=THREADS, decode_f16="outputs")
    nxt = C.c_int32()
    logits = np.empty(cfg["n_vocab"], np.float32)
    ctx.check(lib.gd_stack_prefill(st, ids.ctypes.data, ids.size, C.byref(nxt),
                                   logits.ctypes.data))
    ref_logits = None
    for i in range(0, ids.size, cfg["max_batch"]):     # the GPU's chunks (same result)
        _, ref_logits = ref.prefill(ids[i:i + cfg["max_batch"]])
        ref16.prefill(ids[i:i + cfg["max_batch"]])
    r = rel_diff(logits, ref_logits)
    print(f"  prefill {ids.size}: logits relDiff {r:.2e}")
    assert r < TOL
    if margin_ok(ref_logits):
        assert nxt.value == int(np.argmax(ref_logits))
    check_states(cfg, read, ref, "after prefill")
    tok = int(np.argmax(ref_logits))
    worst = [0.0, 0.0]
    for step in range(n_decode):
        ctx.check(lib.gd_stack_decode(st, tok, C.byref(nxt), logits.ctypes.data))
        _, ref_logits = ref.token(tok)
        _, ref16_logits = ref16.token(tok)
        r, r16 = rel_diff(logits, ref_logits), rel_diff(logits, ref16_logits)
        worst = [max(worst[0], r), max(worst[1], r16)]
        assert r < TOL and r16 < TOL, (step, r, r16)
        tok = int(np.argmax(ref_logits))
    print(f"  {n_decode} decode steps: worst logits relDiff {worst[1]:.2e} (f16 inputs of the "
          f"output projections), {worst[0]:.2e} (f32, the reference's)")
    check_states(cfg, read, ref16, "after decode")
    check_states(cfg, read, ref, "after decode, vs f32 decode inputs", TOL_STATE_F32)
    pos = C.c_int64()
    ctx.check(lib.gd_stack_position(st, C.byref(pos)))
    assert pos.value == ids.size + n_decode
    # Graph-replayed generation continues from the GPU's last pick.
    gen = np.empty(n_gen, np.int32)
    tok = nxt.value
    ctx.check(lib.gd_stack_generate(st, gen.size, gen.ctypes.data))
    agree = 0
    for i in range(gen.size):
        _, ref_logits = ref.token(tok)
        _, ref16_logits = ref16.token(tok)
        if margin_ok(ref16_logits):
            assert gen[i] == int(np.argmax(ref16_logits)), i
            agree += 1
        tok = int(gen[i])
    print(f"  generate {n_gen}: {agree} clear-margin picks agree")
    check_states(cfg, read, ref16, "after generate")
    check_states(cfg, read, ref, "after generate, vs f32 decode inputs", TOL_STATE_F32)
    if chain:
        # Generation equals chained decode calls.
        ctx.check(lib.gd_stack_reset(st))
        ctx.check(lib.gd_stack_prefill(st, ids.ctypes.data, ids.size, C.byref(nxt), None))
        seq = []
        t = nxt.value
        for _ in range(4):
            ctx.check(lib.gd_stack_decode(st, t, C.byref(nxt), None))
            t = nxt.value
            seq.append(t)
        ctx.check(lib.gd_stack_reset(st))
        ctx.check(lib.gd_stack_prefill(st, ids.ctypes.data, ids.size, C.byref(nxt), None))
        g2 = np.empty(4, np.int32)
        ctx.check(lib.gd_stack_generate(st, 4, g2.ctypes.data))
        assert list(g2) == seq


# nk = 4: every value head has its own key head.  A 34-token prompt ends with
# a 2-token chunk, shorter than the conv window: its new conv ring mixes the
# old ring with the chunk's inputs.  max_batch = 64 takes the 40-token prompt
# as one chunk, where the GDN in_proj's split-K partials fit the residual
# partials buffer and are summed by the kernels that read them.
@pytest.mark.parametrize("nk,plen,mb", [(2, 40, 32), (4, 40, 32), (4, 34, 32), (2, 40, 64)])
def test_stack_prefill_decode_generate(ctx, nk, plen, mb):
    """nk = 2 shares key heads between value heads (separate conv, step and
    gated-norm kernels in decode); nk = 4 takes the fused one-launch step."""
    cfg, st = make_stack(ctx, n_k_head=nk, max_batch=mb)
    try:
        ids = (np.arange(plen) * 37 % cfg["n_vocab"]).astype(np.int32)
        print(f"\nstack nk={nk} prompt {plen} max_batch {mb}", flush=True)
        run_parity(ctx, cfg, st, ids, n_decode=6, n_gen=5)
    finally:
        ctx.lib.gd_stack_destroy(st)


@pytest.mark.parametrize("nk", [2, 4])
def test_stack_past_position_64(ctx, nk):
    """A 100-token prompt in one chunk (prefill attention over two 64-query
    blocks, in_proj split-K partials with the T=100 plans), then 20 decode and
    20 generate steps reaching position 140: every decode attention split
    holds two or three cached keys, so the per-wave key loop and its next-key
    prefetch run."""
    cfg, st = make_stack(ctx, n_k_head=nk, max_batch=128, max_ctx=256)
    try:
        ids = ((np.arange(100) * 53 + 11) % cfg["n_vocab"]).astype(np.int32)
        print(f"\nstack nk={nk} prompt 100 in one chunk", flush=True)
        run_parity(ctx, cfg, st, ids, n_decode=20, n_gen=20, chain=False)
    finally:
        ctx.lib.gd_stack_destroy(st)


def test_stack_head_dim_256(ctx):
    """The reference 27B's attention and GDN shape pattern (Model.swift:11-32:
    head_dim 256, 6 q heads per kv head; more value heads than key heads),
    scaled down: 6 q / 1 kv heads of 256, GDN 4 value / 2 key heads; a
    70-token prompt over two chunks, decode and generate."""
    cfg, st = make_stack(ctx, head_dim=256, n_head=6, n_head_kv=1, n_k_head=2, n_v_head=4,
                         max_batch=48)
    try:
        ids = ((np.arange(70) * 29 + 3) % cfg["n_vocab"]).astype(np.int32)
        print("\nstack head_dim 256, 6/1 heads", flush=True)
        run_parity(ctx, cfg, st, ids, n_decode=6, n_gen=6, chain=False)
    finally:
        ctx.lib.gd_stack_destroy(st)


def test_stack_config4_geometry(ctx):
    """BASELINE config 4 at its own per-layer geometry (4 of its 64 layers):
    a 512-id random prompt in one prefill chunk, 8 decode steps, 8 generate
    steps."""
    cfg, st = make_stack(ctx, seed=11, **CONFIG4)
    try:
        ids = np.random.default_rng(2024).integers(0, cfg["n_vocab"], 512).astype(np.int32)
        print(f"\nconfig-4 geometry, 4 layers, prompt 512 (oracle on {THREADS} threads)",
              flush=True)
        run_parity(ctx, cfg, st, ids, n_decode=8, n_gen=8, chain=False)
    finally:
        ctx.lib.gd_stack_destroy(st)


def test_stack_dense(ctx):
    """The dense lineage's attention path (plain q rows, ungated prefill and
    decode, whole-head rope) through prefill over two chunks, decode and
    generate, reset and chained decode."""
    cfg, st = make_stack(ctx, seed=31, max_batch=32, **DENSE)
    try:
        ids = (np.arange(45) * 41 % cfg["n_vocab"]).astype(np.int32)
        print("\nstack dense, 4 attention layers, prompt 45", flush=True)
        run_parity(ctx, cfg, st, ids, n_decode=6, n_gen=5)
    finally:
        ctx.lib.gd_stack_destroy(st)


def test_stack_dense_1p7b_geometry(ctx):
    """The reference 1.7B's per-layer geometry (Model.swift:5-7) with 4 of its
    28 layers: a 128-id prompt in one chunk, 6 decode and 6 generate steps."""
    cfg, st = make_stack(ctx, seed=32, **DENSE_1P7B)
    try:
        ids = np.random.default_rng(17).integers(0, cfg["n_vocab"], 128).astype(np.int32)
        print("\nstack dense 1.7B geometry, 4 layers, prompt 128", flush=True)
        run_parity(ctx, cfg, st, ids, n_decode=6, n_gen=6, chain=False)
    finally:
        ctx.lib.gd_stack_destroy(st)


def test_stack_rejects_bad_input(ctx):
    cfg, st = make_stack(ctx, n_layer=4)
    lib = ctx.lib
    try:
        bad = np.array([5, cfg["n_vocab"]], np.int32)
        assert lib.gd_stack_prefill(st, bad.ctypes.data, 2, None, None) == ga.GD_EINVAL
        assert b"vocab" in lib.gd_last_error(ctx.h)
        ok = np.arange(cfg["max_ctx"] + 1, dtype=np.int32)
        assert lib.gd_stack_prefill(st, ok.ctypes.data, ok.size, None, None) == ga.GD_EINVAL
    finally:
        lib.gd_stack_destroy(st)
    sc = ga.StackConfig(**dict(CFG, head_dim=64))
    h = C.c_void_p()
    assert lib.gd_stack_create(ctx.h, C.byref(sc), 1, C.byref(h)) == ga.GD_EINVAL
    # A dense stack has attention in every layer and no GDN geometry.
    for bad in (dict(DENSE, attn_interval=4), dict(DENSE, d_state=128), dict(DENSE, dense=2)):
        sc = ga.StackConfig(**dict(CFG, **bad))
        assert lib.gd_stack_create(ctx.h, C.byref(sc), 1, C.byref(h)) == ga.GD_EINVAL
        assert b"dense" in lib.gd_last_error(ctx.h)


def test_stack_stop_signal(ctx):
    """MetalEngine's cooperative stop (MetalEngine.swift:15-25, 79-81,
    183-186): a raised stop ends generate before its next step and stays
    raised (shouldStop); the next prefill clears it and runs; a stop raised
    from another thread during a multi-chunk prefill ends it at a chunk
    boundary (or the prefill finishes first)."""
    import threading
    cfg, st = make_stack(ctx, n_layer=4, max_batch=16, max_ctx=1024)
    lib = ctx.lib
    raised = C.c_int()
    try:
        ids = np.arange(40, dtype=np.int32)
        nxt = C.c_int32()
        ctx.check(lib.gd_stack_prefill(st, ids.ctypes.data, ids.size, C.byref(nxt), None))
        ctx.check(lib.gd_stack_should_stop(st, C.byref(raised)))
        assert raised.value == 0
        toks = np.empty(8, np.int32)
        ctx.check(lib.gd_stack_request_stop(st))
        assert lib.gd_stack_generate(st, 8, toks.ctypes.data) == ga.GD_ESTOPPED
        pos = C.c_int64()
        ctx.check(lib.gd_stack_position(st, C.byref(pos)))
        assert pos.value == 40                          # no step was made
        ctx.check(lib.gd_stack_should_stop(st, C.byref(raised)))
        assert raised.value == 1                        # stays raised for the decode loop
        # The next prefill clears it and runs to the end.
        ctx.check(lib.gd_stack_prefill(st, ids.ctypes.data, ids.size, C.byref(nxt), None))
        ctx.check(lib.gd_stack_should_stop(st, C.byref(raised)))
        assert raised.value == 0
        ctx.check(lib.gd_stack_position(st, C.byref(pos)))
        assert pos.value == 80
        ctx.check(lib.gd_stack_generate(st, 8, toks.ctypes.data))
        # A stop from another thread while 60 chunks of 16 are prefilled.
        ctx.check(lib.gd_stack_reset(st))
        long_ids = (np.arange(960) % cfg["n_vocab"]).astype(np.int32)
        out = {}
        th = threading.Thread(target=lambda: out.setdefault(
            "rc", lib.gd_stack_prefill(st, long_ids.ctypes.data, long_ids.size, None, None)))
        th.start()
        while th.is_alive():
            lib.gd_stack_request_stop(st)
            th.join(0.001)
        ctx.check(lib.gd_stack_position(st, C.byref(pos)))
        assert out["rc"] in (ga.GD_OK, ga.GD_ESTOPPED)
        if out["rc"] == ga.GD_ESTOPPED:
            assert pos.value % 16 == 0 and pos.value < 960
        else:
            assert pos.value == 960
        ctx.sync()
    finally:
        lib.gd_stack_destroy(st)
