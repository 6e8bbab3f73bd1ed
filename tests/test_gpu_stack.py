"""GPU parity of the hybrid stack (BASELINE config 4's engine) against the
token-by-token CPU restatement of BonsaiEngine / GDN.step / Attn.step, on a
small random-init geometry: 4 layers (3 GDN + 1 gated attention), GQA on both
the GDN heads (4 value / 2 key) and the attention heads (4 q / 2 kv), a
40-token prompt over two prefill chunks (32 + 8, crossing KV pages of 16),
then decode steps and graph-replayed generation (also a 34-token prompt, 32 + 2).

The oracle stages every mat-vec input and cached K/V in f16, as the
reference's GPU path does (Kernels.metal:428, MetalKVPool.swift); the GPU
computes the GDN prefill chunked and sums in other orders.  Tolerance on
logits and states: norm-wise relative error < 5e-3 (MetalSelfTest.swift:437-448
definition); greedy tokens must agree wherever the oracle's top-2 margin is
clear."""
import ctypes as C

import numpy as np
import pytest

import gadeon_amd as ga
import oracle as O
from conftest import rel_diff

pytestmark = pytest.mark.gpu

CFG = dict(n_layer=4, n_embd=256, n_ff=512, n_head=4, n_head_kv=2, head_dim=128, n_rot=64,
           rope_base=1e7, eps=1e-6, n_vocab=1000, attn_interval=4, d_state=128, n_k_head=2,
           n_v_head=4, d_conv=4, kv_block=16, max_ctx=128, max_batch=32)
TOL = 5e-3


def make_stack(ctx, seed=7, **over):
    cfg = dict(CFG, **over)
    sc = ga.StackConfig(**cfg)
    h = C.c_void_p()
    ctx.check(ctx.lib.gd_stack_create(ctx.h, C.byref(sc), seed, C.byref(h)))
    return cfg, h


def tensor_reader(ctx, st):
    def read(layer, name):
        w = ga.Q2W()
        f = C.POINTER(C.c_float)()
        r0 = C.c_int64()
        n = C.c_int64()
        ctx.check(ctx.lib.gd_stack_tensor(st, layer, name.encode(), C.byref(w), C.byref(r0),
                                          C.byref(f), C.byref(n)))
        if f:
            return ctx.get(C.cast(f, C.c_void_p).value, n.value, np.float32)
        nbytes = n.value * (w.K // 128) * 34
        d = ctx.alloc(nbytes)
        ctx.gd_q2_0_export_rows(C.byref(w), r0.value, n.value, d)
        out = ctx.get(d, nbytes, np.uint8)
        ctx.free(d)
        return out
    return read


def margin_ok(logits):
    top = np.sort(logits)[-2:]
    return top[1] - top[0] > 1e-2 * max(1.0, np.abs(logits).max())


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
    lib = ctx.lib
    try:
        read = tensor_reader(ctx, st)
        ref = O.Stack(cfg, read, stage_f16=True, threads=8)
        ids = (np.arange(plen) * 37 % cfg["n_vocab"]).astype(np.int32)
        nxt = C.c_int32()
        logits = np.empty(cfg["n_vocab"], np.float32)
        ctx.check(lib.gd_stack_prefill(st, ids.ctypes.data, ids.size, C.byref(nxt),
                                       logits.ctypes.data))
        for t in ids:
            _, ref_logits = ref.token(int(t))
        assert rel_diff(logits, ref_logits) < TOL
        if margin_ok(ref_logits):
            assert nxt.value == int(np.argmax(ref_logits))
        # GDN state of layer 0 after the prompt (chunked prefill vs token-serial).
        S_gpu = read(0, "ssm_state")
        assert rel_diff(S_gpu, ref.layer_state(0, "ssm_state")) < TOL
        # Decode steps, fed with the oracle's own greedy picks.
        tok = int(np.argmax(ref_logits))
        for step in range(6):
            ctx.check(lib.gd_stack_decode(st, tok, C.byref(nxt), logits.ctypes.data))
            _, ref_logits = ref.token(tok)
            assert rel_diff(logits, ref_logits) < TOL, step
            tok = int(np.argmax(ref_logits))
        pos = C.c_int64()
        ctx.check(lib.gd_stack_position(st, C.byref(pos)))
        assert pos.value == plen + 6
        # Graph-replayed generation continues from the GPU's last pick.
        gen = np.empty(5, np.int32)
        tok = nxt.value
        ctx.check(lib.gd_stack_generate(st, gen.size, gen.ctypes.data))
        for i in range(gen.size):
            _, ref_logits = ref.token(tok)
            if margin_ok(ref_logits):
                assert gen[i] == int(np.argmax(ref_logits)), i
            tok = int(gen[i])
        # Generation equals chained decode calls.
        ctx.check(lib.gd_stack_reset(st))
        ctx.check(lib.gd_stack_prefill(st, ids.ctypes.data, ids.size, C.byref(nxt), None))
        chain = []
        t = nxt.value
        for _ in range(4):
            ctx.check(lib.gd_stack_decode(st, t, C.byref(nxt), None))
            t = nxt.value
            chain.append(t)
        ctx.check(lib.gd_stack_reset(st))
        ctx.check(lib.gd_stack_prefill(st, ids.ctypes.data, ids.size, C.byref(nxt), None))
        g2 = np.empty(4, np.int32)
        ctx.check(lib.gd_stack_generate(st, 4, g2.ctypes.data))
        assert list(g2) == chain
    finally:
        lib.gd_stack_destroy(st)


def test_stack_rejects_bad_input(ctx):
    cfg, st = make_stack(ctx, n_layer=4)
    lib = ctx.lib
    try:
        bad = np.array([5, cfg["n_vocab"]], np.int32)
        assert lib.gd_stack_prefill(st, bad.ctypes.data, 2, None, None) == ga.GD_EINVAL
        assert b"vocab" in lib.gd_last_error(ctx.h)
        ok = np.arange(cfg["max_ctx"] + 1, dtype=np.int32)
        assert lib.gd_stack_prefill(st, ok.ctypes.data, ok.size, None, None) == ga.GD_EINVAL
        ctx.check(lib.gd_stack_request_stop(st))
        ids = np.arange(40, dtype=np.int32)
        assert lib.gd_stack_prefill(st, ids.ctypes.data, ids.size, None, None) == ga.GD_ESTOPPED
    finally:
        lib.gd_stack_destroy(st)
    sc = ga.StackConfig(**dict(CFG, head_dim=64))
    h = C.c_void_p()
    assert lib.gd_stack_create(ctx.h, C.byref(sc), 1, C.byref(h)) == ga.GD_EINVAL
