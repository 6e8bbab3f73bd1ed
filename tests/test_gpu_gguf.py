"""A stack whose weights come from a GGUF file (gd_stack_create_from_gguf):
BonsaiModel(path:) + upload (Model.swift:133-148, MetalContext.swift:146-191).

A seeded random stack is exported tensor by tensor under the reference's
names (Model.swift:100-145) into a GGUF v3 file written by tests/gguf_writer;
the stack loaded from that file must hold byte-identical weights and give
bit-identical logits, picks and generations (same kernels on the same bytes),
for the qwen35 hybrid and for the dense qwen3 lineage (its own metadata keys
and its ffn_norm name).
With an output.weight in the file the lm_head is that matrix (the untied
branch of Model.swift:145), checked against the CPU oracle.  Files that lack
a tensor or hold one of the wrong type or shape are rejected by name."""
import ctypes as C

import numpy as np
import pytest

import gadeon_amd as ga
import oracle as O
from conftest import rel_diff
from test_gpu_stack import CFG, DENSE, THREADS, TOL, make_stack, tensor_reader
from tests import gguf_writer as W

pytestmark = pytest.mark.gpu

COMMON = ("attn_norm", "ffn_gate", "ffn_up", "ffn_down")
REC = ("attn_qkv", "attn_gate", "ssm_beta", "ssm_alpha", "ssm_out", "ssm_conv1d", "ssm_dt",
       "ssm_a", "ssm_norm")
ATT = ("attn_q", "attn_k", "attn_v", "attn_output", "attn_q_norm", "attn_k_norm")


def export(ctx, cfg, st):
    """{(layer, name): Q2_0 blocks [rows][K/128*34] (uint8) or f32 array}."""
    read = tensor_reader(ctx, st)
    out = {}

    def put(layer, name):
        w, r0, f, n = ga.Q2W(), C.c_int64(), C.POINTER(C.c_float)(), C.c_int64()
        ctx.check(ctx.lib.gd_stack_tensor(st, layer, name.encode(), C.byref(w), C.byref(r0),
                                          C.byref(f), C.byref(n)))
        a = read(layer, name)
        if name == "ssm_conv1d":
            a = a.reshape(-1, cfg["d_conv"])
        elif not f:
            a = a.reshape(n.value, w.K // 128 * 34)
        out[layer, name] = a

    put(-1, "token_embd")
    put(-1, "output_norm")
    for il in range(cfg["n_layer"]):
        rec = (il + 1) % cfg["attn_interval"] != 0
        post = "ffn_norm" if cfg.get("dense") else "post_attention_norm"
        for name in COMMON + (post,) + (REC if rec else ATT):
            put(il, name)
    return out


def load(ctx, path, cfg):
    g = ga.GGUF(path)
    try:
        h = C.c_void_p()
        ctx.check(ctx.lib.gd_stack_create_from_gguf(ctx.h, g.h, cfg["kv_block"], cfg["max_ctx"],
                                                    cfg["max_batch"], C.byref(h)))
    finally:
        g.close()       # the stack keeps no reference to the file
    return h


def run(ctx, st, ids, n_dec=3, n_gen=4):
    lib = ctx.lib
    nxt = C.c_int32()
    lg = np.empty(CFG["n_vocab"], np.float32)
    ctx.check(lib.gd_stack_prefill(st, ids.ctypes.data, ids.size, C.byref(nxt), lg.ctypes.data))
    out = [lg.copy()]
    picks = [nxt.value]
    for _ in range(n_dec):
        ctx.check(lib.gd_stack_decode(st, nxt.value, C.byref(nxt), lg.ctypes.data))
        out.append(lg.copy())
        picks.append(nxt.value)
    gen = np.empty(n_gen, np.int32)
    ctx.check(lib.gd_stack_generate(st, n_gen, gen.ctypes.data))
    return out, picks, list(gen)


@pytest.mark.parametrize("dense", [False, True])
def test_gguf_round_trip_is_bit_identical(ctx, tmp_path, dense):
    cfg, a = make_stack(ctx, seed=11, **(DENSE if dense else {}))
    b = None
    try:
        tensors = export(ctx, cfg, a)
        path = W.write(tmp_path / "stack.gguf", W.stack_kvs(cfg),
                       W.stack_tensors(cfg, tensors))
        with ga.GGUF(path) as g:
            c = g.stack_config()
            for k in ("n_layer", "n_embd", "n_ff", "n_head", "n_head_kv", "head_dim", "n_rot",
                      "n_vocab", "attn_interval", "d_state", "n_k_head", "n_v_head", "d_conv",
                      "dense"):
                assert getattr(c, k) == cfg.get(k, 0), k
        b = load(ctx, path, cfg)
        # The loaded stack holds the file's bytes (repack, then export back).
        loaded = export(ctx, cfg, b)
        for key, arr in tensors.items():
            assert np.array_equal(loaded[key], arr), key
        # The lm_head is tied: "output" names the embedding's matrix.
        read_b = tensor_reader(ctx, b)
        assert np.array_equal(read_b(-1, "output"), read_b(-1, "token_embd"))
        ids = (np.arange(40) * 37 % cfg["n_vocab"]).astype(np.int32)
        la, pa, ga_ = run(ctx, a, ids)
        lb, pb, gb = run(ctx, b, ids)
        for i, (x, y) in enumerate(zip(la, lb)):
            assert np.array_equal(x, y), i
        assert pa == pb and ga_ == gb
        print(f"\n  loaded stack: {len(la)} logits vectors bit-identical, picks {pb}, "
              f"generated {gb}")
    finally:
        ctx.lib.gd_stack_destroy(a)
        if b:
            ctx.lib.gd_stack_destroy(b)


def test_gguf_untied_output(ctx, tmp_path):
    cfg, a = make_stack(ctx, seed=12)
    b = None
    try:
        tensors = export(ctx, cfg, a)
        head = O.lcg_q2_0(cfg["n_embd"], cfg["n_vocab"], 99).reshape(cfg["n_vocab"], -1)
        tensors[-1, "output"] = head
        path = W.write(tmp_path / "untied.gguf", W.stack_kvs(cfg),
                       W.stack_tensors(cfg, tensors))
        b = load(ctx, path, cfg)
        read_b = tensor_reader(ctx, b)
        assert np.array_equal(read_b(-1, "output").reshape(head.shape), head)
        assert np.array_equal(read_b(-1, "token_embd").reshape(tensors[-1, "token_embd"].shape),
                              tensors[-1, "token_embd"])
        ids = (np.arange(24) * 53 % cfg["n_vocab"]).astype(np.int32)
        nxt = C.c_int32()
        lg = np.empty(cfg["n_vocab"], np.float32)
        ctx.check(ctx.lib.gd_stack_prefill(b, ids.ctypes.data, ids.size, C.byref(nxt),
                                           lg.ctypes.data))
        ref = O.Stack(cfg, read_b, stage_f16=True, threads=THREADS, untied=True)
        _, ref_lg = ref.prefill(ids)
        tied = O.Stack(cfg, read_b, stage_f16=True, threads=THREADS)
        _, tied_lg = tied.prefill(ids)
        r, r_tied = rel_diff(lg, ref_lg), rel_diff(lg, tied_lg)
        print(f"\n  untied lm_head: logits relDiff {r:.2e} (vs the tied head: {r_tied:.2e})")
        assert r < TOL
        assert r_tied > 0.1
    finally:
        ctx.lib.gd_stack_destroy(a)
        if b:
            ctx.lib.gd_stack_destroy(b)


@pytest.mark.parametrize("case", ["missing", "type", "shape", "conv"])
def test_gguf_rejects_bad_tensors(ctx, tmp_path, case):
    cfg, a = make_stack(ctx, seed=13)
    try:
        tensors = export(ctx, cfg, a)
    finally:
        ctx.lib.gd_stack_destroy(a)
    entries = W.stack_tensors(cfg, tensors)
    if case == "missing":
        entries = [e for e in entries if e[0] != "blk.1.ssm_alpha.weight"]
        msg = "missing tensor blk.1.ssm_alpha.weight"
    elif case == "type":
        entries = [(n, d, W.GGML_F16, r[:len(r) // 2]) if n == "blk.0.attn_norm.weight"
                   else (n, d, t, r) for n, d, t, r in entries]
        msg = "blk.0.attn_norm.weight must be f32"
    elif case == "shape":
        entries = [(n, [d[0], d[1] - 1], t, r[:len(r) - len(r) // d[1]])
                   if n == "blk.3.attn_k.weight" else (n, d, t, r) for n, d, t, r in entries]
        msg = "blk.3.attn_k.weight must be Q2_0"
    else:
        entries = [(n, [d[1], d[0]], t, r) if n == "blk.2.ssm_conv1d.weight" else (n, d, t, r)
                   for n, d, t, r in entries]
        msg = "blk.2.ssm_conv1d.weight must be"
    path = W.write(tmp_path / f"{case}.gguf", W.stack_kvs(cfg), entries)
    with pytest.raises(ga.GDError, match=msg):
        h = load(ctx, path, cfg)
        ctx.lib.gd_stack_destroy(h)
