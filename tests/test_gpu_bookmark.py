"""Bookmarks of the stack's generation state: MetalEngine.bookmark / restore /
serialize / deserialize (MetalEngine.swift:455-584).

  * bookmark, decode, restore, decode again: bit-identical logits and picks,
    and generate from a restored bookmark continues from its pick;
  * a bookmark outlives a reset and a different prompt (its K/V are its own);
  * serialize writes MetalEngine.serialize's bytes (checked field by field
    against the stack's own state), deserialize into a fresh stack of the
    same weights continues bit-identically, and re-serializing gives the same
    bytes;
  * malformed bytes and bookmarks of another geometry are errors."""
import ctypes as C
import struct

import numpy as np
import pytest

import gadeon_amd as ga
from test_gpu_stack import CFG, DENSE, make_stack, tensor_reader

pytestmark = pytest.mark.gpu


def bookmark(ctx, st):
    h = C.c_void_p()
    ctx.check(ctx.lib.gd_stack_bookmark(st, C.byref(h)))
    return h


def serialize(ctx, st, bm) -> bytes:
    n = C.c_size_t()
    ctx.check(ctx.lib.gd_stack_serialize(st, bm, None, 0, C.byref(n)))
    buf = (C.c_uint8 * n.value)()
    ctx.check(ctx.lib.gd_stack_serialize(st, bm, buf, n.value, C.byref(n)))
    return bytes(buf)


def deserialize(ctx, st, data: bytes):
    h = C.c_void_p()
    buf = (C.c_uint8 * len(data)).from_buffer_copy(data)
    ctx.check(ctx.lib.gd_stack_deserialize(st, buf, len(data), C.byref(h)))
    return h


def prefill(ctx, st, ids):
    nxt = C.c_int32()
    ctx.check(ctx.lib.gd_stack_prefill(st, ids.ctypes.data, ids.size, C.byref(nxt), None))
    return nxt.value


def decode_run(ctx, st, tokens):
    """Decode each of `tokens`; returns (logits list, picks)."""
    lg = np.empty(CFG["n_vocab"], np.float32)
    nxt = C.c_int32()
    out, picks = [], []
    for t in tokens:
        ctx.check(ctx.lib.gd_stack_decode(st, int(t), C.byref(nxt), lg.ctypes.data))
        out.append(lg.copy())
        picks.append(nxt.value)
    return out, picks


def position(ctx, st):
    p = C.c_int64()
    ctx.check(ctx.lib.gd_stack_position(st, C.byref(p)))
    return p.value


def same(a, b):
    return len(a) == len(b) and all(np.array_equal(x, y) for x, y in zip(a, b))


def test_bookmark_restore_repeats_decode(ctx):
    cfg, st = make_stack(ctx, seed=21)
    bm = None
    try:
        ids = (np.arange(40) * 37 % cfg["n_vocab"]).astype(np.int32)
        first = prefill(ctx, st, ids)
        bm = bookmark(ctx, st)
        toks = [first, 5, 77, 300, 9]
        l1, p1 = decode_run(ctx, st, toks)
        ctx.check(ctx.lib.gd_stack_restore(st, bm))
        assert position(ctx, st) == ids.size
        l2, p2 = decode_run(ctx, st, toks)
        assert same(l1, l2) and p1 == p2
        # Generate from the restored pick equals chaining decode on the picks.
        ctx.check(ctx.lib.gd_stack_restore(st, bm))
        gen = np.empty(4, np.int32)
        ctx.check(ctx.lib.gd_stack_generate(st, 4, gen.ctypes.data))
        ctx.check(ctx.lib.gd_stack_restore(st, bm))
        chain = []
        t = first
        for _ in range(4):
            _, (t,) = decode_run(ctx, st, [t])
            chain.append(t)
        assert list(gen) == chain
        print(f"\n  restore: 5 decode steps bit-identical, generate {list(gen)}")
    finally:
        if bm:
            ctx.lib.gd_bookmark_free(bm)
        ctx.lib.gd_stack_destroy(st)


def test_bookmark_outlives_reset(ctx):
    cfg, st = make_stack(ctx, seed=22)
    bm = None
    try:
        a = (np.arange(45) * 11 % cfg["n_vocab"]).astype(np.int32)
        first = prefill(ctx, st, a)
        bm = bookmark(ctx, st)
        l1, p1 = decode_run(ctx, st, [first, 3, 4])
        ctx.check(ctx.lib.gd_stack_reset(st))
        prefill(ctx, st, (np.arange(60) * 29 % cfg["n_vocab"]).astype(np.int32))
        ctx.check(ctx.lib.gd_stack_restore(st, bm))
        l2, p2 = decode_run(ctx, st, [first, 3, 4])
        assert same(l1, l2) and p1 == p2
    finally:
        if bm:
            ctx.lib.gd_bookmark_free(bm)
        ctx.lib.gd_stack_destroy(st)


def parse(data: bytes, cfg):
    """MetalEngine.deserialize's reading order (MetalEngine.swift:515-540)."""
    p = 0

    def i64():
        nonlocal p
        v, = struct.unpack_from("<q", data, p)
        p += 8
        return v

    def floats():
        nonlocal p
        n = i64()
        a = np.frombuffer(data, np.float32, n, p)
        p += 4 * n
        return a

    pos, shift = i64(), i64()
    conv = {}
    for _ in range(i64()):
        il = i64()
        conv[il] = floats()
    rec = {}
    for _ in range(i64()):
        il = i64()
        rec[il] = floats()
    kv = {}
    for _ in range(i64()):
        il, n = i64(), i64()
        kv[il] = (n, floats(), floats())
    assert p == len(data)
    return pos, shift, conv, rec, kv


@pytest.mark.parametrize("dense", [False, True])
def test_serialize_format_and_round_trip(ctx, dense):
    """dense: the qwen3 lineage's bookmark has empty conv and rec dictionaries
    and a K/V entry for every layer."""
    over = DENSE if dense else {}
    cfg, st = make_stack(ctx, seed=23, **over)
    _, st2 = make_stack(ctx, seed=23, **over)
    bm = bm2 = None
    try:
        ids = (np.arange(37) * 13 % cfg["n_vocab"]).astype(np.int32)   # a partial KV page
        first = prefill(ctx, st, ids)
        bm = bookmark(ctx, st)
        data = serialize(ctx, st, bm)
        pos, shift, conv, rec, kv = parse(data, cfg)
        assert pos == ids.size and shift == 0
        gdn = [il for il in range(cfg["n_layer"]) if (il + 1) % cfg["attn_interval"]]
        att = [il for il in range(cfg["n_layer"]) if not (il + 1) % cfg["attn_interval"]]
        assert list(conv) == gdn and list(rec) == gdn and list(kv) == att
        read = tensor_reader(ctx, st)
        for il in gdn:
            assert np.array_equal(conv[il], read(il, "ssm_conv_state"))
            assert np.array_equal(rec[il], read(il, "ssm_state"))
        kv_dim = cfg["n_head_kv"] * cfg["head_dim"]
        for il in att:
            n, k, v = kv[il]
            assert n == ids.size and k.size == v.size == n * kv_dim
            # Widened halves: exactly representable in f16, and not all zero.
            for a in (k, v):
                assert np.array_equal(a.astype(np.float16).astype(np.float32), a)
                assert np.count_nonzero(a) > a.size // 2
        # Into a fresh stack of the same weights: the same continuation.
        bm2 = deserialize(ctx, st2, data)
        ctx.check(ctx.lib.gd_stack_restore(st2, bm2))
        assert position(ctx, st2) == ids.size
        gen = np.empty(2, np.int32)
        with pytest.raises(ga.GDError, match="no previous pick"):
            ctx.check(ctx.lib.gd_stack_generate(st2, 2, gen.ctypes.data))
        toks = [first, 17, 2, 250]
        l1, p1 = decode_run(ctx, st, toks)
        l2, p2 = decode_run(ctx, st2, toks)
        assert same(l1, l2) and p1 == p2
        assert serialize(ctx, st2, bm2) == data
        print(f"\n  serialized {len(data)} bytes at position {pos}; fresh stack continues "
              "bit-identically")
    finally:
        for b in (bm, bm2):
            if b:
                ctx.lib.gd_bookmark_free(b)
        ctx.lib.gd_stack_destroy(st)
        ctx.lib.gd_stack_destroy(st2)


def test_deserialize_rejects_malformed(ctx):
    cfg, st = make_stack(ctx, seed=24)
    _, other = make_stack(ctx, seed=24, n_v_head=2, n_k_head=2)
    bm = None
    try:
        prefill(ctx, st, (np.arange(20) * 7 % cfg["n_vocab"]).astype(np.int32))
        bm = bookmark(ctx, st)
        data = serialize(ctx, st, bm)
        small = C.c_uint8 * 16
        n = C.c_size_t()
        assert ctx.lib.gd_stack_serialize(st, bm, small(), 16, C.byref(n)) == ga.GD_EINVAL

        def bad(b: bytes, msg: str):
            with pytest.raises(ga.GDError, match=msg):
                deserialize(ctx, st, b)

        for cut in (0, 7, 8, 16, 24, 40, len(data) // 2, len(data) - 4):
            bad(data[:cut], "gd_stack_deserialize")
        bad(data + b"\0" * 4, "trailing")
        bad(struct.pack("<q", 1) + data[:8] + data[16:], "ropeShift")       # pos 20 -> shift
        bad(struct.pack("<q", 10 ** 9) + data[8:], "position")
        # The first conv entry names layer 1 instead of 0.
        bad(data[:24] + struct.pack("<q", 1) + data[32:], "GDN layer 1")
        # The first conv run claims one float fewer.
        cnt, = struct.unpack_from("<q", data, 32)
        bad(data[:32] + struct.pack("<q", cnt - 1) + data[40:], "bad count")
        # Another geometry's bookmark does not restore here.
        with pytest.raises(ga.GDError, match="geometry"):
            ctx.check(ctx.lib.gd_stack_restore(other, bm))
    finally:
        if bm:
            ctx.lib.gd_bookmark_free(bm)
        ctx.lib.gd_stack_destroy(st)
        ctx.lib.gd_stack_destroy(other)
