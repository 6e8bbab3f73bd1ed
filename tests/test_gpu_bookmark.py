"""Bookmarks of the stack's generation state: MetalEngine.bookmark / restore /
serialize / deserialize (MetalEngine.swift:455-584).

  * bookmark, decode, restore, decode again: bit-identical logits and picks,
    and generate from a restored bookmark continues from its pick;
  * a bookmark outlives a reset and a different prompt, and the stack it came
    from; it shares the completed KV pages and holds a copy of the partial
    tail page only;
  * serialize writes MetalEngine.serialize's bytes (checked field by field
    against the stack's own state), deserialize into a fresh stack of the
    same weights continues bit-identically, and re-serializing gives the same
    bytes;
  * malformed bytes and bookmarks of another geometry are errors;
  * the CPU engine's parked-state bytes, BonsaiEngine.serialize through
    StateBytes ("GDNS", BonsaiEngine.swift:65-112): written field by field
    from the bookmark, with 512-position KV pages across a page boundary; read
    back bit-identically; a state built from the CPU oracle's own conv rings,
    recurrent states and K/V resumes on the GPU stack and continues within
    the stack tolerance of the oracle; malformed headers, versions, pages and
    truncations are errors."""
import ctypes as C
import struct

import numpy as np
import pytest

import gadeon_amd as ga
import oracle as O
from conftest import rel_diff
from test_gpu_stack import CFG, DENSE, THREADS, TOL, make_stack, tensor_reader

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


def kv_pages(ctx, st):
    live, held, cap = C.c_int64(), C.c_int64(), C.c_int64()
    ctx.check(ctx.lib.gd_stack_kv_pages(st, C.byref(live), C.byref(held), C.byref(cap)))
    return live.value, held.value, cap.value


def test_bookmark_shares_kv_pages(ctx):
    """KV pages are shared, not copied (MetalKVPool.snapshot / restore,
    MetalKVPool.swift:95-120): a bookmark at position 1000 (62 full pages of
    16 and a partial one) takes one page -- its copy of the partial tail --
    and a restore one more -- the live state's own tail -- while the pool
    grew from 10 pages by doubling during the prefill.  The restored state
    continues bit-identically: in the same stack, after a reset and another
    prompt have reused the freed pages, and in a second stack (pages copied
    between pools).  A bookmark on a page boundary takes no page."""
    cfg, st = make_stack(ctx, seed=23, max_ctx=1104, max_batch=64)
    st2 = bm = bm2 = None
    try:
        live, held, cap = kv_pages(ctx, st)
        assert (live, held, cap) == (0, 0, 10)
        ids = (np.arange(1000) * 31 % cfg["n_vocab"]).astype(np.int32)
        first = prefill(ctx, st, ids)
        live, held, cap = kv_pages(ctx, st)
        assert live == 63 and held == 63 and 63 <= cap < 2 * 63 + 10
        bm = bookmark(ctx, st)
        assert kv_pages(ctx, st)[1] == 64                   # one tail page copied
        toks = [first, 5, 77, 300, 9]
        l1, p1 = decode_run(ctx, st, toks)
        ctx.check(ctx.lib.gd_stack_restore(st, bm))
        assert kv_pages(ctx, st)[:2] == (63, 64)            # the old tail freed, a new one taken
        l2, p2 = decode_run(ctx, st, toks)
        assert same(l1, l2) and p1 == p2
        # Another prompt on the freed pages; the shared ones stay the bookmark's.
        ctx.check(ctx.lib.gd_stack_reset(st))
        assert kv_pages(ctx, st)[:2] == (0, 63)
        prefill(ctx, st, (np.arange(300) * 7 % cfg["n_vocab"]).astype(np.int32))
        ctx.check(ctx.lib.gd_stack_restore(st, bm))
        l3, p3 = decode_run(ctx, st, toks)
        assert same(l1, l3) and p1 == p3
        # A second stack of the same weights: its own pool, pages copied in.
        _, st2 = make_stack(ctx, seed=23, max_ctx=1104, max_batch=64)
        ctx.check(ctx.lib.gd_stack_restore(st2, bm))
        assert kv_pages(ctx, st2)[:2] == (63, 63)
        l4, p4 = decode_run(ctx, st2, toks)
        assert same(l1, l4) and p1 == p4
        # On a page boundary nothing is copied.
        ctx.check(ctx.lib.gd_stack_reset(st2))
        prefill(ctx, st2, ids[:992])
        before = kv_pages(ctx, st2)[1]
        bm2 = bookmark(ctx, st2)
        assert kv_pages(ctx, st2)[1] == before == 62
        ctx.lib.gd_bookmark_free(bm)
        bm = None
        assert kv_pages(ctx, st)[1] == 63                   # the live state's pages only
        print(f"\n  KV pages: bookmark at 1000 held 1 extra page; pool capacity {cap}")
    finally:
        for b in (bm, bm2):
            if b:
                ctx.lib.gd_bookmark_free(b)
        ctx.lib.gd_stack_destroy(st)
        if st2:
            ctx.lib.gd_stack_destroy(st2)


def test_bookmark_restores_across_page_sizes(ctx):
    """A bookmark of a stack with 16-position KV pages restores into a stack
    of the same weights with 32-position pages (its positions re-paged) and
    continues bit-identically; serialized bytes do not depend on the page
    size."""
    cfg, st = make_stack(ctx, seed=25)
    st2 = bm = bm2 = None
    try:
        ids = (np.arange(57) * 9 % cfg["n_vocab"]).astype(np.int32)
        first = prefill(ctx, st, ids)
        bm = bookmark(ctx, st)
        l1, p1 = decode_run(ctx, st, [first, 21, 22])
        _, st2 = make_stack(ctx, seed=25, kv_block=32)
        ctx.check(ctx.lib.gd_stack_restore(st2, bm))
        assert kv_pages(ctx, st2)[:2] == (2, 2)            # 57 positions in pages of 32
        l2, p2 = decode_run(ctx, st2, [first, 21, 22])
        assert same(l1, l2) and p1 == p2
        ctx.check(ctx.lib.gd_stack_restore(st2, bm))
        bm2 = bookmark(ctx, st2)
        assert serialize(ctx, st2, bm2) == serialize(ctx, st, bm)
    finally:
        for b in (bm, bm2):
            if b:
                ctx.lib.gd_bookmark_free(b)
        ctx.lib.gd_stack_destroy(st)
        if st2:
            ctx.lib.gd_stack_destroy(st2)


def test_bookmark_outlives_its_stack(ctx):
    """A bookmark holds its pool: the stack it came from can be destroyed and
    the bookmark still restores into another stack bit-identically."""
    cfg, st = make_stack(ctx, seed=24)
    st2 = bm = None
    try:
        ids = (np.arange(70) * 5 % cfg["n_vocab"]).astype(np.int32)
        first = prefill(ctx, st, ids)
        bm = bookmark(ctx, st)
        l1, p1 = decode_run(ctx, st, [first, 11, 12])
        ctx.lib.gd_stack_destroy(st)
        st = None
        _, st2 = make_stack(ctx, seed=24)
        ctx.check(ctx.lib.gd_stack_restore(st2, bm))
        l2, p2 = decode_run(ctx, st2, [first, 11, 12])
        assert same(l1, l2) and p1 == p2
    finally:
        if bm:
            ctx.lib.gd_bookmark_free(bm)
        for s in (st, st2):
            if s:
                ctx.lib.gd_stack_destroy(s)


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
        bad(data[:8] + struct.pack("<q", 1 << 40) + data[16:], "ropeShift")   # out of range
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


def test_rope_shift_restored_from_bytes(ctx):
    """MetalEngine.serialize bytes whose ropeShift is nonzero (what MetalEngine
    keeps after an image span compressed the M-RoPE positions) restore with
    it: later tokens are rotated at position + shift while their K/V land at
    their position (MetalEngine.swift:432-435, 459-480).  Decoded against the
    oracle with the same shift, logits within the stack tolerance; the same
    tokens without the shift give clearly different logits.  The shift
    travels with bookmarks and bytes, GDNS bytes (no such field) refuse it,
    and a reset clears it.  A prefill chunk on the shifted state matches the
    oracle too."""
    cfg, st = make_stack(ctx, seed=29)
    _, st2 = make_stack(ctx, seed=29)
    bms = []
    try:
        read = tensor_reader(ctx, st)
        ref = O.Stack(cfg, read, stage_f16=True, threads=THREADS)
        ids = (np.arange(41) * 29 % cfg["n_vocab"]).astype(np.int32)
        prefill(ctx, st, ids)
        _, rlg = ref.prefill(ids)
        bms.append(bookmark(ctx, st))
        data = serialize(ctx, st, bms[-1])
        assert struct.unpack_from("<q", data, 8)[0] == 0
        shift = -13
        bms.append(deserialize(ctx, st2, data[:8] + struct.pack("<q", shift) + data[16:]))
        ctx.check(ctx.lib.gd_stack_restore(st2, bms[-1]))
        ref.rope_shift = shift
        tok, toks, got, worst = int(np.argmax(rlg)), [], [], 0.0
        for step in range(6):
            (glg,), _ = decode_run(ctx, st2, [tok])
            _, r_lg = ref.token(tok)
            r = rel_diff(glg, r_lg)
            worst = max(worst, r)
            assert r < TOL, (step, r)
            toks.append(tok)
            got.append(glg)
            tok = int(np.argmax(r_lg))
        unshifted, _ = decode_run(ctx, st, toks)
        apart = min(rel_diff(a, b) for a, b in zip(got, unshifted))
        assert apart > 10 * TOL, apart
        # A prefill chunk on the shifted state: the prefill attention rotates
        # its q, and prep its k, at position + shift as well.
        more = (np.arange(9) * 31 % cfg["n_vocab"]).astype(np.int32)
        lgp, nxt = np.empty(cfg["n_vocab"], np.float32), C.c_int32()
        ctx.check(ctx.lib.gd_stack_prefill(st2, more.ctypes.data, more.size, C.byref(nxt),
                                           lgp.ctypes.data))
        _, r_lgp = ref.prefill(more)
        rp = rel_diff(lgp, r_lgp)
        assert rp < TOL, rp
        bms.append(bookmark(ctx, st2))
        assert struct.unpack_from("<q", serialize(ctx, st2, bms[-1]), 8)[0] == shift
        n = C.c_size_t()
        with pytest.raises(ga.GDError, match="ropeShift"):
            ctx.check(ctx.lib.gd_stack_serialize_gdns(st2, bms[-1], None, 0, C.byref(n)))
        ctx.check(ctx.lib.gd_stack_reset(st2))
        bms.append(bookmark(ctx, st2))
        assert struct.unpack_from("<q", serialize(ctx, st2, bms[-1]), 8)[0] == 0
        print(f"\n  ropeShift {shift} restored: 6 decode steps, worst logits relDiff {worst:.2e} "
              f"(unshifted: at least {apart:.2e} apart); a 9-id prefill after them {rp:.2e}")
    finally:
        for b in bms:
            ctx.lib.gd_bookmark_free(b)
        ctx.lib.gd_stack_destroy(st)
        ctx.lib.gd_stack_destroy(st2)


# ---- the CPU engine's parked-state bytes (GDNS) --------------------------------

PAGE = 512      # KVCache.pageP (Attention.swift:16)


def serialize_gdns(ctx, st, bm) -> bytes:
    n = C.c_size_t()
    ctx.check(ctx.lib.gd_stack_serialize_gdns(st, bm, None, 0, C.byref(n)))
    buf = (C.c_uint8 * n.value)()
    ctx.check(ctx.lib.gd_stack_serialize_gdns(st, bm, buf, n.value, C.byref(n)))
    return bytes(buf)


def deserialize_gdns(ctx, st, data: bytes):
    h = C.c_void_p()
    buf = (C.c_uint8 * len(data)).from_buffer_copy(data)
    ctx.check(ctx.lib.gd_stack_deserialize_gdns(st, buf, len(data), C.byref(h)))
    return h


def parse_gdns(data: bytes):
    """BonsaiEngine.deserialize's reading order (BonsaiEngine.swift:89-112)."""
    assert data[:4] == b"GDNS"
    p = 4

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

    version, pos = i64(), i64()
    gdn = {}
    for _ in range(i64()):
        il = i64()
        conv = floats()
        gdn[il] = (conv, floats())
    kv = {}
    for _ in range(i64()):
        il, length, n = i64(), i64(), i64()
        kp = [floats() for _ in range(n)]
        vp = [floats() for _ in range(n)]
        kv[il] = (length, kp, vp)
    assert p == len(data)
    return version, pos, gdn, kv


def build_gdns(pos, gdn, kv, kv_dim, version=1) -> bytes:
    """BonsaiEngine.serialize (BonsaiEngine.swift:65-87) from arrays: gdn maps
    layer -> (conv, rec), kv maps layer -> (K, V) of shape [pos][kv_dim]."""
    out = [b"GDNS", struct.pack("<qq", version, pos), struct.pack("<q", len(gdn))]

    def run(a):
        a = np.ascontiguousarray(a, np.float32).reshape(-1)
        return struct.pack("<q", a.size) + a.tobytes()

    for il in sorted(gdn):
        out += [struct.pack("<q", il), run(gdn[il][0]), run(gdn[il][1])]
    out.append(struct.pack("<q", len(kv)))
    npages = (pos + PAGE - 1) // PAGE
    for il in sorted(kv):
        out.append(struct.pack("<qqq", il, pos, npages))
        for a in kv[il]:
            padded = np.zeros((npages * PAGE, kv_dim), np.float32)
            padded[:pos] = np.asarray(a, np.float32).reshape(pos, kv_dim)
            out += [run(padded[i * PAGE:(i + 1) * PAGE]) for i in range(npages)]
    return b"".join(out)


@pytest.mark.parametrize("dense", [False, True])
def test_gdns_format_and_round_trip(ctx, dense):
    """A 530-position state (two KV pages of 512): the GDNS bytes hold the
    bookmark's conv rings, states and K/V (the same values as MetalEngine's
    format, zero past the position), read back bit-identically, and continue
    the generation bit-identically in a fresh stack."""
    over = dict(DENSE if dense else {}, max_ctx=640, max_batch=128)
    cfg, st = make_stack(ctx, seed=26, **over)
    _, st2 = make_stack(ctx, seed=26, **over)
    bm = bm2 = None
    try:
        ids = (np.arange(530) * 19 % cfg["n_vocab"]).astype(np.int32)
        first = prefill(ctx, st, ids)
        bm = bookmark(ctx, st)
        data = serialize_gdns(ctx, st, bm)
        version, pos, gdn, kv = parse_gdns(data)
        assert version == 1 and pos == ids.size
        rec = [il for il in range(cfg["n_layer"]) if (il + 1) % cfg["attn_interval"]]
        att = [il for il in range(cfg["n_layer"]) if not (il + 1) % cfg["attn_interval"]]
        assert list(gdn) == rec and list(kv) == att
        read = tensor_reader(ctx, st)
        for il in rec:
            assert np.array_equal(gdn[il][0], read(il, "ssm_conv_state"))
            assert np.array_equal(gdn[il][1], read(il, "ssm_state"))
        # K/V against MetalEngine's format of the same bookmark.
        _, _, _, _, mkv = parse(serialize(ctx, st, bm), cfg)
        kv_dim = cfg["n_head_kv"] * cfg["head_dim"]
        for il in att:
            length, kp, vp = kv[il]
            assert length == pos and len(kp) == len(vp) == 2
            for pages, flat in ((kp, mkv[il][1]), (vp, mkv[il][2])):
                assert all(p.size == PAGE * kv_dim for p in pages)
                whole = np.concatenate(pages)
                assert np.array_equal(whole[:pos * kv_dim], flat)
                assert not whole[pos * kv_dim:].any()
        bm2 = deserialize_gdns(ctx, st2, data)
        assert serialize_gdns(ctx, st2, bm2) == data
        assert serialize(ctx, st2, bm2) == serialize(ctx, st, bm)
        ctx.check(ctx.lib.gd_stack_restore(st2, bm2))
        toks = [first, 7, 123, 9]
        l1, p1 = decode_run(ctx, st, toks)
        l2, p2 = decode_run(ctx, st2, toks)
        assert same(l1, l2) and p1 == p2
        print(f"\n  GDNS: {len(data)} bytes at position {pos}, two KV pages; fresh stack "
              "continues bit-identically")
    finally:
        for b in (bm, bm2):
            if b:
                ctx.lib.gd_bookmark_free(b)
        ctx.lib.gd_stack_destroy(st)
        ctx.lib.gd_stack_destroy(st2)


def test_gdns_resumes_a_cpu_parked_state(ctx):
    """The CPU oracle (BonsaiEngine.forward restated) runs a prompt; its own
    conv rings, recurrent states and K/V, written as BonsaiEngine.serialize
    bytes, are read into the GPU stack, which then decodes alongside the
    oracle: logits within the stack tolerance at every step."""
    cfg, st = make_stack(ctx, seed=27)
    bm = None
    try:
        read = tensor_reader(ctx, st)
        ref = O.Stack(cfg, read, stage_f16=True, threads=THREADS)
        ids = (np.arange(37) * 23 % cfg["n_vocab"]).astype(np.int32)
        _, lg = ref.prefill(ids)
        rec = [il for il in range(cfg["n_layer"]) if (il + 1) % cfg["attn_interval"]]
        att = [il for il in range(cfg["n_layer"]) if not (il + 1) % cfg["attn_interval"]]
        kv_dim = cfg["n_head_kv"] * cfg["head_dim"]
        data = build_gdns(ids.size,
                          {il: (ref.layer_state(il, "ssm_conv_state"),
                                ref.layer_state(il, "ssm_state")) for il in rec},
                          {il: (ref.layer_state(il, "k_cache"), ref.layer_state(il, "v_cache"))
                           for il in att}, kv_dim)
        bm = deserialize_gdns(ctx, st, data)
        ctx.check(ctx.lib.gd_stack_restore(st, bm))
        assert position(ctx, st) == ids.size
        tok = int(np.argmax(lg))
        worst = 0.0
        for step in range(6):
            (glg,), _ = decode_run(ctx, st, [tok])
            _, rlg = ref.token(tok)
            r = rel_diff(glg, rlg)
            worst = max(worst, r)
            assert r < TOL, (step, r)
            tok = int(np.argmax(rlg))
        print(f"\n  CPU-parked state resumed on the GPU: 6 decode steps, worst logits relDiff "
              f"{worst:.2e}")
    finally:
        if bm:
            ctx.lib.gd_bookmark_free(bm)
        ctx.lib.gd_stack_destroy(st)


def test_gdns_rejects_malformed(ctx):
    cfg, st = make_stack(ctx, seed=28)
    bm = None
    try:
        prefill(ctx, st, (np.arange(20) * 7 % cfg["n_vocab"]).astype(np.int32))
        bm = bookmark(ctx, st)
        data = serialize_gdns(ctx, st, bm)

        def bad(b: bytes, msg: str):
            with pytest.raises(ga.GDError, match=msg):
                deserialize_gdns(ctx, st, b)

        bad(data[:8], "no GDNS header")
        bad(b"GDNX" + data[4:], "no GDNS header")
        bad(serialize(ctx, st, bm), "no GDNS header")           # MetalEngine's format
        bad(data[:4] + struct.pack("<q", 2) + data[12:], "version 2")
        for cut in (12, 20, 28, len(data) // 2, len(data) - 4):
            bad(data[:cut], "gd_stack_deserialize_gdns")
        bad(data + b"\0" * 8, "trailing")
        bad(data[:12] + struct.pack("<q", 10 ** 9) + data[20:], "position")
        # The last attention layer's first K page claims one float fewer.
        kv_dim = cfg["n_head_kv"] * cfg["head_dim"]
        tail = 2 * (8 + PAGE * kv_dim * 4)                      # its K page and V page
        at = len(data) - tail
        cnt, = struct.unpack_from("<q", data, at)
        assert cnt == PAGE * kv_dim
        bad(data[:at] + struct.pack("<q", cnt - 1) + data[at + 8:], "K page 0")
    finally:
        if bm:
            ctx.lib.gd_bookmark_free(bm)
        ctx.lib.gd_stack_destroy(st)


def test_generate_across_pool_growth(ctx):
    """The KV pool grows (doubling) while a captured decode graph exists: the
    graph, which holds the pools' addresses, is captured again, and 70 greedy
    steps over the growth equal 70 chained decodes on a second stack."""
    cfg, st = make_stack(ctx, seed=26, max_batch=16, max_ctx=128)
    st2 = None
    try:
        _, st2 = make_stack(ctx, seed=26, max_batch=16, max_ctx=128)
        ids = (np.arange(40) * 17 % cfg["n_vocab"]).astype(np.int32)
        first = prefill(ctx, st, ids)
        assert prefill(ctx, st2, ids) == first
        cap0 = kv_pages(ctx, st)[2]
        assert cap0 == 4
        g1 = np.empty(10, np.int32)
        g2 = np.empty(60, np.int32)
        ctx.check(ctx.lib.gd_stack_generate(st, 10, g1.ctypes.data))
        assert kv_pages(ctx, st)[2] == cap0                 # 50 positions: no growth yet
        ctx.check(ctx.lib.gd_stack_generate(st, 60, g2.ctypes.data))
        live, held, cap = kv_pages(ctx, st)
        assert cap > cap0 and live == held == 7             # 110 positions
        chain, t = [], first
        for _ in range(70):
            _, (t,) = decode_run(ctx, st2, [t])
            chain.append(t)
        assert list(g1) + list(g2) == chain
    finally:
        ctx.lib.gd_stack_destroy(st)
        if st2:
            ctx.lib.gd_stack_destroy(st2)
