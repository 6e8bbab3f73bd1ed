"""The library's GGUF v3 reader (gd_gguf_*, host only, no device): metadata of
every value type, tensor placement under the default and a custom alignment,
the qwen35 and qwen3 geometries BonsaiConfig reads, and corrupt files as
errors.  Follows
LLM/src/Shared/GGUF.swift:45-284 and Model.swift:39-69."""
import struct

import numpy as np
import pytest

import gadeon_amd as ga
from tests import gguf_writer as W

STACK_CFG = dict(n_layer=4, n_embd=256, n_ff=384, n_head=4, n_head_kv=2, head_dim=128,
                 n_rot=64, rope_base=1e7, eps=1e-6, n_vocab=512, attn_interval=4, d_state=128,
                 n_k_head=2, n_v_head=4, d_conv=4)

KVS = [
    ("general.architecture", W.STR, "qwen35"),
    ("a.u8", W.U8, 250), ("a.i8", W.I8, -7), ("a.u16", W.U16, 65000), ("a.i16", W.I16, -30000),
    ("a.u32", W.U32, 4000000000), ("a.i32", W.I32, -2000000000), ("a.f32", W.F32, 1.5),
    ("a.bool", W.BOOL, 1), ("a.str", W.STR, "héllo"), ("a.u64", W.U64, 2 ** 63 + 5),
    ("a.i64", W.I64, -(2 ** 62)), ("a.f64", W.F64, 1e-300),
    ("a.ints", W.ARR, (W.I32, [11, 11, 10, 0])), ("a.bools", W.ARR, (W.BOOL, [1, 0, 1])),
    ("a.floats", W.ARR, (W.F32, [0.5, -2.0])), ("a.doubles", W.ARR, (W.F64, [1e100])),
    ("a.strs", W.ARR, (W.STR, ["x", "", "yz"])), ("a.empty", W.ARR, (W.U64, [])),
]


def tensors(rng):
    f = rng.standard_normal(6 * 5).astype(np.float32)
    q = rng.integers(0, 256, size=3 * 34 * 2, dtype=np.uint8)     # [3 rows][2 blocks]
    h = rng.standard_normal(7).astype(np.float16)
    return [("f", [6, 5], W.GGML_F32, f.tobytes()), ("q", [256, 3], W.GGML_Q2_0, q.tobytes()),
            ("h", [7], W.GGML_F16, h.tobytes())]


@pytest.fixture(scope="module")
def lib():
    return ga.load()


@pytest.mark.parametrize("alignment", [32, 64, 1])
def test_reads_every_value_type_and_tensor(tmp_path, lib, alignment):
    rng = np.random.default_rng(alignment)
    ts = tensors(rng)
    kvs = list(KVS)
    if alignment != 32:
        kvs.append(("general.alignment", W.U32, alignment))
    path = W.write(tmp_path / "a.gguf", kvs, ts, alignment=alignment)
    with ga.GGUF(path) as g:
        assert g.info() == (3, len(kvs), 3)
        assert g.string("general.architecture") == "qwen35"
        for key, t, v in KVS[1:]:
            if t in (W.U8, W.I8, W.U16, W.I16, W.U32, W.I32, W.I64):
                assert g.int(key) == v
            elif t == W.U64:
                assert g.int(key) % 2 ** 64 == v        # u64 reads as its int64 bit pattern
        assert g.float("a.f32") == 1.5 and g.float("a.f64") == 1e-300
        assert g.float("a.u8") == 250.0                 # integers read as doubles too
        assert g.bool("a.bool") is True and g.bool("a.u8") is True
        with pytest.raises(ga.GDError):
            g.int("a.bool")                             # GGUF.int does not read a bool
        assert g.string("a.str") == "héllo"
        assert g.ints("a.ints") == [11, 11, 10, 0] and g.ints("a.bools") == [1, 0, 1]
        assert g.floats("a.floats") == [0.5, -2.0] and g.floats("a.doubles") == [1e100]
        assert g.ints("a.empty") == []
        for name, dims, ty, raw in ts:
            d, t, data = g.tensor(name)
            assert d == tuple(dims) and t == ty and data.tobytes() == raw
            # Placement: the first multiple of the alignment after the directory.
            start = data.ctypes.data - g.tensor("f")[2].ctypes.data
            assert start % alignment == 0
        for bad in ("a.missing", "a.str"):
            with pytest.raises(ga.GDError):
                g.int(bad)
        with pytest.raises(ga.GDError, match="no tensor"):
            g.tensor("nope")


def test_data_start_follows_directory(tmp_path, lib):
    """Tensor bytes sit at align_up(end of directory) + offset: check the raw
    file position of each tensor against the writer's layout."""
    rng = np.random.default_rng(1)
    ts = tensors(rng)
    blob = W.encode(KVS, ts)
    path = tmp_path / "b.gguf"
    path.write_bytes(blob)
    with ga.GGUF(path) as g:
        base = g.tensor("f")[2].ctypes.data
        for name, _, _, raw in ts:
            pos = blob.find(raw)
            assert g.tensor(name)[2].ctypes.data - base == pos - blob.find(ts[0][3])
            assert pos % 32 == 0


def test_stack_config_from_metadata(tmp_path, lib):
    rng = np.random.default_rng(2)
    emb = rng.integers(0, 256, size=(STACK_CFG["n_vocab"], 2 * 34), dtype=np.uint8)
    ts = [("token_embd.weight", [256, STACK_CFG["n_vocab"]], W.GGML_Q2_0, emb.tobytes())]
    path = W.write(tmp_path / "c.gguf", W.stack_kvs(STACK_CFG), ts)
    with ga.GGUF(path) as g:
        c = g.stack_config()
    for k, v in STACK_CFG.items():
        assert getattr(c, k) == pytest.approx(v, rel=1e-7), k
    assert (c.kv_block, c.max_ctx, c.max_batch) == (0, 0, 0)
    # Defaults (Model.swift:48, 61): no rope.dimension_count -> head_dim, no
    # full_attention_interval -> 4.
    drop = ("qwen35.rope.dimension_count", "qwen35.full_attention_interval")
    cfg = dict(STACK_CFG, attn_interval=3)
    path = W.write(tmp_path / "d.gguf", W.stack_kvs(cfg, drop=drop), ts)
    with ga.GGUF(path) as g:
        c = g.stack_config()
    assert c.n_rot == cfg["head_dim"] and c.attn_interval == 4


def test_dense_stack_config(tmp_path, lib):
    """general.architecture "qwen3": the dense lineage (Model.swift:41-59) --
    every layer attention, no ssm geometry read (none in the file), the whole
    head rotated when rope.dimension_count is absent."""
    cfg = dict(STACK_CFG, dense=1, attn_interval=1, d_state=0, n_k_head=0, n_v_head=0,
               d_conv=0, n_rot=128, rope_base=1e6)
    emb = np.zeros((cfg["n_vocab"], 2 * 34), np.uint8)
    ts = [("token_embd.weight", [256, cfg["n_vocab"]], W.GGML_Q2_0, emb.tobytes())]
    kvs = W.stack_kvs(cfg)
    assert not any(".ssm." in k or "rope.dimension_count" in k for k, _, _ in kvs)
    path = W.write(tmp_path / "dense.gguf", kvs, ts)
    with ga.GGUF(path) as g:
        c = g.stack_config()
    for k, v in cfg.items():
        assert getattr(c, k) == pytest.approx(v, rel=1e-7), k
    # An explicit rope.dimension_count is honoured on the dense lineage too.
    path = W.write(tmp_path / "dense_rot.gguf",
                   kvs + [("qwen3.rope.dimension_count", W.U32, 64)], ts)
    with ga.GGUF(path) as g:
        assert g.stack_config().n_rot == 64
    # The hybrid needs its ssm keys; a qwen35 file without them is rejected.
    path = W.write(tmp_path / "no_ssm.gguf", W.stack_kvs(cfg, arch="qwen35"), ts)
    with ga.GGUF(path) as g:
        with pytest.raises(ga.GDError, match="missing numeric key qwen35"):
            g.stack_config()


@pytest.mark.parametrize("case", ["arch", "missing", "inner", "width", "nonint"])
def test_stack_config_rejects(tmp_path, lib, case):
    rng = np.random.default_rng(3)
    emb = rng.integers(0, 256, size=(STACK_CFG["n_vocab"], 2 * 34), dtype=np.uint8)
    width = 384 if case == "width" else 256
    emb = np.zeros((STACK_CFG["n_vocab"], width // 128 * 34), np.uint8) if case == "width" else emb
    ts = [("token_embd.weight", [width, STACK_CFG["n_vocab"]], W.GGML_Q2_0, emb.tobytes())]
    kvs = W.stack_kvs(STACK_CFG, arch="llama" if case == "arch" else "qwen35",
                      drop=("qwen35.ssm.state_size",) if case == "missing" else ())
    if case == "inner":
        kvs = [(k, t, 1000 if k.endswith("inner_size") else v) for k, t, v in kvs]
    if case == "nonint":
        kvs = [(k, W.F32 if k.endswith("block_count") else t, 2.5 if k.endswith("block_count")
                else v) for k, t, v in kvs]
    path = W.write(tmp_path / "e.gguf", kvs, ts)
    msg = {"arch": "neither the qwen35", "missing": "state_size", "inner": "inner_size", "width": "width",
           "nonint": "positive integer"}[case]
    with ga.GGUF(path) as g:
        with pytest.raises(ga.GDError, match=msg):
            g.stack_config()


def test_corrupt_files_are_errors(tmp_path, lib):
    rng = np.random.default_rng(4)
    ts = tensors(rng)
    blob = W.encode(KVS, ts)
    p = tmp_path / "x.gguf"

    def opens(b: bytes) -> bool:
        p.write_bytes(b)
        try:
            ga.GGUF(p).close()
            return True
        except ga.GDError:
            return False

    assert opens(blob)
    # Every cut inside the header, directory or tensor data is an error.
    data_end = len(blob)
    for cut in list(range(0, 200)) + list(range(200, data_end, 7)):
        assert not opens(blob[:cut]), cut
    assert not opens(b"GGUX" + blob[4:])                              # magic
    assert not opens(blob[:4] + struct.pack("<I", 1) + blob[8:])      # v1 layout
    assert not opens(blob[:8] + struct.pack("<Q", 2 ** 40) + blob[16:])   # tensor count
    # An unknown metadata type.
    bad = W.encode([("k", W.U8, 1)], [])
    i = bad.find(b"k") + 1
    assert not opens(bad[:i] + struct.pack("<I", 13) + bad[i + 4:])
    # A tensor type outside GGUFType, a tensor past the end, a bad n_dims.
    for mut in (lambda t: (t[0], t[1], 5, t[3]),):
        assert not opens(W.encode(KVS, [mut(ts[0])] + ts[1:]))
    assert not opens(W.encode(KVS, [("f", [6, 5000], W.GGML_F32, ts[0][3])]))
    assert not opens(W.encode(KVS, [("q", [100, 3], W.GGML_Q2_0, ts[1][3])]))  # not whole blocks
    assert not opens(W.encode(KVS, [("f", [1, 1, 1, 1, 30], W.GGML_F32, ts[0][3])]))
    # An array whose count the rest of the file cannot hold (2^40 u8 elements,
    # 2^37 strings) is an error.
    arr = W.encode([("a", W.ARR, (W.U8, [1, 2, 3]))], [])
    i = arr.find(b"a") + 1 + 4 + 4                                  # past key, type, elem type
    assert not opens(arr[:i] + struct.pack("<Q", 2 ** 40) + arr[i + 8:])
    arr = W.encode([("a", W.ARR, (W.STR, ["x"]))], [])
    i = arr.find(b"a") + 1 + 4 + 4
    assert not opens(arr[:i] + struct.pack("<Q", 2 ** 37) + arr[i + 8:])
    # Nonexistent path.
    with pytest.raises(ga.GDError, match="cannot open"):
        ga.GGUF(tmp_path / "absent.gguf")


def test_views_keep_the_mapping(tmp_path, lib):
    """A tensor view outlives close(): the mapping stays until the last view
    (and every array sliced from it) is gone; reads through the object
    itself are refused once it is closed."""
    import gc
    rng = np.random.default_rng(5)
    ts = tensors(rng)
    path = W.write(tmp_path / "v.gguf", list(KVS), ts)
    g = ga.GGUF(path)
    _, _, q = g.tensor("q")
    part = q[34:68]
    del q
    g.close()
    gc.collect()
    assert g.mapped
    assert part.tobytes() == ts[1][3][34:68]
    with pytest.raises(ga.GDError, match="closed"):
        g.tensor("f")
    del part
    gc.collect()
    assert not g.mapped
    with ga.GGUF(path) as g2:                  # no view taken: unmapped at exit
        g2.info()
    assert not g2.mapped
