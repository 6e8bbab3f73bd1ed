"""The C-ABI library loads without a GPU, exports every function the header
declares, and its host-only codec is the exact inverse of the reference's
Q2_0 decoder (Quant.swift:15-30)."""
import re
from pathlib import Path

import numpy as np

import gadeon_amd as ga

ROOT = Path(__file__).resolve().parents[1]


def declared_functions():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(gd_[a-z0-9_]+)\s*\(", text))
    return names


def test_library_exports_every_declared_symbol():
    lib = ga.load()
    names = declared_functions()
    assert len(names) > 30
    for n in sorted(names):
        assert hasattr(lib, n), n
    assert names == set(ga.exported_names())


def test_no_device_is_an_error_not_a_crash():
    if ga.device_count() > 0:
        return
    import ctypes as C
    lib = ga.load()
    h = C.c_void_p()
    assert lib.gd_ctx_create(0, C.byref(h)) == ga.GD_ENODEV
    assert b"device" in lib.gd_last_error(None)


def test_codec_all_byte_values():
    lib = ga.load()
    blocks = np.zeros((2, 34), np.uint8)
    blocks[0, 2:] = np.arange(32)
    blocks[1, 2:] = np.arange(32, 64) + 192       # cover 0..255 across the two
    blocks[0, :2] = [0x00, 0x3C]                  # d = 1.0
    codes = np.empty(256, np.uint8)
    scales = np.empty(2, np.uint16)
    full = np.zeros((8, 34), np.uint8)
    full[:, 2:] = np.arange(256, dtype=np.uint8).reshape(8, 32)
    codes = np.empty(1024, np.uint8)
    scales = np.empty(8, np.uint16)
    assert lib.gd_q2_0_unpack(full.ctypes.data, 1024, codes.ctypes.data, scales.ctypes.data) == 0
    byte_vals = np.arange(256)
    want = np.stack([(byte_vals >> (2 * j)) & 3 for j in range(4)], -1).ravel()
    assert np.array_equal(codes, want)


def test_codec_round_trip():
    lib = ga.load()
    rng = np.random.default_rng(1)
    n = 128 * 37
    codes = rng.integers(0, 4, n).astype(np.uint8)
    scales = rng.standard_normal(n // 128).astype(np.float16).view(np.uint16)
    blocks = np.empty(n // 128 * 34, np.uint8)
    assert lib.gd_q2_0_pack(codes.ctypes.data, scales.ctypes.data, n, blocks.ctypes.data) == 0
    c2 = np.empty_like(codes)
    s2 = np.empty_like(scales)
    assert lib.gd_q2_0_unpack(blocks.ctypes.data, n, c2.ctypes.data, s2.ctypes.data) == 0
    assert np.array_equal(c2, codes) and np.array_equal(s2, scales)
    b2 = np.empty_like(blocks)
    assert lib.gd_q2_0_pack(c2.ctypes.data, s2.ctypes.data, n, b2.ctypes.data) == 0
    assert np.array_equal(b2, blocks)
    # Scale first, little-endian; code j of a block at qs[j>>2] bits 2*(j&3).
    b = blocks.reshape(-1, 34)
    assert np.array_equal(b[:, 0] | (b[:, 1].astype(np.uint16) << 8), scales)
    assert (b[0, 2] & 3) == codes[0] and ((b[0, 2] >> 6) & 3) == codes[3]


def test_codec_rejects_bad_input():
    lib = ga.load()
    codes = np.full(128, 4, np.uint8)
    scales = np.zeros(1, np.uint16)
    out = np.empty(34, np.uint8)
    assert lib.gd_q2_0_pack(codes.ctypes.data, scales.ctypes.data, 128, out.ctypes.data) == ga.GD_EINVAL
    assert lib.gd_q2_0_pack(codes.ctypes.data, scales.ctypes.data, 100, out.ctypes.data) == ga.GD_EINVAL
