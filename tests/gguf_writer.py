"""Minimal GGUF v3 writer for the tests: the layout the reference's reader
parses (LLM/src/Shared/GGUF.swift:45-99) -- magic "GGUF", u32 version, u64
tensor and metadata counts, metadata as (string key, u32 type, value),
tensor directory as (name, u32 n_dims, u64 dims ne0 first, u32 ggml type,
u64 offset), then tensor data from the first multiple of the alignment.

Also builds the qwen35 file of a stack: the metadata keys BonsaiConfig reads
(Model.swift:39-69) and the tensor names BonsaiLayer / BonsaiModel look up
(Model.swift:100-145).
"""
from __future__ import annotations

import struct
from pathlib import Path

import numpy as np

# GGUF metadata value types.
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
        BOOL: "<B", U64: "<Q", I64: "<q", F64: "<d"}

# ggml tensor types used here.
GGML_F32, GGML_F16, GGML_Q2_0 = 0, 1, 42


def _str(s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _scalar(t: int, v) -> bytes:
    if t == STR:
        return _str(v)
    return struct.pack(_FMT[t], v)


def encode_kv(key: str, t: int, v) -> bytes:
    """One metadata entry; an array is t=ARR with v=(element type, values)."""
    out = _str(key) + struct.pack("<I", t)
    if t == ARR:
        et, vals = v
        out += struct.pack("<IQ", et, len(vals)) + b"".join(_scalar(et, x) for x in vals)
    else:
        out += _scalar(t, v)
    return out


def encode(kvs, tensors, alignment: int = 32, version: int = 3) -> bytes:
    """kvs: [(key, type, value)]; tensors: [(name, dims, ggml type, bytes)].
    Each tensor's offset is the running data size rounded up to `alignment`."""
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs))
    head += b"".join(encode_kv(*kv) for kv in kvs)
    data = b""
    for name, dims, ty, raw in tensors:
        off = -len(data) % alignment
        data += b"\0" * off
        head += _str(name) + struct.pack("<I", len(dims))
        head += b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", ty, len(data))
        data += bytes(raw)
    head += b"\0" * (-len(head) % alignment)
    return head + data


def write(path: Path | str, kvs, tensors, alignment: int = 32, version: int = 3) -> Path:
    path = Path(path)
    path.write_bytes(encode(kvs, tensors, alignment, version))
    return path


def stack_kvs(cfg: dict, arch: str | None = None, drop=()) -> list:
    """The metadata BonsaiConfig reads for a stack of geometry cfg (the
    gd_stack_config field names): "qwen35" keys, or for cfg["dense"] the
    dense lineage's "qwen3" keys, which have no ssm geometry, no attention
    interval and no rope.dimension_count (Model.swift:45-59).  Keys named in
    `drop` are left out."""
    dense = bool(cfg.get("dense"))
    arch = arch or ("qwen3" if dense else "qwen35")
    a = arch + "."
    kvs = [("general.architecture", STR, arch),
           (a + "embedding_length", U32, cfg["n_embd"]),
           (a + "feed_forward_length", U32, cfg["n_ff"]),
           (a + "block_count", U32, cfg["n_layer"]),
           (a + "attention.head_count", U32, cfg["n_head"]),
           (a + "attention.head_count_kv", U32, cfg["n_head_kv"]),
           (a + "attention.key_length", U32, cfg["head_dim"]),
           (a + "attention.value_length", U32, cfg["head_dim"]),
           (a + "rope.freq_base", F32, cfg["rope_base"]),
           (a + "attention.layer_norm_rms_epsilon", F32, cfg["eps"])]
    if dense:
        assert cfg["n_rot"] == cfg["head_dim"], "the dense file rotates whole heads"
        return [kv for kv in kvs if kv[0] not in drop]
    kvs += [(a + "rope.dimension_count", U32, cfg["n_rot"]),
            (a + "rope.dimension_sections", ARR, (I32, [11, 11, 10, 0])),
            (a + "full_attention_interval", U32, cfg["attn_interval"]),
            (a + "ssm.state_size", U32, cfg["d_state"]),
            (a + "ssm.group_count", U32, cfg["n_k_head"]),
            (a + "ssm.time_step_rank", U32, cfg["n_v_head"]),
            (a + "ssm.inner_size", U32, cfg["d_state"] * cfg["n_v_head"]),
            (a + "ssm.conv_kernel", U32, cfg["d_conv"])]
    return [kv for kv in kvs if kv[0] not in drop]


def gguf_name(layer: int, name: str) -> str:
    """The file's name of a stack tensor (Model.swift:100-145)."""
    s = name if layer < 0 else f"blk.{layer}.{name}"
    if name == "ssm_dt":
        return s + ".bias"
    if name == "ssm_a":
        return s
    return s + ".weight"


def stack_tensors(cfg: dict, tensors: dict) -> list:
    """Directory entries of a stack's tensors.  tensors maps the reader's
    (layer, short name) to either Q2_0 block bytes of shape [rows][K/128*34]
    (a uint8 array) or an f32 array; conv1d is [conv_dim][d_conv]."""
    out = []
    for (layer, name), arr in tensors.items():
        arr = np.ascontiguousarray(arr)
        if arr.dtype == np.uint8:
            rows = arr.shape[0]
            k = arr.shape[1] // 34 * 128
            out.append((gguf_name(layer, name), [k, rows], GGML_Q2_0, arr.tobytes()))
        elif name == "ssm_conv1d":
            out.append((gguf_name(layer, name), [arr.shape[1], arr.shape[0]], GGML_F32,
                        arr.astype(np.float32).tobytes()))
        else:
            out.append((gguf_name(layer, name), [arr.size], GGML_F32,
                        arr.astype(np.float32).tobytes()))
    return out
