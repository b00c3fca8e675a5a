"""Minimal GGUF v3 writer (numpy arrays in, a Flint-loadable file out), for synthetic models:
the library's tests, the benchmark and users who want a small model file to try the
attention blocks with (include/flint_model.h). Host-side tooling; no GPU work.

File layout written: header (magic "GGUF", version 3, tensor count, key/value count), the
key/value section, the tensor infos, then the tensor data, each tensor aligned to
general.alignment (32 unless given), as /root/reference/src/gguf.cpp:137-194 reads it.
"""
import struct

import numpy as np

GGUF_U32, GGUF_F32, GGUF_BOOL, GGUF_STRING, GGUF_ARRAY = 4, 6, 7, 8, 9
T_F32, T_F16 = 0, 1


def _s(b):
    b = b.encode()
    return struct.pack("<Q", len(b)) + b


# metadata value types of the format and their scalar encodings
GGUF_U8, GGUF_I8, GGUF_U16, GGUF_I16, GGUF_I32, GGUF_U64, GGUF_I64, GGUF_F64 = 0, 1, 2, 3, 5, 10, 11, 12
_SCALAR = {GGUF_U8: "<B", GGUF_I8: "<b", GGUF_U16: "<H", GGUF_I16: "<h", GGUF_U32: "<I", GGUF_I32: "<i",
           GGUF_F32: "<f", GGUF_U64: "<Q", GGUF_I64: "<q", GGUF_F64: "<d"}


def _value(t, v):
    if t in _SCALAR:
        return struct.pack(_SCALAR[t], v)
    if t == GGUF_BOOL:
        return struct.pack("<B", 1 if v else 0)
    if t == GGUF_STRING:
        return _s(v)
    raise ValueError(t)


def write_gguf(path, meta, tensors, alignment=32):
    """Minimal GGUF v3 writer: meta = [(key, type, value)], tensors = [(name, np.ndarray, ggml_type)]
    with array dims in numpy order (outer first; ggml dims are reversed), or
    (name, uint8 rows, ggml_type, ggml dims) for data already in its on-disk encoding.
    An array value is (element type, list); a bare list is a bool array. A non-default
    alignment is also written as general.alignment."""
    if alignment != 32:
        meta = list(meta) + [("general.alignment", GGUF_U32, alignment)]
    out = bytearray()
    out += struct.pack("<IIQQ", 0x46554747, 3, len(tensors), len(meta))
    for key, t, v in meta:
        out += _s(key) + struct.pack("<I", t)
        if t == GGUF_ARRAY:
            et, items = v if isinstance(v, tuple) else (GGUF_BOOL, v)
            out += struct.pack("<IQ", et, len(items)) + b"".join(_value(et, x) for x in items)
        else:
            out += _value(t, v)
    blobs, off = [], 0
    for t in tensors:
        name, arr, gt = t[:3]
        if len(t) == 4:
            data, dims = np.ascontiguousarray(arr, np.uint8).tobytes(), list(t[3])
        else:
            data = arr.astype(np.float32 if gt == T_F32 else np.float16).tobytes()
            dims = list(reversed(arr.shape))
        out += _s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", gt, off)
        blobs.append(data)
        off += (len(data) + alignment - 1) // alignment * alignment
    pad = (-len(out)) % alignment
    with open(path, "wb") as f:
        f.write(out + b"\0" * pad)
        for d in blobs:
            f.write(d + b"\0" * ((-len(d)) % alignment))


def quantize_q8_0(w):
    """float32 rows [n][k] (k a multiple of 32) -> q8_0 blocks as uint8 rows [n][k/32*34]: per 32
    values, an fp16 scale d = max|x| / 127 and int8 q = round(x / d) (ggml's reference q8_0
    quantiser, block_q8_0 = {fp16 d; int8 qs[32]})."""
    w = np.ascontiguousarray(w, np.float32)
    n, k = w.shape
    x = w.reshape(n, k // 32, 32)
    d = np.abs(x).max(axis=2) / 127.0
    inv = np.where(d > 0, 1.0 / np.where(d > 0, d, 1.0), 0.0)
    q = np.clip(np.rint(x * inv[:, :, None]), -127, 127).astype(np.int8)
    blocks = np.concatenate([d.astype(np.float16).view(np.uint8).reshape(n, k // 32, 2), q.view(np.uint8)], axis=2)
    return blocks.reshape(n, k // 32 * 34)


def flint_meta(is_swa, has_rope, n_swa=513, rope_theta=1.0e4, rms_eps=1e-6, n_embd=2048):
    """The metadata HParams::from_gguf reads (/root/reference/src/ref/ref_model.cpp:13-39) for a
    Flint model with one leading dense block, one expert of one row and sigmoid routing."""
    a = "flint."
    return [
        ("general.architecture", GGUF_STRING, "flint"),
        (a + "block_count", GGUF_U32, len(is_swa)),
        (a + "embedding_length", GGUF_U32, n_embd),
        (a + "attention.head_count", GGUF_U32, 32),
        (a + "attention.head_count_kv", GGUF_U32, 4),
        (a + "attention.key_length", GGUF_U32, 128),
        (a + "feed_forward_length", GGUF_U32, 1),
        (a + "expert_feed_forward_length", GGUF_U32, 1),
        (a + "expert_shared_feed_forward_length", GGUF_U32, 1),
        (a + "expert_count", GGUF_U32, 1),
        (a + "expert_used_count", GGUF_U32, 1),
        (a + "leading_dense_block_count", GGUF_U32, 1),
        (a + "attention.sliding_window", GGUF_U32, n_swa),
        (a + "attention.layer_norm_rms_epsilon", GGUF_F32, rms_eps),
        (a + "rope.freq_base", GGUF_F32, rope_theta),
        (a + "attention.sliding_window_pattern", GGUF_ARRAY, [bool(x) for x in is_swa]),
        (a + "attention.rope_pattern", GGUF_ARRAY, [bool(x) for x in has_rope]),
        (a + "expert_gating_func", GGUF_U32, 2),
        (a + "expert_weights_norm", GGUF_BOOL, True),
        (a + "expert_weights_scale", GGUF_F32, 1.0),
    ]


def flint_zero_ffn(il, n_embd=2048):
    """Layer il's FFN tensors, all zero (f16): a dense FFN of width 1 for the leading block, else
    a router, one expert and a shared expert of width 1. A model built with them adds nothing
    in its FFN halves (ref_model.cpp:153-187), so its hidden state is its attention blocks'."""
    b, E = f"blk.{il}.", n_embd
    z = lambda *shape: np.zeros(shape, np.float32)  # noqa: E731
    t = [(b + "ffn_norm.weight", np.ones(E, np.float32), T_F32)]
    if il < 1:
        return t + [(b + "ffn_gate.weight", z(1, E), T_F16), (b + "ffn_up.weight", z(1, E), T_F16),
                    (b + "ffn_down.weight", z(E, 1), T_F16)]
    return t + [(b + "ffn_gate_inp.weight", z(1, E), T_F16), (b + "ffn_gate_exps.weight", z(1, 1, E), T_F16),
                (b + "ffn_up_exps.weight", z(1, 1, E), T_F16), (b + "ffn_down_exps.weight", z(1, E, 1), T_F16),
                (b + "ffn_gate_shexp.weight", z(1, E), T_F16), (b + "ffn_up_shexp.weight", z(1, E), T_F16),
                (b + "ffn_down_shexp.weight", z(E, 1), T_F16)]
