"""The attention blocks loaded from a GGUF model, on the CPU.

* The oracle's block forward (oracle.block_forward: rmsnorm + dequantised q/k/v matvecs +
  sink attention + o matvec + residual) against the reference's own CPU forward
  (RefModel::forward, /root/reference/src/ref/ref_model.cpp:95-187, compiled from its
  sources into oracle/_ref/ref_driver), bit for bit: tests/golden/block_vectors.json holds
  the sha256 of the reference's hidden states for a two-layer quantised model with zero FFN
  weights (tests/golden/make_block_vectors.py).
* The library's GGUF reader and hyper-parameter checks (flint_attn_model_open, flint_open)
  on defective files: each fails on the host, before any device work, with the message the
  reference's loader gives (/root/reference/src/gguf.cpp:137-194, 200-241;
  /root/reference/src/ref/ref_model.cpp:13-39).
"""
import ctypes
import json
import os
import struct

import numpy as np
import pytest

import flint_attn as fa
import oracle as fo
from golden import make_block_vectors as mb
from golden import make_ref_vectors as g

HERE = os.path.dirname(os.path.abspath(__file__))
VECTORS = json.load(open(os.path.join(HERE, "golden", "block_vectors.json")))


@pytest.fixture(scope="module")
def model():
    return mb.make_model(VECTORS["seed"], VECTORS["n_positions"])


@pytest.fixture(scope="module")
def model_file(model, tmp_path_factory):
    path = str(tmp_path_factory.mktemp("gguf") / "blocks.gguf")
    mb.write_model(path, model)
    return path


def test_oracle_blocks_bit_exact_vs_reference_forward(model):
    assert mb.model_sha(model) == VECTORS["model_sha256"], "model generator drifted"
    blocks = mb.oracle_blocks(model, "f32")  # RefModel keeps fp32 K/V
    hidden, _ = fo.block_forward(blocks, model["embd"].astype(np.float32), "f32")
    d = VECTORS["probe_dims"]
    for p, vals in VECTORS["probes"].items():
        assert np.array_equal(hidden[int(p), :d], np.array(vals, np.float32)), f"position {p}"
    assert g.sha(hidden) == VECTORS["hidden_sha256"]


def test_block_step_closed_forms(model):
    """A layer whose attn_output is zero leaves x unchanged; the residual is x + Wo att with
    att the attention oracle's output for the projected q|k|v."""
    blk = mb.oracle_blocks(model, "f16")[1]
    rng = np.random.default_rng(5)
    x = rng.standard_normal(2048).astype(np.float32)
    K = np.zeros((4, 512), np.float32)
    V = np.zeros((4, 512), np.float32)
    x1, att = fo.block_step(blk, x, 0, K, V)
    # position 0 attends to itself only: att = v * e^s0 / (e^s0 + e^sink) per head
    xn = fo.rmsnorm(x, blk.attn_norm)
    qkv = (blk.wqkv.astype(np.float64) @ xn.astype(np.float64)).astype(np.float32)
    q, k, v = fo.qkv_prep(blk.attn, qkv, 0)
    for h in (0, 9, 31):
        s = float(np.dot(q[h * 128:(h + 1) * 128].astype(np.float64), k[(h // 8) * 128:(h // 8 + 1) * 128]))
        s /= np.sqrt(128.0)
        w = 1.0 / (1.0 + np.exp(float(blk.attn.sinks[h]) - s))
        np.testing.assert_allclose(att[h * 128:(h + 1) * 128], w * v[(h // 8) * 128:(h // 8 + 1) * 128],
                                   rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(x1, x + blk.wo.astype(np.float64) @ att, rtol=1e-5, atol=1e-5)
    zero = fo.BlockLayer(blk.attn_norm, blk.wqkv[:4096], blk.wqkv[4096:4608], blk.wqkv[4608:],
                         np.zeros_like(blk.wo), blk.attn)
    x2, _ = fo.block_step(zero, x, 0, np.zeros((4, 512), np.float32), np.zeros((4, 512), np.float32))
    assert np.array_equal(x2, x)


def _err():
    return ctypes.create_string_buffer(512)


def model_open_error(path, n_ctx=256):
    err = _err()
    h = fa.lib().flint_attn_model_open(path.encode(), n_ctx, fa.KV_F16, err, len(err))
    assert not h, "open unexpectedly succeeded"
    return err.value.decode()


class _Cfg(ctypes.Structure):
    _fields_ = [("model_path", ctypes.c_char_p), ("metallib_dir", ctypes.c_char_p), ("pool_gb", ctypes.c_double),
                ("n_ctx", ctypes.c_int32)]


def capi_open_error(path):
    cfg = _Cfg(path.encode(), b".", 0.0, 256)
    err = _err()
    assert not fa.lib().flint_open(ctypes.cast(ctypes.pointer(cfg), ctypes.c_void_p), err, len(err))
    return err.value.decode()


def _drop(name):
    return lambda ts: [t for t in ts if t[0] != name]


def _q4k(name):
    """attn tensor stored as Q4_K (ggml type 12: 256 elements in 144 bytes), a format the
    reference has no attention kernel for."""
    def f(ts):
        return [(name, np.zeros((t[3][1], t[3][0] // 256 * 144), np.uint8), 12, t[3]) if t[0] == name else t
                for t in ts]
    return f


def _reshape(name, dims):
    def f(ts):
        out = []
        for t in ts:
            if t[0] == name:
                t = (name, np.zeros((dims[1], dims[0]), np.float32), g.T_F16)
            out.append(t)
        return out
    return f


CASES = [
    ("arch", {"general.architecture": (g.GGUF_STRING, "llama")}, None, "not a flint model: llama"),
    ("missing_key", {"flint.block_count": None}, None, "gguf: missing key flint.block_count"),
    ("routing", {"flint.expert_gating_func": (g.GGUF_U32, 1)}, None,
     "unexpected routing config (expect sigmoid + norm, scale 1)"),
    ("routing_scale", {"flint.expert_weights_scale": (g.GGUF_F32, 2.5)}, None,
     "unexpected routing config (expect sigmoid + norm, scale 1)"),
    ("key_type", {"flint.block_count": (g.GGUF_STRING, "two")}, None, "gguf: key flint.block_count has the wrong type"),
    ("no_output", None, _drop("output.weight"), "missing tensor output.weight"),
    ("pattern_short", {"flint.attention.rope_pattern": (g.GGUF_ARRAY, [False])}, None,
     "flint: the sliding-window and rope patterns need one entry per layer (2)"),
    ("n_embd", {"flint.embedding_length": (g.GGUF_U32, 4096)}, None, "unsupported attention shape"),
    ("heads", {"flint.attention.head_count_kv": (g.GGUF_U32, 8)}, None, "unsupported attention shape"),
    ("window", {"flint.attention.sliding_window": (g.GGUF_U32, 2000)}, None,
     "attention.sliding_window must be in [1, 1024]"),
]
# defects only the attention-block loader sees (flint_open stops after the hyper-parameters)
TENSOR_CASES = [
    ("missing_k", _drop("blk.1.attn_k.weight"), "missing tensor blk.1.attn_k.weight"),
    ("q4k", _q4k("blk.0.attn_q.weight"), "no kernel for type Q4_K (blk.0.attn_q.weight)"),
    ("shape", _reshape("blk.0.attn_v.weight", (2048, 256)), "tensor blk.0.attn_v.weight has the wrong shape"),
    ("norm_type", lambda ts: [(t[0], t[1], g.T_F16) if t[0] == "blk.1.attn_sinks.weight" else t for t in ts],
     "no kernel for type F16 (blk.1.attn_sinks.weight)"),
]


@pytest.mark.parametrize("name,meta,tens,msg", CASES, ids=[c[0] for c in CASES])
def test_loader_rejects_bad_hparams(model, tmp_path, name, meta, tens, msg):
    path = str(tmp_path / f"{name}.gguf")
    mb.write_model(path, model, meta_edit=meta, tensor_edit=tens)
    assert model_open_error(path).startswith(msg)
    assert capi_open_error(path).startswith(msg)


@pytest.mark.parametrize("name,tens,msg", TENSOR_CASES, ids=[c[0] for c in TENSOR_CASES])
def test_loader_rejects_bad_tensors(model, tmp_path, name, tens, msg):
    path = str(tmp_path / f"{name}.gguf")
    mb.write_model(path, model, tensor_edit=tens)
    assert model_open_error(path).startswith(msg)


def test_loader_file_errors(model_file, tmp_path):
    missing = str(tmp_path / "missing.gguf")
    assert model_open_error(missing) == "cannot open " + missing
    blob = open(model_file, "rb").read()
    bad = tmp_path / "magic.gguf"
    bad.write_bytes(b"GGML" + blob[4:64])
    assert model_open_error(str(bad)) == "not a GGUF file: " + str(bad)
    v2 = tmp_path / "v2.gguf"
    v2.write_bytes(blob[:4] + struct.pack("<I", 2) + blob[8:4096])
    assert model_open_error(str(v2)) == "unsupported GGUF version"
    for cut in (2, 20, 300, 2000):  # inside the header, the metadata and the tensor table
        t = tmp_path / f"cut{cut}.gguf"
        t.write_bytes(blob[:cut])
        assert model_open_error(str(t)) == "gguf: unexpected end of file", cut
    # tensor data cut short: the last tensor's bytes run past the end of the file
    short = tmp_path / "short.gguf"
    short.write_bytes(blob[:-4096])
    assert model_open_error(str(short)).startswith("tensor out of bounds: ")
    empty = tmp_path / "empty.gguf"
    empty.write_bytes(b"")
    assert model_open_error(str(empty)) == "gguf: unexpected end of file"


def test_loader_argument_checks(model_file):
    err = _err()
    assert not fa.lib().flint_attn_model_open(None, 256, fa.KV_F16, err, len(err))
    assert not fa.lib().flint_attn_model_open(model_file.encode(), 0, fa.KV_F16, err, len(err))
    assert "n_ctx" in err.value.decode()
    assert not fa.lib().flint_attn_model_open(model_file.encode(), 256, 7, err, len(err))
    assert "kv_dtype" in err.value.decode()
    L = fa.lib()
    L.flint_attn_model_close(None)
    assert not L.flint_attn_model_engine(None)
    hp = fa.HParams()
    assert L.flint_attn_model_hparams(None, ctypes.byref(hp), None, None) == -1
    assert L.flint_attn_model_block_decode(None, 0, None, 0, None, None, err, len(err)) == -1
    assert L.flint_attn_model_block_prefill(None, 0, None, 0, 1, None, None, err, len(err)) == -1
    assert L.flint_attn_model_embed(None, None, 0, None, None, err, len(err)) == -1
    assert L.flint_attn_model_pos(None) == 0 and L.flint_attn_model_n_ctx(None) == 0
    assert L.flint_attn_model_truncate(None, 0) == -1
    assert L.flint_attn_model_step(None, 0, None, None, err, len(err)) == -1
    assert L.flint_attn_model_prefill(None, None, 0, None, None, err, len(err)) == -1


def test_capi_open_valid_model_names_the_scope(model_file):
    msg = capi_open_error(model_file)
    assert "attention blocks only" in msg and "2-layer model" in msg


def _raw_meta_model(model, tmp_path, name, extra_meta=(), alignment=32, retype=None):
    """The block model with extra metadata entries (raw: any value type) and its tensors at the
    given data alignment; retype = {key: (type, value)} replaces a hyper-parameter's encoding."""
    import gguf_writer as gw
    meta = gw.flint_meta([L["is_swa"] for L in model["layers"]], [L["has_rope"] for L in model["layers"]], mb.N_SWA,
                         mb.THETA, mb.RMS_EPS)
    for key, (t, v) in (retype or {}).items():
        meta = [(k, t, v) if k == key else (k, tt, vv) for k, tt, vv in meta]
    path = str(tmp_path / f"{name}.gguf")
    captured = {}

    def grab(ts):
        captured["t"] = ts
        return ts
    mb.write_model(path, model, tensor_edit=grab)
    gw.write_gguf(path, meta + list(extra_meta), captured["t"], alignment=alignment)
    return path


def test_loader_reads_every_metadata_type(model, tmp_path):
    """Metadata of every GGUF value type, integer hyper-parameters in other integer widths, a
    float one in f64, and a 64-byte data alignment: the file parses and validates (the
    reference's get_int / get_float accept any integer / float width, gguf.cpp:206-213)."""
    import gguf_writer as gw
    extra = [("x.u8", gw.GGUF_U8, 200), ("x.i8", gw.GGUF_I8, -5), ("x.u16", gw.GGUF_U16, 60000),
             ("x.i16", gw.GGUF_I16, -300), ("x.i32", gw.GGUF_I32, -70000), ("x.u64", gw.GGUF_U64, 1 << 40),
             ("x.i64", gw.GGUF_I64, -(1 << 40)), ("x.f64", gw.GGUF_F64, 0.125), ("x.s", gw.GGUF_STRING, "tokens"),
             ("x.ai", gw.GGUF_ARRAY, (gw.GGUF_I32, [1, -2, 3])), ("x.af", gw.GGUF_ARRAY, (gw.GGUF_F32, [0.5, 1.5])),
             ("x.as", gw.GGUF_ARRAY, (gw.GGUF_STRING, ["a", "bc", ""])), ("x.ab", gw.GGUF_ARRAY, [True, False])]
    retype = {"flint.block_count": (gw.GGUF_U64, 2), "flint.attention.head_count": (gw.GGUF_I16, 32),
              "flint.rope.freq_base": (gw.GGUF_F64, mb.THETA)}
    path = _raw_meta_model(model, tmp_path, "types", extra, alignment=64, retype=retype)
    assert "attention blocks only" in capi_open_error(path) and "2-layer model" in capi_open_error(path)
    err = _err()
    h = fa.lib().flint_attn_model_open(path.encode(), 256, fa.KV_F16, err, len(err))
    if h:  # a GPU is present: the model loaded
        hp = fa.HParams()
        assert fa.lib().flint_attn_model_hparams(h, ctypes.byref(hp), None, None) == 0
        assert hp.n_layer == 2 and hp.n_head == 32 and hp.rope_theta == mb.THETA
        fa.lib().flint_attn_model_close(h)
    else:  # no GPU: every host-side check passed and the first device allocation failed
        assert err.value.decode().startswith("hipMalloc"), err.value.decode()


def test_loader_rejects_bad_encodings(model, tmp_path):
    import gguf_writer as gw
    # a metadata value type the format does not have
    path = str(tmp_path / "badtype.gguf")
    blob = bytearray(open(_raw_meta_model(model, tmp_path, "ok", [("x.z", gw.GGUF_U32, 7)]), "rb").read())
    i = blob.index(b"x.z") + 3
    blob[i:i + 4] = struct.pack("<I", 13)
    open(path, "wb").write(bytes(blob))
    assert model_open_error(path) == "gguf: unknown metadata type 13"
    # an array of arrays
    i = blob.index(b"x.z") + 3
    blob[i:i + 4] = struct.pack("<I", gw.GGUF_ARRAY)
    blob[i + 4:i + 8] = struct.pack("<I", gw.GGUF_ARRAY)  # element type (the u32 value's bytes)
    open(path, "wb").write(bytes(blob))
    assert model_open_error(path) == "gguf: unsupported array element type"
    # a tensor type id ggml does not define
    p2 = str(tmp_path / "tensortype.gguf")
    mb.write_model(p2, model, tensor_edit=lambda ts: [(t[0], t[1], 99, (2048, 1)) if t[0] == "output.weight"
                                                      else t for t in ts])
    assert model_open_error(p2) == "unsupported ggml type 99"
    # general.alignment 0
    p3 = _raw_meta_model(model, tmp_path, "align0", [("general.alignment", gw.GGUF_U32, 0)])
    assert model_open_error(p3) == "gguf: general.alignment is 0"


def test_loader_rejects_wrapping_tensor_sizes(model, tmp_path):
    """A tensor whose byte count does not fit 64 bits (an F32 token_embd.weight of 2048 x 2^51
    elements: 2^62 elements, 2^64 bytes) or whose row is not a whole number of blocks is
    rejected on the host, before any device work: no row index past the mapped bytes can
    reach the embedding kernel."""
    p1 = str(tmp_path / "wrap.gguf")
    mb.write_model(p1, model, tensor_edit=lambda ts: [(t[0], np.zeros(16, np.uint8), 0, (2048, 1 << 51))
                                                      if t[0] == "token_embd.weight" else t for t in ts])
    assert model_open_error(p1) == "tensor out of bounds: token_embd.weight"
    p2 = str(tmp_path / "partial_block.gguf")
    mb.write_model(p2, model, tensor_edit=lambda ts: [(t[0], np.zeros(34, np.uint8), 8, (33, 1))
                                                      if t[0] == "output.weight" else t for t in ts])
    assert model_open_error(p2) == "tensor out of bounds: output.weight"
