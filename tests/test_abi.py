"""The C-ABI library on the CPU: it loads, exports every function the headers
declare, and its host-side checks and the engine C API's error paths behave
like the reference's (/root/reference/src/capi.mm:17-73). No GPU work here:
every call below fails its argument checks before touching the device."""
import ctypes
import os
import subprocess

import pytest

import flint_attn as fa


def test_library_exports_every_header_function():
    names = fa.header_functions()
    assert len(names) >= 21
    L = fa.lib()
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    nm = subprocess.run(["nm", "-D", "--defined-only", fa.LIB_PATH], capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in nm.splitlines() if " T " in line}
    assert set(names) <= exported


def test_probe_library_exports_its_entry_points():
    """bench.py's measurement library (streaming read, MFMA rate, launch cost) is built beside the
    attention library and exports the four functions bench_roofline binds; it is not part of the
    attention library's C ABI."""
    path = os.path.join(os.path.dirname(fa.LIB_PATH), "libflint_probe.so")
    assert os.path.exists(path), "build with make -C flint-mac_amd"
    nm = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in nm.splitlines() if " T " in line}
    assert {"flint_probe_stream_read", "flint_probe_mfma", "flint_probe_empty", "flint_probe_chain"} <= exported
    attn = subprocess.run(["nm", "-D", "--defined-only", fa.LIB_PATH], capture_output=True, text=True).stdout
    assert "flint_probe_" not in attn


# The Rust server's bindings, as declared at /root/reference/server/src/ffi.rs:5-11 (the
# #[repr(C)] config) and :19-29 (the extern "C" block), kept here as text.
RUST_FFI = """
fn flint_open(cfg: *const FlintConfig, err: *mut c_char, err_len: i32) -> *mut FlintEngineRaw;
fn flint_close(e: *mut FlintEngineRaw);
fn flint_n_ctx(e: *const FlintEngineRaw) -> i32;
fn flint_n_vocab() -> i32;
fn flint_pos(e: *const FlintEngineRaw) -> i32;
fn flint_truncate(e: *mut FlintEngineRaw, pos: i32) -> i32;
fn flint_prefill(e: *mut FlintEngineRaw, tokens: *const i32, n: i32, err: *mut c_char, err_len: i32) -> i32;
fn flint_decode(e: *mut FlintEngineRaw, token: i32, err: *mut c_char, err_len: i32) -> i32;
fn flint_logits(e: *const FlintEngineRaw) -> *const f32;
"""
RUST_CONFIG = [("model_path", "*const c_char"), ("metallib_dir", "*const c_char"), ("pool_gb", "f64"),
               ("n_ctx", "i32")]
# Rust FFI type -> the C type it binds to (flint_engine is opaque on both sides)
RUST_TO_C = {"*const FlintConfig": "const flint_config*", "*mut c_char": "char*", "*const c_char": "const char*",
             "i32": "int32_t", "f64": "double", "*const i32": "const int32_t*", "*const f32": "const float*",
             "*mut FlintEngineRaw": "flint_engine*", "*const FlintEngineRaw": "const flint_engine*", "": "void"}


def _c_prototypes():
    """{name: (return type, [parameter types])} of include/capi.h, spacing normalised."""
    import re
    src = open(os.path.join(fa.INCLUDE, "capi.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    out = {}
    for ret, name, params in re.findall(r"([A-Za-z_][\w\s\*]*?)\b(flint_\w+)\s*\(([^)]*)\)\s*;", src):
        norm = lambda t: re.sub(r"\s*\*\s*", "*", " ".join(t.split()))
        types = []
        for p in params.split(","):
            p = p.strip()
            if p in ("", "void"):
                continue
            types.append(norm(re.sub(r"\b\w+$", "", p)))  # drop the parameter name
        out[name] = (norm(ret), types)
    return out


def _rust_prototypes():
    import re
    out = {}
    for name, params, ret in re.findall(r"fn (flint_\w+)\(([^)]*)\)(?:\s*->\s*([^;]+))?;", RUST_FFI):
        types = [RUST_TO_C[p.split(":", 1)[1].strip()] for p in params.split(",") if p.strip()]
        out[name] = (RUST_TO_C[(ret or "").strip()], types)
    return out


def test_capi_header_matches_rust_ffi_signatures():
    """Each of the nine entry points the Rust server binds has, in include/capi.h, the return
    type and parameter types that its Rust declaration maps to."""
    rust, c = _rust_prototypes(), _c_prototypes()
    assert len(rust) == 9
    for name, sig in rust.items():
        assert name in c, name
        assert c[name] == sig, (name, c[name], sig)


def test_capi_config_layout_matches_rust_repr_c(tmp_path):
    """flint_config's field offsets and size, compiled from include/capi.h, equal the
    #[repr(C)] layout of the Rust FlintConfig (pointers 8 bytes, f64 8, i32 4, C alignment)."""
    size = {"*const c_char": 8, "f64": 8, "i32": 4}
    off, want = 0, []
    for field, ty in RUST_CONFIG:
        n = size[ty]
        off = (off + n - 1) // n * n
        want.append((field, off))
        off += n
    total = (off + 7) // 8 * 8
    prog = tmp_path / "layout.c"
    prog.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "capi.h"\nint main(void) {\n' +
                    "".join(f'  printf("%zu ", offsetof(flint_config, {f}));\n' for f, _ in RUST_CONFIG) +
                    '  printf("%zu\\n", sizeof(flint_config));\n  return 0;\n}\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", fa.INCLUDE, str(prog), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert got == [o for _, o in want] + [total]


def _err():
    return ctypes.create_string_buffer(256)


class _Cfg(ctypes.Structure):
    _fields_ = [("model_path", ctypes.c_char_p), ("metallib_dir", ctypes.c_char_p), ("pool_gb", ctypes.c_double),
                ("n_ctx", ctypes.c_int32)]


def _open(path):
    cfg = _Cfg(path.encode() if path else None, b".", 0.0, 4096)
    err = _err()
    h = fa.lib().flint_open(ctypes.cast(ctypes.pointer(cfg), ctypes.c_void_p), err, len(err))
    return h, err.value.decode()


def test_capi_open_errors(tmp_path):
    L = fa.lib()
    assert L.flint_n_vocab() == 150144
    h, msg = _open(str(tmp_path / "missing.gguf"))
    assert not h and msg.startswith("cannot open")
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"NOPE" + b"\0" * 60)
    h, msg = _open(str(bad))
    assert not h and msg.startswith("not a GGUF file")
    ok = tmp_path / "model.gguf"
    ok.write_bytes(b"GGUF" + b"\0" * 60)
    h, msg = _open(str(ok))
    assert not h and msg == "unsupported GGUF version"  # version 0 (gguf.cpp:150)
    # a well-formed model: tests/test_model.py::test_capi_open_valid_model_names_the_scope
    # err may be NULL
    cfg = _Cfg(str(tmp_path / "missing.gguf").encode(), b".", 0.0, 0)
    assert not L.flint_open(ctypes.cast(ctypes.pointer(cfg), ctypes.c_void_p), None, 0)


def test_capi_null_handle_paths():
    L = fa.lib()
    L.flint_close(None)
    assert L.flint_truncate(None, 0) == -1
    assert L.flint_pos(None) == 0 and L.flint_n_ctx(None) == 0
    err = _err()
    assert L.flint_decode(None, 1, err, len(err)) == -1 and err.value
    assert L.flint_prefill(None, None, 0, err, len(err)) == -1
    assert not L.flint_logits(None)
    # the model session's timing calls (Engine::last_gpu_ms / enable_profiling / last_profile)
    assert L.flint_attn_model_enable_profiling(None, 1) == -1
    assert L.flint_attn_model_set_weight_planes(None, 0, None, 0) == -1
    assert L.flint_attn_model_weight_planes(None) == -2
    assert L.flint_attn_model_last_gpu_ms(None) == -1.0
    assert L.flint_attn_model_last_encode_ms(None) == -1.0
    assert L.flint_attn_model_last_profile(None, None, 0, None, 0) == -1


def _layer(**kw):
    d = dict(k_cache=0x1000, v_cache=0x2000, n_slots=1024, kv_dtype=fa.KV_F16, is_swa=1, has_rope=1, window=513,
             rope_theta=1e4, rms_eps=1e-6, q_norm=0x3000, k_norm=0x4000, sinks=0x5000)
    d.update(kw)
    return fa.LayerDesc(**d)


@pytest.mark.parametrize("kw,msg", [
    (dict(n_slots=1000), "multiple of 32"),
    (dict(n_slots=992), "power of two"),
    (dict(n_slots=256), "must hold the window"),
    # one slot past FLINT_MAX_SLOTS (a kv head's cache would reach 2^31 bytes), rejected before
    # any launch: the pointers here are not device memory
    (dict(is_swa=0, n_slots=(1 << 23) + 32), "at most 8388608"),
    (dict(kv_dtype=7), "kv_dtype"),
    (dict(k_cache=0), "KV cache pointer"),
    (dict(sinks=0), "sinks"),
    (dict(window=0), "window"),
])
def test_decode_rejects_bad_layer(kw, msg):
    with pytest.raises(fa.FlintAttnError, match=msg):
        fa._call(fa.lib().flint_attn_decode, ctypes.byref(_layer(**kw)), ctypes.c_void_p(0x6000),
                 ctypes.c_void_p(0x7000), 5, 0, None)


def test_decode_rejects_bad_arguments():
    L = fa.lib()
    lay = _layer(is_swa=0, n_slots=2048)
    with pytest.raises(fa.FlintAttnError, match="context full"):
        fa._call(L.flint_attn_decode, ctypes.byref(lay), ctypes.c_void_p(1), ctypes.c_void_p(1), 2048, 0, None)
    with pytest.raises(fa.FlintAttnError, match="multiple of 32"):
        fa._call(L.flint_attn_decode, ctypes.byref(lay), ctypes.c_void_p(1), ctypes.c_void_p(1), 5, 33, None)
    with pytest.raises(fa.FlintAttnError, match="position"):
        fa._call(L.flint_attn_decode, ctypes.byref(lay), ctypes.c_void_p(1), ctypes.c_void_p(1), -1, 0, None)
    with pytest.raises(fa.FlintAttnError, match="NULL"):
        fa._call(L.flint_attn_decode, None, ctypes.c_void_p(1), ctypes.c_void_p(1), 5, 0, None)
    pos = (ctypes.c_int32 * 2)(1, 2)
    with pytest.raises(fa.FlintAttnError, match="n_seq"):
        fa._call(L.flint_attn_decode_batch, ctypes.byref(lay), 0, 0, ctypes.c_void_p(1), ctypes.c_void_p(1), pos, 0,
                 None)
    with pytest.raises(fa.FlintAttnError, match="seq_stride"):
        fa._call(L.flint_attn_decode_batch, ctypes.byref(lay), 2, 100, ctypes.c_void_p(1), ctypes.c_void_p(1), pos,
                 0, None)


def test_prefill_rejects_bad_arguments():
    L = fa.lib()
    full = _layer(is_swa=0, n_slots=4096)
    with pytest.raises(fa.FlintAttnError, match="prefill: empty"):
        fa._call(L.flint_attn_prefill, ctypes.byref(full), ctypes.c_void_p(1), 5120, 0, 0, ctypes.c_void_p(1), None)
    with pytest.raises(fa.FlintAttnError, match="context full"):
        fa._call(L.flint_attn_prefill, ctypes.byref(full), ctypes.c_void_p(1), 5120, 4000, 100, ctypes.c_void_p(1),
                 None)
    with pytest.raises(fa.FlintAttnError, match="q_stride"):
        fa._call(L.flint_attn_prefill, ctypes.byref(full), ctypes.c_void_p(1), 100, 0, 10, ctypes.c_void_p(1), None)


def test_engine_create_rejects_bad_arguments():
    L = fa.lib()
    err = _err()
    flags = (ctypes.c_uint8 * 2)(1, 0)
    assert not L.flint_attn_engine_create(0, flags, flags, 4096, 1, 1e4, err, len(err)) and err.value
    assert not L.flint_attn_engine_create(2, flags, flags, 0, 1, 1e4, err, len(err))
    assert not L.flint_attn_engine_create(2, flags, flags, 4096, 3, 1e4, err, len(err))
    assert b"kv_dtype" in err.value
    assert not L.flint_attn_engine_create(2, flags, flags, (1 << 23) + 1, 1, 1e4, err, len(err))
    assert b"at most 8388608" in err.value
    assert L.flint_attn_engine_n_layer(None) == 0
    assert not L.flint_attn_engine_layer(None, 0)


def test_k_tile_layout_is_a_permutation_read_in_contiguous_units():
    """The K cache tile order (include/flint_attn.h): a bijection of the 32 x 128 tile onto its
    4096 elements, in which the 16-byte unit read by lane l of the decode kernel's load
    instruction (st, c) is unit (st*4 + c)*64 + l and holds 8 consecutive dims of one slot."""
    import numpy as np
    o = fa.k_tile_offsets()
    assert sorted(o.reshape(-1).tolist()) == list(range(4096))
    assert np.all(o[:, 0::8] % 8 == 0) and np.all(np.diff(o.reshape(32, 16, 8), axis=2) == 1)
    for st in range(2):
        for c in range(4):
            units = []
            for lane in range(64):
                n, g = lane & 15, lane >> 4
                slot = 8 * (n >> 2) + 4 * st + (n & 3)
                units.append(o[slot, 32 * c + 8 * g] // 8)
            assert units == list(range((st * 4 + c) * 64, (st * 4 + c) * 64 + 64))
