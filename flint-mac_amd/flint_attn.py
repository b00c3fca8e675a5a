"""Python binding of libflint_attn.so (the MI355X attention hot path) over its C ABI.

Mirrors the reference engine's attention interface (/root/reference/src/engine.h:24-79:
per-layer KV cache, decode step, chunked prefill, debug_attn) for tests and the
benchmark. Device memory and streams come from PyTorch (plumbing only); every
computation runs in the HIP kernels of libflint_attn.so. There is no fallback:
if the library is missing, loading raises.
"""
import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libflint_attn.so")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")

N_HEAD, N_HEAD_KV, HEAD_DIM, GQA = 32, 4, 128, 8
Q_DIM, KV_DIM, QKV_DIM = 4096, 512, 5120
N_SWA, SWA_RING = 513, 1024
KV_F16, KV_BF16 = 1, 2


class FlintAttnError(RuntimeError):
    pass


class LayerDesc(ctypes.Structure):
    """flint_attn_layer (include/flint_attn.h)."""
    _fields_ = [
        ("k_cache", ctypes.c_void_p),
        ("v_cache", ctypes.c_void_p),
        ("n_slots", ctypes.c_int32),
        ("kv_dtype", ctypes.c_int32),
        ("is_swa", ctypes.c_int32),
        ("has_rope", ctypes.c_int32),
        ("window", ctypes.c_int32),
        ("rope_theta", ctypes.c_float),
        ("rms_eps", ctypes.c_float),
        ("q_norm", ctypes.c_void_p),
        ("k_norm", ctypes.c_void_p),
        ("sinks", ctypes.c_void_p),
    ]


class WeightDesc(ctypes.Structure):
    """flint_weight (include/flint_proj.h)."""
    _fields_ = [("data", ctypes.c_void_p), ("type", ctypes.c_int32)]


class HParams(ctypes.Structure):
    """flint_attn_hparams (include/flint_model.h)."""
    _fields_ = [(n, ctypes.c_int32) for n in ("n_layer", "n_embd", "n_head", "n_head_kv", "head_dim", "n_vocab",
                                              "n_ff_dense", "n_ff_exp", "n_ff_shexp", "n_expert", "n_expert_used",
                                              "n_dense_lead", "n_swa")] + [("rms_eps", ctypes.c_float),
                                                                           ("rope_theta", ctypes.c_float)]


# ggml type ids of the weight formats (include/flint_proj.h)
W_TYPES = {"f32": 0, "f16": 1, "q8_0": 8, "q5_K": 13, "q6_K": 14, "iq4_xs": 23, "bf16": 30}
N_EMBD = 2048

_lib = None
_vp, _i32, _i64, _f32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float
_cp = ctypes.c_char_p
_lp = ctypes.POINTER(LayerDesc)
_i32p = ctypes.POINTER(ctypes.c_int32)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_f32p = ctypes.POINTER(ctypes.c_float)

_SIGS = {
    "flint_attn_decode": (_i32, [_lp, _vp, _vp, _i32, _i32, _vp, _cp, _i32]),
    "flint_attn_decode_batch": (_i32, [_lp, _i32, _i64, _vp, _vp, _i32p, _i32, _vp, _cp, _i32]),
    "flint_attn_decode_batch_noalloc": (_i32, [_lp, _i32, _i64, _vp, _vp, _i32p, _i32, _vp, _cp, _i32]),
    "flint_attn_prefill": (_i32, [_lp, _vp, _i32, _i32, _i32, _vp, _vp, _cp, _i32]),
    "flint_attn_sync": (_i32, [_cp, _i32]),
    "flint_attn_engine_create": (_vp, [_i32, _u8p, _u8p, _i32, _i32, _f32, _cp, _i32]),
    "flint_attn_engine_destroy": (None, [_vp]),
    "flint_attn_engine_n_layer": (_i32, [_vp]),
    "flint_attn_engine_set_weights": (_i32, [_vp, _i32, _f32p, _f32p, _f32p, _cp, _i32]),
    "flint_attn_engine_layer": (_lp, [_vp, _i32]),
    "flint_attn_engine_decode": (_i32, [_vp, _i32, _vp, _vp, _i32, _vp, _cp, _i32]),
    "flint_attn_engine_prefill": (_i32, [_vp, _i32, _vp, _i32, _i32, _vp, _vp, _cp, _i32]),
    "flint_attn_engine_debug_attn": (_i32, [_vp, _i32, _f32p, _i32, _i32, _f32p, _cp, _i32]),
    "flint_w_row_bytes": (_i64, [_i32, _i64]),
    "flint_w_get_row": (_i32, [_i32, _vp, _i64, _i64, _vp, _vp, _cp, _i32]),
    "flint_w_get_rows": (_i32, [_i32, _vp, _i64, _i64, _i32p, _i32, _vp, _vp, _cp, _i32]),
    "flint_attn_qkv_proj": (_i32, [ctypes.POINTER(WeightDesc)] * 3 + [_vp, _vp, _f32, _vp, _vp, _cp, _i32]),
    "flint_attn_o_proj": (_i32, [ctypes.POINTER(WeightDesc), _vp, _vp, _vp, _cp, _i32]),
    "flint_attn_qkv_proj_rows": (_i32, [ctypes.POINTER(WeightDesc)] * 3 + [_vp, _i32, _vp, _f32, _vp, _i32, _vp, _cp,
                                                                            _i32]),
    "flint_attn_o_proj_rows": (_i32, [ctypes.POINTER(WeightDesc), _vp, _i32, _vp, _vp, _cp, _i32]),
    "flint_attn_model_open": (_vp, [_cp, _i32, _i32, _cp, _i32]),
    "flint_attn_model_close": (None, [_vp]),
    "flint_attn_model_hparams": (_i32, [_vp, ctypes.POINTER(HParams), _u8p, _u8p]),
    "flint_attn_model_engine": (_vp, [_vp]),
    "flint_attn_model_embed": (_i32, [_vp, _i32p, _i32, _vp, _vp, _cp, _i32]),
    "flint_attn_model_block_decode": (_i32, [_vp, _i32, _vp, _i32, _vp, _vp, _cp, _i32]),
    "flint_attn_model_block_prefill": (_i32, [_vp, _i32, _vp, _i32, _i32, _vp, _vp, _cp, _i32]),
    "flint_attn_model_pos": (_i32, [_vp]),
    "flint_attn_model_n_ctx": (_i32, [_vp]),
    "flint_attn_model_truncate": (_i32, [_vp, _i32]),
    "flint_attn_model_step": (_i32, [_vp, _i32, _vp, _vp, _cp, _i32]),
    "flint_attn_model_prefill": (_i32, [_vp, _i32p, _i32, _vp, _vp, _cp, _i32]),
    "flint_attn_model_enable_profiling": (_i32, [_vp, _i32]),
    "flint_attn_model_set_weight_planes": (_i32, [_vp, _i32, _cp, _i32]),
    "flint_attn_model_weight_planes": (_i32, [_vp]),
    "flint_attn_model_last_gpu_ms": (ctypes.c_double, [_vp]),
    "flint_attn_model_last_encode_ms": (ctypes.c_double, [_vp]),
    "flint_attn_model_last_profile": (_i32, [_vp, _cp, _i32, ctypes.POINTER(ctypes.c_double), _i32]),
    "flint_open": (_vp, [_vp, _cp, _i32]),
    "flint_close": (None, [_vp]),
    "flint_n_ctx": (_i32, [_vp]),
    "flint_n_vocab": (_i32, []),
    "flint_pos": (_i32, [_vp]),
    "flint_truncate": (_i32, [_vp, _i32]),
    "flint_prefill": (_i32, [_vp, _i32p, _i32, _cp, _i32]),
    "flint_decode": (_i32, [_vp, _i32, _cp, _i32]),
    "flint_logits": (_f32p, [_vp]),
}


def lib():
    """Load libflint_attn.so (raises FlintAttnError if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FlintAttnError(f"{LIB_PATH} is missing: run __graft_entry__.build() (make -C flint-mac_amd)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def header_functions():
    """Names of every function declared in include/*.h."""
    names = []
    for fn in sorted(os.listdir(INCLUDE)):
        if fn.endswith(".h"):
            src = open(os.path.join(INCLUDE, fn)).read()
            src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
            src = re.sub(r"//[^\n]*", "", src)
            names += re.findall(r"\b(flint_\w+)\s*\(", src)
    return sorted(set(names))


def _call(fn, *args):
    err = ctypes.create_string_buffer(512)
    rc = fn(*args, err, len(err))
    if rc != 0:
        raise FlintAttnError(err.value.decode())


def k_tile_offsets():
    """[32][128] element offsets, within one 32-slot K tile (4096 elements), of (slot % 32, dim):
    the tile order of the K cache (kt_index in csrc/common.h)."""
    import numpy as np
    r = np.arange(32)[:, None]
    d = np.arange(HEAD_DIM)[None, :]
    st, n = (r >> 2) & 1, ((r >> 3) << 2) | (r & 3)
    c, g = d >> 5, (d >> 3) & 3
    return (((st * 4 + c) * 64 + g * 16 + n) << 3) | (d & 7)


def _stream(stream):
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    return stream


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


class KVLayer:
    """One attention layer on the GPU: KV cache in HBM in 32-slot tiles (K [4][n_slots/32][4096]
    in MFMA-operand order, see k_tile_offsets; V transposed, [4][n_slots/32][128][32]) and its
    q_norm / k_norm / sinks.
    `n_seq` > 1 allocates independent caches for that many sequences."""

    def __init__(self, is_swa, has_rope, n_slots=None, kv_dtype="f16", rope_theta=1e4, window=N_SWA,
                 q_norm=None, k_norm=None, sinks=None, n_seq=1, device="cuda", rms_eps=1e-6):
        import torch
        self.torch_dtype = {"f16": torch.float16, "bf16": torch.bfloat16}[kv_dtype]
        self.kv_dtype = kv_dtype
        if n_slots is None:
            n_slots = SWA_RING if is_swa else 4096
        self.n_slots, self.n_seq = int(n_slots), int(n_seq)
        assert self.n_slots % 32 == 0, "n_slots must be a multiple of 32"
        self.k = torch.zeros((n_seq, N_HEAD_KV, n_slots // 32, 32 * HEAD_DIM), dtype=self.torch_dtype, device=device)
        self.v = torch.zeros((n_seq, N_HEAD_KV, n_slots // 32, HEAD_DIM, 32), dtype=self.torch_dtype, device=device)
        f = lambda a, n, d: torch.as_tensor(a if a is not None else [d] * n, dtype=torch.float32).to(device)
        self.q_norm = f(q_norm, HEAD_DIM, 1.0).contiguous()
        self.k_norm = f(k_norm, HEAD_DIM, 1.0).contiguous()
        self.sinks = f(sinks, N_HEAD, 0.0).contiguous()
        self.desc = LayerDesc(self.k.data_ptr(), self.v.data_ptr(), self.n_slots,
                              KV_F16 if kv_dtype == "f16" else KV_BF16, int(bool(is_swa)), int(bool(has_rope)),
                              int(window), float(rope_theta), float(rms_eps), self.q_norm.data_ptr(),
                              self.k_norm.data_ptr(), self.sinks.data_ptr())
        self.is_swa, self.has_rope, self.window, self.rope_theta = bool(is_swa), bool(has_rope), window, rope_theta

    @property
    def seq_stride(self):
        return N_HEAD_KV * self.n_slots * HEAD_DIM

    def k_slots(self):
        """K as [n_seq][4][n_slots][128] (a copy out of the tiled layout)."""
        import torch
        idx = torch.as_tensor(k_tile_offsets().reshape(-1), device=self.k.device)
        return self.k[..., idx].reshape(self.n_seq, N_HEAD_KV, self.n_slots, HEAD_DIM)

    def v_slots(self):
        """V as [n_seq][4][n_slots][128] (a copy out of the tiled layout)."""
        return self.v.permute(0, 1, 2, 4, 3).reshape(self.n_seq, N_HEAD_KV, self.n_slots, HEAD_DIM)

    def slot(self, pos):
        return pos & (self.n_slots - 1) if self.is_swa else pos

    def decode(self, qkv, att, pos, keys_per_split=0, stream=None):
        """qkv: cuda float32 [5120] (or [n_seq][5120]); att: cuda float32 [4096] (or [n_seq][4096]);
        pos: int or list of ints (one per sequence)."""
        if isinstance(pos, int):
            assert self.n_seq == 1
            _call(lib().flint_attn_decode, ctypes.byref(self.desc), _ptr(qkv), _ptr(att), pos, keys_per_split,
                  _stream(stream))
        else:
            arr = (ctypes.c_int32 * len(pos))(*pos)
            _call(lib().flint_attn_decode_batch, ctypes.byref(self.desc), len(pos), self.seq_stride, _ptr(qkv),
                  _ptr(att), arr, keys_per_split, _stream(stream))

    def prefill(self, qkv, att, p0, T=None, q_stride=QKV_DIM, stream=None):
        """qkv: cuda float32 [T][q_stride] raw rows for positions p0..p0+T-1; att: cuda float32 [T][4096]."""
        if T is None:
            T = qkv.shape[0]
        _call(lib().flint_attn_prefill, ctypes.byref(self.desc), _ptr(qkv), q_stride, p0, T, _ptr(att),
              _stream(stream))


def row_bytes(wtype, k):
    """Bytes of a row of k elements of a weight format, or -1 (flint_w_row_bytes)."""
    return int(lib().flint_w_row_bytes(W_TYPES[wtype], k))


def get_row(wtype, w, k, row, out, stream=None):
    """Dequantise row `row` of the weight bytes `w` (a uint8 device tensor) into out [k] fp32
    (flint_w_get_row; the reference's Engine::debug_get_row)."""
    _call(lib().flint_w_get_row, W_TYPES[wtype], _ptr(w), k, row, _ptr(out), _vp(_stream(stream)))


def get_rows(wtype, w, k, n_rows, rows, out, stream=None):
    """Dequantise rows `rows` (a sequence of ints in [0, n_rows)) of the weight bytes `w` into
    out [len(rows)][k] fp32 in one dispatch per 448 rows (flint_w_get_rows; the reference's
    k_embed_rows)."""
    arr = (ctypes.c_int32 * len(rows))(*[int(r) for r in rows])
    _call(lib().flint_w_get_rows, W_TYPES[wtype], _ptr(w), k, n_rows, arr, len(rows), _ptr(out),
          _vp(_stream(stream)))


def _wdesc(w):
    data, wtype = w
    return ctypes.byref(WeightDesc(data.data_ptr(), W_TYPES[wtype]))


def qkv_proj(wq, wk, wv, x, attn_norm, qkv, rms_eps=1e-6, stream=None):
    """qkv [5120] = [Wq; Wk; Wv] RMSNorm(x) * attn_norm (flint_attn_qkv_proj). Each weight is a
    (uint8 device tensor, type name) pair."""
    _call(lib().flint_attn_qkv_proj, _wdesc(wq), _wdesc(wk), _wdesc(wv), _ptr(x), _ptr(attn_norm), rms_eps,
          _ptr(qkv), _vp(_stream(stream)))


def o_proj(wo, att, x, stream=None):
    """x [2048] += Wo att (flint_attn_o_proj); wo is a (uint8 device tensor, type name) pair."""
    _call(lib().flint_attn_o_proj, _wdesc(wo), _ptr(att), _ptr(x), _vp(_stream(stream)))


def qkv_proj_rows(wq, wk, wv, x, attn_norm, qkv, rms_eps=1e-6, stream=None):
    """qkv [T][>=5120] rows = [Wq; Wk; Wv] RMSNorm(x[t]) * attn_norm for x [T][2048]
    (flint_attn_qkv_proj_rows)."""
    _call(lib().flint_attn_qkv_proj_rows, _wdesc(wq), _wdesc(wk), _wdesc(wv), _ptr(x), x.shape[0], _ptr(attn_norm),
          rms_eps, _ptr(qkv), qkv.stride(0), _vp(_stream(stream)))


def o_proj_rows(wo, att, x, stream=None):
    """x [T][2048] += Wo att[t] for att [T][4096] (flint_attn_o_proj_rows)."""
    _call(lib().flint_attn_o_proj_rows, _wdesc(wo), _ptr(att), att.shape[0], _ptr(x), _vp(_stream(stream)))


def sync():
    _call(lib().flint_attn_sync)


class Model:
    """flint_attn_model: a Flint GGUF's attention blocks in HBM (include/flint_model.h)."""

    def __init__(self, path, n_ctx, kv_dtype="f16"):
        err = ctypes.create_string_buffer(512)
        h = lib().flint_attn_model_open(path.encode(), n_ctx, KV_F16 if kv_dtype == "f16" else KV_BF16, err,
                                        len(err))
        if not h:
            raise FlintAttnError(err.value.decode())
        self.h = ctypes.c_void_p(h)

    def close(self):
        if getattr(self, "h", None) and lib is not None:  # lib is None while the interpreter exits
            lib().flint_attn_model_close(self.h)
            self.h = None

    __del__ = close

    def set_weight_planes(self, on=True):
        """Keep the prefill projections' weight planes (the default) or free them
        (flint_attn_model_set_weight_planes)."""
        _call(lib().flint_attn_model_set_weight_planes, self.h, 1 if on else 0)

    def weight_planes(self):
        """1 kept, 2 allowed and not allocated yet, 0 off, -1 the last allocation failed
        (flint_attn_model_weight_planes)."""
        return lib().flint_attn_model_weight_planes(self.h)

    def enable_profiling(self, on=True):
        """Later steps and prefills time each stage (Engine::enable_profiling;
        flint_attn_model_enable_profiling)."""
        lib().flint_attn_model_enable_profiling(self.h, 1 if on else 0)

    def last_gpu_ms(self):
        """GPU time of the last step or prefill in ms, or None before any (Engine::last_gpu_ms;
        flint_attn_model_last_gpu_ms). Waits for that call's work."""
        t = lib().flint_attn_model_last_gpu_ms(self.h)
        return None if t < 0 else t

    def last_encode_ms(self):
        """Host time the last step or prefill took to enqueue its launches, in ms, or None
        (Engine::last_encode_ms; flint_attn_model_last_encode_ms)."""
        t = lib().flint_attn_model_last_encode_ms(self.h)
        return None if t < 0 else t

    def last_profile(self):
        """[(stage, ms)] of the last step or prefill in order (Engine::last_profile;
        flint_attn_model_last_profile). Waits for that call's work."""
        n = lib().flint_attn_model_last_profile(self.h, None, 0, None, 0)
        if n < 0:
            return []
        width = 32
        labels = ctypes.create_string_buffer(n * width)
        ms = (ctypes.c_double * n)()
        if lib().flint_attn_model_last_profile(self.h, labels, width, ms, n) != n:
            raise FlintAttnError("flint_attn_model_last_profile failed")
        raw = labels.raw
        return [(raw[i * width:(i + 1) * width].split(b"\0")[0].decode(), ms[i]) for i in range(n)]

    def hparams(self):
        """(HParams, is_swa list, has_rope list)."""
        hp = HParams()
        assert lib().flint_attn_model_hparams(self.h, ctypes.byref(hp), None, None) == 0
        a = (ctypes.c_uint8 * hp.n_layer)()
        b = (ctypes.c_uint8 * hp.n_layer)()
        assert lib().flint_attn_model_hparams(self.h, ctypes.byref(hp), a, b) == 0
        return hp, list(a), list(b)

    def layer(self, il):
        p = lib().flint_attn_engine_layer(lib().flint_attn_model_engine(self.h), il)
        if not p:
            raise FlintAttnError(f"bad layer index {il}")
        return p.contents

    def embed(self, tokens, x, stream=None):
        t = (ctypes.c_int32 * len(tokens))(*[int(v) for v in tokens])
        _call(lib().flint_attn_model_embed, self.h, t, len(tokens), _ptr(x), _vp(_stream(stream)))

    def block_decode(self, il, x, pos, att=None, stream=None):
        _call(lib().flint_attn_model_block_decode, self.h, il, _ptr(x), pos, _ptr(att) if att is not None else None,
              _vp(_stream(stream)))

    @property
    def pos(self):
        return lib().flint_attn_model_pos(self.h)

    @property
    def n_ctx(self):
        return lib().flint_attn_model_n_ctx(self.h)

    def truncate(self, pos):
        """0 on success, -1 if pos is outside [0, pos] (flint_attn_model_truncate)."""
        return lib().flint_attn_model_truncate(self.h, pos)

    def step(self, token, x, stream=None):
        """The token through every layer's attention block at the current position; x [2048]
        receives the hidden state (flint_attn_model_step)."""
        _call(lib().flint_attn_model_step, self.h, int(token), _ptr(x), _vp(_stream(stream)))

    def prefill(self, tokens, X, stream=None):
        """tokens at the current position, layer-major; X [n][2048] receives the hidden states
        (flint_attn_model_prefill)."""
        t = (ctypes.c_int32 * len(tokens))(*[int(v) for v in tokens])
        _call(lib().flint_attn_model_prefill, self.h, t, len(tokens), _ptr(X), _vp(_stream(stream)))

    def block_prefill(self, il, X, p0, att=None, stream=None):
        _call(lib().flint_attn_model_block_prefill, self.h, il, _ptr(X), p0, X.shape[0],
              _ptr(att) if att is not None else None, _vp(_stream(stream)))


class Engine:
    """flint_attn_engine: the KV caches and weights of every layer."""

    def __init__(self, is_swa, has_rope, n_ctx, kv_dtype="f16", rope_theta=1e4):
        n = len(is_swa)
        a = (ctypes.c_uint8 * n)(*[int(bool(x)) for x in is_swa])
        b = (ctypes.c_uint8 * n)(*[int(bool(x)) for x in has_rope])
        err = ctypes.create_string_buffer(512)
        h = lib().flint_attn_engine_create(n, a, b, n_ctx, KV_F16 if kv_dtype == "f16" else KV_BF16,
                                           rope_theta, err, len(err))
        if not h:
            raise FlintAttnError(err.value.decode())
        self.h = ctypes.c_void_p(h)

    def close(self):
        if self.h:
            lib().flint_attn_engine_destroy(self.h)
            self.h = None

    __del__ = close

    @property
    def n_layer(self):
        return lib().flint_attn_engine_n_layer(self.h)

    def layer(self, il):
        p = lib().flint_attn_engine_layer(self.h, il)
        if not p:
            raise FlintAttnError(f"bad layer index {il}")
        return p.contents

    def set_weights(self, il, q_norm, k_norm, sinks):
        import numpy as np
        arrs = [np.ascontiguousarray(x, np.float32) for x in (q_norm, k_norm, sinks)]
        _call(lib().flint_attn_engine_set_weights, self.h, il, *[x.ctypes.data_as(_f32p) for x in arrs])

    def decode(self, il, qkv, att, pos, stream=None):
        _call(lib().flint_attn_engine_decode, self.h, il, _ptr(qkv), _ptr(att), pos, _stream(stream))

    def prefill(self, il, qkv, p0, att, stream=None):
        _call(lib().flint_attn_engine_prefill, self.h, il, _ptr(qkv), p0, qkv.shape[0], _ptr(att), _stream(stream))

    def debug_attn(self, il, qkv, chunk):
        """host float32 qkv [n][5120] -> host float32 [n][4096] (Engine::debug_attn)."""
        import numpy as np
        qkv = np.ascontiguousarray(qkv, np.float32)
        n = qkv.shape[0]
        out = np.empty((n, Q_DIM), np.float32)
        _call(lib().flint_attn_engine_debug_attn, self.h, il, qkv.ctypes.data_as(_f32p), n, chunk,
              out.ctypes.data_as(_f32p))
        return out
