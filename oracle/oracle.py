"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker or the timed CPU baseline,
never as the product path. See flint_oracle.h for the reference lines each C
function restates and the checks that pin it.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_DRIVER = os.path.join(HERE, "_ref", "ref_driver")

N_HEAD, N_HEAD_KV, HEAD_DIM, GQA = 32, 4, 128, 8
Q_DIM, KV_DIM, QKV_DIM = 4096, 512, 5120
STORE = {"f32": 0, "f16": 1, "bf16": 2}

_f32p = ctypes.POINTER(ctypes.c_float)


class _Layer(ctypes.Structure):
    _fields_ = [
        ("is_swa", ctypes.c_int),
        ("has_rope", ctypes.c_int),
        ("window", ctypes.c_int),
        ("store", ctypes.c_int),
        ("rope_theta", ctypes.c_float),
        ("rms_eps", ctypes.c_float),
        ("q_norm", _f32p),
        ("k_norm", _f32p),
        ("sinks", _f32p),
    ]


_lib = None


def build():
    """Compile liboracle.so from oracle/flint_oracle.c (gcc)."""
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)


def build_ref():
    """Compile oracle/_ref/ref_driver from the reference sources, if present."""
    if not os.path.isdir("/root/reference/src"):
        return False
    subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)
    return os.path.exists(REF_DRIVER)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.fo_round.restype = ctypes.c_float
        L.fo_round.argtypes = [ctypes.c_float, ctypes.c_int]
        L.fo_round_array.argtypes = [_f32p, ctypes.c_long, ctypes.c_int]
        L.fo_rmsnorm.argtypes = [_f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_float]
        L.fo_rope_neox.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_float]
        L.fo_slot.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.fo_first_key.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int]
        lp = ctypes.POINTER(_Layer)
        L.fo_qkv_prep.argtypes = [lp, _f32p, ctypes.c_int, _f32p, _f32p, _f32p]
        L.fo_attend.argtypes = [lp, _f32p, _f32p, _f32p, ctypes.c_int, _f32p, ctypes.c_int]
        L.fo_attend_split.argtypes = [lp, _f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int, _f32p]
        L.fo_decode_step.argtypes = [lp, _f32p, ctypes.c_int, _f32p, _f32p, _f32p, ctypes.c_int]
        L.fo_prefill.argtypes = [lp, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p, _f32p, _f32p,
                                 ctypes.c_int]
        L.fo_prefill_mt.argtypes = [lp, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    _f32p, _f32p, _f32p, ctypes.c_int]
        for f in ("fo_block_elems", "fo_block_bytes"):
            getattr(L, f).restype = ctypes.c_long
            getattr(L, f).argtypes = [ctypes.c_int]
        L.fo_row_bytes.restype = ctypes.c_long
        L.fo_row_bytes.argtypes = [ctypes.c_int, ctypes.c_long]
        L.fo_dequant_row.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_long, _f32p]
        L.fo_matvec.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_long, ctypes.c_long, _f32p, _f32p]
        L.fo_matvec_f32.argtypes = [_f32p, ctypes.c_long, ctypes.c_long, _f32p, _f32p, ctypes.c_int]
        _lib = L
    return _lib


def _p(a):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return a.ctypes.data_as(_f32p)


class Layer:
    """Per-layer attention parameters, mirroring what the engine binds per layer
    (q_norm/k_norm/sinks tensors, is_swa/has_rope flags, n_swa, rope theta, eps)."""

    def __init__(self, q_norm, k_norm, sinks, is_swa, has_rope, store="f16", rope_theta=1e4, window=513,
                 rms_eps=1e-6):
        self.q_norm = np.ascontiguousarray(q_norm, np.float32)
        self.k_norm = np.ascontiguousarray(k_norm, np.float32)
        self.sinks = np.ascontiguousarray(sinks, np.float32)
        assert self.q_norm.shape == (HEAD_DIM,) and self.k_norm.shape == (HEAD_DIM,)
        assert self.sinks.shape == (N_HEAD,)
        self.is_swa, self.has_rope, self.store = int(is_swa), int(has_rope), store
        self.rope_theta, self.window, self.rms_eps = float(rope_theta), int(window), float(rms_eps)
        self._s = _Layer(self.is_swa, self.has_rope, self.window, STORE[store], self.rope_theta, self.rms_eps,
                         _p(self.q_norm), _p(self.k_norm), _p(self.sinks))

    @property
    def ref(self):
        return ctypes.byref(self._s)


def round_store(x, store):
    x = np.array(x, np.float32, copy=True, order="C")
    lib().fo_round_array(_p(x), x.size, STORE[store])
    return x


def rmsnorm(x, w, eps=1e-6):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    y = np.empty_like(x)
    lib().fo_rmsnorm(_p(x), _p(w), _p(y), x.size, eps)
    return y


def rope_neox(x, pos, theta):
    x = np.array(x, np.float32, copy=True, order="C")
    lib().fo_rope_neox(_p(x), x.size, int(pos), float(theta))
    return x


def slot(pos, is_swa, n_slots=1024):
    return lib().fo_slot(int(pos), int(is_swa), int(n_slots))


def first_key(pos, is_swa, window=513):
    return lib().fo_first_key(int(pos), int(is_swa), int(window))


def qkv_prep(layer, qkv_row, pos):
    qkv_row = np.ascontiguousarray(qkv_row, np.float32)
    q = np.empty(Q_DIM, np.float32)
    k = np.empty(KV_DIM, np.float32)
    v = np.empty(KV_DIM, np.float32)
    lib().fo_qkv_prep(layer.ref, _p(qkv_row), int(pos), _p(q), _p(k), _p(v))
    return q, k, v


def attend(layer, q, K, V, pos, n_threads=1):
    """att [4096] for query q (already normed/roped) at pos over history rows K,V [>=pos+1][512]."""
    q = np.ascontiguousarray(q, np.float32)
    K = np.ascontiguousarray(K, np.float32)
    V = np.ascontiguousarray(V, np.float32)
    assert K.shape[0] >= pos + 1 and V.shape[0] >= pos + 1
    att = np.empty(Q_DIM, np.float32)
    lib().fo_attend(layer.ref, _p(q), _p(K), _p(V), int(pos), _p(att), int(n_threads))
    return att


def attend_split(layer, q, K, V, pos, n_split):
    q = np.ascontiguousarray(q, np.float32)
    K = np.ascontiguousarray(K, np.float32)
    V = np.ascontiguousarray(V, np.float32)
    att = np.empty(Q_DIM, np.float32)
    lib().fo_attend_split(layer.ref, _p(q), _p(K), _p(V), int(pos), int(n_split), _p(att))
    return att


def decode_step(layer, qkv_row, pos, K, V, n_threads=1):
    """Writes history row pos of K, V (arrays [cap][512], modified in place) and returns att [4096]."""
    assert K.dtype == np.float32 and K.flags["C_CONTIGUOUS"] and K.shape[0] > pos
    qkv_row = np.ascontiguousarray(qkv_row, np.float32)
    att = np.empty(Q_DIM, np.float32)
    lib().fo_decode_step(layer.ref, _p(qkv_row), int(pos), _p(K), _p(V), _p(att), int(n_threads))
    return att


def prefill(layer, qkv, p0, K, V, n_threads=1):
    """qkv [T][5120] rows for positions p0..p0+T-1; K,V history [cap][512] (rows < p0 filled).
    Returns att [T][4096]."""
    qkv = np.ascontiguousarray(qkv, np.float32)
    T = qkv.shape[0]
    assert K.shape[0] >= p0 + T
    att = np.empty((T, Q_DIM), np.float32)
    lib().fo_prefill(layer.ref, _p(qkv), QKV_DIM, int(p0), int(T), _p(K), _p(V), _p(att), int(n_threads))
    return att


def prefill_rows(layer, qkv, p0, K, V, r0, r1, n_threads=1):
    """The prefill of qkv [T][5120] at p0 on n_threads threads (fo_prefill_mt): K, V rows
    p0..p0+T-1 are written, att rows [r0, r1) computed (bit-identical to prefill's rows).
    Returns att [T][4096] with the other rows zero."""
    qkv = np.ascontiguousarray(qkv, np.float32)
    T = qkv.shape[0]
    assert K.shape[0] >= p0 + T and 0 <= r0 <= r1 <= T
    att = np.zeros((T, Q_DIM), np.float32)
    assert lib().fo_prefill_mt(layer.ref, _p(qkv), QKV_DIM, int(p0), int(T), int(r0), int(r1), _p(K), _p(V), _p(att),
                               int(n_threads)) == 0
    return att


# ---- weight formats (ggml type ids) ----
W_TYPES = {"f32": 0, "f16": 1, "q8_0": 8, "q5_K": 13, "q6_K": 14, "iq4_xs": 23, "bf16": 30}


def row_bytes(wtype, k):
    return int(lib().fo_row_bytes(W_TYPES[wtype], k))


def dequant_rows(wtype, data, k):
    """All rows of a [n_rows][row_bytes] uint8 array as float32 [n_rows][k]."""
    rb = row_bytes(wtype, k)
    assert rb > 0 and data.dtype == np.uint8 and data.size % rb == 0
    data = np.ascontiguousarray(data).reshape(-1, rb)
    out = np.empty((data.shape[0], k), np.float32)
    for r in range(data.shape[0]):
        assert lib().fo_dequant_row(W_TYPES[wtype], data[r].ctypes.data, k, _p(out[r])) == 0
    return out


def matvec(wtype, data, k, x):
    rb = row_bytes(wtype, k)
    data = np.ascontiguousarray(data)
    n = data.size // rb
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(n, np.float32)
    assert lib().fo_matvec(W_TYPES[wtype], data.ctypes.data, k, n, _p(x), _p(y)) == 0
    return y


REF_DEQUANT = os.path.join(HERE, "_ref", "libref_dequant.so")
_ref_deq = None


def ref_dequant_rows(wtype, data, k):
    """The reference's own ggml dequantize_row_* (oracle/_ref, built from /root/reference);
    None when that build is absent. Only the quantised types (f32/f16/bf16 are plain casts
    in the reference, dequant_row.cpp:23-33)."""
    global _ref_deq
    if not os.path.exists(REF_DEQUANT):
        return None
    if _ref_deq is None:
        _ref_deq = ctypes.CDLL(REF_DEQUANT)
        for t in ("q8_0", "q5_K", "q6_K", "iq4_xs"):
            getattr(_ref_deq, "dequantize_row_" + t).argtypes = [ctypes.c_void_p, _f32p, ctypes.c_int64]
    rb = row_bytes(wtype, k)
    data = np.ascontiguousarray(data).reshape(-1, rb)
    out = np.empty((data.shape[0], k), np.float32)
    fn = getattr(_ref_deq, "dequantize_row_" + wtype)
    for r in range(data.shape[0]):
        fn(data[r].ctypes.data, _p(out[r]), k)
    return out


def random_blocks(wtype, n_rows, k, rng):
    """Random rows of a block format: every byte random except the fp16 scales, which are
    finite halves of moderate size (as quantisers write them)."""
    rb = row_bytes(wtype, k)
    data = rng.integers(0, 256, size=(n_rows, rb), dtype=np.uint8)
    nb = k // int(lib().fo_block_elems(W_TYPES[wtype]))
    bb = int(lib().fo_block_bytes(W_TYPES[wtype]))
    def put_half(off, scale):
        h = (rng.standard_normal((n_rows, nb)) * scale).astype(np.float16).view(np.uint8).reshape(n_rows, nb, 2)
        blocks = data.reshape(n_rows, nb, bb)
        blocks[:, :, off:off + 2] = h
    if wtype == "q8_0":
        put_half(0, 0.01)
    elif wtype == "q5_K":
        put_half(0, 0.002)
        put_half(2, 0.002)
    elif wtype == "q6_K":
        put_half(208, 0.002)
    elif wtype == "iq4_xs":
        put_half(0, 0.001)
    elif wtype in ("f16", "bf16"):
        v = (rng.standard_normal((n_rows, k)) * 0.05).astype(np.float32)
        if wtype == "f16":
            return v.astype(np.float16).view(np.uint8).reshape(n_rows, rb)
        return (v.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).reshape(n_rows, rb)
    elif wtype == "f32":
        return (rng.standard_normal((n_rows, k)) * 0.05).astype(np.float32).view(np.uint8).reshape(n_rows, rb)
    return data


def matvec_f32(W, x, n_threads=8):
    """y = W x for dequantised rows W [n_rows][k], bit-identical to matvec on the packed rows."""
    W = np.ascontiguousarray(W, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(W.shape[0], np.float32)
    lib().fo_matvec_f32(_p(W), W.shape[1], W.shape[0], _p(x), _p(y), int(n_threads))
    return y


class BlockLayer:
    """One layer's attention block as the CPU reference runs it (ref_model.cpp:106-151):
    attn_norm gains, the q/k/v/o weights dequantised to fp32 rows (as dequant_row gives them
    to RefModel::matvec), and the attention parameters (a Layer)."""

    def __init__(self, attn_norm, wq, wk, wv, wo, attn, rms_eps=1e-6):
        self.attn_norm = np.ascontiguousarray(attn_norm, np.float32)
        self.wqkv = np.ascontiguousarray(np.concatenate([wq, wk, wv]), np.float32)
        self.wo = np.ascontiguousarray(wo, np.float32)
        assert self.wqkv.shape == (QKV_DIM, 2048) and self.wo.shape == (2048, Q_DIM)
        self.attn, self.rms_eps = attn, float(rms_eps)


def block_step(blk, x, pos, K, V, n_threads=8):
    """The attention half of RefModel::forward for one layer and one position
    (ref_model.cpp:107-151): xn = rmsnorm(x) * attn_norm, qkv = W xn (double sums),
    att = the sink attention over history rows K, V [cap][512] (row pos written here, in
    the layer's storage type), x + Wo att. Returns (x_new, att)."""
    xn = rmsnorm(x, blk.attn_norm, blk.rms_eps)
    qkv = matvec_f32(blk.wqkv, xn, n_threads)
    att = decode_step(blk.attn, qkv, pos, K, V, n_threads=n_threads)
    o = matvec_f32(blk.wo, att, n_threads)
    return (np.asarray(x, np.float32) + o).astype(np.float32), att


def block_forward(blocks, embd_rows, store, n_threads=8):
    """Hidden state after every position of a model whose layers are `blocks` and whose
    FFN halves are zero (so each layer adds only its attention block): token p at position p,
    embedding row embd_rows[p]. Returns (hidden [n][2048], att [n_layers][n][4096]); the K/V
    history is kept in `store` ("f32": what RefModel keeps; "f16"/"bf16": a GPU cache)."""
    n = embd_rows.shape[0]
    hist = [(np.zeros((n, KV_DIM), np.float32), np.zeros((n, KV_DIM), np.float32)) for _ in blocks]
    hidden = np.empty((n, 2048), np.float32)
    atts = np.empty((len(blocks), n, Q_DIM), np.float32)
    for p in range(n):
        x = np.ascontiguousarray(embd_rows[p], np.float32)
        for il, blk in enumerate(blocks):
            assert blk.attn.store == store
            x, atts[il, p] = block_step(blk, x, p, hist[il][0], hist[il][1], n_threads)
        hidden[p] = x
    return hidden, atts
