"""Weight formats of the attention projections on the CPU: the oracle's dequantisation
(oracle/flint_oracle.c fo_dequant_row) against the reference's own ggml dequantize_row_*
(oracle/_ref, /root/reference/src/ref/dequant_gen.c) and the golden rows made from it, closed
forms of each format, the oracle's matvec (ref_model.cpp:74-93), and the host-side checks of
the C-ABI entry points (include/flint_proj.h), which fail before any GPU work."""
import ctypes
import os

import numpy as np
import pytest

import flint_attn as fa
import oracle

HERE = os.path.dirname(os.path.abspath(__file__))
QUANT = ("q8_0", "q5_K", "q6_K", "iq4_xs")
ALL = QUANT + ("f32", "f16", "bf16")


def test_row_bytes_follow_the_ggml_block_sizes():
    # ggml-common.h static_asserts: q8_0 2+32, q5_K 2*2+12+128+32, q6_K 2+16+192, iq4_xs 2+2+4+128
    sizes = {"q8_0": (32, 34), "q5_K": (256, 176), "q6_K": (256, 210), "iq4_xs": (256, 136),
             "f32": (1, 4), "f16": (1, 2), "bf16": (1, 2)}
    for t, (be, bb) in sizes.items():
        for k in (256, 512, 2048, 4096):
            assert oracle.row_bytes(t, k) == k // be * bb
            assert fa.row_bytes(t, k) == k // be * bb
    assert oracle.row_bytes("q5_K", 300) == -1 and fa.row_bytes("q5_K", 300) == -1
    assert fa.lib().flint_w_row_bytes(2, 2048) == -1  # q4_0: not an attention format


@pytest.mark.parametrize("wtype", QUANT)
def test_dequant_matches_golden_rows(wtype):
    z = np.load(os.path.join(HERE, "golden", "weight_rows.npz"))
    got = oracle.dequant_rows(wtype, z[wtype + "_rows"], 512)
    assert np.array_equal(got.view(np.uint32), z[wtype + "_bits"])


@pytest.mark.parametrize("wtype", QUANT)
@pytest.mark.parametrize("k", [256, 2048, 4096])
def test_dequant_bit_exact_against_reference_ggml(wtype, k):
    rng = np.random.default_rng(k + len(wtype))
    rows = oracle.random_blocks(wtype, 16, k, rng)
    ref = oracle.ref_dequant_rows(wtype, rows, k)
    if ref is None:
        pytest.skip("oracle/_ref/libref_dequant.so not built (needs /root/reference)")
    got = oracle.dequant_rows(wtype, rows, k)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_dequant_closed_forms():
    rng = np.random.default_rng(7)
    # q8_0 with d = 1.0: the int8 quants themselves
    rows = oracle.random_blocks("q8_0", 2, 256, rng)
    blocks = rows.reshape(2, 8, 34)
    blocks[:, :, 0], blocks[:, :, 1] = 0x00, 0x3C
    want = blocks[:, :, 2:].view(np.int8).reshape(2, 256).astype(np.float32)
    assert np.array_equal(oracle.dequant_rows("q8_0", rows, 256), want)
    # zero super-block scales give zero rows (q5_K also needs dmin = 0)
    for t, offs in (("q5_K", (0, 2)), ("q6_K", (208,)), ("iq4_xs", (0,))):
        rows = oracle.random_blocks(t, 2, 512, rng)
        bb = rows.shape[1] // 2
        for o in offs:
            rows.reshape(2, 2, bb)[:, :, o:o + 2] = 0
        assert np.all(oracle.dequant_rows(t, rows, 512) == 0)
    # q6_K: quants 32 (low nibble 0, high bits 2) with scale 1 and d = 1 give zero
    row = np.zeros(210, np.uint8)
    row[128:192] = 0xAA
    row[192:208] = 1
    row[208:210] = (0x00, 0x3C)
    assert np.all(oracle.dequant_rows("q6_K", row[None], 256) == 0)
    # iq4_xs: scale code 33 (ls - 32 = 1) and d = 1 give the code book itself
    row = np.zeros(136, np.uint8)
    row[0:2] = (0x00, 0x3C)
    row[2:4] = (0x00, 0x00)   # scales_h: high bits 0 ...
    row[4:8] = 0x11           # ... scales_l nibbles 1: ls = 1 -> (1 - 32) = -31
    qs = np.arange(16, dtype=np.uint8)
    row[8:24] = qs | (qs << 4)
    table = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.float32)
    got = oracle.dequant_rows("iq4_xs", row[None], 256)[0]
    assert np.array_equal(got[:16], -31 * table) and np.array_equal(got[16:32], -31 * table)
    # f16 / bf16 / f32 rows: plain casts
    v = (rng.standard_normal(64) * 3).astype(np.float32)
    assert np.array_equal(oracle.dequant_rows("f16", v.astype(np.float16).view(np.uint8)[None], 64)[0],
                          v.astype(np.float16).astype(np.float32))
    bf = (v.view(np.uint32) >> 16).astype(np.uint16)
    assert np.array_equal(oracle.dequant_rows("bf16", bf.view(np.uint8)[None], 64)[0],
                          (bf.astype(np.uint32) << 16).view(np.float32))
    assert np.array_equal(oracle.dequant_rows("f32", v.view(np.uint8)[None], 64)[0], v)
    # every half, through f16 rows: subnormals, infinities
    h = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    h = h[(h & 0x7C00) != 0x7C00]  # finite only (nan payloads aside)
    got = oracle.dequant_rows("f16", h.view(np.uint8)[None], h.size)[0]
    assert np.array_equal(got, h.view(np.float16).astype(np.float32))


def test_matvec_selects_and_matches_float64():
    rng = np.random.default_rng(3)
    k = 512
    x = rng.standard_normal(k).astype(np.float32)
    # one-hot q8_0 rows (d = 1, a single quant 1): each row picks one x exactly
    n = 16
    picks = rng.choice(k, n, replace=False)
    rows = np.zeros((n, k // 32, 34), np.uint8)
    rows[:, :, 1] = 0x3C
    for r, i in enumerate(picks):
        rows[r, i // 32, 2 + i % 32] = 1
    assert np.array_equal(oracle.matvec("q8_0", rows.reshape(n, -1), k, x), x[picks])
    for t in ALL:
        w = oracle.random_blocks(t, 24, k, rng)
        dense = oracle.dequant_rows(t, w, k).astype(np.float64)
        want = dense @ x.astype(np.float64)
        got = oracle.matvec(t, w, k, x)
        np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6 * np.abs(dense).sum(1).max())
        # linear in x
        got2 = oracle.matvec(t, w, k, 2 * x)
        np.testing.assert_allclose(got2, 2 * got, rtol=1e-6, atol=1e-6)


def _err():
    return ctypes.create_string_buffer(256)


def test_projection_entry_points_reject_bad_arguments():
    L = fa.lib()
    e = _err()
    assert L.flint_w_get_row(2, ctypes.c_void_p(16), 2048, 0, ctypes.c_void_p(16), None, e, 256) == -1
    assert b"unsupported" in e.value
    assert L.flint_w_get_row(8, None, 2048, 0, ctypes.c_void_p(16), None, e, 256) == -1
    assert b"NULL" in e.value
    assert L.flint_w_get_row(8, ctypes.c_void_p(16), 2048, 0, ctypes.c_void_p(20), None, e, 256) == -1
    assert b"aligned" in e.value
    rows = (ctypes.c_int32 * 3)(0, 7, 3)
    assert L.flint_w_get_rows(8, ctypes.c_void_p(16), 2048, 7, rows, 3, ctypes.c_void_p(16), None, e, 256) == -1
    assert b"get_rows: row 7 out of range" in e.value
    assert L.flint_w_get_rows(8, ctypes.c_void_p(16), 2048, 8, None, 3, ctypes.c_void_p(16), None, e, 256) == -1
    assert b"NULL" in e.value
    assert L.flint_w_get_rows(8, ctypes.c_void_p(16), 2048, 8, rows, 0, ctypes.c_void_p(16), None, e, 256) == -1
    assert b"n must be" in e.value
    neg = (ctypes.c_int32 * 1)(-1)
    assert L.flint_w_get_rows(8, ctypes.c_void_p(16), 2048, 8, neg, 1, ctypes.c_void_p(16), None, e, 256) == -1
    assert b"negative row" in e.value
    good = fa.WeightDesc(16, fa.W_TYPES["q8_0"])
    odd = fa.WeightDesc(24, fa.W_TYPES["q8_0"])
    bad = fa.WeightDesc(16, 2)
    p = ctypes.c_void_p(64)
    assert L.flint_attn_qkv_proj(ctypes.byref(good), ctypes.byref(bad), ctypes.byref(good), p, p, 1e-6, p, None, e,
                                 256) == -1
    assert b"wk" in e.value and b"unsupported" in e.value
    assert L.flint_attn_qkv_proj(ctypes.byref(good), ctypes.byref(good), ctypes.byref(odd), p, p, 1e-6, p, None, e,
                                 256) == -1
    assert b"wv" in e.value and b"aligned" in e.value
    assert L.flint_attn_qkv_proj(None, ctypes.byref(good), ctypes.byref(good), p, p, 1e-6, p, None, e, 256) == -1
    assert b"wq" in e.value
    assert L.flint_attn_o_proj(ctypes.byref(good), None, p, None, e, 256) == -1
    assert b"NULL" in e.value
