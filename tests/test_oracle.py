"""Pins the CPU oracle (oracle/flint_oracle.c) against library routines,
closed forms and invariants, so that a dropped term, a wrong sign or index, or
a transposed operand in the restatement fails here. Its bit-exact agreement
with the reference's own CPU forward is in test_ref_parity.py."""
import numpy as np
import pytest
import scipy.special
import torch

import oracle as fo
from helpers import HEAD_DIM, N_HEAD, Q_DIM, layer_weights


def _sweep_floats(rng, n=200000):
    """Random float32 bit patterns over the f16 range plus exact f16 halfway points."""
    bits = rng.integers(0x33000000, 0x47900000, n, dtype=np.uint32)  # ~3e-8 .. 73728
    x = bits.view(np.float32)
    h = rng.integers(0, 0x7bff, 20000, dtype=np.uint16).view(np.float16).astype(np.float64)
    nxt = np.nextafter(h.astype(np.float16), np.float16(np.inf)).astype(np.float64)
    ties = ((h + nxt) / 2).astype(np.float32)  # exactly representable in float32
    out = np.concatenate([x, -x, ties, -ties, np.float32([0.0, 65504, 65519.99, 65520, 1e-9, 2 ** -25, 2 ** -24])])
    return out[np.isfinite(out)]


def test_round_f16_matches_numpy():
    x = _sweep_floats(np.random.default_rng(0))
    got = fo.round_store(x, "f16")
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_round_bf16_matches_torch():
    rng = np.random.default_rng(1)
    x = np.concatenate([(rng.standard_normal(100000) * 10.0 ** rng.integers(-30, 30, 100000)).astype(np.float32),
                        (rng.integers(0, 1 << 31, 50000, dtype=np.uint32) & 0xFFFF0000 | 0x8000).view(np.float32)])
    x = x[np.isfinite(x)].astype(np.float32)
    got = fo.round_store(x, "bf16")
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_rmsnorm_constant_vector_closed_form():
    g = np.random.default_rng(2).uniform(0.5, 1.5, HEAD_DIM).astype(np.float32)
    for c in (1.0, -3.5, 1e-3, 250.0):
        y = fo.rmsnorm(np.full(HEAD_DIM, c, np.float32), g)
        want = g.astype(np.float64) * c / np.sqrt(c * c + 1e-6)
        np.testing.assert_allclose(y, want, rtol=2e-6)


def test_rmsnorm_random_vs_float64():
    rng = np.random.default_rng(3)
    for _ in range(20):
        x = (rng.standard_normal(HEAD_DIM) * rng.uniform(0.01, 100)).astype(np.float32)
        w = rng.uniform(0.5, 1.5, HEAD_DIM).astype(np.float32)
        x64 = x.astype(np.float64)
        want = x64 / np.sqrt(np.mean(x64 ** 2) + 1e-6) * w
        np.testing.assert_allclose(fo.rmsnorm(x, w), want, rtol=2e-6, atol=1e-7)


def test_rope_pos0_identity():
    x = np.random.default_rng(4).standard_normal(HEAD_DIM).astype(np.float32)
    assert np.array_equal(fo.rope_neox(x, 0, 1e4), x)


@pytest.mark.parametrize("theta", [1e4, 1e6])
def test_rope_unit_vectors_neox_pairing(theta):
    """e_i rotates in the (i, i+64) plane by pos * theta^(-2i/128) (NEOX pairing, not interleaved)."""
    for pos in (1, 7, 100):
        for i in (0, 1, 5, 31, 63):
            e = np.zeros(HEAD_DIM, np.float32)
            e[i] = 1
            y = fo.rope_neox(e, pos, theta)
            ang = pos * theta ** (-2.0 * i / HEAD_DIM)
            want = np.zeros(HEAD_DIM)
            want[i], want[i + 64] = np.cos(ang), np.sin(ang)
            tol = 1e-6 + 1.2e-7 * pos * max(1.0, ang / pos)  # the float angle pos*freq carries ~|ang|*2^-24
            np.testing.assert_allclose(y, want, atol=tol)
            e2 = np.zeros(HEAD_DIM, np.float32)
            e2[i + 64] = 1
            y2 = fo.rope_neox(e2, pos, theta)
            want2 = np.zeros(HEAD_DIM)
            want2[i], want2[i + 64] = -np.sin(ang), np.cos(ang)
            np.testing.assert_allclose(y2, want2, atol=tol)


def test_rope_preserves_pair_norms_and_relative_position():
    rng = np.random.default_rng(5)
    q = rng.standard_normal(HEAD_DIM).astype(np.float32)
    k = rng.standard_normal(HEAD_DIM).astype(np.float32)
    for pos in (3, 250, 1300):
        y = fo.rope_neox(q, pos, 1e4).astype(np.float64)
        q64 = q.astype(np.float64)
        np.testing.assert_allclose(y[:64] ** 2 + y[64:] ** 2, q64[:64] ** 2 + q64[64:] ** 2, rtol=1e-5)
    # <R(m) q, R(n) k> depends on m - n only
    d0 = float(np.dot(fo.rope_neox(q, 40, 1e4).astype(np.float64), fo.rope_neox(k, 10, 1e4)))
    for shift in (5, 37, 200):
        d = float(np.dot(fo.rope_neox(q, 40 + shift, 1e4).astype(np.float64), fo.rope_neox(k, 10 + shift, 1e4)))
        assert abs(d - d0) < 2e-4 * (1 + abs(d0))


def _layer(is_swa=0, has_rope=0, sinks=None, store="f32", seed=6):
    qn, kn, sk = layer_weights(np.random.default_rng(seed))
    if sinks is not None:
        sk = np.full(N_HEAD, sinks, np.float32)
    return fo.Layer(qn, kn, sk, is_swa, has_rope, store)


def _scores64(q, K, pos, first=0):
    qh = q.reshape(N_HEAD, HEAD_DIM).astype(np.float64)
    Kh = K[first:pos + 1].reshape(-1, 4, HEAD_DIM).astype(np.float64)
    return np.einsum("hd,jhd->hj", qh, Kh[:, np.arange(N_HEAD) // 8, :]) / np.sqrt(HEAD_DIM)


def test_attend_one_key_with_sink_closed_form():
    rng = np.random.default_rng(7)
    L = _layer()
    q = rng.standard_normal(Q_DIM).astype(np.float32)
    K = rng.standard_normal((1, 512)).astype(np.float32)
    V = rng.standard_normal((1, 512)).astype(np.float32)
    att = fo.attend(L, q, K, V, 0).reshape(N_HEAD, HEAD_DIM)
    s = _scores64(q, K, 0)[:, 0]
    w = np.exp(s) / (np.exp(s) + np.exp(L.sinks.astype(np.float64)))
    want = w[:, None] * V.reshape(4, HEAD_DIM)[np.arange(N_HEAD) // 8]
    np.testing.assert_allclose(att, want, rtol=2e-5, atol=1e-6)


def test_attend_identical_keys_closed_form():
    rng = np.random.default_rng(8)
    L = _layer()
    n = 50
    q = rng.standard_normal(Q_DIM).astype(np.float32)
    K = np.tile(rng.standard_normal((1, 512)).astype(np.float32), (n, 1))
    V = np.tile(rng.standard_normal((1, 512)).astype(np.float32), (n, 1))
    att = fo.attend(L, q, K, V, n - 1).reshape(N_HEAD, HEAD_DIM)
    s = _scores64(q, K, 0)[:, 0]
    w = n * np.exp(s) / (n * np.exp(s) + np.exp(L.sinks.astype(np.float64)))
    want = w[:, None] * V[0].reshape(4, HEAD_DIM)[np.arange(N_HEAD) // 8]
    np.testing.assert_allclose(att, want, rtol=2e-5, atol=1e-6)


def test_attend_sink_limits():
    rng = np.random.default_rng(9)
    n = 300
    q = rng.standard_normal(Q_DIM).astype(np.float32)
    K = rng.standard_normal((n, 512)).astype(np.float32)
    V = rng.standard_normal((n, 512)).astype(np.float32)
    # sink -> -inf: plain softmax attention
    att = fo.attend(_layer(sinks=-1e4), q, K, V, n - 1).reshape(N_HEAD, HEAD_DIM)
    p = scipy.special.softmax(_scores64(q, K, n - 1), axis=1)
    Vh = V.reshape(n, 4, HEAD_DIM).astype(np.float64)[:, np.arange(N_HEAD) // 8, :]
    want = np.einsum("hj,jhd->hd", p, Vh)
    np.testing.assert_allclose(att, want, rtol=1e-4, atol=2e-6)
    # sink -> +inf: everything goes to the sink
    att = fo.attend(_layer(sinks=80.0), q, K, V, n - 1)
    assert np.abs(att).max() < 1e-20


@pytest.mark.parametrize("is_swa", [0, 1])
def test_attend_window_brute_force(is_swa):
    """With all-zero keys every key in the window weighs exp(0); V[j][d] = j marks which keys count."""
    L = _layer(is_swa=is_swa, sinks=0.0)
    n = 1600
    q = np.random.default_rng(10).standard_normal(Q_DIM).astype(np.float32)
    K = np.zeros((n, 512), np.float32)
    V = np.repeat(np.arange(n, dtype=np.float32)[:, None], 512, axis=1)
    for pos in (0, 1, 511, 512, 513, 600, 1023, 1024, 1599):
        first = max(0, pos - 512) if is_swa else 0
        keys = np.arange(first, pos + 1, dtype=np.float64)
        want = keys.sum() / (len(keys) + 1.0)  # + exp(sink - 0) = 1 in the denominator
        att = fo.attend(L, q, K, V, pos)
        np.testing.assert_allclose(att, want, rtol=1e-6)
        assert fo.first_key(pos, is_swa) == first


@pytest.mark.parametrize("n_split", [1, 2, 16, 32, 64])
def test_attend_split_merge_equals_single_pass(n_split):
    rng = np.random.default_rng(11)
    L = _layer(is_swa=0)
    n = 2000
    q = rng.standard_normal(Q_DIM).astype(np.float32)
    K = rng.standard_normal((n, 512)).astype(np.float32)
    K[rng.random(n) < 0.01] *= 8
    V = rng.standard_normal((n, 512)).astype(np.float32)
    a = fo.attend(L, q, K, V, n - 1)
    b = fo.attend_split(L, q, K, V, n - 1, n_split)
    np.testing.assert_allclose(b, a, rtol=1e-5, atol=1e-6)


def test_ring_slots_brute_force():
    """The window's slots are distinct, slot(pos) never holds a live key of the window, slot = pos mod 1024."""
    for pos in range(4096):
        first = fo.first_key(pos, 1)
        assert first == max(0, pos - 512)
        live = {fo.slot(j, 1) for j in range(first, pos)}
        assert len(live) == pos - first
        s = fo.slot(pos, 1)
        assert s == pos % 1024 and s not in live
        assert fo.slot(pos, 0) == pos


def test_decode_step_rounds_current_kv_and_matches_prefill():
    rng = np.random.default_rng(12)
    qn, kn, sk = layer_weights(rng)
    L = fo.Layer(qn, kn, sk, 1, 1, "f16", 1e6)
    n = 40
    qkv = rng.standard_normal((n, 5120)).astype(np.float32)
    K = np.zeros((n, 512), np.float32)
    V = np.zeros((n, 512), np.float32)
    outs = np.stack([fo.decode_step(L, qkv[p], p, K, V) for p in range(n)])
    # the cache rows hold f16 values; V is the raw v rounded
    assert np.array_equal(V, qkv[:, 4608:].astype(np.float16).astype(np.float32))
    assert np.array_equal(K, K.astype(np.float16).astype(np.float32))
    K2 = np.zeros_like(K)
    V2 = np.zeros_like(V)
    assert np.array_equal(fo.prefill(L, qkv, 0, K2, V2), outs)
    # attending with the rounded history reproduces the step outputs
    q, _, _ = fo.qkv_prep(L, qkv[n - 1], n - 1)
    assert np.array_equal(fo.attend(L, q, K, V, n - 1), outs[-1])


@pytest.mark.parametrize("is_swa,p0", [(0, 0), (1, 37), (1, 600)])
def test_prefill_rows_threaded_equals_prefill(is_swa, p0):
    """fo_prefill_mt (the CPU baseline's prefill: q/k/v of every token, then (row, head) pairs on
    many threads) writes the same K/V history and the same att rows, bit for bit, as the
    token-by-token fo_prefill; rows outside [r0, r1) are left zero."""
    rng = np.random.default_rng(21 + p0)
    qn, kn, sk = layer_weights(rng)
    L = fo.Layer(qn, kn, sk, is_swa, 1, "bf16", 1e6)
    T = 90
    qkv = rng.standard_normal((T, 5120)).astype(np.float32)
    hist = rng.standard_normal((p0, 512)).astype(np.float32)
    K = np.zeros((p0 + T, 512), np.float32)
    V = np.zeros((p0 + T, 512), np.float32)
    K[:p0] = fo.round_store(hist, "bf16")
    V[:p0] = fo.round_store(hist[::-1], "bf16")
    K2, V2 = K.copy(), V.copy()
    want = fo.prefill(L, qkv, p0, K, V)
    got = fo.prefill_rows(L, qkv, p0, K2, V2, 10, 77, n_threads=7)
    assert np.array_equal(K, K2) and np.array_equal(V, V2)
    assert np.array_equal(got[10:77], want[10:77])
    assert not got[:10].any() and not got[77:].any()
