"""Shared input generators and comparison helpers for the attention tests.

Inputs follow the benchmark configs: raw q|k|v ~ N(0,1), RMSNorm gains
~ U(0.5, 1.5), per-head sink logits ~ N(0,1), seeded numpy generators.
"""
import numpy as np

import oracle as fo

N_HEAD, N_HEAD_KV, HEAD_DIM = 32, 4, 128
Q_DIM, KV_DIM, QKV_DIM = 4096, 512, 5120

# attention-output tolerance of the hot path vs the oracle (fp16/bf16 KV)
MAX_ABS = 2e-3
MEAN_ABS = 2e-4


def layer_weights(rng):
    q_norm = rng.uniform(0.5, 1.5, HEAD_DIM).astype(np.float32)
    k_norm = rng.uniform(0.5, 1.5, HEAD_DIM).astype(np.float32)
    sinks = rng.standard_normal(N_HEAD).astype(np.float32)
    return q_norm, k_norm, sinks


def oracle_layer(kv, q_norm, k_norm, sinks, store):
    """fo.Layer with the same settings as a flint_attn.KVLayer."""
    return fo.Layer(q_norm, k_norm, sinks, kv.is_swa, kv.has_rope, store, kv.rope_theta, kv.window)


def assert_close(got, want, what="", max_abs=MAX_ABS, mean_abs=MEAN_ABS):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    d = np.abs(got - want)
    mx, mn = float(d.max()), float(d.mean())
    assert mx <= max_abs and mn <= mean_abs, f"{what}: max-abs {mx:.3e} (<= {max_abs}), mean-abs {mn:.3e} (<= {mean_abs})"
    return mx, mn


def to_cache_layout(K, V, n_slots, slots):
    """Linear history rows K,V [n][512] placed at the given slots -> the cache layout in
    32-slot tiles: K [4][n_slots/32][4096] in the tile order of fa.k_tile_offsets(), V
    transposed, [4][n_slots/32][128][32]."""
    import flint_attn as fa
    n = K.shape[0]
    Ks = np.zeros((N_HEAD_KV, n_slots, HEAD_DIM), np.float32)
    Vs = np.zeros((N_HEAD_KV, n_slots, HEAD_DIM), np.float32)
    slots = np.asarray(slots)
    Ks[:, slots, :] = K.reshape(n, N_HEAD_KV, HEAD_DIM).transpose(1, 0, 2)
    Vs[:, slots, :] = V.reshape(n, N_HEAD_KV, HEAD_DIM).transpose(1, 0, 2)
    Kc = np.zeros((N_HEAD_KV, n_slots // 32, 32 * HEAD_DIM), np.float32)
    Kc[:, :, fa.k_tile_offsets().reshape(-1)] = Ks.reshape(N_HEAD_KV, n_slots // 32, 32 * HEAD_DIM)
    Vc = np.ascontiguousarray(Vs.reshape(N_HEAD_KV, n_slots // 32, 32, HEAD_DIM).transpose(0, 1, 3, 2))
    return Kc, Vc


def k_close(a, b, dtype):
    """Cache K written by the GPU vs the oracle's: both normalise (and rotate) in fp32 before
    rounding to the 16-bit type, so a value may land one unit in the last place away, and
    values that RoPE brings near zero by cancellation may differ by the fp32 error (~1e-7)."""
    a64, b64 = np.asarray(a, np.float64), np.asarray(b, np.float64)
    mant = 10 if dtype == "f16" else 7
    ulp = np.abs(b64) * 2.0 ** -mant
    return bool(np.all(np.abs(a64 - b64) <= ulp * 1.0001 + 1e-5))
