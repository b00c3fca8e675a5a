"""Fused decode attention on the GPU against the CPU oracle (benchmark configs 1-3
and the batched form of config 5), through the C ABI (flint_attn_decode,
flint_attn_decode_batch). Tolerance: max-abs 2e-3 and mean-abs 2e-4 on the
attention output; ring slot contents bit-exact for V (K within 1 ulp of the
cache dtype: its norm/rope runs in fp32 on both sides)."""
import numpy as np
import pytest
import torch

import flint_attn as fa
import oracle as fo
from helpers import (HEAD_DIM, k_close, KV_DIM, N_HEAD_KV, QKV_DIM, Q_DIM, assert_close, layer_weights, oracle_layer,
                     to_cache_layout)

pytestmark = pytest.mark.gpu

TORCH_DT = {"f16": torch.float16, "bf16": torch.bfloat16}


def _say(msg):
    print(f"\n[gpu-test] {msg}", flush=True)


def _fill_cache(kv, K, V, slots, seq=0):
    Kc, Vc = to_cache_layout(K, V, kv.n_slots, slots)
    kv.k[seq].copy_(torch.from_numpy(Kc).to(kv.torch_dtype))
    kv.v[seq].copy_(torch.from_numpy(Vc).to(kv.torch_dtype))


def _history(rng, n, store, outlier_frac=0.0):
    K = rng.standard_normal((n, KV_DIM)).astype(np.float32)
    V = rng.standard_normal((n, KV_DIM)).astype(np.float32)
    if outlier_frac:
        K[rng.random(n) < outlier_frac] *= 8
        V[rng.random(n) < outlier_frac] *= 8
    return fo.round_store(K, store), fo.round_store(V, store)



@pytest.mark.parametrize("store", ["f16", "bf16"])
def test_decode_swa_ring_steps_config2(cuda, store):
    """Config 2: SWA layer, RoPE, 1024-slot ring, window 513, positions 0..1300 one token at a time."""
    n = 1301 if store == "f16" else 700
    _say(f"decode swa ring steps store={store} n={n} seed=1")
    rng = np.random.default_rng(1)
    qn, kn, sk = layer_weights(rng)
    kv = fa.KVLayer(is_swa=True, has_rope=True, kv_dtype=store, rope_theta=1e6, q_norm=qn, k_norm=kn, sinks=sk)
    L = oracle_layer(kv, qn, kn, sk, store)
    qkv = rng.standard_normal((n, QKV_DIM)).astype(np.float32)
    dq = torch.from_numpy(qkv).to(cuda)
    att = torch.zeros((n, Q_DIM), device=cuda)
    for pos in range(n):
        kv.decode(dq[pos], att[pos], pos)
    torch.cuda.synchronize()
    K = np.zeros((n, KV_DIM), np.float32)
    V = np.zeros((n, KV_DIM), np.float32)
    want = fo.prefill(L, qkv, 0, K, V, n_threads=8)
    got = att.cpu().numpy()
    for pos in range(n):
        assert_close(got[pos], want[pos], f"pos {pos}")
    assert_close(got, want, "all steps")
    # ring: slot p & 1023 holds position p for the last 1024 positions
    vc = kv.v_slots()[0].float().cpu().numpy()  # [4][1024][128]
    kc = kv.k_slots()[0].float().cpu().numpy()  # [4][1024][128]
    for p in range(max(0, n - 1024), n):
        s = p & 1023
        assert np.array_equal(vc[:, s, :], V[p].reshape(N_HEAD_KV, HEAD_DIM)), f"V slot {s} pos {p}"
        assert k_close(kc[:, s, :], K[p].reshape(N_HEAD_KV, HEAD_DIM), store), f"K slot {s} pos {p}"


def test_decode_full_rope_config1(cuda):
    """Config 1 shapes on the GPU: full layer with NEOX RoPE theta=1e6, 1024 cached positions, seed 0."""
    _say("decode full rope 1024 cached seed=0")
    rng = np.random.default_rng(0)
    qn, kn, sk = layer_weights(rng)
    n = 1024
    kv = fa.KVLayer(is_swa=False, has_rope=True, n_slots=1056, kv_dtype="f16", rope_theta=1e6, q_norm=qn,
                    k_norm=kn, sinks=sk)
    L = oracle_layer(kv, qn, kn, sk, "f16")
    K, V = _history(rng, n + 1, "f16")
    _fill_cache(kv, K[:n], V[:n], np.arange(n))
    qkv = rng.standard_normal(QKV_DIM).astype(np.float32)
    att = torch.zeros(Q_DIM, device=cuda)
    for kps in (0, 256, 1024):
        kv.decode(torch.from_numpy(qkv).to(cuda), att, n, keys_per_split=kps)
        torch.cuda.synchronize()
        want = fo.decode_step(L, qkv, n, K, V, n_threads=8)
        assert_close(att.cpu().numpy(), want, f"keys_per_split={kps}")


@pytest.mark.parametrize("store", ["f16", "bf16"])
def test_decode_split_k_32k_config3(cuda, store):
    """Config 3: full layer (NoPE), 32768 cached positions, 1% outlier rows x8, seed 2;
    16..128 splits with the LSE merge, all equal to the oracle and to each other."""
    _say(f"decode split-k 32k store={store} seed=2")
    rng = np.random.default_rng(2)
    qn, kn, sk = layer_weights(rng)
    n = 32768
    kv = fa.KVLayer(is_swa=False, has_rope=False, n_slots=n + 32, kv_dtype=store, q_norm=qn, k_norm=kn, sinks=sk)
    L = oracle_layer(kv, qn, kn, sk, store)
    K, V = _history(rng, n + 1, store, outlier_frac=0.01)
    _fill_cache(kv, K[:n], V[:n], np.arange(n))
    qkv = rng.standard_normal(QKV_DIM).astype(np.float32)
    dq = torch.from_numpy(qkv).to(cuda)
    want = fo.decode_step(L, qkv, n, K.copy(), V.copy(), n_threads=8)
    outs = {}
    for kps in (0, 256, 512, 1024, 2048, 32768):  # auto, 128, 64, 32, 16, 1 splits
        att = torch.zeros(Q_DIM, device=cuda)
        kv.decode(dq, att, n, keys_per_split=kps)
        torch.cuda.synchronize()
        outs[kps] = att.cpu().numpy()
        assert_close(outs[kps], want, f"keys_per_split={kps}")
    for kps, o in outs.items():
        np.testing.assert_allclose(o, outs[32768], rtol=0, atol=2e-5 * max(1.0, np.abs(want).max()))
    # the current token's K/V landed in slot n
    vc = kv.v_slots()[0, :, n, :].float().cpu().numpy()
    assert np.array_equal(vc, fo.round_store(qkv[4608:], store).reshape(N_HEAD_KV, HEAD_DIM))


@pytest.mark.parametrize("store", ["f16", "bf16"])
def test_decode_very_long_context(cuda, store):
    """One sequence at 196611 cached positions (a ragged last tile; splits of ~130 tiles from the
    auto plan), and the same call with 9 and 65 splits, against the oracle; the current token's
    K/V land in slot pos."""
    n = 196611
    _say(f"decode very long context n={n} store={store}")
    rng = np.random.default_rng(23)
    qn, kn, sk = layer_weights(rng)
    kv = fa.KVLayer(is_swa=False, has_rope=True, n_slots=n + 29, kv_dtype=store, rope_theta=1e6, q_norm=qn, k_norm=kn,
                    sinks=sk)
    L = oracle_layer(kv, qn, kn, sk, store)
    K, V = _history(rng, n + 1, store)
    _fill_cache(kv, K[:n], V[:n], np.arange(n))
    qkv = rng.standard_normal(QKV_DIM).astype(np.float32)
    dq = torch.from_numpy(qkv).to(cuda)
    want = fo.decode_step(L, qkv, n, K, V, n_threads=8)
    for kps in (0, 24576, 3072):  # auto, 9, 65 splits
        att = torch.zeros(Q_DIM, device=cuda)
        kv.decode(dq, att, n, keys_per_split=kps)
        torch.cuda.synchronize()
        assert_close(att.cpu().numpy(), want, f"keys_per_split={kps}")
    vc = kv.v_slots()[0, :, n, :].float().cpu().numpy()
    assert np.array_equal(vc, fo.round_store(qkv[4608:], store).reshape(N_HEAD_KV, HEAD_DIM))


def test_decode_edge_positions_and_sinks(cuda):
    """pos 0 (current token only), 1, 31/32/33 around a tile edge, extreme sinks."""
    _say("decode edge positions and sinks")
    rng = np.random.default_rng(21)
    for sink_val in (None, -30.0, 30.0):
        qn, kn, sk = layer_weights(rng)
        if sink_val is not None:
            sk[:] = sink_val
        kv = fa.KVLayer(is_swa=False, has_rope=True, n_slots=128, kv_dtype="f16", q_norm=qn, k_norm=kn, sinks=sk)
        L = oracle_layer(kv, qn, kn, sk, "f16")
        n = 70
        qkv = rng.standard_normal((n, QKV_DIM)).astype(np.float32)
        dq = torch.from_numpy(qkv).to(cuda)
        att = torch.zeros((n, Q_DIM), device=cuda)
        for pos in range(n):
            kv.decode(dq[pos], att[pos], pos)
        torch.cuda.synchronize()
        K = np.zeros((n, KV_DIM), np.float32)
        V = np.zeros((n, KV_DIM), np.float32)
        want = fo.prefill(L, qkv, 0, K, V)
        assert_close(att.cpu().numpy(), want, f"sink={sink_val}")


@pytest.mark.parametrize("is_swa", [False, True])
def test_decode_batch_matches_single(cuda, is_swa):
    """Independent sequences at mixed positions in one launch == one launch per sequence == oracle."""
    _say(f"decode batch is_swa={is_swa}")
    rng = np.random.default_rng(4)
    qn, kn, sk = layer_weights(rng)
    positions = [0, 5, 700, 3000, 1025, 64]
    n_slots = 1024 if is_swa else 3072
    kv = fa.KVLayer(is_swa=is_swa, has_rope=is_swa, n_slots=n_slots, kv_dtype="f16", q_norm=qn, k_norm=kn,
                    sinks=sk, n_seq=len(positions))
    kv1 = fa.KVLayer(is_swa=is_swa, has_rope=is_swa, n_slots=n_slots, kv_dtype="f16", q_norm=qn, k_norm=kn,
                     sinks=sk)
    L = oracle_layer(kv, qn, kn, sk, "f16")
    qkv = rng.standard_normal((len(positions), QKV_DIM)).astype(np.float32)
    wants, hist = [], []
    for s, p in enumerate(positions):
        if not is_swa and p >= n_slots:
            positions[s] = p = n_slots - 1
        K, V = _history(rng, p + 1, "f16")
        first = max(0, p - 1023) if is_swa else 0
        _fill_cache(kv, K[first:p], V[first:p], np.arange(first, p) & (n_slots - 1) if is_swa else np.arange(p), s)
        wants.append(fo.decode_step(L, qkv[s], p, K.copy(), V.copy(), n_threads=8))
        hist.append((K, V, first))
    dq = torch.from_numpy(qkv).to(cuda)
    att = torch.zeros((len(positions), Q_DIM), device=cuda)
    kv.decode(dq, att, positions)
    torch.cuda.synchronize()
    got = att.cpu().numpy()
    for s, p in enumerate(positions):
        assert_close(got[s], wants[s], f"seq {s} pos {p}")
        K, V, first = hist[s]
        _fill_cache(kv1, K[first:p], V[first:p], np.arange(first, p) & (n_slots - 1) if is_swa else np.arange(p))
        one = torch.zeros(Q_DIM, device=cuda)
        kv1.decode(dq[s], one, p)
        torch.cuda.synchronize()
        np.testing.assert_allclose(got[s], one.cpu().numpy(), rtol=0, atol=1e-5)


@pytest.mark.parametrize("positions", [[4100, 17000, 40000, 65535, 700], [9000, 33000, 700]],
                         ids=["5seq", "3seq"])
def test_decode_batch_long_contexts_auto_split(cuda, positions):
    """Config-5 shape: independent sequences at long, mixed contexts in one launch, with the
    automatic split plan (each sequence's key range cut into its own number of equal splits,
    so the sequences differ in split count and split length up to the grid's width; a
    sequence with one split is written directly by the decode kernel). Every sequence equals
    the oracle. Up to four sequences, the merge runs four workgroups per head (each a quarter
    of the head's dims); with more, one per head: the 3- and 5-sequence cases take one each."""
    _say(f"decode batch, long mixed contexts {positions}, auto split")
    rng = np.random.default_rng(44)
    qn, kn, sk = layer_weights(rng)
    n_slots = (max(positions) + 1 + 31) // 32 * 32 + 32
    kv = fa.KVLayer(is_swa=False, has_rope=False, n_slots=n_slots, kv_dtype="f16", q_norm=qn, k_norm=kn, sinks=sk,
                    n_seq=len(positions))
    L = oracle_layer(kv, qn, kn, sk, "f16")
    qkv = rng.standard_normal((len(positions), QKV_DIM)).astype(np.float32)
    wants = []
    for s, p in enumerate(positions):
        K, V = _history(rng, p + 1, "f16", outlier_frac=0.01)
        _fill_cache(kv, K[:p], V[:p], np.arange(p), s)
        wants.append(fo.decode_step(L, qkv[s], p, K.copy(), V.copy(), n_threads=8))
    dq = torch.from_numpy(qkv).to(cuda)
    att = torch.zeros((len(positions), Q_DIM), device=cuda)
    kv.decode(dq, att, positions)
    torch.cuda.synchronize()
    got = att.cpu().numpy()
    for s, p in enumerate(positions):
        assert_close(got[s], wants[s], f"seq {s} pos {p}")


@pytest.mark.parametrize("store", ["f16", "bf16"])
def test_decode_batch_64_sequences(cuda, store):
    """The largest batch (64 sequences, every entry of the per-sequence tables the decode
    kernel reads one per lane), full layer, positions from 0 to 4000 (one split each, or
    several with the merge), the first and last sequences the longest; every sequence
    equals the oracle."""
    _say(f"decode batch of 64 sequences store={store}")
    rng = np.random.default_rng(64)
    qn, kn, sk = layer_weights(rng)
    positions = [int(p) for p in rng.integers(0, 4001, 64)]
    positions[0], positions[1], positions[63] = 4000, 0, 3999
    n_slots = 4032
    kv = fa.KVLayer(is_swa=False, has_rope=False, n_slots=n_slots, kv_dtype=store, q_norm=qn, k_norm=kn, sinks=sk,
                    n_seq=64)
    L = oracle_layer(kv, qn, kn, sk, store)
    qkv = rng.standard_normal((64, QKV_DIM)).astype(np.float32)
    wants = []
    for s, p in enumerate(positions):
        K, V = _history(rng, p + 1, store)
        if p:
            _fill_cache(kv, K[:p], V[:p], np.arange(p), s)
        wants.append(fo.decode_step(L, qkv[s], p, K.copy(), V.copy(), n_threads=8))
    dq = torch.from_numpy(qkv).to(cuda)
    att = torch.zeros((64, Q_DIM), device=cuda)
    kv.decode(dq, att, positions)
    torch.cuda.synchronize()
    got = att.cpu().numpy()
    for s, p in enumerate(positions):
        assert_close(got[s], wants[s], f"seq {s} pos {p}")


@pytest.mark.parametrize("store", ["f16", "bf16"])
@pytest.mark.parametrize("n_seq", [1, 3, 8, 16, 17, 24])
def test_decode_batch_swa_v_slices(cuda, store, n_seq):
    """Batched SWA decode with V slices: every sequence has one split, so each kv head's
    output dims are cut over 8 workgroups (up to 8 sequences), 4 (up to 16: 256 workgroups)
    or 2 (17 and 24 sequences: 4 would exceed 256). The launch ids are packed by XCD, two
    sequences per block of ids, so the odd counts leave half of the last block idle.
    Positions before, at and past the ring wrap, and 0; every sequence equals the oracle; the
    current token's K/V land in its ring slot, and every other slot of the sequence's ring
    keeps what it held."""
    _say(f"decode batch SWA v-slices n_seq={n_seq} store={store}")
    rng = np.random.default_rng(100 + n_seq)
    qn, kn, sk = layer_weights(rng)
    positions = [int(p) for p in rng.integers(1, 2600, n_seq)]
    fixed = [0, 1023, 1024] if n_seq >= 3 else [1501]
    positions[:len(fixed)] = fixed
    kv = fa.KVLayer(is_swa=True, has_rope=True, n_slots=1024, kv_dtype=store, q_norm=qn, k_norm=kn, sinks=sk,
                    n_seq=n_seq)
    L = oracle_layer(kv, qn, kn, sk, store)
    qkv = rng.standard_normal((n_seq, QKV_DIM)).astype(np.float32)
    wants, rings = [], []
    for s, p in enumerate(positions):
        K, V = _history(rng, p + 1, store)
        first = max(0, p - 1023)
        if p:
            _fill_cache(kv, K[first:p], V[first:p], np.arange(first, p) & 1023, s)
        Kc, Vc = K.copy(), V.copy()
        wants.append(fo.decode_step(L, qkv[s], p, Kc, Vc, n_threads=8))
        rings.append((Kc, Vc, first))
    dq = torch.from_numpy(qkv).to(cuda)
    att = torch.zeros((n_seq, Q_DIM), device=cuda)
    kv.decode(dq, att, positions)
    torch.cuda.synchronize()
    got = att.cpu().numpy()
    vcs = kv.v_slots().float().cpu().numpy()  # [n_seq][4][1024][128]
    kcs = kv.k_slots().float().cpu().numpy()
    for s, p in enumerate(positions):
        assert_close(got[s], wants[s], f"seq {s} pos {p}")
        Kc, Vc, first = rings[s]
        ring = np.zeros((1024, KV_DIM), np.float32)
        ring[np.arange(first, p + 1) & 1023] = Vc[first:p + 1]
        assert np.array_equal(vcs[s].transpose(1, 0, 2).reshape(1024, KV_DIM), ring), f"seq {s}: V ring"
        cur = p & 1023
        assert k_close(kcs[s][:, cur, :], Kc[p].reshape(N_HEAD_KV, HEAD_DIM), store), f"seq {s}: K slot {cur}"


def config5_contexts():
    """The 16 contexts of benchmark config 5 (bench.py draws them the same way): U[4096, 65536], seed 4."""
    return [int(c) for c in np.random.default_rng(4).integers(4096, 65537, 16)]


@pytest.mark.parametrize("store", ["f16", "bf16"])
@pytest.mark.parametrize("is_swa", [False, True], ids=["full", "swa"])
def test_decode_batch_config5_workload(cuda, store, is_swa):
    """Config 5 at its own workload: 16 sequences at the contexts the benchmark uses (4k-65k),
    one token each, in one batched launch with the automatic plan. Full layer: each
    sequence's key range is cut into its own number of splits over ~192 workgroups, merged
    by the LSE combine. SWA layer (RoPE, 1024-slot ring, window 513): one split per
    sequence, 4 V slices per kv head (256 workgroups). Every sequence equals the oracle, the
    current token's K/V land in its slot, and on the SWA layer every ring slot keeps what it
    held (/root/reference/src/engine.mm:735-766, batched over sequences)."""
    ctx = config5_contexts()
    _say(f"decode config-5 workload store={store} swa={is_swa} contexts={ctx}")
    rng = np.random.default_rng(5 + is_swa)
    qn, kn, sk = layer_weights(rng)
    n_seq = len(ctx)
    n_slots = 1024 if is_swa else (max(ctx) + 1 + 31) // 32 * 32
    kv = fa.KVLayer(is_swa=is_swa, has_rope=is_swa, n_slots=n_slots, kv_dtype=store, rope_theta=1e6, q_norm=qn,
                    k_norm=kn, sinks=sk, n_seq=n_seq)
    L = oracle_layer(kv, qn, kn, sk, store)
    qkv = rng.standard_normal((n_seq, QKV_DIM)).astype(np.float32)
    wants, keep = [], []
    for s, p in enumerate(ctx):
        # the history the cache holds: every position (full) or the last n_slots (ring)
        first = max(0, p - (n_slots - 1)) if is_swa else 0
        K = np.zeros((p + 1, KV_DIM), np.float32)
        V = np.zeros((p + 1, KV_DIM), np.float32)
        K[first:p], V[first:p] = _history(rng, p - first, store, outlier_frac=0.0 if is_swa else 0.01)
        slots = np.arange(first, p) & (n_slots - 1) if is_swa else np.arange(first, p)
        _fill_cache(kv, K[first:p], V[first:p], slots, s)
        wants.append(fo.decode_step(L, qkv[s], p, K, V, n_threads=16))  # writes row p of K, V
        keep.append((K[p].copy(), V[p].copy(), V[max(0, p - (n_slots - 1)):p + 1].copy() if is_swa else None))
        del K, V
    dq = torch.from_numpy(qkv).to(cuda)
    att = torch.zeros((n_seq, Q_DIM), device=cuda)
    kv.decode(dq, att, ctx)
    torch.cuda.synchronize()
    got = att.cpu().numpy()
    for s, p in enumerate(ctx):
        assert_close(got[s], wants[s], f"seq {s} ctx {p}")
        kcur, vcur, ring_hist = keep[s]
        slot = kv.slot(p)
        vc = kv.v[s].permute(0, 1, 3, 2).reshape(N_HEAD_KV, n_slots, HEAD_DIM)[:, slot, :].float().cpu().numpy()
        assert np.array_equal(vc, vcur.reshape(N_HEAD_KV, HEAD_DIM)), f"seq {s}: V slot {slot}"
        kidx = torch.as_tensor(fa.k_tile_offsets()[slot % 32], device=cuda)
        kc = kv.k[s, :, slot // 32][:, kidx].float().cpu().numpy()
        assert k_close(kc, kcur.reshape(N_HEAD_KV, HEAD_DIM), store), f"seq {s}: K slot {slot}"
        if is_swa:
            first = max(0, p - (n_slots - 1))
            ring = np.zeros((n_slots, KV_DIM), np.float32)
            ring[np.arange(first, p + 1) & (n_slots - 1)] = ring_hist
            got_ring = kv.v_slots()[s].float().cpu().numpy().transpose(1, 0, 2).reshape(n_slots, KV_DIM)
            assert np.array_equal(got_ring, ring), f"seq {s}: V ring"
