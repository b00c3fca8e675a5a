"""Batched prefill attention on the GPU against the CPU oracle (benchmark config 4,
the reference's own `flint test-attn` probes, chunk invariance, prefill ==
decode), through the C ABI (flint_attn_prefill, flint_attn_engine_debug_attn).
Tolerance: max-abs 2e-3, mean-abs 2e-4; KV cache / ring slot contents
bit-exact for V and within 1 ulp for K."""
import numpy as np
import pytest
import torch

import flint_attn as fa
import oracle as fo
from helpers import HEAD_DIM, KV_DIM, N_HEAD_KV, QKV_DIM, Q_DIM, assert_close, k_close, layer_weights, oracle_layer

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"\n[gpu-test] {msg}", flush=True)


def _oracle_history(L, qkv, p0=0, K=None, V=None):
    """K,V history rows (normed/roped/rounded) for positions p0..p0+T-1 appended to K,V."""
    T = qkv.shape[0]
    if K is None:
        K = np.zeros((p0 + T, KV_DIM), np.float32)
        V = np.zeros((p0 + T, KV_DIM), np.float32)
    for t in range(T):
        _, K[p0 + t], V[p0 + t] = fo.qkv_prep(L, qkv[t], p0 + t)
    return K, V


def _oracle_at(L, qkv, K, V, positions, p0=0):
    out = {}
    for p in positions:
        q, _, _ = fo.qkv_prep(L, qkv[p - p0], p)
        out[p] = fo.attend(L, q, K, V, p, n_threads=8)
    return out



def _probes(T, extra=()):
    base = [0, 1, 2, 31, 32, 33, 100, 511, 512, 513, 514, 1000, 1023, 1024, 1025, 2047, 2048, 3000, T - 2, T - 1]
    rng = np.random.default_rng(99)
    pts = set(p for p in base if 0 <= p < T) | set(int(x) for x in rng.integers(0, T, 24)) | set(extra)
    return sorted(p for p in pts if 0 <= p < T)


@pytest.mark.parametrize("store", ["bf16", "f16"])
@pytest.mark.parametrize("is_swa", [False, True], ids=["full", "swa"])
def test_prefill_4000_config4(cuda, store, is_swa):
    """Config 4: 4000-token prompt, causal; full layer and SWA-513 layer with ring write of the last 1024.
    Every output row is compared with the oracle."""
    T = 4000
    _say(f"prefill T={T} store={store} swa={is_swa} seed=3")
    rng = np.random.default_rng(3)
    qn, kn, sk = layer_weights(rng)
    kv = fa.KVLayer(is_swa=is_swa, has_rope=is_swa, n_slots=1024 if is_swa else 4096, kv_dtype=store,
                    rope_theta=1e4, q_norm=qn, k_norm=kn, sinks=sk)
    L = oracle_layer(kv, qn, kn, sk, store)
    qkv = rng.standard_normal((T, QKV_DIM)).astype(np.float32)
    att = torch.zeros((T, Q_DIM), device=cuda)
    kv.prefill(torch.from_numpy(qkv).to(cuda), att, 0)
    torch.cuda.synchronize()
    got = att.cpu().numpy()
    assert np.all(np.isfinite(got))
    # every row against the oracle's own prefill (token by token over the linear history)
    K = np.zeros((T, KV_DIM), np.float32)
    V = np.zeros((T, KV_DIM), np.float32)
    want = fo.prefill(L, qkv, 0, K, V, n_threads=16)
    for p in _probes(T):
        assert_close(got[p], want[p], f"pos {p}")
    for r0 in range(0, T, 500):
        assert_close(got[r0:r0 + 500], want[r0:r0 + 500], f"rows {r0}..{r0 + 499}")
    assert_close(got, want, "all rows")
    vc = kv.v_slots()[0].float().cpu().numpy()
    kc = kv.k_slots()[0].float().cpu().numpy()
    lo = T - 1024 if is_swa else 0
    for p in range(lo, T):
        s = kv.slot(p)
        assert np.array_equal(vc[:, s, :], V[p].reshape(N_HEAD_KV, HEAD_DIM)), f"V slot {s} pos {p}"
        assert k_close(kc[:, s, :], K[p].reshape(N_HEAD_KV, HEAD_DIM), store), f"K slot {s} pos {p}"


@pytest.mark.parametrize("n,p0,store,big_v", [(2701, 0, "f16", False), (3000, 517, "bf16", False), (2200, 0, "bf16", True)],
                         ids=["T2701_f16", "p0_517_T2483_bf16", "T2200_bf16_scaled"])
def test_prefill_swa_two_rounds(cuda, n, p0, store, big_v):
    """SWA prefills of more than 64 query blocks (two rounds of workgroups, each kv head's blocks
    dealt to two XCDs in halves, half of the first round started late): odd block counts, a
    last block of 13 rows, a call after a cached prefix at an unaligned position, and the
    scaled path (V rows at 1e5, past f16). Every row against the oracle; the ring bit-exact
    for V."""
    _say(f"SWA two rounds: n={n} p0={p0} store={store} big_v={big_v}")
    rng = np.random.default_rng(5)
    qn, kn, sk = layer_weights(rng)
    qkv = rng.standard_normal((n, QKV_DIM)).astype(np.float32)
    if big_v:
        qkv[3::7, 4608:] *= 1e5
    kv = fa.KVLayer(is_swa=True, has_rope=True, n_slots=1024, kv_dtype=store, rope_theta=1e4, q_norm=qn, k_norm=kn,
                    sinks=sk)
    L = oracle_layer(kv, qn, kn, sk, store)
    dq = torch.from_numpy(qkv).to(cuda)
    att = torch.zeros((n, Q_DIM), device=cuda)
    if p0:
        kv.prefill(dq[:p0], att[:p0], 0)
    kv.prefill(dq[p0:], att[p0:], p0)
    torch.cuda.synchronize()
    got = att.cpu().numpy().astype(np.float64)
    assert np.all(np.isfinite(got))
    K = np.zeros((n, KV_DIM), np.float32)
    V = np.zeros((n, KV_DIM), np.float32)
    want = fo.prefill(L, qkv, 0, K, V, n_threads=16).astype(np.float64)
    scale = np.maximum(1.0, np.abs(want).max(axis=1, keepdims=True)) if big_v else 1.0
    for r0 in range(0, n, 500):
        r1 = min(n, r0 + 500)
        sc = scale[r0:r1] if big_v else 1.0
        assert_close(got[r0:r1] / sc, want[r0:r1] / sc, f"rows {r0}..{r1 - 1}")
    vc = kv.v_slots()[0].float().cpu().numpy()
    for p in range(n - 1024, n):
        assert np.array_equal(vc[:, kv.slot(p), :], V[p].reshape(N_HEAD_KV, HEAD_DIM)), f"V slot of pos {p}"


@pytest.mark.parametrize("n,is_swa,store", [(16384, False, "f16"), (12000, True, "bf16")], ids=["full_16384_f16", "swa_12000_bf16"])
def test_prefill_long_prompt_probes(cuda, n, is_swa, store):
    """One call over a long prompt (512 and 375 query blocks: several rounds of workgroups, the
    longest-first deal of a causal layer over 2048 workgroups): probe rows at block edges, round
    boundaries and random positions against the oracle, and the cache's V rows of sampled
    positions bit-exact."""
    _say(f"long prompt probes n={n} swa={is_swa} store={store}")
    rng = np.random.default_rng(17)
    qn, kn, sk = layer_weights(rng)
    qkv = rng.standard_normal((n, QKV_DIM)).astype(np.float32)
    kv = fa.KVLayer(is_swa=is_swa, has_rope=True, n_slots=1024 if is_swa else n, kv_dtype=store, rope_theta=1e6,
                    q_norm=qn, k_norm=kn, sinks=sk)
    L = oracle_layer(kv, qn, kn, sk, store)
    att = torch.zeros((n, Q_DIM), device=cuda)
    kv.prefill(torch.from_numpy(qkv).to(cuda), att, 0)
    torch.cuda.synchronize()
    got = att.cpu().numpy()
    assert np.all(np.isfinite(got))
    K, V = _oracle_history(L, qkv)
    probes = _probes(n, extra=[4095, 4096, 8191, 8192, 8224, 12287, 12288, n // 2, n - 33, n - 32, n - 31])
    want = _oracle_at(L, qkv, K, V, probes)
    for p in probes:
        assert_close(got[p], want[p], f"pos {p}")
    vc = kv.v_slots()[0].float().cpu().numpy()
    for p in (range(n - 1024, n, 7) if is_swa else range(0, n, 97)):
        assert np.array_equal(vc[:, kv.slot(p), :], V[p].reshape(N_HEAD_KV, HEAD_DIM)), f"V slot of pos {p}"


@pytest.mark.parametrize("il,is_swa", [(0, False), (2, True)], ids=["layer0_full_nope", "layer2_swa_rope"])
def test_debug_attn_reference_test_attn_probes(cuda, il, is_swa):
    """The reference's `flint test-attn` (/root/reference/src/main.mm:241-314): 1300 tokens in
    512-token chunks, inputs uniform on [-2, 2] in steps of 0.002, probes at
    {0,1,31,32,200,511,512,513,600,1023,1024,1100,1299} x heads {0,7,8,31}."""
    _say(f"debug_attn test-attn probes layer {il}")
    flags_swa = [False, False, True]
    eng = fa.Engine(flags_swa, flags_swa, n_ctx=4096, kv_dtype="f16", rope_theta=1e4)
    rng = np.random.default_rng(11 + il)
    qn, kn, sk = layer_weights(rng)
    eng.set_weights(il, qn, kn, sk)
    n = 1300
    qkv = (rng.integers(0, 2001, (n, QKV_DIM)) - 1000).astype(np.float32) / 500.0
    got = eng.debug_attn(il, qkv, 512)
    L = fo.Layer(qn, kn, sk, is_swa, is_swa, "f16", 1e4)
    K, V = _oracle_history(L, qkv)
    probes = [0, 1, 31, 32, 200, 511, 512, 513, 600, 1023, 1024, 1100, 1299]
    want = _oracle_at(L, qkv, K, V, probes)
    heads = [0, 7, 8, 31]
    sel = lambda a: np.concatenate([a[h * HEAD_DIM:(h + 1) * HEAD_DIM] for h in heads])
    g = np.stack([sel(got[p]) for p in probes])
    w = np.stack([sel(want[p]) for p in probes])
    assert_close(g, w, "test-attn probes")
    rel = np.abs(g - w).max() / np.sqrt(np.mean(w.astype(np.float64) ** 2))
    assert rel < 2e-2  # the reference's own pass criterion (main.mm:308)
    eng.close()


@pytest.mark.parametrize("is_swa", [False, True], ids=["full", "swa"])
def test_prefill_chunk_invariance_and_continuation(cuda, is_swa):
    """Chunked prefill (p0 > 0 continuations, including chunks larger than the ring
    headroom) equals one-shot prefill and the oracle."""
    n = 1300
    _say(f"prefill chunk invariance swa={is_swa} n={n}")
    rng = np.random.default_rng(31)
    qn, kn, sk = layer_weights(rng)
    qkv = rng.standard_normal((n, QKV_DIM)).astype(np.float32)
    L = fo.Layer(qn, kn, sk, is_swa, True, "f16", 1e4)
    K, V = _oracle_history(L, qkv)
    want = _oracle_at(L, qkv, K, V, _probes(n, extra=range(590, 610)))
    outs = {}
    for chunk in (n, 512, 600, 97, 1):
        eng = fa.Engine([is_swa], [True], n_ctx=2048, kv_dtype="f16", rope_theta=1e4)
        eng.set_weights(0, qn, kn, sk)
        outs[chunk] = eng.debug_attn(0, qkv, chunk)
        eng.close()
        for p, w in want.items():
            assert_close(outs[chunk][p], w, f"chunk {chunk} pos {p}")
    for chunk, o in outs.items():
        assert_close(o, outs[n], f"chunk {chunk} vs one-shot", max_abs=1e-3, mean_abs=5e-5)


@pytest.mark.parametrize("is_swa", [False, True], ids=["full", "swa"])
def test_prefill_equals_decode(cuda, is_swa):
    """Prefill of 700 tokens == 700 decode steps (outputs within tolerance, V caches bit-identical)."""
    n = 700
    _say(f"prefill == decode swa={is_swa} n={n}")
    rng = np.random.default_rng(41)
    qn, kn, sk = layer_weights(rng)
    mk = lambda: fa.KVLayer(is_swa=is_swa, has_rope=True, n_slots=1024, kv_dtype="f16", q_norm=qn, k_norm=kn,
                            sinks=sk)
    a, b = mk(), mk()
    qkv = rng.standard_normal((n, QKV_DIM)).astype(np.float32)
    dq = torch.from_numpy(qkv).to(cuda)
    att_p = torch.zeros((n, Q_DIM), device=cuda)
    att_d = torch.zeros((n, Q_DIM), device=cuda)
    a.prefill(dq, att_p, 0)
    for pos in range(n):
        b.decode(dq[pos], att_d[pos], pos)
    torch.cuda.synchronize()
    assert_close(att_p.cpu().numpy(), att_d.cpu().numpy(), "prefill vs decode")
    assert torch.equal(a.v, b.v)
    kd = (a.k.float() - b.k.float()).abs()
    assert float(kd.max()) <= float(b.k.float().abs().max()) * 2 ** -10


def test_prefill_short_and_odd_shapes(cuda):
    """T = 1, 33, 65 at p0 = 0 and at p0 = 1000 across the ring wrap (SWA), bf16."""
    _say("prefill short/odd shapes")
    rng = np.random.default_rng(51)
    qn, kn, sk = layer_weights(rng)
    L = fo.Layer(qn, kn, sk, True, True, "bf16", 1e4)
    total = 1000 + 65
    qkv = rng.standard_normal((total, QKV_DIM)).astype(np.float32)
    K, V = _oracle_history(L, qkv)
    for T in (1, 33, 65):
        for p0 in (0, 1000):
            kv = fa.KVLayer(is_swa=True, has_rope=True, kv_dtype="bf16", q_norm=qn, k_norm=kn, sinks=sk)
            if p0:
                pre = torch.zeros((p0, Q_DIM), device=cuda)
                kv.prefill(torch.from_numpy(qkv[:p0]).to(cuda), pre, 0)
            att = torch.zeros((T, Q_DIM), device=cuda)
            kv.prefill(torch.from_numpy(qkv[p0:p0 + T]).to(cuda), att, p0)
            torch.cuda.synchronize()
            want = _oracle_at(L, qkv, K, V, range(p0, p0 + T))
            assert_close(att.cpu().numpy(), np.stack([want[p] for p in range(p0, p0 + T)]), f"T={T} p0={p0}")


@pytest.mark.parametrize("rollback", [300, 700])
def test_prefill_after_rollback_swa_ring(cuda, rollback):
    """Prefix reuse after a rollback (the reference's flint_truncate contract, capi.h:27-29,
    and its caller's rule, server/src/main.rs:95-116): after positions 0..N-1, the sequence
    is cut back to p = N - rollback and continues with new tokens. The 1024-slot SWA ring
    still holds the window of p when the rollback is at most 511 tokens, so prefilling the
    new tokens from p is exact; for a deeper rollback the caller re-prefills from
    max(0, p - 512). Either way the outputs at p.. equal a fresh run of the new sequence."""
    n, m = 1600, 1800
    _say(f"prefill after rollback {rollback} (SWA ring)")
    rng = np.random.default_rng(61)
    qn, kn, sk = layer_weights(rng)
    L = fo.Layer(qn, kn, sk, True, True, "f16", 1e4)
    qkv_a = rng.standard_normal((n, QKV_DIM)).astype(np.float32)
    p = n - rollback
    qkv_b = np.concatenate([qkv_a[:p], rng.standard_normal((m - p, QKV_DIM)).astype(np.float32)])
    kv = fa.KVLayer(is_swa=True, has_rope=True, n_slots=1024, kv_dtype="f16", q_norm=qn, k_norm=kn, sinks=sk,
                    rope_theta=1e4)
    att = torch.zeros((m, Q_DIM), device=cuda)
    kv.prefill(torch.from_numpy(qkv_a).to(cuda), att[:n], 0)
    start = p if rollback <= 511 else max(0, p - 512)
    kv.prefill(torch.from_numpy(qkv_b[start:]).to(cuda), att[start:], start)
    torch.cuda.synchronize()
    got = att.cpu().numpy()
    K, V = _oracle_history(L, qkv_b)
    want = _oracle_at(L, qkv_b, K, V, [p, p + 1, p + 31, p + 300, m - 1])
    for q, w in want.items():
        assert_close(got[q], w, f"rollback {rollback} pos {q}")


@pytest.mark.parametrize("case", ["v_rows_1e5_1e-6", "v_all_1e-6", "k_gain_1e4_q_gain_1e-4"])
@pytest.mark.parametrize("is_swa", [False, True], ids=["full", "swa"])
def test_prefill_then_decode_bf16_beyond_f16_range(cuda, case, is_swa):
    """bf16 K/V outside f16's range on one bf16 cache: V rows scaled to 1e5 (past f16's 65504)
    and to 1e-6 (f16 subnormals), all of V at 1e-6, or K gains x1e4 (normalised K past 65504)
    with q gains x1e-4. Prefill of 1300 tokens in two calls (700 + 600: the second copies whole
    cached tiles and the part-cached tile of p0 = 700), then 4 decode steps on the same cache;
    every position against the oracle. The prefill stores such tiles in f16 scaled by a power
    of two and takes its scaled path; on the SWA layer the window masks large rows of earlier
    positions. Errors are measured relative to each output row's largest magnitude (at least
    1), at the usual bars; the ring / cache slots are bit-exact against the oracle's."""
    _say(f"prefill + decode bf16 beyond f16 range: {case} swa={is_swa}")
    rng = np.random.default_rng(71)
    qn, kn, sk = layer_weights(rng)
    n = 1304
    qkv = rng.standard_normal((n, QKV_DIM)).astype(np.float32)
    if case == "v_rows_1e5_1e-6":
        qkv[3::7, 4608:] *= 1e5
        qkv[5::11, 4608:] *= 1e-6
    elif case == "v_all_1e-6":
        qkv[:, 4608:] *= 1e-6
    else:
        kn = (kn * 1e4).astype(np.float32)
        qn = (qn * 1e-4).astype(np.float32)
    kv = fa.KVLayer(is_swa=is_swa, has_rope=True, n_slots=1024 if is_swa else 1312, kv_dtype="bf16",
                    rope_theta=1e4, q_norm=qn, k_norm=kn, sinks=sk)
    L = oracle_layer(kv, qn, kn, sk, "bf16")
    dq = torch.from_numpy(qkv).to(cuda)
    att = torch.zeros((n, Q_DIM), device=cuda)
    kv.prefill(dq[:700], att[:700], 0)
    kv.prefill(dq[700:1300], att[700:1300], 700)
    for pos in range(1300, n):
        kv.decode(dq[pos], att[pos], pos)
    torch.cuda.synchronize()
    got = att.cpu().numpy().astype(np.float64)
    K = np.zeros((n, KV_DIM), np.float32)
    V = np.zeros((n, KV_DIM), np.float32)
    want = fo.prefill(L, qkv, 0, K, V, n_threads=16).astype(np.float64)
    assert np.all(np.isfinite(got)), "non-finite output"
    scale = np.maximum(1.0, np.abs(want).max(axis=1, keepdims=True))
    if case == "v_all_1e-6":
        scale = np.abs(want).max(axis=1, keepdims=True)
    assert_close(got[:1300] / scale[:1300], want[:1300] / scale[:1300], f"{case}: prefill rows")
    assert_close(got[1300:] / scale[1300:], want[1300:] / scale[1300:], f"{case}: decode rows")
    vc = kv.v_slots()[0].float().cpu().numpy()
    for p in range(max(0, n - 1024) if is_swa else 0, n):
        assert np.array_equal(vc[:, kv.slot(p), :], V[p].reshape(N_HEAD_KV, HEAD_DIM)), f"V slot of pos {p}"


@pytest.mark.parametrize("store", ["f16", "bf16"])
@pytest.mark.parametrize("is_swa", [False, True], ids=["full", "swa"])
def test_prefill_short_at_long_context_split_keys(cuda, store, is_swa):
    """Short prefills after a long one, where the prefill cuts every query block's key range
    into splits merged with the sink by a second kernel: continuations of T = 1, 7, 40, 100
    tokens from p0 = 20005 (full layer: 626-630 key tiles, 63 splits of 10 tiles for the
    first three, 32 of 20 for T = 100) and from p0 = 5003 (SWA ring: at most 18 tiles, 3
    splits of 6). Every new position against the oracle, at the usual bars."""
    p0 = 5003 if is_swa else 20005
    Ts = (1, 7, 40, 100)
    n = p0 + sum(Ts)
    _say(f"short prefills at long context (split keys) swa={is_swa} store={store} p0={p0}")
    rng = np.random.default_rng(81)
    qn, kn, sk = layer_weights(rng)
    qkv = rng.standard_normal((n, QKV_DIM)).astype(np.float32)
    kv = fa.KVLayer(is_swa=is_swa, has_rope=True, n_slots=1024 if is_swa else (n + 31) // 32 * 32,
                    kv_dtype=store, rope_theta=1e4, q_norm=qn, k_norm=kn, sinks=sk)
    L = oracle_layer(kv, qn, kn, sk, store)
    dq = torch.from_numpy(qkv).to(cuda)
    att = torch.zeros((n, Q_DIM), device=cuda)
    kv.prefill(dq[:p0], att[:p0], 0)
    p = p0
    for T in Ts:
        kv.prefill(dq[p:p + T], att[p:p + T], p)
        p += T
    torch.cuda.synchronize()
    got = att.cpu().numpy()
    K, V = _oracle_history(L, qkv)
    want = _oracle_at(L, qkv, K, V, range(p0, n))
    p = p0
    for T in Ts:
        assert_close(got[p:p + T], np.stack([want[q] for q in range(p, p + T)]), f"T={T} at p0={p}")
        p += T


@pytest.mark.parametrize("is_swa", [False, True], ids=["full", "swa"])
def test_prefill_f16_cached_tiles_on_scaled_path(cuda, is_swa):
    """An f16 continuation reads its whole cached tiles from the cache itself; with q gains
    x1e-3 (q below f16's normal range, so q is stored scaled and the tile-by-tile path runs)
    those tiles must count as unscaled. 700 tokens, then 250 from p0 = 700 (21 cached tiles
    read in place, the p0 tile through the copy), against the oracle."""
    _say(f"f16 cached tiles on the scaled path swa={is_swa}")
    rng = np.random.default_rng(91)
    qn, kn, sk = layer_weights(rng)
    qn = (qn * 1e-3).astype(np.float32)
    n = 950
    qkv = rng.standard_normal((n, QKV_DIM)).astype(np.float32)
    kv = fa.KVLayer(is_swa=is_swa, has_rope=True, n_slots=1024, kv_dtype="f16", rope_theta=1e4,
                    q_norm=qn, k_norm=kn, sinks=sk)
    L = oracle_layer(kv, qn, kn, sk, "f16")
    dq = torch.from_numpy(qkv).to(cuda)
    att = torch.zeros((n, Q_DIM), device=cuda)
    kv.prefill(dq[:700], att[:700], 0)
    kv.prefill(dq[700:], att[700:], 700)
    torch.cuda.synchronize()
    K, V = _oracle_history(L, qkv)
    probes = [700, 701, 731, 732, 850, 949]
    want = _oracle_at(L, qkv, K, V, probes)
    got = att.cpu().numpy()
    for p in probes:
        assert_close(got[p], want[p], f"pos {p}")
