"""The attention blocks of a GGUF model on the GPU, through the C ABI (include/flint_model.h),
against the CPU oracle's block forward on the same model.

The model is tests/golden/make_block_vectors.py's two-layer quantised model (layer 0 full
attention without RoPE, q8_0/q6_K weights; layer 1 a 100-token sliding window with RoPE,
q5_K/iq4_xs/q6_K/q8_0 weights), regenerated from its seed and written to a temporary GGUF.
The oracle keeps K/V in f16, as the GPU cache does; the oracle itself is pinned bit for bit
to the reference's RefModel::forward on this model with fp32 K/V (tests/test_model.py).

Bars: each layer is checked on its own input (the GPU's hidden state entering it, run
through the oracle's block for that layer): its attention output at every position within
max-abs 2e-3 and mean-abs 2e-4 of the oracle's, and its output hidden state (x + Wo att,
whose rows have std 1/64, so an attention error passes through at about its own size) within
the same 2e-3 / 2e-4. End to end (the oracle run from the embeddings through both layers)
the hidden state stays within 2e-3 / 2e-4 too. Layer 1's attention is compared end to end
only on the decode path: on the prefill path, whose q enters the MFMAs in f16 as the
reference's does (prefill.metal:158-161), layer 0's output error moves layer 1's inputs and
its end-to-end attention measured 2.3e-3 max-abs (mean 6.7e-5), while the same layer on its
own input stays at 1.2e-3. The embedding rows are exact (f16 -> f32)."""
import numpy as np
import pytest

import flint_attn as fa
import oracle as fo
from golden import make_block_vectors as mb

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-3, 2e-4


@pytest.fixture(scope="module")
def setup(cuda, tmp_path_factory):
    m = mb.make_model()
    path = str(tmp_path_factory.mktemp("gguf") / "blocks.gguf")
    mb.write_model(path, m)
    embd = m["embd"].astype(np.float32)
    blocks = mb.oracle_blocks(m, "f16")
    hidden, att = fo.block_forward(blocks, embd, "f16")
    return path, embd, hidden, att, blocks


def _close(got, want, what, max_abs=MAX_ABS):
    got = np.asarray(got, np.float64)
    err = np.abs(got - want)
    assert np.all(np.isfinite(got)), f"{what}: non-finite"
    assert err.max() <= max_abs and err.mean() <= MEAN_ABS, f"{what}: max {err.max():.3e} mean {err.mean():.3e}"
    print(f"{what}: max-abs {err.max():.2e} mean-abs {err.mean():.2e}")
    return err.max()


def _check_layer(blk, x_in, x_out, att, what):
    """Layer output and attention against the oracle's block run on the GPU's own input."""
    want_x, want_att = fo.block_forward([blk], x_in, "f16")
    _close(att, want_att[0], what + " att")
    _close(x_out, want_x, what + " hidden")


def test_model_hparams_and_layers(setup, cuda):
    path = setup[0]
    model = fa.Model(path, n_ctx=256)
    hp, is_swa, has_rope = model.hparams()
    assert (hp.n_layer, hp.n_embd, hp.n_head, hp.n_head_kv, hp.head_dim) == (2, 2048, 32, 4, 128)
    assert hp.n_swa == mb.N_SWA and hp.n_dense_lead == 1 and hp.n_vocab == 1
    assert abs(hp.rope_theta - mb.THETA) < 1e-3 and abs(hp.rms_eps - mb.RMS_EPS) < 1e-12
    assert is_swa == [0, 1] and has_rope == [0, 1]
    L0, L1 = model.layer(0), model.layer(1)
    assert (L0.is_swa, L0.has_rope, L0.n_slots) == (0, 0, 256)
    assert (L1.is_swa, L1.has_rope, L1.n_slots, L1.window) == (1, 1, fa.SWA_RING, mb.N_SWA)
    model.close()


def test_embed_rows_exact(setup, cuda):
    import torch
    path, embd = setup[0], setup[1]
    model = fa.Model(path, n_ctx=256)
    toks = [0, 5, 159, 77, 5]
    x = torch.zeros((len(toks), 2048), device=cuda)
    model.embed(toks, x)
    torch.cuda.synchronize()
    assert np.array_equal(x.cpu().numpy(), embd[toks])
    with pytest.raises(fa.FlintAttnError, match="out of range"):
        model.embed([160], x)
    model.close()


def test_block_decode_matches_oracle(setup, cuda):
    """Token by token: embedding, then layer 0's and layer 1's block at each position."""
    import torch
    path, embd, hidden, att, blocks = setup
    n = embd.shape[0]
    model = fa.Model(path, n_ctx=256)
    xs = torch.zeros((3, n, 2048), device=cuda)  # hidden state entering layer 0, layer 1, and after
    a = torch.zeros((2, n, 4096), device=cuda)
    for p in range(n):
        model.embed([p], xs[0, p])
        for il in range(2):
            xs[il + 1, p].copy_(xs[il, p])
            model.block_decode(il, xs[il + 1, p], p, a[il, p])
    torch.cuda.synchronize()
    xh = xs.cpu().numpy()
    for il in range(2):
        _check_layer(blocks[il], xh[il], xh[il + 1], a[il].cpu().numpy(), f"decode layer {il}")
        _close(a[il].cpu().numpy(), att[il], f"decode att layer {il}, end to end")
    _close(xh[2], hidden, "decode hidden, end to end")
    model.close()


def test_block_prefill_matches_oracle_and_decode(setup, cuda):
    """Layer-major: every position through layer 0, then through layer 1 (one call each),
    then the same split into a prefill of 70 tokens, 10 decode steps and a prefill of the
    rest (the reference's prefill followed by decode, and prefill after decode)."""
    import torch
    path, embd, hidden, att, blocks = setup
    n = embd.shape[0]
    toks = list(range(n))
    model = fa.Model(path, n_ctx=256)
    X = torch.zeros((n, 2048), device=cuda)
    A = torch.zeros((2, n, 4096), device=cuda)
    model.embed(toks, X)
    for il in range(2):
        x_in = X.cpu().numpy()
        model.block_prefill(il, X, 0, A[il])
        torch.cuda.synchronize()
        _check_layer(blocks[il], x_in, X.cpu().numpy(), A[il].cpu().numpy(), f"prefill layer {il}")
    _close(X.cpu().numpy(), hidden, "prefill hidden, end to end")

    model2 = fa.Model(path, n_ctx=256)
    X2 = torch.zeros((n, 2048), device=cuda)
    model2.embed(toks, X2)
    for il in range(2):
        model2.block_prefill(il, X2[:70], 0)
    for p in range(70, 80):
        for il in range(2):
            model2.block_decode(il, X2[p], p)
    for il in range(2):
        model2.block_prefill(il, X2[80:], 80)
    torch.cuda.synchronize()
    _close(X2.cpu().numpy(), hidden, "prefill/decode/prefill hidden, end to end")
    model.close()
    model2.close()


def test_block_prefill_600_tokens(cuda, tmp_path):
    """A longer layer-major prefill (a model of the same layers with 600 positions): 600 tokens
    through layer 0 and then layer 1 in one call each, so the projections run over five
    128-token tiles and the flash kernel over 19 query blocks (and the 100-token window slides
    over many). Each layer within the bars on its own input, and the hidden state end to end."""
    import torch
    m = mb.make_model(n_pos=600)
    path = str(tmp_path / "blocks600.gguf")
    mb.write_model(path, m)
    embd = m["embd"].astype(np.float32)
    blocks = mb.oracle_blocks(m, "f16")
    n = embd.shape[0]
    model = fa.Model(path, n_ctx=1024)
    X = torch.zeros((n, 2048), device=cuda)
    A = torch.zeros((2, n, 4096), device=cuda)
    model.embed(list(range(n)), X)
    for il in range(2):
        x_in = X.cpu().numpy()
        model.block_prefill(il, X, 0, A[il])
        torch.cuda.synchronize()
        _check_layer(blocks[il], x_in, X.cpu().numpy(), A[il].cpu().numpy(), f"600-token prefill layer {il}")
    hidden, _ = fo.block_forward(blocks, embd, "f16")
    _close(X.cpu().numpy(), hidden, "600-token prefill hidden, end to end")
    model.close()


def test_weight_planes_switch(setup, cuda):
    """The prefill projections' kept weight planes hold the bits the per-call weight prep writes:
    prefill blocks with the planes kept, switched off (freed) and on again give bit-identical
    hidden states, and the accessor reports each state."""
    import torch
    path, embd, hidden, att, blocks = setup
    n = embd.shape[0]
    toks = list(range(n))
    model = fa.Model(path, n_ctx=256)
    assert model.weight_planes() == 2  # allowed, not allocated before the first prefill block
    outs = []
    for state in (1, 0, 1):
        model.set_weight_planes(state == 1)
        X = torch.zeros((n, 2048), device=cuda)
        model.embed(toks, X)
        for il in range(2):
            model.block_prefill(il, X, 0)
        torch.cuda.synchronize()
        assert model.weight_planes() == state
        outs.append(X.cpu().numpy())
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])
    _close(outs[0], hidden, "prefill hidden with kept planes, end to end")
    model.close()


def test_block_errors(setup, cuda):
    import torch
    model = fa.Model(setup[0], n_ctx=64)
    x = torch.zeros((2048,), device=cuda)
    with pytest.raises(fa.FlintAttnError, match="bad layer index"):
        model.block_decode(2, x, 0)
    with pytest.raises(fa.FlintAttnError, match="context full"):
        model.block_decode(0, x, 64)
    X = torch.zeros((65, 2048), device=cuda)
    with pytest.raises(fa.FlintAttnError, match="context full"):
        model.block_prefill(0, X, 0)
    model.block_decode(1, x, 500)  # SWA layer: the ring has no n_ctx limit
    torch.cuda.synchronize()
    model.close()


def test_session_step_prefill_truncate(setup, cuda):
    """The model as one session (flint_attn_model_step / _prefill / _truncate, the reference's
    Engine::step / prefill / truncate): token by token, prefill + steps + prefill, and after a
    rollback the same tokens again give the same hidden states bit for bit (full layer: the
    slots are rewritten with the same values; SWA ring: a 60-token rollback keeps its window)."""
    import torch
    path, embd, hidden, att, blocks = setup
    n = embd.shape[0]
    m = fa.Model(path, n_ctx=256)
    assert (m.pos, m.n_ctx) == (0, 256)
    xs = torch.zeros((n, 2048), device=cuda)
    for p in range(n):
        m.step(p, xs[p])
    torch.cuda.synchronize()
    assert m.pos == n
    first = xs.cpu().numpy()
    _close(first, hidden, "session steps, end to end")
    assert m.truncate(n + 1) == -1 and m.truncate(-1) == -1 and m.pos == n
    assert m.truncate(100) == 0 and m.pos == 100
    again = torch.zeros((n - 100, 2048), device=cuda)
    for i, p in enumerate(range(100, n)):
        m.step(p, again[i])
    torch.cuda.synchronize()
    assert np.array_equal(again.cpu().numpy(), first[100:]), "replay after truncate differs"
    m.close()

    m2 = fa.Model(path, n_ctx=256)
    X = torch.zeros((n, 2048), device=cuda)
    m2.prefill(list(range(70)), X[:70])
    for p in range(70, 80):
        m2.step(p, X[p])
    m2.prefill(list(range(80, n)), X[80:])
    torch.cuda.synchronize()
    assert m2.pos == n
    _close(X.cpu().numpy(), hidden, "session prefill/step/prefill, end to end")
    m2.close()


def test_session_gpu_time_and_profile(setup, cuda):
    """Engine::last_gpu_ms / enable_profiling / last_profile (/root/reference/src/engine.h:54-56,
    63) over the session: the GPU time of the last step or prefill, and with profiling on its
    stages in order (the embedding, then per layer the q/k/v projection, attention and o
    projection), whose times sum to it. Profiling changes no result: the same calls after a
    rollback give the same hidden states bit for bit."""
    import torch
    m = fa.Model(setup[0], n_ctx=256)
    assert m.last_gpu_ms() is None and m.last_profile() == [] and m.last_encode_ms() is None
    n_layer = m.hparams()[0].n_layer
    stages = ["embed"] + [f"blk.{il}.{s}" for il in range(n_layer) for s in ("qkv", "attn", "o")]
    X = torch.zeros((33, 2048), device=cuda)
    m.prefill(list(range(32)), X[:32])
    t = m.last_gpu_ms()
    prof = m.last_profile()
    assert t is not None and t > 0 and m.last_encode_ms() > 0
    assert [s for s, _ in prof] == ["prefill"] and abs(prof[0][1] - t) <= 1e-6 + 1e-6 * t
    m.step(32, X[32])
    assert [s for s, _ in m.last_profile()] == ["step"] and m.last_gpu_ms() > 0
    torch.cuda.synchronize()
    want = X.cpu().numpy()

    m.enable_profiling(True)
    assert m.truncate(0) == 0
    Y = torch.zeros((33, 2048), device=cuda)
    m.prefill(list(range(32)), Y[:32])
    prof = m.last_profile()
    t = m.last_gpu_ms()
    assert [s for s, _ in prof] == stages
    assert all(ms >= 0 for _, ms in prof)
    assert abs(sum(ms for _, ms in prof) - t) <= 1e-3 + 1e-4 * t
    m.step(32, Y[32])
    prof = m.last_profile()
    t = m.last_gpu_ms()
    assert [s for s, _ in prof] == stages
    assert abs(sum(ms for _, ms in prof) - t) <= 1e-3 + 1e-4 * t
    torch.cuda.synchronize()
    assert np.array_equal(Y.cpu().numpy(), want), "profiling changed the hidden states"

    m.enable_profiling(False)
    assert m.truncate(32) == 0
    m.step(32, Y[32])
    assert [s for s, _ in m.last_profile()] == ["step"]
    # a failed call leaves no timing behind
    with pytest.raises(fa.FlintAttnError, match="prefill: empty"):
        m.prefill([], Y)
    assert m.last_gpu_ms() is not None  # the check fails before the call starts its marks
    with pytest.raises(fa.FlintAttnError, match="out of range"):
        m.step(1 << 20, Y[32])
    assert m.last_gpu_ms() is None and m.last_profile() == [] and m.last_encode_ms() is None
    m.close()


def test_session_errors(setup, cuda):
    import torch
    m = fa.Model(setup[0], n_ctx=64)
    X = torch.zeros((65, 2048), device=cuda)
    with pytest.raises(fa.FlintAttnError, match="prefill: empty"):
        m.prefill([], X)
    with pytest.raises(fa.FlintAttnError, match="prefill: context full"):
        m.prefill(list(range(65)), X)
    assert m.pos == 0
    m.prefill(list(range(64)), X[:64])
    with pytest.raises(fa.FlintAttnError, match="context full"):
        m.step(0, X[64])
    assert m.pos == 64
    assert m.truncate(10) == 0
    m.step(10, X[10])
    torch.cuda.synchronize()
    assert m.pos == 11
    m.close()
