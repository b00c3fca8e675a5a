"""GPU parity of the attention projections in the engine's weight formats
(include/flint_proj.h, flint-mac_amd/csrc/proj.hip) against the CPU oracle:
  * get_row bit-identical to fo_dequant_row (itself bit-identical to the reference's ggml
    dequantize_row_*), the reference's check-deq contract (/root/reference/src/main.mm:27-48,
    which allows 1e-5);
  * the q/k/v projection with the attention RMSNorm, and o_proj with the residual add, within
    fp32 reassociation of the oracle's double-accumulated matvec (ref_model.cpp:74-93, 107-110,
    150-151): one token, small batches (bit-identical to one token), and batches on the GEMM
    (proj_gemm.hip, f16 hi/lo planes) in every format and over rows of any range.
"""
import numpy as np
import pytest

import flint_attn as fa
import oracle

pytestmark = pytest.mark.gpu
QUANT = ("q8_0", "q5_K", "q6_K", "iq4_xs")
ALL = QUANT + ("f32", "f16", "bf16")


def _dev(a, cuda):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


@pytest.mark.parametrize("wtype", ALL)
@pytest.mark.parametrize("k", [2048, 4096, 768])
def test_get_row_bit_exact(cuda, wtype, k):
    import torch
    if oracle.row_bytes(wtype, k) < 0:
        pytest.skip("k is not a whole number of blocks")
    rng = np.random.default_rng(k * 7 + len(wtype))
    rows = oracle.random_blocks(wtype, 5, k, rng)
    want = oracle.dequant_rows(wtype, rows, k)
    w = _dev(rows, cuda)
    out = torch.empty(k, dtype=torch.float32, device=cuda)
    for r in range(5):
        out.fill_(float("nan"))
        fa.get_row(wtype, w, k, r, out)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want[r].view(np.uint32)), (wtype, k, r)


@pytest.mark.parametrize("wtype", ["q8_0", "q6_K", "iq4_xs", "f16", "bf16"])
def test_get_rows_matches_get_row(cuda, wtype):
    """The batched row dequantisation (the prefill's token embedding, one dispatch per 448 rows)
    against the oracle row by row: 1000 rows drawn with repeats from a 300-row table, so the
    table crosses two launch boundaries; every row bit-identical."""
    import torch
    k = 2048
    rng = np.random.default_rng(11 + len(wtype))
    table = oracle.random_blocks(wtype, 300, k, rng)
    want = oracle.dequant_rows(wtype, table, k)
    w = _dev(table, cuda)
    rows = rng.integers(0, 300, 1000)
    rows[:3] = [0, 299, 0]
    out = torch.full((1000, k), float("nan"), dtype=torch.float32, device=cuda)
    fa.get_rows(wtype, w, k, 300, rows, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want[rows].view(np.uint32)), wtype
    with pytest.raises(fa.FlintAttnError, match="out of range"):
        fa.get_rows(wtype, w, k, 300, [5, 300], out)


def test_get_row_golden_rows(cuda):
    """The committed reference rows (tests/golden/weight_rows.npz, 512 elements: one wave with
    16 sub-blocks), straight against the reference's float bits."""
    import os
    import torch
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "weight_rows.npz"))
    out = torch.empty(512, dtype=torch.float32, device=cuda)
    for t in QUANT:
        w = _dev(z[t + "_rows"], cuda)
        for r in range(z[t + "_rows"].shape[0]):
            fa.get_row(t, w, 512, r, out)
            torch.cuda.synchronize()
            assert np.array_equal(out.cpu().numpy().view(np.uint32), z[t + "_bits"][r]), (t, r)


def _rows_bound(dense, x):
    """Per-row bound on fp32 reassociation: 2e-6 of the sum of |w x| (a single wrong weight
    moves a 2048-term row by about 5e-4 of it)."""
    return 2e-6 * np.abs(dense.astype(np.float64)) @ np.abs(x.astype(np.float64)) + 1e-7


@pytest.mark.parametrize("types", [("q8_0",) * 3, ("q5_K",) * 3, ("q6_K",) * 3, ("iq4_xs",) * 3,
                                   ("q5_K", "q6_K", "iq4_xs"), ("bf16", "f16", "f32")])
def test_qkv_proj_matches_oracle(cuda, types):
    import torch
    rng = np.random.default_rng(11)
    E = fa.N_EMBD
    x = (rng.standard_normal(E) * 2).astype(np.float32)
    g = rng.uniform(0.5, 1.5, E).astype(np.float32)
    xn = np.empty(E, np.float32)
    oracle.lib().fo_rmsnorm(oracle._p(x), oracle._p(g), oracle._p(xn), E, 1e-6)
    ws, want, bound = [], [], []
    for t, n in zip(types, (4096, 512, 512)):
        rows = oracle.random_blocks(t, n, E, rng)
        ws.append((_dev(rows, cuda), t))
        want.append(oracle.matvec(t, rows, E, xn))
        bound.append(_rows_bound(oracle.dequant_rows(t, rows, E), xn))
    want, bound = np.concatenate(want), np.concatenate(bound)
    qkv = torch.full((5120,), float("nan"), dtype=torch.float32, device=cuda)
    fa.qkv_proj(ws[0], ws[1], ws[2], _dev(x, cuda), _dev(g, cuda), qkv, rms_eps=1e-6)
    torch.cuda.synchronize()
    got = qkv.cpu().numpy()
    err = np.abs(got.astype(np.float64) - want)
    assert np.all(err <= bound), (types, float((err / bound).max()), int(np.argmax(err / bound)))


@pytest.mark.parametrize("wtype", ALL)
def test_o_proj_residual_matches_oracle(cuda, wtype):
    import torch
    rng = np.random.default_rng(12)
    att = rng.standard_normal(4096).astype(np.float32)
    x0 = rng.standard_normal(fa.N_EMBD).astype(np.float32)
    rows = oracle.random_blocks(wtype, fa.N_EMBD, 4096, rng)
    o = oracle.matvec(wtype, rows, 4096, att)
    want = x0 + o  # ref_model.cpp:150-151: x[i] += o[i] in float
    bound = _rows_bound(oracle.dequant_rows(wtype, rows, 4096), att) + 1e-7 * np.abs(x0)
    x = _dev(x0, cuda)
    fa.o_proj((_dev(rows, cuda), wtype), _dev(att, cuda), x)
    torch.cuda.synchronize()
    err = np.abs(x.cpu().numpy().astype(np.float64) - want)
    assert np.all(err <= bound), (wtype, float((err / bound).max()))


def test_projection_block_round_trip(cuda):
    """qkv_proj -> decode attention -> o_proj on one layer, against the oracle's attention
    block (ref_model.cpp:107-151 with the cache in f16): the three stages compose."""
    import torch
    rng = np.random.default_rng(13)
    E, pos = fa.N_EMBD, 40
    g = rng.uniform(0.5, 1.5, E).astype(np.float32)
    qn, kn = rng.uniform(0.5, 1.5, 128).astype(np.float32), rng.uniform(0.5, 1.5, 128).astype(np.float32)
    sinks = rng.standard_normal(32).astype(np.float32)
    wq, wk, wv = (oracle.random_blocks("q8_0", n, E, rng) for n in (4096, 512, 512))
    wo = oracle.random_blocks("q6_K", E, 4096, rng)
    layer = oracle.Layer(qn, kn, sinks, is_swa=False, has_rope=True, store="f16", rope_theta=1e6)
    kv = fa.KVLayer(is_swa=False, has_rope=True, n_slots=64, kv_dtype="f16", q_norm=qn, k_norm=kn, sinks=sinks,
                    rope_theta=1e6, device=cuda)
    K = np.zeros((pos + 1, 512), np.float32)
    V = np.zeros((pos + 1, 512), np.float32)
    dq = (_dev(wq, cuda), "q8_0"), (_dev(wk, cuda), "q8_0"), (_dev(wv, cuda), "q8_0")
    do = (_dev(wo, cuda), "q6_K")
    qkv = torch.empty(5120, dtype=torch.float32, device=cuda)
    att = torch.empty(4096, dtype=torch.float32, device=cuda)
    for p in range(pos + 1):
        x0 = rng.standard_normal(E).astype(np.float32)
        xn = np.empty(E, np.float32)
        oracle.lib().fo_rmsnorm(oracle._p(x0), oracle._p(g), oracle._p(xn), E, 1e-6)
        qkv_ref = np.concatenate([oracle.matvec("q8_0", w, E, xn) for w in (wq, wk, wv)])
        att_ref = oracle.decode_step(layer, qkv_ref, p, K, V)
        x_ref = x0 + oracle.matvec("q6_K", wo, 4096, att_ref)
        x = _dev(x0, cuda)
        fa.qkv_proj(*dq, x, _dev(g, cuda), qkv)
        kv.decode(qkv, att, pos=p)
        fa.o_proj(do, att, x)
        torch.cuda.synchronize()
        got = x.cpu().numpy()
        scale = np.abs(oracle.dequant_rows("q6_K", wo, 4096)).sum(1) * 2e-3 + 1e-5
        assert np.all(np.abs(got - x_ref) <= scale), (p, float(np.abs(got - x_ref).max()))


def test_projection_rows_small_batch_equal_single_token_calls(cuda):
    """Batches below the GEMM's size (flint_attn_qkv_proj_rows / flint_attn_o_proj_rows with
    n_tok < 16) run the one-token kernel per token: each token gets exactly the single-token
    call's bits, also into a strided qkv row (q_stride 5248)."""
    import torch
    rng = np.random.default_rng(41)
    T = 9
    wq = (_dev(oracle.random_blocks("q5_K", 4096, 2048, rng), cuda), "q5_K")
    wk = (_dev(oracle.random_blocks("iq4_xs", 512, 2048, rng), cuda), "iq4_xs")
    wv = (_dev(oracle.random_blocks("q8_0", 512, 2048, rng), cuda), "q8_0")
    wo = (_dev(oracle.random_blocks("q6_K", 2048, 4096, rng), cuda), "q6_K")
    g = _dev(rng.uniform(0.5, 1.5, 2048).astype(np.float32), cuda)
    x = _dev(rng.standard_normal((T, 2048)).astype(np.float32), cuda)
    att = _dev(rng.standard_normal((T, 4096)).astype(np.float32), cuda)
    qkv_rows = torch.full((T, 5248), float("nan"), device=cuda)
    fa.qkv_proj_rows(wq, wk, wv, x, g, qkv_rows)
    y_rows = x.clone()
    fa.o_proj_rows(wo, att, y_rows)
    qkv_one = torch.empty((T, 5120), device=cuda)
    y_one = x.clone()
    for t in range(T):
        fa.qkv_proj(wq, wk, wv, x[t], g, qkv_one[t])
        fa.o_proj(wo, att[t], y_one[t])
    torch.cuda.synchronize()
    assert torch.equal(qkv_rows[:, :5120], qkv_one)
    assert torch.isnan(qkv_rows[:, 5120:]).all()  # the row padding is left alone
    assert torch.equal(y_rows, y_one)


def _gemm_case(cuda, rng, types, wo_type, T, x_scale=None, att_scale=None):
    """qkv_proj_rows and o_proj_rows on T tokens (the GEMM path) against the oracle's matvec of
    every token, within _rows_bound. x_scale / att_scale: per-row factors for the inputs."""
    import torch
    E = fa.N_EMBD
    x = (rng.standard_normal((T, E)) * 2).astype(np.float32)
    if x_scale is not None:
        x *= x_scale[:, None].astype(np.float32)
    g = rng.uniform(0.5, 1.5, E).astype(np.float32)
    ws, dense = [], []
    for t, n in zip(types, (4096, 512, 512)):
        rows = oracle.random_blocks(t, n, E, rng)
        ws.append((_dev(rows, cuda), t))
        dense.append(oracle.dequant_rows(t, rows, E))
    dense = np.concatenate(dense)
    wo_rows = oracle.random_blocks(wo_type, E, 4096, rng)
    wo_dense = oracle.dequant_rows(wo_type, wo_rows, 4096)
    att = rng.standard_normal((T, 4096)).astype(np.float32)
    if att_scale is not None:
        att *= att_scale[:, None].astype(np.float32)
    x0 = rng.standard_normal((T, E)).astype(np.float32)
    qkv = torch.full((T, 5248), float("nan"), device=cuda)
    fa.qkv_proj_rows(ws[0], ws[1], ws[2], _dev(x, cuda), _dev(g, cuda), qkv)
    y = _dev(x0, cuda)
    fa.o_proj_rows((_dev(wo_rows, cuda), wo_type), _dev(att, cuda), y)
    torch.cuda.synchronize()
    got_qkv = qkv.cpu().numpy()[:, :5120].astype(np.float64)
    got_y = y.cpu().numpy().astype(np.float64)
    assert torch.isnan(qkv[:, 5120:]).all()
    for t in range(T):
        xn = np.empty(E, np.float32)
        oracle.lib().fo_rmsnorm(oracle._p(np.ascontiguousarray(x[t])), oracle._p(g), oracle._p(xn), E, 1e-6)
        want = oracle.matvec_f32(dense, xn)
        bound = _rows_bound(dense, xn)
        err = np.abs(got_qkv[t] - want)
        assert np.all(err <= bound), ("qkv", types, t, float((err / bound).max()))
        want_y = x0[t] + oracle.matvec_f32(wo_dense, att[t])
        bound_y = _rows_bound(wo_dense, att[t]) + 1e-7 * np.abs(x0[t])
        err = np.abs(got_y[t] - want_y)
        assert np.all(err <= bound_y), ("o", wo_type, t, float((err / bound_y).max()))


@pytest.mark.parametrize("types,wo_type", [(("q8_0",) * 3, "q8_0"), (("q5_K", "q6_K", "iq4_xs"), "q6_K"),
                                           (("bf16", "f16", "f32"), "iq4_xs"), (("q6_K",) * 3, "q5_K"),
                                           (("iq4_xs",) * 3, "bf16"), (("f16",) * 3, "f16"), (("bf16",) * 3, "q5_K")])
def test_projection_rows_gemm_matches_oracle(cuda, types, wo_type):
    """Batches from 16 tokens (the GEMM on f16 hi/lo planes, or on the weights' integer values
    and block scales for q8_0 / iq4_xs / q5_K / q6_K / f16 / bf16): every output within the fp32
    reassociation bound of the oracle's double-accumulated matvec, at 131 tokens (a partial
    128-token tile) in the engine's formats, the residual added in the o projection."""
    _gemm_case(cuda, np.random.default_rng(51 + len(wo_type)), types, wo_type, 131)


def test_projection_rows_gemm_row_ranges(cuda):
    """The GEMM's per-row power-of-two scaling: hidden rows at 1e4 .. 1e-6 (the RMSNorm makes
    them alike) and attention rows at 1e6 .. 1e-7 (beyond f16's range both ways), each within
    the bound of the oracle; 16 tokens, the smallest GEMM batch."""
    rng = np.random.default_rng(57)
    T = 16
    scales = 10.0 ** np.linspace(4, -6, T)
    att_scales = 10.0 ** np.linspace(6, -7, T)
    _gemm_case(cuda, rng, ("q8_0", "q6_K", "f16"), "q8_0", T, x_scale=scales, att_scale=att_scales)


def test_projection_rows_gemm_1000_tokens(cuda):
    """1000 tokens: eight 128-token tiles and a partial one, dealt over the XCDs tile by tile as a
    long prefill's are, every output within the bound of the oracle."""
    _gemm_case(cuda, np.random.default_rng(61), ("q8_0", "q6_K", "q5_K"), "q8_0", 1000)


def test_projection_rows_gemm_passes_bit_identical(cuda):
    """Beyond 8192 tokens the projections run in passes of 8192 (the workspace's ceiling): each
    token's output does not depend on the batch it came in, so the 8300-token call's rows equal,
    bit for bit, the same rows computed as batches of their own (the first pass's first rows, the
    rows across the pass boundary, the second pass's last rows)."""
    import torch
    rng = np.random.default_rng(67)
    E, T = fa.N_EMBD, 8300
    wq, wk, wv = (oracle.random_blocks("q8_0", n, E, rng) for n in (4096, 512, 512))
    wo = oracle.random_blocks("q6_K", E, 4096, rng)
    ws = [(_dev(w, cuda), "q8_0") for w in (wq, wk, wv)]
    wo_d = (_dev(wo, cuda), "q6_K")
    x = torch.randn((T, E), device=cuda)
    g = torch.rand(E, device=cuda) + 0.5
    att = torch.randn((T, 4096), device=cuda)
    x0 = torch.randn((T, E), device=cuda)
    qkv = torch.empty((T, 5120), device=cuda)
    fa.qkv_proj_rows(ws[0], ws[1], ws[2], x, g, qkv)
    y = x0.clone()
    fa.o_proj_rows(wo_d, att, y)
    for a, b in ((0, 40), (8150, 8250), (8260, 8300)):
        q_part = torch.empty((b - a, 5120), device=cuda)
        fa.qkv_proj_rows(ws[0], ws[1], ws[2], x[a:b].contiguous(), g, q_part)
        y_part = x0[a:b].clone()
        fa.o_proj_rows(wo_d, att[a:b].contiguous(), y_part)
        torch.cuda.synchronize()
        assert torch.equal(qkv[a:b], q_part), ("qkv", a, b)
        assert torch.equal(y[a:b], y_part), ("o", a, b)
