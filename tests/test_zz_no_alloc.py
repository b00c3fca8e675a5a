"""flint_attn_decode_batch_noalloc (the decode entry point that allocates nothing: its split
partials live in the library's static device array) against flint_attn_decode_batch, the entry
point whose kernels it shares, through the C ABI: two calls in a row, the second on a smaller
batch, each bit-identical to the allocating entry point on the same cache. Also its host-side
limit: a plan whose partials exceed the array is rejected before any launch."""
import ctypes

import numpy as np
import pytest
import torch

import flint_attn as fa

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"\n[gpu-test] {msg}", flush=True)


def _both(kv, qkv, positions, kps=0):
    """att from the allocating entry point, then from the no-alloc one, on the same cache (both
    write the same current-token K/V to the same slots and read only keys before them)."""
    n = len(positions)
    arr = (ctypes.c_int32 * n)(*positions)
    outs = []
    for fn in (fa.lib().flint_attn_decode_batch, fa.lib().flint_attn_decode_batch_noalloc):
        att = torch.full((n, fa.Q_DIM), float("nan"), device=qkv.device)
        fa._call(fn, ctypes.byref(kv.desc), n, kv.seq_stride, fa._ptr(qkv), fa._ptr(att), arr, kps,
                 ctypes.c_void_p(fa._stream(None)))
        torch.cuda.synchronize()
        outs.append(att.cpu().numpy())
    return outs


@pytest.mark.parametrize("store", ["f16", "bf16"])
def test_decode_noalloc_matches_decode_batch(cuda, store):
    _say(f"decode no-alloc vs decode_batch store={store}")
    rng = np.random.default_rng(7)
    n_slots = 40000
    kv = fa.KVLayer(is_swa=False, has_rope=True, n_slots=n_slots, kv_dtype=store, rope_theta=1e6,
                    q_norm=rng.uniform(0.5, 1.5, 128), k_norm=rng.uniform(0.5, 1.5, 128),
                    sinks=rng.standard_normal(32), n_seq=3, device=cuda)
    kv.k.normal_()
    kv.v.normal_()
    qkv = torch.randn((3, fa.QKV_DIM), device=cuda)
    # first call: three long sequences (many splits, the largest partial set of the two calls)
    a, b = _both(kv, qkv, [39000, 21000, 9001])
    assert np.isfinite(a).all()
    assert np.array_equal(a, b), f"first call differs: max {np.nanmax(np.abs(a - b)):.3e}"
    # second call, smaller: two sequences, fewer splits, a set keys_per_split
    a, b = _both(kv, qkv[:2], [5000, 3000], kps=256)
    assert np.isfinite(a).all()
    assert np.array_equal(a, b), f"second call differs: max {np.nanmax(np.abs(a - b)):.3e}"
    # one sequence, one split (no partials at all)
    a, b = _both(kv, qkv[:1], [700])
    assert np.array_equal(a, b)


def test_decode_noalloc_rejects_oversized_plans(cuda):
    _say("decode no-alloc plan limit")
    kv = fa.KVLayer(is_swa=False, has_rope=False, n_slots=32800, kv_dtype="f16", device=cuda)
    qkv = torch.zeros((1, fa.QKV_DIM), device=cuda)
    att = torch.zeros((1, fa.Q_DIM), device=cuda)
    arr = (ctypes.c_int32 * 1)(32768)
    with pytest.raises(fa.FlintAttnError, match="more than the 4194304 bytes"):
        # 32-key splits: 1024 splits x 32 heads of partials, more than the array holds
        fa._call(fa.lib().flint_attn_decode_batch_noalloc, ctypes.byref(kv.desc), 1, kv.seq_stride, fa._ptr(qkv),
                 fa._ptr(att), arr, 32, ctypes.c_void_p(fa._stream(None)))
