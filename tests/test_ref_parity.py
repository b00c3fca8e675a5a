"""The oracle against the reference's own CPU forward (RefModel::forward,
/root/reference/src/ref/ref_model.cpp:95-149), bit for bit.

tests/golden/ref_vectors.json was written by tests/golden/make_ref_vectors.py,
which runs oracle/_ref/ref_driver (the reference compiled from its sources) on
a synthetic one-layer Flint model. Each case stores the sha256 of the
reference's float32 attention output over every position and head; the oracle,
run with fp32 storage (what RefModel keeps), must hash to the same value."""
import json
import os

import numpy as np
import pytest

import oracle as fo
from golden import make_ref_vectors as g

HERE = os.path.dirname(os.path.abspath(__file__))
VECTORS = json.load(open(os.path.join(HERE, "golden", "ref_vectors.json")))


@pytest.mark.parametrize("case", VECTORS["cases"], ids=lambda c: c["name"])
def test_oracle_bit_exact_vs_reference_forward(case):
    x, q_norm, k_norm, sinks = g.make_inputs(case["seed"], case["n_positions"])
    qkv = g.raw_qkv(x)
    assert g.sha(qkv) == case["input_sha256"], "input generator drifted"
    L = fo.Layer(q_norm, k_norm, sinks, case["is_swa"], case["has_rope"], "f32", case["rope_theta"],
                 case["window"], case["rms_eps"])
    n = case["n_positions"]
    K = np.zeros((n, 512), np.float32)
    V = np.zeros((n, 512), np.float32)
    att = fo.prefill(L, qkv, 0, K, V, n_threads=8)
    for p, heads in case["probes"].items():
        for h, vals in heads.items():
            got = att[int(p), int(h) * 128:(int(h) + 1) * 128]
            assert np.array_equal(got, np.array(vals, np.float32)), f"pos {p} head {h}"
    assert g.sha(att) == case["output_sha256"]
