"""Generate golden vectors for the attention hot path from the reference's own
CPU forward (oracle/_ref/ref_driver, compiled from /root/reference sources).

Run in the build container (needs /root/reference and `make -C oracle ref`):
    python tests/golden/make_ref_vectors.py
It writes tests/golden/ref_vectors.json. That file holds, per case, the layer
settings, the seed, a sha256 of the generated inputs, a sha256 of the
reference's float32 attention output for every position and head, and the raw
output values at probe positions for four heads (for diagnostics).

How the reference is driven: a synthetic one-layer Flint GGUF (F32/F16
tensors only) whose embedding row for token p carries position p's raw q|k|v
in x[0:5120] (zeros in x[5120:9216]); attn_q/k/v are one-hot selections,
attn_output copies att into hidden rows 5120..9215, the FFN is all zeros, so
RefModel::last_hidden()[5120 + i] is exactly the attention output att[i]
(ref_model.cpp:95-187; each matvec row holds one 1.0, and double(1) * v == v).
The raw q|k|v the attention sees is rmsnorm(x)[0:5120] with unit weights
(ref_model.cpp:107), which the test recomputes with the oracle's fo_rmsnorm.
"""
import hashlib
import json
import os
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle as fo  # noqa: E402

E = 9216  # n_embd of the synthetic model: 5120 (q|k|v) + 4096 (att copy)

# (name, is_swa, has_rope, theta, n_positions, seed, probe positions)
CASES = [
    ("full_nope", 0, 0, 10000.0, 300, 100, [0, 1, 31, 32, 200, 299]),
    ("swa_rope", 1, 1, 10000.0, 600, 101, [0, 1, 31, 32, 200, 511, 512, 513, 514, 599]),
    ("full_rope_1e6", 0, 1, 1.0e6, 300, 102, [0, 1, 63, 64, 299]),
]
PROBE_HEADS = [0, 7, 8, 31]

# the GGUF writer lives with the library (flint-mac_amd/gguf_writer.py)
sys.path.insert(0, os.path.join(ROOT, "flint-mac_amd"))
from gguf_writer import GGUF_ARRAY, GGUF_BOOL, GGUF_F32, GGUF_STRING, GGUF_U32, T_F16, T_F32, write_gguf  # noqa: E402,F401


def make_inputs(seed, n):
    rng = np.random.default_rng(seed)
    x = np.zeros((n, E), np.float32)
    x[:, :5120] = rng.standard_normal((n, 5120), dtype=np.float32)
    q_norm = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    k_norm = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    sinks = rng.standard_normal(32, dtype=np.float32)
    return x, q_norm, k_norm, sinks


def raw_qkv(x):
    """rmsnorm of each embedding row with unit weights (ref_model.cpp:107), first 5120 entries."""
    ones = np.ones(E, np.float32)
    return np.stack([fo.rmsnorm(row, ones)[:5120] for row in x])


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def write_model(path, x, q_norm, k_norm, sinks, is_swa, has_rope, theta):
    n = x.shape[0]
    wq = np.zeros((4096, E), np.float32)
    wq[np.arange(4096), np.arange(4096)] = 1
    wk = np.zeros((512, E), np.float32)
    wk[np.arange(512), 4096 + np.arange(512)] = 1
    wv = np.zeros((512, E), np.float32)
    wv[np.arange(512), 4608 + np.arange(512)] = 1
    wo = np.zeros((E, 4096), np.float32)
    wo[5120 + np.arange(4096), np.arange(4096)] = 1
    a = "flint."
    meta = [
        ("general.architecture", GGUF_STRING, "flint"),
        (a + "block_count", GGUF_U32, 1),
        (a + "embedding_length", GGUF_U32, E),
        (a + "attention.head_count", GGUF_U32, 32),
        (a + "attention.head_count_kv", GGUF_U32, 4),
        (a + "attention.key_length", GGUF_U32, 128),
        (a + "feed_forward_length", GGUF_U32, 1),
        (a + "expert_feed_forward_length", GGUF_U32, 1),
        (a + "expert_shared_feed_forward_length", GGUF_U32, 1),
        (a + "expert_count", GGUF_U32, 1),
        (a + "expert_used_count", GGUF_U32, 1),
        (a + "leading_dense_block_count", GGUF_U32, 1),
        (a + "attention.sliding_window", GGUF_U32, 513),
        (a + "attention.layer_norm_rms_epsilon", GGUF_F32, 1e-6),
        (a + "rope.freq_base", GGUF_F32, theta),
        (a + "attention.sliding_window_pattern", GGUF_ARRAY, [bool(is_swa)]),
        (a + "attention.rope_pattern", GGUF_ARRAY, [bool(has_rope)]),
        (a + "expert_gating_func", GGUF_U32, 2),
        (a + "expert_weights_norm", GGUF_BOOL, True),
        (a + "expert_weights_scale", GGUF_F32, 1.0),
    ]
    b = "blk.0."
    tensors = [
        ("token_embd.weight", x, T_F32),
        ("output_norm.weight", np.ones(E, np.float32), T_F32),
        ("output.weight", np.zeros((1, E), np.float32), T_F16),
        (b + "attn_norm.weight", np.ones(E, np.float32), T_F32),
        (b + "attn_q.weight", wq, T_F16),
        (b + "attn_k.weight", wk, T_F16),
        (b + "attn_v.weight", wv, T_F16),
        (b + "attn_output.weight", wo, T_F16),
        (b + "attn_q_norm.weight", q_norm, T_F32),
        (b + "attn_k_norm.weight", k_norm, T_F32),
        (b + "attn_sinks.weight", sinks, T_F32),
        (b + "ffn_norm.weight", np.ones(E, np.float32), T_F32),
        (b + "ffn_gate.weight", np.zeros((1, E), np.float32), T_F16),
        (b + "ffn_up.weight", np.zeros((1, E), np.float32), T_F16),
        (b + "ffn_down.weight", np.zeros((E, 1), np.float32), T_F16),
    ]
    write_gguf(path, meta, tensors)


def main():
    if not fo.build_ref():
        sys.exit("oracle/_ref/ref_driver cannot be built: /root/reference is absent")
    cases = []
    with tempfile.TemporaryDirectory() as tmp:
        for name, is_swa, has_rope, theta, n, seed, probes in CASES:
            x, q_norm, k_norm, sinks = make_inputs(seed, n)
            model = os.path.join(tmp, name + ".gguf")
            write_model(model, x, q_norm, k_norm, sinks, is_swa, has_rope, theta)
            out = os.path.join(tmp, name + ".f32")
            subprocess.run([fo.REF_DRIVER, model, str(n), out], check=True)
            att = np.fromfile(out, np.float32).reshape(n, 4096)
            cases.append({
                "name": name, "is_swa": is_swa, "has_rope": has_rope, "rope_theta": theta, "window": 513,
                "rms_eps": 1e-6, "n_positions": n, "seed": seed, "input_sha256": sha(raw_qkv(x)),
                "output_sha256": sha(att),
                "probes": {str(p): {str(h): att[p, h * 128:(h + 1) * 128].tolist() for h in PROBE_HEADS}
                           for p in probes},
            })
            print(f"{name}: {n} positions, output sha {cases[-1]['output_sha256'][:16]}", flush=True)
    with open(os.path.join(HERE, "ref_vectors.json"), "w") as f:
        json.dump({"generator": "tests/golden/make_ref_vectors.py", "embedding_length": E,
                   "probe_heads": PROBE_HEADS, "cases": cases}, f)


if __name__ == "__main__":
    main()
