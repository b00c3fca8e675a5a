"""Golden vectors for the attention blocks loaded from a GGUF model, from the reference's
own CPU forward (RefModel::forward, /root/reference/src/ref/ref_model.cpp:95-187, run by
oracle/_ref/ref_driver, which is compiled from the reference's sources).

The synthetic model has Flint's attention shapes (n_embd 2048, 32 q / 4 kv heads,
head_dim 128) and two layers:
  layer 0: full attention, no RoPE; attn_q/k/v in q8_0, attn_output in q6_K;
  layer 1: sliding window N_SWA = 100 (not a multiple of 32), NEOX RoPE theta 1e4;
           attn_q q5_K, attn_k iq4_xs, attn_v q6_K, attn_output q8_0.
Its FFN weights are zero, so each layer adds only its attention block to the hidden state
(ref_model.cpp:151-187 adds a zero FFN output): RefModel::last_hidden() after both layers
is what two attention blocks compute. Token p is fed at position p; its embedding row is
f16 N(0,1). Weights are seeded random blocks whose fp16 scales are set so that the rows
have a standard deviation of about 1/sqrt(row length); norm gains U(0.5, 1.5), sinks N(0,1).

Run in the build container (needs /root/reference and `make -C oracle ref`):
    python tests/golden/make_block_vectors.py
It writes tests/golden/block_vectors.json: a sha256 of the generated model (generator
drift check), a sha256 of the reference's float32 hidden state at every position, and raw
values of the first PROBE_DIMS dims at probe positions. The GGUF itself is regenerated
from the seed by every test that needs it (write_model), so it is not committed.
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
sys.path.insert(0, HERE)
import oracle as fo  # noqa: E402
import make_ref_vectors as g  # noqa: E402
import gguf_writer as gw  # noqa: E402  (flint-mac_amd/, on the path via make_ref_vectors)

E = 2048
SEED = 300
N_POS = 160
N_SWA = 100
THETA = 1.0e4
RMS_EPS = 1e-6
# (is_swa, has_rope, q, k, v, o weight types)
LAYERS = [
    (0, 0, "q8_0", "q8_0", "q8_0", "q6_K"),
    (1, 1, "q5_K", "iq4_xs", "q6_K", "q8_0"),
]
PROBES = [0, 1, 31, 99, 100, 101, 159]
PROBE_DIMS = 32
T_F32, T_F16 = g.T_F32, g.T_F16
SCALE_OFFSETS = {"q8_0": [0], "q5_K": [0, 2], "q6_K": [208], "iq4_xs": [0]}


def scaled_rows(wtype, n_rows, k, rng):
    """Random rows of a block format whose dequantised values have std ~ 1/sqrt(k): the
    fp16 scale fields of random blocks are multiplied by one common factor (the values
    are linear in them)."""
    rows = fo.random_blocks(wtype, n_rows, k, rng).copy()
    std = float(fo.dequant_rows(wtype, rows[:64], k).std())
    c = (1.0 / np.sqrt(k)) / std
    bb = int(fo.lib().fo_block_bytes(fo.W_TYPES[wtype]))
    blocks = rows.reshape(n_rows, -1, bb)
    for off in SCALE_OFFSETS[wtype]:
        h = blocks[:, :, off:off + 2].copy().view(np.float16)
        blocks[:, :, off:off + 2] = (h.astype(np.float32) * c).astype(np.float16).view(np.uint8)
    return rows


def make_model(seed=SEED, n_pos=N_POS):
    rng = np.random.default_rng(seed)
    m = {"embd": rng.standard_normal((n_pos, E)).astype(np.float16), "layers": []}
    for is_swa, has_rope, tq, tk, tv, to in LAYERS:
        m["layers"].append({
            "is_swa": is_swa, "has_rope": has_rope,
            "attn_norm": rng.uniform(0.5, 1.5, E).astype(np.float32),
            "q": (tq, scaled_rows(tq, 4096, E, rng)),
            "k": (tk, scaled_rows(tk, 512, E, rng)),
            "v": (tv, scaled_rows(tv, 512, E, rng)),
            "o": (to, scaled_rows(to, E, 4096, rng)),
            "q_norm": rng.uniform(0.5, 1.5, 128).astype(np.float32),
            "k_norm": rng.uniform(0.5, 1.5, 128).astype(np.float32),
            "sinks": rng.standard_normal(32).astype(np.float32),
        })
    return m


def model_sha(m):
    h = hashlib.sha256(m["embd"].tobytes())
    for L in m["layers"]:
        for key in ("attn_norm", "q_norm", "k_norm", "sinks"):
            h.update(L[key].tobytes())
        for key in ("q", "k", "v", "o"):
            h.update(L[key][0].encode() + L[key][1].tobytes())
    return h.hexdigest()


def write_model(path, m, meta_edit=None, tensor_edit=None):
    """Writes the model as a Flint GGUF. meta_edit {key: None (drop) | (type, value)} and
    tensor_edit (a function of the tensor list) make the defective files of the loader tests."""
    meta = gw.flint_meta([L["is_swa"] for L in m["layers"]], [L["has_rope"] for L in m["layers"]], N_SWA, THETA,
                         RMS_EPS)
    tensors = [
        ("token_embd.weight", m["embd"].astype(np.float32), T_F16),
        ("output_norm.weight", np.ones(E, np.float32), T_F32),
        ("output.weight", np.zeros((1, E), np.float32), T_F16),
    ]
    for il, L in enumerate(m["layers"]):
        b = f"blk.{il}."
        tensors += [(b + "attn_norm.weight", L["attn_norm"], T_F32)]
        for key, name, k, n in (("q", "attn_q", E, 4096), ("k", "attn_k", E, 512), ("v", "attn_v", E, 512),
                                ("o", "attn_output", 4096, E)):
            wtype, rows = L[key]
            tensors.append((b + name + ".weight", rows, fo.W_TYPES[wtype], (k, n)))
        tensors += [
            (b + "attn_q_norm.weight", L["q_norm"], T_F32),
            (b + "attn_k_norm.weight", L["k_norm"], T_F32),
            (b + "attn_sinks.weight", L["sinks"], T_F32),
        ] + gw.flint_zero_ffn(il)
    for key, val in (meta_edit or {}).items():
        meta = [e for e in meta if e[0] != key] + ([(key,) + tuple(val)] if val is not None else [])
    if tensor_edit:
        tensors = tensor_edit(tensors)
    g.write_gguf(path, meta, tensors)


def oracle_blocks(m, store):
    """The model's layers as the oracle's BlockLayers, weights dequantised by the oracle
    (bit-identical to ggml's dequantize_row_*, tests/golden/weight_rows.npz)."""
    out = []
    for L in m["layers"]:
        deq = {key: fo.dequant_rows(L[key][0], L[key][1], 4096 if key == "o" else E) for key in "qkvo"}
        attn = fo.Layer(L["q_norm"], L["k_norm"], L["sinks"], L["is_swa"], L["has_rope"], store, THETA, N_SWA,
                        RMS_EPS)
        out.append(fo.BlockLayer(L["attn_norm"], deq["q"], deq["k"], deq["v"], deq["o"], attn, RMS_EPS))
    return out


def main():
    if not fo.build_ref():
        sys.exit("oracle/_ref/ref_driver cannot be built: /root/reference is absent")
    m = make_model()
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "blocks.gguf")
        write_model(path, m)
        out = os.path.join(tmp, "hidden.f32")
        subprocess.run([fo.REF_DRIVER, path, str(N_POS), out, str(len(LAYERS))], check=True)
        hidden = np.fromfile(out, np.float32).reshape(N_POS, E)
    doc = {
        "generator": "tests/golden/make_block_vectors.py", "seed": SEED, "n_positions": N_POS, "n_swa": N_SWA,
        "rope_theta": THETA, "layers": [list(L) for L in LAYERS], "model_sha256": model_sha(m),
        "hidden_sha256": g.sha(hidden), "probe_dims": PROBE_DIMS,
        "probes": {str(p): hidden[p, :PROBE_DIMS].tolist() for p in PROBES},
    }
    with open(os.path.join(HERE, "block_vectors.json"), "w") as f:
        json.dump(doc, f)
    print(f"hidden sha {doc['hidden_sha256'][:16]}, max |h| {np.abs(hidden).max():.3f}", flush=True)


if __name__ == "__main__":
    main()
