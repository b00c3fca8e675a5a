"""Golden rows for the weight formats of the attention projections, from the reference's own
CPU dequantisation: ggml's dequantize_row_* as vendored by the reference
(/root/reference/src/ref/dequant.c + dequant_gen.c), compiled into oracle/_ref/libref_dequant.so.

Run in the build container (needs /root/reference and `make -C oracle ref`):
    python tests/golden/make_weight_rows.py
It writes tests/golden/weight_rows.npz: for each quantised type, seeded random rows of
512 elements (random quant bytes; fp16 scales drawn as quantisers write them, plus rows
whose scales are 1.0, the smallest subnormal and the largest finite half) and the
reference's float32 output for each row, as raw bits.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle  # noqa: E402

K = 512
SCALE_OFFSETS = {"q8_0": [0], "q5_K": [0, 2], "q6_K": [208], "iq4_xs": [0]}


def special_rows(wtype, rng):
    """Rows whose every fp16 scale is one special half: 1.0, 2^-24 (smallest subnormal),
    65504 (largest finite) and -1.0."""
    out = []
    bb = int(oracle.lib().fo_block_bytes(oracle.W_TYPES[wtype]))
    for h in (0x3C00, 0x0001, 0x7BFF, 0xBC00):
        row = oracle.random_blocks(wtype, 1, K, rng)[0].copy()
        blocks = row.reshape(-1, bb)
        for off in SCALE_OFFSETS[wtype]:
            blocks[:, off] = h & 0xFF
            blocks[:, off + 1] = h >> 8
        out.append(row)
    return np.stack(out)


def main():
    if oracle.ref_dequant_rows("q8_0", np.zeros(34 * K // 32, np.uint8), K) is None:
        sys.exit("oracle/_ref/libref_dequant.so is missing: run `make -C oracle ref` (needs /root/reference)")
    rng = np.random.default_rng(20261201)
    arrays = {}
    for wtype in ("q8_0", "q5_K", "q6_K", "iq4_xs"):
        rows = np.concatenate([oracle.random_blocks(wtype, 8, K, rng), special_rows(wtype, rng)])
        ref = oracle.ref_dequant_rows(wtype, rows, K)
        arrays[wtype + "_rows"] = rows
        arrays[wtype + "_bits"] = ref.view(np.uint32)
    np.savez_compressed(os.path.join(HERE, "weight_rows.npz"), **arrays)
    print("wrote", os.path.join(HERE, "weight_rows.npz"))


if __name__ == "__main__":
    main()
