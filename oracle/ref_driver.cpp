// Drives the reference's own fp32 CPU forward (flint::ref::RefModel, compiled
// from /root/reference/src/ref/ref_model.cpp where it lies) on a synthetic
// one-layer Flint GGUF written by tests/golden/make_ref_vectors.py, and dumps
// the attention output of every position.
//
// TEST INFRASTRUCTURE ONLY (it builds the checker's checker): nothing in the
// product links or runs it.
//
// The synthetic model makes the attention block observable:
//   n_embd E = 9216; token t's embedding row carries the wanted raw q|k|v in
//   x[0:5120] and zeros in x[5120:9216];
//   attn_q/k/v are one-hot selections of xn[0:5120], attn_output copies att
//   into rows 5120..9215 and zeros the rest, and the FFN weights are zero, so
//   after the layer (ref_model.cpp:95-187) last_hidden()[5120 + i] == att[i]
//   exactly: every matvec row holds a single 1.0 and double(1.0) * v == v.
//
// Usage: ref_driver <model.gguf> <n_positions> <out.f32>
//   writes n_positions x 4096 float32 (att of each position, in order).
// Usage: ref_driver <model.gguf> <n_positions> <out.f32> <n_layers>
//   runs the first n_layers layers and writes n_positions x n_embd float32: the hidden
//   state after them (RefModel::last_hidden) at each position, for models of any n_embd.
#include <cstdio>
#include <cstdlib>
#include <exception>
#include <vector>

#include "gguf.h"
#include "ref/ref_model.h"

int main(int argc, char **argv) {
    if (argc != 4 && argc != 5) {
        std::fprintf(stderr, "usage: %s <model.gguf> <n_positions> <out.f32> [n_layers]\n", argv[0]);
        return 2;
    }
    try {
        flint::GgufFile f(argv[1]);
        flint::ref::RefModel model(f, 8);
        const bool hidden = argc == 5;
        model.debug_n_layers = hidden ? std::atoi(argv[4]) : 1;
        const int n = std::atoi(argv[2]);
        std::FILE *out = std::fopen(argv[3], "wb");
        if (!out) {
            std::perror(argv[3]);
            return 1;
        }
        for (int p = 0; p < n; p++) {
            model.forward(p);  // token id p: the embedding row for position p
            const std::vector<float> &h = model.last_hidden();
            if (hidden) {
                std::fwrite(h.data(), sizeof(float), h.size(), out);
                continue;
            }
            if (h.size() != 9216) {
                std::fprintf(stderr, "unexpected hidden size %zu\n", h.size());
                return 1;
            }
            std::fwrite(h.data() + 5120, sizeof(float), 4096, out);
        }
        std::fclose(out);
    } catch (const std::exception &e) {
        std::fprintf(stderr, "ref_driver: %s\n", e.what());
        return 1;
    }
    return 0;
}
