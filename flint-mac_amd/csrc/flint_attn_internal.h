// Kernel parameter blocks and launchers shared by the HIP kernels and the C++
// host code (engine.cpp). Not part of the public C ABI (include/flint_attn.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace flint {

constexpr int MAX_SEQ = 64;  // sequences one batched decode launch can serve

// Decode launch (fused.metal AttnDecArgs {pos, is_full, n_split, keys_per_split},
// /root/reference/src/metal/fused_args.h:15-20, generalised to many sequences).
struct DecodeParams {
    const float *qkv;           // [n_seq][5120] raw q|k|v rows
    const float *q_norm;        // [128]
    const float *k_norm;        // [128]
    const float *sinks;         // [32]
    uint16_t *k_cache;          // sequence 0: [4][n_slots/32][32*128] (kt_index layout)
    uint16_t *v_cache;          // sequence 0: [4][n_slots/32][128][32] (V^T in 32-slot tiles)
    long long seq_stride;       // elements between two sequences' K (and V) caches
    float *att;                 // [n_seq][4096]
    float *partial;             // [n_seq][32][max_split][132]
    int n_slots;                // slots per kv head
    int slot_mask;              // SWA: n_slots - 1 (power of two); full: all ones
    int is_swa, has_rope, window, max_split;
    int tiles_per_split;        // 32-key tiles per split (all sequences)
    float rms_eps;
    int n_seq;
    float rope_freq[64];        // theta^(-2i/128), computed on the host like ref_model.cpp:55
    int pos[MAX_SEQ];           // sequence s decodes the token at pos[s]
    int n_split[MAX_SEQ];       // key splits of sequence s (grid x covers max_split)
};

hipError_t launch_decode(const DecodeParams &P, int dtype, hipStream_t stream);

// Prefill: q/k prep (k_qk_prefill, prefill.metal:99-133) + flash attention
// (k_attn_prefill, prefill.metal:141-266).
struct PrefillParams {
    const float *qkv;     // [T] rows of q_stride floats
    int q_stride;
    int p0, T;
    const float *q_norm, *k_norm, *sinks;
    float rms_eps;
    int is_swa, has_rope, window;
    float rope_freq[64];
    _Float16 *qh;         // [32][T][128] normed/roped q * log2(e)/sqrt(128), f16
    // keys/values the attention reads: key position kp lives at row kp - kbase
    uint16_t *kd;         // [4][k_rows/32][32*128] (kt_index layout)
    uint16_t *vd;         // [4][k_rows/32][128][32]
    int k_rows;           // row capacity per kv head (multiple of 32)
    int kbase;
    // SWA ring (cache) written for positions >= ring_from; copied into kd/vd for [kbase, p0)
    uint16_t *ring_k;     // [4][n_slots/32][32*128] (kt_index layout) or null
    uint16_t *ring_v;     // [4][n_slots/32][128][32]
    int ring_slots, ring_from;
    float *att;           // [T][4096]
};

hipError_t launch_prefill(const PrefillParams &P, int dtype, hipStream_t stream);

}  // namespace flint
