// Kernel parameter blocks and launchers shared by the HIP kernels and the C++
// host code (engine.cpp). Not part of the public C ABI (include/flint_attn.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "flint_proj.h"  // flint_weight (include/, on the include path)

namespace flint {

constexpr int MAX_SEQ = 64;  // sequences one batched decode launch can serve
constexpr int PREFILL_ROW_ALIGN = 128;  // prefill attention-copy rows: a multiple of the LDS stage

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
    float *partial;             // [sum of n_split over sequences of more than one split][32][132]:
                                // sequence s's records start at split0[s], each head's consecutive
    int n_slots;                // slots per kv head
    int slot_mask;              // SWA: n_slots - 1 (power of two); full: all ones
    int is_swa, has_rope, window, max_split;
    float rms_eps;
    int n_seq;
    float rope_freq[64];        // theta^(-2i/128), computed on the host like ref_model.cpp:55
    int pos[MAX_SEQ];           // sequence s decodes the token at pos[s]
    int n_split[MAX_SEQ];       // key splits of sequence s
    int tps[MAX_SEQ];           // 32-key tiles per split of sequence s
    int wg_base[MAX_SEQ + 1];   // first work unit of sequence s (4 x v_slices per split); [n_seq] = the
                                // units of the launch (its grid size without V slices)
    int split0[MAX_SEQ];        // first partial record (in splits) of sequence s: the splits of the
                                // sequences before it that have more than one (one split needs none)
    int v_slices;               // 1, or 2 / 4 / 8 when every sequence has one split: a head's 128 output
                                // dims in that many workgroups (each reads all of K and its part of V)
};

hipError_t launch_decode(const DecodeParams &P, int dtype, hipStream_t stream);

// The static device array that holds the split partials of flint_attn_decode_batch_noalloc, and
// its address on the current device (looked up once per device, no allocation).
constexpr size_t DECODE_SCRATCH_BYTES = 4u << 20;
hipError_t decode_scratch(float **ptr);

// Prefill: k/v prep (k_qk_prefill, prefill.metal:99-133) + flash attention with
// the q prep fused (k_attn_prefill, prefill.metal:141-266).
struct PrefillParams {
    const float *qkv;     // [T] rows of q_stride floats
    int q_stride;
    int p0, T;
    const float *q_norm, *k_norm, *sinks;
    float rms_eps;
    int is_swa, has_rope, window;
    float rope_freq[64];
    // the layer's cache (kt_index / vt_index layouts): position p lives in slot
    // p & cache_mask; positions >= cache_from among the new ones are written to it
    uint16_t *cache_k, *cache_v;
    int n_slots, cache_mask, cache_from;
    // attention copy (f16, pk_index / pv_index layouts) of key positions
    // kbase + 32 n_direct .. p0 + T - 1 at rows 0 .., k_rows rows per kv head (multiple of
    // PREFILL_ROW_ALIGN): position p is copy row p - kbase - 32 n_direct
    _Float16 *sk;
    int k_rows, kbase;
    // per kv head and 32-key tile of the copy: the power-of-two exponents its K and V values
    // were scaled by to fit f16, (eK & 0xffff) | eV << 16 ([4][k_rows / 32], indexed like the
    // copy's tiles; 0 = stored as is)
    int *texp;
    // tiles 0 .. n_direct - 1 of the copy's range (whole tiles of cached positions) are read by
    // the flash kernel from the cache itself and neither copied nor given exponents: set for f16
    // caches, where the copy would hold the same bits, when no cache slot they read is rewritten
    // by this call's kv_prep with a key some query still needs; 0 otherwise
    int n_direct;
    unsigned call_id;     // nonzero id of this call (see g_scaled_call in attn_prefill.hip)
    float *att;           // [T][4096]
    // key splits (few query blocks over a long key range): each query block's tiles in n_split
    // runs of tps tiles, partial records [n_split][T][32][PF_PART_STRIDE] in part, merged by
    // prefill_combine_kernel; n_split = 1: no split, part unused
    int n_split, tps;
    float *part;
};
constexpr int PF_PART_STRIDE = 132;  // acc[128], m (log2 units), l, 2 pad
constexpr int PF_MAX_SPLIT = 64;

hipError_t launch_prefill(const PrefillParams &P, int dtype, hipStream_t stream);

// Weight formats of the attention projections (ggml type ids, /root/reference/src/gguf.h:14-19)
constexpr int W_F32 = 0, W_F16 = 1, W_Q8_0 = 8, W_Q5_K = 13, W_Q6_K = 14, W_IQ4_XS = 23, W_BF16 = 30;
// The batched projections' integer form: q8_0, iq4_xs, q6_K and q5_K weights are v * s (- m for
// q5_K) with v an integer of magnitude at most 127 (exact in f16), s the scale of 32 (q8_0,
// iq4_xs, q5_K) or 16 (q6_K) consecutive elements and m the min of 32 (q5_K); f16 weights are
// v * 1 with v the weight itself, bf16 weights v * 2^e with e putting their block of 32 in f16's
// range; 0: not of that form.
__host__ __device__ constexpr int w_int_sub(int t) {
    return t == W_Q8_0 || t == W_IQ4_XS || t == W_Q5_K || t == W_F16 || t == W_BF16 ? 32 : t == W_Q6_K ? 16 : 0;
}
__host__ __device__ constexpr bool w_int_min(int t) { return t == W_Q5_K; }

struct MatvecSeg {         // rows [row0, row0 + rows) of one launch come from one tensor
    const uint8_t *w;      // its first row (16-byte aligned)
    int type, row0, row_bytes;
};
struct MatvecParams {
    MatvecSeg seg[3];
    int n_seg, n_rows;
    const float *x;        // [n_tok] rows of x_stride floats, K inputs each
    const float *norm_w;   // [K] RMSNorm gains applied to each x row first, or null
    float eps;
    float *y;              // [n_tok] rows of y_stride floats: y = W x, or y += W x when add
    int add;
    int n_tok;             // tokens (grid x), >= 1
    long long x_stride, y_stride;
};
// Rows rows[0 .. n) of a weight tensor (row_bytes each) dequantised into out + i * out_stride.
constexpr int GR_MAX_ROWS = 448;  // rows per launch (the table travels in the kernel arguments)
struct RowsParams {
    const uint8_t *w;
    long long row_bytes, out_stride;
    float *out;
    int type, n_sub, n;   // n_sub: 32-element sub-blocks per row; n <= GR_MAX_ROWS
    int rows[GR_MAX_ROWS];
};
hipError_t launch_get_rows(const RowsParams &P, hipStream_t stream);
hipError_t launch_matvec(const MatvecParams &P, int k, hipStream_t stream);

// Batched projections on the matrix cores (proj_gemm.hip): weight rows and activation rows as
// f16 hi/lo planes scaled by per-row powers of two, then Y[t][n] (+)= 2^(e_t + f_n) sum_k ...
struct GemmWeightParams {  // wprep: rows [0, N) of the segments -> wh, wl [N][K], fexp [N]
    MatvecSeg seg[3];
    int n_seg;
    _Float16 *wh, *wl;
    int *fexp;
    // isub: every segment in the integer form (w_int_sub), 32 if all scales cover 32 elements,
    // else 16; then wh holds the values and wd the scales, [N / 128 row tiles][K / 32 blocks]
    // [32 / isub][128 rows] floats (in wl's memory), and the GEMM takes the integer form.
    // 0: the hi/lo planes. imin: a segment has mins (q5_K); then wm holds them (0 for the other
    // segments), [N / 128][K / 32][128] floats after wd.
    int isub, imin;
    float *wd, *wm;
};
struct GemmActParams {     // xprep: rows [0, T_pad) -> xh, xl [T_pad][K], eexp [T_pad]
    const float *x;        // [T] rows of x_stride floats (16-byte aligned)
    long long x_stride;
    const float *norm_w;   // [K] RMSNorm gains, or null (no norm)
    float eps;
    int T, T_pad;          // T_pad: T rounded up to the GEMM tile (rows past T are zeros)
    _Float16 *xh, *xl;
    int *eexp;
    float *xs;             // or null; else the sums of (xh + xl) over each 32-element block,
                           // [T_pad / 128][K / 32][128] (the integer form's mins need them)
};
struct GemmParams {
    const _Float16 *wh, *wl, *xh, *xl;
    const int *fexp, *eexp;
    int isub, imin;        // the weights as integer values, scales and mins (GemmWeightParams)
    const float *wd, *wm, *xs;
    float *y;              // [T] rows of y_stride floats (16-byte aligned, stride a multiple of 4)
    long long y_stride;
    int add, N, K, T;
};
constexpr int GEMM_TILE = 128;       // tokens and rows per gemm3 workgroup
constexpr int GEMM_MIN_TOKENS = 16;  // batches from this size take the GEMM
constexpr int GEMM_PASS_TOKENS = 8192;  // tokens per GEMM pass (a multiple of GEMM_TILE): bounds the workspace
// prep_weights = false: W's planes already hold the rows (built earlier and kept by the caller)
hipError_t launch_proj_gemm(const GemmWeightParams &W, const GemmActParams &X, const GemmParams &G, bool prep_weights,
                            hipStream_t stream);
int matvec_row_multiple(int k);  // n_rows of a matvec launch must be a multiple of this

// A projection's weight planes kept by a caller that runs many batches through the same weights
// (the model's layer-major prefill): one device block of planes_bytes(N, K, isub) holding wh, wl
// [N][K] and fexp [N], built once with build_*_planes; the *_rows projections given them skip
// their per-call weight prep (the planes are the same bits that prep would write). In the
// integer form (gemm_int_form) wh holds the values and wl's place the scales (N K / sub floats),
// then the mins (N K / 32 floats, if any), with no fexp.
struct WeightPlanes {
    _Float16 *wh = nullptr, *wl = nullptr;
    int *fexp = nullptr;
};
struct IntForm {  // a projection's integer form: sub 32, 16 or 0 (none); min: a segment has mins
    int sub = 0;
    bool min = false;
};
IntForm gemm_int_form(const MatvecSeg *seg, int n_seg);
IntForm qkv_gemm_form(const flint_weight *wq, const flint_weight *wk, const flint_weight *wv);
IntForm o_gemm_form(const flint_weight *wo);
size_t planes_bytes(int N, int K, IntForm f);
WeightPlanes planes_at(void *mem, int N, int K, IntForm f);
void build_qkv_planes(const flint_weight *wq, const flint_weight *wk, const flint_weight *wv, const WeightPlanes &pl,
                      hipStream_t stream);
void build_o_planes(const flint_weight *wo, const WeightPlanes &pl, hipStream_t stream);
// flint_attn_qkv_proj_rows / flint_attn_o_proj_rows with the weights' planes (pl may be null)
void qkv_proj_rows_planes(const flint_weight *wq, const flint_weight *wk, const flint_weight *wv, const float *x,
                          int n_tok, const float *attn_norm, float eps, float *qkv, int qkv_stride,
                          const WeightPlanes *pl, hipStream_t stream);
void o_proj_rows_planes(const flint_weight *wo, const float *att, int n_tok, float *x, const WeightPlanes *pl,
                        hipStream_t stream);

}  // namespace flint

struct flint_attn_engine;

namespace flint {

// Sets layer il's SWA window and RMSNorm epsilon (the GGUF's attention.sliding_window and
// attention.layer_norm_rms_epsilon); throws std::runtime_error on a bad index or window.
void engine_set_layer_params(flint_attn_engine *e, int il, int window, float rms_eps);

}  // namespace flint
