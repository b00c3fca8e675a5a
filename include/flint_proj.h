/*
 * flint attention projections on MI355X (gfx950): the attention block's matvecs in the
 * engine's GGUF weight formats, and the row dequantisation the reference tests them with.
 * Same conventions as flint_attn.h: device pointers, `stream` a hipStream_t as void*
 * (NULL = null stream), 0 / -1 with a NUL-terminated message in err[err_len].
 *
 * Weights are GGUF tensors as stored on disk: row-major, ggml block layouts
 * (/root/reference/third_party/ggml/ggml-common.h: block_q8_0 :251-256, block_q5_K
 * :343-356, block_q6_K :362-368, block_iq4_xs :454-460), rows of K elements in
 * K / block_elems blocks. The type ids are ggml's (/root/reference/src/gguf.h:14-19).
 * The quantised types are the ones the reference builds its attention kernels for
 * (/root/reference/src/metal/fused.metal:641); f32, f16 and bf16 rows are accepted too.
 */
#ifndef FLINT_PROJ_H
#define FLINT_PROJ_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FLINT_W_F32 0
#define FLINT_W_F16 1
#define FLINT_W_Q8_0 8
#define FLINT_W_Q5_K 13
#define FLINT_W_Q6_K 14
#define FLINT_W_IQ4_XS 23
#define FLINT_W_BF16 30

#define FLINT_N_EMBD 2048 /* hidden size (/root/reference/src/metal/flint_config.h:12) */

/* One weight tensor: device data (16-byte aligned) and its ggml type id. */
typedef struct {
    const void *data;
    int32_t type;
} flint_weight;

/* Bytes of one row of k elements, or -1 if the type is unsupported or k is not a whole
 * number of blocks (the reference's Tensor::row_bytes, /root/reference/src/gguf.h:38). */
int64_t flint_w_row_bytes(int32_t type, int64_t k);

/*
 * Row `row` of a weight tensor with rows of k elements, dequantised to fp32 into out[k]
 * (device, 16-byte aligned). Bit-identical to ggml's CPU dequantize_row_* (the reference's
 * check-deq compares its GPU rows with those: /root/reference/src/main.mm:27-48).
 * Replaces Engine::debug_get_row (/root/reference/src/engine.h:37, engine.mm:1370-1383;
 * kernel k_get_row, /root/reference/src/metal/fused.metal:589-600).
 */
int32_t flint_w_get_row(int32_t type, const void *w, int64_t k, int64_t row, float *out, void *stream,
                        char *err, int32_t err_len);

/*
 * Rows rows[0 .. n) (host array; each in [0, n_rows), the tensor's row count) of a weight
 * tensor with rows of k elements, dequantised to fp32 into out[i * k .. (i + 1) * k) (device,
 * 16-byte aligned), each bit-identical to flint_w_get_row of that row. The prefill's token
 * embedding: all n prompt tokens in one dispatch per 448 rows, as k_embed_rows
 * (/root/reference/src/metal/prefill.metal:272) at /root/reference/src/engine.mm:1067-1069.
 */
int32_t flint_w_get_rows(int32_t type, const void *w, int64_t k, int64_t n_rows, const int32_t *rows, int32_t n,
                         float *out, void *stream, char *err, int32_t err_len);

/*
 * The attention block's input side for one token: xn = RMSNorm(x) * attn_norm, then
 * qkv[0:4096] = Wq xn, qkv[4096:4608] = Wk xn, qkv[4608:5120] = Wv xn.
 *   x: device [2048], attn_norm: device [2048] gains, qkv: device [5120] (the raw q|k|v
 *   row flint_attn_decode takes). Wq/Wk/Wv rows have 2048 elements (4096 / 512 / 512 rows);
 *   each may have its own type; data 16-byte aligned.
 * Replaces enc_rmsnorm + three enc_mv at /root/reference/src/engine.mm:728-732 (kernels
 * k_rmsnorm / k_mv, /root/reference/src/metal/flint.metal:48-72, 217-240; the fused
 * variant k_qkv, fused.metal:215-232); CPU reference ref_model.cpp:107-110.
 */
int32_t flint_attn_qkv_proj(const flint_weight *wq, const flint_weight *wk, const flint_weight *wv, const float *x,
                            const float *attn_norm, float rms_eps, float *qkv, void *stream, char *err,
                            int32_t err_len);

/*
 * The attention block's output side: x[r] += sum_i Wo[r][i] * att[i] for r < 2048
 * (the residual add).  att: device [4096]; x: device [2048], updated in place.
 * Replaces enc_mv(L.o, att, x, add = true) at /root/reference/src/engine.mm:811 (k_mv with
 * add, flint.metal:48-72; fused variant k_mv_res, fused.metal:357-378); CPU reference
 * ref_model.cpp:150-151.
 */
int32_t flint_attn_o_proj(const flint_weight *wo, const float *att, float *x, void *stream, char *err,
                          int32_t err_len);

/*
 * The same two projections for n_tok tokens (the prefill side):
 * x: device [n_tok][2048]; qkv: device [n_tok] rows of qkv_stride floats (>= 5120), the raw
 * q|k|v at each row's start; att: device [n_tok][4096].
 * Below 16 tokens (or when the output rows are not 16-byte aligned) each token runs the
 * single-token kernel and gets exactly its bits. From 16 tokens the batch runs as a GEMM on
 * the matrix cores: weight and activation rows split into f16 hi/lo pairs (22 bits, each row
 * scaled by a power of two), products summed in fp32 (q8_0, iq4_xs, q5_K and q6_K weights keep
 * their integer values, exact in f16, and take their block scales and mins in fp32; f16
 * weights are used as they are, bf16 ones scaled by a power of two per block of 32); every
 * output is within fp32 reassociation of the single-token result (both within the oracle's
 * bound). Batches run in passes of at most 8192 tokens, so the device workspace has a ceiling:
 * 4 (rows + p) x K bytes, p = the pass's tokens padded to 128 (and p K / 8 more with q5_K
 * weights), allocated on first use and reused.
 * Replace the prefill's k_rmsnorm_rows + three mm (q, k, v), and mm(o) + k_add_rows, at
 * /root/reference/src/engine.mm:1083-1086 and 1105-1111.
 */
int32_t flint_attn_qkv_proj_rows(const flint_weight *wq, const flint_weight *wk, const flint_weight *wv,
                                 const float *x, int32_t n_tok, const float *attn_norm, float rms_eps, float *qkv,
                                 int32_t qkv_stride, void *stream, char *err, int32_t err_len);
int32_t flint_attn_o_proj_rows(const flint_weight *wo, const float *att, int32_t n_tok, float *x, void *stream,
                               char *err, int32_t err_len);

#ifdef __cplusplus
}
#endif
#endif
