/*
 * flint attention blocks loaded from a GGUF model on MI355X (gfx950).
 *
 * The engine's decode step and layer-major prefill, restricted to the attention half
 * of each layer: RMSNorm -> q/k/v projections -> attention (QK norm, RoPE, KV cache,
 * sinks) -> o projection added to the residual. The FFN / MoE half and the output head
 * are not part of this library; a caller that runs them interleaves its own stages
 * between the blocks, as the reference's encode_token does
 * (/root/reference/src/engine.mm:717-893) and its prefill layer loop
 * (/root/reference/src/engine.mm:1077-1112).
 *
 * Same conventions as flint_attn.h: device pointers, `stream` a hipStream_t as void*
 * (NULL = null stream), 0 / -1 with a NUL-terminated message in err[err_len]. A model
 * is one session; calls on it must be serialised (/root/reference/src/capi.h:1).
 */
#ifndef FLINT_MODEL_H
#define FLINT_MODEL_H

#include <stdint.h>

#include "flint_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct flint_attn_model flint_attn_model;

/* Hyper-parameters read from the GGUF, as HParams::from_gguf reads them
 * (/root/reference/src/ref/ref_model.cpp:13-39). */
typedef struct {
    int32_t n_layer, n_embd, n_head, n_head_kv, head_dim, n_vocab;
    int32_t n_ff_dense, n_ff_exp, n_ff_shexp, n_expert, n_expert_used, n_dense_lead;
    int32_t n_swa;
    float rms_eps, rope_theta;
} flint_attn_hparams;

/*
 * Opens a Flint GGUF: maps the file, reads and validates the hyper-parameters with the
 * reference's checks and messages (gguf.cpp:137-194, ref_model.cpp:13-39: "cannot open
 * <path>", "not a GGUF file: <path>", "gguf: missing key <key>", "not a flint model: <arch>",
 * "unexpected routing config (expect sigmoid + norm, scale 1)", "missing tensor <name>", ...),
 * checks every attention tensor's type and shape, then copies the token embedding and each
 * layer's attention tensors (attn_norm, attn_q/k/v/output, attn_q_norm/k_norm, attn_sinks)
 * to HBM and allocates the KV caches: full layers n_ctx positions, SWA layers a
 * FLINT_SWA_RING-slot ring (/root/reference/src/engine.mm:472-513).
 * kv_dtype: FLINT_KV_F16 (the reference's cache type) or FLINT_KV_BF16.
 * Everything up to the first device allocation runs on the host only.
 */
flint_attn_model *flint_attn_model_open(const char *gguf_path, int32_t n_ctx, int32_t kv_dtype, char *err,
                                        int32_t err_len);
void flint_attn_model_close(flint_attn_model *m);

/* Copies the hyper-parameters into *hp and, when not NULL, the per-layer flags
 * (attention.sliding_window_pattern / attention.rope_pattern) into is_swa[n_layer] and
 * has_rope[n_layer]. 0 / -1. */
int32_t flint_attn_model_hparams(const flint_attn_model *m, flint_attn_hparams *hp, uint8_t *is_swa,
                                 uint8_t *has_rope);

/* The model's attention engine (its KV caches and layer descriptors), or NULL. */
flint_attn_engine *flint_attn_model_engine(flint_attn_model *m);

/*
 * Token embedding rows: x[i][0:n_embd] = token_embd row tokens[i], dequantised to fp32
 * (k_get_row / k_embed_rows, /root/reference/src/engine.mm:719, 1068).
 * tokens: host [n]; x: device [n][n_embd].
 */
int32_t flint_attn_model_embed(flint_attn_model *m, const int32_t *tokens, int32_t n, float *x, void *stream,
                               char *err, int32_t err_len);

/*
 * Decode step of layer il's attention block for the token at position pos:
 *   x += Wo . attention(Wq/Wk/Wv . (RMSNorm(x) * attn_norm), pos)
 * x: device [n_embd], updated in place. att: device [4096] that receives the attention
 * output, or NULL (an internal buffer). The token's K/V go into the layer's cache at
 * slot(pos). Replaces the attention half of encode_token, /root/reference/src/engine.mm:726-812.
 */
int32_t flint_attn_model_block_decode(flint_attn_model *m, int32_t il, float *x, int32_t pos, float *att,
                                      void *stream, char *err, int32_t err_len);

/*
 * Layer-major prefill of layer il's attention block for the T tokens at positions
 * p0 .. p0+T-1: X[t] += Wo . attention_t(...), all tokens in one pass (any T; the
 * reference runs 512-token chunks, engine.mm:1077-1112). X: device [T][n_embd], updated
 * in place; att: device [T][4096] or NULL. The result equals T decode steps in order.
 */
int32_t flint_attn_model_block_prefill(flint_attn_model *m, int32_t il, float *X, int32_t p0, int32_t T,
                                       float *att, void *stream, char *err, int32_t err_len);

/*
 * The prefill projections' kept weight planes (no counterpart in the reference): from the first
 * prefill block of 16 or more tokens, a model keeps every layer's q|k|v and o weights as f16
 * hi/lo planes in one device allocation (75.5 MB a layer; 40.1 MB for q8_0 weights, kept as
 * their values and block scales: 2.0 GB for Flint's 49 layers in q8_0), so later
 * prefill blocks skip their per-call weight prep. on = 0 frees them (after a device
 * synchronize) and prefill rebuilds the planes in its workspace on every call; on = 1 (the
 * default) allows them again. When the allocation fails, prefill goes on without them and
 * tries again in its next call. 0 / -1.
 */
int32_t flint_attn_model_set_weight_planes(flint_attn_model *m, int32_t on, char *err, int32_t err_len);
/* 1: planes kept; 2: allowed, not allocated yet; 0: switched off; -1: allowed, but the last
 * allocation failed (the projections rebuild the planes per call); -2: no model. */
int32_t flint_attn_model_weight_planes(const flint_attn_model *m);

/*
 * The model as one session over its attention blocks, as the reference's Engine drives its
 * layers (/root/reference/src/engine.h:24-79). The position is the number of tokens processed.
 * With the FFN half outside this library, the hidden state these calls return is that of the
 * attention blocks alone: for a model whose FFN weights are zero it is RefModel::last_hidden()
 * (/root/reference/src/ref/ref_model.cpp:95-187).
 */
int32_t flint_attn_model_pos(const flint_attn_model *m);   /* Engine::pos, engine.h:57 */
int32_t flint_attn_model_n_ctx(const flint_attn_model *m); /* Engine::n_ctx, engine.h:60 */

/*
 * Rolls the session back to position pos, 0 <= pos <= the current position (0 / -1), as
 * flint_truncate (/root/reference/src/capi.mm:52-56): the caches keep their contents and the
 * next token goes to position pos. SWA layers keep only their last FLINT_SWA_RING positions,
 * so after a rollback of more than FLINT_SWA_RING - window tokens (511 for Flint) the caller
 * re-prefills from max(0, pos - (window - 1)), the rule of /root/reference/src/capi.h:27-28.
 */
int32_t flint_attn_model_truncate(flint_attn_model *m, int32_t pos);

/*
 * Engine::step (engine.mm:902-940) over the attention blocks: the token's embedding row
 * through every layer's block at the current position, which then advances by one.
 * x: device [n_embd] receives the hidden state after the last layer.
 * Fails with "context full" when the position has reached n_ctx (engine.mm:904).
 */
int32_t flint_attn_model_step(flint_attn_model *m, int32_t token, float *x, void *stream, char *err,
                              int32_t err_len);

/*
 * Engine::prefill (engine.mm:971-1255) over the attention blocks, layer-major: tokens[n]
 * (host) at the current position, every token through layer 0, then layer 1, ...; the
 * position advances by n. X: device [n][n_embd] receives the hidden states.
 * Fails with "prefill: empty" or "prefill: context full" (engine.mm:975-976).
 */
int32_t flint_attn_model_prefill(flint_attn_model *m, const int32_t *tokens, int32_t n, float *X, void *stream,
                                 char *err, int32_t err_len);

/*
 * Engine::enable_profiling (engine.h:54-55, engine.mm:948-951): with `on` set, every later
 * step and prefill also records a HIP event after each of its stages on the call's stream (the
 * embedding "embed", then per layer L "blk.L.qkv", "blk.L.attn" and "blk.L.o"), which
 * flint_attn_model_last_profile reads. The events between stages order nothing, but they add
 * work to the stream, so profiled times are for relative shares, as the reference's are.
 * `on` = 0 turns it off. 0, or -1 without a model.
 */
int32_t flint_attn_model_enable_profiling(flint_attn_model *m, int32_t on);

/*
 * Engine::last_gpu_ms (engine.h:63; engine.mm:931, the command buffer's GPU start to end): the
 * GPU time of the last flint_attn_model_step or _prefill, from HIP events recorded on its stream
 * where it started and ended. Waits for that call's work to finish. -1 when no step or prefill
 * has completed its launches yet.
 */
double flint_attn_model_last_gpu_ms(flint_attn_model *m);

/*
 * Engine::last_encode_ms (engine.h:63; engine.mm:906-915, the host's encoding time): the host
 * time the last flint_attn_model_step or _prefill took to check its arguments and enqueue its
 * launches, in ms. -1 when no step or prefill has completed its launches yet.
 */
double flint_attn_model_last_encode_ms(const flint_attn_model *m);

/*
 * Engine::last_profile (engine.h:56, engine.mm:953-966): the stages of the last step or
 * prefill in order, each with its GPU time in ms (consecutive event marks, so the times sum to
 * flint_attn_model_last_gpu_ms). Unprofiled calls have one stage, "step" or "prefill". Writes
 * min(n, max_n) entries: ms[i], and when labels is given the i-th label, NUL-terminated and cut
 * to label_len - 1 bytes, at labels + i * label_len. Returns n, the number of stages (with ms
 * NULL or max_n <= 0: only n, without waiting), or -1 when there is none (or on a HIP error).
 * Waits for that call's work to finish.
 */
int32_t flint_attn_model_last_profile(flint_attn_model *m, char *labels, int32_t label_len, double *ms,
                                      int32_t max_n);

#ifdef __cplusplus
}
#endif
#endif
