/*
 * flint attention hot path for AMD Instinct MI355X (gfx950): public C ABI.
 *
 * Plain C types only (pointers, sizes, ints, floats). Device pointers are HIP
 * device memory; `stream` is a hipStream_t passed as void* (NULL = the null
 * stream). Every entry point that can fail returns 0 on success and -1 on
 * failure with a NUL-terminated message in err[err_len] (err may be NULL),
 * the error style of the reference's C API (/root/reference/src/capi.mm:17-22).
 * Nothing here is thread-safe across concurrent calls on one engine or one
 * device workspace; callers serialise, as the reference requires of its
 * engine (/root/reference/src/capi.h:1). The workspace (split partials, the
 * prefill's attention copy and partial records, projection scratch) is one set
 * per device, shared by every layer, engine and model, so the calls must also be
 * ordered on the GPU: one stream per device, or an event between streams. Host
 * order alone lets kernels of two streams overlap.
 *
 * KV cache layout per layer and kv head (HBM, 16-bit elements), in tiles of 32 slots:
 *   K: [N_HEAD_KV][n_slots/32][4096]; within a tile, (slot r = slot % 32, dim d) is at
 *      element 8*(((r>>2)&1)*256 + (d>>5)*64 + ((d>>3)&3)*16 + ((r>>3)<<2 | (r&3))) + (d&7)
 *      (the order the decode kernel's MFMA reads K, so each load reads 1 KiB contiguous)
 *   V: [N_HEAD_KV][n_slots/32][HEAD_DIM][32]   (V transposed within the tile)
 * SWA layers: n_slots is a power of two >= window (1024 for Flint) and
 * position p lives in slot p & (n_slots-1); full-attention layers: slot = p.
 * n_slots is at most FLINT_MAX_SLOTS, so a kv head's K (or V) cache stays below 2^31 bytes
 * and the kernels address it with 32-bit offsets (the reference's n_ctx bound,
 * /root/reference/src/metal/flint_config.h:29-31, is far below it).
 * (The reference keeps position-major [slot][kv_head][128] for both,
 * /root/reference/src/engine.mm:509-511, fused.metal:275.)
 */
#ifndef FLINT_ATTN_H
#define FLINT_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Flint's attention shapes (/root/reference/src/metal/flint_config.h:13-31). */
#define FLINT_N_HEAD 32
#define FLINT_N_HEAD_KV 4
#define FLINT_HEAD_DIM 128
#define FLINT_Q_DIM 4096
#define FLINT_KV_DIM 512
#define FLINT_QKV_DIM 5120 /* one raw q|k|v row: q 0..4095, k 4096..4607, v 4608..5119 */
#define FLINT_N_SWA 513    /* SWA window, current token included */
#define FLINT_SWA_RING 1024
#define FLINT_MAX_SLOTS (1 << 23) /* slots per layer and kv head */

/* KV cache element types. */
#define FLINT_KV_F16 1
#define FLINT_KV_BF16 2

/*
 * One attention layer's device state: its KV cache and its attention weights.
 * Mirrors the per-layer binding of the reference engine (Layer.k_cache/v_cache/
 * n_slots, q_norm, k_norm, sinks: /root/reference/src/engine.mm:63-70) plus the
 * per-layer hyper-parameters the CPU reference reads from the GGUF
 * (is_swa, has_rope, n_swa, rope_theta, rms_eps: /root/reference/src/ref/ref_model.h:13-19).
 * is_swa and has_rope are independent flags.
 */
typedef struct {
    void *k_cache;        /* device, layout above (tiled K) */
    void *v_cache;        /* device, layout above (element (h, slot, d) at ((h*n_slots/32 + slot/32)*128 + d)*32 + slot%32) */
    int32_t n_slots;      /* multiple of 32, at most FLINT_MAX_SLOTS; SWA: power of two >= window */
    int32_t kv_dtype;     /* FLINT_KV_F16 or FLINT_KV_BF16 */
    int32_t is_swa;
    int32_t has_rope;
    int32_t window;       /* FLINT_N_SWA */
    float rope_theta;
    float rms_eps;
    const float *q_norm;  /* device [128] */
    const float *k_norm;  /* device [128] */
    const float *sinks;   /* device [32] */
} flint_attn_layer;

/*
 * Fused single-token decode attention of one layer (replaces the k_attn_dec +
 * k_attn_combine dispatch at /root/reference/src/engine.mm:735-766, kernels at
 * /root/reference/src/metal/fused.metal:254-350).
 *   qkv: device [5120] raw q|k|v of the token at `pos` (before norm/rope)
 *   att: device [4096] output
 * Keys [k_begin, pos) come from the cache (k_begin = is_swa ? max(0, pos-window+1) : 0);
 * the current token's K/V (normed, roped, rounded to kv_dtype) is used and
 * written to slot(pos). keys_per_split: multiple of 32, or 0 for the built-in
 * plan. The split workspace is allocated by the library on first use.
 */
int32_t flint_attn_decode(const flint_attn_layer *layer, const float *qkv, float *att, int32_t pos,
                          int32_t keys_per_split, void *stream, char *err, int32_t err_len);

/*
 * Decode one token for each of n_seq independent sequences of one layer in a
 * single launch (no counterpart in the reference, which serves one session;
 * it is the reference's decode stage, engine.mm:735-766, batched over
 * sequences). Sequence s uses the caches at layer->k_cache/v_cache +
 * s * seq_stride elements, qkv row s, att row s and position pos[s] (host array).
 */
int32_t flint_attn_decode_batch(const flint_attn_layer *layer, int32_t n_seq, int64_t seq_stride,
                                const float *qkv, float *att, const int32_t *pos, int32_t keys_per_split,
                                void *stream, char *err, int32_t err_len);

/*
 * flint_attn_decode_batch for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in
 * the reference. It takes the same arguments and launches the same kernels, and allocates
 * nothing: the key-split partials live in a static 4 MiB device array of the library, one
 * per GPU, held until the process ends. That holds 248 key splits, counted over the batch's
 * sequences that take more than one (the built-in plan uses about 48 over all sequences; a
 * sequence of one split needs no partials); a plan that needs more is rejected with an error
 * before any launch. Every call on a GPU shares that
 * GPU's array, so calls that overlap on one GPU (on two streams, or from two threads) race.
 */
int32_t flint_attn_decode_batch_noalloc(const flint_attn_layer *layer, int32_t n_seq, int64_t seq_stride,
                                        const float *qkv, float *att, const int32_t *pos, int32_t keys_per_split,
                                        void *stream, char *err, int32_t err_len);

/*
 * Batched prefill attention of one layer for T tokens at positions p0..p0+T-1
 * (replaces k_qk_prefill + k_attn_prefill, /root/reference/src/metal/prefill.metal:99-266,
 * dispatched per chunk at /root/reference/src/engine.mm:1087-1104).
 *   qkv: device [T] rows of q_stride floats (raw q|k|v at the row start)
 *   att: device [T][4096] output
 * Writes the tokens' K/V into the cache (SWA: the last n_slots positions into
 * the ring). Any T in one call; the reference's 512-token chunking is not needed.
 */
int32_t flint_attn_prefill(const flint_attn_layer *layer, const float *qkv, int32_t q_stride, int32_t p0,
                           int32_t T, float *att, void *stream, char *err, int32_t err_len);

/* Blocks until the device is idle; 0 / -1. */
int32_t flint_attn_sync(char *err, int32_t err_len);

/*
 * Engine-level attention state: the KV caches and weights of every layer,
 * allocated in HBM at creation (the reference's bind_layers + alloc_activations,
 * /root/reference/src/engine.mm:472-527). Layer il is SWA if is_swa[il] != 0
 * (ring of FLINT_SWA_RING slots), else full (n_ctx slots, rounded up to 32).
 */
typedef struct flint_attn_engine flint_attn_engine;

flint_attn_engine *flint_attn_engine_create(int32_t n_layer, const uint8_t *is_swa, const uint8_t *has_rope,
                                            int32_t n_ctx, int32_t kv_dtype, float rope_theta, char *err,
                                            int32_t err_len);
void flint_attn_engine_destroy(flint_attn_engine *e);
int32_t flint_attn_engine_n_layer(const flint_attn_engine *e);
/* Copy one layer's q_norm[128], k_norm[128], sinks[32] (host pointers) into HBM. */
int32_t flint_attn_engine_set_weights(flint_attn_engine *e, int32_t il, const float *q_norm, const float *k_norm,
                                      const float *sinks, char *err, int32_t err_len);
/* The layer descriptor (device pointers owned by the engine), or NULL. */
const flint_attn_layer *flint_attn_engine_layer(const flint_attn_engine *e, int32_t il);
/* Decode / prefill stage of layer il on device buffers (engine.mm:735-766, 1087-1104). */
int32_t flint_attn_engine_decode(flint_attn_engine *e, int32_t il, const float *qkv, float *att, int32_t pos,
                                 void *stream, char *err, int32_t err_len);
int32_t flint_attn_engine_prefill(flint_attn_engine *e, int32_t il, const float *qkv, int32_t p0, int32_t T,
                                  float *att, void *stream, char *err, int32_t err_len);
/*
 * Test entry mirroring Engine::debug_attn (/root/reference/src/engine.h:40,
 * engine.mm:1308-1348): host qkv [n_tok][5120] raw projections, prefilled from
 * position 0 in chunks of `chunk` tokens; host out [n_tok][4096].
 */
int32_t flint_attn_engine_debug_attn(flint_attn_engine *e, int32_t il, const float *qkv, int32_t n_tok,
                                     int32_t chunk, float *out, char *err, int32_t err_len);

#ifdef __cplusplus
}
#endif
#endif
