/*
 * CPU oracle for the flint attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or as the timed CPU baseline). The product path (libflint_attn.so) never
 * links, loads or calls it.
 *
 * It restates the reference's fp32 CPU attention, keeping its order of float
 * and double operations so that, with fp32 KV storage, results are bit-identical
 * to the reference's RefModel::forward (checked by tests/test_ref_parity.py
 * against oracle/_ref, which is compiled from the reference sources):
 *   rmsnorm            /root/reference/src/ref/ref_model.cpp:45-50
 *   rope_neox          /root/reference/src/ref/ref_model.cpp:53-61
 *   per-head q/k prep  /root/reference/src/ref/ref_model.cpp:110-121
 *   sink softmax       /root/reference/src/ref/ref_model.cpp:126-148
 * plus the GPU-path behaviour the reference's own attention test applies:
 *   K/V rounded through the cache dtype    /root/reference/src/main.mm:268-277
 *   current token's K/V rounded before use /root/reference/src/metal/fused.metal:285-289
 *   split-K partials + LSE merge           /root/reference/src/metal/fused.metal:319-350
 *   SWA window / ring slot                 /root/reference/src/metal/flint_config.h:25,29-31
 *
 * Parity pinning (what checks each function; in tests/test_oracle.py, tests/test_ref_parity.py,
 * tests/test_weights.py and tests/test_model.py):
 *   fo_round            numpy float16 / torch bfloat16 casts, bit-exact, all finite inputs of a sweep
 *   fo_rmsnorm          closed form for constant vectors; reference RefModel (bit-exact)
 *   fo_rope_neox        pos 0 identity, pair-norm preservation, relative-position invariance
 *                       of <rope(q,m), rope(k,n)>; reference RefModel (bit-exact)
 *   fo_attend           one key + sink closed form, n identical keys, sink -> -inf equals plain
 *                       softmax (scipy), sink -> +inf gives 0, SWA window brute force;
 *                       reference RefModel (bit-exact, fp32 storage)
 *   fo_attend_split     equals fo_attend for n_split in {1, 2, 16, 32, 64}
 *   fo_slot/fo_first_key brute force over pos in [0, 4096) against a linear history
 *   fo_dequant_row      bit-exact against ggml's dequantize_row_* compiled from the reference's
 *                       vendored sources (oracle/_ref) on random blocks, and against the
 *                       committed fixtures tests/golden/weight_rows.npz made from it; f16/bf16
 *                       against numpy / bit shifts; closed forms (all-zero scales give 0,
 *                       q8_0 with d = 1 gives the int8 values)
 *   fo_matvec           one-hot rows select x exactly; equals a float64 numpy product of
 *                       fo_dequant_row's rows; linearity in x
 *   fo_matvec_f32       with oracle.py's block forward (rmsnorm, q/k/v and o matvecs over
 *                       dequantised rows, the attention above, the residual add): the hidden
 *                       states of a two-layer quantised model with zero FFN weights equal the
 *                       reference's RefModel::forward bit for bit (tests/test_model.py against
 *                       tests/golden/block_vectors.json, written from oracle/_ref); a zero
 *                       o-projection leaves x unchanged; position 0 matches the one-key closed form
 */
#ifndef FLINT_ORACLE_H
#define FLINT_ORACLE_H

#ifdef __cplusplus
extern "C" {
#endif

enum { FO_N_HEAD = 32, FO_N_HEAD_KV = 4, FO_HEAD_DIM = 128, FO_GQA = 8 };
enum { FO_Q_DIM = 4096, FO_KV_DIM = 512, FO_QKV_DIM = 5120 };
enum { FO_STORE_F32 = 0, FO_STORE_F16 = 1, FO_STORE_BF16 = 2 };

typedef struct {
    int is_swa;       /* sliding-window layer: keys [max(0, pos-window+1), pos] */
    int has_rope;     /* NEOX RoPE on q and k (independent of is_swa) */
    int window;       /* 513 for Flint */
    int store;        /* FO_STORE_*: dtype the KV cache holds */
    float rope_theta;
    float rms_eps;
    const float *q_norm; /* [128] shared by all q heads */
    const float *k_norm; /* [128] shared by all kv heads */
    const float *sinks;  /* [32] one logit per q head */
} fo_layer;

float fo_round(float x, int store);
void fo_round_array(float *x, long n, int store);

void fo_rmsnorm(const float *x, const float *w, float *y, int n, float eps);
void fo_rope_neox(float *x, int d, int pos, float theta);

int fo_slot(int pos, int is_swa, int n_slots);
int fo_first_key(int pos, int is_swa, int window);

/* q [32][128], k [4][128], v [4][128] for one token from its raw qkv row [5120].
 * k and v are rounded through the storage dtype (what the cache will hold). */
void fo_qkv_prep(const fo_layer *L, const float *qkv, int pos, float *q, float *k, float *v);

/* Attention output att [32][128] for the query q at position pos over the
 * linear history K, V [pos+1][512] (row j = what the cache holds for position j). */
void fo_attend(const fo_layer *L, const float *q, const float *K, const float *V, int pos, float *att,
               int n_threads);

/* Same result through n_split key splits (float max, double partial sums) and
 * the log-sum-exp merge with the sink. */
void fo_attend_split(const fo_layer *L, const float *q, const float *K, const float *V, int pos,
                     int n_split, float *att);

/* One decode step: prep the token at pos, write its K/V into history row pos,
 * attend. K, V must hold rows 0..pos-1 already. */
void fo_decode_step(const fo_layer *L, const float *qkv, int pos, float *K, float *V, float *att,
                    int n_threads);

/* Prefill of T tokens at positions p0..p0+T-1 (qkv rows q_stride floats apart);
 * identical to T decode steps. att is [T][4096]. */
void fo_prefill(const fo_layer *L, const float *qkv, int q_stride, int p0, int T, float *K, float *V,
                float *att, int n_threads);

/* The same prefill with its attention spread over n_threads threads: every token's
 * q/k/v (K, V rows p0 .. p0+T-1 written), then att rows [r0, r1) of the T, one (row, head)
 * pair per job. The rows written equal fo_prefill's bit for bit (the same per-head code);
 * the CPU baseline times it on a sample of rows. 0 / -1 (bad row range, no memory). */
int fo_prefill_mt(const fo_layer *L, const float *qkv, int q_stride, int p0, int T, int r0, int r1, float *K,
                  float *V, float *att, int n_threads);

/* Weight formats of the attention projections: ggml type ids
 * (/root/reference/src/gguf.h:14-19). fo_row_bytes is -1 for an unsupported type or
 * a k that is not a whole number of blocks. */
enum { FO_W_F32 = 0, FO_W_F16 = 1, FO_W_Q8_0 = 8, FO_W_Q5_K = 13, FO_W_Q6_K = 14, FO_W_IQ4_XS = 23, FO_W_BF16 = 30 };
long fo_block_elems(int type);
long fo_block_bytes(int type);
long fo_row_bytes(int type, long k);
/* One row of k elements to fp32 (0 / -1), bit-identical to ggml's dequantize_row_*. */
int fo_dequant_row(int type, const void *row, long k, float *out);
/* y = W x over n_rows rows, double accumulation per row (0 / -1). */
int fo_matvec(int type, const void *w, long k, long n_rows, const float *x, float *y);
/* The same product for rows already dequantised to fp32 (w [n_rows][k]), rows split over
 * n_threads threads; each row's sum runs in the same order as fo_matvec's, so the result
 * is bit-identical. RefModel::matvec, /root/reference/src/ref/ref_model.cpp:74-93. */
void fo_matvec_f32(const float *w, long k, long n_rows, const float *x, float *y, int n_threads);

#ifdef __cplusplus
}
#endif
#endif
