/*
 * CPU oracle for the flint attention hot path. TEST INFRASTRUCTURE ONLY: see
 * flint_oracle.h for who may use it, which reference lines each function
 * restates, and which checks pin each function.
 *
 * Built with plain gcc -O2 and no -march flags, so float expressions are not
 * contracted into FMAs; the order of float and double operations below follows
 * /root/reference/src/ref/ref_model.cpp line by line so that results with fp32
 * storage are bit-identical to the reference's own CPU forward.
 */
#include "flint_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---- storage rounding (IEEE binary16 / bfloat16, round to nearest even) ---- */

static float round_f16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    const uint32_t sign = u & 0x80000000u, a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) return x; /* inf, nan */
    const int e = (int)(a >> 23) - 127;
    uint32_t r;
    if (e >= -14) {
        /* normal binary16: keep 10 fraction bits, drop 13 with RNE */
        r = a + 0x0fffu + ((a >> 13) & 1u);
        r &= ~0x1fffu;
        if (r >= 0x47800000u) r = 0x7f800000u; /* >= 65536 after rounding: overflow */
    } else if (e >= -25) {
        /* subnormal binary16: multiples of 2^-24 */
        const int shift = 13 + (-14 - e); /* 14..24 */
        const uint32_t m = (a & 0x7fffffu) | 0x800000u;
        const uint32_t half = 1u << (shift - 1), mask = (1u << shift) - 1u;
        uint32_t q = m >> shift;
        const uint32_t rem = m & mask;
        if (rem > half || (rem == half && (q & 1u))) q++;
        float v = ldexpf((float)q, -24);
        memcpy(&r, &v, 4);
    } else {
        r = 0;
    }
    r |= sign;
    float out;
    memcpy(&out, &r, 4);
    return out;
}

static float round_bf16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return x; /* nan */
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
    float out;
    memcpy(&out, &u, 4);
    return out;
}

float fo_round(float x, int store) {
    if (store == FO_STORE_F16) return round_f16(x);
    if (store == FO_STORE_BF16) return round_bf16(x);
    return x;
}

void fo_round_array(float *x, long n, int store) {
    for (long i = 0; i < n; i++) x[i] = fo_round(x[i], store);
}

/* ---- norm / rope: ref_model.cpp:45-61 ---- */

void fo_rmsnorm(const float *x, const float *w, float *y, int n, float eps) {
    double ss = 0;
    for (int i = 0; i < n; i++) ss += (double)x[i] * x[i];
    const float scale = 1.0f / sqrtf((float)(ss / n) + eps);
    for (int i = 0; i < n; i++) y[i] = x[i] * scale * w[i];
}

void fo_rope_neox(float *x, int d, int pos, float theta) {
    for (int i = 0; i < d / 2; i++) {
        const float freq = powf(theta, -2.0f * i / d);
        const float a = pos * freq, c = cosf(a), s = sinf(a);
        const float x0 = x[i], x1 = x[i + d / 2];
        x[i] = x0 * c - x1 * s;
        x[i + d / 2] = x0 * s + x1 * c;
    }
}

/* ---- ring / window: flint_config.h:25,29-31; fused.metal:265,269; prefill.metal:106 ---- */

int fo_slot(int pos, int is_swa, int n_slots) { return is_swa ? (pos & (n_slots - 1)) : pos; }

int fo_first_key(int pos, int is_swa, int window) {
    if (!is_swa) return 0;
    return pos - (window - 1) > 0 ? pos - (window - 1) : 0;
}

/* ---- q/k/v of one token: ref_model.cpp:110-124 ---- */

void fo_qkv_prep(const fo_layer *L, const float *qkv, int pos, float *q, float *k, float *v) {
    const int D = FO_HEAD_DIM;
    memcpy(q, qkv, sizeof(float) * FO_Q_DIM);
    memcpy(k, qkv + FO_Q_DIM, sizeof(float) * FO_KV_DIM);
    memcpy(v, qkv + FO_Q_DIM + FO_KV_DIM, sizeof(float) * FO_KV_DIM);
    for (int hh = 0; hh < FO_N_HEAD; hh++) {
        fo_rmsnorm(&q[hh * D], L->q_norm, &q[hh * D], D, L->rms_eps);
        if (L->has_rope) fo_rope_neox(&q[hh * D], D, pos, L->rope_theta);
    }
    for (int hh = 0; hh < FO_N_HEAD_KV; hh++) {
        fo_rmsnorm(&k[hh * D], L->k_norm, &k[hh * D], D, L->rms_eps);
        if (L->has_rope) fo_rope_neox(&k[hh * D], D, pos, L->rope_theta);
    }
    fo_round_array(k, FO_KV_DIM, L->store);
    fo_round_array(v, FO_KV_DIM, L->store);
}

/* ---- sink softmax over the window: ref_model.cpp:126-148 ---- */

static void attend_heads(const fo_layer *L, const float *q, const float *K, const float *V, int pos,
                         float *att, int h0, int h1) {
    const int D = FO_HEAD_DIM, kv_dim = FO_KV_DIM, group = FO_GQA;
    const int first = fo_first_key(pos, L->is_swa, L->window);
    const float scale = 1.0f / sqrtf((float)D);
    float *s = (float *)malloc(sizeof(float) * (size_t)(pos + 1));
    double acc[FO_HEAD_DIM];
    for (int hh = h0; hh < h1; hh++) {
        const int kvh = hh / group;
        float m = L->sinks[hh];
        for (int j = first; j <= pos; j++) {
            const float *kj = &K[(size_t)j * kv_dim + kvh * D];
            float d = 0;
            for (int i = 0; i < D; i++) d += q[hh * D + i] * kj[i];
            s[j] = d * scale;
            m = m > s[j] ? m : s[j];
        }
        double denom = expf(L->sinks[hh] - m);
        for (int i = 0; i < D; i++) acc[i] = 0.0;
        for (int j = first; j <= pos; j++) {
            const double p = expf(s[j] - m);
            denom += p;
            const float *vj = &V[(size_t)j * kv_dim + kvh * D];
            for (int i = 0; i < D; i++) acc[i] += p * vj[i];
        }
        for (int i = 0; i < D; i++) att[hh * D + i] = (float)(acc[i] / denom);
    }
    free(s);
}

typedef struct {
    const fo_layer *L;
    const float *q, *K, *V;
    int pos, h0, h1;
    float *att;
} attend_job;

static void *attend_thread(void *p) {
    attend_job *j = (attend_job *)p;
    attend_heads(j->L, j->q, j->K, j->V, j->pos, j->att, j->h0, j->h1);
    return NULL;
}

void fo_attend(const fo_layer *L, const float *q, const float *K, const float *V, int pos, float *att,
               int n_threads) {
    if (n_threads <= 1) {
        attend_heads(L, q, K, V, pos, att, 0, FO_N_HEAD);
        return;
    }
    if (n_threads > FO_N_HEAD) n_threads = FO_N_HEAD;
    pthread_t th[FO_N_HEAD];
    attend_job jobs[FO_N_HEAD];
    const int per = (FO_N_HEAD + n_threads - 1) / n_threads;
    int n = 0;
    for (int t = 0; t < n_threads; t++) {
        const int h0 = t * per, h1 = h0 + per < FO_N_HEAD ? h0 + per : FO_N_HEAD;
        if (h0 >= h1) break;
        jobs[n] = (attend_job){L, q, K, V, pos, h0, h1, att};
        if (pthread_create(&th[n], NULL, attend_thread, &jobs[n]) != 0) {
            attend_heads(L, q, K, V, pos, att, h0, h1);
            continue;
        }
        n++;
    }
    for (int t = 0; t < n; t++) pthread_join(th[t], NULL);
}

/* ---- split-K formulation and LSE merge: fused.metal:266-283 (per split), 331-350 (merge) ---- */

void fo_attend_split(const fo_layer *L, const float *q, const float *K, const float *V, int pos,
                     int n_split, float *att) {
    const int D = FO_HEAD_DIM, kv_dim = FO_KV_DIM;
    const int first = fo_first_key(pos, L->is_swa, L->window);
    const int n_keys = pos + 1 - first;
    const float scale = 1.0f / sqrtf((float)D);
    if (n_split < 1) n_split = 1;
    const int kps = (n_keys + n_split - 1) / n_split;
    float *ms = (float *)malloc(sizeof(float) * n_split);
    double *ls = (double *)malloc(sizeof(double) * n_split);
    double *accs = (double *)malloc(sizeof(double) * n_split * D);
    for (int hh = 0; hh < FO_N_HEAD; hh++) {
        const int kvh = hh / FO_GQA;
        for (int sp = 0; sp < n_split; sp++) {
            const int j0 = first + sp * kps;
            int j1 = j0 + kps;
            if (j1 > pos + 1) j1 = pos + 1;
            float m = -INFINITY;
            for (int j = j0; j < j1; j++) {
                const float *kj = &K[(size_t)j * kv_dim + kvh * D];
                float d = 0;
                for (int i = 0; i < D; i++) d += q[hh * D + i] * kj[i];
                const float sj = d * scale;
                m = m > sj ? m : sj;
            }
            double l = 0;
            double *acc = &accs[(size_t)sp * D];
            for (int i = 0; i < D; i++) acc[i] = 0;
            for (int j = j0; j < j1; j++) {
                const float *kj = &K[(size_t)j * kv_dim + kvh * D];
                float d = 0;
                for (int i = 0; i < D; i++) d += q[hh * D + i] * kj[i];
                const double p = exp((double)(d * scale) - m);
                l += p;
                const float *vj = &V[(size_t)j * kv_dim + kvh * D];
                for (int i = 0; i < D; i++) acc[i] += p * vj[i];
            }
            ms[sp] = m;
            ls[sp] = l;
        }
        const float sink = L->sinks[hh];
        float M = sink;
        for (int sp = 0; sp < n_split; sp++)
            if (ls[sp] != 0 && ms[sp] > M) M = ms[sp];
        double Ltot = exp((double)sink - M);
        double out[FO_HEAD_DIM] = {0};
        for (int sp = 0; sp < n_split; sp++) {
            if (ls[sp] == 0) continue; /* empty split, fused.metal:343 */
            const double c = exp((double)ms[sp] - M);
            Ltot += ls[sp] * c;
            for (int i = 0; i < D; i++) out[i] += accs[(size_t)sp * D + i] * c;
        }
        for (int i = 0; i < D; i++) att[hh * D + i] = (float)(out[i] / Ltot);
    }
    free(ms);
    free(ls);
    free(accs);
}

/* ---- decode step / prefill: ref_model.cpp:95-149 (attention block of forward) ---- */

void fo_decode_step(const fo_layer *L, const float *qkv, int pos, float *K, float *V, float *att,
                    int n_threads) {
    float q[FO_Q_DIM];
    fo_qkv_prep(L, qkv, pos, q, &K[(size_t)pos * FO_KV_DIM], &V[(size_t)pos * FO_KV_DIM]);
    fo_attend(L, q, K, V, pos, att, n_threads);
}

void fo_prefill(const fo_layer *L, const float *qkv, int q_stride, int p0, int T, float *K, float *V,
                float *att, int n_threads) {
    for (int t = 0; t < T; t++)
        fo_decode_step(L, qkv + (size_t)t * q_stride, p0 + t, K, V, att + (size_t)t * FO_Q_DIM, n_threads);
}

/* ---- the same prefill on many threads (the CPU baseline): every token's q/k/v first, in
 * position order as fo_prefill writes them, then the attention of rows [r0, r1), each
 * (row, head) pair on one of n_threads threads (interleaved). attend_heads per head is
 * fo_prefill's own, so every row written equals fo_prefill's bit for bit. ---- */

typedef struct {
    const fo_layer *L;
    const float *qkv;
    float *Q, *K, *V;
    int q_stride, p0, T, r0, r1, tid, nth;
    float *att;
} prefill_job;

static void *prep_thread(void *p) {
    prefill_job *j = (prefill_job *)p;
    for (int t = j->tid; t < j->T; t += j->nth)
        fo_qkv_prep(j->L, j->qkv + (size_t)t * j->q_stride, j->p0 + t, j->Q + (size_t)t * FO_Q_DIM,
                    &j->K[(size_t)(j->p0 + t) * FO_KV_DIM], &j->V[(size_t)(j->p0 + t) * FO_KV_DIM]);
    return NULL;
}

static void *prefill_thread(void *p) {
    prefill_job *j = (prefill_job *)p;
    const long n_pairs = (long)(j->r1 - j->r0) * FO_N_HEAD;
    for (long i = j->tid; i < n_pairs; i += j->nth) {
        const int row = j->r0 + (int)(i / FO_N_HEAD), hh = (int)(i % FO_N_HEAD);
        attend_heads(j->L, j->Q + (size_t)row * FO_Q_DIM, j->K, j->V, j->p0 + row, j->att + (size_t)row * FO_Q_DIM,
                     hh, hh + 1);
    }
    return NULL;
}

int fo_prefill_mt(const fo_layer *L, const float *qkv, int q_stride, int p0, int T, int r0, int r1, float *K,
                  float *V, float *att, int n_threads) {
    enum { MAXT = 512 };
    if (r0 < 0 || r1 > T || r0 > r1) return -1;
    float *Q = (float *)malloc(sizeof(float) * (size_t)T * FO_Q_DIM);
    if (!Q) return -1;
    if (n_threads < 1) n_threads = 1;
    if (n_threads > MAXT) n_threads = MAXT;
    pthread_t th[MAXT];
    prefill_job jobs[MAXT];
    /* two phases: every token's q/k/v (tokens interleaved over the threads; each writes its own
     * K, V rows), then the (row, head) pairs */
    for (int phase = 0; phase < 2; phase++) {
        void *(*fn)(void *) = phase == 0 ? prep_thread : prefill_thread;
        int n = 0;
        for (int t = 0; t < n_threads; t++) {
            jobs[t] = (prefill_job){L, qkv, Q, K, V, q_stride, p0, T, r0, r1, t, n_threads, att};
            if (pthread_create(&th[n], NULL, fn, &jobs[t]) != 0) {
                fn(&jobs[t]);
                continue;
            }
            n++;
        }
        for (int t = 0; t < n; t++) pthread_join(th[t], NULL);
    }
    free(Q);
    return 0;
}

/* ---- weight formats of the attention projections ----
 * Restated from ggml's published block formats and dequantisation (the reference
 * vendors them: /root/reference/third_party/ggml/ggml-common.h block_q8_0 :251-256,
 * block_q5_K :343-356, block_q6_K :362-368, block_iq4_xs :454-460, kvalues_iq4nl
 * :1120-1122; dequantize_row_* in /root/reference/src/ref/dequant_gen.c:10-24, 50-106,
 * 209-230), with each float operation in the reference's order and no contraction, so
 * the values are bit-identical. Row dispatch as /root/reference/src/ref/dequant_row.cpp:19-43. */

static float half_bits_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const int exp = (h >> 10) & 0x1f;
    uint32_t mant = h & 0x3ff, bits;
    if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (mant << 13); /* inf / nan */
    } else if (exp != 0) {
        bits = sign | ((uint32_t)(exp - 15 + 127) << 23) | (mant << 13);
    } else if (mant == 0) {
        bits = sign;
    } else { /* subnormal: mant * 2^-24, exact in float */
        int e = -14;
        while (!(mant & 0x400)) {
            mant <<= 1;
            e--;
        }
        bits = sign | ((uint32_t)(e + 127) << 23) | ((mant & 0x3ff) << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static uint16_t rd16(const unsigned char *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

static const signed char iq4nl_values[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                             1,    13,   25,  38,  53,  69,  89,  113};

long fo_block_elems(int type) {
    switch (type) {
        case FO_W_F32: case FO_W_F16: case FO_W_BF16: return 1;
        case FO_W_Q8_0: return 32;
        case FO_W_Q5_K: case FO_W_Q6_K: case FO_W_IQ4_XS: return 256;
        default: return -1;
    }
}

long fo_block_bytes(int type) {
    switch (type) {
        case FO_W_F32: return 4;
        case FO_W_F16: case FO_W_BF16: return 2;
        case FO_W_Q8_0: return 34;
        case FO_W_Q5_K: return 176;
        case FO_W_Q6_K: return 210;
        case FO_W_IQ4_XS: return 136;
        default: return -1;
    }
}

long fo_row_bytes(int type, long k) {
    const long be = fo_block_elems(type);
    if (be <= 0 || k <= 0 || k % be) return -1;
    return k / be * fo_block_bytes(type);
}

/* the 6-bit scale and min of sub-block j (0..7) of a K-quant super-block's 12 scale bytes */
static void kquant_scale_min(const unsigned char *s, int j, int *sc, int *m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 0xf) | ((s[j - 4] >> 6) << 4);
        *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

int fo_dequant_row(int type, const void *row_, long k, float *y) {
    const unsigned char *row = (const unsigned char *)row_;
    if (fo_row_bytes(type, k) < 0) return -1;
    switch (type) {
        case FO_W_F32: memcpy(y, row, (size_t)k * 4); return 0;
        case FO_W_F16:
            for (long i = 0; i < k; i++) y[i] = half_bits_to_float(rd16(row + 2 * i));
            return 0;
        case FO_W_BF16:
            for (long i = 0; i < k; i++) {
                const uint32_t u = (uint32_t)rd16(row + 2 * i) << 16;
                memcpy(&y[i], &u, 4);
            }
            return 0;
        case FO_W_Q8_0: /* y = q * d */
            for (long b = 0; b < k / 32; b++) {
                const unsigned char *blk = row + 34 * b;
                const float d = half_bits_to_float(rd16(blk));
                for (int i = 0; i < 32; i++) y[32 * b + i] = (float)(signed char)blk[2 + i] * d;
            }
            return 0;
        case FO_W_Q5_K: /* 8 sub-blocks of 32: y = (d * sc) * q5 - dmin * m */
            for (long b = 0; b < k / 256; b++) {
                const unsigned char *blk = row + 176 * b;
                const float d = half_bits_to_float(rd16(blk)), dmin = half_bits_to_float(rd16(blk + 2));
                const unsigned char *sc = blk + 4, *qh = blk + 16, *qs = blk + 48;
                for (int j = 0; j < 8; j++) {
                    int s, m;
                    kquant_scale_min(sc, j, &s, &m);
                    const float d1 = d * (float)s, m1 = dmin * (float)m;
                    const unsigned char *ql = qs + 32 * (j / 2);
                    for (int i = 0; i < 32; i++) {
                        const int q = ((j & 1) ? ql[i] >> 4 : ql[i] & 0xf) + (((qh[i] >> j) & 1) ? 16 : 0);
                        const float dq = d1 * (float)q;
                        y[256 * b + 32 * j + i] = dq - m1;
                    }
                }
            }
            return 0;
        case FO_W_Q6_K: /* 16 sub-blocks of 16: y = (d * sc) * (q6 - 32) */
            for (long b = 0; b < k / 256; b++) {
                const unsigned char *blk = row + 210 * b;
                const unsigned char *ql = blk, *qh = blk + 128;
                const signed char *sc = (const signed char *)(blk + 192);
                const float d = half_bits_to_float(rd16(blk + 208));
                for (int e = 0; e < 256; e++) {
                    const int n = e / 128, g = (e % 128) / 32, l = e % 32;
                    const unsigned char lo = ql[64 * n + l + 32 * (g & 1)];
                    const int q = (((g < 2) ? lo & 0xf : lo >> 4) | (((qh[32 * n + l] >> (2 * g)) & 3) << 4)) - 32;
                    const float ds = d * (float)sc[8 * n + l / 16 + 2 * g];
                    y[256 * b + e] = ds * (float)q;
                }
            }
            return 0;
        case FO_W_IQ4_XS: /* 8 sub-blocks of 32: y = (d * (ls - 32)) * table[nibble] */
            for (long b = 0; b < k / 256; b++) {
                const unsigned char *blk = row + 136 * b;
                const float d = half_bits_to_float(rd16(blk));
                const uint16_t sh = rd16(blk + 2);
                const unsigned char *sl = blk + 4, *qs = blk + 8;
                for (int ib = 0; ib < 8; ib++) {
                    const int ls = ((sl[ib / 2] >> (4 * (ib % 2))) & 0xf) | (((sh >> (2 * ib)) & 3) << 4);
                    const float dl = d * (float)(ls - 32);
                    for (int j = 0; j < 16; j++) {
                        y[256 * b + 32 * ib + j] = dl * (float)iq4nl_values[qs[16 * ib + j] & 0xf];
                        y[256 * b + 32 * ib + j + 16] = dl * (float)iq4nl_values[qs[16 * ib + j] >> 4];
                    }
                }
            }
            return 0;
    }
    return -1;
}

/* y[r] = sum_i W[r][i] * x[i] with a double accumulator over the dequantised row
 * (RefModel::matvec, /root/reference/src/ref/ref_model.cpp:74-93) */
int fo_matvec(int type, const void *w, long k, long n_rows, const float *x, float *y) {
    const long rb = fo_row_bytes(type, k);
    if (rb < 0) return -1;
    float *row = (float *)malloc((size_t)k * sizeof(float));
    if (!row) return -1;
    for (long r = 0; r < n_rows; r++) {
        fo_dequant_row(type, (const unsigned char *)w + r * rb, k, row);
        double acc = 0;
        for (long i = 0; i < k; i++) acc += (double)row[i] * x[i];
        y[r] = (float)acc;
    }
    free(row);
    return 0;
}

/* RefModel::matvec (ref_model.cpp:74-93) over dequantised rows: per row, acc += (double)w * x
 * in index order, then rounded to float; rows are independent, so threads change nothing. */
typedef struct {
    const float *w, *x;
    float *y;
    long k, r0, r1;
} mv_job;

static void *mv_thread(void *arg) {
    const mv_job *j = (const mv_job *)arg;
    for (long r = j->r0; r < j->r1; r++) {
        const float *row = j->w + r * j->k;
        double acc = 0;
        for (long i = 0; i < j->k; i++) acc += (double)row[i] * j->x[i];
        j->y[r] = (float)acc;
    }
    return NULL;
}

void fo_matvec_f32(const float *w, long k, long n_rows, const float *x, float *y, int n_threads) {
    enum { MAXT = 64 };
    if (n_threads < 1) n_threads = 1;
    if (n_threads > MAXT) n_threads = MAXT;
    mv_job jobs[MAXT];
    pthread_t th[MAXT];
    const long chunk = (n_rows + n_threads - 1) / n_threads;
    int n = 0;
    for (int t = 0; t < n_threads; t++) {
        const long r0 = t * chunk, r1 = r0 + chunk < n_rows ? r0 + chunk : n_rows;
        if (r0 >= r1) break;
        jobs[n] = (mv_job){w, x, y, k, r0, r1};
        if (pthread_create(&th[n], NULL, mv_thread, &jobs[n]) != 0) {
            mv_thread(&jobs[n]);
            continue;
        }
        n++;
    }
    for (int t = 0; t < n; t++) pthread_join(th[t], NULL);
}
