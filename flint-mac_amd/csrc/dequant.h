// GGUF weight formats of the attention projections: ggml's block layouts
// (/root/reference/third_party/ggml/ggml-common.h), type ids from /root/reference/src/gguf.h:14-19.
// deq32 decodes one 32-element sub-block, the unit every format shares (a q8_0 block, a half of a
// q5_K/iq4_xs 64-element pair, two q6_K 16-element groups), repeating ggml's float operations in
// order with contraction off, so the result is bit-identical to dequantize_row_*
// (/root/reference/src/ref/dequant_gen.c). Shared by proj.hip (matvec, row dequantisation) and
// proj_gemm.hip (the batched projections' weight planes).
#pragma once

#include "common.h"
#include "flint_attn_internal.h"

namespace flint {

__host__ __device__ constexpr int w_block_elems(int t) {
    return t == W_F32 || t == W_F16 || t == W_BF16 ? 1 : t == W_Q8_0 ? 32
         : t == W_Q5_K || t == W_Q6_K || t == W_IQ4_XS ? 256 : 0;
}
__host__ __device__ constexpr int w_block_bytes(int t) {
    return t == W_F32 ? 4 : t == W_F16 || t == W_BF16 ? 2 : t == W_Q8_0 ? 34 : t == W_Q5_K ? 176
         : t == W_Q6_K ? 210 : t == W_IQ4_XS ? 136 : 0;
}

__device__ inline float h2f(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

// iq4_nl code book (ggml-common.h:1120-1122) as int8 bytes, four to a word
constexpr uint32_t IQ4_T0 = 0xbfad9881u, IQ4_T1 = 0xf6eaddcfu, IQ4_T2 = 0x26190d01u, IQ4_T3 = 0x71594535u;
__device__ inline float iq4_value(uint32_t nib) {
    const uint32_t sel = 0x0c0c0c00u | (nib & 7);  // byte nib&7 of the 8-byte half, upper bytes 0
    const uint32_t b = nib & 8 ? __builtin_amdgcn_perm(IQ4_T3, IQ4_T2, sel) : __builtin_amdgcn_perm(IQ4_T1, IQ4_T0, sel);
    return (float)(int8_t)b;
}

// byte i of a little-endian word array
template <int N>
__device__ inline uint32_t byte_of(const uint32_t (&w)[N], int i) { return (w[i >> 2] >> (8 * (i & 3))) & 0xff; }

// The 32 weights of sub-block sb of a row whose bytes start at `row` (LDS or global; for
// the quantised types the row start is 16-byte aligned). Float operations and their order
// follow ggml's dequantize_row_* (dequant_gen.c:10-24, 50-106, 209-230); no contraction.
__device__ inline void deq32(int type, const uint8_t *row, int sb, float (&w)[32]) {
#pragma clang fp contract(off)
    switch (type) {
        case W_Q8_0: {  // y = q * d
            const uint16_t *p = (const uint16_t *)(row + 34 * sb);
            const float d = h2f(p[0]);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const uint32_t v = p[1 + i];
                w[2 * i] = (float)(int8_t)(v & 0xff) * d;
                w[2 * i + 1] = (float)(int8_t)(v >> 8) * d;
            }
            break;
        }
        case W_Q5_K: {  // y = (d * sc) * (q4 + 16 h) - dmin * m
            const uint8_t *blk = row + 176 * (sb >> 3);
            const int j = sb & 7;
            const uint32_t dm = *(const uint32_t *)blk;
            const uint32_t s[3] = {((const uint32_t *)(blk + 4))[0], ((const uint32_t *)(blk + 4))[1],
                                   ((const uint32_t *)(blk + 4))[2]};
            // 6-bit scale and min of sub-block j (ggml's get_scale_min_k4, dequant_gen.c:1-8)
            const uint32_t sc = j < 4 ? byte_of(s, j) & 63 : (byte_of(s, j + 4) & 15) | ((byte_of(s, j - 4) >> 6) << 4);
            const uint32_t mn = j < 4 ? byte_of(s, j + 4) & 63 : (byte_of(s, j + 4) >> 4) | ((byte_of(s, j) >> 6) << 4);
            const float d1 = h2f(dm & 0xffff) * (float)sc, m1 = h2f(dm >> 16) * (float)mn;
            uint32_t qh[8], ql[8];
            *(u32x4 *)&qh[0] = ((const u32x4 *)(blk + 16))[0];
            *(u32x4 *)&qh[4] = ((const u32x4 *)(blk + 16))[1];
            *(u32x4 *)&ql[0] = ((const u32x4 *)(blk + 48 + 32 * (j >> 1)))[0];
            *(u32x4 *)&ql[4] = ((const u32x4 *)(blk + 48 + 32 * (j >> 1)))[1];
            const int ls = 4 * (j & 1);
#pragma unroll
            for (int i = 0; i < 32; i++) {
                const uint32_t q = ((byte_of(ql, i) >> ls) & 15) + (((byte_of(qh, i) >> j) & 1) << 4);
                const float dq = d1 * (float)q;
                w[i] = dq - m1;
            }
            break;
        }
        case W_Q6_K: {  // y = (d * sc) * (q6 - 32); the block is 2-byte aligned
            const uint8_t *blk = row + 210 * (sb >> 3);
            const int j = sb & 7, n = j >> 2, g = j & 3;
            const uint16_t *ql = (const uint16_t *)(blk + 64 * n + 32 * (g & 1));
            const uint16_t *qh = (const uint16_t *)(blk + 128 + 32 * n);
            const uint32_t scw = *(const uint16_t *)(blk + 192 + 8 * n + 2 * g);  // scales 8n+2g, 8n+2g+1
            const float d = h2f(*(const uint16_t *)(blk + 208));
            const float ds0 = d * (float)(int8_t)(scw & 0xff), ds1 = d * (float)(int8_t)(scw >> 8);
            const int lsh = 4 * (g >> 1), hsh = 2 * g;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const uint32_t lo = ql[i], hi = qh[i];
#pragma unroll
                for (int b = 0; b < 2; b++) {
                    const int e = 2 * i + b;
                    const int q = (int)((((lo >> (8 * b)) >> lsh) & 15) | ((((hi >> (8 * b)) >> hsh) & 3) << 4)) - 32;
                    w[e] = (e < 16 ? ds0 : ds1) * (float)q;
                }
            }
            break;
        }
        case W_IQ4_XS: {  // y = (d * (ls - 32)) * table[nibble]; the block is 8-byte aligned
            const uint8_t *blk = row + 136 * (sb >> 3);
            const int ib = sb & 7;
            const uint2 hdr = *(const uint2 *)blk;  // d | scales_h | scales_l[4]
            const uint32_t ls = ((hdr.y >> (8 * (ib >> 1) + 4 * (ib & 1))) & 15) | (((hdr.x >> (16 + 2 * ib)) & 3) << 4);
            const float dl = h2f(hdr.x & 0xffff) * (float)((int)ls - 32);
            const uint2 q0 = *(const uint2 *)(blk + 8 + 16 * ib), q1 = *(const uint2 *)(blk + 16 + 16 * ib);
            const uint32_t qs[4] = {q0.x, q0.y, q1.x, q1.y};
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const uint32_t v = byte_of(qs, i);
                w[i] = dl * iq4_value(v & 15);
                w[i + 16] = dl * iq4_value(v >> 4);
            }
            break;
        }
        case W_F16:
        case W_BF16: {
            uint32_t h[16];
#pragma unroll
            for (int k = 0; k < 4; k++) *(u32x4 *)&h[4 * k] = ((const u32x4 *)(row + 64 * sb))[k];
#pragma unroll
            for (int i = 0; i < 16; i++) {
                if (type == W_F16) {
                    w[2 * i] = h2f(h[i] & 0xffff);
                    w[2 * i + 1] = h2f(h[i] >> 16);
                } else {
                    w[2 * i] = __uint_as_float(h[i] << 16);
                    w[2 * i + 1] = __uint_as_float(h[i] & 0xffff0000u);
                }
            }
            break;
        }
        default: {  // W_F32
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const f32x4 v = ((const f32x4 *)(row + 128 * sb))[k];
                w[4 * k] = v[0];
                w[4 * k + 1] = v[1];
                w[4 * k + 2] = v[2];
                w[4 * k + 3] = v[3];
            }
        }
    }
}

// The integer form of sub-block sb (w_int_sub), for the batched projections: its 32 values v,
// the scales s of elements 0-15 (s[0]) and 16-31 (s[1]) and the min m (q5_K; else 0), computed
// in ggml's float order, so that s * v - m is deq32's weight (s * v when m = 0). Only for types
// with w_int_sub(type) > 0.
__device__ inline void deq32_int(int type, const uint8_t *row, int sb, _Float16 (&v)[32], float (&s)[2], float &m) {
#pragma clang fp contract(off)
    m = 0.f;
    switch (type) {
        case W_Q8_0: {  // y = q * d
            const uint16_t *p = (const uint16_t *)(row + 34 * sb);
            s[0] = s[1] = h2f(p[0]);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const uint32_t u = p[1 + i];
                v[2 * i] = (_Float16)(int8_t)(u & 0xff);
                v[2 * i + 1] = (_Float16)(int8_t)(u >> 8);
            }
            break;
        }
        case W_Q6_K: {  // y = (d * sc) * (q6 - 32)
            const uint8_t *blk = row + 210 * (sb >> 3);
            const int j = sb & 7, n = j >> 2, g = j & 3;
            const uint16_t *ql = (const uint16_t *)(blk + 64 * n + 32 * (g & 1));
            const uint16_t *qh = (const uint16_t *)(blk + 128 + 32 * n);
            const uint32_t scw = *(const uint16_t *)(blk + 192 + 8 * n + 2 * g);
            const float d = h2f(*(const uint16_t *)(blk + 208));
            s[0] = d * (float)(int8_t)(scw & 0xff), s[1] = d * (float)(int8_t)(scw >> 8);
            const int lsh = 4 * (g >> 1), hsh = 2 * g;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const uint32_t lo = ql[i], hi = qh[i];
#pragma unroll
                for (int b = 0; b < 2; b++)
                    v[2 * i + b] = (_Float16)((int)((((lo >> (8 * b)) >> lsh) & 15) | ((((hi >> (8 * b)) >> hsh) & 3) << 4)) - 32);
            }
            break;
        }
        case W_IQ4_XS: {  // y = (d * (ls - 32)) * table[nibble]
            const uint8_t *blk = row + 136 * (sb >> 3);
            const int ib = sb & 7;
            const uint2 hdr = *(const uint2 *)blk;
            const uint32_t ls = ((hdr.y >> (8 * (ib >> 1) + 4 * (ib & 1))) & 15) | (((hdr.x >> (16 + 2 * ib)) & 3) << 4);
            s[0] = s[1] = h2f(hdr.x & 0xffff) * (float)((int)ls - 32);
            const uint2 q0 = *(const uint2 *)(blk + 8 + 16 * ib), q1 = *(const uint2 *)(blk + 16 + 16 * ib);
            const uint32_t qs[4] = {q0.x, q0.y, q1.x, q1.y};
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const uint32_t u = byte_of(qs, i);
                v[i] = (_Float16)iq4_value(u & 15);
                v[i + 16] = (_Float16)iq4_value(u >> 4);
            }
            break;
        }
        case W_Q5_K: {  // y = (d * sc) * (q4 + 16 h) - dmin * m
            const uint8_t *blk = row + 176 * (sb >> 3);
            const int j = sb & 7;
            const uint32_t dm = *(const uint32_t *)blk;
            const uint32_t sw[3] = {((const uint32_t *)(blk + 4))[0], ((const uint32_t *)(blk + 4))[1],
                                    ((const uint32_t *)(blk + 4))[2]};
            const uint32_t sc = j < 4 ? byte_of(sw, j) & 63 : (byte_of(sw, j + 4) & 15) | ((byte_of(sw, j - 4) >> 6) << 4);
            const uint32_t mn = j < 4 ? byte_of(sw, j + 4) & 63 : (byte_of(sw, j + 4) >> 4) | ((byte_of(sw, j) >> 6) << 4);
            s[0] = s[1] = h2f(dm & 0xffff) * (float)sc;
            m = h2f(dm >> 16) * (float)mn;
            uint32_t qh[8], ql[8];
            *(u32x4 *)&qh[0] = ((const u32x4 *)(blk + 16))[0];
            *(u32x4 *)&qh[4] = ((const u32x4 *)(blk + 16))[1];
            *(u32x4 *)&ql[0] = ((const u32x4 *)(blk + 48 + 32 * (j >> 1)))[0];
            *(u32x4 *)&ql[4] = ((const u32x4 *)(blk + 48 + 32 * (j >> 1)))[1];
            const int ls = 4 * (j & 1);
#pragma unroll
            for (int i = 0; i < 32; i++) v[i] = (_Float16)(((byte_of(ql, i) >> ls) & 15) + (((byte_of(qh, i) >> j) & 1) << 4));
            break;
        }
        case W_F16: {  // y = the half itself
            s[0] = s[1] = 1.f;
#pragma unroll
            for (int k = 0; k < 4; k++) *(u32x4 *)&v[8 * k] = ((const u32x4 *)(row + 64 * sb))[k];
            break;
        }
        case W_BF16: {  // y = the bf16 value: 8 significant bits, exact in f16 once the block's
                        // largest magnitude is scaled into [2^14, 2^15) (values below 2^-10 of
                        // it, beneath f16's normal range, round to f16's subnormal steps)
            uint32_t h[16];
#pragma unroll
            for (int k = 0; k < 4; k++) *(u32x4 *)&h[4 * k] = ((const u32x4 *)(row + 64 * sb))[k];
            float w[32], mx = 0.f;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                w[2 * i] = __uint_as_float(h[i] << 16);
                w[2 * i + 1] = __uint_as_float(h[i] & 0xffff0000u);
                mx = fmaxf(mx, fmaxf(fabsf(w[2 * i]), fabsf(w[2 * i + 1])));
            }
            const int e = mx > 0.f && __builtin_isfinite(mx) ? __builtin_amdgcn_frexp_expf(mx) - 15 : 0;
            s[0] = s[1] = __builtin_amdgcn_ldexpf(1.f, e);
#pragma unroll
            for (int i = 0; i < 32; i++) v[i] = (_Float16)__builtin_amdgcn_ldexpf(w[i], -e);
            break;
        }
        default:
            s[0] = s[1] = 0.f;
#pragma unroll
            for (int i = 0; i < 32; i++) v[i] = 0;
    }
}

__device__ inline bool w_is_float(int t) { return t == W_F32 || t == W_F16 || t == W_BF16; }

}  // namespace flint
