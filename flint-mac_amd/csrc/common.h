// Shared constants and CDNA4 (gfx950) building blocks for the flint attention
// kernels. Shapes are Flint's fixed attention shapes
// (/root/reference/src/metal/flint_config.h:13-19).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace flint {

constexpr int N_HEAD = 32;
constexpr int N_HEAD_KV = 4;
constexpr int HEAD_DIM = 128;
constexpr int GQA = N_HEAD / N_HEAD_KV;  // 8
constexpr int Q_DIM = N_HEAD * HEAD_DIM;  // 4096
constexpr int KV_DIM = N_HEAD_KV * HEAD_DIM;  // 512
constexpr int QKV_DIM = Q_DIM + 2 * KV_DIM;  // 5120: one raw q|k|v row
constexpr int N_EMBD = 2048;                  // hidden size (flint_config.h:12)
constexpr float LOG2E = 1.4426950408889634f;

// KV storage dtypes (values of flint_attn_layer.kv_dtype).
constexpr int DT_F16 = 1;
constexpr int DT_BF16 = 2;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // 8 packed 16-bit values

__device__ inline uint32_t pack2(uint16_t lo, uint16_t hi) { return (uint32_t)lo | ((uint32_t)hi << 16); }

// Per-dtype conversions and MFMA calls. The KV cache holds raw 16-bit words.
template <int DT>
struct KvType;

template <>
struct KvType<DT_F16> {
    typedef f16x8 vec8;
    __device__ static inline uint16_t from_float(float x) {
        _Float16 h = (_Float16)x;  // round to nearest even
        return __builtin_bit_cast(uint16_t, h);
    }
    __device__ static inline float to_float(uint16_t u) { return (float)__builtin_bit_cast(_Float16, u); }
    __device__ static inline vec8 as_vec(u16x8 u) { return __builtin_bit_cast(vec8, u); }
    // D(16x16) += A(16x32) * B(32x16)
    __device__ static inline f32x4 mfma16(vec8 a, vec8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};

template <>
struct KvType<DT_BF16> {
    typedef bf16x8 vec8;
    __device__ static inline uint16_t from_float(float x) {
        __bf16 h = (__bf16)x;  // round to nearest even
        return __builtin_bit_cast(uint16_t, h);
    }
    __device__ static inline float to_float(uint16_t u) { return __uint_as_float(uint32_t(u) << 16); }
    __device__ static inline vec8 as_vec(u16x8 u) { return __builtin_bit_cast(vec8, u); }
    __device__ static inline f32x4 mfma16(vec8 a, vec8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};

// f16 operands for the prefill MFMAs (both KV dtypes convert exactly into f16
// within its range; see attn_prefill.hip).
__device__ inline f32x16 mfma32_f16(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// K cache layout: per kv head, tiles of 32 slots (8 KiB each) stored in the order the
// decode kernel's 16x16x32 MFMA A operand reads them, so each of its load
// instructions reads 1 KiB contiguous: 16-byte unit (st*4 + c)*64 + 16g + n of a
// tile holds slot 8(n>>2) + 4st + (n&3) of the tile, dims 32c + 8g .. 32c + 8g + 7.
__host__ __device__ inline size_t kt_index(int kvh, int row, int dim, int rows) {
    const int r = row & 31, st = (r >> 2) & 1, n = ((r >> 3) << 2) | (r & 3);
    const int c = dim >> 5, g = (dim >> 3) & 3;
    return ((size_t)kvh * (rows >> 5) + (row >> 5)) * (32 * HEAD_DIM) + ((((st * 4 + c) * 64 + g * 16 + n) << 3) | (dim & 7));
}

// V cache layout: per kv head, V transposed in tiles of 32 slots,
// [kvh][rows/32][HEAD_DIM][32], so one 32-key tile of V^T is 8 KiB contiguous.
__host__ __device__ inline size_t vt_index(int kvh, int row, int dim, int rows) {
    return (((size_t)kvh * (rows >> 5) + (row >> 5)) * HEAD_DIM + dim) * 32 + (row & 31);
}

// Workgroup barrier that orders LDS only. __syncthreads() also orders global
// memory, which the compiler implements by waiting for every outstanding global
// load (s_waitcnt vmcnt(0)); this one leaves in-flight loads in flight.
// Make the compiler materialise a wave-uniform value at this point: its scalar load is
// issued here, together with the others pinned next to it, instead of being sunk to
// its first use.
template <typename T>
__device__ inline void pin_sgpr(T x) {
    asm volatile("" ::"s"(x));
}

// LDS pointer type of the global_load_lds builtin (loads straight from memory into LDS)
typedef __attribute__((address_space(3))) void lds_void;

template <int N>
__device__ inline void wait_vmcnt() {  // s_waitcnt vmcnt(N), other counters untouched
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ inline void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ inline float wave_sum_xor(float v, int mask) { return v + __shfl_xor(v, mask, 64); }
__device__ inline float wave_max_xor(float v, int mask) { return fmaxf(v, __shfl_xor(v, mask, 64)); }

// Cross-lane steps on VALU lane permutes instead of LDS shuffles (ds_bpermute, one LDS
// round trip each): DPP rotations within a row of 16 lanes, and gfx950's
// v_permlane16_swap / v_permlane32_swap across rows and wave halves.
template <int CTRL>
__device__ inline float dpp(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}
constexpr int DPP_ROR1 = 0x121, DPP_ROR2 = 0x122, DPP_ROR4 = 0x124, DPP_ROR8 = 0x128;  // row_ror:n

// x of lane l ^ 8 (a rotation by 8 within the row of 16)
__device__ inline float lane_xor8(float x) { return dpp<DPP_ROR8>(x); }

constexpr int DPP_QUAD_XOR1 = 0xb1, DPP_QUAD_XOR2 = 0x4e, DPP_HALF_MIRROR = 0x141;
// Sum over the aligned group of 8 lanes; all 8 get the same value.
__device__ inline float lane8_sum(float x) {
    x += dpp<DPP_QUAD_XOR1>(x);
    x += dpp<DPP_QUAD_XOR2>(x);
    return x + dpp<DPP_HALF_MIRROR>(x);
}

// f(x of lane l, x of lane l ^ 16): the swap leaves rows (0,0,2,2) in one register and
// (1,1,3,3) in the other, so every lane combines the same pair in the same order.
__device__ inline float xor16_sum(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ inline float xor16_max(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// f(x of lane l, x of lane l ^ 32): halves (lo, lo) and (hi, hi)
__device__ inline float xor32_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ inline float xor32_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// Sum / max over the 64 lanes of the wave (every lane gets it).
__device__ inline float wave_sum(float x) {
    x += dpp<DPP_ROR8>(x);
    x += dpp<DPP_ROR4>(x);
    x += dpp<DPP_ROR2>(x);
    x += dpp<DPP_ROR1>(x);
    return xor32_sum(xor16_sum(x));
}
__device__ inline float wave_max(float x) {
    x = fmaxf(x, dpp<DPP_ROR8>(x));
    x = fmaxf(x, dpp<DPP_ROR4>(x));
    x = fmaxf(x, dpp<DPP_ROR2>(x));
    x = fmaxf(x, dpp<DPP_ROR1>(x));
    return xor32_max(xor16_max(x));
}

// sin/cos of a RoPE angle (a float, as the reference computes it): the angle
// reaches ~6.5e4 rad at long context, so it is first reduced modulo 2*pi in
// double precision (error ~1e-11 rad) to keep sincosf on its short path.
__device__ inline void rope_sincos(float a, float *sn, float *cs) {
    const double twopi = 6.283185307179586476925286766559;
    const double r = (double)a - twopi * rint((double)a * (1.0 / twopi));
    sincosf((float)r, sn, cs);
}

// RMSNorm (+ NEOX RoPE) of one 128-dim head row by one wave: lane holds dims
// lane and lane + 64 (a NEOX pair, x) with their gains (w), cs/sn the rotation
// of frequency `lane`.
__device__ inline float2 norm_rope_pair(float2 x, float2 w, float eps, bool rope, float cs, float sn) {
    const float ss = wave_sum(x.x * x.x + x.y * x.y);
    const float scale = 1.0f / sqrtf(ss / HEAD_DIM + eps);
    float x0 = x.x * scale * w.x, x1 = x.y * scale * w.y;
    if (rope) {
        const float y0 = x0 * cs - x1 * sn, y1 = x0 * sn + x1 * cs;
        x0 = y0;
        x1 = y1;
    }
    return make_float2(x0, x1);
}

// The same angle's sin/cos on the hardware sine/cosine (v_sin_f32 / v_cos_f32, whose
// argument is in turns), for operands that are rounded to f16 right after (prefill's q).
// The angle is reduced to [-1/2, 1/2] turns in float arithmetic: t + e = a * c_hi
// exactly (e from an fma), t - rint(t) is exact, and a * c_lo carries the rest of
// 1/(2 pi), so r is within ~3e-8 turns of the exact reduction for |a| up to ~1e7.
// Contraction is off so that t stays the rounded product e was taken from.
__device__ inline void rope_sincos_fast(float a, float *sn, float *cs) {
#pragma clang fp contract(off)
    const float c_hi = 0.15915494f, c_lo = 6.4206382e-09f;  // 1/(2 pi) = c_hi + c_lo
    const float t = a * c_hi;
    const float e = __builtin_fmaf(a, c_hi, -t);
    const float r = (t - __builtin_rintf(t)) + __builtin_fmaf(a, c_lo, e);
    *sn = __builtin_amdgcn_sinf(r);
    *cs = __builtin_amdgcn_cosf(r);
}

}  // namespace flint
