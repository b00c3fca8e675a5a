// Layer-major batched prefill attention for CDNA4 (gfx950).
//
// Replaces the reference's k_qk_prefill + k_attn_prefill
// (/root/reference/src/metal/prefill.metal:99-266, dispatched per 512-token
// chunk at /root/reference/src/engine.mm:1087-1104).
//
// Three launches per layer call, stream-ordered:
//  prefix:  positions [kbase, p0) already in the layer's cache are converted
//           into the attention copy (f16, below). kbase = 0 for full layers,
//           max(0, p0 - 512) for SWA layers (the window of the first new token).
//  kv_prep: per new token, RMSNorm (+ NEOX RoPE) of the 4 k heads and the v
//           rows, rounded to the cache dtype, into the cache (SWA: only the last
//           n_slots positions, slot p & (n_slots-1)) and into the attention copy.
//           The prefix runs first because a long SWA prefill overwrites ring
//           slots the prefix reads.
//  flash:   one workgroup per (32-position query block, kv head) serves the 8 q
//           heads of the group (256 query rows, 8 waves x 1 head x 32 rows), so
//           a K/V tile is staged in LDS once per 256 rows. Q is normalised,
//           rotated and scaled in the prologue (q never round-trips through HBM).
//           Scores are S^T = K Q^T and O^T += V^T P^T on v_mfma_f32_32x32x16_f16
//           with fp32 accumulation; K/V stream in 32-key tiles through a 5-tile
//           LDS ring in a software pipeline (the next tile's score MFMAs between
//           this tile's softmax instructions), one barrier per two tiles; the
//           online softmax starts from m = sink, l = 1 (the sink is in the
//           denominator only, prefill.metal:162), raises its running max lazily
//           (only past a margin of 2^8) and masks kp <= qp and, on SWA layers,
//           qp - kp < window (prefill.metal:212).
// Any T in one call: the attention copy is a linear buffer of kbase..p0+T, so
// the reference's 512-token chunking (ring room, flint_config.h:29-31) is not
// needed.
#include <climits>

#include "common.h"
#include "flint_attn_internal.h"

namespace flint {

constexpr int PF_BQ = 32;  // query positions per workgroup
constexpr float PF_RESCALE_LOG2 = 8.f;  // lazy running-max margin (p stays below 2^8)

// S^T row i (MFMA A row) holds key sigma(i) of its 32-key tile: bits 2 and 3 of i
// swapped, so that a lane's 16 score rows are, per 16-key half, 8 consecutive keys
// (the P^T operand of the P*V MFMA then needs no data movement). An involution.
__host__ __device__ inline int pf_sigma(int i) { return (i & 0x13) | ((i & 4) << 1) | ((i & 8) >> 1); }

// Attention copy of K and V (f16), per kv head in 32-key tiles of 16 rows x 64
// units of 16 bytes (16 KiB), in the order the flash kernel's MFMAs read them from
// LDS, one unit per lane:
//   rows 0..7  (K, row st):            unit l = key pf_sigma(l & 31), dims 16st + 8(l>>5) .. +7
//   rows 8..15 (V^T, row 8 + 2dt + kk): unit l = dim 32dt + (l & 31), keys 16kk + 8(l>>5) .. +7
__device__ inline size_t pk_index(int kvh, int row, int dim, int rows) {
    const size_t tile = (size_t)kvh * (rows >> 5) + (row >> 5);
    return (tile * 16 + (dim >> 4)) * 512 + ((((dim >> 3) & 1) * 32 + pf_sigma(row & 31)) << 3) + (dim & 7);
}
__device__ inline size_t pv_index(int kvh, int row, int dim, int rows) {
    const size_t tile = (size_t)kvh * (rows >> 5) + (row >> 5);
    const int k = row & 31;
    return (tile * 16 + 8 + (dim >> 5) * 2 + (k >> 4)) * 512 + ((((k >> 3) & 1) * 32 + (dim & 31)) << 3) + (k & 7);
}

// The id of the last prefill call that stored some tile of the attention copy scaled (its K
// or V values did not fit f16 as they are): written by prefix_kernel and kv_prep_kernel,
// compared with the call's own id by the flash kernel, which then takes its scaled path.
// Ids are unique per call, so the flag needs no reset.
static __device__ uint32_t g_scaled_call;

// The exponent e a tile's values are scaled by (x * 2^-e) to be stored in f16 with its full
// relative precision, from the tile's largest magnitude mx: 0 (stored as is) for mx in
// [2^-6, 2^15), for 0 and for inf / nan (which f16 carries as they are); otherwise
// ilogb(mx) - 14, which puts the scaled maximum in [2^14, 2^15). Tiny tiles are scaled up
// only when `up` (V: the output inherits V's scale; a tiny K only makes its scores tiny,
// which f16 carries to the same absolute accuracy as the reference's fp32).
__device__ inline int tile_exp(float mx, bool up) {
    if (!__builtin_isfinite(mx) || mx == 0.f) return 0;
    if (mx < 32768.f && (!up || mx >= 0.015625f)) return 0;
    return __builtin_amdgcn_frexp_expf(mx) - 15;  // frexp exponent f: mx in [2^(f-1), 2^f)
}

// Maximum over the 256 threads of a workgroup (red: 4 floats of LDS).
__device__ inline float block_max256(float x, float *red) {
    x = wave_max(x);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// A tile's exponents into the table, and the call's flag when the tile is scaled.
__device__ inline void put_texp(const PrefillParams &P, int kvh, int row0, int eK, int eV) {
    P.texp[kvh * (P.k_rows >> 5) + ((row0 - 32 * P.n_direct) >> 5)] = (eK & 0xffff) | (eV << 16);
    if (eK | eV) __hip_atomic_store(&g_scaled_call, P.call_id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// prefix: cache -> attention copy for the cached positions [kbase + 32 n_direct, p0) (the
// n_direct whole tiles before them are read from the cache by the flash kernel itself).
// grid (tiles, kv head), 256 threads. Block x takes tile n_direct + x; a whole tile of cached positions: a
// cache tile and a copy tile both hold 16-byte units of 8 dims of one key (K) or 8 keys of one
// dim (V), so each thread moves 2 + 2 units: read, measure, scale, convert to f16, write at
// the unit's place in the copy. When p0 is not 32-aligned, one more block copies the cached
// positions [p0 & ~31, p0) of the tile that holds p0 into their places in the copy as the
// cache's raw 16-bit values: kv_prep takes them from there (a long SWA prefill overwrites
// their ring slots in its own launch) and writes the tile, new positions included.
template <int DT>
__global__ __launch_bounds__(256) void prefix_kernel(const PrefillParams P) {
    typedef KvType<DT> KT;
    __shared__ float red[2][4];
    const int kvh = blockIdx.y, tid = threadIdx.x;
    const int row0 = 32 * (P.n_direct + (int)blockIdx.x), pos0 = P.kbase + row0;  // the tile's first position
    const int crow = row0 - 32 * P.n_direct;  // its row in the copy, which starts at tile n_direct
    if (pos0 + 32 > P.p0) {  // the tile holding p0: raw values of positions [pos0, p0)
        // every load before the first store: a load after a store that may alias it (both
        // 16-bit) waits for the store, one round trip per element
        constexpr int PER = 32 * HEAD_DIM / 256;  // elements per thread, at most
        uint16_t *raw = (uint16_t *)P.sk;
        const int n = (P.p0 - pos0) * HEAD_DIM;
        uint16_t kx[PER], vx[PER];
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const int i = min(tid + 256 * j, n - 1), r = i >> 7, d = i & 127, slot = (pos0 + r) & P.cache_mask;
            kx[j] = P.cache_k[kt_index(kvh, slot, d, P.n_slots)];
            vx[j] = P.cache_v[vt_index(kvh, slot, d, P.n_slots)];
        }
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const int i = tid + 256 * j, r = i >> 7, d = i & 127;
            if (i < n) {
                raw[pk_index(kvh, crow + r, d, P.k_rows)] = kx[j];
                raw[pv_index(kvh, crow + r, d, P.k_rows)] = vx[j];
            }
        }
        return;
    }
    const size_t ct = (size_t)kvh * (P.n_slots >> 5) + ((pos0 & P.cache_mask) >> 5);  // its cache tile
    const u32x4 *kc = (const u32x4 *)(P.cache_k + ct * (32 * HEAD_DIM));
    const u32x4 *vc = (const u32x4 *)(P.cache_v + ct * (32 * HEAD_DIM));
    u32x4 ku[2], vu[2];
#pragma unroll
    for (int i = 0; i < 2; i++) ku[i] = kc[tid + 256 * i], vu[i] = vc[tid + 256 * i];
    int eK = 0, eV = 0;
    if constexpr (DT == DT_BF16) {
        float mk = 0.f, mv = 0.f;
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int w = 0; w < 4; w++) {
                mk = fmaxf(mk, fmaxf(fabsf(KT::to_float(ku[i][w] & 0xffff)), fabsf(KT::to_float(ku[i][w] >> 16))));
                mv = fmaxf(mv, fmaxf(fabsf(KT::to_float(vu[i][w] & 0xffff)), fabsf(KT::to_float(vu[i][w] >> 16))));
            }
        eK = tile_exp(block_max256(mk, red[0]), false);
        eV = tile_exp(block_max256(mv, red[1]), true);
    }
    if (tid == 0) put_texp(P, kvh, row0, eK, eV);
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int u = tid + 256 * i;
        f16x8 k8, v8;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const uint32_t kw = ku[i][e >> 1], vw = vu[i][e >> 1];
            k8[e] = (_Float16)__builtin_amdgcn_ldexpf(KT::to_float(e & 1 ? kw >> 16 : kw & 0xffff), -eK);
            v8[e] = (_Float16)__builtin_amdgcn_ldexpf(KT::to_float(e & 1 ? vw >> 16 : vw & 0xffff), -eV);
        }
        // K cache unit (st*4 + c)*64 + 16g + n: key 8(n>>2) + 4st + (n&3), dims 32c + 8g .. +7
        const int st = u >> 8, c = (u >> 6) & 3, g = (u >> 4) & 3, n = u & 15;
        const int r = 8 * (n >> 2) + 4 * st + (n & 3);
        *(f16x8 *)(P.sk + pk_index(kvh, crow + r, 32 * c + 8 * g, P.k_rows)) = k8;
        // V cache unit 4d + g: dim d, keys 8g .. 8g+7
        *(f16x8 *)(P.sk + pv_index(kvh, crow + 8 * (u & 3), u >> 2, P.k_rows)) = v8;
    }
}

// ---------------------------------------------------------------------------
// kv_prep: the new tokens' K and V. grid (32-position chunks, kv head), 4 waves.
// Chunk c holds positions 32 c0 + 32 c .. +31 (32-aligned, so it is one tile of the
// attention copy, whose kbase is 32-aligned, and one tile of the cache). Wave w owns the 8
// consecutive rows 8w .. 8w+7, 8 lanes a row (16 dims a lane, so one RMSNorm scale per lane
// serves 16 dims; the row-per-wave layout before it spent ~1 us more per call on per-row
// reductions and divisions): it normalises (+ RoPE) each row's k, rounds k and v to the cache
// dtype into LDS (k row-major, v transposed), then writes every 16-byte unit those rows make: the copy's
// K units (one key, 8 dims) and V units (one dim, these 8 keys), scaled by the tile's
// exponents, and the cache's units of the new positions it keeps. So an f16 chunk needs no
// workgroup barrier (a bf16 chunk has one, for the tile's exponents). The first chunk also
// takes the cached positions before p0 (from the copy, where prefix_kernel left their raw
// values), and rows past the last new position are zero. A V unit of the cache spans the 8
// positions: where some of them are not new (or, for the ring, not kept) its elements are
// stored one by one, so no cache unit is read back and no two workgroups write the same bytes.
constexpr int KP_WAVES = 4, KP_THREADS = 64 * KP_WAVES, KP_ROWS = 32 / KP_WAVES;  // rows per wave
static_assert(KP_ROWS == 8, "a wave's rows make whole V units (8 keys)");
template <int DT>
__global__ __launch_bounds__(KP_THREADS) void kv_prep_kernel(const PrefillParams P) {
    typedef KvType<DT> KT;
    __shared__ __align__(16) uint16_t kl[32][HEAD_DIM + 8];  // k in the cache dtype, [row][dim]
    __shared__ __align__(16) uint16_t vt[HEAD_DIM][32 + 8];  // v in the cache dtype, [dim][row]
    __shared__ float red[2][KP_WAVES];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kvh = blockIdx.y;
    const int c0 = (P.p0 >> 5) + blockIdx.x, pos0 = 32 * c0;  // first position of the chunk
    const int lo = max(P.p0, pos0), hi = min(P.p0 + P.T, pos0 + 32);  // new positions [lo, hi)
    const int r0 = KP_ROWS * wave;  // this wave's rows r0 .. r0 + 7
    // Lane (rr, q8) takes row r0 + rr, dims 32k + 4 q8 + j (k, j < 4): a row's sum of squares is a
    // sum over its 8 lanes, each lane's RMSNorm scale serves its 16 dims, and a NEOX pair
    // (d, d + 64) is (k, k + 2) of one lane. All loads first (rows outside [lo, hi) read the chunk's
    // first new token, in range, and are zeroed), then the maths.
    const int rr = lane >> 3, q8 = lane & 7, r = r0 + rr, pos = pos0 + r;
    const bool is_new = pos >= lo && pos < hi;
    const float *kr = P.qkv + (size_t)((is_new ? pos : lo) - P.p0) * P.q_stride + Q_DIM + kvh * HEAD_DIM + 4 * q8;
    float4 kx[4], vx[4], kw[4], rf[2];
#pragma unroll
    for (int k = 0; k < 4; k++) kw[k] = *(const float4 *)(P.k_norm + 32 * k + 4 * q8);
#pragma unroll
    for (int k = 0; k < 2; k++) rf[k] = *(const float4 *)&P.rope_freq[32 * k + 4 * q8];
#pragma unroll
    for (int k = 0; k < 4; k++) kx[k] = *(const float4 *)(kr + 32 * k);
#pragma unroll
    for (int k = 0; k < 4; k++) vx[k] = *(const float4 *)(kr + KV_DIM + 32 * k);
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) ss += kx[k].x * kx[k].x + kx[k].y * kx[k].y + kx[k].z * kx[k].z + kx[k].w * kx[k].w;
    ss = lane8_sum(ss);
    const float scale = 1.0f / sqrtf(ss / HEAD_DIM + P.rms_eps);  // as norm_rope_pair
    float y[4][4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float *x = &kx[k].x, *w = &kw[k].x;
#pragma unroll
        for (int j = 0; j < 4; j++) y[k][j] = x[j] * scale * w[j];
    }
    if (P.has_rope) {
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const float *f = &rf[k].x;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                float cs, sn;
                rope_sincos((float)pos * f[j], &sn, &cs);
                const float x0 = y[k][j], x1 = y[k + 2][j];
                y[k][j] = x0 * cs - x1 * sn;
                y[k + 2][j] = x0 * sn + x1 * cs;
            }
        }
    }
    float mk = 0.f, mv = 0.f;  // this lane's largest |k| and |v| (bf16: they set the tile's exponents)
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float *v = &vx[k].x;
        uint16_t kh[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            kh[j] = is_new ? KT::from_float(y[k][j]) : 0;
            const uint16_t vh = is_new ? KT::from_float(v[j]) : 0;
            vt[32 * k + 4 * q8 + j][r] = vh;
            if constexpr (DT == DT_BF16) {
                mk = fmaxf(mk, fabsf(KT::to_float(kh[j])));
                mv = fmaxf(mv, fabsf(KT::to_float(vh)));
            }
        }
        *(uint2 *)&kl[r][32 * k + 4 * q8] = make_uint2(pack2(kh[0], kh[1]), pack2(kh[2], kh[3]));
    }
    if (pos0 + r0 < lo) {  // wave-uniform
        // the first chunk of a continuation that starts inside a tile: its cached positions
        // [pos0, p0) come from the copy, where prefix_kernel left the cache's raw values
        // (kbase <= pos0, 32-aligned)
        const uint16_t *raw = (const uint16_t *)P.sk;
        // all rows' loads first (rows from lo on re-read the first row), so they share one round trip
        uint16_t rk[KP_ROWS][2], rv[KP_ROWS][2];
#pragma unroll
        for (int i = 0; i < KP_ROWS; i++) {
            const int r = pos0 + r0 + i < lo ? r0 + i : r0;
            const int row = pos0 + r - P.kbase - 32 * P.n_direct;  // the copy starts at tile n_direct
            rk[i][0] = raw[pk_index(kvh, row, lane, P.k_rows)], rk[i][1] = raw[pk_index(kvh, row, lane + 64, P.k_rows)];
            rv[i][0] = raw[pv_index(kvh, row, lane, P.k_rows)], rv[i][1] = raw[pv_index(kvh, row, lane + 64, P.k_rows)];
        }
#pragma unroll
        for (int i = 0; i < KP_ROWS; i++) {
            const int r = r0 + i;
            if (pos0 + r < lo) {
                const uint16_t k0 = rk[i][0], k1 = rk[i][1], v0 = rv[i][0], v1 = rv[i][1];
                kl[r][lane] = k0, kl[r][lane + 64] = k1, vt[lane][r] = v0, vt[lane + 64][r] = v1;
                if constexpr (DT == DT_BF16) {
                    mk = fmaxf(mk, fmaxf(fabsf(KT::to_float(k0)), fabsf(KT::to_float(k1))));
                    mv = fmaxf(mv, fmaxf(fabsf(KT::to_float(v0)), fabsf(KT::to_float(v1))));
                }
            }
        }
    }
    int eK = 0, eV = 0;
    if constexpr (DT == DT_BF16) {
        mk = wave_max(mk), mv = wave_max(mv);
        if (lane == 0) red[0][wave] = mk, red[1][wave] = mv;
        __syncthreads();  // also makes every wave's rows visible (only this wave's are read)
        float xk = red[0][0], xv = red[1][0];
#pragma unroll
        for (int w = 1; w < KP_WAVES; w++) xk = fmaxf(xk, red[0][w]), xv = fmaxf(xv, red[1][w]);
        eK = tile_exp(xk, false);
        eV = tile_exp(xv, true);
    } else {
        // only this wave's rows are read back
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    const int row0 = pos0 - P.kbase;  // the chunk's first position, from kbase
    const int crow = row0 - 32 * P.n_direct;  // its attention-copy row (the copy starts at tile n_direct)
    if (threadIdx.x == 0) put_texp(P, kvh, row0, eK, eV);
    const int clo = max(lo, P.cache_from);         // positions [clo, hi) go to the cache
    const bool to_cache = hi > clo;
    const int ctile = (pos0 & P.cache_mask) >> 5;  // the cache tile (slot = pos & mask, 32-aligned)
#pragma unroll
    for (int m = 0; m < 2; m++) {
        const int j = lane + 64 * m;  // 128 units per kind: 8 keys x 16 dim groups, 128 dims
        // K units of key r0 + (j & 7), dims 8 (j >> 3) .. +7: the copy's (16 st + 8 hh) and the cache's
        {
            const int r = r0 + (j & 7), d0 = 8 * (j >> 3);
            const u16x8 kv = *(const u16x8 *)&kl[r][d0];
            f16x8 v;
#pragma unroll
            for (int e = 0; e < 8; e++) v[e] = (_Float16)__builtin_amdgcn_ldexpf(KT::to_float(kv[e]), -eK);
            *(f16x8 *)(P.sk + pk_index(kvh, crow + r, d0, P.k_rows)) = v;
            if (to_cache && pos0 + r >= clo && pos0 + r < hi)
                *(u16x8 *)(P.cache_k + kt_index(kvh, 32 * ctile + r, d0, P.n_slots)) = kv;
        }
        // V units of dim j, keys r0 .. r0 + 7
        {
            const u16x8 vv = *(const u16x8 *)&vt[j][r0];
            f16x8 v;
#pragma unroll
            for (int e = 0; e < 8; e++) v[e] = (_Float16)__builtin_amdgcn_ldexpf(KT::to_float(vv[e]), -eV);
            *(f16x8 *)(P.sk + pv_index(kvh, crow + r0, j, P.k_rows)) = v;
            if (to_cache) {
                uint16_t *dst = P.cache_v + vt_index(kvh, 32 * ctile + r0, j, P.n_slots);
                if (pos0 + r0 >= clo && pos0 + r0 + 8 <= hi) {  // wave-uniform
                    *(u16x8 *)dst = vv;
                } else {
#pragma unroll
                    for (int e = 0; e < 8; e++)
                        if (pos0 + r0 + e >= clo && pos0 + r0 + e < hi) dst[e] = vv[e];
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// flash attention
constexpr int PF_WAVES = 8;                  // one q head of the GQA group per wave
constexpr int PF_THREADS = PF_WAVES * 64;
constexpr int PF_TILE_UNITS = 16 * 64;       // 16-byte units per 32-key tile (16 KiB)
constexpr int PF_UNITS_PER_THREAD = PF_TILE_UNITS / PF_THREADS;
constexpr int PF_RING = 5;                   // tiles held in LDS (a barrier every two tiles)

// One tile of the attention copy as 16-byte units, read contiguously: units tid + 512 i.
struct PfTile {
    u32x4 u[PF_UNITS_PER_THREAD];
};
__device__ inline void pf_gload(PfTile &R, const _Float16 *__restrict__ src, int tid) {
#pragma unroll
    for (int i = 0; i < PF_UNITS_PER_THREAD; i++) R.u[i] = *(const u32x4 *)(src + 8 * (tid + PF_THREADS * i));
}
__device__ inline void pf_lstore(const PfTile &R, f16x8 (*dst)[64], int tid) {
#pragma unroll
    for (int i = 0; i < PF_UNITS_PER_THREAD; i++) {
        const int u = tid + PF_THREADS * i;
        dst[u >> 6][u & 63] = __builtin_bit_cast(f16x8, R.u[i]);
    }
}

// Scores S^T = K Q^T of one tile for this wave's head, relative to the running max (the
// chain starts from -m): lane (col, hh) holds query row col, keys
// kp0 + 16(j>>1) + 8hh + 4(j&1) + r in element 4j + r.
__device__ __forceinline__ f32x16 pf_scores(const f16x8 (&kf)[8], const f16x8 (&qf)[8], const f32x16 &negm) {
    f32x16 s = mfma32_f16(kf[0], qf[0], negm);
#pragma unroll
    for (int st = 1; st < 8; st++) s = mfma32_f16(kf[st], qf[st], s);
    return s;
}
// Keys outside the row's [key_lo, key_hi] (causal, SWA window, rows past T) get -inf.
__device__ __forceinline__ void pf_mask(f32x16 &s, int kp0, int hh, int key_lo, int key_hi) {
#pragma unroll
    for (int e = 0; e < 16; e++) {
        const int j = e >> 2, r = e & 3;
        const int kp = kp0 + 16 * (j >> 1) + 8 * hh + 4 * (j & 1) + r;
        s[e] = ((kp >= key_lo) & (kp <= key_hi)) ? s[e] : -INFINITY;
    }
}
// Does any score exceed the running max by more than the margin? Scores are finite or
// -inf, so compared as signed integers every float above the margin is above its bit
// pattern and every negative float below it: an integer max tree.
__device__ __forceinline__ bool pf_over_margin(const f32x16 &s) {
    int mi = __float_as_int(s[0]);
#pragma unroll
    for (int e = 1; e < 16; e++) mi = max(mi, __float_as_int(s[e]));
    return __builtin_amdgcn_ballot_w64(mi > __float_as_int(PF_RESCALE_LOG2)) != 0;
}
// Raise the running max to cover s (wave-uniform call, rare): the row's m grows by d,
// l and acc scale by 2^-d, s is re-expressed against the new m.
__device__ __forceinline__ void pf_rescale(f32x16 &s, float &m, float &l, f32x16 &negm, f32x16 (&acc)[4]) {
    float mt = s[0];
#pragma unroll
    for (int e = 1; e < 16; e++) mt = fmaxf(mt, s[e]);
    const float d = fmaxf(xor32_max(mt), 0.f);
    const float corr = __builtin_amdgcn_exp2f(-d);
    m += d;
#pragma unroll
    for (int e = 0; e < 16; e++) negm[e] = -m;
    l *= corr;
#pragma unroll
    for (int dt = 0; dt < 4; dt++) acc[dt] *= corr;
#pragma unroll
    for (int e = 0; e < 16; e++) s[e] -= d;
}
// P = 2^s in f16 (the MFMA operand); l += P in fp32. (v_dot2 on the f16 pairs would sum
// the rounded values, but it shares the matrix pipe's issue far worse than plain adds:
// measured ~4x the cost of an fma between MFMAs.)
__device__ __forceinline__ void pf_softmax(const f32x16 &s, f16x8 (&pf)[2], float &l) {
#pragma unroll
    for (int e = 0; e < 16; e++) {
        const float p = __builtin_amdgcn_exp2f(s[e]);
        pf[e >> 3][e & 7] = (_Float16)p;
        l += p;
    }
}
__device__ __forceinline__ void pf_pv(f32x16 (&acc)[4], const f16x8 (&vf)[8], const f16x8 (&pf)[2]) {
#pragma unroll
    for (int kk = 0; kk < 2; kk++)
#pragma unroll
        for (int dt = 0; dt < 4; dt++) acc[dt] = mfma32_f16(vf[2 * dt + kk], pf[kk], acc[dt]);
}

// Workgroup: 32 query positions x the 8 q heads of kv head kvh, wave w = head 8 kvh + w.
// Two waves per SIMD (about 250 registers each): while one wave runs softmax
// instructions the other can issue MFMAs.
// DIRECT: some tiles come from the cache itself (n_direct > 0). A separate instantiation: the
// per-tile source selection costs the loop 4 registers and ~7% of a config-4 full layer.
// SWA_DEAL: an SWA layer without key splits (every query block the same length), whose work is
// dealt as described at the block index below.
template <bool DIRECT, bool SWA_DEAL = false>
__global__ __launch_bounds__(PF_THREADS, 1) void flash_prefill_kernel(const PrefillParams P, int n_qblocks) {
    // LDS: five 32-key tiles in the attention-copy order (tile t in ring[(t - t_lo) % 5])
    __shared__ f16x8 ring[PF_RING][16][64];
    // LDS: 8 KiB per wave that hands q over to the operand order, and later the output
    __shared__ f16x8 q_lds[PF_WAVES][8][64];

    // SWA layers of two or more rounds of workgroups (every block the same length): the second
    // half of the first round starts ~4 us late. Otherwise all workgroups of a round load q
    // together, loop together (memory idle) and store together, and the next round's q loads meet
    // the stores; offset by about one q load, half the CUs move data while the other half loop,
    // which stays so in the later rounds (2.0-2.4 us less per T = 4000 call; on full layers the
    // longest-first order already spreads the workgroups out, and the offset measured slower).
    // Workgroups are dealt to CUs in id order, so ids 128 .. 255 are half of the first round.
    if constexpr (SWA_DEAL) {
        if (gridDim.x >= 384 && blockIdx.x >= 128 && blockIdx.x < 256) {
            const unsigned long long t_end = __builtin_amdgcn_s_memrealtime() + 400;  // 100 MHz ticks
            while (__builtin_amdgcn_s_memrealtime() < t_end) __builtin_amdgcn_s_sleep(4);
        }
    }
    // Did this call store some tile of the copy scaled (prefix / kv_prep set the flag before this
    // launch)? Read through the constant address space, so that it is a scalar load issued with
    // the kernel arguments, which the wave waits for anyway: this kernel never writes the flag,
    // and the launch's acquire makes the earlier kernels' store visible. (A plain read of the
    // variable is a vector load, and holding its value in an SGPR from here made every wave wait
    // for that load's round trip before it could issue its q loads.)
    const uint32_t scaled_call = *(const __attribute__((address_space(4))) uint32_t *)&g_scaled_call;
    pin_sgpr(scaled_call);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 31, hh = lane >> 5;
    // workgroup = (query block, key split, kv head), kv head fastest, then split; longest (causal)
    // query blocks first
    const int n_split = P.n_split;
    const int kvh = blockIdx.x & 3, hq = kvh * GQA + wave;
    const int rest = (int)(blockIdx.x >> 2), split = rest % n_split;
    // Longest-first (causal blocks grow with qb). SWA_DEAL: kv head h's workgroups land on XCDs
    // h and h + 4 (the hardware deals workgroup ids to the 8 XCDs in turn); each of the two takes a
    // contiguous half of the head's query blocks, longest first, so that its L2 fetches only its
    // half's copy tiles (a tile is read by the 17 blocks after it): the flash kernel's fetch falls
    // from 1.15x to 1.04x of q plus the copy.
    int qb;
    if constexpr (SWA_DEAL) {
        const int half_blocks = (n_qblocks + 1) >> 1;
        qb = (rest & 1) * half_blocks + (half_blocks - 1 - (rest >> 1));
        if (qb >= n_qblocks) return;  // the second half's first slot when n_qblocks is odd
    } else {
        qb = n_qblocks - 1 - rest / n_split;
    }
    const int t0 = qb * PF_BQ;
    const int q_first = P.p0 + t0, q_last = P.p0 + min(t0 + PF_BQ, P.T) - 1;
    const int my_t = t0 + col, my_qp = P.p0 + my_t;
    const bool row_ok = my_t < P.T;

    const int k_lo = P.is_swa ? max(P.kbase, q_first - (P.window - 1)) : 0;
    // 32-key tiles of this block, then of this split (P.tps tiles each)
    const int tb_lo = (k_lo - P.kbase) >> 5, tb_hi = (q_last - P.kbase) >> 5;
    const int t_lo = tb_lo + split * P.tps, t_hi = min(tb_hi, t_lo + P.tps - 1);
    // the record of row t, head hq of this split (acc[128], m in log2 units, l)
    auto part_row = [&](int t) { return P.part + ((size_t)(split * P.T + t) * N_HEAD + hq) * PF_PART_STRIDE; };
    if (t_lo > t_hi) {  // wave-uniform: a split past this block's keys (shorter blocks of a causal layer)
        if (hh == 0 && row_ok) *(float2 *)(part_row(my_t) + HEAD_DIM) = make_float2(P.sinks[hq] * LOG2E, 0.f);
        return;
    }
    const _Float16 *__restrict__ skv = P.sk + (size_t)kvh * (P.k_rows >> 5) * (16 * 64 * 8);
    // Tile t (32 keys from kbase + 32 t): from the attention copy, or for t < n_direct (whole
    // tiles of cached positions of an f16 cache, whose copy would hold the same bits) from the
    // cache tile itself. Either way thread tid receives copy units tid (K) and 512 + tid (V):
    // from the cache, the K unit of key pf_sigma(col), dims 16 st + 8 hh (kt_index order) and
    // the V unit of dim 32 dt + (tid & 31), keys 16 kk + 8 hh (vt_index order). Branch-free
    // (scalar bases, per-thread offsets), so the loads' wait counts stay static.
    const int n_direct = DIRECT ? P.n_direct : 0;
    const uint16_t *const ck = P.cache_k, *const cv = P.cache_v;
    const int ctile0 = kvh * (P.n_slots >> 5), kbase = P.kbase, cmask = P.cache_mask;
    const int dk = (int)kt_index(0, pf_sigma(tid & 31), 16 * (tid >> 6) + 8 * ((tid >> 5) & 1), 32);
    const int dv = (int)vt_index(0, 16 * ((tid >> 6) & 1) + 8 * ((tid >> 5) & 1), 32 * (tid >> 7) + (tid & 31), 32);
    auto gload = [&](PfTile &R, int t) {
        if constexpr (!DIRECT) {
            pf_gload(R, skv + (size_t)t * (PF_TILE_UNITS * 8), tid);
            return;
        }
        const bool dir = t < n_direct;  // wave-uniform
        const size_t ct = (size_t)ctile0 + (((kbase + 32 * t) & cmask) >> 5);
        const uint16_t *kb = dir ? ck + ct * (32 * HEAD_DIM) : (const uint16_t *)skv + (size_t)(t - n_direct) * (PF_TILE_UNITS * 8);
        const uint16_t *vb = dir ? cv + ct * (32 * HEAD_DIM) : kb + PF_TILE_UNITS * 4;
        const int ok = dir ? dk : 8 * tid, ov = dir ? dv : 8 * tid;
        static_assert(PF_UNITS_PER_THREAD == 2, "one K and one V unit per thread");
        R.u[0] = *(const u32x4 *)(kb + ok);
        R.u[1] = *(const u32x4 *)(vb + ov);
    };

    // ---- Q fragments (B operand of S^T = K Q^T): lane (col, hh) needs query row `col`,
    //      dims 16s + 8hh + e, in f16, after RMSNorm, NEOX RoPE and the scale
    //      log2(e)/sqrt(128) (the reference's half Q block, prefill.metal:158-161).
    //      Loaded row-coalesced instead: lane (rr, q8) = (lane >> 3, lane & 7) reads rows
    //      rr + 8g, dims 32k + 4q8 .. +3, so 8 lanes read one 128-byte line and an
    //      instruction 1 KiB; a row's sum of squares is an 8-lane sum and each NEOX pair
    //      (k, k + 2) sits in one lane. The f16 values go through this wave's LDS area
    //      into the operand order. ----
    // Loads in the order they are waited for (waits count loads in issue order): the
    // norm gains and this lane's 8 RoPE frequencies (32k + 4q8 + j, k < 2), which every
    // q value needs, then the q rows, then the first stage, needed only after q.
    const int q8 = lane & 7, rr = lane >> 3;
    float4 w[4], rf[2], x[4][4];
#pragma unroll
    for (int k = 0; k < 4; k++) w[k] = *(const float4 *)(P.q_norm + 32 * k + 4 * q8);
#pragma unroll
    for (int k = 0; k < 2; k++) rf[k] = *(const float4 *)&P.rope_freq[32 * k + 4 * q8];
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const int t = t0 + rr + 8 * g;
        const float *qp = P.qkv + (size_t)(t < P.T ? t : 0) * P.q_stride + hq * HEAD_DIM + 4 * q8;
#pragma unroll
        for (int k = 0; k < 4; k++) x[g][k] = *(const float4 *)(qp + 32 * k);
    }
    // Without DIRECT, the tiles go straight from memory into their ring slots
    // (global_load_lds_dwordx4: wave w's load i writes units 512 i + 64 w + lane, lane l's 16 bytes
    // at the LDS address in m0 plus 16 l), so no register holds them and no LDS store moves them.
    // Inline asm: for an LDS load it tracks, the compiler makes every later barrier wait for all
    // loads; these are waited for explicitly before the barrier that publishes their slots.
    constexpr bool DMA = !DIRECT;
    const uint32_t dma_voff = 16 * tid;  // the lane's bytes from a tile's start (unit tid)
    const uint32_t dma_lds = (uint32_t)(uintptr_t)(lds_void *)&ring[0][0][0] + 1024 * __builtin_amdgcn_readfirstlane(wave);
    auto dma_tile = [&](int t, int sl) {  // tile t into ring slot sl (wave-uniform)
        const _Float16 *const src = skv + (size_t)t * (PF_TILE_UNITS * 8);
#pragma unroll
        for (int i = 0; i < PF_UNITS_PER_THREAD; i++)
            asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(
                             dma_lds + (uint32_t)(sl * PF_TILE_UNITS * 16 + PF_THREADS * 16 * i)),
                         "v"(dma_voff), "s"(src + PF_THREADS * 8 * i)
                         : "m0");
    };
    PfTile R0, R1, R2, R3;
    if constexpr (DMA) {  // the first four tiles into slots 0..3 (waited for before the loop)
        dma_tile(t_lo, 0);
        if (t_lo + 1 <= t_hi) dma_tile(t_lo + 1, 1);
        if (t_lo + 2 <= t_hi) dma_tile(t_lo + 2, 2);
        if (t_lo + 3 <= t_hi) dma_tile(t_lo + 3, 3);
    } else {
        gload(R0, t_lo);
        if (t_lo + 1 <= t_hi) gload(R1, t_lo + 1);
        if (t_lo + 2 <= t_hi) gload(R2, t_lo + 2);
        if (t_lo + 3 <= t_hi) gload(R3, t_lo + 3);
    }

    // After the RMSNorm |q| <= sqrt(128) |gain|, and the scale log2(e)/sqrt(128) follows: q
    // gains that could take q past f16's range, or keep it below 2^-6, make q be stored scaled
    // by 2^-eQ (wave-uniform; every wave of the block reads the same gains), which the scaled
    // path below undoes.
    float gq = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++)
        gq = fmaxf(gq, fmaxf(fmaxf(fabsf(w[k].x), fabsf(w[k].y)), fmaxf(fabsf(w[k].z), fabsf(w[k].w))));
    const int eQ = tile_exp(wave_max(gq) * (LOG2E * 1.001f), true);
    const bool scaled = eQ != 0 || scaled_call == P.call_id;  // wave-uniform

    f16x8 qf[8];
    {
        const float qs = __builtin_amdgcn_ldexpf(LOG2E / sqrtf((float)HEAD_DIM), -eQ);
        uint2 *const qa = (uint2 *)&q_lds[wave][0][0];  // 8-byte halves of the f16x8 units
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int r = rr + 8 * g;
            float ss = 0.f;
#pragma unroll
            for (int k = 0; k < 4; k++)
                ss += x[g][k].x * x[g][k].x + x[g][k].y * x[g][k].y + x[g][k].z * x[g][k].z + x[g][k].w * x[g][k].w;
            ss = lane8_sum(ss);
            const float scale = t0 + r < P.T ? qs / sqrtf(ss / HEAD_DIM + P.rms_eps) : 0.f;
            const float pos = (float)(P.p0 + t0 + r);
            _Float16 h[4][4];
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const float *x0 = &x[g][k].x, *x1 = &x[g][k + 2].x, *w0 = &w[k].x, *w1 = &w[k + 2].x, *f = &rf[k].x;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float a0 = x0[j] * w0[j], a1 = x1[j] * w1[j];
                    float cs = 1.f, sn = 0.f;
                    if (P.has_rope) rope_sincos_fast(pos * f[j], &sn, &cs);
                    h[k][j] = (_Float16)((a0 * cs - a1 * sn) * scale);
                    h[k + 2][j] = (_Float16)((a0 * sn + a1 * cs) * scale);
                }
            }
            // dims 32k + 4q8 + j: unit [s = 2k + (q8 >> 2)][r + 32((q8 >> 1) & 1)], half q8 & 1
#pragma unroll
            for (int k = 0; k < 4; k++) {
                typedef _Float16 h4 __attribute__((ext_vector_type(4)));
                const h4 v = {h[k][0], h[k][1], h[k][2], h[k][3]};
                qa[((2 * k + (q8 >> 2)) * 64 + r + 32 * ((q8 >> 1) & 1)) * 2 + (q8 & 1)] = __builtin_bit_cast(uint2, v);
            }
        }
#pragma unroll
        for (int st = 0; st < 8; st++) qf[st] = q_lds[wave][st][lane];
    }

    // m starts at the sink; l counts the sink once (l = 1) unless the keys are split, in which
    // case the merge adds it
    float m = P.sinks[hq] * LOG2E, l = hh == 0 && n_split == 1 ? 1.f : 0.f;
    f32x16 negm;  // -m in every element: the C operand of each tile's first score MFMA
#pragma unroll
    for (int e = 0; e < 16; e++) negm[e] = -m;
    f32x16 acc[4];
#pragma unroll
    for (int dt = 0; dt < 4; dt++) acc[dt] = f32x16{};
    // this lane's query row attends to key positions [key_lo, key_hi] (causal, SWA window);
    // rows past T attend to nothing
    const int key_hi = row_ok ? my_qp : -1;
    const int key_lo = P.is_swa ? max(my_qp - (P.window - 1), 0) : 0;
    // wave-uniform: does any row of this block need masking in the tile at key kp0?
    auto edge = [&](int kp0) { return kp0 + 31 > q_first || (P.is_swa && q_last - kp0 >= P.window) || t0 + PF_BQ > P.T; };
    int E = 0;  // acc holds sum p V in units of 2^E (E != 0 only on the scaled path)

    if (scaled) {
        // ---- scaled path: some tile's K or V values were stored scaled by 2^-eK_t / 2^-eV_t to
        //      fit f16, or q by 2^-eQ (rare: values beyond f16's range, or tiny V tiles).
        //      Tile by tile, without the software pipeline: the scores of tile t are
        //      2^(eK_t + eQ) K'Q'^T (exact power-of-two factors), the running max is exact
        //      (no margin), and acc accumulates p V' 2^(eV_t - E) with E the largest V exponent
        //      so far (acc is rescaled when it grows). ----
        const int *te = P.texp + (size_t)kvh * (P.k_rows >> 5);
        if (DMA) wait_vmcnt<0>();  // the first four tiles have landed in the ring (unused here)
        for (int t = t_lo; t <= t_hi; t++) {
            __syncthreads();  // every wave is done with the previous tile's LDS
            {
                PfTile Rt;
                gload(Rt, t);
                pf_lstore(Rt, ring[0], tid);
            }
            __syncthreads();
            f16x8 kf[8], vf[8];
#pragma unroll
            for (int st = 0; st < 8; st++) kf[st] = ring[0][st][lane];
#pragma unroll
            for (int i = 0; i < 8; i++) vf[i] = ring[0][8 + i][lane];
            const int tx = t < n_direct ? 0 : te[t - n_direct];  // wave-uniform (cache tiles: unscaled f16)
            const int eK = (int)(int16_t)(tx & 0xffff), eV = tx >> 16;
            f32x16 sc = pf_scores(kf, qf, f32x16{});
            const float ssc = __builtin_amdgcn_ldexpf(1.f, eK + eQ);
#pragma unroll
            for (int e = 0; e < 16; e++) sc[e] *= ssc;
            if (edge(P.kbase + 32 * t)) pf_mask(sc, P.kbase + 32 * t, hh, key_lo, key_hi);
            float mt = sc[0];
#pragma unroll
            for (int e = 1; e < 16; e++) mt = fmaxf(mt, sc[e]);
            const float m_new = fmaxf(m, xor32_max(mt));  // m is finite (it starts at the sink)
            const float corr = __builtin_amdgcn_exp2f(m - m_new);
            if (t == t_lo) E = eV;
            const float vgrow = eV > E ? __builtin_amdgcn_ldexpf(1.f, E - eV) : 1.f;
            E = max(E, eV);
            m = m_new;
            l *= corr;
#pragma unroll
            for (int dt = 0; dt < 4; dt++) acc[dt] *= corr * vgrow;
            const float pscale = __builtin_amdgcn_ldexpf(1.f, eV - E);
            f16x8 pf[2];
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const float p = __builtin_amdgcn_exp2f(sc[e] - m);
                l += p;
                pf[e >> 3][e & 7] = (_Float16)(p * pscale);
            }
            pf_pv(acc, vf, pf);
        }
    } else {

    // ---- software pipeline over the key tiles. Step t computes P of tile t and its P V
    //      product while the score MFMAs of tile t + 1 run, in explicit slots with a
    //      scheduling fence after each:
    //       * slot g < 8 turns scores 2g, 2g+1 of tile t into P (exp, f16; fp32 row sum) and
    //         issues score MFMA g of tile t + 1; slots 0-2 also store tile t + 4 into the
    //         LDS ring and request tile t + 5;
    //       * slot 8 + j issues P V MFMA j of tile t and reads the V fragment of tile t + 1
    //         and the K fragment of tile t + 2 into the registers that MFMA and score MFMA j
    //         freed, with a step of tile t + 1's rescale test.
    //      Steps run in pairs (t_lo + 2j, t_lo + 2j + 1) with one barrier after each pair.
    //      A pair reads tiles t + 1 .. t + 3 (stored before the previous barrier) and
    //      writes tiles t + 4, t + 5 into the two ring slots whose tiles were last read in
    //      the previous pair, so five slots never conflict. ----
    if constexpr (DMA) {
        wait_vmcnt<0>();  // this wave's part of the first four tiles is in slots 0..3
    } else {
        pf_lstore(R0, ring[0], tid);
        if (t_lo + 1 <= t_hi) pf_lstore(R1, ring[1], tid);
        if (t_lo + 2 <= t_hi) pf_lstore(R2, ring[2], tid);
        if (t_lo + 3 <= t_hi) pf_lstore(R3, ring[3], tid);
    }
    PfTile R;
    if (!DMA && t_lo + 4 <= t_hi) gload(R, t_lo + 4);
    __syncthreads();

    f16x8 kf[8], vf[8];
#pragma unroll
    for (int st = 0; st < 8; st++) kf[st] = ring[0][st][lane];
#pragma unroll
    for (int i = 0; i < 8; i++) vf[i] = ring[0][8 + i][lane];
    f32x16 s_cur = pf_scores(kf, qf, negm);
    if (edge(P.kbase + 32 * t_lo)) pf_mask(s_cur, P.kbase + 32 * t_lo, hh, key_lo, key_hi);
    if (pf_over_margin(s_cur)) pf_rescale(s_cur, m, l, negm, acc);
    if (t_lo + 1 <= t_hi) {
#pragma unroll
        for (int st = 0; st < 8; st++) kf[st] = ring[1][st][lane];
    }
    __syncthreads();  // tile t_lo's slot is rewritten in the first pair

    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    auto slot = [](int r) { return r >= PF_RING ? r - PF_RING : r; };
    int sl0 = 0;  // ring slot of tile t
    auto step = [&](const f32x16 &sc, f32x16 &sn, int t, bool bar) {
        const int kp1 = P.kbase + 32 * (t + 1);
        const int sl1 = slot(sl0 + 1), sl2 = slot(sl0 + 2), sl4 = slot(sl0 + 4);
        const bool st4 = t + 4 <= t_hi, ld5 = t + 5 <= t_hi;
        uint32_t pw[8];  // P of tile t as f16 pairs
#pragma unroll
        for (int g = 0; g < 8; g++) {
            const float e0 = __builtin_amdgcn_exp2f(sc[2 * g]), e1 = __builtin_amdgcn_exp2f(sc[2 * g + 1]);
            const h2 pp = {(_Float16)e0, (_Float16)e1};
            pw[g] = __builtin_bit_cast(uint32_t, pp);
            l += e0 + e1;
            asm volatile("" : "+v"(l));  // keeps the row sum in this slot
            sn = mfma32_f16(kf[g], qf[g], g == 0 ? negm : sn);
            if (!DMA && g < PF_UNITS_PER_THREAD && st4) {
                const int u = tid + PF_THREADS * g;
                ring[sl4][u >> 6][u & 63] = __builtin_bit_cast(f16x8, R.u[g]);
            }
            if (!DMA && g == PF_UNITS_PER_THREAD && ld5) gload(R, t + 5);
            // DMA, first step of a pair: tiles t + 4 and t + 5 into the slots of tiles t - 1 and t,
            // which no wave reads after the barrier before this pair
            if (DMA && g == 0 && !bar && st4) dma_tile(t + 4, sl4);
            if (DMA && g == 1 && !bar && ld5) dma_tile(t + 5, sl0);
            __builtin_amdgcn_sched_barrier(0);
        }
        const f16x8 pf[2] = {__builtin_bit_cast(f16x8, u32x4{pw[0], pw[1], pw[2], pw[3]}),
                             __builtin_bit_cast(f16x8, u32x4{pw[4], pw[5], pw[6], pw[7]})};
        int mi = INT_MIN;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int kk = j >> 2, dt = j & 3;
            acc[dt] = mfma32_f16(vf[2 * dt + kk], pf[kk], acc[dt]);
            vf[2 * dt + kk] = ring[sl1][8 + 2 * dt + kk][lane];
            kf[j] = ring[sl2][j][lane];  // unused after the last tile
            mi = max(mi, max(__float_as_int(sn[2 * j]), __float_as_int(sn[2 * j + 1])));
            __builtin_amdgcn_sched_barrier(0);
        }
        const bool over = __builtin_amdgcn_ballot_w64(mi > __float_as_int(PF_RESCALE_LOG2)) != 0;
        // The test ran before the mask: a masked score can only raise m needlessly, which
        // the rescale handles exactly. Edge tiles are few, so they are masked outside the
        // interleave.
        if (edge(kp1)) pf_mask(sn, kp1, hh, key_lo, key_hi);
        if (over) pf_rescale(sn, m, l, negm, acc);
        if (bar) {
            if (DMA) wait_vmcnt<0>();  // this wave's part of the pair's two tiles is in its slots
            __syncthreads();
        }
        sl0 = sl1;
    };
    // two steps per iteration, so the score buffers alternate without copies
    f32x16 s_alt;
    int t = t_lo;
    for (; t + 2 <= t_hi; t += 2) {
        step(s_cur, s_alt, t, false);
        step(s_alt, s_cur, t + 1, true);
    }
    if (t < t_hi) {
        step(s_cur, s_alt, t, false);
        s_cur = s_alt;
    }
    {  // the last tile
        f16x8 pf[2];
        pf_softmax(s_cur, pf, l);
        pf_pv(acc, vf, pf);
    }
    }  // fast path

    // ---- output rows, normalised, through this wave's LDS area (32 rows x 64 dims of
    //      f32 at a time; float4 column c of row r at r * 16 + (c ^ (r & 15)), so both
    //      sides are conflict-free) and stored row-coalesced: 16 lanes write one row's
    //      256 bytes ----
    // split keys: the unnormalised partial (acc in true units, m, l) goes to this split's records
    const float lsum = xor32_sum(l);
    const float inv = __builtin_amdgcn_ldexpf(n_split == 1 ? 1.0f / lsum : 1.0f, E);  // rows past T: l = 1, acc = 0
    if (n_split > 1 && hh == 0 && row_ok) *(float2 *)(part_row(my_t) + HEAD_DIM) = make_float2(m, lsum);
    float4 *const ob = (float4 *)&q_lds[wave][0][0];
#pragma unroll
    for (int half = 0; half < 2; half++) {
#pragma unroll
        for (int d2 = 0; d2 < 2; d2++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const f32x16 &a = acc[2 * half + d2];
                const int c = 8 * d2 + 2 * j + hh;  // dims 32 d2 + 8j + 4hh of the half
                ob[col * 16 + (c ^ (col & 15))] = float4{a[4 * j] * inv, a[4 * j + 1] * inv, a[4 * j + 2] * inv, a[4 * j + 3] * inv};
            }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int r = 4 * i + (lane >> 4), c = lane & 15;
            const float4 v = ob[r * 16 + (c ^ (r & 15))];
            if (t0 + r < P.T) {
                float *dst = n_split == 1 ? P.att + (size_t)(t0 + r) * Q_DIM + hq * HEAD_DIM : part_row(t0 + r);
                // streaming stores: the output is not read again here, and left in the caches it
                // would evict the K/V tiles the other workgroups of the XCD still read (measured
                // 1.5-2.5 us faster per call on both layer kinds; q read the same way was slower)
                __builtin_nontemporal_store(f32x4{v.x, v.y, v.z, v.w}, (f32x4 *)(dst + 64 * half + 4 * c));
            }
        }
    }
}

// Merge of a split prefill (fused.metal:331-350 per query row): one wave per (row t, head),
// lane l holds dims 2l, 2l + 1 and the (m, l) pair of split l; the records are read 8 splits
// at a time (indices past n_split repeat the last one with weight 0); splits with l = 0 (no
// key of the row) get weight 0 and are skipped.
__global__ __launch_bounds__(256) void prefill_combine_kernel(const PrefillParams P) {
    const int lane = threadIdx.x & 63, pair = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (pair >= P.T * N_HEAD) return;
    const int t = pair / N_HEAD, hq = pair % N_HEAD, ns = P.n_split;
    const float *rec = P.part + ((size_t)t * N_HEAD + hq) * PF_PART_STRIDE;
    const size_t sstride = (size_t)P.T * N_HEAD * PF_PART_STRIDE;
    const float sink = P.sinks[hq] * LOG2E;
    float2 ml = make_float2(sink, 0.f);
    if (lane < ns) ml = *(const float2 *)(rec + lane * sstride + HEAD_DIM);
    const float M = fmaxf(wave_max(ml.y != 0.f ? ml.x : -INFINITY), sink);
    const float w = ml.y != 0.f ? __builtin_amdgcn_exp2f(ml.x - M) : 0.f;
    const float L = wave_sum(ml.y * w) + __builtin_amdgcn_exp2f(sink - M);
    float o0 = 0.f, o1 = 0.f;
    for (int s0 = 0; s0 < ns; s0 += 8) {  // ns <= 64, so s0 + i < 64
        float2 a[8];
#pragma unroll
        for (int i = 0; i < 8; i++) a[i] = *(const float2 *)(rec + min(s0 + i, ns - 1) * sstride + 2 * lane);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float ws = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), s0 + i));
            if (ws != 0.f) o0 += a[i].x * ws, o1 += a[i].y * ws;  // wave-uniform: a skipped split may hold anything
        }
    }
    const float inv = 1.0f / L;
    *(float2 *)(P.att + (size_t)t * Q_DIM + hq * HEAD_DIM + 2 * lane) = make_float2(o0 * inv, o1 * inv);
}

hipError_t launch_prefill(const PrefillParams &P, int dtype, hipStream_t stream) {
    // tiles holding cached positions (kbase 32-aligned) that the copy takes from the cache
    const int n_pre = ((P.p0 - P.kbase + 31) >> 5) - P.n_direct;
    const int nqb = (P.T + PF_BQ - 1) / PF_BQ;
    const dim3 gp(n_pre, N_HEAD_KV), gk(((P.p0 + P.T + 31) >> 5) - (P.p0 >> 5), N_HEAD_KV);
    if (dtype == DT_F16) {
        if (n_pre > 0) hipLaunchKernelGGL(prefix_kernel<DT_F16>, gp, dim3(256), 0, stream, P);
        hipLaunchKernelGGL(kv_prep_kernel<DT_F16>, gk, dim3(KP_THREADS), 0, stream, P);
    } else {
        if (n_pre > 0) hipLaunchKernelGGL(prefix_kernel<DT_BF16>, gp, dim3(256), 0, stream, P);
        hipLaunchKernelGGL(kv_prep_kernel<DT_BF16>, gk, dim3(KP_THREADS), 0, stream, P);
    }
    if (P.n_direct > 0)
        hipLaunchKernelGGL(flash_prefill_kernel<true>, dim3(nqb * P.n_split * N_HEAD_KV), dim3(PF_THREADS), 0, stream, P, nqb);
    else if (P.is_swa && P.n_split == 1)  // both halves of every kv head's blocks: an even count
        hipLaunchKernelGGL((flash_prefill_kernel<false, true>), dim3(2 * ((nqb + 1) >> 1) * N_HEAD_KV), dim3(PF_THREADS), 0,
                           stream, P, nqb);
    else
        hipLaunchKernelGGL(flash_prefill_kernel<false>, dim3(nqb * P.n_split * N_HEAD_KV), dim3(PF_THREADS), 0, stream, P, nqb);
    if (P.n_split > 1)
        hipLaunchKernelGGL(prefill_combine_kernel, dim3((P.T * N_HEAD + 3) / 4), dim3(256), 0, stream, P);
    return hipGetLastError();
}

}  // namespace flint
