// The attention projections of a prefill batch on the matrix cores (gfx950).
//
// Y[t][n] = sum_k W[n][k] X[t][k] for T tokens at once: the q/k/v projection of the RMSNorm'd
// hidden rows and the o projection (added to the residual) of a layer-major prefill step
// (/root/reference/src/engine.mm:1083-1086, 1105-1111). The reference's CPU path sums in double
// (ref_model.cpp:74-93); the one-token kernels here sum fp32 FMAs. The batch reaches the same
// fp32-level accuracy on v_mfma_f32_32x32x16_f16 by splitting both operands into f16 hi/lo
// pairs:
//   * every weight row (dequantised as in proj.hip) and every activation row is scaled by a
//     power of two that puts its largest magnitude in [2^14, 2^15), then split as
//     v = hi + lo with hi = f16(v), lo = f16(v - hi): 22 significant bits, and no value
//     overflows f16 whatever the row's range;
//   * the GEMM accumulates hi*hi + hi*lo + lo*hi in fp32 (the lo*lo term is below 2^-22 of
//     the product) and scales each output by 2^(e_t + f_n), which is exact.
// Three launches: wprep (weights -> planes), xprep (activations -> planes, the RMSNorm fused
// for q/k/v) and gemm3. The stage-level calls rebuild the weight planes from the GGUF rows each
// time (~20 us for a layer's 19M weights); a model keeps every layer's planes after building
// them once, and its calls launch only xprep and gemm3.
#include "common.h"
#include "dequant.h"
#include "flint_attn_internal.h"

namespace flint {

namespace {

// exponent that puts a row's largest magnitude mx in [2^14, 2^15): x * 2^-e fits f16 with its
// full 11 bits at the top of the row (0 for an all-zero row, inf / nan left as they are)
__device__ inline int row_exp(float mx) {
    if (!(mx > 0.f) || !__builtin_isfinite(mx)) return 0;
    return __builtin_amdgcn_frexp_expf(mx) - 15;  // mx in [2^(f-1), 2^f)
}

__device__ inline void split_store(float v, int e, _Float16 *hi, _Float16 *lo) {
    const float s = __builtin_amdgcn_ldexpf(v, -e);
    const _Float16 h = (_Float16)s;
    *hi = h;
    *lo = (_Float16)(s - (float)h);
}

// Planes are stored in the order gemm3 keeps them in LDS, so that a workgroup's chunk of a plane
// (128 rows x 32 k) is one contiguous 8 KiB block that it copies into LDS unchanged: blocks
// [row tile n >> 7][chunk k >> 5], and in a block the 16-byte unit of row r (n & 127), k group
// k8 ((k >> 3) & 3) at unit ((r >> 5) * 2 + (k8 >> 1)) * 64 + (r & 31) + 32 (k8 & 1). The element
// offset of the unit that holds elements 8 g .. 8 g + 7 of row n:
__device__ inline size_t plane_unit(int n, int g, int K) {
    const int r = n & 127, k8 = g & 3;
    const int q = ((r >> 5) * 2 + (k8 >> 1)) * 64 + (r & 31) + 32 * (k8 & 1);
    return (((size_t)(n >> 7) * (K / 32) + (g >> 2)) * 512 + q) * 8;
}

}  // namespace

// ---------------------------------------------------------------------------
// wprep: one 512-thread workgroup per 8 weight rows n0 .. n0 + 7, wave w on row n0 + w: the row's
// bytes staged through its LDS area (2-byte copies: q8_0 and q6_K blocks are only 2-byte aligned),
// dequantised 32 elements per lane per sub-block (lane l owns sub-blocks l, l + 64, ...), the
// row's exponent f_n from its largest magnitude, then its hi/lo values written over the staged
// bytes. After the workgroup's barrier every store writes 8 whole 128-byte lines of the planes'
// chunk order: lane (row rho = lane & 7, group lane gl = lane >> 3) of wave w takes the 16-byte
// units of groups gl + 8 (w + 8 j) of row n0 + rho. The wave areas are 16 bytes longer than a
// row's values, so the 8 rows' reads of one group fall on different banks.
template <int K>
__global__ __launch_bounds__(512) void wprep_kernel(const GemmWeightParams P) {
    constexpr int SUBS = K / 32 / 64;
    constexpr int AREA = K * 4 + 16;  // a staged row (at most K floats), later its hi|lo values
    static_assert(K / 32 * 34 <= K * 4, "a quantised row fits its area");
    __shared__ __align__(16) uint8_t areas[8 * AREA];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = 8 * blockIdx.x + wave;  // this wave's plane row
    uint8_t *const stage = areas + wave * AREA;
    const int in2 = P.n_seg > 2 && n >= P.seg[2].row0, in1 = !in2 && P.n_seg > 1 && n >= P.seg[1].row0;
    const MatvecSeg S = in2 ? P.seg[2] : in1 ? P.seg[1] : P.seg[0];
    const uint8_t *row = S.w + (size_t)(n - S.row0) * S.row_bytes;
    const uint16_t *src = (const uint16_t *)row;
    uint16_t *dst = (uint16_t *)stage;
    for (int i = lane; i < S.row_bytes / 2; i += 64) dst[i] = src[i];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float w[SUBS][32];
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < SUBS; i++) {
        deq32(S.type, stage, lane + 64 * i, w[i]);
#pragma unroll
        for (int e = 0; e < 32; e++) mx = fmaxf(mx, fabsf(w[i][e]));
    }
    const int f = row_exp(wave_max(mx));
    // every lane has read the staged bytes before any lane overwrites them
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    _Float16 *const hi = (_Float16 *)stage, *const lo = hi + K;
#pragma unroll
    for (int i = 0; i < SUBS; i++) {
        const int k0 = 32 * (lane + 64 * i);
        f16x8 h8[4], l8[4];
#pragma unroll
        for (int e = 0; e < 32; e++) {
            _Float16 h, l;
            split_store(w[i][e], f, &h, &l);
            h8[e >> 3][e & 7] = h;
            l8[e >> 3][e & 7] = l;
        }
#pragma unroll
        for (int q = 0; q < 4; q++) {
            *(f16x8 *)(hi + k0 + 8 * q) = h8[q];
            *(f16x8 *)(lo + k0 + 8 * q) = l8[q];
        }
    }
    if (lane == 0) P.fexp[n] = f;
    __syncthreads();
    const int rho = lane & 7, gl = lane >> 3, nr = 8 * blockIdx.x + rho;
    const _Float16 *const rh = (const _Float16 *)(areas + rho * AREA), *const rl = rh + K;
#pragma unroll
    for (int j = 0; j < K / 512; j++) {
        const int g = gl + 8 * (wave + 8 * j);
        const size_t o = plane_unit(nr, g, K);
        *(f16x8 *)(P.wh + o) = *(const f16x8 *)(rh + 8 * g);
        *(f16x8 *)(P.wl + o) = *(const f16x8 *)(rl + 8 * g);
    }
}


// ---------------------------------------------------------------------------
// The integer form. A q8_0, iq4_xs, q5_K or q6_K weight is s v (- m for q5_K), with v an integer
// of magnitude at most 127 (exact in f16), s the scale of its 32 (q8_0, iq4_xs, q5_K) or 16 (q6_K)
// elements and m the min of its 32, and a 32-k chunk of the GEMM is one 32-element sub-block. So
// a chunk's products are sum_k (xh + xl) v on the matrix cores, two products per pair instead of
// gemm3's three and no weight lo plane, and the scale joins in fp32: acc += s T, one s per weight
// row and chunk (SUB = 32) or k-step of 16 (SUB = 16); the min as acc -= m S with S = sum_k
// (xh + xl) over the block, which xprep writes per row and block. The x planes are gemm3's.
//
// wprep_int: thread (row n, sub-block b) writes the sub-block's 32 values as f16 into the plane's
// chunk order (plane_unit), its scales into wd[n / 128][b][32 / SUB][n % 128] and, with mins, its
// min into wm[n / 128][b][n % 128].
template <int K, int SUB>
__global__ __launch_bounds__(256) void wprep_int_kernel(const GemmWeightParams P) {
    constexpr int NB = K / 32, NS = 32 / SUB;
    const int idx = blockIdx.x * 256 + threadIdx.x, n = idx / NB, b = idx % NB;  // sub-block fastest
    const int in2 = P.n_seg > 2 && n >= P.seg[2].row0, in1 = !in2 && P.n_seg > 1 && n >= P.seg[1].row0;
    const MatvecSeg S = in2 ? P.seg[2] : in1 ? P.seg[1] : P.seg[0];
    _Float16 v[32];
    float sc[2], mn;
    deq32_int(S.type, S.w + (size_t)(n - S.row0) * S.row_bytes, b, v, sc, mn);
#pragma unroll
    for (int j = 0; j < 4; j++) {
        f16x8 u;
#pragma unroll
        for (int e = 0; e < 8; e++) u[e] = v[8 * j + e];
        *(f16x8 *)(P.wh + plane_unit(n, 4 * b + j, K)) = u;
    }
    float *const d = P.wd + (((size_t)(n >> 7) * NB + b) * NS) * GEMM_TILE + (n & 127);
    d[0] = sc[0];  // SUB = 32: the two halves' scales are one
    if constexpr (NS == 2) d[GEMM_TILE] = sc[1];
    if (P.imin) P.wm[((size_t)(n >> 7) * NB + b) * GEMM_TILE + (n & 127)] = mn;
}

// ---------------------------------------------------------------------------
// xprep: one 512-thread workgroup per 8 activation rows t0 .. t0 + 7 (rows T .. T_pad - 1 are
// written as zeros). Lane (row rho = lane & 7, group lane gl = lane >> 3) of wave w holds the
// row's 8-element groups gl + 8 (w + 8 j) in registers, read once. The RMSNorm is computed as
// matvec_kernel computes it (double sum of squares, float scale, xn = (x * scale) * g; the sum
// runs in another order), then the row's exponent from the largest |xn|, then the hi/lo planes.
// In the planes' chunk order the 8 rows' units of one group are one 128-byte line, so every
// store instruction writes 8 whole lines.
template <int K>
__global__ __launch_bounds__(512) void xprep_kernel(const GemmActParams P) {
    constexpr int GPJ = K / 8 / 64;  // groups per lane
    __shared__ double red_ss[8][8];  // [wave][row]
    __shared__ float red_mx[8][8];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, rho = lane & 7, gl = lane >> 3;
    const int t = 8 * blockIdx.x + rho;
    const bool live = t < P.T;
    const float *xt = P.x + (size_t)(live ? t : 0) * P.x_stride;
    float v[GPJ][8];
#pragma unroll
    for (int j = 0; j < GPJ; j++) {
        const int g = gl + 8 * (wave + 8 * j);
        const f32x4 a = *(const f32x4 *)(xt + 8 * g), b = *(const f32x4 *)(xt + 8 * g + 4);
        v[j][0] = a[0], v[j][1] = a[1], v[j][2] = a[2], v[j][3] = a[3];
        v[j][4] = b[0], v[j][5] = b[1], v[j][6] = b[2], v[j][7] = b[3];
    }
    if (P.norm_w) {
        double ss = 0;
#pragma unroll
        for (int j = 0; j < GPJ; j++)
#pragma unroll
            for (int e = 0; e < 8; e++) ss += (double)v[j][e] * v[j][e];
#pragma unroll
        for (int m = 8; m < 64; m <<= 1) ss += __shfl_xor(ss, m, 64);
        if (gl == 0) red_ss[wave][rho] = ss;
        __syncthreads();
        ss = 0;
#pragma unroll
        for (int w = 0; w < 8; w++) ss += red_ss[w][rho];
        const float scale = 1.0f / sqrtf((float)(ss / K) + P.eps);
#pragma unroll
        for (int j = 0; j < GPJ; j++) {
            const int g = gl + 8 * (wave + 8 * j);
            const f32x4 a = *(const f32x4 *)(P.norm_w + 8 * g), b = *(const f32x4 *)(P.norm_w + 8 * g + 4);
            const float gg[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
#pragma unroll
            for (int e = 0; e < 8; e++) v[j][e] = v[j][e] * scale * gg[e];
        }
    }
    float mx = 0.f;
#pragma unroll
    for (int j = 0; j < GPJ; j++)
#pragma unroll
        for (int e = 0; e < 8; e++) mx = fmaxf(mx, fabsf(v[j][e]));
#pragma unroll
    for (int m = 8; m < 64; m <<= 1) mx = fmaxf(mx, __shfl_xor(mx, m, 64));
    if (gl == 0) red_mx[wave][rho] = mx;
    __syncthreads();
    mx = red_mx[0][rho];
#pragma unroll
    for (int w = 1; w < 8; w++) mx = fmaxf(mx, red_mx[w][rho]);
    const int e = live ? row_exp(mx) : 0;
#pragma unroll
    for (int j = 0; j < GPJ; j++) {
        f16x8 h8, l8;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            _Float16 h, l;
            split_store(live ? v[j][i] : 0.f, e, &h, &l);
            h8[i] = h;
            l8[i] = l;
        }
        const size_t o = plane_unit(t, gl + 8 * (wave + 8 * j), K);
        *(f16x8 *)(P.xh + o) = h8;
        *(f16x8 *)(P.xl + o) = l8;
        if (P.xs) {  // the block sums: a 32-element block's 4 groups are lanes gl ^ 1, ^ 2, ^ 3
            float gs = 0.f;
#pragma unroll
            for (int i = 0; i < 8; i++) gs += (float)h8[i] + (float)l8[i];
            gs += __shfl_xor(gs, 8, 64);
            gs += __shfl_xor(gs, 16, 64);
            const int b = (gl + 8 * (wave + 8 * j)) >> 2;
            if ((gl & 3) == 0) P.xs[((size_t)(t >> 7) * (K / 32) + b) * GEMM_TILE + (t & 127)] = gs;
        }
    }
    if (tid < 8) P.eexp[t] = e;  // lanes 0..7 of wave 0: rows rho = tid
}

// ---------------------------------------------------------------------------
// gemm3: workgroup tile 128 weight rows (n) x 128 tokens (t), 4 waves in a 2 x 2 grid of
// 64 x 64, each four 32 x 32 MFMA blocks. K runs in chunks of 32 (two MFMA k-steps of 16). A
// chunk of each operand (hi and lo planes, 128 rows x 32 k) goes into LDS in the MFMA operand
// order: per plane, 32-row block and k-step, 1 KiB in which lane l's 16 bytes hold row l & 31,
// k 8 (l >> 5) .. +7 (the same order for the weight rows, operand A, and for the tokens,
// operand B), so every fragment read is one conflict-free ds_read_b128 per lane. The planes
// are stored in that order already (plane_unit), so the chunk's copy into LDS is contiguous on
// both sides. While a chunk is computed from LDS, the next one is stored there and the two
// after it are in flight.
constexpr int GM_TILE = GEMM_TILE, GM_KC = 32, GM_THREADS = 256;
constexpr int GM_PLANE_CHUNK = GM_TILE * GM_KC * 2;  // bytes of one plane's chunk (8 KiB)

__global__ __launch_bounds__(GM_THREADS, 2) void gemm3_kernel(const GemmParams P) {
    // [buffer][operand (A = weights, B = tokens)][plane (hi, lo)]: 8 KiB each
    __shared__ __align__(16) uint8_t lds[2][2][2][GM_PLANE_CHUNK];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wn = wave & 1, wt = wave >> 1;
    // Tile of this workgroup. The hardware deals workgroups to the 8 XCDs in id order (id % 8),
    // each XCD with its own L2: XCD x takes the stripe of weight-row tiles [x w, x w + w) and
    // walks it token-tile-major, so the workgroups resident on one XCD share their weight and
    // token chunks in that L2 (a row-major deal spreads them over the whole output grid).
    const int NT = P.N / GM_TILE, id = blockIdx.x;
    int nt, tt;
    if (NT % 8 == 0) {
        const int w = NT / 8, j = id >> 3;
        nt = (id & 7) * w + j % w;
        tt = j / w;
    } else {
        nt = id % NT;
        tt = id / NT;
    }
    const int n0 = nt * GM_TILE, t0 = tt * GM_TILE;
    const int K = P.K;
    // global -> LDS: a plane's chunk is 512 contiguous units of 16 bytes already in the LDS
    // order (plane_unit); thread tid copies units tid and tid + 256, so a wave's load and its
    // LDS store each cover 1 KiB contiguously (whole cache lines, no bank conflicts)
    const _Float16 *srcA[2] = {P.wh + (size_t)n0 * K, P.wl + (size_t)n0 * K};
    const _Float16 *srcB[2] = {P.xh + (size_t)t0 * K, P.xl + (size_t)t0 * K};
    int goff[2], loff[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int u = tid + GM_THREADS * i;
        goff[i] = 8 * u;
        loff[i] = 16 * u;
    }
    // two register sets of loaded chunks, so two chunks are in flight while one is computed
    u32x4 ga[2][2][2], gb[2][2][2];  // [operand][plane][unit]
    auto gload = [&](u32x4 (&g)[2][2][2], int kc) {
#pragma unroll
        for (int p = 0; p < 2; p++)
#pragma unroll
            for (int i = 0; i < 2; i++) {
                g[0][p][i] = *(const u32x4 *)(srcA[p] + goff[i] + (size_t)kc * GM_TILE);
                g[1][p][i] = *(const u32x4 *)(srcB[p] + goff[i] + (size_t)kc * GM_TILE);
            }
    };
    auto lstore = [&](const u32x4 (&g)[2][2][2], int buf) {
#pragma unroll
        for (int o = 0; o < 2; o++)
#pragma unroll
            for (int p = 0; p < 2; p++)
#pragma unroll
                for (int i = 0; i < 2; i++) *(u32x4 *)(lds[buf][o][p] + loff[i]) = g[o][p][i];
    };
    f32x16 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++) acc[a][b] = f32x16{};
    auto compute = [&](int buf) {
#pragma unroll
        for (int s = 0; s < 2; s++) {  // k-steps of 16
            f16x8 ah[2], al[2], bh[2], bl[2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int ob = ((2 * wn + j) * 2 + s) * 1024 + lane * 16;  // A block 2wn + j
                const int tb = ((2 * wt + j) * 2 + s) * 1024 + lane * 16;  // B block 2wt + j
                ah[j] = *(const f16x8 *)(lds[buf][0][0] + ob);
                al[j] = *(const f16x8 *)(lds[buf][0][1] + ob);
                bh[j] = *(const f16x8 *)(lds[buf][1][0] + tb);
                bl[j] = *(const f16x8 *)(lds[buf][1][1] + tb);
            }
#pragma unroll
            for (int a = 0; a < 2; a++)
#pragma unroll
                for (int b = 0; b < 2; b++) {
                    acc[a][b] = mfma32_f16(ah[a], bh[b], acc[a][b]);
                    acc[a][b] = mfma32_f16(ah[a], bl[b], acc[a][b]);
                    acc[a][b] = mfma32_f16(al[a], bh[b], acc[a][b]);
                }
        }
    };
    // chunk c lives in LDS buffer c & 1; chunks c + 1 and c + 2 are in registers (set gb holds
    // the odd chunks, ga the even ones) while chunk c is computed. K is a multiple of 64, so
    // the chunk count is even. The barriers order LDS only (lds_barrier): a full __syncthreads
    // would also wait for the chunk loads in flight.
    const int n_chunks = K / GM_KC;
    gload(ga, 0);
    gload(gb, GM_KC);
    lstore(ga, 0);
    gload(ga, 2 * GM_KC);
    lds_barrier();
    // Loads and stores are unconditional (past the last chunk they re-read it and store it into
    // a buffer no one reads again), so the compiler's wait counts are static: a store waits for
    // its own register set only, with the other set's loads still in flight.
    const int last = (n_chunks - 1) * GM_KC;
    for (int c = 0; c < n_chunks; c += 2) {
        // chunk c + 1 into buffer 1 (its chunk c - 1 was finished before the last barrier)
        lstore(gb, 1);
        gload(gb, min((c + 3) * GM_KC, last));
        compute(0);
        lds_barrier();
        lstore(ga, 0);
        gload(ga, min((c + 4) * GM_KC, last));
        compute(1);
        lds_barrier();
    }
    // epilogue: block (a, b) element e is weight row n0 + 64 wn + 32 a + 8 (e >> 2) + 4 (lane >> 5) + (e & 3)
    // and token t0 + 64 wt + 32 b + (lane & 31)
#pragma unroll
    for (int b = 0; b < 2; b++) {
        const int t = t0 + 64 * wt + 32 * b + (lane & 31);
        if (t >= P.T) continue;
        const int et = P.eexp[t];
        float *yt = P.y + (size_t)t * P.y_stride;
        // the exponents and the residual (add) first: a load after a store to y that may alias it
        // waits for that store
        int4 f[2][4];
        f32x4 yin[2][4];
#pragma unroll
        for (int a = 0; a < 2; a++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int n = n0 + 64 * wn + 32 * a + 8 * q + 4 * (lane >> 5);
                f[a][q] = *(const int4 *)(P.fexp + n);
                if (P.add) yin[a][q] = *(const f32x4 *)(yt + n);
            }
#pragma unroll
        for (int a = 0; a < 2; a++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int n = n0 + 64 * wn + 32 * a + 8 * q + 4 * (lane >> 5);
                f32x4 v = {__builtin_amdgcn_ldexpf(acc[a][b][4 * q], et + f[a][q].x),
                           __builtin_amdgcn_ldexpf(acc[a][b][4 * q + 1], et + f[a][q].y),
                           __builtin_amdgcn_ldexpf(acc[a][b][4 * q + 2], et + f[a][q].z),
                           __builtin_amdgcn_ldexpf(acc[a][b][4 * q + 3], et + f[a][q].w)};
                if (P.add) v += yin[a][q];
                *(f32x4 *)(yt + n) = v;
            }
    }
}


// gemm_int: gemm3's tiles, deal and LDS order with the tokens as operand A and the weights'
// values as operand B, so that an MFMA output lane holds one weight row (16 tokens of it) and
// takes one scale per chunk (SUB = 32) or k-step (SUB = 16). The chunks go straight from memory
// into LDS (global_load_lds_dwordx4: each wave-wide load writes 1 KiB, lane l's 16 bytes at
// l * 16 from the wave's LDS address), three stages deep: while chunk c is computed, chunks c + 1
// and c + 2 are in flight, and no register holds them. A chunk's 128 (SUB = 32) or 256 scales
// ride along (lanes 0-7 or 0-15 of each wave load 128 or 256 bytes), and with mins (MIN) the
// chunk's block sums of its 128 tokens and mins of its 128 rows (lanes 0-7 again, two loads).
// Each step makes the products T = sum (xh + xl) v of one chunk (SUB = 32: four independent
// chains of four MFMAs) or k-step (SUB = 16: chains of two), and scales the step before's
// (acc += s T) in between, so that those FMAs run beside MFMAs that do not feed them (two
// register sets for T take turns). Against one chunk's MFMAs and FMAs in the same step, q8_0:
// 4000 tokens through 49 Flint blocks 23.2 against 24.0 ms.
template <int SUB>
constexpr int gq_scales() { return (32 / SUB) * GM_TILE; }  // a chunk's scales, per row tile
template <int SUB>
constexpr int gq_stage() { return 3 * GM_PLANE_CHUNK + gq_scales<SUB>() * 4; }  // x hi, x lo, values, scales

template <int SUB, bool MIN>
__global__ __launch_bounds__(GM_THREADS, 2) void gemm_int_kernel(const GemmParams P) {
    constexpr int SCB = gq_scales<SUB>(), SCL = SCB / 16;  // scales per chunk; lanes that load them
    constexpr int STAGE = gq_stage<SUB>(), LOADS = MIN ? 9 : 7;  // direct loads per wave per chunk
    __shared__ __align__(16) uint8_t lds[3][STAGE + (MIN ? 2 * GM_TILE * 4 : 0)];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave & 1, wt = wave >> 1;
    const int NT = P.N / GM_TILE, id = blockIdx.x;
    int nt, tt;
    if (NT % 8 == 0) {  // the XCD deal of gemm3
        const int w = NT / 8, j = id >> 3;
        nt = (id & 7) * w + j % w;
        tt = j / w;
    } else {
        nt = id % NT;
        tt = id / NT;
    }
    const int n0 = nt * GM_TILE, t0 = tt * GM_TILE;
    const int K = P.K;
    // this lane's units tid and tid + 256 of each plane's chunk; its 16 bytes of the scales
    const _Float16 *src[3] = {P.xh + (size_t)t0 * K + 8 * tid, P.xl + (size_t)t0 * K + 8 * tid,
                              P.wh + (size_t)n0 * K + 8 * tid};
    const float *srcd = P.wd + (size_t)nt * (K / GM_KC) * SCB + SCB / 4 * wave + 4 * (lane & (SCL - 1));
    const size_t mo = 32 * wave + 4 * (lane & 7);  // this lane's 16 bytes of the block sums and mins
    const float *srcs = MIN ? P.xs + (size_t)tt * (K / GM_KC) * GM_TILE + mo : nullptr;
    const float *srcm = MIN ? P.wm + (size_t)nt * (K / GM_KC) * GM_TILE + mo : nullptr;
    const int n_chunks = K / GM_KC;
    auto issue = [&](int c, int st) {  // chunk c into stage st
        uint8_t *const base = lds[st];
#pragma unroll
        for (int p = 0; p < 3; p++)
#pragma unroll
            for (int i = 0; i < 2; i++)
                __builtin_amdgcn_global_load_lds(src[p] + (size_t)c * GM_TILE * GM_KC + 2048 * i,
                                                 (lds_void *)(base + p * GM_PLANE_CHUNK + (256 * i + 64 * wave) * 16),
                                                 16, 0, 0);
        if (lane < SCL)
            __builtin_amdgcn_global_load_lds(srcd + (size_t)c * SCB,
                                             (lds_void *)(base + 3 * GM_PLANE_CHUNK + SCB * wave), 16, 0, 0);
        if constexpr (MIN) {
            if (lane < 8) {
                __builtin_amdgcn_global_load_lds(srcs + (size_t)c * GM_TILE, (lds_void *)(base + STAGE + 128 * wave), 16, 0, 0);
                __builtin_amdgcn_global_load_lds(srcm + (size_t)c * GM_TILE,
                                                 (lds_void *)(base + STAGE + 4 * GM_TILE + 128 * wave), 16, 0, 0);
            }
        }
    };
    f32x16 acc[2][2];  // [token block][weight block]
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++) acc[a][b] = f32x16{};
    f32x16 TA[2][2], TB[2][2];  // the products of the even / odd chunks
    float dA[2], dB[2];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++) TB[a][b] = f32x16{};
    dB[0] = dB[1] = 0.f;
    // one step: the products of k-steps s0 .. s1 - 1 of the chunk in stage st into T, the step
    // before's products Tp scaled into acc, this step's scales into dn
    auto step = [&](int st, int s0, int s1, f32x16 (&T)[2][2], float (&dn)[2], const f32x16 (&Tp)[2][2],
                    const float (&dp)[2]) {
        const uint8_t *const base = lds[st];
#pragma unroll
        for (int s = s0; s < s1; s++) {
            f16x8 xh[2], xl[2], wq[2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int tb = ((2 * wt + j) * 2 + s) * 1024 + lane * 16;
                const int ob = ((2 * wn + j) * 2 + s) * 1024 + lane * 16;
                xh[j] = *(const f16x8 *)(base + tb);
                xl[j] = *(const f16x8 *)(base + GM_PLANE_CHUNK + tb);
                wq[j] = *(const f16x8 *)(base + 2 * GM_PLANE_CHUNK + ob);
            }
#pragma unroll
            for (int a = 0; a < 2; a++)
#pragma unroll
                for (int b = 0; b < 2; b++) T[a][b] = mfma32_f16(xh[a], wq[b], s == s0 ? f32x16{} : T[a][b]);
#pragma unroll
            for (int a = 0; a < 2; a++)
#pragma unroll
                for (int b = 0; b < 2; b++) T[a][b] = mfma32_f16(xl[a], wq[b], T[a][b]);
            if (s == s0) {
#pragma unroll
                for (int b = 0; b < 2; b++)
#pragma unroll
                    for (int a = 0; a < 2; a++)
#pragma unroll
                        for (int e = 0; e < 16; e++) acc[a][b][e] = fmaf(dp[b], Tp[a][b][e], acc[a][b][e]);
            }
        }
        if (MIN && s0 == 0) {  // the chunk's mins: acc -= m S, S of element e's token
            const float *const sl = (const float *)(base + STAGE), *const ml = sl + GM_TILE;
#pragma unroll
            for (int a = 0; a < 2; a++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const f32x4 S4 = *(const f32x4 *)(sl + 64 * wt + 32 * a + 8 * q + 4 * (lane >> 5));
#pragma unroll
                    for (int b = 0; b < 2; b++) {
                        const float m = ml[64 * wn + 32 * b + (lane & 31)];
#pragma unroll
                        for (int i = 0; i < 4; i++) acc[a][b][4 * q + i] = fmaf(-m, S4[i], acc[a][b][4 * q + i]);
                    }
                }
        }
        const float *const sc = (const float *)(base + 3 * GM_PLANE_CHUNK) + (SUB == 16 ? GM_TILE * s0 : 0);
#pragma unroll
        for (int b = 0; b < 2; b++) dn[b] = sc[64 * wn + 32 * b + (lane & 31)];
    };
    // Chunk c lives in stage c % 3. Every wave issues the same LOADS loads per chunk (past the
    // last chunk it re-reads the last one into a stage no one reads again), so "chunk c has
    // landed" is vmcnt(LOADS) with chunk c + 1 still in flight; the barrier then makes every
    // wave's part of it visible, and it also ends every wave's reads of stage (c - 1) % 3, which
    // chunk c + 2 overwrites after it. No fence: a workgroup-scope fence would wait for every load
    // in flight (vmcnt(0)); the empty asm keeps the compiler from moving LDS reads across the
    // barrier, and the chunk before's reads have all returned (their registers fed its MFMAs).
    auto sync = [&](int c) {
        wait_vmcnt<LOADS>();
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        const int st = c % 3;
        issue(min(c + 2, n_chunks - 1), st == 0 ? 2 : st - 1);
        return st;
    };
    issue(0, 0);
    issue(1, 1);
    if constexpr (SUB == 32) {
        for (int c = 0; c < n_chunks; c += 2) {  // K is a multiple of 64: the chunk count is even
            step(sync(c), 0, 2, TA, dA, TB, dB);
            step(sync(c + 1), 0, 2, TB, dB, TA, dA);
        }
    } else {
        for (int c = 0; c < n_chunks; c++) {
            const int st = sync(c);
            step(st, 0, 1, TA, dA, TB, dB);
            step(st, 1, 2, TB, dB, TA, dA);
        }
    }
#pragma unroll
    for (int b = 0; b < 2; b++)
#pragma unroll
        for (int a = 0; a < 2; a++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[a][b][e] = fmaf(dB[b], TB[a][b][e], acc[a][b][e]);
    wait_vmcnt<0>();  // the re-read past the last chunk lands before the workgroup's LDS goes
    // epilogue: block (a, b) element e is token t0 + 64 wt + 32 a + 8 (e >> 2) + 4 (lane >> 5) + (e & 3)
    // and weight row n0 + 64 wn + 32 b + (lane & 31): a store instruction writes 32 consecutive
    // floats of each of two token rows. Token block a by token block a, its row exponents and
    // its residual (add) are all read before its first store (rows past T re-read row T - 1): a
    // load after a store that may alias it waits for the store, so loads between the stores cost
    // a round trip each (36 us per o launch at T = 4000).
    auto row = [&](int a, int e) { return min(t0 + 64 * wt + 32 * a + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3), P.T - 1); };
    float *const y0 = P.y + n0 + 64 * wn + (lane & 31);
#pragma unroll
    for (int a = 0; a < 2; a++) {
        int ex[16];
        float yin[16][2];
#pragma unroll
        for (int e = 0; e < 16; e++) ex[e] = P.eexp[row(a, e)];
        if (P.add) {
#pragma unroll
            for (int e = 0; e < 16; e++)
#pragma unroll
                for (int b = 0; b < 2; b++) yin[e][b] = y0[(size_t)row(a, e) * P.y_stride + 32 * b];
        }
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int t = t0 + 64 * wt + 32 * a + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
            if (t >= P.T) continue;
#pragma unroll
            for (int b = 0; b < 2; b++) {
                float v = __builtin_amdgcn_ldexpf(acc[a][b][e], ex[e]);
                if (P.add) v += yin[e][b];
                y0[(size_t)t * P.y_stride + 32 * b] = v;
            }
        }
    }
}

hipError_t launch_proj_gemm(const GemmWeightParams &W, const GemmActParams &X, const GemmParams &G, bool prep_weights,
                            hipStream_t stream) {
    // the planes' chunk order and the GEMM's tiles need whole 128-row tiles of both operands
    if (G.N % GM_TILE != 0 || X.T_pad % GM_TILE != 0 || (G.K != 2048 && G.K != 4096)) return hipErrorInvalidValue;
    if (G.isub == 32 || G.isub == 16) {
        const bool s32 = G.isub == 32;
        if (prep_weights) {
            void (*wk)(GemmWeightParams) = G.K == 2048 ? (s32 ? wprep_int_kernel<2048, 32> : wprep_int_kernel<2048, 16>)
                                                       : (s32 ? wprep_int_kernel<4096, 32> : wprep_int_kernel<4096, 16>);
            hipLaunchKernelGGL(wk, dim3(G.N * (G.K / 32) / 256), dim3(256), 0, stream, W);
        }
        if (X.T_pad > 0) {
            if (G.K == 2048)
                hipLaunchKernelGGL(xprep_kernel<2048>, dim3(X.T_pad / 8), dim3(512), 0, stream, X);
            else
                hipLaunchKernelGGL(xprep_kernel<4096>, dim3(X.T_pad / 8), dim3(512), 0, stream, X);
            void (*gk)(GemmParams) = G.imin ? (s32 ? gemm_int_kernel<32, true> : gemm_int_kernel<16, true>)
                                            : (s32 ? gemm_int_kernel<32, false> : gemm_int_kernel<16, false>);
            hipLaunchKernelGGL(gk, dim3(G.N / GM_TILE * (X.T_pad / GM_TILE)), dim3(GM_THREADS), 0, stream, G);
        }
        return hipGetLastError();
    }
    if (G.K == 2048) {
        if (prep_weights) hipLaunchKernelGGL(wprep_kernel<2048>, dim3(G.N / 8), dim3(512), 0, stream, W);
        if (X.T_pad > 0) hipLaunchKernelGGL(xprep_kernel<2048>, dim3(X.T_pad / 8), dim3(512), 0, stream, X);
    } else {
        if (prep_weights) hipLaunchKernelGGL(wprep_kernel<4096>, dim3(G.N / 8), dim3(512), 0, stream, W);
        if (X.T_pad > 0) hipLaunchKernelGGL(xprep_kernel<4096>, dim3(X.T_pad / 8), dim3(512), 0, stream, X);
    }
    if (X.T_pad > 0)
        hipLaunchKernelGGL(gemm3_kernel, dim3(G.N / GM_TILE * (X.T_pad / GM_TILE)), dim3(GM_THREADS), 0, stream, G);
    return hipGetLastError();
}

}  // namespace flint
