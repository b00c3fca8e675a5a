// Attention projections in the engine's GGUF weight formats, for gfx950:
//   * get_rows_kernel: rows dequantised to fp32 (Engine::debug_get_row,
//     /root/reference/src/engine.mm:1370-1383, kernel k_get_row, fused.metal:589-600; and
//     the prefill's embedding, k_embed_rows, prefill.metal:272, engine.mm:1067-1069);
//   * matvec_kernel: y = W x with 2048- or 4096-element rows, optionally on RMSNorm(x) * g
//     (the q/k/v projections, engine.mm:728-732) or added to y (o_proj with the residual,
//     engine.mm:811).
//
// Formats: ggml's block layouts (/root/reference/third_party/ggml/ggml-common.h), type ids
// from /root/reference/src/gguf.h:14-19. Every row is cut into 32-element sub-blocks, the
// unit all formats share: a q8_0 block, a half of a q5_K/iq4_xs 64-element pair, two q6_K
// 16-element groups. Lane l of a wave owns sub-blocks l, l + 64, ..., so the 32 x values it
// multiplies stay in its registers. Dequantisation repeats ggml's float operations in order
// with contraction off, so get_row is bit-identical to dequantize_row_*
// (/root/reference/src/ref/dequant_gen.c).
//
// Matvec layout (HBM-bound on the weight bytes): a wave takes R consecutive rows. It requests
// their bytes at kernel start (16-byte loads, coalesced) while the workgroup reads x once
// into LDS (normalised there when the RMSNorm is fused). The rows' bytes then go into an
// LDS area of the wave's own; each lane reads the bytes of its sub-block from LDS at the
// alignment the format gives (q8_0 and q6_K blocks are only 2-byte aligned: q8_0 as aligned
// words realigned in registers), decodes 32 weights and accumulates their products with x in
// fp32; a wave-wide sum gives y[row].
// f32/f16/bf16 rows are read straight from HBM (64- or 128-byte sub-blocks, aligned).
#include <hip/hip_runtime.h>

#include "common.h"
#include "dequant.h"
#include "flint_attn_internal.h"

namespace flint {



// ---------------------------------------------------------------------------
// get_rows: workgroup (c, i) dequantises sub-blocks 64c .. 64c+63 of row rows[i] into
// out + i * out_stride, so one launch serves every token of a prefill's embedding (the
// reference's k_embed_rows, prefill.metal:272). The row's bytes start on a block boundary;
// they are staged through LDS with 2-byte loads (any row alignment the block size allows).
constexpr int GR_STAGE = 64 * 32 * 4;  // bytes of 64 f32 sub-blocks, the largest chunk
__global__ __launch_bounds__(64) void get_rows_kernel(const RowsParams P) {
    __shared__ __align__(16) uint8_t stage[GR_STAGE];
    const int lane = threadIdx.x, c = blockIdx.x, i = blockIdx.y;
    const int type = P.type, n_sub = P.n_sub;
    const uint8_t *__restrict__ row = P.w + (size_t)P.rows[i] * (size_t)P.row_bytes;
    float *__restrict__ out = P.out + (size_t)i * (size_t)P.out_stride;
    const int sub0 = 64 * c, nsub = min(64, n_sub - sub0);
    const int be = w_block_elems(type), bb = w_block_bytes(type);
    const size_t off = (size_t)sub0 * 32 / be * bb;
    const int nbytes = nsub * 32 / be * bb;  // chunks are whole blocks (64 is a multiple of 8)
    const uint16_t *src = (const uint16_t *)(row + off);
    uint16_t *dst = (uint16_t *)stage;
    for (int j = lane; j < nbytes / 2; j += 64) dst[j] = src[j];
    __syncthreads();
    if (lane < nsub) {
        float w[32];
        deq32(type, stage, lane, w);
        f32x4 *o = (f32x4 *)(out + 32 * (size_t)(sub0 + lane));
#pragma unroll
        for (int k = 0; k < 8; k++) o[k] = f32x4{w[4 * k], w[4 * k + 1], w[4 * k + 2], w[4 * k + 3]};
    }
}

// ---------------------------------------------------------------------------
// matvec: a workgroup of MV_WAVES waves serves MV_WAVES * R consecutive rows of one token.
// x (times the RMSNorm gains, when norm_w is given; the norm's scale multiplies the row sums)
// is read from HBM once per workgroup into LDS; each wave then takes R rows, whose bytes it
// requested at kernel start, and reads its lanes' 32-element slices of x from LDS.
constexpr int MV_WAVES = 4;

// x in LDS: float4 column c (elements 4c .. 4c+3) of sub-block s at s * 32 + 4 (c ^ ((s >> 1) & 7)).
// Lane l reads its own sub-block's eight columns one instruction at a time; unswizzled, the
// 64 lanes' addresses 128 bytes apart fell on two groups of 4 banks (32-way conflicts), and
// with the swizzle any 8 consecutive lanes read 8 different columns.
__device__ inline int xs_index(int e) {
    const int s = e >> 5, c = (e >> 2) & 7;
    return s * 32 + 4 * (c ^ ((s >> 1) & 7)) + (e & 3);
}

// Sum over the 64 lanes in double, on VALU lane permutes (each 32-bit half moved by DPP within
// rows of 16, then v_permlane16/32_swap across rows): no LDS round trips (a __shfl_xor chain
// costs six dependent ds_bpermute pairs).
template <int CTRL>
__device__ inline double dpp_f64(double v) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, 0xf, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, 0xf, 0xf, false);
    return __builtin_bit_cast(double, ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}
__device__ inline double wave_sum_f64(double v) {
    v += dpp_f64<DPP_ROR8>(v);
    v += dpp_f64<DPP_ROR4>(v);
    v += dpp_f64<DPP_ROR2>(v);
    v += dpp_f64<DPP_ROR1>(v);  // every lane of a row of 16 holds the row's sum
    uint64_t b = __builtin_bit_cast(uint64_t, v);
    const auto l16 = __builtin_amdgcn_permlane16_swap((uint32_t)b, (uint32_t)b, false, false);
    const auto h16 = __builtin_amdgcn_permlane16_swap((uint32_t)(b >> 32), (uint32_t)(b >> 32), false, false);
    v = __builtin_bit_cast(double, ((uint64_t)h16[0] << 32) | l16[0]) + __builtin_bit_cast(double, ((uint64_t)h16[1] << 32) | l16[1]);
    b = __builtin_bit_cast(uint64_t, v);
    const auto l32 = __builtin_amdgcn_permlane32_swap((uint32_t)b, (uint32_t)b, false, false);
    const auto h32 = __builtin_amdgcn_permlane32_swap((uint32_t)(b >> 32), (uint32_t)(b >> 32), false, false);
    return __builtin_bit_cast(double, ((uint64_t)h32[0] << 32) | l32[0]) + __builtin_bit_cast(double, ((uint64_t)h32[1] << 32) | l32[1]);
}

template <int K, int R>
__global__ __launch_bounds__(64 * MV_WAVES) void matvec_kernel(const MatvecParams P) {
    constexpr int SUBS = K / 32 / 64;               // sub-blocks per lane
    constexpr int QBYTES = K / 32 * 34;             // largest quantised row (q8_0)
    constexpr int UNITS = (QBYTES / 16 + 63) / 64;  // 16-byte loads per lane for it
    constexpr int XPT = K / (64 * MV_WAVES);        // x elements per thread in the shared pass
    __shared__ __align__(16) float xs[K];           // the (normalised) x row
    constexpr int QROW = (QBYTES + 4 + 15) / 16 * 16;  // a staged row, + 4 bytes read past a q8_0 row's end
    __shared__ __align__(16) uint8_t stage[MV_WAVES][R][QROW];
    __shared__ double part[MV_WAVES];
    // wave index made scalar: the row segment, its type and its row pointer are then known
    // to be wave-uniform (scalar branches for the format, scalar load bases)
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int row0 = (blockIdx.y * MV_WAVES + wave) * R;  // R rows, all in one segment
    // the segment by selection among constant-index reads: the kernel arguments arrive in one
    // batch of scalar loads (a search loop over P.seg costs a memory round trip per step)
    const MatvecSeg s0 = P.seg[0], s1 = P.seg[1], s2 = P.seg[2];
    const int n_seg = P.n_seg, add = P.add;
    const long long x_stride = P.x_stride, y_stride = P.y_stride;
    const float *const x = P.x, *const norm_w = P.norm_w;
    float *const y = P.y;
    const float eps = P.eps;
    pin_sgpr(s0.w), pin_sgpr(s0.type), pin_sgpr(s0.row0), pin_sgpr(s0.row_bytes);
    pin_sgpr(s1.w), pin_sgpr(s1.type), pin_sgpr(s1.row0), pin_sgpr(s1.row_bytes);
    pin_sgpr(s2.w), pin_sgpr(s2.type), pin_sgpr(s2.row0), pin_sgpr(s2.row_bytes);
    pin_sgpr(n_seg), pin_sgpr(add), pin_sgpr(x_stride), pin_sgpr(y_stride), pin_sgpr(x), pin_sgpr(norm_w);
    pin_sgpr(y), pin_sgpr(eps);
    __builtin_amdgcn_sched_barrier(0);
    const bool in2 = n_seg > 2 && row0 >= s2.row0, in1 = !in2 && n_seg > 1 && row0 >= s1.row0;
    const MatvecSeg S = in2 ? s2 : in1 ? s1 : s0;
    const uint8_t *wrow = S.w + (size_t)(row0 - S.row0) * S.row_bytes;
    const bool fl = w_is_float(S.type);
    // token blockIdx.x: consecutive workgroups take the same rows for successive tokens,
    // so a batch reads each weight row from HBM about once (the rest hit L2)
    const float *__restrict__ xt = x + (size_t)blockIdx.x * x_stride;
    float *__restrict__ yt = y + (size_t)blockIdx.x * y_stride;

    // x and the gains: XPT consecutive elements per thread, 16-byte loads
    f32x4 xv[XPT / 4], gv[XPT / 4];
#pragma unroll
    for (int k = 0; k < XPT / 4; k++) xv[k] = *(const f32x4 *)(xt + XPT * tid + 4 * k);
    if (norm_w) {
#pragma unroll
        for (int k = 0; k < XPT / 4; k++) gv[k] = *(const f32x4 *)(norm_w + XPT * tid + 4 * k);
    }
    // this wave's rows, as quantised-row units (float rows are read again in the dot loop;
    // the units loaded here are within their rows and go unused). Every lane loads (lanes
    // past the row's end re-read its last unit and do not store it), so the loads are
    // unconditional and the RMSNorm below waits for x and the gains only.
    u32x4 u[R][UNITS];
    const int n_units = S.row_bytes >> 4;
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int k = 0; k < UNITS; k++) {
            const int idx = min(lane + 64 * k, n_units - 1);
            u[r][k] = ((const u32x4 *)(wrow + (size_t)r * S.row_bytes))[idx];
        }
    if (norm_w) {
        // RMSNorm as the CPU reference (ref_model.cpp:45-50): double sum of squares, float
        // scale = 1 / sqrt(ss / K + eps). The scale is one number per token, so W (x scale g) =
        // scale (W (x g)): x g goes to LDS at once and the scale multiplies each row's sum at the
        // end (within a few ulp of scaling x first), so the reduction and its barrier are off the
        // path to the dots (one workgroup barrier instead of two).
        double ss = 0;
#pragma unroll
        for (int k = 0; k < XPT / 4; k++)
#pragma unroll
            for (int e = 0; e < 4; e++) ss += (double)xv[k][e] * xv[k][e];
        ss = wave_sum_f64(ss);
        if (lane == 0) part[wave] = ss;
#pragma unroll
        for (int k = 0; k < XPT / 4; k++)
#pragma unroll
            for (int e = 0; e < 4; e++) xv[k][e] = xv[k][e] * gv[k][e];
    }
#pragma unroll
    for (int k = 0; k < XPT / 4; k++) *(f32x4 *)&xs[xs_index(XPT * tid + 4 * k)] = xv[k];
    __syncthreads();
    float scale = 1.f;
    if (norm_w) {
        double ss = 0;
#pragma unroll
        for (int w = 0; w < MV_WAVES; w++) ss += part[w];
        scale = 1.0f / sqrtf((float)(ss / K) + eps);
    }

    // this lane's slices of x: sub-blocks lane + 64 i
    float xl[SUBS][32];
#pragma unroll
    for (int i = 0; i < SUBS; i++)
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const f32x4 v = *(const f32x4 *)&xs[xs_index(32 * (lane + 64 * i) + 4 * k)];
            xl[i][4 * k] = v[0], xl[i][4 * k + 1] = v[1], xl[i][4 * k + 2] = v[2], xl[i][4 * k + 3] = v[3];
        }
    // The two row sources take separate code paths, so that each dequantiser's reads have a
    // known address space: LDS reads for the staged quantised rows, global reads for float
    // rows (one pointer that may be either compiles to generic flat loads, several times slower).
    float acc[R];
    if (!fl) {
        // every row of the wave staged at once, then the dots
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int k = 0; k < UNITS; k++) {
                const int idx = lane + 64 * k;
                if (idx < n_units) ((u32x4 *)stage[wave][r])[idx] = u[r][k];
            }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (S.type == W_Q8_0) {
            // d * sum(q x) per block. The block (2-byte scale, 32 int8) sits at 34 L bytes, 2-byte
            // aligned: it is read as 9 aligned words and realigned (alignbit); each int8 weight is one
            // sign-extending byte convert (SDWA) and an FMA, in two interleaved chains. (Converting
            // unsigned bytes after a sign flip, with 128 sum(x) subtracted per block, measured slower
            // and loses exactness on blocks of small quantised values.)
#pragma unroll
            for (int r = 0; r < R; r++) acc[r] = 0.f;
#pragma unroll
            for (int i = 0; i < SUBS; i++) {
                const int base = 34 * (lane + 64 * i);
                const bool odd = base & 2;  // the block starts 2 bytes into a word
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const uint32_t *dw = (const uint32_t *)(stage[wave][r] + (base & ~3));
                    uint32_t d[9];
#pragma unroll
                    for (int j = 0; j < 9; j++) d[j] = dw[j];
                    const uint32_t sc = odd ? d[0] >> 16 : d[0] & 0xffffu;
                    float b0 = 0.f, b1 = 0.f;
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        const uint32_t q = odd ? d[j + 1] : __builtin_amdgcn_alignbit(d[j + 1], d[j], 16);
                        b0 = fmaf((float)(int8_t)(q & 0xffu), xl[i][4 * j], b0);
                        b1 = fmaf((float)(int8_t)((q >> 8) & 0xffu), xl[i][4 * j + 1], b1);
                        b0 = fmaf((float)(int8_t)((q >> 16) & 0xffu), xl[i][4 * j + 2], b0);
                        b1 = fmaf((float)(int8_t)(q >> 24), xl[i][4 * j + 3], b1);
                    }
                    acc[r] = fmaf(h2f(sc), b0 + b1, acc[r]);
                }
            }
        } else {
#pragma unroll
            for (int r = 0; r < R; r++) {
                float a = 0.f;
#pragma unroll
                for (int i = 0; i < SUBS; i++) {
                    float w[32];
                    deq32(S.type, stage[wave][r], lane + 64 * i, w);
#pragma unroll
                    for (int e = 0; e < 32; e++) a = fmaf(w[e], xl[i][e], a);
                }
                acc[r] = a;
            }
        }
    } else {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint8_t *__restrict__ src = wrow + (size_t)r * S.row_bytes;
            float a = 0.f;
#pragma unroll
            for (int i = 0; i < SUBS; i++) {
                float w[32];
                deq32(S.type, src, lane + 64 * i, w);
#pragma unroll
                for (int e = 0; e < 32; e++) a = fmaf(w[e], xl[i][e], a);
            }
            acc[r] = a;
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = wave_sum(acc[r]);
    if (lane < R) {
        float a = acc[0];
#pragma unroll
        for (int r = 1; r < R; r++) a = lane == r ? acc[r] : a;
        a *= scale;
        const int row = row0 + lane;
        yt[row] = add ? yt[row] + a : a;
    }
}

hipError_t launch_get_rows(const RowsParams &P, hipStream_t stream) {
    hipLaunchKernelGGL(get_rows_kernel, dim3((P.n_sub + 63) / 64, P.n), dim3(64), 0, stream, P);
    return hipGetLastError();
}

// Rows per wave: 2 for the 2048-element rows (q/k/v: 640 workgroups per token) and 1 for the
// 4096-element rows (o: 512 workgroups, two waves per SIMD: with one, each row's LDS reads and
// FMA chain were exposed); measured best of 1, 2, 4 and 8 for either.
constexpr int MV_ROWS_2048 = 2, MV_ROWS_4096 = 1;

int matvec_row_multiple(int k) { return MV_WAVES * (k == 2048 ? MV_ROWS_2048 : MV_ROWS_4096); }

hipError_t launch_matvec(const MatvecParams &P, int k, hipStream_t stream) {
    const dim3 block(64 * MV_WAVES);
    if (k == 2048)
        hipLaunchKernelGGL((matvec_kernel<2048, MV_ROWS_2048>), dim3(P.n_tok, P.n_rows / matvec_row_multiple(k)),
                           block, 0, stream, P);
    else
        hipLaunchKernelGGL((matvec_kernel<4096, MV_ROWS_4096>), dim3(P.n_tok, P.n_rows / matvec_row_multiple(k)),
                           block, 0, stream, P);
    return hipGetLastError();
}

}  // namespace flint
