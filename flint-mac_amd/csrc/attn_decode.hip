// Fused single-token decode attention for CDNA4 (gfx950).
//
// Replaces the reference's k_attn_dec + k_attn_combine
// (/root/reference/src/metal/fused.metal:254-350, dispatched at
// /root/reference/src/engine.mm:735-766). Same maths: per q head, RMSNorm
// (+ NEOX RoPE when the layer has it) of q and of the current k, the current
// token's K/V rounded to the cache dtype, used in this step and written to
// slot(pos); online softmax over the keys [k_begin, pos) read from the cache
// plus the current token; learned sink in the denominator only; split-K over
// the key range with a log-sum-exp merge.
//
// MI355X design:
//  * One workgroup per (kv head, key split) serves all 8 q heads of the GQA
//    group, so every K/V byte is read from HBM once (the reference re-reads
//    K/V per q head).
//  * KV layout is head-major: K [kvh][slot][128], V transposed [kvh][128][slot],
//    so both MFMA operands are single 16-byte loads straight from HBM.
//  * Scores are S^T = K * Q^T on v_mfma_f32_16x16x32: the 16 MFMA columns carry
//    the 8 heads' q split into hi + lo halves of the 16-bit type, so the scores
//    are fp32-accurate at no extra MFMA cost; P*V uses the same hi/lo trick on P.
//  * A tile is 32 keys: 16 x 16-byte loads per lane (16 KiB per wave) in flight.
//  * Batched entry: blockIdx.x walks a flattened (sequence, split) table so one
//    launch serves many independent sequences (one token each).
#include "common.h"
#include "flint_attn_internal.h"

namespace flint {

// partial record per (seq, head, split): acc[128], m (log2 units), l, 2 pad
constexpr int PART_STRIDE = 132;

template <int DT>
__global__ __launch_bounds__(256) void attn_decode_kernel(const DecodeParams P) {
    typedef KvType<DT> KT;
    typedef typename KT::vec8 vec8;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 15, g = lane >> 4;   // MFMA column (q head x hi/lo) and k-group
    const int hloc = n & 7, hl = n >> 3;      // head within the GQA group, 0 = hi half, 1 = lo half
    const int kvh = blockIdx.y;
    const int h = kvh * GQA + hloc;

    // ---- which sequence / split this block serves ----
    int seq = 0;
    while (seq + 1 < P.n_seq && (int)blockIdx.x >= P.split_prefix[seq + 1]) seq++;
    const int split = blockIdx.x - P.split_prefix[seq];
    const int n_split = P.split_prefix[seq + 1] - P.split_prefix[seq];
    const int pos = P.pos[seq];
    const int k_begin = P.is_swa ? max(pos - (P.window - 1), 0) : 0;
    const int tile_lo = k_begin >> 5, tile_hi = (pos + 31) >> 5;  // tiles holding keys [k_begin, pos)
    const int tps = P.tiles_per_split[seq];
    const int t_begin = tile_lo + split * tps;
    const int t_end = min(t_begin + tps, tile_hi);

    const uint16_t *__restrict__ kc = P.k_cache + (size_t)seq * P.seq_stride + (size_t)kvh * P.n_slots * HEAD_DIM;
    const uint16_t *__restrict__ vc = P.v_cache + (size_t)seq * P.seq_stride + (size_t)kvh * HEAD_DIM * P.n_slots;
    const float *__restrict__ row = P.qkv + (size_t)seq * QKV_DIM;

    // ---- q: RMSNorm (+ RoPE), scaled by log2(e)/sqrt(D); lane holds dims 32c + 8g + e ----
    float q[4][8];
    {
        const float *qr = row + h * HEAD_DIM;
        double ss = 0;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float4 a = *(const float4 *)(qr + 32 * c + 8 * g);
            const float4 b = *(const float4 *)(qr + 32 * c + 8 * g + 4);
            q[c][0] = a.x; q[c][1] = a.y; q[c][2] = a.z; q[c][3] = a.w;
            q[c][4] = b.x; q[c][5] = b.y; q[c][6] = b.z; q[c][7] = b.w;
#pragma unroll
            for (int e = 0; e < 8; e++) ss += (double)q[c][e] * q[c][e];
        }
        ss += __shfl_xor(ss, 16, 64);
        ss += __shfl_xor(ss, 32, 64);
        const float scale = 1.0f / sqrtf((float)(ss / HEAD_DIM) + P.rms_eps);
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int e = 0; e < 8; e++) q[c][e] = q[c][e] * scale * P.q_norm[32 * c + 8 * g + e];
        if (P.has_rope) {
#pragma unroll
            for (int c = 0; c < 2; c++)
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const int i = 32 * c + 8 * g + e;  // pairs with i + 64 = 32(c+2) + 8g + e
                    const float a = (float)pos * P.rope_freq[i];
                    const float cs = cosf(a), sn = sinf(a);
                    const float x0 = q[c][e], x1 = q[c + 2][e];
                    q[c][e] = x0 * cs - x1 * sn;
                    q[c + 2][e] = x0 * sn + x1 * cs;
                }
        }
        const float qs = LOG2E / sqrtf((float)HEAD_DIM);
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int e = 0; e < 8; e++) q[c][e] *= qs;
    }
    vec8 qb[4];  // MFMA B operand: column n = this lane's head, hi or lo half
#pragma unroll
    for (int c = 0; c < 4; c++) {
        u16x8 u;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const uint16_t hi = KT::from_float(q[c][e]);
            const uint16_t lo = KT::from_float(q[c][e] - KT::to_float(hi));
            u[e] = hl ? lo : hi;
        }
        qb[c] = KT::as_vec(u);
    }

    // ---- stream the key tiles of this split: wave w takes tiles t_begin + w, + 4, ... ----
    float m = -1e30f, l = 0.f;  // running max (log2 units, per head) and this lane's partial sum
    f32x4 acc[8];
#pragma unroll
    for (int d = 0; d < 8; d++) acc[d] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int slot_mask = P.slot_mask;

    for (int t = t_begin + wave; t < t_end; t += 4) {
        const int kb = t * 32;
        // K rows: sub-tile st, MFMA row i = n holds key kb + 8(i/4) + 4st + (i%4)
        u16x8 kraw[2][4];
#pragma unroll
        for (int st = 0; st < 2; st++) {
            const int key = kb + 8 * (n >> 2) + 4 * st + (n & 3);
            const uint16_t *kp = kc + (size_t)(key & slot_mask) * HEAD_DIM + 8 * g;
#pragma unroll
            for (int c = 0; c < 4; c++) kraw[st][c] = *(const u16x8 *)(kp + 32 * c);
        }
        // V^T: dim row 16d + n, keys kb + 8g .. kb + 8g + 7
        u16x8 vraw[8];
        const int vslot = (kb + 8 * g) & slot_mask;
#pragma unroll
        for (int d = 0; d < 8; d++) vraw[d] = *(const u16x8 *)(vc + (size_t)(16 * d + n) * P.n_slots + vslot);

        f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < 4; c++) {
            s0 = KT::mfma16(KT::as_vec(kraw[0][c]), qb[c], s0);
            s1 = KT::mfma16(KT::as_vec(kraw[1][c]), qb[c], s1);
        }
        float sc[8];  // keys kb + 8g + j for j = 0..7 (j < 4 from s0, j >= 4 from s1)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            sc[r] = s0[r] + __shfl_xor(s0[r], 8, 64);
            sc[4 + r] = s1[r] + __shfl_xor(s1[r], 8, 64);
        }
        const bool partial_tile = kb < k_begin || kb + 32 > pos;  // wave-uniform
        if (partial_tile) {
            // keys outside [k_begin, pos) get score -inf and V = 0 (their slots may hold
            // stale data, and 0 * inf is nan)
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int key = kb + 8 * g + j;
                const bool ok = (key >= k_begin) & (key < pos);
                sc[j] = ok ? sc[j] : -INFINITY;
#pragma unroll
                for (int d = 0; d < 8; d++) vraw[d][j] = ok ? vraw[d][j] : (uint16_t)0;
            }
        }
        float mt = sc[0];
#pragma unroll
        for (int j = 1; j < 8; j++) mt = fmaxf(mt, sc[j]);
        mt = wave_max_xor(mt, 16);
        mt = wave_max_xor(mt, 32);
        const float m_new = fmaxf(m, mt);
        const float corr = exp2f(m - m_new);
        float p[8], psum = 0.f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            p[j] = exp2f(sc[j] - m_new);
            psum += p[j];
        }
        l = l * corr + psum;
        m = m_new;
        u16x8 pu;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint16_t hi = KT::from_float(p[j]);
            const uint16_t lo = KT::from_float(p[j] - KT::to_float(hi));
            pu[j] = hl ? lo : hi;
        }
        const vec8 pb = KT::as_vec(pu);
#pragma unroll
        for (int d = 0; d < 8; d++) {
            acc[d] *= corr;
            acc[d] = KT::mfma16(KT::as_vec(vraw[d]), pb, acc[d]);
        }
    }

    // ---- current token (last split, wave 3): k/v from registers, written to slot(pos) ----
    if (split == n_split - 1 && wave == 3) {
        const float *kr = row + Q_DIM + kvh * HEAD_DIM;
        float k[4][8];
        double ss = 0;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float4 a = *(const float4 *)(kr + 32 * c + 8 * g);
            const float4 b = *(const float4 *)(kr + 32 * c + 8 * g + 4);
            k[c][0] = a.x; k[c][1] = a.y; k[c][2] = a.z; k[c][3] = a.w;
            k[c][4] = b.x; k[c][5] = b.y; k[c][6] = b.z; k[c][7] = b.w;
#pragma unroll
            for (int e = 0; e < 8; e++) ss += (double)k[c][e] * k[c][e];
        }
        ss += __shfl_xor(ss, 16, 64);
        ss += __shfl_xor(ss, 32, 64);
        const float scale = 1.0f / sqrtf((float)(ss / HEAD_DIM) + P.rms_eps);
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int e = 0; e < 8; e++) k[c][e] = k[c][e] * scale * P.k_norm[32 * c + 8 * g + e];
        if (P.has_rope) {
#pragma unroll
            for (int c = 0; c < 2; c++)
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const int i = 32 * c + 8 * g + e;
                    const float a = (float)pos * P.rope_freq[i];
                    const float cs = cosf(a), sn = sinf(a);
                    const float x0 = k[c][e], x1 = k[c + 2][e];
                    k[c][e] = x0 * cs - x1 * sn;
                    k[c + 2][e] = x0 * sn + x1 * cs;
                }
        }
        u16x8 kst[4];
        float dot = 0.f;
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                kst[c][e] = KT::from_float(k[c][e]);
                dot += q[c][e] * KT::to_float(kst[c][e]);
            }
        dot = wave_sum_xor(dot, 16);
        dot = wave_sum_xor(dot, 32);
        const float m_new = fmaxf(m, dot);
        const float corr = exp2f(m - m_new), pc = exp2f(dot - m_new);
        l = l * corr + (g == 0 ? pc : 0.f);
        m = m_new;
        const float *vr = row + Q_DIM + KV_DIM + kvh * HEAD_DIM;
        uint16_t vst[8][4];
#pragma unroll
        for (int d = 0; d < 8; d++) {
            const float4 v4 = *(const float4 *)(vr + 16 * d + 4 * g);
            vst[d][0] = KT::from_float(v4.x);
            vst[d][1] = KT::from_float(v4.y);
            vst[d][2] = KT::from_float(v4.z);
            vst[d][3] = KT::from_float(v4.w);
            acc[d] *= corr;
            if (hl == 0) {
#pragma unroll
                for (int r = 0; r < 4; r++) acc[d][r] += pc * KT::to_float(vst[d][r]);
            }
        }
        if (n == 0) {  // one lane per k-group writes this kv head's row (dims owned by the lane)
            const int slot = pos & slot_mask;
            uint16_t *kw = P.k_cache + (size_t)seq * P.seq_stride + ((size_t)kvh * P.n_slots + slot) * HEAD_DIM;
#pragma unroll
            for (int c = 0; c < 4; c++) *(u16x8 *)(kw + 32 * c + 8 * g) = kst[c];
            uint16_t *vw = P.v_cache + (size_t)seq * P.seq_stride + (size_t)kvh * HEAD_DIM * P.n_slots + slot;
#pragma unroll
            for (int d = 0; d < 8; d++)
#pragma unroll
                for (int r = 0; r < 4; r++) vw[(size_t)(16 * d + 4 * g + r) * P.n_slots] = vst[d][r];
        }
    }

    // ---- merge hi/lo columns and the 4 waves through LDS ----
    __shared__ float sm_acc[4][GQA][HEAD_DIM];
    __shared__ float sm_m[4][GQA], sm_l[4][GQA];
    l = wave_sum_xor(l, 16);
    l = wave_sum_xor(l, 32);
#pragma unroll
    for (int d = 0; d < 8; d++) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float v = acc[d][r] + __shfl_xor(acc[d][r], 8, 64);
            if (hl == 0) sm_acc[wave][hloc][16 * d + 4 * g + r] = v;
        }
    }
    if (hl == 0 && g == 0) {
        sm_m[wave][hloc] = m;
        sm_l[wave][hloc] = l;
    }
    __syncthreads();

    const int th = threadIdx.x >> 5, d4 = (threadIdx.x & 31) * 4;  // head th, dims d4..d4+3
    float M = sm_m[0][th];
#pragma unroll
    for (int w = 1; w < 4; w++) M = fmaxf(M, sm_m[w][th]);
    float L = 0.f;
    float4 A = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < 4; w++) {
        if (sm_l[w][th] == 0.f) continue;
        const float c = exp2f(sm_m[w][th] - M);
        L += sm_l[w][th] * c;
        A.x += sm_acc[w][th][d4 + 0] * c;
        A.y += sm_acc[w][th][d4 + 1] * c;
        A.z += sm_acc[w][th][d4 + 2] * c;
        A.w += sm_acc[w][th][d4 + 3] * c;
    }
    const int hout = kvh * GQA + th;
    if (n_split == 1) {
        const float sink = P.sinks[hout] * LOG2E;
        const float Mf = fmaxf(M, sink), cs = exp2f(M - Mf);
        const float inv = 1.0f / (L * cs + exp2f(sink - Mf));
        float4 o = {A.x * cs * inv, A.y * cs * inv, A.z * cs * inv, A.w * cs * inv};
        *(float4 *)(P.att + (size_t)seq * Q_DIM + hout * HEAD_DIM + d4) = o;
    } else {
        float *pp = P.partial + (((size_t)seq * N_HEAD + hout) * P.max_split + split) * PART_STRIDE;
        *(float4 *)(pp + d4) = A;
        if (d4 == 0) {
            pp[HEAD_DIM] = M;
            pp[HEAD_DIM + 1] = L;
        }
    }
}

// LSE merge of the split partials plus the sink (fused.metal:331-350).
// grid = (N_HEAD, n_seq), 256 threads: the split weights are computed once per
// split (threads over splits), then each thread sums one dim over half the splits.
constexpr int MAX_SPLIT = 1024;
__global__ __launch_bounds__(256) void attn_combine_kernel(const DecodeParams P) {
    __shared__ float w_s[MAX_SPLIT];
    __shared__ float red[2][8];
    __shared__ float half_acc[HEAD_DIM];
    const int hh = blockIdx.x, seq = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int ns = P.split_prefix[seq + 1] - P.split_prefix[seq];
    if (ns <= 1) return;  // written directly by the decode kernel
    const float *pp = P.partial + ((size_t)seq * N_HEAD + hh) * P.max_split * PART_STRIDE;
    const float sink = P.sinks[hh] * LOG2E;
    float M = sink;
    for (int s = tid; s < ns; s += 256) {
        const float ls = pp[s * PART_STRIDE + HEAD_DIM + 1];
        if (ls != 0.f) M = fmaxf(M, pp[s * PART_STRIDE + HEAD_DIM]);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) M = wave_max_xor(M, o);
    if (lane == 0) red[0][wave] = M;
    __syncthreads();
    M = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
    float L = 0.f;
    for (int s = tid; s < ns; s += 256) {
        const float ls = pp[s * PART_STRIDE + HEAD_DIM + 1];
        const float w = ls != 0.f ? exp2f(pp[s * PART_STRIDE + HEAD_DIM] - M) : 0.f;
        w_s[s] = w;
        L += ls * w;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) L = wave_sum_xor(L, o);
    if (lane == 0) red[1][wave] = L;
    __syncthreads();
    L = red[1][0] + red[1][1] + red[1][2] + red[1][3] + exp2f(sink - M);
    const int dim = tid & 127, part = tid >> 7;
    float A = 0.f;
#pragma unroll 8
    for (int s = part; s < ns; s += 2) A += pp[s * PART_STRIDE + dim] * w_s[s];
    if (part == 1) half_acc[dim] = A;
    __syncthreads();
    if (part == 0) P.att[(size_t)seq * Q_DIM + hh * HEAD_DIM + dim] = (A + half_acc[dim]) / L;
}

hipError_t launch_decode(const DecodeParams &P, int dtype, int total_splits, hipStream_t stream) {
    dim3 grid(total_splits, N_HEAD_KV), block(256);
    if (dtype == DT_F16)
        hipLaunchKernelGGL(attn_decode_kernel<DT_F16>, grid, block, 0, stream, P);
    else
        hipLaunchKernelGGL(attn_decode_kernel<DT_BF16>, grid, block, 0, stream, P);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    bool need_combine = false;
    for (int s = 0; s < P.n_seq; s++) need_combine |= (P.split_prefix[s + 1] - P.split_prefix[s]) > 1;
    if (need_combine) {
        hipLaunchKernelGGL(attn_combine_kernel, dim3(N_HEAD, P.n_seq), dim3(256), 0, stream, P);
        e = hipGetLastError();
    }
    return e;
}

}  // namespace flint
