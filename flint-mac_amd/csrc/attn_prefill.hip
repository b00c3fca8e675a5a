// Layer-major batched prefill attention for CDNA4 (gfx950).
//
// Replaces the reference's k_qk_prefill + k_attn_prefill
// (/root/reference/src/metal/prefill.metal:99-266, dispatched per 512-token
// chunk at /root/reference/src/engine.mm:1087-1104).
//
//  qk_prep: per token, RMSNorm (+ NEOX RoPE) of the 32 q heads and 4 k heads;
//    q goes out as f16 [32][T][128] pre-scaled by log2(e)/sqrt(128); K and V
//    go into the key/value buffers in the cache's tiled layouts (kt_index,
//    vt_index: 32-row tiles, K in MFMA-operand order, V transposed).
//    Full-attention layers use the layer's cache directly (row = position).
//    SWA layers attend from a scratch buffer covering [max(0, p0-512), p0+T)
//    (the ring prefix [kbase, p0) is copied in first), and the positions
//    p >= p0 + T - n_slots are also written to ring slot p & (n_slots-1),
//    so one launch serves any T (the reference chunks by 512 for ring room,
//    flint_config.h:29-31).
//  flash attention: one workgroup per (32-position query block, kv head) and
//    all 8 q heads of the group, so a K/V tile is staged in LDS once for 256
//    query rows. Scores are S^T = K * Q^T and O^T += V^T * P^T on
//    v_mfma_f32_32x32x16_f16 with fp32 accumulation; the online softmax starts
//    from m = sink, l = 1 (the sink is in the denominator only, prefill.metal:162);
//    mask: kp <= qp and (full or qp - kp < window) (prefill.metal:212).
#include "common.h"
#include "flint_attn_internal.h"

namespace flint {

template <int DT>
__device__ inline _Float16 to_f16(uint16_t u) {
    return (_Float16)KvType<DT>::to_float(u);
}

// ---------------------------------------------------------------------------
// qk_prep. Blocks [0, T): q/k of one token. Blocks [T, T + nv): a 64-token V
// tile of one kv head.
template <int DT>
__global__ __launch_bounds__(256) void qk_prep_kernel(const PrefillParams P, int nv) {
    typedef KvType<DT> KT;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int b = blockIdx.x;
    if (b < P.T) {
        const int t = b, pos = P.p0 + t;
        const float *row = P.qkv + (size_t)t * P.q_stride;
        float cs = 1.f, sn = 0.f;
        if (P.has_rope) {
            const float a = (float)pos * P.rope_freq[lane];
            cs = cosf(a);
            sn = sinf(a);
        }
        const float qs = LOG2E / sqrtf((float)HEAD_DIM);
        for (int hr = wave; hr < N_HEAD + N_HEAD_KV; hr += 4) {
            const bool is_q = hr < N_HEAD;
            const float *src = is_q ? row + hr * HEAD_DIM : row + Q_DIM + (hr - N_HEAD) * HEAD_DIM;
            const float *w = is_q ? P.q_norm : P.k_norm;
            float x0 = src[lane], x1 = src[lane + 64];
            double ss = (double)x0 * x0 + (double)x1 * x1;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) ss += __shfl_xor(ss, o, 64);
            const float scale = 1.0f / sqrtf((float)(ss / HEAD_DIM) + P.rms_eps);
            x0 = x0 * scale * w[lane];
            x1 = x1 * scale * w[lane + 64];
            if (P.has_rope) {
                const float y0 = x0 * cs - x1 * sn, y1 = x0 * sn + x1 * cs;
                x0 = y0;
                x1 = y1;
            }
            if (is_q) {
                _Float16 *qd = P.qh + ((size_t)hr * P.T + t) * HEAD_DIM;
                qd[lane] = (_Float16)(x0 * qs);
                qd[lane + 64] = (_Float16)(x1 * qs);
            } else {
                const int kvh = hr - N_HEAD;
                const uint16_t k0 = KT::from_float(x0), k1 = KT::from_float(x1);
                P.kd[kt_index(kvh, pos - P.kbase, lane, P.k_rows)] = k0;
                P.kd[kt_index(kvh, pos - P.kbase, lane + 64, P.k_rows)] = k1;
                if (P.ring_k && pos >= P.ring_from) {
                    const int slot = pos & (P.ring_slots - 1);
                    P.ring_k[kt_index(kvh, slot, lane, P.ring_slots)] = k0;
                    P.ring_k[kt_index(kvh, slot, lane + 64, P.ring_slots)] = k1;
                }
            }
        }
        return;
    }
    // V tile: tokens t0..t0+63 of kv head kvh, transposed into [dim][row]
    __shared__ uint16_t tile[64][HEAD_DIM + 2];
    {
        const int vb = b - P.T, kvh = vb & 3, t0 = (vb >> 2) * 64;
        const int nt = min(64, P.T - t0);
        for (int i = threadIdx.x; i < 64 * HEAD_DIM; i += 256) {
            const int tt = i >> 7, d = i & 127;
            if (tt < nt)
                tile[tt][d] = KT::from_float(P.qkv[(size_t)(t0 + tt) * P.q_stride + Q_DIM + KV_DIM + kvh * HEAD_DIM + d]);
        }
        __syncthreads();
        for (int i = threadIdx.x; i < 64 * HEAD_DIM; i += 256) {
            const int d = i >> 6, tt = i & 63;
            if (tt >= nt) continue;
            const int pos = P.p0 + t0 + tt;
            const uint16_t v = tile[tt][d];
            P.vd[vt_index(kvh, pos - P.kbase, d, P.k_rows)] = v;
            if (P.ring_v && pos >= P.ring_from)
                P.ring_v[vt_index(kvh, pos & (P.ring_slots - 1), d, P.ring_slots)] = v;
        }
        return;
    }
}

// SWA ring prefix -> scratch key buffer: positions kbase + c0 .. +63 (< p0) of
// kv head kvh. Runs before qk_prep on the same stream: when T > n_slots - 512
// the new positions' ring writes reuse the slots read here.
__global__ __launch_bounds__(256) void ring_prefix_kernel(const PrefillParams P) {
    const int cb = blockIdx.x, kvh = cb & 3, c0 = (cb >> 2) * 64;
    const int n_pre = P.p0 - P.kbase, nc = min(64, n_pre - c0);
    const int mask = P.ring_slots - 1;
    for (int i = threadIdx.x; i < 64 * 16; i += 256) {  // K rows, 16-byte units
        const int r = i >> 4, u = i & 15;
        if (r >= nc) continue;
        const int pos = P.kbase + c0 + r;
        const u16x8 v = *(const u16x8 *)(P.ring_k + kt_index(kvh, pos & mask, 8 * u, P.ring_slots));
        *(u16x8 *)(P.kd + kt_index(kvh, pos - P.kbase, 8 * u, P.k_rows)) = v;
    }
    for (int i = threadIdx.x; i < 64 * HEAD_DIM; i += 256) {  // V^T columns
        const int d = i >> 6, r = i & 63;
        if (r >= nc) continue;
        const int pos = P.kbase + c0 + r;
        P.vd[vt_index(kvh, pos - P.kbase, d, P.k_rows)] = P.ring_v[vt_index(kvh, pos & mask, d, P.ring_slots)];
    }
}

// ---------------------------------------------------------------------------
// flash attention
constexpr int PF_BQ = 32;  // query positions per workgroup
constexpr int PF_BK = 32;  // keys per tile

// S^T row i (MFMA A row) holds key sigma(i): bits 2 and 3 of i swapped, so that
// a lane's 16 score rows are, per 16-key half, 8 consecutive keys (the P^T
// operand of the P*V MFMA then needs no data movement).
__device__ inline int pf_sigma(int i) { return (i & 0x13) | ((i & 4) << 1) | ((i & 8) >> 1); }

template <int DT>
__global__ __launch_bounds__(256) void flash_prefill_kernel(const PrefillParams P, int n_qblocks) {
    // LDS tiles of 16-byte units (8 f16): K as [dim group][key], V^T as [key group][dim]
    __shared__ f16x8 ks[16][PF_BK];
    __shared__ f16x8 vs[PF_BK / 8][HEAD_DIM];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 31, hh = lane >> 5;
    const int kvh = blockIdx.x & 3;
    const int qb = n_qblocks - 1 - (int)(blockIdx.x >> 2);  // longest (causal) blocks first
    const int t0 = qb * PF_BQ;
    const int q_first = P.p0 + t0, q_last = P.p0 + min(t0 + PF_BQ, P.T) - 1;
    const int my_t = t0 + col, my_qp = P.p0 + my_t;
    const bool row_ok = my_t < P.T;

    // Q fragments (B operand of S^T = K Q^T): column = query row, k = dims 16s + 8hh + e
    f16x8 qf[2][8];
#pragma unroll
    for (int qt = 0; qt < 2; qt++) {
        const int hq = kvh * GQA + 2 * wave + qt;
        const _Float16 *qp = P.qh + ((size_t)hq * P.T + (row_ok ? my_t : 0)) * HEAD_DIM + 8 * hh;
#pragma unroll
        for (int s = 0; s < 8; s++) {
            f16x8 v = *(const f16x8 *)(qp + 16 * s);
            qf[qt][s] = row_ok ? v : f16x8{};
        }
    }
    float m[2], l[2];
    f32x16 acc[2][4];
#pragma unroll
    for (int qt = 0; qt < 2; qt++) {
        m[qt] = P.sinks[kvh * GQA + 2 * wave + qt] * LOG2E;
        l[qt] = hh == 0 ? 1.f : 0.f;
#pragma unroll
        for (int dt = 0; dt < 4; dt++) acc[qt][dt] = f32x16{};
    }

    const int k_lo = P.is_swa ? max(P.kbase, q_first - (P.window - 1)) : 0;
    const int tile_lo = (k_lo - P.kbase) / PF_BK, tile_hi = (q_last - P.kbase) / PF_BK;
    const int n_valid = P.p0 + P.T - P.kbase;  // rows holding keys
    const int sig = pf_sigma(col);
    // this lane's query row attends to key positions [key_lo, key_hi] (causal, SWA window);
    // rows past T attend to nothing
    const int key_hi = row_ok ? my_qp : -1;
    const int key_lo = P.is_swa ? max(my_qp - (P.window - 1), 0) : 0;

    for (int kt = tile_lo; kt <= tile_hi; kt++) {
        const int r0 = kt * PF_BK;  // first row of the tile
        __syncthreads();
        // stage K (32 rows x 16 units) and V^T (128 dims x 4 units); rows >= n_valid are zero
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int u = tid + 256 * i;
            {
                // 16-byte unit u of the tiled K block (contiguous read): key and dim group
                // from the tile order (kt_index)
                const int st = (u >> 8) & 1, c = (u >> 6) & 3, g = (u >> 4) & 3, n = u & 15;
                const int key = 8 * (n >> 2) + 4 * st + (n & 3), dg = 4 * c + g;
                f16x8 v = {};
                if (r0 + key < n_valid) {
                    const u16x8 raw = *(const u16x8 *)(P.kd + kt_index(kvh, r0, 0, P.k_rows) + 8 * u);
#pragma unroll
                    for (int e = 0; e < 8; e++) v[e] = to_f16<DT>(raw[e]);
                }
                ks[dg][key] = v;
            }
            {
                const int d = u & 127, kg = u >> 7;
                f16x8 v = {};
                const int rr = r0 + 8 * kg;
                if (rr < n_valid) {
                    const u16x8 raw = *(const u16x8 *)(P.vd + vt_index(kvh, rr, d, P.k_rows));
#pragma unroll
                    for (int e = 0; e < 8; e++) v[e] = rr + e < n_valid ? to_f16<DT>(raw[e]) : (_Float16)0;
                }
                vs[kg][d] = v;
            }
        }
        __syncthreads();

        const int kp0 = P.kbase + r0;  // key position of row 0
        // wave-uniform: does any row of this block need masking in this tile?
        const bool need_mask = kp0 + PF_BK - 1 > q_first || (P.is_swa && q_last - kp0 >= P.window) ||
                               t0 + PF_BQ > P.T;
#pragma unroll
        for (int qt = 0; qt < 2; qt++) {
            f32x16 s = {};
#pragma unroll
            for (int st = 0; st < 8; st++) s = mfma32_f16(ks[2 * st + hh][sig], qf[qt][st], s);
            // lane holds query row `col`, keys kp0 + 16(j>>1) + 8hh + 4(j&1) + r for element 4j + r
            if (need_mask) {
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int j = e >> 2, r = e & 3;
                    const int kp = kp0 + 16 * (j >> 1) + 8 * hh + 4 * (j & 1) + r;
                    const bool ok = (kp >= key_lo) & (kp <= key_hi);
                    s[e] = ok ? s[e] : -INFINITY;
                }
            }
            float mt = s[0];
#pragma unroll
            for (int e = 1; e < 16; e++) mt = fmaxf(mt, s[e]);
            mt = wave_max_xor(mt, 32);
            const float m_new = fmaxf(m[qt], mt);
            const float corr = exp2f(m[qt] - m_new);
            m[qt] = m_new;
            float psum = 0.f;
            f16x8 pf[2];
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const float p = exp2f(s[e] - m_new);
                psum += p;
                pf[e >> 3][e & 7] = (_Float16)p;
            }
            l[qt] = l[qt] * corr + psum;
#pragma unroll
            for (int dt = 0; dt < 4; dt++) {
                acc[qt][dt] *= corr;
#pragma unroll
                for (int kk = 0; kk < 2; kk++)
                    acc[qt][dt] = mfma32_f16(vs[2 * kk + hh][32 * dt + col], pf[kk], acc[qt][dt]);
            }
        }
    }

    if (!row_ok) return;
#pragma unroll
    for (int qt = 0; qt < 2; qt++) {
        const float lt = l[qt] + __shfl_xor(l[qt], 32, 64);
        const float inv = 1.0f / lt;
        const int hq = kvh * GQA + 2 * wave + qt;
        float *o = P.att + (size_t)my_t * Q_DIM + hq * HEAD_DIM;
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                float4 v = {acc[qt][dt][4 * j] * inv, acc[qt][dt][4 * j + 1] * inv, acc[qt][dt][4 * j + 2] * inv,
                            acc[qt][dt][4 * j + 3] * inv};
                *(float4 *)(o + 32 * dt + 8 * j + 4 * hh) = v;
            }
    }
}

hipError_t launch_prefill(const PrefillParams &P, int dtype, hipStream_t stream) {
    const int nv = ((P.T + 63) / 64) * N_HEAD_KV;
    const int n_pre = P.p0 - P.kbase;
    const int np = (P.ring_k && n_pre > 0 && P.kd != P.ring_k) ? ((n_pre + 63) / 64) * N_HEAD_KV : 0;
    const int nqb = (P.T + PF_BQ - 1) / PF_BQ;
    if (np > 0) hipLaunchKernelGGL(ring_prefix_kernel, dim3(np), dim3(256), 0, stream, P);
    if (dtype == DT_F16) {
        hipLaunchKernelGGL(qk_prep_kernel<DT_F16>, dim3(P.T + nv), dim3(256), 0, stream, P, nv);
        hipLaunchKernelGGL(flash_prefill_kernel<DT_F16>, dim3(nqb * N_HEAD_KV), dim3(256), 0, stream, P, nqb);
    } else {
        hipLaunchKernelGGL(qk_prep_kernel<DT_BF16>, dim3(P.T + nv), dim3(256), 0, stream, P, nv);
        hipLaunchKernelGGL(flash_prefill_kernel<DT_BF16>, dim3(nqb * N_HEAD_KV), dim3(256), 0, stream, P, nqb);
    }
    return hipGetLastError();
}

}  // namespace flint
