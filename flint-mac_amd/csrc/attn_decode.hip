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
//  * One 8-wave workgroup per (sequence, kv head, key split) serves all 8 q
//    heads of the GQA group, so every K/V byte is read from HBM once (the
//    reference re-reads K/V per q head).
//  * KV layout is head-major and tiled by 32 slots: K tiles stored in MFMA
//    A-operand order, V transposed ([dim][slot] per tile), so a 32-key tile is
//    two contiguous 8 KiB blocks, both MFMA operands are single 16-byte loads
//    straight from HBM and every load instruction reads 1 KiB contiguous.
//  * Scores are S^T = K * Q^T on v_mfma_f32_16x16x32: the 16 MFMA columns carry
//    the 8 heads' q split into hi + lo halves of the 16-bit type, so the scores
//    are fp32-accurate at no extra MFMA cost; P*V uses the same hi/lo trick on P.
//  * A tile is 32 keys (16 x 16-byte loads per lane, 16 KiB per wave). Each
//    wave keeps two tiles in flight, and a tile's registers are refilled as
//    soon as it is consumed; the first is requested before the prologue, the
//    second after its barrier.
//  * Compact code on the critical path: each wave runs the straight-line
//    parts of the kernel once, from a cold instruction cache, so the q / k
//    normalisation is cooperative (one q head per wave, a NEOX pair per lane)
//    and hands the MFMA operands over through LDS, and the current token
//    joins the block merge as one more partial.
//  * Every split writes its partial (m, l, acc); a second, short kernel merges
//    them (fused.metal:331-350): one workgroup per head, one wave per 32 dims,
//    one lane per split. (A last-block merge inside the streaming kernel needs
//    coherent stores and a ticket per block and funnels every partial through
//    one CU, which measured slower than the kernel boundary.)
//  * Batched entry: one launch serves many independent sequences (one token each).
//    The grid is flat: sequence s owns 4 x n_split[s] consecutive workgroups (kv head
//    fastest), so no workgroup is idle and the XCDs, dealt workgroups in id order, get
//    equal shares of the stream. Every kernel argument the block needs is read at wave
//    start (the per-sequence tables one entry per lane), so the kernel-argument fetch
//    costs one memory round trip.
//  * Short key ranges (one split per sequence, SWA layers): a kv head's 128 output dims
//    are cut over 8 (4, 2) V-slice workgroups, each reading all of K, and the launch ids
//    are packed so that a kv head's slices share one XCD: its K comes from HBM once and
//    from that XCD's L2 for the other slices.
#include <mutex>

#include "common.h"
#include "flint_attn_internal.h"

namespace flint {

// partial record per (seq, head, split): acc[128], m (log2 units), l, 2 pad
constexpr int PART_STRIDE = 132;
constexpr int DEC_WAVES = 8;
constexpr int DEC_THREADS = DEC_WAVES * 64;
// LDS row of a wave's partial accumulator for one head: 128 floats + 4 of padding, so the
// 32 lanes that write 16 bytes each spread evenly over the banks
constexpr int ACC_ROW = HEAD_DIM + 4;

// VS = V slices: the 128 output dims of a head split over VS workgroups (VS = 1, 2, 4 or 8). Each
// workgroup computes every score (all of K) and the P*V product for its 128/VS dims.
template <int VS>
struct KvTile {
    u32x4 k[2][4];     // K rows: sub-tile st, dim chunk c (8 packed 16-bit values each)
    u32x4 v[8 / VS];   // V^T rows: dim tile 8/VS * slice + d
};

// Issue the 16 loads of tile t (keys 32t .. 32t+31) for this lane: 1 KiB contiguous per
// load instruction in both tiled layouts. kc / vc are wave-uniform bases; offsets stay
// 32-bit (a kv head's cache is < 2^31 elements) so the loads take the scalar-base +
// vector-offset form. A wave with no tile left (live == false) still issues the 16 loads,
// which keeps the compiler's wait counts static, but every lane reads the tile's first
// 16 bytes, so each costs one cache line instead of eight.
template <int VS>
__device__ inline void load_tile(KvTile<VS> &T, const uint16_t *__restrict__ kc, const uint16_t *__restrict__ vc,
                                 int t, int lane, int slot_mask, bool live, int slice) {
    // byte offsets in 32 bits (the host bounds a kv head's cache below 2^31 bytes)
    const uint32_t base = ((uint32_t)(t * 32) & (uint32_t)slot_mask) * (HEAD_DIM * 2);
    const char *kb = (const char *)kc, *vb = (const char *)vc;
    // K: instruction (st, c) reads units (st*4 + c)*64 + lane: MFMA row n = lane & 15 holds
    // key 8(n>>2) + 4st + (n&3) of the tile, dims 32c + 8(lane>>4) .. +7
    const uint32_t ko = base + (live ? lane * 16 : 0);
#pragma unroll
    for (int st = 0; st < 2; st++)
#pragma unroll
        for (int c = 0; c < 4; c++)
            T.k[st][c] = __builtin_nontemporal_load((const u32x4 *)(kb + (ko + (st * 4 + c) * 1024)));
    // V^T tile (8 KiB): row = dim 16d + n, keys 8g .. 8g+7 of the tile
    const uint32_t vo = base + (live ? (lane & 15) * 64 + 16 * (lane >> 4) : 0);
#pragma unroll
    for (int d = 0; d < 8 / VS; d++)
        T.v[d] = __builtin_nontemporal_load((const u32x4 *)(vb + (vo + (8 / VS * slice + d) * 1024)));
}

template <int DT, int VS>
struct DecodeState {
    typedef typename KvType<DT>::vec8 vec8;
    float m, l;          // running max (log2 units) of this lane's head, this lane's partial sum
    f32x4 acc[8 / VS];   // O^T tile d: rows = slice dims 16d + 4g + r, column = this lane's (head, hi/lo)
};

// The running max is raised only when a score exceeds it by more than this (log2 units),
// so p = 2^(s - m) stays below 2^8 and the rescale of l and acc runs on few tiles.
constexpr float RESCALE_LOG2 = 8.f;

// P in two 16-bit halves: word = (p0, p1) packed as hi parts (hl == 0) or as the
// residuals p - hi (hl == 1). Both halves are rounded toward zero; their sum carries p
// to ~2^-22 relative for f16 (2^-16 for bf16).
template <int DT>
__device__ inline uint32_t split_pack(float p0, float p1, int hl);
template <>
__device__ inline uint32_t split_pack<DT_F16>(float p0, float p1, int hl) {
    const auto h = __builtin_amdgcn_cvt_pkrtz(p0, p1);
    const auto l = __builtin_amdgcn_cvt_pkrtz(p0 - (float)h[0], p1 - (float)h[1]);
    return hl ? __builtin_bit_cast(uint32_t, l) : __builtin_bit_cast(uint32_t, h);
}
template <>
__device__ inline uint32_t split_pack<DT_BF16>(float p0, float p1, int hl) {
    const uint32_t b0 = __float_as_uint(p0), b1 = __float_as_uint(p1);
    const float r0 = p0 - __uint_as_float(b0 & 0xffff0000u), r1 = p1 - __uint_as_float(b1 & 0xffff0000u);
    const uint32_t c0 = hl ? __float_as_uint(r0) : b0, c1 = hl ? __float_as_uint(r1) : b1;
    return (c1 & 0xffff0000u) | (c0 >> 16);
}

// Online-softmax update with one 32-key tile.
template <int DT, int VS>
__device__ inline void consume_tile(DecodeState<DT, VS> &S, KvTile<VS> &T, const typename KvType<DT>::vec8 (&qb)[4], int t,
                                    int k_begin, int pos, int g, int hl) {
    typedef KvType<DT> KT;
    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 4; c++) {
        s0 = KT::mfma16(__builtin_bit_cast(typename KT::vec8, T.k[0][c]), qb[c], s0);
        s1 = KT::mfma16(__builtin_bit_cast(typename KT::vec8, T.k[1][c]), qb[c], s1);
    }
    float sc[8];  // keys kb + 8g + j: j < 4 from s0, j >= 4 from s1; hi + lo columns summed
#pragma unroll
    for (int r = 0; r < 4; r++) {
        sc[r] = s0[r] + lane_xor8(s0[r]);
        sc[4 + r] = s1[r] + lane_xor8(s1[r]);
    }
    const int kb = t * 32;
    if (kb < k_begin || kb + 32 > pos) {  // wave-uniform: a tile at either end of the key range
        // keys outside [k_begin, pos) get score -inf and V = 0 (their slots may hold
        // stale data, and 0 * inf is nan); V words hold keys (2w, 2w+1)
        // (-inf is made here, in a register of its own, rather than hoisted out of the
        // stream loop by the compiler, where it would hold a register for the whole loop)
        float ninf;
        asm volatile("v_mov_b32 %0, 0xff800000" : "=v"(ninf));
        uint32_t vmask[4];
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const int key = kb + 8 * g + 2 * w;
            const bool ok0 = (key >= k_begin) & (key < pos), ok1 = (key + 1 >= k_begin) & (key + 1 < pos);
            sc[2 * w] = ok0 ? sc[2 * w] : ninf;
            sc[2 * w + 1] = ok1 ? sc[2 * w + 1] : ninf;
            vmask[w] = ((uint32_t)-(int)ok0 >> 16) | ((uint32_t)-(int)ok1 << 16);
        }
#pragma unroll
        for (int d = 0; d < 8 / VS; d++)
#pragma unroll
            for (int w = 0; w < 4; w++) T.v[d][w] &= vmask[w];
    }
    float mt = fmaxf(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])), fmaxf(fmaxf(sc[4], sc[5]), fmaxf(sc[6], sc[7])));
    mt = xor32_max(xor16_max(mt));
    if (__builtin_amdgcn_ballot_w64(mt > S.m + RESCALE_LOG2) != 0) {  // wave-uniform
        const float m_new = fmaxf(S.m, mt);
        const float corr = __builtin_amdgcn_exp2f(S.m - m_new);
        S.l *= corr;
#pragma unroll
        for (int d = 0; d < 8 / VS; d++) S.acc[d] *= corr;
        S.m = m_new;
    }
    float p[8];
#pragma unroll
    for (int j = 0; j < 8; j++) p[j] = __builtin_amdgcn_exp2f(sc[j] - S.m);
    S.l += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
    const u32x4 pu = {split_pack<DT>(p[0], p[1], hl), split_pack<DT>(p[2], p[3], hl), split_pack<DT>(p[4], p[5], hl),
                      split_pack<DT>(p[6], p[7], hl)};
    const typename KT::vec8 pb = __builtin_bit_cast(typename KT::vec8, pu);
#pragma unroll
    for (int d = 0; d < 8 / VS; d++) S.acc[d] = KT::mfma16(__builtin_bit_cast(typename KT::vec8, T.v[d]), pb, S.acc[d]);
}

template <int DT, int VS>
__global__ __launch_bounds__(DEC_THREADS) void attn_decode_kernel(const DecodeParams P) {
    typedef KvType<DT> KT;
    typedef typename KT::vec8 vec8;
    constexpr int W = DEC_WAVES;

    // the wave index is made scalar, so everything derived from it lives in SGPRs
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15, g = lane >> 4;   // MFMA column (q head x hi/lo) and k-group
    const int hloc = n & 7, hl = n >> 3;      // head within the GQA group, 0 = hi half, 1 = lo half
    static_assert(MAX_SEQ == 64, "one per-sequence table entry per lane");

    // ---- every kernel argument is read here, in one batch of loads at wave start (left to
    //      itself the compiler sinks each load to its first use, and each sunk load is one
    //      more memory round trip on the critical path). The per-sequence tables arrive one
    //      entry per lane, so finding this workgroup's sequence costs no second round trip ----
    const int t_base = P.wg_base[lane], t_pos = P.pos[lane], t_tps = P.tps[lane], t_ns = P.n_split[lane];
    const int t_s0 = P.split0[lane];
    const int n_seq = P.n_seq;
    const int is_swa = P.is_swa, has_rope = P.has_rope, window = P.window;
    const int n_slots = P.n_slots, slot_mask = P.slot_mask;
    const float rms_eps = P.rms_eps;
    const long long seq_stride = P.seq_stride;
    const float *const qkv = P.qkv, *const q_norm = P.q_norm, *const k_norm = P.k_norm, *const sinks = P.sinks;
    uint16_t *const k_cache = P.k_cache, *const v_cache = P.v_cache;
    float *const att = P.att, *const partial = P.partial;
    pin_sgpr(n_seq), pin_sgpr(is_swa), pin_sgpr(has_rope), pin_sgpr(window);
    pin_sgpr(n_slots), pin_sgpr(slot_mask), pin_sgpr(rms_eps), pin_sgpr(seq_stride);
    pin_sgpr(qkv), pin_sgpr(q_norm), pin_sgpr(k_norm), pin_sgpr(sinks), pin_sgpr(k_cache), pin_sgpr(v_cache);
    pin_sgpr(att), pin_sgpr(partial);
    asm volatile("" ::"v"(t_base), "v"(t_pos), "v"(t_tps), "v"(t_ns), "v"(t_s0));

    // The grid is flat and holds exactly the launch's work units: sequence s owns workgroups
    // wg_base[s] .. wg_base[s] + 4 VS n_split[s] - 1 (kv head fastest, then V slice, then
    // split). The hardware deals workgroups to the XCDs in id order, so equal-sized units
    // spread every XCD's share of the stream evenly (a grid with idle slots skews it, and one
    // XCD moves ~1.2 TB/s at most).
    // With V slices (one split per sequence, so wg_base[s] = 4 VS s) the launch ids are packed by
    // XCD instead: 8 VS consecutive ids serve two sequences, the VS slices of kv head h of the
    // first on XCD h and those of the second on XCD h + 4, so the K that all of them read comes
    // from HBM once per kv head and from that XCD's L2 for the other slices. The id is mapped
    // back to the flat order above.
    int wid = blockIdx.x;
    if constexpr (VS > 1) {
        const int j = wid % (8 * VS), s = 2 * (wid / (8 * VS)) + ((j >> 2) & 1);
        if (s >= n_seq) return;  // the second sequence of the last block when n_seq is odd
        wid = 4 * VS * s + (j & 3) + 4 * (j >> 3);  // kv head j & 3, V slice j >> 3
    }
    const int seq = __builtin_popcountll(__builtin_amdgcn_ballot_w64(lane < n_seq && wid >= t_base)) - 1;
    const int n_split = __builtin_amdgcn_readlane(t_ns, seq), pos = __builtin_amdgcn_readlane(t_pos, seq);
    const int tps = __builtin_amdgcn_readlane(t_tps, seq);
    const int local = wid - __builtin_amdgcn_readlane(t_base, seq);
    const int split0 = __builtin_amdgcn_readlane(t_s0, seq);  // this sequence's first partial record
    const int kvh = local & (N_HEAD_KV - 1), slice = (local / N_HEAD_KV) % VS, split = local / (N_HEAD_KV * VS);
    if (seq < 0 || split >= n_split) return;  // not reached: the host sizes the grid exactly
    const bool last_split = split == n_split - 1;
    const int k_begin = is_swa ? max(pos - (window - 1), 0) : 0;
    const int tile_lo = k_begin >> 5, tile_hi = (pos + 31) >> 5;  // tiles holding keys [k_begin, pos)
    const int t_begin = tile_lo + split * tps;
    const int t_end = min(t_begin + tps, tile_hi);

    const uint16_t *__restrict__ kc = k_cache + (size_t)seq * seq_stride + (size_t)kvh * n_slots * HEAD_DIM;
    const uint16_t *__restrict__ vc = v_cache + (size_t)seq * seq_stride + (size_t)kvh * HEAD_DIM * n_slots;
    const float *__restrict__ row = qkv + (size_t)seq * QKV_DIM;

    // LDS: q halves in MFMA-operand order, q in fp32, the current token, the wave merge
    __shared__ uint16_t sm_qh[2][GQA][HEAD_DIM];   // [hi/lo][head][dim]
    __shared__ float sm_q[GQA][HEAD_DIM];          // log2(e)/sqrt(D)-scaled q (for the current token)
    __shared__ float sm_kv[2][HEAD_DIM];           // current token: k and v as the cache holds them
    __shared__ float sm_acc[W][GQA][ACC_ROW];      // wave partial accumulators (padded rows)
    __shared__ float sm_m[W + 1][GQA], sm_l[W + 1][GQA];

    // ---- the prologue's inputs first, then this wave's first tiles: vmcnt counts
    //      completions in issue order, so the prologue can wait for its own small loads
    //      while the tiles stay in flight. Wave w normalises q head w; the last split's last
    //      wave also handles the current token ----
    const bool cur_wave = last_split && wave == W - 1;
    const float *qr = row + (kvh * GQA + wave) * HEAD_DIM;
    const float2 qx = make_float2(qr[lane], qr[lane + 64]);
    const float2 qw = make_float2(q_norm[lane], q_norm[lane + 64]);
    const float rfreq = P.rope_freq[lane];
    // head `wave` of the group, for the final merge: a wave-uniform address read through the
    // constant address space, so it is a scalar load into an SGPR that nothing waits for until
    // the merge (the kernel never writes the sinks). A vector load moved into an SGPR here made
    // every wave wait for its round trip before it issued its first tile loads.
    const float sink = *(const __attribute__((address_space(4))) float *)(sinks + kvh * GQA + wave) * LOG2E;
    float2 kx = {0.f, 0.f}, kw = {0.f, 0.f}, vx = {0.f, 0.f};
    if (cur_wave) {
        const float *kr = row + Q_DIM + kvh * HEAD_DIM, *vr = row + Q_DIM + KV_DIM + kvh * HEAD_DIM;
        kx = make_float2(kr[lane], kr[lane + 64]);
        kw = make_float2(k_norm[lane], k_norm[lane + 64]);
        vx = make_float2(vr[lane], vr[lane + 64]);
    }
    __builtin_amdgcn_sched_barrier(0);
    // The first tile, before the prologue waits for its own loads, so its latency overlaps
    // the prologue; the second after the prologue's barrier. Once the CU's memory pipeline is
    // full a wave's load instructions stall at issue, and a wave still issuing cannot reach
    // the barrier: with both tiles issued here every wave waited for the slowest wave's 32
    // loads to be accepted (q operands ready ~2.9 us after the start of a cold SWA call, ~2.2
    // with one tile). Issuing no tile before the prologue readies q by ~1.2 us but leaves the
    // first tile's latency exposed (slower, also at 32k). Issued unconditionally (a wave
    // without such a tile reads 16 bytes per load of tile t_begin, never consumed), since
    // loads under a branch make the compiler's wait counting at the join conservative.
    KvTile<VS> ta, tb;
    int t_a = t_begin + wave, t_b = t_a + W;
    load_tile(ta, kc, vc, t_a < t_end ? t_a : t_begin, lane, slot_mask, t_a < t_end, slice);
    __builtin_amdgcn_sched_barrier(0);
    // The current token's rows are handed to the prologue here, after the tile's loads: left
    // alone, the compiler rounds v to the cache dtype right after its load, in the branch
    // above, and that wave then waits for the load before it issues its tile.
    asm volatile("" : "+v"(kx.x), "+v"(kx.y), "+v"(kw.x), "+v"(kw.y), "+v"(vx.x), "+v"(vx.y));

    // ---- prologue: wave w normalises q head w (+ RoPE), the last split's last wave also
    //      the current token's k and v (rounded to the cache dtype, written to slot(pos)) ----
    {
        float cs = 1.f, sn = 0.f;  // rotation of frequency `lane`
        if (has_rope) rope_sincos((float)pos * rfreq, &sn, &cs);
        const float qs = LOG2E / sqrtf((float)HEAD_DIM);
        const float2 qv = norm_rope_pair(qx, qw, rms_eps, has_rope, cs, sn);
        const float q0 = qv.x * qs, q1 = qv.y * qs;
        sm_q[wave][lane] = q0;
        sm_q[wave][lane + 64] = q1;
        const uint16_t h0 = KT::from_float(q0), h1 = KT::from_float(q1);
        sm_qh[0][wave][lane] = h0;
        sm_qh[0][wave][lane + 64] = h1;
        sm_qh[1][wave][lane] = KT::from_float(q0 - KT::to_float(h0));
        sm_qh[1][wave][lane + 64] = KT::from_float(q1 - KT::to_float(h1));
        if (cur_wave) {
            // the current token: no key read by this launch lives in slot(pos) (in the ring it
            // held pos - n_slots, outside the window)
            const float2 kv2 = norm_rope_pair(kx, kw, rms_eps, has_rope, cs, sn);
            const uint16_t k0 = KT::from_float(kv2.x), k1 = KT::from_float(kv2.y);
            const uint16_t v0 = KT::from_float(vx.x), v1 = KT::from_float(vx.y);
            sm_kv[0][lane] = KT::to_float(k0);
            sm_kv[0][lane + 64] = KT::to_float(k1);
            sm_kv[1][lane] = KT::to_float(v0);
            sm_kv[1][lane + 64] = KT::to_float(v1);
            const int slot = pos & slot_mask;
            if (slice == 0) {  // one V slice writes the token's K/V (every slice computes them)
                uint16_t *kw_ = k_cache + (size_t)seq * seq_stride;
                kw_[kt_index(kvh, slot, lane, n_slots)] = k0;
                kw_[kt_index(kvh, slot, lane + 64, n_slots)] = k1;
                uint16_t *vw = v_cache + (size_t)seq * seq_stride;
                vw[vt_index(kvh, slot, lane, n_slots)] = v0;
                vw[vt_index(kvh, slot, lane + 64, n_slots)] = v1;
            }
        }
    }
    lds_barrier();  // the q operands are in LDS; the first tile's loads stay in flight
    load_tile(tb, kc, vc, t_b < t_end ? t_b : t_begin, lane, slot_mask, t_b < t_end, slice);
    vec8 qb[4];  // MFMA B operand: column n = head hloc, hi or lo half; k = dims 32c + 8g + e
#pragma unroll
    for (int c = 0; c < 4; c++) qb[c] = *(const vec8 *)&sm_qh[hl][hloc][32 * c + 8 * g];
    if (last_split) {
        // score of the current token for head `wave` (q in fp32, k as the cache holds it),
        // computed while the first tiles stream in
        float dot = sm_q[wave][lane] * sm_kv[0][lane] + sm_q[wave][lane + 64] * sm_kv[0][lane + 64];
        dot = wave_sum(dot);
        if (lane == 0) {
            sm_m[W][wave] = dot;
            sm_l[W][wave] = 1.f;
        }
    }

    // ---- stream this wave's tiles t_begin + wave + 8i, two in flight ----
    DecodeState<DT, VS> S;
    S.m = -1e30f;
    S.l = 0.f;
#pragma unroll
    for (int d = 0; d < 8 / VS; d++) S.acc[d] = f32x4{0.f, 0.f, 0.f, 0.f};
    // Two register sets, each refilled with the tile 16 further on as soon as it is
    // consumed. The steady-state loop runs while both refills are needed, so its loads
    // are unconditional and the wait counts static (consuming a tile waits for its own
    // 16 loads only); the drain then handles the last two or three tiles, issuing no
    // load that will not be consumed except in the three-tile case.
    while (t_b + 2 * W < t_end) {
        consume_tile<DT, VS>(S, ta, qb, t_a, k_begin, pos, g, hl);
        t_a += 2 * W;
        load_tile(ta, kc, vc, t_a, lane, slot_mask, true, slice);
        consume_tile<DT, VS>(S, tb, qb, t_b, k_begin, pos, g, hl);
        t_b += 2 * W;
        load_tile(tb, kc, vc, t_b, lane, slot_mask, true, slice);
    }
    if (t_a < t_end) {
        consume_tile<DT, VS>(S, ta, qb, t_a, k_begin, pos, g, hl);
        t_a += 2 * W;
        const bool third = t_a < t_end;
        // unconditional (16 bytes per load when there is no third tile): tile b's wait
        // stays exact while the third tile streams in
        load_tile(ta, kc, vc, third ? t_a : t_begin, lane, slot_mask, third, slice);
        if (t_b < t_end) consume_tile<DT, VS>(S, tb, qb, t_b, k_begin, pos, g, hl);
        if (third) consume_tile<DT, VS>(S, ta, qb, t_a, k_begin, pos, g, hl);
    }

    // ---- merge hi/lo columns and the waves (and the current token) through LDS ----
    // (the lane's MFMA column and k-group are derived again here from the lane id, so that
    // they hold no register during the stream)
    const int lane2 = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    asm volatile("" ::"v"(lane2));
    const int n2 = lane2 & 15, g2 = lane2 >> 4, hloc2 = n2 & 7, hl2 = n2 >> 3;
    S.l = xor32_sum(xor16_sum(S.l));
#pragma unroll
    for (int d = 0; d < 8 / VS; d++) {
        f32x4 v;
#pragma unroll
        for (int r = 0; r < 4; r++) v[r] = S.acc[d][r] + lane_xor8(S.acc[d][r]);
        if (hl2 == 0) *(f32x4 *)&sm_acc[wave][hloc2][16 * d + 4 * g2] = v;
    }
    if (hl2 == 0 && g2 == 0) {
        sm_m[wave][hloc2] = S.m;
        sm_l[wave][hloc2] = S.l;
    }
    lds_barrier();

    // wave th merges head th: 8 wave partials + the current token, branch-free (a wave
    // without keys has m = -1e30 and l = 0, so its weight is 0). Lane pairs of dims d2, d2+1
    // of this V slice's 128/VS dims (with VS > 1 the upper lanes read unused LDS and store nothing)
    const int th = wave, d2 = lane2 * 2, dg = HEAD_DIM / VS * slice + d2;
    float mw[W + 1], lw[W + 1];
#pragma unroll
    for (int w = 0; w < W; w++) {
        mw[w] = sm_m[w][th];
        lw[w] = sm_l[w][th];
    }
    mw[W] = last_split ? sm_m[W][th] : -1e30f;
    lw[W] = last_split ? 1.f : 0.f;
    float M = mw[0];
#pragma unroll
    for (int w = 1; w <= W; w++) M = fmaxf(M, mw[w]);
    float L = 0.f, A0 = 0.f, A1 = 0.f;
#pragma unroll
    for (int w = 0; w < W; w++) {
        const float c = __builtin_amdgcn_exp2f(mw[w] - M);
        const float2 a = *(const float2 *)&sm_acc[w][th][d2];
        L += lw[w] * c;
        A0 += a.x * c;
        A1 += a.y * c;
    }
    if (last_split) {  // sm_kv is written only in the last split: elsewhere it is stale LDS
        const float c = __builtin_amdgcn_exp2f(mw[W] - M);
        L += lw[W] * c;
        A0 += sm_kv[1][dg & (HEAD_DIM - 1)] * c;
        A1 += sm_kv[1][(dg + 1) & (HEAD_DIM - 1)] * c;
    }
    const int hout = kvh * GQA + th;
    if (n_split == 1) {
        float *out = att + (size_t)seq * Q_DIM + hout * HEAD_DIM + dg;
        const float Mf = fmaxf(M, sink), cs = __builtin_amdgcn_exp2f(M - Mf);
        const float inv = 1.0f / (L * cs + __builtin_amdgcn_exp2f(sink - Mf));
        if (d2 < HEAD_DIM / VS) *(float2 *)out = make_float2(A0 * cs * inv, A1 * cs * inv);
        return;
    }
    if constexpr (VS > 1) return;  // not reached: V slices are planned for one split per sequence
    // partials of a launch: sequence s's records start at split0[s], and each head's splits are
    // consecutive records
    float *pp = partial + ((size_t)split0 * N_HEAD + hout * n_split + split) * PART_STRIDE;
    *(float2 *)(pp + d2) = make_float2(A0, A1);
    if (lane2 == 0) *(float2 *)(pp + HEAD_DIM) = make_float2(M, L);
}

// The merge kernel's arguments: only what it reads (536 bytes instead of the decode kernel's
// 1.3 KB), since a dependent launch waits for its argument block.
struct CombineParams {
    const float *partial, *sinks;
    float *att;
    int n_split[MAX_SEQ];  // key splits of sequence s
    int split0[MAX_SEQ];   // first split record of sequence s
};

// LSE merge of the split partials plus the sink (fused.metal:331-350), with no LDS and no
// workgroup barrier. grid = (N_HEAD, n_seq), 4 waves: wave q writes dims 32q .. 32q + 31 of head
// hh. Lane s takes split s of each chunk of 64 (its (m, l) and its 32 accumulators, all requested
// at once, so the merge waits on one memory round trip after the kernel arguments); the chunk's
// weights 2^(m_s - M) come from a wave max (splits with l = 0 are skipped, as in fused.metal), and
// the 64 lanes' 32 weighted sums are reduced by a reduce-scatter over lane pairs (swaps across
// the wave halves and rows, DPP within rows), which leaves dim lane / 2 in lanes 2d and 2d + 1.
// (A 256-thread workgroup per head quarter, reducing through LDS with three barriers, measured
// ~0.25 us slower per config-3 call.)
__device__ inline float dpp_half_mirror(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), DPP_HALF_MIRROR, 0xf, 0xf, false));
}
// At most 2 waves per SIMD (one workgroup per CU is all the grid needs), so the register
// allocator keeps a lane's 8 accumulator loads and its (m, l) load in flight together instead
// of reusing registers for the last loads after a wait (a second memory round trip).
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void attn_combine_kernel(const CombineParams P) {
    const int hh = blockIdx.x, seq = blockIdx.y, lane = threadIdx.x & 63;
    const int q = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ns = P.n_split[seq], split0 = P.split0[seq];
    const float *const partial = P.partial, *const sinks = P.sinks;
    float *const att = P.att;
    pin_sgpr(ns), pin_sgpr(split0), pin_sgpr(partial), pin_sgpr(sinks), pin_sgpr(att);
    if (ns <= 1) return;  // written directly by the decode kernel
    const float *pp = partial + ((size_t)split0 * N_HEAD + hh * ns) * PART_STRIDE;
    // a scalar load (constant address space: the kernel never writes the sinks), first used
    // after the records' loop, so the records are requested without waiting for it
    const float sink = *(const __attribute__((address_space(4))) float *)(sinks + hh) * LOG2E;
    // M starts finite, so a chunk whose splits all lack keys keeps scale 1 and weight 0
    float M = -1e30f, lsum = 0.f, acc[32];
#pragma unroll
    for (int j = 0; j < 32; j++) acc[j] = 0.f;
    for (int s0 = 0; s0 < ns; s0 += 64) {
        const bool live = s0 + lane < ns;
        const float *rec = pp + (size_t)min(s0 + lane, ns - 1) * PART_STRIDE;
        f32x4 a[8];
#pragma unroll
        for (int i = 0; i < 8; i++) a[i] = *(const f32x4 *)(rec + 32 * q + 4 * i);
        const float2 ml = *(const float2 *)(rec + HEAD_DIM);
        const bool use = live && ml.y != 0.f;  // splits without keys carry no weight
        const float Mn = fmaxf(M, wave_max(use ? ml.x : -INFINITY));
        const float scale = exp2f(M - Mn), w = use ? exp2f(ml.x - Mn) : 0.f;
        lsum = lsum * scale + ml.y * w;
#pragma unroll
        for (int j = 0; j < 32; j++) acc[j] = acc[j] * scale + a[j >> 2][j & 3] * w;
        M = Mn;
    }
    // the sink joins last: Mf = max(M, sink), the sums rescaled by 2^(M - Mf) (folded into the
    // final division, c and L being the same in every lane)
    const float Mf = fmaxf(M, sink), c = exp2f(M - Mf);
    const float L = wave_sum(lsum) * c + exp2f(sink - Mf), cl = c / L;
    // reduce-scatter: 32 values per lane -> one dim per lane pair
#pragma unroll
    for (int j = 0; j < 16; j++) {  // lanes l and l ^ 32: dims j (lower half), j + 16 (upper)
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[j]), __float_as_uint(acc[j + 16]), false, false);
        acc[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
#pragma unroll
    for (int j = 0; j < 8; j++) {  // lanes l and l ^ 16
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(acc[j]), __float_as_uint(acc[j + 8]), false, false);
        acc[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    const bool b3 = lane & 8, b2 = lane & 4, b1 = lane & 2;
#pragma unroll
    for (int j = 0; j < 4; j++) {  // lanes l and l ^ 8 (rotation by 8 within a row of 16)
        const float t0 = acc[j] + dpp<DPP_ROR8>(acc[j]), t1 = acc[j + 4] + dpp<DPP_ROR8>(acc[j + 4]);
        acc[j] = b3 ? t1 : t0;
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {  // lanes l and 7 - l within each 8 (they differ in bit 2)
        const float t0 = acc[j] + dpp_half_mirror(acc[j]), t1 = acc[j + 2] + dpp_half_mirror(acc[j + 2]);
        acc[j] = b2 ? t1 : t0;
    }
    {  // lanes l and l ^ 2, then l ^ 1
        const float t0 = acc[0] + dpp<DPP_QUAD_XOR2>(acc[0]), t1 = acc[1] + dpp<DPP_QUAD_XOR2>(acc[1]);
        acc[0] = b1 ? t1 : t0;
        acc[0] += dpp<DPP_QUAD_XOR1>(acc[0]);
    }
    if ((lane & 1) == 0) att[(size_t)seq * Q_DIM + hh * HEAD_DIM + 32 * q + (lane >> 1)] = acc[0] * cl;
}

// Split partials of the entry point that allocates nothing (flint_attn_decode_batch_noalloc):
// a fixed array in device memory, one copy per GPU, held until the process ends. Host code
// never passes `scratch` itself to a kernel (in host code the name is a stand-in, not a
// device address): it takes the address hipGetSymbolAddress gives on each device.
static __device__ __align__(256) float scratch[DECODE_SCRATCH_BYTES / sizeof(float)];

hipError_t decode_scratch(float **ptr) {
    constexpr int MAX_DEVICES = 64;
    static std::mutex mu;
    static float *addr[MAX_DEVICES] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= MAX_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(mu);
    if (!addr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));  // with this device current
        if (e != hipSuccess) return e;
        addr[dev] = (float *)p;
    }
    *ptr = addr[dev];
    return hipSuccess;
}

hipError_t launch_decode(const DecodeParams &P, int dtype, hipStream_t stream) {
    // V slices: ids packed by XCD, 8 VS per pair of sequences (the kernel maps them back)
    const int n_wg = P.v_slices > 1 ? 8 * P.v_slices * ((P.n_seq + 1) / 2) : P.wg_base[P.n_seq];
    dim3 grid(n_wg), block(DEC_THREADS);
    if (dtype == DT_F16 && P.v_slices == 8)
        hipLaunchKernelGGL((attn_decode_kernel<DT_F16, 8>), grid, block, 0, stream, P);
    else if (dtype == DT_BF16 && P.v_slices == 8)
        hipLaunchKernelGGL((attn_decode_kernel<DT_BF16, 8>), grid, block, 0, stream, P);
    else if (dtype == DT_F16 && P.v_slices == 4)
        hipLaunchKernelGGL((attn_decode_kernel<DT_F16, 4>), grid, block, 0, stream, P);
    else if (dtype == DT_BF16 && P.v_slices == 4)
        hipLaunchKernelGGL((attn_decode_kernel<DT_BF16, 4>), grid, block, 0, stream, P);
    else if (dtype == DT_F16 && P.v_slices == 2)
        hipLaunchKernelGGL((attn_decode_kernel<DT_F16, 2>), grid, block, 0, stream, P);
    else if (dtype == DT_F16)
        hipLaunchKernelGGL((attn_decode_kernel<DT_F16, 1>), grid, block, 0, stream, P);
    else if (P.v_slices == 2)
        hipLaunchKernelGGL((attn_decode_kernel<DT_BF16, 2>), grid, block, 0, stream, P);
    else
        hipLaunchKernelGGL((attn_decode_kernel<DT_BF16, 1>), grid, block, 0, stream, P);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (P.max_split > 1) {
        CombineParams C;
        C.partial = P.partial;
        C.sinks = P.sinks;
        C.att = P.att;
        for (int s = 0; s < MAX_SEQ; s++) {
            C.n_split[s] = s < P.n_seq ? P.n_split[s] : 0;
            C.split0[s] = s < P.n_seq ? P.split0[s] : 0;
        }
        hipLaunchKernelGGL(attn_combine_kernel, dim3(N_HEAD, P.n_seq), dim3(256), 0, stream, C);
        e = hipGetLastError();
    }
    return e;
}

}  // namespace flint
