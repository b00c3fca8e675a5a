// Host side of the flint attention hot path: argument checks, launch plans,
// device workspaces, the per-layer KV-cache engine and the C ABI of the attention
// stage and the projections (include/flint_attn.h, include/flint_proj.h). Compiled by
// hipcc as host C++.
//
// Stage scheduling mirrors the reference engine's attention stages
// (/root/reference/src/engine.mm:735-766 decode, 1077-1104 prefill): one
// stream-ordered launch sequence per layer on the caller's stream.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/flint_attn.h"
#include "../../include/flint_proj.h"
#include "common.h"
#include "flint_attn_internal.h"

namespace flint {
namespace {

struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

void set_err(char *err, int32_t len, const char *msg) {
    if (err && len > 0) {
        std::strncpy(err, msg, len - 1);
        err[len - 1] = 0;
    }
}

void check(hipError_t e, const char *what) {
    if (e != hipSuccess) throw Error(std::string(what) + ": " + hipGetErrorString(e));
}

template <typename F>
int32_t guarded(char *err, int32_t err_len, F &&f) {
    try {
        f();
        return 0;
    } catch (const std::exception &ex) {
        set_err(err, err_len, ex.what());
        return -1;
    }
}

// theta^(-2i/128) with the CPU reference's float expression (ref_model.cpp:55)
void rope_freqs(float theta, float *freq) {
    for (int i = 0; i < HEAD_DIM / 2; i++) freq[i] = std::pow(theta, -2.0f * i / HEAD_DIM);
}

// Device scratch that grows on demand, one set per device.
struct Workspace {
    void *ptr = nullptr;
    size_t bytes = 0;
    void *get(size_t need, bool zero = false) {
        if (need <= bytes) return ptr;
        // earlier launches on any stream may still use the old buffer
        if (ptr) check(hipDeviceSynchronize(), "hipDeviceSynchronize");
        if (ptr) check(hipFree(ptr), "hipFree");
        ptr = nullptr;
        bytes = 0;
        check(hipMalloc(&ptr, need), "hipMalloc workspace");
        if (zero) check(hipMemset(ptr, 0, need), "hipMemset workspace");
        bytes = need;
        return ptr;
    }
};

struct DeviceScratch {
    Workspace partial, kv, gemm, pf_part;
};

std::mutex g_scratch_mu;
std::vector<std::unique_ptr<DeviceScratch>> g_scratch;

DeviceScratch &scratch() {
    int dev = 0;
    check(hipGetDevice(&dev), "hipGetDevice");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if ((int)g_scratch.size() <= dev) g_scratch.resize(dev + 1);
    if (!g_scratch[dev]) g_scratch[dev] = std::make_unique<DeviceScratch>();
    return *g_scratch[dev];
}

void validate_layer(const flint_attn_layer *L) {
    if (!L) throw Error("layer is NULL");
    if (!L->k_cache || !L->v_cache) throw Error("layer KV cache pointer is NULL");
    if (!L->q_norm || !L->k_norm || !L->sinks) throw Error("layer q_norm/k_norm/sinks pointer is NULL");
    if (L->kv_dtype != FLINT_KV_F16 && L->kv_dtype != FLINT_KV_BF16) throw Error("kv_dtype must be F16 or BF16");
    if (L->n_slots <= 0 || L->n_slots % 32 != 0) throw Error("n_slots must be a positive multiple of 32");
    if (L->n_slots > FLINT_MAX_SLOTS)
        throw Error("n_slots must be at most " + std::to_string(FLINT_MAX_SLOTS) + " (32-bit cache offsets)");
    if (L->window < 1) throw Error("window must be >= 1");
    if (((uintptr_t)L->q_norm | (uintptr_t)L->k_norm) & 15) throw Error("q_norm/k_norm must be 16-byte aligned");
    if (L->is_swa) {
        if (L->n_slots & (L->n_slots - 1)) throw Error("SWA ring size must be a power of two");
        if (L->n_slots < L->window) throw Error("SWA ring must hold the window (n_slots >= window)");
    }
}

// Split plan: 32-key tiles per split, per sequence. An 8-wave block is one CU's share.
// Every sequence takes one split while a workgroup's 8 waves need at most 3 tiles each
// (a grid of at most 4 x 64 workgroups, one round of the CUs): the split merge kernel costs
// more than streaming those tiles through one CU. Otherwise the key tiles of all sequences are spread over about 192 workgroups
// (measured on MI355X at 16k-64k keys: ~170-210 workgroups of longer streams beat one per
// CU, e.g. 15.6 vs 17.2 us per call at 32k, 25.1 vs 27.5 at 64k), each sequence's range cut
// into equal splits (a multiple of 4 tiles, 8 at least): the launch lasts as long as its
// longest split, and with one split length for every sequence the short remainders of the
// others left HBM idle at the end (16 sequences at 4k-65k: 221 vs 262 us per layer).
// keys_per_split > 0 overrides the plan with that split length for every sequence.
void plan_splits(int n_seq, const int *tiles, int keys_per_split, int *n_split, int *tps) {
    int total = 0, max_tiles = 0;
    for (int s = 0; s < n_seq; s++) total += tiles[s], max_tiles = std::max(max_tiles, tiles[s]);
    for (int s = 0; s < n_seq; s++) {
        int t;
        if (keys_per_split > 0) {
            t = std::max(1, keys_per_split / 32);
        } else if (max_tiles <= 3 * 8) {
            t = std::max(max_tiles, 1);
        } else {
            const int target_blocks = 192;
            // this sequence's share of the workgroups, then equal splits of its range
            const int64_t want = ((int64_t)tiles[s] * target_blocks + (int64_t)total * N_HEAD_KV - 1) /
                                 ((int64_t)total * N_HEAD_KV);
            const int ns = std::max<int64_t>(1, want);
            t = std::max(8, ((tiles[s] + ns - 1) / ns + 3) / 4 * 4);
        }
        tps[s] = t;
        n_split[s] = std::max(1, (tiles[s] + t - 1) / t);
    }
}

// theta^(-2i/128) table, cached for the last theta
void rope_freqs_cached(float theta, float *freq) {
    static thread_local float last_theta = -1.f, table[HEAD_DIM / 2];
    if (theta != last_theta) {
        rope_freqs(theta, table);
        last_theta = theta;
    }
    std::memcpy(freq, table, sizeof(table));
}

constexpr int PART_STRIDE = 132;

// no_alloc: the split partials go to the library's static device array (decode_scratch), and
// nothing is allocated on the device.
void decode_impl(const flint_attn_layer *L, int n_seq, int64_t seq_stride, const float *qkv, float *att,
                 const int32_t *pos, int32_t keys_per_split, hipStream_t stream, bool no_alloc = false) {
    validate_layer(L);
    if (n_seq < 1 || n_seq > MAX_SEQ) throw Error("n_seq must be in [1, " + std::to_string(MAX_SEQ) + "]");
    if (!qkv || !att || !pos) throw Error("qkv/att/pos pointer is NULL");
    if (keys_per_split < 0 || keys_per_split % 32 != 0) throw Error("keys_per_split must be a multiple of 32");
    if (n_seq > 1 && seq_stride < (int64_t)N_HEAD_KV * L->n_slots * HEAD_DIM)
        throw Error("seq_stride smaller than one sequence's cache");
    DecodeParams P{};
    P.qkv = qkv;
    P.q_norm = L->q_norm;
    P.k_norm = L->k_norm;
    P.sinks = L->sinks;
    P.k_cache = (uint16_t *)L->k_cache;
    P.v_cache = (uint16_t *)L->v_cache;
    P.seq_stride = seq_stride;
    P.att = att;
    P.n_slots = L->n_slots;
    P.slot_mask = L->is_swa ? L->n_slots - 1 : 0x7fffffff;
    P.is_swa = L->is_swa;
    P.has_rope = L->has_rope;
    P.window = L->window;
    P.rms_eps = L->rms_eps;
    rope_freqs_cached(L->rope_theta, P.rope_freq);
    P.n_seq = n_seq;
    int tiles[MAX_SEQ];
    for (int s = 0; s < n_seq; s++) {
        const int p = pos[s];
        if (p < 0) throw Error("position must be >= 0");
        if (!L->is_swa && p >= L->n_slots) throw Error("context full: position beyond the layer's KV capacity");
        const int k_begin = L->is_swa ? std::max(p - (L->window - 1), 0) : 0;
        tiles[s] = p > 0 ? (p + 31) / 32 - k_begin / 32 : 0;
    }
    plan_splits(n_seq, tiles, keys_per_split, P.n_split, P.tps);
    int max_split = 1;
    for (int s = 0; s < n_seq; s++) max_split = std::max(max_split, P.n_split[s]);
    // One split per sequence (short key ranges, SWA layers): one CU streams each kv head's
    // keys (~36 GB/s per CU from HBM, ~63 GB/s from the caches), so 8 (or 4, 2) workgroups per
    // kv head, each reading all of K and its slice of V, shorten the stream without a merge. The
    // launch puts a kv head's slices on one XCD, so the K they all read comes from HBM once and
    // from that XCD's L2 after. Measured on SWA layers (513 keys, rings in the caches): 8.1 us per
    // call with one workgroup per kv head, 6.3 with 2, 5.7 with 4; 16 sequences: 9.8, 9.6, 9.1 us.
    // Cold rings (as a decode step meets them): 7.09 us with 4 slices on two XCDs, 6.62 with 8 on
    // two XCDs, 6.49 with 8 on one.
    P.v_slices = max_split > 1                          ? 1
                 : n_seq * N_HEAD_KV * 8 <= 256 ? 8
                 : n_seq * N_HEAD_KV * 4 <= 256 ? 4
                 : n_seq * N_HEAD_KV * 2 <= 256 ? 2
                                                : 1;
    P.wg_base[0] = 0;
    int n_records = 0;  // partial records (in splits) of the launch: sequences of more than one split
    for (int s = 0; s < n_seq; s++) {
        P.pos[s] = pos[s];
        P.wg_base[s + 1] = P.wg_base[s] + N_HEAD_KV * P.v_slices * P.n_split[s];
        P.split0[s] = n_records;
        if (P.n_split[s] > 1) n_records += P.n_split[s];
    }
    for (int s = n_seq + 1; s <= MAX_SEQ; s++) P.wg_base[s] = P.wg_base[n_seq];
    P.max_split = max_split;
    if (max_split > 1024) throw Error("too many key splits (max 1024): raise keys_per_split");
    if (max_split > 1) {
        // one record per (split, head) of the sequences with more than one split
        const size_t need = (size_t)n_records * N_HEAD * PART_STRIDE * sizeof(float);
        if (no_alloc) {
            if (need > DECODE_SCRATCH_BYTES)
                throw Error("flint_attn_decode_batch_noalloc: the split plan needs " + std::to_string(need) +
                            " bytes of partials, more than the " + std::to_string(DECODE_SCRATCH_BYTES) +
                            " bytes this entry point holds (" +
                            std::to_string(DECODE_SCRATCH_BYTES / (N_HEAD * PART_STRIDE * sizeof(float))) +
                            " key splits over the batch's sequences of more than one split): use fewer "
                            "sequences or a larger keys_per_split");
            check(decode_scratch(&P.partial), "decode scratch address");
        } else {
            P.partial = (float *)scratch().partial.get(need);
        }
    }
    check(launch_decode(P, L->kv_dtype, stream), "decode launch");
}

void prefill_impl(const flint_attn_layer *L, const float *qkv, int q_stride, int p0, int T, float *att,
                  hipStream_t stream) {
    validate_layer(L);
    if (!qkv || !att) throw Error("qkv/att pointer is NULL");
    if (T <= 0) throw Error("prefill: empty");
    if (p0 < 0) throw Error("prefill: negative start position");
    if (q_stride < QKV_DIM || q_stride % 4 != 0) throw Error("q_stride must be >= 5120 and a multiple of 4");
    if (!L->is_swa && p0 + T > L->n_slots) throw Error("prefill: context full");
    PrefillParams P{};
    P.qkv = qkv;
    P.q_stride = q_stride;
    P.p0 = p0;
    P.T = T;
    P.q_norm = L->q_norm;
    P.k_norm = L->k_norm;
    P.sinks = L->sinks;
    P.rms_eps = L->rms_eps;
    P.is_swa = L->is_swa;
    P.has_rope = L->has_rope;
    P.window = L->window;
    rope_freqs_cached(L->rope_theta, P.rope_freq);
    P.att = att;
    P.cache_k = (uint16_t *)L->k_cache;
    P.cache_v = (uint16_t *)L->v_cache;
    P.n_slots = L->n_slots;
    if (L->is_swa) {
        P.cache_mask = L->n_slots - 1;
        P.cache_from = std::max(p0, p0 + T - L->n_slots);  // the ring keeps the last n_slots
        P.kbase = std::max(0, p0 - (L->window - 1)) & ~31;  // 32-aligned: chunks line up with tiles
    } else {
        P.cache_mask = -1;
        P.cache_from = p0;
        P.kbase = 0;
    }
    // f16 caches: whole tiles of cached positions are read in place instead of converted into the
    // copy, for short calls (T <= 256). The flash kernel that can read cache tiles runs its loop
    // ~7% slower, which at 32768 cached positions equals the conversion it saves at T ~ 512
    // (measured per call: T = 1 42.7 against 62.8 us, T = 64 77.1 against 95.1 us). On a ring,
    // kv_prep rewrites the slots of positions p0 - n_slots .. p0 + T - 1 - n_slots; with
    // T <= n_slots - window + 1 those lie before p0 - (window - 1), outside every new query's
    // window (masked keys).
    if (L->kv_dtype == FLINT_KV_F16 && T <= 256 && (!L->is_swa || T <= L->n_slots - L->window + 1))
        P.n_direct = (p0 - P.kbase) >> 5;
    // the attention copy holds the positions from tile n_direct on, then its table of per-tile
    // exponents (every tile the flash kernel reads from it is written in this call, padding
    // rows included): a short call at a long context needs only its own few tiles
    P.k_rows = ((p0 + T - P.kbase - 32 * P.n_direct) + PREFILL_ROW_ALIGN - 1) / PREFILL_ROW_ALIGN * PREFILL_ROW_ALIGN;
    const size_t copy_bytes = (size_t)N_HEAD_KV * P.k_rows * 2 * HEAD_DIM * sizeof(_Float16);
    char *ws = (char *)scratch().kv.get(copy_bytes + (size_t)N_HEAD_KV * (P.k_rows / 32) * sizeof(int));
    P.sk = (_Float16 *)ws;
    P.texp = (int *)(ws + copy_bytes);
    // a nonzero id per call: the kernels flag a call that stored scaled tiles with its id
    static std::atomic<uint32_t> next_call{0};
    uint32_t id = ++next_call;
    if (id == 0) id = ++next_call;
    P.call_id = id;
    // Key splits when the grid of (query block, kv head) workgroups would leave most CUs idle on
    // a long key range (a short prefill at a long context: one workgroup per kv head would stream
    // the whole cache through one CU). Splits of the longest block's tiles, 8 at least, so the
    // launch has about 512 workgroups; the merge kernel adds the sink.
    {
        const int nqb = (T + 31) / 32;
        // tiles of the longest query block: the last one on a full layer; on an SWA layer at
        // most the 18 tiles that a 32-query block's window [first - (window - 1), first + 31] spans
        const int longest = L->is_swa ? std::min(((p0 + T - 1 - P.kbase) >> 5) + 1, (L->window + 62) / 32 + 1)
                                      : ((p0 + T - 1) >> 5) + 1;
        const int base = nqb * N_HEAD_KV;
        int ns = 1;
        if (base < 256 && longest >= 16)
            ns = std::min({PF_MAX_SPLIT, (512 + base - 1) / base, (longest + 7) / 8});
        const int tps = (longest + ns - 1) / ns;
        P.n_split = (longest + tps - 1) / tps;
        P.tps = P.n_split > 1 ? tps : 1 << 24;
        if (P.n_split > 1)
            P.part = (float *)scratch().pf_part.get((size_t)P.n_split * T * N_HEAD * PF_PART_STRIDE * sizeof(float));
    }
    check(launch_prefill(P, L->kv_dtype, stream), "prefill launch");
}

// ---- attention projections (include/flint_proj.h) ----

int64_t w_row_bytes(int type, int64_t k) {
    int be = 0, bb = 0;
    switch (type) {
        case W_F32: be = 1, bb = 4; break;
        case W_F16: case W_BF16: be = 1, bb = 2; break;
        case W_Q8_0: be = 32, bb = 34; break;
        case W_Q5_K: be = 256, bb = 176; break;
        case W_Q6_K: be = 256, bb = 210; break;
        case W_IQ4_XS: be = 256, bb = 136; break;
        default: return -1;
    }
    if (k <= 0 || k % be || k % 32) return -1;
    return k / be * bb;
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

// rows[0 .. n) of a tensor with rows of k elements into out[i * k ..], GR_MAX_ROWS per launch
void get_rows_impl(int type, const void *w, int64_t k, const int64_t *rows, int64_t n_rows_max, int n, float *out,
                   hipStream_t stream, const char *what) {
    const std::string tag(what);
    const int64_t rb = w_row_bytes(type, k);
    if (rb < 0) throw Error(tag + ": unsupported weight type or row length");
    if (!w || !out || !rows) throw Error(tag + ": NULL pointer");
    if (n < 1) throw Error(tag + ": no rows");
    if (k > (int64_t)1 << 30) throw Error(tag + ": row too long");
    if (!aligned16(out)) throw Error(tag + ": out must be 16-byte aligned");
    if (((uintptr_t)w & 1) || (rb & 1)) throw Error(tag + ": row data must be 2-byte aligned");
    for (int i = 0; i < n; i++) {
        if (rows[i] < 0) throw Error(tag + ": negative row");
        if (n_rows_max >= 0 && rows[i] >= n_rows_max)
            throw Error(tag + ": row " + std::to_string(rows[i]) + " out of range");
        if (rows[i] > (int64_t)INT32_MAX) throw Error(tag + ": row index too large");
    }
    RowsParams P{};
    P.w = (const uint8_t *)w;
    P.row_bytes = rb;
    P.out_stride = k;
    P.type = type;
    P.n_sub = (int)(k / 32);
    for (int i0 = 0; i0 < n; i0 += GR_MAX_ROWS) {
        P.n = std::min(GR_MAX_ROWS, n - i0);
        P.out = out + (size_t)i0 * (size_t)k;
        for (int i = 0; i < P.n; i++) P.rows[i] = (int)rows[i0 + i];
        check(launch_get_rows(P, stream), (tag + " launch").c_str());
    }
}

// rows of k elements of one matvec tensor: 16-byte aligned rows are what the kernel reads
void check_weight(const flint_weight *w, int64_t k, const char *name) {
    if (!w || !w->data) throw Error(std::string(name) + ": NULL weight");
    const int64_t rb = w_row_bytes(w->type, k);
    if (rb < 0) throw Error(std::string(name) + ": unsupported weight type");
    if (rb % 16 || !aligned16(w->data)) throw Error(std::string(name) + ": rows must be 16-byte aligned");
}

void check_tokens(int n_tok, const char *name) {
    if (n_tok < 1 || n_tok > 1 << 20) throw Error(std::string(name) + ": n_tok must be in [1, 2^20]");
}

// A batch of T tokens through one projection on the matrix cores (proj_gemm.hip): the weight
// rows of the segments and the activation rows as f16 hi/lo planes in the device workspace, then
// y[t][0:N] (+)= W x[t] (x RMSNorm'd with norm_w when given). The tokens go through in passes of
// at most GEMM_PASS_TOKENS, so the workspace has a fixed ceiling (the weight planes once, built in
// the first pass, and one pass's activation planes).
// pl: the weights' planes, kept by the caller (then no weight prep here); build_only: only build
// them into *pl
void proj_gemm(const MatvecSeg *seg, int n_seg, int N, int K, const float *x, long long x_stride, const float *norm_w,
               float eps, int T, float *y, long long y_stride, int add, const WeightPlanes *pl, hipStream_t stream,
               bool build_only = false) {
    const int T_pass = build_only ? 0 : std::min(T, GEMM_PASS_TOKENS);
    const int T_pad = (T_pass + GEMM_TILE - 1) / GEMM_TILE * GEMM_TILE;
    const size_t wbytes = pl ? 0 : (size_t)N * K * sizeof(_Float16), xbytes = (size_t)T_pad * K * sizeof(_Float16);
    size_t off = 0;
    auto take = [&](size_t b) {
        const size_t o = off;
        off += (b + 255) / 256 * 256;
        return o;
    };
    const size_t o_wh = take(wbytes), o_wl = take(wbytes), o_f = take(pl ? 0 : (size_t)N * sizeof(int));
    const IntForm form = gemm_int_form(seg, n_seg);
    const size_t o_xh = take(xbytes), o_xl = take(xbytes), o_e = take((size_t)T_pad * sizeof(int));
    const size_t o_xs = take(form.min ? (size_t)T_pad * (K / 32) * sizeof(float) : 0);
    char *ws = off ? (char *)scratch().gemm.get(off) : nullptr;
    GemmWeightParams W{};
    for (int i = 0; i < n_seg; i++) W.seg[i] = seg[i];
    W.n_seg = n_seg;
    W.wh = pl ? pl->wh : (_Float16 *)(ws + o_wh);
    W.wl = pl ? pl->wl : (_Float16 *)(ws + o_wl);
    W.fexp = pl ? pl->fexp : (int *)(ws + o_f);
    // every segment in the integer form: the values in wh, the scales, then the mins, in wl's
    // memory (N K (1 / sub + 1 / 32) floats: in the workspace with room to spare, in kept planes
    // laid out for it)
    W.isub = form.sub, W.imin = form.min;
    W.wd = (float *)W.wl;
    W.wm = form.sub ? W.wd + (size_t)N * (K / form.sub) : nullptr;
    if (pl && !W.isub && !pl->fexp) throw Error("projection GEMM: weight planes laid out for the integer form");
    GemmActParams X{};
    X.norm_w = norm_w;
    X.eps = eps;
    X.xh = (_Float16 *)(ws + o_xh);
    X.xl = (_Float16 *)(ws + o_xl);
    X.eexp = (int *)(ws + o_e);
    X.xs = form.min ? (float *)(ws + o_xs) : nullptr;
    GemmParams G{};
    G.wh = W.wh, G.wl = W.wl, G.fexp = W.fexp, G.xh = X.xh, G.xl = X.xl, G.eexp = X.eexp;
    G.isub = W.isub, G.imin = W.imin, G.wd = W.wd, G.wm = W.wm, G.xs = X.xs;
    G.add = add;
    G.N = N;
    G.K = K;
    if (build_only) {
        X.x = x, X.x_stride = x_stride, X.T = 0, X.T_pad = 0;
        G.y = y, G.y_stride = y_stride, G.T = 0;
        check(launch_proj_gemm(W, X, G, true, stream), "projection GEMM launch");
        return;
    }
    for (int t0 = 0; t0 < T; t0 += GEMM_PASS_TOKENS) {
        const int n = std::min(GEMM_PASS_TOKENS, T - t0);
        X.x = x + (size_t)t0 * x_stride;
        X.x_stride = x_stride;
        X.T = n;
        X.T_pad = (n + GEMM_TILE - 1) / GEMM_TILE * GEMM_TILE;
        G.y = y + (size_t)t0 * y_stride;
        G.y_stride = y_stride;
        G.T = n;
        // the weight planes are built once, in the first pass, unless the caller keeps them
        check(launch_proj_gemm(W, X, G, !pl && t0 == 0, stream), "projection GEMM launch");
    }
}

// the GEMM takes batches of GEMM_MIN_TOKENS and more whose output rows are 16-byte aligned
bool use_gemm(int n_tok, const float *y, long long y_stride) {
    return n_tok >= GEMM_MIN_TOKENS && aligned16(y) && y_stride % 4 == 0;
}

// the q/k/v segments of a layer's weights
void qkv_segs(const flint_weight *wq, const flint_weight *wk, const flint_weight *wv, MatvecSeg *seg) {
    check_weight(wq, N_EMBD, "wq");
    check_weight(wk, N_EMBD, "wk");
    check_weight(wv, N_EMBD, "wv");
    const flint_weight *ws[3] = {wq, wk, wv};
    const int row0[3] = {0, Q_DIM, Q_DIM + KV_DIM};
    for (int i = 0; i < 3; i++)
        seg[i] = MatvecSeg{(const uint8_t *)ws[i]->data, ws[i]->type, row0[i], (int)w_row_bytes(ws[i]->type, N_EMBD)};
}

void qkv_proj_impl(const flint_weight *wq, const flint_weight *wk, const flint_weight *wv, const float *x, int n_tok,
                   const float *attn_norm, float eps, float *qkv, int qkv_stride, hipStream_t stream,
                   const WeightPlanes *pl = nullptr) {
    check_weight(wq, N_EMBD, "wq");
    check_weight(wk, N_EMBD, "wk");
    check_weight(wv, N_EMBD, "wv");
    check_tokens(n_tok, "qkv_proj");
    if (!x || !attn_norm || !qkv) throw Error("qkv_proj: NULL pointer");
    if (!aligned16(x) || !aligned16(attn_norm)) throw Error("qkv_proj: x and attn_norm must be 16-byte aligned");
    if (qkv_stride < QKV_DIM) throw Error("qkv_proj: qkv_stride must be >= 5120");
    MatvecParams P{};
    P.n_tok = n_tok;
    P.x_stride = N_EMBD;
    P.y_stride = qkv_stride;
    const flint_weight *ws[3] = {wq, wk, wv};
    const int row0[3] = {0, Q_DIM, Q_DIM + KV_DIM};
    for (int i = 0; i < 3; i++)
        P.seg[i] = MatvecSeg{(const uint8_t *)ws[i]->data, ws[i]->type, row0[i], (int)w_row_bytes(ws[i]->type, N_EMBD)};
    P.n_seg = 3;
    P.n_rows = QKV_DIM;
    static_assert(Q_DIM % 16 == 0 && KV_DIM % 16 == 0, "segments must hold whole row groups");
    if (QKV_DIM % matvec_row_multiple(N_EMBD)) throw Error("qkv_proj: row grouping");
    P.x = x;
    P.norm_w = attn_norm;
    P.eps = eps;
    P.y = qkv;
    P.add = 0;
    if (use_gemm(n_tok, qkv, qkv_stride)) {
        proj_gemm(P.seg, 3, QKV_DIM, N_EMBD, x, N_EMBD, attn_norm, eps, n_tok, qkv, qkv_stride, 0, pl, stream);
        return;
    }
    check(launch_matvec(P, N_EMBD, stream), "qkv_proj launch");
}

void o_proj_impl(const flint_weight *wo, const float *att, int n_tok, float *x, hipStream_t stream,
                 const WeightPlanes *pl = nullptr) {
    check_weight(wo, Q_DIM, "wo");
    check_tokens(n_tok, "o_proj");
    if (!att || !x) throw Error("o_proj: NULL pointer");
    if (!aligned16(att)) throw Error("o_proj: att must be 16-byte aligned");
    MatvecParams P{};
    P.n_tok = n_tok;
    P.x_stride = Q_DIM;
    P.y_stride = N_EMBD;
    P.seg[0] = MatvecSeg{(const uint8_t *)wo->data, wo->type, 0, (int)w_row_bytes(wo->type, Q_DIM)};
    P.n_seg = 1;
    P.n_rows = N_EMBD;
    if (N_EMBD % matvec_row_multiple(Q_DIM)) throw Error("o_proj: row grouping");
    P.x = att;
    P.y = x;
    P.add = 1;
    if (use_gemm(n_tok, x, N_EMBD)) {
        proj_gemm(P.seg, 1, N_EMBD, Q_DIM, att, Q_DIM, nullptr, 0.f, n_tok, x, N_EMBD, 1, pl, stream);
        return;
    }
    check(launch_matvec(P, Q_DIM, stream), "o_proj launch");
}

}  // namespace

// none when a segment is not of the integer form; else the smallest of their scale spans, and
// whether any has mins
static IntForm int_form_of(const int *types, int n) {
    IntForm f;
    f.sub = n > 0 ? 32 : 0;
    for (int i = 0; i < n; i++) f.sub = std::min(f.sub, w_int_sub(types[i])), f.min = f.min || w_int_min(types[i]);
    if (!f.sub) f.min = false;
    return f;
}

IntForm gemm_int_form(const MatvecSeg *seg, int n_seg) {
    int t[3];
    for (int i = 0; i < n_seg; i++) t[i] = seg[i].type;
    return int_form_of(t, n_seg);
}

IntForm qkv_gemm_form(const flint_weight *wq, const flint_weight *wk, const flint_weight *wv) {
    const int t[3] = {wq->type, wk->type, wv->type};
    return int_form_of(t, 3);
}

IntForm o_gemm_form(const flint_weight *wo) { return int_form_of(&wo->type, 1); }

static size_t align256(size_t b) { return (b + 255) / 256 * 256; }

size_t planes_bytes(int N, int K, IntForm f) {
    const size_t w = align256((size_t)N * K * sizeof(_Float16));
    if (f.sub) return w + align256((size_t)N * (K / f.sub + (f.min ? K / 32 : 0)) * sizeof(float));
    return 2 * w + align256((size_t)N * sizeof(int));
}

WeightPlanes planes_at(void *mem, int N, int K, IntForm f) {
    const size_t w = align256((size_t)N * K * sizeof(_Float16));
    WeightPlanes pl;
    pl.wh = (_Float16 *)mem;
    pl.wl = (_Float16 *)((char *)mem + w);
    pl.fexp = f.sub ? nullptr : (int *)((char *)mem + 2 * w);
    return pl;
}

void build_qkv_planes(const flint_weight *wq, const flint_weight *wk, const flint_weight *wv, const WeightPlanes &pl,
                      hipStream_t stream) {
    MatvecSeg seg[3];
    qkv_segs(wq, wk, wv, seg);
    proj_gemm(seg, 3, QKV_DIM, N_EMBD, nullptr, 0, nullptr, 0.f, 0, nullptr, 0, 0, &pl, stream, true);
}

void build_o_planes(const flint_weight *wo, const WeightPlanes &pl, hipStream_t stream) {
    check_weight(wo, Q_DIM, "wo");
    const MatvecSeg seg{(const uint8_t *)wo->data, wo->type, 0, (int)w_row_bytes(wo->type, Q_DIM)};
    proj_gemm(&seg, 1, N_EMBD, Q_DIM, nullptr, 0, nullptr, 0.f, 0, nullptr, 0, 0, &pl, stream, true);
}

void qkv_proj_rows_planes(const flint_weight *wq, const flint_weight *wk, const flint_weight *wv, const float *x,
                          int n_tok, const float *attn_norm, float eps, float *qkv, int qkv_stride,
                          const WeightPlanes *pl, hipStream_t stream) {
    qkv_proj_impl(wq, wk, wv, x, n_tok, attn_norm, eps, qkv, qkv_stride, stream, pl);
}

void o_proj_rows_planes(const flint_weight *wo, const float *att, int n_tok, float *x, const WeightPlanes *pl,
                        hipStream_t stream) {
    o_proj_impl(wo, att, n_tok, x, stream, pl);
}

}  // namespace flint

using namespace flint;

extern "C" {

int64_t flint_w_row_bytes(int32_t type, int64_t k) { return w_row_bytes(type, k); }

int32_t flint_w_get_row(int32_t type, const void *w, int64_t k, int64_t row, float *out, void *stream, char *err,
                        int32_t err_len) {
    return guarded(err, err_len, [&] { get_rows_impl(type, w, k, &row, -1, 1, out, (hipStream_t)stream, "get_row"); });
}

int32_t flint_w_get_rows(int32_t type, const void *w, int64_t k, int64_t n_rows, const int32_t *rows, int32_t n,
                         float *out, void *stream, char *err, int32_t err_len) {
    return guarded(err, err_len, [&] {
        if (!rows) throw Error("get_rows: NULL pointer");
        if (n < 1 || n > 1 << 24) throw Error("get_rows: n must be in [1, 2^24]");
        if (n_rows < 1) throw Error("get_rows: n_rows must be >= 1");
        std::vector<int64_t> r(rows, rows + n);
        get_rows_impl(type, w, k, r.data(), n_rows, n, out, (hipStream_t)stream, "get_rows");
    });
}

int32_t flint_attn_qkv_proj(const flint_weight *wq, const flint_weight *wk, const flint_weight *wv, const float *x,
                            const float *attn_norm, float rms_eps, float *qkv, void *stream, char *err,
                            int32_t err_len) {
    return guarded(err, err_len,
                   [&] { qkv_proj_impl(wq, wk, wv, x, 1, attn_norm, rms_eps, qkv, QKV_DIM, (hipStream_t)stream); });
}

int32_t flint_attn_o_proj(const flint_weight *wo, const float *att, float *x, void *stream, char *err,
                          int32_t err_len) {
    return guarded(err, err_len, [&] { o_proj_impl(wo, att, 1, x, (hipStream_t)stream); });
}

int32_t flint_attn_qkv_proj_rows(const flint_weight *wq, const flint_weight *wk, const flint_weight *wv,
                                 const float *x, int32_t n_tok, const float *attn_norm, float rms_eps, float *qkv,
                                 int32_t qkv_stride, void *stream, char *err, int32_t err_len) {
    return guarded(err, err_len, [&] {
        qkv_proj_impl(wq, wk, wv, x, n_tok, attn_norm, rms_eps, qkv, qkv_stride, (hipStream_t)stream);
    });
}

int32_t flint_attn_o_proj_rows(const flint_weight *wo, const float *att, int32_t n_tok, float *x, void *stream,
                               char *err, int32_t err_len) {
    return guarded(err, err_len, [&] { o_proj_impl(wo, att, n_tok, x, (hipStream_t)stream); });
}

}  // extern "C"

// ---------------------------------------------------------------------------
// engine object

struct flint_attn_engine {
    struct LayerMem {
        flint_attn_layer desc{};
        void *kv = nullptr;   // K then V
        float *w = nullptr;   // q_norm[128] k_norm[128] sinks[32]
    };
    std::vector<LayerMem> layers;
    ~flint_attn_engine() {
        for (auto &l : layers) {
            if (l.kv) (void)hipFree(l.kv);
            if (l.w) (void)hipFree(l.w);
        }
    }
};

extern "C" {

int32_t flint_attn_decode(const flint_attn_layer *layer, const float *qkv, float *att, int32_t pos,
                          int32_t keys_per_split, void *stream, char *err, int32_t err_len) {
    return guarded(err, err_len, [&] { decode_impl(layer, 1, 0, qkv, att, &pos, keys_per_split, (hipStream_t)stream); });
}

int32_t flint_attn_decode_batch(const flint_attn_layer *layer, int32_t n_seq, int64_t seq_stride, const float *qkv,
                                float *att, const int32_t *pos, int32_t keys_per_split, void *stream, char *err,
                                int32_t err_len) {
    return guarded(err, err_len, [&] {
        decode_impl(layer, n_seq, seq_stride, qkv, att, pos, keys_per_split, (hipStream_t)stream);
    });
}

int32_t flint_attn_decode_batch_noalloc(const flint_attn_layer *layer, int32_t n_seq, int64_t seq_stride,
                                        const float *qkv, float *att, const int32_t *pos, int32_t keys_per_split,
                                        void *stream, char *err, int32_t err_len) {
    return guarded(err, err_len, [&] {
        decode_impl(layer, n_seq, seq_stride, qkv, att, pos, keys_per_split, (hipStream_t)stream, true);
    });
}

int32_t flint_attn_prefill(const flint_attn_layer *layer, const float *qkv, int32_t q_stride, int32_t p0, int32_t T,
                           float *att, void *stream, char *err, int32_t err_len) {
    return guarded(err, err_len, [&] { prefill_impl(layer, qkv, q_stride, p0, T, att, (hipStream_t)stream); });
}

int32_t flint_attn_sync(char *err, int32_t err_len) {
    return guarded(err, err_len, [&] { check(hipDeviceSynchronize(), "hipDeviceSynchronize"); });
}

flint_attn_engine *flint_attn_engine_create(int32_t n_layer, const uint8_t *is_swa, const uint8_t *has_rope,
                                            int32_t n_ctx, int32_t kv_dtype, float rope_theta, char *err,
                                            int32_t err_len) {
    try {
        if (n_layer <= 0 || !is_swa || !has_rope) throw Error("engine: n_layer > 0 and the layer flags are required");
        if (n_ctx <= 0) throw Error("engine: n_ctx must be > 0");
        if (n_ctx > FLINT_MAX_SLOTS)
            throw Error("engine: n_ctx must be at most " + std::to_string(FLINT_MAX_SLOTS) + " (32-bit cache offsets)");
        if (kv_dtype != FLINT_KV_F16 && kv_dtype != FLINT_KV_BF16) throw Error("engine: kv_dtype must be F16 or BF16");
        auto e = std::make_unique<flint_attn_engine>();
        e->layers.resize(n_layer);
        // default weights until set_weights: unit norm gains, zero sinks
        std::vector<float> init(HEAD_DIM * 2 + N_HEAD, 0.f);
        std::fill(init.begin(), init.begin() + 2 * HEAD_DIM, 1.f);
        for (int il = 0; il < n_layer; il++) {
            auto &L = e->layers[il];
            const int n_slots = is_swa[il] ? FLINT_SWA_RING : (n_ctx + 31) / 32 * 32;
            const size_t kv_bytes = (size_t)N_HEAD_KV * n_slots * HEAD_DIM * 2;
            check(hipMalloc(&L.kv, 2 * kv_bytes), "hipMalloc KV cache");
            check(hipMemset(L.kv, 0, 2 * kv_bytes), "hipMemset KV cache");
            check(hipMalloc((void **)&L.w, init.size() * sizeof(float)), "hipMalloc layer weights");
            check(hipMemcpy(L.w, init.data(), init.size() * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy");
            L.desc.k_cache = L.kv;
            L.desc.v_cache = (char *)L.kv + kv_bytes;
            L.desc.n_slots = n_slots;
            L.desc.kv_dtype = kv_dtype;
            L.desc.is_swa = is_swa[il] != 0;
            L.desc.has_rope = has_rope[il] != 0;
            L.desc.window = FLINT_N_SWA;
            L.desc.rope_theta = rope_theta;
            L.desc.rms_eps = 1e-6f;
            L.desc.q_norm = L.w;
            L.desc.k_norm = L.w + HEAD_DIM;
            L.desc.sinks = L.w + 2 * HEAD_DIM;
        }
        return e.release();
    } catch (const std::exception &ex) {
        set_err(err, err_len, ex.what());
        return nullptr;
    }
}

void flint_attn_engine_destroy(flint_attn_engine *e) { delete e; }

int32_t flint_attn_engine_n_layer(const flint_attn_engine *e) { return e ? (int32_t)e->layers.size() : 0; }

const flint_attn_layer *flint_attn_engine_layer(const flint_attn_engine *e, int32_t il) {
    if (!e || il < 0 || il >= (int32_t)e->layers.size()) return nullptr;
    return &e->layers[il].desc;
}

}  // extern "C"

void flint::engine_set_layer_params(flint_attn_engine *e, int il, int window, float rms_eps) {
    if (!flint_attn_engine_layer(e, il)) throw Error("engine: bad layer index");
    if (window < 1 || (e->layers[il].desc.is_swa && window > e->layers[il].desc.n_slots))
        throw Error("engine: SWA window must be in [1, ring size]");
    e->layers[il].desc.window = window;
    e->layers[il].desc.rms_eps = rms_eps;
}

extern "C" {

int32_t flint_attn_engine_set_weights(flint_attn_engine *e, int32_t il, const float *q_norm, const float *k_norm,
                                      const float *sinks, char *err, int32_t err_len) {
    return guarded(err, err_len, [&] {
        if (!flint_attn_engine_layer(e, il)) throw Error("engine: bad layer index");
        if (!q_norm || !k_norm || !sinks) throw Error("engine: weight pointer is NULL");
        float *w = e->layers[il].w;
        check(hipMemcpy(w, q_norm, HEAD_DIM * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy q_norm");
        check(hipMemcpy(w + HEAD_DIM, k_norm, HEAD_DIM * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy k_norm");
        check(hipMemcpy(w + 2 * HEAD_DIM, sinks, N_HEAD * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy sinks");
    });
}

int32_t flint_attn_engine_decode(flint_attn_engine *e, int32_t il, const float *qkv, float *att, int32_t pos,
                                 void *stream, char *err, int32_t err_len) {
    return guarded(err, err_len, [&] {
        const flint_attn_layer *L = flint_attn_engine_layer(e, il);
        if (!L) throw Error("engine: bad layer index");
        decode_impl(L, 1, 0, qkv, att, &pos, 0, (hipStream_t)stream);
    });
}

int32_t flint_attn_engine_prefill(flint_attn_engine *e, int32_t il, const float *qkv, int32_t p0, int32_t T,
                                  float *att, void *stream, char *err, int32_t err_len) {
    return guarded(err, err_len, [&] {
        const flint_attn_layer *L = flint_attn_engine_layer(e, il);
        if (!L) throw Error("engine: bad layer index");
        prefill_impl(L, qkv, QKV_DIM, p0, T, att, (hipStream_t)stream);
    });
}

int32_t flint_attn_engine_debug_attn(flint_attn_engine *e, int32_t il, const float *qkv, int32_t n_tok, int32_t chunk,
                                     float *out, char *err, int32_t err_len) {
    return guarded(err, err_len, [&] {
        const flint_attn_layer *L = flint_attn_engine_layer(e, il);
        if (!L) throw Error("engine: bad layer index");
        if (!qkv || !out || n_tok <= 0 || chunk <= 0) throw Error("debug_attn: bad arguments");
        float *dq = nullptr, *dout = nullptr;
        struct Free {
            float *&a, *&b;
            ~Free() {
                if (a) (void)hipFree(a);
                if (b) (void)hipFree(b);
            }
        } fr{dq, dout};
        check(hipMalloc((void **)&dq, (size_t)n_tok * QKV_DIM * sizeof(float)), "hipMalloc");
        check(hipMalloc((void **)&dout, (size_t)n_tok * Q_DIM * sizeof(float)), "hipMalloc");
        check(hipMemcpy(dq, qkv, (size_t)n_tok * QKV_DIM * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy");
        for (int p0 = 0; p0 < n_tok; p0 += chunk) {
            const int T = std::min(chunk, n_tok - p0);
            prefill_impl(L, dq + (size_t)p0 * QKV_DIM, QKV_DIM, p0, T, dout + (size_t)p0 * Q_DIM, nullptr);
        }
        check(hipMemcpy(out, dout, (size_t)n_tok * Q_DIM * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy");
    });
}

}  // extern "C"
