// Host side of the attention blocks loaded from a GGUF model (include/flint_model.h)
// and the engine's C API (include/capi.h). Compiled by hipcc as host C++.
//
// Open: map the GGUF, read the hyper-parameters with the reference's checks
// (HParams::from_gguf, /root/reference/src/ref/ref_model.cpp:13-39), check each layer's
// attention tensors against the shapes the kernels are built for, then copy the token
// embedding and the attention tensors into one HBM allocation and create the attention
// engine (KV caches; the reference's bind_layers, /root/reference/src/engine.mm:472-513).
// A block is three stream-ordered stages on the caller's stream: q/k/v projections with
// the RMSNorm fused, attention, o projection with the residual add (engine.mm:726-812
// decode, 1083-1111 prefill).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/capi.h"
#include "../../include/flint_attn.h"
#include "../../include/flint_model.h"
#include "../../include/flint_proj.h"
#include "common.h"
#include "flint_attn_internal.h"
#include "gguf.h"

namespace flint {
namespace {

void set_err(char *err, int32_t len, const char *msg) {
    if (err && len > 0) {
        std::strncpy(err, msg, len - 1);
        err[len - 1] = 0;
    }
}

void check(hipError_t e, const char *what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// a library call's 0 / -1 turned into an exception carrying its message
void call(int32_t rc, const char *msg) {
    if (rc != 0) throw std::runtime_error(msg);
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

struct HParams {
    flint_attn_hparams h{};
    std::vector<uint8_t> is_swa, has_rope;
};

// The reference's HParams::from_gguf: the same keys, the same order of reads (so a file
// with several problems reports the same first one) and the same routing check.
HParams read_hparams(const gguf::File &f) {
    HParams p;
    const std::string arch = f.get_string("general.architecture");
    if (arch != "flint") throw std::runtime_error("not a flint model: " + arch);
    auto k = [&](const char *s) { return arch + "." + s; };
    auto i32 = [&](const char *s) { return (int32_t)f.get_int(k(s)); };
    flint_attn_hparams &h = p.h;
    h.n_layer = i32("block_count");
    h.n_embd = i32("embedding_length");
    h.n_head = i32("attention.head_count");
    h.n_head_kv = i32("attention.head_count_kv");
    h.head_dim = i32("attention.key_length");
    h.n_ff_dense = i32("feed_forward_length");
    h.n_ff_exp = i32("expert_feed_forward_length");
    h.n_ff_shexp = i32("expert_shared_feed_forward_length");
    h.n_expert = i32("expert_count");
    h.n_expert_used = i32("expert_used_count");
    h.n_dense_lead = i32("leading_dense_block_count");
    h.n_swa = i32("attention.sliding_window");
    h.rms_eps = (float)f.get_float(k("attention.layer_norm_rms_epsilon"));
    h.rope_theta = (float)f.get_float(k("rope.freq_base"));
    p.is_swa = f.get_bool_array(k("attention.sliding_window_pattern"));
    p.has_rope = f.get_bool_array(k("attention.rope_pattern"));
    const gguf::Tensor &out = f.tensor("output.weight");
    h.n_vocab = out.dims.size() > 1 ? (int32_t)out.dims[1] : 0;
    if (f.get_int(k("expert_gating_func")) != 2 || !f.get_bool(k("expert_weights_norm")) ||
        f.get_float(k("expert_weights_scale")) != 1.0)
        throw std::runtime_error("unexpected routing config (expect sigmoid + norm, scale 1)");
    // the reference indexes the layer patterns without a bound check
    if (h.n_layer <= 0) throw std::runtime_error("flint: block_count must be > 0");
    if ((int)p.is_swa.size() < h.n_layer || (int)p.has_rope.size() < h.n_layer)
        throw std::runtime_error("flint: the sliding-window and rope patterns need one entry per layer (" +
                                 std::to_string(h.n_layer) + ")");
    p.is_swa.resize(h.n_layer);
    p.has_rope.resize(h.n_layer);
    return p;
}

// The kernels are built for Flint's attention shapes (flint_config.h:12-17).
void check_shapes(const HParams &p) {
    const flint_attn_hparams &h = p.h;
    if (h.n_embd != FLINT_N_EMBD || h.n_head != FLINT_N_HEAD || h.n_head_kv != FLINT_N_HEAD_KV ||
        h.head_dim != FLINT_HEAD_DIM)
        throw std::runtime_error("unsupported attention shape: n_embd " + std::to_string(h.n_embd) + ", heads " +
                                 std::to_string(h.n_head) + "/" + std::to_string(h.n_head_kv) + ", head_dim " +
                                 std::to_string(h.head_dim) + " (this library serves 2048, 32/4, 128)");
    if (h.n_swa < 1 || h.n_swa > FLINT_SWA_RING)
        throw std::runtime_error("attention.sliding_window must be in [1, " + std::to_string(FLINT_SWA_RING) + "]");
}

bool proj_type(uint32_t t) {
    return t == FLINT_W_F32 || t == FLINT_W_F16 || t == FLINT_W_BF16 || t == FLINT_W_Q8_0 || t == FLINT_W_Q5_K ||
           t == FLINT_W_Q6_K || t == FLINT_W_IQ4_XS;
}

const gguf::Tensor &want(const gguf::File &f, const std::string &name, uint64_t d0, uint64_t d1, bool f32_only) {
    const gguf::Tensor &t = f.tensor(name);
    const bool shape = d1 ? t.dims.size() == 2 && t.dims[0] == d0 && t.dims[1] == d1
                          : t.dims.size() == 1 && t.dims[0] == d0;
    if (!shape)
        throw std::runtime_error("tensor " + name + " has the wrong shape (want " + std::to_string(d0) +
                                 (d1 ? " x " + std::to_string(d1) : std::string()) + ")");
    if (f32_only ? t.type != FLINT_W_F32 : !proj_type(t.type))
        throw std::runtime_error(std::string("no kernel for type ") + gguf::type_name(t.type) + " (" + name + ")");
    return t;
}

// bytes of one 2048-element row of a projection type (proj_type() has accepted it)
int64_t w_row_bytes_of(uint32_t type) { return flint_w_row_bytes((int32_t)type, FLINT_N_EMBD); }

constexpr size_t kAlign = 256;  // every tensor's copy starts 256-byte aligned in HBM

}  // namespace
}  // namespace flint

using namespace flint;

struct flint_attn_model {
    std::unique_ptr<gguf::File> file;
    HParams hp;
    flint_attn_engine *eng = nullptr;
    void *wmem = nullptr;  // every tensor the blocks read, one allocation
    struct Layer {
        flint_weight q, k, v, o;
        const float *attn_norm;
    };
    std::vector<Layer> layers;
    flint_weight embd{};
    int64_t embd_rows = 0;
    // scratch: raw q|k|v rows and attention outputs for up to `cap` tokens
    float *qkv = nullptr, *att = nullptr;
    int cap = 0;
    int32_t n_ctx = 0, pos = 0;  // the session: context length and tokens processed
    // The prefill GEMMs' f16 hi/lo planes of every layer's q|k|v and o weights (75.5 MB a layer;
    // 40.1 MB in q8_0, whose GEMM keeps the integer values and the block scales), one allocation made at
    // the first prefill block that takes the GEMM, layer il's at planes_off[il]; a layer's planes are built
    // on the stream of its first such block and read by every later one. planes_on: the caller's
    // switch (flint_attn_model_set_weight_planes). A failed allocation is tried once per prefill
    // call (planes_failed_call: the call it failed in), and the projections rebuild the planes in
    // the workspace meanwhile.
    void *planes = nullptr;
    bool planes_on = true;
    uint64_t prefill_call = 0, planes_failed_call = 0;
    std::vector<uint8_t> planes_built;
    std::vector<size_t> planes_off;
    // Engine::last_gpu_ms and its profiler (enable_profiling / last_profile, engine.h:54-56, 63):
    // marks are HIP events recorded on the call's stream, mark 0 where a step or prefill starts,
    // then one where it ends or, with profiling on, one after each stage (the embedding, then per
    // layer its q/k/v projection, attention and o projection). labels[i] names the stage between
    // marks i and i + 1. marks_done: the last step or prefill recorded all its marks.
    bool profiling = false, marks_done = false;
    double encode_ms = -1.0;  // host time the last step / prefill took to enqueue its work (Engine::last_encode_ms)
    std::vector<hipEvent_t> marks;
    std::vector<std::string> labels;
    int n_marks = 0;

    ~flint_attn_model() {
        for (hipEvent_t e : marks) (void)hipEventDestroy(e);
        flint_attn_engine_destroy(eng);
        if (wmem) (void)hipFree(wmem);
        if (qkv) (void)hipFree(qkv);
        if (att) (void)hipFree(att);
        if (planes) (void)hipFree(planes);
    }
    static size_t qkv_planes_bytes(const Layer &L) {
        return planes_bytes(FLINT_QKV_DIM, FLINT_N_EMBD, qkv_gemm_form(&L.q, &L.k, &L.v));
    }
    static size_t layer_planes_bytes(const Layer &L) {
        return qkv_planes_bytes(L) + planes_bytes(FLINT_N_EMBD, FLINT_Q_DIM, o_gemm_form(&L.o));
    }
    // the layer's q|k|v and o planes, built on `stream` if this is the first use; false when
    // there is no memory for them
    bool layer_planes(int il, hipStream_t stream, WeightPlanes *pq_out, WeightPlanes *po_out) {
        if (!planes_on) return false;
        if (!planes) {
            if (planes_failed_call == prefill_call) return false;  // already failed in this call
            planes_off.assign(layers.size() + 1, 0);
            for (size_t i = 0; i < layers.size(); i++) planes_off[i + 1] = planes_off[i] + layer_planes_bytes(layers[i]);
            if (hipMalloc(&planes, planes_off.back()) != hipSuccess) {
                (void)hipGetLastError();  // clear the allocation error; the projections work without planes
                planes = nullptr;
                planes_failed_call = prefill_call;
                return false;
            }
            planes_failed_call = 0;
            planes_built.assign(layers.size(), 0);
        }
        const Layer &L = layers[il];
        char *base = (char *)planes + planes_off[il];
        const WeightPlanes pq = planes_at(base, FLINT_QKV_DIM, FLINT_N_EMBD, qkv_gemm_form(&L.q, &L.k, &L.v));
        const WeightPlanes po = planes_at(base + qkv_planes_bytes(L), FLINT_N_EMBD, FLINT_Q_DIM, o_gemm_form(&L.o));
        if (!planes_built[il]) {
            build_qkv_planes(&L.q, &L.k, &L.v, pq, stream);
            build_o_planes(&L.o, po, stream);
            planes_built[il] = 1;
        }
        *pq_out = pq;
        *po_out = po;
        return true;
    }
    void reserve(int n_tok) {
        if (n_tok <= cap) return;
        // earlier calls' kernels may still read the old buffers (they run on the callers' streams)
        if (qkv || att) check(hipDeviceSynchronize(), "hipDeviceSynchronize");
        if (qkv) check(hipFree(qkv), "hipFree");
        if (att) check(hipFree(att), "hipFree");
        qkv = att = nullptr;
        cap = 0;
        check(hipMalloc((void **)&qkv, (size_t)n_tok * FLINT_QKV_DIM * sizeof(float)), "hipMalloc qkv scratch");
        check(hipMalloc((void **)&att, (size_t)n_tok * FLINT_Q_DIM * sizeof(float)), "hipMalloc att scratch");
        cap = n_tok;
    }
    void begin_marks(hipStream_t s) {
        n_marks = 0;
        marks_done = false;
        encode_ms = -1.0;
        labels.clear();
        mark(s, nullptr);
    }
    // the mark after a stage (label: the stage's name; none for mark 0)
    void mark(hipStream_t s, const char *label) {
        if (n_marks == (int)marks.size()) {
            // a device-scope release where each mark is recorded (the default is system scope);
            // a mark still adds a few microseconds to the stream (0.4-0.9 ms over a profiled
            // step's 148 marks)
            hipEvent_t e;
            check(hipEventCreateWithFlags(&e, hipEventReleaseToDevice), "hipEventCreateWithFlags");
            marks.push_back(e);
        }
        check(hipEventRecord(marks[n_marks], s), "hipEventRecord");
        if (n_marks > 0) labels.emplace_back(label);
        n_marks++;
    }
    // the mark after stage `what` of layer il, when profiling
    void stage(hipStream_t s, bool prof, int il, const char *what) {
        if (!prof) return;
        char label[32];
        std::snprintf(label, sizeof(label), "blk.%d.%s", il, what);
        mark(s, label);
    }
    const Layer &layer(int il) const {
        if (il < 0 || il >= (int)layers.size()) throw std::runtime_error("model: bad layer index");
        return layers[il];
    }
};

extern "C" {

flint_attn_model *flint_attn_model_open(const char *gguf_path, int32_t n_ctx, int32_t kv_dtype, char *err,
                                        int32_t err_len) {
    try {
        if (!gguf_path) throw std::runtime_error("flint_attn_model_open: no model path");
        if (n_ctx <= 0) throw std::runtime_error("flint_attn_model_open: n_ctx must be > 0");
        if (kv_dtype != FLINT_KV_F16 && kv_dtype != FLINT_KV_BF16)
            throw std::runtime_error("flint_attn_model_open: kv_dtype must be F16 or BF16");
        auto m = std::make_unique<flint_attn_model>();
        m->n_ctx = n_ctx;
        m->file = std::make_unique<gguf::File>(gguf_path);
        const gguf::File &f = *m->file;
        m->hp = read_hparams(f);
        check_shapes(m->hp);
        const int n_layer = m->hp.h.n_layer;

        // every tensor the blocks read, checked before any device work
        struct Copy {
            const gguf::Tensor *t;
            size_t at;
        };
        std::vector<Copy> copies;
        size_t total = 0;
        auto place = [&](const gguf::Tensor &t) {
            copies.push_back({&t, total});
            total += (t.nbytes + kAlign - 1) / kAlign * kAlign;
            return copies.size() - 1;
        };
        const gguf::Tensor &te = f.tensor("token_embd.weight");
        if (te.dims.size() != 2 || te.dims[0] != (uint64_t)FLINT_N_EMBD || !proj_type(te.type))
            throw std::runtime_error("token_embd.weight: want 2048-element rows of a supported type");
        const size_t c_embd = place(te);
        struct Idx {
            size_t norm, q, k, v, o;
            const gguf::Tensor *qn, *kn, *sk;
        };
        std::vector<Idx> idx(n_layer);
        for (int il = 0; il < n_layer; il++) {
            const std::string b = "blk." + std::to_string(il) + ".";
            Idx &x = idx[il];
            x.norm = place(want(f, b + "attn_norm.weight", FLINT_N_EMBD, 0, true));
            x.q = place(want(f, b + "attn_q.weight", FLINT_N_EMBD, FLINT_Q_DIM, false));
            x.k = place(want(f, b + "attn_k.weight", FLINT_N_EMBD, FLINT_KV_DIM, false));
            x.v = place(want(f, b + "attn_v.weight", FLINT_N_EMBD, FLINT_KV_DIM, false));
            x.o = place(want(f, b + "attn_output.weight", FLINT_Q_DIM, FLINT_N_EMBD, false));
            x.qn = &want(f, b + "attn_q_norm.weight", FLINT_HEAD_DIM, 0, true);
            x.kn = &want(f, b + "attn_k_norm.weight", FLINT_HEAD_DIM, 0, true);
            x.sk = &want(f, b + "attn_sinks.weight", FLINT_N_HEAD, 0, true);
        }

        // device side
        check(hipMalloc(&m->wmem, total), "hipMalloc model weights");
        for (const Copy &c : copies)
            check(hipMemcpy((char *)m->wmem + c.at, c.t->data, c.t->nbytes, hipMemcpyHostToDevice), "hipMemcpy weights");
        auto dev = [&](size_t i) { return (const void *)((const char *)m->wmem + copies[i].at); };
        auto weight = [&](size_t i) { return flint_weight{dev(i), (int32_t)copies[i].t->type}; };
        m->embd = weight(c_embd);
        // rows the copy holds (the reader has checked dims[0] * dims[1] against the tensor's bytes)
        m->embd_rows = (int64_t)std::min<uint64_t>(te.dims[1], te.nbytes / (uint64_t)w_row_bytes_of(te.type));
        char e2[512] = {0};
        m->eng = flint_attn_engine_create(n_layer, m->hp.is_swa.data(), m->hp.has_rope.data(), n_ctx, kv_dtype,
                                          m->hp.h.rope_theta, e2, sizeof(e2));
        if (!m->eng) throw std::runtime_error(e2);
        m->layers.resize(n_layer);
        for (int il = 0; il < n_layer; il++) {
            const Idx &x = idx[il];
            m->layers[il] = {weight(x.q), weight(x.k), weight(x.v), weight(x.o), (const float *)dev(x.norm)};
            call(flint_attn_engine_set_weights(m->eng, il, (const float *)x.qn->data, (const float *)x.kn->data,
                                               (const float *)x.sk->data, e2, sizeof(e2)),
                 e2);
            engine_set_layer_params(m->eng, il, m->hp.h.n_swa, m->hp.h.rms_eps);
        }
        return m.release();
    } catch (const std::exception &ex) {
        set_err(err, err_len, ex.what());
        return nullptr;
    }
}

void flint_attn_model_close(flint_attn_model *m) { delete m; }

int32_t flint_attn_model_hparams(const flint_attn_model *m, flint_attn_hparams *hp, uint8_t *is_swa,
                                 uint8_t *has_rope) {
    if (!m || !hp) return -1;
    *hp = m->hp.h;
    if (is_swa) std::memcpy(is_swa, m->hp.is_swa.data(), m->hp.is_swa.size());
    if (has_rope) std::memcpy(has_rope, m->hp.has_rope.data(), m->hp.has_rope.size());
    return 0;
}

flint_attn_engine *flint_attn_model_engine(flint_attn_model *m) { return m ? m->eng : nullptr; }

int32_t flint_attn_model_embed(flint_attn_model *m, const int32_t *tokens, int32_t n, float *x, void *stream,
                               char *err, int32_t err_len) {
    return guarded(err, err_len, [&] {
        if (!m) throw std::runtime_error("embed: no model");
        if (!tokens || !x || n <= 0) throw std::runtime_error("embed: bad arguments");
        for (int i = 0; i < n; i++)
            if (tokens[i] < 0 || tokens[i] >= m->embd_rows)
                throw std::runtime_error("embed: token " + std::to_string(tokens[i]) + " out of range");
        char e2[512] = {0};
        call(flint_w_get_rows(m->embd.type, m->embd.data, FLINT_N_EMBD, m->embd_rows, tokens, n, x, stream, e2,
                              sizeof(e2)),
             e2);
    });
}

}  // extern "C"

namespace {

// A decode block; prof: a stage mark after each of its three stages (a profiled step).
void block_decode(flint_attn_model *m, int il, float *x, int pos, float *att, void *stream, bool prof) {
    if (!m) throw std::runtime_error("block_decode: no model");
    const flint_attn_model::Layer &L = m->layer(il);
    if (!x) throw std::runtime_error("block_decode: x is NULL");
    m->reserve(1);
    float *a = att ? att : m->att;
    char e2[512] = {0};
    const hipStream_t s = (hipStream_t)stream;
    call(flint_attn_qkv_proj(&L.q, &L.k, &L.v, x, L.attn_norm, m->hp.h.rms_eps, m->qkv, stream, e2, sizeof(e2)), e2);
    m->stage(s, prof, il, "qkv");
    call(flint_attn_engine_decode(m->eng, il, m->qkv, a, pos, stream, e2, sizeof(e2)), e2);
    m->stage(s, prof, il, "attn");
    call(flint_attn_o_proj(&L.o, a, x, stream, e2, sizeof(e2)), e2);
    m->stage(s, prof, il, "o");
}

// A prefill block over T tokens; prof as for block_decode.
void block_prefill(flint_attn_model *m, int il, float *X, int p0, int T, float *att, void *stream, bool prof) {
    if (!m) throw std::runtime_error("block_prefill: no model");
    const flint_attn_model::Layer &L = m->layer(il);
    if (!X) throw std::runtime_error("block_prefill: X is NULL");
    if (T <= 0) throw std::runtime_error("prefill: empty");
    m->reserve(T);
    float *a = att ? att : m->att;
    char e2[512] = {0};
    const hipStream_t s = (hipStream_t)stream;
    WeightPlanes pq, po;
    if (T >= GEMM_MIN_TOKENS && m->layer_planes(il, s, &pq, &po)) {
        // the projections' GEMMs read the layer's cached weight planes
        qkv_proj_rows_planes(&L.q, &L.k, &L.v, X, T, L.attn_norm, m->hp.h.rms_eps, m->qkv, FLINT_QKV_DIM, &pq, s);
        m->stage(s, prof, il, "qkv");
        call(flint_attn_engine_prefill(m->eng, il, m->qkv, p0, T, a, stream, e2, sizeof(e2)), e2);
        m->stage(s, prof, il, "attn");
        o_proj_rows_planes(&L.o, a, T, X, &po, s);
        m->stage(s, prof, il, "o");
        return;
    }
    call(flint_attn_qkv_proj_rows(&L.q, &L.k, &L.v, X, T, L.attn_norm, m->hp.h.rms_eps, m->qkv, FLINT_QKV_DIM,
                                  stream, e2, sizeof(e2)),
         e2);
    m->stage(s, prof, il, "qkv");
    call(flint_attn_engine_prefill(m->eng, il, m->qkv, p0, T, a, stream, e2, sizeof(e2)), e2);
    m->stage(s, prof, il, "attn");
    call(flint_attn_o_proj_rows(&L.o, a, T, X, stream, e2, sizeof(e2)), e2);
    m->stage(s, prof, il, "o");
}

}  // namespace

extern "C" {

int32_t flint_attn_model_block_decode(flint_attn_model *m, int32_t il, float *x, int32_t pos, float *att,
                                      void *stream, char *err, int32_t err_len) {
    return guarded(err, err_len, [&] { block_decode(m, il, x, pos, att, stream, false); });
}

int32_t flint_attn_model_block_prefill(flint_attn_model *m, int32_t il, float *X, int32_t p0, int32_t T,
                                       float *att, void *stream, char *err, int32_t err_len) {
    return guarded(err, err_len, [&] {
        if (m) m->prefill_call++;
        block_prefill(m, il, X, p0, T, att, stream, false);
    });
}

int32_t flint_attn_model_set_weight_planes(flint_attn_model *m, int32_t on, char *err, int32_t err_len) {
    return guarded(err, err_len, [&] {
        if (!m) throw std::runtime_error("set_weight_planes: no model");
        m->planes_on = on != 0;
        m->planes_failed_call = 0;
        if (!m->planes_on && m->planes) {
            // the planes may still be read by work queued on any stream
            check(hipDeviceSynchronize(), "set_weight_planes: device synchronize");
            check(hipFree(m->planes), "set_weight_planes: free");
            m->planes = nullptr;
            m->planes_built.clear();
        }
    });
}

int32_t flint_attn_model_weight_planes(const flint_attn_model *m) {
    if (!m) return -2;
    if (!m->planes_on) return 0;
    if (m->planes) return 1;
    return m->planes_failed_call ? -1 : 2;
}

int32_t flint_attn_model_enable_profiling(flint_attn_model *m, int32_t on) {
    if (!m) return -1;
    m->profiling = on != 0;
    return 0;
}

double flint_attn_model_last_gpu_ms(flint_attn_model *m) {
    if (!m || !m->marks_done || m->n_marks < 2) return -1.0;
    hipEvent_t e0 = m->marks[0], e1 = m->marks[m->n_marks - 1];
    float ms = 0.f;
    if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess) return -1.0;
    return ms;
}

double flint_attn_model_last_encode_ms(const flint_attn_model *m) {
    return m && m->marks_done ? m->encode_ms : -1.0;
}

int32_t flint_attn_model_last_profile(flint_attn_model *m, char *labels, int32_t label_len, double *ms,
                                      int32_t max_n) {
    if (!m || !m->marks_done || m->n_marks < 2) return -1;
    const int n = m->n_marks - 1;
    if (!ms || max_n <= 0) return n;
    if (hipEventSynchronize(m->marks[n]) != hipSuccess) return -1;
    for (int i = 0; i < n && i < max_n; i++) {
        float t = 0.f;
        if (hipEventElapsedTime(&t, m->marks[i], m->marks[i + 1]) != hipSuccess) return -1;
        ms[i] = t;
        if (labels && label_len > 0) set_err(labels + (size_t)i * label_len, label_len, m->labels[i].c_str());
    }
    return n;
}

int32_t flint_attn_model_pos(const flint_attn_model *m) { return m ? m->pos : 0; }
int32_t flint_attn_model_n_ctx(const flint_attn_model *m) { return m ? m->n_ctx : 0; }

int32_t flint_attn_model_truncate(flint_attn_model *m, int32_t pos) {
    if (!m || pos < 0 || pos > m->pos) return -1;
    m->pos = pos;
    return 0;
}

int32_t flint_attn_model_step(flint_attn_model *m, int32_t token, float *x, void *stream, char *err,
                              int32_t err_len) {
    return guarded(err, err_len, [&] {
        if (!m) throw std::runtime_error("step: no model");
        if (!x) throw std::runtime_error("step: x is NULL");
        if (m->pos >= m->n_ctx) throw std::runtime_error("context full");
        const hipStream_t s = (hipStream_t)stream;
        const bool prof = m->profiling;
        const auto t0 = std::chrono::steady_clock::now();
        char e2[512] = {0};
        m->begin_marks(s);
        call(flint_attn_model_embed(m, &token, 1, x, stream, e2, sizeof(e2)), e2);
        if (prof) m->mark(s, "embed");
        for (int il = 0; il < (int)m->layers.size(); il++) block_decode(m, il, x, m->pos, nullptr, stream, prof);
        if (!prof) m->mark(s, "step");
        m->marks_done = true;
        m->encode_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        m->pos++;
    });
}

int32_t flint_attn_model_prefill(flint_attn_model *m, const int32_t *tokens, int32_t n, float *X, void *stream,
                                 char *err, int32_t err_len) {
    return guarded(err, err_len, [&] {
        if (!m) throw std::runtime_error("prefill: no model");
        if (!tokens || n <= 0) throw std::runtime_error("prefill: empty");
        if (!X) throw std::runtime_error("prefill: X is NULL");
        if ((int64_t)m->pos + n > m->n_ctx) throw std::runtime_error("prefill: context full");
        m->prefill_call++;
        const hipStream_t s = (hipStream_t)stream;
        const bool prof = m->profiling;
        const auto t0 = std::chrono::steady_clock::now();
        char e2[512] = {0};
        m->begin_marks(s);
        call(flint_attn_model_embed(m, tokens, n, X, stream, e2, sizeof(e2)), e2);
        if (prof) m->mark(s, "embed");
        for (int il = 0; il < (int)m->layers.size(); il++) block_prefill(m, il, X, m->pos, n, nullptr, stream, prof);
        if (!prof) m->mark(s, "prefill");
        m->marks_done = true;
        m->encode_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        m->pos += n;
    });
}

}  // extern "C"

// ---------------------------------------------------------------------------
// The engine's C API (include/capi.h; /root/reference/src/capi.mm:1-78). flint_open
// reads and validates the model exactly as far as the attention blocks need; the FFN,
// MoE experts and output head are not part of this library, so it then fails with a
// message that says so.

struct flint_engine {
    int32_t n_ctx = 0;
    int32_t pos = 0;
    std::vector<float> logits;
};

extern "C" {

flint_engine *flint_open(const flint_config *cfg, char *err, int32_t err_len) {
    try {
        if (!cfg || !cfg->model_path) throw std::runtime_error("flint_open: no model path");
        gguf::File f(cfg->model_path);
        const HParams p = read_hparams(f);
        check_shapes(p);
        throw std::runtime_error(
            "flint_open: this library implements the attention blocks only (flint_attn_model_open); the FFN, "
            "MoE experts and output head of this " +
            std::to_string(p.h.n_layer) + "-layer model are not part of this build");
    } catch (const std::exception &ex) {
        set_err(err, err_len, ex.what());
        return nullptr;
    }
}

void flint_close(flint_engine *e) { delete e; }

int32_t flint_n_ctx(const flint_engine *e) { return e ? e->n_ctx : 0; }
int32_t flint_n_vocab(void) { return 150144; }
int32_t flint_pos(const flint_engine *e) { return e ? e->pos : 0; }

int32_t flint_truncate(flint_engine *e, int32_t pos) {
    if (!e || pos < 0 || pos > e->pos) return -1;
    e->pos = pos;
    return 0;
}

int32_t flint_prefill(flint_engine *e, const int32_t *tokens, int32_t n, char *err, int32_t err_len) {
    if (!e) {
        set_err(err, err_len, "flint_prefill: no engine");
        return -1;
    }
    if (!tokens || n <= 0) {
        set_err(err, err_len, "prefill: empty");
        return -1;
    }
    set_err(err, err_len, "flint_prefill: the FFN and output head are not part of this build");
    return -1;
}

int32_t flint_decode(flint_engine *e, int32_t token, char *err, int32_t err_len) {
    (void)token;
    if (!e) {
        set_err(err, err_len, "flint_decode: no engine");
        return -1;
    }
    set_err(err, err_len, "flint_decode: the FFN and output head are not part of this build");
    return -1;
}

const float *flint_logits(const flint_engine *e) { return e && !e->logits.empty() ? e->logits.data() : nullptr; }

}  // extern "C"
