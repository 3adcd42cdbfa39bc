// C entry points around the reference engine's own kernels, for parity checks only.
//
// TEST INFRASTRUCTURE ONLY. oracle/Makefile compiles this file together with the reference sources
// (engine/src/ops_ref.cpp, ops_dispatch.cpp, model_file.cpp, model.cpp, threadpool.cpp, tokenizer.cpp, sampler.cpp,
// session.cpp) into
// oracle/_ref/libquanta_ref.so. Nothing of the reference is copied here: the functions below build
// the reference's own Tensor / QuantVec / Model objects over caller buffers and call into it.
//
// Model::shortlist_head is private and Model has no way to load a hidden state other than by running
// the decoder, and Sampler keeps its generator state private, so the Model and Sampler headers are
// included with `private` widened to `public`; all standard headers they pull in are included first so
// the widening reaches only the reference's own classes.
#include <algorithm>
#include <array>
#include <chrono>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <functional>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <utility>
#include <vector>

#define private public
#include "model.h"
#include "sampler.h"
#undef private
#include "session.h"
#include "tokenizer.h"

using quanta::DType;
using quanta::QuantVec;
using quanta::Tensor;

namespace {

Tensor make_tensor(int dtype, int rows, int cols, const uint8_t* data) {
    Tensor t;
    t.dtype = DType(dtype);
    t.rows = rows;
    t.cols = cols;
    t.data = data;
    return t;
}

QuantVec make_qv(const int8_t* q, const float* d, int n) {
    QuantVec v;
    v.n = n;
    v.q.assign(q, q + n);
    v.d.assign(d, d + n / quanta::QK);
    return v;
}

}  // namespace

extern "C" {

float ref_fp16_to_f32(uint16_t h) { return quanta::fp16_to_f32(h); }

void ref_quantize_q8(const float* x, int n, int8_t* q, float* d) {
    QuantVec v;
    quanta::quantize_q8(x, n, v);
    std::memcpy(q, v.q.data(), size_t(n));
    std::memcpy(d, v.d.data(), sizeof(float) * v.d.size());
}

// Model::linear for a quantized W: ThreadPool::parallel_for(rows, 16) over matvec_q (model.cpp:150-157).
void ref_matvec_q(float* out, int dtype, int rows, int cols, const uint8_t* data, const int8_t* xq, const float* xd,
                  int n_threads) {
    const Tensor W = make_tensor(dtype, rows, cols, data);
    const QuantVec x = make_qv(xq, xd, cols);
    quanta::ThreadPool pool(n_threads);
    pool.parallel_for(rows, 16, [&](int r0, int r1) { quanta::matvec_q(out, W, x, r0, r1); });
}

// Model::linear for an F32 / F16 W: ThreadPool::parallel_for(rows, 16) over matvec_ref (model.cpp:154-156).
void ref_matvec_f(float* out, int dtype, int rows, int cols, const uint8_t* data, const float* x, int n_threads) {
    const Tensor W = make_tensor(dtype, rows, cols, data);
    quanta::ThreadPool pool(n_threads);
    pool.parallel_for(rows, 16, [&](int r0, int r1) { quanta::matvec_ref(out, W, x, r0, r1); });
}

// get_row (ops_ref.cpp:162-192) of a tensor of any dtype.
void ref_get_row(float* out, int dtype, int rows, int cols, const uint8_t* data, int row) {
    quanta::get_row(out, make_tensor(dtype, rows, cols, data), row);
}

// Seconds for `reps` calls of Model::linear on one pool (the CPU baseline's timed loop).
double ref_time_matvec_q(float* out, int dtype, int rows, int cols, const uint8_t* data, const int8_t* xq,
                         const float* xd, int n_threads, int reps) {
    const Tensor W = make_tensor(dtype, rows, cols, data);
    const QuantVec x = make_qv(xq, xd, cols);
    quanta::ThreadPool pool(n_threads);
    pool.parallel_for(rows, 16, [&](int r0, int r1) { quanta::matvec_q(out, W, x, r0, r1); });  // warm-up
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < reps; ++i)
        pool.parallel_for(rows, 16, [&](int r0, int r1) { quanta::matvec_q(out, W, x, r0, r1); });
    return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
}

// Model::linear_batch for a quantized W (model.cpp:336-347): out is [n][rows].
void ref_matmul_q(float* out, int dtype, int rows, int cols, const uint8_t* data, const int8_t* xq, const float* xd,
                  int n, int n_threads) {
    const Tensor W = make_tensor(dtype, rows, cols, data);
    std::vector<QuantVec> xs;
    xs.reserve(size_t(n));
    for (int t = 0; t < n; ++t)
        xs.push_back(make_qv(xq + size_t(t) * cols, xd + size_t(t) * (cols / quanta::QK), cols));
    quanta::ThreadPool pool(n_threads);
    pool.parallel_for(rows, 16, [&](int r0, int r1) { quanta::matmul_q(out, rows, W, xs.data(), n, r0, r1); });
}

// Model::shortlist_head (model.cpp:240-334) on a hidden state given already quantized, with the
// reference's own thread pool of n_threads. Writes logits / coarse / upper [V] and the rescored rows
// (the reference's rows_ in its own order); returns last_head_rows().
int ref_shortlist_head(const uint8_t* head8, const uint8_t* head4, const uint16_t* err, int V, int D, const int8_t* xq,
                       const float* xd, int top_k, int n_valid, const int* must, int n_must, int n_threads,
                       float* logits, float* coarse, float* upper, int* rows) {
    const Tensor t8 = make_tensor(int(DType::Q8_0), V, D, head8);
    const Tensor t4 = make_tensor(int(DType::Q4_0), V, D, head4);
    const Tensor te = make_tensor(int(DType::F16), V, D / quanta::QK, reinterpret_cast<const uint8_t*>(err));
    auto m = std::make_unique<quanta::Model>();
    m->lm_head_ = &t8;
    m->head_q4_ = &t4;
    m->head_err_ = &te;
    m->pool_ = std::make_unique<quanta::ThreadPool>(n_threads);
    m->coarse_.assign(size_t(V), 0.f);
    m->upper_.assign(size_t(V), 0.f);
    m->logits_.assign(size_t(V), 0.f);
    m->must_mark_.assign(size_t(V), 0);
    m->xnorm_.assign(size_t(D / quanta::QK), 0.f);
    m->heap_.resize(size_t(m->pool_->size()));
    m->cand_.resize(size_t(m->pool_->size()));
    m->xq_ = make_qv(xq, xd, D);
    quanta::HeadQuery hq;
    hq.top_k = top_k;
    hq.n_valid = n_valid;
    hq.must = must;
    hq.n_must = n_must;
    m->shortlist_head(hq);
    std::memcpy(logits, m->logits_.data(), sizeof(float) * size_t(V));
    std::memcpy(coarse, m->coarse_.data(), sizeof(float) * size_t(V));
    std::memcpy(upper, m->upper_.data(), sizeof(float) * size_t(V));
    std::copy(m->rows_.begin(), m->rows_.end(), rows);
    // The Model never owned these tensors; detach before it is destroyed.
    m->lm_head_ = m->head_q4_ = m->head_err_ = nullptr;
    return m->last_head_rows_;
}

// ---- whole-model entry points (model.cpp:10-228, 349-433; session.cpp:13-52; tools/cli/main.cpp:216-251)

// Loads a .qnt through Model::load with an f16 KV cache (the CLI default). Returns an opaque handle or null.
void* ref_model_load(const char* path, int ctx_len, int n_threads) {
    auto m = std::make_unique<quanta::Model>();
    std::string err;
    if (!m->load(path, ctx_len, &err, n_threads, true)) return nullptr;
    return m.release();
}

// The same with the KV cache's type chosen: kv_f16 0 is the CLI's --kv-f32 (model.cpp:96-104).
void* ref_model_load_kv(const char* path, int ctx_len, int n_threads, int kv_f16) {
    auto m = std::make_unique<quanta::Model>();
    std::string err;
    if (!m->load(path, ctx_len, &err, n_threads, kv_f16 != 0)) return nullptr;
    return m.release();
}

void ref_model_free(void* m) { delete static_cast<quanta::Model*>(m); }

// Replaces a loaded model's thread pool with one of n_threads (n <= 0: ThreadPool::default_threads()), resizing the
// per-thread shortlist state as Model::load sizes it (model.cpp:59, 93-94); returns the pool's size. Lets one
// prefilled cache be decoded at several thread counts.
int ref_model_set_threads(void* mp, int n_threads) {
    auto* m = static_cast<quanta::Model*>(mp);
    m->pool_ = std::make_unique<quanta::ThreadPool>(n_threads);
    if (m->head_q4_) {
        m->heap_.resize(size_t(m->pool_->size()));
        m->cand_.resize(size_t(m->pool_->size()));
    }
    return m->pool_->size();
}

// ThreadPool::default_threads() (threadpool.cpp:21-25): min(8, hardware threads / 2).
int ref_default_threads() { return quanta::ThreadPool::default_threads(); }

// Model::load's verdict on a file (model.cpp:10-106, model_file.cpp:104-218): 1 if it loads, else 0 with the
// reference's error message copied into msg[cap].
int ref_model_load_error(const char* path, char* msg, int cap) {
    quanta::Model m;
    std::string err;
    const bool ok = m.load(path, 16, &err, 1, true);
    if (cap > 0) {
        const size_t n = std::min(err.size(), size_t(cap - 1));
        std::memcpy(msg, err.data(), n);
        msg[n] = '\0';
    }
    return ok ? 1 : 0;
}

// Copies the state a forward leaves behind: logits [V] (exact where the head computed them, -inf elsewhere with the
// shortlist), the final normed hidden state [dim] and its quantization; returns last_head_rows().
static int ref_dump(quanta::Model* m, float* logits, float* hidden, int8_t* hq, float* hd) {
    const auto& hp = m->hparams();
    if (logits) std::memcpy(logits, m->logits_.data(), sizeof(float) * size_t(hp.vocab_size));
    if (hidden) std::memcpy(hidden, m->x_.data(), sizeof(float) * size_t(hp.dim));
    if (hq) std::memcpy(hq, m->xq_.q.data(), size_t(hp.dim));
    if (hd) std::memcpy(hd, m->xq_.d.data(), sizeof(float) * size_t(hp.dim / quanta::QK));
    return m->last_head_rows_;
}

// Model::forward for one token. top_k > 0 uses the shortlist head with n_valid = vocab, else the full head.
int ref_model_forward(void* mp, int token, int pos, int top_k, float* logits, float* hidden, int8_t* hq, float* hd) {
    auto* m = static_cast<quanta::Model*>(mp);
    quanta::HeadQuery q;
    q.top_k = top_k;
    q.n_valid = m->hparams().vocab_size;
    m->forward(token, pos, top_k > 0 ? &q : nullptr);
    return ref_dump(m, logits, hidden, hq, hd);
}

// Model::forward_batch (32-token chunks) for n tokens from pos0.
int ref_model_forward_batch(void* mp, const int* tokens, int n, int pos0, int top_k, float* logits, float* hidden,
                            int8_t* hq, float* hd) {
    auto* m = static_cast<quanta::Model*>(mp);
    quanta::HeadQuery q;
    q.top_k = top_k;
    q.n_valid = m->hparams().vocab_size;
    m->forward_batch(tokens, n, pos0, top_k > 0 ? &q : nullptr);
    return ref_dump(m, logits, hidden, hq, hd);
}

// Copies the f16 KV cache of layer l, positions [0, n_pos): k and v as [n_pos][kv_dim] fp16 bits.
void ref_model_kv(void* mp, int l, int n_pos, uint16_t* k, uint16_t* v) {
    auto* m = static_cast<quanta::Model*>(mp);
    const auto& hp = m->hparams();
    const size_t kv_dim = size_t(hp.n_kv_heads) * hp.head_dim;
    const size_t off = size_t(l) * m->ctx_len_ * kv_dim;
    std::memcpy(k, m->k_cache16_.data() + off, 2 * kv_dim * n_pos);
    std::memcpy(v, m->v_cache16_.data() + off, 2 * kv_dim * n_pos);
}

// `quanta gen --greedy --ids ... -n n_gen` (tools/cli/main.cpp:216-251): batched prefill of the prompt through a
// Session with the greedy sampler parameters (so the shortlist head answers top_k = 1 queries), then n_gen greedy
// tokens. Writes the generated ids, and per step (when non-null) the 8-bit head rows the forward before it read and the
// logit of the chosen id (its exact value, the maximum); returns the count (or -1 if the prompt does not fit).
int ref_gen(void* mp, const int* ids, int n_ids, int n_gen, int* out, int* head_rows, float* top_logit) {
    auto* m = static_cast<quanta::Model*>(mp);
    quanta::Tokenizer tok(m->file().tokenizer());
    quanta::Session s(*m, tok);
    s.set_batch_prefill(true);
    quanta::SamplerParams sp;
    sp.temperature = 0.f;
    sp.repeat_penalty = 1.f;
    s.set_sampler(&sp);
    quanta::SamplerParams greedy;
    greedy.temperature = 0.f;
    greedy.repeat_penalty = 1.f;
    quanta::Sampler sampler(greedy);
    if (!s.feed(std::vector<int>(ids, ids + n_ids), nullptr)) return -1;
    int n = 0;
    s.generate(sampler, n_gen, {}, [&](int id) {
        if (head_rows) head_rows[n] = m->last_head_rows_;
        if (top_logit) top_logit[n] = m->logits_[size_t(id)];
        out[n++] = id;
        return true;
    }, nullptr);
    return n;
}

// Sampler::sample (sampler.cpp:22-85) on logits[0, n_valid) (modified in place) with the generator state *state
// (advanced; the state a Sampler constructed with seed s starts from is s | 1).
int ref_sample(float* logits, int n_valid, const int* history, int n_hist, float temperature, int top_k, float top_p,
               float min_p, float repeat_penalty, int repeat_window, uint64_t* state) {
    quanta::SamplerParams sp;
    sp.temperature = temperature;
    sp.top_k = top_k;
    sp.top_p = top_p;
    sp.min_p = min_p;
    sp.repeat_penalty = repeat_penalty;
    sp.repeat_window = repeat_window;
    sp.seed = 1;
    quanta::Sampler s(sp);
    s.state_ = *state;
    const int id = s.sample(logits, n_valid, std::vector<int>(history, history + n_hist));
    *state = s.state_;
    return id;
}

// A Session over the model with the batched prefill (session.cpp:13-52): the head queries follow the query
// parameters q* (Session::set_sampler, session.cpp:63-79: top_k when temperature > 0, else 1; the history window as
// must ids when the repetition penalty is not 1), the tokens come from Sampler(s*, seed). With q = s this is the chat
// flow; with a greedy s it is `quanta gen` with sampling options (tools/cli/main.cpp:232-244). Writes the n_gen ids
// and per step the 8-bit head rows of the forward before it; returns the count (or -1 if the prompt does not fit).
int ref_gen_sampled(void* mp, const int* ids, int n_ids, int n_gen, float q_temperature, int q_top_k,
                    float q_repeat_penalty, int q_repeat_window, float s_temperature, int s_top_k, float s_top_p,
                    float s_min_p, float s_repeat_penalty, int s_repeat_window, uint64_t seed, int* out,
                    int* head_rows) {
    auto* m = static_cast<quanta::Model*>(mp);
    quanta::Tokenizer tok(m->file().tokenizer());
    quanta::Session s(*m, tok);
    s.set_batch_prefill(true);
    quanta::SamplerParams qp;
    qp.temperature = q_temperature;
    qp.top_k = q_top_k;
    qp.repeat_penalty = q_repeat_penalty;
    qp.repeat_window = q_repeat_window;
    s.set_sampler(&qp);
    quanta::SamplerParams sp;
    sp.temperature = s_temperature;
    sp.top_k = s_top_k;
    sp.top_p = s_top_p;
    sp.min_p = s_min_p;
    sp.repeat_penalty = s_repeat_penalty;
    sp.repeat_window = s_repeat_window;
    sp.seed = seed;
    quanta::Sampler sampler(sp);
    if (!s.feed(std::vector<int>(ids, ids + n_ids), nullptr)) return -1;
    int n = 0;
    s.generate(sampler, n_gen, {}, [&](int id) {
        if (head_rows) head_rows[n] = m->last_head_rows_;
        out[n++] = id;
        return true;
    }, nullptr);
    return n;
}

}  // extern "C"
