// C entry points around the reference engine's own kernels, for parity checks only.
//
// TEST INFRASTRUCTURE ONLY. oracle/Makefile compiles this file together with the reference sources
// (engine/src/ops_ref.cpp, ops_dispatch.cpp, model_file.cpp, model.cpp, threadpool.cpp) into
// oracle/_ref/libquanta_ref.so. Nothing of the reference is copied here: the functions below build
// the reference's own Tensor / QuantVec / Model objects over caller buffers and call into it.
//
// Model::shortlist_head is private and Model has no way to load a hidden state other than by running
// the decoder, so the Model header is included with `private` widened to `public`; all standard
// headers it pulls in are included first so the widening reaches only the reference's own classes.
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
#undef private

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

}  // extern "C"
