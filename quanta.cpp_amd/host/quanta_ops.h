// quanta_ops.h — the reference engine's L1 kernel surface (engine/src/ops.h, with the Tensor view of
// engine/src/model_file.h) served by the gfx950 library. Same names, same argument meaning, same field
// layouts, so engine code written against the reference's ops.h compiles and runs unchanged:
//
//   quantize_q8      reference ops.h:52       (ops_ref.cpp:69-83)
//   matvec_q         reference ops.h:61       (MatvecQFn ops.h:57, ops_ref.cpp:85-120)
//   matmul_q         reference ops.h:69       (MatmulQFn ops.h:68, ops_ref.cpp:122-160)
//   matvec_q_kernel_name / available_matvec_q_kernels / available_matmul_q_kernels   ops.h:62-71
//   shortlist_head   reference Model::shortlist_head (model.cpp:240-334) as a free function
//
// Two ways to build against it:
//
//  - Standalone (the default): this header defines Tensor, QuantVec, DType, QK and HeadQuery itself, with the
//    reference's field layouts, and libquanta_ops.so provides every function above.
//  - Inside the reference engine (QUANTA_HIP_ENGINE defined, the engine's engine/src on the include path): the
//    types come from the engine's own model_file.h / ops.h / model.h, and this header only adds what the engine
//    lacks (HipError, shortlist_head, release_device_tensors). ops_hip.cpp built the same way replaces the engine's
//    ops_dispatch.cpp (matvec_q, matmul_q, matvec_q_kernel_name, available_*); quantize_q8 and the scalar
//    matvec_q_ref / matmul_q_ref stay the engine's own (ops_ref.cpp), so kernel_selftest checks the GPU kernels
//    against them.
//
// Pointers are HOST pointers, as in the reference. Each quantized Tensor is uploaded to the GPU the
// first time it is used (keyed by Tensor::data, so the tensor bytes must not change afterwards) and
// stays resident; activations are staged per calling thread. Calls are thread-safe and may overlap on
// disjoint [r0, r1) row ranges, as ThreadPool::parallel_for issues them (model.cpp:153, 341). The PCIe
// round trip per call makes this surface a drop-in for tests and tools; a GPU-resident engine calls the
// device-pointer C-ABI in quanta_hip.h directly.
//
// Errors: the reference's kernels return void and assume valid input; here a failing call throws
// quanta::HipError (derived from std::runtime_error) with the library's message.
#pragma once

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <utility>
#include <vector>

#if defined(QUANTA_HIP_ENGINE)

#include "model.h"  // the engine's Tensor, DType, QK (model_file.h), QuantVec and kernels (ops.h), HeadQuery

#else

namespace quanta {

enum class DType : uint32_t { F32 = 0, F16 = 1, Q8_0 = 2, Q4_0 = 3 };
constexpr int QK = 32;

// 2-D view of a weight matrix; for Q8_0 / Q4_0 the quants come first, then one fp16 scale per 32 weights.
struct Tensor {
    DType dtype = DType::F32;
    int rows = 0;
    int cols = 0;
    const uint8_t* data = nullptr;

    const float* f32() const { return reinterpret_cast<const float*>(data); }
    size_t quant_bytes() const {
        const size_t n = size_t(rows) * size_t(cols);
        switch (dtype) {
            case DType::F32: return n * 4;
            case DType::F16: return n * 2;
            case DType::Q8_0: return n;
            case DType::Q4_0: return n / 2;
        }
        return 0;
    }
    const uint16_t* scales() const { return reinterpret_cast<const uint16_t*>(data + quant_bytes()); }
};

// Activation quantized to int8 in blocks of 32 with one f32 scale per block.
struct QuantVec {
    std::vector<int8_t> q;
    std::vector<float> d;
    int n = 0;
};

// Which logits the caller needs (reference model.h:24-29).
struct HeadQuery {
    int top_k = 0;
    int n_valid = 0;
    const int* must = nullptr;
    int n_must = 0;
};

inline bool is_quantized(DType t) { return t == DType::Q8_0 || t == DType::Q4_0; }

void quantize_q8(const float* x, int n, QuantVec& out);

using MatvecQFn = void (*)(float* out, const Tensor& W, const QuantVec& x, int r0, int r1);
void matvec_q(float* out, const Tensor& W, const QuantVec& x, int r0, int r1);
const char* matvec_q_kernel_name();
std::vector<std::pair<const char*, MatvecQFn>> available_matvec_q_kernels();

using MatmulQFn = void (*)(float* out, int ldo, const Tensor& W, const QuantVec* x, int n, int r0, int r1);
void matmul_q(float* out, int ldo, const Tensor& W, const QuantVec* x, int n, int r0, int r1);
std::vector<std::pair<const char*, MatmulQFn>> available_matmul_q_kernels();

}  // namespace quanta

#endif  // QUANTA_HIP_ENGINE

namespace quanta {

struct HipError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

// Exact Shortlist Head for the hidden state already quantized in xq: fills logits[V] (exact for the
// rescored rows, -inf elsewhere) and, if given, coarse[V] / upper[V]; returns the number of 8-bit rows
// rescored (reference Model::last_head_rows). head8 Q8_0 [V][D], head4 Q4_0 [V][D], err F16 [V][D/32].
// *top1 (optional) receives the greedy token: the first argmax over [0, n_valid).
int shortlist_head(const Tensor& head8, const Tensor& head4, const Tensor& err, const QuantVec& xq,
                   const HeadQuery& hq, float* logits, int* top1 = nullptr, float* coarse = nullptr,
                   float* upper = nullptr);

// Drops every uploaded tensor (e.g. before the host memory behind Tensor::data is reused).
void release_device_tensors();

}  // namespace quanta
