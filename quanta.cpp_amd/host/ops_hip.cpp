// Host-pointer implementation of quanta_ops.h over the C-ABI (quanta_hip.h). Host C++ only: it needs no
// HIP headers and can be built with any C++17 compiler.
//
// Built with QUANTA_HIP_ENGINE inside the reference engine, it takes the place of engine/src/ops_dispatch.cpp
// (matvec_q, matmul_q, matvec_q_kernel_name, available_*, ops.h:57-71): quantize_q8 then stays the engine's own
// (ops_ref.cpp:69-83, bit-identical to the GPU's), and the kernel lists name the engine's scalar "ref" kernels first,
// as ops_dispatch.cpp does, so kernel_selftest (checks.cpp:64-146) times both families and checks "hip" against
// "ref".
#include "quanta_ops.h"

#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>

#include "quanta_hip.h"

namespace quanta {
namespace {

void check(int rc, const char* what) {
    if (rc != QH_OK) throw HipError(std::string(what) + ": " + qh_last_error());
}

void ensure_init() {
    static const int rc = qh_init(0);  // once per process, thread-safe
    check(rc, "qh_init");
}

struct Resident {
    void* ptr = nullptr;
    qh_tensor view{};
};

std::mutex g_mu;
std::unordered_map<const uint8_t*, Resident> g_resident;

size_t device_bytes(const Tensor& W) {
    size_t b = W.quant_bytes();
    if (is_quantized(W.dtype)) b += size_t(W.rows) * W.cols / QK * 2;
    return b;
}

// Per-thread stream and staging memory; reused across calls, never shrunk.
struct Staging {
    void* stream = nullptr;
    void* dev = nullptr;
    size_t dev_cap = 0;
    std::vector<uint8_t> host;

    Staging() { check(qh_stream_create(&stream), "qh_stream_create"); }
    uint8_t* device(size_t bytes) {
        if (bytes > dev_cap) {
            check(qh_stream_sync(stream), "qh_stream_sync");
            check(qh_free(dev), "qh_free");
            dev = nullptr;
            dev_cap = 0;
            check(qh_malloc(&dev, bytes), "qh_malloc");
            dev_cap = bytes;
        }
        return static_cast<uint8_t*>(dev);
    }
};

Staging& staging() {
    ensure_init();
    // Intentionally leaked: freeing device memory from thread-exit destructors can run after the HIP
    // runtime has been torn down at process exit.
    thread_local Staging* s = new Staging();
    return *s;
}

const qh_tensor* resident(const Tensor& W, void* stream) {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_resident.find(W.data);
    if (it != g_resident.end()) {
        const qh_tensor& v = it->second.view;
        if (v.dtype != int32_t(W.dtype) || v.rows != W.rows || v.cols != W.cols)
            throw HipError("tensor at this address was uploaded with another dtype or shape");
        return &it->second.view;
    }
    Resident r;
    const size_t bytes = device_bytes(W);
    check(qh_malloc(&r.ptr, bytes), "qh_malloc");
    check(qh_memcpy_h2d(r.ptr, W.data, bytes, stream), "qh_memcpy_h2d");
    check(qh_stream_sync(stream), "qh_stream_sync");
    r.view = qh_tensor{int32_t(W.dtype), W.rows, W.cols, r.ptr};
    return &g_resident.emplace(W.data, r).first->second.view;
}

constexpr size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

void hip_matvec(float* out, const Tensor& W, const QuantVec& x, int r0, int r1) { matvec_q(out, W, x, r0, r1); }
void hip_matmul(float* out, int ldo, const Tensor& W, const QuantVec* x, int n, int r0, int r1) {
    matmul_q(out, ldo, W, x, n, r0, r1);
}

}  // namespace

#if !defined(QUANTA_HIP_ENGINE)
void quantize_q8(const float* x, int n, QuantVec& out) {
    Staging& s = staging();
    const int nb = n / QK;
    out.n = n;
    out.q.resize(size_t(n));
    out.d.resize(size_t(nb));
    if (n <= 0) return;
    const size_t ox = 0, oq = align256(sizeof(float) * n), od = oq + align256(size_t(n));
    uint8_t* dev = s.device(od + align256(sizeof(float) * nb));
    check(qh_memcpy_h2d(dev + ox, x, sizeof(float) * n, s.stream), "qh_memcpy_h2d");
    check(qh_quantize_q8(reinterpret_cast<float*>(dev + ox), 1, n, reinterpret_cast<int8_t*>(dev + oq),
                         reinterpret_cast<float*>(dev + od), s.stream),
          "qh_quantize_q8");
    check(qh_memcpy_d2h(out.q.data(), dev + oq, size_t(n), s.stream), "qh_memcpy_d2h");
    check(qh_memcpy_d2h(out.d.data(), dev + od, sizeof(float) * nb, s.stream), "qh_memcpy_d2h");
}
#endif

void matvec_q(float* out, const Tensor& W, const QuantVec& x, int r0, int r1) {
    if (r0 >= r1) return;
    Staging& s = staging();
    const qh_tensor* dw = resident(W, s.stream);
    const int nb = W.cols / QK;
    const size_t oq = 0, od = align256(size_t(W.cols)), oo = od + align256(sizeof(float) * nb);
    uint8_t* dev = s.device(oo + sizeof(float) * size_t(W.rows));
    check(qh_memcpy_h2d(dev + oq, x.q.data(), size_t(W.cols), s.stream), "qh_memcpy_h2d");
    check(qh_memcpy_h2d(dev + od, x.d.data(), sizeof(float) * nb, s.stream), "qh_memcpy_h2d");
    float* dout = reinterpret_cast<float*>(dev + oo);
    check(qh_matvec_q(dout, dw, reinterpret_cast<const int8_t*>(dev + oq), reinterpret_cast<const float*>(dev + od),
                      r0, r1, s.stream),
          "qh_matvec_q");
    check(qh_memcpy_d2h(out + r0, dout + r0, sizeof(float) * size_t(r1 - r0), s.stream), "qh_memcpy_d2h");
}

void matmul_q(float* out, int ldo, const Tensor& W, const QuantVec* x, int n, int r0, int r1) {
    if (r0 >= r1 || n <= 0) return;
    Staging& s = staging();
    const qh_tensor* dw = resident(W, s.stream);
    const int cols = W.cols, nb = cols / QK;
    const size_t oq = 0, od = align256(size_t(n) * cols), oo = od + align256(sizeof(float) * size_t(n) * nb);
    const size_t out_bytes = sizeof(float) * size_t(n) * size_t(ldo);
    uint8_t* dev = s.device(oo + out_bytes);
    for (int t = 0; t < n; ++t) {
        check(qh_memcpy_h2d(dev + oq + size_t(t) * cols, x[t].q.data(), size_t(cols), s.stream), "qh_memcpy_h2d");
        check(qh_memcpy_h2d(dev + od + sizeof(float) * size_t(t) * nb, x[t].d.data(), sizeof(float) * nb, s.stream),
              "qh_memcpy_h2d");
    }
    float* dout = reinterpret_cast<float*>(dev + oo);
    check(qh_matmul_q(dout, ldo, dw, reinterpret_cast<const int8_t*>(dev + oq),
                      reinterpret_cast<const float*>(dev + od), n, r0, r1, s.stream),
          "qh_matmul_q");
    // Only rows [r0, r1) of `out` belong to this call: other threads may be writing the rest.
    s.host.resize(out_bytes);
    check(qh_memcpy_d2h(s.host.data(), dout, out_bytes, s.stream), "qh_memcpy_d2h");
    const float* h = reinterpret_cast<const float*>(s.host.data());
    for (int t = 0; t < n; ++t)
        std::memcpy(out + size_t(t) * ldo + r0, h + size_t(t) * ldo + r0, sizeof(float) * size_t(r1 - r0));
}

const char* matvec_q_kernel_name() { return "hip"; }

#if defined(QUANTA_HIP_ENGINE)
std::vector<std::pair<const char*, MatvecQFn>> available_matvec_q_kernels() {
    return {{"ref", matvec_q_ref}, {"hip", hip_matvec}};
}

std::vector<std::pair<const char*, MatmulQFn>> available_matmul_q_kernels() {
    return {{"ref", matmul_q_ref}, {"hip", hip_matmul}};
}
#else
std::vector<std::pair<const char*, MatvecQFn>> available_matvec_q_kernels() { return {{"hip", hip_matvec}}; }

std::vector<std::pair<const char*, MatmulQFn>> available_matmul_q_kernels() { return {{"hip", hip_matmul}}; }
#endif

int shortlist_head(const Tensor& head8, const Tensor& head4, const Tensor& err, const QuantVec& xq,
                   const HeadQuery& hq, float* logits, int* top1, float* coarse, float* upper) {
    Staging& s = staging();
    const qh_tensor* d8 = resident(head8, s.stream);
    const qh_tensor* d4 = resident(head4, s.stream);
    const qh_tensor* de = resident(err, s.stream);
    const int V = head8.rows, D = head8.cols, nb = D / QK;
    const size_t ws = qh_shortlist_workspace_bytes(V, D, hq.top_k);
    if (ws == 0) throw HipError("shortlist_head: unsupported top_k or shape");
    const int n_must = hq.must ? hq.n_must : 0;
    const size_t o_ws = 0, o_q = align256(ws), o_d = o_q + align256(size_t(D)), o_must = o_d + align256(4 * size_t(nb));
    const size_t o_log = o_must + align256(4 * size_t(n_must)), o_co = o_log + align256(4 * size_t(V));
    const size_t o_up = o_co + align256(4 * size_t(V)), o_rows = o_up + align256(4 * size_t(V));
    const size_t o_st = o_rows + align256(4 * (size_t(V) + n_must));
    uint8_t* dev = s.device(o_st + align256(sizeof(qh_head_stats)));
    check(qh_memcpy_h2d(dev + o_q, xq.q.data(), size_t(D), s.stream), "qh_memcpy_h2d");
    check(qh_memcpy_h2d(dev + o_d, xq.d.data(), 4 * size_t(nb), s.stream), "qh_memcpy_h2d");
    if (n_must) check(qh_memcpy_h2d(dev + o_must, hq.must, 4 * size_t(n_must), s.stream), "qh_memcpy_h2d");
    const qh_head_query q{hq.top_k, hq.n_valid, n_must ? reinterpret_cast<const int32_t*>(dev + o_must) : nullptr,
                          n_must};
    const qh_head_out o{reinterpret_cast<float*>(dev + o_log), reinterpret_cast<float*>(dev + o_co),
                        reinterpret_cast<float*>(dev + o_up), reinterpret_cast<int32_t*>(dev + o_rows),
                        reinterpret_cast<qh_head_stats*>(dev + o_st)};
    check(qh_shortlist_head(d8, d4, de, reinterpret_cast<const int8_t*>(dev + o_q),
                            reinterpret_cast<const float*>(dev + o_d), &q, &o, dev + o_ws, ws, s.stream),
          "qh_shortlist_head");
    qh_head_stats st{};
    check(qh_memcpy_d2h(&st, dev + o_st, sizeof st, s.stream), "qh_memcpy_d2h");
    check(qh_memcpy_d2h(logits, dev + o_log, 4 * size_t(V), s.stream), "qh_memcpy_d2h");
    if (coarse) check(qh_memcpy_d2h(coarse, dev + o_co, 4 * size_t(V), s.stream), "qh_memcpy_d2h");
    if (upper) check(qh_memcpy_d2h(upper, dev + o_up, 4 * size_t(V), s.stream), "qh_memcpy_d2h");
    if (top1) *top1 = st.top1;
    return st.n_rows;
}

void release_device_tensors() {
    std::lock_guard<std::mutex> lk(g_mu);
    for (auto& kv : g_resident) qh_free(kv.second.ptr);
    g_resident.clear();
}

}  // namespace quanta
