// C-ABI layer: argument validation, error reporting and dispatch to the kernel launchers.
// Every entry point returns a status and records a message for the calling thread on failure.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <mutex>

#include "qh_internal.h"

namespace qh {

KernelTimer*& kernel_timer() {
    thread_local KernelTimer* t = nullptr;
    return t;
}

namespace {
thread_local char g_error[512] = "";
std::mutex g_init_mu;
bool g_inited[64] = {};

// The workspace of qh_shortlist_head_noalloc: one array in each GPU's memory, for the life of the process. Host code
// never uses its name as an address (on the host it names a stand-in, not device memory): qh_init records each
// device's own address of it, taken with hipGetSymbolAddress while that device is current, in g_scratch.
__device__ __align__(256) uint8_t scratch[QH_NOALLOC_SCRATCH_BYTES];
void* g_scratch[64] = {};
}  // namespace

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof g_error, fmt, ap);
    va_end(ap);
    return code;
}

int check_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return QH_OK;
    if (e == hipErrorOutOfMemory) return fail(QH_ERR_NOMEM, "%s: %s", what, hipGetErrorString(e));
    return fail(QH_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int validate_quant(const qh_tensor* W, const char* what) {
    if (!W) return fail(QH_ERR_ARG, "%s: null tensor", what);
    if (W->dtype != QH_Q8_0 && W->dtype != QH_Q4_0)
        return fail(QH_ERR_DTYPE, "%s: dtype %d is not q8_0 (2) or q4_0 (3)", what, W->dtype);
    if (W->rows <= 0 || W->cols <= 0) return fail(QH_ERR_SHAPE, "%s: bad shape %d x %d", what, W->rows, W->cols);
    if (W->cols % QH_QK != 0) return fail(QH_ERR_SHAPE, "%s: cols %d is not a multiple of 32", what, W->cols);
    if (W->cols > kMaxCols) return fail(QH_ERR_SHAPE, "%s: cols %d above the supported %d", what, W->cols, kMaxCols);
    if (!W->data) return fail(QH_ERR_ARG, "%s: null data", what);
    if (!aligned16(W->data)) return fail(QH_ERR_ALIGN, "%s: data is not 16-byte aligned", what);
    return QH_OK;
}

// A decoder matrix: Q8_0 / Q4_0 as validate_quant, or F32 / F16 (matvec_ref) with the same shape rules.
int validate_matrix(const qh_tensor* W, const char* what) {
    if (W && (W->dtype == QH_F32 || W->dtype == QH_F16)) {
        if (W->rows <= 0 || W->cols <= 0 || W->cols % QH_QK != 0 || W->cols > kMaxCols)
            return fail(QH_ERR_SHAPE, "%s: bad shape %d x %d", what, W->rows, W->cols);
        if (!W->data) return fail(QH_ERR_ARG, "%s: null data", what);
        if (!aligned16(W->data)) return fail(QH_ERR_ALIGN, "%s: data is not 16-byte aligned", what);
        return QH_OK;
    }
    if (W && W->dtype != QH_Q8_0 && W->dtype != QH_Q4_0)
        return fail(QH_ERR_DTYPE, "%s: dtype %d is not f32 (0), f16 (1), q8_0 (2) or q4_0 (3)", what, W->dtype);
    return validate_quant(W, what);
}

int validate_range(int rows, int r0, int r1, const char* what) {
    if (r0 < 0 || r1 > rows || r0 > r1)
        return fail(QH_ERR_ARG, "%s: row range [%d, %d) outside [0, %d)", what, r0, r1, rows);
    return QH_OK;
}

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

// The sampler parameters the device sampler handles (a finite temperature; at most QH_SAMPLE_MAX_TOPK survivors of
// the top-k cut when sampling).
int check_sampler(const qh_sampler_params& p, int n_valid, const char* who, bool have_ws) {
    if (!(p.temperature == p.temperature) || !(p.repeat_penalty > 0.0f) || p.top_k < 0 || p.repeat_window < 0)
        return fail(QH_ERR_ARG, "%s: bad sampler parameters", who);
    if (p.temperature > 0.0f && !have_ws) {
        const int k = (p.top_k > 0 && p.top_k < n_valid) ? p.top_k : n_valid;
        if (k > QH_SAMPLE_MAX_TOPK)
            return fail(QH_ERR_UNSUPPORTED, "%s: %d survivors of the top-k cut need a workspace (qh_sample_ws)", who,
                        k);
    }
    return QH_OK;
}

// Device checks of qh_init for the current device (gfx950), once per device.
int qh_init_current() {
    int dev = 0;
    if (int rc = check_hip(hipGetDevice(&dev), "hipGetDevice")) return rc;
    return qh_init(dev);
}

// The current device's address of the scratch array (initialising the device on its first use).
int scratch_current(void** ws) {
    int dev = 0;
    if (int rc = check_hip(hipGetDevice(&dev), "hipGetDevice")) return rc;
    if (int rc = qh_init(dev)) return rc;
    std::lock_guard<std::mutex> lk(g_init_mu);
    *ws = g_scratch[dev];
    return *ws ? QH_OK : fail(QH_ERR_HIP, "no scratch array on device %d", dev);
}

// A nibble-plane head: shape as a Q8_0 head of the shortlist (cols a multiple of 64, at most kMaxHeadCols).
int validate_planes(const qh_tensor* W, const char* what) {
    if (!W) return fail(QH_ERR_ARG, "%s: null tensor", what);
    if (W->dtype != QH_Q8_0_PLANES) return fail(QH_ERR_DTYPE, "%s: dtype %d is not q8_0 planes (16)", what, W->dtype);
    if (W->rows <= 0 || W->cols <= 0 || W->cols % 64 != 0 || W->cols > kMaxHeadCols)
        return fail(QH_ERR_SHAPE, "%s: bad shape %d x %d (cols a multiple of 64, at most %d)", what, W->rows, W->cols,
                    kMaxHeadCols);
    if (!W->data) return fail(QH_ERR_ARG, "%s: null data", what);
    if (!aligned16(W->data)) return fail(QH_ERR_ALIGN, "%s: data is not 16-byte aligned", what);
    return QH_OK;
}

// The query, activation and outputs of a shortlist call over a V x D head.
int validate_head_io(int V, int D, const int8_t* xq, const float* xd, const qh_head_query* query,
                     const qh_head_out* out, const char* who) {
    if (!query || !out) return fail(QH_ERR_ARG, "%s: null argument", who);
    if (!xq || !xd || !aligned16(xq)) return fail(QH_ERR_ARG, "%s: bad activation pointers", who);
    if (query->top_k < 1 || query->top_k > QH_HEAD_MAX_TOPK)
        return fail(QH_ERR_UNSUPPORTED, "%s: top_k %d outside [1, %d]", who, query->top_k, QH_HEAD_MAX_TOPK);
    if (query->n_must < 0 || (query->n_must > 0 && !query->must)) return fail(QH_ERR_ARG, "%s: bad must list", who);
    if (!head_select_supported(V, D, query->top_k))
        return fail(QH_ERR_UNSUPPORTED, "%s: %d rows with top_k %d exceed the seed selection", who, V, query->top_k);
    if (!out->logits || !out->coarse || !out->upper || !out->rows || !out->stats)
        return fail(QH_ERR_ARG, "%s: null output buffer", who);
    return QH_OK;
}

// Arguments of the shortlist head entry points (everything but the workspace).
int validate_head(const qh_tensor* head8, const qh_tensor* head4, const qh_tensor* err, const int8_t* xq,
                  const float* xd, const qh_head_query* query, const qh_head_out* out, const char* who) {
    if (!head8 || !head4 || !err || !query || !out) return fail(QH_ERR_ARG, "%s: null argument", who);
    if (int rc = validate_quant(head8, who)) return rc;
    if (int rc = validate_quant(head4, who)) return rc;
    if (head8->dtype != QH_Q8_0 || head4->dtype != QH_Q4_0 || err->dtype != QH_F16)
        return fail(QH_ERR_DTYPE, "%s: needs q8_0 head, q4_0 copy and f16 bounds", who);
    const int V = head8->rows, D = head8->cols;
    if (head4->rows != V || head4->cols != D || err->rows != V || err->cols != D / QH_QK)
        return fail(QH_ERR_SHAPE, "%s: bad shortlist tensors", who);  // as model.cpp:49-58
    if (!head_shape_supported(D))
        return fail(QH_ERR_SHAPE, "%s: hidden size %d must be a multiple of 64 and at most %d", who, D, kMaxHeadCols);
    if (!err->data || !aligned16(err->data)) return fail(QH_ERR_ALIGN, "%s: err not 16-byte aligned", who);
    if (!xq || !xd || !aligned16(xq)) return fail(QH_ERR_ARG, "%s: bad activation pointers", who);
    if (query->top_k < 1 || query->top_k > QH_HEAD_MAX_TOPK)
        return fail(QH_ERR_UNSUPPORTED, "%s: top_k %d outside [1, %d]", who, query->top_k, QH_HEAD_MAX_TOPK);
    if (query->n_must < 0 || (query->n_must > 0 && !query->must)) return fail(QH_ERR_ARG, "%s: bad must list", who);
    if (!head_select_supported(V, D, query->top_k))
        return fail(QH_ERR_UNSUPPORTED, "%s: %d rows with top_k %d exceed the seed selection", who, V, query->top_k);
    if (!out->logits || !out->coarse || !out->upper || !out->rows || !out->stats)
        return fail(QH_ERR_ARG, "%s: null output buffer", who);
    return QH_OK;
}

}  // namespace

std::atomic<int> g_fault_alloc{-1};  // allocations to let through before the forced failure; -1: disarmed

bool fault_alloc_fires() {
    int n = g_fault_alloc.load(std::memory_order_relaxed);
    while (n >= 0) {
        if (g_fault_alloc.compare_exchange_weak(n, n - 1, std::memory_order_relaxed)) return n == 0;
    }
    return false;
}
}  // namespace qh

using namespace qh;

extern "C" {

const char* qh_last_error(void) { return g_error; }

const char* qh_version(void) { return "quanta-hip 0.1 gfx950"; }

int qh_init(int device) {
    int n = 0;
    if (int rc = check_hip(hipGetDeviceCount(&n), "hipGetDeviceCount")) return rc;
    if (device < 0 || device >= n || device >= 64) return fail(QH_ERR_ARG, "qh_init: device %d of %d", device, n);
    if (int rc = check_hip(hipSetDevice(device), "hipSetDevice")) return rc;
    std::lock_guard<std::mutex> lk(g_init_mu);
    if (!g_inited[device]) {
        hipDeviceProp_t prop;
        if (int rc = check_hip(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties")) return rc;
        if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
            return fail(QH_ERR_UNSUPPORTED, "qh_init: device %d is %s, this build targets gfx950", device,
                        prop.gcnArchName);
        void* p = nullptr;
        if (int rc = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)")) return rc;
        if (!p) return fail(QH_ERR_HIP, "qh_init: no device address for the scratch array");
        g_scratch[device] = p;
        g_inited[device] = true;
    }
    return QH_OK;
}

size_t qh_quant_bytes(int dtype, int rows, int cols) {
    const size_t n = (size_t)rows * (size_t)cols;
    switch (dtype) {
        case QH_F32: return n * 4;
        case QH_F16: return n * 2;
        case QH_Q8_0: return n;
        case QH_Q4_0: return n / 2;
        case QH_Q8_0_PLANES: return n;  // both planes
        default: return 0;
    }
}

size_t qh_tensor_bytes(int dtype, int rows, int cols) {
    size_t b = qh_quant_bytes(dtype, rows, cols);
    if (dtype == QH_Q8_0 || dtype == QH_Q4_0 || dtype == QH_Q8_0_PLANES) b += (size_t)rows * cols / QH_QK * 2;
    return b;
}

int qh_validate_tensor(const qh_tensor* W) {
    if (!W) return fail(QH_ERR_ARG, "qh_validate_tensor: null tensor");
    if (W->dtype == QH_Q8_0_PLANES) return validate_planes(W, "qh_validate_tensor");
    if (W->dtype == QH_F32 || W->dtype == QH_F16) {
        if (W->rows <= 0 || W->cols <= 0) return fail(QH_ERR_SHAPE, "bad shape %d x %d", W->rows, W->cols);
        if (!W->data) return fail(QH_ERR_ARG, "null data");
        if (!aligned16(W->data)) return fail(QH_ERR_ALIGN, "data is not 16-byte aligned");
        return QH_OK;
    }
    return validate_quant(W, "qh_validate_tensor");
}

int qh_fault_alloc(int after) {
    g_fault_alloc.store(after < 0 ? -1 : after, std::memory_order_relaxed);
    return QH_OK;
}

int qh_malloc(void** ptr, size_t bytes) {
    if (!ptr) return fail(QH_ERR_ARG, "qh_malloc: null out pointer");
    *ptr = nullptr;
    if (bytes == 0) return QH_OK;
    if (fault_alloc_fires()) return fail(QH_ERR_NOMEM, "qh_malloc: forced allocation failure (%zu bytes)", bytes);
    hipError_t e = hipMalloc(ptr, bytes);
    if (e == hipErrorOutOfMemory) return fail(QH_ERR_NOMEM, "qh_malloc: out of memory (%zu bytes)", bytes);
    return check_hip(e, "hipMalloc");
}

int qh_free(void* ptr) { return ptr ? check_hip(hipFree(ptr), "hipFree") : QH_OK; }

int qh_memcpy_h2d(void* dst, const void* src_host, size_t bytes, void* stream) {
    if (bytes == 0) return QH_OK;
    if (!dst || !src_host) return fail(QH_ERR_ARG, "qh_memcpy_h2d: null pointer");
    return check_hip(hipMemcpyAsync(dst, src_host, bytes, hipMemcpyHostToDevice, as_stream(stream)), "hipMemcpyAsync");
}

int qh_memcpy_d2h(void* dst_host, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return QH_OK;
    if (!dst_host || !src) return fail(QH_ERR_ARG, "qh_memcpy_d2h: null pointer");
    if (int rc = check_hip(hipMemcpyAsync(dst_host, src, bytes, hipMemcpyDeviceToHost, as_stream(stream)),
                           "hipMemcpyAsync"))
        return rc;
    return check_hip(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize");
}

int qh_memset(void* dst, int value, size_t bytes, void* stream) {
    if (bytes == 0) return QH_OK;
    if (!dst) return fail(QH_ERR_ARG, "qh_memset: null pointer");
    return check_hip(hipMemsetAsync(dst, value, bytes, as_stream(stream)), "hipMemsetAsync");
}

int qh_stream_sync(void* stream) { return check_hip(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize"); }

int qh_stream_create(void** stream) {
    if (!stream) return fail(QH_ERR_ARG, "qh_stream_create: null out pointer");
    hipStream_t s = nullptr;
    if (int rc = check_hip(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreateWithFlags")) return rc;
    *stream = s;
    return QH_OK;
}

int qh_stream_destroy(void* stream) {
    return stream ? check_hip(hipStreamDestroy(as_stream(stream)), "hipStreamDestroy") : QH_OK;
}

int qh_quantize_q8(const float* x, int n_tok, int n, int8_t* q, float* d, void* stream) {
    if (!x || !q || !d) return fail(QH_ERR_ARG, "qh_quantize_q8: null pointer");
    if (n_tok < 0 || n <= 0 || n % QH_QK != 0) return fail(QH_ERR_SHAPE, "qh_quantize_q8: n_tok %d, n %d", n_tok, n);
    if (n_tok == 0) return QH_OK;
    return check_hip(launch_quantize_q8(x, n_tok, n, q, d, as_stream(stream)), "qh_quantize_q8 launch");
}

int qh_matvec_ref(float* out, const qh_tensor* W, const float* x, int r0, int r1, void* stream) {
    if (!W || !out || !x || !W->data) return fail(QH_ERR_ARG, "qh_matvec_ref: null pointer");
    if (W->dtype != QH_F32 && W->dtype != QH_F16)
        return fail(QH_ERR_DTYPE, "qh_matvec_ref: dtype %d is not f32 (0) or f16 (1); use qh_matvec_q", W->dtype);
    if (W->rows <= 0 || W->cols <= 0 || W->cols % QH_QK != 0)
        return fail(QH_ERR_SHAPE, "qh_matvec_ref: shape %d x %d (cols must be a multiple of 32)", W->rows, W->cols);
    if (int rc = validate_range(W->rows, r0, r1, "qh_matvec_ref")) return rc;
    if (!aligned16(W->data) || !aligned16(x)) return fail(QH_ERR_ALIGN, "qh_matvec_ref: W or x is not 16-byte aligned");
    if (r0 == r1) return QH_OK;
    return check_hip(launch_gemv_dense(out, 0, *W, x, W->cols, 1, r0, r1, as_stream(stream)), "qh_matvec_ref launch");
}

int qh_matvec_q(float* out, const qh_tensor* W, const int8_t* xq, const float* xd, int r0, int r1, void* stream) {
    if (W && W->dtype == QH_Q8_0_PLANES) {  // a nibble-plane head: the same values as its Q8_0 form
        if (int rc = validate_planes(W, "qh_matvec_q")) return rc;
        if (int rc = validate_range(W->rows, r0, r1, "qh_matvec_q")) return rc;
        if (!out || !xq || !xd) return fail(QH_ERR_ARG, "qh_matvec_q: null pointer");
        if (!aligned16(xq)) return fail(QH_ERR_ALIGN, "qh_matvec_q: xq is not 16-byte aligned");
        return check_hip(launch_gemv_planes(out, *W, xq, xd, r0, r1, as_stream(stream)), "qh_matvec_q launch");
    }
    if (int rc = validate_quant(W, "qh_matvec_q")) return rc;
    if (int rc = validate_range(W->rows, r0, r1, "qh_matvec_q")) return rc;
    if (!out || !xq || !xd) return fail(QH_ERR_ARG, "qh_matvec_q: null pointer");
    if (!aligned16(xq)) return fail(QH_ERR_ALIGN, "qh_matvec_q: xq is not 16-byte aligned");
    if (r0 == r1) return QH_OK;
    const GemvPlan plan = gemv_plan(W->dtype, W->cols, r1 - r0);
    return check_hip(launch_gemv(out, *W, xq, xd, r0, r1, plan, as_stream(stream)), "qh_matvec_q launch");
}

int qh_matmul_q(float* out, int ldo, const qh_tensor* W, const int8_t* xq, const float* xd, int n, int r0, int r1,
                void* stream) {
    if (int rc = validate_quant(W, "qh_matmul_q")) return rc;
    if (int rc = validate_range(W->rows, r0, r1, "qh_matmul_q")) return rc;
    if (!out || !xq || !xd) return fail(QH_ERR_ARG, "qh_matmul_q: null pointer");
    if (n < 0) return fail(QH_ERR_ARG, "qh_matmul_q: n = %d", n);
    if (ldo < r1) return fail(QH_ERR_ARG, "qh_matmul_q: ldo %d < r1 %d", ldo, r1);
    if (!aligned16(xq)) return fail(QH_ERR_ALIGN, "qh_matmul_q: xq is not 16-byte aligned");
    if (n == 0 || r0 == r1) return QH_OK;
    if ((long)n * ldo > 0x7fffffffL) return fail(QH_ERR_SHAPE, "qh_matmul_q: n * ldo too large");
    return check_hip(launch_matmul(out, ldo, *W, xq, xd, n, r0, r1, as_stream(stream)), "qh_matmul_q launch");
}

size_t qh_argmax_workspace_bytes(int n) { return n > 0 ? argmax_workspace_bytes(n) : 0; }

int qh_argmax(const float* logits, int n, int32_t* index, void* workspace, size_t workspace_bytes, void* stream) {
    if (!logits || !index) return fail(QH_ERR_ARG, "qh_argmax: null pointer");
    if (n <= 0) return fail(QH_ERR_ARG, "qh_argmax: n = %d", n);
    const size_t need = argmax_workspace_bytes(n);
    if (!workspace || workspace_bytes < need)
        return fail(QH_ERR_NOMEM, "qh_argmax: workspace %zu bytes, needs %zu", workspace_bytes, need);
    if (!aligned16(workspace)) return fail(QH_ERR_ALIGN, "qh_argmax: workspace not 16-byte aligned");
    return check_hip(launch_argmax(logits, n, index, workspace, as_stream(stream)), "qh_argmax launch");
}

uint64_t qh_sampler_state(uint64_t seed) { return seed | 1u; }

size_t qh_sample_workspace_bytes(int32_t n_valid) {
    if (n_valid < 1 || n_valid > QH_SAMPLE_MAX_VOCAB) return 0;
    return sample_workspace_bytes(n_valid);
}

int qh_sample(const float* logits, int32_t n_valid, const int32_t* rows, const qh_head_stats* head_stats,
              const int32_t* history, int32_t n_hist, const qh_sampler_params* params, uint64_t* state,
              int32_t* out_id, void* stream) {
    return qh_sample_ws(logits, n_valid, rows, head_stats, history, n_hist, params, state, out_id, nullptr, 0,
                        stream);
}

int qh_sample_ws(const float* logits, int32_t n_valid, const int32_t* rows, const qh_head_stats* head_stats,
                 const int32_t* history, int32_t n_hist, const qh_sampler_params* params, uint64_t* state,
                 int32_t* out_id, void* ws, size_t ws_bytes, void* stream) {
    if (!logits || !params || !state || !out_id) return fail(QH_ERR_ARG, "qh_sample: null argument");
    if (n_valid < 1 || n_valid > QH_SAMPLE_MAX_VOCAB)
        return fail(QH_ERR_UNSUPPORTED, "qh_sample: n_valid %d outside [1, %d]", n_valid, QH_SAMPLE_MAX_VOCAB);
    if ((rows == nullptr) != (head_stats == nullptr))
        return fail(QH_ERR_ARG, "qh_sample: rows and head_stats go together");
    if (n_hist < 0 || (n_hist > 0 && !history)) return fail(QH_ERR_ARG, "qh_sample: bad history");
    if (ws && (ws_bytes < sample_workspace_bytes(n_valid) || !aligned16(ws)))
        return fail(QH_ERR_ARG, "qh_sample_ws: workspace of %zu bytes (needs %zu, 16-byte aligned)", ws_bytes,
                    sample_workspace_bytes(n_valid));
    if (int rc = check_sampler(*params, n_valid, "qh_sample", ws != nullptr)) return rc;
    HeadMust hist;
    hist.ids = history;
    hist.n = n_hist;
    hist.window = 0;
    if (params->repeat_window > 0 && n_hist > params->repeat_window) {  // the window, as sampler.cpp:24-27
        hist.ids = history + (n_hist - params->repeat_window);
        hist.n = params->repeat_window;
    }
    return check_hip(
        launch_sample(logits, n_valid, rows, head_stats, hist, *params, state, out_id, ws, as_stream(stream)),
        "qh_sample launch");
}

size_t qh_shortlist_workspace_bytes(int V, int D, int top_k) {
    if (V <= 0 || D <= 0 || top_k <= 0 || top_k > QH_HEAD_MAX_TOPK || !head_shape_supported(D)) return 0;
    return head_workspace_bytes(V, D, top_k);
}

int qh_shortlist_head(const qh_tensor* head8, const qh_tensor* head4, const qh_tensor* err, const int8_t* xq,
                      const float* xd, const qh_head_query* query, const qh_head_out* out, void* workspace,
                      size_t workspace_bytes, void* stream) {
    if (int rc = validate_head(head8, head4, err, xq, xd, query, out, "qh_shortlist_head")) return rc;
    const size_t need = head_workspace_bytes(head8->rows, head8->cols, query->top_k);
    if (!workspace || workspace_bytes < need)
        return fail(QH_ERR_NOMEM, "qh_shortlist_head: workspace %zu bytes, needs %zu", workspace_bytes, need);
    if (!aligned16(workspace)) return fail(QH_ERR_ALIGN, "qh_shortlist_head: workspace not 16-byte aligned");
    HeadMust must;
    must.ids = query->must;
    must.n = query->n_must;
    return check_hip(
        launch_shortlist_head(*head8, *head4, *err, xq, xd, *query, must, *out, workspace, as_stream(stream)),
        "qh_shortlist_head launch");
}

int qh_head_planes(const qh_tensor* head8, void* planes, void* stream) {
    if (int rc = validate_quant(head8, "qh_head_planes")) return rc;
    if (head8->dtype != QH_Q8_0) return fail(QH_ERR_DTYPE, "qh_head_planes: needs a q8_0 head");
    if (head8->cols % 64 != 0 || head8->cols > kMaxHeadCols)
        return fail(QH_ERR_SHAPE, "qh_head_planes: cols %d must be a multiple of 64 and at most %d", head8->cols,
                    kMaxHeadCols);
    if (!planes || !aligned16(planes)) return fail(QH_ERR_ALIGN, "qh_head_planes: planes not 16-byte aligned");
    const size_t n = qh_tensor_bytes(QH_Q8_0, head8->rows, head8->cols);
    const uintptr_t a = reinterpret_cast<uintptr_t>(head8->data), b = reinterpret_cast<uintptr_t>(planes);
    if (a < b + n && b < a + n) return fail(QH_ERR_ARG, "qh_head_planes: planes overlap the q8_0 head");
    return check_hip(launch_head_planes(head8->data, planes, head8->rows, head8->cols, as_stream(stream)),
                     "qh_head_planes launch");
}

int qh_shortlist_planes(const qh_tensor* planes, const int8_t* xq, const float* xd, const qh_head_query* query,
                        const qh_head_out* out, void* workspace, size_t workspace_bytes, void* stream) {
    if (int rc = validate_planes(planes, "qh_shortlist_planes")) return rc;
    if (int rc = validate_head_io(planes->rows, planes->cols, xq, xd, query, out, "qh_shortlist_planes")) return rc;
    const size_t need = head_workspace_bytes(planes->rows, planes->cols, query->top_k);
    if (!workspace || workspace_bytes < need)
        return fail(QH_ERR_NOMEM, "qh_shortlist_planes: workspace %zu bytes, needs %zu", workspace_bytes, need);
    if (!aligned16(workspace)) return fail(QH_ERR_ALIGN, "qh_shortlist_planes: workspace not 16-byte aligned");
    HeadMust must;
    must.ids = query->must;
    must.n = query->n_must;
    const qh_tensor none{QH_F16, 0, 0, nullptr};
    return check_hip(
        launch_shortlist_head(*planes, none, none, xq, xd, *query, must, *out, workspace, as_stream(stream)),
        "qh_shortlist_planes launch");
}

int qh_shortlist_head_noalloc(const qh_tensor* head8, const qh_tensor* head4, const qh_tensor* err, const int8_t* xq,
                              const float* xd, const qh_head_query* query, const qh_head_out* out, void* stream) {
    if (int rc = validate_head(head8, head4, err, xq, xd, query, out, "qh_shortlist_head_noalloc")) return rc;
    const size_t need = head_workspace_bytes(head8->rows, head8->cols, query->top_k);
    if (need > QH_NOALLOC_SCRATCH_BYTES)
        return fail(QH_ERR_NOMEM, "qh_shortlist_head_noalloc: needs %zu bytes of workspace, the scratch array holds %zu",
                    need, (size_t)QH_NOALLOC_SCRATCH_BYTES);
    void* ws = nullptr;
    if (int rc = scratch_current(&ws)) return rc;
    HeadMust must;
    must.ids = query->must;
    must.n = query->n_must;
    return check_hip(launch_shortlist_head(*head8, *head4, *err, xq, xd, *query, must, *out, ws, as_stream(stream)),
                     "qh_shortlist_head_noalloc launch");
}

int qh_decoder_create(const qh_model_desc* hp, const qh_tensor* tensors, int n_tensors, qh_decoder** out) {
    if (!hp || !tensors || !out) return fail(QH_ERR_ARG, "qh_decoder_create: null argument");
    *out = nullptr;
    const int D = hp->dim, L = hp->n_layers;
    if (D <= 0 || D > 8192 || D % 64 || hp->ffn_dim <= 0 || hp->ffn_dim % QH_QK || hp->ffn_dim > kMaxCols || L <= 0 ||
        hp->n_heads <= 0 || hp->n_kv_heads <= 0 || hp->n_heads % hp->n_kv_heads ||
        (hp->head_dim != 64 && hp->head_dim != 128) || hp->n_heads * hp->head_dim != D || hp->ctx_len <= 0 ||
        hp->ctx_len > 8192 || hp->vocab_size <= 0)
        return fail(QH_ERR_SHAPE, "qh_decoder_create: unsupported model shape");  // as model.cpp:39-46
    if (n_tensors != 4 + 12 * L && n_tensors != 5 + 12 * L)
        return fail(QH_ERR_ARG, "qh_decoder_create: %d tensors, needs %d or %d", n_tensors, 4 + 12 * L, 5 + 12 * L);
    if (hp->flags & ~QH_FLAG_HADAMARD_DOWN) return fail(QH_ERR_ARG, "qh_decoder_create: unknown flags %#x", hp->flags);
    if ((hp->flags & QH_FLAG_HADAMARD_DOWN) && hp->ffn_dim % 256 != 0)
        return fail(QH_ERR_SHAPE, "qh_decoder_create: hadamard flag needs ffn_dim %% 256 == 0");  // as model.cpp:39-42
    if (hp->kv_f32 != 0 && hp->kv_f32 != 1) return fail(QH_ERR_ARG, "qh_decoder_create: kv_f32 = %d", hp->kv_f32);
    const int kvd = hp->n_kv_heads * hp->head_dim, F = hp->ffn_dim;
    auto want = [&](int i, int rows, int cols, bool quant, const char* what) -> int {
        const qh_tensor& t = tensors[i];
        if (quant) {
            if (int rc = validate_matrix(&t, what)) return rc;
        } else if (t.dtype != QH_F32 || !t.data) {
            return fail(QH_ERR_DTYPE, "qh_decoder_create: %s must be f32", what);
        }
        if (t.rows != rows || t.cols != cols)
            return fail(QH_ERR_SHAPE, "qh_decoder_create: %s is %d x %d, expected %d x %d", what, t.rows, t.cols, rows,
                        cols);
        return QH_OK;
    };
    // a nibble-plane embedding / LM head (QH_Q8_0_PLANES, qh_head_planes): the Q8_0 values in another layout
    auto want_lm = [&](int i, const char* what) -> int {
        if (tensors[i].dtype != QH_Q8_0_PLANES) return want(i, hp->vocab_size, D, true, what);
        if (int rc = validate_planes(&tensors[i], what)) return rc;
        if (tensors[i].rows != hp->vocab_size || tensors[i].cols != D)
            return fail(QH_ERR_SHAPE, "qh_decoder_create: %s is %d x %d, expected %d x %d", what, tensors[i].rows,
                        tensors[i].cols, hp->vocab_size, D);
        return QH_OK;
    };
    if (int rc = want_lm(0, "embedding")) return rc;
    if (int rc = want(1, 1, D, false, "final norm")) return rc;
    for (int l = 0; l < L; ++l) {
        const int b = 2 + 12 * l;
        const int rows[12] = {1, D, kvd, kvd, D, 1, 1, 1, 1, F, F, D};
        const int cols[12] = {D, D, D, D, D, D, kvd, kvd, D, D, D, F};
        const bool quant[12] = {false, true, true, true, true, false, false, false, false, true, true, true};
        for (int j = 0; j < 12; ++j) {
            if (j >= 5 && j <= 7 && !hp->qkv_bias) continue;
            if (int rc = want(b + j, rows[j], cols[j], quant[j], "layer tensor")) return rc;
        }
    }
    // the LM head: lm_head.weight when untied (model.cpp:16), Q8_0 or Q4_0, else the embedding
    const bool untied = n_tensors == 5 + 12 * L && tensors[4 + 12 * L].data;
    if (untied)
        if (int rc = want_lm(4 + 12 * L, "lm_head")) return rc;
    const int lm_dtype = untied ? tensors[4 + 12 * L].dtype : tensors[0].dtype;
    const qh_tensor& h4 = tensors[2 + 12 * L];
    const qh_tensor& he = tensors[3 + 12 * L];
    if (lm_dtype == QH_Q8_0_PLANES && (h4.data || he.data))
        return fail(QH_ERR_ARG, "qh_decoder_create: a nibble-plane LM head is its own shortlist: no head_q4 / head_err");
    if (h4.data || he.data) {
        if (h4.dtype != QH_Q4_0 || he.dtype != QH_F16 || lm_dtype != QH_Q8_0 || h4.rows != hp->vocab_size ||
            h4.cols != D || he.rows != hp->vocab_size || he.cols != D / QH_QK || !h4.data || !he.data ||
            !head_shape_supported(D))
            return fail(QH_ERR_SHAPE, "qh_decoder_create: bad shortlist head tensors");  // as model.cpp:49-58
    }
    if (int rc = qh_init_current()) return rc;
    if ((h4.data || lm_dtype == QH_Q8_0_PLANES) && !head_select_supported(hp->vocab_size, D, 1))
        return fail(QH_ERR_UNSUPPORTED, "qh_decoder_create: a %d x %d shortlist head is beyond the seed selection",
                    hp->vocab_size, D);
    Decoder* d = nullptr;
    if (int rc = decoder_create(hp, tensors, n_tensors, &d)) return rc;
    *out = reinterpret_cast<qh_decoder*>(d);
    return QH_OK;
}

int qh_decoder_destroy(qh_decoder* d) {
    decoder_destroy(reinterpret_cast<Decoder*>(d));
    return QH_OK;
}

int qh_decoder_prefill(qh_decoder* d, const int32_t* tokens, int n, int pos0, int top_k, void* stream) {
    if (!d || !tokens) return fail(QH_ERR_ARG, "qh_decoder_prefill: null argument");
    Decoder* dd = reinterpret_cast<Decoder*>(d);
    if (n <= 0) return fail(QH_ERR_ARG, "qh_decoder_prefill: n = %d", n);  // as model.cpp:351
    if (pos0 < 0 || pos0 + n > decoder_ctx(dd))
        return fail(QH_ERR_ARG, "qh_decoder_prefill: positions [%d, %d) exceed the context", pos0, pos0 + n);
    if (top_k < 0 || top_k > QH_HEAD_MAX_TOPK) return fail(QH_ERR_UNSUPPORTED, "qh_decoder_prefill: top_k %d", top_k);
    return check_hip(decoder_prefill(dd, tokens, n, pos0, top_k, as_stream(stream)), "qh_decoder_prefill");
}

int qh_decoder_begin(qh_decoder* d, int top_k, int32_t* out_dev, int out_cap, void* stream) {
    if (!d || !out_dev || out_cap <= 0) return fail(QH_ERR_ARG, "qh_decoder_begin: bad argument");
    return check_hip(decoder_begin(reinterpret_cast<Decoder*>(d), top_k, out_dev, out_cap, as_stream(stream)),
                     "qh_decoder_begin");
}

int qh_decoder_step(qh_decoder* d, int top_k, void* stream) {
    if (!d) return fail(QH_ERR_ARG, "qh_decoder_step: null decoder");
    if (top_k < 0 || top_k > QH_HEAD_MAX_TOPK) return fail(QH_ERR_UNSUPPORTED, "qh_decoder_step: top_k %d", top_k);
    return check_hip(decoder_step(reinterpret_cast<Decoder*>(d), top_k, as_stream(stream)), "qh_decoder_step");
}

int qh_decoder_step_timed(qh_decoder* d, int top_k, void* stream, float* us_host, int32_t* stage_host, int cap,
                          int32_t* n_host) {
    if (!d || !us_host || !stage_host || !n_host || cap <= 0) return fail(QH_ERR_ARG, "qh_decoder_step_timed: bad argument");
    if (top_k < 0 || top_k > QH_HEAD_MAX_TOPK) return fail(QH_ERR_UNSUPPORTED, "qh_decoder_step_timed: top_k %d", top_k);
    *n_host = 0;
    return decoder_step_timed(reinterpret_cast<Decoder*>(d), top_k, as_stream(stream), us_host, stage_host, cap + 1,
                              n_host);
}

int qh_decoder_views(qh_decoder* d, qh_decoder_state* v) {
    if (!d || !v) return fail(QH_ERR_ARG, "qh_decoder_views: null argument");
    decoder_views(reinterpret_cast<Decoder*>(d), v);
    return QH_OK;
}

int qh_decoder_set_prefill_stack(qh_decoder* d, int stack) {
    if (!d) return fail(QH_ERR_ARG, "qh_decoder_set_prefill_stack: null decoder");
    if (stack < 32 || stack > 1024 || stack % 32 != 0)
        return fail(QH_ERR_ARG, "qh_decoder_set_prefill_stack: stack %d is not a multiple of 32 in [32, 1024]", stack);
    return check_hip(decoder_set_prefill_stack(reinterpret_cast<Decoder*>(d), stack), "qh_decoder_set_prefill_stack");
}

int qh_decoder_set_query(qh_decoder* d, const qh_sampler_params* p) {
    if (!d) return fail(QH_ERR_ARG, "qh_decoder_set_query: null decoder");
    if (p) {
        if (!(p->repeat_penalty > 0.0f) || p->repeat_window < 0 || p->top_k < 0 || !(p->temperature == p->temperature))
            return fail(QH_ERR_ARG, "qh_decoder_set_query: bad parameters");
        // the shortlist head takes up to QH_HEAD_MAX_TOPK; a model without its tensors runs the full head anyway
        if (p->temperature > 0.0f && p->top_k > QH_HEAD_MAX_TOPK && decoder_has_shortlist(reinterpret_cast<Decoder*>(d)))
            return fail(QH_ERR_UNSUPPORTED, "qh_decoder_set_query: top_k %d above %d with the shortlist head",
                        p->top_k, QH_HEAD_MAX_TOPK);
    }
    decoder_set_query(reinterpret_cast<Decoder*>(d), p);
    return QH_OK;
}

int qh_decoder_set_sampler(qh_decoder* d, const qh_sampler_params* p, uint64_t seed) {
    if (!d) return fail(QH_ERR_ARG, "qh_decoder_set_sampler: null decoder");
    if (p) {
        if (seed == 0) return fail(QH_ERR_ARG, "qh_decoder_set_sampler: seed must be nonzero");
        const int V = decoder_vocab(reinterpret_cast<Decoder*>(d));
        if (V > QH_SAMPLE_MAX_VOCAB)
            return fail(QH_ERR_UNSUPPORTED, "qh_decoder_set_sampler: vocab %d above %d", V, QH_SAMPLE_MAX_VOCAB);
        if (int rc = check_sampler(*p, V, "qh_decoder_set_sampler", true)) return rc;
    }
    return check_hip(decoder_set_sampler(reinterpret_cast<Decoder*>(d), p, seed), "qh_decoder_set_sampler");
}

}  // extern "C"
