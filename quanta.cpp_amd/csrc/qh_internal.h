// Host-side declarations shared between the C-ABI layer (qh_api.hip) and the kernel files.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <utility>
#include <vector>

#include "quanta_hip.h"

namespace qh {

// Device timing of the kernels a call launches (qh_decoder_step_timed): while a timer is set on the calling thread,
// qh_launch launches with start / stop events (hipExtLaunchKernel, the dispatch's own timestamps, no extra packets)
// and records the stage each kernel belongs to.
struct KernelTimer {
    std::vector<hipEvent_t> ev;  // [2 * cap]: start, stop of kernel i
    std::vector<int> stage;      // per timed kernel; -1 until its stage is marked
    int n = 0;                   // kernels timed
    int launched = 0;            // kernels launched while the timer was set (timed or not)
    bool full() const { return 2 * (size_t)n + 1 >= ev.size(); }
    void mark(int id) {  // the kernels launched since the previous mark belong to stage id
        for (int i = n - 1; i >= 0 && stage[i] < 0; --i) stage[i] = id;
    }
};
KernelTimer*& kernel_timer();

// Launch of a kernel (hipLaunchKernelGGL's arguments), timed when a KernelTimer is set on this thread.
template <typename... P, typename... A>
inline void qh_launch(void (*kernel)(P...), dim3 grid, dim3 block, size_t lds, hipStream_t s, A&&... args) {
    KernelTimer* t = kernel_timer();
    if (t) ++t->launched;
    if (t && !t->full()) {
        const hipEvent_t a = t->ev[2 * t->n], b = t->ev[2 * t->n + 1];
        t->stage.push_back(-1);
        ++t->n;
        hipExtLaunchKernelGGL(kernel, grid, block, (std::uint32_t)lds, s, a, b, 0u, static_cast<P>(args)...);
        return;
    }
    kernel<<<grid, block, lds, s>>>(static_cast<P>(args)...);
}

// Records a formatted message as this thread's last error and returns `code`.
int fail(int code, const char* fmt, ...);

// Maps a HIP status to QH_ERR_HIP with context, QH_OK otherwise.
int check_hip(hipError_t e, const char* what);
// True when qh_fault_alloc's forced failure is due for this allocation (counts allocations down while armed).
bool fault_alloc_fires();

// Launch configuration of the decode GEMV for one (dtype, cols) pair.
struct GemvPlan {
    int unroll;     // 16-byte chunks each thread loads per pass (template instance)
    int tile_rows;  // rows per workgroup (per tile for the streaming kernel)
    bool act_lds;   // stage the activation in LDS (large matrices) instead of loading it with the weights
    bool stream;    // persistent streaming kernel (large matrices): `grid` workgroups walk the tiles
    int grid;       // workgroups of the streaming kernel
};
GemvPlan gemv_plan(int dtype, int cols, int rows);
size_t gemv_lds_bytes(int cols, int tile_rows, bool act_lds);

// Compute units of the current device (cached per device).
int device_cus();

// Largest supported cols for the decode GEMV and the prefill matmul.
constexpr int kMaxCols = 32768;

hipError_t launch_quantize_q8(const float* x, int n_tok, int n, int8_t* q, float* d, hipStream_t s);
hipError_t launch_gemv(float* out, const qh_tensor& W, const int8_t* xq, const float* xd, int r0, int r1,
                       const GemvPlan& plan, hipStream_t s);
hipError_t launch_matmul(float* out, int ldo, const qh_tensor& W, const int8_t* xq, const float* xd, int n,
                         int r0, int r1, hipStream_t s);
// matvec_ref for F32 / F16 W over n tokens of f32 activations x [n][ldx]: out[t * ldo + r], rows [r0, r1).
hipError_t launch_gemv_dense(float* out, int ldo, const qh_tensor& W, const float* x, int ldx, int n, int r0, int r1,
                             hipStream_t s);
// One matrix of a fused launch: rows [r0, r1) of W, output row r of token t at out[t * ldo + r].
struct MmOut {
    const qh_tensor* W;
    float* out;
    int ldo, r0, r1;
};
// Up to three matrices of one dtype and width over the same activation in one launch (prefill q / k / v, gate / up).
hipError_t launch_matmul_segs(const MmOut* m, int n_mats, const int8_t* xq, const float* xd, int n, hipStream_t s);
// Gate / up of n >= 128 tokens (a prefill stack) with h = g / (1 + expf(-g)) * u quantized per 32 rows into hq / hd
// ([n][rows], [n][rows / 32]) in one tile launch; hipErrorNotSupported (nothing launched) where the tile plan or the
// shapes do not allow it.
hipError_t launch_matmul_swiglu(const qh_tensor& wg, const qh_tensor& wu, const int8_t* xq, const float* xd, int n,
                                int8_t* hq, float* hd, hipStream_t s);
size_t argmax_workspace_bytes(int n);
hipError_t launch_argmax(const float* logits, int n, int32_t* index, void* ws, hipStream_t s);

// Shortlist head. Workspace layout is private to qh_head.hip. Supported hidden sizes: D % 64 == 0 (whole 4-byte
// words of f16 block errors per row) and D <= kMaxHeadCols (a tile's errors fit one register pass).
constexpr int kMaxHeadCols = 4096;
bool head_shape_supported(int D);
// 0 when the seed selection cannot hold the rows of the top_k + 9 screen shares (very large vocabularies with a
// large top_k).
size_t head_workspace_bytes(int V, int D, int top_k);
bool head_select_supported(int V, int D, int top_k);
// The must ids of a head query (HeadQuery::must, model.h:24-29): ids[0, n) known on the host, or, with len_dev set,
// the last `window` ids (all of them when window <= 0) of a device-resident history ids[0, *len_dev), which the
// kernels read when they run (Session::head_query, session.cpp:63-79), so a captured launch follows the history.
struct HeadMust {
    const int32_t* ids = nullptr;
    int n = 0;
    const int* len_dev = nullptr;
    int window = 0;
};
#if defined(__HIPCC__)
// The must ids a query names, read where the kernel runs (a device-resident history is read at that point).
__device__ __forceinline__ void must_span(const HeadMust& m, const int32_t*& ids, int& n) {
    if (m.len_dev) {
        const int len = *m.len_dev;
        const int from = (m.window > 0 && len > m.window) ? len - m.window : 0;
        ids = m.ids + from;
        n = len > from ? len - from : 0;
    } else {
        ids = m.ids;
        n = m.n;
    }
}
#endif
// The decoder's feedback of a chosen token (session.cpp:45-46): it becomes the next input, is appended to the output
// list and to the token history, and, after a decode step (advance), the position moves on.
struct TokenFeedback {
    int32_t* token = nullptr;
    int* pos = nullptr;
    int* n_out = nullptr;
    int32_t* out = nullptr;
    int out_cap = 0;
    int32_t* hist = nullptr;
    int* hist_len = nullptr;
    int hist_cap = 0;
#if defined(__HIPCC__)
    __device__ __forceinline__ void apply(int id, bool advance) const {
        const int k = *n_out, h = *hist_len;
        const int p = advance ? *pos : 0;
        *token = id;
        if (k < out_cap) out[k] = id;
        *n_out = k + 1;
        if (h < hist_cap) {
            hist[h] = id;
            *hist_len = h + 1;
        }
        if (advance) *pos = p + 1;
    }
#endif
};
// q.must / q.n_must are ignored: the must ids come from `must`. With `advance` set (greedy decoding), the last
// candidate workgroup also feeds the top-1 token back (TokenFeedback::apply with advance), which saves a launch.
hipError_t launch_shortlist_head(const qh_tensor& head8, const qh_tensor& head4, const qh_tensor& err,
                                 const int8_t* xq, const float* xd, const qh_head_query& q, const HeadMust& must,
                                 const qh_head_out& out, void* ws, hipStream_t s,
                                 const TokenFeedback* advance = nullptr);

// The nibble-plane layout (QH_Q8_0_PLANES) of a Q8_0 [V][D] head at planes (the same size, not overlapping it).
hipError_t launch_head_planes(const void* head8, void* planes, int V, int D, hipStream_t s);
// matvec_q over a nibble-plane head (rows [r0, r1) of out), bit-identical to the Q8_0 GEMV of the same values.
hipError_t launch_gemv_planes(float* out, const qh_tensor& planes, const int8_t* xq, const float* xd, int r0, int r1,
                              hipStream_t s);

// Sampler::sample on the device (qh_sample.hip). Candidates: rows[0, hs->n_rows) (the shortlist head's list; every
// other id counts as -inf) or, with rows null, every id below n_valid; the penalty looks at the ids `hist` names.
// Requires 1 <= n_valid <= QH_SAMPLE_MAX_VOCAB; with temperature > 0 and more than QH_SAMPLE_MAX_TOPK survivors, a
// workspace of sample_workspace_bytes(n_valid) (the sorted path), else ws may be null.
size_t sample_workspace_bytes(int n_valid);
hipError_t launch_sample(const float* logits, int n_valid, const int32_t* rows, const qh_head_stats* hs,
                         const HeadMust& hist, const qh_sampler_params& p, uint64_t* state, int32_t* out_id,
                         void* ws, hipStream_t s);

// GPU-resident decoder (qh_decoder.hip). Tensors in qh_decoder_create order; all sizes validated by the caller.
struct Decoder;
int decoder_create(const qh_model_desc* hp, const qh_tensor* tensors, int n_tensors, Decoder** out);
void decoder_destroy(Decoder* d);
// The prefill stack (tokens whose matmuls share a launch, kChunk..1024): reallocates the work buffers (synchronises).
hipError_t decoder_set_prefill_stack(Decoder* d, int c);
hipError_t decoder_prefill(Decoder* d, const int32_t* tokens, int n, int pos0, int top_k, hipStream_t s);
hipError_t decoder_begin(Decoder* d, int top_k, int32_t* out, int out_cap, hipStream_t s);
hipError_t decoder_step(Decoder* d, int top_k, hipStream_t s);
int decoder_step_timed(Decoder* d, int top_k, hipStream_t s, float* us, int32_t* stage, int cap, int32_t* n);
void decoder_views(Decoder* d, qh_decoder_state* v);
int decoder_set_query(Decoder* d, const qh_sampler_params* p);
hipError_t decoder_set_sampler(Decoder* d, const qh_sampler_params* p, uint64_t seed);
int decoder_vocab(const Decoder* d);
bool decoder_has_shortlist(const Decoder* d);
int decoder_ctx(const Decoder* d);

}  // namespace qh
