// GPU-resident decoder for the q4mix Qwen2-shaped model: the reference's Model::forward and forward_batch
// (engine/src/model.cpp:165-228, 349-433) with the operation order of its CPU build, so every hidden state, logit and
// greedy token is bit-identical to the reference.
//
// Per layer and token (decode: one token; prefill: a chunk of up to 32 tokens, all at once):
//   add_rmsnorm_quant  residual add (previous down / o projection), rmsnorm (serial FMA sum of squares, one rounded
//                      1/sqrt), int8 quantization per 32-block              (model.cpp:178-179, 211-213)
//   q, k, v            decode GEMV or prefill int8-MFMA matmul            (model.cpp:180-182, 377-379)
//   bias_rope_kv       biases, RoPE from a host table (glibc powf/cosf/sinf of the reference's formula), f16 K/V
//                      store at the token's position                       (model.cpp:183-195, 385-395)
//   attention          one workgroup per (head, token): scores (serial FMA dot over head_dim), max, glibc-identical
//                      expf, serial sum in position order, normalise, serial weighted V sum in position order
//                      (model.cpp:115-137, ops_ref.cpp:216-226)
//   quantize, o        the attention output is quantized and projected    (model.cpp:207-208)
//   gate, up, swiglu   g / (1 + expf(-g)) * u                              (ops_ref.cpp:243-248)
//   quantize, down     then the next layer's add_rmsnorm_quant adds it to the residual stream
// then the final add + rmsnorm + quantize and the head (Exact Shortlist Head for top-k queries, full 8-bit head
// otherwise). Decoding keeps the position and the token on the device, so one decode step is a fixed sequence of
// launches that a caller can capture in a HIP graph and replay: the step reads the token the previous step chose,
// and its last kernel writes the new token, appends it to the output list and advances the position.
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <vector>

#include "qh_device.h"
#include "qh_internal.h"
#include "qh_math.h"

namespace qh {

namespace {

constexpr int kChunk = 32;  // prefill chunk (reference Model::kBatch, model.h:52)

// glibc-identical expf on the device (all 2^32 inputs checked against the host's expf in tests).
__device__ __forceinline__ float dev_expf(float x) { return expf_variant<2>(x); }

__device__ __forceinline__ float h2f(uint16_t h) { return f16_to_f32(h); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// ------------------------------------------------------------------------------------------------------ kernels

// x[t] = embedding row of tokens[t] (Q8_0 get_row, ops_ref.cpp:176-181): code * f16 scale, exact in f32.
__global__ __launch_bounds__(256) void embed_kernel(const int32_t* __restrict__ tokens, const int8_t* __restrict__ eq,
                                                    const uint16_t* __restrict__ es, int D, float* __restrict__ x) {
    const int t = blockIdx.x;
    const int tok = tokens[t];
    for (int i = threadIdx.x; i < D; i += 256)
        x[(size_t)t * D + i] = (float)eq[(size_t)tok * D + i] * h2f(es[(size_t)tok * (D / QK) + i / QK]);
}

// One workgroup per token: optional residual add x += o, then rmsnorm with weight w and int8 quantization of the
// normed row; the normed row is also written to `normed` when given. D <= 8192.
__global__ __launch_bounds__(256) void add_rmsnorm_quant_kernel(float* __restrict__ x, const float* __restrict__ o,
                                                                const float* __restrict__ w, int D, float eps,
                                                                int8_t* __restrict__ xq, float* __restrict__ xd,
                                                                float* __restrict__ normed) {
    __shared__ float xs[8192];
    __shared__ float scale_sh;
    const int t = blockIdx.x, tid = threadIdx.x;
    float* xr = x + (size_t)t * D;
    for (int i = tid; i < D; i += 256) {
        float v = xr[i];
        if (o) {
            v = v + o[(size_t)t * D + i];
            xr[i] = v;
        }
        xs[i] = v;
    }
    __syncthreads();
    if (tid == 0) {  // ops_ref.cpp:195-196: ss += x*x (one FMA per element, in order), then 1/sqrt(ss/n + eps)
        float ss = 0.0f;
        for (int i = 0; i < D; ++i) ss = __builtin_fmaf(xs[i], xs[i], ss);
        scale_sh = 1.0f / __builtin_sqrtf(ss / (float)D + eps);
    }
    __syncthreads();
    const float scale = scale_sh;
    for (int i = tid; i < D; i += 256) xs[i] = xs[i] * scale * w[i];
    __syncthreads();
    if (normed)
        for (int i = tid; i < D; i += 256) normed[(size_t)t * D + i] = xs[i];
    // quantize_q8 (ops_ref.cpp:69-83): a half-wave per 32-block
    const int nb = D / QK;
    for (int b0 = 0; b0 < nb; b0 += 8) {
        const int b = b0 + (tid >> 5), i = tid & 31;
        const bool ok = b < nb;
        const float v = ok ? xs[b * QK + i] : 0.0f;
        float a = __builtin_fabsf(v);
#pragma unroll
        for (int off = 16; off >= 1; off >>= 1) a = __builtin_fmaxf(a, __shfl_xor(a, off, 64));
        const float d = a / 127.0f;
        const float inv = d > 0.0f ? 1.0f / d : 0.0f;
        if (ok) {
            xq[(size_t)t * D + b * QK + i] = (int8_t)(int)round_half_away(v * inv);
            if (i == 0) xd[(size_t)t * nb + b] = d;
        }
    }
}

// Biases, RoPE and the K/V store for n tokens at positions pos0 + t. One workgroup per token.
// rope (ops_ref.cpp:201-214): p[i] = a*c - b*s and p[i+half] = b*c + a*s with the reference build's contraction,
// i.e. fma(a, c, -(b*s)) and fma(b, c, a*s).
__global__ __launch_bounds__(256) void bias_rope_kv_kernel(float* __restrict__ q, float* __restrict__ k,
                                                           float* __restrict__ v, const float* __restrict__ bq,
                                                           const float* __restrict__ bk, const float* __restrict__ bv,
                                                           const float* __restrict__ cs, const int* __restrict__ pos_dev,
                                                           int n_heads, int n_kv, int hd, uint16_t* __restrict__ kc,
                                                           uint16_t* __restrict__ vc) {
    const int t = blockIdx.x, tid = threadIdx.x;
    const int pos = *pos_dev + t;
    const int qd = n_heads * hd, kvd = n_kv * hd, half = hd / 2;
    float* qt = q + (size_t)t * qd;
    float* kt = k + (size_t)t * kvd;
    float* vt = v + (size_t)t * kvd;
    const float* c = cs + (size_t)pos * hd;  // [half][2]
    for (int e = tid; e < (n_heads + n_kv) * half; e += 256) {
        const int h = e / half, i = e % half;
        const bool isq = h < n_heads;
        float* p = isq ? qt + h * hd : kt + (h - n_heads) * hd;
        const float* bb = isq ? (bq ? bq + h * hd : nullptr) : (bk ? bk + (h - n_heads) * hd : nullptr);
        float a = p[i], b = p[i + half];
        if (bb) {
            a = a + bb[i];
            b = b + bb[i + half];
        }
        const float cc = c[2 * i], ss = c[2 * i + 1];
        const float na = __builtin_fmaf(a, cc, -(b * ss));
        const float nb = __builtin_fmaf(b, cc, a * ss);
        if (isq) {
            p[i] = na;
            p[i + half] = nb;
        } else {
            const int kh = h - n_heads;
            kc[(size_t)pos * kvd + kh * hd + i] = f2h(na);
            kc[(size_t)pos * kvd + kh * hd + i + half] = f2h(nb);
        }
    }
    for (int i = tid; i < kvd; i += 256) {
        float val = vt[i];
        if (bv) val = val + bv[i];
        vc[(size_t)pos * kvd + i] = f2h(val);
    }
}

// Attention of token t (position pos0 + t) and query head h over cached positions [0, pos]. One workgroup per
// (head, token); scores live in LDS (ctx <= 8192).
__global__ __launch_bounds__(256) void attention_kernel(const float* __restrict__ q, const uint16_t* __restrict__ kc,
                                                        const uint16_t* __restrict__ vc, const int* __restrict__ pos_dev,
                                                        int n_heads, int n_kv, int hd, float* __restrict__ out) {
    __shared__ float att[8192];
    __shared__ float qs[256];
    __shared__ float red[4];
    __shared__ float inv_sh;
    const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int pos = *pos_dev + t;
    const int kvd = n_kv * hd, group = n_heads / n_kv, kvh = h / group;
    const float scale = 1.0f / __builtin_sqrtf((float)hd);
    for (int i = tid; i < hd; i += 256) qs[i] = q[(size_t)t * n_heads * hd + h * hd + i];
    __syncthreads();
    // scores: s = sum_i q_i * k_i as one FMA per element in order, then * scale (model.cpp:122-125)
    float mx = -__builtin_inff();
    for (int j = tid; j <= pos; j += 256) {
        const uint16_t* kr = kc + (size_t)j * kvd + kvh * hd;
        float s = 0.0f;
        for (int i = 0; i < hd; i += 8) {
            const uint4 kv8 = *reinterpret_cast<const uint4*>(kr + i);
            const uint32_t wv[4] = {kv8.x, kv8.y, kv8.z, kv8.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                s = __builtin_fmaf(qs[i + 2 * e], h2f((uint16_t)(wv[e] & 0xffffu)), s);
                s = __builtin_fmaf(qs[i + 2 * e + 1], h2f((uint16_t)(wv[e] >> 16)), s);
            }
        }
        const float a = s * scale;
        att[j] = a;
        mx = a > mx ? a : mx;
    }
    // the maximum does not depend on the order of comparison
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float o = __shfl_xor(mx, off, 64);
        mx = o > mx ? o : mx;
    }
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = red[0];
    for (int w = 1; w < 4; ++w) mx = red[w] > mx ? red[w] : mx;
    for (int j = tid; j <= pos; j += 256) att[j] = dev_expf(att[j] - mx);
    __syncthreads();
    if (tid == 0) {  // softmax sum in position order (ops_ref.cpp:220-224)
        float sum = 0.0f;
        for (int j = 0; j <= pos; ++j) sum = sum + att[j];
        inv_sh = 1.0f / sum;
    }
    __syncthreads();
    const float inv = inv_sh;
    for (int j = tid; j <= pos; j += 256) att[j] = att[j] * inv;
    __syncthreads();
    // out_i = sum_j a_j * v_ji, one FMA per position in order (model.cpp:131-135): thread i per dimension
    if (tid < hd) {
        const uint16_t* vr = vc + kvh * hd + tid;
        float acc = 0.0f;
        int j = 0;
        for (; j + 4 <= pos + 1; j += 4) {
            const uint16_t v0 = vr[(size_t)j * kvd], v1 = vr[(size_t)(j + 1) * kvd];
            const uint16_t v2 = vr[(size_t)(j + 2) * kvd], v3 = vr[(size_t)(j + 3) * kvd];
            acc = __builtin_fmaf(att[j], h2f(v0), acc);
            acc = __builtin_fmaf(att[j + 1], h2f(v1), acc);
            acc = __builtin_fmaf(att[j + 2], h2f(v2), acc);
            acc = __builtin_fmaf(att[j + 3], h2f(v3), acc);
        }
        for (; j <= pos; ++j) acc = __builtin_fmaf(att[j], h2f(vr[(size_t)j * kvd]), acc);
        out[(size_t)t * n_heads * hd + h * hd + tid] = acc;
    }
}

// h = g / (1 + expf(-g)) * u over n elements (ops_ref.cpp:243-248).
__global__ __launch_bounds__(256) void swiglu_kernel(const float* __restrict__ g, const float* __restrict__ u, long n,
                                                     float* __restrict__ h) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i < n) {
        const float gv = g[i];
        h[i] = gv / (1.0f + dev_expf(-gv)) * u[i];
    }
}

// Prefill / decode bookkeeping on the device.
__global__ void set_pos_kernel(int* pos_dev, int value) { *pos_dev = value; }

// After a decode step: the chosen token becomes the next input, is appended to out[] and the position advances.
__global__ void advance_kernel(const qh_head_stats* __restrict__ stats, const int32_t* __restrict__ top1_full,
                               int32_t* __restrict__ token, int* __restrict__ pos_dev, int* __restrict__ n_out,
                               int32_t* __restrict__ out, int out_cap) {
    const int id = stats ? stats->top1 : *top1_full;
    *token = id;
    const int k = *n_out;
    if (k < out_cap) out[k] = id;
    *n_out = k + 1;
    *pos_dev = *pos_dev + 1;
}

// Chooses the first generated token from the prefill's head (the reference samples it from the prompt's logits,
// session.cpp:39-41): copies it to the decode input without advancing the position.
__global__ void first_token_kernel(const qh_head_stats* __restrict__ stats, const int32_t* __restrict__ top1_full,
                                   int32_t* __restrict__ token, int* __restrict__ n_out, int32_t* __restrict__ out,
                                   int out_cap) {
    const int id = stats ? stats->top1 : *top1_full;
    *token = id;
    const int k = *n_out;
    if (k < out_cap) out[k] = id;
    *n_out = k + 1;
}

}  // namespace

// ------------------------------------------------------------------------------------------------- host side

struct Decoder {
    qh_model_desc hp;
    std::vector<qh_tensor> t;  // the caller's device tensors, in the qh_decoder_create order
    // device state
    uint16_t *kc = nullptr, *vc = nullptr;
    float* cs = nullptr;
    float *x = nullptr, *o = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *att = nullptr, *g = nullptr,
          *u = nullptr, *hbuf = nullptr, *hidden = nullptr;
    int8_t* xq = nullptr;
    float* xd = nullptr;
    int32_t* tokens = nullptr;  // [kChunk] prefill input / [0] decode input
    int* pos = nullptr;         // current position
    int* n_out = nullptr;
    int32_t* out = nullptr;
    int out_cap = 0;
    // head
    float *logits = nullptr, *coarse = nullptr, *upper = nullptr;
    int32_t* rows = nullptr;
    qh_head_stats* stats = nullptr;
    void* head_ws = nullptr;
    size_t head_ws_bytes = 0;
    void* am_ws = nullptr;
    size_t am_ws_bytes = 0;
    int32_t* top1_full = nullptr;
    std::vector<void*> allocs;
};

namespace {

enum { T_EMBED, T_NORM, T_LAYER0 };
enum { L_ATTN_NORM, L_WQ, L_WK, L_WV, L_WO, L_BQ, L_BK, L_BV, L_FFN_NORM, L_WG, L_WU, L_WD, L_COUNT };

const qh_tensor& lt(const Decoder* d, int l, int which) { return d->t[T_LAYER0 + l * L_COUNT + which]; }
const float* lf(const Decoder* d, int l, int which) { return static_cast<const float*>(lt(d, l, which).data); }
const qh_tensor& head4(const Decoder* d) { return d->t[T_LAYER0 + d->hp.n_layers * L_COUNT]; }
const qh_tensor& head_err(const Decoder* d) { return d->t[T_LAYER0 + d->hp.n_layers * L_COUNT + 1]; }

hipError_t dalloc(Decoder* d, void** p, size_t bytes) {
    hipError_t e = hipMalloc(p, bytes < 256 ? 256 : bytes);
    if (e == hipSuccess) d->allocs.push_back(*p);
    return e;
}

// GEMV for one token, int8-MFMA matmul for several (identical per row).
hipError_t linear(float* out, const qh_tensor& W, const int8_t* xq, const float* xd, int n, hipStream_t s) {
    if (n == 1) return launch_gemv(out, W, xq, xd, 0, W.rows, gemv_plan(W.dtype, W.cols, W.rows), s);
    return launch_matmul(out, W.rows, W, xq, xd, n, 0, W.rows, s);
}

#define QH_TRY(expr)                                 \
    do {                                             \
        const hipError_t e_ = (expr);                \
        if (e_ != hipSuccess) return e_;             \
    } while (0)

// All layers for n tokens whose embeddings are in d->x[0..n) and whose positions start at *d->pos. Leaves the last
// layer's down projection in d->o (not yet added to the residual stream).
hipError_t run_layers(Decoder* d, int n, hipStream_t s) {
    const qh_model_desc& hp = d->hp;
    const int D = hp.dim, F = hp.ffn_dim, hd = hp.head_dim, qd = hp.n_heads * hd, kvd = hp.n_kv_heads * hd;
    const size_t layer_kv = (size_t)hp.ctx_len * kvd;
    for (int l = 0; l < hp.n_layers; ++l) {
        hipLaunchKernelGGL(add_rmsnorm_quant_kernel, dim3(n), dim3(256), 0, s, d->x, l == 0 ? nullptr : d->o,
                           lf(d, l, L_ATTN_NORM), D, hp.norm_eps, d->xq, d->xd, nullptr);
        QH_TRY(hipGetLastError());
        QH_TRY(linear(d->q, lt(d, l, L_WQ), d->xq, d->xd, n, s));
        QH_TRY(linear(d->k, lt(d, l, L_WK), d->xq, d->xd, n, s));
        QH_TRY(linear(d->v, lt(d, l, L_WV), d->xq, d->xd, n, s));
        hipLaunchKernelGGL(bias_rope_kv_kernel, dim3(n), dim3(256), 0, s, d->q, d->k, d->v,
                           hp.qkv_bias ? lf(d, l, L_BQ) : nullptr, hp.qkv_bias ? lf(d, l, L_BK) : nullptr,
                           hp.qkv_bias ? lf(d, l, L_BV) : nullptr, d->cs, d->pos, hp.n_heads, hp.n_kv_heads, hd,
                           d->kc + l * layer_kv, d->vc + l * layer_kv);
        QH_TRY(hipGetLastError());
        hipLaunchKernelGGL(attention_kernel, dim3(hp.n_heads, n), dim3(256), 0, s, d->q, d->kc + l * layer_kv,
                           d->vc + l * layer_kv, d->pos, hp.n_heads, hp.n_kv_heads, hd, d->att);
        QH_TRY(hipGetLastError());
        QH_TRY(launch_quantize_q8(d->att, n, qd, d->xq, d->xd, s));
        QH_TRY(linear(d->o, lt(d, l, L_WO), d->xq, d->xd, n, s));
        hipLaunchKernelGGL(add_rmsnorm_quant_kernel, dim3(n), dim3(256), 0, s, d->x, d->o, lf(d, l, L_FFN_NORM), D,
                           hp.norm_eps, d->xq, d->xd, nullptr);
        QH_TRY(hipGetLastError());
        QH_TRY(linear(d->g, lt(d, l, L_WG), d->xq, d->xd, n, s));
        QH_TRY(linear(d->u, lt(d, l, L_WU), d->xq, d->xd, n, s));
        const long nf = (long)n * F;
        hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((nf + 255) / 256)), dim3(256), 0, s, d->g, d->u, nf, d->hbuf);
        QH_TRY(hipGetLastError());
        QH_TRY(launch_quantize_q8(d->hbuf, n, F, d->xq, d->xd, s));
        QH_TRY(linear(d->o, lt(d, l, L_WD), d->xq, d->xd, n, s));
    }
    return hipSuccess;
}

// Final residual add, norm and quantization of row `row` of d->x, then the head; top_k > 0 uses the shortlist.
hipError_t run_head(Decoder* d, int row, int top_k, hipStream_t s) {
    const qh_model_desc& hp = d->hp;
    const int D = hp.dim;
    float* xr = d->x + (size_t)row * D;
    float* orow = d->o + (size_t)row * D;
    hipLaunchKernelGGL(add_rmsnorm_quant_kernel, dim3(1), dim3(256), 0, s, xr, orow,
                       static_cast<const float*>(d->t[T_NORM].data), D, hp.norm_eps, d->xq, d->xd, d->hidden);
    QH_TRY(hipGetLastError());
    const qh_tensor& h8 = d->t[T_EMBED];
    if (top_k > 0 && head4(d).data) {
        qh_head_query q{top_k, hp.vocab_size, nullptr, 0};
        qh_head_out out{d->logits, d->coarse, d->upper, d->rows, d->stats};
        return launch_shortlist_head(h8, head4(d), head_err(d), d->xq, d->xd, q, out, d->head_ws, s);
    }
    QH_TRY(launch_gemv(d->logits, h8, d->xq, d->xd, 0, h8.rows, gemv_plan(h8.dtype, h8.cols, h8.rows), s));
    return launch_argmax(d->logits, hp.vocab_size, d->top1_full, d->am_ws, s);
}

}  // namespace

// ------------------------------------------------------------------------------------------------- C-ABI glue

int decoder_create(const qh_model_desc* hp, const qh_tensor* tensors, int n_tensors, Decoder** out) {
    auto* d = new Decoder();
    d->hp = *hp;
    d->t.assign(tensors, tensors + n_tensors);
    const int D = hp->dim, F = hp->ffn_dim, V = hp->vocab_size, hd = hp->head_dim;
    const size_t kvd = (size_t)hp->n_kv_heads * hd;
    const size_t kv_bytes = (size_t)hp->n_layers * hp->ctx_len * kvd * 2;
    const int wide = D > F ? D : F;
    hipError_t e = hipSuccess;
    auto A = [&](void** p, size_t b) {
        if (e == hipSuccess) e = dalloc(d, p, b);
    };
    A((void**)&d->kc, kv_bytes);
    A((void**)&d->vc, kv_bytes);
    A((void**)&d->cs, sizeof(float) * (size_t)hp->ctx_len * hd);
    A((void**)&d->x, sizeof(float) * kChunk * D);
    A((void**)&d->o, sizeof(float) * kChunk * D);
    A((void**)&d->q, sizeof(float) * kChunk * D);
    A((void**)&d->k, sizeof(float) * kChunk * kvd);
    A((void**)&d->v, sizeof(float) * kChunk * kvd);
    A((void**)&d->att, sizeof(float) * kChunk * D);
    A((void**)&d->g, sizeof(float) * kChunk * F);
    A((void**)&d->u, sizeof(float) * kChunk * F);
    A((void**)&d->hbuf, sizeof(float) * kChunk * F);
    A((void**)&d->hidden, sizeof(float) * D);
    A((void**)&d->xq, (size_t)kChunk * wide);
    A((void**)&d->xd, sizeof(float) * kChunk * (wide / QK));
    A((void**)&d->tokens, sizeof(int32_t) * kChunk);
    A((void**)&d->pos, 256);
    A((void**)&d->n_out, 256);
    A((void**)&d->logits, sizeof(float) * V);
    A((void**)&d->coarse, sizeof(float) * V);
    A((void**)&d->upper, sizeof(float) * V);
    A((void**)&d->rows, sizeof(int32_t) * (size_t)(V + 64));
    A((void**)&d->stats, sizeof(qh_head_stats));
    A((void**)&d->top1_full, 256);
    d->head_ws_bytes = head_workspace_bytes(V, D, QH_HEAD_MAX_TOPK);
    A(&d->head_ws, d->head_ws_bytes);
    d->am_ws_bytes = argmax_workspace_bytes(V);
    A(&d->am_ws, d->am_ws_bytes);
    if (e != hipSuccess) {
        decoder_destroy(d);
        return check_hip(e, "qh_decoder_create allocation");
    }
    // RoPE angle table with the reference's formula and the host's libm (ops_ref.cpp:201-214).
    std::vector<float> cs((size_t)hp->ctx_len * hd);
    const int half = hd / 2;
    for (int p = 0; p < hp->ctx_len; ++p)
        for (int i = 0; i < half; ++i) {
            const float freq = powf(hp->rope_theta, -2.0f * (float)i / (float)hd);
            const float angle = (float)p * freq;
            cs[((size_t)p * half + i) * 2] = cosf(angle);
            cs[((size_t)p * half + i) * 2 + 1] = sinf(angle);
        }
    e = hipMemcpy(d->cs, cs.data(), sizeof(float) * cs.size(), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemset(d->n_out, 0, 256);
    if (e == hipSuccess) e = hipMemset(d->pos, 0, 256);
    if (e != hipSuccess) {
        decoder_destroy(d);
        return check_hip(e, "qh_decoder_create upload");
    }
    *out = d;
    return QH_OK;
}

void decoder_destroy(Decoder* d) {
    if (!d) return;
    for (void* p : d->allocs) (void)hipFree(p);
    delete d;
}

hipError_t decoder_prefill(Decoder* d, const int32_t* tokens, int n, int pos0, int top_k, hipStream_t s) {
    const qh_model_desc& hp = d->hp;
    const qh_tensor& emb = d->t[T_EMBED];
    const int8_t* eq = static_cast<const int8_t*>(emb.data);
    const uint16_t* es = reinterpret_cast<const uint16_t*>(eq + (size_t)emb.rows * emb.cols);
    int last = 0;
    for (int c0 = 0; c0 < n; c0 += kChunk) {
        const int m = n - c0 < kChunk ? n - c0 : kChunk;
        hipLaunchKernelGGL(set_pos_kernel, dim3(1), dim3(1), 0, s, d->pos, pos0 + c0);
        QH_TRY(hipGetLastError());
        hipLaunchKernelGGL(embed_kernel, dim3(m), dim3(256), 0, s, tokens + c0, eq, es, hp.dim, d->x);
        QH_TRY(hipGetLastError());
        QH_TRY(run_layers(d, m, s));
        last = m - 1;
    }
    QH_TRY(run_head(d, last, top_k, s));
    hipLaunchKernelGGL(set_pos_kernel, dim3(1), dim3(1), 0, s, d->pos, pos0 + n);
    return hipGetLastError();
}

hipError_t decoder_step(Decoder* d, int top_k, hipStream_t s) {
    const qh_model_desc& hp = d->hp;
    const qh_tensor& emb = d->t[T_EMBED];
    const int8_t* eq = static_cast<const int8_t*>(emb.data);
    const uint16_t* es = reinterpret_cast<const uint16_t*>(eq + (size_t)emb.rows * emb.cols);
    hipLaunchKernelGGL(embed_kernel, dim3(1), dim3(256), 0, s, d->tokens, eq, es, hp.dim, d->x);
    QH_TRY(hipGetLastError());
    QH_TRY(run_layers(d, 1, s));
    QH_TRY(run_head(d, 0, top_k, s));
    const bool sl = top_k > 0 && head4(d).data;
    hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(1), 0, s, sl ? d->stats : nullptr, d->top1_full, d->tokens,
                       d->pos, d->n_out, d->out, d->out_cap);
    return hipGetLastError();
}

hipError_t decoder_begin(Decoder* d, int top_k, int32_t* out, int out_cap, hipStream_t s) {
    d->out = out;
    d->out_cap = out_cap;
    hipLaunchKernelGGL(set_pos_kernel, dim3(1), dim3(1), 0, s, d->n_out, 0);
    QH_TRY(hipGetLastError());
    const bool sl = top_k > 0 && head4(d).data;
    hipLaunchKernelGGL(first_token_kernel, dim3(1), dim3(1), 0, s, sl ? d->stats : nullptr, d->top1_full, d->tokens,
                       d->n_out, d->out, d->out_cap);
    return hipGetLastError();
}

int decoder_ctx(const Decoder* d) { return d->hp.ctx_len; }

void decoder_views(Decoder* d, qh_decoder_state* v) {
    v->logits = d->logits;
    v->hidden = d->hidden;
    v->xq = d->xq;
    v->xd = d->xd;
    v->stats = d->stats;
    v->top1_full = d->top1_full;
    v->pos = d->pos;
    v->n_out = d->n_out;
    v->token = d->tokens;
    v->kcache = d->kc;
    v->vcache = d->vc;
}

}  // namespace qh
