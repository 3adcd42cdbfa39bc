/*
 * quanta_hip.h — C-ABI of the MI355X (gfx950) quantized matmul path.
 *
 * Drop-in boundary under the reference's L1 kernels (engine/src/ops.h) and its shortlist head
 * (engine/src/model.cpp:240-334). Plain pointers and sizes only. Every function returns a status
 * (QH_OK = 0); on failure qh_last_error() gives a message for the calling thread.
 *
 * Memory: every tensor, activation and output pointer below is a DEVICE pointer unless the
 * parameter name ends in _host. `stream` is a hipStream_t (NULL = the null stream). Calls only
 * enqueue work; nothing synchronises unless the function says so. Functions are reentrant and may
 * be called from any host thread; the only shared state is the per-device init record.
 *
 * Block layouts are the .qnt layouts, unchanged (reference engine/src/model_file.h:16-38,
 * scripts/export.py:10-13):
 *   Q8_0 [rows][cols]: int8 quants [rows*cols], then fp16 scales [rows*cols/32]
 *   Q4_0 [rows][cols]: packed nibbles [rows*cols/2] (per 32-block, byte j = (q[j]+8) | (q[j+16]+8)<<4),
 *                      then fp16 scales [rows*cols/32]
 *   quantized activation (QuantVec, ops.h:47-51): int8 q[cols], f32 d[cols/32]
 * Results are bit-identical to the reference's scalar kernels (ops_ref.cpp) on the same inputs.
 */
#ifndef QUANTA_HIP_H
#define QUANTA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
enum {
    QH_OK = 0,
    QH_ERR_ARG = 1,         /* null pointer, bad count or range */
    QH_ERR_DTYPE = 2,       /* dtype not allowed for this call */
    QH_ERR_SHAPE = 3,       /* cols % 32 != 0, mismatched tensors, size limits */
    QH_ERR_ALIGN = 4,       /* device pointer not 16-byte aligned */
    QH_ERR_HIP = 5,         /* a HIP runtime call failed */
    QH_ERR_NOMEM = 6,       /* workspace too small / allocation failed */
    QH_ERR_UNSUPPORTED = 7  /* e.g. top_k beyond the supported maximum */
};

/* Tensor dtypes, numbered as the .qnt file stores them (reference model_file.h:16, DType). */
enum { QH_F32 = 0, QH_F16 = 1, QH_Q8_0 = 2, QH_Q4_0 = 3 };

/* A device-only layout, never a .qnt dtype: a Q8_0 [rows][cols] head as nibble planes (qh_head_planes), the same
 * int8 values q = 16 h + l with h = floor(q / 16) in [-8, 7] and l = q - 16 h in [0, 15], in as many bytes as the
 * Q8_0 tensor: the high plane [rows][cols/2] (Q4_0 blocks of the codes h + 8), the low plane [rows][cols/2] (Q4_0
 * blocks of l, no offset), then the Q8_0 fp16 scales [rows][cols/32] unchanged. The shortlist head screens with the
 * high plane alone (reference research/head_deep.py:68-78, docs/PROGRESS.md:121-130). */
enum { QH_Q8_0_PLANES = 16 };

/* Quantization block size (reference model_file.h:17, QK). */
#define QH_QK 32

/* Device view of a .qnt tensor (reference model_file.h:27-38, Tensor): `data` is the device
 * address of the quant section; for Q8_0 / Q4_0 the fp16 scales follow at data + quant bytes. */
typedef struct qh_tensor {
    int32_t dtype;
    int32_t rows;
    int32_t cols;
    const void* data;
} qh_tensor;

/* Message of the last failed call on this thread ("" if none). */
const char* qh_last_error(void);

/* Library version string. */
const char* qh_version(void);

/* Selects `device` for the calling thread and records its properties (idempotent).
 * Replaces: nothing (the reference has no device); called once before the others. */
int qh_init(int device);

/* Size in bytes of the quant section (reference model_file.cpp:29-38, Tensor::quant_bytes). */
size_t qh_quant_bytes(int dtype, int rows, int cols);

/* Quant section plus scale section. */
size_t qh_tensor_bytes(int dtype, int rows, int cols);

/* Checks a tensor view: dtype, shape, cols % 32 and 16-byte alignment of `data`. */
int qh_validate_tensor(const qh_tensor* W);

/* Thin device-memory helpers so C/C++ callers need no HIP headers. */
int qh_malloc(void** ptr, size_t bytes);

/* Forced allocation failure, for tests of the error paths: after `after` more device allocations by the library
 * (qh_malloc and the decoder's own buffers), the next one fails with QH_ERR_NOMEM before any HIP call, and the hook
 * disarms itself; after < 0 disarms it. Process-wide. No counterpart in the reference: it is the fault hook its
 * failure handling is tested with (an allocation failure maps to an error code, nothing is leaked). */
int qh_fault_alloc(int after);
int qh_free(void* ptr);
int qh_memcpy_h2d(void* dst, const void* src_host, size_t bytes, void* stream); /* async */
int qh_memcpy_d2h(void* dst_host, const void* src, size_t bytes, void* stream); /* synchronous */
int qh_memset(void* dst, int value, size_t bytes, void* stream);
int qh_stream_sync(void* stream);
int qh_stream_create(void** stream); /* non-blocking stream at the default priority */
int qh_stream_destroy(void* stream);

/* Per-32-block int8 quantization of n_tok activation rows of length n (x is [n_tok][n] f32):
 * q [n_tok][n] int8, d [n_tok][n/32] f32.
 * Replaces: void quantize_q8(const float* x, int n, QuantVec& out)   (reference ops.h:52,
 *           implementation ops_ref.cpp:69-83), once per token row. */
int qh_quantize_q8(const float* x, int n_tok, int n, int8_t* q, float* d, void* stream);

/* Decode GEMV: out[r] = W[r,:] . x for r in [r0, r1) (out indexed by absolute row), W Q8_0 or Q4_0,
 * x = (xq [cols] int8, xd [cols/32] f32). Per row: int32 block dots, then the serial chain
 * acc = fma(float(s_b) * dw_b, dx_b, acc) in block order.
 * Replaces: void matvec_q(float* out, const Tensor& W, const QuantVec& x, int r0, int r1)
 *           (reference ops.h:61, MatvecQFn ops.h:57; implementation ops_ref.cpp:85-120). */
int qh_matvec_q(float* out, const qh_tensor* W, const int8_t* xq, const float* xd, int r0, int r1,
                void* stream);

/* GEMV over unquantized weights: out[r] = W[r,:] . x for r in [r0, r1), W F32 or F16 ([rows][cols] row-major, cols
 * a multiple of 32), x [cols] f32. Per row the serial chain acc = fma(w_i, x_i, acc) from +0 in column order (the
 * reference build's contraction of acc += w * x; an F16 weight is converted exactly).
 * Replaces: void matvec_ref(float* out, const Tensor& W, const float* x, int r0, int r1) for F32 / F16 W
 *           (reference ops.h:43, implementation ops_ref.cpp:8-27: Model::linear's path for an unquantized W,
 *           model.cpp:154-156). */
int qh_matvec_ref(float* out, const qh_tensor* W, const float* x, int r0, int r1, void* stream);

/* Prefill matmul for n tokens: out[t*ldo + r] for t in [0, n), r in [r0, r1); xq is [n][cols]
 * int8, xd is [n][cols/32] f32 (the n QuantVecs back to back). Every (row, token) value is
 * bit-identical to qh_matvec_q on that token (int8 MFMA, K = 32 per instruction = one block).
 * Replaces: void matmul_q(float* out, int ldo, const Tensor& W, const QuantVec* x, int n, int r0,
 *           int r1) (reference ops.h:69, MatmulQFn ops.h:68; implementation ops_ref.cpp:122-160). */
int qh_matmul_q(float* out, int ldo, const qh_tensor* W, const int8_t* xq, const float* xd, int n, int r0,
                int r1, void* stream);

/* Workspace bytes qh_argmax needs for n logits (0 if n <= 0); no initialisation needed. */
size_t qh_argmax_workspace_bytes(int n);

/* First index of the maximum of logits[0, n) written to *index (device int32). Calls that overlap must not
 * share a workspace.
 * Replaces: the greedy branch of Sampler::sample, std::max_element (reference sampler.cpp:35-37). */
int qh_argmax(const float* logits, int n, int32_t* index, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------ Exact Shortlist Head */

/* Which logits the caller needs (reference model.h:24-29, HeadQuery). `must` is a DEVICE array of
 * n_must ids. top_k must be in [1, QH_HEAD_MAX_TOPK]. */
typedef struct qh_head_query {
    int32_t top_k;
    int32_t n_valid; /* ids >= n_valid are ignored; 0 = whole vocab */
    const int32_t* must;
    int32_t n_must;
} qh_head_query;

#define QH_HEAD_MAX_TOPK 256 /* seeds = top_k + 8 (the sampler's survivor limit, QH_SAMPLE_MAX_TOPK) */

/* Device-side summary of one shortlist call. */
typedef struct qh_head_stats {
    int32_t top1;       /* first argmax of logits over [0, n_valid) (greedy token) */
    int32_t n_rows;     /* 8-bit rows rescored (reference Model::last_head_rows) */
    int32_t n_seeds;    /* seeds rescored first */
    int32_t n_cand;     /* candidates: upper bound >= tau */
    int32_t n_must;     /* must ids rescored */
    int32_t seed_tie;   /* 1 if the last seed's coarse score ties an unselected eligible row */
    float tau;          /* k-th best exact seed logit (-inf if fewer than k seeds) */
    float top1_logit;   /* logits[top1] */
} qh_head_stats;

/* Outputs of qh_shortlist_head, all device buffers owned by the caller. */
typedef struct qh_head_out {
    float* logits;        /* [V]: exact logit for rescored rows, -inf elsewhere */
    float* coarse;        /* [V]: 4-bit score (reference Model::head_coarse) */
    float* upper;         /* [V]: coarse + error bound (reference Model::head_upper) */
    int32_t* rows;        /* [V + n_must]: rescored rows: seeds (best coarse first), then candidates
                             (unordered), then must ids */
    qh_head_stats* stats; /* one record */
} qh_head_out;

/* Workspace bytes qh_shortlist_head needs for a V x D head and top_k (0 if unsupported: D must be a multiple
 * of 64 and at most 4096, V at most 1,048,576 on a 256-CU GPU). The workspace needs no initialisation (each call
 * resets what it uses); calls that overlap must not share one. */
size_t qh_shortlist_workspace_bytes(int V, int D, int top_k);

/* Exact Shortlist Head on one quantized hidden state (xq [D] int8, xd [D/32] f32):
 * 4-bit screen of all V rows with bound = fma(sum_b fma(err_b, xnorm_b), 1.001, 1e-5); seeds = the
 * top_k+8 best eligible coarse scores (lower row first on ties), rescored exactly; tau = k-th best
 * exact seed; candidates {r < n_valid, not seed or must, upper[r] >= tau} and must ids rescored
 * exactly; then the greedy argmax. head8 Q8_0 [V][D], head4 Q4_0 [V][D], err F16 [V][D/32].
 * Replaces: void Model::shortlist_head(const HeadQuery&) (reference model.cpp:240-334) followed by
 *           the greedy sample (sampler.cpp:35-37). */
int qh_shortlist_head(const qh_tensor* head8, const qh_tensor* head4, const qh_tensor* err, const int8_t* xq,
                      const float* xd, const qh_head_query* query, const qh_head_out* out, void* workspace,
                      size_t workspace_bytes, void* stream);

/* Bytes of the scratch array qh_shortlist_head_noalloc works in: one array in each GPU's memory, held by the library
 * until the process ends. Enough for the 151,936-row Qwen2.5 head (0.78 MB, the same at every top_k) and
 * for heads up to about 800,000 rows of 896. */
#define QH_NOALLOC_SCRATCH_BYTES ((size_t)4 << 20)

/* qh_shortlist_head with the same arguments and results but no workspace argument, and no device allocation of any
 * kind: its workspace is the library's scratch array on the current GPU. Fails with QH_ERR_NOMEM, launching nothing,
 * when qh_shortlist_workspace_bytes(V, D, top_k) exceeds QH_NOALLOC_SCRATCH_BYTES. Every call on one GPU works in that
 * GPU's one array, which keeps the last call's contents (the kernels reset what they read, so nothing of one call
 * reaches the next): calls in order on one stream are fine, calls that overlap on one GPU (two streams, or two host
 * threads without an order between them) race and give wrong results. The first call on a device runs qh_init for it
 * (device checks and the scratch array's address); under HIP graph capture, call qh_init for the device (or this entry
 * point once, eagerly) before the capture begins, so that the captured call only launches kernels.
 * No counterpart in the reference (its Model allocates the head's state on the host at load): for callers that cannot
 * allocate device memory, such as code under HIP graph capture, tight serving loops and harnesses that forbid
 * hipMalloc. */
int qh_shortlist_head_noalloc(const qh_tensor* head8, const qh_tensor* head4, const qh_tensor* err, const int8_t* xq,
                              const float* xd, const qh_head_query* query, const qh_head_out* out, void* stream);

/* The nibble-plane layout of a Q8_0 [V][D] head (D a multiple of 64): writes qh_tensor_bytes(QH_Q8_0_PLANES, V, D)
 * bytes (the Q8_0 tensor's size) at `planes`, a 16-byte aligned DEVICE buffer that must not overlap head8's data.
 * The caller may free the Q8_0 copy afterwards: the planes hold the same values, so the exact rows (and an embedding
 * lookup) can be read from them.
 * Replaces: the research layout "the Q8 ints stored as two nibble planes" (reference research/head_deep.py:8-10,
 *           68-78; docs/PROGRESS.md:121-130); the reference engine keeps the Q8_0 head and a separate Q4_0 copy. */
int qh_head_planes(const qh_tensor* head8, void* planes, void* stream);

/* The Exact Shortlist Head over a nibble-plane head alone (planes: QH_Q8_0_PLANES [V][D]), with no extra copy:
 * the screen reads the high plane and the scales (coarse = the chain acc = fma(float(sum_i (16 h_i + 8) x_i) * d_b,
 * dx_b, acc), the values at the midpoints of their high-nibble buckets; bound = fma(sum_b fma(d_b, (8 dx_b) *
 * sum_i |x_i|), 1.001, 1e-5), since |q - (16 h + 8)| = |l - 8| <= 8), then the same seeds, tau, candidates, must ids
 * and greedy argmax as qh_shortlist_head; exact rows are rebuilt from both planes, so every rescored logit is
 * bit-identical to the full Q8_0 head's. Outputs and workspace as qh_shortlist_head
 * (qh_shortlist_workspace_bytes(V, D, top_k)).
 * Replaces: the scope's nibble-plane shortlist variant (reference research/head_deep.py:68-78 "hi4, analytic
 *           bound", docs/PROGRESS.md:121-130) run through Model::shortlist_head's procedure (model.cpp:240-334). */
int qh_shortlist_planes(const qh_tensor* planes, const int8_t* xq, const float* xd, const qh_head_query* query,
                        const qh_head_out* out, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------ sampler */

/* The reference's SamplerParams (sampler.h) without the seed: the generator state lives in device memory. */
typedef struct qh_sampler_params {
    float temperature;    /* <= 0: greedy (first maximum after the penalty) */
    int32_t top_k;        /* 0 = disabled */
    float top_p;          /* 1 = disabled */
    float min_p;          /* 0 = disabled */
    float repeat_penalty; /* 1 = disabled; divides positive logits, multiplies negative ones (HF semantics) */
    int32_t repeat_window; /* how many recent history ids the penalty looks at; 0 = all */
} qh_sampler_params;

#define QH_SAMPLE_MAX_TOPK 256       /* survivors of the top-k cut qh_sample handles without a workspace */
#define QH_SAMPLE_MAX_VOCAB 262144   /* n_valid limit (the history bitmap lives in LDS) */

/* The generator state a reference Sampler constructed with a nonzero seed starts from (sampler.cpp:10-13). */
uint64_t qh_sampler_state(uint64_t seed);

/* One draw of Sampler::sample (sampler.cpp:22-85) on DEVICE logits: repetition penalty over the distinct ids of the
 * history window, then greedy, or top-k, softmax with temperature, min-p, top-p and a draw from the xorshift64*
 * generator whose state is the DEVICE uint64 *state (advanced by one draw when temperature > 0). The chosen id goes
 * to the DEVICE int32 *out_id. The logits are not modified (the reference samples from its own copy).
 *   rows / head_stats: the shortlist head's row list and stats (qh_shortlist_head's out.rows / out.stats), the only
 *                      ids whose logits are finite; NULL / NULL to consider every id below n_valid.
 *   history[0, n_hist): DEVICE token history (the session's prompt and generated ids), NULL when n_hist is 0.
 * Requires 1 <= n_valid <= QH_SAMPLE_MAX_VOCAB and, with temperature > 0, min(top_k or n_valid, n_valid) <=
 * QH_SAMPLE_MAX_TOPK (qh_sample_ws takes any number). Ties between equal logits in the top-k go to the lower id
 * (unspecified in the reference).
 * Replaces: Sampler::sample (reference sampler.cpp:22-85) and Sampler's generator (sampler.cpp:10-21). */
int qh_sample(const float* logits, int32_t n_valid, const int32_t* rows, const qh_head_stats* head_stats,
              const int32_t* history, int32_t n_hist, const qh_sampler_params* params, uint64_t* state,
              int32_t* out_id, void* stream);

/* qh_sample with a DEVICE workspace of qh_sample_workspace_bytes(n_valid) bytes (16-byte aligned), which lifts the
 * QH_SAMPLE_MAX_TOPK limit: any top_k, top_k 0 (every id a survivor) included. More survivors than that are sorted by
 * a device-wide radix sort (4 passes over the logit half); the softmax sum, top-p, total and draw then run in the
 * reference's order and stop where the remaining terms can no longer change a rounded result. Calls that share a
 * workspace must not overlap. Replaces: Sampler::sample (reference sampler.cpp:22-85) with top_k 0 or large. */
size_t qh_sample_workspace_bytes(int32_t n_valid);
int qh_sample_ws(const float* logits, int32_t n_valid, const int32_t* rows, const qh_head_stats* head_stats,
                 const int32_t* history, int32_t n_hist, const qh_sampler_params* params, uint64_t* state,
                 int32_t* out_id, void* ws, size_t ws_bytes, void* stream);

/* ------------------------------------------------------------------ GPU-resident decoder */

/* FLAG_HADAMARD_DOWN (reference engine/src/model_file.h:19-21): the down projection's input is rotated by the
 * block-diagonal 256 x 256 Walsh-Hadamard transform (model.cpp:216-220), the weights having been rotated offline. */
#define QH_FLAG_HADAMARD_DOWN 1u

/* Model shape (reference engine/src/model_file.h:40-45, HParams, with its flags) and the load options: the context
 * length of the KV cache and kv_f32, an f32 cache in place of fp16 (Model::load's kv_f16 = false, the CLI's --kv-f32,
 * model.cpp:96-104). */
typedef struct qh_model_desc {
    int32_t vocab_size, dim, n_layers, n_heads, n_kv_heads, head_dim, ffn_dim, ctx_len, qkv_bias;
    float rope_theta, norm_eps;
    uint32_t flags;  /* QH_FLAG_* */
    int32_t kv_f32;  /* 0: fp16 cache (the reference's default); 1: f32 cache */
} qh_model_desc;

typedef struct qh_decoder qh_decoder;

/* Device addresses of the decoder's results and state, valid until qh_decoder_destroy. */
typedef struct qh_decoder_state {
    float* logits;          /* [vocab]: the last head call's logits (-inf outside the shortlist) */
    float* hidden;          /* [dim]: the last head call's final normed hidden state */
    int8_t* xq;             /* [dim]: its int8 quantization (first dim bytes) */
    float* xd;              /* [dim / 32]: its block scales */
    qh_head_stats* stats;   /* the last shortlist call's summary (top1, n_rows, ...) */
    int32_t* top1_full;     /* the greedy token of the last full-head call */
    int32_t* pos;           /* next position */
    int32_t* n_out;         /* tokens written to the output list since qh_decoder_begin */
    int32_t* token;         /* the token the next step consumes */
    uint16_t* kcache;       /* [n_layers][n_kv_heads][head_dim / 8][ctx_len][8] fp16 bits: chunks of 8 dimensions
                               (position p, KV head h, dimension i at ((h * (head_dim / 8) + i / 8) * ctx_len + p) * 8
                               + i % 8 within its layer) */
    uint16_t* vcache;       /* [n_layers][ceil(ctx_len / 8)][n_kv_heads * head_dim][8] fp16 bits: blocks of 8
                               positions, each dimension's 8 values contiguous (position p, column c at
                               ((p / 8) * kv_dim + c) * 8 + p % 8 within its layer) */
    int32_t* status;        /* 0, or bit 0: a step ran at a position >= ctx_len (it wrote nothing to the cache);
                               bit 1: a prompt token was outside [0, vocab). Cleared by qh_decoder_prefill. */
    int32_t* history;       /* [ctx_len + 1]: the token history (the session's history_, session.cpp:13-52): the
                               prompt ids of every prefill since position 0, then each chosen id */
    int32_t* history_len;   /* its length */
    uint64_t* rng_state;    /* the sampler's xorshift64* state */
    float* kcache_f32;      /* with kv_f32 (kcache and vcache NULL then): [n_layers][ctx_len][n_kv_heads * head_dim],
                               the reference's own layout (model.cpp:96-104); NULL otherwise */
    float* vcache_f32;      /* the same for V */
} qh_decoder_state;

/* Creates a decoder over device tensors, in this order (reference model.cpp:14-33, 47-58):
 *   model.embed_tokens.weight ([vocab][dim], also the LM head when tied), model.norm.weight (F32 [1][dim]);
 *   per layer: input_layernorm (F32), q_proj, k_proj, v_proj, o_proj, q/k/v biases (F32, or data NULL without
 *   qkv_bias), post_attention_layernorm (F32), gate_proj, up_proj, down_proj;
 *   then quanta.head_q4 (Q4_0 [vocab][dim]) and quanta.head_err (F16 [vocab][dim/32]), or both with data NULL;
 *   optionally (n_tensors 5 + 12 n_layers) lm_head.weight ([vocab][dim]), the LM head of an untied model; data NULL
 *   there, or n_tensors 4 + 12 n_layers, means tied.
 * Every matrix (the embedding and LM head included) may be Q8_0, Q4_0, F32 or F16, each on its own, as the exporter
 * writes them (F32 / F16 ones run matvec_ref's float chain on the f32 activation, model.cpp:150-157); the LM head is
 * Q8_0 when the shortlist head tensors are given (model.cpp:49-58).
 * Allocates an fp16 KV cache (f32 with hp->kv_f32) for ctx_len positions and the work buffers. dim, ctx_len <= 8192,
 * head_dim 64 or 128, n_heads * head_dim == dim, ffn_dim % 256 == 0 with QH_FLAG_HADAMARD_DOWN. The tensors must
 * stay alive while the decoder is used.
 * Replaces: Model::load (reference model.cpp:10-106) after the .qnt file is read and uploaded. */
int qh_decoder_create(const qh_model_desc* hp, const qh_tensor* tensors, int n_tensors, qh_decoder** out);
int qh_decoder_destroy(qh_decoder* d);

/* n prompt tokens (device array) at positions [pos0, pos0 + n): every layer in 32-token chunks, then the head for
 * the last token (top_k > 0: shortlist head with n_valid = vocab; 0: full 8-bit head). The next position becomes
 * pos0 + n. Replaces: Model::forward_batch (reference model.cpp:349-433). */
int qh_decoder_prefill(qh_decoder* d, const int32_t* tokens, int n, int pos0, int top_k, void* stream);

/* Starts a greedy generation: the last head call's greedy token becomes the first output (out_dev[0]) and the next
 * input, as Session::generate samples its first token from the prompt's logits (reference session.cpp:33-52). */
int qh_decoder_begin(qh_decoder* d, int top_k, int32_t* out_dev, int out_cap, void* stream);

/* One greedy decode step entirely on the device: forward of the current token at the current position, head,
 * greedy token appended to the output list and made the next input, position + 1. The launch sequence does not
 * depend on host state, so it can be captured in a HIP graph once and replayed for every step.
 * Replaces: one iteration of Session::generate with the greedy sampler (reference session.cpp:39-49, model.cpp:165-228,
 * sampler.cpp:35-37). */
int qh_decoder_step(qh_decoder* d, int top_k, void* stream);

int qh_decoder_views(qh_decoder* d, qh_decoder_state* v);

/* The prefill stack: how many prompt tokens later qh_decoder_prefill calls take through each layer's norms and
 * matmuls at once. 32 (the default) is the reference's chunk (Model::kBatch, model.h:52; forward_batch,
 * model.cpp:349-361); a multiple of 32 up to 1024 runs the same arithmetic on larger batches (the matmul tile kernels
 * at M up to `stack`), attention still in 32-token sub-chunks in order, so every hidden state, cache row and logit is
 * bit-identical to the 32-token chunks. Reallocates the decoder's work buffers: it synchronises the device, the
 * pointers qh_decoder_views gave (xq / xd) change and their contents are lost, and a step captured in a HIP graph
 * before the call must be captured again. On failure the previous stack stays.
 * Replaces: nothing (the reference's chunk is a compile-time constant); a scheduling choice of the GPU path. */
int qh_decoder_set_prefill_stack(qh_decoder* d, int stack);

/* Stages of a decode step, as qh_decoder_step_timed names them: per layer l, id l * QH_STAGES_PER_LAYER + one of
 * QH_STAGE_QKV (rmsnorm + q/k/v projections), QH_STAGE_ATTENTION, QH_STAGE_O (o projection + residual),
 * QH_STAGE_GATE_UP (rmsnorm + gate/up projections + SwiGLU), QH_STAGE_DOWN (down projection + residual); then
 * QH_STAGE_FINAL_NORM, QH_STAGE_HEAD and, when a sampler picks the token, QH_STAGE_PICK. With the fused kernels (the
 * default) each per-layer stage is one kernel. */
enum {
    QH_STAGE_QKV = 0,
    QH_STAGE_ATTENTION = 1,
    QH_STAGE_O = 2,
    QH_STAGE_GATE_UP = 3,
    QH_STAGE_DOWN = 4,
    QH_STAGES_PER_LAYER = 8,
    QH_STAGE_FINAL_NORM = 1 << 20,
    QH_STAGE_HEAD = (1 << 20) + 1,
    QH_STAGE_PICK = (1 << 20) + 2
};

/* One qh_decoder_step with every kernel it launches timed on the device by the dispatch's own start and stop
 * timestamps (no extra packets between the kernels): for the i-th kernel, us_host[i] microseconds and stage_host[i]
 * its stage id; *n_host = the number of kernels. Host arrays; synchronises the stream. When the step launches more
 * than cap kernels the result is QH_ERR_NOMEM with *n_host set to the number it launched (the capacity it needs) and
 * us_host / stage_host unset; the step itself has run all the same (the decoder has advanced one token), so a caller
 * that retries with a larger cap takes the next step.
 * No counterpart in the reference (its CLI times whole tokens); for profiling. */
int qh_decoder_step_timed(qh_decoder* d, int top_k, void* stream, float* us_host, int32_t* stage_host, int cap,
                          int32_t* n_host);

/* The head queries of later prefill / begin / step calls, as Session::head_query builds them from the session's
 * sampler parameters (session.cpp:63-79): top_k = (temperature <= 0 ? 1 : p->top_k), the full head when that is 0,
 * and, when p->repeat_penalty != 1, the last p->repeat_window ids of the token history (all when 0) as must ids. The
 * calls' own top_k argument is then ignored. NULL restores plain queries (the calls' top_k, no must ids). With the
 * shortlist head tensors, top_k is at most QH_HEAD_MAX_TOPK (QH_ERR_UNSUPPORTED above).
 * Replaces: Session::set_sampler and Session::head_query (reference session.h, session.cpp:63-79). */
int qh_decoder_set_query(qh_decoder* d, const qh_sampler_params* p);

/* The token qh_decoder_begin and qh_decoder_step choose: NULL (the default) takes the head's greedy top-1; with p,
 * one qh_sample draw over the head's logits (its row list when the shortlist ran) with the token history, from the
 * generator state `seed | 1` (seed nonzero). The state lives on the device and advances with each draw, so a captured
 * step keeps sampling on replay.
 * Replaces: the Sampler that Session::generate calls (reference sampler.cpp:10-85, session.cpp:32-52). */
int qh_decoder_set_sampler(qh_decoder* d, const qh_sampler_params* p, uint64_t seed);

#ifdef __cplusplus
}
#endif

#endif /* QUANTA_HIP_H */
