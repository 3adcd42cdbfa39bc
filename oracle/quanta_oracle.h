/*
 * Oracle: a plain-C restatement of the reference's quantized matmul path.
 *
 * TEST INFRASTRUCTURE ONLY. This code is the checker, never the product: only tests/,
 * __graft_entry__.smoke() and bench.py's CPU-baseline leg may link or call it. The HIP
 * library never falls back to it.
 *
 * Every function follows one reference function (cited as file:line, relative to the
 * reference repository). Float association is kept explicit (fmaf where the reference
 * build contracts a multiply-add), and the file is compiled with -ffp-contract=off so the
 * compiler cannot fuse anything else.
 *
 * Layouts (reference engine/src/model_file.h:16-38, scripts/export.py:10-13):
 *   Q8_0 tensor [rows][cols]: int8 quants [rows*cols], then fp16 scales [rows*cols/32]
 *   Q4_0 tensor [rows][cols]: packed nibbles [rows*cols/2], then fp16 scales [rows*cols/32];
 *        per 32-block, byte j = (q[j]+8) | (q[j+16]+8) << 4, value = nibble - 8.
 *   Quantized activation ("QuantVec", ops.h:47-51): int8 q[n], f32 d[n/32].
 */
#ifndef QUANTA_ORACLE_H
#define QUANTA_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { QO_F32 = 0, QO_F16 = 1, QO_Q8_0 = 2, QO_Q4_0 = 3 };
enum { QO_QK = 32 };

/* IEEE binary16 -> binary32, exact (ops.h:15-40). */
float qo_fp16_to_f32(uint16_t h);

/* Bytes of the quant section of a tensor (model_file.cpp:29-38). */
uint64_t qo_quant_bytes(int dtype, int rows, int cols);

/* Per-32-block int8 quantization of an activation vector (ops_ref.cpp:69-83). */
void qo_quantize_q8(const float* x, int n, int8_t* q, float* d);

/* Integer-dot matvec over rows [r0, r1) (ops_ref.cpp:85-120). data points at the quants;
 * the fp16 scales follow at data + qo_quant_bytes(). out is indexed by absolute row. */
void qo_matvec_q(float* out, int dtype, int rows, int cols, const uint8_t* data, const int8_t* xq,
                 const float* xd, int r0, int r1);

/* Matvec over F32 / F16 weights with an f32 activation (matvec_ref, ops_ref.cpp:8-27; Model::linear's path for an
 * unquantized W, model.cpp:154-156), rows [r0, r1). data points at the row-major weights. */
void qo_matvec_f(float* out, int dtype, int rows, int cols, const void* data, const float* x, int r0, int r1);

/* Row `row` of a [rows][cols] tensor of any dtype as f32 (get_row, ops_ref.cpp:162-192). */
void qo_get_row(float* out, int dtype, int rows, int cols, const void* data, int row);

/* Multi-token matmul (ops_ref.cpp:122-160, contract ops.h:65-70): out[t*ldo + r] for tokens
 * t in [0, n) and rows r in [r0, r1). xq is [n][cols] int8, xd is [n][cols/32]. Every
 * (row, token) value is bit-identical to qo_matvec_q on that token. */
void qo_matmul_q(float* out, int ldo, int dtype, int rows, int cols, const uint8_t* data,
                 const int8_t* xq, const float* xd, int n, int r0, int r1);

/* Exact Shortlist Head (model.cpp:240-334) for one quantized hidden state.
 *   head8: Q8_0 [V][D] (the exact head), head4: Q4_0 [V][D], err: f16 [V][D/32].
 *   top_k > 0, n_valid (0 = all rows), must[n_must] ids that must come back exact.
 * Outputs (caller-allocated):
 *   logits[V]: exact value for every row that was rescored, -inf elsewhere;
 *   coarse[V], upper[V]: 4-bit score and its upper bound for every row;
 *   rows[V]: rescored rows, seeds first (by coarse score descending, lower row first on ties),
 *            then candidates in ascending row order, then must ids in query order.
 * Returns the number of rescored rows (the reference's last_head_rows). *n_seeds receives the
 * seed count, *tau the cut-off, *seed_tie 1 when the n_seed-th and next-best eligible coarse
 * scores are equal (the reference's per-thread heaps may then pick a different seed). */
int qo_shortlist_head(const uint8_t* head8, const uint8_t* head4, const uint16_t* err, int V, int D,
                      const int8_t* xq, const float* xd, int top_k, int n_valid, const int* must, int n_must,
                      float* logits, float* coarse, float* upper, int* rows, int* n_seeds, float* tau,
                      int* seed_tie);

/* Nibble planes of a Q8_0 [V][D] head (the scope's nibble-plane shortlist variant, research/head_deep.py:68-78,
 * docs/PROGRESS.md:121-130): each int8 q = 16 h + l with h = floor(q / 16) in [-8, 7], l in [0, 15]. planes receives
 * V*D + V*D/16 bytes, the size of the Q8_0 tensor: the high plane [V][D/2] (Q4_0 packing of the codes h + 8), the low
 * plane [V][D/2] (Q4_0 packing of l) and the Q8_0 scales [V][D/32] unchanged. */
void qo_head_planes(const uint8_t* head8, int V, int D, uint8_t* planes);

/* qo_shortlist_head over the nibble planes alone: the screen reads the high plane and the scales (coarse = the chain
 * of float(sum_i (16 h_i + 8) x_i) * d_b, bound = sum_b fma(d_b, (8 dx_b) * sum_i |x_i|), then the same slack,
 * seeds, tau, candidates and must ids), exact rows are the Q8_0 rows rebuilt from both planes. Same outputs. */
int qo_shortlist_planes(const uint8_t* planes, int V, int D, const int8_t* xq, const float* xd, int top_k,
                        int n_valid, const int* must, int n_must, float* logits, float* coarse, float* upper,
                        int* rows, int* n_seeds, float* tau, int* seed_tie);

/* Greedy token: first index of the maximum over logits[0, n) (sampler.cpp:35-37). */
int qo_argmax(const float* logits, int n);

/* Row-parallel drivers for the CPU baseline: rows split in chunks that are multiples of 16 over
 * n_threads pthreads, as ThreadPool::parallel_for(rows, 16, ...) does (threadpool.h:28-40). */
void qo_matvec_q_mt(float* out, int dtype, int rows, int cols, const uint8_t* data, const int8_t* xq,
                    const float* xd, int n_threads);
void qo_matmul_q_mt(float* out, int ldo, int dtype, int rows, int cols, const uint8_t* data,
                    const int8_t* xq, const float* xd, int n, int n_threads);

/* ------------------------------------------------------------------ decoder (model.cpp:10-228, 349-433) */

/* IEEE binary32 -> binary16, round to nearest even (the _Float16 conversion of the reference's KV store,
 * model.cpp:140-143), as bits. */
uint16_t qo_f32_to_f16(float f);

/* glibc-identical expf is the host's own: the oracle calls expf() from libm, as the reference does. */

typedef struct qo_decoder qo_decoder;

/* hp: vocab, dim, n_layers, n_heads, n_kv_heads, head_dim, ffn_dim, ctx_len, qkv_bias, flags (model_file.h:21:
 * bit 0 FLAG_HADAMARD_DOWN), kv_f32 (1: an f32 KV cache, Model::load with kv_f16 false), untied (1: an lm_head.weight
 * tensor, model.cpp:16) (12 ints); hpf: rope_theta, norm_eps. tensors / dtypes: embed (Q8_0 [V][D]), final norm
 * (F32 [D]); per layer attn_norm, wq, wk, wv, wo, bq, bk, bv, ffn_norm, w_gate, w_up, w_down (12 each; biases NULL
 * without qkv_bias, weights Q8_0 or Q4_0); then the shortlist copy head_q4 (Q4_0 [V][D]) and head_err
 * (F16 [V][D/32]), or NULL; then, when untied, lm_head (Q8_0 or Q4_0 [V][D]; Q8_0 with the shortlist copy), the LM
 * head in place of the embedding. Returns NULL on a bad argument (also the Hadamard flag with ffn_dim % 256 != 0,
 * model.cpp:39-42). */
qo_decoder* qo_decoder_create(const int* hp, const float* hpf, const void* const* tensors, const int* dtypes);
void qo_decoder_free(qo_decoder* d);

/* The must ids of the head queries of later forward calls (HeadQuery::must, model.h:24-29; Session::head_query,
 * session.cpp:63-79), NULL / 0 for none. The array stays caller-owned and must outlive those calls. */
void qo_decoder_set_must(qo_decoder* d, const int* must, int n_must);

/* Model::forward (model.cpp:165-228): one token at position pos; top_k > 0 runs the shortlist head with
 * n_valid = vocab, else the full head. logits [V], hidden [D] (the final normed state), hq / hd its quantization
 * (each may be NULL). Returns the 8-bit head rows read. */
int qo_decoder_forward(qo_decoder* d, int token, int pos, int top_k, float* logits, float* hidden, int8_t* hq,
                       float* hd);

/* Model::forward_batch (model.cpp:349-361) for n tokens from pos0: every token's layers (token t attends over
 * positions <= pos0 + t, which is what the 32-token chunks compute), then the head for the last token. */
int qo_decoder_forward_batch(qo_decoder* d, const int* tokens, int n, int pos0, int top_k, float* logits,
                             float* hidden, int8_t* hq, float* hd);

/* Copies the KV cache of layer l, positions [0, n_pos): k and v as [n_pos][n_kv_heads * head_dim] f16 bits, or f32
 * values with kv_f32. */
void qo_decoder_kv(const qo_decoder* d, int l, int n_pos, void* k, void* v);

/* RoPE table of the reference (ops_ref.cpp:201-214) for positions [0, n_pos): cs[pos][i] = (cosf, sinf) of
 * pos * powf(theta, -2 i / head_dim), i < head_dim / 2, as [n_pos][head_dim / 2][2] floats. */
void qo_rope_table(float* cs, int n_pos, int head_dim, float theta);

/* ------------------------------------------------------------------ sampler (sampler.cpp:10-85, sampler.h) */

/* SamplerParams (sampler.h) without the seed. */
typedef struct {
    float temperature;    /* <= 0: greedy */
    int top_k;            /* 0 = disabled */
    float top_p;          /* 1 = disabled */
    float min_p;          /* 0 = disabled */
    float repeat_penalty; /* 1 = disabled; divides positive logits, multiplies negative ones */
    int repeat_window;    /* 0 = the whole history */
} qo_sampler_params;

/* The generator state Sampler's constructor makes from a nonzero seed (sampler.cpp:10-13). */
uint64_t qo_sampler_seed(uint64_t seed);

/* Sampler::sample (sampler.cpp:22-85): repetition penalty over the distinct ids of the history window (logits
 * modified in place), then greedy (first maximum) or top-k, softmax with temperature, min-p, top-p and a draw from
 * the xorshift64* generator whose state is *state (advanced by one draw). Candidates with equal logits are ordered by
 * lower id (the reference's std::sort leaves their order unspecified). */
int qo_sample(float* logits, int n_valid, const int* history, int n_hist, const qo_sampler_params* p,
              uint64_t* state);

#ifdef __cplusplus
}
#endif

#endif
