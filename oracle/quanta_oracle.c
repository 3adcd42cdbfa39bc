/*
 * Oracle: plain-C restatement of the reference's quantized matmul path.
 * TEST INFRASTRUCTURE ONLY (see quanta_oracle.h): the checker and the CPU baseline, never the
 * product. Build with -ffp-contract=off; every fused multiply-add below is an explicit fmaf that
 * mirrors the contraction the reference build performs (clang -O3 with FMA: `acc += a * b`
 * becomes one fused multiply-add, `float(s) * dw * dx` keeps its first product rounded).
 */
#include "quanta_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

float qo_fp16_to_f32(uint16_t h) {
    /* ops.h:15-40. Normal numbers re-bias the exponent; subnormals are m * 2^-24, which is exact
     * in binary32; exponent 31 keeps the payload (inf / NaN). */
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 31u, m = h & 1023u;
    uint32_t bits;
    if (e == 31u) {
        bits = sign | 0x7f800000u | (m << 13);
    } else if (e != 0u) {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    } else {
        const float f = (float)m * 0x1p-24f;
        return sign ? -f : f;
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint64_t qo_quant_bytes(int dtype, int rows, int cols) {
    /* model_file.cpp:29-38 */
    const uint64_t n = (uint64_t)rows * (uint64_t)cols;
    switch (dtype) {
        case QO_F32: return n * 4u;
        case QO_F16: return n * 2u;
        case QO_Q8_0: return n;
        case QO_Q4_0: return n / 2u;
        default: return 0;
    }
}

void qo_quantize_q8(const float* x, int n, int8_t* q, float* d) {
    /* ops_ref.cpp:69-83: amax per 32-block, d = amax/127, q = round-half-away(x * (1/d)). */
    for (int b = 0; b < n / QO_QK; ++b) {
        const float* xb = x + (size_t)b * QO_QK;
        float amax = 0.f;
        for (int i = 0; i < QO_QK; ++i) {
            const float a = fabsf(xb[i]);
            if (a > amax) amax = a;
        }
        const float scale = amax / 127.f;
        const float inv = scale > 0.f ? 1.f / scale : 0.f;
        for (int i = 0; i < QO_QK; ++i) q[(size_t)b * QO_QK + i] = (int8_t)lroundf(xb[i] * inv);
        d[b] = scale;
    }
}

/* Integer dot of one 32-block of weights against one 32-block of the activation. */
static inline int32_t block_dot_q8(const int8_t* w, const int8_t* x) {
    int32_t s = 0;
    for (int i = 0; i < QO_QK; ++i) s += (int32_t)w[i] * (int32_t)x[i];
    return s;
}

static inline int32_t block_dot_q4(const uint8_t* w, const int8_t* x) {
    /* ops_ref.cpp:111-114: low nibble of byte j is element j, high nibble is element j+16. */
    int32_t s = 0;
    for (int j = 0; j < QO_QK / 2; ++j) {
        s += ((int32_t)(w[j] & 15u) - 8) * (int32_t)x[j];
        s += ((int32_t)(w[j] >> 4) - 8) * (int32_t)x[j + QO_QK / 2];
    }
    return s;
}

/* One output value: the serial per-block chain acc = fma(float(s_b) * dw_b, dx_b, acc) in block
 * order (ops_ref.cpp:95-99 / 107-116 as compiled with FMA contraction). */
static float row_dot(int dtype, int cols, const uint8_t* data, const uint16_t* scales, int r, const int8_t* xq,
                     const float* xd) {
    const int nb = cols / QO_QK;
    const uint16_t* dr = scales + (size_t)r * nb;
    float acc = 0.f;
    if (dtype == QO_Q8_0) {
        const int8_t* wr = (const int8_t*)data + (size_t)r * cols;
        for (int b = 0; b < nb; ++b) {
            const int32_t s = block_dot_q8(wr + (size_t)b * QO_QK, xq + (size_t)b * QO_QK);
            const float p = (float)s * qo_fp16_to_f32(dr[b]);
            acc = fmaf(p, xd[b], acc);
        }
    } else {
        const uint8_t* wr = data + (size_t)r * cols / 2;
        for (int b = 0; b < nb; ++b) {
            const int32_t s = block_dot_q4(wr + (size_t)b * QO_QK / 2, xq + (size_t)b * QO_QK);
            const float p = (float)s * qo_fp16_to_f32(dr[b]);
            acc = fmaf(p, xd[b], acc);
        }
    }
    return acc;
}

void qo_matvec_q(float* out, int dtype, int rows, int cols, const uint8_t* data, const int8_t* xq,
                 const float* xd, int r0, int r1) {
    const uint16_t* scales = (const uint16_t*)(data + qo_quant_bytes(dtype, rows, cols));
    for (int r = r0; r < r1; ++r) out[r] = row_dot(dtype, cols, data, scales, r, xq, xd);
}

/* ops_ref.cpp:8-27: acc += w_i * x_i from +0 in column order; the reference build contracts each step into one
 * multiply-add (-march with FMA, GCC's default contraction); an F16 weight is converted exactly first. */
void qo_matvec_f(float* out, int dtype, int rows, int cols, const void* data, const float* x, int r0, int r1) {
    (void)rows;
    for (int r = r0; r < r1; ++r) {
        float acc = 0.f;
        if (dtype == QO_F32) {
            const float* w = (const float*)data + (size_t)r * cols;
            for (int i = 0; i < cols; ++i) acc = fmaf(w[i], x[i], acc);
        } else {
            const uint16_t* w = (const uint16_t*)data + (size_t)r * cols;
            for (int i = 0; i < cols; ++i) acc = fmaf(qo_fp16_to_f32(w[i]), x[i], acc);
        }
        out[r] = acc;
    }
}

/* ops_ref.cpp:162-192; the products q * d are exact in f32 (at most 8 + 11 significant bits) */
void qo_get_row(float* out, int dtype, int rows, int cols, const void* data, int row) {
    const int nb = cols / QO_QK;
    if (dtype == QO_F32) {
        memcpy(out, (const float*)data + (size_t)row * cols, sizeof(float) * (size_t)cols);
    } else if (dtype == QO_F16) {
        const uint16_t* w = (const uint16_t*)data + (size_t)row * cols;
        for (int i = 0; i < cols; ++i) out[i] = qo_fp16_to_f32(w[i]);
    } else if (dtype == QO_Q8_0) {
        const int8_t* q = (const int8_t*)data + (size_t)row * cols;
        const uint16_t* d = (const uint16_t*)((const uint8_t*)data + (size_t)rows * cols) + (size_t)row * nb;
        for (int i = 0; i < cols; ++i) out[i] = (float)q[i] * qo_fp16_to_f32(d[i / QO_QK]);
    } else {
        const uint8_t* q = (const uint8_t*)data + (size_t)row * cols / 2;
        const uint16_t* d = (const uint16_t*)((const uint8_t*)data + (size_t)rows * cols / 2) + (size_t)row * nb;
        for (int b = 0; b < nb; ++b) {
            const float s = qo_fp16_to_f32(d[b]);
            for (int j = 0; j < QO_QK / 2; ++j) {
                out[b * QO_QK + j] = (float)((int)(q[b * QO_QK / 2 + j] & 0xF) - 8) * s;
                out[b * QO_QK + j + QO_QK / 2] = (float)((int)(q[b * QO_QK / 2 + j] >> 4) - 8) * s;
            }
        }
    }
}

void qo_matmul_q(float* out, int ldo, int dtype, int rows, int cols, const uint8_t* data,
                 const int8_t* xq, const float* xd, int n, int r0, int r1) {
    const uint16_t* scales = (const uint16_t*)(data + qo_quant_bytes(dtype, rows, cols));
    const int nb = cols / QO_QK;
    for (int r = r0; r < r1; ++r)
        for (int t = 0; t < n; ++t)
            out[(size_t)t * ldo + r] =
                row_dot(dtype, cols, data, scales, r, xq + (size_t)t * cols, xd + (size_t)t * nb);
}

int qo_argmax(const float* logits, int n) {
    /* sampler.cpp:35-37: std::max_element keeps the first of equal maxima. */
    int best = 0;
    for (int i = 1; i < n; ++i)
        if (logits[i] > logits[best]) best = i;
    return best;
}

/* ---------------------------------------------------------------- shortlist head */

typedef struct {
    float score;
    int row;
} scored_t;

/* Higher score first; lower row first among equal scores. */
static int better(float sa, int ra, float sb, int rb) { return sa > sb || (sa == sb && ra < rb); }

/* Where one head call reads its rows: the Q8_0 head with its Q4_0 copy and f16 block errors (the engine's layout,
 * model.cpp:47-58), or the Q8_0 head alone as nibble planes (qo_head_planes). */
typedef struct {
    int planes;
    const uint8_t* head8;
    const uint16_t* s8;
    const uint8_t* head4;
    const uint16_t* s4;
    const uint16_t* err;
    const uint8_t* hi; /* planes: high nibbles [V][D/2], low nibbles [V][D/2], scales [V][D/32] */
    const uint8_t* lo;
    const uint16_t* ps;
} head_src;

/* One 32-block of the head rebuilt from the nibble planes: q = 16 * h + l, h = (high nibble) - 8, l = low nibble. */
static void planes_block(const head_src* h, int D, int r, int b, int8_t* q) {
    const size_t off = ((size_t)r * (D / QO_QK) + b) * (QO_QK / 2);
    for (int j = 0; j < QO_QK / 2; ++j) {
        const uint8_t hb = h->hi[off + j], lb = h->lo[off + j];
        q[j] = (int8_t)(16 * ((int)(hb & 15u) - 8) + (int)(lb & 15u));
        q[j + QO_QK / 2] = (int8_t)(16 * ((int)(hb >> 4) - 8) + (int)(lb >> 4));
    }
}

/* Exact logit of row r: the Q8_0 chain of row_dot (from the planes, over the rebuilt int8 values). */
static float head_exact(const head_src* h, int D, int r, const int8_t* xq, const float* xd) {
    if (!h->planes) return row_dot(QO_Q8_0, D, h->head8, h->s8, r, xq, xd);
    const int nb = D / QO_QK;
    float acc = 0.f;
    for (int b = 0; b < nb; ++b) {
        int8_t q[QO_QK];
        planes_block(h, D, r, b, q);
        const int32_t s = block_dot_q8(q, xq + (size_t)b * QO_QK);
        const float p = (float)s * qo_fp16_to_f32(h->ps[(size_t)r * nb + b]);
        acc = fmaf(p, xd[b], acc);
    }
    return acc;
}

/* Screen of row r: the coarse score and its bound (before the slack).
 *   engine layout (model.cpp:263-271): coarse = the Q4_0 copy's chain, bound = sum_b fma(err_b, xnorm_b);
 *   planes (research/head_deep.py:68-78, restated over the int8 activation): coarse = the chain of
 *     float(sum_i (16 h_i + 8) x_i) * d_b, i.e. every value at the midpoint of its 16-wide high-nibble bucket, and
 *     bound = sum_b fma(d_b, bop_b) with bop_b = (8 * dx_b) * sum_i |x_i|: |q - (16 h + 8)| = |l - 8| <= 8. */
static float head_screen(const head_src* h, int D, int r, const int8_t* xq, const float* xd, const float* bop,
                         float* bound_out) {
    const int nb = D / QO_QK;
    float bound = 0.f, c = 0.f;
    if (!h->planes) {
        c = row_dot(QO_Q4_0, D, h->head4, h->s4, r, xq, xd);
        const uint16_t* e = h->err + (size_t)r * nb;
        for (int b = 0; b < nb; ++b) bound = fmaf(qo_fp16_to_f32(e[b]), bop[b], bound);
    } else {
        for (int b = 0; b < nb; ++b) {
            /* the high plane only: h = nibble - 8 */
            const uint8_t* hb = h->hi + ((size_t)r * nb + b) * (QO_QK / 2);
            const int8_t* xb = xq + (size_t)b * QO_QK;
            int32_t s = 0;
            for (int j = 0; j < QO_QK / 2; ++j) {
                s += (16 * ((int)(hb[j] & 15u) - 8) + 8) * (int32_t)xb[j];
                s += (16 * ((int)(hb[j] >> 4) - 8) + 8) * (int32_t)xb[j + QO_QK / 2];
            }
            const float d = qo_fp16_to_f32(h->ps[(size_t)r * nb + b]);
            c = fmaf((float)s * d, xd[b], c);
            bound = fmaf(d, bop[b], bound);
        }
    }
    *bound_out = bound;
    return c;
}

static int shortlist_core(const head_src* h, int V, int D, const int8_t* xq, const float* xd, int top_k, int n_valid,
                          const int* must, int n_must, float* logits, float* coarse, float* upper, int* rows,
                          int* n_seeds_out, float* tau_out, int* seed_tie) {
    const int nb = D / QO_QK;
    const int nv = (n_valid > 0 && n_valid < V) ? n_valid : V; /* model.cpp:245 */
    const int k = top_k;
    const int n_seed = k + 8; /* model.cpp:256 */

    /* The bound's per-block operands. Engine layout (model.cpp:247-251): xnorm_b = d_b * sqrt(sum q^2) (an exact
     * integer sum below 2^24). Planes: (8 * d_b) * sum |q| (an exact integer below 2^24). */
    float* bop = (float*)malloc(sizeof(float) * (size_t)nb);
    for (int b = 0; b < nb; ++b) {
        float ss = 0.f;
        int l1 = 0;
        for (int i = 0; i < QO_QK; ++i) {
            const float v = (float)xq[b * QO_QK + i];
            ss = fmaf(v, v, ss);
            l1 += abs((int)xq[b * QO_QK + i]);
        }
        bop[b] = h->planes ? (8.f * xd[b]) * (float)l1 : xd[b] * sqrtf(ss);
    }

    /* mark: 1 = must id (kept out of seeds and candidates), 2 = seed (already exact). */
    uint8_t* mark = (uint8_t*)calloc((size_t)V, 1);
    for (int i = 0; i < n_must; ++i)
        if (must[i] >= 0 && must[i] < nv) mark[must[i]] = 1; /* model.cpp:252-253 */

    /* Screen (model.cpp:259-284): coarse score, bound, upper; logits start at -inf. The seed list
     * keeps the n_seed best eligible coarse scores, sorted best-first. */
    scored_t* seeds = (scored_t*)malloc(sizeof(scored_t) * (size_t)(n_seed + 1));
    int ns = 0;
    for (int r = 0; r < V; ++r) {
        float bound;
        const float c = head_screen(h, D, r, xq, xd, bop, &bound);
        bound = fmaf(bound, 1.001f, 1e-5f); /* model.cpp:271 */
        coarse[r] = c;
        upper[r] = c + bound;
        logits[r] = -INFINITY;
        if (r >= nv || mark[r]) continue;
        /* insertion into the sorted list; rows arrive in ascending order, so an equal score never
         * displaces an earlier row */
        int pos = ns;
        while (pos > 0 && better(c, r, seeds[pos - 1].score, seeds[pos - 1].row)) --pos;
        if (pos < n_seed) {
            const int last = ns < n_seed ? ns : n_seed - 1;
            for (int i = last; i > pos; --i) seeds[i] = seeds[i - 1];
            seeds[pos].score = c;
            seeds[pos].row = r;
            if (ns < n_seed) ++ns;
        }
    }

    /* Tie flag: is some eligible row outside the seed list equal in coarse score to the last seed? */
    int tie = 0;
    if (ns == n_seed) {
        const float cut = seeds[ns - 1].score;
        for (int r = 0; r < nv && !tie; ++r) {
            if (mark[r] || coarse[r] != cut) continue;
            int in = 0;
            for (int i = 0; i < ns; ++i) in |= seeds[i].row == r;
            tie = !in;
        }
    }

    /* Seeds are rescored exactly; tau is the k-th best exact seed logit (model.cpp:302-313). */
    int n_rows = 0;
    for (int i = 0; i < ns; ++i) {
        const int r = seeds[i].row;
        rows[n_rows++] = r;
        mark[r] = 2;
        logits[r] = head_exact(h, D, r, xq, xd);
    }
    float tau = -INFINITY;
    if (ns >= k) {
        /* k-th largest of the exact seed logits */
        float* ex = (float*)malloc(sizeof(float) * (size_t)ns);
        for (int i = 0; i < ns; ++i) ex[i] = logits[seeds[i].row];
        for (int i = 0; i < k; ++i) {
            int m = i;
            for (int j = i + 1; j < ns; ++j)
                if (ex[j] > ex[m]) m = j;
            const float t = ex[i];
            ex[i] = ex[m];
            ex[m] = t;
        }
        tau = ex[k - 1];
        free(ex);
    }

    /* Candidates (model.cpp:315-321): unmarked valid rows whose upper bound reaches tau. */
    for (int r = 0; r < nv; ++r)
        if (!mark[r] && upper[r] >= tau) {
            rows[n_rows++] = r;
            logits[r] = head_exact(h, D, r, xq, xd);
        }
    /* must ids, first occurrence only (model.cpp:324-330) */
    for (int i = 0; i < n_must; ++i) {
        const int id = must[i];
        if (id >= 0 && id < nv && mark[id] == 1) {
            rows[n_rows++] = id;
            mark[id] = 0;
            logits[id] = head_exact(h, D, id, xq, xd);
        }
    }

    if (n_seeds_out) *n_seeds_out = ns;
    if (tau_out) *tau_out = tau;
    if (seed_tie) *seed_tie = tie;
    free(seeds);
    free(mark);
    free(bop);
    return n_rows;
}

int qo_shortlist_head(const uint8_t* head8, const uint8_t* head4, const uint16_t* err, int V, int D,
                      const int8_t* xq, const float* xd, int top_k, int n_valid, const int* must, int n_must,
                      float* logits, float* coarse, float* upper, int* rows, int* n_seeds_out, float* tau_out,
                      int* seed_tie) {
    head_src h;
    memset(&h, 0, sizeof(h));
    h.head8 = head8;
    h.s8 = (const uint16_t*)(head8 + qo_quant_bytes(QO_Q8_0, V, D));
    h.head4 = head4;
    h.s4 = (const uint16_t*)(head4 + qo_quant_bytes(QO_Q4_0, V, D));
    h.err = err;
    return shortlist_core(&h, V, D, xq, xd, top_k, n_valid, must, n_must, logits, coarse, upper, rows, n_seeds_out,
                          tau_out, seed_tie);
}

void qo_head_planes(const uint8_t* head8, int V, int D, uint8_t* planes) {
    /* q = 16 * h + l with h = floor(q / 16) in [-8, 7] and l = q - 16 h in [0, 15] (research/head_deep.py:72-73:
     * h4 = floor(q / 16)); each plane packed as Q4_0 blocks (byte j: element j low, element j + 16 high), the high
     * plane's nibble h + 8 as a Q4_0 code. The scales follow unchanged. */
    const size_t n = (size_t)V * (size_t)D;
    const int8_t* q = (const int8_t*)head8;
    uint8_t* hi = planes;
    uint8_t* lo = planes + n / 2;
    for (size_t blk = 0; blk < n / QO_QK; ++blk) {
        const int8_t* qb = q + blk * QO_QK;
        for (int j = 0; j < QO_QK / 2; ++j) {
            const int a = qb[j], c = qb[j + QO_QK / 2];
            const int ha = (int)floor(a / 16.0), hc = (int)floor(c / 16.0);
            hi[blk * (QO_QK / 2) + j] = (uint8_t)((ha + 8) | ((hc + 8) << 4));
            lo[blk * (QO_QK / 2) + j] = (uint8_t)((a - 16 * ha) | ((c - 16 * hc) << 4));
        }
    }
    memcpy(planes + n, head8 + n, n / QO_QK * 2);
}

int qo_shortlist_planes(const uint8_t* planes, int V, int D, const int8_t* xq, const float* xd, int top_k,
                        int n_valid, const int* must, int n_must, float* logits, float* coarse, float* upper,
                        int* rows, int* n_seeds_out, float* tau_out, int* seed_tie) {
    const size_t n = (size_t)V * (size_t)D;
    head_src h;
    memset(&h, 0, sizeof(h));
    h.planes = 1;
    h.hi = planes;
    h.lo = planes + n / 2;
    h.ps = (const uint16_t*)(planes + n);
    return shortlist_core(&h, V, D, xq, xd, top_k, n_valid, must, n_must, logits, coarse, upper, rows, n_seeds_out,
                          tau_out, seed_tie);
}

/* ---------------------------------------------------------------- threaded CPU baseline */

typedef struct {
    int mm; /* 0 = matvec, 1 = matmul */
    float* out;
    int ldo, dtype, rows, cols, n;
    const uint8_t* data;
    const int8_t* xq;
    const float* xd;
    int r0, r1;
} job_t;

static void* run_job(void* p) {
    const job_t* j = (const job_t*)p;
    if (j->r0 < j->r1) {
        if (j->mm)
            qo_matmul_q(j->out, j->ldo, j->dtype, j->rows, j->cols, j->data, j->xq, j->xd, j->n, j->r0, j->r1);
        else
            qo_matvec_q(j->out, j->dtype, j->rows, j->cols, j->data, j->xq, j->xd, j->r0, j->r1);
    }
    return NULL;
}

static void run_parallel(job_t proto, int n_threads) {
    /* threadpool.h:28-40: rows in chunks of 16, chunk range [chunks*t/nt, chunks*(t+1)/nt). */
    if (n_threads < 1) n_threads = 1;
    const int grain = 16;
    const int chunks = (proto.rows + grain - 1) / grain;
    pthread_t th[256];
    job_t jobs[256];
    if (n_threads > 256) n_threads = 256;
    for (int t = 0; t < n_threads; ++t) {
        const int c0 = (int)((int64_t)chunks * t / n_threads), c1 = (int)((int64_t)chunks * (t + 1) / n_threads);
        jobs[t] = proto;
        jobs[t].r0 = c0 * grain;
        jobs[t].r1 = c1 * grain < proto.rows ? c1 * grain : proto.rows;
    }
    for (int t = 1; t < n_threads; ++t) pthread_create(&th[t], NULL, run_job, &jobs[t]);
    run_job(&jobs[0]);
    for (int t = 1; t < n_threads; ++t) pthread_join(th[t], NULL);
}

void qo_matvec_q_mt(float* out, int dtype, int rows, int cols, const uint8_t* data, const int8_t* xq,
                    const float* xd, int n_threads) {
    job_t j = {0, out, 0, dtype, rows, cols, 1, data, xq, xd, 0, rows};
    run_parallel(j, n_threads);
}

void qo_matmul_q_mt(float* out, int ldo, int dtype, int rows, int cols, const uint8_t* data,
                    const int8_t* xq, const float* xd, int n, int n_threads) {
    job_t j = {1, out, ldo, dtype, rows, cols, n, data, xq, xd, 0, rows};
    run_parallel(j, n_threads);
}

/* ---------------------------------------------------------------- decoder (model.cpp:10-228, 349-433) */

uint16_t qo_f32_to_f16(float f) {
    /* round to nearest even: normals drop 13 mantissa bits, binary16 subnormals are round(|f| * 2^24) */
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, a = x & 0x7fffffffu;
    if (a >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (a > 0x7f800000u ? 0x200u | ((a >> 13) & 0x3ffu) : 0u));
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to infinity */
    if (a < 0x38800000u) {                                   /* below 2^-14: binary16 subnormal */
        const uint32_t e = a >> 23;
        if (e < 102u) return (uint16_t)sign; /* below 2^-25 */
        const uint32_t shift = 126u - e, m = (a & 0x7fffffu) | 0x800000u;
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return (uint16_t)(sign | q);
    }
    uint32_t h = (a - 0x38000000u) >> 13;
    const uint32_t rem = a & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
}

void qo_rope_table(float* cs, int n_pos, int head_dim, float theta) {
    /* ops_ref.cpp:203-206: freq = powf(theta, -2.0f * i / head_dim), angle = pos * freq */
    const int half = head_dim / 2;
    for (int p = 0; p < n_pos; ++p)
        for (int i = 0; i < half; ++i) {
            const float freq = powf(theta, -2.0f * (float)i / (float)head_dim);
            const float angle = (float)p * freq;
            cs[((size_t)p * half + i) * 2] = cosf(angle);
            cs[((size_t)p * half + i) * 2 + 1] = sinf(angle);
        }
}

enum { L_ATTN_NORM, L_WQ, L_WK, L_WV, L_WO, L_BQ, L_BK, L_BV, L_FFN_NORM, L_WG, L_WU, L_WD, L_COUNT };

struct qo_decoder {
    int V, D, nl, nh, nkv, hdim, F, ctx, bias;
    int flags; /* model_file.h:21 FLAG_HADAMARD_DOWN */
    int kv32;  /* f32 KV cache (Model::load kv_f16 = false, the CLI's --kv-f32) */
    int lm;    /* index of the LM head tensor: 0 (tied embedding) or 4 + 12 n_layers (lm_head.weight) */
    float theta, eps;
    const void* const* t;
    const int* dt;
    uint16_t *kc, *vc; /* [layer][ctx][kv_dim] f16 bits */
    float *kcf, *vcf;  /* [layer][ctx][kv_dim] f32, with kv32 */
    float *x, *xb, *xb2, *q, *k, *v, *att, *hb, *hb2, *logits, *coarse, *upper, *cs;
    int8_t *xq, *hq;
    float *xd, *hd;
    int* rows;
    const int* must; /* head query must ids (caller-owned), see qo_decoder_set_must */
    int n_must;
};

static const void* lt(const qo_decoder* d, int l, int which) { return d->t[2 + l * L_COUNT + which]; }
static int ldt(const qo_decoder* d, int l, int which) { return d->dt[2 + l * L_COUNT + which]; }

qo_decoder* qo_decoder_create(const int* hp, const float* hpf, const void* const* tensors, const int* dtypes) {
    qo_decoder* d = (qo_decoder*)calloc(1, sizeof(qo_decoder));
    d->V = hp[0]; d->D = hp[1]; d->nl = hp[2]; d->nh = hp[3]; d->nkv = hp[4]; d->hdim = hp[5]; d->F = hp[6];
    d->ctx = hp[7]; d->bias = hp[8]; d->flags = hp[9]; d->kv32 = hp[10];
    d->lm = hp[11] ? 4 + 12 * d->nl : 0;
    d->theta = hpf[0]; d->eps = hpf[1];
    if (d->nh * d->hdim != d->D || d->nh % d->nkv != 0 || d->D % QO_QK || d->F % QO_QK) { free(d); return NULL; }
    if ((d->flags & 1) && d->F % 256 != 0) { free(d); return NULL; } /* model.cpp:39-42 */
    d->t = tensors;
    d->dt = dtypes;
    const size_t kvd = (size_t)d->nkv * d->hdim;
    if (d->kv32) {
        d->kcf = (float*)calloc((size_t)d->nl * d->ctx * kvd, 4);
        d->vcf = (float*)calloc((size_t)d->nl * d->ctx * kvd, 4);
    } else {
        d->kc = (uint16_t*)calloc((size_t)d->nl * d->ctx * kvd, 2);
        d->vc = (uint16_t*)calloc((size_t)d->nl * d->ctx * kvd, 2);
    }
    d->x = (float*)calloc(d->D, 4); d->xb = (float*)calloc(d->D, 4); d->xb2 = (float*)calloc(d->D, 4);
    d->q = (float*)calloc(d->D, 4); d->k = (float*)calloc(kvd, 4); d->v = (float*)calloc(kvd, 4);
    d->att = (float*)calloc((size_t)d->ctx, 4);
    d->hb = (float*)calloc(d->F, 4); d->hb2 = (float*)calloc(d->F, 4);
    d->logits = (float*)calloc(d->V, 4); d->coarse = (float*)calloc(d->V, 4); d->upper = (float*)calloc(d->V, 4);
    d->rows = (int*)calloc(d->V, 4);
    d->xq = (int8_t*)calloc(d->D > d->F ? d->D : d->F, 1); d->hq = (int8_t*)calloc(d->F, 1);
    d->xd = (float*)calloc(d->D / QO_QK, 4); d->hd = (float*)calloc(d->F / QO_QK, 4);
    d->cs = (float*)malloc(sizeof(float) * (size_t)d->ctx * d->hdim);
    qo_rope_table(d->cs, d->ctx, d->hdim, d->theta);
    return d;
}

/* The KV cache rows of one layer, positions [0, n_pos): f16 bits (2 bytes each) or, with kv32, f32 (4 bytes). */
void qo_decoder_kv(const qo_decoder* d, int l, int n_pos, void* k, void* v) {
    const size_t kvd = (size_t)d->nkv * d->hdim, off = (size_t)l * d->ctx * kvd;
    if (d->kv32) {
        memcpy(k, d->kcf + off, 4 * kvd * (size_t)n_pos);
        memcpy(v, d->vcf + off, 4 * kvd * (size_t)n_pos);
    } else {
        memcpy(k, d->kc + off, 2 * kvd * (size_t)n_pos);
        memcpy(v, d->vc + off, 2 * kvd * (size_t)n_pos);
    }
}

void qo_decoder_free(qo_decoder* d) {
    if (!d) return;
    free(d->kc); free(d->vc); free(d->kcf); free(d->vcf); free(d->x); free(d->xb); free(d->xb2); free(d->q); free(d->k); free(d->v);
    free(d->att); free(d->hb); free(d->hb2); free(d->logits); free(d->coarse); free(d->upper); free(d->rows);
    free(d->xq); free(d->hq); free(d->xd); free(d->hd); free(d->cs); free(d);
}

/* ops_ref.cpp:194-199 */
static void rmsnorm(float* out, const float* x, const float* w, int n, float eps) {
    float ss = 0.f;
    for (int i = 0; i < n; ++i) ss = fmaf(x[i], x[i], ss);
    const float scale = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = 0; i < n; ++i) out[i] = x[i] * scale * w[i];
}

/* ops_ref.cpp:201-214 with the angle table: a*c - b*s and b*c + a*s, each contracted into one multiply-add */
static void rope(float* v, int n_heads, int hd, const float* cs) {
    const int half = hd / 2;
    for (int i = 0; i < half; ++i) {
        const float c = cs[2 * i], s = cs[2 * i + 1];
        for (int h = 0; h < n_heads; ++h) {
            float* p = v + h * hd;
            const float a = p[i], b = p[i + half];
            p[i] = fmaf(a, c, -(b * s));
            p[i + half] = fmaf(b, c, a * s);
        }
    }
}

/* ops_ref.cpp:228-241: in-place Walsh-Hadamard transform of each block of `block` values (butterflies v[j] = a + c,
 * v[j + h] = a - c for h = 1, 2, 4, ...), then * 1 / sqrt(block) */
static void fwht_blocks(float* x, int n, int block) {
    const float norm = 1.0f / sqrtf((float)block);
    for (int b0 = 0; b0 < n; b0 += block) {
        float* v = x + b0;
        for (int h = 1; h < block; h *= 2)
            for (int i = 0; i < block; i += 2 * h)
                for (int j = i; j < i + h; ++j) {
                    const float a = v[j], c = v[j + h];
                    v[j] = a + c;
                    v[j + h] = a - c;
                }
        for (int i = 0; i < block; ++i) v[i] *= norm;
    }
}

/* ops_ref.cpp:216-226 */
static void softmax(float* x, int n) {
    float mx = x[0];
    for (int i = 1; i < n; ++i) mx = x[i] > mx ? x[i] : mx;
    float sum = 0.f;
    for (int i = 0; i < n; ++i) {
        x[i] = expf(x[i] - mx);
        sum += x[i];
    }
    const float inv = 1.0f / sum;
    for (int i = 0; i < n; ++i) x[i] *= inv;
}

/* Model::linear (model.cpp:150-157): the integer-dot matvec on the quantized activation for a Q8_0 / Q4_0 W,
 * matvec_ref on the f32 activation x for an F32 / F16 W */
static void linear(const qo_decoder* d, float* out, int l, int which, int rows, int cols, const float* x,
                   const int8_t* xq, const float* xd) {
    const int dt = ldt(d, l, which);
    if (dt == QO_F32 || dt == QO_F16)
        qo_matvec_f(out, dt, rows, cols, lt(d, l, which), x, 0, rows);
    else
        qo_matvec_q(out, dt, rows, cols, (const uint8_t*)lt(d, l, which), xq, xd, 0, rows);
}

/* One token through every layer (model.cpp:174-222); leaves the residual stream in d->x. */
static void layers(qo_decoder* d, int token, int pos) {
    const int D = d->D, hd = d->hdim, kvd = d->nkv * hd, group = d->nh / d->nkv, F = d->F;
    const float scale = 1.0f / sqrtf((float)hd);
    qo_get_row(d->x, d->dt[0], d->V, D, d->t[0], token); /* get_row on the embedding (model.cpp:173) */
    const float* cs = d->cs + (size_t)pos * hd;
    for (int l = 0; l < d->nl; ++l) {
        rmsnorm(d->xb, d->x, (const float*)lt(d, l, L_ATTN_NORM), D, d->eps);
        qo_quantize_q8(d->xb, D, d->xq, d->xd);
        linear(d, d->q, l, L_WQ, D, D, d->xb, d->xq, d->xd);
        linear(d, d->k, l, L_WK, kvd, D, d->xb, d->xq, d->xd);
        linear(d, d->v, l, L_WV, kvd, D, d->xb, d->xq, d->xd);
        if (d->bias) {
            const float *bq = (const float*)lt(d, l, L_BQ), *bk = (const float*)lt(d, l, L_BK),
                        *bv = (const float*)lt(d, l, L_BV);
            for (int i = 0; i < D; ++i) d->q[i] += bq[i];
            for (int i = 0; i < kvd; ++i) d->k[i] += bk[i];
            for (int i = 0; i < kvd; ++i) d->v[i] += bv[i];
        }
        rope(d->q, d->nh, hd, cs);
        rope(d->k, d->nkv, hd, cs);
        const size_t loff = (size_t)l * d->ctx * kvd;
        /* store (model.cpp:113-114, 197-204): the f16 rounding of k / v, or k / v themselves with kv32 */
        for (int i = 0; i < kvd; ++i) {
            if (d->kv32) {
                d->kcf[loff + (size_t)pos * kvd + i] = d->k[i];
                d->vcf[loff + (size_t)pos * kvd + i] = d->v[i];
            } else {
                d->kc[loff + (size_t)pos * kvd + i] = qo_f32_to_f16(d->k[i]);
                d->vc[loff + (size_t)pos * kvd + i] = qo_f32_to_f16(d->v[i]);
            }
        }
#define QO_KV(c, t, i) (d->kv32 ? d->c##f[loff + (size_t)(t) * kvd + (i)] : qo_fp16_to_f32(d->c[loff + (size_t)(t) * kvd + (i)]))
        /* attend (model.cpp:115-137), head by head */
        for (int h = 0; h < d->nh; ++h) {
            const float* qh = d->q + h * hd;
            const int kvh = h / group;
            for (int t = 0; t <= pos; ++t) {
                float s = 0.f;
                for (int i = 0; i < hd; ++i) s = fmaf(qh[i], QO_KV(kc, t, kvh * hd + i), s);
                d->att[t] = s * scale;
            }
            softmax(d->att, pos + 1);
            float* out = d->xb + h * hd;
            for (int i = 0; i < hd; ++i) out[i] = 0.f;
            for (int t = 0; t <= pos; ++t) {
                const float a = d->att[t];
                for (int i = 0; i < hd; ++i) out[i] = fmaf(a, QO_KV(vc, t, kvh * hd + i), out[i]);
            }
        }
#undef QO_KV
        qo_quantize_q8(d->xb, D, d->xq, d->xd);
        linear(d, d->xb2, l, L_WO, D, D, d->xb, d->xq, d->xd);
        for (int i = 0; i < D; ++i) d->x[i] += d->xb2[i];
        rmsnorm(d->xb, d->x, (const float*)lt(d, l, L_FFN_NORM), D, d->eps);
        qo_quantize_q8(d->xb, D, d->xq, d->xd);
        linear(d, d->hb, l, L_WG, F, D, d->xb, d->xq, d->xd);
        linear(d, d->hb2, l, L_WU, F, D, d->xb, d->xq, d->xd);
        for (int i = 0; i < F; ++i) { /* swiglu, ops_ref.cpp:243-248 */
            const float g = d->hb[i];
            d->hb[i] = g / (1.0f + expf(-g)) * d->hb2[i];
        }
        if (d->flags & 1) fwht_blocks(d->hb, F, 256); /* model.cpp:219 */
        qo_quantize_q8(d->hb, F, d->hq, d->hd);
        linear(d, d->xb2, l, L_WD, D, F, d->hb, d->hq, d->hd);
        for (int i = 0; i < D; ++i) d->x[i] += d->xb2[i];
    }
}

/* final norm, quantization and head (model.cpp:225-238) */
static int head(qo_decoder* d, int top_k, float* logits, float* hidden, int8_t* hq, float* hd) {
    const int D = d->D, V = d->V;
    rmsnorm(d->x, d->x, (const float*)d->t[1], D, d->eps);
    qo_quantize_q8(d->x, D, d->xq, d->xd);
    int rows;
    const void* h4 = d->t[2 + d->nl * L_COUNT];
    const void* he = d->t[3 + d->nl * L_COUNT];
    if (top_k > 0 && h4 && he) {
        int ns, tie;
        float tau;
        rows = qo_shortlist_head((const uint8_t*)d->t[d->lm], (const uint8_t*)h4, (const uint16_t*)he, V, D, d->xq, d->xd,
                                 top_k, V, d->must, d->n_must, d->logits, d->coarse, d->upper, d->rows, &ns, &tau,
                                 &tie);
    } else {
        /* the LM head (model.cpp:16): the embedding when tied, else lm_head.weight; Model::linear by its dtype */
        if (d->dt[d->lm] == QO_F32 || d->dt[d->lm] == QO_F16)
            qo_matvec_f(d->logits, d->dt[d->lm], V, D, d->t[d->lm], d->x, 0, V);
        else
            qo_matvec_q(d->logits, d->dt[d->lm], V, D, (const uint8_t*)d->t[d->lm], d->xq, d->xd, 0, V);
        rows = V;
    }
    if (logits) memcpy(logits, d->logits, sizeof(float) * (size_t)V);
    if (hidden) memcpy(hidden, d->x, sizeof(float) * (size_t)D);
    if (hq) memcpy(hq, d->xq, (size_t)D);
    if (hd) memcpy(hd, d->xd, sizeof(float) * (size_t)(D / QO_QK));
    return rows;
}

void qo_decoder_set_must(qo_decoder* d, const int* must, int n_must) {
    d->must = n_must > 0 ? must : NULL;
    d->n_must = n_must > 0 ? n_must : 0;
}

int qo_decoder_forward(qo_decoder* d, int token, int pos, int top_k, float* logits, float* hidden, int8_t* hq,
                       float* hd) {
    if (pos < 0 || pos >= d->ctx || token < 0 || token >= d->V) return -1;
    layers(d, token, pos);
    return head(d, top_k, logits, hidden, hq, hd);
}

int qo_decoder_forward_batch(qo_decoder* d, const int* tokens, int n, int pos0, int top_k, float* logits,
                             float* hidden, int8_t* hq, float* hd) {
    if (n <= 0 || pos0 < 0 || pos0 + n > d->ctx) return -1;
    for (int t = 0; t < n; ++t) {
        if (tokens[t] < 0 || tokens[t] >= d->V) return -1;
        layers(d, tokens[t], pos0 + t);
    }
    return head(d, top_k, logits, hidden, hq, hd);
}

/* ------------------------------------------------------------------ sampler (sampler.cpp:10-85, sampler.h) */

/* xorshift64* (sampler.cpp:16-21) and the 24-bit uniform in [0, 1) (sampler.h next_uniform). */
static uint64_t sampler_next(uint64_t* s) {
    *s ^= *s >> 12;
    *s ^= *s << 25;
    *s ^= *s >> 27;
    return *s * 0x2545F4914F6CDD1DULL;
}
static float sampler_uniform(uint64_t* s) { return (float)(sampler_next(s) >> 40) * (1.0f / 16777216.0f); }

uint64_t qo_sampler_seed(uint64_t seed) { return seed | 1u; }

typedef struct {
    float v;
    int id;
} scored;

/* larger value first, then the lower id */
static int scored_cmp(const void* a, const void* b) {
    const scored* x = (const scored*)a;
    const scored* y = (const scored*)b;
    if (x->v > y->v) return -1;
    if (x->v < y->v) return 1;
    return (x->id > y->id) - (x->id < y->id);
}

int qo_sample(float* logits, int n_valid, const int* history, int n_hist, const qo_sampler_params* p,
              uint64_t* state) {
    if (n_valid <= 0) return -1;
    /* repetition penalty over the distinct ids of the window (sampler.cpp:23-33) */
    if (p->repeat_penalty != 1.0f && n_hist > 0) {
        const int from = (p->repeat_window > 0 && n_hist > p->repeat_window) ? n_hist - p->repeat_window : 0;
        uint8_t* seen = (uint8_t*)calloc((size_t)n_valid, 1);
        for (int i = from; i < n_hist; ++i) {
            const int id = history[i];
            if (id < 0 || id >= n_valid || seen[id]) continue;
            seen[id] = 1;
            const float l = logits[id];
            logits[id] = l > 0 ? l / p->repeat_penalty : l * p->repeat_penalty;
        }
        free(seen);
    }
    if (p->temperature <= 0.0f) return qo_argmax(logits, n_valid); /* sampler.cpp:35-37 */

    /* top-k by logit (sampler.cpp:39-50) */
    scored* c = (scored*)malloc(sizeof(scored) * (size_t)n_valid);
    for (int i = 0; i < n_valid; ++i) {
        c[i].v = logits[i];
        c[i].id = i;
    }
    qsort(c, (size_t)n_valid, sizeof(scored), scored_cmp);
    int k = n_valid;
    if (p->top_k > 0 && p->top_k < k) k = p->top_k;

    /* softmax with temperature (sampler.cpp:52-59) */
    const float mx = c[0].v;
    float sum = 0.f;
    for (int i = 0; i < k; ++i) {
        c[i].v = expf((c[i].v - mx) / p->temperature);
        sum += c[i].v;
    }
    for (int i = 0; i < k; ++i) c[i].v /= sum;

    /* min-p, top-p (sampler.cpp:61-75) */
    int keep = k;
    if (p->min_p > 0.f) {
        const float floor_p = c[0].v * p->min_p;
        while (keep > 1 && c[keep - 1].v < floor_p) --keep;
    }
    if (p->top_p < 1.f) {
        float cum = 0.f;
        for (int i = 0; i < keep; ++i) {
            cum += c[i].v;
            if (cum >= p->top_p) {
                keep = i + 1;
                break;
            }
        }
    }

    /* draw (sampler.cpp:77-84) */
    float total = 0.f;
    for (int i = 0; i < keep; ++i) total += c[i].v;
    float r = sampler_uniform(state) * total;
    int id = c[keep - 1].id;
    for (int i = 0; i < keep; ++i) {
        r -= c[i].v;
        if (r <= 0.f) {
            id = c[i].id;
            break;
        }
    }
    free(c);
    return id;
}
