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

int qo_shortlist_head(const uint8_t* head8, const uint8_t* head4, const uint16_t* err, int V, int D,
                      const int8_t* xq, const float* xd, int top_k, int n_valid, const int* must, int n_must,
                      float* logits, float* coarse, float* upper, int* rows, int* n_seeds_out, float* tau_out,
                      int* seed_tie) {
    const int nb = D / QO_QK;
    const int nv = (n_valid > 0 && n_valid < V) ? n_valid : V; /* model.cpp:245 */
    const int k = top_k;
    const int n_seed = k + 8; /* model.cpp:256 */
    const uint16_t* s8 = (const uint16_t*)(head8 + qo_quant_bytes(QO_Q8_0, V, D));
    const uint16_t* s4 = (const uint16_t*)(head4 + qo_quant_bytes(QO_Q4_0, V, D));

    /* model.cpp:247-251: xnorm_b = d_b * sqrt(sum q^2) (an exact integer sum below 2^24). */
    float* xnorm = (float*)malloc(sizeof(float) * (size_t)nb);
    for (int b = 0; b < nb; ++b) {
        float ss = 0.f;
        for (int i = 0; i < QO_QK; ++i) {
            const float v = (float)xq[b * QO_QK + i];
            ss = fmaf(v, v, ss);
        }
        xnorm[b] = xd[b] * sqrtf(ss);
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
        const float c = row_dot(QO_Q4_0, D, head4, s4, r, xq, xd);
        const uint16_t* e = err + (size_t)r * nb;
        float bound = 0.f;
        for (int b = 0; b < nb; ++b) bound = fmaf(qo_fp16_to_f32(e[b]), xnorm[b], bound);
        bound = fmaf(bound, 1.001f, 1e-5f);
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
        logits[r] = row_dot(QO_Q8_0, D, head8, s8, r, xq, xd);
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
            logits[r] = row_dot(QO_Q8_0, D, head8, s8, r, xq, xd);
        }
    /* must ids, first occurrence only (model.cpp:324-330) */
    for (int i = 0; i < n_must; ++i) {
        const int id = must[i];
        if (id >= 0 && id < nv && mark[id] == 1) {
            rows[n_rows++] = id;
            mark[id] = 0;
            logits[id] = row_dot(QO_Q8_0, D, head8, s8, id, xq, xd);
        }
    }

    if (n_seeds_out) *n_seeds_out = ns;
    if (tau_out) *tau_out = tau;
    if (seed_tie) *seed_tie = tie;
    free(seeds);
    free(mark);
    free(xnorm);
    return n_rows;
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
