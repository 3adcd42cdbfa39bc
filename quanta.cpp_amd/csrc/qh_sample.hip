// Token sampling on the device: the reference's Sampler::sample (engine/src/sampler.cpp:22-85) in one workgroup, with
// the same float operations in the same order, so the chosen id and the generator state are the reference's.
//
//  1. repetition penalty (sampler.cpp:23-33): the history window's ids go into an LDS bitmap; a candidate whose id is
//     set gets l > 0 ? l / penalty : l * penalty, applied once per id however often it repeats;
//  2. greedy (temperature <= 0, sampler.cpp:35-37): the first maximum, as a block maximum of 64-bit keys (ordered
//     logit bits, then the lower id);
//  3. top-k (sampler.cpp:39-50): the k-th largest key of any k candidates bounds the k-th largest overall from below,
//     so each wave ranks 64 candidates (the first 64 rows of the shortlist head's list are its seeds, the best coarse
//     scores, which makes the bound tight) and only keys at or above the best bound enter an LDS pool, which a
//     bitonic network sorts; a pool that overflows falls back to k rounds of a block maximum below the previous key;
//  4. softmax with temperature, min-p, top-p and the draw (sampler.cpp:52-84): the exponentials and divisions run one
//     per thread, the sums and the draw serially in the reference's order; glibc-identical expf; xorshift64* state in
//     device memory.
// Candidates are the shortlist head's row list (every other id's logit is -inf there) or every id below n_valid. Ties
// in the top-k go to the lower id (the reference's std::sort leaves the order of equal logits unspecified).
#include "qh_device.h"
#include "qh_internal.h"
#include "qh_math.h"

namespace qh {

namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kPool = 4096;

// xorshift64* (sampler.cpp:16-21) and the 24-bit uniform of sampler.h.
__device__ __forceinline__ uint64_t xorshift64s(uint64_t& s) {
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    return s * 0x2545F4914F6CDD1DULL;
}

__device__ uint64_t block_max_u64(uint64_t v, uint64_t* red) {
    v = wave_max_u64(v);
    const int lane = (int)threadIdx.x & 63, wave = (int)threadIdx.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    uint64_t m = red[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) m = red[w] > m ? red[w] : m;
    __syncthreads();  // red is reused
    return m;
}

}  // namespace

__global__ __launch_bounds__(kThreads) void sample_kernel(const float* __restrict__ logits, int n_valid,
                                                          const int32_t* __restrict__ rows,
                                                          const qh_head_stats* __restrict__ hs, HeadMust hist,
                                                          qh_sampler_params p, uint64_t* __restrict__ state,
                                                          int32_t* __restrict__ out_id) {
    extern __shared__ uint32_t seen[];  // [ceil(n_valid / 32)]: history ids, when the penalty is on
    __shared__ uint64_t pool[kPool];
    __shared__ uint64_t red[kWaves];
    __shared__ uint64_t wbound[kWaves];
    __shared__ float cval[QH_SAMPLE_MAX_TOPK];
    __shared__ int cid[QH_SAMPLE_MAX_TOPK];
    __shared__ int pool_n;
    __shared__ float sum_sh;
    __shared__ uint64_t exptab[32];  // expf's table in LDS: the softmax below reads it without a cache round trip
    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint64_t tabv = expf_detail::kTab[min(tid, 31)];
    const bool pen = p.repeat_penalty != 1.0f;
    if (pen) {
        for (int i = tid; i < (n_valid + 31) / 32; i += kThreads) seen[i] = 0u;
        __syncthreads();
        const int32_t* h;
        int nh;
        must_span(hist, h, nh);
        for (int i = tid; i < nh; i += kThreads) {
            const int id = h[i];
            if (id >= 0 && id < n_valid) atomicOr(&seen[id >> 5], 1u << (id & 31));
        }
        __syncthreads();
    }
    const int n = rows ? hs->n_rows : n_valid;
    auto key_of = [&](int i) -> uint64_t {
        const int id = rows ? rows[i] : i;
        if (id < 0 || id >= n_valid) return 0ull;
        float l = logits[id];
        if (pen && ((seen[id >> 5] >> (id & 31)) & 1u)) l = l > 0 ? l / p.repeat_penalty : l * p.repeat_penalty;
        return score_key(l, id);
    };

    if (p.temperature <= 0.0f) {  // first maximum (sampler.cpp:35-37)
        uint64_t m = 0;
        for (int i = tid; i < n; i += kThreads) {
            const uint64_t k = key_of(i);
            m = k > m ? k : m;
        }
        m = block_max_u64(m, red);
        if (tid == 0) *out_id = m ? key_row(m) : 0;
        return;
    }

    const int k = (p.top_k > 0 && p.top_k < n_valid) ? p.top_k : n_valid;  // <= QH_SAMPLE_MAX_TOPK (host check)
    if (tid < 32) exptab[tid] = tabv;  // read after the barriers below
    {  // lower bound on the k-th largest key: the k-th largest of the wave's 64 candidates (when k <= 64)
        const int i = wave * 64 + lane;
        const uint64_t a = i < n ? key_of(i) : 0ull;
        int rank = 0;
        const int lo = (int)(uint32_t)a, hi = (int)(uint32_t)(a >> 32);
        for (int j = 0; j < 64; ++j) {
            const uint64_t kj = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(hi, j) << 32) |
                                (uint64_t)(uint32_t)__builtin_amdgcn_readlane(lo, j);
            rank += kj > a ? 1 : 0;
        }
        const uint64_t b = (a != 0 && rank == k - 1) ? a : 0ull;
        const uint64_t bw = wave_max_u64(b);
        if (lane == 0) wbound[wave] = bw;
        if (tid == 0) pool_n = 0;
    }
    __syncthreads();
    uint64_t thr = wbound[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) thr = wbound[w] > thr ? wbound[w] : thr;
    thr = thr ? thr : 1ull;  // no bound: every real key (keys are nonzero)
    for (int i = tid; i < n; i += kThreads) {
        const uint64_t key = key_of(i);
        if (key >= thr) {
            const int at = atomicAdd(&pool_n, 1);
            if (at < kPool) pool[at] = key;
        }
    }
    __syncthreads();
    const int count = pool_n;
    if (count == 0) {  // uniform; no candidate (an empty row list)
        if (tid == 0) *out_id = 0;
        return;
    }
    int kk = k < count ? k : count;  // the selected keys, largest first, end up in pool[0, kk)
    if (count <= kPool) {
        int p2 = 1;
        while (p2 < count) p2 <<= 1;
        for (int i = count + tid; i < p2; i += kThreads) pool[i] = 0ull;
        __syncthreads();
        bitonic_sort_desc_u64<kThreads>(pool, p2);
    } else {  // k rounds: the largest key below the previous one
        uint64_t prev = ~0ull;
        for (int r = 0; r < k; ++r) {
            uint64_t m = 0;
            for (int i = tid; i < n; i += kThreads) {
                const uint64_t key = key_of(i);
                m = (key < prev && key > m) ? key : m;
            }
            m = block_max_u64(m, red);
            if (tid == 0) pool[r] = m;
            prev = m;
        }
        kk = k;
        __syncthreads();
    }
    // softmax with temperature over the survivors (sampler.cpp:52-59)
    const float mx = key_score(pool[0]);
    for (int i = tid; i < kk; i += kThreads) {
        cval[i] = expf_variant<2>((key_score(pool[i]) - mx) / p.temperature, exptab);
        cid[i] = key_row(pool[i]);
    }
    __syncthreads();
    if (tid == 0) {
        float sum = 0.f;
        for (int i = 0; i < kk; ++i) sum += cval[i];
        sum_sh = sum;
    }
    __syncthreads();
    const float sum = sum_sh;
    for (int i = tid; i < kk; i += kThreads) cval[i] = cval[i] / sum;
    __syncthreads();
    if (tid == 0) {
        int keep = kk;
        if (p.min_p > 0.f) {  // sampler.cpp:61-65
            const float floor_p = cval[0] * p.min_p;
            while (keep > 1 && cval[keep - 1] < floor_p) --keep;
        }
        if (p.top_p < 1.f) {  // sampler.cpp:66-75
            float cum = 0.f;
            for (int i = 0; i < keep; ++i) {
                cum += cval[i];
                if (cum >= p.top_p) {
                    keep = i + 1;
                    break;
                }
            }
        }
        float total = 0.f;  // the draw (sampler.cpp:77-84)
        for (int i = 0; i < keep; ++i) total += cval[i];
        uint64_t st = *state;
        float r = (float)(xorshift64s(st) >> 40) * (1.0f / 16777216.0f) * total;
        *state = st;
        int id = cid[keep - 1];
        for (int i = 0; i < keep; ++i) {
            r -= cval[i];
            if (r <= 0.f) {
                id = cid[i];
                break;
            }
        }
        *out_id = id;
    }
}

size_t sample_lds_bytes(int n_valid) { return (size_t)((n_valid + 31) / 32) * 4; }

hipError_t launch_sample(const float* logits, int n_valid, const int32_t* rows, const qh_head_stats* hs,
                         const HeadMust& hist, const qh_sampler_params& p, uint64_t* state, int32_t* out_id,
                         hipStream_t s) {
    qh_launch(sample_kernel, dim3(1), dim3(kThreads), sample_lds_bytes(n_valid), s, logits, n_valid, rows, hs,
                       hist, p, state, out_id);
    return hipGetLastError();
}

}  // namespace qh
