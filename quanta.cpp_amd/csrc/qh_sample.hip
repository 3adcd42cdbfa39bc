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
// in the top-k go to the lower id (the reference's std::sort leaves the order of equal logits unspecified). More than
// QH_SAMPLE_MAX_TOPK survivors (top_k 0, or larger) take the sorted path below the kernel.
#include "qh_device.h"
#include "qh_internal.h"
#include "qh_math.h"

#include <type_traits>

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
    uint64_t thr;
    // Lower bound on the k-th largest key. The head's row list starts with its seeds (the k + 8 best coarse scores),
    // so for k <= 64 the first 64 entries already hold k candidates: each wave's k-th largest of its 64 bounds it.
    // Past 1024 candidates otherwise: the k-th largest of the threads' own maxima (k distinct candidates are at or
    // above it).
    if (n > kThreads && (!rows || k > 64)) {
        uint64_t m = 0;
#pragma unroll 8
        for (int i = tid; i < n; i += kThreads) {
            const uint64_t key = key_of(i);
            m = key > m ? key : m;
        }
        pool[tid] = m;
        if (tid == 0) pool_n = 0;
        __syncthreads();
        bitonic_sort_desc_u64<kThreads>(pool, kThreads);
        thr = pool[k - 1];
        __syncthreads();  // pool is refilled below
    } else {  // the k-th largest of each wave's 64 candidates (when k <= 64)
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
        __syncthreads();
        thr = wbound[0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) thr = wbound[w] > thr ? wbound[w] : thr;
    }
    thr = thr ? thr : 1ull;  // no bound: every real key (keys are nonzero)
#pragma unroll 8
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

// ---------------------------------------------------------------- any number of survivors (top_k 0 or > 256)
// The candidates' complemented keys (~score_key of the penalised logit: ascending complement = larger logit first,
// equal logits lower id first) start at their ids, so in id order; a device-wide LSD radix sort, stable, of 4 passes
// of 8 bits over the complemented logit half (bits 32-63) leaves them in key order. Each pass is a per-tile digit
// histogram and a stable scatter that scans the histograms itself. One workgroup then runs the softmax, min-p, top-p
// and the draw over the sorted survivors in the reference's order (sampler.cpp:52-84). The serial sums stop where
// the rest cannot change them: the survivors' exponentials (and probabilities) do not increase along the order, so
// once a term is far enough below the running value it and every later term round away (still_bound); for the draw
// r -= p_i, r then stays positive to the end and the last kept survivor is drawn (sampler.cpp:84).
constexpr int kSortThreads = 256, kSortTile = 4096, kSortPer = kSortTile / kSortThreads, kDigits = 256;
constexpr int kFinishBatch = 4096;

int sort_tiles(int n_valid) { return (n_valid + kSortTile - 1) / kSortTile; }

size_t sample_workspace_bytes(int n_valid) {
    const size_t G = (size_t)sort_tiles(n_valid), np = G * kSortTile;
    return 2 * np * 8 + G * kDigits * 4 + 256;
}

// The complemented keys (of the penalised logits) at the candidates' ids, ~0 (no candidate) at every other place of
// the tiles. Without a row list every id below n_valid is a candidate and each thread writes its own places; with
// one, sort_fill_kernel writes ~0 everywhere first and this launch then writes the key of each listed id (entries
// past n_rows or outside [0, n_valid) are skipped; an id listed twice writes the same key twice).
__global__ __launch_bounds__(kSortThreads) void sample_keys_kernel(const float* __restrict__ logits, int n_valid,
                                                                   const int32_t* __restrict__ rows,
                                                                   const qh_head_stats* __restrict__ hs,
                                                                   HeadMust hist, float penalty,
                                                                   uint64_t* __restrict__ out) {
    extern __shared__ uint32_t seen[];  // [ceil(n_valid / 32)] history bitmap, when the penalty is on
    const int tid = (int)threadIdx.x;
    const bool pen = penalty != 1.0f;
    if (pen) {
        for (int i = tid; i < (n_valid + 31) / 32; i += kSortThreads) seen[i] = 0u;
        __syncthreads();
        const int32_t* h;
        int nh;
        must_span(hist, h, nh);
        for (int i = tid; i < nh; i += kSortThreads) {
            const int id = h[i];
            if (id >= 0 && id < n_valid) atomicOr(&seen[id >> 5], 1u << (id & 31));
        }
        __syncthreads();
    }
    auto key_of = [&](int id) {
        float l = logits[id];
        if (pen && ((seen[id >> 5] >> (id & 31)) & 1u)) l = l > 0 ? l / penalty : l * penalty;
        return score_key(l, id);
    };
    if (!rows) {
        for (int j = 0; j < kSortPer; ++j) {
            const int i = (int)blockIdx.x * kSortTile + j * kSortThreads + tid;
            out[i] = i < n_valid ? ~key_of(i) : ~0ull;
        }
        return;
    }
    const int n = hs->n_rows;
    for (int i = (int)blockIdx.x * kSortThreads + tid; i < n; i += (int)gridDim.x * kSortThreads) {
        const int id = rows[i];
        if (id >= 0 && id < n_valid) out[id] = ~key_of(id);
    }
}

__global__ __launch_bounds__(kSortThreads) void sort_fill_kernel(uint64_t* __restrict__ out) {
    for (int j = 0; j < kSortPer; ++j) out[(size_t)blockIdx.x * kSortTile + j * kSortThreads + threadIdx.x] = ~0ull;
}

// Digit histogram of one tile: hist[tile * 256 + d].
__global__ __launch_bounds__(kSortThreads) void sort_hist_kernel(const uint64_t* __restrict__ in, int shift,
                                                                 uint32_t* __restrict__ hist) {
    __shared__ uint32_t cnt[kDigits];
    const int tid = (int)threadIdx.x;
    cnt[tid] = 0u;
    __syncthreads();
    for (int j = 0; j < kSortPer; ++j) {
        const uint64_t k = in[(size_t)blockIdx.x * kSortTile + j * kSortThreads + tid];
        atomicAdd(&cnt[(uint32_t)(k >> shift) & 255u], 1u);
    }
    __syncthreads();
    hist[(size_t)blockIdx.x * kDigits + tid] = cnt[tid];
}

// Stable scatter of one tile. Where the tile's keys of digit d start: the keys of the smaller digits in every tile
// and those of digit d in the tiles before (a scan of the G x 256 histograms). Then the tile's keys in index order,
// 256 at a time; a key's place among the round's keys of its digit from 8 ballots (its wave) and the per-wave digit
// counts in LDS (the waves before it).
__global__ __launch_bounds__(kSortThreads) void sort_scatter_kernel(const uint64_t* __restrict__ in,
                                                                    uint64_t* __restrict__ out, int shift,
                                                                    const uint32_t* __restrict__ hist) {
    constexpr int kW = kSortThreads / 64;
    __shared__ uint32_t base[kDigits];
    __shared__ uint32_t wcnt[kW][kDigits];
    __shared__ uint32_t wtot[kW];
    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6, G = (int)gridDim.x, g = (int)blockIdx.x;
    {
        uint32_t tot = 0u, before = 0u;  // digit tid: in every tile, in the tiles before this one
#pragma unroll 8
        for (int t = 0; t < G; ++t) {
            const uint32_t c = hist[(size_t)t * kDigits + tid];
            tot += c;
            before += t < g ? c : 0u;
        }
        uint32_t incl = tot;  // inclusive scan over the wave's 64 digits
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const uint32_t o = (uint32_t)__shfl_up((int)incl, off, 64);
            incl += lane >= off ? o : 0u;
        }
        if (lane == 63) wtot[wave] = incl;
        for (int w = 0; w < kW; ++w) wcnt[w][tid] = 0u;
        __syncthreads();
        uint32_t wbefore = 0u;
        for (int w = 0; w < wave; ++w) wbefore += wtot[w];
        base[tid] = wbefore + incl - tot + before;
        __syncthreads();
    }
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    for (int j = 0; j < kSortPer; ++j) {
        const uint64_t k = in[(size_t)g * kSortTile + j * kSortThreads + tid];
        const uint32_t d = (uint32_t)(k >> shift) & 255u;
        uint64_t same = ~0ull;
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const uint64_t bal = __ballot((d >> b) & 1u);
            same &= ((d >> b) & 1u) ? bal : ~bal;
        }
        const uint32_t rank = (uint32_t)__popcll(same & below);
        if (rank == 0) wcnt[wave][d] = (uint32_t)__popcll(same);
        __syncthreads();
        uint32_t pos = base[d] + rank;
        for (int w = 0; w < wave; ++w) pos += wcnt[w][d];
        out[pos] = k;
        __syncthreads();
        uint32_t add = 0u;
        for (int w = 0; w < kW; ++w) {
            add += wcnt[w][tid];
            wcnt[w][tid] = 0u;
        }
        base[tid] += add;
        __syncthreads();
    }
}

// A term below this bound leaves a running value v > 0 unchanged when added to or subtracted from it, and so does
// every later term: 2^-26 of v's binade. Added, a term below half an ulp (2^-24 of the binade) rounds away;
// subtracted, one below a quarter (the ulp under a power of two is half the one above); the later terms exceed this
// one by at most the ~1-ulp non-monotonicity that expf's rounding allows, far less than the factor 2 kept here.
// 0 when v is below 2^-100 (no early stop).
__device__ __forceinline__ float still_bound(float v) {
    const uint32_t e = __float_as_uint(v) & 0x7f800000u;
    return e >= (27u << 23) ? __uint_as_float(e - (26u << 23)) : 0.0f;
}

__device__ __forceinline__ float lane_f(float x, int j) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), j));
}

// Softmax, min-p, top-p and the draw over the sorted survivors (sorted[i] = ~key of the i-th best candidate, ~0
// past the last; np places).
// Every thread computes a batch of values (exponentials, probabilities) into LDS; the serial sums over them run on
// wave 0 in the reference's order.
__global__ __launch_bounds__(kThreads) void sample_finish_kernel(const uint64_t* __restrict__ sorted, int n_valid,
                                                                 int np, qh_sampler_params p, uint64_t* __restrict__ state,
                                                                 int32_t* __restrict__ out_id) {
    __shared__ float ev[kFinishBatch];
    __shared__ uint64_t exptab[32];
    __shared__ float f_sh;
    __shared__ int i_sh;
    const int tid = (int)threadIdx.x, lane = tid & 63;
    if (tid < 32) exptab[tid] = expf_detail::kTab[tid];
    if (tid == 0) i_sh = np;  // the number of candidates: where the ~0 places start
    __syncthreads();
    for (int i = tid; i < np; i += kThreads)
        if (sorted[i] == ~0ull) atomicMin(&i_sh, i);
    __syncthreads();
    const int n_real = i_sh;
    const int k = (p.top_k > 0 && p.top_k < n_valid) ? p.top_k : n_valid;
    const int kk = k < n_real ? k : n_real;
    if (kk <= 0) {  // uniform; no candidate
        if (tid == 0) *out_id = 0;
        return;
    }
    const float mx = key_score(~sorted[0]);
    __syncthreads();
    auto e_of = [&](int i) { return expf_variant<2>((key_score(~sorted[i]) - mx) / p.temperature, exptab); };
    // Serial pass over val(0 .. m-1) from the running value acc, in order: mode 0 adds, mode 1 adds and stops at the
    // first running value >= thr, mode 2 subtracts and stops at the first running value <= 0. Returns that index,
    // else -1; the pass also ends where no later value can change acc (still_bound). Wave 0 takes 64 values per LDS
    // read and applies them lane by lane with no test between; a chunk after which the stop condition holds is
    // applied again value by value to find the index (the running values are monotone).
    auto serial = [&](int m, auto val, float& acc, auto modec, float thr) -> int {
        constexpr int mode = decltype(modec)::value;
        int at = -1;  // -1 going on, -2 ended early, >= 0 stopped at
        for (int b0 = 0; b0 < m && at == -1; b0 += kFinishBatch) {
            const int bn = min(kFinishBatch, m - b0);
            for (int i = tid; i < bn; i += kThreads) ev[i] = val(b0 + i);
            __syncthreads();
            if (tid < 64) {
                float a = acc;
                int st = -1;
                for (int c = 0; c < bn && st == -1; c += 64) {
                    const float mine = c + lane < bn ? ev[c + lane] : 0.f;  // zeros leave a running value as it is
                    if (lane_f(mine, 0) < still_bound(a)) {
                        st = -2;
                        break;
                    }
                    float b = a;
#pragma unroll
                    for (int j = 0; j < 64; ++j) b = mode == 2 ? b - lane_f(mine, j) : b + lane_f(mine, j);
                    const bool hit = mode == 1 ? b >= thr : (mode == 2 ? b <= 0.f : false);
                    if (!hit) {
                        a = b;
                        continue;
                    }
                    for (int j = 0; j < 64; ++j) {
                        const float v = lane_f(mine, j);
                        a = mode == 2 ? a - v : a + v;
                        if (mode == 1 ? a >= thr : a <= 0.f) {
                            st = b0 + c + j;
                            break;
                        }
                    }
                }
                if (tid == 0) {
                    f_sh = a;
                    i_sh = st;
                }
            }
            __syncthreads();
            acc = f_sh;
            at = i_sh;
            __syncthreads();
        }
        return at >= 0 ? at : -1;
    };
    using Add = std::integral_constant<int, 0>;
    using AddUntil = std::integral_constant<int, 1>;
    using SubUntil = std::integral_constant<int, 2>;
    // sum of the exponentials in order (sampler.cpp:54-58)
    float sum = 0.f;
    serial(kk, e_of, sum, Add{}, 0.f);
    auto p_of = [&](int i) { return e_of(i) / sum; };
    // min-p (sampler.cpp:61-65): keep ends after the last survivor whose probability is not below the floor
    int keep = kk;
    if (p.min_p > 0.f) {
        const float floor_p = p_of(0) * p.min_p;
        if (tid == 0) i_sh = 0;
        __syncthreads();
        int last = 0;
        for (int i = 1 + tid; i < kk; i += kThreads)
            if (!(p_of(i) < floor_p)) last = i;
        if (last) atomicMax(&i_sh, last);
        __syncthreads();
        keep = i_sh + 1;
        __syncthreads();
    }
    // top-p (sampler.cpp:66-75)
    if (p.top_p < 1.f) {
        float cum = 0.f;
        const float tp = p.top_p;
        const int cut = serial(keep, p_of, cum, AddUntil{}, tp);
        if (cut >= 0) keep = cut + 1;
    }
    // the draw (sampler.cpp:77-84)
    float total = 0.f;
    serial(keep, p_of, total, Add{}, 0.f);
    if (tid == 0) {
        uint64_t st = *state;
        f_sh = (float)(xorshift64s(st) >> 40) * (1.0f / 16777216.0f) * total;
        *state = st;
    }
    __syncthreads();
    float r = f_sh;
    __syncthreads();
    const int chosen = serial(keep, p_of, r, SubUntil{}, 0.f);
    if (tid == 0) *out_id = key_row(~sorted[chosen >= 0 ? chosen : keep - 1]);
}

hipError_t launch_sample(const float* logits, int n_valid, const int32_t* rows, const qh_head_stats* hs,
                         const HeadMust& hist, const qh_sampler_params& p, uint64_t* state, int32_t* out_id,
                         void* ws, hipStream_t s) {
    const int k = (p.top_k > 0 && p.top_k < n_valid) ? p.top_k : n_valid;
    if (p.temperature <= 0.0f || k <= QH_SAMPLE_MAX_TOPK) {
        qh_launch(sample_kernel, dim3(1), dim3(kThreads), sample_lds_bytes(n_valid), s, logits, n_valid, rows, hs,
                  hist, p, state, out_id);
        return hipGetLastError();
    }
    if (!ws) return hipErrorInvalidValue;
    const int G = sort_tiles(n_valid);
    const size_t np = (size_t)G * kSortTile;
    uint64_t* a = static_cast<uint64_t*>(ws);
    uint64_t* b = a + np;
    uint32_t* hist_ws = reinterpret_cast<uint32_t*>(b + np);
    if (rows) qh_launch(sort_fill_kernel, dim3((unsigned)G), dim3(kSortThreads), 0, s, a);
    qh_launch(sample_keys_kernel, dim3((unsigned)G), dim3(kSortThreads),
              p.repeat_penalty != 1.0f ? sample_lds_bytes(n_valid) : 0, s, logits, n_valid, rows, hs, hist,
              p.repeat_penalty, a);
    hipError_t e = hipGetLastError();
    for (int shift = 32; shift < 64 && e == hipSuccess; shift += 8) {  // the keys start in id order
        qh_launch(sort_hist_kernel, dim3((unsigned)G), dim3(kSortThreads), 0, s, a, shift, hist_ws);
        qh_launch(sort_scatter_kernel, dim3((unsigned)G), dim3(kSortThreads), 0, s, a, b, shift, hist_ws);
        e = hipGetLastError();
        uint64_t* t = a;
        a = b;
        b = t;
    }
    if (e != hipSuccess) return e;
    qh_launch(sample_finish_kernel, dim3(1), dim3(kThreads), 0, s, a, n_valid, (int)np, p, state, out_id);
    return hipGetLastError();
}

}  // namespace qh
