// Exact Shortlist Head (reference engine/src/model.cpp:240-334) on gfx950, three launches:
//
//  1. screen    one workgroup per tile of vocab rows: the 4-bit GEMV over the Q4_0 copy (same streaming
//               scheme as the decode GEMV), the per-row bound chain over the f16 block errors and the
//               activation's block norms (bound = fma(sum_b fma(err_b, xnorm_b), 1.001f, 1e-5f)), upper =
//               coarse + bound, logits = -inf; then the tile's best top_k+9 eligible coarse scores
//               (key = score, lower row first on ties) by repeated workgroup max.
//  2. seeds     one workgroup: merges the tile lists into the global top_k+8 seeds (plus one more key to
//               detect a tie at the cut), dedupes the must ids (first occurrence), rescoring seeds and must
//               rows exactly with the Q8_0 row dot, tau = k-th best exact seed.
//  3. cand      one workgroup per 256 rows: candidates {r < n_valid, unmarked, upper[r] >= tau} compacted
//               with a ballot scan, appended to the row list, rescored exactly in the same workgroup, and the
//               greedy argmax key folded in with a 64-bit atomic max; the last workgroup to finish writes the
//               stats record.
//
// Exact rows use the same block products and serial chain as the decode GEMV, so each rescored logit is
// bit-identical to the full Q8_0 head. The mark array (1 byte per row) lives in the workspace: screen clears
// its rows, seeds sets 2 (seed) and 3 (must), cand skips every marked row.
#include "qh_device.h"
#include "qh_internal.h"

namespace qh {

namespace {

struct HeadCtrl {
    unsigned long long argmax_key;
    unsigned int n_cand;
    unsigned int done;
    float tau;
    int n_seeds;
    int n_must;
    int seed_tie;
};

constexpr int kMaxMust = 1024;
constexpr int kScreenThreads = 256;
constexpr int kSeedThreads = 512;
constexpr int kCandThreads = 256;

size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

int screen_tile_rows(int nb) {
    // prod tile (f32, nb+1 per row) + error tile (f16, nb per row) within 48 KB; even row count.
    int t = (48 * 1024) / ((nb + 1) * 4 + nb * 2);
    t = t > 256 ? 256 : t;
    t &= ~1;
    return t < 2 ? 2 : t;
}

struct WsLayout {
    size_t mark, seedpart, ctrl, total;
};

WsLayout ws_layout(int V, int D, int top_k) {
    const int nb = D / QK;
    const int tile = screen_tile_rows(nb);
    const int parts = (V + tile - 1) / tile;
    const int keep = top_k + 9;
    WsLayout l;
    l.mark = 0;
    l.seedpart = align256((size_t)V);
    l.ctrl = l.seedpart + align256((size_t)parts * keep * sizeof(uint64_t));
    l.total = l.ctrl + 256;
    return l;
}

// Block products of one Q8_0 row for the calling wave: lane pairs cover 32-byte blocks; p[b] receives
// float(s_b) * f16(scale_b). Every lane of the wave must call it (DPP inside); `active` masks the work.
__device__ void wave_row_products_q8(const uint8_t* __restrict__ w8, const uint16_t* __restrict__ s8, int row, int nb,
                                     const int8_t* __restrict__ xq, float* p, bool active) {
    const int lane = (int)threadIdx.x & 63;
    const uint8_t* wr = w8 + (size_t)row * nb * QK;
    const int nch = 2 * nb;
    for (int c0 = 0; c0 < nch; c0 += 64) {
        const int c = c0 + lane;
        const bool ok = active && c < nch;
        const uint4 w = ok ? load16(wr + (size_t)c * 16) : make_uint4(0u, 0u, 0u, 0u);
        const int b = min(c >> 1, nb - 1);
        const uint4 xv = load16(xq + b * QK + (c & 1) * 16);
        int s = dot16_i8(w, xv);
        s += swap_pair(s);
        if (ok && !(c & 1)) p[b] = (float)s * f16_to_f32(s8[(size_t)row * nb + b]);
    }
}

__device__ float chain(const float* p, const float* __restrict__ xd, int nb) {
    float acc = 0.0f;
    for (int b = 0; b < nb; ++b) acc = __builtin_fmaf(p[b], xd[b], acc);
    return acc;
}

}  // namespace

template <int U>
__global__ __launch_bounds__(kScreenThreads) void head_screen_kernel(
    const uint8_t* __restrict__ w4, const uint16_t* __restrict__ s4, const uint16_t* __restrict__ err,
    const int8_t* __restrict__ xq, const float* __restrict__ xd, int V, int nb, int nv, const int32_t* __restrict__ must,
    int n_must, int tile, uint32_t nb_magic, float* __restrict__ coarse, float* __restrict__ upper,
    float* __restrict__ logits, uint8_t* __restrict__ mark, uint64_t* __restrict__ seedpart, int n_keep,
    HeadCtrl* __restrict__ ctrl) {
    extern __shared__ float smem[];
    float* prod = smem;                                                    // [tile][nb + 1]
    float* xnorm = prod + (size_t)tile * (nb + 1);                         // [nb]
    uint16_t* errs = reinterpret_cast<uint16_t*>(xnorm + nb);              // [tile][nb]
    uint8_t* mflag = reinterpret_cast<uint8_t*>(errs + (size_t)tile * nb);  // [tile]
    __shared__ uint64_t wbest[2][kScreenThreads / 64];

    const int tid = (int)threadIdx.x;
    const int ra = (int)blockIdx.x * tile;
    const int nrows = min(tile, V - ra);
    const int pstride = nb + 1;
    if (blockIdx.x == 0 && tid == 0) {
        ctrl->argmax_key = 0ull;
        ctrl->n_cand = 0u;
        ctrl->done = 0u;
    }
    for (int i = tid; i < nrows; i += kScreenThreads) {
        mflag[i] = 0;
        mark[ra + i] = 0;
    }
    // xnorm_b = d_b * sqrt(sum q^2) (model.cpp:247-251); the sum is an exact integer in f32.
    for (int b = tid; b < nb; b += kScreenThreads) {
        float ss = 0.0f;
        for (int i = 0; i < QK; ++i) {
            const float v = (float)xq[b * QK + i];
            ss = __builtin_fmaf(v, v, ss);
        }
        xnorm[b] = xd[b] * __builtin_sqrtf(ss);
    }
    // Error tile -> LDS (4-byte loads; ra is even so the tile starts 4-byte aligned).
    {
        const int n16 = nrows * nb;
        const uint32_t* src = reinterpret_cast<const uint32_t*>(err + (size_t)ra * nb);
        uint32_t* dst = reinterpret_cast<uint32_t*>(errs);
        for (int i = tid; i < n16 / 2; i += kScreenThreads) dst[i] = src[i];
        if ((n16 & 1) && tid == 0) errs[n16 - 1] = err[(size_t)ra * nb + n16 - 1];
    }
    __syncthreads();
    for (int i = tid; i < n_must; i += kScreenThreads) {
        const int id = must[i];
        if (id >= ra && id < ra + nrows && id < nv) mflag[id - ra] = 1;
    }

    // 4-bit block products of the tile.
    const int nchunks = nrows * nb;
    const uint8_t* base = w4 + (size_t)ra * nb * (QK / 2);
    const uint16_t* sbase = s4 + (size_t)ra * nb;
    for (int c0 = 0; c0 < nchunks; c0 += kScreenThreads * U) {
        uint4 w[U];
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const int c = c0 + j * kScreenThreads + tid;
            w[j] = c < nchunks ? load16(base + (size_t)c * 16) : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const int c = c0 + j * kScreenThreads + tid;
            const uint32_t g = (uint32_t)c;
            const uint32_t rt = nb == 1 ? g : div_magic(g, nb_magic);
            const uint32_t b = g - rt * (uint32_t)nb;
            const uint4 xlo = load16(xq + b * QK);
            const uint4 xhi = load16(xq + b * QK + 16);
            const int s = dot_q4_block(w[j], xlo, xhi);
            if (c < nchunks) prod[rt * pstride + b] = (float)s * f16_to_f32(sbase[g]);
        }
    }
    __syncthreads();

    uint64_t key = 0;
    if (tid < nrows) {
        const int r = ra + tid;
        const float c = chain(prod + tid * pstride, xd, nb);
        const uint16_t* e = errs + tid * nb;
        float bound = 0.0f;
        for (int b = 0; b < nb; ++b) bound = __builtin_fmaf(f16_to_f32(e[b]), xnorm[b], bound);
        bound = __builtin_fmaf(bound, 1.001f, 1e-5f);  // model.cpp:271
        coarse[r] = c;
        upper[r] = c + bound;
        logits[r] = -__builtin_inff();
        if (r < nv && !mflag[tid]) key = score_key(c, r);
    }
    // Best n_keep keys of the tile, best first.
    const int lane = tid & 63, wave = tid >> 6;
    uint64_t* out = seedpart + (size_t)blockIdx.x * n_keep;
    for (int i = 0; i < n_keep; ++i) {
        const uint64_t m = wave_max_u64(key);
        if (lane == 0) wbest[i & 1][wave] = m;
        __syncthreads();
        uint64_t best = wbest[i & 1][0];
#pragma unroll
        for (int w = 1; w < kScreenThreads / 64; ++w) best = wbest[i & 1][w] > best ? wbest[i & 1][w] : best;
        if (key == best) key = 0;
        if (tid == 0) out[i] = best;
    }
}

__global__ __launch_bounds__(kSeedThreads) void head_seed_kernel(
    const uint8_t* __restrict__ w8, const uint16_t* __restrict__ s8, const int8_t* __restrict__ xq,
    const float* __restrict__ xd, int nb, int nv, int k, int n_keep, int n_parts, uint64_t* __restrict__ seedpart,
    const int32_t* __restrict__ must, int n_must, uint8_t* __restrict__ mark, int32_t* __restrict__ rows,
    float* __restrict__ logits, HeadCtrl* __restrict__ ctrl) {
    extern __shared__ float wprod[];  // [waves][nb]
    __shared__ uint64_t best[QH_HEAD_MAX_TOPK + 9];
    __shared__ uint64_t wb[2][kSeedThreads / 64];
    __shared__ int rowl[QH_HEAD_MAX_TOPK + 8 + kMaxMust];
    __shared__ float exact[QH_HEAD_MAX_TOPK + 8 + kMaxMust];
    __shared__ int counts[2];

    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    constexpr int kWaves = kSeedThreads / 64;
    const int n_seed = n_keep - 1;
    const int total = n_parts * n_keep;
    for (int i = 0; i < n_keep; ++i) {
        uint64_t m = 0;
        int mi = -1;
        for (int j = tid; j < total; j += kSeedThreads) {
            const uint64_t v = seedpart[j];
            if (v > m) {
                m = v;
                mi = j;
            }
        }
        const uint64_t g = wave_max_u64(m);
        if (lane == 0) wb[i & 1][wave] = g;
        __syncthreads();
        uint64_t gb = wb[i & 1][0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) gb = wb[i & 1][w] > gb ? wb[i & 1][w] : gb;
        if (gb != 0 && m == gb) seedpart[mi] = 0;  // keys are unique (one per row)
        if (tid == 0) best[i] = gb;
    }
    __syncthreads();
    if (tid == 0) {
        int ns = 0;
        while (ns < n_seed && best[ns] != 0) ++ns;
        for (int i = 0; i < ns; ++i) {
            const int r = key_row(best[i]);
            rowl[i] = r;
            rows[i] = r;
            mark[r] = 2;
        }
        int nm = 0;
        for (int i = 0; i < n_must; ++i) {  // first occurrence of each valid id (model.cpp:324-330)
            const int id = must[i];
            if (id >= 0 && id < nv && mark[id] == 0) {
                mark[id] = 3;
                rowl[ns + nm] = id;
                rows[ns + nm] = id;
                ++nm;
            }
        }
        counts[0] = ns;
        counts[1] = nm;
        ctrl->n_seeds = ns;
        ctrl->n_must = nm;
        ctrl->seed_tie = (ns == n_seed && best[n_seed] != 0 && (best[n_seed] >> 32) == (best[n_seed - 1] >> 32)) ? 1 : 0;
    }
    __syncthreads();
    const int ns = counts[0], nrow = counts[0] + counts[1];
    float* p = wprod + wave * nb;
    for (int j0 = 0; j0 < nrow; j0 += kWaves) {
        const int j = j0 + wave;
        const bool active = j < nrow;
        const int r = active ? rowl[j] : 0;
        wave_row_products_q8(w8, s8, r, nb, xq, p, active);
        __syncthreads();
        if (active && lane == 0) {
            const float v = chain(p, xd, nb);
            logits[r] = v;
            exact[j] = v;
        }
        __syncthreads();
    }
    if (tid == 0) {
        float tau = -__builtin_inff();
        if (ns >= k) {  // k-th largest exact seed logit (model.cpp:308-313)
            float sel[QH_HEAD_MAX_TOPK + 8];
            for (int i = 0; i < ns; ++i) sel[i] = exact[i];
            for (int i = 0; i < k; ++i) {
                int m = i;
                for (int q = i + 1; q < ns; ++q)
                    if (sel[q] > sel[m]) m = q;
                const float t = sel[i];
                sel[i] = sel[m];
                sel[m] = t;
            }
            tau = sel[k - 1];
        }
        ctrl->tau = tau;
        uint64_t kmax = 0;
        for (int i = 0; i < nrow; ++i) {
            const uint64_t kk = score_key(exact[i], rowl[i]);
            kmax = kk > kmax ? kk : kmax;
        }
        ctrl->argmax_key = kmax;
    }
}

__global__ __launch_bounds__(kCandThreads) void head_cand_kernel(
    const uint8_t* __restrict__ w8, const uint16_t* __restrict__ s8, const int8_t* __restrict__ xq,
    const float* __restrict__ xd, int nb, int nv, const float* __restrict__ upper, const uint8_t* __restrict__ mark,
    int32_t* __restrict__ rows, float* __restrict__ logits, HeadCtrl* __restrict__ ctrl,
    qh_head_stats* __restrict__ stats) {
    extern __shared__ float wprod[];  // [waves][nb]
    __shared__ int candl[kCandThreads];
    __shared__ int wcount[kCandThreads / 64];
    __shared__ int base_sh;
    __shared__ uint64_t wkey[kCandThreads / 64];
    constexpr int kWaves = kCandThreads / 64;
    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = (int)blockIdx.x * kCandThreads + tid;
    const float tau = ctrl->tau;
    const bool cand = r < nv && mark[r] == 0 && upper[r] >= tau;
    const uint64_t ball = __ballot(cand);
    const int pos = __popcll(ball & ((1ull << lane) - 1ull));
    if (lane == 0) wcount[wave] = __popcll(ball);
    __syncthreads();
    int off = 0, count = 0;
    for (int w = 0; w < kWaves; ++w) {
        off += w < wave ? wcount[w] : 0;
        count += wcount[w];
    }
    if (cand) candl[off + pos] = r;
    if (tid == 0 && count > 0) base_sh = (int)atomicAdd(&ctrl->n_cand, (unsigned)count);
    __syncthreads();
    uint64_t kbest = 0;
    if (count > 0) {
        const int row_off = ctrl->n_seeds + ctrl->n_must + base_sh;
        for (int i = tid; i < count; i += kCandThreads) rows[row_off + i] = candl[i];
        float* p = wprod + wave * nb;
        for (int j0 = 0; j0 < count; j0 += kWaves) {
            const int j = j0 + wave;
            const bool active = j < count;
            const int rr = active ? candl[j] : 0;
            wave_row_products_q8(w8, s8, rr, nb, xq, p, active);
            __syncthreads();
            if (active && lane == 0) {
                const float v = chain(p, xd, nb);
                logits[rr] = v;
                const uint64_t kk = score_key(v, rr);
                kbest = kk > kbest ? kk : kbest;
            }
            __syncthreads();
        }
    }
    if (lane == 0) wkey[wave] = kbest;
    __syncthreads();
    if (tid == 0) {
        uint64_t m = wkey[0];
        for (int w = 1; w < kWaves; ++w) m = wkey[w] > m ? wkey[w] : m;
        if (m) atomicMax(&ctrl->argmax_key, (unsigned long long)m);
        __threadfence();
        const unsigned prev = atomicAdd(&ctrl->done, 1u);
        if (prev == gridDim.x - 1) {  // last workgroup: every append and atomic max is visible
            __threadfence();
            const unsigned long long key = atomicAdd(&ctrl->argmax_key, 0ull);
            const int n_cand = (int)atomicAdd(&ctrl->n_cand, 0u);
            stats->top1 = key_row(key);
            stats->top1_logit = key_score(key);
            stats->n_seeds = ctrl->n_seeds;
            stats->n_must = ctrl->n_must;
            stats->n_cand = n_cand;
            stats->n_rows = ctrl->n_seeds + ctrl->n_must + n_cand;
            stats->seed_tie = ctrl->seed_tie;
            stats->tau = ctrl->tau;
        }
    }
}

size_t head_workspace_bytes(int V, int D, int top_k) { return ws_layout(V, D, top_k).total; }

hipError_t launch_shortlist_head(const qh_tensor& head8, const qh_tensor& head4, const qh_tensor& err,
                                 const int8_t* xq, const float* xd, const qh_head_query& q, const qh_head_out& out,
                                 void* ws, hipStream_t s) {
    const int V = head8.rows, D = head8.cols, nb = D / QK;
    if (q.n_must > kMaxMust) return hipErrorInvalidValue;
    const int nv = (q.n_valid > 0 && q.n_valid < V) ? q.n_valid : V;
    const WsLayout l = ws_layout(V, D, q.top_k);
    uint8_t* wsb = static_cast<uint8_t*>(ws);
    uint8_t* mark = wsb + l.mark;
    uint64_t* seedpart = reinterpret_cast<uint64_t*>(wsb + l.seedpart);
    HeadCtrl* ctrl = reinterpret_cast<HeadCtrl*>(wsb + l.ctrl);
    const uint8_t* w8 = static_cast<const uint8_t*>(head8.data);
    const uint16_t* s8 = reinterpret_cast<const uint16_t*>(w8 + qh_quant_bytes(QH_Q8_0, V, D));
    const uint8_t* w4 = static_cast<const uint8_t*>(head4.data);
    const uint16_t* s4 = reinterpret_cast<const uint16_t*>(w4 + qh_quant_bytes(QH_Q4_0, V, D));
    const uint16_t* e16 = static_cast<const uint16_t*>(err.data);

    const int tile = screen_tile_rows(nb);
    const int parts = (V + tile - 1) / tile;
    const int n_keep = q.top_k + 9;
    const uint32_t magic = nb == 1 ? 0u : (uint32_t)((0x100000000ull + (uint64_t)nb - 1) / (uint64_t)nb);
    const size_t lds1 = (size_t)tile * (nb + 1) * 4 + (size_t)nb * 4 + (size_t)tile * nb * 2 + (size_t)tile;
    hipLaunchKernelGGL((head_screen_kernel<4>), dim3(parts), dim3(kScreenThreads), lds1, s, w4, s4, e16, xq, xd, V, nb,
                       nv, q.must, q.n_must, tile, magic, out.coarse, out.upper, out.logits, mark, seedpart, n_keep,
                       ctrl);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const size_t lds2 = (size_t)(kSeedThreads / 64) * nb * 4;
    hipLaunchKernelGGL(head_seed_kernel, dim3(1), dim3(kSeedThreads), lds2, s, w8, s8, xq, xd, nb, nv, q.top_k, n_keep,
                       parts, seedpart, q.must, q.n_must, mark, out.rows, out.logits, ctrl);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    const size_t lds3 = (size_t)(kCandThreads / 64) * nb * 4;
    hipLaunchKernelGGL(head_cand_kernel, dim3((unsigned)((nv + kCandThreads - 1) / kCandThreads)), dim3(kCandThreads),
                       lds3, s, w8, s8, xq, xd, nb, nv, out.upper, mark, out.rows, out.logits, ctrl, out.stats);
    return hipGetLastError();
}

}  // namespace qh
