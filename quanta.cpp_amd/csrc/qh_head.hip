// Exact Shortlist Head (reference engine/src/model.cpp:240-334) on gfx950, three launches:
//
//  1. screen    persistent streaming grid over the vocabulary rows (even row split per workgroup, tiles of up to 64
//               rows, the next tile's Q4_0 chunks and f16 block errors in flight while the current tile is reduced).
//               Per row: the 4-bit score chain (same block products and association as the decode GEMV), the bound
//               chain over the f16 block errors and the activation's block norms
//               (bound = fma(sum_b fma(err_b, xnorm_b), 1.001f, 1e-5f)), upper = coarse + bound, logits = -inf.
//               Wave 0 owns one row per lane and keeps the workgroup's best top_k+9 eligible keys (score, then
//               lower row first) sorted across its lanes, inserting only keys above the current cut.
//  2. seeds     one workgroup: merges the per-workgroup lists (held in registers) into the global top_k+8 seeds
//               plus one more key to detect a tie at the cut, rescores the seeds exactly with the Q8_0 row dot,
//               tau = k-th best exact seed; lists the must ids' first occurrences (valid, not seeds) in query order
//               after the seeds: every occurrence proposes its index with an atomic minimum per row, then a block
//               scan compacts the winners in order.
//  3. cand      one workgroup per 256 rows: candidates {r < n_valid, unmarked, upper[r] >= tau} compacted with a
//               ballot scan, appended to the row list, rescored exactly in the same workgroup; the must rows are
//               split over the workgroups and rescored too; the greedy argmax key is folded in with a 64-bit atomic
//               max; the last workgroup to finish writes the stats record.
//
// Exact rows use the same block products and serial chain as the decode GEMV, so each rescored logit is
// bit-identical to the full Q8_0 head. The mark array (1 byte per row) lives in the workspace: screen clears its
// rows, seeds sets 2 (seed) and 3 (must), cand skips every marked row. With must ids, screen also resets its rows of
// the first-occurrence array (one int per row) that seeds uses.
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
// Completion counters of the candidate workgroups, two levels: workgroup b counts into group b % kDoneGroups (one
// 128-byte line each, after the 256 bytes of HeadCtrl), each group's last workgroup into HeadCtrl::done. Atomics on
// one address are performed one at a time, so 16 groups of 16 finish sooner than one counter of 256.
constexpr int kDoneGroups = 16;
constexpr int kDoneStride = 32;  // unsigned ints per group counter
static_assert(sizeof(HeadCtrl) <= 256, "the group counters follow HeadCtrl's 256 bytes");
__device__ __forceinline__ unsigned* group_done(HeadCtrl* ctrl) {
    return reinterpret_cast<unsigned*>(reinterpret_cast<uint8_t*>(ctrl) + 256);
}

constexpr int kMaxMust = 1 << 22;  // must ids per query (a history window); the screen scans them per tile
constexpr int kNoFirst = 0x7fffffff;
constexpr int kScreenThreads = 256;
constexpr int kScreenU = 5;         // 16-byte weight chunks per thread per tile (two sets fit 128 VGPRs)
constexpr int kScreenMaxRows = 64;  // rows per tile: one per lane of wave 0
constexpr int kScreenErrU = (kScreenU + 1) / 2;  // 4-byte error words per thread per tile (tile * nb / 2 <= 128 U)
constexpr int kScreenMaxShare = 1024;  // rows per screen workgroup: their keys sit in LDS until the final selection
constexpr int kSeedThreads = 1024;
constexpr int kSeedMaxPool = 2048;     // keys that survive the seed threshold, held in LDS
constexpr int kSeedKeysPerThread = 32; // fallback when more survive: every partial key in registers
constexpr int kCandThreads = 256;
constexpr int kCandRowsPerThread = 4;

size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

// Rows per screen tile: even, at most one per wave-0 lane, and at most kScreenU * 256 Q4_0 chunks.
int screen_tile_rows(int nb) {
    int t = kScreenU * kScreenThreads / nb;
    t = t > kScreenMaxRows ? kScreenMaxRows : t;
    t &= ~1;
    return t < 2 ? 2 : t;
}

int screen_grid(int V, int tile) {
    int g = 4 * device_cus();
    const int min_g = (V + kScreenMaxShare - 3) / (kScreenMaxShare - 2);  // shares are rounded to even rows
    g = g > min_g ? g : min_g;
    const int tiles = (V + tile - 1) / tile;
    return g < tiles ? g : tiles;
}

int cand_grid(int nv) {
    int g = device_cus();
    const int min_g = (nv + kCandRowsPerThread * kCandThreads - 1) / (kCandRowsPerThread * kCandThreads);
    g = g > min_g ? g : min_g;
    const int chunks = (nv + kCandThreads - 1) / kCandThreads;
    return g < chunks ? g : chunks;
}

struct WsLayout {
    size_t mark, first, seedpart, ctrl, total;
};

WsLayout ws_layout(int V, int D, int top_k) {
    const int nb = D / QK;
    const int parts = screen_grid(V, screen_tile_rows(nb));
    const int keep = top_k + 9;
    WsLayout l;
    l.mark = 0;
    l.first = align256((size_t)V);
    l.seedpart = l.first + align256((size_t)V * 4);
    l.ctrl = l.seedpart + align256((size_t)parts * keep * sizeof(uint64_t));
    l.total = l.ctrl + 256 + (size_t)kDoneGroups * kDoneStride * 4;
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

// Register set of one screen tile: the Q4_0 chunks with their block scales, and the f16 error words.
struct ScreenRegs {
    uint4 w[kScreenU];
    uint16_t sc[kScreenU];
    uint32_t e[kScreenErrU];

    __device__ __forceinline__ void load(const uint8_t* __restrict__ w4, const uint16_t* __restrict__ s4,
                                         const uint32_t* __restrict__ e32, int r, int nrows, int nb) {
        const int tid = (int)threadIdx.x;
        const int nch = nrows * nb;
        const uint8_t* base = w4 + (size_t)r * nb * (QK / 2);
        const uint16_t* sbase = s4 + (size_t)r * nb;
#pragma unroll
        for (int j = 0; j < kScreenU; ++j) {
            const int c = min(j * kScreenThreads + tid, nch - 1);
            w[j] = load16(base + (size_t)c * 16);
            sc[j] = sbase[c];
        }
        // nb is even, so a tile's errors are nrows * nb / 2 whole 4-byte words starting 4-byte aligned.
        const int n32 = nrows * nb / 2;
        const uint32_t* ebase = e32 + (size_t)r * nb / 2;
#pragma unroll
        for (int j = 0; j < kScreenErrU; ++j) e[j] = ebase[min(j * kScreenThreads + tid, n32 - 1)];
    }

    // Block products and block errors (as f32) into LDS tiles [row][pstride].
    __device__ __forceinline__ void stage(float* prod, float* errf, int pstride, int nrows, int nb, uint32_t nb_magic,
                                          const int8_t* xs) const {
        const int tid = (int)threadIdx.x;
        const int nch = nrows * nb;
#pragma unroll
        for (int j = 0; j < kScreenU; ++j) {
            const int c = j * kScreenThreads + tid;
            const uint32_t g = (uint32_t)min(c, nch - 1);
            const uint32_t rt = nb == 1 ? g : div_magic(g, nb_magic);
            const uint32_t b = g - rt * (uint32_t)nb;
            const uint4 xlo = *reinterpret_cast<const uint4*>(xs + b * QK);
            const uint4 xhi = *reinterpret_cast<const uint4*>(xs + b * QK + 16);
            const int s = dot_q4_block(w[j], xlo, xhi);
            if (c < nch) prod[rt * pstride + b] = (float)s * f16_to_f32(sc[j]);
        }
        const int n32 = nrows * nb / 2;
#pragma unroll
        for (int j = 0; j < kScreenErrU; ++j) {
            const int i = j * kScreenThreads + tid;
            const uint32_t g = 2u * (uint32_t)min(i, n32 - 1);  // first of the word's two blocks (same row)
            const uint32_t rt = div_magic(g, nb_magic);
            const uint32_t b = g - rt * (uint32_t)nb;
            if (i < n32) {
                errf[rt * pstride + b] = f16_to_f32((uint16_t)(e[j] & 0xffffu));
                errf[rt * pstride + b + 1] = f16_to_f32((uint16_t)(e[j] >> 16));
            }
        }
    }
};

// Ranks within a wave: a[s] holds key number s*64 + lane of n keys (n <= 64*NS, missing keys are 0); rank[s]
// receives how many of the n keys are larger than a[s]. Keys are broadcast lane by lane through scalar registers
// (v_readlane), so every lane reads different LDS words beforehand and nothing serialises on one address.
// Every lane of the wave must call it with the same n.
template <int NS>
__device__ __forceinline__ void wave_rank(const uint64_t (&a)[NS], int n, int (&rank)[NS]) {
#pragma unroll
    for (int t = 0; t < NS; ++t) rank[t] = 0;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        if (s * 64 >= n) break;
        const int lo = (int)(uint32_t)a[s], hi = (int)(uint32_t)(a[s] >> 32);
#pragma unroll 16
        for (int j = 0; j < 64; ++j) {
            const uint64_t kj = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(hi, j) << 32) |
                                (uint64_t)(uint32_t)__builtin_amdgcn_readlane(lo, j);
#pragma unroll
            for (int t = 0; t < NS; ++t) rank[t] += kj > a[t] ? 1 : 0;
        }
    }
}

}  // namespace

__global__ __launch_bounds__(kScreenThreads) __attribute__((amdgpu_waves_per_eu(4, 4))) void head_screen_kernel(
    const uint8_t* __restrict__ w4, const uint16_t* __restrict__ s4, const uint32_t* __restrict__ e32,
    const int8_t* __restrict__ xq, const float* __restrict__ xd, int V, int nb, int nv, HeadMust mq, int tile,
    uint32_t nb_magic, float* __restrict__ coarse, float* __restrict__ upper, float* __restrict__ logits,
    uint8_t* __restrict__ mark, int32_t* __restrict__ firsts, uint64_t* __restrict__ seedpart, int n_keep,
    int share_cap) {
    extern __shared__ __align__(16) float smem[];
    // Padded chain rows (chain_lds_pipe): zp zeros, then the nb operands.
    const int L = chain_len32(nb), zp = L - nb, ps = chain_stride32(nb);
    float* xdsp = smem;                                  // [L] activation scales
    float* xnormp = xdsp + L;                            // [L] activation block norms
    float* prod0 = xnormp + L;                           // [tile][ps] block products, two buffers
    float* prod1 = prod0 + (size_t)tile * ps;
    float* errf0 = prod1 + (size_t)tile * ps;            // [tile][ps] block errors, two buffers
    float* errf1 = errf0 + (size_t)tile * ps;
    float* bsh = errf1 + (size_t)tile * ps + kChainPipePad;  // [2][64] bounds of a tile (wave 1 -> wave 0)
    uint64_t* wkeys = reinterpret_cast<uint64_t*>(bsh + 128);                   // [share_cap]
    uint8_t* mflag = reinterpret_cast<uint8_t*>(wkeys + share_cap);             // [2][tile]
    int8_t* xs = reinterpret_cast<int8_t*>(mflag + ((2 * (size_t)tile + 15) & ~size_t(15)));  // [nb * 32]
    uint64_t* lvl2 = reinterpret_cast<uint64_t*>(prod0);  // [4 * 64] after the tile loop
    float* xds = xdsp + zp;
    float* xnorm = xnormp + zp;
    __shared__ int n_elig;

    const int tid = (int)threadIdx.x;
    const int32_t* must;
    int n_must;
    must_span(mq, must, n_must);
    const int ra = (int)((long)blockIdx.x * V / gridDim.x) & ~1;  // even, so error words stay 4-byte aligned
    const int rb = blockIdx.x + 1 == gridDim.x ? V : (int)((long)(blockIdx.x + 1) * V / gridDim.x) & ~1;
    if (ra >= rb) {  // uniform per workgroup: an empty share still publishes an empty list
        if (tid < n_keep) seedpart[(size_t)blockIdx.x * n_keep + tid] = 0ull;
        return;
    }

    ScreenRegs A, B;
    A.load(w4, s4, e32, ra, min(tile, rb - ra), nb);
    zero_chain_prefix(xdsp, prod0, nb, 2 * tile);   // both product buffers
    zero_chain_prefix(xnormp, errf0, nb, 2 * tile);  // both error buffers
    const int cols = nb * QK;
    for (int i = tid; i < cols / 16; i += kScreenThreads) reinterpret_cast<uint4*>(xs)[i] = load16(xq + i * 16);
    for (int i = tid; i < nb; i += kScreenThreads) xds[i] = xd[i];
    __syncthreads();
    // xnorm_b = d_b * sqrt(sum q^2) (model.cpp:247-251); the sum is an exact integer in f32.
    for (int b = tid; b < nb; b += kScreenThreads) {
        float ss = 0.0f;
        for (int i = 0; i < QK; ++i) {
            const float v = (float)xs[b * QK + i];
            ss = __builtin_fmaf(v, v, ss);
        }
        xnorm[b] = xds[b] * __builtin_sqrtf(ss);
    }

    int elig = 0;  // wave 0: eligible keys so far
    // wave 0: the previous tile's rows, coarse scores and bounds buffer, finished once wave 1's bounds are ordered
    // before it by the next barrier
    int prev_r = 0, prev_n = 0, prev_buf = 0;
    float prev_c = 0.0f;
    auto finish_prev = [&]() {
        if (tid < prev_n) upper[prev_r + tid] = prev_c + bsh[prev_buf * 64 + tid];
    };
    // One tile whose chunks sit in `regs`: stage into LDS, then wave 0 (one row per lane) runs the coarse chains and
    // wave 1 the bound chains (model.cpp:263-271).
    int buf = 0;
    auto tile_body = [&](const ScreenRegs& regs, int r, float* prod, float* errf, uint8_t* mf) {
        const int nrows = min(tile, rb - r);
        regs.stage(prod + zp, errf + zp, ps, nrows, nb, nb_magic, xs);
        for (int i = tid; i < nrows; i += kScreenThreads) {
            mf[i] = 0;
            mark[r + i] = 0;
            if (n_must > 0) firsts[r + i] = kNoFirst;
        }
        __syncthreads();
        if (n_must > 0) {
            for (int i = tid; i < n_must; i += kScreenThreads) {
                const int id = must[i];
                if (id >= r && id < r + nrows && id < nv) mf[id - r] = 1;
            }
            __syncthreads();
        }
        if (tid < 64) {
            finish_prev();
            uint64_t key = 0;
            float c = 0.0f;
            if (tid < nrows) {
                const int row = r + tid;
                c = chain_lds_pipe<2>(prod + tid * ps, xdsp, L);
                coarse[row] = c;
                logits[row] = -__builtin_inff();
                if (row < nv && !mf[tid]) key = score_key(c, row);
                wkeys[row - ra] = key;
            }
            elig += __popcll(__ballot(key != 0));
            prev_r = r, prev_n = nrows, prev_buf = buf, prev_c = c;
        } else if (tid < 128) {
            const int l = tid - 64;
            if (l < nrows) {
                const float bound = chain_lds_pipe<2>(errf + l * ps, xnormp, L);
                bsh[buf * 64 + l] = __builtin_fmaf(bound, 1.001f, 1e-5f);  // model.cpp:271
            }
        }
        buf ^= 1;
    };
    // Two register sets in straight-line halves, so the wait before staging one set leaves the other's loads in
    // flight. Loads in the steady-state loop are unconditional (a conditional load makes the compiler's wait
    // counting assume the worst at the join); the last one or two tiles are peeled.
    const int n_tiles = (rb - ra + tile - 1) / tile;
    int t = 0;
    while (t + 2 < n_tiles) {
        B.load(w4, s4, e32, ra + (t + 1) * tile, min(tile, rb - ra - (t + 1) * tile), nb);
        tile_body(A, ra + t * tile, prod0, errf0, mflag);
        A.load(w4, s4, e32, ra + (t + 2) * tile, min(tile, rb - ra - (t + 2) * tile), nb);
        tile_body(B, ra + (t + 1) * tile, prod1, errf1, mflag + tile);
        t += 2;
    }
    if (t + 1 < n_tiles) {
        B.load(w4, s4, e32, ra + (t + 1) * tile, min(tile, rb - ra - (t + 1) * tile), nb);
        tile_body(A, ra + t * tile, prod0, errf0, mflag);
        tile_body(B, ra + (t + 1) * tile, prod1, errf1, mflag + tile);
    } else {
        tile_body(A, ra + t * tile, prod0, errf0, mflag);
    }
    const int R = rb - ra;
    if (tid == 0) n_elig = elig;
    __syncthreads();
    if (tid < 64) finish_prev();
    lvl2[tid] = 0ull;  // over the first product buffer, free now
    __syncthreads();
    // The share's best n_keep keys (keys are unique). Level 1: each wave ranks its quarter of the share (at most
    // 256 keys) and keeps its best n_keep; level 2: wave 0 ranks the 4 * n_keep survivors.
    const int lane = tid & 63, wave = tid >> 6;
    const int Q = (R + 3) / 4;
    const int q0 = min(R, wave * Q), q1 = min(R, q0 + Q);
    {
        uint64_t a[4];
        int rk[4];
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) {
            const int i = q0 + s2 * 64 + lane;
            a[s2] = i < q1 ? wkeys[i] : 0ull;
        }
        if (Q <= 128) {  // uniform
            uint64_t a2[2] = {a[0], a[1]};
            int rk2[2];
            wave_rank<2>(a2, q1 - q0, rk2);
            rk[0] = rk2[0];
            rk[1] = rk2[1];
            rk[2] = rk[3] = n_keep;
        } else {
            wave_rank<4>(a, q1 - q0, rk);
        }
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2)
            if (a[s2] != 0 && rk[s2] < n_keep) lvl2[wave * n_keep + rk[s2]] = a[s2];
    }
    __syncthreads();
    if (wave == 0) {
        uint64_t* part = seedpart + (size_t)blockIdx.x * n_keep;
        uint64_t a[4];
        int rk[4];
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) {
            const int i = s2 * 64 + lane;
            a[s2] = i < 4 * n_keep ? lvl2[i] : 0ull;
        }
        if (4 * n_keep <= 64) {  // uniform
            uint64_t a1[1] = {a[0]};
            int rk1[1];
            wave_rank<1>(a1, 4 * n_keep, rk1);
            rk[0] = rk1[0];
            rk[1] = rk[2] = rk[3] = n_keep;
        } else {
            wave_rank<4>(a, 4 * n_keep, rk);
        }
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2)
            if (a[s2] != 0 && rk[s2] < n_keep) part[rk[s2]] = a[s2];
        if (lane < n_keep && lane >= n_elig) part[lane] = 0ull;
    }
}

__global__ __launch_bounds__(kSeedThreads) void head_seed_kernel(
    const uint8_t* __restrict__ w8, const uint16_t* __restrict__ s8, const int8_t* __restrict__ xq,
    const float* __restrict__ xd, int nb, int nv, int k, int n_keep, int n_parts,
    const uint64_t* __restrict__ seedpart, HeadMust mq, uint8_t* __restrict__ mark, int32_t* __restrict__ firsts,
    int32_t* __restrict__ rows, float* __restrict__ logits, HeadCtrl* __restrict__ ctrl) {
    extern __shared__ float wprod[];  // [waves][nb]
    constexpr int kWaves = kSeedThreads / 64;
    __shared__ uint64_t best[QH_HEAD_MAX_TOPK + 9];
    __shared__ uint64_t wb[2][kWaves];
    __shared__ uint64_t pool[kSeedMaxPool];
    __shared__ int rowl[QH_HEAD_MAX_TOPK + 8];
    __shared__ float exact[QH_HEAD_MAX_TOPK + 8];
    __shared__ int counts[2];
    __shared__ int wsum[kWaves];
    __shared__ int n_pool;

    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n_seed = n_keep - 1;
    // Every partial key in registers. Any n_keep distinct keys bound the global n_keep-th key from below: each
    // wave offers the n_keep-th largest of its lanes' maxima (distinct keys), and L is the largest offer (0 if no
    // wave has n_keep nonzero maxima). Only keys >= L can be selected.
    const int total = n_parts * n_keep;
    uint64_t kv[kSeedKeysPerThread];
#pragma unroll
    for (int j = 0; j < kSeedKeysPerThread; ++j) {
        const int i = j * kSeedThreads + tid;
        kv[j] = i < total ? seedpart[i] : 0ull;
    }
    if (tid < QH_HEAD_MAX_TOPK + 9) best[tid] = 0ull;
    if (tid == 0) n_pool = 0;
    {
        uint64_t lm[1] = {0ull};
#pragma unroll
        for (int j = 0; j < kSeedKeysPerThread; ++j) lm[0] = kv[j] > lm[0] ? kv[j] : lm[0];
        int rk[1];
        wave_rank<1>(lm, 64, rk);
        const uint64_t offer = wave_max_u64((lm[0] != 0 && rk[0] == n_keep - 1) ? lm[0] : 0ull);
        if (lane == 0) wb[0][wave] = offer;
    }
    __syncthreads();
    uint64_t L = wb[0][0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) L = wb[0][w] > L ? wb[0][w] : L;
#pragma unroll
    for (int j = 0; j < kSeedKeysPerThread; ++j) {
        const uint64_t v = kv[j];
        if (v != 0 && v >= L) {
            const int at = atomicAdd(&n_pool, 1);
            if (at < kSeedMaxPool) pool[at] = v;
        }
    }
    __syncthreads();
    const int np = n_pool;
    if (np <= kSeedThreads) {  // uniform: rank each pool key against the pool (broadcast LDS reads); keys are unique
        if (wave * 64 < np) {  // uniform per wave: only the waves that hold pool keys
            const uint64_t mine = tid < np ? pool[tid] : 0ull;
            int rank = 0;
#pragma unroll 8
            for (int j = 0; j < np; ++j) rank += pool[j] > mine ? 1 : 0;
            if (tid < np && rank < n_keep) best[rank] = mine;
        }
    } else {
        // Many survivors (e.g. many equal scores): n_keep rounds of a block-wide maximum over every partial key.
        for (int i = 0; i < n_keep; ++i) {
            uint64_t m = 0;
#pragma unroll
            for (int j = 0; j < kSeedKeysPerThread; ++j) m = kv[j] > m ? kv[j] : m;
            const uint64_t g = wave_max_u64(m);
            if (lane == 0) wb[(i + 1) & 1][wave] = g;
            __syncthreads();
            uint64_t gb = wb[(i + 1) & 1][0];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) gb = wb[(i + 1) & 1][w] > gb ? wb[(i + 1) & 1][w] : gb;
            if (gb != 0 && m == gb) {
#pragma unroll
                for (int j = 0; j < kSeedKeysPerThread; ++j) kv[j] = kv[j] == gb ? 0ull : kv[j];
            }
            if (tid == 0) best[i] = gb;
        }
    }
    __syncthreads();
    if (wave == 0) {  // one lane per seed: the selected keys are best[0, ns), nonzero, best first
        const bool have = lane < n_seed && best[lane] != 0;
        const int ns = __popcll(__ballot(have));
        if (have) {
            const int r = key_row(best[lane]);
            rowl[lane] = r;
            rows[lane] = r;
            mark[r] = 2;
        }
        if (lane == 0) {
            counts[0] = ns;
            ctrl->n_seeds = ns;
            ctrl->seed_tie =
                (ns == n_seed && best[n_seed] != 0 && (best[n_seed] >> 32) == (best[n_seed - 1] >> 32)) ? 1 : 0;
        }
    }
    __syncthreads();
    const int ns = counts[0];
    // The must ids' first occurrences, valid and not seeds, listed after the seeds in query order (model.cpp:324-330;
    // the candidate kernel rescores them): every such occurrence proposes its index for its row with an atomic
    // minimum, then each thread takes a run of the list, counts the occurrences that won, and a block scan of the
    // counts gives each run its place.
    const int32_t* must;
    int n_must;
    must_span(mq, must, n_must);
    if (n_must > 0) {  // uniform
        for (int i = tid; i < n_must; i += kSeedThreads) {
            const int id = must[i];
            if (id >= 0 && id < nv && mark[id] != 2) atomicMin(&firsts[id], i);
        }
        __syncthreads();
        auto first_at = [&](int i, int id) {
            return id >= 0 && id < nv && __hip_atomic_load(&firsts[id], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == i;
        };
        const int per = (n_must + kSeedThreads - 1) / kSeedThreads;
        const int i0 = min(n_must, tid * per), i1 = min(n_must, i0 + per);
        int c = 0;
        for (int i = i0; i < i1; ++i) c += first_at(i, must[i]) ? 1 : 0;
        int incl = c;  // inclusive scan over the wave
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int o = __shfl_up(incl, off, 64);
            incl += lane >= off ? o : 0;
        }
        if (lane == 63) wsum[wave] = incl;
        __syncthreads();
        int base = ns;
        for (int w = 0; w < wave; ++w) base += wsum[w];
        int o = base + incl - c;
        for (int i = i0; i < i1; ++i) {
            const int id = must[i];
            if (first_at(i, id)) {
                rows[o++] = id;
                mark[id] = 3;
            }
        }
        if (tid == kSeedThreads - 1) ctrl->n_must = o - ns;
    } else if (tid == 0) {
        ctrl->n_must = 0;
    }
    float* p = wprod + wave * nb;
    for (int j0 = 0; j0 < ns; j0 += kWaves) {
        const int j = j0 + wave;
        const bool active = j < ns;
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
    if (wave == 0) {  // one lane per seed
        const bool have = lane < ns;
        const float e = have ? exact[lane] : -__builtin_inff();
        float tau = -__builtin_inff();
        if (ns >= k) {  // k-th largest exact seed logit (model.cpp:308-313): fewer than k above it, k at or above
            int gt = 0, ge = 0;
            const int nsu = __builtin_amdgcn_readfirstlane(ns);
            for (int j = 0; j < nsu; ++j) {
                const float ej = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), j));
                gt += ej > e ? 1 : 0;
                ge += ej >= e ? 1 : 0;
            }
            const uint64_t at = __ballot(have && gt < k && ge >= k);  // equal values wherever it is set
            tau = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), __ffsll((long long)at) - 1));
        }
        const uint64_t kmax = wave_max_u64(have ? score_key(e, rowl[lane]) : 0ull);
        if (lane == 0) {
            ctrl->tau = tau;
            ctrl->argmax_key = kmax;
            ctrl->n_cand = 0u;
            ctrl->done = 0u;
        }
        if (lane < kDoneGroups) group_done(ctrl)[lane * kDoneStride] = 0u;
    }
}

__global__ __launch_bounds__(kCandThreads) void head_cand_kernel(
    const uint8_t* __restrict__ w8, const uint16_t* __restrict__ s8, const int8_t* __restrict__ xq,
    const float* __restrict__ xd, int nb, int nv, const float* __restrict__ upper, const uint8_t* __restrict__ mark,
    int32_t* __restrict__ rows, float* __restrict__ logits, HeadCtrl* __restrict__ ctrl,
    qh_head_stats* __restrict__ stats, TokenFeedback fb) {
    extern __shared__ float wprod[];  // [waves][nb]
    constexpr int kWaves = kCandThreads / 64;
    __shared__ int candl[kCandRowsPerThread * kCandThreads];
    __shared__ int wcount[kCandRowsPerThread][kWaves];
    __shared__ int base_sh;
    __shared__ uint64_t wkey[kWaves];
    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Rows [ca, cb) of this workgroup (at most kCandRowsPerThread per thread): every row's bound and mark are
    // loaded up front, candidates are compacted with ballots and rescored, one row per wave at a time.
    const int ca = (int)((long)blockIdx.x * nv / gridDim.x), cb = (int)((long)(blockIdx.x + 1) * nv / gridDim.x);
    const float tau = ctrl->tau;
    const int row_base = ctrl->n_seeds + ctrl->n_must;
    float up[kCandRowsPerThread];
    uint8_t mk[kCandRowsPerThread];
#pragma unroll
    for (int j = 0; j < kCandRowsPerThread; ++j) {
        const int r = min(ca + j * kCandThreads + tid, cb - 1);
        up[j] = upper[r];
        mk[j] = mark[r];
    }
    bool cand[kCandRowsPerThread];
    int pos[kCandRowsPerThread];
#pragma unroll
    for (int j = 0; j < kCandRowsPerThread; ++j) {
        const int r = ca + j * kCandThreads + tid;
        cand[j] = r < cb && mk[j] == 0 && up[j] >= tau;
        const uint64_t ball = __ballot(cand[j]);
        pos[j] = __popcll(ball & ((1ull << lane) - 1ull));
        if (lane == 0) wcount[j][wave] = __popcll(ball);
    }
    __syncthreads();
    int count = 0;
#pragma unroll
    for (int j = 0; j < kCandRowsPerThread; ++j) {
        int off = count;
        for (int w = 0; w < kWaves; ++w) {
            off += w < wave ? wcount[j][w] : 0;
            count += wcount[j][w];
        }
        if (cand[j]) candl[off + pos[j]] = ca + j * kCandThreads + tid;
    }
    uint64_t kbest = 0;
    if (count > 0) {
        if (tid == 0) base_sh = (int)atomicAdd(&ctrl->n_cand, (unsigned)count);
        __syncthreads();
        for (int i = tid; i < count; i += kCandThreads) rows[row_base + base_sh + i] = candl[i];
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
    {  // the must rows, listed after the seeds, split over the workgroups
        const int ns = ctrl->n_seeds, nm = ctrl->n_must;
        const int ma = (int)((long)blockIdx.x * nm / gridDim.x), mb = (int)((long)(blockIdx.x + 1) * nm / gridDim.x);
        float* p = wprod + wave * nb;
        for (int j0 = ma; j0 < mb; j0 += kWaves) {  // uniform bounds
            const int j = j0 + wave;
            const bool active = j < mb;
            const int rr = active ? rows[ns + j] : 0;
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
        // The maximum is performed (its old value has returned) before the completion count moves, so the last
        // workgroup's atomic reads see every maximum and every count (n_cand's were returned before the rescoring).
        // It reads nothing else another workgroup of this launch wrote, so no cache write-back fence is needed.
        // Workgroups without a scored row skip the maximum: atomics on one address serialize.
        if (m) {
            const unsigned long long old = atomicMax(&ctrl->argmax_key, (unsigned long long)m);
            asm volatile("" ::"v"(old));
        }
        const unsigned g = blockIdx.x % kDoneGroups, gsize = (gridDim.x - g + kDoneGroups - 1) / kDoneGroups;
        const bool group_last = atomicAdd(group_done(ctrl) + g * kDoneStride, 1u) == gsize - 1;
        const unsigned ngroups = gridDim.x < (unsigned)kDoneGroups ? gridDim.x : (unsigned)kDoneGroups;
        if (group_last && atomicAdd(&ctrl->done, 1u) == ngroups - 1) {  // last workgroup
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
            if (fb.token) fb.apply(key_row(key), true);
        }
    }
}

size_t head_workspace_bytes(int V, int D, int top_k) { return ws_layout(V, D, top_k).total; }

bool head_shape_supported(int D) { return D % 64 == 0 && D <= kMaxHeadCols; }

hipError_t launch_shortlist_head(const qh_tensor& head8, const qh_tensor& head4, const qh_tensor& err,
                                 const int8_t* xq, const float* xd, const qh_head_query& q, const HeadMust& must,
                                 const qh_head_out& out, void* ws, hipStream_t s, const TokenFeedback* advance) {
    const int V = head8.rows, D = head8.cols, nb = D / QK;
    if (must.n > kMaxMust || !head_shape_supported(D)) return hipErrorInvalidValue;
    const int nv = (q.n_valid > 0 && q.n_valid < V) ? q.n_valid : V;
    const WsLayout l = ws_layout(V, D, q.top_k);
    uint8_t* wsb = static_cast<uint8_t*>(ws);
    uint8_t* mark = wsb + l.mark;
    int32_t* firsts = reinterpret_cast<int32_t*>(wsb + l.first);
    uint64_t* seedpart = reinterpret_cast<uint64_t*>(wsb + l.seedpart);
    HeadCtrl* ctrl = reinterpret_cast<HeadCtrl*>(wsb + l.ctrl);
    const uint8_t* w8 = static_cast<const uint8_t*>(head8.data);
    const uint16_t* s8 = reinterpret_cast<const uint16_t*>(w8 + qh_quant_bytes(QH_Q8_0, V, D));
    const uint8_t* w4 = static_cast<const uint8_t*>(head4.data);
    const uint16_t* s4 = reinterpret_cast<const uint16_t*>(w4 + qh_quant_bytes(QH_Q4_0, V, D));
    const uint32_t* e32 = static_cast<const uint32_t*>(err.data);

    const int tile = screen_tile_rows(nb);
    const int grid = screen_grid(V, tile);
    const int n_keep = q.top_k + 9;
    if (grid * n_keep > kSeedThreads * kSeedKeysPerThread || grid > kSeedMaxPool) return hipErrorInvalidValue;
    const uint32_t magic = nb == 1 ? 0u : (uint32_t)((0x100000000ull + (uint64_t)nb - 1) / (uint64_t)nb);
    // A share holds at most V / grid + 3 rows (its ends are rounded down to even rows); sizing its key array by that
    // instead of kScreenMaxShare keeps the LDS under 40 KB, so four workgroups fit on a CU.
    const int share_cap = V / grid + 4;
    const size_t lds1 = ((size_t)2 * chain_len32(nb) + 4 * (size_t)tile * chain_stride32(nb) + kChainPipePad + 128) * 4 +
                        (size_t)share_cap * 8 + ((2 * (size_t)tile + 15) & ~size_t(15)) + (size_t)D;
    hipLaunchKernelGGL(head_screen_kernel, dim3(grid), dim3(kScreenThreads), lds1, s, w4, s4, e32, xq, xd, V, nb, nv,
                       must, tile, magic, out.coarse, out.upper, out.logits, mark, firsts, seedpart, n_keep,
                       share_cap);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const size_t lds2 = (size_t)(kSeedThreads / 64) * nb * 4;
    hipLaunchKernelGGL(head_seed_kernel, dim3(1), dim3(kSeedThreads), lds2, s, w8, s8, xq, xd, nb, nv, q.top_k, n_keep,
                       grid, seedpart, must, mark, firsts, out.rows, out.logits, ctrl);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    const size_t lds3 = (size_t)(kCandThreads / 64) * nb * 4;
    hipLaunchKernelGGL(head_cand_kernel, dim3((unsigned)cand_grid(nv)), dim3(kCandThreads), lds3, s, w8, s8, xq, xd, nb, nv, out.upper, mark, out.rows, out.logits, ctrl, out.stats,
                       advance ? *advance : TokenFeedback{});
    return hipGetLastError();
}

}  // namespace qh
