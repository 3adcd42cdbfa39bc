// Exact Shortlist Head (reference engine/src/model.cpp:240-334) on gfx950, two launches:
//
//  1. screen    persistent streaming grid over the vocabulary rows (an even row share per workgroup, tiles of up to 64
//               rows, the next tile's Q4_0 chunks and f16 block errors in flight while the current tile is reduced).
//               Per row: the 4-bit score chain (same block products and association as the decode GEMV), the bound
//               chain over the f16 block errors and the activation's block norms
//               (bound = fma(sum_b fma(err_b, xnorm_b), 1.001f, 1e-5f)), upper = coarse + bound, logits = -inf, and
//               the row's mark (1: a valid must id, else 0). Each share publishes its kTops best eligible keys
//               (score, then lower row first; must ids and rows >= n_valid are not eligible).
//  2. select    one workgroup per band of at most 1024 rows. Every workgroup first finds the seeds itself, from the
//               published keys: the top_k+9 best keys overall lie in the top_k+9 shares with the best maxima and are
//               at or above the (top_k+9)-th best maximum T, and a share's published keys hold all of its keys >= T
//               unless its last published key is >= T too (then its rows are read again). The top_k+8 best are the
//               seeds (one more key detects a tie at the cut), rescored exactly; tau = k-th best exact seed. Then
//               the band's candidates {unmarked, not a seed, upper >= tau} and must rows are rescored exactly, the
//               candidates appended to the row list, and the greedy argmax key folded in with 64-bit atomic maxima.
//               The last workgroup to finish lists the must ids' first occurrences in query order after the
//               candidates (every occurrence proposed its index with an atomic minimum per row) and writes the stats.
//
// Exact rows use the same block products and serial chain as the decode GEMV, so each rescored logit is
// bit-identical to the full Q8_0 head. Workspace: the marks (1 byte per row), the first-occurrence array (one int per
// row, reset by the screen when the query has must ids), the published keys and the control words.
#include "qh_device.h"
#include "qh_internal.h"

namespace qh {

// Timeline stamps for phase measurements, compiled in only with -DQH_TIMELINE: thread 0 of every workgroup records the
// constant-rate real-time clock (comparable across compute units) at each stamp of the head kernels
// (qh_timeline_head_read copies them out: [kernel][workgroup < 1024][stamp < 4]).
#if defined(QH_TIMELINE)
__device__ uint64_t qh_tl_head[3][1024][4];
#define QH_HSTAMP(k, i)                                                                                   \
    do {                                                                                                  \
        if (threadIdx.x == 0 && blockIdx.x < 1024) qh_tl_head[k][blockIdx.x][i] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
extern "C" int qh_timeline_head_read(uint64_t* host) {
    return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(qh_tl_head), sizeof(qh_tl_head));
}
#else
#define QH_HSTAMP(k, i) \
    do {                \
    } while (0)
#endif

namespace {

// Control words of one call, reset by the screen's first workgroup for the select kernel that follows: the candidate
// count (each workgroup's base in the row list) and two-level completion counters. Workgroup b counts into group
// b % kDoneGroups and folds its best key into that group's key (one 128-byte line per group after the 256 bytes of
// HeadCtrl); each group's last workgroup counts into HeadCtrl::done. Atomics on one address are performed one at a
// time, so 16 groups finish sooner than one counter.
struct HeadCtrl {
    unsigned int n_cand;
    unsigned int done;
};
constexpr int kDoneGroups = 16;
constexpr int kDoneLine = 128;  // bytes per group: the count, then the group's best key at byte 8
constexpr size_t kCtrlBytes = 256 + (size_t)kDoneGroups * kDoneLine;
static_assert(sizeof(HeadCtrl) <= 256, "the group lines follow HeadCtrl's 256 bytes");
__device__ __forceinline__ unsigned* group_done(HeadCtrl* ctrl, int g) {
    return reinterpret_cast<unsigned*>(reinterpret_cast<uint8_t*>(ctrl) + 256 + g * kDoneLine);
}
__device__ __forceinline__ unsigned long long* group_key(HeadCtrl* ctrl, int g) {
    return reinterpret_cast<unsigned long long*>(reinterpret_cast<uint8_t*>(ctrl) + 256 + g * kDoneLine + 8);
}

constexpr int kMaxMust = 1 << 22;  // must ids per query (a history window); the screen scans them per tile
constexpr int kNoFirst = 0x7fffffff;
constexpr int kScreenThreads = 256;
constexpr int kScreenU = 5;         // 16-byte weight chunks per thread per tile (two sets fit 128 VGPRs)
constexpr int kScreenMaxRows = 64;  // rows per tile: one per lane of wave 0
constexpr int kScreenErrU = (kScreenU + 1) / 2;  // 4-byte error words per thread per tile (tile * nb / 2 <= 128 U)
constexpr int kScreenMaxShare = 1024;  // rows per screen workgroup at most (the grid grows for larger vocabularies)
constexpr int kTops = 4;               // best keys each screen share publishes
static_assert(kTops == 4, "a share's keys are written as two 16-byte stores");
constexpr int kSelThreads = 256;
constexpr int kSelWaves = kSelThreads / 64;
constexpr int kSelShares = 4;   // screen shares per select thread: at most kSelShares * kSelThreads shares
constexpr int kSelRows = 4;     // rows per select thread in the candidate scan
constexpr int kPoolCap = 1024;  // keys an LDS selection pool holds
constexpr int kMaxKeep = QH_HEAD_MAX_TOPK + 9;  // the seeds and the key after them
constexpr int kWaveKeep = 64;                    // up to this many, one lane per key in one wave
constexpr int kBandWords = kSelRows * kSelThreads / 32;  // a bit per band row

size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

// Rows per screen tile: even, at most one per wave-0 lane, and at most kScreenU * 256 Q4_0 chunks.
int screen_tile_rows(int nb) {
    int t = kScreenU * kScreenThreads / nb;
    t = t > kScreenMaxRows ? kScreenMaxRows : t;
    t &= ~1;
    return t < 2 ? 2 : t;
}

// Screen shares: two per compute unit (against four, 1 us less for the 151,936-row head: each workgroup's start-up
// is spread over more tiles), an even number of rows (whole 4-byte error words), at least one tile and at most
// kScreenMaxShare rows each. The first n1 shares (one per compute unit: the workgroups dispatched first, which the
// compute unit's arbitration favours over the second ones) hold s1 rows, the others s2 <= s1: share p holds rows
// [start(p), min(start(p) + len(p), V)).
struct ShareMap {
    int n1, s1, s2;
    __host__ __device__ int start(int p) const { return p < n1 ? p * s1 : n1 * s1 + (p - n1) * s2; }
    __host__ __device__ int len(int p) const { return p < n1 ? s1 : s2; }
};
struct ScreenShape {
    int tile, grid;
    ShareMap map;
};
ScreenShape screen_shape(int V, int nb) {
    ScreenShape sh;
    sh.tile = screen_tile_rows(nb);
    const int cus = device_cus(), g = 2 * cus;
    auto even_clamp = [&](long x) {
        int v = (int)((x + 1) & ~1L);
        v = v > sh.tile ? v : sh.tile;
        return v < kScreenMaxShare ? v : kScreenMaxShare;
    };
    // 15% of a share moves from the second workgroups to the first: with equal shares the second ones ended ~2.4 us
    // after the first (151,936 x 896), with 15% both end together and the screen's span drops 17.8 -> 16.5 us (10%
    // and 20% measured less).
    const long base = (V + g - 1) / g, skew = base * 15 / 100;
    const int s1 = even_clamp(base + skew), s2 = even_clamp(base - skew);
    sh.map = ShareMap{cus, s1, s2};
    const long first = (long)cus * s1;
    sh.grid = V <= first ? (int)((V + s1 - 1) / s1) : cus + (int)((V - first + s2 - 1) / s2);
    return sh;
}

// Select bands: one workgroup per compute unit, 256 to kSelRows * kSelThreads rows each, a multiple of kSelRows;
// workgroup b scans rows [b * band, min((b + 1) * band, n_valid)). Fewer workgroups queue fewer atomics on the
// candidate count and repeat the seed selection fewer times.
int select_band(int nv) {
    static_assert(kSelRows == 4, "a thread's marks are one 4-byte word");
    const int g = device_cus();
    int band = ((nv + g - 1) / g + kSelRows - 1) / kSelRows * kSelRows;
    band = band > kSelThreads ? band : kSelThreads;
    return band < kSelRows * kSelThreads ? band : kSelRows * kSelThreads;
}

// Workspace: marks [V], first occurrences [V], published keys [shares][kTops], control words.
struct WsLayout {
    size_t mark, first, tops, ctrl, total;
};

WsLayout ws_layout(int V, int D) {
    const int parts = screen_shape(V, D / QK).grid;
    WsLayout l;
    l.mark = 0;
    l.first = align256((size_t)V);
    l.tops = l.first + align256((size_t)V * 4);
    l.ctrl = l.tops + align256((size_t)parts * kTops * sizeof(uint64_t));
    l.total = l.ctrl + kCtrlBytes;
    return l;
}

// Register set of one screen tile: the Q4_0 chunks with their block scales, and the f16 error words. PL (nibble
// planes): the high plane's chunks (Q4_0 packing of h + 8) with the Q8_0 scales, and no error words.
template <bool PL>
struct ScreenRegs {
    uint4 w[kScreenU];
    uint16_t sc[kScreenU];
    uint32_t e[PL ? 1 : kScreenErrU];

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
            sc[j] = load_f16_bits(sbase + c);
        }
        if constexpr (PL) return;
        // nb is even, so a tile's errors are nrows * nb / 2 whole 4-byte words starting 4-byte aligned.
        const int n32 = nrows * nb / 2;
        const uint32_t* ebase = e32 + (size_t)r * nb / 2;
#pragma unroll
        for (int j = 0; j < (PL ? 1 : kScreenErrU); ++j) e[j] = ebase[min(j * kScreenThreads + tid, n32 - 1)];
    }

    // Block products and block errors (as f32) into LDS tiles [row][pstride]. PL: the block product of the
    // high-nibble midpoints, sum_i (16 h_i + 8) x_i = 16 sum_i (h_i + 8) x_i - 120 sum_i x_i (sxs: the activation's
    // block sums), and the bound's operand d_b itself.
    __device__ __forceinline__ void stage(float* prod, float* errf, int pstride, int nrows, int nb, uint32_t nb_magic,
                                          const int8_t* xs, const int* sxs) const {
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
            if constexpr (PL) {
                const int s = 16 * dot_u4_block(w[j], xlo, xhi) - 120 * sxs[b];
                const float d = f16_to_f32(sc[j]);
                if (c < nch) {
                    prod[rt * pstride + b] = (float)s * d;
                    errf[rt * pstride + b] = d;
                }
            } else {
                const int s = dot_q4_block(w[j], xlo, xhi);
                if (c < nch) prod[rt * pstride + b] = (float)s * f16_to_f32(sc[j]);
            }
        }
        if constexpr (PL) return;
        const int n32 = nrows * nb / 2;
#pragma unroll
        for (int j = 0; j < (PL ? 1 : kScreenErrU); ++j) {
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
}  // namespace

namespace {


// Workgroup state of block_kth_threshold.
struct RadixShared {
    uint32_t hist[256];
    int digit, need, count;
};

// A threshold for the k largest (k >= 1) of the keys the workgroup's NT threads enumerate (for_each(visit) calls
// visit(key) for each of the thread's keys; 0 = no key; nonzero keys unique): exactly min(k, number of nonzero keys)
// nonzero keys are >= the value returned. MSB-first radix select over 8-bit digits with a 256-bin LDS histogram, one
// pass (one enumeration) per digit, stopping as soon as the digit's bin holds exactly the keys still needed. Every
// thread of the workgroup calls it (barriers inside); the result is uniform.
template <int NT, typename ForEach>
__device__ uint64_t block_kth_threshold(ForEach for_each, int k, RadixShared& sh) {
    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint64_t prefix = 0;  // the digits chosen so far
    int need = k;         // keys still to take among those with that prefix, largest first
    for (int shift = 56;; shift -= 8) {
        for (int i = tid; i < 256; i += NT) sh.hist[i] = 0u;
        __syncthreads();
        const uint64_t hi = shift == 56 ? 0ull : (~0ull << (shift + 8));
        for_each([&](uint64_t v) {
            if (v != 0 && (v & hi) == prefix) atomicAdd(&sh.hist[(uint32_t)(v >> shift) & 255u], 1u);
        });
        __syncthreads();
        if (wave == 0) {  // lane l counts bins 255 - 4l .. 252 - 4l, so the scan over lanes runs from the top digit
            uint32_t c[4], tot = 0;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                c[q] = sh.hist[255 - 4 * lane - q];
                tot += c[q];
            }
            uint32_t incl = tot;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const uint32_t o = (uint32_t)__shfl_up((int)incl, off, 64);
                incl += lane >= off ? o : 0u;
            }
            const uint32_t excl = incl - tot;
            if (excl < (uint32_t)need && (uint32_t)need <= incl) {
                uint32_t above = excl;
                int d = -1, cnt = 0;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    if (d < 0) {
                        if (above + c[q] >= (uint32_t)need) {
                            d = 255 - 4 * lane - q;
                            cnt = (int)c[q];
                        } else {
                            above += c[q];
                        }
                    }
                }
                sh.digit = d;
                sh.need = need - (int)above;
                sh.count = cnt;
            }
            if (lane == 63 && incl < (uint32_t)need) sh.digit = -1;  // fewer keys than k (first pass only)
        }
        __syncthreads();
        const int d = sh.digit, cnt = sh.count, nd = sh.need;
        __syncthreads();  // everyone has read sh before the next pass clears it
        if (d < 0) return 1ull;  // every nonzero key is in
        prefix |= (uint64_t)d << shift;
        need = nd;
        if (cnt == need || shift == 0) return prefix;  // the digit's bin holds exactly the keys still needed
    }
}

// Wave-aggregated append to an LDS list: the lanes with `pred` take consecutive slots from *counter, one LDS atomic
// per wave. Every lane of the wave calls it; returns the lane's slot, or -1 without pred.
__device__ __forceinline__ int wave_append(bool pred, int* counter) {
    const uint64_t b = __ballot(pred);
    if (b == 0) return -1;
    const int lane = (int)threadIdx.x & 63;
    const int leader = __ffsll((unsigned long long)b) - 1;
    int base = 0;
    if (lane == leader) base = atomicAdd(counter, __popcll(b));
    base = __builtin_amdgcn_readlane(base, leader);  // leader is uniform: no LDS round trip
    return pred ? base + __popcll(b & ((1ull << lane) - 1ull)) : -1;
}

// wave_append for N predicates per lane at once: slot[j] receives the position of lane's value j (or -1 without
// pred[j]); one LDS atomic per wave. Every lane of the wave calls it.
template <int N>
__device__ __forceinline__ void wave_append_n(const bool (&pred)[N], int* counter, int (&slot)[N]) {
    const int lane = (int)threadIdx.x & 63;
    uint64_t m[N];
    int tot = 0;
#pragma unroll
    for (int j = 0; j < N; ++j) {
        m[j] = __ballot(pred[j]);
        tot += __popcll(m[j]);
    }
    int base = 0;
    if (tot != 0) {  // uniform
        if (lane == 0) base = atomicAdd(counter, tot);
        base = __builtin_amdgcn_readfirstlane(base);
    }
    const uint64_t below = (1ull << lane) - 1ull;
    int off = base;
#pragma unroll
    for (int j = 0; j < N; ++j) {
        slot[j] = pred[j] ? off + __popcll(m[j] & below) : -1;
        off += __popcll(m[j]);
    }
}

// Sum over the wave (every lane active).
__device__ __forceinline__ int wave_sum_int(int v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Sum over each group of 4 lanes (DPP quad permutations; every lane active).
__device__ __forceinline__ int quad_sum(int v) {
    v += __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);  // lanes 1,0,3,2
    v += __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);  // lanes 2,3,0,1
    return v;
}

// One step of a 64-bit maximum over groups of 4 lanes: the other lane by the DPP quad permutation CTRL.
template <int CTRL>
__device__ __forceinline__ uint64_t quad_max_step(uint64_t v) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, 0xF, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, 0xF, 0xF, false);
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    return o > v ? o : v;
}

// The rank of every entry of an LDS list of np keys (how many entries are larger), four threads per entry: f(i, rank)
// runs once per entry. Every thread of the workgroup calls it with the same np.
template <typename F>
__device__ __forceinline__ void list_ranks(const uint64_t* a, int np, F f) {
    const int tid = (int)threadIdx.x, part = tid & 3;
    for (int i0 = 0; i0 < np; i0 += kSelThreads / 4) {
        const int i = i0 + (tid >> 2);
        const uint64_t mine = i < np ? a[i] : ~0ull;
        int rank = 0;
#pragma unroll 4
        for (int j = part; j < np; j += 4) rank += a[j] > mine ? 1 : 0;
        rank = quad_sum(rank);
        if (i < np && part == 0) f(i, rank);
    }
}

// A list of screen shares whose rows are read again, as one range of n * share indexes: index i is row
// p[i / share] * share + i % share (rows >= V past the head's last share are no rows); `below` is the share's last
// published key (keys at or above it were published).
struct ShareRows {
    int n;
    int p[kMaxKeep];
    uint64_t below[kMaxKeep];
};

// Exact Q8_0 logits of the rows of two LDS lists, a[0, na) then b[0, nb_), for the activation staged in LDS (codes xs
// [nb * 32], scales xds [nb]); na and nb_ are uniform across the workgroup. Passes of 32 rows: each row's 16-byte
// chunks are loaded by a group of 8 lanes with every load of a pass in flight at once, block products go to LDS prod
// [32][nb] (lane pairs cover a 32-byte block), then one lane per row runs the reference chain acc = fma(p_b, dx_b,
// acc) in block order (the decode GEMV's association, so each logit is bit-identical to the full head's) and writes
// it to out[i] (LDS, by list index) when to_out is set, else to logits[row]. Every thread of the workgroup calls it
// (barriers inside). mid() runs once, by every thread, while the first pass's loads are in flight (it may hold
// barriers and must not touch prod). Returns, in each row's chain lane, the best key of the rows it scored (0
// elsewhere).
// The exact head's rows: Q8_0 (w: quants [V][D], s: scales), or with PL the nibble planes (w: high plane, lo: low
// plane, both [V][nb][16 bytes], s: the Q8_0 scales; sxs: the activation's block sums in LDS). A row's chunk ch is
// half ch % 2 of block ch / 2: the block's bytes 16 (ch % 2) .. + 15 (Q8_0), or its high (even) / low (odd) plane.
struct ExactHead {
    const uint8_t* w;
    const uint8_t* lo;
    const uint16_t* s;
    const int* sxs;
};
constexpr int kRescoreLanes = 8, kRescoreRows = kSelThreads / kRescoreLanes;
struct NoMid {
    __device__ void operator()() const {}
};
template <bool PL, typename Mid = NoMid>
__device__ uint64_t rescore_lists(const int* a, int na, const int* b, int nb_, const ExactHead& eh, const int8_t* xs,
                                  const float* xds, int nb, float* prod, float* out, bool to_out,
                                  float* __restrict__ logits, const Mid& mid = Mid()) {
    constexpr int kPer = 8;  // chunks per lane per batch: one batch for rows of up to 1024 columns
    const int tid = (int)threadIdx.x, g = tid / kRescoreLanes, j = tid % kRescoreLanes;
    const int nch = 2 * nb, cnt = na + nb_;
    uint64_t kbest = 0;
    if (cnt == 0) mid();
    for (int p0 = 0; p0 < cnt; p0 += kRescoreRows) {
        const int i = p0 + g;
        const bool act = i < cnt;
        const int r = !act ? 0 : i < na ? a[i] : b[i - na];
        const uint8_t* wr = eh.w + (size_t)r * nb * QK;
        const uint16_t* sr = eh.s + (size_t)r * nb;
        for (int c0 = 0; c0 < nch; c0 += kRescoreLanes * kPer) {  // uniform
            uint4 w[kPer];
            uint16_t sc[kPer];
#pragma unroll
            for (int c = 0; c < kPer; ++c) {  // unconditional (clamped) loads: all in flight before the first wait
                const int ch = min(c0 + j + kRescoreLanes * c, nch - 1);
                if constexpr (PL)
                    w[c] = load16(((ch & 1) ? eh.lo : eh.w) + ((size_t)r * nb + (ch >> 1)) * 16);
                else
                    w[c] = load16(wr + (size_t)ch * 16);
                sc[c] = load_f16_bits(sr + (ch >> 1));
            }
            if (p0 == 0 && c0 == 0) mid();  // with the first pass's loads in flight
            float scf[kPer];
#pragma unroll
            for (int c = 0; c < kPer; ++c) {
                // Used here, outside the store's branch: otherwise the compiler sinks each scale load into that
                // branch and waits for it there, one round trip per chunk.
                scf[c] = f16_to_f32(sc[c]);
                asm volatile("" : "+v"(scf[c]));
            }
#pragma unroll
            for (int c = 0; c < kPer; ++c) {
                const int ch = c0 + j + kRescoreLanes * c;
                const int blk = min(ch >> 1, nb - 1);
                int sdot;
                if constexpr (PL) {  // q = 16 h + l: 16 sum (h + 8) x - 128 sum x from the high plane, sum l x
                    const uint4 xlo = *reinterpret_cast<const uint4*>(xs + blk * QK);
                    const uint4 xhi = *reinterpret_cast<const uint4*>(xs + blk * QK + 16);
                    const int u = dot_u4_block(w[c], xlo, xhi);
                    sdot = (ch & 1) ? u : 16 * u - 128 * eh.sxs[blk];
                } else {
                    const uint4 xv = *reinterpret_cast<const uint4*>(xs + blk * QK + (ch & 1) * 16);
                    sdot = dot16_i8(w[c], xv);
                }
                sdot += swap_pair(sdot);
                if (act && ch < nch && !(ch & 1)) prod[g * nb + blk] = (float)sdot * scf[c];
            }
        }
        __syncthreads();
        if (to_out && p0 == 0) QH_HSTAMP(2, 1);
        if (act && j == 0) {
            float acc = 0.0f;  // nb is even: pairs of operands, reads issued ahead of the serial chain
            const float2* pp = reinterpret_cast<const float2*>(prod + g * nb);
            const float2* xp = reinterpret_cast<const float2*>(xds);
#pragma unroll 8
            for (int h = 0; h < nb / 2; ++h) {
                const float2 pv = pp[h], xv2 = xp[h];
                acc = __builtin_fmaf(pv.x, xv2.x, acc);
                acc = __builtin_fmaf(pv.y, xv2.y, acc);
            }
            if (to_out)
                out[i] = acc;
            else
                logits[r] = acc;
            const uint64_t kk = score_key(acc, r);
            kbest = kk > kbest ? kk : kbest;
        }
        __syncthreads();
        if (to_out && p0 == 0) QH_HSTAMP(2, 2);
    }
    return kbest;
}

}  // namespace

// PL: the nibble-plane head (w4 the high plane, s4 the Q8_0 scales, e32 unused): coarse scores of the high-nibble
// midpoints and the bound sum_b fma(d_b, (8 dx_b) * sum_i |x_i|), since |q - (16 h + 8)| = |l - 8| <= 8.
template <bool PL>
__global__ __launch_bounds__(kScreenThreads) __attribute__((amdgpu_waves_per_eu(4, 4))) void head_screen_kernel(
    const uint8_t* __restrict__ w4, const uint16_t* __restrict__ s4, const uint32_t* __restrict__ e32,
    const int8_t* __restrict__ xq, const float* __restrict__ xd, int V, int nb, int nv, HeadMust mq, int tile, ShareMap sm,
    uint32_t nb_magic, float* __restrict__ coarse, float* __restrict__ upper, float* __restrict__ logits,
    uint8_t* __restrict__ mark, int32_t* __restrict__ firsts, uint64_t* __restrict__ tops, HeadCtrl* __restrict__ ctrl) {
    extern __shared__ __align__(16) float smem[];
    QH_HSTAMP(0, 0);
    // Padded chain rows (chain_lds_pipe): zp zeros, then the nb operands.
    const int L = chain_len32(nb), zp = L - nb, ps = chain_stride32(nb);
    float* xdsp = smem;                                  // [L] activation scales
    float* xnormp = xdsp + L;                            // [L] activation block norms
    float* prod0 = xnormp + L;                           // [tile][ps] block products, two buffers
    float* prod1 = prod0 + (size_t)tile * ps;
    float* errf0 = prod1 + (size_t)tile * ps;            // [tile][ps] block errors, two buffers
    float* errf1 = errf0 + (size_t)tile * ps;
    float* bsh = errf1 + (size_t)tile * ps + kChainPipePad;  // [2][64] bounds of a tile (wave 1 -> wave 0)
    uint8_t* mshare = reinterpret_cast<uint8_t*>(bsh + 128);                    // [kScreenMaxShare] must flags
    int8_t* xs = reinterpret_cast<int8_t*>(mshare + kScreenMaxShare);            // [nb * 32]
    int* sxs = reinterpret_cast<int*>(xs + nb * QK);                             // PL: [nb] block sums of xs
    float* xds = xdsp + zp;
    float* xnorm = xnormp + zp;

    const int tid = (int)threadIdx.x;
    if (blockIdx.x == 0 && tid < kDoneGroups) {  // the select kernel's counters, which it cannot reset itself
        *group_done(ctrl, tid) = 0u;
        *group_key(ctrl, tid) = 0ull;
        if (tid == 0) {
            ctrl->n_cand = 0u;
            ctrl->done = 0u;
        }
    }
    const int32_t* must;
    int n_must;
    must_span(mq, must, n_must);
    const int share = sm.len((int)blockIdx.x);
    const int ra = sm.start((int)blockIdx.x), rb = min(ra + share, V);  // even ra: error words stay 4-byte aligned

    // The activation first, then the first tile: loads return in order, so the block norms below wait only for the
    // activation while the tile is in flight.
    const int cols = nb * QK;
    const int nx = cols / 16;
    uint4 xv[kMaxHeadCols / 16 / kScreenThreads];
    float xdv = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxHeadCols / 16 / kScreenThreads; ++j)
        if (tid + j * kScreenThreads < nx) xv[j] = load16(xq + (tid + j * kScreenThreads) * 16);
    if (tid < nb) xdv = xd[tid];
    ScreenRegs<PL> A, B;
    A.load(w4, s4, e32, ra, min(tile, rb - ra), nb);
    for (int i = 4 * tid; i < share; i += 4 * kScreenThreads) *reinterpret_cast<uint32_t*>(mshare + i) = 0u;
    zero_chain_prefix(xdsp, prod0, nb, 2 * tile);   // both product buffers
    zero_chain_prefix(xnormp, errf0, nb, 2 * tile);  // both error buffers
#pragma unroll
    for (int j = 0; j < kMaxHeadCols / 16 / kScreenThreads; ++j)
        if (tid + j * kScreenThreads < nx) reinterpret_cast<uint4*>(xs)[tid + j * kScreenThreads] = xv[j];
    if (tid < nb) xds[tid] = xdv;
    __syncthreads();
    // xnorm_b = d_b * sqrt(sum q^2) (model.cpp:247-251): every partial sum is an integer below 2^24, so the reference's
    // float accumulation is exact and equals this integer dot.
    // PL: the bound's operand (8 dx_b) * sum_i |x_i| (an exact integer below 2^24; 8 dx_b is exact) and the block sums.
    for (int b = tid; b < nb; b += kScreenThreads) {
        const uint4 lo = *reinterpret_cast<const uint4*>(xs + b * QK), hi = *reinterpret_cast<const uint4*>(xs + b * QK + 16);
        if constexpr (PL) {
            int l1 = 0, sum = 0;
            for (int i = 0; i < QK; ++i) {
                const int v = xs[b * QK + i];
                l1 += v < 0 ? -v : v;
                sum += v;
            }
            sxs[b] = sum;
            xnorm[b] = (8.0f * xds[b]) * (float)l1;
        } else {
            const int ss = dot16_i8(lo, lo) + dot16_i8(hi, hi);
            xnorm[b] = xds[b] * __builtin_sqrtf((float)ss);
        }
    }
    if constexpr (PL) __syncthreads();  // the block sums, read by the first tile's staging
    // The share's must ids as LDS flags (read once; loads batched so they are in flight together), and with must ids
    // the share's rows of the first-occurrence array reset for the select kernel.
    if (n_must > 0) {  // uniform
        constexpr int kB = 8;
        for (int i0 = 0; i0 < n_must; i0 += kScreenThreads * kB) {
            int id[kB];
#pragma unroll
            for (int q = 0; q < kB; ++q) id[q] = must[min(i0 + q * kScreenThreads + tid, n_must - 1)];
#pragma unroll
            for (int q = 0; q < kB; ++q)
                if (i0 + q * kScreenThreads + tid < n_must && id[q] >= ra && id[q] < rb && id[q] < nv) mshare[id[q] - ra] = 1;
        }
        for (int i = tid; i < rb - ra; i += kScreenThreads) firsts[ra + i] = kNoFirst;
        __syncthreads();
    }

    // wave 0: the previous tile's rows, coarse scores and bounds buffer, finished once wave 1's bounds are ordered
    // before it by the next barrier
    int prev_r = 0, prev_n = 0, prev_buf = 0;
    uint64_t kt[kTops] = {};  // wave 0: each lane's best eligible keys, best first
    float prev_c = 0.0f;
    auto finish_prev = [&]() {
        if (tid < prev_n) upper[prev_r + tid] = prev_c + bsh[prev_buf * 64 + tid];
    };
    // One tile whose chunks sit in `regs`: stage into LDS, then wave 0 (one row per lane) runs the coarse chains and
    // wave 1 the bound chains (model.cpp:263-271).
    int buf = 0;
    auto tile_body = [&](const ScreenRegs<PL>& regs, int r, float* prod, float* errf) {
        const int nrows = min(tile, rb - r);
        const uint8_t* mf = mshare + (r - ra);
        regs.stage(prod + zp, errf + zp, ps, nrows, nb, nb_magic, xs, sxs);
        __syncthreads();
        if (tid < 64) {
            finish_prev();
            uint64_t key = 0;
            float c = 0.0f;
            if (tid < nrows) {
                const int row = r + tid;
                c = chain_lds_pipe<2>(prod + tid * ps, xdsp, L);
                coarse[row] = c;
                logits[row] = -__builtin_inff();
                mark[row] = mf[tid];  // 1: a must id (never a seed or candidate), else 0
                if (row < nv && !mf[tid]) key = score_key(c, row);
#pragma unroll
                for (int j = 0; j < kTops; ++j) {  // insertion into the sorted list
                    const uint64_t hi = kt[j] > key ? kt[j] : key;
                    key = kt[j] > key ? key : kt[j];
                    kt[j] = hi;
                }
            }
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
    QH_HSTAMP(0, 1);
    while (t + 2 < n_tiles) {
        B.load(w4, s4, e32, ra + (t + 1) * tile, min(tile, rb - ra - (t + 1) * tile), nb);
        tile_body(A, ra + t * tile, prod0, errf0);
        A.load(w4, s4, e32, ra + (t + 2) * tile, min(tile, rb - ra - (t + 2) * tile), nb);
        tile_body(B, ra + (t + 1) * tile, prod1, errf1);
        t += 2;
    }
    if (t + 1 < n_tiles) {
        B.load(w4, s4, e32, ra + (t + 1) * tile, min(tile, rb - ra - (t + 1) * tile), nb);
        tile_body(A, ra + t * tile, prod0, errf0);
        tile_body(B, ra + (t + 1) * tile, prod1, errf1);
    } else {
        tile_body(A, ra + t * tile, prod0, errf0);
    }
    __syncthreads();  // wave 1's bounds of the last tile
    if (tid < 64) finish_prev();
    QH_HSTAMP(0, 2);
    // The share's kTops best eligible keys, best first (0 where it has fewer), from the lanes' sorted lists: a wave
    // maximum per rank, whose lane (keys are unique) then moves its list up.
    if (tid < 64) {
        uint64_t best[kTops];
#pragma unroll
        for (int j = 0; j < kTops; ++j) {
            best[j] = wave_max_u64(kt[0]);
            if (kt[0] == best[j]) {
#pragma unroll
                for (int i = 0; i + 1 < kTops; ++i) kt[i] = kt[i + 1];
                kt[kTops - 1] = 0ull;
            }
        }
        if (tid == 0) {
            uint4* t = reinterpret_cast<uint4*>(tops + (size_t)blockIdx.x * kTops);
            t[0] = make_uint4((uint32_t)best[0], (uint32_t)(best[0] >> 32), (uint32_t)best[1], (uint32_t)(best[1] >> 32));
            t[1] = make_uint4((uint32_t)best[2], (uint32_t)(best[2] >> 32), (uint32_t)best[3], (uint32_t)(best[3] >> 32));
        }
    }
    QH_HSTAMP(0, 3);
}

// SH: screen shares per thread (2 for grids of up to 512 shares, else kSelShares). PL: the exact rows are the nibble
// planes (w8 the high plane, lo the low plane, s8 the Q8_0 scales); else the Q8_0 head (lo unused).
template <int SH, bool PL>
__global__ __launch_bounds__(kSelThreads) void head_select_kernel(
    const uint8_t* __restrict__ w8, const uint8_t* __restrict__ lo, const uint16_t* __restrict__ s8,
    const int8_t* __restrict__ xq,
    const float* __restrict__ xd, int nb, int nv, int k, int n_parts, ShareMap sm, int band,
    const uint64_t* __restrict__ tops, const float* __restrict__ coarse, const float* __restrict__ upper,
    const uint8_t* __restrict__ mark, int32_t* __restrict__ firsts, HeadMust mq, int32_t* __restrict__ rows,
    float* __restrict__ logits, HeadCtrl* __restrict__ ctrl, qh_head_stats* __restrict__ stats, TokenFeedback fb) {
    // products [32][nb], activation codes [nb * 32], scales [nb], block sums [nb] (PL)
    extern __shared__ __align__(16) float ssm[];
    float* prod = ssm;
    int8_t* xs = reinterpret_cast<int8_t*>(ssm + kRescoreRows * nb);
    float* xds = reinterpret_cast<float*>(xs + nb * QK);
    int* sxs = reinterpret_cast<int*>(xds + nb);
    const ExactHead eh{w8, lo, s8, sxs};
    __shared__ uint64_t pool[kPoolCap];
    __shared__ int prow[kPoolCap];
    __shared__ uint64_t gmax[kSelThreads / 4];
    __shared__ uint64_t best[kMaxKeep];
    __shared__ int seedrow[kMaxKeep];
    __shared__ int seedidx[kMaxKeep];  // early: pool index of the seed of each rank
    __shared__ float exact[kMaxKeep];
    __shared__ ShareRows inc;  // shares whose published keys may miss keys at or above the cut
    __shared__ int selp[kMaxKeep];
    __shared__ RadixShared rsh;
    __shared__ int candl[kSelRows * kSelThreads], mustl[kSelRows * kSelThreads], candf[kSelRows * kSelThreads];
    __shared__ float candu[kSelRows * kSelThreads];              // the speculative candidates' upper bounds
    constexpr int kRxHead = kMaxKeep > 2 * kRescoreRows ? kMaxKeep : 2 * kRescoreRows;
    __shared__ float rx[kRxHead + kSelRows * kSelThreads];  // exact logits: seeds (or pool), then candl
    __shared__ int n_pool, n_sel, n_c, n_m, n_x, n_cf, ns_sh, base_sh, last_sh, n_cand_sh;
    __shared__ uint64_t thr_sh, key_sh, top_sh;
    __shared__ float tau_sh;
    __shared__ uint32_t seedmap[kBandWords];  // more than kWaveKeep seeds: the band's seed rows
    __shared__ int wsum[kSelWaves];
    __shared__ uint64_t wkey[kSelWaves];

    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n_keep = k + 9, n_seed = k + 8;
    QH_HSTAMP(1, 0);
    // Every load that depends on nothing else first: the band's bounds and marks, the published keys of this thread's
    // shares (tid + s * kSelThreads), the activation.
    // Thread t scans rows r0 = ca + 4t .. r0 + 3 (band is a multiple of 4), their marks one 4-byte word.
    const int ca = (int)blockIdx.x * band, cb = min(ca + band, nv), r0 = ca + kSelRows * tid;
    float up[kSelRows];
    uint8_t mk[kSelRows];
    {
        const uint32_t mw = r0 < cb ? *reinterpret_cast<const uint32_t*>(mark + r0) : 0u;
#pragma unroll
        for (int j = 0; j < kSelRows; ++j) {
            up[j] = upper[min(r0 + j, cb - 1)];
            mk[j] = (uint8_t)(mw >> (8 * j));
        }
    }
    uint64_t tk[SH][kTops];
#pragma unroll
    for (int s = 0; s < SH; ++s) {
        const int p = tid + s * kSelThreads;
        uint4 a = make_uint4(0u, 0u, 0u, 0u), b = a;
        if (p < n_parts) {
            a = load16(tops + (size_t)p * kTops);
            b = load16(tops + (size_t)p * kTops + 2);
        }
        tk[s][0] = ((uint64_t)a.y << 32) | a.x;
        tk[s][1] = ((uint64_t)a.w << 32) | a.z;
        tk[s][2] = ((uint64_t)b.y << 32) | b.x;
        tk[s][3] = ((uint64_t)b.w << 32) | b.z;
    }
    for (int i = tid; i < nb * 2; i += kSelThreads) reinterpret_cast<uint4*>(xs)[i] = load16(xq + (size_t)i * 16);
    for (int i = tid; i < nb; i += kSelThreads) xds[i] = xd[i];
    if constexpr (PL) {  // the activation's block sums (from global memory: xs is not complete before the barrier)
        for (int b = tid; b < nb; b += kSelThreads) {
            int sum = 0;
            for (int i = 0; i < QK; ++i) sum += xq[b * QK + i];
            sxs[b] = sum;
        }
    }
    for (int i = tid; i < kMaxKeep; i += kSelThreads) best[i] = 0ull;
    if (tid < kBandWords) seedmap[tid] = 0u;
    if (tid == 0) {
        n_pool = 0;
        n_sel = 0;
        n_c = 0;
        n_m = 0;
        n_x = 0;
        n_cf = 0;
        inc.n = 0;
        thr_sh = 1ull;
        top_sh = 0ull;
    }
    // The must ids' first occurrences: each occurrence in this workgroup's slice of the list proposes its index for its
    // row with an atomic minimum (the screen reset the rows); the last workgroup lists the winners.
    const int32_t* must;
    int n_must;
    must_span(mq, must, n_must);
    unsigned mdep = 0;  // the minima's returned values: each has been performed before this workgroup's completion
    if (n_must > 0) {
        const int per = (n_must + (int)gridDim.x - 1) / (int)gridDim.x;
        const int ma = min(n_must, (int)blockIdx.x * per), mb = min(n_must, ma + per);
        for (int i = ma + tid; i < mb; i += kSelThreads) {
            const int id = must[i];
            if (id >= 0 && id < nv) mdep |= (unsigned)atomicMin(&firsts[id], i);
        }
    }

    // 1. A cut L at most the n_keep-th best key: the n_keep-th best of the maxima of 64 groups of shares (16 each),
    // since n_keep distinct keys reach it (1 or 0 when fewer groups have an eligible row: every key). Every key >= L
    // goes to the pool: the published ones, and the unpublished ones of shares whose last published key is >= L
    // (read again; rare). The pool holds the n_keep best keys; ranking it orders them.
    uint64_t m = 0;
#pragma unroll
    for (int s = 0; s < SH; ++s) m = tk[s][0] > m ? tk[s][0] : m;
    // maximum over groups of 4 lanes by DPP quad permutations (lanes 1,0,3,2, then 2,3,0,1): no LDS round trip
    m = quad_max_step<0xB1>(m);
    m = quad_max_step<0x4E>(m);
    if ((lane & 3) == 0) gmax[tid >> 2] = m;
    __syncthreads();  // (also orders the counters' reset before their first use)
    // The band's must rows open the candidate list (their count is final after the next barrier).
    {
        bool pm[kSelRows];
        int sm_[kSelRows];
#pragma unroll
        for (int j = 0; j < kSelRows; ++j) pm[j] = r0 + j < cb && mk[j] == 1;
        wave_append_n(pm, &n_m, sm_);
#pragma unroll
        for (int j = 0; j < kSelRows; ++j)
            if (sm_[j] >= 0) candl[sm_[j]] = r0 + j;
    }
    list_ranks(gmax, kSelThreads / 4, [&](int i, int rank) {
        if (rank == n_keep - 1) thr_sh = gmax[i];  // zero maxima rank below every nonzero one
        if (rank == 0) top_sh = gmax[i];
    });
    __syncthreads();
    // More keys than group maxima (uniform): the cut is the n_keep-th best published key instead (n_keep distinct keys
    // reach it; radix select over every share's published keys)
    const uint64_t L = n_keep <= kSelThreads / 4 ? thr_sh
                                                 : block_kth_threshold<kSelThreads>(
                                                       [&](auto visit) {
#pragma unroll
                                                           for (int s = 0; s < SH; ++s)
#pragma unroll
                                                               for (int r = 0; r < kTops; ++r) visit(tk[s][r]);
                                                       },
                                                       n_keep, rsh);
    const int nm = n_m;
    // The speculative candidates' cut, a sixteenth of the k-th best coarse score below it: for k = 1 the best key
    // overall, known here (the best group maximum); for k > 1 once the pool is ranked.
    auto cut_below = [](uint64_t kth) {
        if (kth == 0) return -__builtin_inff();
        const float c = key_score(kth);
        return c - (__builtin_fabsf(c) * 0.0625f + 1e-3f);
    };
    // The band's unmarked rows with upper >= cut follow the must rows in candl, their bounds in candu.
    auto spec_append = [&](float cut) {
        bool pc[kSelRows];
        int sc_[kSelRows];
#pragma unroll
        for (int j = 0; j < kSelRows; ++j) pc[j] = r0 + j < cb && mk[j] == 0 && up[j] >= cut;
        wave_append_n(pc, &n_c, sc_);
#pragma unroll
        for (int j = 0; j < kSelRows; ++j)
            if (sc_[j] >= 0) {
                candl[nm + sc_[j]] = r0 + j;
                candu[sc_[j]] = up[j];
            }
    };
    float cut = k == 1 ? cut_below(top_sh) : 0.0f;
    if (k == 1) spec_append(cut);  // in the pool's phase: no barrier of its own
    {
        bool pr[SH * kTops];
        int slot[SH * kTops];
#pragma unroll
        for (int s = 0; s < SH; ++s)
#pragma unroll
            for (int r = 0; r < kTops; ++r) pr[s * kTops + r] = tk[s][r] != 0 && tk[s][r] >= L;
        wave_append_n(pr, &n_pool, slot);
#pragma unroll
        for (int s = 0; s < SH; ++s)
#pragma unroll
            for (int r = 0; r < kTops; ++r)
                if (slot[s * kTops + r] >= 0 && slot[s * kTops + r] < kPoolCap) {
                    pool[slot[s * kTops + r]] = tk[s][r];
                    prow[slot[s * kTops + r]] = key_row(tk[s][r]);
                }
        bool pi[SH];
        int si[SH];
#pragma unroll
        for (int s = 0; s < SH; ++s) pi[s] = pr[s * kTops + kTops - 1];
        wave_append_n(pi, &inc.n, si);
#pragma unroll
        for (int s = 0; s < SH; ++s)
            if (si[s] >= 0 && si[s] < kMaxKeep) {
                inc.p[si[s]] = tid + s * kSelThreads;
                inc.below[si[s]] = tk[s][kTops - 1];
            }
    }
    __syncthreads();
    QH_HSTAMP(2, 0);
    if (inc.n > 0 && inc.n <= kMaxKeep) {  // uniform; rare: a share holding kTops of the keys >= L
        const int smax = sm.s1, n = inc.n * smax;
#pragma unroll 1
        for (int i0 = 0; i0 < n; i0 += kSelThreads) {  // uniform trip count: wave_append needs whole waves
            const int i = i0 + tid;
            uint64_t v = 0;
            if (i < n) {
                const int sh = i / smax, off = i - sh * smax;
                const int r = off < sm.len(inc.p[sh]) ? sm.start(inc.p[sh]) + off : nv;
                if (r < nv && mark[r] == 0) v = score_key(coarse[r], r);
                if (v >= inc.below[sh]) v = 0;  // published
            }
            const int slot = wave_append(v != 0 && v >= L, &n_pool);
            if (slot >= 0 && slot < kPoolCap) {
                pool[slot] = v;
                prow[slot] = key_row(v);
            }
        }
        __syncthreads();
    }
    if (n_pool > kPoolCap || inc.n > kMaxKeep) {  // uniform; a pathological tie structure
        // The exact n_keep-th best share maximum T (radix select), then the n_keep-th best key th over the rows of the
        // shares reaching T (radix select, streaming their rows), and the keys >= th.
        const uint64_t T = block_kth_threshold<kSelThreads>(
            [&](auto visit) {
#pragma unroll
                for (int s = 0; s < SH; ++s) visit(tk[s][0]);
            },
            n_keep, rsh);
#pragma unroll 1
        for (int s = 0; s < SH; ++s) {
            const int slot = wave_append(tk[s][0] != 0 && tk[s][0] >= T, &n_sel);  // at most n_keep shares
            if (slot >= 0) selp[slot] = tid + s * kSelThreads;
        }
        __syncthreads();
        const int smax = sm.s1, n = n_sel * smax;
        auto key_at = [&](int i) -> uint64_t {
            const int sh = i / smax, off = i - sh * smax;
            const int r = off < sm.len(selp[sh]) ? sm.start(selp[sh]) + off : nv;
            return (r < nv && mark[r] == 0) ? score_key(coarse[r], r) : 0ull;
        };
        const uint64_t th = block_kth_threshold<kSelThreads>(
            [&](auto visit) {
                for (int i = tid; i < n; i += kSelThreads) visit(key_at(i));
            },
            n_keep, rsh);
        if (tid == 0) n_pool = 0;
        __syncthreads();
        for (int i0 = 0; i0 < n; i0 += kSelThreads) {
            const int i = i0 + tid;
            const uint64_t v = i < n ? key_at(i) : 0ull;
            const int slot = wave_append(v != 0 && v >= th, &n_pool);  // exactly min(n_keep, eligible rows)
            if (slot >= 0) {
                pool[slot] = v;
                prow[slot] = key_row(v);
            }
        }
        __syncthreads();
    }
    const int np = n_pool;

    // 2. The seeds: the pool's n_seed best keys (model.cpp:295-304), rescored exactly (model.cpp:305-307); tau = the
    // k-th best exact seed logit (model.cpp:308-313). 3. The band's candidates {unmarked, not a seed, upper >= tau}
    // (model.cpp:315-322) and must rows, rescored exactly. The candidates are rescored in the seeds' pass, before tau
    // is known: every unmarked band row with upper >= cut (listed above: the cut sits a sixteenth below the k-th best
    // coarse score, and the k-th best exact seed logit is that score within its rounding error, whose bound is loose
    // but whose actual size is small), and once tau is known the rows with upper >= tau that are no seeds are kept. Rows with tau <= upper < cut
    // (tau below the cut, rare) take a second pass. For greedy queries a pool of up to two rescoring passes is rescored
    // whole in that pass and ranked while its loads are in flight, which keeps the ranking off the path.
    const bool early = k == 1 && np <= 2 * kRescoreRows;  // uniform
    auto rank_pool = [&]() {
        list_ranks(pool, np, [&](int i, int rank) {  // keys are unique
            if (rank < n_keep) {
                best[rank] = pool[i];
                if (rank < n_seed) {
                    seedrow[rank] = prow[i];
                    if (early) seedidx[rank] = i;
                }
            }
        });
        __syncthreads();
    };
    if (!early) rank_pool();
    if (k > 1) {
        cut = cut_below(best[k - 1]);
        spec_append(cut);
        __syncthreads();
    }
    const int nsp = n_c;  // candl: nm must rows, then nsp speculative candidates (at most band rows in all)
    const int na = early ? np : min(np, n_seed);
    // (early: the pool is ranked while the pass's loads are in flight)
    rescore_lists<PL>(early ? prow : seedrow, na, candl, nm + nsp, eh, xs, xds, nb, prod, rx, true, logits,
                      [&]() {
                          if (early) rank_pool();
                      });
    for (int i = tid; i < min(np, n_seed); i += kSelThreads) exact[i] = rx[early ? seedidx[i] : i];
    __syncthreads();
    QH_HSTAMP(2, 3);
    QH_HSTAMP(1, 1);
    int ns = 0;
    if (n_seed < kWaveKeep) {  // uniform
        if (wave == 0) {  // one lane per seed
            ns = __popcll(__ballot(lane < n_seed && best[lane] != 0));
            const bool have = lane < ns;
            const float e = have ? exact[lane] : -__builtin_inff();
            float t = -__builtin_inff();
            const uint64_t ks = wave_max_u64(have ? score_key(e, seedrow[lane]) : 0ull);
            if (k == 1) {  // the best exact seed logit
                if (ns >= 1) t = key_score(ks);
            } else if (ns >= k) {  // fewer than k seeds above it, k at or above
                int gt = 0, ge = 0;
                for (int j = 0; j < ns; ++j) {
                    const float ej = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), j));
                    gt += ej > e ? 1 : 0;
                    ge += ej >= e ? 1 : 0;
                }
                const uint64_t at = __ballot(have && gt < k && ge >= k);  // equal values wherever it is set
                t = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), __ffsll((long long)at) - 1));
            }
            if (lane == 0) {
                tau_sh = t;
                key_sh = ks;
                ns_sh = ns;
            }
        }
        __syncthreads();
    } else {
        // Many seeds (k > 55): the same over the workgroup. The ranked keys are nonzero first, so ns counts them; tau
        // is the exact logit with fewer than k seeds above it and k at or above (equal values wherever that holds).
        int have = 0;
        uint64_t ks = 0;
        for (int i = tid; i < n_seed; i += kSelThreads) {
            if (best[i] != 0) {
                ++have;
                const uint64_t kk = score_key(exact[i], seedrow[i]);
                ks = kk > ks ? kk : ks;
            }
        }
        have = wave_sum_int(have);
        ks = wave_max_u64(ks);
        if (lane == 0) {
            wsum[wave] = have;
            wkey[wave] = ks;
        }
        if (tid == 0) tau_sh = -__builtin_inff();
        __syncthreads();
        ns = 0;
        ks = 0;
#pragma unroll
        for (int w = 0; w < kSelWaves; ++w) {
            ns += wsum[w];
            ks = wkey[w] > ks ? wkey[w] : ks;
        }
        if (ns >= k)
            for (int i = tid; i < ns; i += kSelThreads) {
                const float e = exact[i];
                int gt = 0, ge = 0;
                for (int j = 0; j < ns; ++j) {
                    const float ej = exact[j];
                    gt += ej > e ? 1 : 0;
                    ge += ej >= e ? 1 : 0;
                }
                if (gt < k && ge >= k) tau_sh = e;
            }
        // the band's seed rows as bits, for the candidate filter below
        for (int i = tid; i < ns; i += kSelThreads) {
            const int r = seedrow[i];
            if (r >= ca && r < cb) atomicOr(&seedmap[(r - ca) >> 5], 1u << ((r - ca) & 31));
        }
        if (tid == 0) {
            key_sh = ks;
            ns_sh = ns;
        }
        __syncthreads();
    }
    const float tau = tau_sh;
    ns = ns_sh;
    if (blockIdx.x == 0)
        for (int i = tid; i < ns; i += kSelThreads) {
            rows[i] = seedrow[i];
            logits[seedrow[i]] = exact[i];
        }
    QH_HSTAMP(1, 2);
    // The kept candidates and the must rows: logits out, their best key.
    uint64_t kbest = 0;
    auto not_seed = [&](int r) {  // r is a row of the band
        if (n_seed >= kWaveKeep) return ((seedmap[(r - ca) >> 5] >> ((r - ca) & 31)) & 1u) == 0u;
        bool ok = true;
        for (int q = 0; q < ns; ++q) ok = ok && seedrow[q] != r;
        return ok;
    };
    for (int i0 = 0; i0 < nm + nsp; i0 += kSelThreads) {  // uniform trip count: wave_append needs whole waves
        const int i = i0 + tid;
        bool keep = false;
        int r = 0;
        if (i < nm + nsp) {
            r = candl[i];
            keep = i >= nm && candu[i - nm] >= tau && not_seed(r);
            if (keep || i < nm) {
                const float e = rx[na + i];
                logits[r] = e;
                const uint64_t kk = score_key(e, r);
                kbest = kk > kbest ? kk : kbest;
            }
        }
        const int slot = wave_append(keep, &n_cf);
        if (slot >= 0) candf[slot] = r;
    }
    if (tau < cut) {  // uniform; the rows between tau and the cut, in a pass of their own
#pragma unroll
        for (int j = 0; j < kSelRows; ++j) {
            const int r = r0 + j;
            const bool c = r < cb && mk[j] == 0 && up[j] >= tau && up[j] < cut && not_seed(r);
            const int slot = wave_append(c, &n_x);
            if (slot >= 0) mustl[slot] = r;
        }
        __syncthreads();
        const int nx = n_x;
        const uint64_t kb = rescore_lists<PL>(mustl, nx, candl, 0, eh, xs, xds, nb, prod, rx, false, logits);
        kbest = kb > kbest ? kb : kbest;
        for (int i0 = 0; i0 < nx; i0 += kSelThreads) {
            const int i = i0 + tid;
            const int slot = wave_append(i < nx, &n_cf);
            if (slot >= 0) candf[slot] = mustl[i];
        }
    }
    if (blockIdx.x == 0 && tid == 0) kbest = key_sh > kbest ? key_sh : kbest;  // the seeds' best key, once
    kbest = wave_max_u64(kbest);
    if (lane == 0) wkey[wave] = kbest;
    asm volatile("" ::"v"(mdep));  // the must minima have returned
    __syncthreads();
    const int nc = n_cf;
    QH_HSTAMP(1, 3);

    // 4. Completion. The candidates' slot request and the maximum go out together; both are performed (their old
    // values have returned) before the counts move, so the last workgroup's atomic reads see every maximum, every
    // count and every first occurrence. It reads nothing else another workgroup of this launch wrote, so no cache
    // write-back fence is needed; the candidate rows are written after the counts (nothing in this launch reads them).
    if (tid == 0) {
        uint64_t kw = wkey[0];
        for (int w = 1; w < kSelWaves; ++w) kw = wkey[w] > kw ? wkey[w] : kw;
        const int g = (int)(blockIdx.x % kDoneGroups);
        unsigned base = 0;
        unsigned long long old = 0;
        if (nc > 0) base = atomicAdd(&ctrl->n_cand, (unsigned)nc);
        if (kw) old = atomicMax(group_key(ctrl, g), (unsigned long long)kw);
        asm volatile("" ::"v"(base), "v"(old));
        base_sh = (int)base;
        const unsigned gsize = (gridDim.x - (unsigned)g + kDoneGroups - 1) / kDoneGroups;
        const bool group_last = atomicAdd(group_done(ctrl, g), 1u) == gsize - 1;
        const unsigned ngroups = gridDim.x < (unsigned)kDoneGroups ? gridDim.x : (unsigned)kDoneGroups;
        last_sh = group_last && atomicAdd(&ctrl->done, 1u) == ngroups - 1;
    }
    __syncthreads();
    for (int i = tid; i < nc; i += kSelThreads) rows[ns + base_sh + i] = candf[i];
    __syncthreads();
    if (!last_sh) return;
    if (wave == 0) {  // the group keys, one lane each, and the candidate count, all in flight at once
        const unsigned nc_all = __hip_atomic_load(&ctrl->n_cand, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint64_t v = __hip_atomic_load(group_key(ctrl, lane < kDoneGroups ? lane : 0), __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
        const uint64_t key = wave_max_u64(lane < kDoneGroups ? v : 0ull);
        if (lane == 0) {
            key_sh = key;
            n_cand_sh = (int)nc_all;
        }
    }
    __syncthreads();
    const int n_cand = n_cand_sh;
    // The must ids' first occurrences, valid (model.cpp:324-330: must ids are never seeds), after the candidates in
    // query order. Batches of kSelThreads * kMustBatch ids: each thread takes a run of up to kMustBatch, loads its ids
    // and then their first-occurrence words (every load in flight before the first wait), counts the occurrences that
    // won, and a block scan of the counts gives each run its place.
    int n_listed = 0;
    constexpr int kMustBatch = 16;
    for (int b0 = 0; b0 < n_must; b0 += kSelThreads * kMustBatch) {  // uniform
        const int bn = min(n_must - b0, kSelThreads * kMustBatch);
        const int per = (bn + kSelThreads - 1) / kSelThreads;
        const int i0 = b0 + min(bn, tid * per), i1 = b0 + min(bn, tid * per + per);
        int id[kMustBatch], fw[kMustBatch];
#pragma unroll
        for (int q = 0; q < kMustBatch; ++q) id[q] = must[min(i0 + q, n_must - 1)];
#pragma unroll
        for (int q = 0; q < kMustBatch; ++q)
            fw[q] = __hip_atomic_load(&firsts[min(max(id[q], 0), nv - 1)], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        unsigned wins = 0;  // bit q: occurrence i0 + q is its id's first
#pragma unroll
        for (int q = 0; q < kMustBatch; ++q)
            wins |= (i0 + q < i1 && id[q] >= 0 && id[q] < nv && fw[q] == i0 + q) ? 1u << q : 0u;
        const int c = __popc(wins);
        int incl = c;  // inclusive scan over the wave
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int o = __shfl_up(incl, off, 64);
            incl += lane >= off ? o : 0;
        }
        if (lane == 63) wsum[wave] = incl;
        __syncthreads();
        int before = 0, total = 0;
        for (int w = 0; w < kSelWaves; ++w) {
            before += w < wave ? wsum[w] : 0;
            total += wsum[w];
        }
        int o = ns + n_cand + n_listed + before + incl - c;
#pragma unroll
        for (int q = 0; q < kMustBatch; ++q)
            if (wins >> q & 1u) rows[o++] = id[q];
        n_listed += total;
        __syncthreads();  // wsum is read before the next batch writes it
    }
    if (tid == 0) {
        const uint64_t key = key_sh;
        stats->top1 = key_row(key);
        stats->top1_logit = key_score(key);
        stats->n_seeds = ns;
        stats->n_must = n_listed;
        stats->n_cand = n_cand;
        stats->n_rows = ns + n_cand + n_listed;
        stats->seed_tie =
            (ns == n_seed && best[n_seed] != 0 && (best[n_seed] >> 32) == (best[n_seed - 1] >> 32)) ? 1 : 0;
        stats->tau = tau;
        if (fb.token) fb.apply(key_row(key), true);
    }
}

// The nibble planes of a Q8_0 head, one 32-block per thread: q = 16 h + l with h = floor(q / 16) in [-8, 7] and
// l = q mod 16. A byte's high nibble u (as unsigned) gives h + 8 = u ^ 8, its low nibble is l; each plane keeps the
// Q4_0 packing (byte j: element j in the low nibble, element j + 16 in the high one).
__global__ __launch_bounds__(256) void head_planes_kernel(const uint8_t* __restrict__ q8, uint8_t* __restrict__ hi,
                                                          uint8_t* __restrict__ lo, long n_blocks) {
    const long b = (long)blockIdx.x * 256 + threadIdx.x;
    if (b >= n_blocks) return;
    const uint4 a = load16(q8 + b * QK), c = load16(q8 + b * QK + 16);
    auto hw = [](uint32_t x, uint32_t y) {
        return ((((x >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u) | ((((y >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u) << 4));
    };
    auto lw = [](uint32_t x, uint32_t y) { return (x & 0x0F0F0F0Fu) | ((y & 0x0F0F0F0Fu) << 4); };
    *reinterpret_cast<uint4*>(hi + b * 16) = make_uint4(hw(a.x, c.x), hw(a.y, c.y), hw(a.z, c.z), hw(a.w, c.w));
    *reinterpret_cast<uint4*>(lo + b * 16) = make_uint4(lw(a.x, c.x), lw(a.y, c.y), lw(a.z, c.z), lw(a.w, c.w));
}

// matvec_q over a nibble-plane head: rows [r0, r1), 256 per workgroup in passes of 32 through rescore_lists (8 lanes
// a row, every load of a pass in flight, then the row's serial chain acc = fma(float(s_b) * d_b, dx_b, acc)), so each
// value equals the Q8_0 GEMV's bit for bit. out is indexed by absolute row.
__global__ __launch_bounds__(kSelThreads) void gemv_planes_kernel(const uint8_t* __restrict__ hi,
                                                                  const uint8_t* __restrict__ lo,
                                                                  const uint16_t* __restrict__ sc,
                                                                  const int8_t* __restrict__ xq,
                                                                  const float* __restrict__ xd, int nb, int r0, int r1,
                                                                  float* __restrict__ out) {
    extern __shared__ __align__(16) float ssm[];  // products [32][nb], activation codes, scales, block sums
    float* prod = ssm;
    int8_t* xs = reinterpret_cast<int8_t*>(ssm + kRescoreRows * nb);
    float* xds = reinterpret_cast<float*>(xs + nb * QK);
    int* sxs = reinterpret_cast<int*>(xds + nb);
    __shared__ int list[kSelThreads];
    const int tid = (int)threadIdx.x, ra = r0 + (int)blockIdx.x * kSelThreads;
    for (int i = tid; i < nb * 2; i += kSelThreads) reinterpret_cast<uint4*>(xs)[i] = load16(xq + (size_t)i * 16);
    for (int b = tid; b < nb; b += kSelThreads) {
        xds[b] = xd[b];
        int sum = 0;
        for (int i = 0; i < QK; ++i) sum += xq[b * QK + i];
        sxs[b] = sum;
    }
    list[tid] = ra + tid;
    __syncthreads();
    const ExactHead eh{hi, lo, sc, sxs};
    rescore_lists<true>(list, min(kSelThreads, r1 - ra), list, 0, eh, xs, xds, nb, prod, nullptr, false, out);
}

hipError_t launch_gemv_planes(float* out, const qh_tensor& planes, const int8_t* xq, const float* xd, int r0, int r1,
                              hipStream_t s) {
    if (r1 <= r0) return hipSuccess;
    const int V = planes.rows, D = planes.cols, nb = D / QK;
    const uint8_t* hi = static_cast<const uint8_t*>(planes.data);
    const uint8_t* lo = hi + (size_t)V * D / 2;
    const uint16_t* sc = reinterpret_cast<const uint16_t*>(hi + (size_t)V * D);
    const size_t lds = (size_t)kRescoreRows * nb * 4 + (size_t)nb * QK + (size_t)nb * 8;
    qh_launch(gemv_planes_kernel, dim3((unsigned)((r1 - r0 + kSelThreads - 1) / kSelThreads)), dim3(kSelThreads), lds,
              s, hi, lo, sc, xq, xd, nb, r0, r1, out);
    return hipGetLastError();
}

hipError_t launch_head_planes(const void* head8, void* planes, int V, int D, hipStream_t s) {
    const size_t n = (size_t)V * D;
    const long nblk = (long)(n / QK);
    uint8_t* out = static_cast<uint8_t*>(planes);
    qh_launch(head_planes_kernel, dim3((unsigned)((nblk + 255) / 256)), dim3(256), 0, s,
              static_cast<const uint8_t*>(head8), out, out + n / 2, nblk);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return hipMemcpyAsync(out + n, static_cast<const uint8_t*>(head8) + n, n / QK * 2, hipMemcpyDeviceToDevice, s);
}

bool head_select_supported(int V, int D, int top_k) {
    return top_k >= 1 && top_k <= QH_HEAD_MAX_TOPK && screen_shape(V, D / QK).grid <= kSelShares * kSelThreads;
}

size_t head_workspace_bytes(int V, int D, int top_k) {
    return head_select_supported(V, D, top_k) ? ws_layout(V, D).total : 0;
}

bool head_shape_supported(int D) { return D % 64 == 0 && D <= kMaxHeadCols; }

hipError_t launch_shortlist_head(const qh_tensor& head8, const qh_tensor& head4, const qh_tensor& err,
                                 const int8_t* xq, const float* xd, const qh_head_query& q, const HeadMust& must,
                                 const qh_head_out& out, void* ws, hipStream_t s, const TokenFeedback* advance) {
    const int V = head8.rows, D = head8.cols, nb = D / QK;
    if (must.n > kMaxMust || !head_shape_supported(D) || !head_select_supported(V, D, q.top_k))
        return hipErrorInvalidValue;
    const int nv = (q.n_valid > 0 && q.n_valid < V) ? q.n_valid : V;
    const WsLayout l = ws_layout(V, D);
    uint8_t* wsb = static_cast<uint8_t*>(ws);
    uint8_t* mark = wsb + l.mark;
    int32_t* firsts = reinterpret_cast<int32_t*>(wsb + l.first);
    uint64_t* tops = reinterpret_cast<uint64_t*>(wsb + l.tops);
    HeadCtrl* ctrl = reinterpret_cast<HeadCtrl*>(wsb + l.ctrl);
    // The nibble-plane head (QH_Q8_0_PLANES) screens with its high plane and rescores from both planes; head4 and err
    // are not read then.
    const bool pl = head8.dtype == QH_Q8_0_PLANES;
    const uint8_t* w8 = static_cast<const uint8_t*>(head8.data);
    const uint16_t* s8 = reinterpret_cast<const uint16_t*>(w8 + qh_quant_bytes(QH_Q8_0, V, D));
    const uint8_t* lo = pl ? w8 + (size_t)V * D / 2 : nullptr;
    const uint8_t* w4 = pl ? w8 : static_cast<const uint8_t*>(head4.data);
    const uint16_t* s4 = pl ? s8 : reinterpret_cast<const uint16_t*>(w4 + qh_quant_bytes(QH_Q4_0, V, D));
    const uint32_t* e32 = pl ? nullptr : static_cast<const uint32_t*>(err.data);

    const ScreenShape sh = screen_shape(V, nb);
    const int tile = sh.tile;
    const uint32_t magic = nb == 1 ? 0u : (uint32_t)((0x100000000ull + (uint64_t)nb - 1) / (uint64_t)nb);
    const size_t lds1 = ((size_t)2 * chain_len32(nb) + 4 * (size_t)tile * chain_stride32(nb) + kChainPipePad + 128) * 4 +
                        kScreenMaxShare + (size_t)D + (pl ? (size_t)nb * 4 : 0);
    qh_launch(pl ? head_screen_kernel<true> : head_screen_kernel<false>, dim3(sh.grid), dim3(kScreenThreads), lds1, s,
              w4, s4, e32, xq, xd, V, nb, nv, must, tile, sh.map, magic, out.coarse, out.upper, out.logits, mark, firsts,
              tops, ctrl);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int band = select_band(nv);
    const size_t lds2 = (size_t)kRescoreRows * nb * 4 + (size_t)nb * QK + (size_t)nb * 4 + (pl ? (size_t)nb * 4 : 0);
    auto* sel = sh.grid <= 2 * kSelThreads ? (pl ? head_select_kernel<2, true> : head_select_kernel<2, false>)
                                           : (pl ? head_select_kernel<kSelShares, true> : head_select_kernel<kSelShares, false>);
    qh_launch(sel, dim3((unsigned)((nv + band - 1) / band)), dim3(kSelThreads), lds2, s, w8, lo, s8, xq, xd, nb, nv,
              q.top_k, sh.grid, sh.map, band, tops, out.coarse, out.upper, mark, firsts, must, out.rows, out.logits,
              ctrl, out.stats, advance ? *advance : TokenFeedback{});
    return hipGetLastError();
}

}  // namespace qh
