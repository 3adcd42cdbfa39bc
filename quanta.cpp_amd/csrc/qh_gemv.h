// One workgroup's tile of the Q8_0 / Q4_0 integer-dot GEMV (reference ops_ref.cpp:85-120), shared by the plain
// GEMV kernel and the decoder's fused kernels (projection + residual + norm, gate/up + SwiGLU).
//
// A tile is a run of consecutive rows; in the .qnt layout their quants are one contiguous byte range, streamed
// with coalesced 16-byte loads (thread t takes chunks t, t+256, ...). A Q8_0 block is two chunks (a lane pair,
// combined with one DPP swap), a Q4_0 block is one chunk. Each block's exact int32 dot becomes
// p = float(s) * f16(scale) (one rounded multiply) parked in LDS at [row][block]; after one barrier, thread r runs
// row r's serial chain acc = fma(p_b, dx_b, acc) over the blocks in order, which is the reference's float
// association, so the result is bit-identical. Every load of a pass is issued before the first wait; longer tiles
// prefetch the next pass while computing the current one.
//
// A tile may span NSEG segments of equal row count from up to three matrices of one dtype and width (gate and up;
// one head's q, k and v rows): virtual rows [s*n, (s+1)*n) come from segment s, so one round trip covers them all.
#pragma once

#include <limits.h>

#include "qh_device.h"

namespace qh {

// Per-workgroup timeline stamps of the decode GEMV kernels, compiled in only with -DQH_TIMELINE: thread 0 of each
// workgroup records the constant-rate real-time clock ([kernel][workgroup < 1024][stamp < 6]; each translation unit
// has its own array, read out by the decoder's qh_timeline_wg_read).
#if defined(QH_TIMELINE)
static __device__ uint64_t qh_tl_wg[8][1024][6];
#define QH_WSTAMP(k, i)                                                                                     \
    do {                                                                                                    \
        if ((k) >= 0 && threadIdx.x == 0 && blockIdx.x < 1024 && blockIdx.y == 0)                          \
            qh_tl_wg[(k)][blockIdx.x][(i)] = __builtin_amdgcn_s_memrealtime();                              \
    } while (0)
#else
#define QH_WSTAMP(k, i) \
    do {                \
    } while (0)
#endif

// One pass of a workgroup: U chunks of 16 bytes per thread, the block scale of each chunk and, unless the
// activation is staged in LDS (XL), the activation bytes the chunk pairs with. The chunk index is clamped
// into the tile, so every load is unconditional and all of them go out back to back.
// Tile sources: segment s starts at row 0 of w[s] / sc[s] (the caller offsets them to the tile's first row).
template <int NSEG>
struct GemvSegs {
    const uint8_t* w[NSEG];
    const uint16_t* sc[NSEG];
};

template <int DT, int U, bool XL, int NSEG = 1>
struct GemvPass {
    uint4 w[U];
    uint4 xa[XL ? 1 : U];
    uint4 xb[(XL || DT == kQ8) ? 1 : U];
    uint16_t sc[U];
    uint32_t rt[U], b[U];

    // split: chunks per segment (NSEG > 1).
    __device__ __forceinline__ void load(const GemvSegs<NSEG>& sg, int split, const int8_t* __restrict__ xq, int c0,
                                         int last, int nb, uint32_t nb_magic) {
        constexpr int kChunksPerBlock = DT == kQ8 ? 2 : 1;
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const int c = min(c0 + j * 256 + (int)threadIdx.x, last);
            const uint32_t g = (uint32_t)c / kChunksPerBlock;  // block index within the tile
            rt[j] = nb == 1 ? g : div_magic(g, nb_magic);      // tile row
            b[j] = g - rt[j] * (uint32_t)nb;                    // block within the row
            if constexpr (NSEG > 1) {
                const int s1 = c >= split, s2 = NSEG > 2 && c >= 2 * split;
                const int cc = c - (s1 + s2) * split;
                const uint8_t* wb = s2 ? sg.w[NSEG - 1] : s1 ? sg.w[1] : sg.w[0];
                const uint16_t* sb = s2 ? sg.sc[NSEG - 1] : s1 ? sg.sc[1] : sg.sc[0];
                w[j] = load16(wb + (size_t)cc * 16);
                sc[j] = sb[(uint32_t)cc / kChunksPerBlock];
            } else {
                w[j] = load16(sg.w[0] + (size_t)c * 16);
                sc[j] = sg.sc[0][g];
            }
            if constexpr (!XL) {
                if constexpr (DT == kQ8) {
                    xa[j] = load16(xq + b[j] * QK + (c & 1) * 16);
                } else {
                    xa[j] = load16(xq + b[j] * QK);
                    xb[j] = load16(xq + b[j] * QK + 16);
                }
            }
        }
    }

    // Block products of the pass into LDS (only chunks below nchunks are stored). xs: LDS activation (XL).
    __device__ __forceinline__ void products(float* prod, int pstride, int c0, int nchunks, const int8_t* xs) const {
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const int c = c0 + j * 256 + (int)threadIdx.x;
            if constexpr (DT == kQ8) {
                const uint4 xv = XL ? *reinterpret_cast<const uint4*>(xs + b[j] * QK + (c & 1) * 16) : xa[XL ? 0 : j];
                int s = dot16_i8(w[j], xv);
                s += swap_pair(s);
                if (c < nchunks && !(c & 1)) prod[rt[j] * pstride + b[j]] = (float)s * f16_to_f32(sc[j]);
            } else {
                const uint4 xlo = XL ? *reinterpret_cast<const uint4*>(xs + b[j] * QK) : xa[XL ? 0 : j];
                const uint4 xhi = XL ? *reinterpret_cast<const uint4*>(xs + b[j] * QK + 16) : xb[XL ? 0 : j];
                const int s = dot_q4_block(w[j], xlo, xhi);
                if (c < nchunks) prod[rt[j] * pstride + b[j]] = (float)s * f16_to_f32(sc[j]);
            }
        }
    }
};

// LDS floats of a tile before the staged codes: activation scales and block products as padded chain rows
// (chain_lds_pipe: [chain_len32(nb)] scales, then [tile_rows][chain_stride32(nb)] products) and the chain's read
// slack.
__host__ __device__ __forceinline__ size_t gemv_tile_lds_floats(int nb, int tile_rows) {
    return (size_t)chain_len32(nb) + (size_t)tile_rows * chain_stride32(nb) + kChainPipePad;
}

// LDS bytes of a tile of tile_rows virtual rows (PAIR tiles count both matrices' rows).
__host__ __device__ __forceinline__ size_t gemv_tile_lds_bytes(int cols, int tile_rows, bool xl) {
    const size_t f = gemv_tile_lds_floats(cols / QK, tile_rows) * 4;
    return xl ? f + (size_t)cols : f;
}

// The serial row chain acc = fma(p_b, dx_b, acc) for b in [0, nb) (nb % 4 == 0, nb >= 32) with the products p from
// LDS (16-byte aligned) and the activation scales dx as scalar operands straight from global memory (dx uniform across
// the wave, 4-byte aligned, nothing in the kernel writes it): per 32 blocks, two 64-byte scalar loads and eight
// 16-byte LDS reads instead of sixteen LDS reads, so a long chain runs at the FMA latency (chain_lds_pipe is bound by
// its LDS read issue: ~13 cycles per block at 152 blocks). Scalar loads return out of order, so each batch waits for
// everything outstanding, the next batch being issued right after that wait; the last batch is read from
// dx + nb - 32, so nothing past dx + nb is read. Every lane of the wave calls it (lanes without a row ignore the result).
typedef float gv16f __attribute__((ext_vector_type(16)));
typedef const __attribute__((address_space(4))) gv16f* const_gv16f_ptr;
__device__ __forceinline__ void gemv_wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xc07f); }  // lgkmcnt(0) only
__device__ __forceinline__ float chain_lds_sdx(const float* p, const float* dx, int nb) {
    struct Batch {
        gv16f d0, d1;
        float4 q[8];
    };
    const int nfull = nb & ~31;  // blocks in whole batches of 32
    auto ld = [&](Batch& bt, int b) {  // b: a whole batch's start, or the tail's nb - 32
        const const_gv16f_ptr d = (const_gv16f_ptr)(dx + b);
        bt.d0 = d[0];
        bt.d1 = d[1];
#pragma unroll
        for (int i = 0; i < 8; ++i) bt.q[i] = *reinterpret_cast<const float4*>(p + b + 4 * i);
    };
    float acc = 0.0f;
    auto use = [&](const Batch& bt, int from) {  // blocks from .. 31 of the batch (from uniform, a multiple of 4)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (4 * i < from) continue;
            const gv16f& d = i < 4 ? bt.d0 : bt.d1;
            const int o = (4 * i) & 15;
            acc = __builtin_fmaf(bt.q[i].x, d[o], acc);
            acc = __builtin_fmaf(bt.q[i].y, d[o + 1], acc);
            acc = __builtin_fmaf(bt.q[i].z, d[o + 2], acc);
            acc = __builtin_fmaf(bt.q[i].w, d[o + 3], acc);
        }
    };
    Batch A, B;
    ld(A, nfull > 0 ? 0 : nb - 32);
    int b = 0;
#pragma unroll 1
    for (; b + 64 <= nfull; b += 64) {
        gemv_wait_lgkm0();
        __builtin_amdgcn_sched_barrier(0);
        ld(B, b + 32);
        __builtin_amdgcn_sched_barrier(0);
        use(A, 0);
        gemv_wait_lgkm0();
        __builtin_amdgcn_sched_barrier(0);
        ld(A, b + 64 < nfull ? b + 64 : nb - 32);
        __builtin_amdgcn_sched_barrier(0);
        use(B, 0);
    }
    gemv_wait_lgkm0();
    __builtin_amdgcn_sched_barrier(0);
    if (b < nfull) {  // one whole batch left in A, then the tail (if any)
        if (nfull < nb) ld(B, nb - 32);
        __builtin_amdgcn_sched_barrier(0);
        use(A, 0);
        if (nfull < nb) {
            gemv_wait_lgkm0();
            __builtin_amdgcn_sched_barrier(0);
            use(B, 32 - (nb - nfull));
        }
    } else if (nfull < nb) {  // A holds the tail
        use(A, 32 - (nb - nfull));
    }
    return acc;
}

// Stages the activation for a tile: its block scales into xds and, when the codes are read from LDS (XL), its codes
// into xs, straight from the quantized activation in global memory: begin() issues the first loads (ahead of the
// tile's weight loads), fill() stores them and loads the rest.
struct GlobalAct {
    static constexpr bool kGlobalScales = true;  // xd holds the scales in global memory (scalar-operand chains)
    const int8_t* __restrict__ xq;
    const float* __restrict__ xd;
    int nb;
    struct Pre {
        uint4 xv;
        float dv;
    };
    template <bool XL>
    __device__ __forceinline__ Pre begin() const {
        const int tid = (int)threadIdx.x, xch = nb * QK / 16;
        Pre p{make_uint4(0u, 0u, 0u, 0u), 0.0f};
        if constexpr (XL) p.xv = load16(xq + min(tid, xch - 1) * 16);
        p.dv = xd[min(tid, nb - 1)];
        return p;
    }
    template <bool XL>
    __device__ __forceinline__ void fill(const Pre& p, int8_t* xs, float* xds) const {
        const int tid = (int)threadIdx.x, xch = nb * QK / 16;
        if (XL && tid < xch) reinterpret_cast<uint4*>(xs)[tid] = p.xv;
        if (tid < nb) xds[tid] = p.dv;
        if constexpr (XL)
            for (int i = tid + 256; i < xch; i += 256) reinterpret_cast<uint4*>(xs)[i] = load16(xq + i * 16);
        for (int i = tid + 256; i < nb; i += 256) xds[i] = xd[i];
    }
};

// nrows rows of each of the NSEG segments of sg . x, for one workgroup of 256 threads: virtual row v is row v % nrows
// of segment v / nrows. tile_rows: the virtual row capacity the LDS layout is sized for (>= NSEG * nrows). Returns
// the value of virtual row threadIdx.x for threads below NSEG * nrows, 0 for the others. smem: dynamic LDS of
// gemv_tile_lds_bytes(nb * 32, tile_rows, XL) bytes. act.begin<XL>() issues the activation's first loads, before the
// first pass of weight loads; act.fill<XL>(pre, xs, xds) then stages the activation (codes in LDS when XL; it may use
// its own barriers, all 256 threads call it); xq / xd are read per chunk when !XL. The LDS is free for reuse only
// after a barrier.
template <int DT, int U, bool XL, int NSEG = 1, typename Act = GlobalAct>
__device__ __forceinline__ float gemv_tile(const GemvSegs<NSEG>& sg, const int8_t* __restrict__ xq,
                                           const float* __restrict__ xd, int nb, int nrows, int tile_rows,
                                           uint32_t nb_magic, float* smem, const Act& act, int tlk = -1) {
    (void)tlk;
    constexpr int kChunksPerBlock = DT == kQ8 ? 2 : 1;
    const int L = chain_len32(nb), zp = L - nb, pstride = chain_stride32(nb);
    float* dxs = smem;                          // [L] activation scales, zp zeros first
    float* xds = dxs + zp;
    float* prod = smem + L;                     // [tile_rows][pstride] block products, zp zeros first per row
    int8_t* xs = reinterpret_cast<int8_t*>(smem + gemv_tile_lds_floats(nb, tile_rows));  // [cols] codes (XL)
    const int tid = (int)threadIdx.x;
    const int vrows = NSEG * nrows;
    const int nchunks = vrows * nb * kChunksPerBlock;
    const int split = nrows * nb * kChunksPerBlock;

    const auto pre = act.template begin<XL>();  // the activation's loads go out first: the products wait for them
    GemvPass<DT, U, XL, NSEG> cur;
    cur.load(sg, split, xq, 0, nchunks - 1, nb, nb_magic);
    // The scalar-operand chain's scales: one scalar load per 64-byte line into the scalar cache, on the chain's wave,
    // while the weights stream.
    constexpr int kWarm = 16;
    uint32_t warm[kWarm];
    bool warmed = false;
    if constexpr (Act::kGlobalScales) {
        warmed = nb >= 64 && (nb & 3) == 0 && NSEG * nrows <= 64;
        if (warmed && tid < 64) {
            const __attribute__((address_space(4))) uint32_t* q = (const __attribute__((address_space(4))) uint32_t*)act.xd;
#pragma unroll
            for (int i = 0; i < kWarm; ++i) warm[i] = q[min(i * 16, nb - 1)];
        }
    }
    act.template fill<XL>(pre, xs, xds);
    zero_chain_prefix(dxs, prod, nb, vrows);
    if constexpr (XL) __syncthreads();
    QH_WSTAMP(tlk, 1);
    float* prow = prod + zp;
    if (nchunks <= 256 * U) {  // uniform: a single pass
        cur.products(prow, pstride, 0, nchunks, xs);
    } else {
        for (int c0 = 0; c0 < nchunks; c0 += 256 * U) {
            if (c0 + 256 * U < nchunks) {  // uniform: prefetch the next pass, then compute this one
                GemvPass<DT, U, XL, NSEG> nxt;
                nxt.load(sg, split, xq, c0 + 256 * U, nchunks - 1, nb, nb_magic);
                cur.products(prow, pstride, c0, nchunks, xs);
                cur = nxt;
            } else {
                cur.products(prow, pstride, c0, nchunks, xs);
            }
        }
    }
    QH_WSTAMP(tlk, 2);
    if constexpr (Act::kGlobalScales) {
        if (warmed && tid < 64) {  // the warm-up loads are held until here, so they cannot be dropped
            asm volatile("" ::"s"(warm[0]), "s"(warm[1]), "s"(warm[2]), "s"(warm[3]), "s"(warm[4]), "s"(warm[5]),
                         "s"(warm[6]), "s"(warm[7]));
            asm volatile("" ::"s"(warm[8]), "s"(warm[9]), "s"(warm[10]), "s"(warm[11]), "s"(warm[12]), "s"(warm[13]),
                         "s"(warm[14]), "s"(warm[15]));
        }
    }
    __syncthreads();
    if constexpr (Act::kGlobalScales) {
        // Long rows: the scalar-operand chain, on the wave holding the row lanes (vrows <= 64, uniform).
        if (warmed) {
            if (tid >= 64) return 0.0f;
            const float v = chain_lds_sdx(prod + min(tid, vrows - 1) * pstride + zp, act.xd, nb);
            return tid < vrows ? v : 0.0f;
        }
    }
    return tid < vrows ? chain_lds_pipe(prod + tid * pstride, dxs, L) : 0.0f;
}

// Rows [ra, ra + nrows) of one matrix, activation from global memory.
template <int DT, int U, bool XL>
__device__ __forceinline__ float gemv_tile(const uint8_t* __restrict__ wq, const uint16_t* __restrict__ wscale,
                                           const int8_t* __restrict__ xq, const float* __restrict__ xd, int nb,
                                           int ra, int nrows, int tile_rows, uint32_t nb_magic, float* smem,
                                           int tlk = -1) {
    constexpr int kBlockBytes = DT == kQ8 ? QK : QK / 2;
    const GemvSegs<1> sg{{wq + (size_t)ra * nb * kBlockBytes}, {wscale + (size_t)ra * nb}};
    return gemv_tile<DT, U, XL, 1>(sg, xq, xd, nb, nrows, tile_rows, nb_magic, smem, GlobalAct{xq, xd, nb}, tlk);
}

}  // namespace qh
