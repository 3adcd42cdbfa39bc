// Prefill matmul for n tokens (reference ops_ref.cpp:122-160, contract ops.h:65-70) on gfx950 int8 MFMA.
//
// v_mfma_i32_16x16x32_i8 takes K = 32 per instruction, exactly one Q8_0 / Q4_0 block, so every block's exact
// int32 dot s(row, token, b) comes out on its own. The per-(row, token) f32 chain acc = fma(float(s) * dw_b, dx_b,
// acc) then runs in block order in one thread, so each output equals the decode GEMV bit for bit. (The K = 64
// forms would merge two scale blocks.)
//
// Workgroup: 16 consecutive rows x 16*TT tokens, all of K, in chunks of KC blocks.
//  * MFMA phase: wave w takes blocks [w*KC/4, (w+1)*KC/4) of the chunk for all TT token tiles (the weight
//    operand is loaded once and reused across the tiles) and parks the int32 sums in LDS as s[block][row][token];
//    the chunk's row scales (f16 -> f32) and token scales go to LDS beside them.
//  * chain phase: each thread owns TT (row, token) pairs (one token, TT rows) and advances their chains over the
//    chunk's blocks. The chains live in registers across chunks, so LDS only ever holds one chunk.
//  * two register sets alternate in straight-line halves: the operands of chunk c+1 are loaded before chunk c is
//    reduced, and the loads of the steady-state loop are unconditional (the tail is peeled).
// Operand layout of one MFMA (block b): lane l supplies row (l % 16) / token (l % 16) and k-group (l / 16) as 8 int8
// values; Q4_0 nibbles are unpacked in registers (k-groups 0, 1 take the low nibbles of bytes 0-7 / 8-15, k-groups
// 2, 3 the high ones). Result register i of lane l is row 4*(l/16)+i, token l%16.
// Workgroups that share a row tile (different token groups) are numbered so that they land on the same XCD
// (workgroups are dealt to the 8 XCDs round-robin), where the weights they all read stay in that XCD's L2.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "qh_device.h"
#include "qh_internal.h"

namespace qh {

namespace {

constexpr int kMmThreads = 256;  // 4 waves
constexpr int kXcds = 8;

template <int TT, int KC>
struct MmShape {
    static constexpr int kTok = 16 * TT;           // tokens per workgroup
    static constexpr int kTokPad = kTok + 4;       // LDS row stride: the 4 row groups of one MFMA store hit different banks
    static constexpr int kBpw = KC / 4;            // blocks per wave per chunk
    static constexpr int kDxPer = kTok * KC / kMmThreads;  // token scales each thread stages per chunk
    static_assert(KC % 4 == 0 && (kTok * KC) % kMmThreads == 0 && 16 * KC <= kMmThreads, "chunk shape");
};

template <int DT, int TT, int KC>
struct MmRegs {
    using S = MmShape<TT, KC>;
    long a[S::kBpw];          // weight bytes of the wave's blocks (Q4_0: packed, unpacked at use)
    long x[S::kBpw][TT];      // activation operand per block and token tile
    float dx[S::kDxPer];      // staged token scales
    uint16_t dw;              // staged row scale (threads < 16 * KC)
};

}  // namespace

// Up to three matrices of one dtype and width, same activation, in one launch (q / k / v, gate / up): their row tiles
// are numbered one after another, segment s covering rows [r0[s], r1[s]) of its matrix and writing its output rows to
// out[s][token * ldo[s] + row].
struct MmSegs {
    const uint8_t* wq[3];
    const uint16_t* ws[3];
    float* out[3];
    int ldo[3], r0[3], r1[3];
    int tiles[3];  // row tiles of 16 per segment (0 for unused ones)
};

// The segment of row tile rt (launch-wide numbering) and its matrix, rows and output; rt becomes the tile's index
// within the segment. Uniform per workgroup: all of it stays in scalar registers.
struct MmSeg {
    const uint8_t* wq;
    const uint16_t* ws;
    float* out;
    int ldo, r0, r1;
    __device__ __forceinline__ MmSeg(const MmSegs& sg, int& rt) {
        int s = 0;
        if (rt >= sg.tiles[0]) {
            rt -= sg.tiles[0];
            s = 1;
            if (rt >= sg.tiles[1]) {
                rt -= sg.tiles[1];
                s = 2;
            }
        }
        wq = s == 0 ? sg.wq[0] : s == 1 ? sg.wq[1] : sg.wq[2];
        ws = s == 0 ? sg.ws[0] : s == 1 ? sg.ws[1] : sg.ws[2];
        out = s == 0 ? sg.out[0] : s == 1 ? sg.out[1] : sg.out[2];
        ldo = s == 0 ? sg.ldo[0] : s == 1 ? sg.ldo[1] : sg.ldo[2];
        r0 = s == 0 ? sg.r0[0] : s == 1 ? sg.r0[1] : sg.r0[2];
        r1 = s == 0 ? sg.r1[0] : s == 1 ? sg.r1[1] : sg.r1[2];
    }
};

template <int DT, int TT, int KC>
__global__ __launch_bounds__(kMmThreads) void matmul_lds_kernel(MmSegs segs, const int8_t* __restrict__ xq,
                                                            const float* __restrict__ xd, int cols, int n, int n_tg) {
    using S = MmShape<TT, KC>;
    constexpr int kTok = S::kTok, kTokPad = S::kTokPad, kBpw = S::kBpw;
    __shared__ int sl[KC][16][kTokPad];     // int32 block sums
    __shared__ float dxs[kTok][KC + 1];     // token scales of the chunk
    __shared__ float dws[16][KC + 1];       // row scales of the chunk (f32)
    const int nb = cols / QK;
    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lq = lane >> 4;

    // XCD-aware numbering: physical workgroup p runs on XCD p % 8; logical tiles [start(x), start(x+1)) go to XCD x.
    const int G = (int)gridDim.x, p = (int)blockIdx.x;
    const int xcd = p % kXcds, per = G / kXcds, rem = G % kXcds;
    const int logical = xcd * per + min(xcd, rem) + p / kXcds;
    int rt = logical / n_tg;
    const int tg = logical % n_tg;
    const MmSeg sg(segs, rt);
    const uint8_t* __restrict__ wq = sg.wq;
    const uint16_t* __restrict__ wscale = sg.ws;
    float* __restrict__ out = sg.out;
    const int ldo = sg.ldo, r0 = sg.r0, r1 = sg.r1;
    const int rbase = r0 + rt * 16, tbase = tg * kTok;

    // MFMA operands: row (rbase + li) for the weights, tokens (tbase + tt*16 + li) for the activations; rows and
    // tokens past the end are clamped for loading and never stored.
    const int arow = min(rbase + li, r1 - 1);
    const uint8_t* wrow;
    int shift = 0;
    if (DT == kQ8) {
        wrow = wq + (size_t)arow * cols + lq * 8;
    } else {
        wrow = wq + (size_t)arow * (cols / 2) + (lq & 1) * 8;
        shift = (lq >> 1) * 4;
    }
    const int8_t* xrow[TT];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) xrow[tt] = xq + (size_t)min(tbase + tt * 16 + li, n - 1) * cols + lq * 8;
    // Staging of the chunk scales: token scale e = j*256 + tid is (token e / KC, block e % KC); row scale tid is
    // (row tid / KC, block tid % KC) for tid < 16 * KC.
    const int dw_row = min(rbase + (tid / KC) % 16, r1 - 1);

    auto load = [&](MmRegs<DT, TT, KC>& R, int c0) {
#pragma unroll
        for (int i = 0; i < kBpw; ++i) {
            const int b = min(c0 + wave * kBpw + i, nb - 1);
            R.a[i] = *reinterpret_cast<const long*>(wrow + (size_t)b * (DT == kQ8 ? QK : QK / 2));
#pragma unroll
            for (int tt = 0; tt < TT; ++tt) R.x[i][tt] = *reinterpret_cast<const long*>(xrow[tt] + (size_t)b * QK);
        }
#pragma unroll
        for (int j = 0; j < S::kDxPer; ++j) {
            const int e = j * kMmThreads + tid;
            const int t = min(tbase + e / KC, n - 1), b = min(c0 + e % KC, nb - 1);
            R.dx[j] = xd[(size_t)t * nb + b];
        }
        R.dw = wscale[(size_t)dw_row * nb + min(c0 + tid % KC, nb - 1)];
    };

    // Chain pairs of this thread: token ctok, rows crow(j) = j * (256 / kTok) + tid / kTok.
    const int ctok = tid % kTok;
    float acc[TT];
#pragma unroll
    for (int j = 0; j < TT; ++j) acc[j] = 0.0f;

    auto reduce = [&](const MmRegs<DT, TT, KC>& R, int c0) {
#pragma unroll
        for (int i = 0; i < kBpw; ++i) {
            const int bl = wave * kBpw + i;
            long a = R.a[i];
            if (DT == kQ4) {
                const uint64_t v = (uint64_t)a;
                const uint32_t lo = nibbles_to_i8(((uint32_t)v >> shift) & 0x0F0F0F0Fu);
                const uint32_t hi = nibbles_to_i8(((uint32_t)(v >> 32) >> shift) & 0x0F0F0F0Fu);
                a = (long)(((uint64_t)hi << 32) | lo);
            }
#pragma unroll
            for (int tt = 0; tt < TT; ++tt) {
                v4i c = {0, 0, 0, 0};
                c = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, R.x[i][tt], c, 0, 0, 0);
#pragma unroll
                for (int k = 0; k < 4; ++k) sl[bl][4 * lq + k][tt * 16 + li] = c[k];
            }
        }
#pragma unroll
        for (int j = 0; j < S::kDxPer; ++j) {
            const int e = j * kMmThreads + tid;
            dxs[e / KC][e % KC] = R.dx[j];
        }
        if (tid < 16 * KC) dws[tid / KC][tid % KC] = f16_to_f32(R.dw);
        __syncthreads();
        // The chunk's operands are read first (the loop is unrolled, so the LDS reads overlap), then the chains
        // advance block by block; blocks past the end of the row leave them unchanged.
        const int nblk = min(KC, nb - c0);
        float dxv[KC], pv[KC][TT];
#pragma unroll
        for (int k = 0; k < KC; ++k) {
            dxv[k] = dxs[ctok][k];
#pragma unroll
            for (int j = 0; j < TT; ++j) {
                const int row = j * (kMmThreads / kTok) + tid / kTok;
                pv[k][j] = (float)sl[k][row][ctok] * dws[row][k];
            }
        }
#pragma unroll
        for (int k = 0; k < KC; ++k) {
#pragma unroll
            for (int j = 0; j < TT; ++j) {
                const float nx = __builtin_fmaf(pv[k][j], dxv[k], acc[j]);
                acc[j] = k < nblk ? nx : acc[j];
            }
        }
        __syncthreads();
    };

    // sched_barrier keeps each chunk's loads issued ahead of the reduction they overlap (the scheduler would otherwise
    // sink them below that reduction's waits, leaving no load in flight while a chunk is reduced).
    const int n_chunks = (nb + KC - 1) / KC;
    MmRegs<DT, TT, KC> A, B;
    load(A, 0);
    int c = 0;
    while (c + 2 < n_chunks) {
        load(B, (c + 1) * KC);
        __builtin_amdgcn_sched_barrier(0);
        reduce(A, c * KC);
        load(A, (c + 2) * KC);
        __builtin_amdgcn_sched_barrier(0);
        reduce(B, (c + 1) * KC);
        c += 2;
    }
    if (c + 1 < n_chunks) {
        load(B, (c + 1) * KC);
        __builtin_amdgcn_sched_barrier(0);
        reduce(A, c * KC);
        reduce(B, (c + 1) * KC);
    } else {
        reduce(A, c * KC);
    }

    const int tok = tbase + ctok;
    if (tok < n) {
#pragma unroll
        for (int j = 0; j < TT; ++j) {
            const int r = rbase + j * (kMmThreads / kTok) + tid / kTok;
            if (r < r1) out[(size_t)tok * ldo + r] = acc[j];
        }
    }
}

// Staged variant for few (row tile, token tile) pairs: the chunk's weights, activation codes and scales are brought
// into LDS by coalesced 16-byte loads (8 full cache lines per wave instruction, against 16 partly used lines for an
// operand loaded in MFMA layout, whose per-CU address processing bounds the other kernels at 32 tokens), chunks ahead
// in registers; the waves then read their MFMA operands from LDS. Tile and block split as in the LDS kernel: wave w
// multiplies blocks 4w..4w+3 of each 16-block chunk, 256 threads run one (row, token) chain each. Rows of one or two
// chunks run on 4 waves (the same threads multiply and chain); longer rows on 8, four that load, stage and multiply
// and four that run the chains of the chunk before.
constexpr int kStKC = 16;  // blocks per chunk
template <int DT>
struct StageRegs {
    static constexpr int kBw = DT == kQ8 ? QK : QK / 2;         // weight bytes per block
    static constexpr int kAu = 16 * kStKC * kBw / 16 / kMmThreads;  // 16-byte weight units per thread (2 / 1)
    static constexpr int kXu = 16 * kStKC * QK / 16 / kMmThreads;   // 16-byte activation units per thread (2)
    uint4 a[kAu];
    uint4 x[kXu];
    uint16_t dw;  // row tid / 16, block tid % 16
    float dx;     // token tid / 16, block tid % 16
};

// LDS operand rows of the tile kernel: rows 8-15 of each 16 hold every 16-byte unit with its 8-byte halves swapped
// (an operand read's lane takes half h ^ 1 there), so the rows li and li + 8 of one 8-byte operand read fall in
// different banks (measured: bank-conflict cycles 27-31% -> 9-10% of the LDS's active cycles; the same layout made the
// 32-token staged kernel slower, 9.9 -> 11.4 us on 896x4864, so it keeps plain rows).
__device__ __forceinline__ uint4 swz16(const uint4& v, int row) {
    const bool h = (row >> 3) & 1;
    return make_uint4(h ? v.z : v.x, h ? v.w : v.y, h ? v.x : v.z, h ? v.y : v.w);
}

template <int DT, int NS>
__global__ __launch_bounds__(NS == 0 ? kMmThreads : 2 * kMmThreads) void matmul_stage_kernel(MmSegs segs, const int8_t* __restrict__ xq,
                                                              const float* __restrict__ xd, int cols, int n,
                                                              int n_tg) {
    using R = StageRegs<DT>;
    constexpr int KC = kStKC, kBw = R::kBw;
    constexpr int kArow = KC * kBw + 16;  // LDS row strides in bytes: = 4 dwords mod 64 banks, so the 16 rows x 2
    constexpr int kXrow = KC * QK + 16;   // lane groups of a half-wave operand read hit 64 distinct banks
    constexpr int kAupr = KC * kBw / 16, kXupr = KC * QK / 16;  // 16-byte units per row
    __shared__ __align__(16) uint8_t as[2][16 * kArow];
    __shared__ __align__(16) int8_t xs[2][16 * kXrow];
    // Block sums and token scales by (row or token, block): a chain reads its chunk as 16-byte units, unit u of
    // token t stored at u ^ ((t >> 2) & 3) so that 8 lanes of consecutive tokens hit distinct banks.
    constexpr int kSb = NS == 0 ? 2 : 3, kLb = NS == 0 ? 1 : 2;  // scale and block-sum buffers
    __shared__ float4 dws[kSb][16][KC / 4];  // [row][block]: chunk c in buffer c % kSb
    __shared__ float4 dxs[kSb][16][KC / 4];  // [token][block], swizzled
    __shared__ int4 sl[kLb][16][16][KC / 4];  // [row][token][block], swizzled: chunk c in buffer c % kLb
    const int nb = cols / QK;
    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lq = lane >> 4;

    const int G = (int)gridDim.x, p = (int)blockIdx.x;
    const int xcd = p % kXcds, per = G / kXcds, rem = G % kXcds;
    const int logical = xcd * per + min(xcd, rem) + p / kXcds;
    int rt = logical / n_tg;
    const int tg = logical % n_tg;
    const MmSeg sg(segs, rt);
    const int r0 = sg.r0, r1 = sg.r1;
    const int rbase = r0 + rt * 16, tbase = tg * 16;
    const size_t wrow_bytes = (size_t)nb * kBw;

    // Per-thread source rows of the staged units (rows and tokens past the end clamped: loaded, never stored).
    const uint8_t* asrc[R::kAu];
    int aoff[R::kAu];
#pragma unroll
    for (int j = 0; j < R::kAu; ++j) {
        const int e = j * kMmThreads + tid;
        asrc[j] = sg.wq + (size_t)min(rbase + e / kAupr, r1 - 1) * wrow_bytes;
        aoff[j] = (e % kAupr) * 16;
    }
    const int8_t* xsrc[R::kXu];
    int xoff[R::kXu];
#pragma unroll
    for (int j = 0; j < R::kXu; ++j) {
        const int e = j * kMmThreads + tid;
        xsrc[j] = xq + (size_t)min(tbase + e / kXupr, n - 1) * cols;
        xoff[j] = (e % kXupr) * 16;
    }
    const uint16_t* dwsrc = sg.ws + (size_t)min(rbase + tid / 16, r1 - 1) * nb;
    const float* dxsrc = xd + (size_t)min(tbase + tid / 16, n - 1) * nb;
    const int sk = tid % 16;

    // Chunk c0's operands into registers; byte offsets past the end of a row are clamped to its last unit.
    auto load = [&](R& S, int c0) {
#pragma unroll
        for (int j = 0; j < R::kAu; ++j)
            S.a[j] = load16(asrc[j] + min((size_t)c0 * kBw + aoff[j], wrow_bytes - 16));
#pragma unroll
        for (int j = 0; j < R::kXu; ++j)
            S.x[j] = load16(xsrc[j] + min(c0 * QK + xoff[j], cols - 16));
        const int b = min(c0 + sk, nb - 1);
        S.dw = dwsrc[b];
        S.dx = dxsrc[b];
    };
    auto stage = [&](const R& S, int buf, int sbuf) {
#pragma unroll
        for (int j = 0; j < R::kAu; ++j) {
            const int e = j * kMmThreads + tid;
            *reinterpret_cast<uint4*>(&as[buf][(e / kAupr) * kArow + (e % kAupr) * 16]) = S.a[j];
        }
#pragma unroll
        for (int j = 0; j < R::kXu; ++j) {
            const int e = j * kMmThreads + tid;
            *reinterpret_cast<uint4*>(&xs[buf][(e / kXupr) * kXrow + (e % kXupr) * 16]) = S.x[j];
        }
        const int t = tid / 16;
        uint32_t h = S.dw;
        asm volatile("" : "+v"(h));  // keeps the conversion here (hoisted, it would wait for every set's loads)
        reinterpret_cast<float*>(&dws[sbuf][t][0])[sk] = f16_to_f32((uint16_t)h);
        reinterpret_cast<float*>(&dxs[sbuf][t][0])[4 * ((sk >> 2) ^ ((t >> 2) & 3)) + (sk & 3)] = S.dx;
    };
    const int shift = DT == kQ8 ? 0 : (lq >> 1) * 4;
    // The wave's 4 blocks: operands read together, 4 independent MFMAs, then the block sums out.
    auto products = [&](int buf, int lbuf) {
        long a[4], x[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int bl = wave * 4 + i;
            a[i] = *reinterpret_cast<const long*>(&as[buf][li * kArow + bl * kBw + (DT == kQ8 ? lq * 8 : (lq & 1) * 8)]);
            x[i] = *reinterpret_cast<const long*>(&xs[buf][li * kXrow + bl * QK + lq * 8]);
        }
        v4i c[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            long ai = a[i];
            if (DT == kQ4) {
                const uint64_t v = (uint64_t)ai;
                const uint32_t lo = nibbles_to_i8(((uint32_t)v >> shift) & 0x0F0F0F0Fu);
                const uint32_t hi = nibbles_to_i8(((uint32_t)(v >> 32) >> shift) & 0x0F0F0F0Fu);
                ai = (long)(((uint64_t)hi << 32) | lo);
            }
            c[i] = __builtin_amdgcn_mfma_i32_16x16x32_i8(ai, x[i], (v4i){0, 0, 0, 0}, 0, 0, 0);
        }
        // row 4 lq + k, token li: the sums of blocks 4 wave .. 4 wave + 3 as one unit
#pragma unroll
        for (int k = 0; k < 4; ++k) sl[lbuf][4 * lq + k][li][wave ^ ((li >> 2) & 3)] = (int4){c[0][k], c[1][k], c[2][k], c[3][k]};
    };
    // Chain of this thread: row tid / 16, token tid % 16 (the LDS kernel's pairing at one token tile).
    const int ctid = NS == 0 ? tid : tid - kMmThreads;
    const int crow = ctid / 16, ctok = ctid % 16;
    float acc = 0.0f;
    auto chains = [&](int lbuf, int sbuf, int c0) {
        const int nblk = min(KC, nb - c0);
        float pv[KC], dxv[KC];
        const int sw = (ctok >> 2) & 3;
#pragma unroll
        for (int u = 0; u < KC / 4; ++u) {
            const int4 si = sl[lbuf][crow][ctok][u ^ sw];
            const float4 w = dws[sbuf][crow][u], d = dxs[sbuf][ctok][u ^ sw];
            pv[4 * u + 0] = (float)si.x * w.x;
            pv[4 * u + 1] = (float)si.y * w.y;
            pv[4 * u + 2] = (float)si.z * w.z;
            pv[4 * u + 3] = (float)si.w * w.w;
            dxv[4 * u + 0] = d.x;
            dxv[4 * u + 1] = d.y;
            dxv[4 * u + 2] = d.z;
            dxv[4 * u + 3] = d.w;
        }
#pragma unroll
        for (int k = 0; k < KC; ++k) {
            const float nx = __builtin_fmaf(pv[k], dxv[k], acc);
            acc = k < nblk ? nx : acc;
        }
    };

    if constexpr (NS == 0) {
        // At most two chunks (nb <= 2 KC), straight-line with one block-sum buffer (the LDS of three workgroups per
        // CU): a chain past nb adds nothing, and the products of a chunk past nb read clamped rows no chain uses.
        R A, B;
        load(A, 0);
        load(B, KC);
        __builtin_amdgcn_sched_barrier(0);
        stage(A, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        products(0, 0);
        stage(B, 1, 1);
        __syncthreads();
        chains(0, 0, 0);
        __syncthreads();
        products(1, 0);
        __syncthreads();
        chains(0, 1, KC);
    } else {
        // Eight waves: waves 0-3 load, stage and multiply, waves 4-7 run the chains, each SIMD holding one wave of
        // each; the two kinds run separate loops that meet at one barrier per chunk (1 + n_chunks barriers each).
        // Between two barriers the products of chunk c + 1 (operand buffer (c + 1) % 2 -> block sums (c + 1) % 2)
        // and the chains of chunk c (block sums c % 2, scales c % 3) run together, and chunk c + 2 is staged
        // (operands into buffer c % 2, last read by chunk c's products; scales into c + 2 mod 3). NS register sets,
        // set k holding a chunk = k mod NS, each refilled with the chunk NS past the one it stages; loads and stages
        // past the last chunk are clamped re-reads into buffers no later phase reads, issued on every pass so that
        // each wait counts only the loads it needs.
        const int n_chunks = (nb + KC - 1) / KC;
        if (tid < kMmThreads) {
            R S[NS];
#pragma unroll
            for (int i = 0; i < NS; ++i) load(S[i], i * KC);
            __builtin_amdgcn_sched_barrier(0);
            stage(S[0], 0, 0);
            load(S[0], NS * KC);
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();
            products(0, 0);
            stage(S[1], 1, 1);
            load(S[1], (NS + 1) * KC);
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();
            for (int c = 0;; c += NS) {
#pragma unroll
                for (int j = 0; j < NS; ++j) {
                    const int cc = c + j;
                    if (cc + 1 >= n_chunks) return;
                    products((cc + 1) & 1, (cc + 1) & 1);
                    stage(S[(j + 2) % NS], cc & 1, (cc + 2) % 3);
                    load(S[(j + 2) % NS], (cc + 2 + NS) * KC);
                    __builtin_amdgcn_sched_barrier(0);
                    __syncthreads();
                }
            }
        }
        __syncthreads();
        __syncthreads();
        for (int cc = 0;; ++cc) {
            chains(cc & 1, cc % 3, cc * KC);
            if (cc + 1 >= n_chunks) break;
            __syncthreads();
        }
    }

    const int tok = tbase + ctok, r = rbase + crow;
    if (tok < n && r < r1) sg.out[(size_t)tok * sg.ldo + r] = acc;
}

// Tile variant for batches of 128 tokens and more: a workgroup of NW = 4 or 8 waves owns 64 rows x TT tokens
// (TT = 16, 32 or 64) over all of K, in chunks of KC blocks brought into LDS by coalesced 16-byte loads (a row's chunk
// is KC x 16 (Q4_0) or KC x 32 (Q8_0) contiguous bytes, a token's KC x 32; Q4_0 codes are unpacked to int8 as they
// are staged, so both formats share the LDS layout and the compute loop), double-buffered with two register sets:
// the loads of chunk c + 3 are issued as chunk c + 1 is staged. Wave (wr, wt) multiplies 16 NRS rows by 16 NTS tokens
// (four waves at TT >= 32: 32 rows x TT / 2 tokens; at TT = 16: 16 rows x 16 tokens; eight waves: 16 rows x TT / 2
// tokens, two waves per SIMD): per block one MFMA per (16-row, 16-token) tile, each weight operand read once for
// every token tile and each activation operand once for every row tile, and the wave runs the chains of its lanes'
// outputs in registers (lane l: rows 4 (l / 16) + i of each row tile, token l % 16 of each token tile), so no block
// sum goes through LDS. A whole chunk runs straight-line two blocks deep (block b's chains, block b + 1's MFMAs,
// block b + 2's operand reads). Operand loads in MFMA layout (8 bytes per lane from 16 rows) kept the texture-address
// units busy for most of the register kernel's time at 512 tokens; here they are busy about a third of the time, and
// the exact f32 chains (a convert, a scale multiply and an FMA per output and block; two FMAs with eight waves) and
// the per-chunk staging and barrier are what is left.
// Timeline stamps of workgroup 0, wave 0 (compiled in only with -DQH_TIMELINE; qh_timeline_mm_read copies them out).
#if defined(QH_TIMELINE)
__device__ uint64_t qh_tl_mm[64];
#define QH_MMSTAMP(i)                                                                                     \
    do {                                                                                                  \
        if (blockIdx.x == 0 && threadIdx.x == 0 && (i) < 64) qh_tl_mm[i] = __builtin_readcyclecounter(); \
    } while (0)
#else
#define QH_MMSTAMP(i) \
    do {              \
    } while (0)
#endif
template <int DT, int KC, int TT, int NT>
struct TileRegs {
    static constexpr int kBw = DT == kQ8 ? QK : QK / 2;   // weight bytes per block
    static constexpr int kAu = 64 * KC * kBw / 16 / NT;  // 16-byte weight units per thread
    static constexpr int kXu = TT * KC * QK / 16 / NT;   // 16-byte activation units per thread
    static constexpr int kTpr = NT / 64;                 // threads per row (and per token) of the scales
    static constexpr int kSp = KC / kTpr;                // scales per thread and chunk
    uint4 a[kAu];
    uint4 x[kXu];
    uint16_t dw[kSp];  // row tid / kTpr, blocks kSp (tid % kTpr) + j of the chunk
    float dx[kSp];     // token tid / kTpr, blocks kSp (tid % kTpr) + j of the chunk
};

// TT: tokens per workgroup, 64 (waves of 32 rows x 32 tokens), 32 (waves of 32 rows x 16 tokens: twice the
// workgroups for matrices with few row tiles) or 16 (four waves of 16 rows x 16 tokens: four times, for long rows,
// KC = 8).
// SW: the prefill stack's gate / up launch with SwiGLU and the down projection's input quantization in the epilogue
// (model.cpp:212-218; ops_ref.cpp:243-248, 69-83): workgroup row tile rt stages gate rows [32 rt, 32 rt + 32) of segment
// 0 as its rows 0-31 and the same up rows of segment 1 as rows 32-63, so the row-0 waves hold g and the row-1 waves u
// of the same (row, token) outputs; h = g / (1 + expf(-g)) * u of each token's 32 rows is one 32-block of hq / hd
// (rows = segs.r1[0] values per token).
template <int DT, int KC, int TT, int NW, bool SW>
__global__ __launch_bounds__(64 * NW) void matmul_tile_kernel(MmSegs segs, const int8_t* __restrict__ xq,
                                                             const float* __restrict__ xd, int cols, int n, int n_tg,
                                                             int8_t* __restrict__ hq, float* __restrict__ hd) {
    constexpr int NT = 64 * NW;  // threads
    static_assert(TT == 64 || TT == 32 || TT == 16, "token tile");
    static_assert(NW == 4 || (NW == 8 && TT >= 32), "waves");
    static_assert(!SW || (NW == 4 && TT == 32), "SwiGLU epilogue: four waves, 32 tokens");
    // With eight waves (two per SIMD) the chains' VALU issue is what bounds the kernel: the integer sums start from
    // kSumBias and each block product is one FMA with a staged -(B * dw) (two-step products in a chunk with an inf or
    // NaN row scale)
    constexpr bool BIAS = NW == 8;
    static_assert(64 * KC * (DT == kQ8 ? QK : QK / 2) / 16 % NT == 0 && TT * KC * QK / 16 % NT == 0 &&
                      KC % (NT / 64) == 0,
                  "whole units and scales per thread");
    constexpr int WT = TT == 16 ? 1 : 2;  // waves across the tokens
    constexpr int WR = NW / WT;           // waves across the 64 rows
    constexpr int NRS = 4 / WR;           // 16-row tiles per wave
    constexpr int NTS = TT / (16 * WT);   // 16-token tiles per wave
    using R = TileRegs<DT, KC, TT, NT>;
    constexpr int kBw = R::kBw, kSp = R::kSp, kTpr = R::kTpr;
    // Weights are staged as int8 codes whatever the format (Q4_0 nibbles are unpacked once, as they are staged, not by
    // both token waves at every block): LDS row strides in bytes
    constexpr int kArow = KC * QK + 16, kXrow = KC * QK + 16;
    constexpr int kAupr = KC * kBw / 16, kXupr = KC * QK / 16;  // 16-byte units per row and chunk
    __shared__ __align__(16) uint8_t as[2][64 * kArow];
    __shared__ __align__(16) int8_t xs[2][TT * kXrow];
    // Row scales as f16 bits in the order the waves read them: [block][row wave wr][lane group lq][row tile rs][i]
    // holds row 16 NRS wr + 16 rs + 4 lq + i, so a lane's scales of a block are one 16-byte (8-byte) read
    __shared__ __align__(16) uint16_t dws[2][KC][WR][4][4 * NRS];
    __shared__ __align__(16) float cws[BIAS ? 2 : 1][BIAS ? KC : 1][WR][4][4 * NRS];  // -(kSumBiasF * dw), same order
    __shared__ __align__(16) float dxs[2][KC][TT];  // [block][token]
    __shared__ int first_nonfinite;  // lowest chunk with an inf or NaN row scale (INT_MAX if none)
    const int nb = cols / QK;
    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lq = lane >> 4;
    const int wr = wave / WT, wt = wave % WT;
    ExpTab et;  // SW: the expf table, loaded first thing
    if constexpr (SW) et.load();
    const int lqs = lq ^ ((li >> 3) & 1);  // the 8-byte half this lane reads in its row (rows 8-15 swapped, swz16)

    // XCD-aware numbering as in the other variants; segment tiles count 64-row tiles here
    const int G = (int)gridDim.x, p = (int)blockIdx.x;
    const int xcd = p % kXcds, per = G / kXcds, rem = G % kXcds;
    const int logical = xcd * per + min(xcd, rem) + p / kXcds;
    int rt = logical / n_tg;
    const int tg = logical % n_tg;
    const MmSeg sg(segs, rt);
    const int r1 = sg.r1;
    const int rbase = sg.r0 + rt * 64, tbase = tg * TT;
    const size_t wrow_bytes = (size_t)nb * kBw;
    const bool dx_thread = tid < kTpr * TT;  // threads of a token's scales (wave-uniform)

    // Source rows of this thread's staged units; rows and tokens past the end are clamped (loaded, never stored), and
    // byte offsets past the end of a row onto its last unit (blocks no chain adds).
    // SW: staged row t is row 32 rt + (t & 31) of segment t / 32 (gate, up)
    auto wrow = [&](int t) {
        return SW ? (t < 32 ? segs.wq[0] : segs.wq[1]) + (size_t)(32 * rt + (t & 31)) * wrow_bytes
                  : sg.wq + (size_t)min(rbase + t, r1 - 1) * wrow_bytes;
    };
    const uint8_t* asrc[R::kAu];
    int aoff[R::kAu];
#pragma unroll
    for (int j = 0; j < R::kAu; ++j) {
        const int e = j * NT + tid;
        asrc[j] = wrow(e / kAupr);
        aoff[j] = (e % kAupr) * 16;
    }
    const int8_t* xsrc[R::kXu];
    int xoff[R::kXu];
#pragma unroll
    for (int j = 0; j < R::kXu; ++j) {
        const int e = j * NT + tid;
        xsrc[j] = xq + (size_t)min(tbase + e / kXupr, n - 1) * cols;
        xoff[j] = (e % kXupr) * 16;
    }
    const uint16_t* dwsrc = SW ? (tid / kTpr < 32 ? segs.ws[0] : segs.ws[1]) + (size_t)(32 * rt + (tid / kTpr & 31)) * nb
                               : sg.ws + (size_t)min(rbase + tid / kTpr, r1 - 1) * nb;
    const float* dxsrc = xd + (size_t)min(tbase + tid / kTpr, n - 1) * nb;
    const int sk = kSp * (tid % kTpr);

    auto load = [&](R& S, int c0) {
#pragma unroll
        for (int j = 0; j < R::kAu; ++j)
            S.a[j] = load16(asrc[j] + min((size_t)c0 * kBw + aoff[j], wrow_bytes - 16));
#pragma unroll
        for (int j = 0; j < R::kXu; ++j)
            S.x[j] = load16(xsrc[j] + min(c0 * QK + xoff[j], cols - 16));
#pragma unroll
        for (int j = 0; j < kSp; ++j) {
            const int b = min(c0 + sk + j, nb - 1);
            S.dw[j] = dwsrc[b];
            if (dx_thread) S.dx[j] = dxsrc[b];
        }
    };
    auto stage = [&](const R& S, int buf, int c) {
#pragma unroll
        for (int j = 0; j < R::kAu; ++j) {
            const int e = j * NT + tid;
            if (DT == kQ8) {
                *reinterpret_cast<uint4*>(&as[buf][(e / kAupr) * kArow + (e % kAupr) * 16]) = swz16(S.a[j], e / kAupr);
            } else {  // one block: element i < 16 in the low nibble of byte i, element 16 + i in its high nibble
                const uint4 v = swz16(S.a[j], e / kAupr);  // both unpacked units come out with their halves swapped
                const uint32_t w[4] = {v.x, v.y, v.z, v.w};
                uint32_t lo[4], hi[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    lo[q] = nibbles_to_i8(w[q] & 0x0F0F0F0Fu);
                    hi[q] = nibbles_to_i8((w[q] >> 4) & 0x0F0F0F0Fu);
                }
                uint8_t* dst = &as[buf][(e / kAupr) * kArow + (e % kAupr) * QK];
                *reinterpret_cast<uint4*>(dst) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
                *reinterpret_cast<uint4*>(dst + 16) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
            }
        }
#pragma unroll
        for (int j = 0; j < R::kXu; ++j) {
            const int e = j * NT + tid;
            *reinterpret_cast<uint4*>(&xs[buf][(e / kXupr) * kXrow + (e % kXupr) * 16]) = swz16(S.x[j], e / kXupr);
        }
        const int t = tid / kTpr;
        bool nonfinite = false;
#pragma unroll
        for (int j = 0; j < kSp; ++j) {
            dws[buf][sk + j][t / (16 * NRS)][(t >> 2) & 3][((t >> 4) % NRS) * 4 + (t & 3)] = S.dw[j];
            if constexpr (BIAS) {
                cws[buf][sk + j][t / (16 * NRS)][(t >> 2) & 3][((t >> 4) % NRS) * 4 + (t & 3)] =
                    -(kSumBiasF * f16_to_f32(S.dw[j]));
                nonfinite = nonfinite || f16_nonfinite(S.dw[j]);
            }
            if (dx_thread) dxs[buf][sk + j][t] = S.dx[j];
        }
        if (BIAS && nonfinite) atomicMin(&first_nonfinite, c);  // rare: that chunk takes the two-step products
    };

    float acc[NRS][NTS][4];
#pragma unroll
    for (int rs = 0; rs < NRS; ++rs)
#pragma unroll
        for (int ts = 0; ts < NTS; ++ts)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[rs][ts][i] = 0.0f;
    // One block's operands (NRS weight tiles, NTS token tiles) and its products.
    struct Ops {
        long a[NRS], x[NTS];
        uint32_t dw[2 * NRS];  // f16 scales of rows 16 rs + 4 lq + i (i = 0..3) of the wave's rows
        float dx[NTS];
        float cw[BIAS ? 4 * NRS : 1];
    };
    auto ld_ops = [&](Ops& o, int buf, int b) {
#pragma unroll
        for (int rs = 0; rs < NRS; ++rs) {
            o.a[rs] = *reinterpret_cast<const long*>(
                &as[buf][(wr * 16 * NRS + rs * 16 + li) * kArow + b * QK + lqs * 8]);
        }
        if constexpr (NRS == 2) {
            const uint4 w = *reinterpret_cast<const uint4*>(&dws[buf][b][wr][lq][0]);
            o.dw[0] = w.x, o.dw[1] = w.y, o.dw[2] = w.z, o.dw[3] = w.w;
        } else {
            const uint2 w = *reinterpret_cast<const uint2*>(&dws[buf][b][wr][lq][0]);
            o.dw[0] = w.x, o.dw[1] = w.y;
        }
        if constexpr (BIAS) {
#pragma unroll
            for (int rs = 0; rs < NRS; ++rs) {
                const float4 w = *reinterpret_cast<const float4*>(&cws[buf][b][wr][lq][4 * rs]);
                o.cw[4 * rs] = w.x, o.cw[4 * rs + 1] = w.y, o.cw[4 * rs + 2] = w.z, o.cw[4 * rs + 3] = w.w;
            }
        }
#pragma unroll
        for (int ts = 0; ts < NTS; ++ts) {
            o.x[ts] = *reinterpret_cast<const long*>(
                &xs[buf][(wt * (TT / WT) + ts * 16 + li) * kXrow + b * QK + lqs * 8]);
            o.dx[ts] = dxs[buf][b][wt * (TT / WT) + ts * 16 + li];
        }
    };
    auto mma = [&](const Ops& o, v4i(&c)[NRS][NTS]) {
#pragma unroll
        for (int rs = 0; rs < NRS; ++rs)
#pragma unroll
            for (int ts = 0; ts < NTS; ++ts)
                c[rs][ts] = BIAS ? __builtin_amdgcn_mfma_i32_16x16x32_i8(o.a[rs], o.x[ts],
                                                                         (v4i){kSumBias, kSumBias, kSumBias, kSumBias},
                                                                         0, 0, 0)
                                 : __builtin_amdgcn_mfma_i32_16x16x32_i8(o.a[rs], o.x[ts], (v4i){0, 0, 0, 0}, 0, 0, 0);
    };
    // acc = fma(float(s) * dw, dx, acc) (ops_ref.cpp:97-98) for one block. float(s) * dw is taken as
    // fma(float(s), dw, 0) with the f16 scale as a mixed-precision operand (v_fma_mix_f32: the scale widens exactly,
    // one rounding, as the product; a zero product comes out +0 where the product could be -0, which a chain from +0
    // never shows, since +0 + -0 = +0). With BIAS the sums are B + s: fma(B + s, dw, -(B * dw)) (FAST), else
    // fma(B + s - B, dw, 0).
    auto chain = [&](auto fast, const Ops& o, const v4i(&c)[NRS][NTS]) {
        const uint32_t* dww = o.dw;
#pragma unroll
        for (int rs = 0; rs < NRS; ++rs) {
#pragma unroll
            for (int ts = 0; ts < NTS; ++ts)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t w = dww[2 * rs + (i >> 1)];
                    const float dw = (float)__builtin_bit_cast(_Float16, (uint16_t)(i & 1 ? w >> 16 : w & 0xffffu));
                    float pr;
                    if constexpr (!BIAS)
                        pr = __builtin_fmaf((float)c[rs][ts][i], dw, 0.0f);
                    else if constexpr (decltype(fast)::value)
                        pr = __builtin_fmaf(__int_as_float(c[rs][ts][i]), dw, o.cw[4 * rs + i]);
                    else
                        pr = __builtin_fmaf(__int_as_float(c[rs][ts][i]) - kSumBiasF, dw, 0.0f);
                    acc[rs][ts][i] = __builtin_fmaf(pr, o.dx[ts], acc[rs][ts][i]);
                }
        }
    };
    // Blocks 0 .. nblk - 1 of buffer buf in order, software-pipelined: block b + 1's operands are read and its
    // products issued while block b's chains run.
    auto compute = [&](auto fast, int buf, int nblk) {
        Ops o0, o1;
        v4i c0[NRS][NTS], c1[NRS][NTS];
        ld_ops(o0, buf, 0);
        mma(o0, c0);
        int b = 0;
        for (; b + 2 <= nblk; b += 2) {
            ld_ops(o1, buf, b + 1);
            __builtin_amdgcn_sched_barrier(0);
            chain(fast, o0, c0);
            mma(o1, c1);
            if (b + 2 < nblk) ld_ops(o0, buf, b + 2);
            __builtin_amdgcn_sched_barrier(0);
            chain(fast, o1, c1);
            if (b + 2 < nblk) mma(o0, c0);
        }
        if (b < nblk) chain(fast, o0, c0);
    };
    // A whole chunk (KC blocks), straight-line and two blocks deep: while block b's chains run, block b + 1's MFMAs
    // are in flight and block b + 2's operands are being read, so neither the LDS latency nor the MFMA latency waits
    // in front of a chain.
    auto compute_full = [&](auto fast, int buf) {
        Ops o[3];
        v4i c[2][NRS][NTS];
        ld_ops(o[0], buf, 0);
        if (KC > 1) ld_ops(o[1], buf, 1);
        mma(o[0], c[0]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int b = 0; b < KC; ++b) {
            if (b + 2 < KC) ld_ops(o[(b + 2) % 3], buf, b + 2);
            if (b + 1 < KC) mma(o[(b + 1) % 3], c[(b + 1) & 1]);
            __builtin_amdgcn_sched_barrier(0);
            chain(fast, o[b % 3], c[b & 1]);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // Two register sets, chunk j in set j % 2: chunk c + 1 is staged after chunk c is multiplied (its buffer was last
    // read by chunk c - 1, before the previous barrier), and the loads of chunk c + 3 go into the set it leaves, so
    // two chunks' products cover each load.
    const int n_chunks = (nb + KC - 1) / KC;
    QH_MMSTAMP(0);
    R S0, S1;
    load(S0, 0);
    if (n_chunks > 1) load(S1, KC);
    if constexpr (BIAS) {
        if (tid == 0) first_nonfinite = 0x7fffffff;
        __syncthreads();  // the loads above are in flight
    }
    stage(S0, 0, 0);
    if (n_chunks > 2) load(S0, 2 * KC);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    QH_MMSTAMP(1);
    auto step = [&](int c, R& Sn) {  // Sn holds chunk c + 1
        // Chunk c's scales were staged before the last barrier; a later chunk's flag only lowers the bound to c + 1
        const bool fast = !BIAS || __builtin_amdgcn_readfirstlane(first_nonfinite) > c;
        if ((c + 1) * KC <= nb) {
            if (fast)
                compute_full(std::true_type{}, c & 1);
            else
                compute_full(std::false_type{}, c & 1);
        } else if (fast) {
            compute(std::true_type{}, c & 1, nb - c * KC);
        } else {
            compute(std::false_type{}, c & 1, nb - c * KC);
        }
        QH_MMSTAMP(2 + 3 * c);
        if (c + 1 < n_chunks) {
            stage(Sn, (c + 1) & 1, c + 1);
            QH_MMSTAMP(3 + 3 * c);
            if (c + 3 < n_chunks) load(Sn, (c + 3) * KC);
            __builtin_amdgcn_sched_barrier(0);
        }
        __syncthreads();
        QH_MMSTAMP(4 + 3 * c);
    };
    for (int c = 0; c < n_chunks; c += 2) {
        step(c, S1);
        if (c + 1 < n_chunks) step(c + 1, S0);
    }

    if constexpr (SW) {
        __shared__ float hsw[2][32][TT + 1];  // [gate, up][row][token]
        __shared__ uint64_t exptab[32];
#pragma unroll
        for (int rs = 0; rs < NRS; ++rs)
#pragma unroll
            for (int ts = 0; ts < NTS; ++ts)
#pragma unroll
                for (int i = 0; i < 4; ++i) hsw[wr][16 * rs + 4 * lq + i][wt * (TT / WT) + ts * 16 + li] = acc[rs][ts][i];
        et.store(exptab);
        __syncthreads();
        const int F = segs.r1[0];
#pragma unroll
        for (int pass = 0; pass < TT / 8; ++pass) {  // 32 lanes per token's block
            const int tk = pass * 8 + tid / 32, rr = tid % 32, tok = tbase + tk;
            if (tok < n) {  // uniform per 32-lane group
                const float gv = hsw[0][rr][tk], uv = hsw[1][rr][tk];
                quant_block32(gv / (1.0f + dev_expf(-gv, exptab)) * uv, hq + (size_t)tok * F + 32 * rt,
                              hd + (size_t)tok * (F / QK) + rt);
            }
        }
        return;
    }
#pragma unroll
    for (int ts = 0; ts < NTS; ++ts) {
        const int tok = tbase + wt * (TT / WT) + ts * 16 + li;
        if (tok < n) {
#pragma unroll
            for (int rs = 0; rs < NRS; ++rs)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = rbase + wr * 16 * NRS + rs * 16 + 4 * lq + i;
                    if (r < r1) sg.out[(size_t)tok * sg.ldo + r] = acc[rs][ts][i];
                }
        }
    }
}

// Register-chain variant: a wave owns 16 rows x 16*TT tokens over all of K and runs the chains of its own MFMA
// outputs in registers (lane l: rows 4*(l/16)+i, token l%16 of each tile), so no block sum goes through LDS. The NW
// waves of a workgroup share the 16 rows (their weight loads hit L1) and take consecutive token tiles. Blocks go in
// chunks of 4: two register sets alternate in straight-line halves, the operands of chunk c+1 in flight while chunk c
// is reduced. VEC (nb % 4 == 0 and 16-byte aligned token scales): the 4 row scales and the token scales of a chunk
// are single 8- and 16-byte loads.
template <int DT, int TT, bool VEC>
struct RegChunk {
    long a[4];          // weight bytes per block (Q4_0 packed, unpacked at use)
    long x[4][TT];      // activation operand per block and token tile
    uint2 dw[4];        // row 4*(l/16)+i: fp16 scales of the chunk's 4 blocks (VEC)
    float4 dx[TT];      // token of tile tt: f32 scales of the chunk's 4 blocks (VEC)
    uint16_t dws[VEC ? 1 : 4][VEC ? 1 : 4];  // scalar path: [row i][block]
    float dxs[VEC ? 1 : TT][VEC ? 1 : 4];    // scalar path: [tile][block]
};

template <int DT, int TT, int NW, bool VEC>
__global__ __launch_bounds__(64 * NW) void matmul_reg_kernel(MmSegs segs, const int8_t* __restrict__ xq,
                                                            const float* __restrict__ xd, int cols, int n, int n_tg) {
    const int nb = cols / QK;
    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lq = lane >> 4;
    const int G = (int)gridDim.x, p = (int)blockIdx.x;
    const int xcd = p % kXcds, per = G / kXcds, rem = G % kXcds;
    const int logical = xcd * per + min(xcd, rem) + p / kXcds;
    int rt = logical / n_tg;
    const int tg = logical % n_tg;
    const MmSeg sg(segs, rt);
    const uint8_t* __restrict__ wq = sg.wq;
    const uint16_t* __restrict__ wscale = sg.ws;
    float* __restrict__ out = sg.out;
    const int ldo = sg.ldo, r0 = sg.r0, r1 = sg.r1;
    const int rbase = r0 + rt * 16;
    const int tbase = (tg * NW + wave) * TT * 16;
    if (tbase >= n) return;  // uniform per wave; nothing below synchronises across waves

    const int arow = min(rbase + li, r1 - 1);
    const uint8_t* wrow;
    int shift = 0;
    if (DT == kQ8) {
        wrow = wq + (size_t)arow * cols + lq * 8;
    } else {
        wrow = wq + (size_t)arow * (cols / 2) + (lq & 1) * 8;
        shift = (lq >> 1) * 4;
    }
    const int8_t* xrow[TT];
    const float* dxrow[TT];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
        const int t = min(tbase + tt * 16 + li, n - 1);
        xrow[tt] = xq + (size_t)t * cols + lq * 8;
        dxrow[tt] = xd + (size_t)t * nb;
    }
    const uint16_t* dwrow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) dwrow[i] = wscale + (size_t)min(rbase + 4 * lq + i, r1 - 1) * nb;

    auto load = [&](RegChunk<DT, TT, VEC>& R, int c0) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int b = min(c0 + k, nb - 1);
            R.a[k] = *reinterpret_cast<const long*>(wrow + (size_t)b * (DT == kQ8 ? QK : QK / 2));
#pragma unroll
            for (int tt = 0; tt < TT; ++tt) R.x[k][tt] = *reinterpret_cast<const long*>(xrow[tt] + (size_t)b * QK);
        }
        if constexpr (VEC) {
#pragma unroll
            for (int i = 0; i < 4; ++i) R.dw[i] = *reinterpret_cast<const uint2*>(dwrow[i] + c0);
#pragma unroll
            for (int tt = 0; tt < TT; ++tt) R.dx[tt] = *reinterpret_cast<const float4*>(dxrow[tt] + c0);
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int b = min(c0 + k, nb - 1);
#pragma unroll
                for (int i = 0; i < 4; ++i) R.dws[i][k] = dwrow[i][b];
#pragma unroll
                for (int tt = 0; tt < TT; ++tt) R.dxs[tt][k] = dxrow[tt][b];
            }
        }
    };

    float acc[TT][4];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[tt][i] = 0.0f;

    auto reduce = [&](const RegChunk<DT, TT, VEC>& R, int c0) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            long a = R.a[k];
            if (DT == kQ4) {
                const uint64_t v = (uint64_t)a;
                const uint32_t lo = nibbles_to_i8(((uint32_t)v >> shift) & 0x0F0F0F0Fu);
                const uint32_t hi = nibbles_to_i8(((uint32_t)(v >> 32) >> shift) & 0x0F0F0F0Fu);
                a = (long)(((uint64_t)hi << 32) | lo);
            }
            float dw[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint16_t h;
                if constexpr (VEC) {
                    const uint32_t w2 = k < 2 ? R.dw[i].x : R.dw[i].y;
                    h = (uint16_t)((k & 1) ? (w2 >> 16) : (w2 & 0xffffu));
                } else {
                    h = R.dws[i][k];
                }
                dw[i] = f16_to_f32(h);
            }
            const bool live = c0 + k < nb;
#pragma unroll
            for (int tt = 0; tt < TT; ++tt) {
                v4i c = {0, 0, 0, 0};
                c = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, R.x[k][tt], c, 0, 0, 0);
                float dx;
                if constexpr (VEC) {
                    dx = k == 0 ? R.dx[tt].x : k == 1 ? R.dx[tt].y : k == 2 ? R.dx[tt].z : R.dx[tt].w;
                } else {
                    dx = R.dxs[tt][k];
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float nx = __builtin_fmaf((float)c[i] * dw[i], dx, acc[tt][i]);
                    acc[tt][i] = live ? nx : acc[tt][i];
                }
            }
        }
    };

    // sched_barrier: as in the LDS kernel, each chunk's loads stay issued ahead of the reduction they overlap.
    const int n_chunks = (nb + 3) / 4;
    RegChunk<DT, TT, VEC> A, B;
    load(A, 0);
    int c = 0;
    while (c + 2 < n_chunks) {
        load(B, (c + 1) * 4);
        __builtin_amdgcn_sched_barrier(0);
        reduce(A, c * 4);
        load(A, (c + 2) * 4);
        __builtin_amdgcn_sched_barrier(0);
        reduce(B, (c + 1) * 4);
        c += 2;
    }
    if (c + 1 < n_chunks) {
        load(B, (c + 1) * 4);
        __builtin_amdgcn_sched_barrier(0);
        reduce(A, c * 4);
        reduce(B, (c + 1) * 4);
    } else {
        reduce(A, c * 4);
    }

#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
        const int tok = tbase + tt * 16 + li;
        if (tok < n) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = rbase + 4 * lq + i;
                if (r < r1) out[(size_t)tok * ldo + r] = acc[tt][i];
            }
        }
    }
}

namespace {

// Launch plan: kernel family, token tiles (per workgroup for the LDS kernel, per wave for the register kernel) and
// waves per workgroup. QH_MM="stage", "stage:NS", "tile", "tile:KC", "lds:TT" or "reg:TT:NW" overrides the heuristic
// (tuning sweeps).
struct MmPlan {
    bool reg;
    int tt, nw;
    bool stage = false;  // the LDS-staged kernel (one token tile per workgroup)
    int ns = 0;          // its register sets in flight past two chunks (2, 3 or 4; 0: default)
    bool tile = false;   // the 64-row tile kernel
    int kc = 4;          // its blocks per chunk (4 or 8)
    int ttile = 64;      // its tokens per workgroup (64, 32 or 16)
};

MmPlan matmul_plan(int rows, int cols, int n) {
    MmPlan pl{true, 1, 1};
    const char* env = getenv("QH_MM");
    if (env) {
        int a = 0, b = 0;
        if (sscanf(env, "lds:%d", &a) == 1 && (a == 1 || a == 2 || a == 4)) return MmPlan{false, a, 4};
        if (strcmp(env, "stage") == 0) return MmPlan{false, 1, 4, true};
        if (strcmp(env, "tile") == 0) return MmPlan{false, 1, 4, false, 0, true, 4};
        if (sscanf(env, "tile:%d", &a) == 1 && (a == 4 || a == 8)) return MmPlan{false, 1, 4, false, 0, true, a};
        if (strcmp(env, "tile32") == 0) return MmPlan{false, 1, 4, false, 0, true, 4, 32};
        if (sscanf(env, "tile32:%d", &a) == 1 && (a == 4 || a == 8)) return MmPlan{false, 1, 4, false, 0, true, a, 32};
        if (strcmp(env, "tile16") == 0) return MmPlan{false, 1, 4, false, 0, true, 8, 16};
        if (strcmp(env, "tile32w8") == 0) return MmPlan{false, 1, 8, false, 0, true, 8, 32};
        if (strcmp(env, "tile32w8:16") == 0) return MmPlan{false, 1, 8, false, 0, true, 16, 32};
        if (sscanf(env, "stage:%d", &a) == 1 && a >= 2 && a <= 4) return MmPlan{false, 1, 4, true, a};
        if (sscanf(env, "reg:%d:%d", &a, &b) == 2 && (a == 1 || a == 2 || a == 4) && (b == 1 || b == 2 || b == 4))
            return MmPlan{true, a, b};
    }
    (void)pl;
    // From sweeps on MI355X (cold weights) at the Qwen2.5-0.5B shapes, M = 32 / 64 / 128 / 256 / 512: the tile kernel
    // with 32-token workgroups wins from 128 tokens once there are about 192 tiles or more, with 4-block chunks on rows
    // of up to 64 blocks (Q4_0 4864x896 at M = 512: 20.2 us, against 24.4 with 8-block chunks, 21.2-24.2 for 64-token
    // workgroups, 45.0 staged and 54.2 register-chain; M = 128: 10.8 against 14.4 staged; Q8_0 896x896 at M = 512:
    // 8.4 against 11.9 and 13.3) and eight waves with 16-block chunks on longer rows (Q4_0 896x4864 at M = 512: 22.4,
    // against 23.0 with 8-block chunks, 24.4 with four waves, 25.4 with 16-token workgroups). Long rows with too few
    // 32-token tiles take 16-token workgroups when they make about 192 (896x4864 at M = 256: 19.4 against 24.7
    // staged). Everywhere else (32 and 64 tokens, few row tiles) the LDS-staged kernel wins, also over the
    // register-chain kernel; it measured 4-12% under the LDS and register kernels at 32 tokens (q/k/v, o, gate/up,
    // down).
    const long row_tiles = (rows + 63) / 64;
    const long tiles32 = row_tiles * ((n + 31) / 32), tiles16 = row_tiles * ((n + 15) / 16);
    if (n >= 128 && tiles32 >= 192)
        return cols >= 2048 ? MmPlan{false, 1, 8, false, 0, true, 16, 32} : MmPlan{false, 1, 4, false, 0, true, 4, 32};
    if (n >= 128 && cols >= 2048 && tiles16 >= 192) return MmPlan{false, 1, 4, false, 0, true, 8, 16};
    return MmPlan{false, 1, 4, true};
}

template <int DT, int TT, int KC>
void launch_mm_lds(const MmSegs& sg, int row_tiles, const int8_t* xq, const float* xd, int cols, int n, hipStream_t s) {
    const int n_tg = (n + 16 * TT - 1) / (16 * TT);
    qh_launch((matmul_lds_kernel<DT, TT, KC>), dim3((unsigned)(row_tiles * n_tg)), dim3(kMmThreads), 0, s, sg, xq,
              xd, cols, n, n_tg);
}

template <int DT, int TT, int NW, bool VEC>
void launch_mm_reg(const MmSegs& sg, int row_tiles, const int8_t* xq, const float* xd, int cols, int n, hipStream_t s) {
    const int waves = (n + 16 * TT - 1) / (16 * TT);
    const int n_tg = (waves + NW - 1) / NW;
    qh_launch((matmul_reg_kernel<DT, TT, NW, VEC>), dim3((unsigned)(row_tiles * n_tg)), dim3(64 * NW), 0, s, sg, xq,
              xd, cols, n, n_tg);
}

}  // namespace

// The matrices of one launch: up to three of one dtype and width (row ranges [r0, r1) each), same activation.
hipError_t launch_matmul_segs(const MmOut* m, int n_mats, const int8_t* xq, const float* xd, int n, hipStream_t s) {
    if (n_mats < 1 || n_mats > 3) return hipErrorInvalidValue;
    MmSegs sg{};
    int row_tiles = 0;
    const qh_tensor& W = *m[0].W;
    for (int i = 0; i < n_mats; ++i) {
        const qh_tensor& Wi = *m[i].W;
        if (Wi.dtype != W.dtype || Wi.cols != W.cols) return hipErrorInvalidValue;
        const uint8_t* wq = static_cast<const uint8_t*>(Wi.data);
        sg.wq[i] = wq;
        sg.ws[i] = reinterpret_cast<const uint16_t*>(wq + qh_quant_bytes(Wi.dtype, Wi.rows, Wi.cols));
        sg.out[i] = m[i].out;
        sg.ldo[i] = m[i].ldo;
        sg.r0[i] = m[i].r0;
        sg.r1[i] = m[i].r1;
        sg.tiles[i] = (m[i].r1 - m[i].r0 + 15) / 16;
        row_tiles += sg.tiles[i];
    }
    const MmPlan pl = matmul_plan(row_tiles * 16, W.cols, n);
    const bool vec = (W.cols / QK) % 4 == 0 && (reinterpret_cast<uintptr_t>(xd) & 15u) == 0;
    bool aligned = (reinterpret_cast<uintptr_t>(xq) & 15u) == 0;
    for (int i = 0; i < n_mats; ++i) aligned = aligned && (reinterpret_cast<uintptr_t>(sg.wq[i]) & 15u) == 0;
    if (pl.tile && aligned) {
        MmSegs sg64 = sg;
        int row_tiles64 = 0;
        for (int i = 0; i < n_mats; ++i) {
            sg64.tiles[i] = (m[i].r1 - m[i].r0 + 63) / 64;
            row_tiles64 += sg64.tiles[i];
        }
        const int n_tg = (n + pl.ttile - 1) / pl.ttile;
        const dim3 grid((unsigned)(row_tiles64 * n_tg));
#define QH_MM_TILE(DT, KC, TT, NW)                                                                             \
    if (W.dtype == DT && pl.kc == KC && pl.ttile == TT && pl.nw == NW)                                                \
        qh_launch((matmul_tile_kernel<DT, KC, TT, NW, false>), grid, dim3(64 * NW), 0, s, sg64, xq, xd, W.cols, n, n_tg, \
                  (int8_t*)nullptr, (float*)nullptr);
        QH_MM_TILE(kQ8, 4, 64, 4) QH_MM_TILE(kQ8, 8, 64, 4) QH_MM_TILE(kQ4, 4, 64, 4) QH_MM_TILE(kQ4, 8, 64, 4)
        QH_MM_TILE(kQ8, 4, 32, 4) QH_MM_TILE(kQ8, 8, 32, 4) QH_MM_TILE(kQ4, 4, 32, 4) QH_MM_TILE(kQ4, 8, 32, 4)
        QH_MM_TILE(kQ8, 8, 16, 4) QH_MM_TILE(kQ4, 8, 16, 4) QH_MM_TILE(kQ8, 8, 32, 8) QH_MM_TILE(kQ4, 8, 32, 8)
        QH_MM_TILE(kQ8, 16, 32, 8) QH_MM_TILE(kQ4, 16, 32, 8)
#undef QH_MM_TILE
        return hipGetLastError();
    }
    if (pl.stage && aligned) {
        const int n_tg = (n + 15) / 16;
        // Register sets in flight: the two chunks of short rows, else pl.ns (default 2)
        const int ns = W.cols / QK <= 2 * kStKC ? 0 : pl.ns ? pl.ns : 2;
        const dim3 grid((unsigned)(row_tiles * n_tg));
#define QH_MM_STAGE(DT, NS)                                                                                \
    if (W.dtype == DT && ns == NS)                                                                         \
        qh_launch((matmul_stage_kernel<DT, NS>), grid, dim3(NS ? 2 * kMmThreads : kMmThreads), 0, s, sg, xq, xd, \
                  W.cols, n, n_tg);
        QH_MM_STAGE(kQ8, 0) QH_MM_STAGE(kQ8, 2) QH_MM_STAGE(kQ8, 3) QH_MM_STAGE(kQ8, 4)
        QH_MM_STAGE(kQ4, 0) QH_MM_STAGE(kQ4, 2) QH_MM_STAGE(kQ4, 3) QH_MM_STAGE(kQ4, 4)
#undef QH_MM_STAGE
        return hipGetLastError();
    }
    if (!pl.reg) {
#define QH_MM_LDS(DT, TT, KC)                                                  \
        if (W.dtype == DT && pl.tt == TT) {                                    \
            launch_mm_lds<DT, TT, KC>(sg, row_tiles, xq, xd, W.cols, n, s);    \
            return hipGetLastError();                                          \
        }
        QH_MM_LDS(kQ8, 1, 16) QH_MM_LDS(kQ8, 2, 16) QH_MM_LDS(kQ8, 4, 8)
        QH_MM_LDS(kQ4, 1, 16) QH_MM_LDS(kQ4, 2, 16) QH_MM_LDS(kQ4, 4, 8)
#undef QH_MM_LDS
        return hipErrorInvalidValue;
    }
#define QH_MM_REG(DT, TT, NW)                                                                \
    if (W.dtype == DT && pl.tt == TT && pl.nw == NW) {                                       \
        if (vec)                                                                             \
            launch_mm_reg<DT, TT, NW, true>(sg, row_tiles, xq, xd, W.cols, n, s);            \
        else                                                                                 \
            launch_mm_reg<DT, TT, NW, false>(sg, row_tiles, xq, xd, W.cols, n, s);           \
        return hipGetLastError();                                                            \
    }
    QH_MM_REG(kQ8, 1, 1) QH_MM_REG(kQ8, 1, 2) QH_MM_REG(kQ8, 1, 4) QH_MM_REG(kQ8, 2, 1) QH_MM_REG(kQ8, 2, 2)
    QH_MM_REG(kQ8, 2, 4) QH_MM_REG(kQ8, 4, 1) QH_MM_REG(kQ8, 4, 2) QH_MM_REG(kQ8, 4, 4)
    QH_MM_REG(kQ4, 1, 1) QH_MM_REG(kQ4, 1, 2) QH_MM_REG(kQ4, 1, 4) QH_MM_REG(kQ4, 2, 1) QH_MM_REG(kQ4, 2, 2)
    QH_MM_REG(kQ4, 2, 4) QH_MM_REG(kQ4, 4, 1) QH_MM_REG(kQ4, 4, 2) QH_MM_REG(kQ4, 4, 4)
#undef QH_MM_REG
    return hipErrorInvalidValue;
}

#if defined(QH_TIMELINE)
extern "C" int qh_timeline_mm_read(uint64_t* host, int n) {
    return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(qh_tl_mm), sizeof(uint64_t) * (size_t)n);
}
#endif

hipError_t launch_matmul(float* out, int ldo, const qh_tensor& W, const int8_t* xq, const float* xd, int n, int r0,
                         int r1, hipStream_t s) {
    const MmOut m{&W, out, ldo, r0, r1};
    return launch_matmul_segs(&m, 1, xq, xd, n, s);
}

hipError_t launch_matmul_swiglu(const qh_tensor& wg, const qh_tensor& wu, const int8_t* xq, const float* xd, int n,
                                int8_t* hq, float* hd, hipStream_t s) {
    const int F = wg.rows;
    if (wg.dtype != wu.dtype || (wg.dtype != kQ8 && wg.dtype != kQ4) || wu.rows != F || wu.cols != wg.cols ||
        F % QK != 0 || wg.cols % QK != 0 || wg.cols < 16 || n < 128)
        return hipErrorNotSupported;
    const MmPlan pl = matmul_plan(2 * F, wg.cols, n);
    if (!pl.tile || pl.nw != 4 || pl.kc != 4 || pl.ttile != 32) return hipErrorNotSupported;
    const uint8_t *qg = static_cast<const uint8_t*>(wg.data), *qu = static_cast<const uint8_t*>(wu.data);
    if (((reinterpret_cast<uintptr_t>(qg) | reinterpret_cast<uintptr_t>(qu) | reinterpret_cast<uintptr_t>(xq)) & 15u) != 0)
        return hipErrorNotSupported;
    MmSegs sg{};
    sg.wq[0] = qg;
    sg.wq[1] = qu;
    sg.ws[0] = reinterpret_cast<const uint16_t*>(qg + qh_quant_bytes(wg.dtype, F, wg.cols));
    sg.ws[1] = reinterpret_cast<const uint16_t*>(qu + qh_quant_bytes(wu.dtype, F, wu.cols));
    sg.r0[0] = 0;
    sg.r1[0] = F;
    sg.tiles[0] = F / QK;  // 32-row pairs: every tile in segment 0
    const int n_tg = (n + 31) / 32;
    const dim3 grid((unsigned)(F / QK * n_tg));
    if (wg.dtype == kQ8)
        qh_launch((matmul_tile_kernel<kQ8, 4, 32, 4, true>), grid, dim3(256), 0, s, sg, xq, xd, wg.cols, n, n_tg, hq, hd);
    else
        qh_launch((matmul_tile_kernel<kQ4, 4, 32, 4, true>), grid, dim3(256), 0, s, sg, xq, xd, wg.cols, n, n_tg, hq, hd);
    return hipGetLastError();
}

}  // namespace qh
