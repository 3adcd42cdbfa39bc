// GPU-resident decoder for the q4mix Qwen2-shaped model: the reference's Model::forward and forward_batch
// (engine/src/model.cpp:165-228, 349-433) with the operation order of its CPU build, so every hidden state, logit and
// greedy token is bit-identical to the reference.
//
// Decode (one token) runs five kernels per layer, each with its elementwise work fused in:
//   qkv        one launch for the q, k and v GEMVs (three row segments, same activation); every workgroup first runs
//              the layer's rmsnorm (serial FMA sum of squares, one rounded 1/sqrt) and quantizes the normed row into
//              its LDS (layer 0: the token's embedding row)                (model.cpp:179-182, ops_ref.cpp:195-199)
//   attention  one 16-wave workgroup per query head: biases, RoPE (host table of glibc powf/cosf/sinf of the
//              reference's formula), this token's f16 K/V row into the cache, scores (serial FMA dot over head_dim),
//              max, glibc-identical expf, serial sum in position order, normalise, serial weighted V sum in position
//              order, and the int8 quantization of the head's two 32-blocks of output
//                                                                         (model.cpp:115-137, 183-208, ops_ref.cpp:201-226)
//   o          GEMV and residual add                                     (model.cpp:207-209)
//   gate/up    the MLP's rmsnorm in every workgroup's prologue as above, one GEMV over the same rows of both matrices,
//              g / (1 + expf(-g)) * u, quantization                     (model.cpp:212-218, ops_ref.cpp:243-248)
//   down       GEMV and residual add                                     (model.cpp:219-221)
// then the final norm and the head (Exact Shortlist Head for top-k queries, full 8-bit head + argmax otherwise). The
// position and the token live on the device, so a decode step is a fixed launch sequence that can be captured in a HIP
// graph and replayed: the step reads the token the previous step chose, and its last kernel writes the new token,
// appends it to the output list and advances the position. A step at a position beyond the context writes nothing
// into the cache and raises bit 0 of the status word; a prompt token outside the vocabulary raises bit 1.
//
// Prefill (chunks of up to 32 tokens) uses the int8-MFMA matmul for every projection (q / k / v in one launch, gate /
// up in one launch) and an attention kernel over a (head, token) grid: a token's keys and values for the chunk's
// positions come from the chunk's own projections, so no kernel reads a cache row another workgroup of the same launch
// writes.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <type_traits>
#include <vector>

#include "qh_device.h"
#include "qh_gemv.h"
#include "qh_internal.h"
#include "qh_math.h"

namespace qh {

namespace {

constexpr int kChunk = 32;            // prefill chunk (reference Model::kBatch, model.h:52)
constexpr int kMaxStack = 1024;       // prefill stack limit (tokens whose matmuls share a launch)
constexpr int kMaxCtx = 8192;         // positions the attention kernel's score array holds
constexpr int kVStageBytes = 96 * 1024;  // LDS for staged V rows (768 rows at head_dim 64)
constexpr int kFuseLds = 65536;       // dynamic LDS limit of the fused GEMV kernels

// Positions the V cache holds per layer: the context rounded up to its 8-position blocks.
inline int v_ctx(int ctx) { return (ctx + 7) & ~7; }

// Floats per attention workgroup's exp row: the context rounded up to 16 (64-byte aligned rows) plus 64 of slack for
// whole-batch scalar reads past the last position.
inline int escr_stride(int ctx) { return ((ctx + 15) & ~15) + 64; }

enum { kStatusCtx = 1, kStatusToken = 2 };


__device__ __forceinline__ float h2f(uint16_t h) { return f16_to_f32(h); }

// A 16-byte register value as a native vector (register arrays of HIP's uint4 struct are not always split into
// registers by the compiler; native vectors are).
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
__device__ __forceinline__ v4u ld4(const void* p) { return *reinterpret_cast<const v4u*>(p); }

// LDS DMA (global_load_lds_dwordx4): lane l's 16 bytes at g go to lds_wave + 16 l, where lds_wave is the same LDS
// address in every lane of the wave. Counted by vmcnt; the LDS data is valid after s_waitcnt vmcnt(0). Issued in
// inline assembly, behind the compiler's back: the compiler counts a DMA it knows of as a transfer that may complete
// out of order, so after one it waits for every outstanding load (vmcnt(0)) before using any earlier load's result
// and before any LDS access. This way the earlier loads keep their waits, LDS accesses wait for nothing, the caller
// waits for the transfer itself (s_waitcnt vmcnt(0)) before reading its LDS, and the compiler's waits for loads
// issued before it become conservative (they also cover the transfers), never short. M0, which the transfer takes
// its LDS address from, is an input operand of the asm ("{m0}" constraint): the compiler writes it and knows what M0
// holds afterwards. The s_nop covers the wait state between an M0 write and the transfer that reads it. The body
// exists only in the device pass (the host pass cannot form an LDS address).
__device__ __forceinline__ void lds_dma16_async(const void* g, void* lds_wave) {
#if defined(__HIP_DEVICE_COMPILE__)
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds_wave);
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(m0) : "memory");
#endif
}
// f32 -> f16 (round to nearest even) of an already rounded f32 value, as the reference stores its f32 K / V results
// into the f16 cache. The empty asm makes the value opaque, so the compiler cannot fuse the FMA that produced it and
// this conversion into one v_fma_mixlo_f16, which rounds only once (straight to f16) and differs on double-rounding
// cases.
__device__ __forceinline__ uint16_t f2h(float f) {
    asm volatile("" : "+v"(f));
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// quantize_q8 of one 32-block held one value per lane of a half-wave (ops_ref.cpp:69-83): the block's absolute
// maximum / 127, codes rounded half away from zero. Every lane of the half-wave must be active.
// Maximum over the whole wave (every lane active) with the select o > a ? o : a at each step: DPP within rows of
// 16, then the gfx950 row swaps (16 and 32 lanes apart).
__device__ __forceinline__ float wave_max_sel(float a) {
    auto step = [](float x, float o) { return o > x ? o : x; };
    a = step(a, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a), 0xB1, 0xF, 0xF, false)));
    a = step(a, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a), 0x4E, 0xF, 0xF, false)));
    a = step(a, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a), 0x141, 0xF, 0xF, false)));
    a = step(a, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a), 0x140, 0xF, 0xF, false)));
    uint32_t u = __builtin_bit_cast(uint32_t, a);
    const auto s16 = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    a = step(__builtin_bit_cast(float, (uint32_t)s16[0]), __builtin_bit_cast(float, (uint32_t)s16[1]));
    u = __builtin_bit_cast(uint32_t, a);
    const auto s32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return step(__builtin_bit_cast(float, (uint32_t)s32[0]), __builtin_bit_cast(float, (uint32_t)s32[1]));
}

// The same for a block held four consecutive values per lane by an aligned group of 8 lanes (lane j of the group
// holds elements 4j .. 4j + 3): one 4-byte store of codes per lane.
__device__ __forceinline__ void quant_block_x8(float4 v, int8_t* __restrict__ q, float* __restrict__ d) {
    const float a = max8_lanes(__builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(v.x), __builtin_fabsf(v.y)),
                                               __builtin_fmaxf(__builtin_fabsf(v.z), __builtin_fabsf(v.w))));
    const float sc = a / 127.0f;
    const float inv = sc > 0.0f ? 1.0f / sc : 0.0f;
    const int j = (int)threadIdx.x & 7;
    const uint32_t c0 = (uint32_t)(uint8_t)(int8_t)(int)round_half_away(v.x * inv);
    const uint32_t c1 = (uint32_t)(uint8_t)(int8_t)(int)round_half_away(v.y * inv);
    const uint32_t c2 = (uint32_t)(uint8_t)(int8_t)(int)round_half_away(v.z * inv);
    const uint32_t c3 = (uint32_t)(uint8_t)(int8_t)(int)round_half_away(v.w * inv);
    *reinterpret_cast<uint32_t*>(q + 4 * j) = c0 | (c1 << 8) | (c2 << 16) | (c3 << 24);
    if (j == 0) *d = sc;
}

// quantize_q8 of the row xs[0, D) (16-byte aligned, D % 32 == 0) into q / d: 8 lanes per block, 32 blocks per pass
// of 256 threads.
__device__ __forceinline__ void quant_row_x8(const float* xs, int D, int8_t* __restrict__ q, float* __restrict__ d) {
    const int nb = D / QK;
    for (int t = (int)threadIdx.x; t < nb * 8; t += 256) {  // whole 8-lane groups
        const int b = t >> 3;
        quant_block_x8(reinterpret_cast<const float4*>(xs)[t], q + b * QK, d + b);
    }
}

// acc = op(acc, p[i]) for i = 0 .. n-1 in order, by one thread, over floats in LDS (16-byte aligned, n >= 1). A wave
// issues about one instruction per 4 cycles whatever its kind, so the loop is shaped for the fewest instructions
// per element: batches of 32 values read as 8 b128 at immediate offsets from one base, two register sets that
// alternate without copies (the next batch in flight while the current one is consumed), no clamping. It reads up
// to kChainPad floats past n: callers size the array n + kChainPad.
constexpr int kChainPad = 64;

// An LDS address the compiler treats as per-lane: uniform LDS addresses otherwise get rematerialized into a VGPR for
// every read, costing an instruction each (mbcnt_lo(0, 0) is 0 in every lane).
template <typename T>
__device__ __forceinline__ const T* lane_ptr(const T* p) {
    return p + __builtin_amdgcn_mbcnt_lo(0u, 0u);
}

template <typename Op>
__device__ __forceinline__ float lds_chain(const float* p, int n, Op op, float acc0 = 0.0f) {
    float4 a[8], b[8];
    auto ld = [](float4(&r)[8], const float* q) {
        const float4* q4 = reinterpret_cast<const float4*>(q);
#pragma unroll
        for (int k = 0; k < 8; ++k) r[k] = q4[k];
    };
    float acc = acc0;
    auto use = [&](const float4(&r)[8], int cnt) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            if (4 * k + 0 < cnt) acc = op(acc, r[k].x);
            if (4 * k + 1 < cnt) acc = op(acc, r[k].y);
            if (4 * k + 2 < cnt) acc = op(acc, r[k].z);
            if (4 * k + 3 < cnt) acc = op(acc, r[k].w);
        }
    };
    int j = 0;
    p = lane_ptr(p);
    ld(a, p);
    // sched_barrier keeps each prefetch ahead of the values it overlaps (the scheduler would sink it)
    for (; j + 64 <= n; j += 64) {
        ld(b, p + j + 32);
        __builtin_amdgcn_sched_barrier(0);
        use(a, 32);
        ld(a, p + j + 64);
        __builtin_amdgcn_sched_barrier(0);
        use(b, 32);
    }
    if (j + 32 <= n) {
        ld(b, p + j + 32);
        __builtin_amdgcn_sched_barrier(0);
        use(a, 32);
        use(b, n - j - 32);  // cnt is uniform
    } else {
        use(a, n - j);
    }
    return acc;
}

// R float4 per thread of a row of n4 <= 256 R float4 with every load issued before the first use: slot k holds
// element tid + 256 k (clamped onto the last element, so the loads are unconditional). Kernels take R = row_slots(n4):
// one load per thread up to D = 1024, eight (D <= 8192) above.
template <int R>
struct RowF4 {
    float4 v[R];
    __device__ __forceinline__ void load(const float* __restrict__ src, int n4) {
        const float4* s4 = reinterpret_cast<const float4*>(src);
#pragma unroll
        for (int k = 0; k < R; ++k) v[k] = s4[min((int)threadIdx.x + 256 * k, n4 - 1)];
    }
};
constexpr int row_slots(int n4) { return n4 <= 256 ? 1 : 8; }

// ------------------------------------------------------------------------------ segmented sum of squares
// rmsnorm's sum of squares is one serial chain, ss = fma(x_i, x_i, ss) for i = 0 .. D-1 in order (ops_ref.cpp:195-197):
// D dependent FMAs, the longest dependency of a decode layer. seg_sum_squares runs it as four segments at once, one
// per wave, and still returns the chain's value bit for bit:
//  - wave 0 runs segment 0 from 0;
//  - the wave of segment k >= 1 runs it from 64 start values at once, one per lane: the f32 rounding of the exact
//    (double) sum of squares before the segment, and its neighbours 32 below to 31 above in bit order. The chain's
//    value at the segment start differs from that guess only by the chain's own accumulated rounding (at most 26 ulps
//    over 2*10^5 random rows of 896, including rows with outliers), so some lane almost always started at exactly
//    the chain's value, and that lane's result is then the chain's value at the segment end;
//  - every thread then follows the chain from segment 0 through the lanes whose start matches bit for bit; a value
//    outside a window (rare) is continued by running that segment serially from it.
// The chains read x through scalar loads (x is in global memory and no workgroup writes it during the kernel): one
// 64-byte load feeds 16 FMAs of all 64 lanes with scalar operands, and the LDS stays free for the other waves.
// Scalar loads can return out of order, so the loop waits for everything outstanding after each 32-value batch,
// with the next batch already issued; each wave first touches every 64-byte line of its segment (SegWarm) so these
// loads hit the scalar cache.
typedef float v16f __attribute__((ext_vector_type(16)));
typedef const __attribute__((address_space(4))) v16f* const_v16f_ptr;
typedef const __attribute__((address_space(4))) uint32_t* const_u32_ptr;

// lgkmcnt(0) with the vector-memory and export counters left alone (gfx9 s_waitcnt encoding).
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xc07f); }

// acc = fma(g[i], g[i], acc) for i = 0 .. n-1 in order, g uniform across the wave and 64-byte aligned, n % 32 == 0.
__device__ __forceinline__ float ss_chain_scalar(const float* g, int n, float acc) {
    const_v16f_ptr p = (const_v16f_ptr)g;
    const int nv = n / 16;  // even
    v16f a0 = p[0], a1 = p[1];
    wait_lgkm0();
    __builtin_amdgcn_sched_barrier(0);
    int i = 0;
#pragma unroll 1
    for (; i + 4 <= nv; i += 4) {
        const v16f b0 = p[i + 2], b1 = p[i + 3];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < 16; ++k) acc = __builtin_fmaf(a0[k], a0[k], acc);
#pragma unroll
        for (int k = 0; k < 16; ++k) acc = __builtin_fmaf(a1[k], a1[k], acc);
        __builtin_amdgcn_sched_barrier(0);
        wait_lgkm0();
        __builtin_amdgcn_sched_barrier(0);
        a0 = p[min(i + 4, nv - 2)];
        a1 = p[min(i + 5, nv - 1)];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < 16; ++k) acc = __builtin_fmaf(b0[k], b0[k], acc);
#pragma unroll
        for (int k = 0; k < 16; ++k) acc = __builtin_fmaf(b1[k], b1[k], acc);
        __builtin_amdgcn_sched_barrier(0);
        wait_lgkm0();
        __builtin_amdgcn_sched_barrier(0);
    }
    if (i + 2 <= nv) {  // nv % 4 == 2: the last batch, loaded by the loop (or before it)
#pragma unroll
        for (int k = 0; k < 16; ++k) acc = __builtin_fmaf(a0[k], a0[k], acc);
#pragma unroll
        for (int k = 0; k < 16; ++k) acc = __builtin_fmaf(a1[k], a1[k], acc);
    }
    return acc;
}

// One scalar load per 64-byte line of the first 256 values of g[0, n): brings them into the scalar cache; the values
// are held until consume() so the loads cannot be dropped.
struct SegWarm {
    uint32_t v[16];
    __device__ __forceinline__ void issue(const float* g, int n) {
        const_u32_ptr q = (const_u32_ptr)g;
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = q[min(i * 16, n - 1)];
    }
    __device__ __forceinline__ void consume() const {
        asm volatile("" ::"s"(v[0]), "s"(v[1]), "s"(v[2]), "s"(v[3]), "s"(v[4]), "s"(v[5]), "s"(v[6]), "s"(v[7]));
        asm volatile("" ::"s"(v[8]), "s"(v[9]), "s"(v[10]), "s"(v[11]), "s"(v[12]), "s"(v[13]), "s"(v[14]), "s"(v[15]));
    }
};

// Sum over the wave of a double, in lane 63 (DPP: pairs, quads, half rows, rows, then rows 0+1 and 2+3 across).
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ double dpp_f64(double v) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, ROWS, 0xf, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, ROWS, 0xf, false);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ double wave_sum_lane63(double v) {
    v += dpp_f64<0xb1>(v);         // quad_perm [1,0,3,2]
    v += dpp_f64<0x4e>(v);         // quad_perm [2,3,0,1]
    v += dpp_f64<0x141>(v);        // row_half_mirror
    v += dpp_f64<0x140>(v);        // row_mirror
    v += dpp_f64<0x142, 0xa>(v);   // row_bcast:15 into rows 1, 3
    v += dpp_f64<0x143, 0xc>(v);   // row_bcast:31 into rows 2, 3
    return v;
}

// acc = op(acc, g[i]) for i = 0 .. n-1 in order (n >= 1), g uniform across the wave and 4-byte aligned. Whole
// batches of 32 values are read, so up to 32 values past n must be readable.
template <typename Op>
__device__ __forceinline__ float chain_scalar(const float* g, int n, float acc, Op op) {
    const_v16f_ptr p = (const_v16f_ptr)g;
    const int nb = n >> 5, rem = n & 31;
    auto use = [&](const v16f& x0, const v16f& x1, int cnt) {  // cnt is uniform
#pragma unroll
        for (int k = 0; k < 16; ++k)
            if (k < cnt) acc = op(acc, x0[k]);
#pragma unroll
        for (int k = 0; k < 16; ++k)
            if (16 + k < cnt) acc = op(acc, x1[k]);
    };
    v16f a0 = p[0], a1 = p[1];
    wait_lgkm0();
    __builtin_amdgcn_sched_barrier(0);
    int b = 0;
#pragma unroll 1
    for (; b + 2 <= nb; b += 2) {
        const v16f c0 = p[2 * b + 2], c1 = p[2 * b + 3];
        __builtin_amdgcn_sched_barrier(0);
        use(a0, a1, 32);
        __builtin_amdgcn_sched_barrier(0);
        wait_lgkm0();
        __builtin_amdgcn_sched_barrier(0);
        a0 = p[2 * b + 4];
        a1 = p[2 * b + 5];
        __builtin_amdgcn_sched_barrier(0);
        use(c0, c1, 32);
        __builtin_amdgcn_sched_barrier(0);
        wait_lgkm0();
        __builtin_amdgcn_sched_barrier(0);
    }
    if (b < nb) {  // a full batch in a, the partial one after it
        const v16f c0 = p[2 * b + 2], c1 = p[2 * b + 3];
        __builtin_amdgcn_sched_barrier(0);
        use(a0, a1, 32);
        __builtin_amdgcn_sched_barrier(0);
        wait_lgkm0();
        __builtin_amdgcn_sched_barrier(0);
        use(c0, c1, rem);
    } else {
        use(a0, a1, rem);
    }
    return acc;
}

// Four segments of a chain over n values, wave w running segment w: [0, b1), [b1, b1 + L), [b1 + L, b1 + 2 L),
// [b1 + 2 L, n).
struct Segs4 {
    int b1, L, n;
    __device__ __forceinline__ int start(int k) const { return k == 0 ? 0 : b1 + (k - 1) * L; }
    __device__ __forceinline__ int len(int k) const { return k == 0 ? b1 : k == 3 ? n - b1 - 2 * L : L; }
};

// Workgroup state of one segmented chain.
struct SegShared {
    double part[4][4];  // [wave][k]: the wave's share of the exact sum of the chain's terms below segment k's start
    float res[256];     // every lane's segment result
    uint32_t gbits[4];  // segment k's guess
};

// Sums three per-lane partials over the wave into part[wave][1..3]; a barrier must follow before seg_chain_run.
__device__ __forceinline__ void seg_partials(SegShared& sh, double p1, double p2, double p3) {
    p1 = wave_sum_lane63(p1);
    p2 = wave_sum_lane63(p2);
    p3 = wave_sum_lane63(p3);
    if ((threadIdx.x & 63) == 63) {
        const int w = (int)threadIdx.x >> 6;
        sh.part[w][1] = p1;
        sh.part[w][2] = p2;
        sh.part[w][3] = p3;
    }
}

// Runs the segments (wave 0 from 0, the wave of segment k from the 64 candidates around its guess), a barrier, then
// follows the chain through the candidates; returns the chain's end value in every thread. chain(k, start) runs
// segment k from start in the calling wave (k and start uniform across the wave) and returns its end value. All 256
// threads call it after the barrier that published part.
template <typename Chain>
__device__ __forceinline__ float seg_chain_run(SegShared& sh, Chain chain) {
    const int tid = (int)threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    float start = 0.0f;
    if (wave > 0) {
        const double g = sh.part[0][wave] + sh.part[1][wave] + sh.part[2][wave] + sh.part[3][wave];
        const uint32_t gb = __float_as_uint((float)g);
        start = __uint_as_float(gb + (uint32_t)lane - 32u);
        if (lane == 0) sh.gbits[wave] = gb;
    }
    sh.res[tid] = chain(wave, start);
    __syncthreads();
    float s = sh.res[0];
    const uint32_t g1 = sh.gbits[1], g2 = sh.gbits[2], g3 = sh.gbits[3];
#pragma unroll
    for (int k = 1; k < 4; ++k) {
        const uint32_t j = __float_as_uint(s) - (k == 1 ? g1 : k == 2 ? g2 : g3) + 32u;
        if (j < 64u)
            s = sh.res[64 * k + j];
        else
            s = chain(k, s);
    }
    return s;
}

// The chain's value ss of x[0, D) in every thread: segments [0, S0) and three of L = (D / 4) rounded down to a
// multiple of 32 (S0 = D - 3 L >= L). x: global, 64-byte aligned, not written during the kernel; xr: this thread's
// RowF4 of x; warm: seg_warm(x, D), issued by the same thread. All 256 threads of the workgroup call it (two barriers
// inside). D % 64 == 0, 128 <= D <= 8192.
__device__ __forceinline__ Segs4 seg_split(int D) {
    const int L = (D / 4) & ~31;
    return Segs4{D - 3 * L, L, D};
}
// The scalar loads that bring this wave's segment of x into the scalar cache (issued early, consumed by
// seg_sum_squares).
__device__ __forceinline__ SegWarm seg_warm(const float* __restrict__ x, int D) {
    const Segs4 sg = seg_split(D);
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    SegWarm warm;
    warm.issue(x + sg.start(wave), sg.len(wave));
    return warm;
}
template <int R>
__device__ float seg_sum_squares(const float* __restrict__ x, int D, const RowF4<R>& xr, const SegWarm& warm,
                                 int tlk = -1) {
    (void)tlk;
    __shared__ SegShared sh;
    const int tid = (int)threadIdx.x, n4 = D / 4;
    const Segs4 sg = seg_split(D);
    double p1 = 0.0, p2 = 0.0, p3 = 0.0;
#pragma unroll
    for (int k = 0; k < R; ++k) {
        const int i4 = tid + 256 * k;
        if (i4 < n4) {
            const float4 v = xr.v[k];
            const double s = (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
            const int e = 4 * i4;
            p1 += e < sg.start(1) ? s : 0.0;
            p2 += e < sg.start(2) ? s : 0.0;
            p3 += e < sg.start(3) ? s : 0.0;
        }
    }
    seg_partials(sh, p1, p2, p3);
    __syncthreads();
    QH_WSTAMP(tlk, 4);
    warm.consume();
    const float r = seg_chain_run(sh, [&](int k, float s0) { return ss_chain_scalar(x + sg.start(k), sg.len(k), s0); });
    QH_WSTAMP(tlk, 5);
    return r;
}

// seg_sum_squares for a row held in LDS (xs, complete, 16-byte aligned, kChainPad floats of slack; written in this
// kernel, so not readable through scalar loads): the same segments and candidate starts, each segment's chain reading
// its operands from LDS (the four waves' broadcast reads slow each other, ~12 cycles per element, against ~6 for
// scalar operands, still a quarter of the serial chain). xr: this thread's RowF4 of the row's values. All 256 threads
// call it (two barriers inside).
template <int R>
__device__ float seg_sum_squares_lds(const float* xs, int D, const RowF4<R>& xr) {
    __shared__ SegShared sh;
    const int tid = (int)threadIdx.x, n4 = D / 4;
    const Segs4 sg = seg_split(D);
    double p1 = 0.0, p2 = 0.0, p3 = 0.0;
#pragma unroll
    for (int k = 0; k < R; ++k) {
        const int i4 = tid + 256 * k;
        if (i4 < n4) {
            const float4 v = xr.v[k];
            const double s = (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
            const int e = 4 * i4;
            p1 += e < sg.start(1) ? s : 0.0;
            p2 += e < sg.start(2) ? s : 0.0;
            p3 += e < sg.start(3) ? s : 0.0;
        }
    }
    seg_partials(sh, p1, p2, p3);
    __syncthreads();
    return seg_chain_run(sh, [&](int k, float s0) {
        return lds_chain(xs + sg.start(k), sg.len(k), [](float acc, float v) { return __builtin_fmaf(v, v, acc); }, s0);
    });
}

// rmsnorm scale 1 / sqrt(ss / D + eps) (ops_ref.cpp:197-198).
__device__ __forceinline__ float rms_scale(float ss, int D, float eps) {
    return 1.0f / __builtin_sqrtf(ss / (float)D + eps);
}

// The sum of squares of xs[0, D) (LDS, complete, kChainPad floats of slack) by thread 0, in every thread.
__device__ __forceinline__ float lds_sum_squares(const float* xs, int D) {
    __shared__ float ss_sh;
    if (threadIdx.x == 0) ss_sh = lds_chain(xs, D, [](float acc, float v) { return __builtin_fmaf(v, v, acc); });
    __syncthreads();
    return ss_sh;
}

// y = x * scale * w of the row xs[0..D) (LDS; each thread reads and rewrites its own float4s, slot k = tid + 256 k),
// also to `normed` when given, then quantize_q8 of y. All 256 threads call it; xs is free after its return only
// after a barrier.
template <int R>
__device__ void normalize_quant_lds(float* xs, int D, float scale, const RowF4<R>& wr, int8_t* __restrict__ oq,
                                    float* __restrict__ od, float* __restrict__ normed) {
    const int tid = (int)threadIdx.x, n4 = D / 4;
    float4* x4 = reinterpret_cast<float4*>(xs);
#pragma unroll
    for (int k = 0; k < R; ++k) {
        const int i4 = tid + 256 * k;
        if (i4 < n4) {
            float4 xv = x4[i4];
            xv.x = xv.x * scale * wr.v[k].x;
            xv.y = xv.y * scale * wr.v[k].y;
            xv.z = xv.z * scale * wr.v[k].z;
            xv.w = xv.w * scale * wr.v[k].w;
            x4[i4] = xv;
            if (normed) reinterpret_cast<float4*>(normed)[i4] = xv;
        }
    }
    __syncthreads();
    quant_row_x8(xs, D, oq, od);
}

// rmsnorm of the row xs[0..D) (LDS, 16-byte aligned, complete) with weight w (loaded into wr by the caller before
// the row was complete, so its latency is hidden), then quantize_q8 of the normed row; also written to `normed`
// when given (ops_ref.cpp:195-199: ss += x*x as one FMA per element in order, scale = 1/sqrt(ss/n + eps),
// y = x * scale * w). Called by all 256 threads of a workgroup; D % 64 == 0, D <= 8192.
template <int R>
__device__ void norm_quant_lds(float* xs, int D, const RowF4<R>& wr, float eps, int8_t* __restrict__ oq,
                               float* __restrict__ od, float* __restrict__ normed) {
    normalize_quant_lds(xs, D, rms_scale(lds_sum_squares(xs, D), D, eps), wr, oq, od, normed);
}

// Activation fill for a GEMV tile whose input is rmsnorm(x) * w quantized (the decode step's q/k/v and gate/up
// inputs): every workgroup normalises the residual row itself, while its first pass of weight loads is in flight,
// and quantizes it straight into the tile's LDS codes / scales, so no kernel of its own and no cross-workgroup
// synchronisation is needed. With eq set, the row is instead the embedding of token *tok (the first layer), and
// workgroup 0 also stores it as the residual stream x_out. tmp: LDS scratch of D + kChainPad floats (16-byte
// aligned).
struct NormAct {
    static constexpr bool kGlobalScales = false;  // the scales are computed into LDS
    const float* x;
    const int8_t* eq;
    const uint16_t* es;
    const int32_t* tok;
    int V;
    float* x_out;
    int* status;
    const float* w;
    float eps;
    int D;
    float* tmp;
    int tlk;  // timeline id of the kernel (stamps compiled in only with QH_TIMELINE)

    // The loads the norm starts from (issued before the tile's weight loads, whose issue would otherwise hold them
    // up): the residual row and its scalar-cache warm-up, and the norm weight.
    template <int R>
    struct Pre {
        RowF4<R> wr, xr;
        SegWarm warm;
    };
    // EMB: the row is the embedding of *tok (eq set); the same loads whatever the branch below, so the compiler counts
    // the outstanding loads exactly where the row is first used.
    template <int R, bool EMB>
    __device__ __forceinline__ Pre<R> begin() const {
        Pre<R> p;
        load_row<R, EMB>(p.xr, (int)threadIdx.x, D / 4);
        if (!EMB && D >= 128) p.warm = seg_warm(x, D);  // uniform
        p.wr.load(w, D / 4);
        return p;
    }

    template <bool XL, int R, bool EMB>
    __device__ __forceinline__ void fill(const Pre<R>& p, int8_t* xs, float* xds) const {
        static_assert(XL, "the normed activation is produced in LDS");
        const int tid = (int)threadIdx.x, n4 = D / 4;
        const RowF4<R>& wr = p.wr;
        const RowF4<R>& xr = p.xr;
        float4* t4 = reinterpret_cast<float4*>(tmp);
        float ss;
        if (!EMB && D >= 128) {  // uniform
            ss = seg_sum_squares(x, D, xr, p.warm, tlk);
        } else {
#pragma unroll
            for (int k = 0; k < R; ++k) {
                const int i4 = tid + 256 * k;
                if (i4 < n4) {
                    t4[i4] = xr.v[k];
                    if (x_out && blockIdx.x == 0) reinterpret_cast<float4*>(x_out)[i4] = xr.v[k];
                }
            }
            __syncthreads();
            ss = lds_sum_squares(tmp, D);
        }
        const float scale = rms_scale(ss, D, eps);
        if constexpr (R == 1) {
            // thread t holds float4 t, so the 8-lane groups of quant_block_x8 are the row's 32-blocks: each thread
            // quantizes its own values, with no LDS round trip and no barrier (n4 % 8 == 0: whole groups)
            if (tid < n4) {
                float4 y = xr.v[0];
                y.x = y.x * scale * wr.v[0].x;
                y.y = y.y * scale * wr.v[0].y;
                y.z = y.z * scale * wr.v[0].z;
                y.w = y.w * scale * wr.v[0].w;
                quant_block_x8(y, xs + (tid >> 3) * QK, xds + (tid >> 3));
            }
        } else {
#pragma unroll
            for (int k = 0; k < R; ++k) {
                const int i4 = tid + 256 * k;
                if (i4 < n4) {
                    float4 y = xr.v[k];
                    y.x = y.x * scale * wr.v[k].x;
                    y.y = y.y * scale * wr.v[k].y;
                    y.z = y.z * scale * wr.v[k].z;
                    y.w = y.w * scale * wr.v[k].w;
                    t4[i4] = y;
                }
            }
            __syncthreads();
            quant_row_x8(tmp, D, xs, xds);
        }
    }

    // The row to normalise into xr: the embedding of *tok (EMB) or x.
    template <int R, bool EMB>
    __device__ __forceinline__ void load_row(RowF4<R>& xr, int tid, int n4) const {
        const int nb = D / QK;
        if constexpr (EMB) {
            int t = *tok;
            const bool bad = t < 0 || t >= V;
            if (bad && tid == 0 && blockIdx.x == 0) atomicOr(status, kStatusToken);
            t = bad ? 0 : t;
            const int8_t* er = eq + (size_t)t * D;
            const uint16_t* sr = es + (size_t)t * nb;
#pragma unroll
            for (int k = 0; k < R; ++k) {
                const int i4 = min(tid + 256 * k, n4 - 1);
                const uint32_t c4 = *reinterpret_cast<const uint32_t*>(er + 4 * i4);
                const float sc = h2f(sr[i4 / (QK / 4)]);
                xr.v[k].x = bad ? 0.0f : (float)(int8_t)(c4 & 0xff) * sc;
                xr.v[k].y = bad ? 0.0f : (float)(int8_t)((c4 >> 8) & 0xff) * sc;
                xr.v[k].z = bad ? 0.0f : (float)(int8_t)((c4 >> 16) & 0xff) * sc;
                xr.v[k].w = bad ? 0.0f : (float)(int8_t)(c4 >> 24) * sc;
            }
        } else {
            xr.load(x, n4);
        }
    }
};

// A NormAct with its row slots (R = row_slots(D / 4)) and row source (EMB: the embedding, eq set) fixed, in the
// interface gemv_tile takes.
template <int R, bool EMB>
struct NormActR {
    static constexpr bool kGlobalScales = false;
    NormAct a;
    template <bool XL>
    __device__ __forceinline__ NormAct::Pre<R> begin() const { return a.template begin<R, EMB>(); }
    template <bool XL>
    __device__ __forceinline__ void fill(const NormAct::Pre<R>& p, int8_t* xs, float* xds) const {
        a.template fill<XL, R, EMB>(p, xs, xds);
    }
};

// ------------------------------------------------------------------------------------------------------ kernels

// x[t] = embedding row of tokens[t] (get_row, ops_ref.cpp:162-192: F32 as stored, F16 converted, Q8_0 / Q4_0 code *
// f16 scale, all exact in f32), then the first layer's rmsnorm and quantization; the normed row also to normed[t]
// when given (the f32 input of unquantized matrices). One workgroup per token.
template <int R>
__global__ __launch_bounds__(256) void embed_norm_quant_kernel(const int32_t* __restrict__ tokens,
                                                               const uint8_t* __restrict__ emb, int dtype, int D,
                                                               int V, float* __restrict__ x,
                                                               const float* __restrict__ w, float eps,
                                                               int8_t* __restrict__ oq, float* __restrict__ od,
                                                               float* __restrict__ normed, int* __restrict__ status) {
    __shared__ __align__(16) float xs[8192 + kChainPad];
    const int t = blockIdx.x, tid = threadIdx.x;
    RowF4<R> wr;
    wr.load(w, D / 4);
    int tok = tokens[t];
    const bool bad = tok < 0 || tok >= V;
    if (bad) {
        if (tid == 0) atomicOr(status, kStatusToken);
        tok = 0;
    }
    const size_t nq = dtype == kQ4 ? (size_t)V * D / 2 : (size_t)V * D;  // quant bytes (both planes) before the scales
    const uint16_t* sr = reinterpret_cast<const uint16_t*>(emb + nq) + (size_t)tok * (D / QK);
    for (int i4 = tid; i4 < D / 4; i4 += 256) {  // elements 4 i4 .. 4 i4 + 3 (one block, one half of a Q4_0 block)
        float4 v;
        if (dtype == kF32) {
            v = reinterpret_cast<const float4*>(emb + (size_t)tok * D * 4)[i4];
        } else if (dtype == kF16) {
            const uint2 h = reinterpret_cast<const uint2*>(emb + (size_t)tok * D * 2)[i4];
            v = make_float4(h2f((uint16_t)(h.x & 0xffffu)), h2f((uint16_t)(h.x >> 16)), h2f((uint16_t)(h.y & 0xffffu)),
                            h2f((uint16_t)(h.y >> 16)));
        } else {
            const float sc = h2f(sr[i4 / (QK / 4)]);
            uint32_t c4;
            if (dtype == kQ8) {
                c4 = *reinterpret_cast<const uint32_t*>(emb + (size_t)tok * D + 4 * i4);
            } else if (dtype == kQ8P) {  // q = 16 (h + 8) + l - 128: the byte (h + 8) << 4 | l, top bit flipped
                const int e = 4 * i4, j = e % QK;
                const size_t off = (size_t)tok * D / 2 + (e / QK) * 16 + j % 16;
                const uint32_t hb = *reinterpret_cast<const uint32_t*>(emb + off);
                const uint32_t lb = *reinterpret_cast<const uint32_t*>(emb + (size_t)V * D / 2 + off);
                const uint32_t hn = j < 16 ? hb & 0x0F0F0F0Fu : (hb >> 4) & 0x0F0F0F0Fu;
                const uint32_t ln = j < 16 ? lb & 0x0F0F0F0Fu : (lb >> 4) & 0x0F0F0F0Fu;
                c4 = ((hn << 4) | ln) ^ 0x80808080u;
            } else {  // element j of a block: low nibble of byte j (j < 16), high nibble of byte j - 16
                const int e = 4 * i4, j = e % QK;
                const uint32_t b4 = *reinterpret_cast<const uint32_t*>(emb + (size_t)tok * D / 2 + (e / QK) * 16 + j % 16);
                c4 = nibbles_to_i8(j < 16 ? b4 & 0x0F0F0F0Fu : (b4 >> 4) & 0x0F0F0F0Fu);
            }
            v = make_float4((float)(int8_t)(c4 & 0xff) * sc, (float)(int8_t)((c4 >> 8) & 0xff) * sc,
                            (float)(int8_t)((c4 >> 16) & 0xff) * sc, (float)(int8_t)(c4 >> 24) * sc);
        }
        if (bad) v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        reinterpret_cast<float4*>(x + (size_t)t * D)[i4] = v;
        reinterpret_cast<float4*>(xs)[i4] = v;
    }
    __syncthreads();
    norm_quant_lds(xs, D, wr, eps, oq + (size_t)t * D, od + (size_t)t * (D / QK), normed ? normed + (size_t)t * D : nullptr);
}

// One workgroup per token: residual add x += o, then rmsnorm with weight w and int8 quantization of the normed row;
// the normed row is also written to normed[t] when given. D <= 8192.
template <int R>
__global__ __launch_bounds__(256) void add_rmsnorm_quant_kernel(float* __restrict__ x, const float* __restrict__ o,
                                                                const float* __restrict__ w, int D, float eps,
                                                                int8_t* __restrict__ xq, float* __restrict__ xd,
                                                                float* __restrict__ normed) {
    __shared__ __align__(16) float xs[8192 + kChainPad];
    const int t = blockIdx.x, tid = threadIdx.x, n4 = D / 4;
    RowF4<R> wr, xr, orow;
    wr.load(w, n4);
    xr.load(x + (size_t)t * D, n4);
    orow.load(o + (size_t)t * D, n4);
#pragma unroll
    for (int k = 0; k < R; ++k) {
        const int i4 = tid + 256 * k;
        if (i4 < n4) {
            float4 v = xr.v[k];
            v.x = v.x + orow.v[k].x;
            v.y = v.y + orow.v[k].y;
            v.z = v.z + orow.v[k].z;
            v.w = v.w + orow.v[k].w;
            xr.v[k] = v;
            reinterpret_cast<float4*>(x + (size_t)t * D)[i4] = v;
            reinterpret_cast<float4*>(xs)[i4] = v;
        }
    }
    __syncthreads();
    const float ss = D >= 128 ? seg_sum_squares_lds(xs, D, xr) : lds_sum_squares(xs, D);  // uniform
    normalize_quant_lds(xs, D, rms_scale(ss, D, eps), wr, xq + (size_t)t * D, xd + (size_t)t * (D / QK),
                        normed ? normed + (size_t)t * D : nullptr);
}

// Attention of token t (position pos0 + t) and query head h over positions [0, pos0 + t], for a chunk of n <= 32
// tokens whose raw projections are q [n][n_heads*HD], k / v [n][n_kv*HD]. One workgroup per (head, token).
// Cache layouts (f16 bits, per layer): K in 16-byte chunks of 8 dimensions, [n_kv][HD/8][ctx][8], so the lanes of a
// wave that read chunk c of 64 consecutive positions read 1 KB of contiguous memory (one row per lane, each lane's
// row complete after HD/8 reads); V in blocks of 8 positions, [pos/8][n_kv*HD][8], so one 16-byte read gives a lane 8
// consecutive positions of its dimension. Rows below pos0 come from the cache; the
// chunk's own rows are rebuilt from k / v (bias, RoPE, f16 rounding, exactly as stored), and workgroups of the first
// query head of each KV group store their token's row. The output (HD values) is quantized straight into oq / od
// ([n][n_heads*HD] codes, one scale per 32 values).
// WPE = 1: a 96 KB V stage, one workgroup per CU (one wave per SIMD, which lets the compiler keep three cached K rows
// per thread in registers). WPE = 2 (prefill chunks at head_dim 64): a 32 KB stage (256 rows) and two cached K rows
// per thread, so two workgroups share a CU (LDS under 80 KB, registers under 256 each) and the 448 workgroups of a
// 14-head chunk run in one round instead of two; their serial chains leave each SIMD mostly idle.
// Timeline stamps of the chunk's last token, query head 0 (compiled in only with -DQH_TIMELINE; the last launch's
// stamps stay in qh_tl_pa, qh_timeline_pa_read copies them out).
#if defined(QH_TIMELINE)
__device__ uint64_t qh_tl_pa[16];
#define QH_PASTAMP(i)                                                                                        \
    do {                                                                                                     \
        if (blockIdx.x == 0 && blockIdx.y == gridDim.y - 1 && threadIdx.x == 0) qh_tl_pa[i] = __builtin_readcyclecounter(); \
    } while (0)
#else
#define QH_PASTAMP(i) \
    do {              \
    } while (0)
#endif
template <int HD, int WPE = 1>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WPE, WPE))) void attention_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ bq, const float* __restrict__ bk, const float* __restrict__ bv,
    const float* __restrict__ cs, const int* __restrict__ pos_dev, int ctx, int n_heads, int n_kv,
    uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int8_t* __restrict__ oq, float* __restrict__ od,
    int* __restrict__ status, float* __restrict__ of, int single) {
    constexpr int HALF = HD / 2, CPR = HD / 8;           // 16-byte chunks per f16 K row
    constexpr int kVRows = (WPE == 1 ? kVStageBytes : 32 * 1024) / (HD * 2);  // V rows one LDS stage holds (mult. of 8)
    constexpr int kVBlk = kVRows / 8;                    // 8-row blocks per stage
    __shared__ __align__(16) float att[kMaxCtx + kChainPad];
    __shared__ __align__(16) uint4 vst[(kVBlk + 4) * HD];  // [block][dim] -> 8 rows; 4 blocks of read padding
    __shared__ __align__(16) uint16_t kloc[kChunk * HD];
    __shared__ __align__(16) uint16_t vloc[kChunk * HD];
    __shared__ __align__(16) float qs[HD];
    __shared__ float red[4];
    __shared__ float sum_sh;
    __shared__ uint64_t exptab[32];
    ExpTab et;
    et.load();
    // single: every token of a prefill stack is its own chunk (token y = blockIdx.y at position *pos_dev + y), its
    // earlier rows all in the cache already (kv_store_kernel), so the workgroup rebuilds only its own row and stores
    // none.
    const int h = blockIdx.x, y = blockIdx.y, t = single ? 0 : y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int pos0 = *pos_dev + (single ? y : 0), pos = pos0 + t, nrows = pos + 1;
    if (pos >= ctx || pos0 < 0) {  // uniform: a step past the context touches no cache row
        if (tid == 0 && h == 0) atomicOr(status, kStatusCtx);
        return;
    }
    const int qd = n_heads * HD, kvd = n_kv * HD, group = n_heads / n_kv, kvh = h / group;
    if (single) {  // uniform: this token's rows of the projections and of the output
        q += (size_t)y * qd;
        k += (size_t)y * kvd;
        v += (size_t)y * kvd;
        oq += (size_t)y * qd;
        od += (size_t)y * (qd / QK);
        if (of) of += (size_t)y * qd;
    }
    QH_PASTAMP(0);
    // V block b of this head: HD uint4 at vbase + b * kvd (in uint4 units, kvd / 8 per position... see vblock())
    const uint4* vc4 = reinterpret_cast<const uint4*>(vc);
    auto vchunk = [&](int blk, int d) { return (size_t)blk * kvd + kvh * HD + d; };  // uint4 index of (block, dim)
    // K chunk (8 dimensions, 16 bytes) c of position p of this KV head, in 16-byte units: [kv head][HD/8][ctx]
    auto kchunk = [&](int c, int p) { return ((size_t)kvh * CPR + c) * ctx + p; };

    // this token's q (this head), k and v (its KV head) rows among the chunk's projections
    const float* qsrc = q + (size_t)t * qd + h * HD;  // row r of k / v: ksrc + r * kvd
    const float* ksrc = k + kvh * HD;
    const float* vsrc = v + kvh * HD;
    const int nk = (t + 1) * HALF, nv = (t + 1) * HD;
    // q of this head with bias, rotated; keys and values of the chunk's tokens 0..t (model.cpp:183-195, rope
    // ops_ref.cpp:201-214: a*c - b*s and b*c + a*s with the reference build's contraction fma(a, c, -(b*s)) and
    // fma(b, c, a*s)). A pair's inputs: the raw values a = row[i], b = row[i + HALF], their biases, cos / sin.
    struct Pair {
        float a, b, ba, bb, c, s;
    };
    auto load_pair = [&](const float* row, const float* bias, int i, const float* crow) {
        Pair pr;
        pr.a = row[i];
        pr.b = row[i + HALF];
        pr.ba = bias ? bias[i] : 0.0f;
        pr.bb = bias ? bias[i + HALF] : 0.0f;
        pr.c = crow[2 * i];
        pr.s = crow[2 * i + 1];
        return pr;
    };
    auto rope = [](const Pair& pr, bool has_bias, float& lo, float& hi) {
        float a = pr.a, b = pr.b;
        if (has_bias) {
            a = a + pr.ba;
            b = b + pr.bb;
        }
        lo = __builtin_fmaf(a, pr.c, -(b * pr.s));
        hi = __builtin_fmaf(b, pr.c, a * pr.s);
    };
    const float* bqh = bq ? bq + h * HD : nullptr;
    const float* bkh = bk ? bk + kvh * HD : nullptr;
    // Every element this thread rebuilds is loaded before any is used (indices clamped, so every load is
    // unconditional and the loads are one round trip): K pair elements tid + 256 i and V elements tid + 256 i of the
    // chunk's rows 0..t. 256 is a multiple of HD, so a thread's elements share their dimension, and its biases.
    static_assert(256 % HD == 0, "a thread's rebuilt elements share one dimension");
    constexpr int KPT = kChunk * HALF / 256, VPT = kChunk * HD / 256;  // elements per thread at n = kChunk
    const int tq = min(tid, HALF - 1);
    const Pair qp = load_pair(qsrc, bqh, tq, cs + (size_t)pos * HD);
    const int ik = tid % HALF, iv = tid % HD;
    const float kba = bkh ? bkh[ik] : 0.0f, kbb = bkh ? bkh[ik + HALF] : 0.0f;
    const float vb = bv ? bv[kvh * HD + iv] : 0.0f;
    float ka[KPT], kb[KPT], vv[VPT];
    float2 kcs[KPT];
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
        const int rk = min(tid + 256 * i, nk - 1) / HALF;
        const float* row = ksrc + (size_t)rk * kvd;
        ka[i] = row[ik];
        kb[i] = row[ik + HALF];
        kcs[i] = *reinterpret_cast<const float2*>(cs + (size_t)(pos0 + rk) * HD + 2 * ik);
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) vv[i] = vsrc[(size_t)(min(tid + 256 * i, nv - 1) / HD) * kvd + iv];
    __builtin_amdgcn_sched_barrier(0);

    // This thread's cached K rows for the first score rows (registers) go out behind those (a load waits for every
    // load issued before it), and their issue, which stalls while the memory pipeline drains, covers the q / k / v
    // latency. No row read here is written by this launch: K rows stop below pos0.
    constexpr int kKPre = WPE == 1 ? 3 : 2;  // score rows per thread loaded up front (768 / 512 positions)
    const int grow = pos0 > 0 ? pos0 - 1 : 0;
    v4u kpre[kKPre][CPR];
#pragma unroll
    for (int r = 0; r < kKPre; ++r) {
        const uint16_t* kg = kc + (kchunk(0, min(tid + 256 * r, grow)) << 3);
#pragma unroll
        for (int i = 0; i < CPR; ++i) kpre[r][i] = ld4(kg + (size_t)i * ctx * 8);
    }
    if (tid < HALF) rope(qp, bq != nullptr, qs[tid], qs[tid + HALF]);
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
        const int e = tid + 256 * i;
        if (e < nk) {
            const int r = e / HALF;
            float lo, hi;
            rope(Pair{ka[i], kb[i], kba, kbb, kcs[i].x, kcs[i].y}, bk != nullptr, lo, hi);
            kloc[r * HD + ik] = f2h(lo);
            kloc[r * HD + ik + HALF] = f2h(hi);
        }
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int e = tid + 256 * i;
        if (e < nv) vloc[(e / HD) * HD + iv] = f2h(bv ? vv[i] + vb : vv[i]);
    }
    et.store(exptab);
    __syncthreads();
    QH_PASTAMP(1);
    if (!single && h % group == 0)
        for (int i = tid; i < HD; i += 256) {
            kc[(kchunk(i >> 3, pos) << 3) + (i & 7)] = kloc[t * HD + i];
            vc[vchunk(pos / 8, i) * 8 + (pos & 7)] = vloc[t * HD + i];
        }

    // scores: s = sum_i q_i * k_i as one FMA per element in order, then * scale (model.cpp:122-125)
    float qv[HD];
#pragma unroll
    for (int i = 0; i < HD; ++i) qv[i] = qs[i];
    const float scale = 1.0f / __builtin_sqrtf((float)HD);
    float mx = -__builtin_inff();
    // one dot product: s = fma(q_i, k_i, s) in dimension order
    auto dot_row = [&](const v4u(&kk)[CPR]) {
        float sc = 0.0f;
#pragma unroll
        for (int i = 0; i < CPR; ++i) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                sc = __builtin_fmaf(qv[i * 8 + 2 * e], h2f((uint16_t)(kk[i][e] & 0xffffu)), sc);
                sc = __builtin_fmaf(qv[i * 8 + 2 * e + 1], h2f((uint16_t)(kk[i][e] >> 16)), sc);
            }
        }
        return sc;
    };
    // the chunk's own rows j >= pos0 (keys in LDS)
    for (int j = pos0 + tid; j < nrows; j += 256) {
        v4u kk[CPR];
        const uint16_t* kl = kloc + (j - pos0) * HD;
#pragma unroll
        for (int i = 0; i < CPR; ++i) kk[i] = ld4(kl + i * 8);
        const float a = dot_row(kk) * scale;
        att[j] = a;
        mx = a > mx ? a : mx;
    }
    // The first stage's V blocks go straight into LDS (DMA, no registers), in two halves of the whole stage per wave
    // (clamped onto the last block, whose repeats write the same data): the first once the scores are done and the
    // second after the exp row (the issue of a half stalls its wave while the memory pipeline drains, so neither
    // holds up the scores, and the second is issued after the wait that completes the first). Everything is waited
    // for before the stage is built. Cache blocks stop below pos0: none is written by
    // this launch (the block holding pos0 carries stale rows from pos0 on, replaced when the stage is built).
    const int ncb = min((pos0 + 7) / 8, kVBlk);  // cache blocks of the first stage (the last may be partial)
    constexpr int kDmaPerBlk = HD / 64;          // 1 KB (one wave instruction) per DMA chunk
    constexpr int kVEarly = kVBlk * kDmaPerBlk / 4;  // DMA chunks per wave
    auto dma_v = [&](int e0, int e1) {           // chunks wave + 4 e, e in [e0, e1)
        const int last = max(ncb * kDmaPerBlk - 1, 0);
#pragma unroll
        for (int e = e0; e < e1; ++e) {
            const int c = min(wave + 4 * e, last);
            lds_dma16_async(vc4 + vchunk(c / kDmaPerBlk, (c % kDmaPerBlk) * 64 + lane), vst + c * 64);
        }
    };

    // the cached rows tid + 256 r (registers only), their chains interleaved; stored after the barrier below
    float sc[kKPre];
    {
#pragma unroll
        for (int r = 0; r < kKPre; ++r)  // uniform: no thread has a cached row tid + 256 r at or past pos0
            sc[r] = 256 * r < pos0 ? dot_row(kpre[r]) * scale : 0.0f;
#pragma unroll
        for (int r = 0; r < kKPre; ++r) {
            const int j = tid + 256 * r;
            if (j < pos0) mx = sc[r] > mx ? sc[r] : mx;
        }
    }
    for (int j = tid + 256 * kKPre; j < pos0; j += 256) {  // longer contexts: one row at a time
        v4u kk[CPR];
        const uint16_t* kg = kc + (kchunk(0, j) << 3);
#pragma unroll
        for (int i = 0; i < CPR; ++i) kk[i] = ld4(kg + (size_t)i * ctx * 8);
        const float a = dot_row(kk) * scale;
        att[j] = a;
        mx = a > mx ? a : mx;
    }
    // the maximum does not depend on the order of comparison
    QH_PASTAMP(2);
    mx = wave_max_sel(mx);
    if (lane == 0) red[wave] = mx;
    dma_v(0, kVEarly / 2);
#pragma unroll
    for (int r = 0; r < kKPre; ++r) {
        const int j = tid + 256 * r;
        if (j < pos0) att[j] = sc[r];
    }
    __syncthreads();
    mx = red[0];
    for (int w = 1; w < 4; ++w) mx = red[w] > mx ? red[w] : mx;
    QH_PASTAMP(3);
    // exp, kept in LDS, with each lane's exact partial sums below the segment starts
    const bool seg = nrows >= 128;  // uniform; shorter rows keep the single chain
    const int Ls = (nrows / 4) & ~15;
    const Segs4 sg{(nrows - 3 * Ls) & ~15, Ls, nrows};
    double p1 = 0.0, p2 = 0.0, p3 = 0.0;
    for (int j = tid; j < nrows; j += 256) {
        const float e = dev_expf(att[j] - mx, exptab);
        att[j] = e;
        p1 += j < sg.start(1) ? (double)e : 0.0;
        p2 += j < sg.start(2) ? (double)e : 0.0;
        p3 += j < sg.start(3) ? (double)e : 0.0;
    }
    QH_PASTAMP(4);
    __shared__ SegShared ssh;
    if (seg) seg_partials(ssh, p1, p2, p3);
    __builtin_amdgcn_s_waitcnt(0);  // the first half of the V DMA
    dma_v(kVEarly / 2, kVEarly);
    __syncthreads();
    // softmax sum in position order (ops_ref.cpp:220-224)
    auto add = [](float acc, float a) { return acc + a; };
    float sum;
    if (seg) {
        // segments read as LDS broadcasts (through scalar loads of a global copy written just before, the sum of
        // 512 positions took 2.3 us against 1.4 us)
        sum = seg_chain_run(ssh, [&](int k, float s0) { return lds_chain(att + sg.start(k), sg.len(k), add, s0); });
    } else {
        __syncthreads();
        if (tid == 0) sum_sh = lds_chain(att, nrows, add);
        __syncthreads();
        sum = sum_sh;
    }
    QH_PASTAMP(5);
    const float inv = 1.0f / sum;
    for (int j = tid; j < nrows; j += 256) {
        att[j] = att[j] * inv;
    }
    // the V DMA is complete before the barrier; then the chunk's rows that fall inside
    // the first stage are written over the DMA's blocks
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    uint16_t* vst16 = reinterpret_cast<uint16_t*>(vst);
    {
        const int s1 = min(nrows, kVRows);
        for (int e = tid; e < (s1 - pos0) * HD; e += 256) {  // empty when pos0 >= kVRows
            const int r = pos0 + e / HD, d = e % HD;
            vst16[((r >> 3) * HD + d) * 8 + (r & 7)] = vloc[(r - pos0) * HD + d];
        }
        __syncthreads();
    }
    QH_PASTAMP(6);

    // out_i = sum_j a_j * v_ji, one FMA per position in order (model.cpp:131-135): thread i per dimension, over
    // the rows of each LDS stage. The weights are broadcast LDS reads of att (every lane the same address), so a
    // batch of 32 positions is 4 V reads, 8 weight reads and 32 FMAs, the next batch's reads in flight while one is
    // consumed. (With scalar operands from a global copy of the weights, written just before, the first stage's
    // chain ran 1.4x slower at two workgroups per CU.) V reads past the stage stay inside its padding, weight reads
    // inside att's padding.
    // Past the first stage, the threads without a dimension load the next stage's cache blocks into registers while
    // the chain runs (kPreload: at most 12 16-byte units each), so only LDS stores stand between two stages.
    constexpr int kLoaders = 256 - HD, kPre = (kVBlk * HD + kLoaders - 1) / kLoaders;
    constexpr bool kPreload = kPre <= 12;
    uint4 nxt[kPreload ? kPre : 1];
    float acc = 0.0f;
    for (int s0 = 0;;) {
        const int se = min(nrows, s0 + kVRows);
        if (kPreload && tid >= HD && se < nrows) {  // uniform per wave; pos0 >= 1 here (a second stage)
            const int nb8 = (min(nrows, se + kVRows) - se + 7) / 8, lastc = (pos0 - 1) / 8;
#pragma unroll
            for (int u = 0; u < kPre; ++u) {
                const int c = tid - HD + kLoaders * u, blk = se / 8 + c / HD, d = c % HD;
                const uint4 x = vc4[vchunk(min(blk, lastc), d)];
                nxt[u] = c < nb8 * HD && blk * 8 < pos0 ? x : make_uint4(0u, 0u, 0u, 0u);
            }
        }
        if (tid < HD) {
            // The weights are LDS broadcast reads of att (one 16-byte read gives every lane 4 weights), a batch
            // ahead of the chain.
            const float4* ap = reinterpret_cast<const float4*>(att + s0);  // s0 is a multiple of 32
            auto ldv = [&](uint4(&vv)[4], float4(&w)[8], int jr) {  // rows s0 + jr .. + 31 (jr % 32 == 0)
                const uint4* vp = vst + (jr >> 3) * HD + tid;
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) vv[q4] = vp[q4 * HD];
#pragma unroll
                for (int q = 0; q < 8; ++q) w[q] = ap[jr / 4 + q];
            };
            auto use = [&](const uint4(&vv)[4], const float4(&w)[8], int cnt) {
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                    const uint32_t v[4] = {vv[q4].x, vv[q4].y, vv[q4].z, vv[q4].w};
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const int k = 8 * q4 + e;
                        const float4 wq = w[k >> 2];
                        const float wk = (k & 3) == 0 ? wq.x : (k & 3) == 1 ? wq.y : (k & 3) == 2 ? wq.z : wq.w;
                        if (k < cnt)
                            acc = __builtin_fmaf(wk, h2f((uint16_t)(e & 1 ? v[e >> 1] >> 16 : v[e >> 1] & 0xffffu)),
                                                 acc);
                    }
                }
            };
            const int n = se - s0;
            uint4 vA[4], vB[4];
            float4 wA[8], wB[8];
            // sched_barrier keeps each batch's reads ahead of the chain steps they overlap (the scheduler would sink
            // them next to their first use)
            ldv(vA, wA, 0);
            int jr = 0;
#pragma unroll 1
            for (; jr + 64 <= n; jr += 64) {
                ldv(vB, wB, jr + 32);
                __builtin_amdgcn_sched_barrier(0);
                use(vA, wA, 32);
                ldv(vA, wA, jr + 64);
                __builtin_amdgcn_sched_barrier(0);
                use(vB, wB, 32);
            }
            if (jr + 32 <= n) {
                ldv(vB, wB, jr + 32);
                __builtin_amdgcn_sched_barrier(0);
                use(vA, wA, 32);
                use(vB, wB, n - jr - 32);
            } else {
                use(vA, wA, n - jr);
            }
        }
        s0 = se;
        if (s0 >= nrows) break;
        __syncthreads();  // the stage is consumed; load rows [s0, min(nrows, s0 + kVRows)) (s0 % 8 == 0)
        const int sn = min(nrows, s0 + kVRows);
        const int nb8 = (sn - s0 + 7) / 8;
        if constexpr (kPreload) {
            if (tid >= HD) {
#pragma unroll
                for (int u = 0; u < kPre; ++u) {
                    const int c = tid - HD + kLoaders * u;
                    if (c < nb8 * HD) vst[c] = nxt[u];
                }
            }
        } else {
            for (int c = tid; c < nb8 * HD; c += 256) {  // whole cache blocks; the chunk's rows are written after
                const int blk = s0 / 8 + c / HD, d = c % HD;
                vst[c] = blk * 8 < pos0 ? vc4[vchunk(blk, d)] : make_uint4(0u, 0u, 0u, 0u);
            }
        }
        __syncthreads();
        for (int e = tid; e < (sn - max(s0, pos0)) * HD; e += 256) {
            const int r = max(s0, pos0) + e / HD, d = e % HD;
            vst16[(((r - s0) >> 3) * HD + d) * 8 + (r & 7)] = vloc[(r - pos0) * HD + d];
        }
        __syncthreads();
    }
    QH_PASTAMP(7);
    if (tid < HD) {  // quantize_q8 of the attention output, two 32-blocks per 64 dimensions
        const int col = h * HD + (tid & ~31);
        if (of) of[(size_t)t * qd + h * HD + tid] = acc;  // the f32 input of an unquantized o projection
        quant_block32(acc, oq + (size_t)t * qd + col, od + (size_t)t * (qd / QK) + col / QK);
    }
}

// The f16 cache rows of n tokens at positions *pos_dev .. + n - 1 (a prefill stack) from their projections k / v
// ([n][n_kv * HD]): bias, RoPE as a*c - b*s and b*c + a*s with the reference build's contraction
// (fma(a, c, -(b*s)), fma(b, c, a*s)), rounded to f16, exactly what attention_kernel rebuilds and stores
// (model.cpp:183-206, ops_ref.cpp:201-214), in the K chunk and V block layouts. One workgroup per token; positions
// past the context store nothing (attention_kernel raises the status).
template <int HD>
__global__ __launch_bounds__(256) void kv_store_kernel(const float* __restrict__ k, const float* __restrict__ v,
                                                       const float* __restrict__ bk, const float* __restrict__ bv,
                                                       const float* __restrict__ cs, const int* __restrict__ pos_dev,
                                                       int ctx, int n_kv, uint16_t* __restrict__ kc,
                                                       uint16_t* __restrict__ vc) {
    constexpr int HALF = HD / 2, CPR = HD / 8;
    const int t = blockIdx.x, tid = threadIdx.x, pos = *pos_dev + t;
    if (pos >= ctx || pos < 0) return;
    const int kvd = n_kv * HD;
    const float* krow = k + (size_t)t * kvd;
    const float* crow = cs + (size_t)pos * HD;
    for (int e = tid; e < n_kv * HALF; e += 256) {
        const int kvh = e / HALF, i = e % HALF;
        float a = krow[kvh * HD + i], b = krow[kvh * HD + i + HALF];
        if (bk) {
            a = a + bk[kvh * HD + i];
            b = b + bk[kvh * HD + i + HALF];
        }
        const float c = crow[2 * i], sn = crow[2 * i + 1];
        const float lo = __builtin_fmaf(a, c, -(b * sn)), hi = __builtin_fmaf(b, c, a * sn);
        const size_t base = (size_t)kvh * CPR * ctx;
        kc[((base + (size_t)(i >> 3) * ctx + pos) << 3) + (i & 7)] = f2h(lo);
        kc[((base + (size_t)((i + HALF) >> 3) * ctx + pos) << 3) + ((i + HALF) & 7)] = f2h(hi);
    }
    for (int e = tid; e < kvd; e += 256) {
        const float x = v[(size_t)t * kvd + e];
        vc[((size_t)(pos / 8) * kvd + e) * 8 + (pos & 7)] = f2h(bv ? x + bv[e] : x);
    }
}

// Attention of a prefill stack at head_dim 64 with kStackTok consecutive tokens of one query head per workgroup, once
// kv_store_kernel has stored every row of the stack, so the workgroup rebuilds nothing and its tokens share the K and
// V rows it reads: positions *pos_dev + y0 .. + kStackTok - 1 (y0 = kStackTok * blockIdx.y, tokens below n), all
// below kStackCtx. The same arithmetic and order as attention_kernel for each token (model.cpp:115-137,
// ops_ref.cpp:216-226): q with bias and RoPE in f32; wave i takes token i: its q as 64 scalar operands, lane l
// scores cached rows l, l + 64, ... up to the token's row count (s = fma(q_i, k_i, s) in dimension order, the f16 key
// as a mixed-precision operand, then * 1/sqrt(64)), the next row's key loaded while a row is scored; the maximum over
// the wave; glibc expf; the softmax sum in position order, its normalisation, and the weighted V chain over V rows
// staged in LDS (lane d for dimension d, the weights as LDS broadcast reads), the four tokens' chains on four SIMDs
// at once. The V stages' loads are issued a stage ahead (the first at the start), so their latency hides under the
// scores and the previous stage's chains. The output is quantized per 32-block. Its LDS holds two workgroups per CU,
// so the register budget is that of two waves per SIMD.
constexpr int kStackTok = 4;
constexpr int kStackCtx = 1024;
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void attention_stack_kernel(
    const float* __restrict__ q, const float* __restrict__ bq, const float* __restrict__ cs,
    const int* __restrict__ pos_dev, int n, int ctx, int n_heads, int n_kv, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, int8_t* __restrict__ oq, float* __restrict__ od, int* __restrict__ status,
    float* __restrict__ of) {
    constexpr int HD = 64, HALF = HD / 2, CPR = HD / 8, NTK = kStackTok;
    constexpr int kVRows = 256, kVBlk = kVRows / 8;  // V rows per LDS stage (32 KB)
    constexpr int kVPer = kVBlk * HD / 256;          // 16-byte V units per thread and stage
    __shared__ __align__(16) float att[NTK][kStackCtx + kChainPad];
    __shared__ __align__(16) uint4 vst[(kVBlk + 4) * HD];  // [block][dim] -> 8 rows; 4 blocks of read padding
    __shared__ __align__(16) float qs[NTK][HD];
    __shared__ uint64_t exptab[32];
    ExpTab et;
    et.load();
    // groups in reverse order: the longest (the stack's last tokens) are dispatched first, the short ones fill in
    const int h = blockIdx.x, y0 = ((int)gridDim.y - 1 - (int)blockIdx.y) * NTK, tid = threadIdx.x, lane = tid & 63,
              wave = tid >> 6;
    const int nt = min(NTK, n - y0);  // tokens of this workgroup (uniform)
    const int base = *pos_dev + y0;   // position of token 0
    const int nmax = base + nt;       // rows of the last token
    if (base < 0 || nmax > ctx || nmax > kStackCtx) {  // uniform; the host launches this only within both limits
        if (tid == 0) atomicOr(status, kStatusCtx);
        return;
    }
    const int qd = n_heads * HD, kvd = n_kv * HD, group = n_heads / n_kv, kvh = h / group;
    auto kchunk = [&](int c, int p) { return ((size_t)kvh * CPR + c) * ctx + p; };
    auto vchunk = [&](int blk, int d) { return (size_t)blk * kvd + kvh * HD + d; };
    const uint4* vc4 = reinterpret_cast<const uint4*>(vc);
    // V units of the stage at s0 (whole cache blocks of 8 positions below nmax) into registers, then into vst
    v4u vreg[kVPer];
    auto vload = [&](int s0) {  // units past the stage's blocks: re-reads, never stored
        const int nb8 = (min(nmax, s0 + kVRows) - s0 + 7) / 8;
#pragma unroll
        for (int k = 0; k < kVPer; ++k) {
            const int c = min(tid + 256 * k, nb8 * HD - 1);
            vreg[k] = ld4(vc4 + vchunk(s0 / 8 + c / HD, c % HD));
        }
    };
    auto vput = [&]() {  // the whole stage area (rows past the stage: never read)
#pragma unroll
        for (int k = 0; k < kVPer; ++k) *reinterpret_cast<v4u*>(&vst[tid + 256 * k]) = vreg[k];
    };
    vload(0);
    // q of token `wave` (lanes 0-31: one rotated pair each), with bias (model.cpp:183-195, ops_ref.cpp:201-214)
    if (wave < nt && lane < HALF) {
        const float* src = q + (size_t)(y0 + wave) * qd + h * HD;
        const float* crow = cs + (size_t)(base + wave) * HD;
        float a = src[lane], b = src[lane + HALF];
        if (bq) {
            a = a + bq[h * HD + lane];
            b = b + bq[h * HD + lane + HALF];
        }
        const float c = crow[2 * lane], sn = crow[2 * lane + 1];
        qs[wave][lane] = __builtin_fmaf(a, c, -(b * sn));
        qs[wave][lane + HALF] = __builtin_fmaf(b, c, a * sn);
    }
    et.store(exptab);
    __syncthreads();

    // wave tk: token tk's scores, maximum, exponentials, softmax sum in position order (ops_ref.cpp:220-224) and
    // normalisation, all within the wave (its rows of att are its own)
    const int tk = wave, nrows = base + tk + 1;
    if (tk < nt) {
        const float scale = 1.0f / __builtin_sqrtf((float)HD);
        const float qv = qs[tk][lane];
        float qsg[HD];  // q_i, wave-uniform
#pragma unroll
        for (int d = 0; d < HD; ++d) qsg[d] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, qv), d));
        float mx = -__builtin_inff();
        v4u kA[CPR], kB[CPR];
        auto kload = [&](v4u(&kk)[CPR], int j) {  // row j's key, clamped to the token's last row
            const uint16_t* kg = kc + (kchunk(0, min(j, nrows - 1)) << 3);
#pragma unroll
            for (int c = 0; c < CPR; ++c) kk[c] = ld4(kg + (size_t)c * ctx * 8);
        };
        auto score = [&](const v4u(&kk)[CPR], int j) {
            float sc = 0.0f;
#pragma unroll
            for (int c = 0; c < CPR; ++c)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    sc = __builtin_fmaf(qsg[8 * c + 2 * e], h2f((uint16_t)(kk[c][e] & 0xffffu)), sc);
                    sc = __builtin_fmaf(qsg[8 * c + 2 * e + 1], h2f((uint16_t)(kk[c][e] >> 16)), sc);
                }
            if (j < nrows) {
                const float a = sc * scale;
                att[tk][j] = a;
                mx = a > mx ? a : mx;
            }
        };
        kload(kA, lane);
        int j0 = 0;
        for (; j0 + 64 < nrows; j0 += 128) {
            kload(kB, j0 + 64 + lane);
            score(kA, j0 + lane);
            kload(kA, j0 + 128 + lane);
            score(kB, j0 + 64 + lane);
        }
        if (j0 < nrows) score(kA, j0 + lane);
        mx = wave_max_sel(mx);  // the maximum does not depend on the order of comparison
        __builtin_amdgcn_wave_barrier();
        for (int j = lane; j < nrows; j += 64) att[tk][j] = dev_expf(att[tk][j] - mx, exptab);
        __builtin_amdgcn_wave_barrier();
        const float sum = lds_chain(att[tk], nrows, [](float acc, float a) { return acc + a; });
        const float inv = 1.0f / sum;
        for (int j = lane; j < nrows; j += 64) att[tk][j] = att[tk][j] * inv;
    }
    // out_i = sum_j a_j * v_ji, one FMA per position in order (model.cpp:131-135): wave i, lane d, over the rows of
    // each V stage (whole cache blocks of 8 positions; rows past a token's count are never used)
    float acc = 0.0f;
    for (int s0 = 0; s0 < nmax; s0 += kVRows) {
        const int sn = min(nmax, s0 + kVRows);
        __syncthreads();  // the previous stage is consumed (and, for the first, the normalised rows are written)
        vput();
        if (s0 + kVRows < nmax) vload(s0 + kVRows);  // the next stage's loads run under this stage's chains
        __syncthreads();
        if (tk < nt && s0 < nrows) {
            const int n_ = min(nrows, sn) - s0;
            const float4* ap = reinterpret_cast<const float4*>(lane_ptr(att[tk] + s0));  // s0 % 32 == 0
            auto ldv = [&](uint4(&vv)[4], float4(&w)[8], int jr) {  // rows s0 + jr .. + 31 (jr % 32 == 0)
                const uint4* vp = vst + (jr >> 3) * HD + lane;
#pragma unroll
                for (int q4i = 0; q4i < 4; ++q4i) vv[q4i] = vp[q4i * HD];
#pragma unroll
                for (int qi = 0; qi < 8; ++qi) w[qi] = ap[jr / 4 + qi];
            };
            auto use = [&](const uint4(&vv)[4], const float4(&w)[8], int cnt) {
#pragma unroll
                for (int q4i = 0; q4i < 4; ++q4i) {
                    const uint32_t vw[4] = {vv[q4i].x, vv[q4i].y, vv[q4i].z, vv[q4i].w};
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const int kx = 8 * q4i + e;
                        const float4 wq = w[kx >> 2];
                        const float wk = (kx & 3) == 0 ? wq.x : (kx & 3) == 1 ? wq.y : (kx & 3) == 2 ? wq.z : wq.w;
                        if (kx < cnt)
                            acc = __builtin_fmaf(wk, h2f((uint16_t)(e & 1 ? vw[e >> 1] >> 16 : vw[e >> 1] & 0xffffu)),
                                                 acc);
                    }
                }
            };
            uint4 vA[4], vB[4];
            float4 wA[8], wB[8];
            ldv(vA, wA, 0);
            int jr = 0;
#pragma unroll 1
            for (; jr + 64 <= n_; jr += 64) {
                ldv(vB, wB, jr + 32);
                __builtin_amdgcn_sched_barrier(0);
                use(vA, wA, 32);
                ldv(vA, wA, jr + 64);
                __builtin_amdgcn_sched_barrier(0);
                use(vB, wB, 32);
            }
            if (jr + 32 <= n_) {
                ldv(vB, wB, jr + 32);
                __builtin_amdgcn_sched_barrier(0);
                use(vA, wA, 32);
                use(vB, wB, n_ - jr - 32);
            } else {
                use(vA, wA, n_ - jr);
            }
        }
    }
    if (tk < nt) {  // quantize_q8 of the output, two 32-blocks per 64 dimensions
        const size_t row = (size_t)(y0 + tk) * qd;
        const int col = h * HD + (lane & ~31);
        if (of) of[row + h * HD + lane] = acc;
        quant_block32(acc, oq + row + col, od + row / QK + col / QK);
    }
}

// Attention over an f32 KV cache (the reference's --kv-f32, model.cpp:96-104, 197-204: the cache keeps k / v as
// computed, no f16 rounding), laid out as the reference keeps it, [ctx][n_kv * head_dim] per layer. One 256-thread
// workgroup per (query head, token of the chunk), prefill and decode alike: the chunk's K / V rows 0..t are rebuilt
// from the projections (bias, RoPE) in LDS, so no workgroup reads a cache row another one writes; scores
// s = fma(q_i, k_i, s) in dimension order, * 1 / sqrt(head_dim); max; glibc expf; the sum in position order (four
// segments with candidate starts, as attention_kernel); normalise; out_i = fma(a_j, v_ji, out_i) in position order
// over V rows staged in LDS; the output quantized per 32-block (model.cpp:115-137, ops_ref.cpp:201-226).
template <int HD>
__global__ __launch_bounds__(256) void attention_f32_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ bq, const float* __restrict__ bk, const float* __restrict__ bv,
    const float* __restrict__ cs, const int* __restrict__ pos_dev, int ctx, int n_heads, int n_kv,
    float* __restrict__ kc, float* __restrict__ vc, int8_t* __restrict__ oq, float* __restrict__ od,
    int* __restrict__ status, float* __restrict__ of) {
    constexpr int HALF = HD / 2, C4 = HD / 4;
    constexpr int kVR = 16384 / HD;  // V rows per LDS stage (64 KB)
    __shared__ __align__(16) float att[kMaxCtx + kChainPad];
    __shared__ __align__(16) float vst[kVR * HD];
    __shared__ __align__(16) float kloc[kChunk * HD];
    __shared__ __align__(16) float vloc[kChunk * HD];
    __shared__ __align__(16) float qs[HD];
    __shared__ float red[4];
    __shared__ float sum_sh;
    __shared__ uint64_t exptab[32];
    __shared__ SegShared ssh;
    ExpTab et;
    et.load();
    const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int pos0 = *pos_dev, pos = pos0 + t, nrows = pos + 1;
    if (pos >= ctx || pos0 < 0) {  // uniform: a step past the context touches no cache row
        if (tid == 0 && h == 0) atomicOr(status, kStatusCtx);
        return;
    }
    const int qd = n_heads * HD, kvd = n_kv * HD, group = n_heads / n_kv, kvh = h / group;
    // add_bias, then rope: a * c - b * s and b * c + a * s with the reference build's contraction
    for (int e = tid; e < (t + 1) * HALF; e += 256) {
        const int r = e / HALF, i = e % HALF;
        const float* row = k + (size_t)r * kvd + kvh * HD;
        float a = row[i], b = row[i + HALF];
        if (bk) {
            a = a + bk[kvh * HD + i];
            b = b + bk[kvh * HD + i + HALF];
        }
        const float* crow = cs + (size_t)(pos0 + r) * HD;
        kloc[r * HD + i] = __builtin_fmaf(a, crow[2 * i], -(b * crow[2 * i + 1]));
        kloc[r * HD + i + HALF] = __builtin_fmaf(b, crow[2 * i], a * crow[2 * i + 1]);
    }
    for (int e = tid; e < (t + 1) * HD; e += 256) {
        const int r = e / HD, i = e % HD;
        const float x = v[(size_t)r * kvd + kvh * HD + i];
        vloc[e] = bv ? x + bv[kvh * HD + i] : x;
    }
    if (tid < HALF) {
        const float* row = q + (size_t)t * qd + h * HD;
        float a = row[tid], b = row[tid + HALF];
        if (bq) {
            a = a + bq[h * HD + tid];
            b = b + bq[h * HD + tid + HALF];
        }
        const float* crow = cs + (size_t)pos * HD;
        qs[tid] = __builtin_fmaf(a, crow[2 * tid], -(b * crow[2 * tid + 1]));
        qs[tid + HALF] = __builtin_fmaf(b, crow[2 * tid], a * crow[2 * tid + 1]);
    }
    et.store(exptab);
    __syncthreads();
    if (h % group == 0)
        for (int i = tid; i < HD; i += 256) {
            kc[(size_t)pos * kvd + kvh * HD + i] = kloc[t * HD + i];
            vc[(size_t)pos * kvd + kvh * HD + i] = vloc[t * HD + i];
        }
    // scores (model.cpp:122-125): cached rows below pos0 from the cache, the chunk's rows from LDS
    const float scale = 1.0f / __builtin_sqrtf((float)HD);
    const float4* q4 = reinterpret_cast<const float4*>(qs);
    float mx = -__builtin_inff();
    for (int j = tid; j < nrows; j += 256) {
        const float* kr = j < pos0 ? kc + (size_t)j * kvd + kvh * HD : kloc + (j - pos0) * HD;
        float sc = 0.0f;
#pragma unroll 4
        for (int c = 0; c < C4; ++c) {
            const float4 kk = reinterpret_cast<const float4*>(kr)[c], qq = q4[c];
            sc = __builtin_fmaf(qq.x, kk.x, sc);
            sc = __builtin_fmaf(qq.y, kk.y, sc);
            sc = __builtin_fmaf(qq.z, kk.z, sc);
            sc = __builtin_fmaf(qq.w, kk.w, sc);
        }
        const float a = sc * scale;
        att[j] = a;
        mx = a > mx ? a : mx;
    }
    mx = wave_max_sel(mx);  // the maximum does not depend on the order of comparison
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = red[0];
    for (int w = 1; w < 4; ++w) mx = red[w] > mx ? red[w] : mx;
    // exp, with each lane's exact partial sums below the segment starts; the sum in position order (ops_ref.cpp:216-226)
    const bool seg = nrows >= 128;  // uniform; shorter rows keep the single chain
    const int Ls = (nrows / 4) & ~15;
    const Segs4 sg{(nrows - 3 * Ls) & ~15, Ls, nrows};
    double p1 = 0.0, p2 = 0.0, p3 = 0.0;
    for (int j = tid; j < nrows; j += 256) {
        const float e = dev_expf(att[j] - mx, exptab);
        att[j] = e;
        p1 += j < sg.start(1) ? (double)e : 0.0;
        p2 += j < sg.start(2) ? (double)e : 0.0;
        p3 += j < sg.start(3) ? (double)e : 0.0;
    }
    if (seg) seg_partials(ssh, p1, p2, p3);
    __syncthreads();
    auto add = [](float acc, float a) { return acc + a; };
    float sum;
    if (seg) {
        sum = seg_chain_run(ssh, [&](int kk, float s0) { return lds_chain(att + sg.start(kk), sg.len(kk), add, s0); });
    } else {
        if (tid == 0) sum_sh = lds_chain(att, nrows, add);
        __syncthreads();
        sum = sum_sh;
    }
    const float inv = 1.0f / sum;
    for (int j = tid; j < nrows; j += 256) att[j] = att[j] * inv;
    // out_i = sum_j a_j * v_ji (model.cpp:131-135): thread i per dimension, V rows staged in LDS
    float acc = 0.0f;
    for (int s0 = 0; s0 < nrows; s0 += kVR) {
        const int sn = min(nrows, s0 + kVR);
        __syncthreads();  // the weights are final, the previous stage is consumed
        for (int e = tid; e < (sn - s0) * C4; e += 256) {
            const int r = s0 + e / C4, c = e % C4;
            const float* src = r < pos0 ? vc + (size_t)r * kvd + kvh * HD : vloc + (r - pos0) * HD;
            reinterpret_cast<float4*>(vst + (r - s0) * HD)[c] = reinterpret_cast<const float4*>(src)[c];
        }
        __syncthreads();
        if (tid < HD)
            for (int j = s0; j < sn; ++j) acc = __builtin_fmaf(att[j], vst[(j - s0) * HD + tid], acc);
    }
    if (tid < HD) {  // quantize_q8 of the attention output
        const int col = h * HD + (tid & ~31);
        if (of) of[(size_t)t * qd + h * HD + tid] = acc;  // the f32 input of an unquantized o projection
        quant_block32(acc, oq + (size_t)t * qd + col, od + (size_t)t * (qd / QK) + col / QK);
    }
}

// h = g / (1 + expf(-g)) * u (ops_ref.cpp:243-248) over a 256-value block, then the block's Walsh-Hadamard transform
// (FLAG_HADAMARD_DOWN, model.cpp:219, 424: fwht_blocks, ops_ref.cpp:228-241: butterflies v[j] = a + c, v[j + h] = a - c
// for h = 1, 2, .., 128, then * 1 / sqrt(256)) and the quantization of its 8 32-blocks for the down projection. Each
// butterfly adds or subtracts the same two values as the reference's loop, so the result does not depend on the
// order the butterflies of a stage run in. Grid (ffn_dim / 256, tokens).
__global__ __launch_bounds__(256) void swiglu_fwht_quant_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                                int F, int8_t* __restrict__ oq, float* __restrict__ od,
                                                                float* __restrict__ of) {
    __shared__ float vb[256];
    const int tid = threadIdx.x;
    const size_t b0 = (size_t)blockIdx.y * F + (size_t)blockIdx.x * 256;
    const float gv = g[b0 + tid];
    vb[tid] = gv / (1.0f + dev_expf(-gv)) * u[b0 + tid];
    __syncthreads();
    for (int hh = 1; hh < 256; hh *= 2) {
        const int j = (tid / hh) * 2 * hh + tid % hh;  // butterfly tid (< 128): v[j], v[j + hh]
        float a = 0.0f, c = 0.0f;
        if (tid < 128) {
            a = vb[j];
            c = vb[j + hh];
        }
        __syncthreads();
        if (tid < 128) {
            vb[j] = a + c;
            vb[j + hh] = a - c;
        }
        __syncthreads();
    }
    const float norm = 1.0f / __builtin_sqrtf(256.0f);
    const size_t blk = b0 + (tid & ~31);
    const float hv = vb[tid] * norm;
    if (of) of[b0 + tid] = hv;
    quant_block32(hv, oq + blk, od + blk / QK);
}

// ------------------------------------------------------------------------------ decode attention, 16 waves per head
// Timeline stamps for phase measurements: compiled in only with -DQH_TIMELINE (thread 0 of workgroup 0 records the
// shader clock at each stamp; qh_timeline_read copies them out).
#if defined(QH_TIMELINE)
__device__ uint64_t qh_tl[64];
#define QH_STAMP(i)                                                                    \
    do {                                                                               \
        if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) qh_tl[i] = __builtin_readcyclecounter(); \
    } while (0)
#else
#define QH_STAMP(i) \
    do {            \
    } while (0)
#endif

// Brings every 64-byte line of g[0, n) (g uniform across the wave, 4-byte aligned) into the scalar cache: one scalar
// load per line, all in flight at once, then one wait. The loads land in one scratch register, since only their
// cache fill matters.
__device__ __forceinline__ void warm_lines(const float* g, int n) {
#if defined(__HIP_DEVICE_COMPILE__)
    uint32_t sink;
    for (int i = 0; i < n; i += 16)
        asm volatile("s_load_dword %0, %1, 0x0" : "=s"(sink) : "s"(g + i) : "memory");
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#endif
}

// Workgroup state of a four-segment chain run by waves 0-3 of a 16-wave workgroup (seg16_*).
struct SegShared16 {
    double part[16][4];  // [wave][k]: the wave's share of the exact sum of the chain's terms below segment k's start
    float res[256];      // every lane's segment result (waves 0-3)
    uint32_t gbits[4];   // segment k's guess
};

// Sums three per-lane partials over the wave into part[wave][1..3]; a barrier must follow before seg16_run.
__device__ __forceinline__ void seg16_partials(SegShared16& sh, double p1, double p2, double p3) {
    p1 = wave_sum_lane63(p1);
    p2 = wave_sum_lane63(p2);
    p3 = wave_sum_lane63(p3);
    if ((threadIdx.x & 63) == 63) {
        const int w = (int)threadIdx.x >> 6;
        sh.part[w][1] = p1;
        sh.part[w][2] = p2;
        sh.part[w][3] = p3;
    }
}

// seg_chain_run for a 16-wave workgroup: waves 0-3 run the four segments (wave 0 from 0, wave k from the 64 candidates
// around its guess, the f32 rounding of the exact sum below the segment), the others wait at the barrier; then every
// thread follows the chain through the candidates and returns its end value. chain(k, start) runs segment k from
// start in the calling wave (k and start uniform across the wave). All 1024 threads call it after the barrier that
// published part.
template <typename Chain>
__device__ __forceinline__ float seg16_run(SegShared16& sh, Chain chain) {
    const int tid = (int)threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    if (wave < 4) {
        float start = 0.0f;
        if (wave > 0) {
            double g = 0.0;
#pragma unroll
            for (int w = 0; w < 16; ++w) g += sh.part[w][wave];
            const uint32_t gb = __float_as_uint((float)g);
            start = __uint_as_float(gb + (uint32_t)lane - 32u);
            if (lane == 0) sh.gbits[wave] = gb;
        }
        sh.res[tid] = chain(wave, start);
    }
    __syncthreads();
    float s = sh.res[0];
    const uint32_t g1 = sh.gbits[1], g2 = sh.gbits[2], g3 = sh.gbits[3];
#pragma unroll
    for (int k = 1; k < 4; ++k) {
        const uint32_t j = __float_as_uint(s) - (k == 1 ? g1 : k == 2 ? g2 : g3) + 32u;
        if (j < 64u)
            s = sh.res[64 * k + j];
        else
            s = chain(k, s);
    }
    return s;
}

// Decode attention of one token (position *pos_dev) for query head h = blockIdx.x over positions [0, pos], head_dim 64:
// the same arithmetic, order and cache layouts as attention_kernel with one token, spread over 16 waves. Every thread
// scores one cached row held in registers (rows beyond 1024 in a loop), the 16 waves share the V DMA of the first LDS
// stage (a few transfers each, issued after their scores, so the scores keep exact load waits), and the exp and
// normalisation run one position per thread. The serial softmax sum runs as four segments on waves 0-3 (seg16_run), the
// weighted V chain on wave 0 with the weights as scalar operands while the other waves bring the weight row into the
// scalar cache. Workgroups of the first query head of each KV group store the token's K / V row.
// Grid (group, n_kv) with group = n_heads / n_kv: query head h = blockIdx.y * group + blockIdx.x of KV head blockIdx.y,
// so no division is needed. The arguments the first loads need come first: the first 16 dwords arrive in registers at
// dispatch, the rest (and the grid's size) take a load.
template <int HD>
__global__ __launch_bounds__(1024) void attention_decode_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    uint16_t* __restrict__ kc, const int* __restrict__ pos_dev, int ctx, int group, const float* __restrict__ bq,
    const float* __restrict__ bk, int n_kv, const float* __restrict__ bv, const float* __restrict__ cs,
    uint16_t* __restrict__ vc, int8_t* __restrict__ oq, float* __restrict__ od, float* __restrict__ escr,
    int escr_stride, int* __restrict__ status, float* __restrict__ of) {
    static_assert(HD == 64, "one chain wave and one K row of 8 chunks per thread");
    constexpr int NT = 1024, NW = NT / 64;
    constexpr int HALF = HD / 2, CPR = HD / 8;
    constexpr int kVRows = kVStageBytes / (HD * 2);  // V rows one LDS stage holds (a multiple of 8)
    constexpr int kVBlk = kVRows / 8;                // 8-row blocks per stage
    __shared__ __align__(16) float att[kMaxCtx + kChainPad];
    __shared__ __align__(16) uint4 vst[(kVBlk + 4) * HD];  // [block][dim] -> 8 rows; 4 blocks of read padding
    __shared__ __align__(16) uint16_t kloc[HD];
    __shared__ __align__(16) uint16_t vloc[HD];
    __shared__ __align__(16) float qs[HD];
    __shared__ float red[NW];
    __shared__ float sum_sh;
    __shared__ uint64_t exptab[32];
    __shared__ SegShared16 ssh;
    QH_STAMP(0);
    QH_WSTAMP(1, 0);
    const int n_heads = group * n_kv;
    const int kvh = (int)blockIdx.y, h = kvh * group + (int)blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kvd = n_kv * HD;
    // The token's raw q (wave 0), k (wave 1) and v (wave 2) values and biases do not depend on the position: their
    // loads go out before it arrives.
    float pa = 0.0f, pb = 0.0f, ba = 0.0f, bb = 0.0f, pc = 0.0f, ps = 0.0f;
    if (wave < 2 && lane < HALF) {
        const float* src = wave == 0 ? q + h * HD : k + kvh * HD;
        const float* bias = wave == 0 ? (bq ? bq + h * HD : nullptr) : (bk ? bk + kvh * HD : nullptr);
        pa = src[lane];
        pb = src[lane + HALF];
        ba = bias ? bias[lane] : 0.0f;
        bb = bias ? bias[lane + HALF] : 0.0f;
    } else if (wave == 2) {
        pa = v[kvh * HD + lane];
        ba = bv ? bv[kvh * HD + lane] : 0.0f;
    }
    ExpTab et;
    et.load();
    const uint4* vc4 = reinterpret_cast<const uint4*>(vc);
    auto vchunk = [&](int blk, int d) { return (size_t)blk * kvd + kvh * HD + d; };  // uint4 index of (block, dim)
    auto kchunk = [&](int c, int p) { return ((size_t)kvh * CPR + c) * ctx + p; };    // 16-byte K chunk c of row p
    // The position (a scalar load, back before the vector loads above), then this thread's K row: cached rows only
    // (tid < pos; row pos is the token's own, written by this launch). The K rows are the largest of the kernel's first
    // transfers and one CU issues them at ~40 bytes per cycle, so rows past the position are not read.
    const int pos = *pos_dev, nrows = pos + 1;
    if (pos >= ctx || pos < 0) {  // uniform: a step past the context touches no cache row
        if (tid == 0 && h == 0) atomicOr(status, kStatusCtx);
        return;
    }
    v4u kk[CPR];
    if (tid < pos) {
        const uint16_t* kg = kc + (kchunk(0, tid) << 3);
#pragma unroll
        for (int i = 0; i < CPR; ++i) kk[i] = ld4(kg + (size_t)i * ctx * 8);
    }
    QH_STAMP(8);
    // Then the RoPE angles of the position (ops_ref.cpp:201-214, with the reference build's contraction).
    if (wave < 2 && lane < HALF) {
        const float* crow = cs + (size_t)pos * HD;
        pc = crow[2 * lane];
        ps = crow[2 * lane + 1];
    }
    const bool has_bias = wave == 0 ? bq != nullptr : wave == 1 ? bk != nullptr : bv != nullptr;
    if (wave < 2 && lane < HALF) {
        float a = pa, b = pb;
        if (has_bias) {
            a = a + ba;
            b = b + bb;
        }
        const float lo = __builtin_fmaf(a, pc, -(b * ps)), hi = __builtin_fmaf(b, pc, a * ps);
        QH_STAMP(9);
        if (wave == 0) {
            qs[lane] = lo;
            qs[lane + HALF] = hi;
        } else {
            kloc[lane] = f2h(lo);
            kloc[lane + HALF] = f2h(hi);
        }
    } else if (wave == 2) {
        vloc[lane] = f2h(has_bias ? pa + ba : pa);
    }
    et.store(exptab);
    __syncthreads();
    QH_STAMP(1);
    if (h % group == 0 && tid < HD) {
        kc[(kchunk(tid >> 3, pos) << 3) + (tid & 7)] = kloc[tid];
        vc[vchunk(pos / 8, tid) * 8 + (pos & 7)] = vloc[tid];
    }

    // scores s_j = (sum_i q_i * k_ji as one FMA per element in dimension order) * (1 / sqrt(HD)) (model.cpp:122-125);
    // q comes from LDS by broadcast reads (every lane the same address), which keeps the kernel within the 128
    // registers a 16-wave workgroup allows
    const float scale = 1.0f / __builtin_sqrtf((float)HD);
    const float4* q4 = reinterpret_cast<const float4*>(lane_ptr(qs));
    auto dot_row = [&](const v4u(&r)[CPR], const float4* q4) {
        float sc = 0.0f;
#pragma unroll
        for (int i = 0; i < CPR; ++i) {
            const float4 qa = q4[2 * i], qb = q4[2 * i + 1];
            const float qq[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                sc = __builtin_fmaf(qq[2 * e], h2f((uint16_t)(r[i][e] & 0xffffu)), sc);
                sc = __builtin_fmaf(qq[2 * e + 1], h2f((uint16_t)(r[i][e] >> 16)), sc);
            }
        }
        return sc;
    };
    float mx = -__builtin_inff();
    if (tid < nrows) {  // row tid: the cached row in registers, or the token's own row (tid == pos)
        if (tid == pos) {
#pragma unroll
            for (int i = 0; i < CPR; ++i) kk[i] = ld4(kloc + i * 8);
        }
        const float a = dot_row(kk, q4) * scale;
        att[tid] = a;
        mx = a;
    }
    if (pos >= NT) {  // contexts beyond NT positions: the other cached rows one at a time, then the token's own row
        for (int j = tid + NT; j < pos; j += NT) {
            const uint16_t* kg = kc + (kchunk(0, j) << 3);
#pragma unroll
            for (int i = 0; i < CPR; ++i) kk[i] = ld4(kg + (size_t)i * ctx * 8);
            const float4* qo = q4;
            asm volatile("" : "+v"(qo));  // keeps the q reads inside the loop (hoisted, they would not fit)
            const float a = dot_row(kk, qo) * scale;
            att[j] = a;
            mx = a > mx ? a : mx;
        }
        if (tid == pos % NT) {
#pragma unroll
            for (int i = 0; i < CPR; ++i) kk[i] = ld4(kloc + i * 8);
            const float a = dot_row(kk, q4) * scale;
            att[pos] = a;
            mx = a > mx ? a : mx;
        }
    }
    QH_STAMP(2);
    mx = wave_max_sel(mx);  // the maximum does not depend on the order of comparison
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) mx = red[w] > mx ? red[w] : mx;
    QH_STAMP(3);
    // exp (the exp row also goes to global memory for the segmented sum's scalar loads), with each lane's exact partial
    // sums below the segment starts
    float* erow = escr + (size_t)h * escr_stride;
    float* arow = escr + (size_t)(n_heads + h) * escr_stride;
    const bool seg = nrows >= 128;  // uniform; shorter rows keep the single chain
    const int Ls = (nrows / 4) & ~15;
    const Segs4 sg{(nrows - 3 * Ls) & ~15, Ls, nrows};
    double p1 = 0.0, p2 = 0.0, p3 = 0.0;
    for (int j = tid; j < nrows; j += NT) {
        const float e = dev_expf(att[j] - mx, exptab);
        att[j] = e;
        erow[j] = e;
        p1 += j < sg.start(1) ? (double)e : 0.0;
        p2 += j < sg.start(2) ? (double)e : 0.0;
        p3 += j < sg.start(3) ? (double)e : 0.0;
    }
    QH_STAMP(10);
    if (seg) seg16_partials(ssh, p1, p2, p3);
    QH_STAMP(11);
    __builtin_amdgcn_s_waitcnt(0);  // the exp row's stores (read through scalar loads after the barrier)
    QH_STAMP(12);
    __syncthreads();
    QH_STAMP(4);
    // The first stage's V blocks straight into LDS by DMA while waves 0-3 run the softmax sum: waves 4-15 take 1 KB
    // chunks wave - 4, wave + 8, ... (clamped onto the last chunk, whose repeats write the same data). A wave's DMA
    // issue waits while the memory pipeline drains, so the chain waves issue none. Cache blocks stop below pos: the
    // block holding pos, if any, carries a stale row pos that the stage build replaces. The normalisation's
    // s_waitcnt(0) completes the transfers before the barrier that precedes the V chain.
    const int ncb = min((pos + 7) / 8, kVBlk);
    if (wave >= 4) {
        constexpr int kDmaWaves = NW - 4, kPerWave = (kVBlk + kDmaWaves - 1) / kDmaWaves;
        const int last = max(ncb - 1, 0);
#pragma unroll
        for (int e = 0; e < kPerWave; ++e) {
            const int c = min(wave - 4 + kDmaWaves * e, last);
            lds_dma16_async(vc4 + vchunk(c, lane), vst + c * 64);
        }
    }
    // softmax sum in position order (ops_ref.cpp:220-224)
    auto add = [](float acc, float a) { return acc + a; };
    float sum;
    if (seg) {
        sum = seg16_run(ssh, [&](int kk_, float s0) {
            warm_lines(erow + sg.start(kk_), sg.len(kk_));  // the exp row was just written: not in the scalar cache
            return chain_scalar(erow + sg.start(kk_), sg.len(kk_), s0, add);
        });
    } else {
        if (tid == 0) sum_sh = lds_chain(att, nrows, add);
        __syncthreads();
        sum = sum_sh;
    }
    QH_STAMP(5);
    const float inv = 1.0f / sum;
    for (int j = tid; j < nrows; j += NT) {
        const float a = att[j] * inv;
        att[j] = a;
        arow[j] = a;
    }
    QH_STAMP(13);
    // the weight row's stores and the V DMA complete before the barrier; then the token's own row, if it falls inside
    // the first stage, is written over the DMA's block
    __builtin_amdgcn_s_waitcnt(0);
    QH_STAMP(14);
    __syncthreads();
    uint16_t* vst16 = reinterpret_cast<uint16_t*>(vst);
    if (pos < kVRows && tid < HD) vst16[((pos >> 3) * HD + tid) * 8 + (pos & 7)] = vloc[tid];
    __syncthreads();
    QH_STAMP(6);

    // out_i = sum_j a_j * v_ji, one FMA per position in order (model.cpp:131-135): lane i of wave 0 per dimension,
    // the weights as scalar operands (as in attention_kernel); the other waves warm the weight row's lines.
    float acc = 0.0f;
    for (int s0 = 0;;) {
        const int se = min(nrows, s0 + kVRows);
        if (tid < HD) {
            const_v16f_ptr wp = (const_v16f_ptr)(arow + s0);  // s0 is a multiple of 32: 64-byte aligned
            auto ldv = [&](uint4(&vv)[4], int jr) {  // rows s0 + jr .. + 31 (jr % 32 == 0)
                const uint4* vp = vst + (jr >> 3) * HD + tid;
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) vv[q4] = vp[q4 * HD];
            };
            auto use = [&](const uint4(&vv)[4], const v16f& w0, const v16f& w1, int cnt) {
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                    const uint32_t w[4] = {vv[q4].x, vv[q4].y, vv[q4].z, vv[q4].w};
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const int kx = 8 * q4 + e;
                        if (kx < cnt)
                            acc = __builtin_fmaf(kx < 16 ? w0[kx & 15] : w1[kx & 15],
                                                 h2f((uint16_t)(e & 1 ? w[e >> 1] >> 16 : w[e >> 1] & 0xffffu)), acc);
                    }
                }
            };
            const int n = se - s0;
            uint4 vA[4], vB[4];
            v16f wA0 = wp[0], wA1 = wp[1], wB0, wB1;
            ldv(vA, 0);
            int jr = 0;
#pragma unroll 1
            for (; jr + 64 <= n; jr += 64) {
                wait_lgkm0();
                __builtin_amdgcn_sched_barrier(0);
                wB0 = wp[(jr + 32) / 16];
                wB1 = wp[(jr + 32) / 16 + 1];
                ldv(vB, jr + 32);
                __builtin_amdgcn_sched_barrier(0);
                use(vA, wA0, wA1, 32);
                wait_lgkm0();
                __builtin_amdgcn_sched_barrier(0);
                wA0 = wp[(jr + 64) / 16];
                wA1 = wp[(jr + 64) / 16 + 1];
                ldv(vA, jr + 64);
                __builtin_amdgcn_sched_barrier(0);
                use(vB, wB0, wB1, 32);
            }
            wait_lgkm0();
            __builtin_amdgcn_sched_barrier(0);
            if (jr + 32 <= n) {
                wB0 = wp[(jr + 32) / 16];
                wB1 = wp[(jr + 32) / 16 + 1];
                ldv(vB, jr + 32);
                __builtin_amdgcn_sched_barrier(0);
                use(vA, wA0, wA1, 32);
                wait_lgkm0();
                __builtin_amdgcn_sched_barrier(0);
                use(vB, wB0, wB1, n - jr - 32);
            } else {
                use(vA, wA0, wA1, n - jr);
            }
        } else if (s0 == 0) {  // the other waves: 16 lines of the weight row per scalar-load batch
            const int wi = __builtin_amdgcn_readfirstlane(wave - 1);
            for (int b = wi * 256; b < nrows; b += (NW - 1) * 256) {
                SegWarm warm;
                warm.issue(arow + b, nrows - b);
                warm.consume();
            }
        }
        s0 = se;
        if (s0 >= nrows) break;
        __syncthreads();  // the stage is consumed; load rows [s0, min(nrows, s0 + kVRows)) (s0 % 8 == 0)
        const int sn = min(nrows, s0 + kVRows);
        const int nb8 = (sn - s0 + 7) / 8;
        for (int c = tid; c < nb8 * HD; c += NT) {  // whole cache blocks; the token's row is written after
            const int blk = s0 / 8 + c / HD, d = c % HD;
            vst[c] = blk * 8 < pos ? vc4[vchunk(blk, d)] : make_uint4(0u, 0u, 0u, 0u);
        }
        __syncthreads();
        if (pos >= s0 && pos < sn && tid < HD) vst16[(((pos - s0) >> 3) * HD + tid) * 8 + (pos & 7)] = vloc[tid];
        __syncthreads();
    }
    QH_STAMP(7);
    QH_WSTAMP(1, 3);
    if (tid < HD) {  // quantize_q8 of the attention output, two 32-blocks per 64 dimensions
        const int col = h * HD + (tid & ~31);
        if (of) of[h * HD + tid] = acc;  // the f32 input of an unquantized o projection
        quant_block32(acc, oq + col, od + col / QK);
    }
}

// h = g / (1 + expf(-g)) * u (ops_ref.cpp:243-248) over n_blocks 32-blocks, quantized per block.
__global__ __launch_bounds__(256) void swiglu_quant_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                           long n_blocks, int8_t* __restrict__ oq,
                                                           float* __restrict__ od, float* __restrict__ of) {
    const long blk = ((long)blockIdx.x * 256 + threadIdx.x) >> 5;
    if (blk >= n_blocks) return;  // whole half-waves leave together
    const long i = blk * QK + (threadIdx.x & 31);
    const float gv = g[i];
    const float hv = gv / (1.0f + dev_expf(-gv)) * u[i];
    if (of) of[i] = hv;  // the f32 input of an unquantized down projection
    quant_block32(hv, oq + blk * QK, od + blk);
}

// Prefill gate / up, SwiGLU and quantization of the down projection's input in one launch (model.cpp:212-218 for a
// chunk of n tokens; ops_ref.cpp:122-160, 243-248, 69-83). Workgroup (b, g): rows [32 b, 32 b + 32) of gate and of up
// for tokens [16 g, 16 g + 16). The chunk's 64 weight rows, 16 activation rows and their scales are staged in LDS
// by coalesced 16-byte loads, 16 blocks at a time (the next chunk's loads in flight); wave w multiplies row tile w
// (gate rows 0-15, 16-31, up rows 0-15, 16-31 of the block) by the token tile with one int8 MFMA per block and runs
// the chains of its own results in registers: lane l holds rows 4 (l / 16) + i, token l % 16, acc = fma(float(s) *
// dw, dx, acc) in block order, as the other matmul kernels. Then h = g / (1 + expf(-g)) * u and the quantization of
// each token's 32 values (one block of the down projection's input) by 32 lanes. SHORT: at most two chunks
// (cols <= 1024), straight-line.
constexpr int kSwKC = 16;  // blocks per chunk
template <int DT>
struct SwRegs {
    static constexpr int kBw = DT == kQ8 ? QK : QK / 2;           // weight bytes per block
    static constexpr int kAu = 64 * kSwKC * kBw / 16 / 256;        // 16-byte weight units per thread (8 / 4)
    static constexpr int kXu = 16 * kSwKC * QK / 16 / 256;         // 16-byte activation units per thread (2)
    static constexpr int kWu = 64 * kSwKC / 256;                   // row scales per thread (4)
    uint4 a[kAu];
    uint4 x[kXu];
    uint16_t dw[kWu];
    float dx;
};

template <int DT, bool SHORT>
__global__ __launch_bounds__(256) void matmul_swiglu_kernel(const uint8_t* __restrict__ wg,
                                                            const uint16_t* __restrict__ sgt,
                                                            const uint8_t* __restrict__ wu,
                                                            const uint16_t* __restrict__ sut,
                                                            const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                            int cols, int rows, int n, int n_tg,
                                                            int8_t* __restrict__ oq, float* __restrict__ od) {
    using R = SwRegs<DT>;
    constexpr int KC = kSwKC, kBw = R::kBw;
    constexpr int kArow = KC * kBw + 16;  // LDS row strides in bytes (= 4 dwords mod 64 banks: the 16 rows of an
    constexpr int kXrow = KC * QK + 16;   // operand read hit distinct banks)
    constexpr int kAupr = KC * kBw / 16, kXupr = KC * QK / 16;
    constexpr int kDxRow = KC + 4;        // token scale row stride (floats): 16-byte reads of 16 tokens, no conflict
    __shared__ __align__(16) uint8_t as[2][64 * kArow];
    __shared__ __align__(16) int8_t xs[2][16 * kXrow];
    __shared__ __align__(16) float dws[2][64 * KC];
    __shared__ __align__(16) float dxs[2][16 * kDxRow];
    __shared__ float hg[32][17], hu[32][17];
    __shared__ uint64_t exptab[32];
    ExpTab et;
    et.load();
    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lq = lane >> 4;
    // workgroups of one row block (its token groups) are numbered onto one XCD, as in the matmul kernels
    const int G = (int)gridDim.x, p = (int)blockIdx.x;
    const int xcd = p % 8, per = G / 8, rem = G % 8;
    const int logical = xcd * per + min(xcd, rem) + p / 8;
    const int rb = logical / n_tg, tg = logical % n_tg;
    const int r0 = rb * 32, tbase = tg * 16;
    const int nb = cols / QK;
    const size_t wrow = (size_t)nb * kBw;

    // staged row s (0..63): gate row r0 + s for s < 32, else up row r0 + s - 32; tokens past n are clamped
    const uint8_t* asrc[R::kAu];
    int aoff[R::kAu];
#pragma unroll
    for (int j = 0; j < R::kAu; ++j) {
        const int e = j * 256 + tid, r = e / kAupr;
        asrc[j] = r < 32 ? wg + (size_t)(r0 + r) * wrow : wu + (size_t)(r0 + r - 32) * wrow;
        aoff[j] = (e % kAupr) * 16;
    }
    const int8_t* xsrc[R::kXu];
    int xoff[R::kXu];
#pragma unroll
    for (int j = 0; j < R::kXu; ++j) {
        const int e = j * 256 + tid;
        xsrc[j] = xq + (size_t)min(tbase + e / kXupr, n - 1) * cols;
        xoff[j] = (e % kXupr) * 16;
    }
    const uint16_t* wsrc[R::kWu];
#pragma unroll
    for (int j = 0; j < R::kWu; ++j) {
        const int r = (j * 256 + tid) / KC;
        wsrc[j] = r < 32 ? sgt + (size_t)(r0 + r) * nb : sut + (size_t)(r0 + r - 32) * nb;
    }
    const float* dxsrc = xd + (size_t)min(tbase + tid / KC, n - 1) * nb;
    const int sk = tid % KC;  // the block of this thread's staged scales (256 is a multiple of KC)

    auto load = [&](R& S, int c0) {
#pragma unroll
        for (int j = 0; j < R::kAu; ++j)
            S.a[j] = load16(asrc[j] + min((size_t)c0 * kBw + aoff[j], wrow - 16));
#pragma unroll
        for (int j = 0; j < R::kXu; ++j) S.x[j] = load16(xsrc[j] + min(c0 * QK + xoff[j], cols - 16));
        const int b = min(c0 + sk, nb - 1);
#pragma unroll
        for (int j = 0; j < R::kWu; ++j) S.dw[j] = wsrc[j][b];
        S.dx = dxsrc[b];
    };
    auto stage = [&](const R& S, int buf) {
#pragma unroll
        for (int j = 0; j < R::kAu; ++j) {
            const int e = j * 256 + tid;
            *reinterpret_cast<uint4*>(&as[buf][(e / kAupr) * kArow + (e % kAupr) * 16]) = S.a[j];
        }
#pragma unroll
        for (int j = 0; j < R::kXu; ++j) {
            const int e = j * 256 + tid;
            *reinterpret_cast<uint4*>(&xs[buf][(e / kXupr) * kXrow + (e % kXupr) * 16]) = S.x[j];
        }
#pragma unroll
        for (int j = 0; j < R::kWu; ++j) {
            uint32_t h = S.dw[j];
            asm volatile("" : "+v"(h));  // keeps the conversion here (hoisted, it would wait for later loads)
            dws[buf][j * 256 + tid] = f16_to_f32((uint16_t)h);
        }
        dxs[buf][(tid / KC) * kDxRow + sk] = S.dx;
    };
    // wave w: staged rows 16 w + li (operand) / 16 w + 4 lq + i (results); chains acc[i] of (row 16 w + 4 lq + i,
    // token li)
    const int shift = DT == kQ8 ? 0 : (lq >> 1) * 4;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    auto compute = [&](int buf, int c0) {
        const int nblk = min(KC, nb - c0);
        const float4* dw4 = reinterpret_cast<const float4*>(dws[buf]) + (16 * wave + 4 * lq) * (KC / 4);
        const float4* dx4 = reinterpret_cast<const float4*>(dxs[buf] + li * kDxRow);
#pragma unroll
        for (int g4 = 0; g4 < KC / 4; ++g4) {
            long a[4], x[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int b = 4 * g4 + i;
                a[i] = *reinterpret_cast<const long*>(
                    &as[buf][(16 * wave + li) * kArow + b * kBw + (DT == kQ8 ? lq * 8 : (lq & 1) * 8)]);
                x[i] = *reinterpret_cast<const long*>(&xs[buf][li * kXrow + b * QK + lq * 8]);
            }
            float4 dwv[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) dwv[r] = dw4[r * (KC / 4) + g4];
            const float4 dxv = dx4[g4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                long ai = a[i];
                if (DT == kQ4) {
                    const uint64_t v = (uint64_t)ai;
                    const uint32_t lo = nibbles_to_i8(((uint32_t)v >> shift) & 0x0F0F0F0Fu);
                    const uint32_t hi = nibbles_to_i8(((uint32_t)(v >> 32) >> shift) & 0x0F0F0F0Fu);
                    ai = (long)(((uint64_t)hi << 32) | lo);
                }
                const v4i c = __builtin_amdgcn_mfma_i32_16x16x32_i8(ai, x[i], (v4i){0, 0, 0, 0}, 0, 0, 0);
                const float dx = i == 0 ? dxv.x : i == 1 ? dxv.y : i == 2 ? dxv.z : dxv.w;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float dw = i == 0 ? dwv[r].x : i == 1 ? dwv[r].y : i == 2 ? dwv[r].z : dwv[r].w;
                    const float nx = __builtin_fmaf((float)c[r] * dw, dx, acc[r]);
                    acc[r] = 4 * g4 + i < nblk ? nx : acc[r];
                }
            }
        }
    };

    const int n_chunks = (nb + KC - 1) / KC;
    if constexpr (SHORT) {
        R A, B;
        load(A, 0);
        load(B, KC);
        __builtin_amdgcn_sched_barrier(0);
        stage(A, 0);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        compute(0, 0);
        stage(B, 1);  // buffer 1 is not read by chunk 0
        __syncthreads();
        compute(1, KC);  // a chunk past nb adds nothing
    } else {
        // chunk c in buffer c % 2 and register set c % 2, refilled with chunk c + 2 once staged (clamped re-reads
        // past the last chunk)
        R S[2];
        load(S[0], 0);
        load(S[1], KC);
        __builtin_amdgcn_sched_barrier(0);
        stage(S[0], 0);
        load(S[0], 2 * KC);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        for (int c = 0;; c += 2) {
            compute(0, c * KC);
            if (c + 1 >= n_chunks) break;
            stage(S[1], 1);
            load(S[1], (c + 3) * KC);
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();
            compute(1, (c + 1) * KC);
            if (c + 2 >= n_chunks) break;
            stage(S[0], 0);
            load(S[0], (c + 4) * KC);
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();
        }
    }
    (void)n_chunks;

    // h = g / (1 + expf(-g)) * u (ops_ref.cpp:243-248) and its quantization per token: 32 lanes per block
    {
        float(*dst)[17] = wave < 2 ? hg : hu;
#pragma unroll
        for (int r = 0; r < 4; ++r) dst[16 * (wave & 1) + 4 * lq + r][li] = acc[r];
    }
    et.store(exptab);
    __syncthreads();
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
        const int tk = pass * 8 + tid / 32, rr = tid % 32, tok = tbase + tk;
        if (tok < n) {  // uniform per 32-lane group
            const float gv = hg[rr][tk], uv = hu[rr][tk];
            quant_block32(gv / (1.0f + dev_expf(-gv, exptab)) * uv, oq + (size_t)tok * rows + r0,
                          od + (size_t)tok * (rows / QK) + rb);
        }
    }
}

// q, k and v GEMVs of one token in one launch: three row segments of one dtype and width over one activation,
// the layer's normed input, which every workgroup builds itself (NormAct).
struct QkvSegs {
    const uint8_t *w0, *w1, *w2;
    const uint16_t *s0, *s1, *s2;
    float *o0, *o1, *o2;
    int rows0, rows1, rows2;
    int tiles0, tiles1;
};

template <int DT, int U, int R, bool EMB>
__global__ __launch_bounds__(256) void gemv_qkv_norm_kernel(QkvSegs a, NormAct act, int nb, int tile_rows,
                                                            uint32_t nb_magic) {
    extern __shared__ __align__(16) float smem[];
    QH_WSTAMP(0, 0);
    int blk = (int)blockIdx.x;
    const uint8_t* w = a.w0;
    const uint16_t* sc = a.s0;
    float* out = a.o0;
    int rows = a.rows0;
    if (blk >= a.tiles0) {
        blk -= a.tiles0;
        if (blk >= a.tiles1) {
            blk -= a.tiles1;
            w = a.w2, sc = a.s2, out = a.o2, rows = a.rows2;
        } else {
            w = a.w1, sc = a.s1, out = a.o1, rows = a.rows1;
        }
    }
    const int ra = blk * tile_rows;
    const int nrows = min(tile_rows, rows - ra);
    act.tmp = smem + gemv_tile_lds_bytes(nb * QK, tile_rows, true) / 4;
    constexpr int kBlockBytes = DT == kQ8 ? QK : QK / 2;
    const GemvSegs<1> segs{{w + (size_t)ra * nb * kBlockBytes}, {sc + (size_t)ra * nb}};
    const float val =
        gemv_tile<DT, U, true, 1>(segs, nullptr, nullptr, nb, nrows, tile_rows, nb_magic, smem,
                                  NormActR<R, EMB>{act}, 0);
    QH_WSTAMP(0, 3);
    if ((int)threadIdx.x < nrows) out[ra + threadIdx.x] = val;
}

// One token's projection added into the residual stream: x[r] += (W . xq)[r] (model.cpp:208-210, 224-226).
template <int DT, int U, bool XL>
__global__ __launch_bounds__(256) void gemv_residual_kernel(const uint8_t* __restrict__ wq,
                                                            const uint16_t* __restrict__ wscale,
                                                            const int8_t* __restrict__ xq,
                                                            const float* __restrict__ xd, int nb, int rows,
                                                            int tile_rows, uint32_t nb_magic, float* __restrict__ x) {
    extern __shared__ __align__(16) float smem[];
    const int tlk = nb > 64 ? 4 : 2;  // timeline id: the down projection (K = 4864) or o (K = 896)
    (void)tlk;
    QH_WSTAMP(tlk, 0);
    const int tid = (int)threadIdx.x;
    const int ra = (int)blockIdx.x * tile_rows;
    const int nrows = min(tile_rows, rows - ra);
    const float x0 = x[ra + min(tid, nrows - 1)];  // the residual row, in flight with the weights
    const float val = gemv_tile<DT, U, XL>(wq, wscale, xq, xd, nb, ra, nrows, tile_rows, nb_magic, smem, tlk);
    QH_WSTAMP(tlk, 3);
    if (tid < nrows) x[ra + tid] = x0 + val;
}

// One token's gate and up GEMVs over the same 32 rows of both matrices, from the normed MLP input each workgroup
// builds itself (NormAct), then h = g / (1 + expf(-g)) * u and the quantization of those 32 values (one block) for
// the down projection.
template <int DT, int U, int R>
__global__ __launch_bounds__(256) void gemv_swiglu_norm_kernel(const uint8_t* __restrict__ wg,
                                                               const uint16_t* __restrict__ sg,
                                                               const uint8_t* __restrict__ wu,
                                                               const uint16_t* __restrict__ su, NormAct act, int nb,
                                                               uint32_t nb_magic, int8_t* __restrict__ oq,
                                                               float* __restrict__ od) {
    extern __shared__ __align__(16) float smem[];
    __shared__ uint64_t exptab[32];
    QH_WSTAMP(3, 0);
    ExpTab et;
    et.load();
    const int tid = (int)threadIdx.x, ra = (int)blockIdx.x * QK;
    act.tmp = smem + gemv_tile_lds_bytes(nb * QK, 2 * QK, true) / 4;
    constexpr int kBlockBytes = DT == kQ8 ? QK : QK / 2;
    const GemvSegs<2> segs{{wg + (size_t)ra * nb * kBlockBytes, wu + (size_t)ra * nb * kBlockBytes},
                           {sg + (size_t)ra * nb, su + (size_t)ra * nb}};
    const float val =
        gemv_tile<DT, U, true, 2>(segs, nullptr, nullptr, nb, QK, 2 * QK, nb_magic, smem, NormActR<R, false>{act}, 3);
    QH_WSTAMP(3, 3);
    // wave 0 holds the block's 32 gate rows in lanes 0-31 and its 32 up rows in lanes 32-63: one half swap hands
    // lane l its up value (the exp table is stored by lanes 0-31 of the same wave, so no barrier is needed)
    if (tid < 2 * QK) {  // wave 0
        et.store(exptab);
        const uint32_t vb = __builtin_bit_cast(uint32_t, val);
        const auto sw = __builtin_amdgcn_permlane32_swap(vb, vb, false, false);
        const float u = __builtin_bit_cast(float, (uint32_t)sw[1]);
        if (tid < QK) quant_block32(val / (1.0f + dev_expf(-val, exptab)) * u, oq + ra, od + blockIdx.x);
    }
}

__global__ __launch_bounds__(256) void residual_add_kernel(float* __restrict__ x, const float* __restrict__ o, int n) {
    const int i = (int)(blockIdx.x * 256 + threadIdx.x);
    if (i < n) x[i] = x[i] + o[i];
}

// rmsnorm + quantization of one row (the final norm before the head), normed row also to `normed`.
template <int R>
__global__ __launch_bounds__(256) void norm_quant_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                         int D, float eps, int8_t* __restrict__ oq,
                                                         float* __restrict__ od, float* __restrict__ normed) {
    __shared__ __align__(16) float xs[8192 + kChainPad];
    const int tid = threadIdx.x, n4 = D / 4;
    RowF4<R> wr, xr;
    xr.load(x, n4);
    const SegWarm warm = D >= 128 ? seg_warm(x, D) : SegWarm{};
    wr.load(w, n4);
#pragma unroll
    for (int k = 0; k < R; ++k)
        if (tid + 256 * k < n4) reinterpret_cast<float4*>(xs)[tid + 256 * k] = xr.v[k];
    if (D >= 128) {  // uniform
        normalize_quant_lds(xs, D, rms_scale(seg_sum_squares(x, D, xr, warm), D, eps), wr, oq, od, normed);
    } else {
        __syncthreads();
        norm_quant_lds(xs, D, wr, eps, oq, od, normed);
    }
}

// Prefill / decode bookkeeping on the device.
__global__ void set_int_kernel(int* p, int value) { *p = value; }

// The first positions of a prefill stack's 32-token attention sub-chunks: p[i] = base + 32 i, i < n.
__global__ void set_subpos_kernel(int* p, int base, int n) {
    const int i = (int)threadIdx.x;
    if (i < n) p[i] = base + kChunk * i;
}

// The token a step chose: the sampler's pick when there is one, else the head's greedy top-1.
struct Pick {
    const int32_t* sampled;
    const qh_head_stats* stats;
    const int32_t* top1_full;
    __device__ __forceinline__ int id() const { return sampled ? *sampled : stats ? stats->top1 : *top1_full; }
};

// The chosen token becomes the next input, is appended to out[] and to the token history (session.cpp:45-46), and,
// after a decode step (advance), the position moves on.
__global__ void advance_kernel(Pick pick, TokenFeedback fb, int advance) { fb.apply(pick.id(), advance != 0); }

// Appends a prompt chunk to the token history (Session::feed, session.cpp:13-30), first emptying it when the chunk
// starts a sequence (reset). One workgroup.
__global__ __launch_bounds__(256) void history_append_kernel(const int32_t* __restrict__ tokens, int n, int reset,
                                                             int32_t* __restrict__ hist, int* __restrict__ hist_len,
                                                             int hist_cap) {
    __shared__ int base;
    if (threadIdx.x == 0) base = reset ? 0 : *hist_len;
    __syncthreads();
    const int b = base;
    for (int i = (int)threadIdx.x; i < n; i += 256)
        if (b + i < hist_cap) hist[b + i] = tokens[i];
    if (threadIdx.x == 0) *hist_len = b + n < hist_cap ? b + n : hist_cap;
}

}  // namespace

// ------------------------------------------------------------------------------------------------- host side

struct Decoder {
    qh_model_desc hp;
    std::vector<qh_tensor> t;  // the caller's device tensors, in the qh_decoder_create order
    const qh_tensor* lmh = nullptr;  // the LM head: the embedding, or lm_head.weight when untied (model.cpp:16)
    bool hadamard = false;           // FLAG_HADAMARD_DOWN (model_file.h:21)
    bool kv32 = false;               // an f32 KV cache (Model::load kv_f16 false)
    bool dense = false;              // some matrix is F32 / F16 (matvec_ref): f32 copies of the activations are kept
    float *fa = nullptr, *fb = nullptr;  // f32 normed layer input [kChunk][dim]; attention / SwiGLU output
                                         // [kChunk][max(dim, ffn_dim)] (the unquantized matrices' inputs)
    // device state
    uint16_t *kc = nullptr, *vc = nullptr;  // f16 cache (the default)
    float *kcf = nullptr, *vcf = nullptr;   // f32 cache, [n_layers][ctx][kv_dim] each
    float* cs = nullptr;
    float *x = nullptr, *o = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *g = nullptr, *u = nullptr,
          *hidden = nullptr;
    // int8 activations: qa holds a layer's normed input (and the head's), qb the attention / MLP inner activation
    int8_t *qa = nullptr, *qb = nullptr;
    float *da = nullptr, *db = nullptr;
    float* escr = nullptr;      // decode attention: a row of exp values, then one of weights, per head
    int escr_stride = 0;
    int32_t* tokens = nullptr;  // [kChunk] prefill input / [0] decode input
    // Prefill stack: the tokens whose norms and matmuls share one launch (kChunk, the reference's Model::kBatch, by
    // default; larger stacks run the matmul tile kernels at M up to kMaxStack). Attention runs each stack as 32-token
    // sub-chunks in order, the sub-chunk i starting at subpos[i].
    int stack = kChunk;
    int* subpos = nullptr;
    int stack_end = 0;  // the current prefill stack's end position (host-side, for the attention plan)
    // token history (prompt ids since position 0, then each chosen id) and the optional query / sampler settings
    int32_t* hist = nullptr;  // [ctx_len + 1]
    int* hist_len = nullptr;
    bool has_query = false, has_sampler = false;
    qh_sampler_params qp{}, sp{};
    uint64_t* rng = nullptr;
    int32_t* sampled = nullptr;
    int* pos = nullptr;         // current position
    int* n_out = nullptr;
    int* status = nullptr;
    int32_t* out = nullptr;
    int out_cap = 0;
    // head
    float *logits = nullptr, *coarse = nullptr, *upper = nullptr;
    int32_t* rows = nullptr;
    qh_head_stats* stats = nullptr;
    void* head_ws = nullptr;
    size_t head_ws_bytes = 0;
    void* am_ws = nullptr;
    size_t am_ws_bytes = 0;
    void* sample_ws = nullptr;  // the sampler's sorted path (more than QH_SAMPLE_MAX_TOPK survivors)
    int32_t* top1_full = nullptr;
    bool fuse = true;  // fused decode kernels (QH_DECODER_FUSE=0 at creation selects one launch per operation)
    std::vector<void*> allocs;
    // The stage the kernels launched since the previous mark belong to (qh_decoder_step_timed).
    void mark(int id) const {
        if (KernelTimer* t = kernel_timer()) t->mark(id);
    }
};

namespace {

enum { T_EMBED, T_NORM, T_LAYER0 };
enum { L_ATTN_NORM, L_WQ, L_WK, L_WV, L_WO, L_BQ, L_BK, L_BV, L_FFN_NORM, L_WG, L_WU, L_WD, L_COUNT };

const qh_tensor& lt(const Decoder* d, int l, int which) { return d->t[T_LAYER0 + l * L_COUNT + which]; }
const float* lf(const Decoder* d, int l, int which) { return static_cast<const float*>(lt(d, l, which).data); }
const float* bias(const Decoder* d, int l, int which) { return d->hp.qkv_bias ? lf(d, l, which) : nullptr; }
const qh_tensor& head4(const Decoder* d) { return d->t[T_LAYER0 + d->hp.n_layers * L_COUNT]; }
const qh_tensor& head_err(const Decoder* d) { return d->t[T_LAYER0 + d->hp.n_layers * L_COUNT + 1]; }
const float* final_norm(const Decoder* d) { return static_cast<const float*>(d->t[T_NORM].data); }
bool dense_w(const qh_tensor& W) { return W.dtype == kF32 || W.dtype == kF16; }

const uint8_t* quants(const qh_tensor& W) { return static_cast<const uint8_t*>(W.data); }
const uint16_t* scales(const qh_tensor& W) {
    return reinterpret_cast<const uint16_t*>(quants(W) + qh_quant_bytes(W.dtype, W.rows, W.cols));
}
uint32_t nb_magic(int nb) { return nb == 1 ? 0u : (uint32_t)((0x100000000ull + (uint64_t)nb - 1) / (uint64_t)nb); }

hipError_t dalloc(Decoder* d, void** p, size_t bytes) {
    if (fault_alloc_fires()) return hipErrorOutOfMemory;  // qh_fault_alloc's forced failure
    hipError_t e = hipMalloc(p, bytes < 256 ? 256 : bytes);
    if (e == hipSuccess) d->allocs.push_back(*p);
    return e;
}

void dfree(Decoder* d, void* p) {
    if (!p) return;
    for (size_t i = 0; i < d->allocs.size(); ++i)
        if (d->allocs[i] == p) {
            d->allocs.erase(d->allocs.begin() + (long)i);
            break;
        }
    (void)hipFree(p);
}

// The work buffers of a prefill stack of c tokens: the residual stream, projections, MLP rows, int8 activations and
// their scales, the f32 copies for unquantized matrices and the attention sub-chunks' positions. On failure the ones
// allocated stay listed (the caller frees them).
hipError_t alloc_stack(Decoder* d, int c) {
    const qh_model_desc& hp = d->hp;
    const size_t D = hp.dim, F = hp.ffn_dim, wide = D > F ? D : F, kvd = (size_t)hp.n_kv_heads * hp.head_dim;
    hipError_t e = hipSuccess;
    auto A = [&](void** p, size_t b) {
        if (e == hipSuccess) e = dalloc(d, p, b);
    };
    A((void**)&d->x, sizeof(float) * c * D);
    A((void**)&d->o, sizeof(float) * c * D);
    A((void**)&d->q, sizeof(float) * c * D);
    A((void**)&d->k, sizeof(float) * c * kvd);
    A((void**)&d->v, sizeof(float) * c * kvd);
    A((void**)&d->g, sizeof(float) * c * F);
    A((void**)&d->u, sizeof(float) * c * F);
    A((void**)&d->qa, c * wide);
    A((void**)&d->qb, c * wide);
    A((void**)&d->da, sizeof(float) * c * (wide / QK));
    A((void**)&d->db, sizeof(float) * c * (wide / QK));
    if (d->dense) {
        A((void**)&d->fa, sizeof(float) * c * D);
        A((void**)&d->fb, sizeof(float) * c * wide);
    }
    A((void**)&d->subpos, sizeof(int) * (kMaxStack / kChunk));
    return e;
}

#define QH_TRY(expr)                                 \
    do {                                             \
        const hipError_t e_ = (expr);                \
        if (e_ != hipSuccess) return e_;             \
    } while (0)

// Calls f(dt, u, xl) with std::integral_constant arguments for the plan's dtype, unroll and activation staging, so a
// caller can launch KERNEL<dt, u, xl> for any plan gemv_plan makes.
// Calls f with the row-slot count (std::integral_constant) of rows of D floats.
template <typename F>
void by_row_slots(int D, F&& f) {
    if (row_slots(D / 4) == 1)
        f(std::integral_constant<int, 1>{});
    else
        f(std::integral_constant<int, 8>{});
}

template <typename F>
hipError_t plan_dispatch(int dtype, const GemvPlan& p, F&& f) {
    using std::integral_constant;
    auto go = [&](auto dt, auto u) {
        if (p.act_lds)
            f(dt, u, std::true_type{});
        else
            f(dt, u, std::false_type{});
        return hipGetLastError();
    };
    auto by_unroll = [&](auto dt) {
        switch (p.unroll) {
            case 1: return go(dt, integral_constant<int, 1>{});
            case 2: return go(dt, integral_constant<int, 2>{});
            case 4: return go(dt, integral_constant<int, 4>{});
            case 8: return go(dt, integral_constant<int, 8>{});
            default: return hipErrorInvalidValue;
        }
    };
    if (dtype == kQ8) return by_unroll(integral_constant<int, kQ8>{});
    if (dtype == kQ4) return by_unroll(integral_constant<int, kQ4>{});
    return hipErrorInvalidValue;
}

hipError_t embed(Decoder* d, const int32_t* tokens, int n, hipStream_t s) {
    const qh_tensor& emb = d->t[T_EMBED];
    by_row_slots(d->hp.dim, [&](auto r) {
        qh_launch((embed_norm_quant_kernel<decltype(r)::value>), dim3(n), dim3(256), 0, s, tokens, quants(emb),
                  emb.dtype, d->hp.dim, d->hp.vocab_size, d->x, lf(d, 0, L_ATTN_NORM), d->hp.norm_eps, d->qa, d->da,
                  d->fa, d->status);
    });
    return hipGetLastError();
}

// Model::linear / linear_batch (model.cpp:150-157, 336-347) of n tokens into out [n][ldo] (n == 1: out[r]): the
// integer-dot GEMV / matmul on the quantized activation for a Q8_0 / Q4_0 W, matvec_ref on its f32 copy for an
// F32 / F16 W. inner: the attention / SwiGLU output (qb / db / fb), else the normed layer input (qa / da / fa).
hipError_t linear(Decoder* d, float* out, int ldo, const qh_tensor& W, bool inner, int n, hipStream_t s) {
    if (dense_w(W)) return launch_gemv_dense(out, ldo, W, inner ? d->fb : d->fa, W.cols, n, 0, W.rows, s);
    const int8_t* xq = inner ? d->qb : d->qa;
    const float* xd = inner ? d->db : d->da;
    if (n == 1) return launch_gemv(out, W, xq, xd, 0, W.rows, gemv_plan(W.dtype, W.cols, W.rows), s);
    return launch_matmul(out, ldo, W, xq, xd, n, 0, W.rows, s);
}

// The normed-input fill of a decode kernel: layer input from the residual stream x, or (first layer) from the
// embedding of the current token, which workgroup 0 also stores as x.
NormAct make_norm(Decoder* d, bool embedding, const float* w) {
    NormAct a{};
    if (embedding) {
        const qh_tensor& emb = d->t[T_EMBED];
        a.eq = reinterpret_cast<const int8_t*>(quants(emb));
        a.es = reinterpret_cast<const uint16_t*>(quants(emb) + (size_t)emb.rows * emb.cols);
        a.tok = d->tokens;
        a.V = d->hp.vocab_size;
        a.x_out = d->x;
    } else {
        a.x = d->x;
    }
    a.status = d->status;
    a.w = w;
    a.eps = d->hp.norm_eps;
    a.D = d->hp.dim;
    a.tlk = -1;
    return a;
}

// LDS of a normed-input GEMV tile: the tile (codes staged in LDS) plus the D-float scratch of the norm.
size_t norm_tile_lds(int cols, int tile_rows, int D) {
    return gemv_tile_lds_bytes(cols, tile_rows, true) + 4 * ((size_t)D + kChainPad);
}

// Plan of the fused q/k/v launch, or false (one launch per operation) where the three projections differ in dtype
// or the plain GEMV would stream or the tile does not fit.
bool qkv_plan(const Decoder* d, int l, GemvPlan* p, size_t* lds) {
    const qh_tensor &wq = lt(d, l, L_WQ), &wk = lt(d, l, L_WK), &wv = lt(d, l, L_WV);
    if (!d->fuse || dense_w(wq) || wq.dtype != wk.dtype || wq.dtype != wv.dtype) return false;
    *p = gemv_plan(wq.dtype, wq.cols, wq.rows);
    *lds = norm_tile_lds(wq.cols, p->tile_rows, d->hp.dim);
    return !p->stream && *lds <= kFuseLds;
}

hipError_t launch_qkv_norm(Decoder* d, int l, const GemvPlan& p, size_t lds, const NormAct& act, hipStream_t s) {
    const qh_tensor &wq = lt(d, l, L_WQ), &wk = lt(d, l, L_WK), &wv = lt(d, l, L_WV);
    const int T = p.tile_rows;
    QkvSegs a{quants(wq), quants(wk), quants(wv), scales(wq), scales(wk), scales(wv), d->q, d->k, d->v,
              wq.rows, wk.rows, wv.rows, (wq.rows + T - 1) / T, (wk.rows + T - 1) / T};
    const unsigned grid = (unsigned)(a.tiles0 + a.tiles1 + (wv.rows + T - 1) / T);
    const int nb = wq.cols / QK;
    return plan_dispatch(wq.dtype, p, [&](auto dt, auto u, auto) {
        by_row_slots(act.D, [&](auto r) {
            if (act.eq)
                qh_launch((gemv_qkv_norm_kernel<decltype(dt)::value, decltype(u)::value, decltype(r)::value,
                                                         true>),
                                   dim3(grid), dim3(256), lds, s, a, act, nb, T, nb_magic(nb));
            else
                qh_launch((gemv_qkv_norm_kernel<decltype(dt)::value, decltype(u)::value, decltype(r)::value,
                                                         false>),
                                   dim3(grid), dim3(256), lds, s, a, act, nb, T, nb_magic(nb));
        });
    });
}

// x += W . (xq, xd) for one token: the GEMV tile kernel with the add in its epilogue, or (a streaming-size W, or
// one launch per operation) GEMV into d->o and a separate add.
hipError_t residual(Decoder* d, const qh_tensor& W, hipStream_t s) {
    const int8_t* xq = d->qb;
    const float* xd = d->db;
    if (dense_w(W)) {
        QH_TRY(linear(d, d->o, 0, W, true, 1, s));
        qh_launch(residual_add_kernel, dim3((unsigned)((W.rows + 255) / 256)), dim3(256), 0, s, d->x, d->o, W.rows);
        return hipGetLastError();
    }
    const GemvPlan p = gemv_plan(W.dtype, W.cols, W.rows);
    if (d->fuse && !p.stream) {
        const int T = p.tile_rows, nb = W.cols / QK;
        const unsigned grid = (unsigned)((W.rows + T - 1) / T);
        const size_t lds = gemv_lds_bytes(W.cols, T, p.act_lds);
        return plan_dispatch(W.dtype, p, [&](auto dt, auto u, auto xl) {
            qh_launch((gemv_residual_kernel<decltype(dt)::value, decltype(u)::value, decltype(xl)::value>),
                               dim3(grid), dim3(256), lds, s, quants(W), scales(W), xq, xd, nb, W.rows, T,
                               nb_magic(nb), d->x);
        });
    }
    QH_TRY(launch_gemv(d->o, W, xq, xd, 0, W.rows, p, s));
    qh_launch(residual_add_kernel, dim3((unsigned)((W.rows + 255) / 256)), dim3(256), 0, s, d->x, d->o,
                       W.rows);
    return hipGetLastError();
}

// The down projection's input from gate / up rows g, u of n tokens (ffn values each): SwiGLU and quantization, with
// the block-256 Walsh-Hadamard transform between them when the model has FLAG_HADAMARD_DOWN (model.cpp:216-220).
hipError_t swiglu_down_input(Decoder* d, int F, int n, hipStream_t s) {
    if (d->hadamard) {
        qh_launch(swiglu_fwht_quant_kernel, dim3((unsigned)(F / 256), (unsigned)n), dim3(256), 0, s, d->g, d->u, F,
                  d->qb, d->db, d->fb);
    } else {
        const long nblk = (long)n * F / QK;
        qh_launch(swiglu_quant_kernel, dim3((unsigned)((nblk * QK + 255) / 256)), dim3(256), 0, s, d->g, d->u, nblk,
                  d->qb, d->db, d->fb);
    }
    return hipGetLastError();
}

hipError_t norm_quant(Decoder* d, const float* w, float* normed, hipStream_t s) {
    by_row_slots(d->hp.dim, [&](auto r) {
        qh_launch((norm_quant_kernel<decltype(r)::value>), dim3(1), dim3(256), 0, s, d->x, w, d->hp.dim,
                           d->hp.norm_eps, d->qa, d->da, normed);
    });
    return hipGetLastError();
}

// rmsnorm (ffn_norm) of one token, gate / up, SwiGLU and quantization into qb / db.
hipError_t gate_up(Decoder* d, int l, hipStream_t s) {
    const qh_tensor &wg = lt(d, l, L_WG), &wu = lt(d, l, L_WU);
    const int nb = wg.cols / QK;
    const size_t lds = norm_tile_lds(wg.cols, 2 * QK, d->hp.dim);
    if (d->fuse && !d->hadamard && !d->dense && wg.dtype == wu.dtype && lds <= kFuseLds) {
        const unsigned grid = (unsigned)(wg.rows / QK);
        NormAct act = make_norm(d, false, lf(d, l, L_FFN_NORM));
        act.tlk = 3;
        by_row_slots(d->hp.dim, [&](auto r) {
            constexpr int R = decltype(r)::value;
            if (wg.dtype == kQ8)
                qh_launch((gemv_swiglu_norm_kernel<kQ8, 8, R>), dim3(grid), dim3(256), lds, s, quants(wg),
                                   scales(wg), quants(wu), scales(wu), act, nb, nb_magic(nb), d->qb, d->db);
            else
                qh_launch((gemv_swiglu_norm_kernel<kQ4, 8, R>), dim3(grid), dim3(256), lds, s, quants(wg),
                                   scales(wg), quants(wu), scales(wu), act, nb, nb_magic(nb), d->qb, d->db);
        });
        return hipGetLastError();
    }
    QH_TRY(norm_quant(d, lf(d, l, L_FFN_NORM), d->fa, s));
    QH_TRY(linear(d, d->g, 0, wg, false, 1, s));
    QH_TRY(linear(d, d->u, 0, wu, false, 1, s));
    return swiglu_down_input(d, wg.rows, 1, s);
}

// Attention of a chunk of n <= kChunk tokens at positions *pos_dev .. + n - 1 whose projections start at row r0 of
// q / k / v; outputs to rows r0 .. of qb / db (and fb).
hipError_t attention_chunk(Decoder* d, int l, int n, int r0, const int* pos_dev, hipStream_t s) {
    const qh_model_desc& hp = d->hp;
    const size_t layer_k = (size_t)hp.ctx_len * hp.n_kv_heads * hp.head_dim;
    const size_t layer_v = (size_t)v_ctx(hp.ctx_len) * hp.n_kv_heads * hp.head_dim;
    const size_t qd = (size_t)hp.n_heads * hp.head_dim, kvd = (size_t)hp.n_kv_heads * hp.head_dim;
    const float *q = d->q + r0 * qd, *k = d->k + r0 * kvd, *v = d->v + r0 * kvd;
    int8_t* oq = d->qb + r0 * qd;
    float* od = d->db + r0 * (qd / QK);
    float* of = d->fb ? d->fb + r0 * qd : nullptr;
    const dim3 grid(hp.n_heads, n);
    if (d->kv32) {  // the f32 cache: prefill and decode alike
        const size_t layer_kv = (size_t)hp.ctx_len * hp.n_kv_heads * hp.head_dim;
        if (hp.head_dim == 64)
            qh_launch((attention_f32_kernel<64>), grid, dim3(256), 0, s, q, k, v, bias(d, l, L_BQ),
                      bias(d, l, L_BK), bias(d, l, L_BV), d->cs, pos_dev, hp.ctx_len, hp.n_heads, hp.n_kv_heads,
                      d->kcf + l * layer_kv, d->vcf + l * layer_kv, oq, od, d->status, of);
        else
            qh_launch((attention_f32_kernel<128>), grid, dim3(256), 0, s, q, k, v, bias(d, l, L_BQ),
                      bias(d, l, L_BK), bias(d, l, L_BV), d->cs, pos_dev, hp.ctx_len, hp.n_heads, hp.n_kv_heads,
                      d->kcf + l * layer_kv, d->vcf + l * layer_kv, oq, od, d->status, of);
    } else if (hp.head_dim == 64) {
        qh_launch((attention_kernel<64, 2>), grid, dim3(256), 0, s, q, k, v, bias(d, l, L_BQ), bias(d, l, L_BK),
                  bias(d, l, L_BV), d->cs, pos_dev, hp.ctx_len, hp.n_heads, hp.n_kv_heads, d->kc + l * layer_k,
                  d->vc + l * layer_v, oq, od, d->status, of, 0);
    } else {
        qh_launch((attention_kernel<128>), grid, dim3(256), 0, s, q, k, v, bias(d, l, L_BQ), bias(d, l, L_BK),
                  bias(d, l, L_BV), d->cs, pos_dev, hp.ctx_len, hp.n_heads, hp.n_kv_heads, d->kc + l * layer_k,
                  d->vc + l * layer_v, oq, od, d->status, of, 0);
    }
    return hipGetLastError();
}

// Attention of a prefill stack of n > kChunk tokens at positions *d->pos ..: the f16 cache rows of every token of the
// stack first (kv_store_kernel), then one attention launch in which each token is its own chunk (every earlier row
// read from the cache), so the stack's (head, token) workgroups fill the GPU together.
hipError_t attention_stack(Decoder* d, int l, int n, hipStream_t s) {
    const qh_model_desc& hp = d->hp;
    const size_t layer_k = (size_t)hp.ctx_len * hp.n_kv_heads * hp.head_dim;
    const size_t layer_v = (size_t)v_ctx(hp.ctx_len) * hp.n_kv_heads * hp.head_dim;
    uint16_t *kc = d->kc + l * layer_k, *vc = d->vc + l * layer_v;
    const dim3 grid(hp.n_heads, n);
    if (hp.head_dim == 64) {
        qh_launch((kv_store_kernel<64>), dim3(n), dim3(256), 0, s, d->k, d->v, bias(d, l, L_BK), bias(d, l, L_BV),
                  d->cs, d->pos, hp.ctx_len, hp.n_kv_heads, kc, vc);
        QH_TRY(hipGetLastError());
        if (d->stack_end <= kStackCtx) {  // the stack's last row within the four-token kernel's score rows
            qh_launch(attention_stack_kernel, dim3(hp.n_heads, (n + kStackTok - 1) / kStackTok), dim3(256), 0, s,
                      d->q, bias(d, l, L_BQ), d->cs, d->pos, n, hp.ctx_len, hp.n_heads, hp.n_kv_heads, kc, vc, d->qb,
                      d->db, d->status, d->fb);
            return hipGetLastError();
        }
        qh_launch((attention_kernel<64, 2>), grid, dim3(256), 0, s, d->q, d->k, d->v, bias(d, l, L_BQ),
                  bias(d, l, L_BK), bias(d, l, L_BV), d->cs, d->pos, hp.ctx_len, hp.n_heads, hp.n_kv_heads, kc, vc,
                  d->qb, d->db, d->status, d->fb, 1);
    } else {
        qh_launch((kv_store_kernel<128>), dim3(n), dim3(256), 0, s, d->k, d->v, bias(d, l, L_BK), bias(d, l, L_BV),
                  d->cs, d->pos, hp.ctx_len, hp.n_kv_heads, kc, vc);
        QH_TRY(hipGetLastError());
        qh_launch((attention_kernel<128>), grid, dim3(256), 0, s, d->q, d->k, d->v, bias(d, l, L_BQ),
                  bias(d, l, L_BK), bias(d, l, L_BV), d->cs, d->pos, hp.ctx_len, hp.n_heads, hp.n_kv_heads, kc, vc,
                  d->qb, d->db, d->status, d->fb, 1);
    }
    return hipGetLastError();
}

hipError_t attention(Decoder* d, int l, int n, hipStream_t s) {
    const qh_model_desc& hp = d->hp;
    if (n > kChunk && !d->kv32 && d->fuse) return attention_stack(d, l, n, s);
    if (n > kChunk) {  // a prefill stack: its 32-token sub-chunks in order (each reads the rows the ones before wrote)
        for (int i = 0; i * kChunk < n; ++i)
            QH_TRY(attention_chunk(d, l, min(kChunk, n - i * kChunk), i * kChunk, d->subpos + i, s));
        return hipSuccess;
    }
    if (n == 1 && hp.head_dim == 64 && d->fuse && !d->kv32) {  // decode: one 16-wave workgroup per head
        const size_t layer_k = (size_t)hp.ctx_len * hp.n_kv_heads * hp.head_dim;
        const size_t layer_v = (size_t)v_ctx(hp.ctx_len) * hp.n_kv_heads * hp.head_dim;
        qh_launch((attention_decode_kernel<64>), dim3(hp.n_heads / hp.n_kv_heads, hp.n_kv_heads), dim3(1024), 0, s,
                  d->q, d->k, d->v, d->kc + l * layer_k, d->pos, hp.ctx_len, hp.n_heads / hp.n_kv_heads,
                  bias(d, l, L_BQ), bias(d, l, L_BK), hp.n_kv_heads, bias(d, l, L_BV), d->cs, d->vc + l * layer_v,
                  d->qb, d->db, d->escr, d->escr_stride, d->status, d->fb);
        return hipGetLastError();
    }
    return attention_chunk(d, l, n, 0, d->pos, s);  // a chunk of the prefill (either cache), or the f32 cache
}

// One decode step's layers for the token in d->tokens[0], from its embedding. Leaves the final normed hidden state
// in d->hidden and its quantization in qa / da for the head.
hipError_t decode_layers(Decoder* d, hipStream_t s) {
    const qh_model_desc& hp = d->hp;
    for (int l = 0; l < hp.n_layers; ++l) {
        GemvPlan p;
        size_t lds = 0;
        if (qkv_plan(d, l, &p, &lds) && (l > 0 || d->t[T_EMBED].dtype == kQ8)) {
            NormAct act = make_norm(d, l == 0, lf(d, l, L_ATTN_NORM));
            act.tlk = 0;
            QH_TRY(launch_qkv_norm(d, l, p, lds, act, s));
        } else {
            if (l == 0)
                QH_TRY(embed(d, d->tokens, 1, s));
            else
                QH_TRY(norm_quant(d, lf(d, l, L_ATTN_NORM), d->fa, s));
            QH_TRY(linear(d, d->q, 0, lt(d, l, L_WQ), false, 1, s));
            QH_TRY(linear(d, d->k, 0, lt(d, l, L_WK), false, 1, s));
            QH_TRY(linear(d, d->v, 0, lt(d, l, L_WV), false, 1, s));
        }
        d->mark(l * QH_STAGES_PER_LAYER + QH_STAGE_QKV);
        QH_TRY(attention(d, l, 1, s));
        d->mark(l * QH_STAGES_PER_LAYER + QH_STAGE_ATTENTION);
        QH_TRY(residual(d, lt(d, l, L_WO), s));
        d->mark(l * QH_STAGES_PER_LAYER + QH_STAGE_O);
        QH_TRY(gate_up(d, l, s));
        d->mark(l * QH_STAGES_PER_LAYER + QH_STAGE_GATE_UP);
        QH_TRY(residual(d, lt(d, l, L_WD), s));
        d->mark(l * QH_STAGES_PER_LAYER + QH_STAGE_DOWN);
    }
    QH_TRY(norm_quant(d, final_norm(d), d->hidden, s));
    d->mark(QH_STAGE_FINAL_NORM);
    return hipSuccess;
}

// Matrices over one activation, in as few launches as their formats allow: runs of one dtype and width share one.
// Gate / up / SwiGLU / quantization of a prefill chunk as one launch (matmul_swiglu_kernel) into qb / db, or false
// (the matmul launch and swiglu_quant_kernel instead: one launch per operation, different formats or widths, rows
// not a multiple of 32, unaligned operands).
bool swiglu_fused(Decoder* d, const qh_tensor& wg, const qh_tensor& wu, int n, hipStream_t s) {
    if (n > kChunk || !d->fuse || d->hadamard || d->dense || wg.dtype != wu.dtype || wg.rows != wu.rows || wg.cols != wu.cols || wg.rows % QK != 0 ||
        (wg.dtype != kQ8 && wg.dtype != kQ4) || wg.cols % QK != 0 || wg.cols < 2 * QK)
        return false;
    const uint8_t *qg = quants(wg), *qu = quants(wu);
    if (((reinterpret_cast<uintptr_t>(qg) | reinterpret_cast<uintptr_t>(qu) | reinterpret_cast<uintptr_t>(d->qa)) &
         15u) != 0)
        return false;
    const int n_tg = (n + 15) / 16;
    const dim3 grid((unsigned)(wg.rows / QK * n_tg));
    const bool short_rows = wg.cols / QK <= 2 * kSwKC;
#define QH_SW(DT, SH)                                                                                            \
    qh_launch((matmul_swiglu_kernel<DT, SH>), grid, dim3(256), 0, s, qg, scales(wg), qu, scales(wu), d->qa, d->da, \
              wg.cols, wg.rows, n, n_tg, d->qb, d->db)
    if (wg.dtype == kQ4) {
        if (short_rows)
            QH_SW(kQ4, true);
        else
            QH_SW(kQ4, false);
    } else {
        if (short_rows)
            QH_SW(kQ8, true);
        else
            QH_SW(kQ8, false);
    }
#undef QH_SW
    return true;
}

hipError_t matmul_group(const MmOut* m, int k, const int8_t* xq, const float* xd, int n, hipStream_t s) {
    for (int i = 0; i < k;) {
        int j = i + 1;
        while (j < k && m[j].W->dtype == m[i].W->dtype && m[j].W->cols == m[i].W->cols) ++j;
        QH_TRY(launch_matmul_segs(m + i, j - i, xq, xd, n, s));
        i = j;
    }
    return hipSuccess;
}

// All layers for a chunk of n tokens whose embeddings are in d->x[0..n) and normed inputs in qa / da, positions
// from *d->pos. Leaves the last layer's down projection in d->o (not yet added to the residual stream).
hipError_t prefill_layers(Decoder* d, int n, hipStream_t s) {
    const qh_model_desc& hp = d->hp;
    const int D = hp.dim, F = hp.ffn_dim;
    for (int l = 0; l < hp.n_layers; ++l) {
        if (l > 0) {
            by_row_slots(D, [&](auto r) {
                qh_launch((add_rmsnorm_quant_kernel<decltype(r)::value>), dim3(n), dim3(256), 0, s, d->x,
                                   d->o, lf(d, l, L_ATTN_NORM), D, hp.norm_eps, d->qa, d->da, d->fa);
            });
            QH_TRY(hipGetLastError());
        }
        const qh_tensor &wq = lt(d, l, L_WQ), &wk = lt(d, l, L_WK), &wv = lt(d, l, L_WV);
        const MmOut qkv[3] = {{&wq, d->q, wq.rows, 0, wq.rows}, {&wk, d->k, wk.rows, 0, wk.rows},
                              {&wv, d->v, wv.rows, 0, wv.rows}};
        if (dense_w(wq) || dense_w(wk) || dense_w(wv)) {
            for (const MmOut& m : qkv) QH_TRY(linear(d, m.out, m.ldo, *m.W, false, n, s));
        } else {
            QH_TRY(matmul_group(qkv, 3, d->qa, d->da, n, s));
        }
        QH_TRY(attention(d, l, n, s));
        const qh_tensor& wo = lt(d, l, L_WO);
        QH_TRY(linear(d, d->o, wo.rows, wo, true, n, s));
        by_row_slots(D, [&](auto r) {
            qh_launch((add_rmsnorm_quant_kernel<decltype(r)::value>), dim3(n), dim3(256), 0, s, d->x, d->o,
                               lf(d, l, L_FFN_NORM), D, hp.norm_eps, d->qa, d->da, d->fa);
        });
        QH_TRY(hipGetLastError());
        const qh_tensor &wg = lt(d, l, L_WG), &wu = lt(d, l, L_WU), &wd = lt(d, l, L_WD);
        // a prefill stack: gate / up with the SwiGLU epilogue in one tile launch where the plan allows it
        const hipError_t sw = n > kChunk && d->fuse && !d->hadamard && !d->dense
                                  ? launch_matmul_swiglu(wg, wu, d->qa, d->da, n, d->qb, d->db, s)
                                  : hipErrorNotSupported;
        if (sw != hipErrorNotSupported) {
            QH_TRY(sw);
        } else if (!swiglu_fused(d, wg, wu, n, s)) {
            const MmOut gu[2] = {{&wg, d->g, wg.rows, 0, wg.rows}, {&wu, d->u, wu.rows, 0, wu.rows}};
            if (dense_w(wg) || dense_w(wu)) {
                for (const MmOut& m : gu) QH_TRY(linear(d, m.out, m.ldo, *m.W, false, n, s));
            } else {
                QH_TRY(matmul_group(gu, 2, d->qa, d->da, n, s));
            }
            QH_TRY(swiglu_down_input(d, F, n, s));
        }
        QH_TRY(hipGetLastError());
        QH_TRY(linear(d, d->o, wd.rows, wd, true, n, s));
    }
    return hipSuccess;
}

// The head on the quantized final hidden state in qa / da; top_k > 0 uses the shortlist.
// The head query of a forward (Session::head_query, session.cpp:63-79): with a query set, top_k follows its
// temperature and top_k, and its repetition penalty makes the history window the must ids; else the caller's top_k.
int query_top_k(const Decoder* d, int top_k) {
    if (!d->has_query) return top_k;
    return d->qp.temperature <= 0.f ? 1 : d->qp.top_k;
}

// The token history as a device-resident id list: its last `window` ids (all when window <= 0).
HeadMust history_window(const Decoder* d, int window) {
    HeadMust m;
    m.ids = d->hist;
    m.len_dev = d->hist_len;
    m.window = window;
    return m;
}

// The shortlist head runs for top_k > 0 queries on a model with head_q4 / head_err or with a nibble-plane LM head.
bool has_shortlist(const Decoder* d) { return head4(d).data != nullptr || d->lmh->dtype == kQ8P; }
bool shortlist_on(const Decoder* d, int top_k) { return query_top_k(d, top_k) > 0 && has_shortlist(d); }

// The feedback of a chosen token into the decoder's state.
TokenFeedback token_feedback(Decoder* d) {
    TokenFeedback fb;
    fb.token = d->tokens;
    fb.pos = d->pos;
    fb.n_out = d->n_out;
    fb.out = d->out;
    fb.out_cap = d->out_cap;
    fb.hist = d->hist;
    fb.hist_len = d->hist_len;
    fb.hist_cap = d->hp.ctx_len + 1;
    return fb;
}

// advance: a greedy decode step through the shortlist head, whose last kernel then also feeds the token back.
hipError_t run_head(Decoder* d, int top_k, hipStream_t s, bool advance = false) {
    const qh_tensor& h8 = *d->lmh;
    if (shortlist_on(d, top_k)) {
        qh_head_query q{query_top_k(d, top_k), d->hp.vocab_size, nullptr, 0};
        qh_head_out out{d->logits, d->coarse, d->upper, d->rows, d->stats};
        const HeadMust must = d->has_query && d->qp.repeat_penalty != 1.f ? history_window(d, d->qp.repeat_window)
                                                                           : HeadMust{};
        const TokenFeedback fb = token_feedback(d);
        return launch_shortlist_head(h8, head4(d), head_err(d), d->qa, d->da, q, must, out, d->head_ws, s,
                                     advance ? &fb : nullptr);
    }
    if (dense_w(h8))  // Model::linear on the final normed state itself (matvec_ref)
        QH_TRY(launch_gemv_dense(d->logits, 0, h8, d->hidden, h8.cols, 1, 0, h8.rows, s));
    else if (h8.dtype == kQ8P)
        QH_TRY(launch_gemv_planes(d->logits, h8, d->qa, d->da, 0, h8.rows, s));
    else
        QH_TRY(launch_gemv(d->logits, h8, d->qa, d->da, 0, h8.rows, gemv_plan(h8.dtype, h8.cols, h8.rows), s));
    return launch_argmax(d->logits, d->hp.vocab_size, d->top1_full, d->am_ws, s);
}


}  // namespace

// ------------------------------------------------------------------------------------------------- C-ABI glue

int decoder_create(const qh_model_desc* hp, const qh_tensor* tensors, int n_tensors, Decoder** out) {
    auto* d = new Decoder();
    d->hp = *hp;
    const char* fuse = getenv("QH_DECODER_FUSE");
    d->fuse = !(fuse && strcmp(fuse, "0") == 0);
    d->t.assign(tensors, tensors + n_tensors);
    const size_t n_lm = T_LAYER0 + (size_t)hp->n_layers * L_COUNT + 2;  // lm_head.weight's slot, when given
    d->lmh = d->t.size() > n_lm && d->t[n_lm].data ? &d->t[n_lm] : &d->t[T_EMBED];
    d->hadamard = (hp->flags & QH_FLAG_HADAMARD_DOWN) != 0;
    d->kv32 = hp->kv_f32 != 0;
    d->dense = dense_w(*d->lmh);
    for (int l = 0; l < hp->n_layers; ++l)
        for (int m : {L_WQ, L_WK, L_WV, L_WO, L_WG, L_WU, L_WD}) d->dense = d->dense || dense_w(lt(d, l, m));
    const int D = hp->dim, V = hp->vocab_size, hd = hp->head_dim;
    const size_t kvd = (size_t)hp->n_kv_heads * hd;
    const size_t kv_bytes = (size_t)hp->n_layers * hp->ctx_len * kvd * 2;
    const size_t v_bytes = (size_t)hp->n_layers * v_ctx(hp->ctx_len) * kvd * 2;
    const size_t kv32_bytes = (size_t)hp->n_layers * hp->ctx_len * kvd * 4;
    hipError_t e = hipSuccess;
    auto A = [&](void** p, size_t b) {
        if (e == hipSuccess) e = dalloc(d, p, b);
    };
    if (d->kv32) {
        A((void**)&d->kcf, kv32_bytes);
        A((void**)&d->vcf, kv32_bytes);
    } else {
        A((void**)&d->kc, kv_bytes);
        A((void**)&d->vc, v_bytes);
    }
    A((void**)&d->cs, sizeof(float) * (size_t)hp->ctx_len * hd);
    if (e == hipSuccess) e = alloc_stack(d, kChunk);
    A((void**)&d->hidden, sizeof(float) * D);
    d->escr_stride = escr_stride(hp->ctx_len);
    A((void**)&d->escr, sizeof(float) * 2 * (size_t)hp->n_heads * d->escr_stride);  // exp rows, weight rows
    A((void**)&d->tokens, sizeof(int32_t) * kChunk);
    A((void**)&d->hist, sizeof(int32_t) * ((size_t)hp->ctx_len + 1));
    A((void**)&d->hist_len, 256);
    A((void**)&d->rng, 256);
    A((void**)&d->sampled, 256);
    A((void**)&d->pos, 256);
    A((void**)&d->n_out, 256);
    A((void**)&d->status, 256);
    A((void**)&d->logits, sizeof(float) * V);
    A((void**)&d->coarse, sizeof(float) * V);
    A((void**)&d->upper, sizeof(float) * V);
    A((void**)&d->rows, sizeof(int32_t) * (size_t)(V + 64));
    A((void**)&d->stats, sizeof(qh_head_stats));
    A((void**)&d->top1_full, 256);
    if (has_shortlist(d)) {
        d->head_ws_bytes = head_workspace_bytes(V, D, 1);  // the same for every top_k the selection holds
        A(&d->head_ws, d->head_ws_bytes);
    }
    d->am_ws_bytes = argmax_workspace_bytes(V);
    A(&d->am_ws, d->am_ws_bytes);
    if (V <= QH_SAMPLE_MAX_VOCAB) A(&d->sample_ws, sample_workspace_bytes(V));
    if (e != hipSuccess) {
        decoder_destroy(d);
        return check_hip(e, "qh_decoder_create allocation");
    }
    // RoPE angle table with the reference's formula and the host's libm (ops_ref.cpp:201-214).
    std::vector<float> cs((size_t)hp->ctx_len * hd);
    const int half = hd / 2;
    for (int p = 0; p < hp->ctx_len; ++p)
        for (int i = 0; i < half; ++i) {
            const float freq = powf(hp->rope_theta, -2.0f * (float)i / (float)hd);
            const float angle = (float)p * freq;
            cs[((size_t)p * half + i) * 2] = cosf(angle);
            cs[((size_t)p * half + i) * 2 + 1] = sinf(angle);
        }
    e = hipMemcpy(d->cs, cs.data(), sizeof(float) * cs.size(), hipMemcpyHostToDevice);
    for (int* p : {d->n_out, d->pos, d->status, d->hist_len})
        if (e == hipSuccess) e = hipMemset(p, 0, 256);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        decoder_destroy(d);
        return check_hip(e, "qh_decoder_create upload");
    }
    *out = d;
    return QH_OK;
}

void decoder_destroy(Decoder* d) {
    if (!d) return;
    for (void* p : d->allocs) (void)hipFree(p);
    delete d;
}

hipError_t decoder_set_prefill_stack(Decoder* d, int c) {
    if (c == d->stack) return hipSuccess;
    QH_TRY(hipDeviceSynchronize());  // nothing in flight uses the buffers that are replaced
    void** slots[] = {(void**)&d->x,  (void**)&d->o,  (void**)&d->q,  (void**)&d->k,  (void**)&d->v,
                      (void**)&d->g,  (void**)&d->u,  (void**)&d->qa, (void**)&d->qb, (void**)&d->da,
                      (void**)&d->db, (void**)&d->fa, (void**)&d->fb, (void**)&d->subpos};
    constexpr int kSlots = (int)(sizeof(slots) / sizeof(slots[0]));
    void* old[kSlots];
    for (int i = 0; i < kSlots; ++i) {
        old[i] = *slots[i];
        *slots[i] = nullptr;
    }
    const hipError_t e = alloc_stack(d, c);
    for (int i = 0; i < kSlots; ++i) {
        void* drop = e == hipSuccess ? old[i] : *slots[i];
        if (e != hipSuccess) *slots[i] = old[i];  // keep the previous stack on failure
        dfree(d, drop);
    }
    if (e == hipSuccess) d->stack = c;
    return e;
}

hipError_t decoder_prefill(Decoder* d, const int32_t* tokens, int n, int pos0, int top_k, hipStream_t s) {
    const qh_model_desc& hp = d->hp;
    const int D = hp.dim;
    qh_launch(set_int_kernel, dim3(1), dim3(1), 0, s, d->status, 0);
    QH_TRY(hipGetLastError());
    qh_launch(history_append_kernel, dim3(1), dim3(256), 0, s, tokens, n, pos0 == 0 ? 1 : 0, d->hist,
                       d->hist_len, hp.ctx_len + 1);
    QH_TRY(hipGetLastError());
    int last = 0;
    for (int c0 = 0; c0 < n; c0 += d->stack) {
        const int m = n - c0 < d->stack ? n - c0 : d->stack;
        if (m > kChunk) {
            qh_launch(set_subpos_kernel, dim3(1), dim3(kMaxStack / kChunk), 0, s, d->subpos, pos0 + c0,
                      (m + kChunk - 1) / kChunk);
            QH_TRY(hipGetLastError());
        }
        qh_launch(set_int_kernel, dim3(1), dim3(1), 0, s, d->pos, pos0 + c0);
        QH_TRY(hipGetLastError());
        d->stack_end = pos0 + c0 + m;
        QH_TRY(embed(d, tokens + c0, m, s));
        QH_TRY(prefill_layers(d, m, s));
        last = m - 1;
    }
    // final residual add, norm and quantization of the last token only, then the head
    by_row_slots(D, [&](auto r) {
        qh_launch((add_rmsnorm_quant_kernel<decltype(r)::value>), dim3(1), dim3(256), 0, s,
                           d->x + (size_t)last * D, d->o + (size_t)last * D, final_norm(d), D, hp.norm_eps, d->qa,
                           d->da, d->hidden);
    });
    QH_TRY(hipGetLastError());
    QH_TRY(run_head(d, top_k, s));
    qh_launch(set_int_kernel, dim3(1), dim3(1), 0, s, d->pos, pos0 + n);
    return hipGetLastError();
}

// Picks the token from the last head call (the sampler when one is set) and feeds it back (advance: a decode step).
hipError_t pick_and_advance(Decoder* d, int top_k, bool advance, hipStream_t s) {
    const bool sl = shortlist_on(d, top_k);
    Pick pick{nullptr, sl ? d->stats : nullptr, d->top1_full};
    if (d->has_sampler) {
        const HeadMust hist = d->sp.repeat_penalty != 1.f ? history_window(d, d->sp.repeat_window) : HeadMust{};
        QH_TRY(launch_sample(d->logits, d->hp.vocab_size, sl ? d->rows : nullptr, sl ? d->stats : nullptr, hist,
                             d->sp, d->rng, d->sampled, d->sample_ws, s));
        pick.sampled = d->sampled;
    }
    qh_launch(advance_kernel, dim3(1), dim3(1), 0, s, pick, token_feedback(d), advance ? 1 : 0);
    return hipGetLastError();
}

hipError_t decoder_step(Decoder* d, int top_k, hipStream_t s) {
    QH_TRY(decode_layers(d, s));
    if (!d->has_sampler && shortlist_on(d, top_k)) {  // greedy: fed back in the head
        QH_TRY(run_head(d, top_k, s, true));
        d->mark(QH_STAGE_HEAD);
        return hipSuccess;
    }
    QH_TRY(run_head(d, top_k, s));
    d->mark(QH_STAGE_HEAD);
    QH_TRY(pick_and_advance(d, top_k, true, s));
    d->mark(QH_STAGE_PICK);
    return hipSuccess;
}

int decoder_step_timed(Decoder* d, int top_k, hipStream_t s, float* us, int32_t* stage, int cap, int32_t* n) {
    KernelTimer t;
    t.ev.assign(2 * (size_t)cap, nullptr);
    int rc = QH_OK;
    for (hipEvent_t& e : t.ev)
        if (!rc) rc = check_hip(hipEventCreate(&e), "hipEventCreate");
    if (!rc) {
        kernel_timer() = &t;
        const hipError_t e = decoder_step(d, top_k, s);
        kernel_timer() = nullptr;
        rc = check_hip(e, "qh_decoder_step_timed");
    }
    if (!rc) rc = check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
    if (!rc && t.launched > cap)
        rc = fail(QH_ERR_NOMEM, "qh_decoder_step_timed: the step launched %d kernels, more than the %d timing slots (the "
                  "step has run)", t.launched, cap);
    for (int i = 0; !rc && i < t.n; ++i) {
        rc = check_hip(hipEventElapsedTime(&us[i], t.ev[2 * i], t.ev[2 * i + 1]), "hipEventElapsedTime");
        us[i] *= 1e3f;
        stage[i] = t.stage[i];
    }
    for (hipEvent_t e : t.ev)
        if (e) (void)hipEventDestroy(e);
    if (!rc || t.launched > cap) *n = t.launched;
    return rc;
}

hipError_t decoder_begin(Decoder* d, int top_k, int32_t* out, int out_cap, hipStream_t s) {
    d->out = out;
    d->out_cap = out_cap;
    qh_launch(set_int_kernel, dim3(1), dim3(1), 0, s, d->n_out, 0);
    QH_TRY(hipGetLastError());
    return pick_and_advance(d, top_k, false, s);
}

int decoder_ctx(const Decoder* d) { return d->hp.ctx_len; }

#if defined(QH_TIMELINE)
extern "C" int qh_timeline_pa_read(uint64_t* host, int n) {
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(qh_tl_pa), sizeof(uint64_t) * (n < 16 ? n : 16)) == hipSuccess ? 0 : 1;
}

extern "C" int qh_timeline_read(uint64_t* host, int n) {
    return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(qh_tl), sizeof(uint64_t) * (size_t)n);
}
extern "C" int qh_timeline_wg_read(uint64_t* host) {
    return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(qh_tl_wg), sizeof(qh_tl_wg));
}
#endif

void decoder_views(Decoder* d, qh_decoder_state* v) {
    v->logits = d->logits;
    v->hidden = d->hidden;
    v->xq = d->qa;
    v->xd = d->da;
    v->stats = d->stats;
    v->top1_full = d->top1_full;
    v->pos = d->pos;
    v->n_out = d->n_out;
    v->token = d->tokens;
    v->kcache = d->kc;
    v->vcache = d->vc;
    v->kcache_f32 = d->kcf;
    v->vcache_f32 = d->vcf;
    v->status = d->status;
    v->history = d->hist;
    v->history_len = d->hist_len;
    v->rng_state = d->rng;
}

int decoder_vocab(const Decoder* d) { return d->hp.vocab_size; }

bool decoder_has_shortlist(const Decoder* d) { return has_shortlist(d); }

int decoder_set_query(Decoder* d, const qh_sampler_params* p) {
    d->has_query = p != nullptr;
    if (p) d->qp = *p;
    return 0;
}

hipError_t decoder_set_sampler(Decoder* d, const qh_sampler_params* p, uint64_t seed) {
    d->has_sampler = p != nullptr;
    if (!p) return hipSuccess;
    d->sp = *p;
    const uint64_t st = seed | 1u;  // Sampler's constructor (sampler.cpp:10-13)
    return hipMemcpy(d->rng, &st, sizeof st, hipMemcpyHostToDevice);
}

}  // namespace qh
