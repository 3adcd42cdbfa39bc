// Device helpers shared by the gfx950 kernels: exact conversions, int8 dot products, wave reductions.
//
// Float rules (all kernels are compiled with -ffp-contract=off): a fused multiply-add appears only as an
// explicit __builtin_fmaf, division and sqrt stay correctly rounded, and f32 / f16 denormals are kept,
// so every f32 result matches the reference's scalar CPU code bit for bit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

#include "qh_math.h"

namespace qh {

constexpr int QK = 32;
constexpr int kF32 = 0;  // dtype numbers as in the .qnt file
constexpr int kF16 = 1;
constexpr int kQ8 = 2;
constexpr int kQ4 = 3;
constexpr int kQ8P = 16;  // the device-only nibble-plane layout of a Q8_0 head (QH_Q8_0_PLANES)

// IEEE binary16 bits -> binary32 (exact for every input, subnormals included): v_cvt_f32_f16.
__device__ __forceinline__ float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// A block product float(s) * d in one FMA. An integer sum that starts from kSumBias (the bits of B = 1.5 * 2^23) ends
// at the bits of the float B + s, exactly, for |s| < 2^22 (a block's |s| <= 32 * 128 * 128 = 2^19); then
// fma(B + s, d, -(B * d)) is the exact value s * d rounded once, the same f32 as float(s) * d, because B * d needs at
// most 13 significant bits for an f16 scale d, so -(B * d) is exact (checked on the CPU for every finite f16 d and
// |s| <= 2^19, apart from the sign of a zero product, which a chain acc = fma(p, dx, acc) from +0 never shows). Not
// for d = inf or NaN (the terms cancel into NaN, or the NaN's sign flips): callers take (B + s - B) * d there, which
// is float(s) * d again.
constexpr int kSumBias = 0x4B400000;
constexpr float kSumBiasF = 12582912.0f;
// True for the f16 bits of inf and NaN (the scales the one-FMA product cannot take).
__device__ __forceinline__ bool f16_nonfinite(uint32_t h) { return (h & 0x7C00u) == 0x7C00u; }

// The f16 bits at p (2-byte aligned) through a 4-byte load of the aligned word holding them: 16-bit global loads cost
// gfx950 far more than 32-bit ones (measured: eight per lane add about 1.8 us to a scattered row fetch against 0.2 us
// as words). The word starts inside the array, so it stays inside the allocation's granule even where it reaches
// 2 bytes past the array's last element.
// The word's address is p stepped back by one element (not an integer cast), so the load keeps p's address space.
__device__ __forceinline__ uint16_t load_f16_bits(const uint16_t* p) {
    const int odd = (int)((reinterpret_cast<uintptr_t>(p) >> 1) & 1);
    const uint32_t w = *reinterpret_cast<const uint32_t*>(p - odd);
    return (uint16_t)(odd ? (w >> 16) : w);
}

// Round half away from zero (lroundf semantics) of a value whose magnitude is below 2^23.
__device__ __forceinline__ float round_half_away(float y) {
    const float t = __builtin_truncf(y);
    return __builtin_fabsf(y - t) >= 0.5f ? t + __builtin_copysignf(1.0f, y) : t;
}

// Signed 4 x int8 dot product with int32 accumulate (v_dot4_i32_i8); exact.
__device__ __forceinline__ int dot4(int a, int b, int acc) { return __builtin_amdgcn_sdot4(a, b, acc, false); }

// Value of the neighbouring lane (lane ^ 1) via DPP quad_perm [1,0,3,2].
__device__ __forceinline__ int swap_pair(int v) { return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false); }

// Exact floor(g / d) for g < 2^32 / d, with magic = ceil(2^32 / d) computed on the host.
__device__ __forceinline__ uint32_t div_magic(uint32_t g, uint32_t magic) { return __umulhi(g, magic); }

// Monotone map of a float onto uint32 (larger float -> larger key); finite values and infinities.
__device__ __forceinline__ uint32_t ordered_bits(float f) {
    const uint32_t u = __builtin_bit_cast(uint32_t, f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float from_ordered_bits(uint32_t k) {
    const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return __builtin_bit_cast(float, u);
}

// Score key: higher score first, then lower row first; 0 means "no entry".
__device__ __forceinline__ uint64_t score_key(float score, int row) {
    return ((uint64_t)ordered_bits(score) << 32) | (uint64_t)(0xffffffffu - (uint32_t)row);
}
__device__ __forceinline__ int key_row(uint64_t k) { return (int)(0xffffffffu - (uint32_t)k); }
__device__ __forceinline__ float key_score(uint64_t k) { return from_ordered_bits((uint32_t)(k >> 32)); }

// Whole-wave reductions (every lane active) in registers: DPP exchanges within rows of 16 lanes (quad_perm
// [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror), then the gfx950 row swaps 16 and 32 lanes apart; every lane
// ends with the result. No LDS round trips.
template <typename T, typename Op>
__device__ __forceinline__ T wave_reduce32x2(T v, Op op) {
    static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit values");
    auto dpp = [](T x, auto ctrl) {
        if constexpr (sizeof(T) == 4) {
            return __builtin_bit_cast(T, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), decltype(ctrl)::value,
                                                                  0xF, 0xF, false));
        } else {
            const uint64_t u = __builtin_bit_cast(uint64_t, x);
            const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)u, decltype(ctrl)::value, 0xF, 0xF, false);
            const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(u >> 32), decltype(ctrl)::value, 0xF,
                                                                  0xF, false);
            return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
        }
    };
    auto swap = [](T x, auto rows32) {  // {x of this lane's pair partner row or half, x}
        if constexpr (sizeof(T) == 4) {
            const uint32_t u = __builtin_bit_cast(uint32_t, x);
            const auto r = decltype(rows32)::value ? __builtin_amdgcn_permlane32_swap(u, u, false, false)
                                                   : __builtin_amdgcn_permlane16_swap(u, u, false, false);
            return std::pair<T, T>{__builtin_bit_cast(T, (uint32_t)r[0]), __builtin_bit_cast(T, (uint32_t)r[1])};
        } else {
            const uint64_t u = __builtin_bit_cast(uint64_t, x);
            const uint32_t lo = (uint32_t)u, hi = (uint32_t)(u >> 32);
            const auto a = decltype(rows32)::value ? __builtin_amdgcn_permlane32_swap(lo, lo, false, false)
                                                   : __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
            const auto b = decltype(rows32)::value ? __builtin_amdgcn_permlane32_swap(hi, hi, false, false)
                                                   : __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
            return std::pair<T, T>{__builtin_bit_cast(T, ((uint64_t)(uint32_t)b[0] << 32) | (uint32_t)a[0]),
                                   __builtin_bit_cast(T, ((uint64_t)(uint32_t)b[1] << 32) | (uint32_t)a[1])};
        }
    };
    v = op(v, dpp(v, std::integral_constant<int, 0xB1>{}));
    v = op(v, dpp(v, std::integral_constant<int, 0x4E>{}));
    v = op(v, dpp(v, std::integral_constant<int, 0x141>{}));
    v = op(v, dpp(v, std::integral_constant<int, 0x140>{}));
    const auto p16 = swap(v, std::false_type{});
    v = op(p16.first, p16.second);
    const auto p32 = swap(v, std::true_type{});
    return op(p32.first, p32.second);
}

// Lane exchanges for block maxima, all in registers (DPP and the gfx950 row swap; no LDS round trips).
template <int kCtrl>
__device__ __forceinline__ float dpp_max(float a) {
    const float o = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a), kCtrl, 0xF, 0xF, false));
    return __builtin_fmaxf(a, o);
}
// Maximum over each aligned group of 8 lanes (every lane of the group active).
__device__ __forceinline__ float max8_lanes(float a) {
    a = dpp_max<0xB1>(a);   // quad_perm [1,0,3,2]
    a = dpp_max<0x4E>(a);   // quad_perm [2,3,0,1]
    return dpp_max<0x141>(a);  // row_half_mirror: lane i <-> 7 - i within each 8
}
// Maximum over each aligned group of 32 lanes (every lane of the group active).
__device__ __forceinline__ float max32_lanes(float a) {
    a = max8_lanes(a);
    a = dpp_max<0x140>(a);  // row_mirror: lane i <-> 15 - i within each 16
    const uint32_t u = __builtin_bit_cast(uint32_t, a);
    const auto sw = __builtin_amdgcn_permlane16_swap(u, u, false, false);  // rows 0 <-> 1 and 2 <-> 3
    return __builtin_fmaxf(__builtin_bit_cast(float, (uint32_t)sw[0]), __builtin_bit_cast(float, (uint32_t)sw[1]));
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    return wave_reduce32x2(v, [](uint64_t a, uint64_t b) { return a > b ? a : b; });
}

// Sorts a[0, p2) (p2 a power of two) largest first with a bitonic network; every thread of the workgroup (kThreads of
// them) calls it, and a barrier ends every stage. The caller pads a to p2 with zeros.
template <int kThreads>
__device__ void bitonic_sort_desc_u64(uint64_t* a, int p2) {
    const int tid = (int)threadIdx.x;
    for (int size = 2; size <= p2; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int t = tid; t < p2 / 2; t += kThreads) {
                const int lo = 2 * t - (t & (stride - 1)), hi = lo + stride;
                const bool desc = (lo & size) == 0;
                const uint64_t x = a[lo], y = a[hi];
                if (desc ? x < y : x > y) {
                    a[lo] = y;
                    a[hi] = x;
                }
            }
            __syncthreads();
        }
    }
}

__device__ __forceinline__ int wave_sum_i32(int v) {
    return wave_reduce32x2(v, [](int a, int b) { return a + b; });
}

// 16 signed int8 weights . 16 signed int8 activations.
__device__ __forceinline__ int dot16_i8(const uint4 w, const uint4 x) {
    int s = dot4((int)w.x, (int)x.x, 0);
    s = dot4((int)w.y, (int)x.y, s);
    s = dot4((int)w.z, (int)x.z, s);
    return dot4((int)w.w, (int)x.w, s);
}

// One Q4_0 block (16 packed bytes) . its 32 int8 activations: low nibbles pair with elements 0-15,
// high nibbles with 16-31, each nibble minus 8. The -8 offset is applied as 4-byte dots against
// 0xF8F8F8F8 (= -8 in every byte), so the whole sum stays in exact int32 arithmetic.
__device__ __forceinline__ int dot_q4_block(const uint4 w, const uint4 xlo, const uint4 xhi) {
    constexpr int kLo = 0x0F0F0F0F, kM8 = (int)0xF8F8F8F8u;
    int s = dot4((int)w.x & kLo, (int)xlo.x, 0);
    s = dot4((int)w.y & kLo, (int)xlo.y, s);
    s = dot4((int)w.z & kLo, (int)xlo.z, s);
    s = dot4((int)w.w & kLo, (int)xlo.w, s);
    s = dot4((int)(w.x >> 4) & kLo, (int)xhi.x, s);
    s = dot4((int)(w.y >> 4) & kLo, (int)xhi.y, s);
    s = dot4((int)(w.z >> 4) & kLo, (int)xhi.z, s);
    s = dot4((int)(w.w >> 4) & kLo, (int)xhi.w, s);
    s = dot4(kM8, (int)xlo.x, s);
    s = dot4(kM8, (int)xlo.y, s);
    s = dot4(kM8, (int)xlo.z, s);
    s = dot4(kM8, (int)xlo.w, s);
    s = dot4(kM8, (int)xhi.x, s);
    s = dot4(kM8, (int)xhi.y, s);
    s = dot4(kM8, (int)xhi.z, s);
    return dot4(kM8, (int)xhi.w, s);
}

// 32 unsigned nibbles (Q4_0 packing: low nibbles are elements 0-15, high nibbles 16-31, no offset) . 32 int8
// activations: 8 four-byte dots, exact int32.
__device__ __forceinline__ int dot_u4_block(const uint4 w, const uint4 xlo, const uint4 xhi) {
    constexpr int kLo = 0x0F0F0F0F;
    int s = dot4((int)w.x & kLo, (int)xlo.x, 0);
    s = dot4((int)w.y & kLo, (int)xlo.y, s);
    s = dot4((int)w.z & kLo, (int)xlo.z, s);
    s = dot4((int)w.w & kLo, (int)xlo.w, s);
    s = dot4((int)(w.x >> 4) & kLo, (int)xhi.x, s);
    s = dot4((int)(w.y >> 4) & kLo, (int)xhi.y, s);
    s = dot4((int)(w.z >> 4) & kLo, (int)xhi.z, s);
    return dot4((int)(w.w >> 4) & kLo, (int)xhi.w, s);
}

__device__ __forceinline__ uint4 load16(const void* p) { return *reinterpret_cast<const uint4*>(p); }

// Accumulator of one 16x16x32 int8 MFMA.
typedef int v4i __attribute__((ext_vector_type(4)));

// Nibbles (0..15 per byte) -> signed bytes (nibble - 8), no borrow between bytes.
__device__ __forceinline__ uint32_t nibbles_to_i8(uint32_t v) { return ((v | 0x80808080u) - 0x08080808u) ^ 0x80808080u; }

// Pipelined chain rows (chain_lds_pipe): a row of nb operands is stored as chain_len32(nb) - nb zeros followed by
// the nb operands, rows chain_stride32(nb) floats apart (16-byte aligned, 4 mod 32 floats, so 16-byte reads of
// neighbouring rows fall in different banks), and kChainPipePad readable floats follow the last row.
constexpr int kChainPipePad = 32;
__host__ __device__ __forceinline__ int chain_len32(int nb) { return (nb + 31) & ~31; }
__host__ __device__ __forceinline__ int chain_stride32(int nb) { return chain_len32(nb) + 4; }

// Zeros in front of the padded chain rows of dxs and of rows [0, nrows) of prod (rows chain_stride32(nb) apart), by a
// workgroup of 256 threads.
__device__ __forceinline__ void zero_chain_prefix(float* dxs, float* prod, int nb, int nrows) {
    const int zp = chain_len32(nb) - nb, ps = chain_stride32(nb), tid = (int)threadIdx.x;
    if (zp == 0) return;
    if ((zp & 3) == 0) {  // uniform (nb % 4 == 0): thread r writes the 16-byte zero groups of padded row r
        for (int r = tid; r <= nrows; r += 256) {
            float4* z = reinterpret_cast<float4*>(r == 0 ? dxs : prod + (size_t)(r - 1) * ps);
            for (int k = 0; k < (zp >> 2); ++k) z[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        return;
    }
    for (int i = tid; i < (nrows + 1) * 32; i += 256) {  // 256-thread workgroups
        const int r = i >> 5, j = i & 31;
        if (j < zp) (r == 0 ? dxs : prod + (size_t)(r - 1) * ps)[j] = 0.0f;
    }
}

// The serial chain over a padded row: acc = fma(p[i], dx[i], acc) for i in [0, L), L a multiple of 32. The leading
// zeros of p and dx leave acc = +0 exactly (fma(0, 0, +0) = +0), so the result is the chain over the nb operands
// from +0, the reference's order. Operands arrive 8 at a time (two 16-byte LDS reads of each) in NB rotating
// batches, NB - 1 in flight while one is consumed, so the chain runs at the FMA latency rather than the LDS
// latency (NB = 4; NB = 2 holds 32 fewer registers); the reads reach 32 floats past p + L and dx + L. p and dx are
// 16-byte aligned.
template <int NB = 4>
__device__ __forceinline__ float chain_lds_pipe(const float* p, const float* dx, int L) {
    static_assert(NB == 2 || NB == 4, "two or four batches");
    struct Batch {
        float4 p0, p1, x0, x1;
    };
    auto ld = [&](Batch& q, int b) {
        q.p0 = *reinterpret_cast<const float4*>(p + b);
        q.p1 = *reinterpret_cast<const float4*>(p + b + 4);
        q.x0 = *reinterpret_cast<const float4*>(dx + b);
        q.x1 = *reinterpret_cast<const float4*>(dx + b + 4);
    };
    float acc = 0.0f;
    auto use = [&](const Batch& q) {
        acc = __builtin_fmaf(q.p0.x, q.x0.x, acc);
        acc = __builtin_fmaf(q.p0.y, q.x0.y, acc);
        acc = __builtin_fmaf(q.p0.z, q.x0.z, acc);
        acc = __builtin_fmaf(q.p0.w, q.x0.w, acc);
        acc = __builtin_fmaf(q.p1.x, q.x1.x, acc);
        acc = __builtin_fmaf(q.p1.y, q.x1.y, acc);
        acc = __builtin_fmaf(q.p1.z, q.x1.z, acc);
        acc = __builtin_fmaf(q.p1.w, q.x1.w, acc);
    };
    // The first batch passes through an empty asm: the loop's reload of a batch is then not merged with its first
    // load into one load at the top of the loop, which would leave nothing in flight across iterations. Only the
    // first: the asm waits for its operands, and the other batches' reads stay in flight into the loop.
    auto pin = [](Batch& q) {
        asm volatile("" : "+v"(q.p0.x), "+v"(q.p0.y), "+v"(q.p0.z), "+v"(q.p0.w), "+v"(q.p1.x), "+v"(q.p1.y),
                     "+v"(q.p1.z), "+v"(q.p1.w));
        asm volatile("" : "+v"(q.x0.x), "+v"(q.x0.y), "+v"(q.x0.z), "+v"(q.x0.w), "+v"(q.x1.x), "+v"(q.x1.y),
                     "+v"(q.x1.z), "+v"(q.x1.w));
    };
    Batch q[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) ld(q[i], 8 * i);
    pin(q[0]);
    for (int b = 0; b < L; b += 8 * NB) {  // the scheduling barriers keep each batch's reads ahead of the next FMAs
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            use(q[i]);
            ld(q[i], b + 8 * (NB + i));
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    return acc;
}

// glibc-identical expf on the device (all 2^32 inputs checked against the host's expf in tests).
__device__ __forceinline__ float dev_expf(float x) { return expf_variant<2>(x); }
// The same with its table in LDS (ExpTab): a table read from global memory costs a cache round trip per call.
struct ExpTab {
    uint64_t v;  // thread t < 32: entry t, loaded first thing
    __device__ __forceinline__ void load() { v = expf_detail::kTab[min((int)threadIdx.x, 31)]; }
    __device__ __forceinline__ void store(uint64_t* lds) const {
        if (threadIdx.x < 32) lds[threadIdx.x] = v;
    }
};
__device__ __forceinline__ float dev_expf(float x, const uint64_t* lds_tab) { return expf_variant<2>(x, lds_tab); }

// quantize_q8 of one 32-block (ops_ref.cpp:69-83) held one value per lane by an aligned group of 32 lanes: amax
// (the maximum does not depend on the order of comparison), d = amax / 127, inv = d > 0 ? 1 / d : 0, and
// q = lround(v * inv).
__device__ __forceinline__ void quant_block32(float v, int8_t* __restrict__ q, float* __restrict__ d) {
    const float a = max32_lanes(__builtin_fabsf(v));
    const float sc = a / 127.0f;
    const float inv = sc > 0.0f ? 1.0f / sc : 0.0f;
    const int i = (int)threadIdx.x & 31;
    q[i] = (int8_t)(int)round_half_away(v * inv);
    if (i == 0) *d = sc;
}

}  // namespace qh
