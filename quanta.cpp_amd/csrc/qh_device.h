// Device helpers shared by the gfx950 kernels: exact conversions, int8 dot products, wave reductions.
//
// Float rules (all kernels are compiled with -ffp-contract=off): a fused multiply-add appears only as an
// explicit __builtin_fmaf, division and sqrt stay correctly rounded, and f32 / f16 denormals are kept,
// so every f32 result matches the reference's scalar CPU code bit for bit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qh {

constexpr int QK = 32;
constexpr int kQ8 = 2;  // dtype numbers as in the .qnt file
constexpr int kQ4 = 3;

// IEEE binary16 bits -> binary32 (exact for every input, subnormals included): v_cvt_f32_f16.
__device__ __forceinline__ float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

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

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const uint64_t o = __shfl_xor(v, off, 64);
        v = o > v ? o : v;
    }
    return v;
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
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
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

__device__ __forceinline__ uint4 load16(const void* p) { return *reinterpret_cast<const uint4*>(p); }

// The same chain over 16-byte aligned operands, read four blocks per LDS access.
__device__ __forceinline__ float chain_lds4(const float* p, const float* dx, int nb) {
    float acc = 0.0f;
    int b = 0;
#pragma unroll 4
    for (; b + 4 <= nb; b += 4) {
        const float4 pv = *reinterpret_cast<const float4*>(p + b);
        const float4 xv = *reinterpret_cast<const float4*>(dx + b);
        acc = __builtin_fmaf(pv.x, xv.x, acc);
        acc = __builtin_fmaf(pv.y, xv.y, acc);
        acc = __builtin_fmaf(pv.z, xv.z, acc);
        acc = __builtin_fmaf(pv.w, xv.w, acc);
    }
    for (; b < nb; ++b) acc = __builtin_fmaf(p[b], dx[b], acc);
    return acc;
}

// Row stride (floats) of an LDS product tile read by chain_lds4: a multiple of 4, and not a multiple of 32, so
// the 16-byte reads of neighbouring rows fall in different banks.
__host__ __device__ __forceinline__ int prod_stride4(int nb) {
    const int p = (nb + 3) & ~3;
    return (p & 31) == 0 ? p + 4 : p;
}


}  // namespace qh
