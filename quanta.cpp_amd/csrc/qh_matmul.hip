// Prefill matmul for n tokens (reference ops_ref.cpp:122-160, contract ops.h:65-70) on gfx950 int8 MFMA.
//
// v_mfma_i32_16x16x32_i8 takes K = 32 per instruction, exactly one Q8_0 / Q4_0 block, so every block's
// exact int32 dot s(row, token, b) arrives in registers on its own and the per-(row, token) chain
// acc = fma(float(s) * dw_b, dx_b, acc) runs in block order in the lane that holds the element: each
// output equals the decode GEMV bit for bit. (The K = 64 forms would merge two scale blocks.)
//
// Tiling: a wave computes a 16-row x 16-token tile over the whole K; a workgroup of four waves covers
// 64 consecutive rows and shares the 16 token rows through L1. Operand layout for one block b: lane l
// supplies row (l % 16) and k-group (l / 16) as 8 int8 values; the activation operand uses the same
// k-group split, so the integer sum pairs the same elements. Q4_0 nibbles are unpacked in registers to
// signed bytes (k-groups 0,1 take the low nibbles of bytes 0-7 / 8-15, k-groups 2,3 the high ones).
// The result register i of lane l is row 4*(l/16)+i, token l%16.
#include "qh_device.h"
#include "qh_internal.h"

namespace qh {

typedef int v4i __attribute__((ext_vector_type(4)));

// Nibbles (0..15 per byte) -> signed bytes (nibble - 8), no borrow between bytes.
__device__ __forceinline__ uint32_t nibbles_to_i8(uint32_t v) { return ((v | 0x80808080u) - 0x08080808u) ^ 0x80808080u; }

template <int DT>
__global__ __launch_bounds__(256) void matmul_kernel(float* __restrict__ out, int ldo, const uint8_t* __restrict__ wq,
                                                     const uint16_t* __restrict__ wscale,
                                                     const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                     int cols, int n, int r0, int r1) {
    const int nb = cols / QK;
    const int lane = (int)threadIdx.x & 63, wave = (int)threadIdx.x >> 6;
    const int li = lane & 15, lq = lane >> 4;
    const int rbase = r0 + (int)blockIdx.x * 64 + wave * 16;
    const int tbase = (int)blockIdx.y * 16;
    if (rbase >= r1) return;  // whole wave past the last row (uniform per wave)

    // Operand rows; rows / tokens past the end are clamped for loading and never stored.
    const int arow = min(rbase + li, r1 - 1);
    const int btok = min(tbase + li, n - 1);
    const int8_t* xrow = xq + (size_t)btok * cols + lq * 8;
    const float* dxrow = xd + (size_t)btok * nb;
    const uint16_t* srow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) srow[i] = wscale + (size_t)min(rbase + 4 * lq + i, r1 - 1) * nb;

    const uint8_t* wrow;
    int shift = 0;
    if (DT == kQ8) {
        wrow = wq + (size_t)arow * cols + lq * 8;
    } else {
        wrow = wq + (size_t)arow * (cols / 2) + (lq & 1) * 8;
        shift = (lq >> 1) * 4;
    }

    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int b = 0; b < nb; ++b) {
        long a;
        if (DT == kQ8) {
            a = *reinterpret_cast<const long*>(wrow + (size_t)b * QK);
        } else {
            const uint2 v = *reinterpret_cast<const uint2*>(wrow + (size_t)b * (QK / 2));
            const uint32_t lo = nibbles_to_i8((v.x >> shift) & 0x0F0F0F0Fu);
            const uint32_t hi = nibbles_to_i8((v.y >> shift) & 0x0F0F0F0Fu);
            a = (long)(((uint64_t)hi << 32) | lo);
        }
        const long x = *reinterpret_cast<const long*>(xrow + (size_t)b * QK);
        v4i c = {0, 0, 0, 0};
        c = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, x, c, 0, 0, 0);
        const float dx = dxrow[b];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = __builtin_fmaf((float)c[i] * f16_to_f32(srow[i][b]), dx, acc[i]);
    }
    const int tok = tbase + li;
    if (tok < n) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = rbase + 4 * lq + i;
            if (r < r1) out[(size_t)tok * ldo + r] = acc[i];
        }
    }
}

hipError_t launch_matmul(float* out, int ldo, const qh_tensor& W, const int8_t* xq, const float* xd, int n, int r0,
                         int r1, hipStream_t s) {
    const uint8_t* wq = static_cast<const uint8_t*>(W.data);
    const uint16_t* ws = reinterpret_cast<const uint16_t*>(wq + qh_quant_bytes(W.dtype, W.rows, W.cols));
    const dim3 grid((unsigned)((r1 - r0 + 63) / 64), (unsigned)((n + 15) / 16));
    if (W.dtype == kQ8)
        hipLaunchKernelGGL(matmul_kernel<kQ8>, grid, dim3(256), 0, s, out, ldo, wq, ws, xq, xd, W.cols, n, r0, r1);
    else
        hipLaunchKernelGGL(matmul_kernel<kQ4>, grid, dim3(256), 0, s, out, ldo, wq, ws, xq, xd, W.cols, n, r0, r1);
    return hipGetLastError();
}

}  // namespace qh
