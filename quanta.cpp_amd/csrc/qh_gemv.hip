// Decode-side kernels: activation quantization (reference ops_ref.cpp:69-83) and the Q8_0 / Q4_0
// integer-dot GEMV (reference ops_ref.cpp:85-120), for gfx950.
//
// GEMV data flow. A workgroup owns a tile of consecutive rows. In the .qnt layout the quants of those
// rows are one contiguous byte range, so the workgroup streams it with coalesced 16-byte loads
// (thread t takes chunks t, t+256, ...), independent of the row length. A Q8_0 block is two chunks
// (a lane pair, combined with one DPP swap), a Q4_0 block is one chunk. Each block's exact int32 dot
// is turned into p = float(s) * f16(scale) (one rounded multiply, order-free) and parked in LDS at
// [row][block]. After one barrier, thread r runs row r's serial chain acc = fma(p_b, dx_b, acc) over
// the blocks in order, which is the reference's float association, so the result is bit-identical.
// The activation (at most a few KB) is read straight from global memory and stays in L1/L2.
#include <stdio.h>
#include <stdlib.h>

#include "qh_device.h"
#include "qh_internal.h"

namespace qh {

// One wave quantizes two 32-blocks (one per half-wave, one element per lane).
__global__ __launch_bounds__(256) void quantize_q8_kernel(const float* __restrict__ x, long total_blocks,
                                                          int8_t* __restrict__ q, float* __restrict__ d) {
    const long blk = ((long)blockIdx.x * 256 + threadIdx.x) >> 5;
    const int i = threadIdx.x & 31;
    const bool ok = blk < total_blocks;
    const float v = ok ? x[blk * QK + i] : 0.0f;
    float a = __builtin_fabsf(v);
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1) a = __builtin_fmaxf(a, __shfl_xor(a, off, 64));
    const float scale = a / 127.0f;
    const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    if (ok) {
        q[blk * QK + i] = (int8_t)(int)round_half_away(v * inv);
        if (i == 0) d[blk] = scale;
    }
}

hipError_t launch_quantize_q8(const float* x, int n_tok, int n, int8_t* q, float* d, hipStream_t s) {
    const long total = (long)n_tok * (n / QK);
    const long threads = total * QK;
    const unsigned grid = (unsigned)((threads + 255) / 256);
    hipLaunchKernelGGL(quantize_q8_kernel, dim3(grid), dim3(256), 0, s, x, total, q, d);
    return hipGetLastError();
}

template <int DT, int U>
__global__ __launch_bounds__(256) void gemv_kernel(float* __restrict__ out, const uint8_t* __restrict__ wq,
                                                   const uint16_t* __restrict__ wscale,
                                                   const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                   int nb, int r0, int r1, int tile_rows, uint32_t nb_magic) {
    extern __shared__ float prod[];  // [tile_rows][nb + 1]
    constexpr int kChunksPerBlock = DT == kQ8 ? 2 : 1;
    constexpr int kBlockBytes = DT == kQ8 ? QK : QK / 2;
    const int pstride = nb + 1;
    const int ra = r0 + (int)blockIdx.x * tile_rows;
    const int nrows = min(tile_rows, r1 - ra);
    const int nchunks = nrows * nb * kChunksPerBlock;
    const uint8_t* base = wq + (size_t)ra * nb * kBlockBytes;
    const uint16_t* sbase = wscale + (size_t)ra * nb;

    for (int c0 = 0; c0 < nchunks; c0 += 256 * U) {
        uint4 w[U];
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const int c = c0 + j * 256 + (int)threadIdx.x;
            w[j] = c < nchunks ? load16(base + (size_t)c * 16) : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const int c = c0 + j * 256 + (int)threadIdx.x;
            const uint32_t g = (uint32_t)c / kChunksPerBlock;  // block index within the tile
            const uint32_t rt = nb == 1 ? g : div_magic(g, nb_magic);  // tile row
            const uint32_t b = g - rt * (uint32_t)nb;           // block within the row, always < nb
            if (DT == kQ8) {
                const uint4 xv = load16(xq + b * QK + (c & 1) * 16);
                int s = dot16_i8(w[j], xv);
                s += swap_pair(s);
                if (c < nchunks && !(c & 1)) prod[rt * pstride + b] = (float)s * f16_to_f32(sbase[g]);
            } else {
                const uint4 xlo = load16(xq + b * QK);
                const uint4 xhi = load16(xq + b * QK + 16);
                const int s = dot_q4_block(w[j], xlo, xhi);
                if (c < nchunks) prod[rt * pstride + b] = (float)s * f16_to_f32(sbase[g]);
            }
        }
    }
    __syncthreads();
    const int t = (int)threadIdx.x;
    if (t < nrows) {
        const float* p = prod + t * pstride;
        float acc = 0.0f;
        for (int b = 0; b < nb; ++b) acc = __builtin_fmaf(p[b], xd[b], acc);
        out[ra + t] = acc;
    }
}

namespace {

int round_unroll(int need) { return need <= 1 ? 1 : need <= 2 ? 2 : need <= 4 ? 4 : 8; }

bool env_plan(GemvPlan* p) {
    // QH_GEMV_PLAN="unroll:tile_rows" overrides the heuristic (tuning sweeps); read once.
    static const char* env = getenv("QH_GEMV_PLAN");
    if (!env) return false;
    int u = 0, t = 0;
    if (sscanf(env, "%d:%d", &u, &t) != 2) return false;
    p->unroll = round_unroll(u);
    p->tile_rows = t;
    return true;
}

}  // namespace

GemvPlan gemv_plan(int dtype, int cols, int rows) {
    const int nb = cols / QK;
    const int chunks_per_row = dtype == kQ8 ? 2 * nb : nb;
    const int lds_rows = 16384 / (nb + 1);  // prod tile <= 64 KB
    GemvPlan p;
    if (!env_plan(&p)) {
        // Aim for about two workgroups per CU on the 256-CU part; short rows get several per tile.
        int t = (rows + 511) / 512;
        p.tile_rows = t;
        p.unroll = round_unroll((t * chunks_per_row + 255) / 256);
    }
    p.tile_rows = p.tile_rows < 1 ? 1 : p.tile_rows;
    p.tile_rows = p.tile_rows > 256 ? 256 : p.tile_rows;
    p.tile_rows = p.tile_rows > lds_rows ? lds_rows : p.tile_rows;
    return p;
}

template <int DT, int U>
static void launch_gemv_t(float* out, const qh_tensor& W, const int8_t* xq, const float* xd, int r0, int r1,
                          int tile_rows, hipStream_t s) {
    const int nb = W.cols / QK;
    const uint8_t* wq = static_cast<const uint8_t*>(W.data);
    const uint16_t* ws = reinterpret_cast<const uint16_t*>(wq + qh_quant_bytes(W.dtype, W.rows, W.cols));
    const uint32_t magic = nb == 1 ? 0u : (uint32_t)((0x100000000ull + (uint64_t)nb - 1) / (uint64_t)nb);
    const unsigned grid = (unsigned)((r1 - r0 + tile_rows - 1) / tile_rows);
    const size_t lds = (size_t)tile_rows * (nb + 1) * sizeof(float);
    hipLaunchKernelGGL((gemv_kernel<DT, U>), dim3(grid), dim3(256), lds, s, out, wq, ws, xq, xd, nb, r0, r1,
                       tile_rows, magic);
}

hipError_t launch_gemv(float* out, const qh_tensor& W, const int8_t* xq, const float* xd, int r0, int r1,
                       const GemvPlan& plan, hipStream_t s) {
#define QH_GEMV_CASE(DT, U)                                                       \
    if (W.dtype == DT && plan.unroll == U) {                                      \
        launch_gemv_t<DT, U>(out, W, xq, xd, r0, r1, plan.tile_rows, s);          \
        return hipGetLastError();                                                 \
    }
    QH_GEMV_CASE(kQ8, 1) QH_GEMV_CASE(kQ8, 2) QH_GEMV_CASE(kQ8, 4) QH_GEMV_CASE(kQ8, 8)
    QH_GEMV_CASE(kQ4, 1) QH_GEMV_CASE(kQ4, 2) QH_GEMV_CASE(kQ4, 4) QH_GEMV_CASE(kQ4, 8)
#undef QH_GEMV_CASE
    return hipErrorInvalidValue;
}

// Greedy token: first index of the maximum (reference sampler.cpp:35-37). One 1024-thread workgroup.
__global__ __launch_bounds__(1024) void argmax_kernel(const float* __restrict__ logits, int n,
                                                      int32_t* __restrict__ index) {
    __shared__ uint64_t part[16];
    uint64_t best = 0;
    for (int i = (int)threadIdx.x; i < n; i += 1024) {
        const uint64_t k = score_key(logits[i], i);
        best = k > best ? k : best;
    }
    best = wave_max_u64(best);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t m = part[0];
        for (int w = 1; w < 16; ++w) m = part[w] > m ? part[w] : m;
        *index = key_row(m);
    }
}

hipError_t launch_argmax(const float* logits, int n, int32_t* index, hipStream_t s) {
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, s, logits, n, index);
    return hipGetLastError();
}

}  // namespace qh
