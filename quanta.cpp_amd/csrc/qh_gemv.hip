// Decode-side kernels: activation quantization (reference ops_ref.cpp:69-83) and the Q8_0 / Q4_0
// integer-dot GEMV (reference ops_ref.cpp:85-120), for gfx950.
//
// GEMV data flow: a workgroup owns a tile of consecutive rows (qh_gemv.h: coalesced 16-byte loads of the
// tile's contiguous bytes, exact int32 block dots, one rounded product per block parked in LDS, then one serial
// FMA chain per row in the reference's order). Small matrices use one tile per workgroup; vocabulary-sized
// ones use the persistent streaming kernel below.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "qh_device.h"
#include "qh_gemv.h"
#include "qh_internal.h"

namespace qh {

// One wave quantizes two 32-blocks (one per half-wave, one element per lane).
__global__ __launch_bounds__(256) void quantize_q8_kernel(const float* __restrict__ x, long total_blocks,
                                                          int8_t* __restrict__ q, float* __restrict__ d) {
    const long blk = ((long)blockIdx.x * 256 + threadIdx.x) >> 5;
    const int i = threadIdx.x & 31;
    const bool ok = blk < total_blocks;
    const float v = ok ? x[blk * QK + i] : 0.0f;
    const float a = max32_lanes(__builtin_fabsf(v));  // every lane takes part (v = 0 past the end)
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
    qh_launch(quantize_q8_kernel, dim3(grid), dim3(256), 0, s, x, total, q, d);
    return hipGetLastError();
}

// XL = false: activation read with the weights (best for small, latency-bound matrices).
// XL = true: activation staged once in LDS (best for large matrices, where per-chunk activation loads
// would compete with the weight stream).
template <int DT, int U, bool XL>
__global__ __launch_bounds__(256) void gemv_kernel(float* __restrict__ out, const uint8_t* __restrict__ wq,
                                                   const uint16_t* __restrict__ wscale,
                                                   const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                   int nb, int r0, int r1, int tile_rows, uint32_t nb_magic) {
    extern __shared__ __align__(16) float smem[];
    const int ra = r0 + (int)blockIdx.x * tile_rows;
    const int nrows = min(tile_rows, r1 - ra);
    const float v = gemv_tile<DT, U, XL>(wq, wscale, xq, xd, nb, ra, nrows, tile_rows, nb_magic, smem);
    if ((int)threadIdx.x < nrows) out[ra + threadIdx.x] = v;
}

// Streaming GEMV for large matrices (vocabulary-sized heads). The grid is persistent: workgroup g walks the
// contiguous run of row tiles [g*nt/G, (g+1)*nt/G), so each workgroup streams one long byte range. Two register
// sets alternate: the 16-byte chunks (and block scales) of tile t+1 are in flight while tile t's block products
// and row chains are computed. The activation codes and scales are staged in LDS once per launch. Products go to
// one of two LDS buffers, so one barrier per tile suffices: the chain of tile t-1 (same buffer as t+1) finishes
// before any thread passes the barrier of tile t.
template <int DT, int U>
struct StreamRegs {
    uint4 w[U];
    uint16_t sc[U];

    // Loads the chunks of the tile starting at `base` (nchunks valid, later slots clamped onto the last one).
    __device__ __forceinline__ void load(const uint8_t* __restrict__ base, const uint16_t* __restrict__ sbase,
                                         int nchunks) {
        constexpr int kChunksPerBlock = DT == kQ8 ? 2 : 1;
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const int c = min(j * 256 + (int)threadIdx.x, nchunks - 1);
            w[j] = load16(base + (size_t)c * 16);
            sc[j] = sbase[c / kChunksPerBlock];
        }
    }

    __device__ __forceinline__ void products(float* prod, int pstride, int nchunks, int nb, uint32_t nb_magic,
                                             const int8_t* xs) const {
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const int c = j * 256 + (int)threadIdx.x;
            const int cc = min(c, nchunks - 1);
            if constexpr (DT == kQ8) {
                const uint32_t g = (uint32_t)cc >> 1;
                const uint32_t rt = nb == 1 ? g : div_magic(g, nb_magic);
                const uint32_t b = g - rt * (uint32_t)nb;
                const uint4 xv = *reinterpret_cast<const uint4*>(xs + b * QK + (cc & 1) * 16);
                int s = dot16_i8(w[j], xv);
                s += swap_pair(s);
                if (c < nchunks && !(c & 1)) prod[rt * pstride + b] = (float)s * f16_to_f32(sc[j]);
            } else {
                const uint32_t g = (uint32_t)cc;
                const uint32_t rt = nb == 1 ? g : div_magic(g, nb_magic);
                const uint32_t b = g - rt * (uint32_t)nb;
                const uint4 xlo = *reinterpret_cast<const uint4*>(xs + b * QK);
                const uint4 xhi = *reinterpret_cast<const uint4*>(xs + b * QK + 16);
                const int s = dot_q4_block(w[j], xlo, xhi);
                if (c < nchunks) prod[rt * pstride + b] = (float)s * f16_to_f32(sc[j]);
            }
        }
    }
};

template <int DT, int U>
__global__ __launch_bounds__(256) void gemv_stream_kernel(float* __restrict__ out, const uint8_t* __restrict__ wq,
                                                          const uint16_t* __restrict__ wscale,
                                                          const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                          int nb, int r0, int r1, int tile_rows, uint32_t nb_magic) {
    extern __shared__ __align__(16) float smem[];
    constexpr int kChunksPerBlock = DT == kQ8 ? 2 : 1;
    constexpr int kBlockBytes = DT == kQ8 ? QK : QK / 2;
    const int cols = nb * QK;
    const int L = chain_len32(nb), zp = L - nb, pstride = chain_stride32(nb);
    float* dxs = smem;                                          // [L] padded chain row (zp zeros first)
    float* xds = dxs + zp;
    float* prod0 = smem + L;                                    // [tile_rows][pstride] padded chain rows
    float* prod1 = prod0 + (size_t)tile_rows * pstride;
    int8_t* xs = reinterpret_cast<int8_t*>(prod1 + (size_t)tile_rows * pstride + kChainPipePad);  // [cols]
    const int tid = (int)threadIdx.x;
    // Rows [ra, rb) of this workgroup: an even split, so no workgroup carries more than one extra partial tile.
    const int n = r1 - r0;
    const int ra = r0 + (int)((long)blockIdx.x * n / gridDim.x);
    const int rb = r0 + (int)((long)(blockIdx.x + 1) * n / gridDim.x);
    if (ra >= rb) return;  // uniform per workgroup; nothing below synchronises across workgroups

    const size_t row_bytes = (size_t)nb * kBlockBytes;
    auto chunks_of = [&](int r) { return min(tile_rows, rb - r) * nb * kChunksPerBlock; };

    StreamRegs<DT, U> A, B;
    A.load(wq + (size_t)ra * row_bytes, wscale + (size_t)ra * nb, chunks_of(ra));
    for (int i = tid; i < cols / 16; i += 256) reinterpret_cast<uint4*>(xs)[i] = load16(xq + i * 16);
    for (int i = tid; i < nb; i += 256) xds[i] = xd[i];
    zero_chain_prefix(dxs, prod0, nb, 2 * tile_rows);  // both product buffers (contiguous)
    __syncthreads();

    // One tile: block products into `prod`, then one barrier, then one chain thread per row.
    auto tile_body = [&](const StreamRegs<DT, U>& regs, int r, float* prod) {
        const int nrows = min(tile_rows, rb - r);
        regs.products(prod + zp, pstride, nrows * nb * kChunksPerBlock, nb, nb_magic, xs);
        __syncthreads();
        if (tid < nrows) out[r + tid] = chain_lds_pipe(prod + tid * pstride, dxs, L);
    };
    // Loads in the steady-state loop are unconditional (a conditional load makes the compiler's wait counting
    // assume the worst at the join); the last one or two tiles are peeled.
    const int n_tiles = (rb - ra + tile_rows - 1) / tile_rows;
    int t = 0;
    while (t + 2 < n_tiles) {
        const int r = ra + t * tile_rows;
        B.load(wq + (size_t)(r + tile_rows) * row_bytes, wscale + (size_t)(r + tile_rows) * nb, chunks_of(r + tile_rows));
        tile_body(A, r, prod0);
        A.load(wq + (size_t)(r + 2 * tile_rows) * row_bytes, wscale + (size_t)(r + 2 * tile_rows) * nb,
               chunks_of(r + 2 * tile_rows));
        tile_body(B, r + tile_rows, prod1);
        t += 2;
    }
    const int r = ra + t * tile_rows;
    if (t + 1 < n_tiles) {
        B.load(wq + (size_t)(r + tile_rows) * row_bytes, wscale + (size_t)(r + tile_rows) * nb, chunks_of(r + tile_rows));
        tile_body(A, r, prod0);
        tile_body(B, r + tile_rows, prod1);
    } else {
        tile_body(A, r, prod0);
    }
}

namespace {

int round_unroll(int need) { return need <= 1 ? 1 : need <= 2 ? 2 : need <= 4 ? 4 : 8; }

bool env_plan(GemvPlan* p) {
    // Tuning sweeps override the heuristic with QH_GEMV_PLAN:
    //   "unroll:tile_rows[:lds]"      one-pass tile kernel
    //   "s:unroll:wg_per_cu"          streaming kernel (tile_rows derived from unroll)
    const char* env = getenv("QH_GEMV_PLAN");
    if (!env) return false;
    int u = 0, t = 0;
    if (sscanf(env, "s:%d:%d", &u, &t) == 2) {
        p->stream = true;
        p->unroll = round_unroll(u);
        p->grid = t * device_cus();
        p->act_lds = true;
        return true;
    }
    if (sscanf(env, "%d:%d", &u, &t) != 2) return false;
    p->stream = false;
    p->unroll = round_unroll(u);
    p->tile_rows = t;
    p->act_lds = strstr(env, ":lds") != nullptr;
    return true;
}

}  // namespace

int device_cus() {
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int n = 0;
        cus[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
    }
    return cus[dev];
}

size_t gemv_lds_bytes(int cols, int tile_rows, bool xl) { return gemv_tile_lds_bytes(cols, tile_rows, xl); }

static size_t gemv_stream_lds_bytes(int cols, int tile_rows) {
    const int nb = cols / QK;
    return ((size_t)chain_len32(nb) + 2 * (size_t)tile_rows * chain_stride32(nb) + kChainPipePad) * 4 + (size_t)cols;
}

GemvPlan gemv_plan(int dtype, int cols, int rows) {
    const int nb = cols / QK;
    const int cpr = dtype == kQ8 ? 2 * nb : nb;  // 16-byte chunks per row
    const int lds_rows = (65536 - cols - 4 * (chain_len32(nb) + kChainPipePad)) / (chain_stride32(nb) * 4);  // 64 KB
    GemvPlan p;
    p.stream = false;
    p.grid = 0;
    if (!env_plan(&p)) {
        // Measured on MI355X (cold HBM, graph-replayed): small matrices are latency-bound and do best with
        // about one 16-byte load per thread per workgroup (4 Q8 / 8 Q4 rows of 896); rows of 4864 as below.
        // Matrices of several MB and up go to the streaming kernel, which keeps two tiles per workgroup in
        // flight with a persistent grid of two workgroups per CU.
        const long chunks = (long)rows * cpr;
        if (chunks >= 512L * 1024) {
            p.stream = true;
            p.unroll = 8;
            p.grid = 2 * device_cus();
            p.act_lds = true;
        } else {
            // Rows longer than 256 chunks (4,864 columns) take 4 per workgroup where that is at most 8 chunks per
            // thread: half the workgroups of 2-row tiles, so a shorter dispatch ramp, while the rows' chains still
            // run side by side (Q4_0 896x4864 3.17 -> 2.91 us, Q8_0 3.53 -> 3.42 us cold).
            int t = 256 / cpr;
            if (t < 1) t = 1;
            if (t == 1) t = 4 * cpr <= 8 * 256 ? 4 : cpr < 512 ? 2 : 1;
            // Over 512 such tiles, twice the rows per workgroup (two loads per thread): Q4_0 4864x896 2.68 -> 2.63
            // us, Q8_0 2.95 -> 2.84 us cold; at 896 rows the one-load tiles stay ahead.
            else if ((rows + t - 1) / t > 512 && 2 * t * cpr <= 512) t *= 2;
            p.tile_rows = t;
            p.unroll = round_unroll((t * cpr + 255) / 256);
            p.act_lds = false;
        }
    }
    if (p.stream) {
        // Rows per tile: as many whole rows as unroll * 256 chunk slots hold, within 64 KB of LDS.
        int t = p.unroll * 256 / cpr;
        const int lds_stream_rows = (65536 - cols - 4 * (chain_len32(nb) + kChainPipePad)) / (2 * chain_stride32(nb) * 4);
        t = t < 1 ? 1 : t;
        t = t > 256 ? 256 : t;  // one chain thread per row
        t = t > lds_stream_rows ? lds_stream_rows : t;
        p.tile_rows = t;
        if (p.tile_rows * cpr > p.unroll * 256) p.stream = false;  // row longer than the register tile
        else return p;
        p.unroll = round_unroll((cpr + 255) / 256);
        p.tile_rows = 1;
        p.act_lds = true;
    }
    p.tile_rows = p.tile_rows < 1 ? 1 : p.tile_rows;
    p.tile_rows = p.tile_rows > 256 ? 256 : p.tile_rows;
    p.tile_rows = p.tile_rows > lds_rows ? lds_rows : p.tile_rows;
    return p;
}

template <int DT, int U, bool XL>
static void launch_gemv_t(float* out, const qh_tensor& W, const int8_t* xq, const float* xd, int r0, int r1,
                          int tile_rows, hipStream_t s) {
    const int nb = W.cols / QK;
    const uint8_t* wq = static_cast<const uint8_t*>(W.data);
    const uint16_t* ws = reinterpret_cast<const uint16_t*>(wq + qh_quant_bytes(W.dtype, W.rows, W.cols));
    const uint32_t magic = nb == 1 ? 0u : (uint32_t)((0x100000000ull + (uint64_t)nb - 1) / (uint64_t)nb);
    const unsigned grid = (unsigned)((r1 - r0 + tile_rows - 1) / tile_rows);
    const size_t lds = gemv_lds_bytes(W.cols, tile_rows, XL);
    qh_launch((gemv_kernel<DT, U, XL>), dim3(grid), dim3(256), lds, s, out, wq, ws, xq, xd, nb, r0, r1,
                       tile_rows, magic);
}

template <int DT, int U>
static void launch_gemv_stream_t(float* out, const qh_tensor& W, const int8_t* xq, const float* xd, int r0, int r1,
                                 int tile_rows, int grid, hipStream_t s) {
    const int nb = W.cols / QK;
    const uint8_t* wq = static_cast<const uint8_t*>(W.data);
    const uint16_t* ws = reinterpret_cast<const uint16_t*>(wq + qh_quant_bytes(W.dtype, W.rows, W.cols));
    const uint32_t magic = nb == 1 ? 0u : (uint32_t)((0x100000000ull + (uint64_t)nb - 1) / (uint64_t)nb);
    const int n = r1 - r0;
    const int n_tiles = (n + tile_rows - 1) / tile_rows;
    const int g = grid < n_tiles ? grid : n_tiles;
    // Even tiles within a workgroup's share: the fewest tiles of at most tile_rows rows, all the same size.
    const int per = (n + g - 1) / g;
    const int k = (per + tile_rows - 1) / tile_rows;
    tile_rows = (per + k - 1) / k;
    const size_t lds = gemv_stream_lds_bytes(W.cols, tile_rows);
    qh_launch((gemv_stream_kernel<DT, U>), dim3((unsigned)g), dim3(256), lds, s, out, wq, ws, xq, xd, nb, r0,
                       r1, tile_rows, magic);
}

hipError_t launch_gemv(float* out, const qh_tensor& W, const int8_t* xq, const float* xd, int r0, int r1,
                       const GemvPlan& plan, hipStream_t s) {
#define QH_GEMV_CASE(DT, U)                                                               \
    if (W.dtype == DT && plan.unroll == U) {                                              \
        if (plan.stream) {                                                                \
            launch_gemv_stream_t<DT, U>(out, W, xq, xd, r0, r1, plan.tile_rows, plan.grid, s); \
            return hipGetLastError();                                                     \
        }                                                                                 \
        if (plan.act_lds)                                                                 \
            launch_gemv_t<DT, U, true>(out, W, xq, xd, r0, r1, plan.tile_rows, s);        \
        else                                                                              \
            launch_gemv_t<DT, U, false>(out, W, xq, xd, r0, r1, plan.tile_rows, s);       \
        return hipGetLastError();                                                         \
    }
    QH_GEMV_CASE(kQ8, 1) QH_GEMV_CASE(kQ8, 2) QH_GEMV_CASE(kQ8, 4) QH_GEMV_CASE(kQ8, 8)
    QH_GEMV_CASE(kQ4, 1) QH_GEMV_CASE(kQ4, 2) QH_GEMV_CASE(kQ4, 4) QH_GEMV_CASE(kQ4, 8)
#undef QH_GEMV_CASE
    return hipErrorInvalidValue;
}

// Greedy token: first index of the maximum (reference sampler.cpp:35-37), in two launches. Each workgroup folds
// a contiguous slice into one 64-bit key (ordered score bits, then the complement of the index, so equal scores
// prefer the lower index); one workgroup then folds the partial keys and writes the index.
constexpr int kArgmaxThreads = 256;
constexpr int kArgmaxPerThread = 8;
constexpr int kArgmaxMaxParts = 1024;

int argmax_parts(int n) {
    const int p = (n + kArgmaxThreads * kArgmaxPerThread - 1) / (kArgmaxThreads * kArgmaxPerThread);
    return p < kArgmaxMaxParts ? p : kArgmaxMaxParts;
}

size_t argmax_workspace_bytes(int n) { return ((size_t)argmax_parts(n) * 8 + 255) & ~size_t(255); }

__global__ __launch_bounds__(kArgmaxThreads) void argmax_part_kernel(const float* __restrict__ logits, int n,
                                                                     uint64_t* __restrict__ part) {
    __shared__ uint64_t wbest[kArgmaxThreads / 64];
    const int a = (int)((long)blockIdx.x * n / gridDim.x), b = (int)((long)(blockIdx.x + 1) * n / gridDim.x);
    uint64_t best = 0;
    for (int i0 = a; i0 < b; i0 += kArgmaxThreads * kArgmaxPerThread) {
        float v[kArgmaxPerThread];
#pragma unroll
        for (int j = 0; j < kArgmaxPerThread; ++j) {
            const int i = i0 + j * kArgmaxThreads + (int)threadIdx.x;
            v[j] = logits[min(i, b - 1)];
        }
#pragma unroll
        for (int j = 0; j < kArgmaxPerThread; ++j) {
            const int i = i0 + j * kArgmaxThreads + (int)threadIdx.x;
            const uint64_t k = i < b ? score_key(v[j], i) : 0ull;
            best = k > best ? k : best;
        }
    }
    best = wave_max_u64(best);
    if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t m = wbest[0];
        for (int w = 1; w < kArgmaxThreads / 64; ++w) m = wbest[w] > m ? wbest[w] : m;
        part[blockIdx.x] = m;
    }
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_final_kernel(const uint64_t* __restrict__ part, int n_parts,
                                                                      int32_t* __restrict__ index) {
    __shared__ uint64_t wbest[kArgmaxThreads / 64];
    uint64_t best = 0;
    for (int i = (int)threadIdx.x; i < n_parts; i += kArgmaxThreads) best = part[i] > best ? part[i] : best;
    best = wave_max_u64(best);
    if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t m = wbest[0];
        for (int w = 1; w < kArgmaxThreads / 64; ++w) m = wbest[w] > m ? wbest[w] : m;
        *index = key_row(m);
    }
}

// ------------------------------------------------------------------------- unquantized weights (F32 / F16)
// matvec_ref (ops_ref.cpp:8-27) for n tokens: out[t * ldo + r] = acc with acc = fma(w_ri, x_ti, acc) from +0 in column
// order (the reference build contracts acc += w * x into one multiply-add; an F16 weight converts exactly). Every
// (row, token) chain is serial, so a workgroup owns 64 rows x 4 tokens: each 64-column tile of the rows (coalesced
// 16-byte loads, F16 widened to f32 as it is staged) and of the 4 tokens' activations is staged in LDS, the next
// tile's loads in flight while this one is used, and wave w runs the 64 chains of token 4 blockIdx.y + w, lane r on
// row r (LDS rows padded to 65 floats: the lanes' reads of one column fall in 64 different banks; the activation
// value is a broadcast). An option off the benchmark's path (the quantized GEMVs are its hot path): written for the
// exact order first; the serial chain of a row (cols FMAs) bounds it.
constexpr int kDenseT = 64, kDenseStride = kDenseT + 1;
template <int DT>
__global__ __launch_bounds__(256) void gemv_dense_kernel(const uint8_t* __restrict__ W, int cols, int r0, int r1,
                                                         const float* __restrict__ x, int ldx, int n,
                                                         float* __restrict__ out, int ldo) {
    __shared__ float ws[2][64 * kDenseStride];
    __shared__ __align__(16) float xs[2][4 * kDenseT];
    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int rbase = r0 + (int)blockIdx.x * 64;
    const int t = (int)blockIdx.y * 4 + wave;
    const int ntiles = (cols + kDenseT - 1) / kDenseT;
    // 16-byte units u = 256 j + tid of the 64 x 64 tile: F32 four per thread (row u / 16, columns 4 (u % 16) ..), F16
    // two (row u / 8, columns 8 (u % 8) ..). Rows past r1 and columns past cols are clamped (loaded, never used).
    constexpr int kUnits = DT == kF32 ? 4 : 2;
    uint4 wr[kUnits];
    float4 xr = make_float4(0.f, 0.f, 0.f, 0.f);
    auto load = [&](int tile) {
        const int c0 = tile * kDenseT;
#pragma unroll
        for (int j = 0; j < kUnits; ++j) {
            const int u = 256 * j + tid;
            const int row = min(rbase + (DT == kF32 ? u / 16 : u / 8), r1 - 1);
            if (DT == kF32) {
                const int c = min(c0 + 4 * (u % 16), cols - 4);
                wr[j] = *reinterpret_cast<const uint4*>(W + ((size_t)row * cols + c) * 4);
            } else {
                const int c = min(c0 + 8 * (u % 8), cols - 8);
                wr[j] = *reinterpret_cast<const uint4*>(W + ((size_t)row * cols + c) * 2);
            }
        }
        if (tid < 64) {
            const int tt = min((int)blockIdx.y * 4 + tid / 16, n - 1);
            const int c = min(c0 + 4 * (tid % 16), cols - 4);
            xr = *reinterpret_cast<const float4*>(x + (size_t)tt * ldx + c);
        }
    };
    auto stage = [&](int buf) {
#pragma unroll
        for (int j = 0; j < kUnits; ++j) {
            const int u = 256 * j + tid;
            if (DT == kF32) {
                float* d = &ws[buf][(u / 16) * kDenseStride + 4 * (u % 16)];
                d[0] = __uint_as_float(wr[j].x);
                d[1] = __uint_as_float(wr[j].y);
                d[2] = __uint_as_float(wr[j].z);
                d[3] = __uint_as_float(wr[j].w);
            } else {
                float* d = &ws[buf][(u / 8) * kDenseStride + 8 * (u % 8)];
                const uint32_t h[4] = {wr[j].x, wr[j].y, wr[j].z, wr[j].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    d[2 * e] = f16_to_f32((uint16_t)(h[e] & 0xffffu));
                    d[2 * e + 1] = f16_to_f32((uint16_t)(h[e] >> 16));
                }
            }
        }
        if (tid < 64) reinterpret_cast<float4*>(&xs[buf][(tid / 16) * kDenseT])[tid % 16] = xr;
    };
    float acc = 0.0f;
    const bool run = t < n && rbase + lane < r1;
    load(0);
    stage(0);
    __syncthreads();
    for (int tile = 0; tile < ntiles; ++tile) {
        const int buf = tile & 1;
        if (tile + 1 < ntiles) load(tile + 1);
        if (run) {
            const float* wrow = &ws[buf][lane * kDenseStride];
            const float* xt = &xs[buf][wave * kDenseT];
            const int cnt = min(kDenseT, cols - tile * kDenseT);  // 64, or 32 for the last tile (cols % 32 == 0)
            if (cnt == kDenseT) {
#pragma unroll
                for (int c = 0; c < kDenseT; ++c) acc = __builtin_fmaf(wrow[c], xt[c], acc);
            } else {
#pragma unroll
                for (int c = 0; c < kDenseT / 2; ++c) acc = __builtin_fmaf(wrow[c], xt[c], acc);
            }
        }
        if (tile + 1 < ntiles) stage(buf ^ 1);
        __syncthreads();
    }
    if (run) out[(size_t)t * ldo + rbase + lane] = acc;
}

hipError_t launch_gemv_dense(float* out, int ldo, const qh_tensor& W, const float* x, int ldx, int n, int r0, int r1,
                             hipStream_t s) {
    const dim3 grid((unsigned)((r1 - r0 + 63) / 64), (unsigned)((n + 3) / 4));
    const uint8_t* w = static_cast<const uint8_t*>(W.data);
    if (W.dtype == kF32)
        qh_launch(gemv_dense_kernel<kF32>, grid, dim3(256), 0, s, w, W.cols, r0, r1, x, ldx, n, out, ldo);
    else if (W.dtype == kF16)
        qh_launch(gemv_dense_kernel<kF16>, grid, dim3(256), 0, s, w, W.cols, r0, r1, x, ldx, n, out, ldo);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_argmax(const float* logits, int n, int32_t* index, void* ws, hipStream_t s) {
    const int parts = argmax_parts(n);
    uint64_t* part = static_cast<uint64_t*>(ws);
    qh_launch(argmax_part_kernel, dim3((unsigned)parts), dim3(kArgmaxThreads), 0, s, logits, n, part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    qh_launch(argmax_final_kernel, dim3(1), dim3(kArgmaxThreads), 0, s, part, parts, index);
    return hipGetLastError();
}

}  // namespace qh
