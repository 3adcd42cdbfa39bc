// Evaluates qh::expf_variant<2> (quanta.cpp_amd/csrc/qh_math.h) on the GPU for every one of the 2^32 binary32 inputs
// and compares each result with the same function evaluated on the host, which tests/cpp/expf_exhaustive.cpp checks
// against the host libm. The decoder's softmax and SwiGLU call this function on the device, so together the two
// programs show the device exp equals glibc's expf everywhere. Exits 0 when no input differs (NaNs compared as
// "both NaN"). Built with hipcc for gfx950 by tests/cpp/Makefile.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <thread>
#include <vector>

#include "qh_math.h"

namespace {

constexpr uint64_t kChunk = 1ull << 26;

__global__ void eval_chunk(uint64_t base, uint32_t* out) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;  // the grid covers exactly kChunk inputs
    const uint32_t u = (uint32_t)(base + i);
    float x;
    memcpy(&x, &u, 4);
    const float y = qh::expf_variant<2>(x);
    uint32_t r;
    memcpy(&r, &y, 4);
    out[i] = r;
}

}  // namespace

int main() {
    uint32_t* dev = nullptr;
    if (hipMalloc(&dev, kChunk * 4) != hipSuccess) {
        fprintf(stderr, "hipMalloc failed\n");
        return 2;
    }
    std::vector<uint32_t> host(kChunk);
    const unsigned nt = std::thread::hardware_concurrency() ? (std::thread::hardware_concurrency() > 16 ? 16 : std::thread::hardware_concurrency()) : 8;
    uint64_t bad = 0;
    std::atomic<int> shown{0};
    for (uint64_t base = 0; base < (1ull << 32); base += kChunk) {
        hipLaunchKernelGGL(eval_chunk, dim3((unsigned)(kChunk / 256)), dim3(256), 0, 0, base, dev);
        if (hipMemcpy(host.data(), dev, kChunk * 4, hipMemcpyDeviceToHost) != hipSuccess) {
            fprintf(stderr, "hipMemcpy failed\n");
            return 2;
        }
        std::atomic<uint64_t> b{0};
        std::vector<std::thread> th;
        for (unsigned t = 0; t < nt; ++t)
            th.emplace_back([&, t] {
                uint64_t lb = 0;
                for (uint64_t i = kChunk * t / nt; i < kChunk * (t + 1) / nt; ++i) {
                    const uint32_t u = (uint32_t)(base + i);
                    float x;
                    memcpy(&x, &u, 4);
                    const float y = qh::expf_variant<2>(x);
                    uint32_t r;
                    memcpy(&r, &y, 4);
                    const bool dev_nan = (host[i] & 0x7f800000u) == 0x7f800000u && (host[i] & 0x7fffffu);
                    if (r != host[i] && !(y != y && dev_nan)) {
                        ++lb;
                        if (shown.fetch_add(1) < 8) printf("  x=0x%08x host 0x%08x device 0x%08x\n", u, r, host[i]);
                    }
                }
                b += lb;
            });
        for (auto& x : th) x.join();
        bad += b;
        if ((base & ((1ull << 30) - 1)) == 0) {
            printf("inputs from 0x%08llx checked\n", (unsigned long long)base);
            fflush(stdout);
        }
    }
    printf("device expf_variant<2>: %llu of 4294967296 inputs differ from the host\n", (unsigned long long)bad);
    (void)hipFree(dev);
    return bad == 0 ? 0 : 1;
}
