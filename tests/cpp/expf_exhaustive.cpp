// Compares qh::expf_variant<F> (quanta.cpp_amd/csrc/qh_math.h) with the host libm's expf on every one of the 2^32
// binary32 inputs, for F = 0, 1, 2. Prints the number of differing results per variant (NaN payloads compared as
// "both NaN") and the first few differences; exits 0 when the variant the decoder uses (QH_EXPF_FUSED) has none.
// Host C++ only: built with -ffp-contract=off so that only the explicit fma calls fuse.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <thread>
#include <vector>

#define QH_HD
#include "qh_math.h"

#ifndef QH_EXPF_FUSED
#define QH_EXPF_FUSED 2
#endif

namespace {

float from_bits(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
uint32_t to_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

}  // namespace

int main(int argc, char** argv) {
    const unsigned nt = std::thread::hardware_concurrency() ? std::thread::hardware_concurrency() : 8;
    // optional range [lo, hi) of input bit patterns (hex) for quick runs
    uint64_t lo = 0, hi = 1ull << 32;
    if (argc == 3) {
        lo = strtoull(argv[1], nullptr, 16);
        hi = strtoull(argv[2], nullptr, 16);
    }
    std::atomic<uint64_t> bad[3] = {{0}, {0}, {0}};
    std::vector<std::thread> th;
    std::atomic<int> shown{0};
    for (unsigned t = 0; t < nt; ++t)
        th.emplace_back([&, t] {
            uint64_t b0 = 0, b1 = 0, b2 = 0;
            const uint64_t a = lo + (hi - lo) * t / nt, e = lo + (hi - lo) * (t + 1) / nt;
            for (uint64_t u = a; u < e; ++u) {
                const float x = from_bits((uint32_t)u);
                const float want = expf(x);
                const float g[3] = {qh::expf_variant<0>(x), qh::expf_variant<1>(x), qh::expf_variant<2>(x)};
                for (int v = 0; v < 3; ++v) {
                    const bool same = (isnan(want) && isnan(g[v])) || to_bits(want) == to_bits(g[v]);
                    if (!same) {
                        (v == 0 ? b0 : v == 1 ? b1 : b2)++;
                        if (v == QH_EXPF_FUSED && shown.fetch_add(1) < 8)
                            printf("  differs: x=%a (0x%08x) libm=%a ours=%a\n", x, (unsigned)u, want, g[v]);
                    }
                }
            }
            bad[0] += b0;
            bad[1] += b1;
            bad[2] += b2;
        });
    for (auto& x : th) x.join();
    for (int v = 0; v < 3; ++v)
        printf("expf variant %d (fused=%d): %llu of %llu inputs differ from libm\n", v, v,
               (unsigned long long)bad[v].load(), (unsigned long long)(hi - lo));
    return bad[QH_EXPF_FUSED] == 0 ? 0 : 1;
}
