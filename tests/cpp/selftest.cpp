// Model-free kernel self-test of the drop-in C++ surface (quanta_ops.h), in the shape of the reference's
// kernel_selftest (engine/src/checks.cpp:64-146): the same xorshift64 fixture recipe (seed
// 0x9E3779B97F4A7C15, random quant bytes including -128, fp16 scales 0x2000 + r % 0x800, activations
// (r % 2001 - 1000) / 1000) on one 4864 x 896 MLP matrix per dtype. It checks, for Q8_0 and Q4_0:
//   * quantize_q8 on the GPU equals the oracle's restatement byte for byte;
//   * every available kernel's matvec equals the oracle bit for bit, and passes the reference's own
//     criterion max|diff| / max|want| < 1e-4;
//   * matmul for n = 32 and a ragged n = 7 equals looped matvec of the same family, bit for bit;
//   * the engine's threading pattern (parallel_for over rows, grain 16, concurrent calls) gives the same rows.
// Prints one line per check and exits 0 only if all pass. Timings include the PCIe round trip of the
// host-pointer surface.
#include <chrono>
#include <cmath>
#include <cstdio>
#include <thread>
#include <vector>

#include "quanta_ops.h"
#include "quanta_oracle.h"

using namespace quanta;

namespace {

using Clock = std::chrono::steady_clock;

struct XorShift {
    uint64_t s = 0x9E3779B97F4A7C15ULL;
    uint64_t operator()() {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        return s;
    }
};

bool same_bits(const float* a, const float* b, size_t n) { return std::memcmp(a, b, n * sizeof(float)) == 0; }

}  // namespace

int main() {
    XorShift next;
    bool ok = true;
    for (DType dt : {DType::Q8_0, DType::Q4_0}) {
        const char* name = dt == DType::Q8_0 ? "q8_0" : "q4_0";
        const int rows = 4864, cols = 896, nb = cols / QK;
        const size_t qbytes = dt == DType::Q8_0 ? size_t(rows) * cols : size_t(rows) * cols / 2;
        std::vector<uint8_t> buf(qbytes + size_t(rows) * nb * 2);
        for (size_t i = 0; i < qbytes; ++i) buf[i] = uint8_t(next());
        uint16_t* scales = reinterpret_cast<uint16_t*>(buf.data() + qbytes);
        for (int i = 0; i < rows * nb; ++i) scales[i] = uint16_t(0x2000 + next() % 0x800);
        Tensor W;
        W.dtype = dt;
        W.rows = rows;
        W.cols = cols;
        W.data = buf.data();

        std::vector<float> x(cols);
        for (float& v : x) v = float(int(next() % 2001) - 1000) / 1000.f;
        QuantVec xq;
        quantize_q8(x.data(), cols, xq);
        std::vector<int8_t> oq(cols);
        std::vector<float> od(nb);
        qo_quantize_q8(x.data(), cols, oq.data(), od.data());
        const bool qok = std::memcmp(oq.data(), xq.q.data(), cols) == 0 && same_bits(od.data(), xq.d.data(), nb);
        ok &= qok;
        std::printf("%-5s quantize_q8 vs oracle: %s\n", name, qok ? "PASS" : "FAIL");

        std::vector<float> want(rows), got(rows);
        qo_matvec_q(want.data(), int(dt), rows, cols, buf.data(), oq.data(), od.data(), 0, rows);
        for (const auto& [kname, fn] : available_matvec_q_kernels()) {
            fn(got.data(), W, xq, 0, rows);
            double max_abs = 0, scale = 0;
            for (int r = 0; r < rows; ++r) {
                max_abs = std::max(max_abs, std::fabs(double(got[r]) - want[r]));
                scale = std::max(scale, std::fabs(double(want[r])));
            }
            const bool exact = same_bits(got.data(), want.data(), rows);
            const bool pass = exact && max_abs / scale < 1e-4;
            ok &= pass;
            const int iters = 50;
            const auto t0 = Clock::now();
            for (int i = 0; i < iters; ++i) fn(got.data(), W, xq, 0, rows);
            const double sec = std::chrono::duration<double>(Clock::now() - t0).count() / iters;
            std::printf("%-5s %-4s matvec bit-exact vs oracle %s, max err %.2e of output scale  %8.1f us  %7.2f GB/s "
                        "(host pointers, PCIe included)\n",
                        name, kname, pass ? "PASS" : "FAIL", max_abs / scale, sec * 1e6, double(buf.size()) / sec / 1e9);
        }

        // Engine threading pattern: ThreadPool::parallel_for(rows, 16) issues concurrent calls on disjoint ranges.
        {
            std::vector<float> par(rows, -1.f);
            const int nt = 8, grain = 16, chunks = (rows + grain - 1) / grain;
            std::vector<std::thread> th;
            for (int t = 0; t < nt; ++t)
                th.emplace_back([&, t] {
                    const int c0 = int(int64_t(chunks) * t / nt), c1 = int(int64_t(chunks) * (t + 1) / nt);
                    const int r0 = c0 * grain, r1 = std::min(rows, c1 * grain);
                    if (r0 < r1) matvec_q(par.data(), W, xq, r0, r1);
                });
            for (auto& t : th) t.join();
            const bool pok = same_bits(par.data(), want.data(), rows);
            ok &= pok;
            std::printf("%-5s hip  matvec from 8 threads on disjoint row ranges: %s\n", name, pok ? "PASS" : "FAIL");
        }

        const int n = 32;
        std::vector<QuantVec> xs(n);
        for (auto& v : xs) {
            for (float& f : x) f = float(int(next() % 2001) - 1000) / 1000.f;
            quantize_q8(x.data(), cols, v);
        }
        const auto mvs = available_matvec_q_kernels();
        const auto mms = available_matmul_q_kernels();
        std::vector<float> want_mm(size_t(n) * rows), got_mm(size_t(n) * rows);
        for (size_t k = 0; k < mms.size(); ++k) {
            for (int t = 0; t < n; ++t) mvs[k].second(want_mm.data() + size_t(t) * rows, W, xs[t], 0, rows);
            bool exact = true;
            for (int n_try : {n, 7}) {
                std::fill(got_mm.begin(), got_mm.end(), 0.f);
                mms[k].second(got_mm.data(), rows, W, xs.data(), n_try, 0, rows);
                exact &= same_bits(got_mm.data(), want_mm.data(), size_t(n_try) * rows);
            }
            ok &= exact;
            const int iters = 5;
            auto t0 = Clock::now();
            for (int i = 0; i < iters; ++i) mms[k].second(got_mm.data(), rows, W, xs.data(), n, 0, rows);
            const double mm_sec = std::chrono::duration<double>(Clock::now() - t0).count() / iters;
            t0 = Clock::now();
            for (int i = 0; i < iters; ++i)
                for (int t = 0; t < n; ++t) mvs[k].second(got_mm.data() + size_t(t) * rows, W, xs[t], 0, rows);
            const double mv_sec = std::chrono::duration<double>(Clock::now() - t0).count() / iters;
            std::printf("%-5s %-4s matmul x%d (and x7): bit-exact vs looped matvec %s  %7.2f ms vs %7.2f ms looped\n",
                        name, mms[k].first, n, exact ? "PASS" : "FAIL", mm_sec * 1e3, mv_sec * 1e3);
        }
    }
    std::printf("selftest: %s\n", ok ? "ALL PASS" : "FAIL");
    release_device_tensors();
    return ok ? 0 : 1;
}
