// ref_shim.cpp -- a C entry point over the reference's own header-only CPU
// FFT (include/butterfly/fft.hpp:70-96 of TruNcat3/kunlunxin-fft), compiled
// from the reference tree in place by oracle/Makefile into oracle/_ref/.
// Test infrastructure only: it lets the parity tests compare the oracle's C
// restatement with the reference code itself, and lets bench.py time the
// reference CPU path (cpu_baseline kind "reference").  No reference source is
// copied here; this file only calls butterfly::fft_dit / fft_dif.
#include <algorithm>
#include <chrono>
#include <complex>
#include <cstdint>
#include <thread>
#include <vector>

#include "butterfly/fft.hpp"

extern "C" {

// In-place forward FFT of `batch` contiguous rows of interleaved
// complex<double>.  dif != 0 selects butterfly::fft_dif.
int ref_fft_batch(double* a, int64_t n, int64_t batch, int dif) {
    if (!butterfly::is_power_of_two(static_cast<std::size_t>(n))) return -1;
    std::vector<std::complex<double>> row(static_cast<std::size_t>(n));
    for (int64_t r = 0; r < batch; ++r) {
        double* p = a + 2 * r * n;
        for (int64_t i = 0; i < n; ++i) row[i] = {p[2 * i], p[2 * i + 1]};
        row = dif ? butterfly::fft_dif(row) : butterfly::fft_dit(row);
        for (int64_t i = 0; i < n; ++i) { p[2 * i] = row[i].real(); p[2 * i + 1] = row[i].imag(); }
    }
    return 0;
}

// Median seconds (std::chrono::steady_clock) over `reps` calls of
// ref_fft_batch on a fresh copy of `a` each time.
double ref_time_fft_batch(const double* a, int64_t n, int64_t batch, int dif, int reps) {
    if (reps < 1) reps = 1;
    std::vector<double> work(static_cast<std::size_t>(2 * n * batch));
    std::vector<double> t;
    for (int r = 0; r < reps; ++r) {
        std::copy(a, a + 2 * n * batch, work.begin());
        auto s0 = std::chrono::steady_clock::now();
        ref_fft_batch(work.data(), n, batch, dif);
        auto s1 = std::chrono::steady_clock::now();
        t.push_back(std::chrono::duration<double>(s1 - s0).count());
    }
    std::sort(t.begin(), t.end());
    return t[t.size() / 2];
}

// As ref_time_fft_batch, with the rows split into `threads` contiguous
// ranges, one std::thread each (the reference path is single-threaded per
// transform; this is the all-cores figure of the same work).
double ref_time_fft_batch_mt(const double* a, int64_t n, int64_t batch, int dif, int reps, int threads) {
    if (reps < 1) reps = 1;
    if (threads < 1) threads = 1;
    if (threads > batch) threads = static_cast<int>(batch);
    std::vector<double> work(static_cast<std::size_t>(2 * n * batch));
    std::vector<double> t;
    for (int r = 0; r < reps; ++r) {
        std::copy(a, a + 2 * n * batch, work.begin());
        auto s0 = std::chrono::steady_clock::now();
        std::vector<std::thread> pool;
        for (int k = 0; k < threads; ++k) {
            const int64_t r0 = batch * k / threads, r1 = batch * (k + 1) / threads;
            pool.emplace_back([&, r0, r1] { ref_fft_batch(work.data() + 2 * r0 * n, n, r1 - r0, dif); });
        }
        for (auto& th : pool) th.join();
        auto s1 = std::chrono::steady_clock::now();
        t.push_back(std::chrono::duration<double>(s1 - s0).count());
    }
    std::sort(t.begin(), t.end());
    return t[t.size() / 2];
}

unsigned ref_bit_reverse(unsigned x, int bits) { return butterfly::bit_reverse(x, bits); }

}  // extern "C"
