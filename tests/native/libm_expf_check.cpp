// Host-side check of q3x::libm_expf (qwen3x_amd/csrc/libm_expf.h) against
// the host libm's expf, on every float of the ranges given on the command
// line as bit patterns [lo, hi] (inclusive).  Prints the count of values
// checked and of mismatches, and the first mismatch; exits 1 on any.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <thread>
#include <vector>

#include "libm_expf.h"

static float from_bits(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static uint32_t to_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

int main(int argc, char** argv) {
    if (argc < 3 || (argc - 1) % 2) { fprintf(stderr, "usage: %s lo hi [lo hi ...]\n", argv[0]); return 2; }
    std::atomic<unsigned long long> checked{0}, bad{0};
    std::atomic<uint32_t> first{0};
    const unsigned threads = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    for (int a = 1; a + 1 < argc; a += 2) {
        const uint64_t lo = strtoull(argv[a], nullptr, 0), hi = strtoull(argv[a + 1], nullptr, 0);
        std::vector<std::thread> pool;
        for (unsigned t = 0; t < threads; ++t)
            pool.emplace_back([&, t] {
                unsigned long long n = 0, m = 0;
                for (uint64_t u = lo + t; u <= hi; u += threads) {
                    const float x = from_bits(static_cast<uint32_t>(u));
                    const uint32_t want = to_bits(expf(x)), got = to_bits(q3x::libm_expf(x));
                    ++n;
                    if (want != got && !(x != x)) {
                        if (m++ == 0) first = static_cast<uint32_t>(u);
                    }
                }
                checked += n;
                bad += m;
            });
        for (auto& th : pool) th.join();
    }
    printf("checked %llu mismatches %llu first 0x%08x\n", checked.load(), bad.load(), first.load());
    return bad.load() ? 1 : 0;
}
