// Host check of expf_libm (agent-serve_amd/csrc/expf_libm.hpp, the expf the GPU sampler
// uses) against the host libm's expf: every float in [-128, -0], the arguments
// sample_logits (sampler.cpp:29) passes. Prints the number of differing results.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>

#include "expf_libm.hpp"

int main() {
    static const uint64_t tab[32] = TF_EXP2_TABLE;
    const uint32_t lo = 0x80000000u, hi = 0xC3000000u;  // -0 .. -128
    const int nt = (int)std::max(1u, std::thread::hardware_concurrency());
    std::vector<long> bad(nt, 0);
    std::vector<std::thread> th;
    for (int t = 0; t < nt; ++t)
        th.emplace_back([&, t] {
            for (uint64_t u = lo + (uint64_t)t; u <= hi; u += (uint64_t)nt) {
                float x;
                const uint32_t b = (uint32_t)u;
                std::memcpy(&x, &b, 4);
                const float a = expf(x), g = tfk::expf_libm(x, tab);
                if (std::memcmp(&a, &g, 4) != 0) ++bad[t];
            }
        });
    for (auto& x : th) x.join();
    long total = 0;
    for (long b : bad) total += b;
    std::printf("%ld\n", total);
    return 0;
}
