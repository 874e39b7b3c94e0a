// hb_fill.cpp -- the seeded synthetic inputs: bf16 ~ N(0, std^2) from
// splitmix64 and Box-Muller.  Element i depends on (seed, i) only: pair
// j = i / 2 draws two uniforms from splitmix64 outputs 2j and 2j+1 of the
// seed's stream; element 2j is r cos(2 pi u2), element 2j+1 r sin(2 pi u2),
// r = sqrt(-2 ln(1 - u1)), all in double, then f32, then rounded to nearest
// even.  (The reference's own generators, fill_random16 at qwen.rs:2613-2627
// and random16 at bin/herbert-metal-probe.rs:446-463, draw uniform bf16;
// the graded inputs are the normal ones this file makes.)
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "herbert_hip.h"

namespace {

// Output `i` (0-based) of splitmix64 seeded with `seed` (Steele, Lea and
// Flood, "Fast splittable pseudorandom number generators", OOPSLA 2014).
inline uint64_t splitmix64(uint64_t seed, uint64_t i) {
    uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

inline uint16_t rne(float f) {
    uint32_t b;
    std::memcpy(&b, &f, 4);
    return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

void fill_range(uint64_t seed, double sd, uint16_t* out, uint64_t lo, uint64_t hi) {
    const double two_pi = 6.283185307179586476925286766559;
    for (uint64_t j = lo / 2; 2 * j < hi; j++) {
        double u1 = (double)(splitmix64(seed, 2 * j) >> 11) * 0x1.0p-53;
        double u2 = (double)(splitmix64(seed, 2 * j + 1) >> 11) * 0x1.0p-53;
        double r = std::sqrt(-2.0 * std::log(1.0 - u1));
        double a = two_pi * u2;
        if (2 * j >= lo) out[2 * j] = rne((float)(r * std::cos(a) * sd));
        if (2 * j + 1 < hi && 2 * j + 1 >= lo) out[2 * j + 1] = rne((float)(r * std::sin(a) * sd));
    }
}

}  // namespace

extern "C" void hb_fill_normal_bf16(uint64_t seed, float std_, uint16_t* out, uint64_t n,
                                    int threads) {
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    if (n < (1u << 16)) threads = 1;
    uint64_t per = ((n + threads - 1) / threads + 1) & ~1ull;  // even, covers n
    std::vector<std::thread> t;
    for (int i = 0; i < threads; i++) {
        uint64_t lo = per * i, hi = lo + per < n ? lo + per : n;
        if (lo >= n) break;
        t.emplace_back(fill_range, seed, (double)std_, out, lo, hi);
    }
    for (auto& th : t) th.join();
}
