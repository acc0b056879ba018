// synth.cpp - the seeded synthetic inputs of bench.py (host code in
// libhephbench.so, not part of the FP8 linear library).
//
// Counter-based splitmix64 with Box-Muller in double: element i of a stream
// draws two uniforms from the pair i >> 1 and takes the cosine (even i) or
// sine (odd i) branch, so any range of a stream can be generated on its own
// and in parallel. This is the sequence of the parity tests' generator (the
// bench's activations for a seed are the bytes the tests draw for that seed;
// tests/test_bench_synth.py checks it bit for bit), restated here because the
// bench may use the CPU restatement only for its CPU baseline. Compiled with
// -ffp-contract=off, as that generator is: every product and sum rounds
// separately.
#include <algorithm>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

namespace {

inline uint64_t splitmix64(uint64_t z)
{
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// [0, 1) with 53 random bits
inline double uniform01(uint64_t seed, uint64_t i)
{
    const uint64_t z = splitmix64(splitmix64(seed) ^ (i * 0xD1B54A32D192ED03ull));
    return (double)(z >> 11) * (1.0 / 9007199254740992.0);
}

inline float normal_at(uint64_t seed, uint64_t idx, float mean, float stddev)
{
    const double two_pi = 6.283185307179586476925286766559;
    const uint64_t pair = idx >> 1;
    double u1 = uniform01(seed, 2 * pair);
    const double u2 = uniform01(seed, 2 * pair + 1);
    if (u1 < 1e-300) u1 = 1e-300;
    const double r = std::sqrt(-2.0 * std::log(u1));
    const double z = (idx & 1) ? r * std::sin(two_pi * u2) : r * std::cos(two_pi * u2);
    return (float)((double)mean + (double)stddev * z);
}

// f32 -> bf16 bits, round to nearest even (NaN kept quiet)
inline uint16_t to_bf16(float f)
{
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// Runs body(begin, end) over [0, n) on up to 16 threads.
template <class F>
void parallel(size_t n, F body)
{
    const unsigned hw = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    const size_t parts = n < (1u << 16) ? 1 : hw;
    if (parts == 1) {
        body((size_t)0, n);
        return;
    }
    std::vector<std::thread> ts;
    for (size_t p = 0; p < parts; ++p) {
        const size_t b = n * p / parts, e = n * (p + 1) / parts;
        ts.emplace_back([=] { body(b, e); });
    }
    for (auto& t : ts) t.join();
}

}  // namespace

extern "C" {

// out[i] = element offset + i of the normal stream of `seed`, mean + std * z.
void heph_bench_gen_normal(uint64_t seed, uint64_t offset, size_t n, float mean, float stddev,
                           float* out)
{
    parallel(n, [&](size_t b, size_t e) {
        for (size_t i = b; i < e; ++i) out[i] = normal_at(seed, offset + i, mean, stddev);
    });
}

// The same values rounded to bf16.
void heph_bench_gen_normal_bf16(uint64_t seed, uint64_t offset, size_t n, float mean,
                                float stddev, uint16_t* out)
{
    parallel(n, [&](size_t b, size_t e) {
        for (size_t i = b; i < e; ++i) out[i] = to_bf16(normal_at(seed, offset + i, mean, stddev));
    });
}

// Activations: N(0,1) element i, times outlier_mul where the uniform stream
// of seed ^ 0x5eed is below outlier_p at i, rounded to bf16.
void heph_bench_gen_act_bf16(uint64_t seed, size_t n, double outlier_p, float outlier_mul,
                             uint16_t* out)
{
    parallel(n, [&](size_t b, size_t e) {
        for (size_t i = b; i < e; ++i) {
            float v = normal_at(seed, i, 0.0f, 1.0f);
            if (outlier_p > 0.0 && uniform01(seed ^ 0x5eedull, i) < outlier_p) v *= outlier_mul;
            out[i] = to_bf16(v);
        }
    });
}

// FNV-1a 64 of n bytes (the digests bench.py checks its inputs against).
uint64_t heph_bench_fnv1a64(const void* data, size_t n)
{
    const uint8_t* p = static_cast<const uint8_t*>(data);
    uint64_t h = 0xcbf29ce484222325ull;
    for (size_t i = 0; i < n; ++i) {
        h ^= p[i];
        h *= 0x100000001b3ull;
    }
    return h;
}

}  // extern "C"
