// Deterministic synthetic weights (include/qlm_engine.h, "synthetic
// checkpoints"). Element i of a tensor is a pure function of (seed, i):
//   u1, u2 = uniforms from splitmix64(seed + 2i), splitmix64(seed + 2i + 1)
//   z = sqrt(-2 ln u1) * cos(2 pi u2)           (Box-Muller, double)
// so any partition of the work over threads gives identical bytes.

#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "qlm_engine.h"

namespace {

inline uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// (0, 1]: never 0, so log() is finite.
inline double unit_open0(uint64_t r) { return ((double)(r >> 11) + 1.0) * (1.0 / 9007199254740992.0); }
// [0, 1)
inline double unit(uint64_t r) { return (double)(r >> 11) * (1.0 / 9007199254740992.0); }

inline double normal_at(uint64_t seed, uint64_t i) {
    const double u1 = unit_open0(splitmix64(seed + 2 * i));
    const double u2 = unit(splitmix64(seed + 2 * i + 1));
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}

inline uint16_t f32_to_bf16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    u += 0x7FFFu + ((u >> 16) & 1u);  // round to nearest even (finite inputs)
    return (uint16_t)(u >> 16);
}

template <typename F>
void parallel_for(size_t n, F&& f) {
    unsigned nt = std::thread::hardware_concurrency();
    if (nt == 0) nt = 1;
    if (nt > 16) nt = 16;
    if (n < (size_t)1 << 16) nt = 1;
    std::vector<std::thread> th;
    const size_t chunk = (n + nt - 1) / nt;
    for (unsigned t = 0; t < nt; ++t) {
        const size_t lo = t * chunk, hi = std::min(n, lo + chunk);
        if (lo >= hi) break;
        th.emplace_back([=, &f] { f(lo, hi); });
    }
    for (auto& x : th) x.join();
}

}  // namespace

extern "C" {

uint64_t qlm_synth_tensor_seed(uint64_t base, const char* name) {
    uint64_t h = 0xCBF29CE484222325ull;  // FNV-1a 64
    for (const char* p = name; p && *p; ++p) {
        h ^= (uint8_t)*p;
        h *= 0x100000001B3ull;
    }
    return splitmix64(base ^ h);
}

int qlm_synth_normal_f32(float* out, size_t n, uint64_t seed, float mean, float std_dev) {
    if (!out) return 1;
    parallel_for(n, [&](size_t lo, size_t hi) {
        for (size_t i = lo; i < hi; ++i) out[i] = (float)((double)mean + (double)std_dev * normal_at(seed, i));
    });
    return 0;
}

int qlm_synth_normal_bf16(uint16_t* out, size_t n, uint64_t seed, float mean, float std_dev) {
    if (!out) return 1;
    parallel_for(n, [&](size_t lo, size_t hi) {
        for (size_t i = lo; i < hi; ++i)
            out[i] = f32_to_bf16((float)((double)mean + (double)std_dev * normal_at(seed, i)));
    });
    return 0;
}

int qlm_synth_uniform_f32(float* out, size_t n, uint64_t seed, float lo, float hi) {
    if (!out) return 1;
    parallel_for(n, [&](size_t a, size_t b) {
        for (size_t i = a; i < b; ++i)
            out[i] = (float)((double)lo + ((double)hi - (double)lo) * unit(splitmix64(seed + i)));
    });
    return 0;
}

}  // extern "C"
