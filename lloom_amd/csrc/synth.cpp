// synth.cpp -- the deterministic synthetic-input generator used by the
// benchmark and the tests (it has no counterpart in the reference).
//
// Element i of a stream belongs to chunk i / 65536; chunk c runs its own
// xoshiro256** generator whose state is four SplitMix64 outputs seeded by
// (seed, c).  Normals are Box-Muller pairs from two 53-bit uniforms.  The
// chunking makes the output independent of how many threads fill it.
#include <cmath>
#include <cstdint>
#include <thread>
#include <vector>

#include "../../include/lloom_hip.h"

namespace {

constexpr int64_t CHUNK = 65536;

inline uint64_t splitmix64(uint64_t& s) {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

struct Xoshiro {
    uint64_t s[4];
    Xoshiro(uint64_t seed, uint64_t chunk) {
        uint64_t sm = seed ^ (chunk * 0xD1B54A32D192ED03ull);
        for (auto& v : s) v = splitmix64(sm);
    }
    static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
    uint64_t next() {
        uint64_t r = rotl(s[1] * 5, 7) * 9;
        uint64_t t = s[1] << 17;
        s[2] ^= s[0];
        s[3] ^= s[1];
        s[1] ^= s[2];
        s[0] ^= s[3];
        s[2] ^= t;
        s[3] = rotl(s[3], 45);
        return r;
    }
    double uniform() { return (double)(next() >> 11) * 0x1.0p-53; }
};

template <typename F>
void parallel_chunks(int64_t count, F fill) {
    int64_t nchunks = (count + CHUNK - 1) / CHUNK;
    unsigned hw = std::thread::hardware_concurrency();
    int nt = (int)(hw == 0 ? 1 : (hw > 16 ? 16 : hw));
    if (nchunks < nt) nt = (int)(nchunks > 0 ? nchunks : 1);
    std::vector<std::thread> th;
    for (int t = 0; t < nt; t++)
        th.emplace_back([=]() {
            for (int64_t c = t; c < nchunks; c += nt) fill(c, c * CHUNK, std::min(count, (c + 1) * CHUNK));
        });
    for (auto& x : th) x.join();
}

}  // namespace

extern "C" int lloom_hip_synth_normal(uint64_t seed, float mean, float std_, float* out, int64_t count) {
    if (!out || count < 0) return LLOOM_HIP_EINVAL;
    parallel_chunks(count, [=](int64_t c, int64_t lo, int64_t hi) {
        Xoshiro g(seed, (uint64_t)c);
        for (int64_t i = lo; i < hi; i += 2) {
            double u1 = 1.0 - g.uniform(), u2 = g.uniform();
            double r = std::sqrt(-2.0 * std::log(u1));
            out[i] = (float)(mean + std_ * r * std::cos(2.0 * M_PI * u2));
            if (i + 1 < hi) out[i + 1] = (float)(mean + std_ * r * std::sin(2.0 * M_PI * u2));
        }
    });
    return LLOOM_HIP_OK;
}

extern "C" int lloom_hip_synth_uniform(uint64_t seed, float lo_, float hi_, float* out, int64_t count) {
    if (!out || count < 0) return LLOOM_HIP_EINVAL;
    parallel_chunks(count, [=](int64_t c, int64_t lo, int64_t hi) {
        Xoshiro g(seed, (uint64_t)c);
        for (int64_t i = lo; i < hi; i++) out[i] = (float)(lo_ + (hi_ - lo_) * g.uniform());
    });
    return LLOOM_HIP_OK;
}
