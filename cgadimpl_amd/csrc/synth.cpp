// synth.cpp -- seeded synthetic inputs for the RMSNorm layer configurations.
//
// The stream is std::mt19937_64(seed), whose output sequence the C++ standard
// fixes, so the same seed gives the same inputs on every host.  Normal draws
// use the Box-Muller transform (Box & Muller, 1958) coded out in double, not
// std::normal_distribution (its algorithm is implementation-defined).
//
// Draw rules:
//   uniform53()   = (next() >> 11) * 2^-53                in [0, 1)
//   normal pair   : u1 = 1 - uniform53() (in (0, 1]), u2 = uniform53(),
//                   rad = sqrt(-2 ln u1), z0 = rad cos(2 pi u2),
//                   z1 = rad sin(2 pi u2); values are emitted z0, z1, z0, ...
//                   and an odd count drops the last z1.
//   uniform(a,b)  = a + (b - a) * uniform53()
//   outliers(p,s) : one uniform53() per element; elements with u < p are
//                   multiplied by s.
// Values are produced in double and rounded once to fp32; bf16 storage rounds
// that fp32 value to nearest-even.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <random>

namespace {

struct Gen {
    std::mt19937_64 eng;
    explicit Gen(uint64_t seed) : eng(seed) {}
    double uniform53() { return static_cast<double>(eng() >> 11) * 0x1.0p-53; }
};

uint16_t bf16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu))
        return static_cast<uint16_t>((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

}  // namespace

extern "C" {

void* agk_synth_new(uint64_t seed) { return new Gen(seed); }

void agk_synth_free(void* g) { delete static_cast<Gen*>(g); }

// Raw engine output, for known-answer checks of the stream.
void agk_synth_raw_u64(void* gp, uint64_t* out, int64_t n) {
    Gen& g = *static_cast<Gen*>(gp);
    for (int64_t i = 0; i < n; ++i) out[i] = g.eng();
}

void agk_synth_normal_f32(void* gp, float* out, int64_t n, double mean, double stddev) {
    Gen& g = *static_cast<Gen*>(gp);
    const double two_pi = 6.283185307179586476925286766559;
    int64_t i = 0;
    while (i < n) {
        const double u1 = 1.0 - g.uniform53();
        const double u2 = g.uniform53();
        const double rad = sqrt(-2.0 * log(u1));
        out[i++] = static_cast<float>(mean + stddev * rad * cos(two_pi * u2));
        if (i < n) out[i++] = static_cast<float>(mean + stddev * rad * sin(two_pi * u2));
    }
}

void agk_synth_uniform_f32(void* gp, float* out, int64_t n, double lo, double hi) {
    Gen& g = *static_cast<Gen*>(gp);
    for (int64_t i = 0; i < n; ++i) out[i] = static_cast<float>(lo + (hi - lo) * g.uniform53());
}

// Scales elements of x whose independent uniform draw is below p; returns
// how many were scaled.
int64_t agk_synth_outliers_f32(void* gp, float* x, int64_t n, double p, double scale) {
    Gen& g = *static_cast<Gen*>(gp);
    int64_t hits = 0;
    for (int64_t i = 0; i < n; ++i) {
        if (g.uniform53() < p) {
            x[i] = static_cast<float>(static_cast<double>(x[i]) * scale);
            ++hits;
        }
    }
    return hits;
}

void agk_synth_to_bf16(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = bf16_rne(in[i]);
}

}  // extern "C"
