// nerf_math.h — scalar helpers compiled identically for the host and for gfx950.
//
// Everything here is plain C++ with no intrinsics so that host (g++/clang) and
// device (hipcc, gfx950) builds execute the same sequence of correctly rounded
// IEEE-754 binary32 operations.  Translation units that include it must be
// built with -ffp-contract=off; that is what makes occupancy bits, hash indices
// and sample counts bit-identical between the GPU kernels and a CPU build.
#pragma once

#include <math.h>
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define NERF_HD __host__ __device__ __forceinline__
#else
#define NERF_HD static inline
#endif

namespace nerf_math {

// Spatial-hash primes of Mueller et al., "Instant Neural Graphics Primitives"
// (SIGGRAPH 2022), section 3: pi_1 = 1, pi_2 = 2654435761, pi_3 = 805459861.
constexpr uint32_t kPrime1 = 1u;
constexpr uint32_t kPrime2 = 2654435761u;
constexpr uint32_t kPrime3 = 805459861u;

// splitmix64 constants (Steele, Lea, Flood, "Fast splittable pseudorandom
// number generators", OOPSLA 2014), as used by the reference's weight init
// (backend-cuda.cu:1811-1824).
constexpr uint64_t kGolden = 0x9e3779b97f4a7c15ull;
constexpr uint64_t kMix1   = 0xbf58476d1ce4e5b9ull;
constexpr uint64_t kMix2   = 0x94d049bb133111ebull;

NERF_HD uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof(u));
    return u;
}
NERF_HD float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, sizeof(f));
    return f;
}

// Initial state of one splitmix64 stream keyed by (a, b); the reference seeds
// its two MLP streams this way (backend-cuda.cu:1811, :1830).
NERF_HD uint64_t stream_state(uint64_t a, uint64_t b) {
    return (a + kGolden) ^ (b * kMix1);
}

// Output number i (0-based) of a splitmix64 stream.  The sequential generator
// adds kGolden before each draw, so draw i sees state0 + (i + 1) * kGolden;
// computing it directly lets every GPU lane produce its element independently.
NERF_HD uint64_t splitmix_at(uint64_t state0, uint64_t i) {
    uint64_t z = state0 + (i + 1ull) * kGolden;
    z = (z ^ (z >> 30)) * kMix1;
    z = (z ^ (z >> 27)) * kMix2;
    return z ^ (z >> 31);
}

// 24-bit uniform in [0, 1) from the high word of a splitmix64 output
// (backend-cuda.cu:1824: (u32)(z >> 32) >> 8, times 2^-24).
NERF_HD float unit24(uint64_t z) {
    return (float)((uint32_t)(z >> 32) >> 8) * (1.0f / 16777216.0f);
}

// Deterministic exp for binary32, used where host and device must agree bit for
// bit (the analytic Gaussian density that feeds the occupancy bitfield).
// Method: Cody & Waite argument reduction x = k ln2 + r with ln2 split into
// ln2_hi = 0.693359375 (exact in 9 bits) and ln2_lo = -2.12194440e-4, followed by the
// degree-7 minimax polynomial for exp(r) on [-ln2/2, ln2/2] from S. L. Moshier's
// Cephes library (expf.c), and scaling by 2^k through the exponent field.
// Inputs below -87 return 0 (results that would be subnormal are flushed) and
// inputs above 88 are clamped to 88.  Accuracy: within 2 ulp of the correctly
// rounded exp on [-87, 88] (checked against libm by the CPU tests).
NERF_HD float det_expf(float x) {
    if (!(x >= -87.0f)) return 0.0f;  // also maps NaN to 0
    if (x > 88.0f) x = 88.0f;
    const float kf = floorf(x * 1.44269504088896341f + 0.5f);
    float r        = x - kf * 0.693359375f;
    r              = r - kf * -2.12194440e-4f;
    const float r2 = r * r;
    float p        = 1.9875691500e-4f;
    p              = p * r + 1.3981999507e-3f;
    p              = p * r + 8.3334519073e-3f;
    p              = p * r + 4.1665795894e-2f;
    p              = p * r + 1.6666665459e-1f;
    p              = p * r + 5.0000001201e-1f;
    p              = p * r2 + r;
    p              = p + 1.0f;
    const int32_t k = (int32_t)kf;  // in [-125, 127], so the result stays normal
    return bits_f32(f32_bits(p) + ((uint32_t)k << 23));
}

}  // namespace nerf_math
