// mlp_device.hpp — device building blocks of the register-resident fp16
// MFMA MLPs and of the hash-grid gather that feeds them (see field.hip for the
// layout argument).  Shared by the forward kernels (field.hip) and the
// training kernels (train_kernels.hip).
#pragma once

#include "common.hpp"

namespace nerf_hip {
namespace mlp {

constexpr uint32_t kWaveSize    = 64;
constexpr uint32_t kBlockWaves  = 4;
constexpr uint32_t kBlockThreads = kWaveSize * kBlockWaves;

__device__ __forceinline__ floatx4 mfma16x16x32(const half8_t a, const half8_t b, const floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// k-index maps (see file header).  Returns -1 for a padded slot.
enum class KMap { Identity, Hidden, ColorIn };

__device__ __forceinline__ int logical_k(KMap m, uint32_t t, uint32_t g, uint32_t e) {
    switch (m) {
    case KMap::Identity: return (int)(32u * t + 8u * g + e);
    case KMap::Hidden: return (int)(32u * t + (e < 4u ? 4u * g + e : 16u + 4u * g + (e - 4u)));
    case KMap::ColorIn:
    default:
        if (e < 4u) {
            const uint32_t slot = 4u * g + e;  // density output neuron
            return slot == 0u ? -1 : (int)(slot - 1u);
        }
        return (int)(15u + 4u * g + (e - 4u));  // SH coefficient
    }
}

// A fragment of W [n_out][n_in] for output block b, k-step t.
__device__ __forceinline__ half8_t load_a(const half_t* W, uint32_t n_in, uint32_t b, uint32_t t, KMap m, uint32_t lane) {
    const uint32_t i = lane & 15u, g = lane >> 4;
    const half_t* row = W + (16u * b + i) * n_in;
    half8_t a;
#pragma unroll
    for (uint32_t e = 0; e < 8u; ++e) {
        const int k = logical_k(m, t, g, e);
        a[e]        = k < 0 ? (half_t)0.0f : row[k];
    }
    return a;
}

struct DensityFrags {
    half8_t w1[4];  // 64 x 32: blocks 0..3, one k-step
    half8_t w2[2];  // 16 x 64: one block, k-steps 0..1
};
struct ColorFrags {
    half8_t w1[4];  // 64 x 32
    half8_t w2[8];  // 64 x 64: [block * 2 + kstep]
    half8_t w3[2];  // 16 x 64
};

// Fragments of layers whose k-map is Identity or Hidden are contiguous runs
// of the weight row (8 halves, or two runs of 4), so they are read from LDS
// as one 16-byte or two 8-byte loads.  P must be 16-byte aligned.
__device__ __forceinline__ half8_t frag_identity(const half_t* W, uint32_t n_in, uint32_t b, uint32_t t, uint32_t lane) {
    const uint32_t i = lane & 15u, g = lane >> 4;
    return *reinterpret_cast<const half8_t*>(W + (16u * b + i) * n_in + 32u * t + 8u * g);
}
__device__ __forceinline__ half8_t frag_hidden(const half_t* row, uint32_t g) {
    const half4_t lo = *reinterpret_cast<const half4_t*>(row + 4u * g);
    const half4_t hi = *reinterpret_cast<const half4_t*>(row + 16u + 4u * g);
    return half8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

__device__ __forceinline__ void load_density(const half_t* P, DensityFrags& f, uint32_t lane) {
    const uint32_t i = lane & 15u, g = lane >> 4;
#pragma unroll
    for (uint32_t b = 0; b < 4u; ++b) f.w1[b] = frag_identity(P, 32u, b, 0u, lane);
#pragma unroll
    for (uint32_t t = 0; t < 2u; ++t) f.w2[t] = frag_hidden(P + 2048 + i * 64u + 32u * t, g);
}

__device__ __forceinline__ void load_color(const half_t* P, ColorFrags& f, uint32_t lane) {
    const uint32_t i = lane & 15u, g = lane >> 4;
#pragma unroll
    for (uint32_t b = 0; b < 4u; ++b) f.w1[b] = load_a(P, 32u, b, 0u, KMap::ColorIn, lane);
#pragma unroll
    for (uint32_t b = 0; b < 4u; ++b)
#pragma unroll
        for (uint32_t t = 0; t < 2u; ++t) f.w2[2u * b + t] = frag_hidden(P + 2048 + (16u * b + i) * 64u + 32u * t, g);
    // Colour output: MFMA row 4c (c = 1..3) computes output c - 1 and every
    // other row is zero, so lane group c holds colour c - 1 in element 0 (and
    // lane group 0 takes sigma from the density output, row 0).
    const bool used   = (i & 3u) == 0u && i != 0u;
    const half_t* row = P + 2048 + 4096 + (used ? (i / 4u - 1u) : 0u) * 64u;
    const half8_t z   = {};
#pragma unroll
    for (uint32_t t = 0; t < 2u; ++t) {
        const half8_t v = frag_hidden(row + 32u * t, g);
        f.w3[t]         = used ? v : z;
    }
}

// Copies the density (3072) and colour (7168) fp16 parameters into LDS,
// colour after density, as 1,280 16-byte chunks; every thread issues all of
// its loads before its first LDS store, so the copy costs about one memory
// latency instead of one per element.  Element copies when a source is not
// 16-byte aligned.  The caller synchronises the workgroup afterwards.
template <uint32_t kThreads>
__device__ __forceinline__ void stage_weights(half_t* lds, const half_t* __restrict__ dp, const half_t* __restrict__ cp) {
    constexpr uint32_t kD = NERF_EXT_DENSITY_PARAMS / 8u, kN = kD + NERF_EXT_COLOR_PARAMS / 8u;
    constexpr uint32_t kPer = (kN + kThreads - 1u) / kThreads;
    if (((reinterpret_cast<uintptr_t>(dp) | reinterpret_cast<uintptr_t>(cp)) & 15u) == 0u) {
        const uint4* d4 = reinterpret_cast<const uint4*>(dp);
        const uint4* c4 = reinterpret_cast<const uint4*>(cp);
        uint4 r[kPer];
#pragma unroll
        for (uint32_t k = 0; k < kPer; ++k) {
            const uint32_t c = threadIdx.x + kThreads * k;
            if (c < kN) r[k] = c < kD ? d4[c] : c4[c - kD];
        }
#pragma unroll
        for (uint32_t k = 0; k < kPer; ++k) {
            const uint32_t c = threadIdx.x + kThreads * k;
            if (c < kN) reinterpret_cast<uint4*>(lds)[c] = r[k];
        }
    } else {
        for (uint32_t i = threadIdx.x; i < NERF_EXT_DENSITY_PARAMS; i += kThreads) lds[i] = dp[i];
        for (uint32_t i = threadIdx.x; i < NERF_EXT_COLOR_PARAMS; i += kThreads) lds[NERF_EXT_DENSITY_PARAMS + i] = cp[i];
    }
}

// The density parameters alone (3072 halves, 384 chunks).
template <uint32_t kThreads>
__device__ __forceinline__ void stage_density(half_t* lds, const half_t* __restrict__ dp) {
    constexpr uint32_t kN = NERF_EXT_DENSITY_PARAMS / 8u, kPer = (kN + kThreads - 1u) / kThreads;
    if ((reinterpret_cast<uintptr_t>(dp) & 15u) == 0u) {
        uint4 r[kPer];
#pragma unroll
        for (uint32_t k = 0; k < kPer; ++k) {
            const uint32_t c = threadIdx.x + kThreads * k;
            if (c < kN) r[k] = reinterpret_cast<const uint4*>(dp)[c];
        }
#pragma unroll
        for (uint32_t k = 0; k < kPer; ++k) {
            const uint32_t c = threadIdx.x + kThreads * k;
            if (c < kN) reinterpret_cast<uint4*>(lds)[c] = r[k];
        }
    } else {
        for (uint32_t i = threadIdx.x; i < NERF_EXT_DENSITY_PARAMS; i += kThreads) lds[i] = dp[i];
    }
}

// ReLU in fp16 after the conversion (packed convert, packed max): the same
// values as converting max(v, 0), at a quarter of the fp32 max/canonicalise
// instructions.
__device__ __forceinline__ half4_t relu_half(const floatx4 v) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 z = {(half_t)0.0f, (half_t)0.0f};
    const h2 a = __builtin_elementwise_max(h2{(half_t)v[0], (half_t)v[1]}, z);
    const h2 b = __builtin_elementwise_max(h2{(half_t)v[2], (half_t)v[3]}, z);
    return half4_t{a[0], a[1], b[0], b[1]};
}

__device__ __forceinline__ half8_t cat(const half4_t a, const half4_t b) {
    return half8_t{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// 64 hidden neurons from a 32-wide B operand (4 output blocks, ReLU, fp16).
__device__ __forceinline__ void layer_32_64(const half8_t* w, const half8_t x, half4_t h[4]) {
    const floatx4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (uint32_t b = 0; b < 4u; ++b) h[b] = relu_half(mfma16x16x32(w[b], x, zero));
}

// 16 linear outputs from 64 hidden (one block, two k-steps).
__device__ __forceinline__ floatx4 layer_64_16(const half8_t* w, const half4_t h[4]) {
    const floatx4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
    floatx4 o          = mfma16x16x32(w[0], cat(h[0], h[1]), zero);
    return mfma16x16x32(w[1], cat(h[2], h[3]), o);
}

__device__ __forceinline__ floatx4 density_mlp(const DensityFrags& f, const half8_t x) {
    half4_t h[4];
    layer_32_64(f.w1, x, h);
    return layer_64_16(f.w2, h);
}

__device__ __forceinline__ floatx4 color_mlp(const ColorFrags& f, const half8_t x) {
    half4_t h1[4], h2[4];
    layer_32_64(f.w1, x, h1);
    const floatx4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (uint32_t b = 0; b < 4u; ++b) {
        floatx4 a = mfma16x16x32(f.w2[2u * b], cat(h1[0], h1[1]), zero);
        a         = mfma16x16x32(f.w2[2u * b + 1u], cat(h1[2], h1[3]), a);
        h2[b]     = relu_half(a);
    }
    return layer_64_16(f.w3, h2);
}

// Hash encoding of levels 4g..4g+3 of one point: features 8g..8g+7 as fp32.
template <typename TableT>
__device__ __forceinline__ void encode_quad(const GridParams& g, const TableT* __restrict__ table, const float p[3], uint32_t grp, float feat[8]) {
#pragma unroll
    for (uint32_t j = 0; j < 4u; ++j) {
        // Level 4*grp + j, selected without dynamic indexing of the kernel argument.
        const uint32_t l0 = j, l1 = 4u + j, l2 = 8u + j, l3 = 12u + j;
        const uint32_t N  = grp == 0u ? g.resolution[l0] : grp == 1u ? g.resolution[l1] : grp == 2u ? g.resolution[l2] : g.resolution[l3];
        const uint32_t dn = grp == 0u ? g.dense[l0] : grp == 1u ? g.dense[l1] : grp == 2u ? g.dense[l2] : g.dense[l3];
        const uint32_t level = 4u * grp + j;
        float a0 = 0.0f, a1 = 0.0f;
        // Lanes s and s ^ 1 of a lane group hold the same level of two
        // points, so they fetch each point's x-neighbour corners together
        // (one cache line per point and edge), dense and hashed levels alike:
        // the lane groups of a wave hold both kinds at once, and the 8-byte
        // x-pair loads of encode_level_xpair ran both branches (measured 1.5x
        // slower than one load per corner).
        if (level < g.n_levels) encode_level_lanepair(g, table, p, level, N, dn != 0u, a0, a1);
        feat[2u * j]      = a0;
        feat[2u * j + 1u] = a1;
    }
}

__device__ __forceinline__ half8_t to_half8(const float f[8]) {
    half8_t h;
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = (half_t)f[e];
    return h;
}

// Real SH bands 0..3 (Sloan 2008), coefficients 4g..4g+3 of a unit direction.
// c ? a : b as a bit blend (no branch; exact).
__device__ __forceinline__ float select_bits(bool c, float a, float b) {
    const uint32_t m = 0u - (uint32_t)c;
    return __uint_as_float((__float_as_uint(a) & m) | (__float_as_uint(b) & ~m));
}

// All 16 coefficients of a unit direction.
__device__ __forceinline__ void sh16(const float d[3], float s[16]) {
    const float x = d[0], y = d[1], z = d[2];
    const float xy = x * y, yz = y * z, xz = x * z;
    const float x2 = x * x, y2 = y * y, z2 = z * z;
    s[0]  = 0.28209479177387814f;
    s[1]  = -0.48860251190291987f * y;
    s[2]  = 0.48860251190291987f * z;
    s[3]  = -0.48860251190291987f * x;
    s[4]  = 1.0925484305920792f * xy;
    s[5]  = -1.0925484305920792f * yz;
    s[6]  = 0.94617469575755997f * z2 - 0.31539156525251999f;
    s[7]  = -1.0925484305920792f * xz;
    s[8]  = 0.54627421529603959f * (x2 - y2);
    s[9]  = 0.59004358992664352f * y * (3.0f * x2 - y2) * -1.0f;
    s[10] = 2.8906114426405538f * xy * z;
    s[11] = 0.45704579946446572f * y * (1.0f - 5.0f * z2);
    s[12] = 0.3731763325901154f * z * (5.0f * z2 - 3.0f);
    s[13] = 0.45704579946446572f * x * (1.0f - 5.0f * z2);
    s[14] = 1.4453057213202769f * z * (x2 - y2);
    s[15] = 0.59004358992664352f * x * (3.0f * y2 - x2);
}

// Coefficients 4g..4g+3 (lane group g) of a unit direction.
__device__ __forceinline__ void sh4_quad(const float d[3], uint32_t grp, float out[4]) {
    float s[16];
    sh16(d, s);
    // Lane group g takes s[4g .. 4g + 3]: bitwise selects, so the four groups
    // of a wave never take divergent branches.
#pragma unroll
    for (uint32_t e = 0; e < 4u; ++e) {
        const float lo = select_bits((grp & 1u) != 0u, s[4u + e], s[e]);
        const float hi = select_bits((grp & 1u) != 0u, s[12u + e], s[8u + e]);
        out[e]         = select_bits((grp & 2u) != 0u, hi, lo);
    }
}

// Output activation spread over the wave: lane (g, s) holds channel g of
// sample s in element 0 (sigma from the density output o, colour g - 1 from
// the row-permuted colour output c) and applies its activation (g = 0: exp,
// else sigmoid 1 / (1 + exp(-c)) with the hardware reciprocal, 1 ulp), so
// each lane evaluates one exponential and one reciprocal; bit selects keep
// the wave convergent.
__device__ __forceinline__ float field_channel(const floatx4 o, const floatx4 c, uint32_t grp) {
    const bool sigma = grp == 0u;
    const float e    = __expf(select_bits(sigma, o[0], -c[0]));
    return select_bits(sigma, e, __builtin_amdgcn_rcpf(1.0f + e));
}

// Colour input of lane group grp from density outputs 4g..4g+3 and the four
// fp16 SH coefficients 4g..4g+3; the slot of density output 0 (sigma) carries
// a zero weight and a zero value.
__device__ __forceinline__ half8_t color_input(const floatx4 o, const half4_t sh, uint32_t grp) {
    half8_t xc;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        xc[e]     = (half_t)o[e];
        xc[4 + e] = sh[e];
    }
    if (grp == 0u) xc[0] = (half_t)0.0f;
    return xc;
}

}  // namespace mlp
}  // namespace nerf_hip
