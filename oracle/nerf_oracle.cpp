// nerf_oracle.cpp — scalar C++ CPU oracle of the NeRF hot path.
//
// TEST INFRASTRUCTURE ONLY.  This file is the oracle: tests/, the smoke check
// in __graft_entry__.py and the cpu_baseline leg of bench.py call it through
// ctypes (oracle/liboracle.so).  The product (nerf_amd/libnerf.so) never links,
// loads or calls it.
//
// It restates, one scalar operation at a time, the semantics of each stage:
//   * stages the reference has (ray generation, AABB clip, occupancy lookup,
//     march, composite, RGBA8 packing, RNG, weight init) follow
//     Xayah-Graphics/NeRF backend-cuda.cu at the cited lines, with two
//     documented substitutions: 1/sqrtf replaces rsqrtf (:384) so that the
//     result is correctly rounded on every target, and libm expf replaces
//     __expf;
//   * stages the reference lacks (hash-grid encoding, SH degree-4 direction
//     encoding, exp density activation, analytic Gaussian scene) follow their
//     published definitions, cited at each function.
// Build flags: -O2 -ffp-contract=off, no SIMD intrinsics (oracle/Makefile).
//
// How each part is pinned (tests/test_oracle_*.py): fp16 conversion against
// numpy's IEEE conversion; splitmix64 against Vigna's published seed-0
// outputs; hash indices against brute-force closed forms and dense-level
// injectivity; trilinear interpolation against exact reproduction of linear
// tables; MLP against an fp64 numpy GEMM with the same rounding points; SH
// against quadrature orthonormality; rays, AABB and march against analytic
// axis-aligned cases; composite against the closed form for constant density;
// the Huber loss against a one-sample closed form in both branches.
// hash_u32, rand01, the training pixel draws and the camera pick
// (:321-332, :438-440, :1482) have no published test vector: they are pinned
// by a numpy uint32 restatement of the reference's recurrences, compared bit
// for bit (tests/test_oracle_rng_pins.py), plus bijectivity and avalanche.

#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <thread>
#include <vector>

#include "../nerf_amd/csrc/nerf_math.h"  // det_expf only (shared on purpose: bit-exact occupancy)

// ---------------------------------------------------------------------------
// IEEE binary16 conversion (round to nearest even), written from the format
// definition (IEEE 754-2008, section 3.6).
// ---------------------------------------------------------------------------
extern "C" uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t a    = x & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);  // NaN
    if (a >= 0x47800000u) return (uint16_t)(sign | 0x7c00u); // >= 2^16: inf
    if (a >= 0x38800000u) {                                   // normal half
        const uint32_t mant = a & 0x7fffffu;
        const uint32_t exp  = (a >> 23) - 127u + 15u;
        uint32_t h          = (exp << 10) | (mant >> 13);
        const uint32_t rem  = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;  // may carry into inf
        return (uint16_t)(sign | h);
    }
    if (a < 0x33000000u) return (uint16_t)sign;  // below 2^-25: rounds to zero
    const uint32_t mant  = (a & 0x7fffffu) | 0x800000u;
    const uint32_t shift = 126u - (a >> 23);      // 14..24
    uint32_t h           = mant >> shift;
    const uint32_t rem   = mant & ((1u << shift) - 1u);
    const uint32_t half  = 1u << (shift - 1u);
    if (rem > half || (rem == half && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

extern "C" float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e    = (h >> 10) & 0x1fu;
    uint32_t m          = h & 0x3ffu;
    uint32_t x;
    if (e == 0u) {
        if (m == 0u) {
            x = sign;
        } else {  // subnormal: normalise
            uint32_t ee = 113u;
            while (!(m & 0x400u)) {
                m <<= 1;
                --ee;
            }
            x = sign | (ee << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (e == 31u) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

extern "C" void orc_f32_to_f16_array(const float* src, uint16_t* dst, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) dst[i] = orc_f32_to_f16(src[i]);
}

static inline float r16(float x) { return orc_f16_to_f32(orc_f32_to_f16(x)); }

// ---------------------------------------------------------------------------
// Integer RNG.
// ---------------------------------------------------------------------------
// backend-cuda.cu:321-328 (== :1439-1446).
extern "C" uint32_t orc_hash_u32(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}
// backend-cuda.cu:329-332.
extern "C" float orc_rand01(uint32_t seed) {
    return (float)(orc_hash_u32(seed) & 0x00ffffffu) / (float)0x01000000u;
}

// Sequential splitmix64 exactly as the reference's init loop runs it
// (backend-cuda.cu:1811, :1819-1823): state += golden; mix.
extern "C" void orc_splitmix_sequence(uint64_t state, uint64_t n, uint64_t* out) {
    for (uint64_t i = 0; i < n; ++i) {
        state += 0x9e3779b97f4a7c15ull;
        uint64_t z = state;
        z          = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z          = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        out[i]     = z ^ (z >> 31);
    }
}

// State seeding of backend-cuda.cu:1811 / :1830.
extern "C" uint64_t orc_stream_state(uint64_t a, uint64_t b) {
    return (a + 0x9e3779b97f4a7c15ull) ^ (b * 0xbf58476d1ce4e5b9ull);
}

// n uniforms lo + (hi - lo) * u24, u24 = ((u32)(z >> 32) >> 8) / 2^24, from the
// sequential stream (a, b).  Used for the hash table init U(-1e-4, 1e-4) and for
// all synthetic inputs; written as (2u - 1) * half_range + mid to mirror
// backend-cuda.cu:1824 when lo = -hi.
extern "C" void orc_uniform_fill(uint64_t a, uint64_t b, uint64_t n, float lo, float hi, float* out) {
    uint64_t state = orc_stream_state(a, b);
    for (uint64_t i = 0; i < n; ++i) {
        state += 0x9e3779b97f4a7c15ull;
        uint64_t z     = state;
        z              = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z              = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        z              = z ^ (z >> 31);
        const float u  = (float)((uint32_t)(z >> 32) >> 8) * (1.0f / 16777216.0f);
        if (lo == -hi)
            out[i] = (u * 2.0f - 1.0f) * hi;
        else
            out[i] = lo + (hi - lo) * u;
    }
}

// Xavier-uniform MLP init of backend-cuda.cu:1810-1847 applied to the target
// shapes: density 32->64->16 (seeds 0x1234/0x5678), colour 32->64->64->16
// (seeds 0x9abc/0xdef0).  Matrices are packed [out][in], input layer first.
extern "C" uint32_t orc_mlp_param_count(uint32_t network) { return network == 0u ? 3072u : 7168u; }

extern "C" void orc_mlp_init(uint32_t network, float* out) {
    const uint32_t dens_shape[2][2] = {{64u, 32u}, {16u, 64u}};
    const uint32_t col_shape[3][2]  = {{64u, 32u}, {64u, 64u}, {16u, 64u}};
    const uint32_t n_mat            = network == 0u ? 2u : 3u;
    uint64_t state = network == 0u ? orc_stream_state(0x1234ull, 0x5678ull) : orc_stream_state(0x9abcull, 0xdef0ull);
    uint64_t off   = 0;
    for (uint32_t m = 0; m < n_mat; ++m) {
        const uint32_t fan_out = network == 0u ? dens_shape[m][0] : col_shape[m][0];
        const uint32_t fan_in  = network == 0u ? dens_shape[m][1] : col_shape[m][1];
        const float scale      = sqrtf(6.0f / (float)(fan_in + fan_out));
        for (uint64_t i = 0; i < (uint64_t)fan_in * fan_out; ++i) {
            state += 0x9e3779b97f4a7c15ull;
            uint64_t z = state;
            z          = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
            z          = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
            z ^= z >> 31;
            out[off + i] = ((float)((uint32_t)(z >> 32) >> 8) * (1.0f / 16777216.0f) * 2.0f - 1.0f) * scale;
        }
        off += (uint64_t)fan_in * fan_out;
    }
}

// ---------------------------------------------------------------------------
// Multiresolution hash grid (Mueller et al. 2022, section 3).
// ---------------------------------------------------------------------------
struct OrcGrid {
    uint32_t n_levels;
    uint32_t n_features;
    uint32_t table_size;  // T, a power of two
    uint32_t table_dtype; // 0 f32, 1 f16
    uint32_t resolution[16];
    uint32_t dense[16];
};

// N_l = floor(N_min * b^l + 1e-9) in double; b = (finest / base)^(1 / (L - 1))
// when finest > 0.  A level is dense (1:1 indexing) when (N_l + 1)^3 <= T.
extern "C" void orc_grid_levels(uint32_t n_levels, uint32_t base, float per_level_scale, uint32_t finest, uint32_t log2_table_size, uint32_t* resolution, uint32_t* dense) {
    double b = (double)per_level_scale;
    if (finest > 0u && n_levels > 1u) b = exp(log((double)finest / (double)base) / (double)(n_levels - 1u));
    const uint64_t T = 1ull << log2_table_size;
    for (uint32_t l = 0; l < n_levels; ++l) {
        const double nl   = floor((double)base * pow(b, (double)l) + 1e-9);
        resolution[l]     = (uint32_t)nl;
        const uint64_t v  = (uint64_t)resolution[l] + 1ull;
        dense[l]          = (v * v * v <= T) ? 1u : 0u;
    }
}

static inline float table_value(const OrcGrid& g, const void* table, uint32_t level, uint32_t idx, uint32_t f) {
    const uint64_t off = ((uint64_t)level * g.table_size + idx) * g.n_features + f;
    if (g.table_dtype == 0u) return ((const float*)table)[off];
    return orc_f16_to_f32(((const uint16_t*)table)[off]);
}

static void encode_point(const OrcGrid& g, const void* table, const float* p, float* feat, uint32_t* idx_out, float* w_out) {
    for (uint32_t l = 0; l < g.n_levels; ++l) {
        const uint32_t N = g.resolution[l];
        const float s    = (float)N;
        uint32_t i0[3];
        float w[3];
        for (int a = 0; a < 3; ++a) {
            const float x   = fminf(fmaxf(p[a], 0.0f), 1.0f);
            const float pos = x * s;
            uint32_t c      = (uint32_t)floorf(pos);
            if (c >= N) c = N - 1u;
            i0[a] = c;
            w[a]  = pos - (float)c;
        }
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (uint32_t c = 0; c < 8u; ++c) {
            const uint32_t cx = i0[0] + (c & 1u);
            const uint32_t cy = i0[1] + ((c >> 1) & 1u);
            const uint32_t cz = i0[2] + ((c >> 2) & 1u);
            uint32_t idx;
            if (g.dense[l]) {
                const uint32_t stride = N + 1u;
                idx                   = cx + cy * stride + cz * stride * stride;
            } else {
                idx = ((cx * 1u) ^ (cy * 2654435761u) ^ (cz * 805459861u)) & (g.table_size - 1u);
            }
            const float wx     = (c & 1u) ? w[0] : 1.0f - w[0];
            const float wy     = (c & 2u) ? w[1] : 1.0f - w[1];
            const float wz     = (c & 4u) ? w[2] : 1.0f - w[2];
            const float weight = (wx * wy) * wz;
            if (idx_out) idx_out[l * 8u + c] = idx;
            if (w_out) w_out[l * 8u + c] = weight;
            for (uint32_t f = 0; f < g.n_features; ++f) acc[f] += weight * table_value(g, table, l, idx, f);
        }
        for (uint32_t f = 0; f < g.n_features; ++f) feat[l * g.n_features + f] = acc[f];
    }
}

// features: [n][L*F] f32; optional indices/weights: [n][L][8].
extern "C" void orc_encode(const OrcGrid* g, const void* table, const float* pos, uint32_t n, float* features, uint32_t* indices, float* weights) {
    const uint32_t width = g->n_levels * g->n_features;
    for (uint32_t i = 0; i < n; ++i)
        encode_point(*g, table, pos + 3ull * i, features + (uint64_t)i * width, indices ? indices + (uint64_t)i * g->n_levels * 8u : nullptr,
            weights ? weights + (uint64_t)i * g->n_levels * 8u : nullptr);
}

// ---------------------------------------------------------------------------
// MLPs: no biases, ReLU hidden layers, W row-major [out][in] (backend-cuda.cu
// :668-783 semantics), fp16 operands and fp16-rounded hidden activations,
// accumulation carried in fp64 and rounded once to fp32.
// ---------------------------------------------------------------------------
static void matvec(const uint16_t* W, uint32_t n_out, uint32_t n_in, const float* x, float* y) {
    for (uint32_t o = 0; o < n_out; ++o) {
        double acc = 0.0;
        for (uint32_t k = 0; k < n_in; ++k) acc += (double)orc_f16_to_f32(W[(uint64_t)o * n_in + k]) * (double)x[k];
        y[o] = (float)acc;
    }
}

// Density network 32 -> 64 -> 16 on one feature row; out16 = raw outputs.
static void density_row(const uint16_t* params, const float* feat32, float* out16) {
    float x[32], h[64];
    for (int k = 0; k < 32; ++k) x[k] = r16(feat32[k]);
    matvec(params, 64, 32, x, h);
    for (int k = 0; k < 64; ++k) h[k] = r16(fmaxf(h[k], 0.0f));
    matvec(params + 2048, 16, 64, h, out16);
}

// Real spherical harmonics, bands 0..3 (16 values) with the Condon-Shortley
// phase, of a unit direction (Sloan, "Stupid Spherical Harmonics Tricks", 2008).
extern "C" void orc_sh4(const float* d, float* out) {
    const float x = d[0], y = d[1], z = d[2];
    const float xy = x * y, yz = y * z, xz = x * z;
    const float x2 = x * x, y2 = y * y, z2 = z * z;
    out[0]  = 0.28209479177387814f;
    out[1]  = -0.48860251190291987f * y;
    out[2]  = 0.48860251190291987f * z;
    out[3]  = -0.48860251190291987f * x;
    out[4]  = 1.0925484305920792f * xy;
    out[5]  = -1.0925484305920792f * yz;
    out[6]  = 0.94617469575755997f * z2 - 0.31539156525251999f;
    out[7]  = -1.0925484305920792f * xz;
    out[8]  = 0.54627421529603959f * (x2 - y2);
    out[9]  = 0.59004358992664352f * y * (3.0f * x2 - y2) * -1.0f;
    out[10] = 2.8906114426405538f * xy * z;
    out[11] = 0.45704579946446572f * y * (1.0f - 5.0f * z2);
    out[12] = 0.3731763325901154f * z * (5.0f * z2 - 3.0f);
    out[13] = 0.45704579946446572f * x * (1.0f - 5.0f * z2);
    out[14] = 1.4453057213202769f * z * (x2 - y2);
    out[15] = 0.59004358992664352f * x * (3.0f * y2 - x2);
}

// Colour network [geo 15 | SH 16 | 0] -> 64 -> 64 -> 16 (3 used), sigmoid.
static void color_row(const uint16_t* params, const float* dens_out16, const float* dir, float* rgb) {
    float sh[16], x[32], h1[64], h2[64], o[16];
    orc_sh4(dir, sh);
    for (int k = 0; k < 15; ++k) x[k] = r16(dens_out16[1 + k]);
    for (int k = 0; k < 16; ++k) x[15 + k] = r16(sh[k]);
    x[31] = 0.0f;
    matvec(params, 64, 32, x, h1);
    for (int k = 0; k < 64; ++k) h1[k] = r16(fmaxf(h1[k], 0.0f));
    matvec(params + 2048, 64, 64, h1, h2);
    for (int k = 0; k < 64; ++k) h2[k] = r16(fmaxf(h2[k], 0.0f));
    matvec(params + 2048 + 4096, 16, 64, h2, o);
    for (int c = 0; c < 3; ++c) rgb[c] = 1.0f / (1.0f + expf(-o[c]));
}

// Density MLP on given features (rounded to fp16 inside): raw outputs [n][16].
extern "C" void orc_density_mlp(const uint16_t* params, const float* features, uint32_t n, float* out) {
    for (uint32_t i = 0; i < n; ++i) density_row(params, features + 32ull * i, out + 16ull * i);
}

// Config-1 pipeline: encode -> density MLP -> exp on channel 0.  out [n][16].
extern "C" void orc_density_forward(const OrcGrid* g, const void* table, const uint16_t* params, const float* pos, uint32_t n, float* out) {
    float feat[32];
    for (uint32_t i = 0; i < n; ++i) {
        encode_point(*g, table, pos + 3ull * i, feat, nullptr, nullptr);
        float* o = out + 16ull * i;
        density_row(params, feat, o);
        o[0] = expf(o[0]);
    }
}

// Full field: out [n][4] = (sigma = exp(raw), r, g, b).
static void field_point(const OrcGrid& g, const void* table, const uint16_t* dparams, const uint16_t* cparams, const float* p, const float* d, float* out4) {
    float feat[32], o[16], rgb[3];
    encode_point(g, table, p, feat, nullptr, nullptr);
    density_row(dparams, feat, o);
    color_row(cparams, o, d, rgb);
    out4[0] = expf(o[0]);
    out4[1] = rgb[0];
    out4[2] = rgb[1];
    out4[3] = rgb[2];
}

extern "C" void orc_field_forward(const OrcGrid* g, const void* table, const uint16_t* dparams, const uint16_t* cparams, const float* pos, const float* dirs, uint32_t n, float* out) {
    for (uint32_t i = 0; i < n; ++i) field_point(*g, table, dparams, cparams, pos + 3ull * i, dirs + 3ull * i, out + 4ull * i);
}

// ---------------------------------------------------------------------------
// Analytic Gaussian scene: density(p) = sum_g A_g exp(k_g |p - c_g|^2) with
// k_g = -0.5 / sigma_g^2.  Record per Gaussian: cx cy cz sigma A r g b.
// ---------------------------------------------------------------------------
extern "C" float orc_det_expf(float x) { return nerf_math::det_expf(x); }
extern "C" void orc_det_expf_array(const float* x, uint64_t n, float* out) {
    for (uint64_t i = 0; i < n; ++i) out[i] = nerf_math::det_expf(x[i]);
}

static inline float scene_density(const float* gs, uint32_t count, const float* p) {
    float acc = 0.0f;
    for (uint32_t i = 0; i < count; ++i) {
        const float* g = gs + 8ull * i;
        const float dx = p[0] - g[0];
        const float dy = p[1] - g[1];
        const float dz = p[2] - g[2];
        const float d2 = (dx * dx + dy * dy) + dz * dz;
        const float k  = -0.5f / (g[3] * g[3]);
        acc            = acc + g[4] * nerf_math::det_expf(d2 * k);
    }
    return acc;
}

extern "C" void orc_scene_density(const float* gs, uint32_t count, const float* pos, uint32_t n, float* out) {
    for (uint32_t i = 0; i < n; ++i) out[i] = scene_density(gs, count, pos + 3ull * i);
}

// ---------------------------------------------------------------------------
// Occupancy grid over one box or nested cascades: cascade 0 is the box,
// cascade c > 0 the box scaled by 2^c about its centre (centre -/+ half * 2^c,
// fp32); a point belongs to the first cascade whose box holds it, and to the
// cell min(res - 1, floor(r * res)) of r = (p - lo) / (hi - lo) there
// (backend-cuda.cu:338-351 within one box).  Cascade c occupies words
// [c W, (c + 1) W), W = ceil(res^3 / 32).
// ---------------------------------------------------------------------------
struct OrcOcc {
    const uint32_t* bits;
    uint32_t res, cascades, words;
    float bmin[3], bmax[3], omin[3], omax[3];
};

static void occ_box(const OrcOcc& o, uint32_t c, float* lo, float* hi) {
    for (int a = 0; a < 3; ++a) {
        if (c == 0u) {
            lo[a] = o.bmin[a];
            hi[a] = o.bmax[a];
        } else {
            const float centre = 0.5f * (o.bmin[a] + o.bmax[a]);
            const float half   = 0.5f * (o.bmax[a] - o.bmin[a]);
            const float sc     = (float)(1u << c);
            lo[a]              = centre - half * sc;
            hi[a]              = centre + half * sc;
        }
    }
}

static OrcOcc make_occ(const uint32_t* bits, uint32_t res, uint32_t cascades, const float* aabb) {
    OrcOcc o;
    o.bits     = bits;
    o.res      = res;
    o.cascades = cascades == 0u ? 1u : cascades;
    o.words    = (uint32_t)(((uint64_t)res * res * res + 31u) / 32u);
    for (int a = 0; a < 3; ++a) {
        o.bmin[a] = aabb[a];
        o.bmax[a] = aabb[3 + a];
    }
    occ_box(o, o.cascades - 1u, o.omin, o.omax);
    return o;
}

static const uint32_t kOrcOutside = 0xFFFFFFFFu;

static uint32_t occ_cell(const OrcOcc& o, const float* p) {
    for (uint32_t c = 0; c < o.cascades; ++c) {
        float lo[3], hi[3];
        occ_box(o, c, lo, hi);
        const float rx = (p[0] - lo[0]) / (hi[0] - lo[0]);
        const float ry = (p[1] - lo[1]) / (hi[1] - lo[1]);
        const float rz = (p[2] - lo[2]) / (hi[2] - lo[2]);
        if (rx < 0.0f || rx >= 1.0f || ry < 0.0f || ry >= 1.0f || rz < 0.0f || rz >= 1.0f) continue;
        const uint32_t ix = std::min(o.res - 1u, (uint32_t)(rx * (float)o.res));
        const uint32_t iy = std::min(o.res - 1u, (uint32_t)(ry * (float)o.res));
        const uint32_t iz = std::min(o.res - 1u, (uint32_t)(rz * (float)o.res));
        return c * 32u * o.words + ix + iy * o.res + iz * o.res * o.res;
    }
    return kOrcOutside;
}

// A null bitfield marks every cell of every cascade occupied.
static bool occ_occupied(const OrcOcc& o, const float* p) {
    const uint32_t idx = occ_cell(o, p);
    if (idx == kOrcOutside) return false;
    return !o.bits || (o.bits[idx >> 5] & (1u << (idx & 31u))) != 0u;
}

// Cell index (as above) of each point; kOrcOutside outside every cascade.
extern "C" void orc_occ_cell(uint32_t res, uint32_t cascades, const float* aabb, const float* pos, uint32_t n, uint32_t* out) {
    const OrcOcc o = make_occ(nullptr, res, cascades, aabb);
    for (uint32_t i = 0; i < n; ++i) out[i] = occ_cell(o, pos + 3ull * i);
}

// Centre of cell (x, y, z) of cascade c: lo + (i + 0.5) * ((hi - lo) / res).
static void cell_centre(const OrcOcc& o, uint32_t c, uint64_t cell, float* p) {
    const uint64_t rr = (uint64_t)o.res * o.res;
    const uint32_t z  = (uint32_t)(cell / rr);
    const uint32_t r  = (uint32_t)(cell - (uint64_t)z * rr);
    const uint32_t y  = r / o.res;
    const uint32_t x  = r - y * o.res;
    float lo[3], hi[3];
    occ_box(o, c, lo, hi);
    const float step[3] = {(hi[0] - lo[0]) / (float)o.res, (hi[1] - lo[1]) / (float)o.res, (hi[2] - lo[2]) / (float)o.res};
    p[0] = lo[0] + ((float)x + 0.5f) * step[0];
    p[1] = lo[1] + ((float)y + 0.5f) * step[1];
    p[2] = lo[2] + ((float)z + 0.5f) * step[2];
}

// Bit (x + y*res + z*res^2) of cascade c is set iff density(cell centre) >
// threshold (backend-cuda.cu :1607-1608 cell centres, :1632-1633 strict
// threshold, :347-350 packing).  bits: cascades * W words.
extern "C" void orc_occupancy_from_scene(const float* gs, uint32_t count, uint32_t res, uint32_t cascades, const float* aabb, float threshold, uint32_t* bits) {
    const OrcOcc o       = make_occ(nullptr, res, cascades, aabb);
    const uint64_t cells = (uint64_t)res * res * res;
    memset(bits, 0, (uint64_t)o.cascades * o.words * 4u);
    for (uint32_t c = 0; c < o.cascades; ++c) {
        uint32_t* w = bits + (uint64_t)c * o.words;
        for (uint64_t k = 0; k < cells; ++k) {
            float p[3];
            cell_centre(o, c, k, p);
            if (scene_density(gs, count, p) > threshold) w[k >> 5] |= 1u << (k & 31u);
        }
    }
}

// Uniform background shell: ORs the bit of every cell (every cascade) whose
// centre q has r_inner^2 <= |q - centre|^2 <= r_outer^2.
extern "C" void orc_occupancy_mark_shell(uint32_t res, uint32_t cascades, const float* aabb, const float* centre, float r_inner, float r_outer, uint32_t* bits) {
    const OrcOcc o       = make_occ(nullptr, res, cascades, aabb);
    const uint64_t cells = (uint64_t)res * res * res;
    const float r2i = r_inner * r_inner, r2o = r_outer * r_outer;
    for (uint32_t c = 0; c < o.cascades; ++c) {
        uint32_t* w = bits + (uint64_t)c * o.words;
        for (uint64_t k = 0; k < cells; ++k) {
            float p[3];
            cell_centre(o, c, k, p);
            const float dx = p[0] - centre[0], dy = p[1] - centre[1], dz = p[2] - centre[2];
            const float d2 = (dx * dx + dy * dy) + dz * dz;
            if (d2 >= r2i && d2 <= r2o) w[k >> 5] |= 1u << (k & 31u);
        }
    }
}

// ---------------------------------------------------------------------------
// Cameras, rays, AABB and occupancy march.
// ---------------------------------------------------------------------------
struct OrcCamera {
    float c2w[12];  // rows 0..2 of the row-major camera-to-world matrix
    float fx, fy, cx, cy;
    uint32_t width, height;
};

struct OrcRay {
    float o[3], d[3], tn, tf;
};

// backend-cuda.cu:373-390 (ray direction; 1/sqrtf instead of rsqrtf) and
// :391-408 (slab test).
static bool make_ray(const OrcCamera& c, float px, float py_flipped, const float* lo, const float* hi, OrcRay& r) {
    const float dcx = (px - c.cx) / c.fx;
    const float dcy = (py_flipped - c.cy) / c.fy;
    const float dcz = -1.0f;
    float d[3];
    for (int a = 0; a < 3; ++a) d[a] = c.c2w[4 * a + 0] * dcx + c.c2w[4 * a + 1] * dcy + c.c2w[4 * a + 2] * dcz;
    const float len2 = d[0] * d[0] + d[1] * d[1] + d[2] * d[2];
    if (len2 <= 1e-16f) return false;
    const float inv = 1.0f / sqrtf(len2);
    for (int a = 0; a < 3; ++a) {
        r.d[a] = d[a] * inv;
        r.o[a] = c.c2w[4 * a + 3];
    }
    float tmin = -INFINITY, tmax = INFINITY;
    float tmins[3], tmaxs[3];
    for (int a = 0; a < 3; ++a) {
        const float inv_d = fabsf(r.d[a]) > 1e-8f ? 1.0f / r.d[a] : (r.d[a] >= 0.0f ? 1e8f : -1e8f);
        const float t0    = (lo[a] - r.o[a]) * inv_d;
        const float t1    = (hi[a] - r.o[a]) * inv_d;
        tmins[a]          = fminf(t0, t1);
        tmaxs[a]          = fmaxf(t0, t1);
    }
    tmin = fmaxf(fmaxf(tmins[0], tmins[1]), tmins[2]);
    tmax = fminf(fminf(tmaxs[0], tmaxs[1]), tmaxs[2]);
    if (!(tmin <= tmax && tmax > 0.0f)) return false;
    if (tmin < 0.0f) tmin = 0.0f;
    r.tn = tmin;
    r.tf = tmax;
    return true;
}

// Inference ray of pixel (x, y): pixel centre, y flipped (backend-cuda.cu:561-563).
static bool pixel_ray(const OrcCamera& c, uint32_t x, uint32_t y, const float* lo, const float* hi, OrcRay& r) {
    const float px = (float)x + 0.5f;
    const float py = (float)y + 0.5f;
    return make_ray(c, px, (float)c.height - 1.0f - py, lo, hi, r);
}

// March of backend-cuda.cu:448-469; emit(t_mid, dt) for occupied steps.
template <typename Emit>
static uint32_t march(const OrcCamera& c, const OrcRay& r, const OrcOcc& occ, uint32_t max_steps, Emit emit) {
    const float t_range = r.tf - r.tn;
    if (!(t_range > 0.0f)) return 0u;
    const float dt_min = t_range / (float)max_steps;
    const float ifx    = c.fx > 0.0f ? 1.0f / c.fx : 0.0f;
    const float ify    = c.fy > 0.0f ? 1.0f / c.fy : 0.0f;
    const float cone   = 0.5f * (ifx + ify);
    uint32_t count = 0, i = 0;
    float t = r.tn;
    while (t < r.tf && i < max_steps) {
        const float dt    = fminf(fmaxf(dt_min, t * cone), r.tf - t);
        const float tm    = t + 0.5f * dt;
        const float p[3]  = {r.o[0] + tm * r.d[0], r.o[1] + tm * r.d[1], r.o[2] + tm * r.d[2]};
        if (occ_occupied(occ, p)) {
            emit(count, tm, dt);
            ++count;
        }
        t += dt;
        ++i;
    }
    return count;
}

// Per-ray occupied-sample counts for rays [ray_begin, ray_begin + n) of one
// view; rays are clipped to the outermost cascade's box.
extern "C" void orc_march_count(const OrcCamera* cam, const uint32_t* bits, uint32_t res, uint32_t cascades, const float* aabb, uint32_t max_steps, uint32_t ray_begin, uint32_t n, uint32_t* counts) {
    const OrcOcc occ = make_occ(bits, res, cascades, aabb);
    for (uint32_t k = 0; k < n; ++k) {
        const uint32_t ray = ray_begin + k;
        OrcRay r;
        counts[k] = 0u;
        if (!pixel_ray(*cam, ray % cam->width, ray / cam->width, occ.omin, occ.omax, r)) continue;
        counts[k] = march(*cam, r, occ, max_steps, [](uint32_t, float, float) {});
    }
}

// Samples (t_mid, dt) of one ray, up to cap; returns the count.
extern "C" uint32_t orc_march_ray(const OrcCamera* cam, const uint32_t* bits, uint32_t res, uint32_t cascades, const float* aabb, uint32_t max_steps, uint32_t ray, float* t_dt, uint32_t cap) {
    const OrcOcc occ = make_occ(bits, res, cascades, aabb);
    OrcRay r;
    if (!pixel_ray(*cam, ray % cam->width, ray / cam->width, occ.omin, occ.omax, r)) return 0u;
    return march(*cam, r, occ, max_steps, [&](uint32_t k, float tm, float dt) {
        if (k < cap) {
            t_dt[2 * k]     = tm;
            t_dt[2 * k + 1] = dt;
        }
    });
}

// Ray origin/direction/t-range of one pixel ray against a box; returns 0 if
// it misses.
extern "C" int orc_pixel_ray(const OrcCamera* cam, uint32_t ray, const float* aabb, float* out8) {
    OrcRay r;
    if (!pixel_ray(*cam, ray % cam->width, ray / cam->width, aabb, aabb + 3, r)) return 0;
    for (int a = 0; a < 3; ++a) {
        out8[a]     = r.o[a];
        out8[3 + a] = r.d[a];
    }
    out8[6] = r.tn;
    out8[7] = r.tf;
    return 1;
}

// ---------------------------------------------------------------------------
// Composite (backend-cuda.cu:601-635) with early stop: after sample i updates
// T, stop when T < t_stop.  Background bg added as C + T * bg; clamp; RGBA8 by
// round-to-nearest-even of x * 255 (:628-634).
// ---------------------------------------------------------------------------
static uint32_t pack_rgba8(const float* rgb) {
    uint32_t u[3];
    for (int c = 0; c < 3; ++c) u[c] = (uint32_t)nearbyintf(fminf(1.0f, fmaxf(0.0f, rgb[c])) * 255.0f);
    return (255u << 24) | (u[2] << 16) | (u[1] << 8) | u[0];
}

// sigma_rgb: [count][4]; dt: [count].  Writes rgb[3]; returns samples used.
extern "C" uint32_t orc_composite_ray(const float* sigma_rgb, const float* dt, uint32_t count, float t_stop, const float* bg, float* rgb_out, uint32_t* rgba8_out) {
    float T = 1.0f, C[3] = {0, 0, 0};
    uint32_t used = 0;
    for (uint32_t i = 0; i < count; ++i) {
        const float a = 1.0f - expf(-(sigma_rgb[4 * i] * fmaxf(dt[i], 0.0f)));
        const float w = T * a;
        for (int c = 0; c < 3; ++c) C[c] += w * sigma_rgb[4 * i + 1 + c];
        T *= 1.0f - a;
        ++used;
        if (T < t_stop) break;
    }
    for (int c = 0; c < 3; ++c) rgb_out[c] = C[c] + T * bg[c];
    if (rgba8_out) *rgba8_out = pack_rgba8(rgb_out);
    return used;
}

// ---------------------------------------------------------------------------
// Whole render of a list of rays of one view: march -> field -> composite.
// Rays are split statically over n_threads std::threads.
// ---------------------------------------------------------------------------
struct OrcModel {
    OrcGrid grid;
    const void* table;
    const uint16_t* density_params;
    const uint16_t* color_params;
    uint32_t kind;  // 0 hash grid, 1 the reference's own network (world positions)
};

static void ref_field_point(const uint16_t* dp, const uint16_t* cp, const float* p, const float* d, float* out4, float* raw4);

// The field sees positions normalised to the outermost cascade's box,
// (w - lo) / (hi - lo) per axis (exact for the unit box).
// Optional per-ray outputs of the early stop: used_out = samples composited
// (the sample after which T < t_stop is the last one, :601-635 plus the
// stop), t_prev_out = T before the last composited sample, t_final_out = T
// after it.
extern "C" void orc_render_rays(const OrcModel* model, const OrcCamera* cam, const uint32_t* bits, uint32_t res, uint32_t cascades, const float* aabb, uint32_t max_steps, float t_stop, const float* bg, const uint32_t* rays, uint32_t n_rays,
    float* rgb_out, uint32_t* rgba8_out, uint32_t* counts_out, uint32_t n_threads, uint32_t* used_out, float* t_prev_out, float* t_final_out) {
    if (n_threads == 0u) n_threads = 1u;
    const OrcOcc occ = make_occ(bits, res, cascades, aabb);
    auto work = [&](uint32_t begin, uint32_t end) {
        std::vector<float> t_dt, sig, dts;
        for (uint32_t k = begin; k < end; ++k) {
            const uint32_t ray = rays[k];
            OrcRay r;
            uint32_t count = 0;
            t_dt.clear();
            if (pixel_ray(*cam, ray % cam->width, ray / cam->width, occ.omin, occ.omax, r)) {
                count = march(*cam, r, occ, max_steps, [&](uint32_t, float tm, float dt) {
                    t_dt.push_back(tm);
                    t_dt.push_back(dt);
                });
            }
            float T = 1.0f, T_prev = 1.0f, C[3] = {0, 0, 0};
            uint32_t used = 0;
            for (uint32_t i = 0; i < count; ++i) {
                const float tm   = t_dt[2 * i];
                const float dt   = t_dt[2 * i + 1];
                const float wp[3] = {r.o[0] + tm * r.d[0], r.o[1] + tm * r.d[1], r.o[2] + tm * r.d[2]};
                float p[3];
                for (int a = 0; a < 3; ++a) p[a] = (wp[a] - occ.omin[a]) / (occ.omax[a] - occ.omin[a]);
                float s4[4];
                if (model->kind == 1u) ref_field_point(model->density_params, model->color_params, wp, r.d, s4, nullptr);
                else field_point(model->grid, model->table, model->density_params, model->color_params, p, r.d, s4);
                const float a = 1.0f - expf(-(s4[0] * fmaxf(dt, 0.0f)));
                const float w = T * a;
                for (int c = 0; c < 3; ++c) C[c] += w * s4[1 + c];
                T_prev = T;
                T *= 1.0f - a;
                ++used;
                if (T < t_stop) break;
            }
            if (used_out) used_out[k] = used;
            if (t_prev_out) t_prev_out[k] = T_prev;
            if (t_final_out) t_final_out[k] = T;
            float rgb[3];
            for (int c = 0; c < 3; ++c) rgb[c] = C[c] + T * bg[c];
            if (rgb_out)
                for (int c = 0; c < 3; ++c) rgb_out[3ull * k + c] = rgb[c];
            if (rgba8_out) rgba8_out[k] = pack_rgba8(rgb);
            if (counts_out) counts_out[k] = count;
        }
    };
    std::vector<std::thread> pool;
    const uint32_t chunk = (n_rays + n_threads - 1u) / n_threads;
    for (uint32_t t = 0; t < n_threads; ++t) {
        const uint32_t b = t * chunk, e = std::min(n_rays, b + chunk);
        if (b >= e) break;
        pool.emplace_back(work, b, e);
    }
    for (auto& th : pool) th.join();
}


// Inference with the reference's sampling (backend-cuda.cu:534-600): the
// pixel-centre ray (y flipped, :561-563) clipped to the box; dt = (t_far -
// t_near) / spp; no samples when the ray misses the box or dt is not
// positive (:570-583), else spp samples at t_mid = t_near + (i + 0.5) dt,
// position o + t_mid d (:585-599).  Composite of :601-635 over every sample
// (no early stop): alpha = 1 - exp(-sigma max(dt, 0)), w = T alpha,
// C += w c, T *= 1 - alpha; output C + T bg, clamped, rounded to RGBA8.
// The field is the model's: the hash grid reads positions normalised by the
// box, the reference's network world positions.
extern "C" void orc_render_uniform(const OrcModel* model, const OrcCamera* cam, const float* aabb, uint32_t spp, const float* bg, const uint32_t* rays, uint32_t n_rays, float* rgb_out, uint32_t* rgba8_out,
                                   uint32_t* counts_out, uint32_t n_threads) {
    if (n_threads == 0u) n_threads = 1u;
    auto work = [&](uint32_t begin, uint32_t end) {
        for (uint32_t k = begin; k < end; ++k) {
            const uint32_t ray = rays[k];
            OrcRay r;
            uint32_t count = 0;
            float dt       = 0.0f;
            if (pixel_ray(*cam, ray % cam->width, ray / cam->width, aabb, aabb + 3, r)) {
                dt = (r.tf - r.tn) / (float)spp;
                if (dt > 0.0f) count = spp;
            }
            float T = 1.0f, Cc[3] = {0, 0, 0};
            for (uint32_t i = 0; i < count; ++i) {
                const float tm    = r.tn + ((float)i + 0.5f) * dt;
                const float wp[3] = {r.o[0] + tm * r.d[0], r.o[1] + tm * r.d[1], r.o[2] + tm * r.d[2]};
                float s4[4];
                if (model->kind == 1u) {
                    ref_field_point(model->density_params, model->color_params, wp, r.d, s4, nullptr);
                } else {
                    float p[3];
                    for (int a = 0; a < 3; ++a) p[a] = (wp[a] - aabb[a]) / (aabb[3 + a] - aabb[a]);
                    field_point(model->grid, model->table, model->density_params, model->color_params, p, r.d, s4);
                }
                const float a = 1.0f - expf(-(s4[0] * fmaxf(dt, 0.0f)));
                const float w = T * a;
                for (int c = 0; c < 3; ++c) Cc[c] += w * s4[1 + c];
                T *= 1.0f - a;
            }
            float rgb[3];
            for (int c = 0; c < 3; ++c) rgb[c] = Cc[c] + T * bg[c];
            if (rgb_out)
                for (int c = 0; c < 3; ++c) rgb_out[3ull * k + c] = rgb[c];
            if (rgba8_out) rgba8_out[k] = pack_rgba8(rgb);
            if (counts_out) counts_out[k] = count;
        }
    };
    std::vector<std::thread> pool;
    const uint32_t chunk = (n_rays + n_threads - 1u) / n_threads;
    for (uint32_t t = 0; t < n_threads; ++t) {
        const uint32_t b = t * chunk, e = std::min(n_rays, b + chunk);
        if (b >= e) break;
        pool.emplace_back(work, b, e);
    }
    for (auto& th : pool) th.join();
}

// ===========================================================================
// Training: composite backward with Huber loss, MLP backward, hash-grid
// scatter-add, Adam.
// ===========================================================================

// Huber loss of x with threshold delta (Huber 1964): 0.5 x^2 for |x| <= delta,
// delta (|x| - delta / 2) otherwise; derivative clamp(x, -delta, delta).
static inline double huber(double x, double d) { return fabs(x) <= d ? 0.5 * x * x : d * (fabs(x) - 0.5 * d); }

// Forward + backward of front-to-back compositing for one ray (reference
// backend-cuda.cu:1095-1182 generalised to exp density, Huber loss and a
// background colour).  sigma = exp(raw), c = sigmoid(raw_rgb),
// alpha_i = 1 - exp(-sigma_i max(dt_i, 0)), T_{i+1} = T_i (1 - alpha_i),
// pred = sum_i T_i alpha_i c_i + T_n bg.  Loss = inv_norm * sum_c huber(pred_c
// - gt_c).  Gradients wrt the raw network outputs, with the suffix
// S_i = sum_{j>i} w_j c_j + T_n bg (:1140-1170):
//   d raw_rgb_ic   = w_i g_c c_ic (1 - c_ic)
//   d raw_sigma_i  = dt_i sigma_i sum_c g_c (T_{i+1} c_ic - S_ic)
// (the reference's T_i c - S / (1 - alpha) times d alpha / d raw =
// dt sigma (1 - alpha)).  Evaluated in fp64; returns the un-normalised loss.
static double composite_backward_core(const std::vector<double>& sig, const std::vector<double>& c, const float* dt, uint32_t n, const float* gt, const float* bg, float delta, float inv_norm, float* dsraw, float* drgbraw,
                                      float* pred_out) {
    std::vector<double> a(n), T(n + 1);
    T[0] = 1.0;
    double pred[3] = {0, 0, 0};
    for (uint32_t i = 0; i < n; ++i) {
        const double dti = dt[i] > 0.0f ? (double)dt[i] : 0.0;
        a[i]             = 1.0 - exp(-sig[i] * dti);
        for (int k = 0; k < 3; ++k) pred[k] += T[i] * a[i] * c[3 * i + k];
        T[i + 1] = T[i] * (1.0 - a[i]);
    }
    double loss = 0.0, g[3];
    for (int k = 0; k < 3; ++k) {
        pred[k] += T[n] * bg[k];
        const double x = pred[k] - gt[k];
        loss += huber(x, delta);
        g[k] = (x > delta ? delta : (x < -delta ? -delta : x)) * inv_norm;
        if (pred_out) pred_out[k] = (float)pred[k];
    }
    double S[3] = {T[n] * bg[0], T[n] * bg[1], T[n] * bg[2]};
    for (int i = (int)n - 1; i >= 0; --i) {
        const double dti = dt[i] > 0.0f ? (double)dt[i] : 0.0;
        const double w   = T[i] * a[i];
        double ds        = 0.0;
        for (int k = 0; k < 3; ++k) {
            const double ci    = c[3 * i + k];
            drgbraw[3 * i + k] = (float)(w * g[k] * ci * (1.0 - ci));
            ds += g[k] * (T[i + 1] * ci - S[k]);
            S[k] += w * ci;
        }
        dsraw[i] = (float)(dti * sig[i] * ds);
    }
    return loss;
}

extern "C" double orc_composite_backward_ray(const float* sraw, const float* rgbraw, const float* dt, uint32_t n, const float* gt, const float* bg, float delta, float inv_norm, float* dsraw, float* drgbraw, float* pred_out) {
    std::vector<double> sig(n), c(3 * (size_t)n);
    for (uint32_t i = 0; i < n; ++i) {
        sig[i] = exp((double)sraw[i]);
        for (int k = 0; k < 3; ++k) c[3 * i + k] = 1.0 / (1.0 + exp(-(double)rgbraw[3 * i + k]));
    }
    return composite_backward_core(sig, c, dt, n, gt, bg, delta, inv_norm, dsraw, drgbraw, pred_out);
}

// The same with the activations given (sigma, rgb in [0, 1]) instead of raw
// outputs; gradients are still with respect to the raw outputs.
extern "C" double orc_composite_backward_act(const float* sigma, const float* rgb, const float* dt, uint32_t n, const float* gt, const float* bg, float delta, float inv_norm, float* dsraw, float* drgbraw, float* pred_out) {
    std::vector<double> sig(n), c(3 * (size_t)n);
    for (uint32_t i = 0; i < n; ++i) {
        sig[i] = (double)sigma[i];
        for (int k = 0; k < 3; ++k) c[3 * i + k] = (double)rgb[3 * i + k];
    }
    return composite_backward_core(sig, c, dt, n, gt, bg, delta, inv_norm, dsraw, drgbraw, pred_out);
}

// MLP backward for n samples with the GPU's fp16 rounding points.
// Inputs: features [n][32] (fp16 values), directions [n][3], upstream
// d_sigma_raw [n] and d_rgb_raw [n][3], loss_scale.  Forward activations are
// recomputed exactly as in density_row / color_row.  Deltas are scaled by
// loss_scale and rounded to fp16 where the GPU feeds them to MFMA:
//   do3 = f16(ls * d_rgb_raw) (rows 0..2), dh2 = f16(mask(h2) C3^T do3),
//   dh1 = f16(mask(h1) C2^T dh2), dgeo = (C1^T dh1)[geo],
//   do = f16(ls * d_sigma_raw | dgeo), dhd = f16(mask(hd) D2^T do),
//   dfeat = D1^T dhd (fp32, still scaled by ls).
// Weight gradients (scaled by ls) accumulate in fp64: dW = sum delta (x) act.
// Layouts of dD (3072) and dC (7168) follow the parameter packing.
extern "C" void orc_mlp_backward(const uint16_t* dp, const uint16_t* cp, const float* features, const float* dirs, const float* dsraw, const float* drgbraw, uint32_t n, float loss_scale, float* dfeat, double* dD, double* dC) {
    auto W = [](const uint16_t* P, uint32_t off, uint32_t n_in, uint32_t o, uint32_t k) { return (double)orc_f16_to_f32(P[off + o * n_in + k]); };
    for (uint32_t s = 0; s < n; ++s) {
        float x[32], hd[64], o[16], xc[32], h1[64], h2[64], sh[16];
        for (int k = 0; k < 32; ++k) x[k] = r16(features[32ull * s + k]);
        matvec(dp, 64, 32, x, hd);
        for (int k = 0; k < 64; ++k) hd[k] = r16(fmaxf(hd[k], 0.0f));
        matvec(dp + 2048, 16, 64, hd, o);
        orc_sh4(dirs + 3ull * s, sh);
        for (int k = 0; k < 15; ++k) xc[k] = r16(o[1 + k]);
        for (int k = 0; k < 16; ++k) xc[15 + k] = r16(sh[k]);
        xc[31] = 0.0f;
        matvec(cp, 64, 32, xc, h1);
        for (int k = 0; k < 64; ++k) h1[k] = r16(fmaxf(h1[k], 0.0f));
        matvec(cp + 2048, 64, 64, h1, h2);
        for (int k = 0; k < 64; ++k) h2[k] = r16(fmaxf(h2[k], 0.0f));
        // colour backward
        float do3[16] = {0};
        for (int c = 0; c < 3; ++c) do3[c] = r16(loss_scale * drgbraw[3ull * s + c]);
        float dh2[64], dh1[64];
        for (int k = 0; k < 64; ++k) {
            double acc = 0.0;
            for (int q = 0; q < 16; ++q) acc += W(cp, 6144, 64, q, k) * do3[q];
            dh2[k] = h2[k] > 0.0f ? r16((float)acc) : 0.0f;
        }
        for (int k = 0; k < 64; ++k) {
            double acc = 0.0;
            for (int q = 0; q < 64; ++q) acc += W(cp, 2048, 64, q, k) * dh2[q];
            dh1[k] = h1[k] > 0.0f ? r16((float)acc) : 0.0f;
        }
        float dgeo[15];
        for (int k = 0; k < 15; ++k) {
            double acc = 0.0;
            for (int q = 0; q < 64; ++q) acc += W(cp, 0, 32, q, k) * dh1[q];
            dgeo[k] = (float)acc;
        }
        // density backward
        float dout[16];
        dout[0] = r16(loss_scale * dsraw[s]);
        for (int k = 0; k < 15; ++k) dout[1 + k] = r16(dgeo[k]);
        float dhd[64];
        for (int k = 0; k < 64; ++k) {
            double acc = 0.0;
            for (int q = 0; q < 16; ++q) acc += W(dp, 2048, 64, q, k) * dout[q];
            dhd[k] = hd[k] > 0.0f ? r16((float)acc) : 0.0f;
        }
        for (int k = 0; k < 32; ++k) {
            double acc = 0.0;
            for (int q = 0; q < 64; ++q) acc += W(dp, 0, 32, q, k) * dhd[q];
            dfeat[32ull * s + k] = (float)acc;
        }
        // weight gradients
        for (int q = 0; q < 64; ++q)
            for (int k = 0; k < 32; ++k) dD[q * 32 + k] += (double)dhd[q] * x[k];
        for (int q = 0; q < 16; ++q)
            for (int k = 0; k < 64; ++k) dD[2048 + q * 64 + k] += (double)dout[q] * hd[k];
        for (int q = 0; q < 64; ++q)
            for (int k = 0; k < 32; ++k) dC[q * 32 + k] += (double)dh1[q] * xc[k];
        for (int q = 0; q < 64; ++q)
            for (int k = 0; k < 64; ++k) dC[2048 + q * 64 + k] += (double)dh2[q] * h1[k];
        for (int q = 0; q < 16; ++q)
            for (int k = 0; k < 64; ++k) dC[6144 + q * 64 + k] += (double)do3[q] * h2[k];
    }
}

// Hash-grid backward: dtable[l][idx_c][f] += w_c * dfeat[2l + f] over the 8
// corners of every level of every point (fp64 accumulation, so the result does
// not depend on summation order).  dtable: [L][T][F] doubles.
extern "C" void orc_encode_backward(const OrcGrid* g, const float* pos, const float* dfeat, uint32_t n, double* dtable) {
    for (uint32_t s = 0; s < n; ++s) {
        for (uint32_t l = 0; l < g->n_levels; ++l) {
            const uint32_t N = g->resolution[l];
            const float sc   = (float)N;
            uint32_t i0[3];
            float wa[3];
            for (int a = 0; a < 3; ++a) {
                const float x = fminf(fmaxf(pos[3ull * s + a], 0.0f), 1.0f);
                const float p = x * sc;
                uint32_t cidx = (uint32_t)floorf(p);
                if (cidx >= N) cidx = N - 1u;
                i0[a] = cidx;
                wa[a] = p - (float)cidx;
            }
            for (uint32_t c = 0; c < 8u; ++c) {
                const uint32_t cx = i0[0] + (c & 1u), cy = i0[1] + ((c >> 1) & 1u), cz = i0[2] + ((c >> 2) & 1u);
                uint32_t id;
                if (g->dense[l]) {
                    const uint32_t st = N + 1u;
                    id                = cx + cy * st + cz * st * st;
                } else {
                    id = ((cx * 1u) ^ (cy * 2654435761u) ^ (cz * 805459861u)) & (g->table_size - 1u);
                }
                const float wx  = (c & 1u) ? wa[0] : 1.0f - wa[0];
                const float wy  = (c & 2u) ? wa[1] : 1.0f - wa[1];
                const float wz  = (c & 4u) ? wa[2] : 1.0f - wa[2];
                const double wt = (double)((wx * wy) * wz);
                for (uint32_t f = 0; f < g->n_features; ++f)
                    dtable[((uint64_t)l * g->table_size + id) * g->n_features + f] += wt * (double)dfeat[(uint64_t)s * g->n_levels * g->n_features + l * g->n_features + f];
            }
        }
    }
}

// Adam step of backend-cuda.cu:1513-1554 on n parameters: grads are scaled by
// loss_scale; skip when non-finite or norm > guard; lr decays by 0.1 per
// decay_ksteps * 1000 steps; global-norm clip; bias corrections 1/(1 - b^t).
// step is the 1-based optimizer step t.  Returns 1 if the update was skipped.
extern "C" int orc_adam(float* w, float* m, float* v, const float* g, uint64_t n, float lr, float b1, float b2, float eps, float clip, float guard, float loss_scale, uint32_t decay_ksteps, uint32_t step, double grad_norm, int nonfinite) {
    if (nonfinite || !(grad_norm == grad_norm) || grad_norm > guard) return 1;
    const float decay = (float)decay_ksteps * 1000.0f;
    const float lr_t  = decay > 0.0f ? lr * powf(0.1f, (float)step / decay) : lr;
    const float scale = (grad_norm > clip && grad_norm > 0.0) ? (float)(clip / grad_norm) : 1.0f;
    const float bc1   = 1.0f / (1.0f - powf(b1, (float)step));
    const float bc2   = 1.0f / (1.0f - powf(b2, (float)step));
    for (uint64_t i = 0; i < n; ++i) {
        const float gr = g[i] / loss_scale * scale;
        m[i]           = b1 * m[i] + (1.0f - b1) * gr;
        v[i]           = b2 * v[i] + (1.0f - b2) * gr * gr;
        w[i] -= lr_t * (m[i] * bc1) / (sqrtf(v[i] * bc2) + eps);
    }
    return 0;
}

// Training rays of one step (backend-cuda.cu:438-499): random pixel of ray r,
// ray through (px, H - 1 - py), march, ground truth bilinear over the
// RGBA8 image (top row first) composited over white.  Outputs per ray:
// counts[r], gt[r][4] (r, g, b, alpha), pixel[r][2]; samples (t_mid, dt) are
// written ray-major into t_dt (capacity cap), offsets[r] = start of ray r.
extern "C" void orc_train_rays(const OrcCamera* cam, const uint8_t* image, const uint32_t* bits, uint32_t res, const float* aabb, uint32_t max_steps, uint32_t frame, uint32_t n_rays, uint32_t* counts, float* gt, float* pixel, uint32_t* offsets,
                               float* t_dt, uint32_t cap) {
    uint32_t off = 0;
    const uint32_t W = cam->width, H = cam->height;
    for (uint32_t r = 0; r < n_rays; ++r) {
        const uint32_t seed = frame * 1315423911u ^ r * 9781u;
        const float px      = orc_rand01(seed ^ 0xA511E9B3u) * (float)W;
        const float py      = orc_rand01(seed ^ 0x63D83595u) * (float)H;
        pixel[2 * r]        = px;
        pixel[2 * r + 1]    = py;
        OrcRay ray;
        uint32_t count = 0;
        offsets[r]     = off;
        if (make_ray(*cam, px, (float)H - 1.0f - py, aabb, aabb + 3, ray)) {
            count = march(*cam, ray, make_occ(bits, res, 1u, aabb), max_steps, [&](uint32_t k, float tm, float dt) {
                if (off + k < cap) {
                    t_dt[2 * (off + k)]     = tm;
                    t_dt[2 * (off + k) + 1] = dt;
                }
            });
        }
        counts[r] = count;
        off += count;
        float g4[4] = {1.0f, 1.0f, 1.0f, 0.0f};
        if (count > 0) {
            const float cx = fmaxf(0.0f, fminf(px, (float)W - 1.0f)), cy = fmaxf(0.0f, fminf(py, (float)H - 1.0f));
            const int x0 = (int)floorf(cx), y0 = (int)floorf(cy);
            const int x1 = std::min(x0 + 1, (int)W - 1), y1 = std::min(y0 + 1, (int)H - 1);
            const float tx = cx - (float)x0, ty = cy - (float)y0;
            const float inv255 = 1.0f / 255.0f;
            const uint8_t* p00 = image + ((uint64_t)y0 * W + x0) * 4;
            const uint8_t* p10 = image + ((uint64_t)y0 * W + x1) * 4;
            const uint8_t* p01 = image + ((uint64_t)y1 * W + x0) * 4;
            const uint8_t* p11 = image + ((uint64_t)y1 * W + x1) * 4;
            float c[4];
            for (int k = 0; k < 4; ++k) {
                const float a = (float)p00[k] * inv255 * (1.0f - tx) + (float)p10[k] * inv255 * tx;
                const float b = (float)p01[k] * inv255 * (1.0f - tx) + (float)p11[k] * inv255 * tx;
                c[k]          = a * (1.0f - ty) + b * ty;
            }
            const float al = c[3];
            g4[0] = c[0] * al + (1.0f - al);
            g4[1] = c[1] * al + (1.0f - al);
            g4[2] = c[2] * al + (1.0f - al);
            g4[3] = al;
        }
        for (int k = 0; k < 4; ++k) gt[4 * r + k] = g4[k];
    }
}

// Camera index of training step `frame` (backend-cuda.cu:1482).
extern "C" uint32_t orc_train_camera(uint32_t frame, uint32_t image_count) { return orc_hash_u32(frame * 747796405u + 2891336453u) % image_count; }

// Ground-truth images of the analytic scene: `steps` uniform steps over the
// ray's AABB interval, emission = density-weighted Gaussian albedo,
// alpha = 1 - exp(-density dt), stop below transmittance 1e-4, RGB over white,
// A = 1 - T; RGBA8 packed little-endian (R in the low byte), pixel (x, y) at
// index y * W + x with the reference's pixel-centre and row flip.
extern "C" void orc_scene_render(const float* gs, uint32_t count, const OrcCamera* cam, const float* aabb, uint32_t steps, uint32_t* rgba) {
    const uint32_t W = cam->width, H = cam->height;
    for (uint32_t y = 0; y < H; ++y) {
        for (uint32_t x = 0; x < W; ++x) {
            OrcRay r;
            float T = 1.0f, Cc[3] = {0.0f, 0.0f, 0.0f};
            if (pixel_ray(*cam, x, y, aabb, aabb + 3, r)) {
                const float dt = (r.tf - r.tn) / (float)steps;
                for (uint32_t i = 0; i < steps && dt > 0.0f; ++i) {
                    const float t    = r.tn + ((float)i + 0.5f) * dt;
                    const float p[3] = {r.o[0] + t * r.d[0], r.o[1] + t * r.d[1], r.o[2] + t * r.d[2]};
                    float sig = 0.0f, cr = 0.0f, cg = 0.0f, cb = 0.0f;
                    for (uint32_t k = 0; k < count; ++k) {
                        const float* g = gs + 8ull * k;
                        const float dx = p[0] - g[0], dy = p[1] - g[1], dz = p[2] - g[2];
                        const float kk = -0.5f / (g[3] * g[3]);
                        const float v  = g[4] * nerf_math::det_expf(((dx * dx + dy * dy) + dz * dz) * kk);
                        sig += v;
                        cr += v * g[5];
                        cg += v * g[6];
                        cb += v * g[7];
                    }
                    if (sig <= 0.0f) continue;
                    const float a = 1.0f - expf(-sig * dt);
                    const float w = T * a / sig;
                    Cc[0] += w * cr;
                    Cc[1] += w * cg;
                    Cc[2] += w * cb;
                    T *= 1.0f - a;
                    if (T < 1e-4f) break;
                }
            }
            uint32_t u[3];
            for (int c = 0; c < 3; ++c) u[c] = (uint32_t)rintf(fminf(1.0f, fmaxf(0.0f, Cc[c] + T)) * 255.0f);
            const uint32_t ua     = (uint32_t)rintf(fminf(1.0f, fmaxf(0.0f, 1.0f - T)) * 255.0f);
            rgba[(uint64_t)y * W + x] = (ua << 24) | (u[2] << 16) | (u[1] << 8) | u[0];
        }
    }
}

// Field MLPs on given features (rounded to fp16 inside) and unit directions:
// out [n][4] = (sigma = exp(raw), r, g, b), the network part of field_point.
extern "C" void orc_field_mlp(const uint16_t* dparams, const uint16_t* cparams, const float* features, const float* dirs, uint32_t n, float* out) {
    for (uint32_t i = 0; i < n; ++i) {
        float o[16], rgb[3];
        density_row(dparams, features + 32ull * i, o);
        color_row(cparams, o, dirs + 3ull * i, rgb);
        float* out4 = out + 4ull * i;
        out4[0]     = expf(o[0]);
        out4[1]     = rgb[0];
        out4[2]     = rgb[1];
        out4[3]     = rgb[2];
    }
}

// ===========================================================================
// Reference-model mode: the reference's own network (backend-cuda.cu:23-54).
// Frequency encoding of the world position (10 levels) and of the direction
// (4 levels) (:252-277); density MLP 64 -> 128 -> 128 x 4 -> 16 on the 63
// encoded values and a zero (:918-927); colour MLP on [raw density outputs
// 1..15 | direction encoding (27) | 0 x 6] (:928-943) -> 128 -> 128 x 2 -> 16
// (3 used); sigma = softplus(raw 0) (:913-917), rgb = sigmoid(raw) (:910-912).
// Rounding points: fp16 inputs, fp16 hidden activations and fp16 raw outputs
// (the reference's output buffers are fp16, :1063-1083); accumulation in fp64.
// ===========================================================================
static const uint32_t kRefDensity[6][2] = {{128u, 64u}, {128u, 128u}, {128u, 128u}, {128u, 128u}, {128u, 128u}, {16u, 128u}};
static const uint32_t kRefColor[4][2]   = {{128u, 48u}, {128u, 128u}, {128u, 128u}, {16u, 128u}};

extern "C" uint32_t orc_ref_param_count(uint32_t network) { return network == 0u ? 75776u : 40960u; }

// The reference's Xavier-uniform init (:1810-1847) on its own shapes.
extern "C" void orc_ref_mlp_init(uint32_t network, float* out) {
    const uint32_t n_mat = network == 0u ? 6u : 4u;
    uint64_t state       = network == 0u ? orc_stream_state(0x1234ull, 0x5678ull) : orc_stream_state(0x9abcull, 0xdef0ull);
    uint64_t off         = 0;
    for (uint32_t m = 0; m < n_mat; ++m) {
        const uint32_t fan_out = network == 0u ? kRefDensity[m][0] : kRefColor[m][0];
        const uint32_t fan_in  = network == 0u ? kRefDensity[m][1] : kRefColor[m][1];
        const float scale      = sqrtf(6.0f / (float)(fan_in + fan_out));
        for (uint64_t i = 0; i < (uint64_t)fan_in * fan_out; ++i) {
            state += 0x9e3779b97f4a7c15ull;
            uint64_t z = state;
            z          = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
            z          = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
            z ^= z >> 31;
            out[off + i] = ((float)((uint32_t)(z >> 32) >> 8) * (1.0f / 16777216.0f) * 2.0f - 1.0f) * scale;
        }
        off += (uint64_t)fan_in * fan_out;
    }
}

// [x, y, z, then per level l: sin(2^l x), sin(2^l y), sin(2^l z), cos(2^l x),
// cos(2^l y), cos(2^l z)] (:252-277).  The argument x * 2^l is exact in fp32;
// sin and cos of it are correctly rounded to fp32 (fp64 evaluation).
extern "C" void orc_freq_encode(const float* p, uint32_t levels, float* out) {
    out[0] = p[0];
    out[1] = p[1];
    out[2] = p[2];
    float freq = 1.0f;
    for (uint32_t l = 0; l < levels; ++l) {
        for (int a = 0; a < 3; ++a) {
            const double arg    = (double)(p[a] * freq);
            out[3 + 6 * l + a]     = (float)sin(arg);
            out[3 + 6 * l + 3 + a] = (float)cos(arg);
        }
        freq *= 2.0f;
    }
}

// softplus with the reference's branches (:913-917), evaluated in fp64.
extern "C" float orc_softplus(float x) {
    if (x > 20.0f) return x;
    if (x < -20.0f) return (float)exp((double)x);
    return (float)log1p(exp((double)x));
}

static float sigmoid64(float x) { return (float)(1.0 / (1.0 + exp(-(double)x))); }

// Layers of one network on an fp16-valued input row; out = fp16-rounded raw
// outputs of the last layer.
static void ref_mlp_row(const uint16_t* W, const uint32_t (*shape)[2], uint32_t layers, const float* x_in, float* out) {
    std::vector<float> a(x_in, x_in + shape[0][1]), b;
    uint64_t off = 0;
    for (uint32_t m = 0; m < layers; ++m) {
        b.assign(shape[m][0], 0.0f);
        matvec(W + off, shape[m][0], shape[m][1], a.data(), b.data());
        off += (uint64_t)shape[m][0] * shape[m][1];
        for (float& v : b) v = m + 1u < layers ? r16(fmaxf(v, 0.0f)) : r16(v);
        a.swap(b);
    }
    std::copy(a.begin(), a.end(), out);
}

static void ref_field_point(const uint16_t* dp, const uint16_t* cp, const float* p, const float* d, float* out4, float* raw4) {
    float pe[64], de[27], dens[16], ci[48], col[16];
    orc_freq_encode(p, 10u, pe);
    for (int k = 0; k < 63; ++k) pe[k] = r16(pe[k]);
    pe[63] = 0.0f;
    ref_mlp_row(dp, kRefDensity, 6u, pe, dens);
    orc_freq_encode(d, 4u, de);
    for (int k = 0; k < 15; ++k) ci[k] = dens[1 + k];
    for (int k = 0; k < 27; ++k) ci[15 + k] = r16(de[k]);
    for (int k = 42; k < 48; ++k) ci[k] = 0.0f;
    ref_mlp_row(cp, kRefColor, 4u, ci, col);
    out4[0] = orc_softplus(dens[0]);
    for (int c = 0; c < 3; ++c) out4[1 + c] = sigmoid64(col[c]);
    if (raw4) {
        raw4[0] = dens[0];
        for (int c = 0; c < 3; ++c) raw4[1 + c] = col[c];
    }
}

// out [n][4] = (sigma, r, g, b); raw (optional) [n][4] = fp16-rounded raw
// density output 0 and colour outputs 0..2.  Positions in world coordinates.
extern "C" void orc_ref_field_forward(const uint16_t* dparams, const uint16_t* cparams, const float* pos, const float* dirs, uint32_t n, float* out, float* raw) {
    for (uint32_t i = 0; i < n; ++i) ref_field_point(dparams, cparams, pos + 3ull * i, dirs + 3ull * i, out + 4ull * i, raw ? raw + 4ull * i : nullptr);
}

// Composite forward + backward of one ray with the reference's loss
// (:1095-1182): sigma = softplus(raw), rgb = sigmoid(raw), white background,
// ray weight w_r = 0.1 + 0.9 clamp(gt_a, 0, 1), loss w_r |pred - gt|^2,
// output gradient g = 2 w_r (pred - gt) inv_norm.  d raw sigma_i =
// dt_i (T_{i+1} c_i - S_i) . g sigmoid(raw_i) with S_i the colour composited
// behind sample i plus T_n (the exact derivative; the reference divides by
// max(1 - alpha, 1e-6), equal wherever 1 - alpha >= 1e-6); d raw rgb_i =
// T_i alpha_i g c (1 - c).  fp64 throughout; returns the ray's loss.
extern "C" double orc_ref_composite_backward_ray(const float* sraw, const float* rgbraw, const float* dt, uint32_t n, const float* gt4, float inv_norm, float* dsraw, float* drgbraw, float* pred_out) {
    auto softplus = [](double x) { return x > 20.0 ? x : (x < -20.0 ? exp(x) : log1p(exp(x))); };
    auto sigm     = [](double x) { return 1.0 / (1.0 + exp(-x)); };
    std::vector<double> T(n + 1), a(n), c(3ull * n), d(n);
    T[0] = 1.0;
    double pred[3] = {0.0, 0.0, 0.0};
    for (uint32_t i = 0; i < n; ++i) {
        d[i] = fmax((double)dt[i], 0.0);
        a[i] = 1.0 - exp(-softplus(sraw[i]) * d[i]);
        for (int k = 0; k < 3; ++k) {
            c[3ull * i + k] = sigm(rgbraw[3ull * i + k]);
            pred[k] += T[i] * a[i] * c[3ull * i + k];
        }
        T[i + 1] = T[i] * (1.0 - a[i]);
    }
    const double wr = 0.1 + 0.9 * fmin(1.0, fmax(0.0, (double)gt4[3]));
    double loss = 0.0, g[3];
    for (int k = 0; k < 3; ++k) {
        pred[k] += T[n];
        const double x = pred[k] - gt4[k];
        loss += wr * x * x;
        g[k] = 2.0 * wr * x * inv_norm;
        if (pred_out) pred_out[k] = (float)pred[k];
    }
    double S[3] = {T[n], T[n], T[n]};  // composited behind sample i
    for (int i = (int)n - 1; i >= 0; --i) {
        double ds = 0.0;
        for (int k = 0; k < 3; ++k) {
            const double ck = c[3ull * i + k];
            ds += g[k] * (T[i + 1] * ck - S[k]);
            if (drgbraw) drgbraw[3ull * i + k] = (float)(T[i] * a[i] * g[k] * ck * (1.0 - ck));
            S[k] += T[i] * a[i] * ck;
        }
        if (dsraw) dsraw[i] = (float)(d[i] * ds * sigm(sraw[i]));
    }
    return loss;
}

// MLP backward of the reference-model network for a batch: given d loss /
// d raw outputs draw [n][4] (raw sigma, raw r, g, b), weight gradients
// dD [75776], dC [40960] (accumulated in fp64, multiplied by loss_scale).
// Rounding points as the product path: output deltas fp16(loss_scale x draw);
// every propagated delta fp16(mask . W^T delta) with the mask from the
// forward activation (> 0); the geometry features' delta
// fp16((W_c0^T delta_c0) [0, 15)) becomes density output deltas 1..15
// (:1069-1083); activations as the forward (fp16).
extern "C" void orc_ref_mlp_backward(const uint16_t* dp, const uint16_t* cp, const float* pos, const float* dirs, const float* draw, uint32_t n, float loss_scale, double* dD, double* dC) {
    auto W = [](const uint16_t* P, uint64_t off, uint32_t n_in, uint32_t o, uint32_t i) { return (double)orc_f16_to_f32(P[off + (uint64_t)o * n_in + i]); };
    uint64_t doff[6], coff[4], o = 0;
    for (int m = 0; m < 6; ++m) doff[m] = o, o += (uint64_t)kRefDensity[m][0] * kRefDensity[m][1];
    o = 0;
    for (int m = 0; m < 4; ++m) coff[m] = o, o += (uint64_t)kRefColor[m][0] * kRefColor[m][1];
    // Forward with every layer's input kept: net input, then each layer's output.
    auto forward = [&](const uint16_t* P, const uint32_t (*shape)[2], const uint64_t* off, uint32_t layers, std::vector<std::vector<float>>& acts) {
        for (uint32_t m = 0; m < layers; ++m) {
            const std::vector<float>& a = acts[m];
            std::vector<float> b(shape[m][0]);
            for (uint32_t q = 0; q < shape[m][0]; ++q) {
                double acc = 0.0;
                for (uint32_t k = 0; k < shape[m][1]; ++k) acc += W(P, off[m], shape[m][1], q, k) * (double)a[k];
                b[q] = m + 1u < layers ? r16(fmaxf((float)acc, 0.0f)) : r16((float)acc);
            }
            acts.push_back(b);
        }
    };
    // Backward from output delta; returns the delta of the network input (unmasked).
    auto backward = [&](const uint16_t* P, const uint32_t (*shape)[2], const uint64_t* off, uint32_t layers, const std::vector<std::vector<float>>& acts, std::vector<float> delta, double* dW) {
        std::vector<double> din;
        for (int m = (int)layers - 1; m >= 0; --m) {
            const uint32_t n_out = shape[m][0], n_in = shape[m][1];
            const std::vector<float>& a = acts[m];
            for (uint32_t q = 0; q < n_out; ++q)
                for (uint32_t k = 0; k < n_in; ++k) dW[off[m] + (uint64_t)q * n_in + k] += (double)delta[q] * (double)a[k];
            din.assign(n_in, 0.0);
            for (uint32_t k = 0; k < n_in; ++k)
                for (uint32_t q = 0; q < n_out; ++q) din[k] += W(P, off[m], n_in, q, k) * (double)delta[q];
            if (m > 0) {
                std::vector<float> nd(n_in);
                for (uint32_t k = 0; k < n_in; ++k) nd[k] = a[k] > 0.0f ? r16((float)din[k]) : 0.0f;
                delta.swap(nd);
            }
        }
        return din;
    };
    for (uint32_t s = 0; s < n; ++s) {
        float pe[64], de[27];
        orc_freq_encode(pos + 3ull * s, 10u, pe);
        for (int k = 0; k < 63; ++k) pe[k] = r16(pe[k]);
        pe[63] = 0.0f;
        std::vector<std::vector<float>> da{std::vector<float>(pe, pe + 64)};
        forward(dp, kRefDensity, doff, 6u, da);
        const std::vector<float>& dens = da.back();
        orc_freq_encode(dirs + 3ull * s, 4u, de);
        std::vector<float> ci(48, 0.0f);
        for (int k = 0; k < 15; ++k) ci[k] = dens[1 + k];
        for (int k = 0; k < 27; ++k) ci[15 + k] = r16(de[k]);
        std::vector<std::vector<float>> ca{ci};
        forward(cp, kRefColor, coff, 4u, ca);
        std::vector<float> dc(16, 0.0f), dd(16, 0.0f);
        for (int k = 0; k < 3; ++k) dc[k] = r16(loss_scale * draw[4ull * s + 1 + k]);
        const std::vector<double> dci = backward(cp, kRefColor, coff, 4u, ca, dc, dC);
        dd[0] = r16(loss_scale * draw[4ull * s]);
        for (int k = 0; k < 15; ++k) dd[1 + k] = r16((float)dci[k]);
        backward(dp, kRefDensity, doff, 6u, da, dd, dD);
    }
}
