// field.hip — fused hash-grid encode + fp16 MFMA MLPs on gfx950.
//
// Network semantics follow the reference's fully fused MLP (backend-cuda.cu
// :668-835: no biases, ReLU hidden layers, W row-major [out][in], packed input
// layer first) at the target widths: density 32 -> 64 -> 16, colour
// [geo 15 | SH4 16 | 0] -> 64 -> 64 -> 16 (3 used).  Unlike the reference
// (WMMA with an fp16 accumulator, activations staged through shared memory),
// everything here is register resident on v_mfma_f32_16x16x32_f16:
//
//   * Transposed products.  A layer computes out^T = W . in^T with W as the A
//     operand (16 output neurons x 32 inputs) and the activations as the B
//     operand (32 inputs x 16 samples).  The 16x16 fp32 result leaves lane l
//     holding out[4 (l / 16) + e][sample l % 16], e = 0..3.
//   * No transposes between layers.  The reduction index k of a 16x16x32 MFMA
//     is paired between A and B by (lane / 16, element), whatever order the
//     hardware sums in.  So the next layer consumes the result registers as
//     they are: lane group g supplies, for k-step t, neurons
//     {32t + 4g + 0..3, 32t + 16 + 4g + 0..3} (its results of blocks 2t and
//     2t+1), and the weights of that layer are loaded once, permuted the same
//     way.  No LDS round trip, no shuffles.
//   * The first B operand is the hash encoding itself: lane (g, s) encodes
//     levels 4g..4g+3 of sample s (features 8g..8g+7), straight into
//     registers.
//   * Weights are staged once per workgroup into LDS, then each wave keeps its
//     A fragments in VGPRs (80 VGPRs for both networks) and loops over tiles
//     of 16 samples (persistent grid).
#include "common.hpp"

namespace nerf_hip {

namespace {

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

__device__ __forceinline__ void load_density(const half_t* P, DensityFrags& f, uint32_t lane) {
#pragma unroll
    for (uint32_t b = 0; b < 4u; ++b) f.w1[b] = load_a(P, 32u, b, 0u, KMap::Identity, lane);
#pragma unroll
    for (uint32_t t = 0; t < 2u; ++t) f.w2[t] = load_a(P + 2048, 64u, 0u, t, KMap::Hidden, lane);
}

__device__ __forceinline__ void load_color(const half_t* P, ColorFrags& f, uint32_t lane) {
#pragma unroll
    for (uint32_t b = 0; b < 4u; ++b) f.w1[b] = load_a(P, 32u, b, 0u, KMap::ColorIn, lane);
#pragma unroll
    for (uint32_t b = 0; b < 4u; ++b)
#pragma unroll
        for (uint32_t t = 0; t < 2u; ++t) f.w2[2u * b + t] = load_a(P + 2048, 64u, b, t, KMap::Hidden, lane);
#pragma unroll
    for (uint32_t t = 0; t < 2u; ++t) f.w3[t] = load_a(P + 2048 + 4096, 64u, 0u, t, KMap::Hidden, lane);
}

__device__ __forceinline__ half4_t relu_half(const floatx4 v) {
    half4_t h;
#pragma unroll
    for (int e = 0; e < 4; ++e) h[e] = (half_t)fmaxf(v[e], 0.0f);
    return h;
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
// Corner order, weights and accumulation order are those of the oracle.
template <typename TableT>
__device__ __forceinline__ void encode_quad(const GridParams& g, const TableT* __restrict__ table, const float p[3], uint32_t grp, float feat[8]) {
    const uint32_t mask = g.table_size - 1u;
#pragma unroll
    for (uint32_t j = 0; j < 4u; ++j) {
        // Level 4*grp + j, selected without dynamic indexing of the kernel argument.
        const uint32_t l0 = j, l1 = 4u + j, l2 = 8u + j, l3 = 12u + j;
        const uint32_t N  = grp == 0u ? g.resolution[l0] : grp == 1u ? g.resolution[l1] : grp == 2u ? g.resolution[l2] : g.resolution[l3];
        const uint32_t dn = grp == 0u ? g.dense[l0] : grp == 1u ? g.dense[l1] : grp == 2u ? g.dense[l2] : g.dense[l3];
        const uint32_t level = 4u * grp + j;
        float a0 = 0.0f, a1 = 0.0f;
        if (level < g.n_levels) {
            const LevelCell c  = level_cell(p, N);
            const TableT* base = table + (uint64_t)level * g.table_size * 2u;
            uint32_t idx[8];
#pragma unroll
            for (uint32_t k = 0; k < 8u; ++k) idx[k] = corner_index(c, k, N, dn != 0u, mask);
            float v0[8], v1[8];
#pragma unroll
            for (uint32_t k = 0; k < 8u; ++k) {
                v0[k] = (float)base[2u * idx[k]];
                v1[k] = (float)base[2u * idx[k] + 1u];
            }
#pragma unroll
            for (uint32_t k = 0; k < 8u; ++k) {
                const float w = corner_weight(c, k);
                a0            = a0 + w * v0[k];
                a1            = a1 + w * v1[k];
            }
        }
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
__device__ __forceinline__ void sh4_quad(const float d[3], uint32_t grp, float out[4]) {
    const float x = d[0], y = d[1], z = d[2];
    const float xy = x * y, yz = y * z, xz = x * z;
    const float x2 = x * x, y2 = y * y, z2 = z * z;
    float s[16];
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
#pragma unroll
    for (uint32_t e = 0; e < 4u; ++e) out[e] = grp == 0u ? s[e] : grp == 1u ? s[4u + e] : grp == 2u ? s[8u + e] : s[12u + e];
}

__device__ __forceinline__ void stage_params(half_t* lds, const half_t* src, uint32_t count) {
    for (uint32_t i = threadIdx.x; i < count; i += blockDim.x) lds[i] = src[i];
    __syncthreads();
}

// ---------------------------------------------------------------- kernels
// Density MLP on fp16 features [n][32] -> raw outputs [n][16].
__global__ __launch_bounds__(kBlockThreads) void k_density_mlp(const half_t* __restrict__ params, const half_t* __restrict__ features, uint32_t n, float* __restrict__ out) {
    __shared__ half_t sp[NERF_EXT_DENSITY_PARAMS];
    stage_params(sp, params, NERF_EXT_DENSITY_PARAMS);
    const uint32_t lane = threadIdx.x & 63u, grp = lane >> 4, s16 = lane & 15u;
    DensityFrags f;
    load_density(sp, f, lane);
    const uint32_t tiles  = (n + 15u) / 16u;
    const uint32_t nwaves = gridDim.x * kBlockWaves;
    for (uint32_t tile = blockIdx.x * kBlockWaves + (threadIdx.x >> 6); tile < tiles; tile += nwaves) {
        const uint32_t s = tile * 16u + s16;
        half8_t x;
        if (s < n) {
            x = *reinterpret_cast<const half8_t*>(features + (uint64_t)s * 32u + 8u * grp);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = (half_t)0.0f;
        }
        const floatx4 o = density_mlp(f, x);
        if (s < n) *reinterpret_cast<float4*>(out + (uint64_t)s * 16u + 4u * grp) = make_float4(o[0], o[1], o[2], o[3]);
    }
}

// Fused encode + density MLP on points: out [n][16] = (exp(raw0), raw1..15).
template <typename TableT>
__global__ __launch_bounds__(kBlockThreads) void k_density_forward(GridParams g, const TableT* __restrict__ table, const half_t* __restrict__ params, const float* __restrict__ pos, uint32_t n, float* __restrict__ out) {
    __shared__ half_t sp[NERF_EXT_DENSITY_PARAMS];
    stage_params(sp, params, NERF_EXT_DENSITY_PARAMS);
    const uint32_t lane = threadIdx.x & 63u, grp = lane >> 4, s16 = lane & 15u;
    DensityFrags f;
    load_density(sp, f, lane);
    const uint32_t tiles  = (n + 15u) / 16u;
    const uint32_t nwaves = gridDim.x * kBlockWaves;
    for (uint32_t tile = blockIdx.x * kBlockWaves + (threadIdx.x >> 6); tile < tiles; tile += nwaves) {
        const uint32_t s = tile * 16u + s16;
        const uint32_t q = s < n ? s : n - 1u;
        const float p[3] = {pos[3ull * q], pos[3ull * q + 1], pos[3ull * q + 2]};
        float feat[8];
        encode_quad(g, table, p, grp, feat);
        floatx4 o = density_mlp(f, to_half8(feat));
        if (grp == 0u) o[0] = expf(o[0]);
        if (s < n) *reinterpret_cast<float4*>(out + (uint64_t)s * 16u + 4u * grp) = make_float4(o[0], o[1], o[2], o[3]);
    }
}

// Full field: sigma, rgb per sample.  Inputs either explicit (positions,
// directions) or march samples (t_mid, dt, ray) with per-ray o, d.
template <typename TableT, bool kFromSamples>
__global__ __launch_bounds__(kBlockThreads) void k_field_forward(GridParams g, const TableT* __restrict__ table, const half_t* __restrict__ dparams, const half_t* __restrict__ cparams, FieldInputs in, uint32_t n, float4* __restrict__ out) {
    __shared__ half_t sp[NERF_EXT_DENSITY_PARAMS + NERF_EXT_COLOR_PARAMS];
    for (uint32_t i = threadIdx.x; i < NERF_EXT_DENSITY_PARAMS; i += blockDim.x) sp[i] = dparams[i];
    for (uint32_t i = threadIdx.x; i < NERF_EXT_COLOR_PARAMS; i += blockDim.x) sp[NERF_EXT_DENSITY_PARAMS + i] = cparams[i];
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63u, grp = lane >> 4, s16 = lane & 15u;
    DensityFrags fd;
    ColorFrags fc;
    load_density(sp, fd, lane);
    load_color(sp + NERF_EXT_DENSITY_PARAMS, fc, lane);
    const uint32_t tiles  = (n + 15u) / 16u;
    const uint32_t nwaves = gridDim.x * kBlockWaves;
    for (uint32_t tile = blockIdx.x * kBlockWaves + (threadIdx.x >> 6); tile < tiles; tile += nwaves) {
        const uint32_t s = tile * 16u + s16;
        const uint32_t q = s < n ? s : n - 1u;
        float p[3], d[3];
        if constexpr (kFromSamples) {
            const float2 td  = in.samples[q];
            const uint32_t r = in.sample_ray[q];
            const float4 ro  = in.rays[2ull * r];
            const float4 rd  = in.rays[2ull * r + 1ull];
            d[0]             = rd.x;
            d[1]             = rd.y;
            d[2]             = rd.z;
            p[0]             = ro.x + td.x * rd.x;
            p[1]             = ro.y + td.x * rd.y;
            p[2]             = ro.z + td.x * rd.z;
        } else {
#pragma unroll
            for (int a = 0; a < 3; ++a) {
                p[a] = in.positions[3ull * q + a];
                d[a] = in.directions[3ull * q + a];
            }
        }
        float feat[8];
        encode_quad(g, table, p, grp, feat);
        const floatx4 o = density_mlp(fd, to_half8(feat));
        // Colour input: (density outputs 4g..4g+3, SH 4g..4g+3); the slot of
        // density output 0 (sigma) carries a zero weight and a zero value.
        float sh[4];
        sh4_quad(d, grp, sh);
        half8_t xc;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            xc[e]     = (half_t)o[e];
            xc[4 + e] = (half_t)sh[e];
        }
        if (grp == 0u) xc[0] = (half_t)0.0f;
        const floatx4 c = color_mlp(fc, xc);
        if (grp == 0u && s < n) {
            const float sigma = expf(o[0]);
            const float r     = 1.0f / (1.0f + expf(-c[0]));
            const float gg    = 1.0f / (1.0f + expf(-c[1]));
            const float b     = 1.0f / (1.0f + expf(-c[2]));
            out[s]            = make_float4(sigma, r, gg, b);
        }
    }
}

uint32_t persistent_blocks(uint32_t n, uint32_t per_cu) {
    const uint32_t tiles  = (n + 15u) / 16u;
    const uint32_t needed = (tiles + kBlockWaves - 1u) / kBlockWaves;
    const uint32_t cap    = device_cu_count() * per_cu;
    return needed < cap ? (needed > 0u ? needed : 1u) : cap;
}

}  // namespace

hipError_t launch_field(const GridParams& g, const void* table, const FieldWeights& w, const FieldInputs& in, uint32_t n, float4* out4, hipStream_t stream) {
    if (n == 0u) return hipSuccess;
    const uint32_t blocks = persistent_blocks(n, 8u);
    const bool from_samples = in.samples != nullptr;
    if (g.table_dtype == NERF_EXT_F32) {
        if (from_samples)
            k_field_forward<float, true><<<blocks, kBlockThreads, 0, stream>>>(g, (const float*)table, w.density, w.color, in, n, out4);
        else
            k_field_forward<float, false><<<blocks, kBlockThreads, 0, stream>>>(g, (const float*)table, w.density, w.color, in, n, out4);
    } else {
        if (from_samples)
            k_field_forward<half_t, true><<<blocks, kBlockThreads, 0, stream>>>(g, (const half_t*)table, w.density, w.color, in, n, out4);
        else
            k_field_forward<half_t, false><<<blocks, kBlockThreads, 0, stream>>>(g, (const half_t*)table, w.density, w.color, in, n, out4);
    }
    return hipGetLastError();
}

hipError_t launch_density(const GridParams& g, const void* table, const half_t* dparams, const float* positions, const half_t* features, uint32_t n, float* out, hipStream_t stream) {
    if (n == 0u) return hipSuccess;
    const uint32_t blocks = persistent_blocks(n, 8u);
    if (features) {
        k_density_mlp<<<blocks, kBlockThreads, 0, stream>>>(dparams, features, n, out);
    } else if (g.table_dtype == NERF_EXT_F32) {
        k_density_forward<float><<<blocks, kBlockThreads, 0, stream>>>(g, (const float*)table, dparams, positions, n, out);
    } else {
        k_density_forward<half_t><<<blocks, kBlockThreads, 0, stream>>>(g, (const half_t*)table, dparams, positions, n, out);
    }
    return hipGetLastError();
}

// Float -> fp16 (round to nearest even), e.g. master weights -> MLP params.
__global__ __launch_bounds__(256) void k_float_to_half(const float* __restrict__ src, half_t* __restrict__ dst, uint64_t n) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = (half_t)src[i];
}

// Host-side Xavier-uniform init of backend-cuda.cu:1810-1847 on the target shapes.
static void mlp_init_host(uint32_t network, float* out) {
    static const uint32_t dens[2][2] = {{64u, 32u}, {16u, 64u}};
    static const uint32_t col[3][2]  = {{64u, 32u}, {64u, 64u}, {16u, 64u}};
    const uint32_t n_mat             = network == 0u ? 2u : 3u;
    const uint64_t state0            = network == 0u ? nerf_math::stream_state(0x1234ull, 0x5678ull) : nerf_math::stream_state(0x9abcull, 0xdef0ull);
    uint64_t draw = 0, off = 0;
    for (uint32_t m = 0; m < n_mat; ++m) {
        const uint32_t fan_out = network == 0u ? dens[m][0] : col[m][0];
        const uint32_t fan_in  = network == 0u ? dens[m][1] : col[m][1];
        const float scale      = sqrtf(6.0f / (float)(fan_in + fan_out));
        const uint64_t count   = (uint64_t)fan_in * fan_out;
        for (uint64_t i = 0; i < count; ++i, ++draw) {
            const uint64_t z = nerf_math::splitmix_at(state0, draw);
            out[off + i]     = ((float)((uint32_t)(z >> 32) >> 8) * (1.0f / 16777216.0f) * 2.0f - 1.0f) * scale;
        }
        off += count;
    }
}

}  // namespace nerf_hip

using namespace nerf_hip;

extern "C" {

NERF_API NerfStatus nerf_ext_mlp_init(uint32_t network, float* params_host) {
    NERF_CHECK_ARG(network <= 1u, "nerf_ext_mlp_init: network must be 0 (density) or 1 (colour)");
    NERF_CHECK_ARG(params_host, "nerf_ext_mlp_init: null output");
    mlp_init_host(network, params_host);
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_float_to_half(const float* src, uint16_t* dst, uint64_t n, void* stream) {
    if (n == 0u) return NERF_STATUS_OK;
    NERF_CHECK_ARG(src && dst, "nerf_ext_float_to_half: null pointer");
    const uint64_t blocks = (n + 255u) / 256u;
    k_float_to_half<<<(uint32_t)(blocks < 65536u ? blocks : 65536u), 256, 0, (hipStream_t)stream>>>(src, (half_t*)dst, n);
    NERF_LAUNCH_CHECK("k_float_to_half");
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_density_mlp(const uint16_t* params, const uint16_t* features, uint32_t n, float* out, void* stream) {
    if (n == 0u) return NERF_STATUS_OK;
    NERF_CHECK_ARG(params && features && out, "nerf_ext_density_mlp: null pointer");
    GridParams g{};
    NERF_HIP_TRY(launch_density(g, nullptr, (const half_t*)params, nullptr, (const half_t*)features, n, out, (hipStream_t)stream));
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_density_forward(const NerfExtGridDesc* grid, const void* table, const uint16_t* params, const float* positions, uint32_t n, float* out, void* stream) {
    GridParams g;
    const NerfStatus s = make_grid(grid, g);
    if (s != NERF_STATUS_OK) return s;
    NERF_CHECK_ARG(g.n_levels * g.n_features == 32u, "nerf_ext_density_forward: the density MLP takes 32 features (16 levels x 2)");
    if (n == 0u) return NERF_STATUS_OK;
    NERF_CHECK_ARG(table && params && positions && out, "nerf_ext_density_forward: null pointer");
    NERF_HIP_TRY(launch_density(g, table, (const half_t*)params, positions, nullptr, n, out, (hipStream_t)stream));
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_field_forward(const NerfExtModel* model, const float* positions, const float* directions, uint32_t n, float* out, void* stream) {
    NERF_CHECK_ARG(model, "nerf_ext_field_forward: null model");
    GridParams g;
    const NerfStatus s = make_grid(&model->grid, g);
    if (s != NERF_STATUS_OK) return s;
    NERF_CHECK_ARG(g.n_levels * g.n_features == 32u, "nerf_ext_field_forward: the density MLP takes 32 features (16 levels x 2)");
    if (n == 0u) return NERF_STATUS_OK;
    NERF_CHECK_ARG(model->table && model->density_params && model->color_params && positions && directions && out, "nerf_ext_field_forward: null pointer");
    FieldInputs in{};
    in.positions  = positions;
    in.directions = directions;
    const FieldWeights w{(const half_t*)model->density_params, (const half_t*)model->color_params};
    NERF_HIP_TRY(launch_field(g, model->table, w, in, n, (float4*)out, (hipStream_t)stream));
    return NERF_STATUS_OK;
}

}  // extern "C"
