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
//   * The 20 A fragments of both networks (1 KiB each) are built once per
//     workgroup.  The level-major render kernel keeps them in VGPRs (80 per
//     lane); the tile kernel and the MLP pass keep them in LDS in lane order
//     and read each where it is used (one conflict-free 16-byte read).
#include "mlp_device.hpp"

namespace nerf_hip {

using namespace mlp;

namespace {

// Position (normalised by the AABB), direction and dt of march sample q.
__device__ __forceinline__ void sample_point(const FieldInputs& in, uint32_t q, uint32_t r, float p[3], float d[3], float& dt) {
    const float2 td  = in.samples[q];
    dt               = td.y;
    const float4 ro  = in.rays[2ull * r];
    const float4 rd  = in.rays[2ull * r + 1ull];
    d[0]             = rd.x;
    d[1]             = rd.y;
    d[2]             = rd.z;
    const float w[3] = {ro.x + td.x * rd.x, ro.y + td.x * rd.y, ro.z + td.x * rd.z};
    box_relative(w, in.bmin, in.bmax, p);
}

// Colour input from per-sample fp32 SH coefficients (lane group grp's four).
__device__ __forceinline__ half8_t color_input_dir(const floatx4 o, const float d[3], uint32_t grp) {
    float sh[4];
    sh4_quad(d, grp, sh);
    return color_input(o, half4_t{(half_t)sh[0], (half_t)sh[1], (half_t)sh[2], (half_t)sh[3]}, grp);
}

constexpr uint32_t kGroupSamples = 64u;
constexpr uint32_t kFieldFrags   = 20u;  // density w1[4] w2[2], colour w1[4] w2[8] w3[2]
constexpr uint32_t kMlpWaves     = 4u;   // waves per SIMD the register budget is built for

// Fragment f of the two MLPs for lane `lane`, read from the global parameters
// element by element (any alignment); same values as load_density /
// load_color give from the staged copy.
__device__ half8_t mlp_fragment(const half_t* __restrict__ dp, const half_t* __restrict__ cp, uint32_t f, uint32_t lane) {
    const uint32_t i = lane & 15u;
    if (f < 4u) return load_a(dp, 32u, f, 0u, KMap::Identity, lane);
    if (f < 6u) return load_a(dp + 2048, 64u, 0u, f - 4u, KMap::Hidden, lane);
    if (f < 10u) return load_a(cp, 32u, f - 6u, 0u, KMap::ColorIn, lane);
    if (f < 18u) return load_a(cp + 2048, 64u, (f - 10u) >> 1, (f - 10u) & 1u, KMap::Hidden, lane);
    // Colour output: row 4c (c = 1..3) of the MFMA computes colour c - 1,
    // every other row is zero (see load_color).
    const bool used = (i & 3u) == 0u && i != 0u;
    const half8_t v = load_a(cp + 2048 + 4096 + (used ? (i / 4u - 1u) : 0u) * 64u, 64u, 0u, f - 18u, KMap::Hidden, lane & 48u);
    const half8_t z = {};
    return used ? v : z;
}

// The MLPs of one 16-sample tile with the 20 fragments in LDS in lane order
// (W = &frag[0][0] + lane): density 32 -> 64 -> 16 from the encoding x, then
// colour [geo | SH] -> 64 -> 64 -> 16 from the colour input that xc_of builds
// out of the density outputs.  Same products and order as density_mlp /
// color_mlp on register fragments.
template <typename ColorIn>
__device__ __forceinline__ void tile_mlp(const half8_t* W, const half8_t x, ColorIn xc_of, floatx4& o, floatx4& c) {
    const floatx4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
    half4_t h[4], h2[4];
#pragma unroll
    for (uint32_t b = 0; b < 4u; ++b) h[b] = relu_half(mfma16x16x32(W[64u * b], x, zero));
    o                = mfma16x16x32(W[64u * 5u], cat(h[2], h[3]), mfma16x16x32(W[64u * 4u], cat(h[0], h[1]), zero));
    const half8_t xc = xc_of(o);
#pragma unroll
    for (uint32_t b = 0; b < 4u; ++b) h[b] = relu_half(mfma16x16x32(W[64u * (6u + b)], xc, zero));
#pragma unroll
    for (uint32_t b = 0; b < 4u; ++b) h2[b] = relu_half(mfma16x16x32(W[64u * (11u + 2u * b)], cat(h[2], h[3]), mfma16x16x32(W[64u * (10u + 2u * b)], cat(h[0], h[1]), zero)));
    c = mfma16x16x32(W[64u * 19u], cat(h2[2], h2[3]), mfma16x16x32(W[64u * 18u], cat(h2[0], h2[1]), zero));
}

// Fragment base for this lane, through an opaque offset: with a visible lane
// index the compiler hoists all 20 fragment reads out of the sample loop
// into 80 VGPRs, which is what keeping them in LDS avoids.
__device__ __forceinline__ const half8_t* lane_frags(const half8_t (&frag)[kFieldFrags][kWaveSize], uint32_t lane) {
    uint32_t lo = lane;
    asm volatile("" : "+v"(lo));
    return &frag[0][0] + lo;
}

// ---------------------------------------------------------------- kernels
// Density MLP on fp16 features [n][32] -> raw outputs [n][16].
__global__ __launch_bounds__(kBlockThreads) void k_density_mlp(const half_t* __restrict__ params, const half_t* __restrict__ features, uint32_t n, float* __restrict__ out) {
    __shared__ __align__(16) half_t sp[NERF_EXT_DENSITY_PARAMS];
    stage_density<kBlockThreads>(sp, params);
    __syncthreads();
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
    __shared__ __align__(16) half_t sp[NERF_EXT_DENSITY_PARAMS];
    stage_density<kBlockThreads>(sp, params);
    __syncthreads();
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
// directions) or march samples (t_mid, dt, ray) with per-ray o, d.  The
// weight fragments stay in LDS (84 VGPRs instead of 157): on a training
// batch (2^18 samples, one ray's consecutive samples per tile) the gathers
// of a tile then get more registers in flight, 75 -> 71 us at the same 3
// workgroups per CU.
template <typename TableT, bool kFromSamples>
__global__ __launch_bounds__(kBlockThreads) void k_field_forward(GridParams g, const TableT* __restrict__ table, const half_t* __restrict__ dparams, const half_t* __restrict__ cparams, FieldInputs in, uint32_t n_cap, float4* __restrict__ out) {
    const uint32_t n = in.n_dev ? min(*in.n_dev, n_cap) : n_cap;
    __shared__ __align__(16) half8_t frag[kFieldFrags][kWaveSize];
    const uint32_t lane = threadIdx.x & 63u, grp = lane >> 4, s16 = lane & 15u;
    for (uint32_t f = threadIdx.x >> 6; f < kFieldFrags; f += kBlockWaves) frag[f][lane] = mlp_fragment(dparams, cparams, f, lane);
    __syncthreads();
    // Round r covers tiles [r * W, (r + 1) * W) of the stream (W = all waves),
    // XCD x (workgroups b with b % 8 == x) taking the x-th eighth of it, so
    // a ray's consecutive tiles share one XCD's L2 while the whole device
    // works on one band of neighbouring rays.
    const uint32_t tiles   = (n + 15u) / 16u;
    const uint32_t per_xcd = (gridDim.x >> 3) * kBlockWaves;
    const uint32_t lw      = (blockIdx.x >> 3) * kBlockWaves + (threadIdx.x >> 6);
    const uint32_t first   = (blockIdx.x & 7u) * per_xcd + lw;
    for (uint32_t tile = first; tile < tiles; tile += 8u * per_xcd) {
        const uint32_t s = tile * 16u + s16;
        const uint32_t q = s < n ? s : n - 1u;
        float p[3], d[3], dt = 0.0f;
        uint32_t dst = s;  // output slot
        if constexpr (kFromSamples) {
            const uint32_t qs = in.sample_index ? in.sample_index[q] : q;
            dst               = in.sample_index && !in.alpha_in_order ? qs : s;
            sample_point(in, qs, sample_owner(in, q, qs), p, d, dt);
        } else {
#pragma unroll
            for (int a = 0; a < 3; ++a) {
                p[a] = in.positions[3ull * q + a];
                d[a] = in.directions[3ull * q + a];
            }
        }
        float feat[8];
        encode_quad(g, table, p, grp, feat);
        const half8_t x = to_half8(feat);
        if (in.features_out && s < n) *reinterpret_cast<half8_t*>(in.features_out + (uint64_t)s * 32u + 8u * grp) = x;
        floatx4 o, c;
        tile_mlp(lane_frags(frag, lane), x, [&](const floatx4& od) { return color_input_dir(od, d, grp); }, o, c);
        float v = field_channel(o, c, grp);
        if (kFromSamples && in.alpha_in_order && grp == 0u) v = render_alpha(v, dt);
        if (s < n) reinterpret_cast<float*>(out)[4ull * dst + grp] = v;
    }
}

// Full field, level-major gather.  A wave takes 64 samples at a time, lane l
// owning sample l: it gathers the 16 levels of its sample one level after
// another, so every load instruction of the wave reads one level for 64
// consecutive samples (neighbouring samples share the lines of the coarse
// levels within one instruction) and a level's dense/hashed branch is
// uniform across the wave.  Dense levels take one load per x-neighbour
// pair.  On hashed levels the two lanes of a pair fetch the x-neighbour
// corners of one sample in the same load instruction (encode_level_lanepair:
// one 128-byte line per sample where a lane per sample asks for two), which
// halves the cache-line lookups of the fine levels, the kernel's bound
// (800x800 render: field 81.9 -> 54.8 ms; pairing only the even-x corners
// in one 8-byte load, as the encode kernel does, measured 11 % slower).
// The fp16 features go through LDS (rows of 80 bytes: 16-byte
// stores of four levels, 16-byte reads of lane group g's levels 4g..4g+3,
// no bank conflicts) into the MLP's B-operand layout, four 16-sample tiles
// per group; the SH coefficients go through LDS as in k_field_mlp.
constexpr uint32_t kFeatPitch = 40u;  // halves per LDS feature row (80 bytes)
template <typename TableT, bool kFromSamples>
__global__ __launch_bounds__(kBlockThreads) void k_field_forward_lv(GridParams g, const TableT* __restrict__ table, const half_t* __restrict__ dparams, const half_t* __restrict__ cparams, FieldInputs in, uint32_t n_cap,
                                                                   float4* __restrict__ out) {
    const uint32_t n = in.n_dev ? min(*in.n_dev, n_cap) : n_cap;
    __shared__ __align__(16) half_t sp[NERF_EXT_DENSITY_PARAMS + NERF_EXT_COLOR_PARAMS];
    __shared__ __align__(16) half_t feat[kBlockWaves][64 * kFeatPitch];
    __shared__ half4_t shl[kBlockWaves][64][4];
    __shared__ float dts[kBlockWaves][64];  // dt per sample (alpha_in_order)
    stage_weights<kBlockThreads>(sp, dparams, cparams);
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63u, grp = lane >> 4, s16 = lane & 15u, wv = threadIdx.x >> 6;
    DensityFrags fd;
    ColorFrags fc;
    load_density(sp, fd, lane);
    load_color(sp + NERF_EXT_DENSITY_PARAMS, fc, lane);
    half_t* F = feat[wv];
    // Round r covers groups [r * W, (r + 1) * W) (W = all waves), XCD x
    // (workgroups b with b % 8 == x) taking the x-th eighth of it.
    const uint32_t groups  = (n + 63u) / 64u;
    const uint32_t per_xcd = (gridDim.x >> 3) * kBlockWaves;
    const uint32_t first   = (blockIdx.x & 7u) * per_xcd + (blockIdx.x >> 3) * kBlockWaves + wv;
    for (uint32_t gi = first; gi < groups; gi += 8u * per_xcd) {
        const uint32_t s = gi * 64u + lane;
        const uint32_t q = s < n ? s : n - 1u;
        float p[3], d[3];
        if constexpr (kFromSamples) {
            const uint32_t qs = in.sample_index ? in.sample_index[q] : q;
            const uint32_t r  = sample_owner(in, q, qs);
            float dt;
            sample_point(in, qs, r, p, d, dt);
            dts[wv][lane] = dt;
        } else {
#pragma unroll
            for (int a = 0; a < 3; ++a) {
                p[a] = in.positions[3ull * q + a];
                d[a] = in.directions[3ull * q + a];
            }
        }
        float sh[16];
        sh16(d, sh);
#pragma unroll
        for (uint32_t j = 0; j < 4u; ++j) shl[wv][lane][j] = half4_t{to_half_rne(sh[4u * j]), to_half_rne(sh[4u * j + 1u]), to_half_rne(sh[4u * j + 2u]), to_half_rne(sh[4u * j + 3u])};
        // Gather, four levels per 16-byte LDS store.
#pragma unroll
        for (uint32_t k = 0; k < 4u; ++k) {
            half8_t h;
#pragma unroll
            for (uint32_t j = 0; j < 4u; ++j) {
                const uint32_t l = 4u * k + j;
                float a0 = 0.0f, a1 = 0.0f;
                if (l < g.n_levels) {
                    if (g.dense[l] != 0u) encode_level_xpair<TableT, false>(g, table, p, l, g.resolution[l], true, a0, a1);
                    else encode_level_lanepair<TableT>(g, table, p, l, g.resolution[l], false, a0, a1);
                }
                h[2u * j]      = to_half_rne(a0);
                h[2u * j + 1u] = to_half_rne(a1);
            }
            *reinterpret_cast<half8_t*>(F + lane * kFeatPitch + 8u * k) = h;
            if (in.features_out && s < n) *reinterpret_cast<half8_t*>(in.features_out + (uint64_t)s * 32u + 8u * k) = h;
        }
        __builtin_amdgcn_wave_barrier();  // LDS traffic of one wave completes in order
        float v[4];
#pragma unroll
        for (uint32_t t = 0; t < 4u; ++t) {
            const uint32_t row = 16u * t + s16;
            const half8_t x    = *reinterpret_cast<const half8_t*>(F + row * kFeatPitch + 8u * grp);
            const floatx4 o    = density_mlp(fd, x);
            const floatx4 c    = color_mlp(fc, color_input(o, shl[wv][row][grp], grp));
            v[t]               = field_channel(o, c, grp);
            if (kFromSamples && in.alpha_in_order && grp == 0u) v[t] = render_alpha(v[t], dts[wv][row]);
        }
#pragma unroll
        for (uint32_t t = 0; t < 4u; ++t) {
            const uint32_t st = gi * 64u + 16u * t + s16;
            if (st < n) {
                const uint32_t dst = (kFromSamples && in.sample_index && !in.alpha_in_order) ? in.sample_index[st] : st;
                reinterpret_cast<float*>(out)[4ull * dst + grp] = v[t];
            }
        }
        __builtin_amdgcn_wave_barrier();
    }
}

// MLP pass on given encodings, in groups of 64 samples (four 16-sample
// tiles) per wave.  Lane l first evaluates all 16 SH coefficients of sample
// l of the group and leaves them in LDS as fp16; lane (g, s) of tile t then
// reads coefficients 4g..4g+3 of sample 16t + s back (8 bytes) instead of
// evaluating the 16 polynomials and selecting four.  Lane (g, s) loads
// features 8g..8g+7 of sample s of each tile (one 16-byte load), the B
// operand of the density MLP.
//
// The 20 weight fragments (A operands: density 4 + 2, colour 4 + 8 + 2) live
// in LDS in lane order, 1 KiB each, and the group runs layer by layer over
// its four tiles: each fragment is read once per group (one conflict-free
// ds_read_b128) and feeds four MFMAs.  Holding them in registers instead
// costs 80 VGPRs per lane and limits the pass to 3 waves per SIMD; this way
// it runs 4 (2^24 samples: 434 vs 445 us; 2^18: 12.4 vs 17.7 us, where
// staging the weights once per workgroup dominated), with identical results.
//
// Directions come from a source: an array [n][3], or the owning rays of a
// march sample stream whose count is read on the device.
struct DirsFromArray {
    const float* dirs;
    uint32_t n;
    __device__ __forceinline__ uint32_t count() const { return n; }
    __device__ __forceinline__ void at(uint32_t q, float d[3]) const {
#pragma unroll
        for (int a = 0; a < 3; ++a) d[a] = dirs[3ull * q + a];
    }
};

struct DirsFromSamples {
    const uint32_t* sample_ray;
    const float4* rays;
    const uint32_t* n_dev;
    uint32_t cap;
    __device__ __forceinline__ uint32_t count() const { return n_dev ? min(*n_dev, cap) : cap; }
    __device__ __forceinline__ void at(uint32_t q, float d[3]) const {
        const float4 rd = rays[2ull * sample_ray[q] + 1ull];
        d[0]            = rd.x;
        d[1]            = rd.y;
        d[2]            = rd.z;
    }
};

// Features come from rows [n][32] or from level-major fp16 pairs (the
// sparse training batch's encode, which the backward reads too).
struct FeatsFromRows {
    const half_t* rows;
    __device__ __forceinline__ half8_t at(uint32_t q, uint32_t grp, bool) const { return *reinterpret_cast<const half8_t*>(rows + (uint64_t)q * 32u + 8u * grp); }
};
struct FeatsFromLevels {
    const uint32_t* lm;  // [16][stride]
    uint32_t stride;
    __device__ __forceinline__ half8_t at(uint32_t q, uint32_t grp, bool) const {
        uint32_t v[4];
#pragma unroll
        for (uint32_t j = 0; j < 4u; ++j) v[j] = lm[(uint64_t)(4u * grp + j) * stride + q];
        return __builtin_bit_cast(half8_t, v);
    }
};

template <typename Dirs, typename Feats>
__global__ __launch_bounds__(kBlockThreads) __attribute__((amdgpu_waves_per_eu(kMlpWaves, 8))) void k_field_mlp(const half_t* __restrict__ dparams, const half_t* __restrict__ cparams, Feats features,
                                                                                                                  Dirs dirs, float4* __restrict__ out) {
    const uint32_t n = dirs.count();
    __shared__ __align__(16) half8_t frag[kFieldFrags][kWaveSize];
    __shared__ half4_t shl[kBlockWaves][kGroupSamples][4];
    const uint32_t lane = threadIdx.x & 63u, grp = lane >> 4, s16 = lane & 15u, wv = threadIdx.x >> 6;
    for (uint32_t f = wv; f < kFieldFrags; f += kBlockWaves) frag[f][lane] = mlp_fragment(dparams, cparams, f, lane);
    __syncthreads();
    const uint32_t groups = (n + kGroupSamples - 1u) / kGroupSamples;
    const uint32_t nwaves = gridDim.x * kBlockWaves;
    const floatx4 zero    = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t gi = blockIdx.x * kBlockWaves + wv; gi < groups; gi += nwaves) {
        const uint32_t base = gi * kGroupSamples;
        // The fragment reads stay inside the loop (an opaque lane offset):
        // hoisted, they would be the 80 VGPRs this layout saves.
        uint32_t lo = lane;
        asm volatile("" : "+v"(lo));
        const half8_t* W = &frag[0][0] + lo;
        half8_t x[4];
#pragma unroll
        for (uint32_t t = 0; t < 4u; ++t) {
            const uint32_t q = min(base + 16u * t + s16, n - 1u);
            x[t]             = features.at(q, grp, base + 16u * t + s16 < n);
        }
        float d[3];
        dirs.at(min(base + lane, n - 1u), d);
        float sh[16];
        sh16(d, sh);
#pragma unroll
        for (uint32_t j = 0; j < 4u; ++j)
            shl[wv][lane][j] = half4_t{to_half_rne(sh[4u * j]), to_half_rne(sh[4u * j + 1u]), to_half_rne(sh[4u * j + 2u]), to_half_rne(sh[4u * j + 3u])};
        __builtin_amdgcn_wave_barrier();  // LDS traffic of one wave completes in order
        half4_t h[4][4], h2[4][4];
        floatx4 o[4], c[4];
        // Density 32 -> 64 (ReLU) -> 16.
#pragma unroll
        for (uint32_t b = 0; b < 4u; ++b) {
            const half8_t w = W[64u * b];
#pragma unroll
            for (uint32_t t = 0; t < 4u; ++t) h[t][b] = relu_half(mfma16x16x32(w, x[t], zero));
        }
        {
            const half8_t w0 = W[64u * 4u], w1 = W[64u * 5u];
#pragma unroll
            for (uint32_t t = 0; t < 4u; ++t) o[t] = mfma16x16x32(w1, cat(h[t][2], h[t][3]), mfma16x16x32(w0, cat(h[t][0], h[t][1]), zero));
        }
        // Colour 32 -> 64 -> 64 (ReLU both) -> 16 (rows 4, 8, 12 used).
        half8_t xc[4];
#pragma unroll
        for (uint32_t t = 0; t < 4u; ++t) xc[t] = color_input(o[t], shl[wv][16u * t + s16][grp], grp);
#pragma unroll
        for (uint32_t b = 0; b < 4u; ++b) {
            const half8_t w = W[64u * (6u + b)];
#pragma unroll
            for (uint32_t t = 0; t < 4u; ++t) h[t][b] = relu_half(mfma16x16x32(w, xc[t], zero));
        }
#pragma unroll
        for (uint32_t b = 0; b < 4u; ++b) {
            const half8_t w0 = W[64u * (10u + 2u * b)], w1 = W[64u * (11u + 2u * b)];
#pragma unroll
            for (uint32_t t = 0; t < 4u; ++t) h2[t][b] = relu_half(mfma16x16x32(w1, cat(h[t][2], h[t][3]), mfma16x16x32(w0, cat(h[t][0], h[t][1]), zero)));
        }
        {
            const half8_t w0 = W[64u * 18u], w1 = W[64u * 19u];
#pragma unroll
            for (uint32_t t = 0; t < 4u; ++t) c[t] = mfma16x16x32(w1, cat(h2[t][2], h2[t][3]), mfma16x16x32(w0, cat(h2[t][0], h2[t][1]), zero));
        }
#pragma unroll
        for (uint32_t t = 0; t < 4u; ++t) {
            const uint32_t s = base + 16u * t + s16;
            const float v    = field_channel(o[t], c[t], grp);
            if (s < n) reinterpret_cast<float*>(out)[4ull * s + grp] = v;
        }
        __builtin_amdgcn_wave_barrier();
    }
}

// Twice as many workgroups as stay resident (4 per CU at 4 waves per SIMD):
// the second half refills CUs whose first workgroups finish early, which
// evens out the end of the pass (2^22 samples: 4 per CU 103-110 us, 6 per CU
// 96-100 us, 8 per CU 97-99 us, 16 per CU 99 us); the fragment build per
// workgroup (20 KiB from L2) stays small beside the groups each one runs.
uint32_t mlp_pass_blocks(uint32_t n) {
    const uint32_t groups = (n + kGroupSamples - 1u) / kGroupSamples;
    return max(1u, min((groups + kBlockWaves - 1u) / kBlockWaves, device_cu_count() * 2u * kMlpWaves));
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
    // Renders (more than 2^20 samples) take the level-major kernel, 3
    // workgroups per CU (its LDS and register budget); training-sized
    // batches the tile kernel, whose 16-sample tiles leave a shorter tail
    // when a launch is only one or two rounds of work (2^18 samples: 67 vs
    // 93 us).  The tile kernel runs 4 workgroups per CU: 2^18 samples are
    // 16,384 tiles, exactly 4 per wave (67 us; 3 per CU leave 5 or 6 tiles
    // per wave, 71 us; 5 and 6 per CU, 77 us).  The level-major kernel
    // measured no faster with its fragments in LDS (49.9 vs 49.8 ms per
    // render) and slower with 8-wave workgroups at 4 waves per SIMD (52.5
    // ms: more waves than its L1 serves).
    const bool level_major  = n > (1u << 20);
    const uint32_t blocks   = (persistent_blocks(n, level_major ? 3u : 4u) + 7u) / 8u * 8u;  // whole XCD rounds
    const bool from_samples = in.samples != nullptr;
    if (in.sparse && from_samples && in.features_out && !in.sample_index && !in.alpha_in_order && g.table_dtype != NERF_EXT_F32 && g.n_levels == 16u) {
        // Sparse samples: encode level group by level group, one group per
        // XCD, into features_out, then the MLPs over those features.
        const hipError_t e = launch_encode_samples(g, (const half_t*)table, in, n, in.features_out, in.features_lm, stream);
        if (e != hipSuccess) return e;
        const DirsFromSamples dirs{in.sample_ray, in.rays, in.n_dev, n};
        if (in.features_lm)
            k_field_mlp<<<mlp_pass_blocks(n), kBlockThreads, 0, stream>>>(w.density, w.color, FeatsFromLevels{in.features_lm, n}, dirs, out4);
        else
            k_field_mlp<<<mlp_pass_blocks(n), kBlockThreads, 0, stream>>>(w.density, w.color, FeatsFromRows{in.features_out}, dirs, out4);
        return hipGetLastError();
    }
#define NERF_FIELD_LAUNCH(K)                                                                                                                   \
    do {                                                                                                                                       \
        if (g.table_dtype == NERF_EXT_F32) {                                                                                                   \
            if (from_samples) K<float, true><<<blocks, kBlockThreads, 0, stream>>>(g, (const float*)table, w.density, w.color, in, n, out4);      \
            else K<float, false><<<blocks, kBlockThreads, 0, stream>>>(g, (const float*)table, w.density, w.color, in, n, out4);                \
        } else {                                                                                                                               \
            if (from_samples) K<half_t, true><<<blocks, kBlockThreads, 0, stream>>>(g, (const half_t*)table, w.density, w.color, in, n, out4);  \
            else K<half_t, false><<<blocks, kBlockThreads, 0, stream>>>(g, (const half_t*)table, w.density, w.color, in, n, out4);              \
        }                                                                                                                                      \
    } while (0)
    if (level_major) NERF_FIELD_LAUNCH(k_field_forward_lv);
    else NERF_FIELD_LAUNCH(k_field_forward);
#undef NERF_FIELD_LAUNCH
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

NERF_API NerfStatus nerf_ext_field_mlp(const uint16_t* density_params, const uint16_t* color_params, const uint16_t* features, const float* directions, uint32_t n, float* out, void* stream) {
    if (n == 0u) return NERF_STATUS_OK;
    NERF_CHECK_ARG(density_params && color_params && features && directions && out, "nerf_ext_field_mlp: null pointer");
    NERF_CHECK_ARG(((uintptr_t)features & 15u) == 0u, "nerf_ext_field_mlp: features must be 16-byte aligned");
    k_field_mlp<<<mlp_pass_blocks(n), kBlockThreads, 0, (hipStream_t)stream>>>((const half_t*)density_params, (const half_t*)color_params, FeatsFromRows{(const half_t*)features}, DirsFromArray{directions, n},
                                                                                reinterpret_cast<float4*>(out));
    NERF_LAUNCH_CHECK("k_field_mlp");
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_field_forward(const NerfExtModel* model, const float* positions, const float* directions, uint32_t n, float* out, void* stream) {
    NERF_CHECK_ARG(model, "nerf_ext_field_forward: null model");
    NERF_CHECK_ARG(model->kind <= NERF_EXT_MODEL_REFERENCE, "nerf_ext_field_forward: unknown model kind");
    if (model->kind == NERF_EXT_MODEL_REFERENCE) return nerf_ext_ref_field_forward(model->density_params, model->color_params, positions, directions, n, out, nullptr, stream);
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
