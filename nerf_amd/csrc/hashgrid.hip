// hashgrid.hip — multiresolution hash-grid encoding (Mueller et al., "Instant
// Neural Graphics Primitives", SIGGRAPH 2022, section 3).  The reference has no
// hash grid (its encoder is the frequency encoding of backend-cuda.cu:252-277);
// the semantics below are the published ones, fixed in detail by
// include/nerf_ext.h and restated scalar by the CPU oracle.
//
// Standalone forward kernel layout: grid.y = level, so at any moment the
// resident workgroups gather from one or two levels' tables and each XCD's L2
// holds the level being read (512 KiB per level for T = 2^16 fp32, 2 MiB for
// T = 2^19 fp16).
#include <math.h>

#include "common.hpp"

namespace nerf_hip {

NerfStatus make_grid(const NerfExtGridDesc* d, GridParams& g) {
    NERF_CHECK_ARG(d, "grid descriptor is null");
    NERF_CHECK_ARG(d->n_levels >= 1u && d->n_levels <= NERF_EXT_MAX_LEVELS, "grid: n_levels must be 1..16");
    NERF_CHECK_ARG(d->n_features == 2u, "grid: n_features must be 2");
    NERF_CHECK_ARG(d->log2_table_size >= 2u && d->log2_table_size <= 24u, "grid: log2_table_size must be 2..24");
    NERF_CHECK_ARG(d->base_resolution >= 1u, "grid: base_resolution must be >= 1");
    NERF_CHECK_ARG(d->table_dtype == NERF_EXT_F32 || d->table_dtype == NERF_EXT_F16, "grid: table_dtype must be F32 or F16");
    double b = (double)d->per_level_scale;
    if (d->finest_resolution > 0u && d->n_levels > 1u) b = exp(log((double)d->finest_resolution / (double)d->base_resolution) / (double)(d->n_levels - 1u));
    NERF_CHECK_ARG(b >= 1.0, "grid: per-level scale must be >= 1");
    g.n_levels    = d->n_levels;
    g.n_features  = d->n_features;
    g.table_size  = 1u << d->log2_table_size;
    g.table_dtype = d->table_dtype;
    for (uint32_t l = 0; l < NERF_EXT_MAX_LEVELS; ++l) {
        g.resolution[l] = 0u;
        g.dense[l]      = 0u;
    }
    for (uint32_t l = 0; l < d->n_levels; ++l) {
        const double nl = floor((double)d->base_resolution * pow(b, (double)l) + 1e-9);
        NERF_CHECK_ARG(nl >= 1.0 && nl < 16777216.0, "grid: level resolution out of range (must be < 2^24)");
        g.resolution[l]  = (uint32_t)nl;
        const uint64_t v = (uint64_t)g.resolution[l] + 1ull;
        g.dense[l]       = (v * v * v <= (uint64_t)g.table_size) ? 1u : 0u;
    }
    return NERF_STATUS_OK;
}

// Table init: element i (memory order) = U(-range, range) from splitmix64
// stream (0x7ab1e, seed), the same generator as the reference's weight init
// (backend-cuda.cu:1819-1824) evaluated at its closed form per element.
__device__ __forceinline__ void store_value(float* p, float v) { *p = v; }
__device__ __forceinline__ void store_value(half_t* p, float v) { *p = to_half_rne(v); }

template <typename T>
__global__ __launch_bounds__(256) void k_init_table(T* table, uint64_t count, uint64_t state0, float range) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride) {
        const float u = nerf_math::unit24(nerf_math::splitmix_at(state0, i));
        store_value(table + i, (u * 2.0f - 1.0f) * range);
    }
}

// Tile encode, for tables too large for the level split: workgroup of 16
// points x 16 level slots, thread (level l, point p) =
// threadIdx.x = 16 l + p gathers the 8 corners of one level of one point.
// The 16 positions are staged in LDS once, and the 16 x 2L features go out
// through an LDS tile as one contiguous store of the workgroup's points.
constexpr uint32_t kEncPoints = 16u;

template <typename TableT, typename OutT>
__global__ __launch_bounds__(256) void k_encode_tile(GridParams g, const TableT* __restrict__ table, const float* __restrict__ pos, uint32_t n, OutT* __restrict__ out) {
    __shared__ float sp[3u * kEncPoints];
    __shared__ OutT tile[kEncPoints * 2u * NERF_EXT_MAX_LEVELS];
    const uint32_t first = blockIdx.x * kEncPoints;
    const uint32_t count = n - first < kEncPoints ? n - first : kEncPoints;
    if (threadIdx.x < 3u * count) sp[threadIdx.x] = pos[3ull * first + threadIdx.x];
    __syncthreads();
    const uint32_t p = threadIdx.x & (kEncPoints - 1u), level = threadIdx.x / kEncPoints;
    const uint32_t width = 2u * g.n_levels;
    if (level < g.n_levels) {  // uniform over the 16 lanes of a level
        // Lanes p and p ^ 1 fetch each other's x-neighbour corners
        // (encode_level_lanepair), so lanes past the last point gather too.
        const uint32_t pq = p < count ? p : count - 1u;
        const float x[3]  = {sp[3u * pq], sp[3u * pq + 1u], sp[3u * pq + 2u]};
        float a0, a1;
        encode_level_lanepair(g, table, x, level, g.resolution[level], g.dense[level] != 0u, a0, a1);
        if (p < count) {
            store_value(&tile[p * width + 2u * level], a0);
            store_value(&tile[p * width + 2u * level + 1u], a1);
        }
    }
    __syncthreads();
    OutT* o = out + (uint64_t)first * width;
    for (uint32_t i = threadIdx.x; i < count * width; i += blockDim.x) o[i] = tile[i];
}

// XCD-aware encode.  Workgroup b runs on XCD b % 8 (the dispatcher's round
// robin) and gathers only kLevels levels of the table, so each XCD's L2
// holds those levels rather than all of them:
//   * kLevels = 2: XCD x takes levels 2x, 2x + 1 for every point;
//   * kLevels = 4 (16 levels): XCD x takes levels 4 (x % 4) .. + 3 for the
//     points of every other 256-point block (x / 4 picks which), so a point's
//     position is read by 4 XCDs instead of 8 and each thread writes 32
//     contiguous bytes of the output row instead of 16;
//   * kLevels = 1 (16 levels): XCD x takes level x + 8 phase for every
//     point, so its L2 holds one level; phase 2 runs phase 0 on the first
//     half of the workgroups and phase 1 on the second.
// One point per thread (the launch gives every thread exactly one).  The
// placement is a locality choice only: any workgroup-to-XCD mapping gives
// the same result.  The x-neighbour corners of a dense level are adjacent
// entries, fetched by one load; on a hashed level the lanes of a pair fetch
// them for each other's points in one load instruction (one cache line per
// point and edge; encode_level_lanepair), so every lane runs the gathers and
// only lanes holding a point store.
// Points come from a source (PointsFromArray, PointsFromSamples) whose count
// may be read on the device.
// With lm (fp16 output only), the features go level-major instead: level
// l's pair of sample i at lm[l * lm_stride + i] (a workgroup writes whole
// lines; rows of [n][32] would collect their 16 levels from 8 XCDs' L2s as
// partial lines: 134 MB written per 4,096 x 64-step batch for 16 MB of
// features).
template <typename TableT, typename OutT, uint32_t kLevels, typename Points>
__global__ __launch_bounds__(256) void k_encode_split(GridParams g, const TableT* __restrict__ table, Points src, OutT* __restrict__ out, bool nt, uint32_t phase, uint32_t* __restrict__ lm = nullptr,
                                                      uint32_t lm_stride = 0u) {
    constexpr uint32_t kParts = kLevels >= 2u ? kLevels / 2u : 1u;  // XCDs sharing one level group
    const uint32_t xcd = blockIdx.x & 7u, group = xcd % (8u / kParts), part = xcd / (8u / kParts);
    uint32_t slot = blockIdx.x >> 3, slots = gridDim.x >> 3;
    if (kLevels == 1u && phase > 1u) {  // both phases in one launch: the first half of the slots, then the second
        slots /= 2u;
        phase = slot >= slots ? 1u : 0u;
        slot -= phase * slots;
    }
    const uint32_t l0 = kLevels * group + (kLevels == 1u ? 8u * phase : 0u);
    if (l0 >= g.n_levels) return;  // uniform per workgroup
    const uint32_t n = src.count();
    const uint32_t width = 2u * g.n_levels;
    for (uint32_t blk = slot * kParts + part; blk * 256u < n; blk += slots * kParts) {
        const uint32_t i  = blk * 256u + threadIdx.x;
        const uint32_t iq = i < n ? i : n - 1u;
        float x[3];
        src.at(iq, x);
        float f[2u * kLevels];
#pragma unroll
        for (uint32_t j = 0; j < kLevels; ++j) {
            const uint32_t l = l0 + j;
            f[2u * j] = f[2u * j + 1u] = 0.0f;
            if (l < g.n_levels) {
                if (g.dense[l] != 0u) encode_level_xpair(g, table, x, l, g.resolution[l], true, f[2u * j], f[2u * j + 1u]);
                else encode_level_lanepair(g, table, x, l, g.resolution[l], false, f[2u * j], f[2u * j + 1u]);
            }
        }
        if (i >= n) continue;
        if constexpr (sizeof(OutT) == 2u) {
            if (lm) {
#pragma unroll
                for (uint32_t j = 0; j < kLevels; ++j)
                    if (l0 + j < g.n_levels)
                        lm[(uint64_t)(l0 + j) * lm_stride + i] =
                            (uint32_t)__builtin_bit_cast(uint16_t, to_half_rne(f[2u * j])) | ((uint32_t)__builtin_bit_cast(uint16_t, to_half_rne(f[2u * j + 1u])) << 16);
                continue;
            }
        }
        OutT* o = out + (uint64_t)i * width + 2u * l0;
        if (l0 + kLevels <= g.n_levels) {  // uniform: every level of the group exists
            // 16-byte stores.  With nt (large launches) non-temporal: the
            // features are written once and not read back here, and keeping
            // them out of L2 leaves it to the table (2^24 points: 4.93 ->
            // 4.57 ms); small launches are faster with ordinary stores.
            if constexpr (sizeof(OutT) == 4u) {
#pragma unroll
                for (uint32_t q = 0; q < kLevels / 2u; ++q) {
                    const floatx4 v = floatx4{f[4u * q], f[4u * q + 1u], f[4u * q + 2u], f[4u * q + 3u]};
                    if (nt) __builtin_nontemporal_store(v, reinterpret_cast<floatx4*>(o) + q);
                    else reinterpret_cast<floatx4*>(o)[q] = v;
                }
            } else {
#pragma unroll
                for (uint32_t q = 0; q < kLevels / 4u; ++q) {
                    const half8_t v = half8_t{to_half_rne(f[8u * q]), to_half_rne(f[8u * q + 1u]), to_half_rne(f[8u * q + 2u]), to_half_rne(f[8u * q + 3u]), to_half_rne(f[8u * q + 4u]), to_half_rne(f[8u * q + 5u]),
                                              to_half_rne(f[8u * q + 6u]), to_half_rne(f[8u * q + 7u])};
                    if (nt) __builtin_nontemporal_store(v, reinterpret_cast<half8_t*>(o) + q);
                    else reinterpret_cast<half8_t*>(o)[q] = v;
                }
                if constexpr (kLevels % 4u != 0u) {
#pragma unroll
                    for (uint32_t j = 4u * (kLevels / 4u); j < kLevels; ++j) {
                        const uint32_t v = (uint32_t)__builtin_bit_cast(uint16_t, to_half_rne(f[2u * j])) | ((uint32_t)__builtin_bit_cast(uint16_t, to_half_rne(f[2u * j + 1u])) << 16);
                        *reinterpret_cast<uint32_t*>(o + 2u * j) = v;
                    }
                }
            }
        } else {
#pragma unroll
            for (uint32_t j = 0; j < kLevels; ++j) {
                if (l0 + j < g.n_levels) {
                    store_value(o + 2u * j, f[2u * j]);
                    store_value(o + 2u * j + 1u, f[2u * j + 1u]);
                }
            }
        }
    }
}

__global__ __launch_bounds__(256) void k_encode_indices(GridParams g, const float* __restrict__ pos, uint32_t n, uint32_t* __restrict__ indices, float* __restrict__ weights) {
    const uint32_t level = blockIdx.y;
    const uint32_t i     = blockIdx.x * 256u + threadIdx.x;
    if (i >= n) return;
    const float p[3]  = {pos[3ull * i], pos[3ull * i + 1], pos[3ull * i + 2]};
    const uint32_t N  = g.resolution[level];
    const LevelCell c = level_cell(p, N);
    const uint64_t o  = ((uint64_t)i * g.n_levels + level) * 8u;
#pragma unroll
    for (uint32_t k = 0; k < 8u; ++k) {
        if (indices) indices[o + k] = corner_index(c, k, N, g.dense[level] != 0u, g.table_size - 1u);
        if (weights) weights[o + k] = corner_weight(c, k);
    }
}

hipError_t launch_encode_samples(const GridParams& g, const half_t* table, const FieldInputs& in, uint32_t cap, half_t* features, uint32_t* lm, hipStream_t stream) {
    if (cap == 0u) return hipSuccess;
    if (g.n_levels != 16u || g.table_dtype != NERF_EXT_F16) return hipErrorInvalidValue;
    PointsFromSamples src{in.samples, in.sample_ray, in.rays, in.n_dev, cap, {in.bmin[0], in.bmin[1], in.bmin[2]}, {in.bmax[0], in.bmax[1], in.bmax[2]}};
    const uint64_t level_bytes = (uint64_t)g.table_size * g.n_features * 2u;
    const uint32_t blocks_256  = (cap + 255u) / 256u;
    // Four levels per XCD when four fit in half of its L2; else one level per
    // XCD in two phases (levels 0-7, then 8-15; one launch whose second half
    // of workgroups, dispatched after the first, takes the second phase):
    // with T = 2^19 fp16 a level is 2 MiB, and two of them (4 MiB) left no
    // room in the XCD's L2 for the feature rows streaming through it (the
    // reference host's 4,096 rays x <= 64 steps: 117 us for two levels per
    // XCD, 95 us for the two phases as two launches).
    if (4u * level_bytes <= (2ull << 20)) {
        k_encode_split<half_t, half_t, 4u><<<8u * ((blocks_256 + 1u) / 2u), 256, 0, stream>>>(g, table, src, features, false, 0u, lm, cap);
    } else {
        k_encode_split<half_t, half_t, 1u><<<16u * blocks_256, 256, 0, stream>>>(g, table, src, features, false, 2u, lm, cap);
    }
    return hipGetLastError();
}

}  // namespace nerf_hip

using namespace nerf_hip;

extern "C" {

NERF_API NerfStatus nerf_ext_grid_levels(const NerfExtGridDesc* grid, NerfExtGridLevels* out) {
    NERF_CHECK_ARG(out, "nerf_ext_grid_levels: null output");
    GridParams g;
    const NerfStatus s = make_grid(grid, g);
    if (s != NERF_STATUS_OK) return s;
    out->n_levels   = g.n_levels;
    out->table_size = g.table_size;
    for (uint32_t l = 0; l < NERF_EXT_MAX_LEVELS; ++l) {
        out->resolution[l] = g.resolution[l];
        out->dense[l]      = g.dense[l];
    }
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_grid_init_table(const NerfExtGridDesc* grid, uint64_t seed, float range, void* table, void* stream) {
    GridParams g;
    const NerfStatus s = make_grid(grid, g);
    if (s != NERF_STATUS_OK) return s;
    NERF_CHECK_ARG(table, "nerf_ext_grid_init_table: null table");
    const uint64_t count  = (uint64_t)g.n_levels * g.table_size * g.n_features;
    const uint64_t state0 = nerf_math::stream_state(0x7ab1eull, seed);
    const uint32_t blocks = (uint32_t)((count + 255u) / 256u < 65536u ? (count + 255u) / 256u : 65536u);
    if (g.table_dtype == NERF_EXT_F32)
        k_init_table<float><<<blocks, 256, 0, (hipStream_t)stream>>>((float*)table, count, state0, range);
    else
        k_init_table<half_t><<<blocks, 256, 0, (hipStream_t)stream>>>((half_t*)table, count, state0, range);
    NERF_LAUNCH_CHECK("k_init_table");
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_encode_forward(const NerfExtGridDesc* grid, const void* table, const float* positions, uint32_t n, void* features, uint32_t features_dtype, void* stream) {
    GridParams g;
    const NerfStatus s = make_grid(grid, g);
    if (s != NERF_STATUS_OK) return s;
    if (n == 0u) return NERF_STATUS_OK;
    NERF_CHECK_ARG(table && positions && features, "nerf_ext_encode_forward: null pointer");
    NERF_CHECK_ARG(features_dtype == NERF_EXT_F32 || features_dtype == NERF_EXT_F16, "nerf_ext_encode_forward: bad features dtype");
    hipStream_t st = (hipStream_t)stream;
    // Level split when two levels of the table fit in one XCD's L2 (4 MiB),
    // four levels per XCD when four fit in half of it (16-level grids only);
    // otherwise every workgroup gathers all levels.  (fp16 T = 2^19, two 2 MiB
    // levels per XCD: 2^18 random points 188 -> 113 us against all levels
    // per workgroup.)
    const uint64_t level_bytes = (uint64_t)g.table_size * g.n_features * (g.table_dtype == NERF_EXT_F32 ? 4u : 2u);
    const bool split           = 2u * level_bytes <= (4ull << 20);
    const bool quad            = split && g.n_levels == 16u && 4u * level_bytes <= (2ull << 20);
    // One point per thread (no persistent grid): workgroups that finish early
    // are replaced by new ones, so the CUs stay full to the end instead of
    // draining through a long tail of the oldest-first wave scheduling.
    const uint32_t blocks_256 = (n + 255u) / 256u;
    const bool nt             = n >= (1u << 20);  // non-temporal feature stores for large launches
    const dim3 grid_dim = quad ? dim3(8u * ((blocks_256 + 1u) / 2u)) : split ? dim3(8u * blocks_256) : dim3((n + kEncPoints - 1u) / kEncPoints);
#define NERF_ENC(TT, OT)                                                                                                   \
    do {                                                                                                                   \
        if (quad)                                                                                                          \
            k_encode_split<TT, OT, 4u><<<grid_dim, 256, 0, st>>>(g, (const TT*)table, PointsFromArray{positions, n}, (OT*)features, nt, 0u);  \
        else if (split)                                                                                                    \
            k_encode_split<TT, OT, 2u><<<grid_dim, 256, 0, st>>>(g, (const TT*)table, PointsFromArray{positions, n}, (OT*)features, nt, 0u);  \
        else                                                                                                               \
            k_encode_tile<TT, OT><<<grid_dim, 256, 0, st>>>(g, (const TT*)table, positions, n, (OT*)features);             \
    } while (0)
    if (g.table_dtype == NERF_EXT_F32) {
        if (features_dtype == NERF_EXT_F32) NERF_ENC(float, float);
        else NERF_ENC(float, half_t);
    } else {
        if (features_dtype == NERF_EXT_F32) NERF_ENC(half_t, float);
        else NERF_ENC(half_t, half_t);
    }
#undef NERF_ENC
    NERF_LAUNCH_CHECK("k_encode_forward");
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_encode_indices(const NerfExtGridDesc* grid, const float* positions, uint32_t n, uint32_t* indices, float* weights, void* stream) {
    GridParams g;
    const NerfStatus s = make_grid(grid, g);
    if (s != NERF_STATUS_OK) return s;
    if (n == 0u) return NERF_STATUS_OK;
    NERF_CHECK_ARG(positions && (indices || weights), "nerf_ext_encode_indices: null pointer");
    const dim3 grid_dim((n + 255u) / 256u, g.n_levels);
    k_encode_indices<<<grid_dim, 256, 0, (hipStream_t)stream>>>(g, positions, n, indices, weights);
    NERF_LAUNCH_CHECK("k_encode_indices");
    return NERF_STATUS_OK;
}

}  // extern "C"
