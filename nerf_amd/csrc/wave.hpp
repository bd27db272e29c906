// wave.hpp — wavefront-wide scans and reductions (wave64) for the
// one-wave-per-ray kernels: march sample compaction and compositing.
#pragma once

#include "common.hpp"

namespace nerf_hip {
namespace wave {

__device__ __forceinline__ uint32_t lane_id() { return threadIdx.x & 63u; }

// Inclusive scans over the 64 lanes (Hillis-Steele, log2(64) = 6 steps).
__device__ __forceinline__ float inclusive_sum(float v) {
    const uint32_t lane = lane_id();
#pragma unroll
    for (uint32_t d = 1; d < 64u; d <<= 1) {
        const float o = __shfl_up(v, d, 64);
        if (lane >= d) v += o;
    }
    return v;
}

__device__ __forceinline__ float inclusive_product(float v) {
    const uint32_t lane = lane_id();
#pragma unroll
    for (uint32_t d = 1; d < 64u; d <<= 1) {
        const float o = __shfl_up(v, d, 64);
        if (lane >= d) v *= o;
    }
    return v;
}

__device__ __forceinline__ float sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float broadcast(float v, uint32_t lane) { return __shfl(v, (int)lane, 64); }

// Number of set bits of `mask` below this lane.
__device__ __forceinline__ uint32_t rank_below(uint64_t mask) {
    const uint32_t lane = lane_id();
    const uint64_t below = lane == 0u ? 0ull : (mask & (~0ull >> (64u - lane)));
    return (uint32_t)__popcll(below);
}

// Occupancy march of one ray by a group of G lanes (G divides 64; the wave
// marches 64 / G rays), with the step rule of backend-cuda.cu:450-469.  The
// lanes of a group run the same scalar recurrence for t, so t and dt are
// bit-identical to a one-thread march; lane j of the group keeps step i + j of
// each run of G steps, the G occupancy tests run in parallel, and
// emit(k, t_mid, dt) is called by the lanes holding the k-th occupied step
// with k < limit, consecutive k on consecutive lanes.  Returns the number of
// occupied steps seen (all of them when limit is ~0u).  Larger G shortens a
// ray's latency chain; smaller G shares each recurrence instruction among
// more rays.
template <uint32_t G, typename Occupied, typename Emit>
__device__ __forceinline__ uint32_t march(float4 ro, float4 rd, float cone, uint32_t max_steps, uint32_t limit, Occupied occupied, Emit emit) {
    static_assert(G >= 1u && G <= 64u && 64u % G == 0u, "group size must divide 64");
    const uint32_t lane = lane_id(), j_own = lane % G, shift = lane - j_own;
    const uint64_t group_bits = G == 64u ? ~0ull : ((1ull << G) - 1ull);
    const float tn = ro.w, tf = rd.w;
    if (!(tf - tn > 0.0f)) return 0u;
    const float dt_min = (tf - tn) / (float)max_steps;
    float t = tn;
    uint32_t i = 0u, seen = 0u;
    while (t < tf && i < max_steps && seen < limit) {
        float my_tm = 0.0f, my_dt = 0.0f;
        bool has = false;
        for (uint32_t j = 0; j < G && t < tf && i < max_steps; ++j, ++i) {
            const float dt = fminf(fmaxf(dt_min, t * cone), tf - t);
            const float tm = t + 0.5f * dt;
            if (j_own == j) {
                my_tm = tm;
                my_dt = dt;
                has   = true;
            }
            t += dt;
        }
        const float p[3]    = {ro.x + my_tm * rd.x, ro.y + my_tm * rd.y, ro.z + my_tm * rd.z};
        const bool hit      = has && occupied(p);
        const uint64_t mask = (__ballot(hit) >> shift) & group_bits;
        const uint32_t k    = seen + (uint32_t)__popcll(mask & ((1ull << j_own) - 1ull));
        if (hit && k < limit) emit(k, my_tm, my_dt);
        seen += (uint32_t)__popcll(mask);
    }
    return seen;
}

}  // namespace wave
}  // namespace nerf_hip
