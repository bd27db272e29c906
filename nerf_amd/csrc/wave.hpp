// wave.hpp — wavefront-wide scans and reductions (wave64) for the
// one-wave-per-ray kernels: march sample compaction and compositing.
#pragma once

#include "common.hpp"

namespace nerf_hip {
namespace wave {

__device__ __forceinline__ uint32_t lane_id() { return threadIdx.x & 63u; }

// Wave-wide scans and broadcasts on DPP lane moves (VALU only, no LDS round
// trip): an inclusive scan is four row shifts (1, 2, 4, 8 lanes within each
// row of 16) and two row broadcasts (lane 15 of a row into the next row,
// lane 31 into rows 2 and 3); a lane whose source is outside its row keeps
// the identity.  With __shfl_up each of the six steps was a ds_bpermute and
// a wait (about 25 serial LDS round trips per 64-sample group in the
// composite backward).  The association differs from a sequential product
// or sum by rounding only.
namespace dpp {
constexpr int kRowShr1 = 0x111, kRowShr2 = 0x112, kRowShr4 = 0x114, kRowShr8 = 0x118;
constexpr int kRowBcast15 = 0x142, kRowBcast31 = 0x143, kWaveShr1 = 0x138;
template <int kCtrl, int kRowMask = 0xf>
__device__ __forceinline__ float move(float v, float fill) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(fill), __float_as_int(v), kCtrl, kRowMask, 0xf, false));
}
}  // namespace dpp

__device__ __forceinline__ float inclusive_sum(float v) {
    v += dpp::move<dpp::kRowShr1>(v, 0.0f);
    v += dpp::move<dpp::kRowShr2>(v, 0.0f);
    v += dpp::move<dpp::kRowShr4>(v, 0.0f);
    v += dpp::move<dpp::kRowShr8>(v, 0.0f);
    v += dpp::move<dpp::kRowBcast15, 0xa>(v, 0.0f);
    v += dpp::move<dpp::kRowBcast31, 0xc>(v, 0.0f);
    return v;
}

__device__ __forceinline__ float inclusive_product(float v) {
    v *= dpp::move<dpp::kRowShr1>(v, 1.0f);
    v *= dpp::move<dpp::kRowShr2>(v, 1.0f);
    v *= dpp::move<dpp::kRowShr4>(v, 1.0f);
    v *= dpp::move<dpp::kRowShr8>(v, 1.0f);
    v *= dpp::move<dpp::kRowBcast15, 0xa>(v, 1.0f);
    v *= dpp::move<dpp::kRowBcast31, 0xc>(v, 1.0f);
    return v;
}

// The value of the lane below (lane 0: fill), e.g. an exclusive scan from an
// inclusive one.
__device__ __forceinline__ float shift_up1(float v, float fill) { return dpp::move<dpp::kWaveShr1>(v, fill); }

// `lane` must be the same on every lane of the wave.
__device__ __forceinline__ float broadcast(float v, uint32_t lane) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), (int)lane)); }

__device__ __forceinline__ float sum(float v) { return broadcast(inclusive_sum(v), 63u); }

// Number of set bits of `mask` below this lane.
__device__ __forceinline__ uint32_t rank_below(uint64_t mask) {
    const uint32_t lane = lane_id();
    const uint64_t below = lane == 0u ? 0ull : (mask & (~0ull >> (64u - lane)));
    return (uint32_t)__popcll(below);
}

constexpr uint32_t kOutside = 0xFFFFFFFFu;

// Occupancy march of one ray by a group of G lanes (G divides 64; the wave
// marches 64 / G rays), with the step rule of backend-cuda.cu:450-469.  The
// lanes of a group run the same scalar recurrence for t, so t and dt are
// bit-identical to a one-thread march; lane j of the group keeps step i + j of
// each run of G steps and tests its cell: cell(p) gives the cell index or
// kOutside, and bit (index & 31) of bits[index >> 5] marks it occupied (a
// null bitfield marks every cell inside the box).  The loads of run k + 1 are
// issued before the cells of run k are consumed, so their latency overlaps
// the recurrence.
//
// march_range covers steps [i_begin, i_end) starting from t = t_begin (any t
// the full march passes at step i_begin: the recurrence depends on t alone,
// so a march resumed there is bit-identical).  emit(k, t_mid, dt) is called by
// the lanes holding the k-th occupied step of the range with k < limit,
// consecutive k on consecutive lanes; mark(i, t, seen) is called by every
// lane of the group at the start of each run, with the occupied steps seen
// before it.  Returns the number of occupied steps seen (all of them when
// limit is ~0u).
template <uint32_t G, bool kMed3Chain, typename Cell, typename Emit, typename Mark>
__device__ __forceinline__ uint32_t march_range_impl(float4 ro, float4 rd, float cone, float dt_min, float t_begin, uint32_t i_begin, uint32_t i_end, uint32_t limit, const uint32_t* __restrict__ bits, Cell cell,
                                                     Emit emit, Mark mark) {
    static_assert(G >= 1u && G <= 64u && 64u % G == 0u, "group size must divide 64");
    const uint32_t lane = lane_id(), j_own = lane % G, shift = lane - j_own;
    const uint64_t group_bits = G == 64u ? ~0ull : ((1ull << G) - 1ull);
    const float tf = rd.w;
    float t        = t_begin;
    uint32_t i = i_begin, seen = 0u;
    // One run of G steps: this lane's step (if any) and its cell word in flight.
    // The G steps run unconditionally, branch-free: once t reaches tf the
    // step is clamped to zero, so t stays put and every later step of the run
    // is marked dead, which leaves t and dt of the live steps bit-identical
    // to the conditional loop.  Each lane keeps only the t at which its own
    // step starts (one select per step) and recomputes that step's dt, mid
    // point and liveness from it afterwards with the same operations.
    auto step_dt = [&](float tt) { return fminf(fmaxf(dt_min, tt * cone), fmaxf(tf - tt, 0.0f)); };
    // With kMed3Chain the shared chain advances by med3(dt_min, t * cone,
    // tf - t), three instructions per step instead of five.  It equals
    // step_dt while the step stays short of tf (tf - t is then at least the
    // clamped step) and whenever tf - t lies between the two candidates; when
    // both candidates exceed tf - t, step_dt lands exactly on tf and med3
    // beyond it, so the ray is dead either way and every live t is the same.
    // (tf - t is exact there by Sterbenz's lemma: such a step starts beyond
    // tf / (1 + cone) and beyond tf - dt_min, both above tf / 2 under the
    // bounds march_range checks.)  Lanes recompute their own step with
    // step_dt.
    auto chain_dt = [&](float tt) { return kMed3Chain ? __builtin_amdgcn_fmed3f(dt_min, tt * cone, tf - tt) : step_dt(tt); };
    // Lanes keeping step j of a run: lane j of every group.
    constexpr uint64_t kOwnPattern = G == 64u ? 1ull : G == 32u ? 0x0000000100000001ull : G == 16u ? 0x0001000100010001ull : G == 8u ? 0x0101010101010101ull : 0ull;
    static_assert(kOwnPattern != 0ull, "group size 8, 16, 32 or 64");
    struct Run {
        float tm, dt, t0;
        uint32_t i0, idx, word;
        bool has;
    };
    auto run = [&](Run& r) {
        r.t0        = t;
        r.i0        = i;
        float t_own = tf;
#pragma unroll
        for (uint32_t j = 0; j < G; ++j) {
            // t_own = t on the lanes keeping step j: one v_cndmask on a
            // constant lane mask (two scalar moves), where a compare against
            // the lane index costs a v_cmp and a wait state more per step.
            asm("v_cndmask_b32_e64 %0, %0, %1, %2" : "+v"(t_own) : "v"(t), "s"(kOwnPattern << j));
            t += chain_dt(t);
        }
        r.dt             = step_dt(t_own);
        r.tm             = t_own + 0.5f * r.dt;
        r.has            = t_own < tf && i + j_own < i_end;
        i += G;
        const float p[3] = {ro.x + r.tm * rd.x, ro.y + r.tm * rd.y, ro.z + r.tm * rd.z};
        r.idx            = r.has ? cell(p) : kOutside;
        r.word           = (r.idx != kOutside && bits) ? bits[r.idx >> 5] : 0u;
    };
    Run cur{}, nxt{};
    bool more = t < tf && i < i_end;  // uniform per group
    if (more) run(cur);
    while (more) {
        const bool next = t < tf && i < i_end;
        if (next) run(nxt);
        mark(cur.i0, cur.t0, seen);
        const bool hit      = cur.has && cur.idx != kOutside && (!bits || ((cur.word >> (cur.idx & 31u)) & 1u));
        const uint64_t mask = (__ballot(hit) >> shift) & group_bits;
        const uint32_t k    = seen + (uint32_t)__popcll(mask & ((1ull << j_own) - 1ull));
        if (hit && k < limit) emit(k, cur.tm, cur.dt);
        seen += (uint32_t)__popcll(mask);
        more = next && seen < limit;
        cur  = nxt;
    }
    return seen;
}

template <uint32_t G, typename Cell, typename Emit, typename Mark>
__device__ __forceinline__ uint32_t march_range(float4 ro, float4 rd, float cone, float dt_min, float t_begin, uint32_t i_begin, uint32_t i_end, uint32_t limit, const uint32_t* __restrict__ bits, Cell cell, Emit emit,
                                                Mark mark) {
    // The three-instruction chain where a step that reaches tf starts well
    // beyond tf / 2 (cone <= 1/2: focal lengths of two pixels or more;
    // dt_min <= tf / 4: four or more steps over [0, tf]); otherwise the exact
    // one.
    if (cone <= 0.5f && dt_min <= 0.25f * rd.w) return march_range_impl<G, true>(ro, rd, cone, dt_min, t_begin, i_begin, i_end, limit, bits, cell, emit, mark);
    return march_range_impl<G, false>(ro, rd, cone, dt_min, t_begin, i_begin, i_end, limit, bits, cell, emit, mark);
}

// The whole march of a ray: steps [0, max_steps) from t_near = ro.w.
template <uint32_t G, typename Cell, typename Emit, typename Mark>
__device__ __forceinline__ uint32_t march(float4 ro, float4 rd, float cone, uint32_t max_steps, uint32_t limit, const uint32_t* __restrict__ bits, Cell cell, Emit emit, Mark mark) {
    const float tn = ro.w, tf = rd.w;
    if (!(tf - tn > 0.0f)) return 0u;
    const float dt_min = (tf - tn) / (float)max_steps;
    return march_range<G>(ro, rd, cone, dt_min, tn, 0u, max_steps, limit, bits, cell, emit, mark);
}
template <uint32_t G, typename Cell, typename Emit>
__device__ __forceinline__ uint32_t march(float4 ro, float4 rd, float cone, uint32_t max_steps, uint32_t limit, const uint32_t* __restrict__ bits, Cell cell, Emit emit) {
    return march<G>(ro, rd, cone, max_steps, limit, bits, cell, emit, [](uint32_t, float, uint32_t) {});
}

}  // namespace wave
}  // namespace nerf_hip
