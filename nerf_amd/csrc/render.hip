// render.hip — inference rendering: occupancy march with compacted sample
// streams, fused field evaluation, front-to-back compositing to RGBA8.
//
// Stages (one HIP stream); with the default chunk size 1-3 are one pass per
// chunk of at most kSlotSamples slot entries, k_march_slots (eight lanes per
// ray, the whole march, samples into per-ray slots of max_steps rounded up
// to a power of two); with an explicit sample budget per chunk:
//   1. k_march_count   one thread per ray: pixel ray + AABB (backend-cuda.cu
//                      :373-408, :561-563), occupancy march (:448-469),
//                      per-ray occupied-step count; ray record (o, tn, d, tf).
//   2. scan            exclusive prefix sum of counts -> sample offsets.
//   3. k_march_samples eight lanes per ray: re-marches from the stored ray
//                      record 8 steps at a time and writes the compacted
//                      stream (t_mid, dt), ray-major, in contiguous segments.
//   4. rounds          k_round_list lists the next slice of every active
//                      ray's samples (step-major per group of 64 rays, each
//                      entry with its ray), the fused field (hash encode +
//                      MFMA MLPs -> sigma, r, g, b) shades the list, and
//                      k_round_composite (lane = ray, replaying the list
//                      order, front to back, :601-635) composites the field's
//                      (alpha, rgb) onto the ray's carried (T, C), retiring
//                      rays at T < min_transmittance or at the end of their
//                      samples: background C + T * bg, RGBA8.
// The reference instead samples spp uniform steps per ray with no occupancy
// test and no early stop (:534-600) and writes 28 B per step whether or not
// the step is occupied.
#include <algorithm>
#include <mutex>
#include <vector>

#include "common.hpp"
#include "wave.hpp"

namespace nerf_hip {

namespace {

__device__ __forceinline__ float cone_angle(const NerfExtCamera& c) {
    const float ifx = c.fx > 0.0f ? 1.0f / c.fx : 0.0f;
    const float ify = c.fy > 0.0f ? 1.0f / c.fy : 0.0f;
    return 0.5f * (ifx + ify);
}

// The march loop of backend-cuda.cu:450-469, one scalar fp32 op at a time.
template <typename Emit>
__device__ __forceinline__ uint32_t march_ray(const float4 ro, const float4 rd, float cone, uint32_t max_steps, const OccView& occ, Emit emit) {
    const float tn = ro.w, tf = rd.w;
    const float t_range = tf - tn;
    if (!(t_range > 0.0f)) return 0u;
    const float dt_min = t_range / (float)max_steps;
    uint32_t count = 0u, i = 0u;
    float t = tn;
    while (t < tf && i < max_steps) {
        const float dt   = fminf(fmaxf(dt_min, t * cone), tf - t);
        const float tm   = t + 0.5f * dt;
        const float p[3] = {ro.x + tm * rd.x, ro.y + tm * rd.y, ro.z + tm * rd.z};
        if (occ_occupied(occ, p)) {
            emit(count, tm, dt);
            ++count;
        }
        t += dt;
        ++i;
    }
    return count;
}

__global__ __launch_bounds__(256) void k_march_count(const NerfExtCamera* __restrict__ cams, uint32_t pixels_per_view, uint32_t n_rays, OccView occ, uint32_t max_steps, float4* __restrict__ rays, uint32_t* __restrict__ counts) {
    const uint32_t ray = blockIdx.x * 256u + threadIdx.x;
    if (ray >= n_rays) return;
    const uint32_t view     = ray / pixels_per_view;
    const NerfExtCamera cam = cams[view];
    Ray r;
    float4 ro = make_float4(0.0f, 0.0f, 0.0f, 0.0f), rd = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    uint32_t count = 0u;
    if (pixel_ray(cam, ray - view * pixels_per_view, occ.omin, occ.omax, r)) {
        ro    = make_float4(r.o[0], r.o[1], r.o[2], r.tn);
        rd    = make_float4(r.d[0], r.d[1], r.d[2], r.tf);
        count = march_ray(ro, rd, cone_angle(cam), max_steps, occ, [](uint32_t, float, float) {});
    }
    rays[2ull * ray]      = ro;
    rays[2ull * ray + 1u] = rd;
    counts[ray]           = count;
}

// Writes one camera, passed by value, to device memory (the allocation-free
// march stages its camera this way instead of a host-to-device copy).
__global__ void k_stage_camera(NerfExtCamera cam, NerfExtCamera* __restrict__ dst) {
    if (threadIdx.x == 0u && blockIdx.x == 0u) *dst = cam;
}

// Eight rays per wave, eight lanes per ray (wave::march<8>): the step
// sequence is bit-identical to the count pass and the occupied steps of each
// run of 8 are written contiguously, so samples leave in 64-byte segments
// instead of one 8-byte store per ray and step; k < count keeps every write
// inside the ray's slice.  Only (t_mid, dt) is written: the round lists carry
// each entry's ray to the field and composite passes.
constexpr uint32_t kMarchGroup = 8u;

__global__ __launch_bounds__(256) void k_march_samples(const NerfExtCamera* __restrict__ cams, uint32_t pixels_per_view, uint32_t ray0, uint32_t ray_end, OccView occ, uint32_t max_steps, const float4* __restrict__ rays,
                                                      const uint32_t* __restrict__ counts, const uint32_t* __restrict__ offsets, float2* __restrict__ samples) {
    const uint32_t ray = ray0 + (blockIdx.x * 256u + threadIdx.x) / kMarchGroup;
    if (ray >= ray_end) return;
    const uint32_t count = counts[ray];
    if (count == 0u) return;
    const uint32_t view = ray / pixels_per_view;
    const float cone    = cone_angle(cams[view]);
    const uint32_t base = offsets[ray];
    wave::march<kMarchGroup>(rays[2ull * ray], rays[2ull * ray + 1u], cone, max_steps, count, occ.bits, [&](const float p[3]) { return occ_cell(occ, p); }, [&](uint32_t k, float tm, float dt) {
        samples[base + k] = make_float2(tm, dt);
    });
}

// box_relative on n points [n][3] -> [n][3] (nerf_ext_box_relative).
__global__ __launch_bounds__(256) void k_box_relative(const float* __restrict__ pts, uint32_t n, float3 lo, float3 hi, float* __restrict__ out) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n) return;
    const float p[3] = {pts[3ull * i], pts[3ull * i + 1u], pts[3ull * i + 2u]};
    const float l[3] = {lo.x, lo.y, lo.z}, h[3] = {hi.x, hi.y, hi.z};
    float q[3];
    box_relative(p, l, h, q);
#pragma unroll
    for (int a = 0; a < 3; ++a) out[3ull * i + a] = q[a];
}

// One march per ray into per-ray slots (the default chunking: chunks of at
// most kSlotSamples slot entries): ray r's samples at [(r - ray0) 2^shift,
// + count) of the chunk's buffer (2^shift >= max_steps, so a sample's index
// also names its ray), its count and that offset, and its ray record, all
// from one pass of wave::march<8> to the end of the ray (no count is known
// beforehand).  The same steps, cells and samples as k_march_count followed
// by k_march_samples; the slots are 8 KiB-aligned per ray at 1,024 steps, so
// each run's 64-byte segment falls within one cache line.
__global__ __launch_bounds__(256) void k_march_slots(const NerfExtCamera* __restrict__ cams, uint32_t pixels_per_view, uint32_t ray0, uint32_t ray_end, OccView occ, uint32_t max_steps, uint32_t shift,
                                                    float4* __restrict__ rays, uint32_t* __restrict__ counts, uint32_t* __restrict__ offsets, float2* __restrict__ samples) {
    const uint32_t ray = ray0 + (blockIdx.x * 256u + threadIdx.x) / kMarchGroup;
    if (ray >= ray_end) return;
    const uint32_t view     = ray / pixels_per_view;
    const NerfExtCamera cam = cams[view];
    Ray r;
    float4 ro = make_float4(0.0f, 0.0f, 0.0f, 0.0f), rd = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    uint32_t count = 0u;
    if (pixel_ray(cam, ray - view * pixels_per_view, occ.omin, occ.omax, r)) {
        ro             = make_float4(r.o[0], r.o[1], r.o[2], r.tn);
        rd             = make_float4(r.d[0], r.d[1], r.d[2], r.tf);
        float2* slot   = samples + ((uint64_t)(ray - ray0) << shift);
        count          = wave::march<kMarchGroup>(ro, rd, cone_angle(cam), max_steps, ~0u, occ.bits, [&](const float p[3]) { return occ_cell(occ, p); }, [&](uint32_t k, float tm, float dt) {
            slot[k] = make_float2(tm, dt);
        });
    }
    if ((threadIdx.x & (kMarchGroup - 1u)) == 0u) {
        rays[2ull * ray]      = ro;
        rays[2ull * ray + 1u] = rd;
        counts[ray]           = count;
        offsets[ray]          = (ray - ray0) << shift;
    }
}

__global__ void k_fill_u32(uint32_t* __restrict__ p, uint32_t n, uint32_t v) {
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) p[i] = v;
}

// -------------------------------------------------------------- rounds
// Shading and compositing run in rounds over slices of each ray's sample
// stream.  Every ray carries its progress p (samples composited so far) and
// the quota q of its next round: round r shades samples [p, p + min(q, count
// - p)) of every active ray, composites them front to back onto the ray's
// carried (T, C) (reference :601-635) and retires the rays whose
// transmittance fell below t_stop or whose samples are exhausted.  The
// quota follows a schedule of round ends E_r = 256, 512, 1024, 2048, ...
// (q = E_r - p catches a ray up with it), except where the ray's own decay
// predicts its stop sooner: from T0 -> T1 over the m samples of the last
// round the per-sample rate ln(T0 / T1) / m gives the samples still needed
// to fall below t_stop, and the quota is that plus a margin when it is
// smaller than the catch-up.  A ray whose prediction fell short catches up
// in the following round, and the last round never predicts, so every ray
// is done after the scheduled rounds plus two.  Only active rays are shaded:
// an opaque surface ends a ray's field work within the round it is reached,
// and a ray that thins out gradually stops close to its predicted sample.
// The split into rounds changes which samples share a field launch, never a
// value: images are the same for any quotas.

__device__ __forceinline__ void write_pixel(uint32_t ray, float cr, float cg, float cb, float T, float3 bg, uint32_t* __restrict__ rgba8, float* __restrict__ rgb_out) {
    const float r = cr + T * bg.x, g = cg + T * bg.y, b = cb + T * bg.z;
    if (rgb_out) {
        rgb_out[3ull * ray]      = r;
        rgb_out[3ull * ray + 1u] = g;
        rgb_out[3ull * ray + 2u] = b;
    }
    const uint32_t ur = (uint32_t)rintf(fminf(1.0f, fmaxf(0.0f, r)) * 255.0f);
    const uint32_t ug = (uint32_t)rintf(fminf(1.0f, fmaxf(0.0f, g)) * 255.0f);
    const uint32_t ub = (uint32_t)rintf(fminf(1.0f, fmaxf(0.0f, b)) * 255.0f);
    rgba8[ray]        = (255u << 24) | (ub << 16) | (ug << 8) | ur;
}

// ------------------------------------------------------- uniform sampling
// The reference's inference sampling (backend-cuda.cu:534-600): spp samples
// per pixel ray at t_near + (i + 0.5) dt, dt = (t_far - t_near) / spp, over
// the box, no occupancy test; a ray that misses the box (or whose dt is not
// positive) has none.  Composite (:601-635) without early stop.
__global__ __launch_bounds__(256) void k_uniform_rays(const NerfExtCamera* __restrict__ cams, uint32_t pixels_per_view, uint32_t n_rays, float3 bmin, float3 bmax, uint32_t spp, float4* __restrict__ rays,
                                                     uint32_t* __restrict__ counts) {
    const uint32_t ray = blockIdx.x * 256u + threadIdx.x;
    if (ray >= n_rays) return;
    const uint32_t view     = ray / pixels_per_view;
    const NerfExtCamera cam = cams[view];
    const float lo[3] = {bmin.x, bmin.y, bmin.z}, hi[3] = {bmax.x, bmax.y, bmax.z};
    Ray r;
    float4 ro = make_float4(0.0f, 0.0f, 0.0f, 0.0f), rd = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    uint32_t count = 0u;
    if (pixel_ray(cam, ray - view * pixels_per_view, lo, hi, r)) {
        const float dt = (r.tf - r.tn) / (float)spp;
        if (dt > 0.0f) {
            ro    = make_float4(r.o[0], r.o[1], r.o[2], r.tn);
            rd    = make_float4(r.d[0], r.d[1], r.d[2], r.tf);
            count = spp;
        }
    }
    rays[2ull * ray]      = ro;
    rays[2ull * ray + 1u] = rd;
    counts[ray]           = count;
}

// Sample layout of a chunk: its rays in groups of 64 neighbouring pixels
// (lane = ray), each group's spp samples step-major, sample i of ray
// ray0 + 64 g + l at (g spp + i) 64 + l, so that the field pass evaluates 64
// neighbouring rays at one step per wave (in ray-major order every wave's
// gathers were one ray's segment, whose fine-level corners are all fresh
// lines).  One wave per group writes the (t_mid, dt) of :588-594 and the
// owning ray; lanes past the chunk or of rays that miss the box get (0, 0)
// and a valid ray (the field evaluates them, the composite skips them).
__global__ __launch_bounds__(256) void k_uniform_samples(uint32_t ray0, uint32_t ray_end, uint32_t spp, const float4* __restrict__ rays, const uint32_t* __restrict__ counts, float2* __restrict__ samples,
                                                        uint32_t* __restrict__ sample_ray) {
    const uint32_t lane = threadIdx.x & 63u, nw = gridDim.x * 4u;
    const uint32_t groups = (ray_end - ray0 + 63u) / 64u;
    for (uint32_t g = blockIdx.x * 4u + (threadIdx.x >> 6); g < groups; g += nw) {
        const uint32_t ray   = ray0 + g * 64u + lane;
        const bool live      = ray < ray_end && counts[ray] > 0u;
        const float tn       = live ? rays[2ull * ray].w : 0.0f;
        const float tf       = live ? rays[2ull * ray + 1u].w : 0.0f;
        const float dt       = live ? (tf - tn) / (float)spp : 0.0f;  // a live ray has spp samples
        const uint32_t owner = ray < ray_end ? ray : ray_end - 1u;
        const uint64_t base  = (uint64_t)g * spp * 64u + lane;
        for (uint32_t i = 0; i < spp; ++i) {
            samples[base + 64ull * i]    = live ? make_float2(tn + ((float)i + 0.5f) * dt, dt) : make_float2(0.0f, 0.0f);
            sample_ray[base + 64ull * i] = owner;
        }
    }
}

// One wave per group of 64 rays (lane = ray), each lane compositing its
// ray's samples front to back (:601-635, every sample composited), then
// C + T bg, clamped, to RGBA8.  A step's loads are 64 consecutive outputs.
__global__ __launch_bounds__(256) void k_uniform_composite(uint32_t ray0, uint32_t ray_end, uint32_t spp, const uint32_t* __restrict__ counts, const float2* __restrict__ samples, const float4* __restrict__ field,
                                                          float3 bg, uint32_t* __restrict__ rgba8, float* __restrict__ rgb_out) {
    const uint32_t lane = threadIdx.x & 63u, nw = gridDim.x * 4u;
    const uint32_t groups = (ray_end - ray0 + 63u) / 64u;
    for (uint32_t g = blockIdx.x * 4u + (threadIdx.x >> 6); g < groups; g += nw) {
        const uint32_t ray = ray0 + g * 64u + lane;
        if (ray >= ray_end) continue;
        const uint32_t count = counts[ray];
        const uint64_t base  = (uint64_t)g * spp * 64u + lane;
        float T = 1.0f, cr = 0.0f, cg = 0.0f, cb = 0.0f;
#pragma unroll 8
        for (uint32_t i = 0; i < count; ++i) {
            const float4 f = field[base + 64ull * i];
            const float dt = fmaxf(samples[base + 64ull * i].y, 0.0f);
            const float al = 1.0f - __expf(-(f.x * dt));
            const float w  = T * al;
            cr += w * f.y;
            cg += w * f.z;
            cb += w * f.w;
            T *= 1.0f - al;
        }
        write_pixel(ray, cr, cg, cb, T, bg, rgba8, rgb_out);
    }
}

// Spatial order of the sample lists.  The field kernel evaluates 64
// consecutive list entries per wave; its table gathers are served by the
// caches only as far as those 64 samples are close in space.  So the first
// round lists rays in tiles of kTile x kTile pixels (a wave's 64 rays are
// four tiles side by side, a 16 x 4 pixel block), k_round_list emits each
// group of 64 listed rays step by step (a wave's samples are 64 neighbouring
// rays at one march step, then the next step), and k_round_composite keeps
// each group's surviving rays together for the next round.  The order only
// changes which samples share a wave; every value is the same.
constexpr uint32_t kTile = 4u;

// Tile-major enumeration of the rays [ray0, ray_end) of equally sized views
// of width W: rays are numbered ray = row * W + x over rows of all views;
// thread t covers tile t / 16 (tile rows from row0_tile, tiles_x per row),
// pixel (t % 16) of it in Z order.  Threads that map outside the range are
// idle.
__device__ __forceinline__ bool tiled_ray(uint32_t t, uint32_t W, uint32_t tiles_x, uint32_t row0_tile, uint32_t ray0, uint32_t ray_end, uint32_t& ray) {
    const uint32_t tile = t / (kTile * kTile), in = t % (kTile * kTile);
    // Z order inside the tile: each lane quad is a 2 x 2 pixel block, so the
    // samples of a quad (the unit the texture address path handles at once)
    // more often share cache lines (field 51.0 -> 49.8 ms against row-major
    // tiles; 8 x 8 Z-order tiles: 52.1 ms).
    const uint32_t ix = ((in >> 1) & 1u) | (((in >> 3) & 1u) << 1), iy = (in & 1u) | (((in >> 2) & 1u) << 1);
    const uint32_t x      = (tile % tiles_x) * kTile + ix;
    const uint64_t row    = (uint64_t)(row0_tile + tile / tiles_x) * kTile + iy;
    const uint64_t r      = row * W + x;
    ray                   = (uint32_t)r;
    return x < W && r >= ray0 && r < ray_end;
}

// Rays without samples get the background; the others start the first
// round's list (wave-aggregated appends, tile-major order) with T = 1, C = 0,
// progress 0 and the first round's quota.
__global__ __launch_bounds__(256) void k_round_init(uint32_t ray0, uint32_t ray_end, uint32_t W, uint32_t tiles_x, uint32_t row0_tile, const uint32_t* __restrict__ counts, float3 bg, uint32_t* __restrict__ rgba8,
                                                   float* __restrict__ rgb_out, float4* __restrict__ state, uint2* __restrict__ prog, uint32_t first_quota, uint32_t* __restrict__ list,
                                                   uint32_t* __restrict__ n_active, uint32_t* __restrict__ composited, uint32_t* __restrict__ shaded) {
    uint32_t ray       = 0u;
    const bool valid   = tiled_ray(blockIdx.x * 256u + threadIdx.x, W, tiles_x, row0_tile, ray0, ray_end, ray);
    const bool take    = valid && counts[ray] > 0u;
    const uint64_t m   = __ballot(take);
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t base       = 0u;
    const uint32_t lead = m ? (uint32_t)__ffsll((long long)m) - 1u : 0u;
    if (m && lane == lead) base = atomicAdd(n_active, (uint32_t)__popcll(m));
    base = (uint32_t)__shfl((int)base, (int)lead, 64);
    if (take) {
        list[base + wave::rank_below(m)] = ray;
        state[ray]                       = make_float4(1.0f, 0.0f, 0.0f, 0.0f);
        prog[ray]                        = make_uint2(0u, first_quota);
    } else if (valid) {
        write_pixel(ray, 0.0f, 0.0f, 0.0f, 1.0f, bg, rgba8, rgb_out);
        if (composited) composited[ray] = 0u;
        if (shaded) shaded[ray] = 0u;
    }
}

// Samples of this round per list slot (zero past the active count, so the
// scans run over a fixed length); keep flags start at zero.
__global__ __launch_bounds__(256) void k_round_counts(uint32_t n_slots, const uint32_t* __restrict__ list, const uint32_t* __restrict__ n_active, const uint32_t* __restrict__ counts, const uint2* __restrict__ prog,
                                                     uint32_t* __restrict__ cnt, uint32_t* __restrict__ keep) {
    const uint32_t a = blockIdx.x * 256u + threadIdx.x;
    if (a >= n_slots) return;
    keep[a] = 0u;
    uint32_t v = 0u;
    if (a < *n_active) {
        const uint32_t ray = list[a];
        const uint32_t c   = counts[ray];
        const uint2 pq     = prog[ray];
        v                  = c > pq.x ? min(pq.y, c - pq.x) : 0u;
    }
    cnt[a] = v;
}

// Stream indices of this round's samples, and with qray non-null each
// entry's ray (samples in per-ray slots need none: the index names the ray).
// One wave per group of 64 list slots (lane = slot): the group's samples
// fill the same range of the list as slot by slot (from off of its first
// slot), but step-major: step i of every slot that has one, in slot order,
// then step i + 1.
__global__ __launch_bounds__(256) void k_round_list(const uint32_t* __restrict__ list, const uint32_t* __restrict__ n_active, const uint32_t* __restrict__ offsets, const uint2* __restrict__ prog, const uint32_t* __restrict__ cnt,
                                                   const uint32_t* __restrict__ off, uint32_t* __restrict__ qlist, uint32_t* __restrict__ qray) {
    const uint32_t lane = threadIdx.x & 63u, nw = gridDim.x * 4u;
    const uint32_t n    = *n_active;
    for (uint32_t g = blockIdx.x * 4u + (threadIdx.x >> 6); g * 64u < n; g += nw) {
        const uint32_t a  = g * 64u + lane;
        const bool slot   = a < n;
        const uint32_t m  = slot ? cnt[a] : 0u;
        const uint32_t ray = slot && m ? list[a] : 0u;
        const uint32_t q0  = slot && m ? offsets[ray] + prog[ray].x : 0u;
        uint32_t dst      = off[g * 64u];
        uint32_t steps    = m;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) steps = max(steps, (uint32_t)__shfl_xor((int)steps, o, 64));
        for (uint32_t i = 0; i < steps; ++i) {
            const uint64_t act = __ballot(i < m);
            if (i < m) {
                const uint32_t at = dst + wave::rank_below(act);
                qlist[at]         = q0 + i;
                if (qray) qray[at] = ray;
            }
            dst += (uint32_t)__popcll(act);
        }
    }
}

// One wave per group of 64 list slots (lane = slot), the grouping of
// k_round_list: the field pass left the group's entries of this round in
// the order k_round_list listed them (step by step, compacted by ballot) as
// (alpha, r, g, b), so the lanes replay that order and each composites its
// own ray front to back (backend-cuda.cu:601-635: w = T alpha, C += w c,
// T *= 1 - alpha; the sample after which T < t_stop is the last one
// composited) onto the (T, C) the ray carries between rounds.  Then the
// pixel is written or (T, C) carried, and the slot flagged in keep
// (k_round_compact then lists the kept rays in slot order).  The entries of
// eight steps are loaded before they are composited; each load reads the
// group's entries of one step, consecutive in the output.  A kept ray's
// progress and next quota are updated (next_end: the schedule's end of the
// next round; predict: whether that round may take a predicted quota).  A
// retiring ray optionally reports the samples it composited (the early-stop
// index) and the samples the field evaluated for it (to the end of this
// round).
__device__ __forceinline__ uint32_t next_quota(float T0, float T1, uint32_t m, uint32_t p, uint32_t next_end, float t_stop, bool predict) {
    const uint32_t catch_up = next_end - p;
    if (!predict || !(T1 < T0) || m == 0u) return catch_up;
    // Samples until T < t_stop at the last round's rate, with a margin of a
    // thirty-second plus four samples (C5, 8 x 1280x720: 86 samples shaded
    // past the stop per ray with an eighth plus eight, 24 with this; a ray
    // that falls short takes another round).  Only the amount of work
    // depends on it.
    const float need = (__logf(T1) - __logf(t_stop)) * (float)m / (__logf(T0) - __logf(T1));
    const float q    = need * 1.03125f + 4.0f;
    return q < (float)catch_up ? max(1u, (uint32_t)q) : catch_up;
}

__global__ __launch_bounds__(256) void k_round_composite(const uint32_t* __restrict__ list, const uint32_t* __restrict__ n_active, const uint32_t* __restrict__ counts, uint2* __restrict__ prog, const uint32_t* __restrict__ cnt,
                                                        const uint32_t* __restrict__ off, const float4* __restrict__ field, float t_stop, float3 bg, float4* __restrict__ state, uint32_t* __restrict__ rgba8,
                                                        float* __restrict__ rgb_out, uint32_t* __restrict__ keep, uint32_t next_end, uint32_t predict, uint32_t* __restrict__ composited,
                                                        uint32_t* __restrict__ shaded) {
    const uint32_t lane = threadIdx.x & 63u, nw = gridDim.x * 4u;
    const uint32_t n    = *n_active;
    for (uint32_t g = blockIdx.x * 4u + (threadIdx.x >> 6); g * 64u < n; g += nw) {
        const uint32_t a   = g * 64u + lane;
        const bool slot    = a < n;
        const uint32_t m   = slot ? cnt[a] : 0u;
        const uint32_t ray = slot ? list[a] : 0u;
        const float4 st0   = slot ? state[ray] : make_float4(1.0f, 0.0f, 0.0f, 0.0f);
        float T = st0.x, cr = st0.y, cg = st0.z, cb = st0.w;
        bool stopped   = false;
        uint32_t used  = 0u;
        uint32_t dst   = off[g * 64u];
        uint32_t steps = m;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) steps = max(steps, (uint32_t)__shfl_xor((int)steps, o, 64));
        constexpr uint32_t kBatch = 8u;
        for (uint32_t i0 = 0; i0 < steps; i0 += kBatch) {
            float4 f[kBatch];
#pragma unroll
            for (uint32_t k = 0; k < kBatch; ++k) {
                const uint32_t i   = i0 + k;
                const uint64_t act = __ballot(i < m);
                f[k]               = i < m && !stopped ? field[dst + wave::rank_below(act)] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                dst += (uint32_t)__popcll(act);
            }
#pragma unroll
            for (uint32_t k = 0; k < kBatch; ++k) {
                if (i0 + k < m && !stopped) {
                    const float w = T * f[k].x;
                    cr += w * f[k].y;
                    cg += w * f[k].z;
                    cb += w * f[k].w;
                    T *= 1.0f - f[k].x;
                    stopped = T < t_stop;
                    ++used;
                }
            }
        }
        if (slot) {
            const uint32_t p = prog[ray].x;
            const bool done  = stopped || p + m >= counts[ray];
            if (done) {
                write_pixel(ray, cr, cg, cb, T, bg, rgba8, rgb_out);
                if (composited) composited[ray] = p + used;
                if (shaded) shaded[ray] = p + m;
            } else {
                state[ray] = make_float4(T, cr, cg, cb);
                prog[ray]  = make_uint2(p + m, next_quota(st0.x, T, m, p + m, next_end, t_stop, predict != 0u));
            }
            keep[a] = done ? 0u : 1u;
        }
    }
}

// The next round's list: the kept slots' rays in slot order (kept groups
// stay together), at positions from the exclusive scan of keep; the count
// is the low word of the scan's 64-bit total.
__global__ __launch_bounds__(256) void k_round_compact(const uint32_t* __restrict__ list, const uint32_t* __restrict__ n_active, const uint32_t* __restrict__ keep, const uint32_t* __restrict__ koff,
                                                      const unsigned long long* __restrict__ total, uint32_t* __restrict__ next_list, uint32_t* __restrict__ n_next) {
    const uint32_t a = blockIdx.x * 256u + threadIdx.x;
    if (a == 0u) *n_next = (uint32_t)*total;
    if (a < *n_active && keep[a]) next_list[koff[a]] = list[a];
}

}  // namespace

// ------------------------------------------------------------------- scan
// Exclusive prefix sum of n u32 values (n < 2^32 total).  Three passes over
// 1024-element blocks: block sums, scan of the sums in one workgroup, then
// the per-block scan with the block's base added.  total (device) receives the
// grand total as u64 so that overflow of the u32 offsets is detectable.
namespace {

constexpr uint32_t kScanBlock = 1024u;  // elements per workgroup (256 threads x 4)

__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t v) {
    const uint32_t lane = threadIdx.x & 63u;
#pragma unroll
    for (uint32_t d = 1; d < 64u; d <<= 1) {
        const uint32_t o = __shfl_up(v, d, 64);
        if (lane >= d) v += o;
    }
    return v;
}

// Block-wide exclusive scan of one value per thread (256 threads); returns the
// exclusive prefix and writes the block total to *total.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* lds4, uint32_t* total) {
    const uint32_t inc  = wave_inclusive_scan(v);
    const uint32_t wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63u) == 63u) lds4[wave] = inc;
    __syncthreads();
    uint32_t wave_base = 0u;
    for (uint32_t w = 0; w < wave; ++w) wave_base += lds4[w];
    *total = lds4[0] + lds4[1] + lds4[2] + lds4[3];
    __syncthreads();
    return wave_base + inc - v;
}

__global__ __launch_bounds__(256) void k_scan_reduce(const uint32_t* __restrict__ in, uint32_t n, uint32_t* __restrict__ block_sums) {
    __shared__ uint32_t lds4[4];
    const uint64_t base = (uint64_t)blockIdx.x * kScanBlock + 4u * threadIdx.x;
    uint32_t v          = 0u;
#pragma unroll
    for (uint32_t k = 0; k < 4u; ++k) v += base + k < n ? in[base + k] : 0u;
    uint32_t total;
    block_exclusive_scan(v, lds4, &total);
    if (threadIdx.x == 0u) block_sums[blockIdx.x] = total;
}

__global__ __launch_bounds__(256) void k_scan_sums(uint32_t* __restrict__ block_sums, uint32_t n_blocks, unsigned long long* __restrict__ total_out) {
    __shared__ uint32_t lds4[4];
    uint64_t carry = 0u;
    for (uint32_t b0 = 0; b0 < n_blocks; b0 += 256u) {
        const uint32_t i = b0 + threadIdx.x;
        const uint32_t v = i < n_blocks ? block_sums[i] : 0u;
        uint32_t total;
        const uint32_t ex = block_exclusive_scan(v, lds4, &total);
        if (i < n_blocks) block_sums[i] = (uint32_t)(carry + ex);
        carry += total;
        __syncthreads();
    }
    if (threadIdx.x == 0u) *total_out = carry;
}

__global__ __launch_bounds__(256) void k_scan_apply(const uint32_t* __restrict__ in, uint32_t n, const uint32_t* __restrict__ block_sums, uint32_t* __restrict__ out) {
    __shared__ uint32_t lds4[4];
    const uint64_t base = (uint64_t)blockIdx.x * kScanBlock + 4u * threadIdx.x;
    uint32_t v[4], s = 0u;
#pragma unroll
    for (uint32_t k = 0; k < 4u; ++k) {
        v[k] = base + k < n ? in[base + k] : 0u;
        s += v[k];
    }
    uint32_t total;
    uint32_t run = block_exclusive_scan(s, lds4, &total) + block_sums[blockIdx.x];
#pragma unroll
    for (uint32_t k = 0; k < 4u; ++k) {
        if (base + k < n) out[base + k] = run;
        run += v[k];
    }
}

// Apply pass for up to kScanDirect blocks, which sums the preceding block
// totals itself (k_scan_sums is then not needed); the last block writes the
// grand total.
constexpr uint32_t kScanDirect = 2048u;
__global__ __launch_bounds__(256) void k_scan_apply_direct(const uint32_t* __restrict__ in, uint32_t n, const uint32_t* __restrict__ block_sums, uint32_t* __restrict__ out, unsigned long long* __restrict__ total_out) {
    __shared__ uint32_t lds4[4];
    __shared__ unsigned long long wsum[4];
    unsigned long long before = 0ull;  // 64-bit: the grand total may pass 2^32
    for (uint32_t b = threadIdx.x; b < blockIdx.x; b += 256u) before += block_sums[b];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) before += __shfl_xor(before, o, 64);
    if ((threadIdx.x & 63u) == 0u) wsum[threadIdx.x >> 6] = before;
    __syncthreads();
    const unsigned long long prefix = wsum[0] + wsum[1] + wsum[2] + wsum[3];
    const uint64_t base = (uint64_t)blockIdx.x * kScanBlock + 4u * threadIdx.x;
    uint32_t v[4], s = 0u;
#pragma unroll
    for (uint32_t k = 0; k < 4u; ++k) {
        v[k] = base + k < n ? in[base + k] : 0u;
        s += v[k];
    }
    uint32_t total;
    uint32_t run = block_exclusive_scan(s, lds4, &total) + (uint32_t)prefix;
#pragma unroll
    for (uint32_t k = 0; k < 4u; ++k) {
        if (base + k < n) out[base + k] = run;
        run += v[k];
    }
    if (blockIdx.x == gridDim.x - 1u && threadIdx.x == 0u) *total_out = prefix + total;
}

}  // namespace

uint64_t scan_tmp_words(uint32_t n) { return (n + kScanBlock - 1u) / kScanBlock + 2u; }

// Sums of in[] over consecutive blocks of 1024 elements (the scan's first pass).
hipError_t block_sums_u32(const uint32_t* in, uint32_t n, uint32_t* sums, hipStream_t stream) {
    const uint32_t blocks = (n + kScanBlock - 1u) / kScanBlock;
    if (blocks) k_scan_reduce<<<blocks, 256, 0, stream>>>(in, n, sums);
    return hipGetLastError();
}
static_assert(kScanBlock == 1024u, "the renderer plans chunks in blocks of 1024 rays");

hipError_t exclusive_scan_u32(const uint32_t* in, uint32_t* out, uint32_t n, uint32_t* tmp, unsigned long long* total, hipStream_t stream) {
    const uint32_t blocks = (n + kScanBlock - 1u) / kScanBlock;
    if (blocks == 0u) return hipMemsetAsync(total, 0, sizeof(unsigned long long), stream);
    k_scan_reduce<<<blocks, 256, 0, stream>>>(in, n, tmp);
    if (blocks <= kScanDirect) {
        k_scan_apply_direct<<<blocks, 256, 0, stream>>>(in, n, tmp, out, total);
    } else {
        k_scan_sums<<<1, 256, 0, stream>>>(tmp, blocks, total);
        k_scan_apply<<<blocks, 256, 0, stream>>>(in, n, tmp, out);
    }
    return hipGetLastError();
}

}  // namespace nerf_hip

// ----------------------------------------------------------------- renderer
constexpr uint32_t kFirstRound = 256u;  // samples per ray in the first round (a multiple of 64)
constexpr uint32_t kScanBlockRays = 1024u;        // rays per block of the chunk plan (the scan's block)
constexpr uint64_t kChunkSamples  = 1ull << 29;   // samples per chunk: 32 B each in the stream buffers (16 GiB)
constexpr uint32_t kSlotMaxSteps  = 8192u;       // steps per ray up to which the default chunking uses slots
constexpr uint64_t kSlotSamples   = 1ull << 30;   // slot entries (rays x max_steps rounded up to a power of two) per chunk of the default chunking
constexpr uint32_t kMaxSteps      = 1u << 19;     // so that a block of rays holds at most kChunkSamples samples
constexpr uint32_t kMaxRounds  = 24u;   // round ends double from 256 (12 cover 2^19 steps), plus two

struct NerfExtRenderer {
    template <typename T>
    struct Buf {
        T* ptr       = nullptr;
        uint64_t cap = 0;
        hipError_t reserve(uint64_t n) {
            if (n <= cap) return hipSuccess;
            if (ptr) (void)hipFree(ptr);
            ptr = nullptr;
            cap = 0;
            const uint64_t want = n + n / 8u + 256u;
            hipError_t e        = hipMalloc(&ptr, want * sizeof(T));
            if (e == hipSuccess) cap = want;
            return e;
        }
        void release() {
            if (ptr) (void)hipFree(ptr);
            ptr = nullptr;
            cap = 0;
        }
    };
    Buf<NerfExtCamera> cams;
    Buf<float4> rays;
    Buf<uint32_t> counts, offsets, scan_tmp;
    Buf<unsigned long long> total;
    Buf<float2> samples;
    Buf<uint32_t> sample_ray;
    Buf<float4> field;
    // rounds
    Buf<float4> state;                 // per ray (T, C.rgb)
    Buf<uint2> prog;                   // per ray (samples composited, quota of its next round)
    Buf<uint32_t> list[2], n_active;   // active rays of this / the next round, and their counts
    Buf<uint32_t> cnt, off, qlist;     // samples per slot, their offsets, stream indices
    Buf<uint32_t> qray;                // owning ray of each qlist entry
    Buf<uint32_t> keep, koff;          // slots carried into the next round, their positions there
    Buf<unsigned long long> keep_total;
    Buf<unsigned long long> round_total;
    Buf<nerf_hip::half8_t> ref_frags;           // reference-model weights in MFMA fragment order
    hipEvent_t ev[6] = {};
    hipEvent_t fev[2 * kMaxRounds] = {};
    std::vector<uint32_t> host_sums;  // per-block sample counts (chunk plan)

    ~NerfExtRenderer() {
        cams.release();
        rays.release();
        counts.release();
        offsets.release();
        scan_tmp.release();
        total.release();
        samples.release();
        sample_ray.release();
        field.release();
        state.release();
        prog.release();
        list[0].release();
        list[1].release();
        n_active.release();
        cnt.release();
        off.release();
        keep.release();
        koff.release();
        keep_total.release();
        qlist.release();
        qray.release();
        round_total.release();
        for (hipEvent_t& e : fev)
            if (e) (void)hipEventDestroy(e);
        for (hipEvent_t& e : ev)
            if (e) (void)hipEventDestroy(e);
    }
};

namespace nerf_hip {
namespace {

// Scratch of nerf_ext_march_count_noalloc, one copy per GPU, held until the
// process ends: the staged camera in the first 256 bytes, then the per-ray
// records (o, t_near), (d, t_far) that k_march_count writes, 32 bytes per
// ray, for at most kNoAllocMaxRays rays (32 MiB + 256 B).  In host code the
// name `scratch` is a host-side stand-in, not a device address: kernels get
// the address hipGetSymbolAddress returns for the current device.
constexpr uint32_t kNoAllocMaxRays  = 1u << 20;
constexpr uint64_t kNoAllocCamBytes = 256u;
constexpr uint64_t kNoAllocBytes    = kNoAllocCamBytes + 2ull * sizeof(float4) * kNoAllocMaxRays;
static_assert(sizeof(NerfExtCamera) <= kNoAllocCamBytes, "camera slot");
__device__ __align__(256) unsigned char scratch[kNoAllocBytes];

constexpr int kNoAllocMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kNoAllocMaxDevices];  // device address of each GPU's copy of `scratch`

// Address of the current device's copy of `scratch`, looked up once per
// device with that device current.
hipError_t scratch_address(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kNoAllocMaxDevices) return hipErrorInvalidDevice;
    std::scoped_lock lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e       = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return hipSuccess;
}

}  // namespace
}  // namespace nerf_hip

using namespace nerf_hip;

extern "C" {

NERF_API NerfStatus nerf_ext_renderer_create(NerfExtRenderer** out) {
    NERF_CHECK_ARG(out, "nerf_ext_renderer_create: null output");
    *out = nullptr;
    NerfExtRenderer* r = new (std::nothrow) NerfExtRenderer();
    if (!r) {
        set_error("nerf_ext_renderer_create: out of host memory");
        return NERF_STATUS_FAILURE;
    }
    for (hipEvent_t& e : r->fev) {
        const hipError_t err = hipEventCreate(&e);
        if (err != hipSuccess) {
            delete r;
            return hip_fail(err, "hipEventCreate");
        }
    }
    for (hipEvent_t& e : r->ev) {
        const hipError_t err = hipEventCreate(&e);
        if (err != hipSuccess) {
            delete r;
            return hip_fail(err, "hipEventCreate");
        }
    }
    *out = r;
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_renderer_destroy(NerfExtRenderer* renderer) {
    if (!renderer) return NERF_STATUS_OK;
    (void)hipDeviceSynchronize();
    delete renderer;
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_box_relative(const float* points, uint32_t n, const float* box_lo, const float* box_hi, float* out, void* stream) {
    NERF_CHECK_ARG(points && box_lo && box_hi && out, "nerf_ext_box_relative: null argument");
    if (n == 0u) return NERF_STATUS_OK;
    k_box_relative<<<(n + 255u) / 256u, 256, 0, (hipStream_t)stream>>>(points, n, make_float3(box_lo[0], box_lo[1], box_lo[2]), make_float3(box_hi[0], box_hi[1], box_hi[2]), out);
    NERF_LAUNCH_CHECK("k_box_relative");
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_march_count(const NerfExtCamera* camera, const NerfExtOccupancy* occupancy, uint32_t max_steps, uint32_t* counts, void* stream) {
    NERF_CHECK_ARG(camera && occupancy && counts, "nerf_ext_march_count: null pointer");
    NERF_CHECK_ARG(max_steps > 0u, "nerf_ext_march_count: max_steps must be > 0");
    NERF_CHECK_ARG(camera->width > 0u && camera->height > 0u, "nerf_ext_march_count: empty image");
    const uint64_t n64 = (uint64_t)camera->width * camera->height;
    NERF_CHECK_ARG(n64 < (1ull << 31), "nerf_ext_march_count: too many rays");
    const uint32_t n = (uint32_t)n64;
    hipStream_t st   = (hipStream_t)stream;
    NerfExtCamera* dcam = nullptr;
    float4* rays        = nullptr;
    NERF_HIP_TRY(hipMallocAsync((void**)&dcam, sizeof(NerfExtCamera), st));
    NERF_HIP_TRY(hipMallocAsync((void**)&rays, sizeof(float4) * 2ull * n, st));
    NERF_HIP_TRY(hipMemcpyAsync(dcam, camera, sizeof(NerfExtCamera), hipMemcpyHostToDevice, st));
    OccView occ;
    NERF_CHECK_ARG(make_occ_view(*occupancy, occ), "nerf_ext_march_count: bad occupancy (empty box, more than 8 cascades or too many cells)");
    k_march_count<<<(n + 255u) / 256u, 256, 0, st>>>(dcam, n, n, occ, max_steps, rays, counts);
    NERF_LAUNCH_CHECK("k_march_count");
    NERF_HIP_TRY(hipFreeAsync(rays, st));
    NERF_HIP_TRY(hipFreeAsync(dcam, st));
    return NERF_STATUS_OK;
}

// nerf_ext_march_count without any allocation: the camera and the ray
// records live in the library's per-GPU scratch (at most 2^20 rays).  Calls
// that overlap on one GPU share that scratch and race.
NERF_API NerfStatus nerf_ext_march_count_noalloc(const NerfExtCamera* camera, const NerfExtOccupancy* occupancy, uint32_t max_steps, uint32_t* counts, void* stream) {
    NERF_CHECK_ARG(camera && occupancy && counts, "nerf_ext_march_count_noalloc: null pointer");
    NERF_CHECK_ARG(max_steps > 0u, "nerf_ext_march_count_noalloc: max_steps must be > 0");
    NERF_CHECK_ARG(camera->width > 0u && camera->height > 0u, "nerf_ext_march_count_noalloc: empty image");
    const uint64_t n64 = (uint64_t)camera->width * camera->height;
    if (n64 > kNoAllocMaxRays) {
        set_error("nerf_ext_march_count_noalloc: " + std::to_string(camera->width) + " x " + std::to_string(camera->height) + " = " + std::to_string(n64) +
                  " rays exceeds the scratch maximum of 1048576 (2^20) rays; use nerf_ext_march_count");
        return NERF_STATUS_INVALID_USAGE;
    }
    OccView occ;
    NERF_CHECK_ARG(make_occ_view(*occupancy, occ), "nerf_ext_march_count_noalloc: bad occupancy (empty box, more than 8 cascades or too many cells)");
    const uint32_t n = (uint32_t)n64;
    hipStream_t st   = (hipStream_t)stream;
    void* base       = nullptr;
    NERF_HIP_TRY(scratch_address(&base));
    NerfExtCamera* dcam = static_cast<NerfExtCamera*>(base);
    float4* rays        = reinterpret_cast<float4*>(static_cast<unsigned char*>(base) + kNoAllocCamBytes);
    k_stage_camera<<<1, 64, 0, st>>>(*camera, dcam);
    NERF_LAUNCH_CHECK("k_stage_camera");
    k_march_count<<<(n + 255u) / 256u, 256, 0, st>>>(dcam, n, n, occ, max_steps, rays, counts);
    NERF_LAUNCH_CHECK("k_march_count");
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_render(NerfExtRenderer* R, const NerfExtRenderDesc* d, uint32_t* rgba8, float* rgb_f32, uint32_t* counts_out, NerfExtRenderStats* stats) {
    NERF_CHECK_ARG(R && d && d->model && d->occupancy && d->cameras && rgba8, "nerf_ext_render: null argument");
    NERF_CHECK_ARG(d->view_count >= 1u, "nerf_ext_render: view_count must be >= 1");
    NERF_CHECK_ARG(d->max_steps >= 1u && d->max_steps <= kMaxSteps, "nerf_ext_render: max_steps must be 1..2^19");
    NERF_CHECK_ARG(d->model->kind <= NERF_EXT_MODEL_REFERENCE, "nerf_ext_render: unknown model kind");
    const bool ref_model = d->model->kind == NERF_EXT_MODEL_REFERENCE;
    GridParams g{};
    if (!ref_model) {
        const NerfStatus gs = make_grid(&d->model->grid, g);
        if (gs != NERF_STATUS_OK) return gs;
        NERF_CHECK_ARG(g.n_levels * g.n_features == 32u, "nerf_ext_render: the density MLP takes 32 features (16 levels x 2)");
    }
    NERF_CHECK_ARG((ref_model || d->model->table) && d->model->density_params && d->model->color_params, "nerf_ext_render: model has null buffers");
    const uint32_t W = d->cameras[0].width, H = d->cameras[0].height;
    for (uint32_t v = 0; v < d->view_count; ++v) NERF_CHECK_ARG(d->cameras[v].width == W && d->cameras[v].height == H && W > 0u && H > 0u, "nerf_ext_render: all views must share a non-empty image size");
    const uint64_t n64 = (uint64_t)W * H * d->view_count;
    NERF_CHECK_ARG(n64 < (1ull << 31), "nerf_ext_render: too many rays");
    const uint32_t n_rays = (uint32_t)n64;
    hipStream_t st        = (hipStream_t)d->stream;

    NERF_HIP_TRY(R->cams.reserve(d->view_count));
    NERF_HIP_TRY(R->rays.reserve(2ull * n_rays));
    NERF_HIP_TRY(R->counts.reserve(n_rays));
    NERF_HIP_TRY(R->offsets.reserve(n_rays));
    NERF_HIP_TRY(R->scan_tmp.reserve(scan_tmp_words(n_rays)));
    NERF_HIP_TRY(R->total.reserve(1));
    NERF_HIP_TRY(hipMemcpyAsync(R->cams.ptr, d->cameras, sizeof(NerfExtCamera) * d->view_count, hipMemcpyHostToDevice, st));

    OccView occ;
    NERF_CHECK_ARG(make_occ_view(*d->occupancy, occ), "nerf_ext_render: bad occupancy (empty box, more than 8 cascades or too many cells)");
    const uint32_t ppv    = W * H;
    const uint32_t blocks = (n_rays + 255u) / 256u;
    const bool timed      = stats != nullptr;

    if (timed) NERF_HIP_TRY(hipEventRecord(R->ev[0], st));
    struct Chunk {
        uint32_t ray0, ray_end;
        uint64_t samples;
    };
    std::vector<Chunk> chunks;
    uint64_t total = 0, biggest = 0;
    const uint32_t n_blocks = (n_rays + kScanBlockRays - 1u) / kScanBlockRays;
    NERF_HIP_TRY(R->scan_tmp.reserve(std::max<uint64_t>(scan_tmp_words(n_rays), n_blocks)));
    // With the default chunk size and at most kSlotMaxSteps steps per ray the
    // chunks are whole blocks of rays holding at most kSlotSamples slot
    // entries, each marched once into per-ray slots of 2^slot_shift
    // (k_march_slots): no count pass, no plan on the host, no scan.  Their
    // buffers are sized by rays x 2^slot_shift, so longer marches (whose
    // samples rarely fill their slots) keep the count pass and buffers sized
    // by the samples.
    const bool slots = !d->chunk_samples && d->max_steps <= kSlotMaxSteps;
    uint32_t slot_shift = 0u;  // slots of 2^slot_shift >= max_steps samples
    while ((1u << slot_shift) < d->max_steps) ++slot_shift;
    if (slots) {
        if (timed) NERF_HIP_TRY(hipEventRecord(R->ev[1], st));
        if (timed) NERF_HIP_TRY(hipEventRecord(R->ev[2], st));
        const uint32_t per_chunk = std::max<uint32_t>(1u, (uint32_t)(kSlotSamples / ((1ull << slot_shift) * kScanBlockRays))) * kScanBlockRays;
        for (uint32_t r0 = 0; r0 < n_rays; r0 += std::min(per_chunk, n_rays - r0)) {
            const uint32_t r1 = r0 + std::min(per_chunk, n_rays - r0);
            chunks.push_back(Chunk{r0, r1, (uint64_t)(r1 - r0) << slot_shift});
            biggest = std::max(biggest, (uint64_t)(r1 - r0) << slot_shift);
        }
    } else {
        k_march_count<<<blocks, 256, 0, st>>>(R->cams.ptr, ppv, n_rays, occ, d->max_steps, R->rays.ptr, R->counts.ptr);
        NERF_LAUNCH_CHECK("k_march_count");
        if (timed) NERF_HIP_TRY(hipEventRecord(R->ev[1], st));
        // Chunk plan: the per-ray counts summed over blocks of kScanBlock rays
        // (exact; at most kScanBlock * 2^19 < 2^32 each), copied to the host,
        // which groups whole blocks into chunks of at most kChunkSamples
        // samples.  Each chunk is marched, shaded and composited on its own,
        // so the sample buffers hold one chunk; offsets are relative to the
        // chunk.
        NERF_HIP_TRY(block_sums_u32(R->counts.ptr, n_rays, R->scan_tmp.ptr, st));
        R->host_sums.resize(n_blocks);
        NERF_HIP_TRY(hipMemcpyAsync(R->host_sums.data(), R->scan_tmp.ptr, sizeof(uint32_t) * n_blocks, hipMemcpyDeviceToHost, st));
        NERF_HIP_TRY(hipStreamSynchronize(st));
        if (timed) NERF_HIP_TRY(hipEventRecord(R->ev[2], st));
        const uint64_t budget = d->chunk_samples ? std::min<uint64_t>(d->chunk_samples, kChunkSamples) : kChunkSamples;
        for (uint32_t b = 0; b < n_blocks;) {
            Chunk c{b * kScanBlockRays, 0u, 0u};
            while (b < n_blocks && (c.ray0 == (uint64_t)b * kScanBlockRays || c.samples + R->host_sums[b] <= budget)) c.samples += R->host_sums[b++];
            c.ray_end = std::min<uint64_t>((uint64_t)b * kScanBlockRays, n_rays);
            total += c.samples;
            biggest = std::max(biggest, c.samples);
            chunks.push_back(c);
        }
    }
    NERF_HIP_TRY(R->samples.reserve(biggest));
    NERF_HIP_TRY(R->field.reserve(biggest));
    NERF_HIP_TRY(R->qlist.reserve(biggest));
    if (!slots) NERF_HIP_TRY(R->qray.reserve(biggest));

    // Every field launch of the rounds reads its entries' rays from the round
    // list (qray), so the march writes no per-sample ray index.
    FieldInputs in{};
    in.samples = R->samples.ptr;
    in.rays    = R->rays.ptr;
    for (int a = 0; a < 3; ++a) {  // the field's box is the outermost cascade's
        in.bmin[a] = occ.omin[a];
        in.bmax[a] = occ.omax[a];
    }
    const FieldWeights w{(const half_t*)d->model->density_params, (const half_t*)d->model->color_params};
    if (ref_model) {
        NERF_HIP_TRY(R->ref_frags.reserve(64ull * kRefFragments));
        NERF_HIP_TRY(ref_pack_weights(w.density, w.color, R->ref_frags.ptr, st));
    }
    const float3 bg = make_float3(d->background[0], d->background[1], d->background[2]);
    // Rounds: the schedule's round ends 256, 512, 1024, ... until every
    // ray's stream (at most max_steps samples) is covered; when there is more
    // than one, two more rounds at the last end let rays whose predicted
    // quota fell short catch up.  Round r + 1 may take predicted quotas
    // unless it is the last.
    uint32_t n_rounds = 0u;
    uint32_t Es[kMaxRounds];
    for (uint64_t E = kFirstRound;; E *= 2u) {
        Es[n_rounds++] = (uint32_t)E;
        if (E >= d->max_steps) break;
    }
    if (n_rounds >= 2u)
        for (int k = 0; k < 2; ++k, ++n_rounds) Es[n_rounds] = Es[n_rounds - 1u];
    const uint32_t chunk_rays_max = n_rays;
    NERF_HIP_TRY(R->state.reserve(n_rays));
    NERF_HIP_TRY(R->prog.reserve(n_rays));
    NERF_HIP_TRY(R->list[0].reserve(chunk_rays_max));
    NERF_HIP_TRY(R->list[1].reserve(chunk_rays_max));
    NERF_HIP_TRY(R->n_active.reserve(2));
    NERF_HIP_TRY(R->cnt.reserve(chunk_rays_max));
    NERF_HIP_TRY(R->off.reserve(chunk_rays_max));
    NERF_HIP_TRY(R->round_total.reserve(kMaxRounds));
    NERF_HIP_TRY(R->keep.reserve(chunk_rays_max));
    NERF_HIP_TRY(R->koff.reserve(chunk_rays_max));
    NERF_HIP_TRY(R->keep_total.reserve(1));
    in.sample_index     = R->qlist.ptr;
    in.sample_index_ray = slots ? nullptr : R->qray.ptr;  // slots: the ray from the index
    in.slot_rays        = slots;
    in.slot_shift       = slot_shift;
    in.alpha_in_order   = true;  // k_round_composite reads (alpha, rgb) in list order

    float ms_scan = 0.0f, ms_samples = 0.0f, field_ms = 0.0f;
    uint64_t shaded = 0;
    for (const Chunk& c : chunks) {
        const uint32_t nr = c.ray_end - c.ray0;
        in.slot_ray0       = c.ray0;
        if (timed) NERF_HIP_TRY(hipEventRecord(R->ev[3], st));
        if (!slots) NERF_HIP_TRY(exclusive_scan_u32(R->counts.ptr + c.ray0, R->offsets.ptr + c.ray0, nr, R->scan_tmp.ptr, R->total.ptr, st));
        if (timed) NERF_HIP_TRY(hipEventRecord(R->ev[4], st));
        if (slots) {
            k_march_slots<<<(nr + 256u / kMarchGroup - 1u) / (256u / kMarchGroup), 256, 0, st>>>(R->cams.ptr, ppv, c.ray0, c.ray_end, occ, d->max_steps, slot_shift, R->rays.ptr, R->counts.ptr, R->offsets.ptr, R->samples.ptr);
            NERF_LAUNCH_CHECK("k_march_slots");
        } else {
            k_march_samples<<<(nr + 256u / kMarchGroup - 1u) / (256u / kMarchGroup), 256, 0, st>>>(R->cams.ptr, ppv, c.ray0, c.ray_end, occ, d->max_steps, R->rays.ptr, R->counts.ptr, R->offsets.ptr, R->samples.ptr);
            NERF_LAUNCH_CHECK("k_march_samples");
        }
        if (timed) NERF_HIP_TRY(hipEventRecord(R->ev[5], st));
        uint32_t* n_cur = R->n_active.ptr;
        uint32_t* n_nxt = R->n_active.ptr + 1;
        uint32_t* l_cur = R->list[0].ptr;
        uint32_t* l_nxt = R->list[1].ptr;
        const uint32_t cblocks = (nr + 255u) / 256u;
        k_fill_u32<<<1, 64, 0, st>>>(n_cur, 2u, 0u);
        // Tile-major enumeration of the chunk's rays: tile rows from the
        // chunk's first pixel row to its last.
        const uint32_t tiles_x = (W + kTile - 1u) / kTile, row0_tile = (c.ray0 / W) / kTile, row1_tile = ((c.ray_end - 1u) / W) / kTile;
        const uint64_t tile_threads = (uint64_t)(row1_tile - row0_tile + 1u) * tiles_x * kTile * kTile;
        k_round_init<<<(uint32_t)((tile_threads + 255u) / 256u), 256, 0, st>>>(c.ray0, c.ray_end, W, tiles_x, row0_tile, R->counts.ptr, bg, rgba8, rgb_f32, R->state.ptr, R->prog.ptr, Es[0], l_cur, n_cur, d->composited, d->shaded);
        NERF_LAUNCH_CHECK("k_round_init");
        const uint32_t ray_waves = std::min<uint32_t>((nr + 3u) / 4u, device_cu_count() * 16u);  // workgroups of one-wave-per-slot kernels
        for (uint32_t r = 0; r < n_rounds; ++r) {
            k_round_counts<<<cblocks, 256, 0, st>>>(nr, l_cur, n_cur, R->counts.ptr, R->prog.ptr, R->cnt.ptr, R->keep.ptr);
            NERF_HIP_TRY(exclusive_scan_u32(R->cnt.ptr, R->off.ptr, nr, R->scan_tmp.ptr, R->round_total.ptr + r, st));
            k_round_list<<<ray_waves, 256, 0, st>>>(l_cur, n_cur, R->offsets.ptr, R->prog.ptr, R->cnt.ptr, R->off.ptr, R->qlist.ptr, slots ? nullptr : R->qray.ptr);
            NERF_LAUNCH_CHECK("k_round_list");
            // The field reads this round's sample count on the device: the low
            // word of the 64-bit scan total (little-endian; totals < 2^32).
            in.n_dev = reinterpret_cast<const uint32_t*>(R->round_total.ptr + r);
            if (timed) NERF_HIP_TRY(hipEventRecord(R->fev[2u * r], st));
            if (ref_model) NERF_HIP_TRY(launch_ref_field(R->ref_frags.ptr, in, (uint32_t)c.samples, R->field.ptr, nullptr, st));
            else NERF_HIP_TRY(launch_field(g, d->model->table, w, in, (uint32_t)c.samples, R->field.ptr, st));
            if (timed) NERF_HIP_TRY(hipEventRecord(R->fev[2u * r + 1u], st));
            const uint32_t nxt = std::min(r + 1u, n_rounds - 1u);
            k_round_composite<<<ray_waves, 256, 0, st>>>(l_cur, n_cur, R->counts.ptr, R->prog.ptr, R->cnt.ptr, R->off.ptr, R->field.ptr, d->min_transmittance, bg, R->state.ptr, rgba8, rgb_f32, R->keep.ptr, Es[nxt],
                                                         r + 2u < n_rounds ? 1u : 0u, d->composited, d->shaded);
            NERF_LAUNCH_CHECK("k_round_composite");
            NERF_HIP_TRY(exclusive_scan_u32(R->keep.ptr, R->koff.ptr, nr, R->scan_tmp.ptr, R->keep_total.ptr, st));
            k_round_compact<<<cblocks, 256, 0, st>>>(l_cur, n_cur, R->keep.ptr, R->koff.ptr, R->keep_total.ptr, l_nxt, n_nxt);
            NERF_LAUNCH_CHECK("k_round_compact");
            std::swap(l_cur, l_nxt);
            std::swap(n_cur, n_nxt);
        }
        if (timed) {
            // Per-chunk stage times (the events are reused by the next chunk).
            NERF_HIP_TRY(hipStreamSynchronize(st));
            float t_scan = 0.0f, t_samp = 0.0f;
            NERF_HIP_TRY(hipEventElapsedTime(&t_scan, R->ev[3], R->ev[4]));
            NERF_HIP_TRY(hipEventElapsedTime(&t_samp, R->ev[4], R->ev[5]));
            ms_scan += t_scan;
            ms_samples += t_samp;
            for (uint32_t r = 0; r < n_rounds; ++r) {
                float f = 0.0f;
                NERF_HIP_TRY(hipEventElapsedTime(&f, R->fev[2u * r], R->fev[2u * r + 1u]));
                field_ms += f;
            }
            std::vector<unsigned long long> totals(n_rounds);
            NERF_HIP_TRY(hipMemcpy(totals.data(), R->round_total.ptr, sizeof(unsigned long long) * n_rounds, hipMemcpyDeviceToHost));
            for (unsigned long long t : totals) shaded += t;
        }
    }
    if (counts_out) NERF_HIP_TRY(hipMemcpyAsync(counts_out, R->counts.ptr, sizeof(uint32_t) * n_rays, hipMemcpyDeviceToDevice, st));
    if (timed) {
        hipEvent_t end = nullptr;
        NERF_HIP_TRY(hipEventCreate(&end));
        NERF_HIP_TRY(hipEventRecord(end, st));
        NERF_HIP_TRY(hipEventSynchronize(end));
        float ms_count = 0.0f, ms_plan = 0.0f, total_ms = 0.0f;
        NERF_HIP_TRY(hipEventElapsedTime(&ms_count, R->ev[0], R->ev[1]));
        NERF_HIP_TRY(hipEventElapsedTime(&ms_plan, R->ev[1], R->ev[2]));
        NERF_HIP_TRY(hipEventElapsedTime(&total_ms, R->ev[0], end));
        (void)hipEventDestroy(end);
        if (slots) {  // the marched total, from the per-block sums of the counts
            NERF_HIP_TRY(block_sums_u32(R->counts.ptr, n_rays, R->scan_tmp.ptr, st));
            R->host_sums.resize(n_blocks);
            NERF_HIP_TRY(hipMemcpyAsync(R->host_sums.data(), R->scan_tmp.ptr, sizeof(uint32_t) * n_blocks, hipMemcpyDeviceToHost, st));
            NERF_HIP_TRY(hipStreamSynchronize(st));
            for (uint32_t b = 0; b < n_blocks; ++b) total += R->host_sums[b];
        }
        stats->rays           = n_rays;
        stats->samples        = total;
        stats->samples_shaded = shaded;
        stats->ms_count       = ms_count;
        stats->ms_scan        = ms_plan + ms_scan;
        stats->ms_samples     = ms_samples;
        stats->ms_field       = field_ms;
        stats->ms_composite   = total_ms - stats->ms_count - stats->ms_scan - ms_samples - field_ms;
        stats->ms_total       = total_ms;
    }
    return NERF_STATUS_OK;
}

// The reference's inference sampling (backend-cuda.cu:534-635) for any
// model: rays in chunks of whole 1,024-ray blocks whose spp samples each fit
// the chunk budget; per chunk the samples, the field, the composite.
NERF_API NerfStatus nerf_ext_render_uniform(NerfExtRenderer* R, const NerfExtModel* model, const NerfExtCamera* cameras, uint32_t view_count, const float* aabb6, uint32_t samples_per_ray, const float* background3,
                                          uint32_t* rgba8, float* rgb_f32, void* stream) {
    NERF_CHECK_ARG(R && model && cameras && aabb6 && rgba8, "nerf_ext_render_uniform: null argument");
    NERF_CHECK_ARG(view_count >= 1u, "nerf_ext_render_uniform: view_count must be >= 1");
    NERF_CHECK_ARG(samples_per_ray >= 1u && samples_per_ray <= kMaxSteps, "nerf_ext_render_uniform: samples_per_ray must be 1..2^19");
    NERF_CHECK_ARG(model->kind <= NERF_EXT_MODEL_REFERENCE, "nerf_ext_render_uniform: unknown model kind");
    const bool ref_model = model->kind == NERF_EXT_MODEL_REFERENCE;
    GridParams g{};
    if (!ref_model) {
        const NerfStatus gs = make_grid(&model->grid, g);
        if (gs != NERF_STATUS_OK) return gs;
        NERF_CHECK_ARG(g.n_levels * g.n_features == 32u, "nerf_ext_render_uniform: the density MLP takes 32 features (16 levels x 2)");
    }
    NERF_CHECK_ARG((ref_model || model->table) && model->density_params && model->color_params, "nerf_ext_render_uniform: model has null buffers");
    for (int a = 0; a < 3; ++a) NERF_CHECK_ARG(aabb6[3 + a] > aabb6[a], "nerf_ext_render_uniform: empty box");
    const uint32_t W = cameras[0].width, H = cameras[0].height;
    for (uint32_t v = 0; v < view_count; ++v) NERF_CHECK_ARG(cameras[v].width == W && cameras[v].height == H && W > 0u && H > 0u, "nerf_ext_render_uniform: all views must share a non-empty image size");
    const uint64_t n64 = (uint64_t)W * H * view_count;
    NERF_CHECK_ARG(n64 < (1ull << 31), "nerf_ext_render_uniform: too many rays");
    const uint32_t n_rays = (uint32_t)n64;
    hipStream_t st        = (hipStream_t)stream;
    // Chunk: whole blocks of kScanBlockRays rays, at most kChunkSamples samples.
    const uint64_t blocks_per_chunk = std::max<uint64_t>(1u, kChunkSamples / ((uint64_t)samples_per_ray * kScanBlockRays));
    const uint32_t chunk_rays       = (uint32_t)std::min<uint64_t>(blocks_per_chunk * kScanBlockRays, (uint64_t)(n_rays + kScanBlockRays - 1u) / kScanBlockRays * kScanBlockRays);
    const uint64_t chunk_samples    = (uint64_t)chunk_rays * samples_per_ray;
    NERF_HIP_TRY(R->cams.reserve(view_count));
    NERF_HIP_TRY(R->rays.reserve(2ull * n_rays));
    NERF_HIP_TRY(R->counts.reserve(n_rays));
    NERF_HIP_TRY(R->offsets.reserve(n_rays));
    NERF_HIP_TRY(R->scan_tmp.reserve(scan_tmp_words(chunk_rays)));
    NERF_HIP_TRY(R->total.reserve(1));
    NERF_HIP_TRY(R->samples.reserve(chunk_samples));
    NERF_HIP_TRY(R->sample_ray.reserve(chunk_samples));
    NERF_HIP_TRY(R->field.reserve(chunk_samples));
    NERF_HIP_TRY(hipMemcpyAsync(R->cams.ptr, cameras, sizeof(NerfExtCamera) * view_count, hipMemcpyHostToDevice, st));
    const float3 bmin = make_float3(aabb6[0], aabb6[1], aabb6[2]), bmax = make_float3(aabb6[3], aabb6[4], aabb6[5]);
    k_uniform_rays<<<(n_rays + 255u) / 256u, 256, 0, st>>>(R->cams.ptr, W * H, n_rays, bmin, bmax, samples_per_ray, R->rays.ptr, R->counts.ptr);
    NERF_LAUNCH_CHECK("k_uniform_rays");
    FieldInputs in{};
    in.samples    = R->samples.ptr;
    in.sample_ray = R->sample_ray.ptr;
    in.rays       = R->rays.ptr;
    for (int a = 0; a < 3; ++a) {
        in.bmin[a] = aabb6[a];
        in.bmax[a] = aabb6[3 + a];
    }
    const FieldWeights w{(const half_t*)model->density_params, (const half_t*)model->color_params};
    if (ref_model) {
        NERF_HIP_TRY(R->ref_frags.reserve(64ull * kRefFragments));
        NERF_HIP_TRY(ref_pack_weights(w.density, w.color, R->ref_frags.ptr, st));
    }
    const float3 bg = background3 ? make_float3(background3[0], background3[1], background3[2]) : make_float3(1.0f, 1.0f, 1.0f);
    for (uint32_t ray0 = 0; ray0 < n_rays; ray0 += chunk_rays) {
        const uint32_t ray_end = std::min(n_rays, ray0 + chunk_rays), nr = ray_end - ray0;
        const uint32_t groups = (nr + 63u) / 64u, waves = std::min<uint32_t>((groups + 3u) / 4u, device_cu_count() * 16u);
        const uint32_t n_smp  = (uint32_t)((uint64_t)groups * 64u * samples_per_ray);  // the groups' whole layout
        k_uniform_samples<<<waves, 256, 0, st>>>(ray0, ray_end, samples_per_ray, R->rays.ptr, R->counts.ptr, R->samples.ptr, R->sample_ray.ptr);
        NERF_LAUNCH_CHECK("k_uniform_samples");
        if (ref_model) NERF_HIP_TRY(launch_ref_field(R->ref_frags.ptr, in, n_smp, R->field.ptr, nullptr, st));
        else NERF_HIP_TRY(launch_field(g, model->table, w, in, n_smp, R->field.ptr, st));
        k_uniform_composite<<<waves, 256, 0, st>>>(ray0, ray_end, samples_per_ray, R->counts.ptr, R->samples.ptr, R->field.ptr, bg, rgba8, rgb_f32);
        NERF_LAUNCH_CHECK("k_uniform_composite");
    }
    return NERF_STATUS_OK;
}

}  // extern "C"
