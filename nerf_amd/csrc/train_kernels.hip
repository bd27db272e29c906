// train_kernels.hip — one training step of the hash-grid NeRF on gfx950.
//
// Stage                     reference                      here
// begin step / camera       backend-cuda.cu:1479-1488      k_step_begin
// occupancy maintenance     :1555-1634                     k_occ_eval (window), k_occ_bits (decay, bits)
// ray sampling + march      :422-533                       k_train_rays, k_train_samples (or, for rays of
//                                                          one segment, k_ray_offsets, k_train_samples_one)
// field forward             :1328-1339                     launch_field (field.hip)
// composite fwd/bwd + loss  :1095-1182 (MSE)               k_composite_train (Huber)
// MLP backward              :784-909, 1267-1301 (cuBLAS)   k_bwd_dx (dfeat, dW partials)
// hash-table backward       (hash-grid model)              k_bin_pass<false> (record count, on a second
//                                                          stream) and its scan; k_scatter_fill (coarse-level
//                                                          slabs and the record fill, direct or staged)
// gradient sums             :1286-1301                     k_grad_reduce (bins, coarse chunks, dW partials)
// grad stats, Adam          :1447-1554                     in the gradient writers, summed by k_grad_norm
//                                                          (which may also end the step); k_adam
// end step                  :1495-1512                     k_step_end
//
// MI355X choices: every count lives in device memory and every launch has a
// fixed shape, so a whole step is one stream of kernels (graph-capturable;
// HIP has no conditional graph nodes, so the reference's bucket switch
// (:1489-1494) becomes kernels that read their counts and exit early).  The
// MLP backward recomputes the forward per 16-sample tile in registers (MFMA
// is cheap next to moving activations through HBM) and, in the same pass,
// moves each tile's deltas and activations through LDS onto the MFMA
// reduction axis for the weight gradients (deterministic per-workgroup
// partials); the hash-table gradient goes through sorted bins with exact
// fixed-point sums.
#include "mlp_device.hpp"
#include "wave.hpp"
#include "train.hpp"

namespace nerf_hip {

using namespace mlp;

namespace {

constexpr uint32_t kWave   = 64;
constexpr uint32_t kWaves  = 4;
constexpr uint32_t kThreads = kWave * kWaves;

__device__ __forceinline__ uint32_t hash_u32(uint32_t x) {  // backend-cuda.cu:321-328
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}
__device__ __forceinline__ float rand01(uint32_t seed) {  // :329-332
    return (float)(hash_u32(seed) & 0x00ffffffu) / (float)0x01000000u;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += (uint32_t)__shfl_xor((int)v, o, 64);
    return v;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o, 64));
    return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Orders LDS traffic of one wavefront (writes by some lanes, reads by others)
// without a workgroup barrier.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// ------------------------------------------------------------ step control
// What the start of a step decides (:1479-1488): its index, camera,
// occupancy work and ray count, from the previous step's index and the ray
// count its sampler chose.
struct StepBegin {
    uint32_t frame, camera, occ_mode, n_rays;
    float rays_f;
    uint32_t skip;  // the latest Adam's, carried until this step's Adam
};
__device__ __forceinline__ StepBegin step_begin_values(const TrainParams& P, const TrainDevState* prev) {
    StepBegin b;
    const uint32_t f = prev->frame + 1u;
    b.frame          = f;
    b.camera = hash_u32(f * 747796405u + 2891336453u) % P.image_count;  // :1482
    if (f < P.occ_warmup)
        b.occ_mode = f == 0u ? kOccWarmupInit : kOccNone;                // :1483-1485
    else
        b.occ_mode = (P.occ_interval != 0u && f % P.occ_interval == 0u) ? kOccRefresh : kOccNone;
    b.rays_f            = prev->rays_next;
    b.skip              = prev->skip;
    const uint32_t rays = (uint32_t)(b.rays_f + 0.5f);
    b.n_rays            = rays < P.min_rays ? P.min_rays : (rays > P.max_rays ? P.max_rays : rays);
    return b;
}
__device__ __forceinline__ void step_begin_store(TrainDevState* S, const StepBegin& b) {
    S->frame      = b.frame;
    S->rays_f     = b.rays_f;
    S->skip       = b.skip;
    S->camera     = b.camera;
    S->occ_mode   = b.occ_mode;
    S->n_rays     = b.n_rays;
    S->n_samples  = 0u;
    S->n_active   = 0u;
    S->total      = 0ull;
    S->nonfinite  = 0u;
    S->grad_sumsq = 0.0;
    S->loss_sum   = 0.0f;
}
// A step's first kernel may do the begin itself (begin = true): every
// workgroup derives the values from the previous step's slot, which nothing
// changes meanwhile, and workgroup 0 stores them; later kernels read them
// from the state.
__device__ __forceinline__ StepBegin step_begin_in(const TrainParams& P, TrainDevState* S, const TrainDevState* prev, bool begin) {
    if (!begin) return StepBegin{S->frame, S->camera, S->occ_mode, S->n_rays, S->rays_f, S->skip};
    const StepBegin b = step_begin_values(P, prev);
    if (blockIdx.x == 0u && threadIdx.x == 0u) step_begin_store(S, b);
    return b;
}

__global__ void k_step_begin(TrainParams P, TrainDevState* S, const TrainDevState* prev) {
    if (threadIdx.x != 0u || blockIdx.x != 0u) return;
    step_begin_store(S, step_begin_values(P, prev));
}

// The ray-count adaptation, once the step's occupied samples are known (the
// sampler's totals): aim the next batch at target_samples (exponentially
// smoothed), from the occupied samples before the capacity cut (the kept
// count is capped, so it cannot show an overshoot).
__device__ __forceinline__ void ray_count_next(const TrainParams& P, TrainDevState* S, unsigned long long total) {
    float r = S->rays_f;
    if (P.target_samples != 0u && total > 0ull) {
        const float want = r * (float)P.target_samples / (float)total;
        r                = 0.5f * r + 0.5f * want;
        r                = fminf(fmaxf(r, (float)P.min_rays), (float)P.max_rays);
    }
    S->rays_next = r;
}

// :1495-1512.  Reads only what the step's kernels up to the gradient norm
// wrote and the previous step's sample total, and Adam reads none of what it
// writes, so the gradient-norm kernel may run it (end = true in k_grad_norm).
__device__ __forceinline__ void step_end(const TrainParams& P, TrainDevState* S, const TrainDevState* prev) {
    const float inv = S->n_active ? 1.0f / (float)S->n_active : 0.0f;
    const float loss = S->loss_sum * inv;                                          // :1499
    const float gn   = (float)sqrt(S->grad_sumsq > 0.0 ? S->grad_sumsq : 0.0) / P.loss_scale;
    S->stats.loss              = loss;
    S->stats.grad_norm         = gn;
    S->stats.has_nonfinite     = (S->nonfinite || !isfinite(loss) || !isfinite(gn)) ? 1u : 0u;
    S->stats.completed_steps   = S->frame + 1u;
    S->stats.last_train_camera = S->camera;
    S->samples_done            = prev->samples_done + S->n_samples;
}

__global__ void k_step_end(TrainParams P, TrainDevState* S, const TrainDevState* prev) {
    if (threadIdx.x != 0u || blockIdx.x != 0u) return;
    step_end(P, S, prev);
}

// ----------------------------------------------------------- occupancy grid
// A refresh decays every cell (:1563) and then takes, over the rotating
// window of cells_per_update cells, max(density, sigma(cell centre))
// (:1575-1627).  The window's cells are decayed by the kernel that evaluates
// them and every other cell by k_occ_bits, which then sets the bits, so the
// refresh is two launches: the same products and maxima as a decay pass
// before the evaluation.
__device__ __forceinline__ bool occ_in_window(uint32_t cell, uint32_t start, uint32_t window, uint32_t cells) {
    return (cell >= start ? cell - start : cell + cells - start) < window;
}

// density[cell] = max(decay x density[cell], exp(raw sigma(cell centre))).
// bits non-null (whole words: cells and window multiples of 32): the whole
// occupancy stage in one launch, without k_occ_bits: for a refresh the
// workgroups first decay the cells of the words outside the window and set
// those words' bits, then evaluate the window a tile of 16 cells (half a
// word, stored as 16 bits) per wave; the warm-up start as in k_occ_bits.
// (Words assembled from two waves' tiles through LDS took two workgroup
// barriers per four tiles: 2^21 cells 225 -> 284 us.)
template <typename TableT>
__global__ __launch_bounds__(kThreads) void k_occ_eval(TrainParams P, GridParams g, const TableT* __restrict__ table, const half_t* __restrict__ dparams, TrainDevState* S, const TrainDevState* prev,
                                                       bool begin, float* density, uint32_t* __restrict__ bits) {
    const StepBegin sb  = step_begin_in(P, S, prev, begin);
    const uint32_t mode = sb.occ_mode;  // uniform across the grid
    if (bits && mode == kOccWarmupInit) {  // as k_occ_bits
        for (uint32_t c = blockIdx.x * blockDim.x + threadIdx.x; c < P.occ_cells; c += gridDim.x * blockDim.x) density[c] = 1.0f;
        for (uint32_t w = blockIdx.x * blockDim.x + threadIdx.x; w < P.occ_cells / 32u; w += gridDim.x * blockDim.x) bits[w] = ~0u;
        return;
    }
    if (mode != kOccRefresh) return;
    __shared__ __align__(16) half_t sp[NERF_EXT_DENSITY_PARAMS];
    stage_density<kThreads>(sp, dparams);
    const uint32_t lane = threadIdx.x & 63u, grp = lane >> 4, s16 = lane & 15u, wave = threadIdx.x >> 6;
    const uint32_t count = P.occ_cells_per_update < P.occ_cells ? P.occ_cells_per_update : P.occ_cells;
    const uint32_t start = (uint32_t)((uint64_t)sb.frame * count % P.occ_cells);
    if (bits) {
        const uint32_t words = P.occ_cells / 32u, w_start = start / 32u, w_count = count / 32u;
        for (uint32_t w = blockIdx.x * blockDim.x + threadIdx.x; w < words - w_count; w += gridDim.x * blockDim.x) {
            const uint32_t word = (w_start + w_count + w) % words;  // the words after the window, wrapping
            float4* d4          = reinterpret_cast<float4*>(density + 32ull * word);
            uint32_t b          = 0u;
#pragma unroll
            for (uint32_t k = 0; k < 8u; ++k) {
                float4 v = d4[k];
                v.x *= P.occ_decay;
                v.y *= P.occ_decay;
                v.z *= P.occ_decay;
                v.w *= P.occ_decay;
                d4[k] = v;
                b |= (v.x > P.occ_threshold ? 1u : 0u) << (4u * k);
                b |= (v.y > P.occ_threshold ? 1u : 0u) << (4u * k + 1u);
                b |= (v.z > P.occ_threshold ? 1u : 0u) << (4u * k + 2u);
                b |= (v.w > P.occ_threshold ? 1u : 0u) << (4u * k + 3u);
            }
            bits[word] = b;
        }
    }
    __syncthreads();
    DensityFrags f;
    load_density(sp, f, lane);
    const uint32_t res   = P.occ_res;
    const float step[3]  = {(P.bmax[0] - P.bmin[0]) / (float)res, (P.bmax[1] - P.bmin[1]) / (float)res, (P.bmax[2] - P.bmin[2]) / (float)res};
    const uint32_t tiles = (count + 15u) / 16u;
    for (uint32_t tile = blockIdx.x * kWaves + wave; tile < tiles; tile += gridDim.x * kWaves) {
        const uint32_t k    = tile * 16u + s16;
        const uint32_t kq   = k < count ? k : count - 1u;
        const uint32_t cell = (start + kq) % P.occ_cells;
        const uint32_t z = cell / (res * res), rem = cell - z * res * res, y = rem / res, x = rem - y * res;
        float p[3] = {P.bmin[0] + ((float)x + 0.5f) * step[0], P.bmin[1] + ((float)y + 0.5f) * step[1], P.bmin[2] + ((float)z + 0.5f) * step[2]};
        // The hash grid encodes the unit cube: normalise by the AABB.
        const float w[3] = {p[0], p[1], p[2]};
        box_relative(w, P.bmin, P.bmax, p);
        float feat[8];
        encode_quad(g, table, p, grp, feat);
        const floatx4 o = density_mlp(f, to_half8(feat));
        bool occ        = false;
        if (grp == 0u && k < count) {
            const float sigma = expf(o[0]);
            const float d     = fmaxf(density[cell] * P.occ_decay, sigma);
            density[cell]     = d;
            occ               = d > P.occ_threshold;
        }
        if (bits) {
            // The tile's 16 cells are one half of a bit word (the window
            // starts on a word): lanes 0..15 hold them, stored as 16 bits.
            const uint32_t b = (uint32_t)__ballot(occ) & 0xFFFFu;
            if (lane == 0u) reinterpret_cast<uint16_t*>(bits)[(start + tile * 16u) % P.occ_cells / 16u] = (uint16_t)b;
        }
    }
}

// Warmup start: density 1 and every word all ones (:1559-1561, :1569-1571);
// refresh: the decay of the cells outside the window, then bit = density >
// threshold, strict (:1628-1634).  window: the refresh window's size (the
// window's own cells were decayed when they were evaluated).
__global__ __launch_bounds__(256) void k_occ_bits(TrainParams P, const TrainDevState* S, uint32_t window, float* density, uint32_t* bits) {
    const uint32_t mode = S->occ_mode;
    if (mode == kOccNone) return;
    const uint32_t cell = blockIdx.x * 256u + threadIdx.x;
    bool occ            = false;
    if (cell < P.occ_cells) {
        if (mode == kOccWarmupInit) {
            density[cell] = 1.0f;
            occ           = true;
        } else {
            const uint32_t start = (uint32_t)((uint64_t)S->frame * window % P.occ_cells);
            float d              = density[cell];
            if (!occ_in_window(cell, start, window, P.occ_cells)) {
                d *= P.occ_decay;
                density[cell] = d;
            }
            occ = d > P.occ_threshold;
        }
    }
    const uint64_t b    = mode == kOccWarmupInit ? ~0ull : __ballot(occ);
    const uint32_t words = (P.occ_cells + 31u) / 32u;
    const uint32_t w0    = (blockIdx.x * 256u + (threadIdx.x & ~63u)) >> 5;
    if ((threadIdx.x & 63u) == 0u) {
        if (w0 < words) bits[w0] = (uint32_t)b;
        if (w0 + 1u < words) bits[w0 + 1u] = (uint32_t)(b >> 32);
    }
}

// Reference model: the refresh window's cell centres in world coordinates
// (:1575-1611; direction (0, 0, 1), which the density does not read), for a
// field evaluation, then density[cell] = max(density[cell], sigma) with
// sigma = softplus of the raw density output (:1617-1627).
__global__ __launch_bounds__(256) void k_occ_points(TrainParams P, const TrainDevState* S, uint32_t window, float* __restrict__ points, float* __restrict__ dirs) {
    const uint32_t k = blockIdx.x * 256u + threadIdx.x;
    if (k >= window || S->occ_mode != kOccRefresh) return;
    const uint32_t start = (uint32_t)((uint64_t)S->frame * window % P.occ_cells);
    const uint32_t cell  = (start + k) % P.occ_cells;
    const uint32_t res = P.occ_res, z = cell / (res * res), rem = cell - z * res * res, y = rem / res, x = rem - y * res;
    const uint32_t c[3] = {x, y, z};
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        const float step    = (P.bmax[a] - P.bmin[a]) / (float)res;
        points[3u * k + a]  = P.bmin[a] + ((float)c[a] + 0.5f) * step;
        dirs[3u * k + a]    = a == 2 ? 1.0f : 0.0f;
    }
}

__global__ __launch_bounds__(256) void k_occ_apply_field(TrainParams P, const TrainDevState* S, uint32_t window, const float4* __restrict__ field, float* __restrict__ density) {
    const uint32_t k = blockIdx.x * 256u + threadIdx.x;
    if (k >= window || S->occ_mode != kOccRefresh) return;
    const uint32_t start = (uint32_t)((uint64_t)S->frame * window % P.occ_cells);
    const uint32_t cell  = (start + k) % P.occ_cells;
    density[cell]        = fmaxf(density[cell] * P.occ_decay, field[k].x);
}

// ---------------------------------------------------------------- sampling
// Occupancy cell of p (backend-cuda.cu:338-351), or wave::kOutside.
__device__ __forceinline__ uint32_t occ_cell_at(const TrainParams& P, const float p[3]) {
    float rel[3];
    box_relative(p, P.bmin, P.bmax, rel);
    const float rx = rel[0], ry = rel[1], rz = rel[2];
    if (rx < 0.0f || rx >= 1.0f || ry < 0.0f || ry >= 1.0f || rz < 0.0f || rz >= 1.0f) return wave::kOutside;
    const uint32_t res = P.occ_res;
    const uint32_t ix = min(res - 1u, (uint32_t)(rx * (float)res)), iy = min(res - 1u, (uint32_t)(ry * (float)res)), iz = min(res - 1u, (uint32_t)(rz * (float)res));
    return ix + iy * res + iz * res * res;
}

__device__ __forceinline__ float cone_of(const NerfExtCamera& c) {  // :333-337
    const float ifx = c.fx > 0.0f ? 1.0f / c.fx : 0.0f, ify = c.fy > 0.0f ? 1.0f / c.fy : 0.0f;
    return 0.5f * (ifx + ify);
}

// Random pixel per ray (:438-441), ray, march count, bilinear ground truth
// composited over white (:471-499).  kRayGroup lanes per ray (wave::march); ray
// slots from n_rays to max_rays get a zero count so the scan over all slots
// stays valid (their ray, ground-truth and checkpoint records are not
// written: every reader stops at n_rays).
constexpr uint32_t kTrainGroup = 16u;  // lanes per ray in the emission pass (4 units per wave)
// The count pass marches each ray with a whole wave: a step has only a few
// hundred rays (a wave each, under one per SIMD), so the pass is the latency
// of the t recurrence, which the three-instruction chain of
// wave::march_range keeps near 22 cycles per step.
constexpr uint32_t kRayGroup = 64u;

__global__ __launch_bounds__(256) void k_train_rays(TrainParams P, TrainDevState* S, const TrainDevState* prev, bool begin, const NerfExtCamera* __restrict__ cams, const uint8_t* __restrict__ images, const uint32_t* __restrict__ bits, float4* __restrict__ rays,
                                                     float4* __restrict__ gt, uint32_t* __restrict__ counts, float* __restrict__ seg_t, uint32_t* __restrict__ seg_seen, uint32_t* __restrict__ seg_reached, uint32_t segs) {
    constexpr uint32_t kPer = 64u / kRayGroup;  // rays per wave
    const uint32_t lane = threadIdx.x & 63u, stride = gridDim.x * kWaves * kPer;
    const StepBegin sb = step_begin_in(P, S, prev, begin);
    const uint32_t n_rays = sb.n_rays, cam_idx = sb.camera, frame = sb.frame;
    const NerfExtCamera cam = cams[cam_idx];
    const float cone        = cone_of(cam);
    const uint32_t n_live   = min(n_rays, P.max_rays);
    // Slots past the step's rays get only their count (the scan runs over
    // every slot), in coalesced stores; nothing reads their other records.
    // (One lane writing four records per empty slot cost 30 us of a 36 us
    // pass at 2^18 slots and ~320 rays.)
    for (uint32_t r = n_live + blockIdx.x * blockDim.x + threadIdx.x; r < P.max_rays; r += gridDim.x * blockDim.x) counts[r] = 0u;
    for (uint32_t r = (blockIdx.x * kWaves + (threadIdx.x >> 6)) * kPer + lane / kRayGroup; r < n_live; r += stride) {
        uint32_t count = 0u, reached = 0u;
        float4 ro = make_float4(0.0f, 0.0f, 0.0f, 0.0f), rd = make_float4(0.0f, 0.0f, 0.0f, 0.0f), g4 = make_float4(1.0f, 1.0f, 1.0f, 0.0f);
        if (r < n_rays) {
            const uint32_t seed = frame * 1315423911u ^ r * 9781u;
            const float px      = rand01(seed ^ 0xA511E9B3u) * (float)P.width;
            const float py      = rand01(seed ^ 0x63D83595u) * (float)P.height;
            const float pyf     = (float)P.height - 1.0f - py;
            Ray ray;
            if (make_ray(cam, px, pyf, P.bmin, P.bmax, ray)) {
                ro    = make_float4(ray.o[0], ray.o[1], ray.o[2], ray.tn);
                rd    = make_float4(ray.d[0], ray.d[1], ray.d[2], ray.tf);
                // Checkpoints every kSegSteps steps (t and the occupied steps
                // before), from which k_train_samples resumes each segment.
                count = wave::march<kRayGroup>(ro, rd, cone, P.max_steps, ~0u, bits, [&](const float p[3]) { return occ_cell_at(P, p); }, [](uint32_t, float, float) {},
                                                 [&](uint32_t i0, float t0, uint32_t seen) {
                                                     if (i0 % kSegSteps == 0u) {
                                                         reached = i0 / kSegSteps + 1u;
                                                         if (lane % kRayGroup == 0u) {
                                                             seg_t[(uint64_t)r * segs + i0 / kSegSteps]    = t0;
                                                             seg_seen[(uint64_t)r * segs + i0 / kSegSteps] = seen;
                                                         }
                                                     }
                                                 });
            }
            if (count > 0u) {
                const uint8_t* img = images + (uint64_t)cam_idx * P.width * P.height * 4u;
                const float cx = fmaxf(0.0f, fminf(px, (float)P.width - 1.0f)), cy = fmaxf(0.0f, fminf(py, (float)P.height - 1.0f));
                const int x0 = (int)floorf(cx), y0 = (int)floorf(cy);
                const int x1 = min(x0 + 1, (int)P.width - 1), y1 = min(y0 + 1, (int)P.height - 1);
                const float tx = cx - (float)x0, ty = cy - (float)y0;
                const int stride = (int)P.width * 4;
                const uint8_t* p00 = img + y0 * stride + x0 * 4;
                const uint8_t* p10 = img + y0 * stride + x1 * 4;
                const uint8_t* p01 = img + y1 * stride + x0 * 4;
                const uint8_t* p11 = img + y1 * stride + x1 * 4;
                const float inv255 = 1.0f / 255.0f;
                float c[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float a = (float)p00[k] * inv255 * (1.0f - tx) + (float)p10[k] * inv255 * tx;
                    const float b = (float)p01[k] * inv255 * (1.0f - tx) + (float)p11[k] * inv255 * tx;
                    c[k]          = a * (1.0f - ty) + b * ty;
                }
                const float alpha = c[3];
                g4 = make_float4(c[0] * alpha + (1.0f - alpha), c[1] * alpha + (1.0f - alpha), c[2] * alpha + (1.0f - alpha), alpha);
            }
        }
        if (lane % kRayGroup == 0u) {
            rays[2ull * r]      = ro;
            rays[2ull * r + 1u] = rd;
            gt[r]               = g4;
            counts[r]           = count;
            seg_reached[r]      = reached;
        }
    }
}

// Writes the samples of every ray whose whole range fits the stream capacity;
// kept[r] is its count or 0.  The kept rays form a prefix (offsets grow with
// r), so n_samples = max(offset + count) over kept rays.  kTrainGroup lanes
// per ray.
// Emission pass: one unit per (ray, segment of kSegSteps steps), resumed from
// the checkpoint k_train_rays left, so the serial step chain of a unit is
// kSegSteps long rather than the whole ray.  A ray is kept only if all its
// samples fit under the capacity (its offset + count); unit (r, 0) records
// the ray's kept count and the step totals.
__global__ __launch_bounds__(256) void k_train_samples(TrainParams P, TrainDevState* S, const NerfExtCamera* __restrict__ cams, const uint32_t* __restrict__ bits, const float4* __restrict__ rays, const uint32_t* __restrict__ counts,
                                                        uint32_t* __restrict__ offsets, const float* __restrict__ seg_t, const uint32_t* __restrict__ seg_seen, const uint32_t* __restrict__ seg_reached, uint32_t segs,
                                                        uint32_t* __restrict__ kept,
                                                        float2* __restrict__ samples, uint32_t* __restrict__ sample_ray) {
    constexpr uint32_t kPer = 64u / kTrainGroup;
    const uint32_t lane = threadIdx.x & 63u, stride = gridDim.x * kWaves * kPer, j = lane % kTrainGroup;
    const bool leader   = j == 0u;
    const uint32_t n_rays = min(S->n_rays, P.max_rays);
    const float cone      = cone_of(cams[S->camera]);
    for (uint32_t r = blockIdx.x * blockDim.x + threadIdx.x; r < P.max_rays; r += gridDim.x * blockDim.x)
        if (r >= n_rays) kept[r] = 0u;
    // Sum of counts[0, end) over the whole wave (every lane gets it; integer
    // sums, so the order does not matter): a ray's offset in the stream is
    // the sum over the rays before it, computed where it is used (a separate
    // scan took two launches, about 9 us).  The kPer units of a wave share one
    // such sum, for the first unit's ray, and each unit adds the counts of the
    // at most kPer - 1 rays between (4,096 rays of 64 steps: 40 -> 31 us for
    // the pass, against one sum per unit by its 16 lanes).
    auto wave_count_sum = [&](uint32_t end) {
        uint32_t a = 0u, b = 0u, c = 0u, d = 0u, k = lane;
        for (; k + 192u < end; k += 256u) {
            a += counts[k];
            b += counts[k + 64u];
            c += counts[k + 128u];
            d += counts[k + 192u];
        }
        for (; k < end; k += 64u) a += counts[k];
        uint32_t part = (a + b) + (c + d);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) part += (uint32_t)__shfl_xor((int)part, o, 64);
        return part;
    };
    if (blockIdx.x == 0u && threadIdx.x < 64u) {
        const uint32_t total = wave_count_sum(n_rays);  // occupied samples before the capacity cut
        if (threadIdx.x == 0u) {
            S->total = total;
            ray_count_next(P, S, total);
        }
    }
    const uint64_t units = (uint64_t)n_rays * segs;
    // The loop runs per wave (every lane takes part in the wave's sum); lane
    // group g of the wave takes unit uw + g.
    for (uint64_t uw = (uint64_t)(blockIdx.x * kWaves + (threadIdx.x >> 6)) * kPer; uw < units; uw += stride) {
        const uint32_t ra    = (uint32_t)(uw / segs);
        const uint32_t first = wave_count_sum(ra);
        const uint64_t u     = uw + lane / kTrainGroup;
        if (u >= units) continue;
        const uint32_t r = (uint32_t)(u / segs), sg = (uint32_t)(u % segs);
        uint32_t base    = first;
        for (uint32_t k = ra; k < r; ++k) base += counts[k];
        const uint32_t count = counts[r];
        const bool fits      = count > 0u && (uint64_t)base + count <= (uint64_t)P.sample_cap;
        if (sg == 0u && leader) {
            offsets[r] = base;
            kept[r]    = fits ? count : 0u;
            if (fits) {
                atomicMax(&S->n_samples, base + count);
                atomicAdd(&S->n_active, 1u);
            }
        }
        const uint32_t reached = seg_reached[r];
        if (!fits || sg >= reached) continue;
        const uint32_t s0 = seg_seen[u], s1 = sg + 1u < reached ? seg_seen[u + 1u] : count;
        if (s1 <= s0) continue;
        const float4 ro = rays[2ull * r], rd = rays[2ull * r + 1u];
        const float dt_min = (rd.w - ro.w) / (float)P.max_steps;  // as in wave::march
        const uint32_t i0 = sg * kSegSteps, i1 = min(i0 + kSegSteps, P.max_steps);
        const uint32_t at = base + s0;
        wave::march_range<kTrainGroup>(ro, rd, cone, dt_min, seg_t[u], i0, i1, s1 - s0, bits, [&](const float p[3]) { return occ_cell_at(P, p); },
                                       [&](uint32_t k, float tm, float dt) {
                                           samples[at + k]    = make_float2(tm, dt);
                                           sample_ray[at + k] = r;
                                       },
                                       [](uint32_t, float, uint32_t) {});
    }
}

// Rays of one segment (at most kSegSteps steps, the reference host's 64):
// one workgroup scans the step's counts into the offsets, the kept counts and
// the step totals (what the leading units of k_train_samples record), and
// k_train_samples_one marches each ray with a whole wave (one run of 64
// steps: one cell-word round trip instead of four) from its offset.  At
// 4,096 rays of 64 steps the per-wave prefix sums of k_train_samples cost
// more than the march (31 us for the pass; this pair 7.4 + 5.9 us).
constexpr uint32_t kOffsetThreads = 1024u;
__global__ __launch_bounds__(kOffsetThreads) void k_ray_offsets(TrainParams P, TrainDevState* S, const uint32_t* __restrict__ counts, uint32_t* __restrict__ offsets, uint32_t* __restrict__ kept) {
    constexpr uint32_t kT = kOffsetThreads;
    __shared__ uint32_t wsum[kT / 64u], wend[kT / 64u], wact[kT / 64u];
    const uint32_t n_rays = min(S->n_rays, P.max_rays);
    const uint32_t lane = threadIdx.x & 63u, wv = threadIdx.x >> 6;
    uint32_t carry = 0u, end_max = 0u, active = 0u;
    for (uint32_t r0 = 0; r0 < n_rays; r0 += 4u * kT) {
        uint32_t c[4], own = 0u;
#pragma unroll
        for (uint32_t k = 0; k < 4u; ++k) {
            const uint32_t r = r0 + 4u * threadIdx.x + k;
            c[k]             = r < n_rays ? counts[r] : 0u;
            own += c[k];
        }
        uint32_t inc = own;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t up = (uint32_t)__shfl_up((int)inc, o, 64);
            if (lane >= (uint32_t)o) inc += up;
        }
        if (lane == 63u) wsum[wv] = inc;
        __syncthreads();
        uint32_t before = 0u, chunk = 0u;
        for (uint32_t w = 0; w < kT / 64u; ++w) {
            before += w < wv ? wsum[w] : 0u;
            chunk += wsum[w];
        }
        uint32_t base = carry + before + inc - own;
#pragma unroll
        for (uint32_t k = 0; k < 4u; ++k) {
            const uint32_t r = r0 + 4u * threadIdx.x + k;
            if (r < n_rays) {
                const bool fits = c[k] > 0u && (uint64_t)base + c[k] <= (uint64_t)P.sample_cap;
                offsets[r]      = base;
                kept[r]         = fits ? c[k] : 0u;
                if (fits) {
                    end_max = max(end_max, base + c[k]);
                    ++active;
                }
            }
            base += c[k];
        }
        carry += chunk;
        __syncthreads();  // wsum is rewritten by the next chunk
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        end_max = max(end_max, (uint32_t)__shfl_xor((int)end_max, o, 64));
        active += (uint32_t)__shfl_xor((int)active, o, 64);
    }
    if (lane == 0u) {
        wend[wv] = end_max;
        wact[wv] = active;
    }
    __syncthreads();
    if (threadIdx.x == 0u) {
        uint32_t e = 0u, a = 0u;
        for (uint32_t w = 0; w < kT / 64u; ++w) {
            e = max(e, wend[w]);
            a += wact[w];
        }
        S->n_samples = e;
        S->n_active  = a;
        S->total     = carry;  // occupied samples before the capacity cut
        ray_count_next(P, S, carry);
    }
}

__global__ __launch_bounds__(256) void k_train_samples_one(TrainParams P, const TrainDevState* S, const NerfExtCamera* __restrict__ cams, const uint32_t* __restrict__ bits, const float4* __restrict__ rays,
                                                            const uint32_t* __restrict__ offsets, uint32_t* __restrict__ kept, const float* __restrict__ seg_t, float2* __restrict__ samples,
                                                            uint32_t* __restrict__ sample_ray) {
    const uint32_t n_rays = min(S->n_rays, P.max_rays);
    const float cone      = cone_of(cams[S->camera]);
    for (uint32_t r = blockIdx.x * blockDim.x + threadIdx.x; r < P.max_rays; r += gridDim.x * blockDim.x)
        if (r >= n_rays) kept[r] = 0u;
    for (uint32_t r = blockIdx.x * kWaves + (threadIdx.x >> 6); r < n_rays; r += gridDim.x * kWaves) {
        const uint32_t count = kept[r];
        if (count == 0u) continue;
        const uint32_t at = offsets[r];
        const float4 ro = rays[2ull * r], rd = rays[2ull * r + 1u];
        const float dt_min = (rd.w - ro.w) / (float)P.max_steps;  // as in wave::march
        wave::march_range<64u>(ro, rd, cone, dt_min, seg_t[r], 0u, P.max_steps, count, bits, [&](const float p[3]) { return occ_cell_at(P, p); },
                               [&](uint32_t k, float tm, float dt) {
                                   samples[at + k]    = make_float2(tm, dt);
                                   sample_ray[at + k] = r;
                               },
                               [](uint32_t, float, uint32_t) {});
    }
}

// Rays of one segment with at most kPrefixRays ray slots (the reference
// host's 4,096 rays of 64 steps): one launch instead of k_ray_offsets and
// k_train_samples_one.  Workgroup b owns rays 4b..4b+3, a wave each; it adds
// the counts of the rays before them itself (at 4,096 rays 8 MB of L2 reads
// over the whole grid, against a launch of its own for the scan), and the
// workgroup that owns the last ray scans all counts for the step totals.
// The kept rays are those whose samples all fit the capacity, a prefix of
// the rays with samples (offsets only grow): the kept count is the largest
// inclusive prefix sum within the capacity.
constexpr uint32_t kPrefixRays = 8192u;
__global__ __launch_bounds__(256) void k_train_samples_prefix(TrainParams P, TrainDevState* S, const NerfExtCamera* __restrict__ cams, const uint32_t* __restrict__ bits, const float4* __restrict__ rays,
                                                               const uint32_t* __restrict__ counts, uint32_t* __restrict__ offsets, uint32_t* __restrict__ kept, const float* __restrict__ seg_t,
                                                               float2* __restrict__ samples, uint32_t* __restrict__ sample_ray) {
    __shared__ uint32_t red[3][kWaves];
    const uint32_t n_rays = min(S->n_rays, P.max_rays);
    const uint32_t lane = threadIdx.x & 63u, wv = threadIdx.x >> 6;
    const uint32_t r0 = blockIdx.x * kWaves, r = r0 + wv;
    // Counts before this workgroup's rays (r0 is a multiple of 4: 16-byte loads).
    uint32_t before = 0u;
    const uint32_t upto = min(r0, n_rays & ~3u);
    for (uint32_t i = 4u * threadIdx.x; i < upto; i += 4u * blockDim.x) {
        const uint4 c = *reinterpret_cast<const uint4*>(counts + i);
        before += c.x + c.y + c.z + c.w;
    }
    for (uint32_t i = upto + threadIdx.x; i < min(r0, n_rays); i += blockDim.x) before += counts[i];
    before = wave_sum_u32(before);
    if (lane == 0u) red[0][wv] = before;
    __syncthreads();
    uint32_t base = 0u;
    for (uint32_t w = 0; w < kWaves; ++w) base += red[0][w];
    for (uint32_t w = 0; w < wv; ++w) base += r0 + w < n_rays ? counts[r0 + w] : 0u;
    const uint32_t count = r < n_rays ? counts[r] : 0u;
    const bool fits      = count > 0u && (uint64_t)base + count <= (uint64_t)P.sample_cap;
    if (r < P.max_rays && lane == 0u) {
        kept[r] = fits ? count : 0u;
        if (r < n_rays) offsets[r] = base;
    }
    if (n_rays > 0u && blockIdx.x == (n_rays - 1u) / kWaves) {
        // Step totals: thread t takes a run of `per` counts, the runs' sums
        // are scanned across the workgroup, then each thread walks its run.
        const uint32_t per = (n_rays + blockDim.x - 1u) / blockDim.x;
        const uint32_t a = min(threadIdx.x * per, n_rays), e = min(a + per, n_rays);
        uint32_t own = 0u;
        for (uint32_t i = a; i < e; ++i) own += counts[i];
        uint32_t inc = own;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t up = (uint32_t)__shfl_up((int)inc, o, 64);
            if (lane >= (uint32_t)o) inc += up;
        }
        __syncthreads();  // red[0] was read above
        if (lane == 63u) red[0][wv] = inc;
        __syncthreads();
        uint32_t run = inc - own, total = 0u;
        for (uint32_t w = 0; w < kWaves; ++w) {
            run += w < wv ? red[0][w] : 0u;
            total += red[0][w];
        }
        uint32_t end_max = 0u, active = 0u;
        for (uint32_t i = a; i < e; ++i) {
            const uint32_t c = counts[i];
            run += c;
            if (c > 0u && (uint64_t)run <= (uint64_t)P.sample_cap) {
                end_max = run;
                ++active;
            }
        }
        end_max = wave_max_u32(end_max);
        active  = wave_sum_u32(active);
        if (lane == 0u) {
            red[1][wv] = end_max;
            red[2][wv] = active;
        }
        __syncthreads();
        if (threadIdx.x == 0u) {
            uint32_t em = 0u, ac = 0u;
            for (uint32_t w = 0; w < kWaves; ++w) {
                em = max(em, red[1][w]);
                ac += red[2][w];
            }
            S->n_samples = em;
            S->n_active  = ac;
            S->total     = total;  // occupied samples before the capacity cut
            ray_count_next(P, S, total);
        }
    }
    if (!fits) return;
    const float cone   = cone_of(cams[S->camera]);
    const float4 ro = rays[2ull * r], rd = rays[2ull * r + 1u];
    const float dt_min = (rd.w - ro.w) / (float)P.max_steps;  // as in wave::march
    wave::march_range<64u>(ro, rd, cone, dt_min, seg_t[r], 0u, P.max_steps, count, bits, [&](const float p[3]) { return occ_cell_at(P, p); },
                           [&](uint32_t k, float tm, float dt) {
                               samples[base + k]    = make_float2(tm, dt);
                               sample_ray[base + k] = r;
                           },
                           [](uint32_t, float, uint32_t) {});
}

// ----------------------------------------------------- composite fwd + bwd
// Huber loss (Huber 1964) on the white-composited RGB; gradients with respect
// to the raw network outputs (see the oracle's orc_composite_backward_ray for
// the derivation).  One wave per ray over groups of 64 samples: transmittance
// from the carried T times the exclusive product of (1 - alpha) across the
// group; the backward pass forms the suffix S_i = pred - prefix_i from an
// inclusive scan of w c, so both passes run front to back.
constexpr uint32_t kCompositeBatch = 8u;  // groups of 64 samples loaded together per ray

__global__ __launch_bounds__(256) void k_composite_train(TrainParams P, TrainDevState* S, const uint32_t* __restrict__ kept, const uint32_t* __restrict__ offsets, const float2* __restrict__ samples, const float4* __restrict__ field,
                                                          const float4* __restrict__ gt, float4* __restrict__ draw) {
    __shared__ float wsum[kWaves];
    const uint32_t lane = threadIdx.x & 63u, nw = gridDim.x * kWaves;
    const uint32_t active = S->n_active;
    const float inv_norm  = active ? 1.0f / (float)active : 0.0f;
    const uint32_t n_rays = min(S->n_rays, P.max_rays);
    const float d         = P.huber_delta;
    float wave_loss       = 0.0f;
    for (uint32_t r = blockIdx.x * kWaves + (threadIdx.x >> 6); r < n_rays; r += nw) {
        const uint32_t count = kept[r];
        if (count == 0u) continue;
        const uint32_t base = offsets[r];
        // The field and step of kCompositeBatch groups of 64 samples are
        // loaded together before any of them is composited: a ray has only
        // its own wave, so each load round trip is exposed.
        float4 fb[kCompositeBatch];
        float db[kCompositeBatch];
        auto load_batch = [&](uint32_t c0) {
#pragma unroll
            for (uint32_t b = 0; b < kCompositeBatch; ++b) {
                const uint32_t i = c0 + 64u * b + lane;
                const bool valid = i < count;
                fb[b]            = valid ? field[base + i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                db[b]            = valid ? fmaxf(samples[base + i].y, 0.0f) : 0.0f;
            }
        };
        float T = 1.0f, C[3] = {0.0f, 0.0f, 0.0f};
        for (uint32_t c0 = 0; c0 < count; c0 += 64u * kCompositeBatch) {
            load_batch(c0);
#pragma unroll
            for (uint32_t b = 0; b < kCompositeBatch; ++b) {
                if (c0 + 64u * b >= count) break;  // uniform
                const bool valid = c0 + 64u * b + lane < count;
                const float4 f   = fb[b];
                const float dt   = db[b];
                const float a    = valid ? 1.0f - __expf(-(f.x * dt)) : 0.0f;
                const float incl = wave::inclusive_product(1.0f - a);
                const float excl = wave::shift_up1(incl, 1.0f);
                const float w    = T * excl * a;
                C[0] += w * f.y;
                C[1] += w * f.z;
                C[2] += w * f.w;
                T *= wave::broadcast(incl, 63u);
            }
        }
        const float4 g4    = gt[r];
        const float gtv[3] = {g4.x, g4.y, g4.z};
        float pred[3], gr[3];
        float ray_loss = 0.0f;
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            pred[c]        = wave::sum(C[c]) + T;  // white background
            const float x  = pred[c] - gtv[c];
            const float ax = fabsf(x);
            ray_loss += ax <= d ? 0.5f * x * x : d * (ax - 0.5f * d);
            gr[c] = fminf(fmaxf(x, -d), d) * inv_norm;
        }
        wave_loss += ray_loss;
        T = 1.0f;
        float carry[3] = {0.0f, 0.0f, 0.0f};
        for (uint32_t c00 = 0; c00 < count; c00 += 64u * kCompositeBatch) {
            load_batch(c00);
#pragma unroll
            for (uint32_t b = 0; b < kCompositeBatch; ++b) {
                const uint32_t c0 = c00 + 64u * b;
                if (c0 >= count) break;  // uniform
                const uint32_t i  = c0 + lane;
                const bool valid  = i < count;
                const float4 f    = fb[b];
                const float dt    = db[b];
                const float a     = valid ? 1.0f - __expf(-(f.x * dt)) : 0.0f;
                const float incl  = wave::inclusive_product(1.0f - a);
                const float excl  = wave::shift_up1(incl, 1.0f);
                const float w     = T * excl * a;
                const float Tn    = T * incl;
                const float c3[3] = {f.y, f.z, f.w};
                float ds = 0.0f, dc[3];
#pragma unroll
                for (int c = 0; c < 3; ++c) {
                    const float prefix = carry[c] + wave::inclusive_sum(w * c3[c]);
                    ds += gr[c] * (Tn * c3[c] - (pred[c] - prefix));
                    dc[c]    = w * gr[c] * c3[c] * (1.0f - c3[c]);
                    carry[c] = wave::broadcast(prefix, 63u);
                }
                if (valid) draw[base + i] = make_float4(dt * f.x * ds, dc[0], dc[1], dc[2]);
                T *= wave::broadcast(incl, 63u);
            }
        }
    }
    if (lane == 0u) wsum[threadIdx.x >> 6] = wave_loss;
    __syncthreads();
    if (threadIdx.x == 0u) {
        const float b = wsum[0] + wsum[1] + wsum[2] + wsum[3];
        if (b != 0.0f) atomicAdd(&S->loss_sum, b);
    }
}

// ------------------------------------------------------------ MLP backward
// Transposed-weight fragments (A operands of the backward products).
// C3^T: rows = h2 neurons, k = colour output neuron (identity map, < 16).
__device__ __forceinline__ half8_t frag_c3t(const half_t* cp, uint32_t b, uint32_t lane) {
    const uint32_t i = lane & 15u, g = lane >> 4;
    half8_t a;
#pragma unroll
    for (uint32_t e = 0; e < 8u; ++e) {
        const uint32_t k = 8u * g + e;
        a[e]             = k < 16u ? cp[6144u + k * 64u + 16u * b + i] : (half_t)0.0f;
    }
    return a;
}
// W^T for a 64-output layer W [64][n_in] (C2: n_in 64, D1/C1 handled below):
// rows = W's input index 16b + i, k = W's output index via the Hidden map.
__device__ __forceinline__ half8_t frag_hidden_t(const half_t* W, uint32_t n_in, uint32_t b, uint32_t t, uint32_t lane) {
    const uint32_t i = lane & 15u, g = lane >> 4;
    half8_t a;
#pragma unroll
    for (uint32_t e = 0; e < 8u; ++e) {
        const int k = logical_k(KMap::Hidden, t, g, e);
        a[e]        = W[(uint32_t)k * n_in + 16u * b + i];
    }
    return a;
}
// C1^T with rows = density-output slots 0..15 (slot 0 -> zero row, slot j ->
// colour input j - 1), k = h1 neuron via the Hidden map.
__device__ __forceinline__ half8_t frag_c1t(const half_t* cp, uint32_t t, uint32_t lane) {
    const uint32_t i = lane & 15u, g = lane >> 4;
    half8_t a;
#pragma unroll
    for (uint32_t e = 0; e < 8u; ++e) {
        const int k = logical_k(KMap::Hidden, t, g, e);
        a[e]        = i == 0u ? (half_t)0.0f : cp[(uint32_t)k * 32u + (i - 1u)];
    }
    return a;
}
// D2^T: rows = hd neurons 16b + i, k = density output slot 4g + e (e < 4).
__device__ __forceinline__ half8_t frag_d2t(const half_t* dp, uint32_t b, uint32_t lane) {
    const uint32_t i = lane & 15u, g = lane >> 4;
    half8_t a;
#pragma unroll
    for (uint32_t e = 0; e < 8u; ++e) a[e] = e < 4u ? dp[2048u + (4u * g + e) * 64u + 16u * b + i] : (half_t)0.0f;
    return a;
}

__device__ __forceinline__ half4_t mask_half(const floatx4 v, const half4_t act) {
    half4_t h;
#pragma unroll
    for (int e = 0; e < 4; ++e) h[e] = act[e] > (half_t)0.0f ? (half_t)v[e] : (half_t)0.0f;
    return h;
}

// Everything one 16-sample tile needs in the backward passes.
struct TileGrad {
    half8_t x;        // density input (hash features), B layout
    half4_t hd[4];    // density hidden
    half4_t dhd[4];   // its delta
    half4_t dout;     // density output delta (slots 4g..4g+3)
    half8_t xc;       // colour input, B layout (ColorIn map)
    half4_t h1[4], dh1[4], h2[4], dh2[4];
    half8_t do3;      // colour output delta, identity map
    floatx4 dx[2];    // hash-feature gradient: features 16b + 4g + e
};

// Recomputes the forward of one tile and back-propagates (loss-scaled fp16
// deltas, fp32 MFMA accumulation): the chain of the oracle's orc_mlp_backward.
// Every A operand of the tile's products, in MFMA fragment order: fragment
// f of lane l is the 16 bytes at F[64 f + l], so each is one conflict-free
// 128-bit LDS read.
enum : uint32_t {
    kFragCF1 = 0,   // colour layer 1 (ColorIn map), blocks 0..3
    kFragCF2 = 4,   // colour layer 2, [2 block + k-step]
    kFragC3T = 12,  // colour output, transposed, blocks 0..3
    kFragC2T = 16,  // colour layer 2, transposed, [2 block + k-step]
    kFragC1T = 24,  // colour layer 1, transposed, k-steps 0..1
    kFragD2T = 26,  // density output, transposed, blocks 0..3
    kFragD1T = 30,  // density layer 1, transposed, [2 block + k-step]
    kFragDW1 = 34,  // density layer 1, blocks 0..3
    kFragDW2 = 38,  // density output, k-steps 0..1
    kFrags   = 40,
};
__device__ half8_t build_frag(uint32_t f, const half_t* dp, const half_t* cp, uint32_t lane) {
    if (f < kFragCF2) return load_a(cp, 32u, f - kFragCF1, 0u, KMap::ColorIn, lane);
    if (f < kFragC3T) return load_a(cp + 2048, 64u, (f - kFragCF2) >> 1, (f - kFragCF2) & 1u, KMap::Hidden, lane);
    if (f < kFragC2T) return frag_c3t(cp, f - kFragC3T, lane);
    if (f < kFragC1T) return frag_hidden_t(cp + 2048, 64u, (f - kFragC2T) >> 1, (f - kFragC2T) & 1u, lane);
    if (f < kFragD2T) return frag_c1t(cp, f - kFragC1T, lane);
    if (f < kFragD1T) return frag_d2t(dp, f - kFragD2T, lane);
    if (f < kFragDW1) return frag_hidden_t(dp, 32u, (f - kFragD1T) >> 1, (f - kFragD1T) & 1u, lane);
    if (f < kFragDW2) return load_a(dp, 32u, f - kFragDW1, 0u, KMap::Identity, lane);
    return load_a(dp + 2048, 64u, 0u, f - kFragDW2, KMap::Hidden, lane);
}

__device__ __forceinline__ void tile_backward(const half8_t* F, const half8_t x, const float d[3], const float4 g, float ls, uint32_t grp, TileGrad& T) {
    const floatx4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
    const uint32_t lane = threadIdx.x & 63u;
    auto frag = [&](uint32_t f) { return F[64u * f + lane]; };
    T.x = x;
    const half8_t dw1[4] = {frag(kFragDW1), frag(kFragDW1 + 1u), frag(kFragDW1 + 2u), frag(kFragDW1 + 3u)};
    const half8_t dw2[2] = {frag(kFragDW2), frag(kFragDW2 + 1u)};
    layer_32_64(dw1, x, T.hd);
    const floatx4 o = layer_64_16(dw2, T.hd);
    float sh[4];
    sh4_quad(d, grp, sh);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        T.xc[e]     = (half_t)o[e];
        T.xc[4 + e] = (half_t)sh[e];
    }
    if (grp == 0u) T.xc[0] = (half_t)0.0f;
    // colour forward
#pragma unroll
    for (uint32_t b = 0; b < 4u; ++b) T.h1[b] = relu_half(mfma16x16x32(frag(kFragCF1 + b), T.xc, zero));
#pragma unroll
    for (uint32_t b = 0; b < 4u; ++b) {
        floatx4 a = mfma16x16x32(frag(kFragCF2 + 2u * b), cat(T.h1[0], T.h1[1]), zero);
        a         = mfma16x16x32(frag(kFragCF2 + 2u * b + 1u), cat(T.h1[2], T.h1[3]), a);
        T.h2[b]   = relu_half(a);
    }
    // colour backward
#pragma unroll
    for (uint32_t e = 0; e < 8u; ++e) {
        const uint32_t k = 8u * grp + e;
        const float v    = k == 0u ? g.y : (k == 1u ? g.z : (k == 2u ? g.w : 0.0f));
        T.do3[e]         = to_half_rne(ls * v);
    }
#pragma unroll
    for (uint32_t b = 0; b < 4u; ++b) T.dh2[b] = mask_half(mfma16x16x32(frag(kFragC3T + b), T.do3, zero), T.h2[b]);
#pragma unroll
    for (uint32_t b = 0; b < 4u; ++b) {
        floatx4 a = mfma16x16x32(frag(kFragC2T + 2u * b), cat(T.dh2[0], T.dh2[1]), zero);
        a         = mfma16x16x32(frag(kFragC2T + 2u * b + 1u), cat(T.dh2[2], T.dh2[3]), a);
        T.dh1[b]  = mask_half(a, T.h1[b]);
    }
    floatx4 dgeo = mfma16x16x32(frag(kFragC1T), cat(T.dh1[0], T.dh1[1]), zero);
    dgeo         = mfma16x16x32(frag(kFragC1T + 1u), cat(T.dh1[2], T.dh1[3]), dgeo);
    // density backward
#pragma unroll
    for (int e = 0; e < 4; ++e) T.dout[e] = (half_t)dgeo[e];
    if (grp == 0u) T.dout[0] = to_half_rne(ls * g.x);
    const half4_t z4 = {(half_t)0.0f, (half_t)0.0f, (half_t)0.0f, (half_t)0.0f};
#pragma unroll
    for (uint32_t b = 0; b < 4u; ++b) T.dhd[b] = mask_half(mfma16x16x32(frag(kFragD2T + b), cat(T.dout, z4), zero), T.hd[b]);
#pragma unroll
    for (uint32_t b = 0; b < 2u; ++b) {
        floatx4 a = mfma16x16x32(frag(kFragD1T + 2u * b), cat(T.dhd[0], T.dhd[1]), zero);
        T.dx[b]   = mfma16x16x32(frag(kFragD1T + 2u * b + 1u), cat(T.dhd[2], T.dhd[3]), a);
    }
}

__device__ __forceinline__ void sample_position(float t, float4 ro, float4 rd, const float* bmin, const float* bmax, float p[3]) {
    const float w[3] = {ro.x + t * rd.x, ro.y + t * rd.y, ro.z + t * rd.z};
    box_relative(w, bmin, bmax, p);
}
__device__ __forceinline__ void sample_geometry(const float2* samples, const uint32_t* sample_ray, const float4* rays, const float* bmin, const float* bmax, uint32_t q, float p[3], float d[3]) {
    const float2 td  = samples[q];
    const uint32_t r = sample_ray[q];
    const float4 ro = rays[2ull * r], rd = rays[2ull * r + 1u];
    d[0] = rd.x;
    d[1] = rd.y;
    d[2] = rd.z;
    sample_position(td.x, ro, rd, bmin, bmax, p);
}

// Value of lane i + o of the same 16-lane row (0 past the row's end): DPP
// row_shl:o.
template <int o>
__device__ __forceinline__ float row_next(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x100 + o, 0xF, 0xF, false));
}
template <int o>
__device__ __forceinline__ uint32_t row_next_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x100 + o, 0xF, 0xF, false);
}
// Value of lane i - 1 of the same 16-lane row (`fill` on the row's first
// lane): DPP row_shr:1, a VALU move rather than an LDS round trip.
__device__ __forceinline__ uint32_t row_prev_u(uint32_t v, uint32_t fill) { return (uint32_t)__builtin_amdgcn_update_dpp((int)fill, (int)v, 0x111, 0xF, 0xF, false); }

template <int o>
__device__ __forceinline__ void combine_step(float v[16], uint32_t seg) {
    const uint32_t ns = row_next_u<o>(seg);
    const bool same   = ns == seg;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const float nv = row_next<o>(v[k]);
        v[k]           = same ? v[k] + nv : v[k];
    }
}

// Coarse-level hash-grid backward: the first n_dense levels (dense, at most
// kCoarseMaxEntries entries).  Consecutive samples mostly share cells there,
// so binned records would crowd into a few bins and global atomics would
// queue on a few hot addresses.  Instead workgroup (chunk, slab) adds the
// contributions of one chunk of samples to the slab's entries in LDS and
// writes them to the chunk's row of the partials, which k_coarse_reduce adds
// in chunk order.  Runs of consecutive samples of a 16-lane row in the same
// cell touch the same 8 corners: their 16 corner values (8 corners x 2
// features) are summed across the run with a segmented suffix scan over DPP
// row shifts, and only the run's first lane adds to LDS.
// The LDS sums are int32 fixed point (fp32 LDS atomics run at a twelfth of
// the rate of integer ones, and 32-bit entries let a slab hold a whole level
// of up to 2^14 entries): a first pass over the chunk's d(feature) pairs of
// the level bounds every entry's sum by S = sum of max(|d0|, |d1|) (the
// corner weights of a sample add to 1), values are scaled by 2^e with
// S * 2^e < 2^30 and rounded to integers, and each entry's exact sum is
// scaled back once; the rounding of a value is at most 2^-31 S, below the
// rounding of the fp16 gradients the reference accumulates.  A non-finite S
// makes the slab's partials NaN, which the statistics report as non-finite.
constexpr uint32_t kCoarseThreads = 1024u;
constexpr uint32_t kCoarseBatch   = 4u;
// Workgroup blk of the coarse scatter; slab: [count][2] LDS words (two's
// complement), wsum: kCoarseThreads / 64 floats.
__device__ __forceinline__ void coarse_scatter_wg(const TrainParams& P, const GridParams& g, const CoarsePlan& C, const TrainDevState* S, const float2* __restrict__ samples, const uint32_t* __restrict__ sample_ray,
                                                  const float4* __restrict__ rays, const float2* __restrict__ dfeat, float2* __restrict__ partials, uint32_t blk, uint32_t* slab, float* wsum) {
    // Workgroup b runs on XCD b % 8: the slabs of one chunk share an XCD, and
    // with it the L2 lines of the chunk's samples.
    const uint32_t xcd = blk & 7u, r = blk >> 3;
    const uint32_t k = r % C.n_slabs, chunk = (r / C.n_slabs) * 8u + xcd;
    const uint32_t level = C.level[k], e0 = C.begin[k], ne = C.count[k];
    for (uint32_t i = threadIdx.x; i < 2u * ne; i += blockDim.x) slab[i] = 0u;
    const uint32_t n   = min(S->n_samples, P.sample_cap);
    const uint32_t per = (n + kCoarseChunks - 1u) / kCoarseChunks;
    const uint32_t s0 = min(n, chunk * per), s1 = min(n, s0 + per);
    const float2* df_level = dfeat + (uint64_t)level * P.sample_cap;
    // kCoarseBatch samples per thread have their loads in flight together.
    float bound = 0.0f;
    for (uint32_t q0 = s0 + threadIdx.x; q0 < s1; q0 += kCoarseBatch * kCoarseThreads) {
        float2 df[kCoarseBatch];
#pragma unroll
        for (uint32_t b = 0; b < kCoarseBatch; ++b) {
            const uint32_t q = q0 + b * kCoarseThreads;
            df[b]            = q < s1 ? df_level[q] : make_float2(0.0f, 0.0f);
        }
#pragma unroll
        for (uint32_t b = 0; b < kCoarseBatch; ++b) {
            bound += fmaxf(fabsf(df[b].x), fabsf(df[b].y));
            if (!isfinite(df[b].x) || !isfinite(df[b].y)) bound = __builtin_inff();  // fmaxf would drop a NaN
        }
    }
    bound = wave_sum(bound);
    if ((threadIdx.x & 63u) == 0u) wsum[threadIdx.x >> 6] = bound;
    __syncthreads();
    bound = 0.0f;
    for (uint32_t w = 0; w < kCoarseThreads / 64u; ++w) bound += wsum[w];
    float4* out = reinterpret_cast<float4*>(partials + (uint64_t)chunk * C.row + C.level_part[level] + e0);
    if (!isfinite(bound)) {  // uniform
        const float nan = __builtin_nanf("");
        for (uint32_t i = threadIdx.x; i < ne / 2u; i += blockDim.x) out[i] = make_float4(nan, nan, nan, nan);
        return;
    }
    const int e = bound > 0.0f ? 29 - ilogbf(bound) : 0;  // bound * 2^e < 2^30
    const uint32_t N = g.resolution[level], s16 = threadIdx.x & 15u;
    for (uint32_t base = s0; base < s1; base += kCoarseBatch * kCoarseThreads) {  // uniform over the workgroup
        float2 td[kCoarseBatch], df[kCoarseBatch];
        uint32_t ray[kCoarseBatch];
#pragma unroll
        for (uint32_t b = 0; b < kCoarseBatch; ++b) {
            const uint32_t q = base + b * kCoarseThreads + threadIdx.x;
            const bool live  = q < s1;
            td[b]            = samples[live ? q : s0];
            ray[b]           = sample_ray[live ? q : s0];
            df[b]            = live ? df_level[q] : make_float2(0.0f, 0.0f);
        }
        float4 ro[kCoarseBatch], rd[kCoarseBatch];
#pragma unroll
        for (uint32_t b = 0; b < kCoarseBatch; ++b) {
            ro[b] = rays[2ull * ray[b]];
            rd[b] = rays[2ull * ray[b] + 1u];
        }
#pragma unroll
        for (uint32_t b = 0; b < kCoarseBatch; ++b) {
            const bool live = base + b * kCoarseThreads + threadIdx.x < s1;
            float p[3];
            sample_position(td[b].x, ro[b], rd[b], P.bmin, P.bmax, p);
            const LevelCell c = level_cell(p, N);
            // The cell's corners span entries [lo, lo + 1 + (N + 1) + (N + 1)^2];
            // a wave none of whose cells reach the slab skips the rest (the
            // samples of a wave are mostly one ray, in a few slabs).
            const uint32_t lo = corner_index(c, 0u, N, true, 0u), hi = lo + 1u + (N + 1u) * (N + 2u);
            if (__ballot(live && hi >= e0 && lo < e0 + ne) == 0ull) continue;  // uniform per wave
            // Cell key; dead lanes get a key no live lane has.
            const uint32_t kx = live ? c.i0[0] : 0xFFFFFFFFu, ky = c.i0[1], kz = c.i0[2];
            const uint32_t px = row_prev_u(kx, ~0u), py = row_prev_u(ky, ~0u), pz = row_prev_u(kz, ~0u);
            const bool head      = s16 == 0u || kx != px || ky != py || kz != pz || !live;
            const uint64_t heads = __ballot(head);
            float v[16];
#pragma unroll
            for (uint32_t j = 0; j < 8u; ++j) {
                const float w  = corner_weight(c, j);
                v[2u * j]      = w * df[b].x;
                v[2u * j + 1u] = w * df[b].y;
            }
            if (heads != ~0ull) {  // some run longer than one sample in the wave
                const uint32_t lane      = threadIdx.x & 63u;
                const uint32_t row_heads = (uint32_t)(heads >> (lane & 48u)) & 0xFFFFu;
                const uint32_t seg       = (uint32_t)__popc(row_heads & ((2u << s16) - 1u));
                combine_step<1>(v, seg);
                combine_step<2>(v, seg);
                combine_step<4>(v, seg);
                combine_step<8>(v, seg);
            }
            if (live && head) {
#pragma unroll
                for (uint32_t j = 0; j < 8u; ++j) {
                    const uint32_t idx = corner_index(c, j, N, true, 0u) - e0;  // wraps past ne below the slab
                    if (idx < ne) {
                        atomicAdd(&slab[2u * idx], (uint32_t)(int32_t)rintf(ldexpf(v[2u * j], e)));
                        atomicAdd(&slab[2u * idx + 1u], (uint32_t)(int32_t)rintf(ldexpf(v[2u * j + 1u], e)));
                    }
                }
            }
        }
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < ne / 2u; i += blockDim.x) {
        float f[4];
#pragma unroll
        for (uint32_t m = 0; m < 4u; ++m) f[m] = ldexpf((float)(int32_t)slab[4u * i + m], -e);
        out[i] = make_float4(f[0], f[1], f[2], f[3]);
    }
}

__global__ __launch_bounds__(kCoarseThreads) void k_coarse_scatter(TrainParams P, GridParams g, CoarsePlan C, const TrainDevState* S, const float2* __restrict__ samples, const uint32_t* __restrict__ sample_ray,
                                                                   const float4* __restrict__ rays, const float2* __restrict__ dfeat, float2* __restrict__ partials) {
    extern __shared__ __align__(16) uint32_t slab[];
    __shared__ float wsum[kCoarseThreads / 64u];
    coarse_scatter_wg(P, g, C, S, samples, sample_ray, rays, dfeat, partials, blockIdx.x, slab, wsum);
}

// Input-gradient pass: d(features) of each tile, loss-scaled, to dfeat
// (level-major: [level][sample] pairs) for the coarse-slab and binned table
// scatters.  Lane (g, s) holds
// features 16b + 4g + e of sample s, i.e. levels 2g, 2g+1 (b = 0) and 8+2g,
// 9+2g (b = 1).
// Weight gradients inside the same pass.  dW = sum over samples of delta
// act^T needs the sample axis on the MFMA reduction axis, so each phase every
// wave puts its tile's deltas and activations of some layers into LDS,
// neuron-major (row = neuron, 16 samples per row); after a barrier the four
// tiles (64 samples = two k-steps of 32) are multiplied out.  The 40 16x16
// blocks of the five weight matrices are split 10 per wave: wave w owns
// output block w of the colour hidden, colour input and density input
// layers and input block w of the two 16-wide output layers, and keeps them
// in registers for the whole pass; the workgroup writes one partial per
// parameter at the end (fixed order throughout, so the result is
// deterministic).  Phases (rows per tile):
//   1: dh2 [0,64) h1 [64,128)
//   2: dh1 [0,64) xc [64,96) do3 [96,112) h2 [112,176)
//   3: dhd [0,64) x  [64,96) dout [96,112) hd [112,176)
// Rows are 48 bytes (16 samples + pad): 16-byte aligned fragment reads, and
// the four rows one 16-bit store instruction writes (r + 4g) fall in two
// bank groups.
constexpr uint32_t kPhaseRows    = 176u;
constexpr uint32_t kOpPitch      = 24u;  // halves per LDS row
constexpr uint32_t kDxFragBytes  = kFrags * 64u * 16u;
constexpr uint32_t kDxOpBytes    = kWaves * kPhaseRows * kOpPitch * 2u;
constexpr uint32_t kDxLds        = kDxFragBytes + kDxOpBytes;  // bytes of dynamic LDS: two workgroups per CU
static_assert(kDxLds <= 81920u, "two workgroups per CU");
static_assert(kMlpParams * 2u <= kDxOpBytes, "raw weights are staged in the operand area");

__device__ __forceinline__ void put_row(half_t* L, uint32_t row, uint32_t s16, half_t v) { L[row * kOpPitch + s16] = v; }
// Rows 16b + 4g + e of a 64-row block starting at row0.  Lanes s16 and
// s16 ^ 1 hold the same rows of neighbouring samples: after one DPP swap of
// a packed pair of rows, the even lane writes the first row and the odd lane
// the second, each as one 4-byte store of both samples (half the LDS store
// instructions of one 2-byte store per value: 49.5 -> 47.8 us per 2^18
// samples, the same rows).
__device__ __forceinline__ void put16(half_t* L, uint32_t row0, const half4_t v[4], uint32_t s16, uint32_t grp) {
    const bool odd = (s16 & 1u) != 0u;
#pragma unroll
    for (uint32_t b = 0; b < 4u; ++b)
#pragma unroll
        for (uint32_t e = 0; e < 4u; e += 2u) {
            const uint32_t own   = __builtin_bit_cast(uint32_t, half2_t{v[b][e], v[b][e + 1u]});
            const uint32_t other = (uint32_t)__builtin_amdgcn_mov_dpp((int)own, 0xB1, 0xf, 0xf, false);  // quad_perm [1, 0, 3, 2]
            // even: (own row e, partner row e); odd: (partner row e + 1, own row e + 1)
            const uint32_t word = odd ? __builtin_amdgcn_perm(own, other, 0x07060302u) : __builtin_amdgcn_perm(other, own, 0x05040100u);
            const uint32_t row  = row0 + 16u * b + 4u * grp + e + (odd ? 1u : 0u);
            *reinterpret_cast<uint32_t*>(L + row * kOpPitch + (s16 & ~1u)) = word;
        }
}
// A or B fragment of rows [row0, row0 + 16) over k-step ks: lane (r, g) takes
// row r, samples 8 (g & 1) .. + 7 of the tile of wave 2 ks + (g >> 1).
__device__ __forceinline__ half8_t op_frag(const half_t* ops, uint32_t row0, uint32_t ks, uint32_t lane) {
    const uint32_t r = lane & 15u, g = lane >> 4;
    const half_t* region = ops + (2u * ks + (g >> 1)) * kPhaseRows * kOpPitch;
    return *reinterpret_cast<const half8_t*>(region + (row0 + r) * kOpPitch + 8u * (g & 1u));
}

// features: rows [n][32], or (features_lm non-null) level-major pairs
// [16][sample_cap].
__global__ __launch_bounds__(kThreads) void k_bwd_dx(TrainParams P, const TrainDevState* S, const half_t* __restrict__ dparams, const half_t* __restrict__ cparams, const half_t* __restrict__ features,
                                                     const uint32_t* __restrict__ features_lm, const float4* __restrict__ draw,
                                                     const float2* __restrict__ samples, const uint32_t* __restrict__ sample_ray, const float4* __restrict__ rays, float2* __restrict__ dfeat, float* __restrict__ partials) {
    extern __shared__ __align__(16) half_t dyn[];
    half8_t* F  = reinterpret_cast<half8_t*>(dyn);
    half_t* ops = dyn + kDxFragBytes / 2u;
    // Raw weights into the operand area, then every fragment built once.
    stage_weights<kThreads>(ops, dparams, cparams);
    __syncthreads();
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u, grp = lane >> 4, s16 = lane & 15u;
    for (uint32_t f = wave; f < kFrags; f += kWaves) F[64u * f + lane] = build_frag(f, ops, ops + NERF_EXT_DENSITY_PARAMS, lane);
    __syncthreads();
    const uint32_t n     = min(S->n_samples, P.sample_cap);
    const uint32_t tiles = (n + 15u) / 16u;
    half_t* W            = ops + wave * kPhaseRows * kOpPitch;  // this wave's operand rows
    const floatx4 zero   = {0.0f, 0.0f, 0.0f, 0.0f};
    floatx4 acc_h[4], acc_ci[2], acc_di[2], acc_co = zero, acc_do = zero;
#pragma unroll
    for (uint32_t i = 0; i < 4u; ++i) acc_h[i] = zero;
    acc_ci[0] = acc_ci[1] = acc_di[0] = acc_di[1] = zero;
    // Every wave of the workgroup runs the same number of iterations (the
    // barriers); a wave past the last tile runs one with zero deltas.
    const uint32_t first = blockIdx.x * kWaves, stride = gridDim.x * kWaves;
    const uint32_t iters = tiles > first ? (tiles - first + stride - 1u) / stride : 0u;
    for (uint32_t it = 0; it < iters; ++it) {
        const uint32_t tile = first + wave + it * stride;
        const uint32_t s    = tile * 16u + s16;
        const bool live     = tile < tiles && s < n;
        const uint32_t q    = live ? s : n - 1u;  // n > 0 here
        float p[3], d[3];
        sample_geometry(samples, sample_ray, rays, P.bmin, P.bmax, q, p, d);
        half8_t x;
        if (features_lm) {
            uint32_t v[4];
#pragma unroll
            for (uint32_t j = 0; j < 4u; ++j) v[j] = features_lm[(uint64_t)(4u * grp + j) * P.sample_cap + q];
            x = __builtin_bit_cast(half8_t, v);
        } else {
            x = *reinterpret_cast<const half8_t*>(features + (uint64_t)q * 32u + 8u * grp);
        }
        float4 gr       = draw[q];
        if (!live) gr = make_float4(0.0f, 0.0f, 0.0f, 0.0f);  // padding samples add nothing to the weight gradients
        TileGrad T;
        tile_backward(F, x, d, gr, P.loss_scale, grp, T);
        if (live) {
#pragma unroll
            for (uint32_t b = 0; b < 2u; ++b) {
                const uint64_t l = 8u * b + 2u * grp;
                dfeat[l * P.sample_cap + s]        = make_float2(T.dx[b][0], T.dx[b][1]);
                dfeat[(l + 1u) * P.sample_cap + s] = make_float2(T.dx[b][2], T.dx[b][3]);
            }
        }
        // Phase 1: colour hidden layer.
        put16(W, 0u, T.dh2, s16, grp);
        put16(W, 64u, T.h1, s16, grp);
        __syncthreads();
#pragma unroll
        for (uint32_t ks = 0; ks < 2u; ++ks) {
            const half8_t a = op_frag(ops, 16u * wave, ks, lane);
#pragma unroll
            for (uint32_t ib = 0; ib < 4u; ++ib) acc_h[ib] = mfma16x16x32(a, op_frag(ops, 64u + 16u * ib, ks, lane), acc_h[ib]);
        }
        __syncthreads();
        // Phase 2: colour input and output layers.
        put16(W, 0u, T.dh1, s16, grp);
#pragma unroll
        for (uint32_t e = 0; e < 8u; ++e) {  // colour input in logical order; row 31 is the zero pad
            const int k = logical_k(KMap::ColorIn, 0u, grp, e);
            put_row(W, 64u + (k < 0 ? 31u : (uint32_t)k), s16, k < 0 ? (half_t)0.0f : T.xc[e]);
            if (8u * grp + e < 16u) put_row(W, 96u + 8u * grp + e, s16, T.do3[e]);
        }
        put16(W, 112u, T.h2, s16, grp);
        __syncthreads();
#pragma unroll
        for (uint32_t ks = 0; ks < 2u; ++ks) {
            const half8_t a = op_frag(ops, 16u * wave, ks, lane);
#pragma unroll
            for (uint32_t ib = 0; ib < 2u; ++ib) acc_ci[ib] = mfma16x16x32(a, op_frag(ops, 64u + 16u * ib, ks, lane), acc_ci[ib]);
            acc_co = mfma16x16x32(op_frag(ops, 96u, ks, lane), op_frag(ops, 112u + 16u * wave, ks, lane), acc_co);
        }
        __syncthreads();
        // Phase 3: density input and output layers.
        put16(W, 0u, T.dhd, s16, grp);
#pragma unroll
        for (uint32_t e = 0; e < 8u; ++e) put_row(W, 64u + 8u * grp + e, s16, T.x[e]);
#pragma unroll
        for (uint32_t e = 0; e < 4u; ++e) put_row(W, 96u + 4u * grp + e, s16, T.dout[e]);
        put16(W, 112u, T.hd, s16, grp);
        __syncthreads();
#pragma unroll
        for (uint32_t ks = 0; ks < 2u; ++ks) {
            const half8_t a = op_frag(ops, 16u * wave, ks, lane);
#pragma unroll
            for (uint32_t ib = 0; ib < 2u; ++ib) acc_di[ib] = mfma16x16x32(a, op_frag(ops, 64u + 16u * ib, ks, lane), acc_di[ib]);
            acc_do = mfma16x16x32(op_frag(ops, 96u, ks, lane), op_frag(ops, 112u + 16u * wave, ks, lane), acc_do);
        }
        __syncthreads();
    }
    // This workgroup's partial of every weight gradient (parameter order:
    // density 0..3071, colour 3072..10239).  Lane (g, s16) of a block holds
    // rows 4g + e (delta neurons), column s16 (activation neurons).
    float* out = partials + (uint64_t)blockIdx.x * kMlpParams;
    constexpr uint32_t D = NERF_EXT_DENSITY_PARAMS;
#pragma unroll
    for (uint32_t e = 0; e < 4u; ++e) {
        const uint32_t o = 16u * wave + 4u * grp + e;  // output neuron of the 64-wide layers
#pragma unroll
        for (uint32_t ib = 0; ib < 4u; ++ib) out[D + 2048u + o * 64u + 16u * ib + s16] = acc_h[ib][e];
#pragma unroll
        for (uint32_t ib = 0; ib < 2u; ++ib) {
            out[D + o * 32u + 16u * ib + s16] = acc_ci[ib][e];
            out[o * 32u + 16u * ib + s16]     = acc_di[ib][e];
        }
        const uint32_t o16 = 4u * grp + e;  // output of the 16-wide layers
        out[D + 6144u + o16 * 64u + 16u * wave + s16] = acc_co[e];
        out[2048u + o16 * 64u + 16u * wave + s16]     = acc_do[e];
    }
}

// Hash-grid backward of the levels past the first n_dense (hashed levels and
// the finer dense ones), binned.  Entry e = (level - n_dense) * T + index
// belongs to bin e / kBinEntries.  k_bin_pass<false> counts each workgroup's
// records per bin (LDS histogram, stored as hist[bin][workgroup]); an exclusive scan of
// that matrix gives every (bin, workgroup) its record range; k_bin_pass<true>
// revisits the same samples in the same order and writes each record
// (entry within the bin, w * d(feature 0), w * d(feature 1)) into its range;
// k_bin_accumulate then sums one bin per workgroup in LDS and writes the
// bin's slice of the gradient once.  No global atomics, and the gradient is
// overwritten rather than accumulated, so it needs no clearing.
// A record is 8 bytes: the two values, each rounded to 17 explicit mantissa
// bits (relative change at most 2^-18), with the entry's 12-bit index within
// its bin in their low 6 bits.  Non-finite values stay non-finite or are
// caught by the bin's maximum, which is taken before packing.
static_assert(kBinEntries == 4096u, "records hold 12 bits of entry index");
__device__ __forceinline__ uint2 pack_record(float v0, float v1, uint32_t entry) {
    return make_uint2(((__float_as_uint(v0) + 32u) & ~63u) | (entry & 63u), ((__float_as_uint(v1) + 32u) & ~63u) | (entry >> 6));
}
__device__ __forceinline__ uint32_t record_entry(uint2 r) { return (r.x & 63u) | ((r.y & 63u) << 6); }
__device__ __forceinline__ float2 record_value(uint2 r) { return make_float2(__uint_as_float(r.x & ~63u), __uint_as_float(r.y & ~63u)); }

// 16 waves per workgroup: the 128 KiB of LDS counters allow one workgroup
// per CU, and the LDS atomics and record stores need several waves per SIMD
// to hide their latency.  Measured no faster: counters sized to the grid's
// bins with two workgroups per CU (236 vs 229 us for the backward), 16-byte
// stores of each x-neighbour record pair (bins padded to even counts).
constexpr uint32_t kBinThreads = 1024u;
// Workgroup blk of nblk; cursor: n_bins LDS words, vmax (kFill): n_bins
// LDS words, the bits of the largest |record value| per bin.
template <bool kFill>
__device__ __forceinline__ void bin_pass_wg(const TrainParams& P, const GridParams& g, const TrainDevState* S, const float2* __restrict__ samples, const uint32_t* __restrict__ sample_ray,
                                            const float4* __restrict__ rays, const float2* __restrict__ dfeat, uint32_t n_dense, uint32_t n_bins, uint32_t* __restrict__ hist, uint2* __restrict__ rec,
                                            uint32_t* __restrict__ bin_max, uint32_t blk, uint32_t nblk, uint32_t* cursor, uint32_t* vmax) {
    for (uint32_t i = threadIdx.x; i < n_bins; i += blockDim.x) {
        cursor[i] = kFill ? hist[(uint64_t)i * nblk + blk] : 0u;
        if constexpr (kFill) vmax[i] = 0u;
    }
    __syncthreads();
    const uint32_t n    = min(S->n_samples, P.sample_cap);
    const uint32_t mask = g.table_size - 1u;
    const uint32_t lane = threadIdx.x & 63u, s16 = lane & 15u;
    // Waves take 64 consecutive samples; all lanes stay active (rows of 16
    // combine runs of samples in the same cell, as in k_coarse_scatter, and only
    // a run's first lane emits its 8 records).
    for (uint32_t base = blk * blockDim.x + (threadIdx.x & ~63u); base < n; base += nblk * blockDim.x) {
        const uint32_t s = base + lane;
        const bool live  = s < n;
        const uint32_t q = live ? s : n - 1u;
        float p[3], d[3];
        sample_geometry(samples, sample_ray, rays, P.bmin, P.bmax, q, p, d);
        for (uint32_t l = n_dense; l < g.n_levels; ++l) {
            const uint32_t N  = g.resolution[l];
            const bool dense  = g.dense[l] != 0u;
            const uint32_t e0 = (l - n_dense) * g.table_size;
            const LevelCell c = level_cell(p, N);
            const uint32_t kx = live ? c.i0[0] : 0xFFFFFFFFu, ky = c.i0[1], kz = c.i0[2];
            const uint32_t px = row_prev_u(kx, ~0u), py = row_prev_u(ky, ~0u), pz = row_prev_u(kz, ~0u);
            const bool head   = s16 == 0u || kx != px || ky != py || kz != pz || !live;
            float v[16];
            if constexpr (kFill) {
                const float2 df = live ? dfeat[(uint64_t)l * P.sample_cap + q] : make_float2(0.0f, 0.0f);
                const float d0 = df.x, d1 = df.y;
#pragma unroll
                for (uint32_t k = 0; k < 8u; ++k) {
                    const float w  = corner_weight(c, k);
                    v[2u * k]      = w * d0;
                    v[2u * k + 1u] = w * d1;
                }
                const uint64_t heads = __ballot(head);
                if (heads != ~0ull) {
                    const uint32_t row_heads = (uint32_t)(heads >> (lane & 48u)) & 0xFFFFu;
                    const uint32_t seg       = (uint32_t)__popc(row_heads & ((2u << s16) - 1u));
                    combine_step<1>(v, seg);
                    combine_step<2>(v, seg);
                    combine_step<4>(v, seg);
                    combine_step<8>(v, seg);
                }
            }
            if (!(live && head)) continue;
            // Corners k (x) and k + 1 (x + 1) of each (y, z) edge: adjacent
            // entries on a dense level, entries differing in their low bits
            // (x's prime is 1) on a hashed one, so almost always in one bin:
            // one cursor increment reserves both records' slots (and one
            // maximum covers their four values), which halves the LDS atomics
            // of both passes.  A pair that straddles a bin edge takes a slot
            // in each bin.
#pragma unroll
            for (uint32_t k = 0; k < 8u; k += 2u) {
                const uint32_t ea = e0 + corner_index(c, k, N, dense, mask);
                const uint32_t eb = e0 + corner_index(c, k + 1u, N, dense, mask);
                const uint32_t ba = ea / kBinEntries, bb = eb / kBinEntries;
                uint32_t sa, sb;
                if (ba == bb) {
                    sa = atomicAdd(&cursor[ba], 2u);
                    sb = sa + 1u;
                } else {
                    sa = atomicAdd(&cursor[ba], 1u);
                    sb = atomicAdd(&cursor[bb], 1u);
                }
                if constexpr (kFill) {
                    // |x| as bits orders like |x| for finite x; NaN and inf compare above every finite value.
                    const uint32_t ma = max(__float_as_uint(v[2u * k]) & 0x7FFFFFFFu, __float_as_uint(v[2u * k + 1u]) & 0x7FFFFFFFu);
                    const uint32_t mb = max(__float_as_uint(v[2u * k + 2u]) & 0x7FFFFFFFu, __float_as_uint(v[2u * k + 3u]) & 0x7FFFFFFFu);
                    if (ba == bb) {
                        atomicMax(&vmax[ba], max(ma, mb));
                    } else {
                        atomicMax(&vmax[ba], ma);
                        atomicMax(&vmax[bb], mb);
                    }
                    rec[sa] = pack_record(v[2u * k], v[2u * k + 1u], ea % kBinEntries);
                    rec[sb] = pack_record(v[2u * k + 2u], v[2u * k + 3u], eb % kBinEntries);
                }
            }
        }
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < n_bins; i += blockDim.x) {
        if constexpr (kFill) bin_max[(uint64_t)i * nblk + blk] = vmax[i];
        else hist[(uint64_t)i * nblk + blk] = cursor[i];
    }
}

template <bool kFill>
__global__ __launch_bounds__(kBinThreads) void k_bin_pass(TrainParams P, GridParams g, const TrainDevState* S, const float2* __restrict__ samples, const uint32_t* __restrict__ sample_ray, const float4* __restrict__ rays,
                                                  const float2* __restrict__ dfeat, uint32_t n_dense, uint32_t n_bins, uint32_t* __restrict__ hist, uint2* __restrict__ rec,
                                                  uint32_t* __restrict__ bin_max) {
    __shared__ uint32_t cursor[kMaxBins];
    __shared__ uint32_t vmax[kFill ? kMaxBins : 1u];
    bin_pass_wg<kFill>(P, g, S, samples, sample_ray, rays, dfeat, n_dense, n_bins, hist, rec, bin_max, blockIdx.x, gridDim.x, cursor, vmax);
}

// Fill pass with the records staged in LDS, for grids whose per-bin state
// fits beside the stage (n_bins <= kStagedMaxBins).  The workgroup takes one
// level of its chunk of samples per round: every head lane reserves its
// records' slots as in k_bin_pass<true> (the same slots, since the cursors
// advance the same way), then the round's records are placed in LDS by bin
// (an exclusive scan of the round's per-bin counts) and written out in that
// order, so consecutive lanes store consecutive slots of one bin's range
// instead of one scattered 8-byte store per record.  (Left out, those
// stores were half of k_bin_pass<true>: 74 -> 38 us at 2^18 samples of 1,024
// steps, 136 -> 32 us at 4,096 rays of 64 steps; staged: 90 and 98 us.)
// Records, slots and the per-bin maxima are those of k_bin_pass<true>; only
// the order in which they reach memory differs.
constexpr uint32_t kStageRecords  = kBinThreads * 8u;  // at most 8 records per lane and level
constexpr uint32_t kStageBytes    = kStageRecords * (sizeof(uint2) + sizeof(uint32_t));
constexpr uint32_t kStagedMaxBins = (160u * 1024u - kStageBytes - 1024u) / (4u * sizeof(uint32_t));
__host__ __device__ constexpr uint32_t staged_fill_lds(uint32_t n_bins) { return kStageBytes + 4u * sizeof(uint32_t) * ((n_bins + 1u) & ~1u); }

// Workgroup barrier for LDS data only: waits for this wave's LDS operations,
// not for its global loads and stores (which __syncthreads also drains).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Workgroup blk of nblk; lds_words: staged_fill_lds(n_bins) bytes; wave_tot:
// kBinThreads / 64 LDS words.
__device__ __forceinline__ void bin_fill_staged_wg(const TrainParams& P, const GridParams& g, const TrainDevState* S, const float2* __restrict__ samples, const uint32_t* __restrict__ sample_ray,
                                                   const float4* __restrict__ rays, const float2* __restrict__ dfeat, uint32_t n_dense, uint32_t n_bins, const uint32_t* __restrict__ hist,
                                                   uint2* __restrict__ rec, uint32_t* __restrict__ bin_max, uint32_t blk, uint32_t nblk, uint32_t* lds_words, uint32_t* wave_tot) {
    uint2* st_rec      = reinterpret_cast<uint2*>(lds_words);  // [kStageRecords]
    uint32_t* st_slot  = lds_words + 2u * kStageRecords;       // [kStageRecords] global slot of each staged record
    const uint32_t nb2 = (n_bins + 1u) & ~1u;
    uint32_t* cursor   = st_slot + kStageRecords;  // [n_bins] next global slot of each bin's range
    uint32_t* vmax     = cursor + nb2;             // [n_bins] bits of the largest |record value|
    uint32_t* start    = vmax + nb2;               // [n_bins] the round's first slot
    uint32_t* pos      = start + nb2;              // [n_bins] LDS position of slot x of bin b: x + pos[b]
    for (uint32_t i = threadIdx.x; i < n_bins; i += blockDim.x) {
        const uint32_t h = hist[(uint64_t)i * nblk + blk];
        cursor[i]        = h;
        start[i]         = h;
        vmax[i]          = 0u;
    }
    __syncthreads();
    const uint32_t n    = min(S->n_samples, P.sample_cap);
    const uint32_t mask = g.table_size - 1u;
    const uint32_t lane = threadIdx.x & 63u, s16 = lane & 15u, wave = threadIdx.x >> 6;
    const uint32_t per  = (n_bins + blockDim.x - 1u) / blockDim.x;  // bins per thread in the scan
    // Chunks of blockDim.x consecutive samples, the same samples per wave as
    // k_bin_pass (wave w of the workgroup holds samples chunk + 64 w ..).
    for (uint32_t chunk = blk * blockDim.x; chunk < n; chunk += nblk * blockDim.x) {
        const uint32_t s = chunk + threadIdx.x;
        const bool live  = s < n;
        const uint32_t q = live ? s : n - 1u;
        float p[3], d[3];
        sample_geometry(samples, sample_ray, rays, P.bmin, P.bmax, q, p, d);
        // d(features) of the next level are loaded a round ahead.
        float2 df_next = live ? dfeat[(uint64_t)n_dense * P.sample_cap + q] : make_float2(0.0f, 0.0f);
        for (uint32_t l = n_dense; l < g.n_levels; ++l) {
            const float2 df = df_next;
            if (l + 1u < g.n_levels) df_next = live ? dfeat[(uint64_t)(l + 1u) * P.sample_cap + q] : make_float2(0.0f, 0.0f);
            const uint32_t N  = g.resolution[l];
            const bool dense  = g.dense[l] != 0u;
            const uint32_t e0 = (l - n_dense) * g.table_size;
            const LevelCell c = level_cell(p, N);
            const uint32_t kx = live ? c.i0[0] : 0xFFFFFFFFu, ky = c.i0[1], kz = c.i0[2];
            const uint32_t px = row_prev_u(kx, ~0u), py = row_prev_u(ky, ~0u), pz = row_prev_u(kz, ~0u);
            const bool head   = s16 == 0u || kx != px || ky != py || kz != pz || !live;
            float v[16];
#pragma unroll
            for (uint32_t k = 0; k < 8u; ++k) {
                const float w  = corner_weight(c, k);
                v[2u * k]      = w * df.x;
                v[2u * k + 1u] = w * df.y;
            }
            const uint64_t heads = __ballot(head);
            if (heads != ~0ull) {
                const uint32_t row_heads = (uint32_t)(heads >> (lane & 48u)) & 0xFFFFu;
                const uint32_t seg       = (uint32_t)__popc(row_heads & ((2u << s16) - 1u));
                combine_step<1>(v, seg);
                combine_step<2>(v, seg);
                combine_step<4>(v, seg);
                combine_step<8>(v, seg);
            }
            const bool emits = live && head;
            // This lane's records: the corners of edge (y, z) k / 2 as records k, k + 1.
            uint2 r[8];
            uint32_t rbin[8], rslot[8];
#pragma unroll
            for (uint32_t k = 0; k < 8u; k += 2u) {
                rbin[k] = rbin[k + 1u] = 0xFFFFFFFFu;
                if (!emits) continue;
                const uint32_t ea = e0 + corner_index(c, k, N, dense, mask);
                const uint32_t eb = e0 + corner_index(c, k + 1u, N, dense, mask);
                const uint32_t ba = ea / kBinEntries, bb = eb / kBinEntries;
                uint32_t sa, sb;
                const uint32_t ma = max(__float_as_uint(v[2u * k]) & 0x7FFFFFFFu, __float_as_uint(v[2u * k + 1u]) & 0x7FFFFFFFu);
                const uint32_t mb = max(__float_as_uint(v[2u * k + 2u]) & 0x7FFFFFFFu, __float_as_uint(v[2u * k + 3u]) & 0x7FFFFFFFu);
                if (ba == bb) {
                    sa = atomicAdd(&cursor[ba], 2u);
                    sb = sa + 1u;
                    atomicMax(&vmax[ba], max(ma, mb));
                } else {
                    sa = atomicAdd(&cursor[ba], 1u);
                    sb = atomicAdd(&cursor[bb], 1u);
                    atomicMax(&vmax[ba], ma);
                    atomicMax(&vmax[bb], mb);
                }
                r[k]          = pack_record(v[2u * k], v[2u * k + 1u], ea % kBinEntries);
                r[k + 1u]     = pack_record(v[2u * k + 2u], v[2u * k + 3u], eb % kBinEntries);
                rbin[k]       = ba;
                rbin[k + 1u]  = bb;
                rslot[k]      = sa;
                rslot[k + 1u] = sb;
            }
            lds_barrier();
            // Exclusive scan of the round's per-bin counts: thread t sums bins
            // [t per, (t + 1) per), waves scan the thread sums, the wave totals
            // are added in LDS; each bin's round then starts at its cursor.
            const uint32_t b0 = min(threadIdx.x * per, n_bins), b1 = min(b0 + per, n_bins);
            uint32_t own = 0u;
            for (uint32_t b = b0; b < b1; ++b) own += cursor[b] - start[b];
            uint32_t inc = own;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t up = (uint32_t)__shfl_up((int)inc, o, 64);
                if (lane >= (uint32_t)o) inc += up;
            }
            if (lane == 63u) wave_tot[wave] = inc;
            lds_barrier();
            uint32_t before = 0u, total = 0u;
            for (uint32_t w = 0; w < blockDim.x / 64u; ++w) {
                const uint32_t t = wave_tot[w];
                before += w < wave ? t : 0u;
                total += t;
            }
            uint32_t off = before + inc - own;
            for (uint32_t b = b0; b < b1; ++b) {
                const uint32_t first = start[b], end = cursor[b];
                pos[b]   = off - first;
                start[b] = end;
                off += end - first;
            }
            lds_barrier();
#pragma unroll
            for (uint32_t k = 0; k < 8u; ++k) {
                if (rbin[k] == 0xFFFFFFFFu) continue;
                const uint32_t at = rslot[k] + pos[rbin[k]];
                st_rec[at]        = r[k];
                st_slot[at]       = rslot[k];
            }
            lds_barrier();
            for (uint32_t i = threadIdx.x; i < total; i += blockDim.x) rec[st_slot[i]] = st_rec[i];
            // The next round's atomics touch only the cursors, and its stage
            // writes come after two more barriers.
        }
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < n_bins; i += blockDim.x) bin_max[(uint64_t)i * nblk + blk] = vmax[i];
}

// The coarse levels' scatter and the record fill in one launch: the first
// n_coarse workgroups take the coarse slabs (their dynamic LDS is the slab),
// the other kBinBlocks the fill (the same LDS as its cursors and maxima, or
// its stage).  One launch instead of two: the fill's workgroups start on each
// CU as the coarse ones finish there.
template <bool kStaged>
__global__ __launch_bounds__(kBinThreads) void k_scatter_fill(TrainParams P, GridParams g, CoarsePlan C, const TrainDevState* S, const float2* __restrict__ samples, const uint32_t* __restrict__ sample_ray,
                                                              const float4* __restrict__ rays, const float2* __restrict__ dfeat, float2* __restrict__ partials, uint32_t n_coarse, uint32_t n_dense,
                                                              uint32_t n_bins, uint32_t* __restrict__ hist, uint2* __restrict__ rec, uint32_t* __restrict__ bin_max) {
    static_assert(kCoarseThreads == kBinThreads, "one workgroup size for both parts");
    extern __shared__ __align__(16) uint32_t lds_words[];
    __shared__ float wsum[kBinThreads / 64u];
    __shared__ uint32_t wave_tot[kBinThreads / 64u];
    if (blockIdx.x < n_coarse) {
        coarse_scatter_wg(P, g, C, S, samples, sample_ray, rays, dfeat, partials, blockIdx.x, lds_words, wsum);
        return;
    }
    const uint32_t blk = blockIdx.x - n_coarse;
    if constexpr (kStaged) bin_fill_staged_wg(P, g, S, samples, sample_ray, rays, dfeat, n_dense, n_bins, hist, rec, bin_max, blk, kBinBlocks, lds_words, wave_tot);
    else bin_pass_wg<true>(P, g, S, samples, sample_ray, rays, dfeat, n_dense, n_bins, hist, rec, bin_max, blk, kBinBlocks, lds_words, lds_words + n_bins);
}

// One bin per workgroup.  fp32 LDS atomics run at a twelfth of the rate of
// 64-bit integer ones on gfx950, so the bin is accumulated in fixed point:
// a first pass over the bin's records finds max |v|, every value is scaled
// by the power of two 2^e that puts that maximum at 2^40 and rounded to an
// int64, and the int64 sums (exact, so independent of the order of the
// records) are scaled back once.  Contributions below 2^-40 of the bin's
// largest one round to zero.  A non-finite record makes the whole slice
// NaN, which the gradient statistics report as non-finite.
// grad points at the first hashed level; entries = hashed levels x T.
// acc: 2 kBinEntries int64 of LDS; wmax, wsq: 16 each.
__device__ void bin_accumulate(uint32_t bin, const uint32_t* __restrict__ offsets, uint32_t n_blocks, uint32_t n_bins, const unsigned long long* __restrict__ total, const uint2* __restrict__ rec,
                               const uint32_t* __restrict__ bin_max, uint64_t entries, float2* __restrict__ grad, double* __restrict__ norm, unsigned long long* acc, uint32_t* wmax, double* wsq) {
    for (uint32_t i = threadIdx.x; i < 2u * kBinEntries; i += blockDim.x) acc[i] = 0ull;
    const uint32_t begin = offsets[(uint64_t)bin * n_blocks];
    const uint32_t end   = bin + 1u < n_bins ? offsets[(uint64_t)(bin + 1u) * n_blocks] : (uint32_t)*total;
    // Largest |record value| of the bin, as bits: the maximum of the fill
    // pass's per-workgroup maxima (bits above 0x7F800000 - NaN - or equal to
    // it - inf - mark a non-finite record).
    uint32_t mb = 0u;
    for (uint32_t i = threadIdx.x; i < n_blocks; i += blockDim.x) mb = max(mb, bin_max[(uint64_t)bin * n_blocks + i]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mb = max(mb, (uint32_t)__shfl_xor((int)mb, o, 64));
    if ((threadIdx.x & 63u) == 0u) wmax[threadIdx.x >> 6] = mb;
    __syncthreads();
    mb = 0u;
    for (uint32_t w = 0; w < blockDim.x / 64u; ++w) mb = max(mb, wmax[w]);
    const float mx      = __uint_as_float(mb);
    const uint64_t base = (uint64_t)bin * kBinEntries;
    if (mb >= 0x7F800000u) {  // NaN or inf among the records
        for (uint32_t i = threadIdx.x; i < kBinEntries; i += blockDim.x)
            if (base + i < entries) grad[base + i] = make_float2(__builtin_nanf(""), __builtin_nanf(""));
        if (threadIdx.x == 0u) norm[bin] = -1.0;
        return;
    }
    const int e        = mx > 0.0f ? 39 - ilogbf(mx) : 0;  // mx * 2^e in [2^39, 2^40)
    const double scale = ldexp(1.0, e);
    // Batches of 8 coalesced record loads per thread are issued before their
    // LDS atomics, so the loads of a batch are in flight together.
    constexpr uint32_t kBatch = 8u;
    for (uint32_t r0 = begin; r0 < end; r0 += kBatch * blockDim.x) {
        uint32_t idx[kBatch];
        float2 val[kBatch];
#pragma unroll
        for (uint32_t k = 0; k < kBatch; ++k) {
            const uint32_t r = r0 + k * blockDim.x + threadIdx.x;
            const uint2 w    = r < end ? rec[r] : make_uint2(0u, 0u);
            idx[k]           = record_entry(w);
            val[k]           = record_value(w);
        }
#pragma unroll
        for (uint32_t k = 0; k < kBatch; ++k) {
            if (r0 + k * blockDim.x + threadIdx.x < end) {
                atomicAdd(&acc[2u * idx[k]], (unsigned long long)llrint((double)val[k].x * scale));
                atomicAdd(&acc[2u * idx[k] + 1u], (unsigned long long)llrint((double)val[k].y * scale));
            }
        }
    }
    __syncthreads();
    // The bin's gradient, and its share of the squared gradient norm (one
    // partial per workgroup, added by the last workgroup to finish).
    const double inv = ldexp(1.0, -e);
    double sq        = 0.0;
    for (uint32_t i = threadIdx.x; i < kBinEntries; i += blockDim.x)
        if (base + i < entries) {
            const float gx = (float)((double)(long long)acc[2u * i] * inv), gy = (float)((double)(long long)acc[2u * i + 1u] * inv);
            grad[base + i] = make_float2(gx, gy);
            sq += (double)gx * (double)gx + (double)gy * (double)gy;
        }
    sq = wave_sum_d(sq);
    if ((threadIdx.x & 63u) == 0u) wsq[threadIdx.x >> 6] = sq;
    __syncthreads();
    if (threadIdx.x == 0u) {
        double b = 0.0;
        for (uint32_t w = 0; w < blockDim.x / 64u; ++w) b += wsq[w];
        norm[bin] = b;
    }
}

// Sum of the per-workgroup partials: a workgroup takes 16 columns of 4
// parameters; its 16 slices of 16 threads each add every 16th partial (16
// independent four-wide loads per thread), then the slices are added in a
// fixed order.  The MLP gradient's share of the squared norm is taken here,
// from the values written: one partial per workgroup, added by the last
// workgroup to finish.
constexpr uint32_t kReduceSlices = 16u;
// Part vb of the MLP weight-gradient reduction, run by the 256 threads t of
// half h of a 512-thread workgroup (each half has its own slice sums; both
// halves reach the barrier, an out-of-range part only takes part in it).
// part_h: LDS of 2 x kReduceSlices x 16 float4.
__device__ void dw_reduce(uint32_t vb, uint32_t t, uint32_t h, const float* __restrict__ partials, uint32_t blocks, float* __restrict__ grad, double* __restrict__ norm, float4 (*part_h)[kReduceSlices][16]) {
    static_assert(kMlpParams % 64u == 0u, "whole columns per workgroup");
    float4 (*part)[16] = part_h[h];
    const bool valid   = vb < kMlpParams / 64u;
    const uint32_t col = t & 15u, slice = t >> 4;
    const uint32_t c   = vb * 16u + col;  // float4 column
    const float4* p4   = reinterpret_cast<const float4*>(partials);
    float4 s           = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    // Batches of 8 loads in flight, added in partial order.
    for (uint32_t b0 = slice; valid && b0 < blocks; b0 += 8u * kReduceSlices) {
        float4 v[8];
#pragma unroll
        for (uint32_t k = 0; k < 8u; ++k) {
            const uint32_t b = b0 + k * kReduceSlices;
            v[k]             = b < blocks ? p4[(uint64_t)b * (kMlpParams / 4u) + c] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (uint32_t k = 0; k < 8u; ++k) {
            s.x += v[k].x;
            s.y += v[k].y;
            s.z += v[k].z;
            s.w += v[k].w;
        }
    }
    part[slice][col] = s;
    __syncthreads();
    if (t >= 64u || !valid) return;
    // Thread t < 64: parameter 4 * (vb * 16) + t.
    const uint32_t cc = t >> 2, e = t & 3u;
    float gi          = 0.0f;
    for (uint32_t k = 0; k < kReduceSlices; ++k) {
        const float4 v = part[k][cc];
        gi += e == 0u ? v.x : e == 1u ? v.y : e == 2u ? v.z : v.w;
    }
    grad[vb * 64u + t] = gi;
    const bool finite = isfinite(gi);
    const double sq   = wave_sum_d(finite ? (double)gi * (double)gi : 0.0);
    if (t == 0u) norm[vb] = __ballot(!finite) != 0ull ? -1.0 - sq : sq;
}

// Sum of the coarse levels' chunk partials, in chunk order (the same layout
// of work as k_dw_reduce: 16 columns of two entries per workgroup, 16 slices
// of the chunks), written to the levels' gradient; their share of the squared
// norm is taken from the values written, as in k_dw_reduce.  Entries
// past a level's (N + 1)^3 are never written and stay zero.
static_assert(kCoarseChunks % kReduceSlices == 0u, "whole slices of chunks");
// Part vb of the coarse levels' reduction, by the 256 threads t of half h of
// a 512-thread workgroup, as dw_reduce.
__device__ void coarse_reduce(uint32_t vb, uint32_t t, uint32_t h, const float2* __restrict__ partials, const CoarsePlan& C, uint32_t n_levels, uint32_t table_size, float* __restrict__ grad, double* __restrict__ norm,
                              float4 (*part_h)[kReduceSlices][16]) {
    float4 (*part)[16] = part_h[h];
    const bool in_range = vb < coarse_reduce_blocks(C);
    const uint32_t col = t & 15u, slice = t >> 4;
    const uint32_t cols = C.row / 2u;
    const uint32_t c    = vb * 16u + col;  // entries 2c, 2c + 1 of a partial row
    const float4* p4    = reinterpret_cast<const float4*>(partials);
    float4 s            = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (in_range && c < cols) {
        constexpr uint32_t kPer = kCoarseChunks / kReduceSlices;
        float4 v[kPer];
#pragma unroll
        for (uint32_t k = 0; k < kPer; ++k) v[k] = p4[(uint64_t)(slice + k * kReduceSlices) * cols + c];
#pragma unroll
        for (uint32_t k = 0; k < kPer; ++k) {
            s.x += v[k].x;
            s.y += v[k].y;
            s.z += v[k].z;
            s.w += v[k].w;
        }
    }
    part[slice][col] = s;
    __syncthreads();
    if (t >= 64u || !in_range) return;
    // Thread t < 64: component t & 3 (entry t >> 1 & 1, feature t & 1) of column t >> 2.
    const uint32_t cc = t >> 2, comp = t & 3u;
    float gi          = 0.0f;
    for (uint32_t k = 0; k < kReduceSlices; ++k) {
        const float4 v = part[k][cc];
        gi += comp == 0u ? v.x : comp == 1u ? v.y : comp == 2u ? v.z : v.w;
    }
    const uint32_t e = 2u * (vb * 16u + cc) + (comp >> 1);  // entry of the partial row
    uint32_t l       = 0u;
    while (l + 1u < n_levels && e >= C.level_part[l + 1u]) ++l;
    const uint32_t el = e - C.level_part[l];
    const bool valid  = e < C.row && el < C.level_entries[l];
    if (valid) grad[((uint64_t)l * table_size + el) * 2u + (comp & 1u)] = gi;
    const bool finite = !valid || isfinite(gi);
    const double sq   = wave_sum_d(valid && finite ? (double)gi * (double)gi : 0.0);
    if (t == 0u) norm[vb] = __ballot(!finite) != 0ull ? -1.0 - sq : sq;
}

// The gradient reductions of a step in one launch of 512-thread workgroups
// (each launch costs about 4.5 us here, and the three parts are independent):
// the first workgroups take pairs of coarse-level parts, the next pairs of
// MLP weight-gradient parts (two 256-thread parts per workgroup; first, so
// that these short parts run beside the bins rather than after them), the
// rest one bin each.  norm gets one partial per part: coarse parts first,
// then the bins, then the MLP parts.
struct GradReduceArgs {
    const uint32_t* bin_off;
    uint32_t n_bins;
    const unsigned long long* bin_total;
    const uint2* rec;
    const uint32_t* bin_max;
    uint64_t hashed_entries;
    float2* hashed_grad;
    const float2* coarse_partials;
    CoarsePlan coarse;
    uint32_t n_dense;
    uint32_t table_size;
    float* table_grad;
    const float* dw_partials;
    uint32_t dw_blocks;
    float* mlp_grad;
    double* norm;
};
__global__ __launch_bounds__(512) void k_grad_reduce(GradReduceArgs a) {
    // One LDS allocation for every part (the bins' 64 KiB of sums, which the
    // reduction parts reuse for their slice sums), so two workgroups fit a CU.
    __shared__ unsigned long long acc[2u * kBinEntries];
    __shared__ uint32_t wmax[16];
    __shared__ double wsq[16];
    static_assert(2u * kReduceSlices * 16u * sizeof(float4) <= sizeof(acc), "slice sums fit the bins' LDS");
    float4 (*part_h)[kReduceSlices][16] = reinterpret_cast<float4 (*)[kReduceSlices][16]>(acc);
    const uint32_t coarse_parts = coarse_reduce_blocks(a.coarse);  // norm partials of the coarse levels
    const uint32_t coarse_pairs = a.n_dense ? (coarse_parts + 1u) / 2u : 0u;
    const uint32_t t = threadIdx.x & 255u, h = threadIdx.x >> 8;
    const uint32_t b = blockIdx.x;
    if (b < coarse_pairs) {
        const uint32_t vb = 2u * b + h;
        coarse_reduce(vb < coarse_parts ? vb : 0xFFFFFFFFu, t, h, a.coarse_partials, a.coarse, a.n_dense, a.table_size, a.table_grad, a.norm, part_h);
    } else if (b < coarse_pairs + kMlpParams / 128u) {
        dw_reduce(2u * (b - coarse_pairs) + h, t, h, a.dw_partials, a.dw_blocks, a.mlp_grad, a.norm + coarse_parts + a.n_bins, part_h);
    } else {
        bin_accumulate(b - coarse_pairs - kMlpParams / 128u, a.bin_off, kBinBlocks, a.n_bins, a.bin_total, a.rec, a.bin_max, a.hashed_entries, a.hashed_grad, a.norm + coarse_parts, acc, wmax,
                       wsq);
    }
}

// The step's squared gradient norm: the sum, in a fixed order, of the
// per-workgroup partials of the gradient sums (coarse chunks, bins, weight
// gradients; the reference model's weight-gradient reduction).  A partial is
// the sum of squares of the workgroup's finite gradient values, or -1 minus
// that sum when one of its values is not finite (the statistics of
// backend-cuda.cu:1451-1476: finite values summed, a separate flag).
// Per-workgroup atomics on one address would serialize; this sum is also
// independent of the order the workgroups ran in.  Each thread adds every
// kNormThreads-th partial, then the waves are added in order.  Writes the
// statistics and Adam's copy of them; end: then the end of the step.
constexpr uint32_t kNormThreads = 1024u;
__global__ __launch_bounds__(kNormThreads) void k_grad_norm(TrainParams P, const double* __restrict__ norm, uint32_t n, TrainDevState* S, const TrainDevState* prev, bool end) {
    __shared__ double ws[kNormThreads / 64u];
    __shared__ uint32_t bad;
    if (threadIdx.x == 0u) bad = 0u;
    __syncthreads();
    double acc      = 0.0;
    bool nonfinite  = false;
    for (uint32_t i = threadIdx.x; i < n; i += kNormThreads) {
        const double v = norm[i];
        nonfinite      = nonfinite || v < 0.0;
        acc += v < 0.0 ? -1.0 - v : v;
    }
    acc = wave_sum_d(acc);
    if ((threadIdx.x & 63u) == 0u) ws[threadIdx.x >> 6] = acc;
    if (nonfinite) bad = 1u;
    __syncthreads();
    if (threadIdx.x == 0u) {
        double t = 0.0;
        for (uint32_t w = 0; w < kNormThreads / 64u; ++w) t += ws[w];
        S->grad_sumsq     = t;
        S->nonfinite      = bad;
        if (end) step_end(P, S, prev);
    }
}

// ------------------------------------------------------------------ Adam
// :1513-1536: skip guard, lr decay, clip factor, bias corrections, from the
// step's gradient statistics.
struct AdamCoef {
    float lr, gs, bc1, bc2;  // gs: clip factor / loss scale
    uint32_t skip;
};
// From the step's own state slot (the next step's begin writes the other).
__device__ AdamCoef adam_coef(const TrainParams& P, const TrainDevState* S) {
    const float gn   = (float)sqrt(S->grad_sumsq > 0.0 ? S->grad_sumsq : 0.0) / P.loss_scale;
    const uint32_t t = S->frame + 1u;  // optimizer step
    AdamCoef c;
    c.skip = (S->nonfinite != 0u || !isfinite(gn) || gn > P.guard) ? 1u : 0u;
    if (c.skip) {
        c.lr = 0.0f;
        c.gs = 1.0f / P.loss_scale;
        c.bc1 = c.bc2 = 1.0f;
        return c;
    }
    const float decay = (float)P.lr_decay_ksteps * 1000.0f;
    c.lr              = decay > 0.0f ? P.lr * powf(0.1f, (float)t / decay) : P.lr;
    c.gs              = ((gn > P.clip && gn > 0.0f) ? P.clip / gn : 1.0f) * (1.0f / P.loss_scale);
    c.bc1             = 1.0f / (1.0f - powf(P.beta1, (float)t));
    c.bc2             = 1.0f / (1.0f - powf(P.beta2, (float)t));
    return c;
}

struct AdamSeg {
    float* w;
    half_t* w16;
    const float* g;
    float* m;
    float* v;
};

__device__ __forceinline__ float adam_one(const AdamCoef& c, const TrainParams& P, float& w, float g, float& m, float& v) {
    const float gr = g * c.gs;
    m              = P.beta1 * m + (1.0f - P.beta1) * gr;
    v              = P.beta2 * v + (1.0f - P.beta2) * gr * gr;
    w              = w - c.lr * (m * c.bc1) / (sqrtf(v * c.bc2) + P.eps);
    return w;
}

// :1537-1554 on fp32 masters with fp16 working copies, all parameters in one
// launch: the hash table four at a time (n_table is a multiple of 4), then
// the density and colour MLPs (contiguous masters, moments and gradients;
// separate fp16 copies).  Every workgroup derives the step's coefficients
// itself.  The backward pass overwrites the gradients every step, so they
// are not cleared here.
__global__ __launch_bounds__(256) void k_adam(TrainParams P, TrainDevState* S, AdamSeg table, uint64_t n_table, AdamSeg mlp, half_t* __restrict__ w16_color, uint32_t n_density, uint32_t n_mlp) {
    __shared__ AdamCoef coef;
    if (threadIdx.x == 0u) {
        coef = adam_coef(P, S);
        if (blockIdx.x == 0u) S->skip = coef.skip;
    }
    __syncthreads();
    const AdamCoef c = coef;
    if (c.skip) return;
    const uint64_t step = (uint64_t)gridDim.x * blockDim.x;
    const uint64_t n4 = n_table / 4u, total = n4 + n_mlp;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += step) {
        if (i < n4) {
            // The fp32 streams (64 MiB each) pass through once per step:
            // non-temporal, so they do not sweep the caches.
            floatx4 w = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(table.w) + i), m = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(table.m) + i);
            floatx4 v = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(table.v) + i);
            const floatx4 g = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(table.g) + i);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                float wk = w[k], mk = m[k], vk = v[k];
                adam_one(c, P, wk, g[k], mk, vk);
                w[k] = wk;
                m[k] = mk;
                v[k] = vk;
            }
            __builtin_nontemporal_store(w, reinterpret_cast<floatx4*>(table.w) + i);
            __builtin_nontemporal_store(m, reinterpret_cast<floatx4*>(table.m) + i);
            __builtin_nontemporal_store(v, reinterpret_cast<floatx4*>(table.v) + i);
            half4_t h = {to_half_rne(w[0]), to_half_rne(w[1]), to_half_rne(w[2]), to_half_rne(w[3])};
            reinterpret_cast<half4_t*>(table.w16)[i] = h;
        } else {
            const uint32_t j = (uint32_t)(i - n4);
            float w = mlp.w[j], m = mlp.m[j], v = mlp.v[j];
            adam_one(c, P, w, mlp.g[j], m, v);
            mlp.w[j] = w;
            mlp.m[j] = m;
            mlp.v[j] = v;
            if (j < n_density) mlp.w16[j] = to_half_rne(w);
            else w16_color[j - n_density] = to_half_rne(w);
        }
    }
}

// Workgroups of a one-wave-per-ray kernel: one wave per ray slot, at most
// 16 workgroups (64 waves) per CU; the kernels loop over the remaining slots.
uint32_t ray_wave_blocks(uint32_t max_rays) {
    const uint32_t need = (max_rays + kWaves - 1u) / kWaves;
    const uint32_t cap  = device_cu_count() * 16u;
    return need < cap ? (need > 0u ? need : 1u) : cap;
}

uint32_t grid_for(uint64_t n, uint32_t cap) {
    const uint64_t b = (n + 255u) / 256u;
    return (uint32_t)(b < cap ? (b > 0u ? b : 1u) : cap);
}

}  // namespace

hipError_t launch_composite_train(const TrainParams& P, const TrainBuffers& B, hipStream_t st) {
    k_composite_train<<<ray_wave_blocks(P.max_rays), 256, 0, st>>>(P, B.state, B.kept, B.offsets, B.samples, B.field, B.gt, B.draw);
    return hipGetLastError();
}

// The hashed levels' record count per (bin, workgroup) and its exclusive
// scan (the record ranges of the fill pass).
static hipError_t launch_bin_count(const TrainParams& P, const TrainBuffers& B, hipStream_t st) {
    k_bin_pass<false><<<kBinBlocks, kBinThreads, 0, st>>>(P, B.grid, B.state, B.samples, B.sample_ray, B.rays, B.dfeat, B.n_dense, B.n_bins, B.bin_hist, nullptr, nullptr);
    return exclusive_scan_u32(B.bin_hist, B.bin_off, B.n_bins * kBinBlocks, B.bin_scan_tmp, B.bin_total, st);
}

hipError_t launch_mlp_backward(const TrainParams& P, const TrainBuffers& B, hipStream_t st, StepStreams* ss, bool end) {
    const uint32_t cus = device_cu_count();
    if (B.grid.table_dtype != NERF_EXT_F16) return hipErrorInvalidValue;
    static bool lds_set = false;  // once per process: the kernels' dynamic LDS exceeds the 64 KiB default
    if (!lds_set) {
        hipError_t e = hipFuncSetAttribute((const void*)k_bwd_dx, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kDxLds);
        if (e == hipSuccess) e = hipFuncSetAttribute((const void*)k_coarse_scatter, hipFuncAttributeMaxDynamicSharedMemorySize, (int)(kCoarseSlabEntries * 2u * sizeof(uint32_t)));
        const uint32_t slab_lds = kCoarseSlabEntries * 2u * sizeof(uint32_t);
        if (e == hipSuccess) e = hipFuncSetAttribute((const void*)k_scatter_fill<true>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)max(slab_lds, staged_fill_lds(kStagedMaxBins)));
        if (e == hipSuccess) e = hipFuncSetAttribute((const void*)k_scatter_fill<false>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)max(slab_lds, 2u * kMaxBins * (uint32_t)sizeof(uint32_t)));
        if (e != hipSuccess) return e;
        lds_set = true;
    }
    const uint32_t dx_blocks = min(cus * 2u, kDxMaxBlocks);  // two per CU (LDS)
    k_bwd_dx<<<dx_blocks, kThreads, kDxLds, st>>>(P, B.state, B.dparams, B.cparams, B.features, sparse_features(P, B) ? B.features_lm : nullptr, B.draw, B.samples, B.sample_ray, B.rays, B.dfeat, B.dw_partials);
    // Coarse levels: LDS slabs per chunk of samples, summed over the chunks
    // by the gradient reduction; hashed levels: binned.  One launch when both
    // are present.
    const CoarsePlan& C = B.coarse;
    uint32_t lds_entries = 0u;
    for (uint32_t k = 0; k < C.n_slabs; ++k) lds_entries = max(lds_entries, C.count[k]);
    const uint32_t n_coarse = B.n_dense ? kCoarseChunks * C.n_slabs : 0u, slab_lds = lds_entries * 2u * (uint32_t)sizeof(uint32_t);
    if (!B.n_bins && n_coarse)
        k_coarse_scatter<<<n_coarse, kCoarseThreads, slab_lds, st>>>(P, B.grid, C, B.state, B.samples, B.sample_ray, B.rays, B.dfeat, B.coarse_partials);
    if (B.n_bins) {
        // The count started beside the forward pass by the sample stage, or
        // here when no count followed the step's sample stage.
        const uint32_t sl = ss ? ss->slot : 0u;
        hipError_t e      = ss && ss->counted[sl] ? hipStreamWaitEvent(st, ss->done[sl], 0) : launch_bin_count(P, B, st);
        if (e != hipSuccess) return e;
        if (ss) ss->counted[sl] = false;  // consumed
        // Staged for sparse batches (<= 128 steps per ray: records rarely
        // combine and the scattered stores dominate: 4,096 rays of 64 steps
        // 136 -> 98 us); dense batches keep the direct stores, whose records
        // are fewer and whose pass is shorter than the staging rounds (2^18
        // samples of 1,024 steps: 74 us direct, 90 us staged).
        if (P.max_steps <= 128u && B.n_bins <= kStagedMaxBins)
            k_scatter_fill<true><<<n_coarse + kBinBlocks, kBinThreads, max(slab_lds, staged_fill_lds(B.n_bins)), st>>>(P, B.grid, C, B.state, B.samples, B.sample_ray, B.rays, B.dfeat, B.coarse_partials, n_coarse, B.n_dense,
                                                                                                                        B.n_bins, B.bin_off, B.rec, B.bin_max);
        else
            k_scatter_fill<false><<<n_coarse + kBinBlocks, kBinThreads, max(slab_lds, 2u * B.n_bins * (uint32_t)sizeof(uint32_t)), st>>>(P, B.grid, C, B.state, B.samples, B.sample_ray, B.rays, B.dfeat, B.coarse_partials,
                                                                                                                                     n_coarse, B.n_dense, B.n_bins, B.bin_off, B.rec, B.bin_max);
        // The fill is the step's last reader of its sample stream.
        if (ss && ss->record_filled && (e = hipEventRecord(ss->filled, st)) != hipSuccess) return e;
    }
    // Bin accumulation, the coarse levels' chunk sums and the MLP weight
    // gradients' partial sums, in one launch.
    GradReduceArgs a{};
    a.bin_off         = B.bin_off;
    a.n_bins          = B.n_bins;
    a.bin_total       = B.bin_total;
    a.rec             = B.rec;
    a.bin_max         = B.bin_max;
    a.hashed_entries  = (uint64_t)(B.grid.n_levels - B.n_dense) * B.grid.table_size;
    a.hashed_grad     = reinterpret_cast<float2*>(B.table_grad) + (uint64_t)B.n_dense * B.grid.table_size;
    a.coarse_partials = B.coarse_partials;
    a.coarse          = B.coarse;
    a.n_dense         = B.n_dense;
    a.table_size      = B.grid.table_size;
    a.table_grad      = B.table_grad;
    a.dw_partials     = B.dw_partials;
    a.dw_blocks       = dx_blocks;
    a.mlp_grad        = B.mlp_grad;
    a.norm            = B.norm_partials;
    const uint32_t coarse_pairs = B.n_dense ? (coarse_reduce_blocks(B.coarse) + 1u) / 2u : 0u;
    k_grad_reduce<<<B.n_bins + coarse_pairs + kMlpParams / 128u, 512, 0, st>>>(a);
    k_grad_norm<<<1, kNormThreads, 0, st>>>(P, B.norm_partials, norm_partial_count(B), B.state, B.prev, end);
    return hipGetLastError();
}

hipError_t launch_adam(const TrainParams& P, const TrainBuffers& B, hipStream_t st) {
    // One item (four table entries or one MLP weight) per thread: a grid
    // that loops leaves its CUs draining unevenly at the end of the stream.
    const uint32_t cap = 1u << 30;
    // The gradient statistics were taken when the gradients were written.
    if (B.table_elems % 4u) return hipErrorInvalidValue;
    const AdamSeg table{B.table_f32, B.table, B.table_grad, B.table_m, B.table_v};
    const AdamSeg mlp{B.mlp_f32, B.dparams, B.mlp_grad, B.mlp_m, B.mlp_v};
    k_adam<<<grid_for(B.table_elems / 4u + B.mlp_params, cap), 256, 0, st>>>(P, B.state, table, B.table_elems, mlp, B.cparams, B.density_params, B.mlp_params);
    return hipGetLastError();
}

// Stages both models share: the sampler, Adam (over whatever parameters the
// run has) and the end of the step.
static hipError_t launch_train_stage_common(const TrainParams& P, const TrainBuffers& B, uint32_t stage, hipStream_t st, uint32_t fold) {
    switch (stage) {
    case NERF_EXT_STAGE_SAMPLE: {
        k_train_rays<<<ray_wave_blocks(P.max_rays), 256, 0, st>>>(P, B.state, B.prev, (fold & kFoldBegin) != 0u, B.cams, B.images, B.bits, B.rays, B.gt, B.counts, B.seg_t, B.seg_seen, B.seg_reached,
                                                                  B.segs);
        if (B.segs == 1u && P.max_rays <= kPrefixRays) {
            k_train_samples_prefix<<<(P.max_rays + kWaves - 1u) / kWaves, 256, 0, st>>>(P, B.state, B.cams, B.bits, B.rays, B.counts, B.offsets, B.kept, B.seg_t, B.samples, B.sample_ray);
        } else if (B.segs == 1u) {
            k_ray_offsets<<<1, kOffsetThreads, 0, st>>>(P, B.state, B.counts, B.offsets, B.kept);
            k_train_samples_one<<<ray_wave_blocks(P.max_rays), 256, 0, st>>>(P, B.state, B.cams, B.bits, B.rays, B.offsets, B.kept, B.seg_t, B.samples, B.sample_ray);
        } else {
            k_train_samples<<<ray_wave_blocks(P.max_rays * B.segs), 256, 0, st>>>(P, B.state, B.cams, B.bits, B.rays, B.counts, B.offsets, B.seg_t, B.seg_seen, B.seg_reached, B.segs, B.kept, B.samples,
                                                                                  B.sample_ray);
        }
        break;
    }
    case NERF_EXT_STAGE_ADAM: return launch_adam(P, B, st);
    case NERF_EXT_STAGE_END:
        if (!(fold & kFoldEnd)) k_step_end<<<1, 64, 0, st>>>(P, B.state, B.prev);
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Stages of the reference model: the same step with the reference's network
// (packed into MFMA fragments once per step, at its start), its loss and its
// backward; no hash table.
static hipError_t launch_ref_train_stage(const TrainParams& P, const TrainBuffers& B, uint32_t stage, bool occupancy_update, hipStream_t st, uint32_t fold) {
    FieldInputs in{};
    in.samples    = B.samples;
    in.sample_ray = B.sample_ray;
    in.rays       = B.rays;
    in.n_dev      = &B.state->n_samples;
    switch (stage) {
    case NERF_EXT_STAGE_BEGIN:
        k_step_begin<<<1, 64, 0, st>>>(P, B.state, B.prev);
        return ref_pack_weights(B.dparams, B.cparams, B.ref.frags, st);
    case NERF_EXT_STAGE_OCCUPANCY:
        if (occupancy_update) {
            const uint32_t wb = (B.occ_window + 255u) / 256u;
            k_occ_points<<<wb, 256, 0, st>>>(P, B.state, B.occ_window, B.occ_points, B.occ_dirs);
            FieldInputs q{};
            q.positions  = B.occ_points;
            q.directions = B.occ_dirs;
            const hipError_t e = launch_ref_field(B.ref.frags, q, B.occ_window, B.occ_field, nullptr, st);
            if (e != hipSuccess) return e;
            k_occ_apply_field<<<wb, 256, 0, st>>>(P, B.state, B.occ_window, B.occ_field, B.density);
            k_occ_bits<<<(P.occ_cells + 255u) / 256u, 256, 0, st>>>(P, B.state, B.occ_window, B.density, B.bits);
        }
        break;
    case NERF_EXT_STAGE_FORWARD: return launch_ref_field(B.ref.frags, in, P.sample_cap, B.field, nullptr, st);
    case NERF_EXT_STAGE_COMPOSITE: return launch_ref_composite_train(B.ref, B.kept, B.offsets, B.samples, B.field, B.gt, B.draw, &B.state->loss_sum, &B.state->n_rays, &B.state->n_active, st);
    case NERF_EXT_STAGE_BACKWARD: {
        const hipError_t e = launch_ref_backward_train(B.ref, in, B.draw, P.loss_scale, B.mlp_grad, B.norm_partials, st);
        if (e != hipSuccess) return e;
        k_grad_norm<<<1, kNormThreads, 0, st>>>(P, B.norm_partials, norm_partial_count(B), B.state, B.prev, (fold & kFoldEnd) != 0u);
        break;
    }
    default: return launch_train_stage_common(P, B, stage, st, fold & kFoldEnd);
    }
    return hipGetLastError();
}

hipError_t launch_train_stage(const TrainParams& P, const TrainBuffers& B, uint32_t stage, bool occupancy_update, hipStream_t st, StepStreams* ss, uint32_t fold) {
    if (B.model_kind == NERF_EXT_MODEL_REFERENCE) return launch_ref_train_stage(P, B, stage, occupancy_update, st, fold);
    const uint32_t cus = device_cu_count();
    switch (stage) {
    case NERF_EXT_STAGE_BEGIN:
        if (!(fold & kFoldBegin)) k_step_begin<<<1, 64, 0, st>>>(P, B.state, B.prev);
        break;
    case NERF_EXT_STAGE_OCCUPANCY:
        if (occupancy_update) {
            // Refreshes over whole bit words take one launch.
            const uint32_t window = min(P.occ_cells_per_update, P.occ_cells);
            const bool one        = P.occ_cells % 32u == 0u && window % 32u == 0u;
            k_occ_eval<half_t><<<cus * 4u, kThreads, 0, st>>>(P, B.grid, B.table, B.dparams, B.state, B.prev, (fold & kFoldBegin) != 0u, B.density, one ? B.bits : nullptr);
            if (!one) k_occ_bits<<<(P.occ_cells + 255u) / 256u, 256, 0, st>>>(P, B.state, window, B.density, B.bits);
        }
        break;
    case NERF_EXT_STAGE_FORWARD: {
        FieldInputs in{};
        in.samples      = B.samples;
        in.sample_ray   = B.sample_ray;
        in.rays         = B.rays;
        in.n_dev        = &B.state->n_samples;
        in.features_out = B.features;
        for (int a = 0; a < 3; ++a) {
            in.bmin[a] = P.bmin[a];
            in.bmax[a] = P.bmax[a];
        }
        // At up to 128 steps per ray a ray's samples are spread over the
        // whole box (neighbouring samples rarely share a fine-level cell), so
        // the batch takes the level-split encode and a separate MLP pass.
        in.sparse      = sparse_features(P, B);
        in.features_lm = in.sparse ? B.features_lm : nullptr;
        return launch_field(B.grid, B.table, FieldWeights{B.dparams, B.cparams}, in, P.sample_cap, B.field, st);
    }
    case NERF_EXT_STAGE_COMPOSITE: return launch_composite_train(P, B, st);
    case NERF_EXT_STAGE_SAMPLE: {
        hipError_t e = launch_train_stage_common(P, B, stage, st, fold);
        if (e != hipSuccess || !ss || !ss->aux || !B.n_bins) return e;
        // The record count needs only the samples: it runs on the second
        // stream while this one runs the forward pass, the composite and the
        // MLP backward (2^18 samples: 17.5 + 9.5 us off the step's chain).
        const uint32_t sl = ss->slot;
        ss->counted[sl] = false;
        if ((e = hipEventRecord(ss->sampled[sl], st)) != hipSuccess) return e;
        if (st != ss->aux && (e = hipStreamWaitEvent(ss->aux, ss->sampled[sl], 0)) != hipSuccess) return e;
        if ((e = launch_bin_count(P, B, ss->aux)) != hipSuccess) return e;
        if ((e = hipEventRecord(ss->done[sl], ss->aux)) != hipSuccess) return e;
        ss->counted[sl] = true;
        return hipSuccess;
    }
    case NERF_EXT_STAGE_BACKWARD: return launch_mlp_backward(P, B, st, ss, (fold & kFoldEnd) != 0u);
    default: return launch_train_stage_common(P, B, stage, st, fold);
    }
    return hipGetLastError();
}

}  // namespace nerf_hip
