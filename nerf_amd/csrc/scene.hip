// scene.hip — analytic Gaussian scene, its occupancy bitfield, and orbit
// cameras.  The Gaussian density is evaluated with nerf_math::det_expf so that
// the bitfield is bit-identical to a CPU evaluation of the same field.
//
// Occupancy packing follows backend-cuda.cu:347-350 (cell x + y res + z res^2,
// word idx >> 5, bit idx & 31) and the strict threshold of :1632; cell centres
// follow :1607-1608.  The reference builds its bitfield with one atomicOr per
// cell (:1628-1634); here each wavefront ballots its 64 cells and one lane
// stores the two resulting words, so there are no atomics.
#include <math.h>

#include "common.hpp"

namespace nerf_hip {
namespace {

constexpr uint32_t kMaxSceneLds = 1024;  // Gaussians staged in LDS per pass

struct GaussLds {
    float cx, cy, cz, k, a;
};

__device__ __forceinline__ float eval_density(const GaussLds* gs, uint32_t count, const float p[3], float acc) {
    for (uint32_t i = 0; i < count; ++i) {
        const float dx = p[0] - gs[i].cx;
        const float dy = p[1] - gs[i].cy;
        const float dz = p[2] - gs[i].cz;
        const float d2 = (dx * dx + dy * dy) + dz * dz;
        acc            = acc + gs[i].a * nerf_math::det_expf(d2 * gs[i].k);
    }
    return acc;
}

__device__ __forceinline__ void stage_gaussians(GaussLds* lds, const NerfExtGaussian* g, uint32_t begin, uint32_t count) {
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < count; i += blockDim.x) {
        const NerfExtGaussian q = g[begin + i];
        lds[i]                  = GaussLds{q.cx, q.cy, q.cz, -0.5f / (q.sigma * q.sigma), q.amplitude};
    }
    __syncthreads();
}

__global__ __launch_bounds__(256) void k_scene_density(const NerfExtGaussian* __restrict__ gaussians, uint32_t count, const float* __restrict__ pos, uint32_t n, float* __restrict__ out) {
    __shared__ GaussLds lds[kMaxSceneLds];
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    const uint32_t q = i < n ? i : n - 1u;
    const float p[3] = {pos[3ull * q], pos[3ull * q + 1], pos[3ull * q + 2]};
    float acc        = 0.0f;
    for (uint32_t b = 0; b < count; b += kMaxSceneLds) {
        const uint32_t c = count - b < kMaxSceneLds ? count - b : kMaxSceneLds;
        stage_gaussians(lds, gaussians, b, c);
        acc = eval_density(lds, c, p, acc);
    }
    if (i < n) out[i] = acc;
}

// Cell c of cascade blockIdx.y: centre lo + (i + 0.5) * ((hi - lo) / res) per
// axis.
__device__ __forceinline__ void cell_centre(const OccView& o, uint32_t cascade, uint64_t cell, float p[3]) {
    const uint64_t rr  = (uint64_t)o.res * o.res;
    const uint32_t z   = (uint32_t)(cell / rr);
    const uint32_t rem = (uint32_t)(cell - (uint64_t)z * rr);
    const uint32_t y   = rem / o.res;
    const uint32_t x   = rem - y * o.res;
    float lo[3], hi[3];
    occ_box(o, cascade, lo, hi);
    const float sx = (hi[0] - lo[0]) / (float)o.res, sy = (hi[1] - lo[1]) / (float)o.res, sz = (hi[2] - lo[2]) / (float)o.res;
    p[0] = lo[0] + ((float)x + 0.5f) * sx;
    p[1] = lo[1] + ((float)y + 0.5f) * sy;
    p[2] = lo[2] + ((float)z + 0.5f) * sz;
}

// Each wavefront ballots 64 consecutive cells of one cascade into two words
// (kOr: ORed into the existing words, else stored); cascades start at word
// boundaries, so a word never mixes cascades.
template <bool kOr>
__device__ __forceinline__ void store_ballot(const OccView& o, uint32_t* bits, uint32_t cascade, bool occ) {
    const uint64_t ballot    = __ballot(occ);
    const uint32_t lane      = threadIdx.x & 63u;
    const uint64_t wave_base = ((uint64_t)blockIdx.x * 256u + (threadIdx.x & ~63u)) >> 5;  // first word of this wave in the cascade
    uint32_t* w              = bits + (uint64_t)cascade * o.words;
    if (lane == 0u) {
#pragma unroll
        for (uint32_t k = 0; k < 2u; ++k) {
            if (wave_base + k >= o.words) break;
            const uint32_t v = (uint32_t)(ballot >> (32u * k));
            if constexpr (kOr) {
                if (v) w[wave_base + k] |= v;
            } else {
                w[wave_base + k] = v;
            }
        }
    }
}

__global__ __launch_bounds__(256) void k_occupancy_from_scene(const NerfExtGaussian* __restrict__ gaussians, uint32_t count, float threshold, OccView o, uint32_t* __restrict__ bits) {
    __shared__ GaussLds lds[kMaxSceneLds];
    const uint64_t cells = (uint64_t)o.res * o.res * o.res;
    const uint64_t cell  = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    float p[3];
    cell_centre(o, blockIdx.y, cell < cells ? cell : cells - 1u, p);
    float acc = 0.0f;
    for (uint32_t b = 0; b < count; b += kMaxSceneLds) {
        const uint32_t c = count - b < kMaxSceneLds ? count - b : kMaxSceneLds;
        stage_gaussians(lds, gaussians, b, c);
        acc = eval_density(lds, c, p, acc);
    }
    store_ballot<false>(o, bits, blockIdx.y, cell < cells && acc > threshold);
}

__global__ __launch_bounds__(256) void k_occupancy_mark_shell(OccView o, float3 centre, float r2_inner, float r2_outer, uint32_t* __restrict__ bits) {
    const uint64_t cells = (uint64_t)o.res * o.res * o.res;
    const uint64_t cell  = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    float p[3];
    cell_centre(o, blockIdx.y, cell < cells ? cell : cells - 1u, p);
    const float dx = p[0] - centre.x, dy = p[1] - centre.y, dz = p[2] - centre.z;
    const float d2 = (dx * dx + dy * dy) + dz * dz;
    store_ballot<true>(o, bits, blockIdx.y, cell < cells && d2 >= r2_inner && d2 <= r2_outer);
}

struct GaussColorLds {
    float cx, cy, cz, k, a, r, g, b;
};

// Ground-truth volume rendering of the analytic scene: uniform steps, colour
// = density-weighted albedo, white background, alpha = 1 - T; stops once
// T < 1e-4.  Gaussians (<= kMaxSceneLds) staged in LDS.
__global__ __launch_bounds__(256) void k_scene_render(const NerfExtGaussian* __restrict__ gs, uint32_t count, const NerfExtCamera* __restrict__ cams, uint32_t ppv, uint32_t n_rays, float3 bmin3, float3 bmax3, uint32_t steps,
                                                      uint32_t* __restrict__ rgba) {
    __shared__ GaussColorLds lds[kMaxSceneLds];
    for (uint32_t i = threadIdx.x; i < count; i += blockDim.x) {
        const NerfExtGaussian q = gs[i];
        lds[i]                  = GaussColorLds{q.cx, q.cy, q.cz, -0.5f / (q.sigma * q.sigma), q.amplitude, q.r, q.g, q.b};
    }
    __syncthreads();
    const uint32_t ray = blockIdx.x * 256u + threadIdx.x;
    if (ray >= n_rays) return;
    const uint32_t view = ray / ppv;
    const float bmin[3] = {bmin3.x, bmin3.y, bmin3.z}, bmax[3] = {bmax3.x, bmax3.y, bmax3.z};
    Ray r;
    float T = 1.0f, C[3] = {0.0f, 0.0f, 0.0f};
    if (pixel_ray(cams[view], ray - view * ppv, bmin, bmax, r)) {
        const float dt = (r.tf - r.tn) / (float)steps;
        for (uint32_t i = 0; i < steps && dt > 0.0f; ++i) {
            const float t    = r.tn + ((float)i + 0.5f) * dt;
            const float p[3] = {r.o[0] + t * r.d[0], r.o[1] + t * r.d[1], r.o[2] + t * r.d[2]};
            float sig = 0.0f, cr = 0.0f, cg = 0.0f, cb = 0.0f;
            for (uint32_t k = 0; k < count; ++k) {
                const float dx = p[0] - lds[k].cx, dy = p[1] - lds[k].cy, dz = p[2] - lds[k].cz;
                const float v  = lds[k].a * nerf_math::det_expf(((dx * dx + dy * dy) + dz * dz) * lds[k].k);
                sig += v;
                cr += v * lds[k].r;
                cg += v * lds[k].g;
                cb += v * lds[k].b;
            }
            if (sig <= 0.0f) continue;
            const float a = 1.0f - expf(-sig * dt);
            const float w = T * a / sig;
            C[0] += w * cr;
            C[1] += w * cg;
            C[2] += w * cb;
            T *= 1.0f - a;
            if (T < 1e-4f) break;
        }
    }
    uint32_t u[3];
#pragma unroll
    for (int c = 0; c < 3; ++c) u[c] = (uint32_t)rintf(fminf(1.0f, fmaxf(0.0f, C[c] + T)) * 255.0f);
    const uint32_t ua = (uint32_t)rintf(fminf(1.0f, fmaxf(0.0f, 1.0f - T)) * 255.0f);
    rgba[ray]         = (ua << 24) | (u[2] << 16) | (u[1] << 8) | u[0];
}

}  // namespace

bool make_occ_view(const NerfExtOccupancy& o, OccView& v) {
    const uint32_t casc = o.cascades == 0u ? 1u : o.cascades;
    if (casc > 8u || o.resolution == 0u) return false;
    for (int a = 0; a < 3; ++a)
        if (!(o.aabb_max[a] > o.aabb_min[a])) return false;
    const uint64_t cells = (uint64_t)o.resolution * o.resolution * o.resolution;
    const uint64_t words = (cells + 31u) / 32u;
    if ((uint64_t)casc * words * 32u >= 0xFFFFFFFFull) return false;
    v.bits     = o.bitfield;
    v.res      = o.resolution;
    v.cascades = casc;
    v.words    = (uint32_t)words;
    for (int a = 0; a < 3; ++a) {
        v.bmin[a] = o.aabb_min[a];
        v.bmax[a] = o.aabb_max[a];
        // The device's occ_box for the last cascade, on the host (same fp32
        // operations; this file is built with -ffp-contract=off).
        if (casc == 1u) {
            v.omin[a] = v.bmin[a];
            v.omax[a] = v.bmax[a];
        } else {
            const float centre = 0.5f * (v.bmin[a] + v.bmax[a]);
            const float half   = 0.5f * (v.bmax[a] - v.bmin[a]);
            const float s      = (float)(1u << (casc - 1u));
            v.omin[a]          = centre - half * s;
            v.omax[a]          = centre + half * s;
        }
    }
    return true;
}

}  // namespace nerf_hip

using namespace nerf_hip;

extern "C" {

NERF_API NerfStatus nerf_ext_scene_gaussians(const NerfExtSceneDesc* d, NerfExtGaussian* out) {
    NERF_CHECK_ARG(d && out, "nerf_ext_scene_gaussians: null argument");
    const uint64_t s0 = nerf_math::stream_state(0x6a55ull, d->seed);
    for (uint32_t i = 0; i < d->count; ++i) {
        float u[8];
        for (uint32_t k = 0; k < 8u; ++k) u[k] = nerf_math::unit24(nerf_math::splitmix_at(s0, 8ull * i + k));
        NerfExtGaussian& g = out[i];
        g.cx               = d->centre_lo + (d->centre_hi - d->centre_lo) * u[0];
        g.cy               = d->centre_lo + (d->centre_hi - d->centre_lo) * u[1];
        g.cz               = d->centre_lo + (d->centre_hi - d->centre_lo) * u[2];
        g.sigma            = d->sigma_lo + (d->sigma_hi - d->sigma_lo) * u[3];
        g.amplitude        = d->amplitude_lo + (d->amplitude_hi - d->amplitude_lo) * u[4];
        g.r                = u[5];
        g.g                = u[6];
        g.b                = u[7];
    }
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_scene_density(const NerfExtGaussian* gaussians, uint32_t count, const float* positions, uint32_t n, float* out, void* stream) {
    if (n == 0u) return NERF_STATUS_OK;
    NERF_CHECK_ARG(gaussians && positions && out, "nerf_ext_scene_density: null pointer");
    k_scene_density<<<(n + 255u) / 256u, 256, 0, (hipStream_t)stream>>>(gaussians, count, positions, n, out);
    NERF_LAUNCH_CHECK("k_scene_density");
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_occupancy_from_scene(const NerfExtGaussian* gaussians, uint32_t count, float threshold, const NerfExtOccupancy* occ, void* stream) {
    NERF_CHECK_ARG(occ && occ->bitfield && gaussians, "nerf_ext_occupancy_from_scene: null pointer");
    NERF_CHECK_ARG(occ->resolution >= 1u && occ->resolution <= 2048u, "nerf_ext_occupancy_from_scene: resolution must be 1..2048");
    OccView v;
    NERF_CHECK_ARG(make_occ_view(*occ, v), "nerf_ext_occupancy_from_scene: empty box, more than 8 cascades or too many cells");
    const uint64_t cells = (uint64_t)v.res * v.res * v.res;
    const dim3 grid((uint32_t)((cells + 255u) / 256u), v.cascades);
    k_occupancy_from_scene<<<grid, 256, 0, (hipStream_t)stream>>>(gaussians, count, threshold, v, occ->bitfield);
    NERF_LAUNCH_CHECK("k_occupancy_from_scene");
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_occupancy_mark_shell(const NerfExtOccupancy* occ, const float* centre3, float r_inner, float r_outer, void* stream) {
    NERF_CHECK_ARG(occ && occ->bitfield && centre3, "nerf_ext_occupancy_mark_shell: null pointer");
    NERF_CHECK_ARG(occ->resolution >= 1u && occ->resolution <= 2048u, "nerf_ext_occupancy_mark_shell: resolution must be 1..2048");
    NERF_CHECK_ARG(r_inner >= 0.0f && r_outer >= r_inner, "nerf_ext_occupancy_mark_shell: need 0 <= r_inner <= r_outer");
    OccView v;
    NERF_CHECK_ARG(make_occ_view(*occ, v), "nerf_ext_occupancy_mark_shell: empty box, more than 8 cascades or too many cells");
    const uint64_t cells = (uint64_t)v.res * v.res * v.res;
    const dim3 grid((uint32_t)((cells + 255u) / 256u), v.cascades);
    k_occupancy_mark_shell<<<grid, 256, 0, (hipStream_t)stream>>>(v, make_float3(centre3[0], centre3[1], centre3[2]), r_inner * r_inner, r_outer * r_outer, occ->bitfield);
    NERF_LAUNCH_CHECK("k_occupancy_mark_shell");
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_scene_render(const NerfExtGaussian* gaussians, uint32_t count, const NerfExtCamera* cameras, uint32_t view_count, const float* aabb6, uint32_t steps, uint32_t* rgba8, void* stream) {
    NERF_CHECK_ARG(gaussians && cameras && aabb6 && rgba8, "nerf_ext_scene_render: null pointer");
    NERF_CHECK_ARG(count >= 1u && count <= kMaxSceneLds, "nerf_ext_scene_render: 1..1024 Gaussians");
    NERF_CHECK_ARG(view_count >= 1u && steps >= 1u, "nerf_ext_scene_render: need views and steps");
    const uint32_t W = cameras[0].width, H = cameras[0].height;
    for (uint32_t v = 0; v < view_count; ++v) NERF_CHECK_ARG(cameras[v].width == W && cameras[v].height == H && W > 0u && H > 0u, "nerf_ext_scene_render: views must share a size");
    const uint64_t n64 = (uint64_t)W * H * view_count;
    NERF_CHECK_ARG(n64 < (1ull << 31), "nerf_ext_scene_render: too many rays");
    hipStream_t st      = (hipStream_t)stream;
    NerfExtCamera* dcam = nullptr;
    NERF_HIP_TRY(hipMallocAsync((void**)&dcam, sizeof(NerfExtCamera) * view_count, st));
    NERF_HIP_TRY(hipMemcpyAsync(dcam, cameras, sizeof(NerfExtCamera) * view_count, hipMemcpyHostToDevice, st));
    const uint32_t n = (uint32_t)n64;
    k_scene_render<<<(n + 255u) / 256u, 256, 0, st>>>(gaussians, count, dcam, W * H, n, make_float3(aabb6[0], aabb6[1], aabb6[2]), make_float3(aabb6[3], aabb6[4], aabb6[5]), steps, rgba8);
    NERF_LAUNCH_CHECK("k_scene_render");
    NERF_HIP_TRY(hipFreeAsync(dcam, st));
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_camera_orbit(uint64_t seed, uint32_t index, float radius, const float* centre3, uint32_t width, uint32_t height, float focal, NerfExtCamera* out) {
    NERF_CHECK_ARG(centre3 && out, "nerf_ext_camera_orbit: null argument");
    NERF_CHECK_ARG(width > 0u && height > 0u && focal > 0.0f, "nerf_ext_camera_orbit: bad image size or focal");
    const uint64_t s0 = nerf_math::stream_state(0xca3eull, seed);
    const double u    = (double)nerf_math::unit24(nerf_math::splitmix_at(s0, 2ull * index));
    const double v    = (double)nerf_math::unit24(nerf_math::splitmix_at(s0, 2ull * index + 1ull));
    const double cz   = 1.0 - 2.0 * u;  // uniform on the sphere
    const double sz   = sqrt(fmax(0.0, 1.0 - cz * cz));
    const double phi  = 2.0 * 3.14159265358979323846 * v;
    const double back[3] = {sz * cos(phi), cz, sz * sin(phi)};  // camera +z (it looks along -z)
    double upw[3]        = {0.0, 1.0, 0.0};
    if (fabs(back[1]) > 0.999) {
        upw[1] = 0.0;
        upw[2] = 1.0;
    }
    double right[3] = {upw[1] * back[2] - upw[2] * back[1], upw[2] * back[0] - upw[0] * back[2], upw[0] * back[1] - upw[1] * back[0]};
    const double rn = sqrt(right[0] * right[0] + right[1] * right[1] + right[2] * right[2]);
    for (double& c : right) c /= rn;
    const double up[3] = {back[1] * right[2] - back[2] * right[1], back[2] * right[0] - back[0] * right[2], back[0] * right[1] - back[1] * right[0]};
    for (int a = 0; a < 3; ++a) {
        out->c2w[4 * a + 0] = (float)right[a];
        out->c2w[4 * a + 1] = (float)up[a];
        out->c2w[4 * a + 2] = (float)back[a];
        out->c2w[4 * a + 3] = (float)((double)centre3[a] + (double)radius * back[a]);
    }
    out->fx     = focal;
    out->fy     = focal;
    out->cx     = 0.5f * ((float)width - 1.0f);   // benchmark.cpp:213-214 convention
    out->cy     = 0.5f * ((float)height - 1.0f);
    out->width  = width;
    out->height = height;
    return NERF_STATUS_OK;
}

}  // extern "C"
