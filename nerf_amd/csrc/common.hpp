// common.hpp — internal declarations shared by the HIP translation units of
// libnerf.so.  Not a public header: the C interface is include/nerf.h and
// include/nerf_ext.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#ifndef NERF_BUILD_SHARED
#define NERF_BUILD_SHARED 1
#endif
#include "../../include/nerf.h"
#include "../../include/nerf_ext.h"
#include "nerf_math.h"

namespace nerf_hip {

// ------------------------------------------------------------------ errors
void set_error(const std::string& msg);
void clear_error();

// Records a HIP failure as the thread's last error and maps it to the ABI code.
NerfStatus hip_fail(hipError_t e, const char* what);

#define NERF_HIP_TRY(expr)                                       \
    do {                                                         \
        const hipError_t nerf_e_ = (expr);                       \
        if (nerf_e_ != hipSuccess) return ::nerf_hip::hip_fail(nerf_e_, #expr); \
    } while (0)

#define NERF_CHECK_ARG(cond, msg)                        \
    do {                                                 \
        if (!(cond)) {                                   \
            ::nerf_hip::set_error(msg);                  \
            return NERF_STATUS_INVALID_USAGE;            \
        }                                                \
    } while (0)

// Launch error check: kernel launches report configuration errors through
// hipGetLastError().
#define NERF_LAUNCH_CHECK(name) NERF_HIP_TRY(hipGetLastError())

// ------------------------------------------------------------ vector types
typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// fp32 -> fp16, round to nearest even, of an fp32 value that has been rounded
// to fp32 first.  The empty asm makes the value opaque, which stops the
// compiler from fusing a preceding multiply into the conversion
// (v_fma_mixlo_f16 rounds the exact product once, straight to fp16, which can
// differ from rounding to fp32 and then to fp16).
__device__ __forceinline__ half_t to_half_rne(float x) {
    asm volatile("" : "+v"(x));
    return (half_t)x;
}

// ------------------------------------------------------------- hash grid
// Per-level parameters of a hash grid, passed by value to kernels.
struct GridParams {
    uint32_t n_levels;
    uint32_t n_features;
    uint32_t table_size;   // T
    uint32_t table_dtype;  // NERF_EXT_F32 / NERF_EXT_F16
    uint32_t resolution[NERF_EXT_MAX_LEVELS];
    uint32_t dense[NERF_EXT_MAX_LEVELS];
};

// Validates a descriptor and computes its level table (host, fp64).
NerfStatus make_grid(const NerfExtGridDesc* desc, GridParams& out);

// Index and trilinear weight of corner c (bit 0 = x, 1 = y, 2 = z) for one
// level; shared by every kernel that touches the table.  All arithmetic is the
// scalar fp32/u32 sequence of the oracle's encode_point().
struct LevelCell {
    uint32_t i0[3];
    float w[3];
};

__device__ __forceinline__ LevelCell level_cell(const float p[3], uint32_t N) {
    LevelCell c;
    const float s = (float)N;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        const float x   = fminf(fmaxf(p[a], 0.0f), 1.0f);
        const float pos = x * s;
        uint32_t i      = (uint32_t)floorf(pos);
        i               = i >= N ? N - 1u : i;
        c.i0[a]         = i;
        c.w[a]          = pos - (float)i;
    }
    return c;
}

__device__ __forceinline__ uint32_t corner_index(const LevelCell& c, uint32_t corner, uint32_t N, bool dense, uint32_t mask) {
    const uint32_t cx = c.i0[0] + (corner & 1u);
    const uint32_t cy = c.i0[1] + ((corner >> 1) & 1u);
    const uint32_t cz = c.i0[2] + ((corner >> 2) & 1u);
    if (dense) {
        const uint32_t stride = N + 1u;
        return cx + cy * stride + cz * stride * stride;
    }
    return ((cx * nerf_math::kPrime1) ^ (cy * nerf_math::kPrime2) ^ (cz * nerf_math::kPrime3)) & mask;
}

__device__ __forceinline__ float corner_weight(const LevelCell& c, uint32_t corner) {
    const float wx = (corner & 1u) ? c.w[0] : 1.0f - c.w[0];
    const float wy = (corner & 2u) ? c.w[1] : 1.0f - c.w[1];
    const float wz = (corner & 4u) ? c.w[2] : 1.0f - c.w[2];
    return (wx * wy) * wz;
}

// Hash encoding of one level of one point: features (a0, a1) as fp32.
// Corner order, weights and accumulation order are those of the oracle.
template <typename TableT>
__device__ __forceinline__ void encode_level(const GridParams& g, const TableT* __restrict__ table, const float p[3], uint32_t level, uint32_t N, bool dense, float& a0, float& a1) {
    const LevelCell c  = level_cell(p, N);
    const TableT* base = table + (uint64_t)level * g.table_size * 2u;
    uint32_t idx[8];
#pragma unroll
    for (uint32_t k = 0; k < 8u; ++k) idx[k] = corner_index(c, k, N, dense, g.table_size - 1u);
    float v0[8], v1[8];
#pragma unroll
    for (uint32_t k = 0; k < 8u; ++k) {
        v0[k] = (float)base[2u * idx[k]];
        v1[k] = (float)base[2u * idx[k] + 1u];
    }
    a0 = 0.0f;
    a1 = 0.0f;
#pragma unroll
    for (uint32_t k = 0; k < 8u; ++k) {
        const float w = corner_weight(c, k);
        a0            = a0 + w * v0[k];
        a1            = a1 + w * v1[k];
    }
}

// ------------------------------------------------- box-relative coordinates
// (p - lo) / (hi - lo) per axis, bit-identical to the three fp32 divisions:
// the occupancy cell rule's coordinates and the hash grid's unit-cube
// positions of march samples.
// A divisor fixed over many divisions (a box size) lets the division become
// four FMAs and a multiply: r = the refined reciprocal of d (v_rcp_f32, then
// one Newton step r0 + r0 (1 - d r0)), q0 = x r, then two residual
// corrections q <- q + (x - d q) r (Markstein's method).  That is the
// operation sequence hipcc emits for a correctly rounded x / d on gfx950,
// less its operand scaling (v_div_scale) and special-value fix-up
// (v_div_fixup), which change nothing while d and 1 / d are normal, x is
// finite with |x| >= 2^-103, and 2^-126 <= |x / d| < 2^95.  The fast
// quotients are kept when d lies in [2^-20, 2^20] (the reciprocal and its
// refinement are then loop invariants for the cascade-0 box) and every
// computed |q| lies in [2^-80, 2^80]: operands outside those ranges cannot
// give a computed quotient there.  Otherwise (a degenerate box, a point on
// or within 2^-80 box lengths of a face, non-finite input) all three axes
// are divided.  The march's cell test had spent 33 of its 65 instructions
// per step on the divisions.
__device__ __forceinline__ float quotient_by(float x, float d, float r) {
    const float q0 = x * r;
    const float q1 = __builtin_fmaf(__builtin_fmaf(-d, q0, x), r, q0);
    return __builtin_fmaf(__builtin_fmaf(-d, q1, x), r, q1);
}

__device__ __forceinline__ void box_relative(const float p[3], const float lo[3], const float hi[3], float q[3]) {
    float d[3], x[3];
    bool d_ok = true;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        d[a] = hi[a] - lo[a];
        x[a] = p[a] - lo[a];
        d_ok = d_ok && d[a] >= 0x1p-20f && d[a] <= 0x1p20f;
        const float r0 = __builtin_amdgcn_rcpf(d[a]);
        const float r  = __builtin_fmaf(__builtin_fmaf(-d[a], r0, 1.0f), r0, r0);
        q[a]           = quotient_by(x[a], d[a], r);
    }
    const float lo_q = fminf(fminf(fabsf(q[0]), fabsf(q[1])), fabsf(q[2]));
    const float sum  = fabsf(q[0]) + fabsf(q[1]) + fabsf(q[2]);  // NaN if any q is
    if (!(d_ok && lo_q >= 0x1p-80f && sum <= 0x1p80f)) {
#pragma unroll
        for (int a = 0; a < 3; ++a) q[a] = x[a] / d[a];
    }
}

// ------------------------------------------------------------- occupancy
// Occupancy grid over one box or over nested cascades (NerfExtOccupancy in
// include/nerf_ext.h): cascade 0 is [bmin, bmax], cascade c > 0 that box
// scaled by 2^c about its centre; a point belongs to the first cascade whose
// box holds it.  Scalar fp32 throughout, the same operations as the oracle,
// so cells (and with them occupancy bits and sample counts) are bit-exact.
struct OccView {
    const uint32_t* bits;  // cascades * words words, or null: every cell occupied
    uint32_t res;
    uint32_t cascades;     // >= 1
    uint32_t words;        // per cascade: ceil(res^3 / 32)
    float bmin[3], bmax[3];  // cascade 0
    float omin[3], omax[3];  // outermost cascade: the box rays are clipped to
};

constexpr uint32_t kCellOutside = 0xFFFFFFFFu;

__device__ __forceinline__ void occ_box(const OccView& o, uint32_t c, float lo[3], float hi[3]) {
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        if (c == 0u) {
            lo[a] = o.bmin[a];
            hi[a] = o.bmax[a];
        } else {
            const float centre = 0.5f * (o.bmin[a] + o.bmax[a]);
            const float half   = 0.5f * (o.bmax[a] - o.bmin[a]);
            const float s      = (float)(1u << c);
            lo[a]              = centre - half * s;
            hi[a]              = centre + half * s;
        }
    }
}

// Bit index of the cell holding p (cascade c: c * 32 * words + x + y res +
// z res^2; cell rule of backend-cuda.cu:338-351 within the cascade's box),
// or kCellOutside.
__device__ __forceinline__ uint32_t occ_cell(const OccView& o, const float p[3]) {
    for (uint32_t c = 0; c < o.cascades; ++c) {
        float lo[3], hi[3], rel[3];
        occ_box(o, c, lo, hi);
        box_relative(p, lo, hi, rel);
        const float rx = rel[0], ry = rel[1], rz = rel[2];
        if (rx < 0.0f || rx >= 1.0f || ry < 0.0f || ry >= 1.0f || rz < 0.0f || rz >= 1.0f) continue;
        const uint32_t ix = min(o.res - 1u, (uint32_t)(rx * (float)o.res));
        const uint32_t iy = min(o.res - 1u, (uint32_t)(ry * (float)o.res));
        const uint32_t iz = min(o.res - 1u, (uint32_t)(rz * (float)o.res));
        return c * 32u * o.words + ix + iy * o.res + iz * o.res * o.res;
    }
    return kCellOutside;
}

__device__ __forceinline__ bool occ_occupied(const OccView& o, const float p[3]) {
    const uint32_t idx = occ_cell(o, p);
    if (idx == kCellOutside) return false;
    return !o.bits || ((o.bits[idx >> 5] >> (idx & 31u)) & 1u);
}

// Host: view of a NerfExtOccupancy (cascades 0 means 1), with the outermost
// box computed by the same fp32 operations as occ_box; false if the box is
// empty, the cascade count is above 8 or the bit indices overflow 32 bits.
bool make_occ_view(const NerfExtOccupancy& o, OccView& v);

// One level with the x-neighbour corners of each (y, z) edge (corners 2e and
// 2e + 1) fetched by as few loads as the index structure allows:
//   * dense level: the two entries are adjacent (i1 = i0 + 1): one load of
//     two entries at i0 (entry aligned, not necessarily pair aligned; the
//     hardware serves unaligned dword loads);
//   * hashed level: when x is even, i1 = i0 ^ 1 (x's prime is 1): one load
//     of that aligned entry pair; otherwise two single-entry loads (also
//     merging the odd-x cases whose entries happen to be adjacent measured
//     no faster).
// Same entries, weights and summation order as encode_level.
template <typename TableT>
__device__ __forceinline__ void load_entry_pair(const TableT* p, float q[4]) {
    if constexpr (sizeof(TableT) == 4) {
        float4 w;
        __builtin_memcpy(&w, p, 16);
        q[0] = w.x;
        q[1] = w.y;
        q[2] = w.z;
        q[3] = w.w;
    } else {
        half4_t w;
        __builtin_memcpy(&w, p, 8);
#pragma unroll
        for (int k = 0; k < 4; ++k) q[k] = (float)w[k];
    }
}

template <typename TableT, bool kHashPairs = true>
__device__ __forceinline__ void encode_level_xpair(const GridParams& g, const TableT* __restrict__ table, const float p[3], uint32_t level, uint32_t N, bool dense, float& a0, float& a1) {
    const LevelCell c  = level_cell(p, N);
    const TableT* base = table + (uint64_t)level * g.table_size * 2u;
    float v0[8], v1[8];
#pragma unroll
    for (uint32_t e = 0; e < 4u; ++e) {  // (y, z) edge e: corners 2e (x) and 2e + 1 (x + 1)
        const uint32_t i0 = corner_index(c, 2u * e, N, dense, g.table_size - 1u);
        const uint32_t i1 = corner_index(c, 2u * e + 1u, N, dense, g.table_size - 1u);
        float q[4];
        if (dense) {
            load_entry_pair(base + 2u * i0, q);
            v0[2u * e]      = q[0];
            v1[2u * e]      = q[1];
            v0[2u * e + 1u] = q[2];
            v1[2u * e + 1u] = q[3];
        } else if (kHashPairs && i1 == (i0 ^ 1u)) {
            load_entry_pair(base + 2u * (i0 & ~1u), q);
            const bool odd  = (i0 & 1u) != 0u;
            v0[2u * e]      = odd ? q[2] : q[0];
            v1[2u * e]      = odd ? q[3] : q[1];
            v0[2u * e + 1u] = odd ? q[0] : q[2];
            v1[2u * e + 1u] = odd ? q[1] : q[3];
        } else {
            v0[2u * e]      = (float)base[2u * i0];
            v1[2u * e]      = (float)base[2u * i0 + 1u];
            v0[2u * e + 1u] = (float)base[2u * i1];
            v1[2u * e + 1u] = (float)base[2u * i1 + 1u];
        }
    }
    a0 = 0.0f;
    a1 = 0.0f;
#pragma unroll
    for (uint32_t k = 0; k < 8u; ++k) {
        const float w = corner_weight(c, k);
        a0            = a0 + w * v0[k];
        a1            = a1 + w * v1[k];
    }
}

// One level of one point per lane, with the x-neighbour corners of each
// point fetched by a lane pair (lanes 2k and 2k + 1 of a wave, both active,
// same level).  On a hashed level x's prime is 1, so corners x and x + 1 of
// a (y, z) edge have entries i and i ^ (x ^ (x + 1)) = i ^ (2^(t+1) - 1), t
// the trailing ones of x: one 128-byte line holds both unless x ends in five
// or more ones (fp16 entries; four for fp32); on a dense level they are
// adjacent entries.  Load e of a lane reads corner 2e + h
// (h = lane parity) of the even lane's point, load 4 + e the same corner of
// the odd lane's point, so each load instruction asks for one line per
// point where one lane per point asks for two; a quad_perm swap per edge
// then hands each lane the other half of its own point's corners.  Same
// entries, weights and summation order as encode_level.
__device__ __forceinline__ uint32_t pair_swap(uint32_t v) { return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xf, 0xf, false); }  // quad_perm [1, 0, 3, 2]

template <typename TableT>
__device__ __forceinline__ void encode_level_lanepair(const GridParams& g, const TableT* __restrict__ table, const float p[3], uint32_t level, uint32_t N, bool dense, float& a0, float& a1) {
    constexpr uint32_t kWords = sizeof(TableT) == 4 ? 2u : 1u;  // dwords per entry
    const LevelCell c = level_cell(p, N);
    const bool odd    = (threadIdx.x & 1u) != 0u;
    const uint32_t h  = odd ? 1u : 0u;
    LevelCell ce, co;  // cells of the even and the odd lane's point
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        const uint32_t other = pair_swap(c.i0[a]);
        ce.i0[a]             = odd ? other : c.i0[a];
        co.i0[a]             = odd ? c.i0[a] : other;
    }
    const uint32_t mask    = g.table_size - 1u;
    const uint32_t* base   = reinterpret_cast<const uint32_t*>(table + (uint64_t)level * g.table_size * 2u);
    uint32_t ve[4][kWords], vo[4][kWords];
#pragma unroll
    for (uint32_t e = 0; e < 4u; ++e) {
        const uint32_t ie = corner_index(ce, 2u * e + h, N, dense, mask);
#pragma unroll
        for (uint32_t w = 0; w < kWords; ++w) ve[e][w] = base[kWords * ie + w];
    }
#pragma unroll
    for (uint32_t e = 0; e < 4u; ++e) {
        const uint32_t io = corner_index(co, 2u * e + h, N, dense, mask);
#pragma unroll
        for (uint32_t w = 0; w < kWords; ++w) vo[e][w] = base[kWords * io + w];
    }
    float v0[8], v1[8];
#pragma unroll
    for (uint32_t e = 0; e < 4u; ++e) {
        uint32_t lo[kWords], hi[kWords];  // corners 2e and 2e + 1 of this lane's point
#pragma unroll
        for (uint32_t w = 0; w < kWords; ++w) {
            const uint32_t recv = pair_swap(odd ? ve[e][w] : vo[e][w]);
            const uint32_t own  = odd ? vo[e][w] : ve[e][w];
            lo[w]               = odd ? recv : own;
            hi[w]               = odd ? own : recv;
        }
        if constexpr (sizeof(TableT) == 4) {
            v0[2u * e]      = __uint_as_float(lo[0]);
            v1[2u * e]      = __uint_as_float(lo[kWords - 1u]);
            v0[2u * e + 1u] = __uint_as_float(hi[0]);
            v1[2u * e + 1u] = __uint_as_float(hi[kWords - 1u]);
        } else {
            v0[2u * e]      = (float)__builtin_bit_cast(half_t, (uint16_t)(lo[0] & 0xffffu));
            v1[2u * e]      = (float)__builtin_bit_cast(half_t, (uint16_t)(lo[0] >> 16));
            v0[2u * e + 1u] = (float)__builtin_bit_cast(half_t, (uint16_t)(hi[0] & 0xffffu));
            v1[2u * e + 1u] = (float)__builtin_bit_cast(half_t, (uint16_t)(hi[0] >> 16));
        }
    }
    a0 = 0.0f;
    a1 = 0.0f;
#pragma unroll
    for (uint32_t k = 0; k < 8u; ++k) {
        const float w = corner_weight(c, k);
        a0            = a0 + w * v0[k];
        a1            = a1 + w * v1[k];
    }
}

// --------------------------------------------------------------- cameras
struct Ray {
    float o[3];
    float d[3];
    float tn, tf;
};

// Pixel ray of backend-cuda.cu:373-408 with 1/sqrtf in place of rsqrtf; all
// scalar IEEE fp32 (the library is built with -ffp-contract=off).
__device__ __forceinline__ bool make_ray(const NerfExtCamera& c, float px, float py_flipped, const float* bmin, const float* bmax, Ray& r) {
    const float dcx = (px - c.cx) / c.fx;
    const float dcy = (py_flipped - c.cy) / c.fy;
    const float dcz = -1.0f;
    float d[3];
#pragma unroll
    for (int a = 0; a < 3; ++a) d[a] = c.c2w[4 * a + 0] * dcx + c.c2w[4 * a + 1] * dcy + c.c2w[4 * a + 2] * dcz;
    const float len2 = d[0] * d[0] + d[1] * d[1] + d[2] * d[2];
    if (len2 <= 1e-16f) return false;
    const float inv = 1.0f / sqrtf(len2);
    float tmins[3], tmaxs[3];
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        r.d[a]            = d[a] * inv;
        r.o[a]            = c.c2w[4 * a + 3];
        const float inv_d = fabsf(r.d[a]) > 1e-8f ? 1.0f / r.d[a] : (r.d[a] >= 0.0f ? 1e8f : -1e8f);
        const float t0    = (bmin[a] - r.o[a]) * inv_d;
        const float t1    = (bmax[a] - r.o[a]) * inv_d;
        tmins[a]          = fminf(t0, t1);
        tmaxs[a]          = fmaxf(t0, t1);
    }
    float tn       = fmaxf(fmaxf(tmins[0], tmins[1]), tmins[2]);
    const float tf = fminf(fminf(tmaxs[0], tmaxs[1]), tmaxs[2]);
    if (!(tn <= tf && tf > 0.0f)) return false;
    if (tn < 0.0f) tn = 0.0f;
    r.tn = tn;
    r.tf = tf;
    return true;
}

// Inference pixel ray (pixel centre, y flipped: backend-cuda.cu:561-563).
__device__ __forceinline__ bool pixel_ray(const NerfExtCamera& c, uint32_t pix, const float* bmin, const float* bmax, Ray& r) {
    const uint32_t x = pix % c.width;
    const uint32_t y = pix / c.width;
    const float px   = (float)x + 0.5f;
    const float py   = (float)y + 0.5f;
    return make_ray(c, px, (float)c.height - 1.0f - py, bmin, bmax, r);
}

// ------------------------------------------------------------ field eval
// Where the fused field kernel gets its sample positions and directions.
// Opacity of a render sample from the field's density (backend-cuda.cu
// :601-635 with dt clamped at zero); the renderer's rounds take it from the
// field pass.
__device__ __forceinline__ float render_alpha(float sigma, float dt) { return 1.0f - __expf(-(sigma * fmaxf(dt, 0.0f))); }

struct FieldInputs {
    // Mode A: explicit positions [n][3] and directions [n][3].
    const float* positions;
    const float* directions;
    // Mode B: march output — (t_mid, dt) per sample, owning ray per sample and
    // per-ray origin/direction records (float4 o, float4 d).
    const float2* samples;
    const uint32_t* sample_ray;
    const float4* rays;  // [ray][2]: (o.xyz, tn), (d.xyz, tf)
    // Optional: sample count read on the device (clamped to the launch's
    // capacity) and an fp16 copy of the hash features [n][32] for training.
    const uint32_t* n_dev;
    half_t* features_out;
    // Optional (mode B): the j-th sample evaluated is stream sample
    // sample_index[j], and its output goes to out[sample_index[j]].
    const uint32_t* sample_index;
    // Optional with sample_index: the owning ray of the j-th evaluated
    // sample, read in order instead of sample_ray at a scattered stream index.
    const uint32_t* sample_index_ray;
    // With slot_rays the samples sit in per-ray slots of 2^slot_shift: stream
    // sample q belongs to ray slot_ray0 + (q >> slot_shift) (no ray array).
    bool slot_rays;
    uint32_t slot_shift, slot_ray0;
    // With sample_index (the renderer's rounds): output j goes to out[j] in
    // evaluation order as (alpha, r, g, b), alpha = 1 - exp(-sigma max(dt, 0))
    // with the sample's dt, instead of (sigma, r, g, b) at out[sample_index[j]].
    bool alpha_in_order;
    // Mode B positions are world positions inside [bmin, bmax]; the grid
    // encodes the unit cube, so they are mapped by (p - bmin) / (bmax - bmin).
    float bmin[3];
    float bmax[3];
    // Mode B with features_out, fp16 table: the samples are far apart (a few
    // march steps per ray), so caches see no reuse between them and the
    // table is gathered level group by level group, each on its own XCD
    // (whose L2 then holds those levels), followed by the MLPs as a pass over
    // the features.  Same values as the fused kernel.
    bool sparse;
    // With sparse: level-major [16][capacity] fp16 feature pairs, which the
    // level-split encode writes (each XCD whole lines of its levels) instead
    // of features_out, and the MLP pass reads.
    uint32_t* features_lm;
};

// Owning ray of evaluated sample j (stream index qs), per FieldInputs.
__device__ __forceinline__ uint32_t sample_owner(const FieldInputs& in, uint32_t j, uint32_t qs) {
    if (in.slot_rays) return in.slot_ray0 + (qs >> in.slot_shift);
    return in.sample_index && in.sample_index_ray ? in.sample_index_ray[j] : in.sample_ray[qs];
}

struct PointsFromSamples {
    const float2* samples;
    const uint32_t* sample_ray;
    const float4* rays;
    const uint32_t* n_dev;
    uint32_t cap;
    float bmin[3], bmax[3];
    __device__ __forceinline__ uint32_t count() const { return n_dev ? min(*n_dev, cap) : cap; }
    __device__ __forceinline__ void at(uint32_t q, float x[3]) const {
        const float2 td  = samples[q];
        const uint32_t r = sample_ray[q];
        const float4 ro  = rays[2ull * r];
        const float4 rd  = rays[2ull * r + 1ull];
        const float w[3] = {ro.x + td.x * rd.x, ro.y + td.x * rd.y, ro.z + td.x * rd.z};
        box_relative(w, bmin, bmax, x);
    }
};

// Point sources of the XCD-split encode (hashgrid.hip): positions in the
// grid's unit cube from an array, or from a march sample stream (FieldInputs
// mode B, the same operations as the field kernels use).
struct PointsFromArray {
    const float* pos;
    uint32_t n;
    __device__ __forceinline__ uint32_t count() const { return n; }
    __device__ __forceinline__ void at(uint32_t i, float x[3]) const {
        const float3 p = *reinterpret_cast<const float3*>(pos + 3ull * i);
        x[0]           = p.x;
        x[1]           = p.y;
        x[2]           = p.z;
    }
};

struct FieldWeights {
    const half_t* density;  // 3072
    const half_t* color;    // 7168
};

// XCD-split encode of a sample stream's positions into fp16 features [n][32]
// (16-level grids, fp16 table), the sample count read on the device.
// Level-split encode of a march sample stream: features [cap][32] fp16 rows,
// or with lm, level-major fp16 pairs lm[level * cap + sample].
hipError_t launch_encode_samples(const GridParams& g, const half_t* table, const FieldInputs& in, uint32_t cap, half_t* features, uint32_t* lm, hipStream_t stream);
// out4 [n] float4 (sigma, r, g, b).
hipError_t launch_field(const GridParams& g, const void* table, const FieldWeights& w, const FieldInputs& in, uint32_t n, float4* out4, hipStream_t stream);
// Density network only, on points or on fp16 features: out [n][16] = (exp(raw0), raw1..15).
hipError_t launch_density(const GridParams& g, const void* table, const half_t* dparams, const float* positions, const half_t* features, uint32_t n, float* out, hipStream_t stream);

// Reference-model mode (refmodel.hip): the reference's own network.  Its
// weights are packed into kRefFragments MFMA A fragments (64 lanes x 8 halves
// each; the forward's first, then the backward's transposed ones) by
// ref_pack_weights; launch_ref_field evaluates the field from them (world
// positions), out4 = (softplus sigma, sigmoid rgb), raw4 optional.
constexpr uint32_t kRefFragments = 444u;
hipError_t ref_pack_weights(const half_t* dparams, const half_t* cparams, half8_t* frags, hipStream_t stream);
hipError_t launch_ref_field(const half8_t* frags, const FieldInputs& in, uint32_t n, float4* out4, float4* raw4, hipStream_t stream);
// Training of the reference model (the trainer's stages).  Rows of the
// neuron-major fp16 buffers (blocks of 32 samples) the backward writes per sample: every layer's
// input (acts) and output delta (dlts); weight-gradient partials per chunk of
// kRefDwChunk samples; kRefReduceBlocks squared-norm partials.
constexpr uint32_t kRefActRows = 1136u, kRefDltRows = 1056u;
constexpr uint32_t kRefDwChunk = 4096u;
constexpr uint32_t kRefParams = NERF_EXT_REF_DENSITY_PARAMS + NERF_EXT_REF_COLOR_PARAMS;
constexpr uint32_t kRefReduceBlocks = (kRefParams + 255u) / 256u;  // one parameter per thread
constexpr uint32_t kRefMaxSamples = 1u << 20;  // per backward call: the buffers stay below 4 GiB (buffer-descriptor range)
struct RefTrainLaunch {
    half8_t* frags;    // 64 x kRefFragments
    half_t* acts;      // [kRefActRows][np]
    half_t* dlts;      // [kRefDltRows][np]
    float* partial;    // [chunks][kRefParams]
    uint32_t np;       // sample capacity rounded up to 64
    uint32_t chunks;   // ceil(np / kRefDwChunk)
    uint32_t max_rays;
};
// Composite forward/backward with the reference's loss on the trainer's
// stream: counts = kept, ray and active-ray counts on the device.
hipError_t launch_ref_composite_train(const RefTrainLaunch& T, const uint32_t* kept, const uint32_t* offsets, const float2* samples, const float4* field, const float4* gt, float4* draw, float* loss_sum,
                                      const uint32_t* n_rays_dev, const uint32_t* n_active_dev, hipStream_t stream);
// MLP backward (forward recomputed from the sample stream, in.n_dev samples)
// and the weight gradients x loss_scale into grad [kRefParams] (density then
// colour), with kRefReduceBlocks squared-norm partials in norm.
hipError_t launch_ref_backward_train(const RefTrainLaunch& T, const FieldInputs& in, const float4* draw, float loss_scale, float* grad, double* norm, hipStream_t stream);

// Number of compute units of the current device (cached).
uint32_t device_cu_count();

}  // namespace nerf_hip
