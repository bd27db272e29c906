/*
 * nerf_ext.h — additive C interface of the MI355X NeRF backend.
 *
 * nerf.h (the reference ABI) fixes the model shape at compile time, renders
 * only uploaded cameras and caps training at 256 steps per ray.  The benchmark
 * configurations need more: hash-grid shapes, an analytic scene, novel views,
 * multi-view batches and kernel-level calls on device buffers.  Those live
 * here, in a separate header that never changes nerf.h.  None of these entry
 * points has a counterpart in the reference's nerf.h; each comment names the
 * reference code whose behaviour the kernel behind it follows, or the
 * publication that defines it where the reference has no such stage.
 *
 * Conventions
 *   - Plain pointers and sizes; "device" pointers come from nerf_ext_malloc
 *     (or any HIP allocation on the current device), "host" pointers are
 *     ordinary process memory.
 *   - stream: a hipStream_t passed as void*; NULL is the null stream.
 *     Kernel launches are asynchronous; nothing synchronises unless stated.
 *   - Every function returns a NerfStatus.  On failure nerf_ext_last_error()
 *     returns a message for the calling thread.
 *   - Arithmetic contract: hash indices, occupancy bits and sample counts are
 *     bit-exact with the scalar CPU oracle (oracle/nerf_oracle.cpp); MLP
 *     outputs and RGB agree within 1e-3 relative.
 */
#ifndef NERF_EXT_H
#define NERF_EXT_H

#include "nerf.h"

#ifdef __cplusplus
extern "C" {
#endif

enum { NERF_EXT_F32 = 0, NERF_EXT_F16 = 1 };
enum { NERF_EXT_H2D = 1, NERF_EXT_D2H = 2, NERF_EXT_D2D = 3 };
enum { NERF_EXT_DENSITY_PARAMS = 3072, NERF_EXT_COLOR_PARAMS = 7168 };
/* Parameter counts of the reference's own network (reference-model mode):
 * density 128x64 + 4 x 128x128 + 16x128, colour 128x48 + 2 x 128x128 + 16x128. */
enum { NERF_EXT_REF_DENSITY_PARAMS = 75776, NERF_EXT_REF_COLOR_PARAMS = 40960 };
/* NerfExtModel.kind */
enum { NERF_EXT_MODEL_HASHGRID = 0, NERF_EXT_MODEL_REFERENCE = 1 };
enum { NERF_EXT_MAX_LEVELS = 16 };

/* ---------------------------------------------------------------- runtime */
typedef struct NerfExtDeviceInfo {
    char name[64];
    char arch[32];              /* e.g. "gfx950" */
    uint32_t compute_units;
    uint32_t lds_bytes_per_block;
    uint64_t global_mem_bytes;
    uint32_t clock_khz;
    uint32_t memory_clock_khz;
    uint32_t memory_bus_bits;
    uint32_t l2_bytes;
} NerfExtDeviceInfo;

NERF_API const char* nerf_ext_last_error(void);
NERF_API NerfStatus nerf_ext_device_info(NerfExtDeviceInfo* out);
NERF_API NerfStatus nerf_ext_malloc(void** out_ptr, uint64_t bytes);
NERF_API NerfStatus nerf_ext_free(void* ptr);
NERF_API NerfStatus nerf_ext_memcpy(void* dst, const void* src, uint64_t bytes, uint32_t kind);
NERF_API NerfStatus nerf_ext_memset(void* dst, int value, uint64_t bytes);
NERF_API NerfStatus nerf_ext_synchronize(void);
NERF_API NerfStatus nerf_ext_stream_create(void** out_stream);
NERF_API NerfStatus nerf_ext_stream_destroy(void* stream);
NERF_API NerfStatus nerf_ext_stream_synchronize(void* stream);
NERF_API NerfStatus nerf_ext_event_create(void** out_event);
NERF_API NerfStatus nerf_ext_event_destroy(void* event);
NERF_API NerfStatus nerf_ext_event_record(void* event, void* stream);
NERF_API NerfStatus nerf_ext_event_elapsed_ms(void* start, void* stop, float* out_ms);

/* ------------------------------------------------------ hash-grid encoding */
/* Multiresolution hash encoding of Mueller et al., "Instant Neural Graphics
 * Primitives", SIGGRAPH 2022, section 3 (no counterpart in the reference,
 * whose encoder is the frequency encoding of backend-cuda.cu:252-277).
 * Level l has resolution N_l = floor(N_min * b^l + 1e-9), with
 * b = (finest / N_min)^(1 / (L - 1)) when finest_resolution != 0 and
 * b = per_level_scale otherwise.  A point x in [0,1]^3 (clamped) maps to
 * p = x * N_l; corners floor(p) (clamped to N_l - 1) + {0,1}^3; index
 * cx + cy (N_l+1) + cz (N_l+1)^2 when (N_l+1)^3 <= T, else
 * (cx * 1 ^ cy * 2654435761 ^ cz * 805459861) mod T; trilinear weights. */
typedef struct NerfExtGridDesc {
    uint32_t n_levels;          /* L, at most 16 */
    uint32_t n_features;        /* F, must be 2 */
    uint32_t log2_table_size;   /* log2 T, 2..24 */
    uint32_t base_resolution;   /* N_min >= 1 */
    float per_level_scale;      /* b, used when finest_resolution == 0 */
    uint32_t finest_resolution; /* optional N_max */
    uint32_t table_dtype;       /* NERF_EXT_F32 or NERF_EXT_F16 */
    uint32_t reserved;
} NerfExtGridDesc;

typedef struct NerfExtGridLevels {
    uint32_t n_levels;
    uint32_t table_size;
    uint32_t resolution[NERF_EXT_MAX_LEVELS];
    uint32_t dense[NERF_EXT_MAX_LEVELS];
} NerfExtGridLevels;

NERF_API NerfStatus nerf_ext_grid_levels(const NerfExtGridDesc* grid, NerfExtGridLevels* out);
/* Table of L * T * F elements of grid->table_dtype, layout [level][entry][feature],
 * filled with U(-range, range) from the splitmix64 stream keyed by
 * (0x7ab1e, seed), element order = memory order (bit-exact with the oracle). */
NERF_API NerfStatus nerf_ext_grid_init_table(const NerfExtGridDesc* grid, uint64_t seed, float range, void* table, void* stream);
/* features: [n][L*F] of features_dtype. */
NERF_API NerfStatus nerf_ext_encode_forward(const NerfExtGridDesc* grid, const void* table, const float* positions, uint32_t n, void* features, uint32_t features_dtype, void* stream);
/* Debug view of the gather: indices [n][L][8] and trilinear weights [n][L][8]. */
NERF_API NerfStatus nerf_ext_encode_indices(const NerfExtGridDesc* grid, const float* positions, uint32_t n, uint32_t* indices, float* weights, void* stream);

/* ------------------------------------------------------------------- MLPs */
/* Density network 32 -> 64 -> 16 and colour network [geo 15 | SH4 16 | 0]
 * -> 64 -> 64 -> 16 (3 used), no biases, ReLU, fp16 weights packed [out][in]
 * input layer first (reference semantics backend-cuda.cu:668-835, packing
 * :828-834), fp32 MFMA accumulation.  Weight init: the reference's
 * splitmix64 Xavier (backend-cuda.cu:1810-1847) on the target shapes. */
NERF_API NerfStatus nerf_ext_mlp_init(uint32_t network /* 0 density, 1 colour */, float* params_host);
NERF_API NerfStatus nerf_ext_float_to_half(const float* src, uint16_t* dst, uint64_t n, void* stream);
/* Density MLP on fp16 features [n][32]: raw outputs [n][16] fp32. */
NERF_API NerfStatus nerf_ext_density_mlp(const uint16_t* params, const uint16_t* features, uint32_t n, float* out, void* stream);
/* Fused hash encode + density MLP; out [n][16] = (exp(raw0), raw1..raw15). */
NERF_API NerfStatus nerf_ext_density_forward(const NerfExtGridDesc* grid, const void* table, const uint16_t* params, const float* positions, uint32_t n, float* out, void* stream);

typedef struct NerfExtModel {
    NerfExtGridDesc grid;
    const void* table;              /* device, [L][T][F] */
    const uint16_t* density_params; /* device, 3072 fp16 (reference model: 75776) */
    const uint16_t* color_params;   /* device, 7168 fp16 (reference model: 40960) */
    uint32_t kind;                  /* NERF_EXT_MODEL_HASHGRID (0) or
                                       NERF_EXT_MODEL_REFERENCE: the reference's
                                       own network (grid and table unused; field
                                       positions are world coordinates) */
    uint32_t reserved;
} NerfExtModel;

/* Full field at points with view directions: out [n][4] = (sigma, r, g, b),
 * sigma = exp(density raw 0), rgb = sigmoid(colour raw 0..2); positions in
 * the unit cube of the grid.  A model of kind NERF_EXT_MODEL_REFERENCE runs
 * nerf_ext_ref_field_forward instead (world positions, softplus sigma). */
NERF_API NerfStatus nerf_ext_field_forward(const NerfExtModel* model, const float* positions, const float* directions, uint32_t n, float* out, void* stream);
/* Reference-model mode: the reference's own network (backend-cuda.cu:23-54).
 * Frequency encoding of the world position (10 levels) and of the direction
 * (4 levels) (:252-277); density 64 -> 128 -> 128 x 4 -> 16; colour
 * [raw density 1..15 | direction encoding 27 | 0 x 6] -> 128 -> 128 x 2 -> 16
 * (3 used) (:918-943); fp16 weights packed [out][in], input layer first
 * (:828-834, :1213-1241).  out [n][4] = (softplus(raw density 0), sigmoid of
 * raw colour 0..2) (:909-917); raw (optional) [n][4] = the fp16-rounded raw
 * outputs.  Init: :1810-1847 on these shapes. */
NERF_API NerfStatus nerf_ext_ref_mlp_init(uint32_t network /* 0 density, 1 colour */, float* params_host);
NERF_API NerfStatus nerf_ext_ref_field_forward(const uint16_t* density_params, const uint16_t* color_params, const float* positions, const float* directions, uint32_t n, float* out, float* raw, void* stream);
/* Composite forward + backward with the reference's loss (backend-cuda.cu
 * :1095-1182) for rays whose samples are stored contiguously: ray r owns
 * samples [offsets[r], offsets[r] + counts[r]) of samples [n][2] = (t, dt)
 * and field [n][4] = (sigma = softplus(raw), sigmoid rgb) as
 * nerf_ext_ref_field_forward writes it; gt [n_rays][4] = (r, g, b) composited
 * over white and alpha.  Loss per ray (0.1 + 0.9 clamp(alpha, 0, 1)) |pred -
 * gt|^2, white background, output gradient 2 w (pred - gt) inv_norm.  draw
 * [n][4] = d loss / d (raw sigma, raw r, raw g, raw b); the batch's loss is
 * added to *loss_sum (device). */
/* MLP backward of the reference-model network (forward recomputed): weight
 * gradients ddensity [75776], dcolor [40960] (fp32, device, overwritten) of
 * the loss whose derivatives in the raw outputs are draw [n][4] = (raw sigma,
 * raw r, g, b) (as nerf_ext_ref_composite_backward writes them), multiplied
 * by loss_scale (:1066, :1079; Adam divides it out).  fp16 deltas, fp32
 * accumulation; the colour network's input gradient flows into density
 * outputs 1..15 (:1069-1083).  n <= 2^20 per call. */
NERF_API NerfStatus nerf_ext_ref_backward(const uint16_t* density_params, const uint16_t* color_params, const float* positions, const float* directions, const float* draw, uint32_t n, float loss_scale, float* ddensity, float* dcolor, void* stream);
/* nerf_ext_ref_backward that also leaves the backward's per-layer fp16 rows
 * for inspection, in caller-allocated device buffers: acts [1136][np] (the
 * input of every layer, recomputed), dlts [1056][np] (the delta of every
 * layer's output), np = n rounded up to 64, neuron-major in blocks of 32
 * samples: row r of sample s at element (s / 32 * rows + r) * 32 + s % 32,
 * rows = 1136 or 1056.  Layers 0..9 in the order density 64->128, 128->128
 * x 4, 128->16, colour 48->128, 128->128 x 2, 128->16; layer l's input rows
 * start at acts row {0, 64, 192, 320, 448, 576, 704, 752, 880, 1008}[l]
 * (layer 0: the position encoding 63 + 1 zero; layer 6: [raw density 1..15 |
 * direction encoding 27 | 0 x 6]) and its output delta rows at dlts row
 * {0, 128, 256, 384, 512, 640, 656, 784, 912, 1040}[l] (layer 5: output 0 =
 * fp16(loss_scale d raw sigma), outputs 1..15 = the colour input's geometry
 * deltas; layer 9: fp16(loss_scale d raw r, g, b), then zeros). */
NERF_API NerfStatus nerf_ext_ref_backward_rows(const uint16_t* density_params, const uint16_t* color_params, const float* positions, const float* directions, const float* draw, uint32_t n, float loss_scale, float* ddensity,
                                             float* dcolor, uint16_t* acts, uint16_t* dlts, void* stream);
NERF_API NerfStatus nerf_ext_ref_composite_backward(const uint32_t* counts, const uint32_t* offsets, const float* samples, const float* field, const float* gt, uint32_t n_rays, float inv_norm, float* draw, float* loss_sum, void* stream);
/* The density and colour MLPs of nerf_ext_field_forward on given encodings:
 * features fp16 [n][32], unit directions [n][3] -> out [n][4] = (sigma, r, g, b).
 * The fused fp16-MFMA MLP pass on its own (no table gathers). */
NERF_API NerfStatus nerf_ext_field_mlp(const uint16_t* density_params, const uint16_t* color_params, const uint16_t* features, const float* directions, uint32_t n, float* out, void* stream);

/* ------------------------------------------------------- context options */
/* Options of a nerf.h context (void* from nerf_create_context); nerf.h itself
 * cannot express them.
 *   model_kind: NERF_EXT_MODEL_HASHGRID (the default) or
 *     NERF_EXT_MODEL_REFERENCE, the reference's own network
 *     (backend-cuda.cu:23-54) trained, rendered and checkpointed as the
 *     reference does it.  Changing it replaces the model by a freshly
 *     initialised one (the reference's init, :1810-1847), clears the
 *     occupancy grid and, if training is configured, rebuilds the training
 *     run with the same NerfTrainingConfig (step counter 0).
 *     nerf_load_network_weights also switches it to the model a file holds
 *     ("nerf/network-v1": the reference's; "nerf/hashgrid-network-v1").
 *   inference_sampling: what nerf_inference's samples_per_ray means.
 *     NERF_EXT_SAMPLING_UNIFORM: the reference's sampling (:534-635),
 *     exactly samples_per_ray uniform samples over the box per ray, no
 *     occupancy test, no early stop.  NERF_EXT_SAMPLING_MARCH: the
 *     occupancy-grid march with samples_per_ray as the step budget and early
 *     stop at transmittance 1e-4.  NERF_EXT_SAMPLING_DEFAULT: uniform for the
 *     reference model, march for the hash grid. */
enum { NERF_EXT_SAMPLING_DEFAULT = 0, NERF_EXT_SAMPLING_UNIFORM = 1, NERF_EXT_SAMPLING_MARCH = 2 };
typedef struct NerfExtContextOptions {
    uint32_t model_kind;
    uint32_t inference_sampling;
} NerfExtContextOptions;
NERF_API NerfStatus nerf_ext_context_configure(void* context, const NerfExtContextOptions* options);
NERF_API NerfStatus nerf_ext_context_options(void* context, NerfExtContextOptions* out);

/* ---------------------------------------------------------- analytic scene */
typedef struct NerfExtGaussian {
    float cx, cy, cz;   /* centre */
    float sigma;        /* isotropic standard deviation */
    float amplitude;    /* peak density */
    float r, g, b;      /* albedo */
} NerfExtGaussian;

/* count Gaussians from the splitmix64 stream (0x6a55, seed): per Gaussian
 * centre = lo + (hi - lo) u (3 draws), sigma = s0 + (s1 - s0) u,
 * amplitude = a0 + (a1 - a0) u, albedo u (3 draws); 8 draws per Gaussian. */
typedef struct NerfExtSceneDesc {
    uint32_t count;
    uint32_t reserved;
    uint64_t seed;
    float centre_lo, centre_hi;
    float sigma_lo, sigma_hi;
    float amplitude_lo, amplitude_hi;
} NerfExtSceneDesc;

NERF_API NerfStatus nerf_ext_scene_gaussians(const NerfExtSceneDesc* desc, NerfExtGaussian* out_host);
/* density(p) = sum_g A_g exp(-|p - c_g|^2 / (2 sigma_g^2)), host/device bit-identical. */
NERF_API NerfStatus nerf_ext_scene_density(const NerfExtGaussian* gaussians, uint32_t count, const float* positions, uint32_t n, float* out, void* stream);

/* Occupancy grid (reference bitfield backend-cuda.cu:338-351) over one box
 * or over nested cascades for unbounded scenes.  Cascade 0 is the box
 * [aabb_min, aabb_max]; cascade c > 0 is that box scaled by 2^c about its
 * centre: centre = 0.5 (min + max), half = 0.5 (max - min), bounds
 * centre -/+ half * 2^c (fp32).  A point belongs to the first cascade c whose
 * box holds it (r = (p - lo_c) / (hi_c - lo_c) in [0, 1) on every axis) and
 * to its cell min(res - 1, floor(r * res)) there; points outside every
 * cascade are unoccupied.  Rays are clipped to the outermost box.  Cascade c
 * occupies words [c * W, (c + 1) * W), W = ceil(res^3 / 32), of the
 * bitfield, cell x + y res + z res^2 at bit (index & 31) of word index >> 5. */
typedef struct NerfExtOccupancy {
    uint32_t* bitfield;  /* device, cascades * ceil(res^3 / 32) words */
    uint32_t resolution;
    float aabb_min[3];
    float aabb_max[3];
    uint32_t cascades;   /* 0 or 1: one grid over the box; at most 8 */
} NerfExtOccupancy;

/* Bit set iff density(cell centre) > threshold (reference cell centres
 * backend-cuda.cu:1607-1608, strict threshold :1632), every cascade. */
NERF_API NerfStatus nerf_ext_occupancy_from_scene(const NerfExtGaussian* gaussians, uint32_t count, float threshold, const NerfExtOccupancy* occupancy, void* stream);
/* Uniform-density background shell: sets (ORs) the bit of every cell, in
 * every cascade, whose centre q has r_inner^2 <= |q - centre|^2 <= r_outer^2
 * (fp32, (dx dx + dy dy) + dz dz) — the occupancy of a shell whose density
 * exceeds the threshold. */
NERF_API NerfStatus nerf_ext_occupancy_mark_shell(const NerfExtOccupancy* occupancy, const float* centre3, float r_inner, float r_outer, void* stream);

/* ----------------------------------------------------------- rays and march */
typedef struct NerfExtCamera {
    float c2w[12];          /* rows 0..2 of the row-major camera-to-world 4x4 */
    float fx, fy, cx, cy;
    uint32_t width, height;
} NerfExtCamera;

/* Camera on a sphere of the given radius around centre, looking at it, +y up,
 * direction from the splitmix64 stream (0xca3e, seed), draw index 2*index. */
NERF_API NerfStatus nerf_ext_camera_orbit(uint64_t seed, uint32_t index, float radius, const float* centre3, uint32_t width, uint32_t height, float focal, NerfExtCamera* out);

/* The occupancy cell rule's box-relative coordinates (p - lo) / (hi - lo) of
 * n points (device [n][3] in and out; box_lo, box_hi: host float[3]), as the
 * march kernels compute them: bit-identical to fp32 division (the reference
 * divides inline, backend-cuda.cu:342).  For tests of that computation. */
NERF_API NerfStatus nerf_ext_box_relative(const float* points, uint32_t n, const float* box_lo, const float* box_hi, float* out, void* stream);

/* Per-ray occupied-step counts of the pixel rays of one view (pixel centres,
 * y flipped: backend-cuda.cu:561-563; march :448-469).  counts [W*H]. */
NERF_API NerfStatus nerf_ext_march_count(const NerfExtCamera* camera, const NerfExtOccupancy* occupancy, uint32_t max_steps, uint32_t* counts, void* stream);

/* nerf_ext_march_count for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc); it has no counterpart in the reference.  Same arguments, same
 * counts, bit for bit.  The camera and the per-ray records live in a static
 * per-GPU scratch array of the library (32 MiB + 256 B, held by every GPU the
 * library runs on until the process ends), so width x height is limited to
 * 2^20 rays: larger images return NERF_STATUS_INVALID_USAGE.  Calls that
 * overlap on one GPU (several streams or threads) share the scratch and race;
 * serialise them. */
NERF_API NerfStatus nerf_ext_march_count_noalloc(const NerfExtCamera* camera, const NerfExtOccupancy* occupancy, uint32_t max_steps, uint32_t* counts, void* stream);

/* ------------------------------------------------------------------ render */
typedef struct NerfExtRenderer NerfExtRenderer;

typedef struct NerfExtRenderDesc {
    const NerfExtModel* model;
    const NerfExtOccupancy* occupancy;
    const NerfExtCamera* cameras;   /* host array of view_count cameras */
    uint32_t view_count;
    uint32_t max_steps;             /* march steps per ray */
    float min_transmittance;        /* early stop threshold, e.g. 1e-4 */
    float background[3];            /* composited as C + T * background */
    void* stream;
    uint64_t chunk_samples;         /* Rays are marched, shaded and
                                       composited in chunks of whole blocks of
                                       1024 rays (a block is never split).
                                       0 with max_steps <= 8192: chunks of
                                       at most 2^30 slot entries (rays x
                                       max_steps rounded up to a power of
                                       two), each marched once into per-ray
                                       slots (28 B per entry in the
                                       buffers).  Else: chunks of at most
                                       this many samples (0: 2^29; capped at
                                       2^29) after a count pass over all
                                       rays (32 B per sample) */
    uint32_t* composited;           /* optional device [view][H][W]: samples
                                       composited per ray, i.e. up to and
                                       including the one after which T <
                                       min_transmittance (all of them if T
                                       stays above it) */
    uint32_t* shaded;               /* optional device [view][H][W]: samples
                                       the field evaluated per ray (whole
                                       rounds: >= composited) */
} NerfExtRenderDesc;

typedef struct NerfExtRenderStats {
    uint64_t rays;
    uint64_t samples;          /* occupied samples marched (before early stop) */
    float ms_count;            /* march count pass */
    float ms_scan;             /* exclusive scan of counts */
    float ms_samples;          /* march write pass */
    float ms_field;            /* fused encode + MLP, summed over the rounds */
    float ms_composite;        /* composite rounds and their bookkeeping */
    float ms_total;
    uint64_t samples_shaded;   /* samples evaluated by the field (rays retire early) */
} NerfExtRenderStats;

NERF_API NerfStatus nerf_ext_renderer_create(NerfExtRenderer** out);
NERF_API NerfStatus nerf_ext_renderer_destroy(NerfExtRenderer* renderer);
/* Renders view_count views into rgba8 [view][H][W] (device), max_steps at
 * most 2^19.  Optional device
 * outputs: rgb_f32 [view][H][W][3] (unclamped composite) and counts
 * [view][H][W] (occupied samples per ray).  With stats != NULL the call
 * synchronises and times each stage with HIP events on desc->stream. */
NERF_API NerfStatus nerf_ext_render(NerfExtRenderer* renderer, const NerfExtRenderDesc* desc, uint32_t* rgba8, float* rgb_f32, uint32_t* counts, NerfExtRenderStats* stats);

/* Ground truth of the analytic scene: volume rendering of density(p) with
 * colour(p) = sum_g A_g G_g(p) albedo_g / density(p), uniform steps of
 * (t_far - t_near) / steps over the AABB, white background; RGBA8 with
 * alpha = 1 - T.  rgba8: device [view][H][W]. */
NERF_API NerfStatus nerf_ext_scene_render(const NerfExtGaussian* gaussians, uint32_t count, const NerfExtCamera* cameras, uint32_t view_count, const float* aabb6, uint32_t steps, uint32_t* rgba8, void* stream);

/* The reference's inference sampling (backend-cuda.cu:534-635) for
 * view_count views of one size: per pixel ray (pixel centre, y flipped) clipped
 * to the box aabb6 = (min xyz, max xyz), samples_per_ray (1..2^19) samples at
 * t_near + (i + 0.5) dt, dt = (t_far - t_near) / samples_per_ray, no
 * occupancy test; composite front to back over every sample, then
 * C + T * background3 (NULL: white), clamped to RGBA8 (rgba8 [view][H][W],
 * device) and, optionally, the unclamped RGB (rgb_f32 [view][H][W][3]).
 * Either model kind; hash-grid positions are normalised by the box. */
NERF_API NerfStatus nerf_ext_render_uniform(NerfExtRenderer* renderer, const NerfExtModel* model, const NerfExtCamera* cameras, uint32_t view_count, const float* aabb6, uint32_t samples_per_ray, const float* background3,
                                          uint32_t* rgba8, float* rgb_f32, void* stream);

/* ---------------------------------------------------------------- training */
/* One training step (the reference's nerf_train_step, backend-cuda.cu:2405,
 * with the graph of :2199-2402): pick a camera (hash of the step, :1482),
 * occupancy maintenance on its schedule (:1479-1634), random pixels per ray
 * (:438-441), occupancy march with compaction (:422-533) into a sample stream
 * of fixed capacity, fused field forward, composite forward/backward with a
 * Huber loss on white-composited RGB, MLP backward on MFMA, hash-grid
 * scatter-add, global-norm clip / skip guard / Adam (:1447-1554) on fp32
 * masters with fp16 working copies.  With target_samples != 0 the ray count
 * adapts so that each step marches about target_samples samples. */
typedef struct NerfExtTrainer NerfExtTrainer;

typedef struct NerfExtTrainDesc {
    NerfExtGridDesc grid;            /* table_dtype must be NERF_EXT_F16 */
    const uint8_t* images_rgba8;     /* host, image_count * W * H * 4 */
    const NerfExtCamera* cameras;    /* host, image_count (all of size W x H) */
    uint32_t image_count;
    uint32_t occupancy_res;
    float aabb_min[3];
    float aabb_max[3];
    NerfHyperParams hyper;
    NerfOccupancyParams occupancy;
    uint32_t initial_rays;           /* rays of the first step */
    uint32_t max_rays;               /* ray-buffer capacity */
    uint32_t target_samples;         /* 0: keep the ray count fixed */
    uint32_t sample_capacity;        /* sample-stream capacity */
    uint32_t max_steps_per_ray;      /* march step budget */
    float huber_delta;               /* hash-grid model's Huber loss */
    float table_init_range;          /* hash table init U(-r, r) */
    uint32_t model_kind;             /* NERF_EXT_MODEL_HASHGRID (0), or
                                        NERF_EXT_MODEL_REFERENCE: the reference's
                                        own network (grid unused), trained as the
                                        reference trains it: its loss
                                        (backend-cuda.cu:1095-1182), softplus
                                        occupancy refresh (:1617-1627), Adam over
                                        its 116,736 weights; sample_capacity at
                                        most 2^20 */
    uint64_t seed;                   /* hash table init seed */
} NerfExtTrainDesc;

typedef struct NerfExtTrainStats {
    NerfTrainStats last;             /* last completed step */
    uint32_t rays;                   /* rays marched in the step in progress (some of
                                        its stages enqueued), else in the last step */
    uint32_t samples;                /* samples kept in that step */
    uint32_t active_rays;
    uint32_t skipped;                /* Adam update skipped */
    uint64_t occupied_samples;       /* before the capacity cut */
    uint64_t samples_total;          /* samples trained on since creation or the last reset */
} NerfExtTrainStats;

/* Device buffers of a trainer, for inspection (read-only use by callers). */
typedef struct NerfExtTrainBuffers {
    void* state;                     /* opaque device state */
    float* rays;                     /* [max_rays][2][4]: (o, t_near), (d, t_far) */
    float* gt;                       /* [max_rays][4] */
    uint32_t* counts;                /* [max_rays] occupied samples per ray */
    uint32_t* kept;                  /* [max_rays] samples kept */
    uint32_t* offsets;               /* [max_rays] */
    float* samples;                  /* [cap][2] (t_mid, dt) */
    uint32_t* sample_ray;            /* [cap] */
    float* field;                    /* [cap][4] (sigma, r, g, b) */
    uint16_t* features;              /* [cap][32] fp16 (not written when
                                        features_lm is set) */
    float* draw;                     /* [cap][4] d loss / d raw outputs */
    float* table_grad;               /* [L][T][2] fp32, loss-scaled */
    float* mlp_grad;                 /* [3072 + 7168] fp32, loss-scaled */
    float* table_f32;                /* fp32 master table */
    float* mlp_f32;                  /* fp32 master MLP weights */
    float* table_m;
    float* table_v;
    float* mlp_m;
    float* mlp_v;
    uint32_t* bitfield;
    float* density_grid;
    uint32_t max_rays;
    uint32_t sample_capacity;
    uint64_t table_elems;
    float* dfeat;                    /* [16 levels][cap][2] d loss / d features,
                                        loss-scaled, level-major (hash-grid
                                        model; NULL for the reference model) */
    uint32_t* features_lm;           /* [16 levels][cap] fp16 feature pairs,
                                        level-major: where the step's features
                                        are kept for batches of at most 128
                                        steps per ray; NULL otherwise */
} NerfExtTrainBuffers;

enum {
    NERF_EXT_STAGE_BEGIN = 0,     /* camera, occupancy schedule, counters */
    NERF_EXT_STAGE_OCCUPANCY = 1, /* occupancy maintenance (if scheduled) */
    NERF_EXT_STAGE_SAMPLE = 2,    /* rays, march, scan, sample stream */
    NERF_EXT_STAGE_FORWARD = 3,   /* field forward (+ fp16 features) */
    NERF_EXT_STAGE_COMPOSITE = 4, /* composite fwd/bwd + loss */
    NERF_EXT_STAGE_BACKWARD = 5,  /* MLP backward, hash scatter-add, dW */
    NERF_EXT_STAGE_ADAM = 6,      /* grad stats, Adam, fp16 copies */
    NERF_EXT_STAGE_END = 7        /* stats, sample total, step++ (the ray-count
                                     adaptation runs in the sample stage) */
};

NERF_API NerfStatus nerf_ext_trainer_create(const NerfExtTrainDesc* desc, NerfExtTrainer** out);
NERF_API NerfStatus nerf_ext_trainer_destroy(NerfExtTrainer* trainer);
/* Enqueues `steps` full training steps (asynchronous).  Consecutive steps of
   one call overlap on the trainer's second stream (each step samples beside
   the previous step's gradient sums and Adam); the results are those of the
   steps enqueued one stage at a time, bit for bit. */
NERF_API NerfStatus nerf_ext_trainer_step(NerfExtTrainer* trainer, uint32_t steps);
/* Enqueues stages first..last of the current step (parity tests). */
NERF_API NerfStatus nerf_ext_trainer_run_stages(NerfExtTrainer* trainer, uint32_t first, uint32_t last);
NERF_API NerfStatus nerf_ext_trainer_synchronize(NerfExtTrainer* trainer);
NERF_API NerfStatus nerf_ext_trainer_stats(NerfExtTrainer* trainer, NerfExtTrainStats* out);
NERF_API NerfStatus nerf_ext_trainer_buffers(NerfExtTrainer* trainer, NerfExtTrainBuffers* out);
/* Current fp16 model and occupancy (device pointers owned by the trainer). */
NERF_API NerfStatus nerf_ext_trainer_model(NerfExtTrainer* trainer, NerfExtModel* model, NerfExtOccupancy* occupancy);
/* The trainer's stream (hipStream_t as void*). */
NERF_API void* nerf_ext_trainer_stream(NerfExtTrainer* trainer);

#ifdef __cplusplus
}
#endif

#endif /* NERF_EXT_H */
