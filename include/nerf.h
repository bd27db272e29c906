/*
 * nerf.h — C ABI of the NeRF backend.
 *
 * This header re-declares, type for type and field for field, the public C
 * interface of the reference project (nerf.h:1-129 of Xayah-Graphics/NeRF,
 * MPL-2.0), so that a host program written against that header links against
 * this MI355X/HIP backend without edits.  Names, enum values, struct layouts
 * (LP64) and calling conventions are identical; the layouts are checked by
 * tests/test_abi_layout.py.  Nothing here refers to CUDA: the enum names
 * NERF_STATUS_CUDA_ERROR and NERF_MEMORY_CUDA_DEVICE are kept for source
 * compatibility and mean "GPU runtime error" and "device pointer".
 */
#ifndef NERF_H
#define NERF_H

#include <stdint.h>

#if defined(_WIN32) || defined(__CYGWIN__)
#  if defined(NERF_BUILD_SHARED) && defined(NERF_BUILD_EXPORTS)
#    define NERF_API __declspec(dllexport)
#  elif defined(NERF_BUILD_SHARED)
#    define NERF_API __declspec(dllimport)
#  else
#    define NERF_API
#  endif
#elif defined(__GNUC__) || defined(__clang__)
#  if defined(NERF_BUILD_SHARED)
#    define NERF_API __attribute__((visibility("default")))
#  else
#    define NERF_API
#  endif
#else
#  define NERF_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes returned by every entry point (reference nerf.h:29). */
typedef enum NerfStatus {
    NERF_STATUS_OK            = 0,
    NERF_STATUS_INVALID_USAGE = 1,
    NERF_STATUS_STATE_ERROR   = 2,
    NERF_STATUS_IO_ERROR      = 3,
    NERF_STATUS_CUDA_ERROR    = 4, /* GPU runtime error (HIP on this backend) */
    NERF_STATUS_FAILURE       = 5
} NerfStatus;

/* Context creation (reference nerf.h:31-58).  88 bytes on LP64. */
typedef struct NerfCreateDesc {
    uint32_t occupancy_grid_res;      /* cells per axis of the occupancy grid */
    uint32_t max_sample_steps;        /* capacity of the per-batch sample stream */
    uint32_t max_batch_rays;          /* capacity of the per-batch ray list */
    uint64_t arena_alignment_bytes;   /* power of two */

    const uint8_t* images_rgba8;      /* image_count * width * height * 4 bytes */
    uint64_t images_bytes;

    /* image_count row-major camera-to-world 4x4 matrices:
     *   [ r00 r01 r02 tx ; r10 r11 r12 ty ; r20 r21 r22 tz ; 0 0 0 1 ] */
    const float* cameras_4x4_packed;
    uint64_t cameras_bytes;

    uint32_t image_count;
    uint32_t image_width;
    uint32_t image_height;

    float fx;
    float fy;
    float cx;
    float cy;
} NerfCreateDesc;

NERF_API NerfStatus nerf_create_context(const NerfCreateDesc* desc, void** out_context);
NERF_API NerfStatus nerf_destroy_context(void* context);

/* Optimiser settings (reference nerf.h:60-69).  32 bytes. */
typedef struct NerfHyperParams {
    float learning_rate;
    float adam_beta1;
    float adam_beta2;
    float adam_eps;
    float grad_clip_norm;
    float update_guard_grad_norm;
    float loss_scale;
    uint32_t lr_decay_ksteps;
} NerfHyperParams;

/* Occupancy-grid schedule (reference nerf.h:70-76).  20 bytes. */
typedef struct NerfOccupancyParams {
    float decay;
    float threshold;
    uint32_t cells_per_update;
    uint32_t update_interval;
    uint32_t warmup_steps;
} NerfOccupancyParams;

/* Training configuration (reference nerf.h:77-90).  84 bytes. */
typedef struct NerfTrainingConfig {
    float aabb_min_x;
    float aabb_min_y;
    float aabb_min_z;
    float aabb_max_x;
    float aabb_max_y;
    float aabb_max_z;
    NerfHyperParams hyper_params;
    NerfOccupancyParams occupancy_params;
    uint32_t rays_per_batch;
    uint32_t max_sample_steps_per_ray;
} NerfTrainingConfig;

NERF_API NerfStatus nerf_configure_training(void* context, const NerfTrainingConfig* config);
NERF_API NerfStatus nerf_train_step(void* context);

/* Statistics of the last completed step (reference nerf.h:92-99).  20 bytes. */
typedef struct NerfTrainStats {
    float loss;
    float grad_norm;
    uint32_t has_nonfinite;
    uint32_t completed_steps;
    uint32_t last_train_camera;
} NerfTrainStats;

NERF_API NerfStatus nerf_read_train_stats(void* context, NerfTrainStats* out_stats);

/* Inference (reference nerf.h:101-117). */
typedef enum NerfMemoryKind {
    NERF_MEMORY_HOST        = 1,
    NERF_MEMORY_CUDA_DEVICE = 2 /* device pointer (HIP on this backend) */
} NerfMemoryKind;

typedef struct NerfInferenceRequest {  /* 32 bytes */
    uint32_t camera_idx;
    uint32_t samples_per_ray;
    uint32_t memory_kind;
    void* dst_rgba8;
    uint64_t dst_bytes;
} NerfInferenceRequest;

typedef struct NerfInferenceInfo {     /* 32 bytes */
    uint64_t capacity_bytes;
    uint64_t valid_bytes;
    uint32_t row_stride_bytes;
    uint32_t width;
    uint32_t height;
    uint32_t generation;
} NerfInferenceInfo;

NERF_API NerfStatus nerf_inference(void* context, const NerfInferenceRequest* request, NerfInferenceInfo* out_info);

/* Weight checkpoints (reference nerf.h:119-123). */
typedef struct NerfCheckpointFileDesc {
    const char* path_utf8;
} NerfCheckpointFileDesc;

NERF_API NerfStatus nerf_save_network_weights(void* context, const NerfCheckpointFileDesc* desc);
NERF_API NerfStatus nerf_load_network_weights(void* context, const NerfCheckpointFileDesc* desc);

#ifdef __cplusplus
}
#endif

#endif /* NERF_H */
