// train.hip — training entry points of include/nerf.h on the trainer.
//
// Argument and state validation follow backend-cuda.cu:2125-2140 and
// :2405-2435.  nerf_configure_training builds a trainer that borrows the
// context's model and occupancy buffers, with the configured AABB, Adam
// hyper-parameters, occupancy schedule, a fixed rays_per_batch and
// max_sample_steps_per_ray as the march budget; the sample stream holds
// rays_per_batch * max_sample_steps_per_ray samples, so no ray is ever cut.
// nerf_train_step enqueues one step asynchronously (:2417);
// nerf_read_train_stats synchronises (:2431).  The loss is the Huber loss
// (delta 0.1) for the hash-grid model, and the reference's alpha-weighted
// squared error (:1095-1182) for the reference model.
#include "context.hpp"
#include "trainer.hpp"

namespace nerf_hip {

void Context::train_release() {
    delete train;
    train               = nullptr;
    training_configured = false;
}

// The trainer of a validated NerfTrainingConfig for the context's current
// model, built without touching the context: it borrows the context's model,
// occupancy buffers and device images; rays_per_batch rays per step,
// max_sample_steps_per_ray as the march budget, a stream of rays_per_batch *
// max_sample_steps_per_ray samples (no ray is ever cut).
NerfStatus Context::train_build(const NerfTrainingConfig& c, Trainer** out) {
    *out = nullptr;
    const uint64_t total = (uint64_t)c.rays_per_batch * c.max_sample_steps_per_ray;
    std::vector<NerfExtCamera> cams(image_count);
    for (uint32_t i = 0; i < image_count; ++i) {
        const float* m = cameras.data() + 16ull * i;
        for (int r = 0; r < 3; ++r)
            for (int k = 0; k < 4; ++k) cams[i].c2w[4 * r + k] = m[4 * r + k];
        cams[i].fx     = fx;
        cams[i].fy     = fy;
        cams[i].cx     = cx;
        cams[i].cy     = cy;
        cams[i].width  = width;
        cams[i].height = height;
    }
    NerfExtTrainDesc d{};
    d.grid          = grid;
    d.images_rgba8  = nullptr;  // borrowed on the device below
    d.cameras       = cams.data();
    d.image_count   = image_count;
    d.occupancy_res = occupancy_res;
    d.aabb_min[0]   = c.aabb_min_x;
    d.aabb_min[1]   = c.aabb_min_y;
    d.aabb_min[2]   = c.aabb_min_z;
    d.aabb_max[0]   = c.aabb_max_x;
    d.aabb_max[1]   = c.aabb_max_y;
    d.aabb_max[2]   = c.aabb_max_z;
    d.hyper             = c.hyper_params;
    d.occupancy         = c.occupancy_params;
    d.initial_rays      = c.rays_per_batch;
    d.max_rays          = c.rays_per_batch;
    d.target_samples    = 0u;
    d.sample_capacity   = (uint32_t)total;
    d.max_steps_per_ray = c.max_sample_steps_per_ray;
    d.huber_delta       = 0.1f;
    d.model_kind        = model_kind;
    if (d.hyper.loss_scale <= 0.0f) d.hyper.loss_scale = 1.0f;
    const BorrowedModel bm{(half_t*)table, table_f32, (half_t*)dparams, (half_t*)cparams, mlp_f32, bitfield, density_grid, images};
    const NerfStatus s = trainer_create(&d, &bm, stream, out);
    return s == NERF_STATUS_OK || s == NERF_STATUS_INVALID_USAGE ? s : NERF_STATUS_CUDA_ERROR;
}

// Replaces the training run by one for config c; on failure the previous
// run stays configured.
NerfStatus Context::train_configure_locked(const NerfTrainingConfig& c) {
    Trainer* t         = nullptr;
    const NerfStatus s = train_build(c, &t);
    if (s != NERF_STATUS_OK) return s;
    train_release();
    train               = t;
    train_config        = c;
    host_generation     = 0u;
    training_configured = true;
    return NERF_STATUS_OK;
}

NerfStatus Context::train_reset_state() {
    const uint64_t cells = (uint64_t)occupancy_res * occupancy_res * occupancy_res;
    if (cells) {
        NERF_HIP_TRY(hipMemsetAsync(bitfield, 0, (cells + 31u) / 32u * 4u, stream));
        NERF_HIP_TRY(hipMemsetAsync(density_grid, 0, cells * sizeof(float), stream));
    }
    NERF_HIP_TRY(hipStreamSynchronize(stream));
    // Training stays configured; moments, gradients and the step counter restart.
    return train ? train->reset() : NERF_STATUS_OK;
}

}  // namespace nerf_hip

using namespace nerf_hip;

extern "C" {

// backend-cuda.cu:2125-2140 (validation), :2205-2215 (state reset).
NERF_API NerfStatus nerf_configure_training(void* context, const NerfTrainingConfig* config) {
    if (!context || !config) return NERF_STATUS_INVALID_USAGE;
    Context* ctx = static_cast<Context*>(context);
    if (!ctx->scene_ready) return NERF_STATUS_STATE_ERROR;
    const NerfTrainingConfig c = *config;
    const uint64_t total       = (uint64_t)c.rays_per_batch * c.max_sample_steps_per_ray;
    if (c.rays_per_batch == 0u || c.max_sample_steps_per_ray == 0u || c.max_sample_steps_per_ray > 256u) return NERF_STATUS_INVALID_USAGE;
    if (c.occupancy_params.update_interval == 0u || ctx->image_count == 0u) return NERF_STATUS_INVALID_USAGE;
    if (c.rays_per_batch > ctx->max_batch_rays || total > ctx->max_sample_steps || total > 0xffffffffull) return NERF_STATUS_INVALID_USAGE;
    if (!(c.aabb_max_x > c.aabb_min_x && c.aabb_max_y > c.aabb_min_y && c.aabb_max_z > c.aabb_min_z)) {
        set_error("nerf_configure_training: empty AABB");
        return NERF_STATUS_INVALID_USAGE;
    }
    if (ctx->occupancy_res == 0u) {
        set_error("nerf_configure_training: the context has no occupancy grid (occupancy_grid_res 0)");
        return NERF_STATUS_INVALID_USAGE;
    }
    std::scoped_lock lock(ctx->mutex);
    return ctx->train_configure_locked(c);
}

// backend-cuda.cu:2405-2420.
NERF_API NerfStatus nerf_train_step(void* context) {
    if (!context) return NERF_STATUS_INVALID_USAGE;
    Context* ctx = static_cast<Context*>(context);
    // The trainer is replaced under the mutex (nerf_configure_training), so
    // it is checked under the mutex too.
    std::scoped_lock lock(ctx->mutex);
    if (!ctx->scene_ready || !ctx->training_configured || !ctx->train) return NERF_STATUS_STATE_ERROR;
    const NerfStatus s = ctx->train->run_stages(NERF_EXT_STAGE_BEGIN, NERF_EXT_STAGE_END);
    if (s != NERF_STATUS_OK) return NERF_STATUS_CUDA_ERROR;
    ++ctx->host_generation;
    return NERF_STATUS_OK;
}

// backend-cuda.cu:2421-2435.
NERF_API NerfStatus nerf_read_train_stats(void* context, NerfTrainStats* out_stats) {
    if (!context || !out_stats) return NERF_STATUS_INVALID_USAGE;
    Context* ctx = static_cast<Context*>(context);
    std::scoped_lock lock(ctx->mutex);
    if (!ctx->training_configured || !ctx->train) return NERF_STATUS_STATE_ERROR;
    TrainDevState st{}, last{};
    if (ctx->train->read_state(st, &last) != NERF_STATUS_OK) return NERF_STATUS_CUDA_ERROR;
    *out_stats           = last.stats;
    ctx->host_generation = out_stats->completed_steps;
    return NERF_STATUS_OK;
}

}  // extern "C"
