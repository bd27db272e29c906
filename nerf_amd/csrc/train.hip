// train.hip — training entry points of include/nerf.h.
//
// Argument and state validation follow backend-cuda.cu:2125-2140 and
// :2405-2435.  The training step itself (march, field forward, composite
// backward with Huber loss, MLP backward on MFMA, hash-grid scatter-add,
// fused Adam, occupancy schedule) is not in this build yet: nerf_train_step
// reports NERF_STATUS_FAILURE with an explanatory last-error message.
#include "common.hpp"
#include "context.hpp"

namespace nerf_hip {

struct TrainState {
    NerfTrainStats stats{};
};

void Context::train_release() {
    delete train;
    train = nullptr;
    training_configured = false;
}

NerfStatus Context::train_reset_state() {
    const uint64_t cells = (uint64_t)occupancy_res * occupancy_res * occupancy_res;
    if (cells) {
        NERF_HIP_TRY(hipMemsetAsync(bitfield, 0, (cells + 31u) / 32u * 4u, stream));
        NERF_HIP_TRY(hipMemsetAsync(density_grid, 0, cells * sizeof(float), stream));
    }
    if (train) train->stats = NerfTrainStats{};
    NERF_HIP_TRY(hipStreamSynchronize(stream));
    return NERF_STATUS_OK;
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
    std::scoped_lock lock(ctx->mutex);
    if (!ctx->train) ctx->train = new TrainState();
    ctx->train_config        = c;
    ctx->host_generation     = 0u;
    const NerfStatus s       = ctx->train_reset_state();
    if (s != NERF_STATUS_OK) return s;
    ctx->training_configured = true;
    return NERF_STATUS_OK;
}

// backend-cuda.cu:2405-2420.
NERF_API NerfStatus nerf_train_step(void* context) {
    if (!context) return NERF_STATUS_INVALID_USAGE;
    Context* ctx = static_cast<Context*>(context);
    if (!ctx->scene_ready || !ctx->training_configured) return NERF_STATUS_STATE_ERROR;
    set_error("nerf_train_step: the training step is not part of this build yet");
    return NERF_STATUS_FAILURE;
}

// backend-cuda.cu:2421-2435.
NERF_API NerfStatus nerf_read_train_stats(void* context, NerfTrainStats* out_stats) {
    if (!context || !out_stats) return NERF_STATUS_INVALID_USAGE;
    Context* ctx = static_cast<Context*>(context);
    if (!ctx->training_configured || !ctx->train) return NERF_STATUS_STATE_ERROR;
    std::scoped_lock lock(ctx->mutex);
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) return NERF_STATUS_CUDA_ERROR;
    *out_stats           = ctx->train->stats;
    ctx->host_generation = out_stats->completed_steps;
    return NERF_STATUS_OK;
}

}  // extern "C"
