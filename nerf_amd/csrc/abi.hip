// abi.hip — the reference's C ABI (include/nerf.h) on the MI355X backend.
//
// Behaviour follows backend-cuda.cu:1993-2593: argument and state checks,
// status codes, ownership (create deep-copies images and cameras, destroy is
// null-safe), synchronisation points (inference, stats, save and load
// synchronise; train_step is asynchronous).  The model behind it is the
// hash-grid NeRF of this backend: 16 levels x 2 fp16 features, T = 2^19,
// N_min 16, b 1.3819, density 32->64->16 (exp), colour SH4 -> 64 -> 64 -> 3
// (sigmoid).  Deliberate differences, each for a reason:
//   * inference marches the occupancy bitfield (all cells occupied until
//     training has built one) with samples_per_ray as the step budget, and
//     stops a ray once its transmittance falls below 1e-4; the reference
//     samples spp uniform steps without occupancy (:534-600);
//   * camera_idx is range-checked (the reference reads out of bounds, :539).
#include <string.h>

#include <memory>
#include <mutex>
#include <vector>

#include "checkpoint.hpp"
#include "common.hpp"
#include "context.hpp"

using namespace nerf_hip;

namespace nerf_hip {

NerfExtGridDesc abi_grid_desc() {
    NerfExtGridDesc g{};
    g.n_levels          = 16u;
    g.n_features        = 2u;
    g.log2_table_size   = 19u;
    g.base_resolution   = 16u;
    g.per_level_scale   = 1.3819f;
    g.finest_resolution = 0u;
    g.table_dtype       = NERF_EXT_F16;
    return g;
}

Context::~Context() { release(); }

void Context::release() {
    if (stream) (void)hipStreamSynchronize(stream);
    if (renderer) (void)nerf_ext_renderer_destroy(renderer);
    renderer = nullptr;
    train_release();
    for (void* p : {(void*)images, (void*)rgba, (void*)bitfield, (void*)density_grid, (void*)table, (void*)table_f32, (void*)dparams, (void*)cparams, (void*)mlp_f32})
        if (p) (void)hipFree(p);
    images = nullptr;
    rgba   = nullptr;
    bitfield = nullptr;
    density_grid = nullptr;
    table = nullptr;
    table_f32 = nullptr;
    dparams = cparams = nullptr;
    mlp_f32 = nullptr;
    if (stream) (void)hipStreamDestroy(stream);
    stream = nullptr;
}

// Uploads fp32 master weights and refreshes their fp16 working copies.
NerfStatus Context::upload_weights(const float* mlp32, const float* t32) {
    NERF_HIP_TRY(hipMemcpyAsync(mlp_f32, mlp32, sizeof(float) * (NERF_EXT_DENSITY_PARAMS + NERF_EXT_COLOR_PARAMS), hipMemcpyHostToDevice, stream));
    if (t32) NERF_HIP_TRY(hipMemcpyAsync(table_f32, t32, sizeof(float) * table_elems, hipMemcpyHostToDevice, stream));
    NERF_HIP_TRY(hipStreamSynchronize(stream));
    NerfStatus s = nerf_ext_float_to_half(mlp_f32, dparams, NERF_EXT_DENSITY_PARAMS, stream);
    if (s == NERF_STATUS_OK) s = nerf_ext_float_to_half(mlp_f32 + NERF_EXT_DENSITY_PARAMS, cparams, NERF_EXT_COLOR_PARAMS, stream);
    if (s == NERF_STATUS_OK) s = nerf_ext_float_to_half(table_f32, (uint16_t*)table, table_elems, stream);
    if (s != NERF_STATUS_OK) return s;
    NERF_HIP_TRY(hipStreamSynchronize(stream));
    return NERF_STATUS_OK;
}

NerfStatus Context::init_model() {
    grid = abi_grid_desc();
    NerfStatus s = make_grid(&grid, grid_params);
    if (s != NERF_STATUS_OK) return s;
    table_elems = (uint64_t)grid_params.n_levels * grid_params.table_size * grid_params.n_features;
    NERF_HIP_TRY(hipMalloc(&table, table_elems * sizeof(uint16_t)));
    NERF_HIP_TRY(hipMalloc(&table_f32, table_elems * sizeof(float)));
    NERF_HIP_TRY(hipMalloc(&dparams, NERF_EXT_DENSITY_PARAMS * sizeof(uint16_t)));
    NERF_HIP_TRY(hipMalloc(&cparams, NERF_EXT_COLOR_PARAMS * sizeof(uint16_t)));
    NERF_HIP_TRY(hipMalloc(&mlp_f32, (NERF_EXT_DENSITY_PARAMS + NERF_EXT_COLOR_PARAMS) * sizeof(float)));
    NerfExtGridDesc g32 = grid;
    g32.table_dtype     = NERF_EXT_F32;
    s                   = nerf_ext_grid_init_table(&g32, 0u, 1e-4f, table_f32, stream);
    if (s != NERF_STATUS_OK) return s;
    std::vector<float> w(NERF_EXT_DENSITY_PARAMS + NERF_EXT_COLOR_PARAMS);
    nerf_ext_mlp_init(0u, w.data());
    nerf_ext_mlp_init(1u, w.data() + NERF_EXT_DENSITY_PARAMS);
    return upload_weights(w.data(), nullptr);
}

}  // namespace nerf_hip

extern "C" {

// backend-cuda.cu:1994-2097.
NERF_API NerfStatus nerf_create_context(const NerfCreateDesc* desc, void** out_context) {
    if (!desc || !out_context) return NERF_STATUS_INVALID_USAGE;
    *out_context          = nullptr;
    const NerfCreateDesc d = *desc;
    if (d.arena_alignment_bytes == 0u || (d.arena_alignment_bytes & (d.arena_alignment_bytes - 1u)) != 0u) {
        set_error("nerf_create_context: arena_alignment_bytes must be a power of two");
        return NERF_STATUS_INVALID_USAGE;
    }
    const uint64_t image_bytes = (uint64_t)d.image_width * d.image_height * 4u * d.image_count;
    if ((d.image_count && (!d.images_rgba8 || d.images_bytes < image_bytes)) || (d.image_count && (!d.cameras_4x4_packed || d.cameras_bytes < 64ull * d.image_count))) {
        set_error("nerf_create_context: dataset buffers smaller than image_count images/cameras");
        return NERF_STATUS_INVALID_USAGE;
    }
    auto ctx = std::make_unique<Context>();
    int dev  = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
        set_error("nerf_create_context: no HIP device");
        return NERF_STATUS_FAILURE;
    }
    ctx->occupancy_res    = d.occupancy_grid_res;
    ctx->max_sample_steps = d.max_sample_steps;
    ctx->max_batch_rays   = d.max_batch_rays;
    ctx->alignment        = d.arena_alignment_bytes;
    ctx->image_count      = d.image_count;
    ctx->width            = d.image_width;
    ctx->height           = d.image_height;
    ctx->fx = d.fx;
    ctx->fy = d.fy;
    ctx->cx = d.cx;
    ctx->cy = d.cy;
    if (d.image_count) ctx->cameras.assign(d.cameras_4x4_packed, d.cameras_4x4_packed + 16ull * d.image_count);
    const uint64_t cells = (uint64_t)d.occupancy_grid_res * d.occupancy_grid_res * d.occupancy_grid_res;
    NerfStatus s         = NERF_STATUS_OK;
    if (cells) {
        if (hipMalloc(&ctx->bitfield, (cells + 31u) / 32u * 4u) != hipSuccess || hipMalloc(&ctx->density_grid, cells * sizeof(float)) != hipSuccess) return NERF_STATUS_CUDA_ERROR;
        if (hipMemset(ctx->bitfield, 0, (cells + 31u) / 32u * 4u) != hipSuccess || hipMemset(ctx->density_grid, 0, cells * sizeof(float)) != hipSuccess) return NERF_STATUS_CUDA_ERROR;
    }
    s = ctx->init_model();
    if (s != NERF_STATUS_OK) return NERF_STATUS_FAILURE;
    if (image_bytes) {
        if (hipMalloc(&ctx->images, image_bytes) != hipSuccess) return NERF_STATUS_CUDA_ERROR;
        if (hipMemcpy(ctx->images, d.images_rgba8, image_bytes, hipMemcpyHostToDevice) != hipSuccess) return NERF_STATUS_CUDA_ERROR;
    }
    const uint64_t frame_bytes = (uint64_t)d.image_width * d.image_height * 4u;
    if (frame_bytes) {
        if (hipMalloc(&ctx->rgba, frame_bytes) != hipSuccess) return NERF_STATUS_CUDA_ERROR;
        if (hipMemset(ctx->rgba, 0, frame_bytes) != hipSuccess) return NERF_STATUS_CUDA_ERROR;
    }
    if (nerf_ext_renderer_create(&ctx->renderer) != NERF_STATUS_OK) return NERF_STATUS_FAILURE;
    ctx->scene_ready = true;
    *out_context     = ctx.release();
    return NERF_STATUS_OK;
}

// backend-cuda.cu:2098-2124.
NERF_API NerfStatus nerf_destroy_context(void* context) {
    if (!context) return NERF_STATUS_OK;
    Context* ctx = static_cast<Context*>(context);
    {
        std::scoped_lock lock(ctx->mutex);
        ctx->release();
    }
    delete ctx;
    return NERF_STATUS_OK;
}

// backend-cuda.cu:2436-2465.
NERF_API NerfStatus nerf_inference(void* context, const NerfInferenceRequest* request, NerfInferenceInfo* out_info) {
    if (!context || !request) return NERF_STATUS_INVALID_USAGE;
    Context* ctx = static_cast<Context*>(context);
    if (!ctx->scene_ready || !ctx->rgba) return NERF_STATUS_STATE_ERROR;
    if (request->samples_per_ray == 0u) return NERF_STATUS_INVALID_USAGE;
    if (request->camera_idx >= ctx->image_count) {
        set_error("nerf_inference: camera_idx out of range");
        return NERF_STATUS_INVALID_USAGE;
    }
    std::scoped_lock lock(ctx->mutex);
    const uint64_t expected = (uint64_t)ctx->width * ctx->height * 4u;
    NerfExtCamera cam{};
    const float* m = ctx->cameras.data() + 16ull * request->camera_idx;
    for (int r = 0; r < 3; ++r)
        for (int c = 0; c < 4; ++c) cam.c2w[4 * r + c] = m[4 * r + c];
    cam.fx     = ctx->fx;
    cam.fy     = ctx->fy;
    cam.cx     = ctx->cx;
    cam.cy     = ctx->cy;
    cam.width  = ctx->width;
    cam.height = ctx->height;
    NerfExtOccupancy occ{};
    occ.resolution = ctx->occupancy_res;
    if (ctx->training_configured) {
        const NerfTrainingConfig& t = ctx->train_config;
        occ.bitfield                = ctx->bitfield;
        const float mn[3] = {t.aabb_min_x, t.aabb_min_y, t.aabb_min_z}, mx[3] = {t.aabb_max_x, t.aabb_max_y, t.aabb_max_z};
        for (int a = 0; a < 3; ++a) {
            occ.aabb_min[a] = mn[a];
            occ.aabb_max[a] = mx[a];
        }
    } else {
        occ.bitfield = nullptr;  // no occupancy yet: every cell of [0,1]^3 (:1884-1889)
        for (int a = 0; a < 3; ++a) {
            occ.aabb_min[a] = 0.0f;
            occ.aabb_max[a] = 1.0f;
        }
    }
    const NerfExtModel model{ctx->grid, ctx->table, ctx->dparams, ctx->cparams};
    NerfExtRenderDesc rd{};
    rd.model             = &model;
    rd.occupancy         = &occ;
    rd.cameras           = &cam;
    rd.view_count        = 1u;
    rd.max_steps         = request->samples_per_ray;
    rd.min_transmittance = 1e-4f;
    rd.background[0] = rd.background[1] = rd.background[2] = 1.0f;
    rd.stream = ctx->stream;
    if (nerf_ext_render(ctx->renderer, &rd, ctx->rgba, nullptr, nullptr, nullptr) != NERF_STATUS_OK) return NERF_STATUS_CUDA_ERROR;
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) return NERF_STATUS_CUDA_ERROR;
    if (request->dst_rgba8) {
        const hipMemcpyKind kind = request->memory_kind == NERF_MEMORY_CUDA_DEVICE ? hipMemcpyDeviceToDevice : hipMemcpyDeviceToHost;
        if (hipMemcpy(request->dst_rgba8, ctx->rgba, expected, kind) != hipSuccess) return NERF_STATUS_CUDA_ERROR;
    }
    if (out_info) {
        out_info->capacity_bytes   = expected;
        out_info->valid_bytes      = expected;
        out_info->row_stride_bytes = ctx->width * 4u;
        out_info->width            = ctx->width;
        out_info->height           = ctx->height;
        out_info->generation       = ctx->host_generation;
    }
    return NERF_STATUS_OK;
}

static std::vector<nerf_ckpt::Tensor> checkpoint_tensors(std::vector<float>& w32, std::vector<float>& t32, const Context& ctx) {
    w32.resize(NERF_EXT_DENSITY_PARAMS + NERF_EXT_COLOR_PARAMS);
    t32.resize(ctx.table_elems);
    float* d32 = w32.data();
    float* c32 = w32.data() + NERF_EXT_DENSITY_PARAMS;
    return {
        {"density.input.weight", {64, 32}, d32},
        {"density.output.weight", {16, 64}, d32 + 2048},
        {"color.input.weight", {64, 32}, c32},
        {"color.hidden.0.weight", {64, 64}, c32 + 2048},
        {"color.output.weight", {16, 64}, c32 + 2048 + 4096},
        {"encoding.hash_table", {ctx.grid.n_levels, 1ull << ctx.grid.log2_table_size, ctx.grid.n_features}, t32.data()},
    };
}

// backend-cuda.cu:2466-2525.
NERF_API NerfStatus nerf_save_network_weights(void* context, const NerfCheckpointFileDesc* desc) {
    if (!context || !desc || !desc->path_utf8) return NERF_STATUS_INVALID_USAGE;
    Context* ctx = static_cast<Context*>(context);
    std::scoped_lock lock(ctx->mutex);
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) return NERF_STATUS_CUDA_ERROR;
    std::vector<float> w32, t32;
    auto tensors = checkpoint_tensors(w32, t32, *ctx);
    if (hipMemcpy(w32.data(), ctx->mlp_f32, w32.size() * 4u, hipMemcpyDeviceToHost) != hipSuccess) return NERF_STATUS_CUDA_ERROR;
    if (hipMemcpy(t32.data(), ctx->table_f32, t32.size() * 4u, hipMemcpyDeviceToHost) != hipSuccess) return NERF_STATUS_CUDA_ERROR;
    const std::vector<std::pair<std::string, std::string>> ms = {{"format", "nerf/hashgrid-network-v1"}};
    const std::vector<std::pair<std::string, uint64_t>> mn    = {{"density_input_dim", 32}, {"density_hidden_layers", 1}, {"density_width", 64}, {"density_output_dim", 16}, {"color_input_dim", 32}, {"color_hidden_layers", 2},
           {"color_width", 64}, {"color_output_dim", 16}, {"hash_levels", ctx->grid.n_levels}, {"hash_features", ctx->grid.n_features}, {"hash_log2_table_size", ctx->grid.log2_table_size}, {"hash_base_resolution", ctx->grid.base_resolution}};
    if (!nerf_ckpt::save(desc->path_utf8, tensors, ms, mn)) return NERF_STATUS_IO_ERROR;
    return NERF_STATUS_OK;
}

// backend-cuda.cu:2526-2592: load resets optimiser moments, occupancy and the
// step counter.
NERF_API NerfStatus nerf_load_network_weights(void* context, const NerfCheckpointFileDesc* desc) {
    if (!context || !desc || !desc->path_utf8) return NERF_STATUS_INVALID_USAGE;
    Context* ctx = static_cast<Context*>(context);
    std::vector<float> w32, t32;
    auto tensors = checkpoint_tensors(w32, t32, *ctx);
    std::string err;
    if (!nerf_ckpt::load(desc->path_utf8, tensors, err)) {
        set_error("nerf_load_network_weights: " + err);
        return NERF_STATUS_IO_ERROR;
    }
    std::scoped_lock lock(ctx->mutex);
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) return NERF_STATUS_CUDA_ERROR;
    if (ctx->upload_weights(w32.data(), t32.data()) != NERF_STATUS_OK) return NERF_STATUS_CUDA_ERROR;
    const NerfStatus s = ctx->train_reset_state();
    if (s != NERF_STATUS_OK) return s;
    ctx->host_generation = 0u;
    return NERF_STATUS_OK;
}

}  // extern "C"
