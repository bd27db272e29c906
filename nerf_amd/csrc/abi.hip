// abi.hip — the reference's C ABI (include/nerf.h) on the MI355X backend.
//
// Behaviour follows backend-cuda.cu:1993-2593: argument and state checks,
// status codes, ownership (create deep-copies images and cameras, destroy is
// null-safe), synchronisation points (inference, stats, save and load
// synchronise; train_step is asynchronous).  Two models can sit behind it
// (nerf_ext_context_configure): the hash-grid NeRF of this backend (the
// default: 16 levels x 2 fp16 features, T = 2^19, N_min 16, b 1.3819, density
// 32->64->16 (exp), colour SH4 -> 64 -> 64 -> 3 (sigmoid)), or the
// reference's own network (frequency encoding, 128-wide MLPs, softplus),
// trained with the reference's loss and saved in its checkpoint format.
// nerf_inference samples as the reference does (spp uniform samples over the
// box, no occupancy, no early stop, :534-635) for the reference model; for
// the hash grid it marches the occupancy bitfield (all cells occupied until
// training has built one) with samples_per_ray as the step budget and stops
// a ray below transmittance 1e-4, unless the context selects uniform
// sampling.  camera_idx is range-checked (the reference reads out of bounds,
// :539).
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
    free_model();
    for (void* p : {(void*)images, (void*)rgba, (void*)bitfield, (void*)density_grid})
        if (p) (void)hipFree(p);
    images = nullptr;
    rgba   = nullptr;
    bitfield = nullptr;
    density_grid = nullptr;
    if (stream) (void)hipStreamDestroy(stream);
    stream = nullptr;
}

// Uploads fp32 master weights (density then colour; the table for the hash
// grid, when given) and refreshes their fp16 working copies.
NerfStatus Context::upload_weights(const float* mlp32, const float* t32) {
    const uint32_t nd = density_params(), nc = color_params();
    NERF_HIP_TRY(hipMemcpyAsync(mlp_f32, mlp32, sizeof(float) * (nd + nc), hipMemcpyHostToDevice, stream));
    if (t32 && table_elems) NERF_HIP_TRY(hipMemcpyAsync(table_f32, t32, sizeof(float) * table_elems, hipMemcpyHostToDevice, stream));
    NERF_HIP_TRY(hipStreamSynchronize(stream));
    NerfStatus s = nerf_ext_float_to_half(mlp_f32, dparams, nd, stream);
    if (s == NERF_STATUS_OK) s = nerf_ext_float_to_half(mlp_f32 + nd, cparams, nc, stream);
    if (s == NERF_STATUS_OK && table_elems) s = nerf_ext_float_to_half(table_f32, (uint16_t*)table, table_elems, stream);
    if (s != NERF_STATUS_OK) return s;
    NERF_HIP_TRY(hipStreamSynchronize(stream));
    return NERF_STATUS_OK;
}

Context::ModelSlot Context::take_model() {
    const ModelSlot m{model_kind, grid, grid_params, table_elems, table, table_f32, dparams, cparams, mlp_f32};
    table     = nullptr;
    table_f32 = nullptr;
    dparams = cparams = nullptr;
    mlp_f32     = nullptr;
    table_elems = 0;
    return m;
}

void Context::put_model(const ModelSlot& m) {
    model_kind  = m.kind;
    grid        = m.grid;
    grid_params = m.grid_params;
    table_elems = m.table_elems;
    table       = m.table;
    table_f32   = m.table_f32;
    dparams     = m.dparams;
    cparams     = m.cparams;
    mlp_f32     = m.mlp_f32;
}

void Context::free_slot(ModelSlot& m) {
    for (void* p : {(void*)m.table, (void*)m.table_f32, (void*)m.dparams, (void*)m.cparams, (void*)m.mlp_f32})
        if (p) (void)hipFree(p);
    m.table = m.table_f32 = nullptr;
    m.dparams = m.cparams = nullptr;
    m.mlp_f32 = nullptr;
}

void Context::free_model() {
    ModelSlot m = take_model();
    free_slot(m);
}

NerfStatus Context::init_model() {
    const bool ref = model_kind == NERF_EXT_MODEL_REFERENCE;
    grid           = abi_grid_desc();
    NerfStatus s   = make_grid(&grid, grid_params);
    if (s != NERF_STATUS_OK) return s;
    const uint32_t nd = density_params(), nc = color_params();
    table_elems       = ref ? 0u : (uint64_t)grid_params.n_levels * grid_params.table_size * grid_params.n_features;
    if (!ref) {
        NERF_HIP_TRY(hipMalloc(&table, table_elems * sizeof(uint16_t)));
        NERF_HIP_TRY(hipMalloc(&table_f32, table_elems * sizeof(float)));
    }
    NERF_HIP_TRY(hipMalloc(&dparams, nd * sizeof(uint16_t)));
    NERF_HIP_TRY(hipMalloc(&cparams, nc * sizeof(uint16_t)));
    NERF_HIP_TRY(hipMalloc(&mlp_f32, (uint64_t)(nd + nc) * sizeof(float)));
    if (!ref) {
        NerfExtGridDesc g32 = grid;
        g32.table_dtype     = NERF_EXT_F32;
        s                   = nerf_ext_grid_init_table(&g32, 0u, 1e-4f, table_f32, stream);
        if (s != NERF_STATUS_OK) return s;
    }
    std::vector<float> w(nd + nc);
    if (ref) {
        nerf_ext_ref_mlp_init(0u, w.data());
        nerf_ext_ref_mlp_init(1u, w.data() + nd);
    } else {
        nerf_ext_mlp_init(0u, w.data());
        nerf_ext_mlp_init(1u, w.data() + nd);
    }
    return upload_weights(w.data(), nullptr);
}

NerfStatus Context::switch_model(uint32_t kind) {
    if (kind == model_kind) return NERF_STATUS_OK;
    if (stream) NERF_HIP_TRY(hipStreamSynchronize(stream));
    // Build the new model (and, when training is configured, its trainer for
    // the same config) beside the current ones; commit only if all of it
    // succeeds.
    ModelSlot old = take_model();
    model_kind    = kind;
    NerfStatus s  = init_model();
    Trainer* nt   = nullptr;
    if (s == NERF_STATUS_OK && training_configured) s = train_build(train_config, &nt);
    if (s != NERF_STATUS_OK) {
        if (stream) (void)hipStreamSynchronize(stream);
        free_model();
        put_model(old);
        return s;
    }
    const bool was_training = training_configured;
    train_release();  // the previous run borrowed the previous model
    train               = nt;
    training_configured = was_training;
    free_slot(old);
    const uint64_t cells = (uint64_t)occupancy_res * occupancy_res * occupancy_res;
    if (cells) {
        NERF_HIP_TRY(hipMemsetAsync(bitfield, 0, (cells + 31u) / 32u * 4u, stream));
        NERF_HIP_TRY(hipMemsetAsync(density_grid, 0, cells * sizeof(float), stream));
        NERF_HIP_TRY(hipStreamSynchronize(stream));
    }
    host_generation = 0u;
    return NERF_STATUS_OK;
}

NerfExtModel Context::model() const {
    NerfExtModel m{};
    m.grid           = grid;
    m.table          = table;
    m.density_params = dparams;
    m.color_params   = cparams;
    m.kind           = model_kind;
    return m;
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
    const NerfExtModel model = ctx->model();
    const bool uniform       = ctx->inference_sampling == NERF_EXT_SAMPLING_UNIFORM || (ctx->inference_sampling == NERF_EXT_SAMPLING_DEFAULT && ctx->model_kind == NERF_EXT_MODEL_REFERENCE);
    if (uniform) {
        // The reference's sampling over the training box, or [0,1]^3 before
        // training is configured (:1884-1889).
        const float box[6] = {occ.aabb_min[0], occ.aabb_min[1], occ.aabb_min[2], occ.aabb_max[0], occ.aabb_max[1], occ.aabb_max[2]};
        const float white[3] = {1.0f, 1.0f, 1.0f};
        if (nerf_ext_render_uniform(ctx->renderer, &model, &cam, 1u, box, request->samples_per_ray, white, ctx->rgba, nullptr, ctx->stream) != NERF_STATUS_OK) return NERF_STATUS_CUDA_ERROR;
    } else {
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
    }
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

// Checkpoint contents of the context's model.  The reference model's tensors
// are the reference's (names :1223-1241, [rows][cols] = [out][in], density
// then colour, input layer first: the packing of the masters here);
// the hash-grid model's follow the same scheme plus "encoding.hash_table".
struct CheckpointLayout {
    std::vector<nerf_ckpt::Tensor> tensors;
    std::vector<std::pair<std::string, std::string>> meta_strings;
    std::vector<std::pair<std::string, uint64_t>> meta_numbers;
};

static const char* kRefFormat      = "nerf/network-v1";
static const char* kHashgridFormat = "nerf/hashgrid-network-v1";

static CheckpointLayout checkpoint_layout(std::vector<float>& w32, std::vector<float>& t32, uint32_t kind, const NerfExtGridDesc& grid) {
    CheckpointLayout c;
    const bool ref    = kind == NERF_EXT_MODEL_REFERENCE;
    const uint32_t nd = ref ? (uint32_t)NERF_EXT_REF_DENSITY_PARAMS : (uint32_t)NERF_EXT_DENSITY_PARAMS;
    const uint32_t nc = ref ? (uint32_t)NERF_EXT_REF_COLOR_PARAMS : (uint32_t)NERF_EXT_COLOR_PARAMS;
    w32.assign(nd + nc, 0.0f);
    float* d32 = w32.data();
    float* c32 = w32.data() + nd;
    if (ref) {
        // density 64 -> 128 -> 128 x 4 -> 16; colour 48 -> 128 -> 128 x 2 -> 16.
        c.tensors.push_back({"density.input.weight", {128, 64}, d32});
        for (uint32_t k = 0; k < 4u; ++k) c.tensors.push_back({"density.hidden." + std::to_string(k) + ".weight", {128, 128}, d32 + 8192 + 16384 * k});
        c.tensors.push_back({"density.output.weight", {16, 128}, d32 + 73728});
        c.tensors.push_back({"color.input.weight", {128, 48}, c32});
        for (uint32_t k = 0; k < 2u; ++k) c.tensors.push_back({"color.hidden." + std::to_string(k) + ".weight", {128, 128}, c32 + 6144 + 16384 * k});
        c.tensors.push_back({"color.output.weight", {16, 128}, c32 + 38912});
        c.meta_strings = {{"format", kRefFormat}};
        c.meta_numbers = {{"density_input_dim", 64}, {"density_hidden_layers", 5}, {"density_width", 128}, {"density_output_dim", 16},
                          {"color_input_dim", 48},   {"color_hidden_layers", 3},   {"color_width", 128},   {"color_output_dim", 16}};
        return c;
    }
    t32.resize((uint64_t)grid.n_levels * (1ull << grid.log2_table_size) * grid.n_features);
    c.tensors = {
        {"density.input.weight", {64, 32}, d32},
        {"density.output.weight", {16, 64}, d32 + 2048},
        {"color.input.weight", {64, 32}, c32},
        {"color.hidden.0.weight", {64, 64}, c32 + 2048},
        {"color.output.weight", {16, 64}, c32 + 2048 + 4096},
        {"encoding.hash_table", {grid.n_levels, 1ull << grid.log2_table_size, grid.n_features}, t32.data()},
    };
    c.meta_strings = {{"format", kHashgridFormat}};
    c.meta_numbers = {{"density_input_dim", 32}, {"density_hidden_layers", 1}, {"density_width", 64}, {"density_output_dim", 16}, {"color_input_dim", 32}, {"color_hidden_layers", 2},
                      {"color_width", 64}, {"color_output_dim", 16}, {"hash_levels", grid.n_levels}, {"hash_features", grid.n_features}, {"hash_log2_table_size", grid.log2_table_size},
                      {"hash_base_resolution", grid.base_resolution}};
    return c;
}

// backend-cuda.cu:2466-2525.
NERF_API NerfStatus nerf_save_network_weights(void* context, const NerfCheckpointFileDesc* desc) {
    if (!context || !desc || !desc->path_utf8) return NERF_STATUS_INVALID_USAGE;
    Context* ctx = static_cast<Context*>(context);
    std::scoped_lock lock(ctx->mutex);
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) return NERF_STATUS_CUDA_ERROR;
    std::vector<float> w32, t32;
    const CheckpointLayout c = checkpoint_layout(w32, t32, ctx->model_kind, ctx->grid);
    if (hipMemcpy(w32.data(), ctx->mlp_f32, w32.size() * 4u, hipMemcpyDeviceToHost) != hipSuccess) return NERF_STATUS_CUDA_ERROR;
    if (!t32.empty() && hipMemcpy(t32.data(), ctx->table_f32, t32.size() * 4u, hipMemcpyDeviceToHost) != hipSuccess) return NERF_STATUS_CUDA_ERROR;
    if (!nerf_ckpt::save(desc->path_utf8, c.tensors, c.meta_strings, c.meta_numbers)) return NERF_STATUS_IO_ERROR;
    return NERF_STATUS_OK;
}

// backend-cuda.cu:2526-2592: load resets optimiser moments, occupancy and the
// step counter.  A file of the other model kind switches the context to it
// (a reference checkpoint, "nerf/network-v1", loads into the reference
// model).
NERF_API NerfStatus nerf_load_network_weights(void* context, const NerfCheckpointFileDesc* desc) {
    if (!context || !desc || !desc->path_utf8) return NERF_STATUS_INVALID_USAGE;
    Context* ctx = static_cast<Context*>(context);
    std::string format, err;
    if (!nerf_ckpt::read_format(desc->path_utf8, format, err)) {
        set_error("nerf_load_network_weights: " + err);
        return NERF_STATUS_IO_ERROR;
    }
    uint32_t kind = 0u;
    if (format == kRefFormat) kind = NERF_EXT_MODEL_REFERENCE;
    else if (format == kHashgridFormat) kind = NERF_EXT_MODEL_HASHGRID;
    else {
        set_error("nerf_load_network_weights: unknown format \"" + format + "\"");
        return NERF_STATUS_IO_ERROR;
    }
    std::scoped_lock lock(ctx->mutex);
    // Read the file against the layout of its model kind before touching the
    // context, so a bad file leaves the context as it was.
    std::vector<float> w32, t32;
    CheckpointLayout c = checkpoint_layout(w32, t32, kind, abi_grid_desc());
    if (!nerf_ckpt::load(desc->path_utf8, c.tensors, err)) {
        set_error("nerf_load_network_weights: " + err);
        return NERF_STATUS_IO_ERROR;
    }
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) return NERF_STATUS_CUDA_ERROR;
    NerfStatus s = ctx->switch_model(kind);
    if (s != NERF_STATUS_OK) return s == NERF_STATUS_INVALID_USAGE ? s : NERF_STATUS_CUDA_ERROR;
    if (ctx->upload_weights(w32.data(), t32.empty() ? nullptr : t32.data()) != NERF_STATUS_OK) return NERF_STATUS_CUDA_ERROR;
    s = ctx->train_reset_state();
    if (s != NERF_STATUS_OK) return s;
    ctx->host_generation = 0u;
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_context_configure(void* context, const NerfExtContextOptions* options) {
    NERF_CHECK_ARG(context && options, "nerf_ext_context_configure: null argument");
    NERF_CHECK_ARG(options->model_kind <= NERF_EXT_MODEL_REFERENCE, "nerf_ext_context_configure: unknown model_kind");
    NERF_CHECK_ARG(options->inference_sampling <= NERF_EXT_SAMPLING_MARCH, "nerf_ext_context_configure: unknown inference_sampling");
    Context* ctx = static_cast<Context*>(context);
    std::scoped_lock lock(ctx->mutex);
    const NerfStatus s = ctx->switch_model(options->model_kind);
    if (s == NERF_STATUS_OK) ctx->inference_sampling = options->inference_sampling;  // a failed switch changes nothing
    return s;
}

NERF_API NerfStatus nerf_ext_context_options(void* context, NerfExtContextOptions* out) {
    NERF_CHECK_ARG(context && out, "nerf_ext_context_options: null argument");
    Context* ctx = static_cast<Context*>(context);
    std::scoped_lock lock(ctx->mutex);
    out->model_kind         = ctx->model_kind;
    out->inference_sampling = ctx->inference_sampling;
    return NERF_STATUS_OK;
}

}  // extern "C"
