// context.hpp — the object behind the opaque void* context of include/nerf.h.
#pragma once

#include <mutex>
#include <vector>

#include "common.hpp"

namespace nerf_hip {

struct Trainer;  // training run (trainer.hip)

NerfExtGridDesc abi_grid_desc();

struct Context {
    std::mutex mutex;  // serialises all GPU work of one context (backend-cuda.cu:1407)
    hipStream_t stream = nullptr;

    // dataset (deep copies, backend-cuda.cu:1970-1977)
    uint8_t* images = nullptr;
    std::vector<float> cameras;  // host, 16 floats per image
    uint32_t image_count = 0, width = 0, height = 0;
    float fx = 0, fy = 0, cx = 0, cy = 0;
    uint32_t* rgba = nullptr;  // last inference image
    bool scene_ready = false;

    // occupancy
    uint32_t occupancy_res = 0;
    uint32_t* bitfield     = nullptr;
    float* density_grid    = nullptr;

    // capacities from NerfCreateDesc
    uint32_t max_sample_steps = 0, max_batch_rays = 0;
    uint64_t alignment = 0;

    // model: fp32 masters + fp16 working copies.  NERF_EXT_MODEL_HASHGRID:
    // table + 3,072 + 7,168 weights; NERF_EXT_MODEL_REFERENCE: the reference's
    // own network, 75,776 + 40,960 weights, no table.
    uint32_t model_kind         = NERF_EXT_MODEL_HASHGRID;
    uint32_t inference_sampling = NERF_EXT_SAMPLING_DEFAULT;
    NerfExtGridDesc grid{};
    GridParams grid_params{};
    uint64_t table_elems = 0;
    void* table          = nullptr;  // fp16 [L][T][2]
    float* table_f32     = nullptr;
    uint16_t* dparams    = nullptr;
    uint16_t* cparams    = nullptr;
    float* mlp_f32       = nullptr;  // density then colour fp32 masters

    NerfExtRenderer* renderer = nullptr;

    // training
    bool training_configured = false;
    NerfTrainingConfig train_config{};
    uint32_t host_generation = 0;
    Trainer* train           = nullptr;

    ~Context();
    void release();
    uint32_t density_params() const { return model_kind == NERF_EXT_MODEL_REFERENCE ? (uint32_t)NERF_EXT_REF_DENSITY_PARAMS : (uint32_t)NERF_EXT_DENSITY_PARAMS; }
    uint32_t color_params() const { return model_kind == NERF_EXT_MODEL_REFERENCE ? (uint32_t)NERF_EXT_REF_COLOR_PARAMS : (uint32_t)NERF_EXT_COLOR_PARAMS; }
    // Allocates and initialises a model of model_kind (the reference's init).
    NerfStatus init_model();
    void free_model();
    // Replaces the model by a freshly initialised one of `kind`, clears the
    // occupancy grid and rebuilds a configured training run for it (caller
    // holds the mutex).  Atomic: the new model and trainer are built beside
    // the current ones, and on any failure the context is left as it was.
    NerfStatus switch_model(uint32_t kind);
    NerfStatus upload_weights(const float* mlp32, const float* t32);
    NerfExtModel model() const;
    // The model's buffers, moved out of (take) or into (put) the context.
    struct ModelSlot {
        uint32_t kind;
        NerfExtGridDesc grid;
        GridParams grid_params;
        uint64_t table_elems;
        void* table;
        float* table_f32;
        uint16_t* dparams;
        uint16_t* cparams;
        float* mlp_f32;
    };
    ModelSlot take_model();
    void put_model(const ModelSlot& m);
    static void free_slot(ModelSlot& m);
    // Builds a trainer for config c and the current model without changing
    // the context (caller holds the mutex).
    NerfStatus train_build(const NerfTrainingConfig& c, Trainer** out);
    // Replaces the training run by one for config c; on failure the previous
    // run stays (caller holds the mutex).
    NerfStatus train_configure_locked(const NerfTrainingConfig& c);
    // Zeroes optimiser moments, gradients, occupancy and the step counter.
    NerfStatus train_reset_state();
    void train_release();
};

}  // namespace nerf_hip
