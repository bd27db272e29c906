// trainer.hpp — host object of a training run (trainer.hip).
#pragma once

#include <memory>
#include <vector>

#include "train.hpp"

namespace nerf_hip {

// Model buffers lent by the owner of a model (the nerf.h context) instead of
// being allocated by the trainer.
struct BorrowedModel {
    half_t* table;
    float* table_f32;
    half_t* dparams;
    half_t* cparams;
    float* mlp_f32;
    uint32_t* bits;
    float* density;
    const uint8_t* images;  // device RGBA8 dataset, or null: the trainer copies desc->images_rgba8 (host)
};

struct Trainer {
    TrainParams P{};
    TrainBuffers B{};  // the buffers; at(k) gives step k's view (its state slot, the previous one, its bin ranges)
    TrainDevState* slot_state[2]            = {nullptr, nullptr};
    uint32_t* slot_bin_off[2]               = {nullptr, nullptr};
    unsigned long long* slot_bin_total[2]   = {nullptr, nullptr};
    bool open = false;  // stages of step host_frame have been enqueued, its end not yet
    NerfExtGridDesc grid_desc{};
    hipStream_t stream = nullptr;
    bool own_stream    = false;
    StepStreams side;  // the second stream of a step (hash-grid model)
    uint32_t host_frame = 0;  // steps enqueued so far (drives the occupancy schedule)
    float initial_rays  = 1.0f;
    std::vector<void*> owned;

    ~Trainer();
    bool occupancy_due(uint32_t frame) const;
    TrainBuffers at(uint32_t step) const;
    uint32_t fold_for(uint32_t stage, uint32_t first, uint32_t last, bool occupancy_update) const;
    NerfStatus run_stages(uint32_t first, uint32_t last);
    NerfStatus run_steps(uint32_t steps);  // whole steps, consecutive ones overlapped
    TrainDevState* current_state() const;
    // The state of the step in progress, else of the last completed step;
    // last: also the last completed step's.
    NerfStatus read_state(TrainDevState& host, TrainDevState* last = nullptr);
    // Zeroes gradients, Adam moments, the occupancy grid and the step state
    // (frame 0, initial ray count); the weights are left as they are.
    NerfStatus reset();
};

NerfStatus trainer_create(const NerfExtTrainDesc* desc, const BorrowedModel* borrowed, hipStream_t stream, Trainer** out);

}  // namespace nerf_hip
