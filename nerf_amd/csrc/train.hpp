// train.hpp — device-resident training state and the kernels of one step.
#pragma once

#include "common.hpp"

namespace nerf_hip {

enum : uint32_t { kOccNone = 0u, kOccWarmupInit = 1u, kOccRefresh = 2u };

// Per-step scalars kept in device memory, so that every kernel of a step reads
// its counts on the device (fixed launch shapes: the step can be captured in
// a HIP graph).  Mirrors the reference's TrainingDeviceState
// (backend-cuda.cu:79-85) plus the batch counters and Adam scalars.  Steps
// alternate between two of these (step k in slot k % 2): a step's begin
// reads the previous step's slot, so the next step can sample while this
// one still trains.
struct TrainDevState {
    uint32_t frame;       // this step's index (reference frame_index): the previous step's + 1
    uint32_t camera;      // camera of the current step
    uint32_t occ_mode;    // kOcc* of the current step
    uint32_t n_rays;      // rays marched this step
    uint32_t n_samples;   // samples kept this step (a prefix of the stream)
    uint32_t n_active;    // rays with at least one kept sample
    uint32_t nonfinite;   // gradient contains inf/nan
    uint32_t skip;        // Adam update skipped
    unsigned long long total;  // occupied samples before the capacity cut
    unsigned long long samples_done;  // samples trained on since the last reset, this step's included
    double grad_sumsq;    // sum of squared (loss-scaled) gradients
    float loss_sum;       // sum of per-ray Huber losses
    float rays_f;         // this step's adaptive ray count
    float rays_next;      // the next step's, from this step's occupied samples
    NerfTrainStats stats; // this step's, once it has ended
};

// Fixed parameters of a configured run (kernel argument).
struct TrainParams {
    uint32_t image_count, width, height;
    uint32_t occ_res;
    float bmin[3], bmax[3];
    uint32_t max_steps;       // march steps per ray
    uint32_t max_rays;        // capacity of the ray buffers
    uint32_t sample_cap;      // capacity of the sample stream
    uint32_t target_samples;  // adaptive ray count target (0: fixed)
    uint32_t min_rays;
    float huber_delta;
    float loss_scale;
    float lr, beta1, beta2, eps, clip, guard;
    uint32_t lr_decay_ksteps;
    float occ_decay, occ_threshold;
    uint32_t occ_cells_per_update, occ_interval, occ_warmup;
    uint32_t occ_cells;
};

// The coarse dense levels' gradient is summed in LDS: workgroup (chunk c,
// slab k) adds the contributions of sample chunk c to entries [begin, begin +
// count) of one level and writes them to row c of the partials, where the
// levels lie one after another (level l from level_part[l], its entry count
// rounded up to even).  A level of more than kCoarseSlabEntries entries takes
// several slabs.
constexpr uint32_t kCoarseMaxEntries  = 1u << 15;  // largest level on the slab path
constexpr uint32_t kCoarseSlabEntries = 1u << 14;  // entries per slab: 128 KiB of int32 pairs in LDS
constexpr uint32_t kCoarseChunks      = 64u;       // sample chunks, a multiple of 8 (the slabs of a chunk share an XCD)
constexpr uint32_t kCoarseMaxSlabs    = NERF_EXT_MAX_LEVELS * (kCoarseMaxEntries / kCoarseSlabEntries);
struct CoarsePlan {
    uint32_t n_slabs;
    uint32_t row;                                  // entries of a partial row (even)
    uint32_t level[kCoarseMaxSlabs];               // per slab: level
    uint32_t begin[kCoarseMaxSlabs];               // first entry within the level
    uint32_t count[kCoarseMaxSlabs];               // entries (even)
    uint32_t level_part[NERF_EXT_MAX_LEVELS + 1];  // per level: first entry in the partial row
    uint32_t level_entries[NERF_EXT_MAX_LEVELS];   // (N + 1)^3
};

// Device buffers of a run.
struct TrainBuffers {
    TrainDevState* state;        // this step's slot
    TrainDevState* prev;         // the previous step's slot
    const NerfExtCamera* cams;   // [image_count]
    const uint8_t* images;       // [image_count][H][W][4]
    uint32_t* bits;              // occupancy bitfield
    float* density;              // occupancy density grid
    float4* rays;                // [max_rays][2]
    float4* gt;                  // [max_rays] (r, g, b, a)
    uint32_t* counts;            // [max_rays] occupied samples
    uint32_t* kept;              // [max_rays] samples kept (0 if cut)
    uint32_t* offsets;           // [max_rays]
    float* seg_t;                // [max_rays][segs] t at the start of each kSegSteps-step segment of the march
    uint32_t* seg_seen;          // [max_rays][segs] occupied steps before the segment
    uint32_t* seg_reached;       // [max_rays] segments the march started
    uint32_t segs;               // ceil(max_steps / kSegSteps)
    float2* samples;             // [sample_cap] (t_mid, dt)
    uint32_t* sample_ray;        // [sample_cap]
    float4* field;               // [sample_cap] (sigma, r, g, b)
    half_t* features;            // [sample_cap][32]
    uint32_t* features_lm;         // [16][sample_cap] fp16 feature pairs, level-major (sparse batches' encode)
    float4* draw;                // [sample_cap] (d sigma_raw, d r, d g, d b)
    float2* dfeat;               // [16 levels][sample_cap] d(features), loss-scaled
    // binned hash-grid scatter: records (entry within bin, 2 values) grouped
    // by bin of kBinEntries table entries
    uint32_t* bin_hist;          // [n_bins][kBinBlocks] record counts
    uint32_t* bin_off;           // [n_bins][kBinBlocks] exclusive scan of bin_hist (one per slot)
    uint32_t* bin_max;           // [n_bins][kBinBlocks] bits of the largest |record value|
    uint32_t* bin_scan_tmp;
    unsigned long long* bin_total;  // one per slot
    uint2* rec;                  // [rec_cap] packed (entry within bin, 2 values)
    uint32_t n_bins;             // bins of the levels past the coarse ones
    uint32_t n_dense;            // leading (coarse) levels accumulated in LDS slabs (dense, <= kCoarseMaxEntries entries)
    uint64_t rec_cap;
    CoarsePlan coarse;           // slabs of the coarse levels
    float2* coarse_partials;     // [kCoarseChunks][coarse.row] per-chunk sums of the coarse levels' gradient
    // model
    GridParams grid;
    half_t* table;               // fp16 working copy [L][T][2]
    float* table_f32;            // fp32 master
    float* table_grad;           // fp32, loss-scaled
    float* table_m;
    float* table_v;
    half_t* dparams;             // 3072 fp16
    half_t* cparams;             // 7168 fp16
    float* mlp_f32;              // 10240 fp32 masters (density then colour)
    float* mlp_grad;             // 10240, loss-scaled
    float* mlp_m;
    float* mlp_v;
    float* dw_partials;          // [kDxMaxBlocks][10240] per-workgroup weight-gradient partials
    double* norm_partials;       // [norm_partial_count] per-workgroup squared-gradient-norm partials
    uint64_t table_elems;        // 0 for the reference model (no hash grid)
    // Which network trains: NERF_EXT_MODEL_HASHGRID (the buffers above) or
    // NERF_EXT_MODEL_REFERENCE (the reference's own network: no table, no
    // features; the backward's buffers below).
    uint32_t model_kind;
    uint32_t mlp_params;         // kMlpParams or kRefParams (masters, moments, gradients)
    uint32_t density_params;     // the density network's share (first in mlp_f32)
    RefTrainLaunch ref;          // reference model: packed weights, backward buffers
    float* occ_points;           // reference model: [occ_window][3] world cell centres of a refresh
    float* occ_dirs;             // [occ_window][3] (0, 0, 1)
    float4* occ_field;           // [occ_window] field at those points
    uint32_t occ_window;         // min(cells_per_update, cells)
};

// Batches of at most 128 steps per ray (sparse samples) keep the step's
// features level-major only (features_lm): the level-split encode writes
// them, the MLP pass and the input-gradient pass read them.
inline bool sparse_features(const TrainParams& P, const TrainBuffers& B) {
    return B.model_kind != NERF_EXT_MODEL_REFERENCE && P.max_steps <= 128u && B.grid.n_levels == 16u && B.features_lm != nullptr;
}

constexpr uint32_t kDxMaxBlocks = 1024;  // workgroups of the input-gradient pass (two per CU)
constexpr uint32_t kBinEntries = 4096;  // table entries per scatter bin (64 KiB of int64 pairs in LDS)
constexpr uint32_t kBinBlocks  = 256;   // workgroups of the bin count / fill passes
constexpr uint32_t kSegSteps = 64;  // march steps per resumable segment of the training sampler
constexpr uint32_t kMaxBins    = 16384; // bins; the fill pass keeps a cursor and a maximum per bin in LDS (128 KiB)
constexpr uint32_t kMlpParams  = NERF_EXT_DENSITY_PARAMS + NERF_EXT_COLOR_PARAMS;

// Workgroups of the coarse-level reduction (16 columns of two entries each).
__host__ __device__ inline uint32_t coarse_reduce_blocks(const CoarsePlan& C) { return (C.row / 2u + 15u) / 16u; }
// Squared-norm partials of a step: coarse reduction, bins, weight gradients
// (the reference model: its weight-gradient reduction only).
inline uint32_t norm_partial_count(const TrainBuffers& B) {
    return B.model_kind == NERF_EXT_MODEL_REFERENCE ? kRefReduceBlocks : coarse_reduce_blocks(B.coarse) + B.n_bins + kMlpParams / 64u;
}

// A second stream beside a step's own: the hash table's record count and its
// scan depend only on the step's samples, so the sample stage starts them
// there and the backward waits for them, instead of running them between
// the MLP backward and the record fill.  counted[s] is true once a count has
// been started for the step in slot s.  A run of several steps also puts
// each step's begin, occupancy and sample stages there, after the previous
// step's record fill (`filled`: the last reader of the sample stream), so
// that they overlap its gradient sums and Adam pass.
struct StepStreams {
    hipStream_t aux       = nullptr;
    hipEvent_t sampled[2] = {nullptr, nullptr};  // per slot: the sample stage's end, on the stream it ran on
    hipEvent_t done[2]    = {nullptr, nullptr};  // per slot: the count and scan's end, on aux
    hipEvent_t ready      = nullptr;             // a point on the step's stream the second stream waits for
    hipEvent_t filled     = nullptr;             // the record fill's end, on the step's stream (record_filled)
    bool counted[2]       = {false, false};
    bool record_filled    = false;
    uint32_t slot         = 0u;                  // the slot of the step being enqueued
};

// Folds of a step's one-thread stages into their neighbours, for callers that
// enqueue the neighbours too (each launch costs a few microseconds whatever
// it does).  kFoldBegin: the begin stage launches nothing and the step's
// first kernel (the occupancy refresh, else the ray pass; hash-grid model)
// does the begin.  kFoldEnd: the end stage launches nothing and the
// backward's gradient-norm kernel does the end (before Adam, which reads its
// own copy of the step index).
enum : uint32_t { kFoldBegin = 1u, kFoldEnd = 2u };

// Launches one stage (NERF_EXT_STAGE_*) of a training step on `stream`.
// `occupancy_update` selects the occupancy-maintenance kernels (the schedule
// is a function of the step index, which the host tracks).  ss may be null
// (then the count runs in the backward, on `stream`).  fold: kFold* bits,
// passed to the stages on either side of the one folded away.
hipError_t launch_train_stage(const TrainParams& P, const TrainBuffers& B, uint32_t stage, bool occupancy_update, hipStream_t stream, StepStreams* ss, uint32_t fold = 0u);

// Individual stages, exposed for the parity tests through nerf_ext.h.
hipError_t launch_composite_train(const TrainParams& P, const TrainBuffers& B, hipStream_t stream);
// end: the gradient-norm kernel also ends the step (kFoldEnd).
hipError_t launch_mlp_backward(const TrainParams& P, const TrainBuffers& B, hipStream_t stream, StepStreams* ss, bool end = false);
hipError_t launch_adam(const TrainParams& P, const TrainBuffers& B, hipStream_t stream);

uint64_t scan_tmp_words(uint32_t n);
hipError_t exclusive_scan_u32(const uint32_t* in, uint32_t* out, uint32_t n, uint32_t* tmp, unsigned long long* total, hipStream_t stream);

}  // namespace nerf_hip
