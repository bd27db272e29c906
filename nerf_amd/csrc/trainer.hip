// trainer.hip — the training run object behind nerf_ext_trainer_* and the
// reference ABI's nerf_configure_training / nerf_train_step.
//
// Owns the device state, the ray/sample buffers of one step and (unless the
// caller lends them) the model: fp32 master table and MLP weights, their
// fp16 working copies, Adam moments and gradients, and the occupancy grid.
#include <string.h>

#include <vector>

#include "trainer.hpp"

namespace nerf_hip {

Trainer::~Trainer() {
    if (side.aux) (void)hipStreamSynchronize(side.aux);
    if (stream) (void)hipStreamSynchronize(stream);
    for (int k = 0; k < 2; ++k) {
        if (side.sampled[k]) (void)hipEventDestroy(side.sampled[k]);
        if (side.done[k]) (void)hipEventDestroy(side.done[k]);
    }
    if (side.ready) (void)hipEventDestroy(side.ready);
    if (side.filled) (void)hipEventDestroy(side.filled);
    if (side.aux) (void)hipStreamDestroy(side.aux);
    for (void* p : owned)
        if (p) (void)hipFree(p);
    if (stream && own_stream) (void)hipStreamDestroy(stream);
}

template <typename T>
static hipError_t alloc(Trainer& t, T*& ptr, uint64_t count) {
    void* p        = nullptr;
    const hipError_t e = hipMalloc(&p, count * sizeof(T) > 0 ? count * sizeof(T) : 16u);
    if (e != hipSuccess) return e;
    t.owned.push_back(p);
    ptr = static_cast<T*>(p);
    return hipSuccess;
}

bool Trainer::occupancy_due(uint32_t frame) const {
    if (frame < P.occ_warmup) return frame == 0u;                      // backend-cuda.cu:1483-1485
    return P.occ_interval != 0u && frame % P.occ_interval == 0u;       // :1487
}

// The fold bits for stage s of a range that starts at `first` and ends at
// `last` (kFoldBegin: hash-grid model, the range holds the begin and the
// step's first kernel; kFoldEnd: the range holds the backward and the end).
uint32_t Trainer::fold_for(uint32_t s, uint32_t first, uint32_t last, bool occ) const {
    uint32_t fold = 0u;
    if (B.model_kind != NERF_EXT_MODEL_REFERENCE && first == NERF_EXT_STAGE_BEGIN && last >= NERF_EXT_STAGE_SAMPLE &&
        (s == NERF_EXT_STAGE_BEGIN || s == (occ ? NERF_EXT_STAGE_OCCUPANCY : NERF_EXT_STAGE_SAMPLE)))
        fold |= kFoldBegin;
    if (first <= NERF_EXT_STAGE_BACKWARD && last == NERF_EXT_STAGE_END && (s == NERF_EXT_STAGE_BACKWARD || s == NERF_EXT_STAGE_END)) fold |= kFoldEnd;
    return fold;
}

TrainBuffers Trainer::at(uint32_t step) const {
    TrainBuffers b = B;
    b.state        = slot_state[step & 1u];
    b.prev         = slot_state[(step + 1u) & 1u];
    b.bin_off      = slot_bin_off[step & 1u];
    b.bin_total    = slot_bin_total[step & 1u];
    return b;
}

NerfStatus Trainer::run_stages(uint32_t first, uint32_t last) {
    for (uint32_t s = first; s <= last; ++s) {
        const bool occ = occupancy_due(host_frame);
        side.slot      = host_frame & 1u;
        NERF_HIP_TRY(launch_train_stage(P, at(host_frame), s, occ, stream, &side, fold_for(s, first, last, occ)));
        open = s != NERF_EXT_STAGE_END;
        if (s == NERF_EXT_STAGE_END) ++host_frame;
    }
    return NERF_STATUS_OK;
}

// Several whole steps.  With a second stream each step's begin, occupancy
// and sample stages and its record count run there; the step's own stream
// waits for the samples before its forward pass and for the count before
// its record fill (the count runs beside the forward: beside the gradient
// sums and Adam it slowed them and ended after them).  Step k + 1's are
// enqueued there after step k's record fill, the last reader of the sample
// stream, so they run beside step k's gradient sums and Adam pass: the two
// steps' counters live in different state slots (TrainBuffers::state and
// prev) and their record ranges in different bin-offset buffers.  A step that
// refreshes the occupancy grid evaluates the weights the previous step's Adam
// writes, so its stages wait for that Adam instead.  The first step waits for
// all the work already on the step's stream, so the overlap stays inside one
// call and work a caller enqueues between calls is ordered as before.  Every
// stage of a step ends before the step's stream passes its forward pass, so
// synchronizing that stream covers the whole run.
NerfStatus Trainer::run_steps(uint32_t steps) {
    if (!side.aux || !side.ready || !side.filled || steps < 2u) {
        for (uint32_t i = 0; i < steps; ++i) {
            const NerfStatus s = run_stages(NERF_EXT_STAGE_BEGIN, NERF_EXT_STAGE_END);
            if (s != NERF_STATUS_OK) return s;
        }
        return NERF_STATUS_OK;
    }
    auto sample_aux = [&](uint32_t k) -> hipError_t {
        const bool occ = occupancy_due(k);
        side.slot      = k & 1u;
        for (uint32_t s = NERF_EXT_STAGE_BEGIN; s <= NERF_EXT_STAGE_SAMPLE; ++s) {
            const hipError_t e = launch_train_stage(P, at(k), s, occ, side.aux, &side, fold_for(s, NERF_EXT_STAGE_BEGIN, NERF_EXT_STAGE_SAMPLE, occ));
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    };
    NERF_HIP_TRY(hipEventRecord(side.ready, stream));
    NERF_HIP_TRY(hipStreamWaitEvent(side.aux, side.ready, 0));
    NERF_HIP_TRY(sample_aux(host_frame));
    open = true;
    for (uint32_t i = 0; i < steps; ++i) {
        const uint32_t k    = host_frame;
        const bool more     = i + 1u < steps;
        const bool occ_next = more && occupancy_due(k + 1u);
        const TrainBuffers Bk = at(k);
        side.slot = k & 1u;
        // The step's samples; its record count, which runs beside the forward
        // pass, is waited for by the backward before the fill.
        NERF_HIP_TRY(hipStreamWaitEvent(stream, side.sampled[k & 1u], 0));
        side.record_filled = more && !occ_next;
        for (uint32_t s = NERF_EXT_STAGE_FORWARD; s <= NERF_EXT_STAGE_BACKWARD; ++s)
            NERF_HIP_TRY(launch_train_stage(P, Bk, s, false, stream, &side, fold_for(s, NERF_EXT_STAGE_BEGIN, NERF_EXT_STAGE_END, false)));  // the backward ends the step
        side.record_filled = false;
        ++host_frame;
        if (more && !occ_next) {
            NERF_HIP_TRY(hipStreamWaitEvent(side.aux, side.filled, 0));
            NERF_HIP_TRY(sample_aux(k + 1u));
        }
        side.slot = k & 1u;
        NERF_HIP_TRY(launch_train_stage(P, Bk, NERF_EXT_STAGE_ADAM, false, stream, &side));
        if (occ_next) {
            NERF_HIP_TRY(hipEventRecord(side.ready, stream));  // after this step's Adam
            NERF_HIP_TRY(hipStreamWaitEvent(side.aux, side.ready, 0));
            NERF_HIP_TRY(sample_aux(k + 1u));
        }
    }
    open = false;
    return NERF_STATUS_OK;
}

NerfStatus trainer_create(const NerfExtTrainDesc* d, const BorrowedModel* borrowed, hipStream_t stream, Trainer** out) {
    NERF_CHECK_ARG(d && out, "trainer: null argument");
    *out = nullptr;
    NERF_CHECK_ARG(d->image_count >= 1u && d->cameras && (d->images_rgba8 || (borrowed && borrowed->images)), "trainer: a dataset of at least one image is required");
    NERF_CHECK_ARG(d->model_kind <= NERF_EXT_MODEL_REFERENCE, "trainer: unknown model_kind");
    const bool ref = d->model_kind == NERF_EXT_MODEL_REFERENCE;
    NERF_CHECK_ARG(ref || d->grid.table_dtype == NERF_EXT_F16, "trainer: the hash table must be fp16");
    NERF_CHECK_ARG(!ref || d->sample_capacity <= kRefMaxSamples, "trainer: the reference model takes at most 2^20 samples per step (sample_capacity)");
    NERF_CHECK_ARG(d->max_rays >= 1u && d->sample_capacity >= 1u && d->max_steps_per_ray >= 1u, "trainer: capacities must be >= 1");
    // Per-ray sample offsets are a u32 exclusive scan of counts of at most
    // max_steps_per_ray each: the sum must not wrap.
    NERF_CHECK_ARG((uint64_t)d->max_rays * d->max_steps_per_ray < (1ull << 32), "trainer: max_rays x max_steps_per_ray must stay below 2^32");
    NERF_CHECK_ARG(d->occupancy_res >= 1u && d->occupancy_res <= 1024u, "trainer: occupancy_res must be 1..1024");
    NERF_CHECK_ARG(d->hyper.loss_scale > 0.0f, "trainer: loss_scale must be > 0");
    const uint32_t W = d->cameras[0].width, H = d->cameras[0].height;
    for (uint32_t i = 0; i < d->image_count; ++i) NERF_CHECK_ARG(d->cameras[i].width == W && d->cameras[i].height == H && W > 0u && H > 0u, "trainer: all images must share one non-empty size");
    for (int a = 0; a < 3; ++a) NERF_CHECK_ARG(d->aabb_max[a] > d->aabb_min[a], "trainer: empty AABB");

    auto t = std::make_unique<Trainer>();
    GridParams g{};
    NerfStatus st = NERF_STATUS_OK;
    if (!ref) {
        st = make_grid(&d->grid, g);
        if (st != NERF_STATUS_OK) return st;
        NERF_CHECK_ARG(g.n_levels * g.n_features == 32u, "trainer: the density MLP takes 32 features (16 levels x 2)");
        NERF_CHECK_ARG((uint64_t)g.n_levels * g.table_size <= (uint64_t)kMaxBins * kBinEntries, "trainer: at most 2^26 table entries (16 levels x 2^22)");
        NERF_CHECK_ARG((uint64_t)d->sample_capacity * g.n_levels * 8u < (1ull << 32), "trainer: sample_capacity x 128 must stay below 2^32 gradient records");
    }
    if (stream) {
        t->stream = stream;
    } else {
        NERF_HIP_TRY(hipStreamCreateWithFlags(&t->stream, hipStreamNonBlocking));
        t->own_stream = true;
    }
    TrainParams& P = t->P;
    P.image_count  = d->image_count;
    P.width        = W;
    P.height       = H;
    P.occ_res      = d->occupancy_res;
    for (int a = 0; a < 3; ++a) {
        P.bmin[a] = d->aabb_min[a];
        P.bmax[a] = d->aabb_max[a];
    }
    P.max_steps            = d->max_steps_per_ray;
    P.max_rays             = d->max_rays;
    P.sample_cap           = d->sample_capacity;
    P.target_samples       = d->target_samples;
    P.min_rays             = d->target_samples ? 64u : 1u;
    if (P.min_rays > P.max_rays) P.min_rays = P.max_rays;
    P.huber_delta          = d->huber_delta > 0.0f ? d->huber_delta : 0.1f;
    P.loss_scale           = d->hyper.loss_scale;
    P.lr                   = d->hyper.learning_rate;
    P.beta1                = d->hyper.adam_beta1;
    P.beta2                = d->hyper.adam_beta2;
    P.eps                  = d->hyper.adam_eps;
    P.clip                 = d->hyper.grad_clip_norm;
    P.guard                = d->hyper.update_guard_grad_norm;
    P.lr_decay_ksteps      = d->hyper.lr_decay_ksteps;
    P.occ_decay            = d->occupancy.decay;
    P.occ_threshold        = d->occupancy.threshold;
    P.occ_cells_per_update = d->occupancy.cells_per_update;
    P.occ_interval         = d->occupancy.update_interval;
    P.occ_warmup           = d->occupancy.warmup_steps;
    P.occ_cells            = d->occupancy_res * d->occupancy_res * d->occupancy_res;

    TrainBuffers& B    = t->B;
    B.grid             = g;
    B.model_kind       = d->model_kind;
    B.table_elems      = ref ? 0ull : (uint64_t)g.n_levels * g.table_size * g.n_features;
    B.mlp_params       = ref ? kRefParams : kMlpParams;
    B.density_params   = ref ? (uint32_t)NERF_EXT_REF_DENSITY_PARAMS : (uint32_t)NERF_EXT_DENSITY_PARAMS;
    Trainer& T      = *t;
    NERF_HIP_TRY(alloc(T, T.slot_state[0], 2));
    T.slot_state[1] = T.slot_state[0] + 1;
    B.state         = T.slot_state[0];
    B.prev          = T.slot_state[1];
    NerfExtCamera* cams = nullptr;
    NERF_HIP_TRY(alloc(T, cams, d->image_count));
    B.cams = cams;
    uint8_t* images = nullptr;  // the trainer's own copy, unless the dataset is borrowed on the device
    if (borrowed && borrowed->images) {
        B.images = borrowed->images;
    } else {
        NERF_HIP_TRY(alloc(T, images, (uint64_t)d->image_count * W * H * 4u));
        B.images = images;
    }
    NERF_HIP_TRY(alloc(T, B.rays, 2ull * P.max_rays));
    NERF_HIP_TRY(alloc(T, B.gt, P.max_rays));
    NERF_HIP_TRY(alloc(T, B.counts, P.max_rays));
    NERF_HIP_TRY(alloc(T, B.kept, P.max_rays));
    NERF_HIP_TRY(alloc(T, B.offsets, P.max_rays));
    B.segs = (P.max_steps + kSegSteps - 1u) / kSegSteps;
    NERF_HIP_TRY(alloc(T, B.seg_t, (uint64_t)P.max_rays * B.segs));
    NERF_HIP_TRY(alloc(T, B.seg_seen, (uint64_t)P.max_rays * B.segs));
    NERF_HIP_TRY(alloc(T, B.seg_reached, P.max_rays));
    NERF_HIP_TRY(alloc(T, B.samples, P.sample_cap));
    NERF_HIP_TRY(alloc(T, B.sample_ray, P.sample_cap));
    NERF_HIP_TRY(alloc(T, B.field, P.sample_cap));
    NERF_HIP_TRY(alloc(T, B.draw, P.sample_cap));
    B.n_dense = 0u;
    B.coarse  = CoarsePlan{};
    B.n_bins  = 0u;
    if (ref) {
        RefTrainLaunch& R = B.ref;
        R.np              = (P.sample_cap + 63u) / 64u * 64u;
        R.chunks          = (R.np + kRefDwChunk - 1u) / kRefDwChunk;
        R.max_rays        = P.max_rays;
        NERF_HIP_TRY(alloc(T, R.frags, 64ull * kRefFragments));
        NERF_HIP_TRY(alloc(T, R.acts, (uint64_t)kRefActRows * R.np));
        NERF_HIP_TRY(alloc(T, R.dlts, (uint64_t)kRefDltRows * R.np));
        NERF_HIP_TRY(alloc(T, R.partial, (uint64_t)R.chunks * kRefParams));
        B.occ_window = P.occ_cells_per_update < P.occ_cells ? P.occ_cells_per_update : P.occ_cells;
        NERF_HIP_TRY(alloc(T, B.occ_points, 3ull * B.occ_window));
        NERF_HIP_TRY(alloc(T, B.occ_dirs, 3ull * B.occ_window));
        NERF_HIP_TRY(alloc(T, B.occ_field, B.occ_window));
        NERF_HIP_TRY(hipMemsetAsync(B.occ_points, 0, 12ull * B.occ_window, T.stream));
        NERF_HIP_TRY(hipMemsetAsync(B.occ_dirs, 0, 12ull * B.occ_window, T.stream));
    } else {
    NERF_HIP_TRY(alloc(T, B.features, 32ull * P.sample_cap));
    NERF_HIP_TRY(alloc(T, B.features_lm, 16ull * P.sample_cap));
    NERF_HIP_TRY(alloc(T, B.dfeat, 16ull * P.sample_cap));
    // Leading dense levels of at most kCoarseMaxEntries entries are summed in
    // LDS slabs; binned, the records of every sample would crowd into their
    // few bins.  Every other level is binned.
    B.n_dense          = 0u;
    CoarsePlan& C      = B.coarse;
    C                  = CoarsePlan{};
    while (B.n_dense < g.n_levels && g.dense[B.n_dense]) {
        const uint64_t v = (uint64_t)g.resolution[B.n_dense] + 1u;
        if (v * v * v > kCoarseMaxEntries) break;
        const uint32_t l     = B.n_dense++;
        const uint32_t e     = (uint32_t)(v * v * v);
        const uint32_t e_pad = (e + 1u) & ~1u;
        C.level_entries[l]   = e;
        C.level_part[l]      = C.row;
        for (uint32_t b = 0; b < e_pad; b += kCoarseSlabEntries) {
            C.level[C.n_slabs] = l;
            C.begin[C.n_slabs] = b;
            C.count[C.n_slabs] = e_pad - b < kCoarseSlabEntries ? e_pad - b : kCoarseSlabEntries;
            ++C.n_slabs;
        }
        C.row += e_pad;
    }
    C.level_part[B.n_dense] = C.row;
    if (C.row) NERF_HIP_TRY(alloc(T, B.coarse_partials, (uint64_t)kCoarseChunks * C.row));
    B.n_bins  = (uint32_t)(((uint64_t)(g.n_levels - B.n_dense) * g.table_size + kBinEntries - 1u) / kBinEntries);
    B.rec_cap = (uint64_t)P.sample_cap * (g.n_levels - B.n_dense) * 8u;
    NERF_HIP_TRY(alloc(T, B.bin_hist, (uint64_t)B.n_bins * kBinBlocks));
    NERF_HIP_TRY(alloc(T, T.slot_bin_off[0], 2ull * B.n_bins * kBinBlocks));
    T.slot_bin_off[1] = T.slot_bin_off[0] + (uint64_t)B.n_bins * kBinBlocks;
    B.bin_off         = T.slot_bin_off[0];
    NERF_HIP_TRY(alloc(T, B.bin_max, (uint64_t)B.n_bins * kBinBlocks));
    NERF_HIP_TRY(alloc(T, B.bin_scan_tmp, scan_tmp_words(B.n_bins * kBinBlocks + 1u)));
    NERF_HIP_TRY(alloc(T, T.slot_bin_total[0], 2));
    T.slot_bin_total[1] = T.slot_bin_total[0] + 1;
    B.bin_total         = T.slot_bin_total[0];
    NERF_HIP_TRY(alloc(T, B.rec, B.rec_cap));
    NERF_HIP_TRY(alloc(T, B.dw_partials, (uint64_t)kDxMaxBlocks * kMlpParams));
    if (B.n_bins) {
        NERF_HIP_TRY(hipStreamCreateWithFlags(&T.side.aux, hipStreamNonBlocking));
        for (int k = 0; k < 2; ++k) {
            NERF_HIP_TRY(hipEventCreateWithFlags(&T.side.sampled[k], hipEventDisableTiming));
            NERF_HIP_TRY(hipEventCreateWithFlags(&T.side.done[k], hipEventDisableTiming));
        }
        NERF_HIP_TRY(hipEventCreateWithFlags(&T.side.ready, hipEventDisableTiming));
        NERF_HIP_TRY(hipEventCreateWithFlags(&T.side.filled, hipEventDisableTiming));
    }
    }
    NERF_HIP_TRY(alloc(T, B.table_grad, B.table_elems));
    NERF_HIP_TRY(alloc(T, B.table_m, B.table_elems));
    NERF_HIP_TRY(alloc(T, B.table_v, B.table_elems));
    NERF_HIP_TRY(alloc(T, B.mlp_grad, B.mlp_params));
    NERF_HIP_TRY(alloc(T, B.mlp_m, B.mlp_params));
    NERF_HIP_TRY(alloc(T, B.mlp_v, B.mlp_params));
    NERF_HIP_TRY(alloc(T, B.norm_partials, norm_partial_count(B)));
    if (borrowed) {
        B.table     = borrowed->table;
        B.table_f32 = borrowed->table_f32;
        B.dparams   = borrowed->dparams;
        B.cparams   = borrowed->cparams;
        B.mlp_f32   = borrowed->mlp_f32;
        B.bits      = borrowed->bits;
        B.density   = borrowed->density;
    } else {
        NERF_HIP_TRY(alloc(T, B.table, B.table_elems));
        NERF_HIP_TRY(alloc(T, B.table_f32, B.table_elems));
        NERF_HIP_TRY(alloc(T, B.dparams, B.density_params));
        NERF_HIP_TRY(alloc(T, B.cparams, B.mlp_params - B.density_params));
        NERF_HIP_TRY(alloc(T, B.mlp_f32, B.mlp_params));
        NERF_HIP_TRY(alloc(T, B.bits, (P.occ_cells + 31u) / 32u));
        NERF_HIP_TRY(alloc(T, B.density, P.occ_cells));
    }
    hipStream_t s = T.stream;
    NERF_HIP_TRY(hipMemcpyAsync(cams, d->cameras, sizeof(NerfExtCamera) * d->image_count, hipMemcpyHostToDevice, s));
    if (images) NERF_HIP_TRY(hipMemcpyAsync(images, d->images_rgba8, (uint64_t)d->image_count * W * H * 4u, hipMemcpyHostToDevice, s));
    T.initial_rays = (float)(d->initial_rays ? d->initial_rays : 1u);
    st             = T.reset();
    if (st != NERF_STATUS_OK) return st;
    if (!borrowed) {
        if (!ref) {
            NerfExtGridDesc g32 = d->grid;
            g32.table_dtype     = NERF_EXT_F32;
            st                  = nerf_ext_grid_init_table(&g32, d->seed, d->table_init_range, B.table_f32, s);
            if (st != NERF_STATUS_OK) return st;
            st = nerf_ext_float_to_half(B.table_f32, (uint16_t*)B.table, B.table_elems, s);
            if (st != NERF_STATUS_OK) return st;
        }
        // The reference's Xavier init (backend-cuda.cu:1810-1847) on the
        // network's shapes.
        std::vector<float> w(B.mlp_params);
        if (ref) {
            nerf_ext_ref_mlp_init(0u, w.data());
            nerf_ext_ref_mlp_init(1u, w.data() + B.density_params);
        } else {
            nerf_ext_mlp_init(0u, w.data());
            nerf_ext_mlp_init(1u, w.data() + B.density_params);
        }
        NERF_HIP_TRY(hipMemcpyAsync(B.mlp_f32, w.data(), sizeof(float) * B.mlp_params, hipMemcpyHostToDevice, s));
        NERF_HIP_TRY(hipStreamSynchronize(s));
        st = nerf_ext_float_to_half(B.mlp_f32, (uint16_t*)B.dparams, B.density_params, s);
        if (st == NERF_STATUS_OK) st = nerf_ext_float_to_half(B.mlp_f32 + B.density_params, (uint16_t*)B.cparams, B.mlp_params - B.density_params, s);
        if (st != NERF_STATUS_OK) return st;
    }
    NERF_HIP_TRY(hipStreamSynchronize(s));
    T.grid_desc = d->grid;
    *out       = t.release();
    return NERF_STATUS_OK;
}

NerfStatus Trainer::reset() {
    hipStream_t s = stream;
    NERF_HIP_TRY(hipMemsetAsync(B.table_grad, 0, B.table_elems * 4u, s));
    NERF_HIP_TRY(hipMemsetAsync(B.table_m, 0, B.table_elems * 4u, s));
    NERF_HIP_TRY(hipMemsetAsync(B.table_v, 0, B.table_elems * 4u, s));
    NERF_HIP_TRY(hipMemsetAsync(B.mlp_grad, 0, B.mlp_params * 4ull, s));
    NERF_HIP_TRY(hipMemsetAsync(B.mlp_m, 0, B.mlp_params * 4ull, s));
    NERF_HIP_TRY(hipMemsetAsync(B.mlp_v, 0, B.mlp_params * 4ull, s));
    NERF_HIP_TRY(hipMemsetAsync(B.bits, 0, (P.occ_cells + 31u) / 32u * 4u, s));
    NERF_HIP_TRY(hipMemsetAsync(B.density, 0, (uint64_t)P.occ_cells * 4u, s));
    // Slot 1 stands for the step before step 0: index -1, the initial ray
    // count as its choice for the next step, no samples yet.
    TrainDevState init[2]{};
    init[1].frame     = 0xFFFFFFFFu;
    init[1].rays_f    = initial_rays;
    init[1].rays_next = initial_rays;
    NERF_HIP_TRY(hipMemcpyAsync(slot_state[0], init, sizeof(init), hipMemcpyHostToDevice, s));
    NERF_HIP_TRY(hipStreamSynchronize(s));
    host_frame = 0u;
    open       = false;
    for (int k = 0; k < 2; ++k) side.counted[k] = false;
    return NERF_STATUS_OK;
}

// The state of the step in progress (some of its stages enqueued), else of
// the last completed step.
TrainDevState* Trainer::current_state() const { return slot_state[(open ? host_frame : host_frame - 1u) & 1u]; }

NerfStatus Trainer::read_state(TrainDevState& host, TrainDevState* last) {
    NERF_HIP_TRY(hipStreamSynchronize(stream));
    NERF_HIP_TRY(hipMemcpy(&host, current_state(), sizeof(host), hipMemcpyDeviceToHost));
    if (last) NERF_HIP_TRY(hipMemcpy(last, slot_state[(host_frame - 1u) & 1u], sizeof(*last), hipMemcpyDeviceToHost));
    return NERF_STATUS_OK;
}

}  // namespace nerf_hip

using namespace nerf_hip;

struct NerfExtTrainer {
    nerf_hip::Trainer* t = nullptr;
};

extern "C" {

NERF_API NerfStatus nerf_ext_trainer_create(const NerfExtTrainDesc* desc, NerfExtTrainer** out) {
    NERF_CHECK_ARG(out, "nerf_ext_trainer_create: null output");
    *out       = nullptr;
    Trainer* t = nullptr;
    const NerfStatus s = trainer_create(desc, nullptr, nullptr, &t);
    if (s != NERF_STATUS_OK) return s;
    *out      = new NerfExtTrainer();
    (*out)->t = t;
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_trainer_destroy(NerfExtTrainer* trainer) {
    if (!trainer) return NERF_STATUS_OK;
    delete trainer->t;
    delete trainer;
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_trainer_step(NerfExtTrainer* trainer, uint32_t steps) {
    NERF_CHECK_ARG(trainer && trainer->t, "nerf_ext_trainer_step: null trainer");
    return trainer->t->run_steps(steps);
}

NERF_API NerfStatus nerf_ext_trainer_run_stages(NerfExtTrainer* trainer, uint32_t first, uint32_t last) {
    NERF_CHECK_ARG(trainer && trainer->t, "nerf_ext_trainer_run_stages: null trainer");
    NERF_CHECK_ARG(first <= last && last <= NERF_EXT_STAGE_END, "nerf_ext_trainer_run_stages: bad stage range");
    return trainer->t->run_stages(first, last);
}

NERF_API NerfStatus nerf_ext_trainer_synchronize(NerfExtTrainer* trainer) {
    NERF_CHECK_ARG(trainer && trainer->t, "nerf_ext_trainer_synchronize: null trainer");
    NERF_HIP_TRY(hipStreamSynchronize(trainer->t->stream));
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_trainer_stats(NerfExtTrainer* trainer, NerfExtTrainStats* out) {
    NERF_CHECK_ARG(trainer && trainer->t && out, "nerf_ext_trainer_stats: null argument");
    // The step in progress (or the last one) for its counters; the last
    // completed step for its statistics and the running sample total.
    TrainDevState s{}, done{};
    const NerfStatus st = trainer->t->read_state(s, &done);
    if (st != NERF_STATUS_OK) return st;
    out->last             = done.stats;
    out->rays             = s.n_rays;
    out->samples          = s.n_samples;
    out->active_rays      = s.n_active;
    out->skipped          = s.skip;
    out->occupied_samples = s.total;
    out->samples_total    = done.samples_done;
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_trainer_buffers(NerfExtTrainer* trainer, NerfExtTrainBuffers* o) {
    NERF_CHECK_ARG(trainer && trainer->t && o, "nerf_ext_trainer_buffers: null argument");
    const TrainBuffers& B = trainer->t->B;
    memset(o, 0, sizeof(*o));
    o->state           = trainer->t->current_state();
    o->rays            = (float*)B.rays;
    o->gt              = (float*)B.gt;
    o->counts          = B.counts;
    o->kept            = B.kept;
    o->offsets         = B.offsets;
    o->samples         = (float*)B.samples;
    o->sample_ray      = B.sample_ray;
    o->field           = (float*)B.field;
    o->features        = (uint16_t*)B.features;
    o->draw            = (float*)B.draw;
    o->table_grad      = B.table_grad;
    o->mlp_grad        = B.mlp_grad;
    o->table_f32       = B.table_f32;
    o->mlp_f32         = B.mlp_f32;
    o->table_m         = B.table_m;
    o->table_v         = B.table_v;
    o->mlp_m           = B.mlp_m;
    o->mlp_v           = B.mlp_v;
    o->bitfield        = B.bits;
    o->density_grid    = B.density;
    o->max_rays        = trainer->t->P.max_rays;
    o->sample_capacity = trainer->t->P.sample_cap;
    o->table_elems     = B.table_elems;
    o->dfeat           = (float*)B.dfeat;
    o->features_lm     = sparse_features(trainer->t->P, B) ? B.features_lm : nullptr;
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_trainer_model(NerfExtTrainer* trainer, NerfExtModel* model, NerfExtOccupancy* occ) {
    NERF_CHECK_ARG(trainer && trainer->t, "nerf_ext_trainer_model: null trainer");
    const Trainer& t = *trainer->t;
    if (model) {
        model->grid           = t.grid_desc;
        model->table          = t.B.table;
        model->density_params = (const uint16_t*)t.B.dparams;
        model->color_params   = (const uint16_t*)t.B.cparams;
        model->kind           = t.B.model_kind;
        model->reserved       = 0u;
    }
    if (occ) {
        occ->bitfield   = t.B.bits;
        occ->resolution = t.P.occ_res;
        occ->cascades   = 1u;
        for (int a = 0; a < 3; ++a) {
            occ->aabb_min[a] = t.P.bmin[a];
            occ->aabb_max[a] = t.P.bmax[a];
        }
    }
    return NERF_STATUS_OK;
}

NERF_API void* nerf_ext_trainer_stream(NerfExtTrainer* trainer) { return trainer && trainer->t ? (void*)trainer->t->stream : nullptr; }

}  // extern "C"
