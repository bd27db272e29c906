// nerf_bench — the reference's host program (benchmark.cpp) on this backend:
// the same command line, training loop, logging, periodic inference with
// PSNR and checkpoint save/load, all through the reference ABI (nerf.h).
// Besides a NeRF-synthetic dataset directory (--dataset), it can train on
// the analytic Gaussian scene rendered on the device (--synthetic VIEWS).
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <iostream>
#include <limits>
#include <stdexcept>
#include <string>
#include <string_view>
#include <vector>

#include "../../include/nerf.h"
#include "../../include/nerf_ext.h"
#include "dataset.hpp"
#include "png.hpp"

using namespace nerf_host;

namespace {

void check(NerfStatus s, const char* what) {
    if (s != NERF_STATUS_OK) {
        const char* msg = nerf_ext_last_error();
        throw std::runtime_error(std::string(what) + " failed: status=" + std::to_string((int)s) + (msg && *msg ? std::string(" (") + msg + ")" : std::string()));
    }
}

// The analytic scene (count Gaussians from `seed`) seen from `views` orbit
// cameras of radius 1.32 around the box centre (radius 4 in the Blender
// frame), rendered on the device with `steps` quadrature steps.
HostDataset synthetic_dataset(uint32_t views, uint32_t size, uint32_t count, uint64_t seed, uint32_t steps) {
    HostDataset d;
    d.count = views, d.width = size, d.height = size;
    NerfExtSceneDesc sd{};
    sd.count = count;
    sd.seed  = seed;
    sd.centre_lo = 0.2f, sd.centre_hi = 0.8f, sd.sigma_lo = 0.02f, sd.sigma_hi = 0.1f, sd.amplitude_lo = 5.0f, sd.amplitude_hi = 50.0f;
    std::vector<NerfExtGaussian> g(count);
    check(nerf_ext_scene_gaussians(&sd, g.data()), "nerf_ext_scene_gaussians");
    std::vector<NerfExtCamera> cams(views);
    const float centre[3] = {0.5f, 0.5f, 0.5f};
    const float focal     = 1111.0f * (float)size / 800.0f;
    for (uint32_t i = 0; i < views; ++i) check(nerf_ext_camera_orbit(seed, i, 1.32f, centre, size, size, focal, &cams[i]), "nerf_ext_camera_orbit");
    void* dg = nullptr;
    void* dimg = nullptr;
    const uint64_t img_bytes = (uint64_t)views * size * size * 4u;
    check(nerf_ext_malloc(&dg, sizeof(NerfExtGaussian) * count), "nerf_ext_malloc");
    check(nerf_ext_malloc(&dimg, img_bytes), "nerf_ext_malloc");
    check(nerf_ext_memcpy(dg, g.data(), sizeof(NerfExtGaussian) * count, NERF_EXT_H2D), "nerf_ext_memcpy");
    const float box[6] = {0.0f, 0.0f, 0.0f, 1.0f, 1.0f, 1.0f};
    check(nerf_ext_scene_render((const NerfExtGaussian*)dg, count, cams.data(), views, box, steps, (uint32_t*)dimg, nullptr), "nerf_ext_scene_render");
    check(nerf_ext_synchronize(), "nerf_ext_synchronize");
    d.images_rgba8.resize(img_bytes);
    check(nerf_ext_memcpy(d.images_rgba8.data(), dimg, img_bytes, NERF_EXT_D2H), "nerf_ext_memcpy");
    nerf_ext_free(dg);
    nerf_ext_free(dimg);
    d.cameras_4x4.resize((size_t)views * 16);
    for (uint32_t i = 0; i < views; ++i) {
        float* m = d.cameras_4x4.data() + (size_t)i * 16;
        for (int r = 0; r < 3; ++r)
            for (int c = 0; c < 4; ++c) m[4 * r + c] = cams[i].c2w[4 * r + c];
        m[12] = m[13] = m[14] = 0.0f;
        m[15] = 1.0f;
    }
    d.fx = cams[0].fx, d.fy = cams[0].fy, d.cx = cams[0].cx, d.cy = cams[0].cy;
    return d;
}

bool parse_u32(std::string_view v, uint32_t& out) {
    char* end = nullptr;
    const std::string s(v);
    const unsigned long x = std::strtoul(s.c_str(), &end, 10);
    if (s.empty() || !end || *end != '\0' || x > 0xFFFFFFFFul) return false;
    out = (uint32_t)x;
    return true;
}

}  // namespace

int main(int argc, char** argv) {
    std::string dataset_path, load_weights, save_weights, inference_out = "nerf_inference_final.png", model_name = "hashgrid";
    uint32_t steps = 10000u, rays = 4096u, max_sample_steps = 64u, log_interval = 200u, inference_interval = 2000u, inference_camera = 0u, inference_samples = 64u;
    uint32_t synthetic = 0u, synthetic_size = 800u, synthetic_gaussians = 32u, seed = 0u;

    auto help = [&]() {
        std::cout << "Usage: " << (argc > 0 ? argv[0] : "nerf_bench") << " (--dataset <path> | --synthetic <views>) [options]\n"
                  << "  --steps <N> default " << steps << "\n  --rays <N> default " << rays << "\n  --max-sample-steps <N> default " << max_sample_steps << "\n  --log-interval <N> default " << log_interval
                  << "\n  --inference-interval <N> default " << inference_interval << "\n  --inference-camera <N> default " << inference_camera << "\n  --inference-samples <N> default " << inference_samples
                  << "\n  --inference-out <path> default " << inference_out << "\n  --load-weights <path> optional\n  --save-weights <path> optional\n"
                  << "  --synthetic <views>: train on the analytic Gaussian scene instead of a dataset\n  --synthetic-size <N> default " << synthetic_size << "\n  --synthetic-gaussians <N> default " << synthetic_gaussians
                  << "\n  --seed <N> default " << seed << "\n  --model <hashgrid|reference> default hashgrid (reference: the reference's own network, nerf_ext_context_configure)\n";
    };
    for (int i = 1; i < argc; ++i) {
        const std::string_view key = argv[i];
        if (key == "--help" || key == "-h") {
            help();
            return 0;
        }
        if (i + 1 >= argc) {
            std::cerr << "missing value for " << key << '\n';
            return 2;
        }
        const std::string_view value = argv[++i];
        struct U32Opt {
            const char* name;
            uint32_t* dst;
        } const opts[] = {{"--steps", &steps}, {"--rays", &rays}, {"--max-sample-steps", &max_sample_steps}, {"--log-interval", &log_interval}, {"--inference-interval", &inference_interval},
                          {"--inference-camera", &inference_camera}, {"--inference-samples", &inference_samples}, {"--synthetic", &synthetic}, {"--synthetic-size", &synthetic_size},
                          {"--synthetic-gaussians", &synthetic_gaussians}, {"--seed", &seed}};
        bool handled = false;
        for (const U32Opt& o : opts) {
            if (key == o.name) {
                if (!parse_u32(value, *o.dst)) {
                    std::cerr << "invalid value for " << key << ": " << value << '\n';
                    return 2;
                }
                handled = true;
            }
        }
        if (handled) continue;
        if (key == "--dataset") dataset_path = value;
        else if (key == "--load-weights") load_weights = value;
        else if (key == "--save-weights") save_weights = value;
        else if (key == "--inference-out") inference_out = value;
        else if (key == "--model") model_name = value;
        else {
            std::cerr << "unknown argument: " << key << '\n';
            return 2;
        }
    }
    if (dataset_path.empty() == (synthetic == 0u)) {
        std::cerr << "exactly one of --dataset and --synthetic is required\n";
        return 2;
    }
    if (model_name != "hashgrid" && model_name != "reference") {
        std::cerr << "--model must be hashgrid or reference\n";
        return 2;
    }
    if (log_interval == 0u || inference_interval == 0u) {
        std::cerr << "--log-interval and --inference-interval must be positive\n";
        return 2;
    }

    void* ctx = nullptr;
    struct Guard {
        void** c;
        ~Guard() {
            if (*c) nerf_destroy_context(*c);
        }
    } guard{&ctx};
    // The reference host program's settings (benchmark.cpp:416-432, :446-474).
    NerfHyperParams hp{};
    hp.learning_rate = 5e-4f, hp.adam_beta1 = 0.9f, hp.adam_beta2 = 0.999f, hp.adam_eps = 1e-8f, hp.grad_clip_norm = 1.0f, hp.update_guard_grad_norm = 100.0f, hp.loss_scale = 128.0f, hp.lr_decay_ksteps = 250u;
    NerfOccupancyParams occ{};
    occ.decay = 0.98f, occ.threshold = 0.01f, occ.cells_per_update = 65536u, occ.update_interval = 1u, occ.warmup_steps = 32u;
    try {
        HostDataset data;
        if (synthetic) {
            data = synthetic_dataset(synthetic, synthetic_size, synthetic_gaussians, seed, 512u);
        } else {
            std::string err;
            if (!load_nerf_synthetic(dataset_path, data, &err)) throw std::runtime_error(err);
        }
        if (inference_camera >= data.count) throw std::runtime_error("--inference-camera is not a frame of the dataset");
        std::vector<uint8_t> pred((size_t)data.width * data.height * 4u);
        NerfCreateDesc cd{};
        cd.occupancy_grid_res = 128u, cd.max_sample_steps = 1u << 21, cd.max_batch_rays = 1u << 16, cd.arena_alignment_bytes = 256u;
        cd.images_rgba8 = data.images_rgba8.data(), cd.images_bytes = data.images_rgba8.size();
        cd.cameras_4x4_packed = data.cameras_4x4.data(), cd.cameras_bytes = data.cameras_4x4.size() * sizeof(float);
        cd.image_count = data.count, cd.image_width = data.width, cd.image_height = data.height;
        cd.fx = data.fx, cd.fy = data.fy, cd.cx = data.cx, cd.cy = data.cy;
        check(nerf_create_context(&cd, &ctx), "nerf_create_context");
        if (model_name == "reference") {
            const NerfExtContextOptions o{NERF_EXT_MODEL_REFERENCE, NERF_EXT_SAMPLING_DEFAULT};
            check(nerf_ext_context_configure(ctx, &o), "nerf_ext_context_configure");
        }
        if (!load_weights.empty()) {
            const NerfCheckpointFileDesc f{load_weights.c_str()};
            check(nerf_load_network_weights(ctx, &f), "nerf_load_network_weights");
        }
        NerfTrainingConfig tc{};
        tc.aabb_min_x = tc.aabb_min_y = tc.aabb_min_z = 0.0f;
        tc.aabb_max_x = tc.aabb_max_y = tc.aabb_max_z = 1.0f;
        tc.hyper_params = hp, tc.occupancy_params = occ, tc.rays_per_batch = rays, tc.max_sample_steps_per_ray = max_sample_steps;
        check(nerf_configure_training(ctx, &tc), "nerf_configure_training");
        const auto t0 = std::chrono::steady_clock::now();
        float loss_ema = 0.0f;
        for (uint32_t step = 0; step < steps; ++step) {
            check(nerf_train_step(ctx), "nerf_train_step");
            const uint32_t done = step + 1u;
            if (done % log_interval == 0u || done == steps) {
                NerfTrainStats st{};
                check(nerf_read_train_stats(ctx, &st), "nerf_read_train_stats");
                loss_ema             = step == 0u ? st.loss : 0.95f * loss_ema + 0.05f * st.loss;
                const float sec      = std::chrono::duration<float>(std::chrono::steady_clock::now() - t0).count();
                const float sps      = sec > 0.0f ? (float)done / sec : 0.0f;
                const double eta_sec = sps > 0.0f ? (double)(steps - done) / (double)sps : std::numeric_limits<double>::infinity();
                std::cout << "[train] step=" << done << " loss=" << st.loss << " loss_ema=" << loss_ema << " grad_norm=" << st.grad_norm << " sps=" << sps << " eta_sec=" << eta_sec
                          << " nonfinite=" << (st.has_nonfinite ? 1 : 0) << std::endl;
            }
            if (done % inference_interval == 0u || done == steps) {
                NerfInferenceInfo info{};
                const NerfInferenceRequest req{inference_camera, inference_samples, NERF_MEMORY_HOST, pred.data(), pred.size()};
                check(nerf_inference(ctx, &req, &info), "nerf_inference");
                const Metrics m = evaluate_rgba8(data, inference_camera, pred.data());
                std::cout << "[eval] step=" << done << " camera=" << inference_camera << " psnr=" << m.psnr << " pred_luma=" << m.pred_luma << std::endl;
                if (done == steps) {
                    if (!png_write_file(inference_out, info.width, info.height, pred.data())) throw std::runtime_error("cannot write " + inference_out);
                    std::cout << "[eval] saved=" << inference_out << std::endl;
                }
            }
        }
        if (!save_weights.empty()) {
            const NerfCheckpointFileDesc f{save_weights.c_str()};
            check(nerf_save_network_weights(ctx, &f), "nerf_save_network_weights");
        }
    } catch (const std::exception& ex) {
        std::cerr << ex.what() << '\n';
        return 1;
    }
    return 0;
}
