// dataset.hpp — host-side datasets for the reference ABI (nerf.h): the
// NeRF-synthetic layout (transforms JSON + PNG frames, as benchmark.cpp:148-303
// reads it) and the analytic Gaussian scene rendered on the device, plus the
// PSNR evaluation of benchmark.cpp:47-86.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace nerf_host {

struct HostDataset {
    std::vector<uint8_t> images_rgba8;  // [count][height][width][4]
    std::vector<float> cameras_4x4;     // [count][16] row-major camera-to-world, already in the backend's frame
    uint32_t count = 0, width = 0, height = 0;
    float fx = 0.0f, fy = 0.0f, cx = 0.0f, cy = 0.0f;
};

// Signed axis of a coordinate basis: axis 0..2 (x, y, z) with sign +-1.
struct SignedAxis {
    uint32_t axis;
    float sign;
};
struct Basis {
    SignedAxis x, y, z;
};

// The NeRF-synthetic convention (benchmark.cpp:149-156): world axes (x, -z,
// y) of the Blender frame map to the backend's (x, y, z), camera axes are
// kept, translations are scaled by 0.33 and offset by 0.5 per axis.
struct SceneTransform {
    Basis src_world{{0, 1.0f}, {2, -1.0f}, {1, 1.0f}};
    Basis src_camera{{0, 1.0f}, {1, 1.0f}, {2, 1.0f}};
    Basis dst_world{{0, 1.0f}, {1, 1.0f}, {2, 1.0f}};
    Basis dst_camera{{0, 1.0f}, {1, 1.0f}, {2, 1.0f}};
    float scale = 0.33f;
    float bias[3] = {0.5f, 0.5f, 0.5f};
};

// Maps one row-major 4x4 camera-to-world matrix of the source convention to
// the backend's: R' = W R C, t' = scale (W t) + bias, with W taking source
// world coordinates to destination ones and C destination camera
// coordinates to source ones.
void transform_camera(const SceneTransform& tf, const float src[16], float dst[16]);

// Loads <path>/transforms_train.json (or the .json file given) and its
// frames.  Intrinsics from camera_angle_x: fx = fy = W / (2 tan(angle / 2)),
// cx = (W - 1) / 2, cy = (H - 1) / 2.
bool load_nerf_synthetic(const std::string& path, HostDataset& out, std::string* error, const SceneTransform& tf = SceneTransform{});

// PSNR of an RGBA8 prediction against frame `camera` (the ground truth
// composited over white with its alpha, mean squared error over RGB and
// pixels in double), and the prediction's mean Rec. 709 luma.
struct Metrics {
    double psnr = 0.0, pred_luma = 0.0;
};
Metrics evaluate_rgba8(const HostDataset& data, uint32_t camera, const uint8_t* pred_rgba8);

}  // namespace nerf_host
