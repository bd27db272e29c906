// host_capi.cpp — C entry points of the host harness pieces (PNG, JSON,
// dataset loading, camera transform, PSNR), built into libnerf_host.so so
// that they can be driven from Python without a GPU.
#include <cstring>
#include <string>

#include "dataset.hpp"
#include "json.hpp"
#include "png.hpp"

using namespace nerf_host;

#define HOST_API extern "C" __attribute__((visibility("default")))

namespace {
thread_local std::string g_error;
}

HOST_API const char* nerf_host_last_error() { return g_error.c_str(); }

// Decodes a PNG; with out == nullptr only the size is returned.  0 on success.
HOST_API int nerf_host_png_decode(const uint8_t* data, uint64_t n, uint32_t* w, uint32_t* h, uint8_t* out, uint64_t out_bytes) {
    Image im;
    if (!png_decode(data, n, im, &g_error)) return 1;
    *w = im.width, *h = im.height;
    if (out) {
        if (out_bytes < im.rgba.size()) {
            g_error = "nerf_host_png_decode: output too small";
            return 2;
        }
        std::memcpy(out, im.rgba.data(), im.rgba.size());
    }
    return 0;
}

// Encodes RGBA8; returns the PNG's size (the bytes are written when it fits in cap).
HOST_API uint64_t nerf_host_png_encode(uint32_t w, uint32_t h, const uint8_t* rgba, uint8_t* out, uint64_t cap) {
    const std::vector<uint8_t> png = png_encode_rgba(w, h, rgba);
    if (out && cap >= png.size()) std::memcpy(out, png.data(), png.size());
    return png.size();
}

HOST_API uint32_t nerf_host_crc32(const uint8_t* d, uint64_t n) { return crc32(d, n); }
HOST_API uint32_t nerf_host_adler32(const uint8_t* d, uint64_t n) { return adler32(d, n); }

// 0 if `text` is valid JSON; the number of top-level object keys in *keys.
HOST_API int nerf_host_json_check(const char* text, uint32_t* keys) {
    Json j;
    if (!json_parse(text, j, &g_error)) return 1;
    if (keys) *keys = j.kind == Json::Object ? (uint32_t)j.obj.size() : 0u;
    return 0;
}

// The NeRF-synthetic camera transform of one row-major 4x4 matrix.
HOST_API void nerf_host_transform_camera(const float src[16], float dst[16]) { transform_camera(SceneTransform{}, src, dst); }

// Loads a dataset: with images == nullptr only count/width/height/intrinsics
// are filled.  intrinsics = (fx, fy, cx, cy).  0 on success.
HOST_API int nerf_host_load_dataset(const char* path, uint32_t* count, uint32_t* width, uint32_t* height, float* intrinsics, float* cameras, uint64_t camera_floats, uint8_t* images, uint64_t image_bytes) {
    HostDataset d;
    if (!load_nerf_synthetic(path, d, &g_error)) return 1;
    *count = d.count, *width = d.width, *height = d.height;
    intrinsics[0] = d.fx, intrinsics[1] = d.fy, intrinsics[2] = d.cx, intrinsics[3] = d.cy;
    if (cameras) {
        if (camera_floats < d.cameras_4x4.size() || image_bytes < d.images_rgba8.size()) {
            g_error = "nerf_host_load_dataset: output too small";
            return 2;
        }
        std::memcpy(cameras, d.cameras_4x4.data(), d.cameras_4x4.size() * sizeof(float));
        if (images) std::memcpy(images, d.images_rgba8.data(), d.images_rgba8.size());
    }
    return 0;
}

// PSNR of pred against gt (both RGBA8 [h][w]); luma of pred in *luma.
HOST_API double nerf_host_psnr(const uint8_t* gt, const uint8_t* pred, uint32_t w, uint32_t h, double* luma) {
    HostDataset d;
    d.count = 1, d.width = w, d.height = h;
    d.images_rgba8.assign(gt, gt + (size_t)w * h * 4);
    const Metrics m = evaluate_rgba8(d, 0, pred);
    if (luma) *luma = m.pred_luma;
    return m.psnr;
}
