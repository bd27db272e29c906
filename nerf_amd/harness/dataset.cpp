// dataset.cpp — see dataset.hpp.
#include "dataset.hpp"

#include <cmath>
#include <cstdio>
#include <filesystem>
#include <fstream>
#include <limits>
#include <sstream>

#include "json.hpp"
#include "png.hpp"

namespace nerf_host {
namespace {

bool fail(std::string* e, const std::string& m) {
    if (e) *e = m;
    return false;
}

// Column c of the matrix of basis b holds the unit vector of its c-th axis.
void basis_matrix(const Basis& b, float m[9]) {
    for (int i = 0; i < 9; ++i) m[i] = 0.0f;
    const SignedAxis cols[3] = {b.x, b.y, b.z};
    for (uint32_t c = 0; c < 3; ++c) m[cols[c].axis * 3 + c] = cols[c].sign;
}

}  // namespace

void transform_camera(const SceneTransform& tf, const float src[16], float dst[16]) {
    float sw[9], sc[9], dw[9], dc[9];
    basis_matrix(tf.src_world, sw);
    basis_matrix(tf.src_camera, sc);
    basis_matrix(tf.dst_world, dw);
    basis_matrix(tf.dst_camera, dc);
    // W = Dw^T Sw (source world -> destination world), C = Sc^T Dc.
    float W[9] = {}, C[9] = {};
    for (int r = 0; r < 3; ++r)
        for (int c = 0; c < 3; ++c)
            for (int k = 0; k < 3; ++k) {
                W[r * 3 + c] += dw[k * 3 + r] * sw[k * 3 + c];
                C[r * 3 + c] += sc[k * 3 + r] * dc[k * 3 + c];
            }
    const float R[9] = {src[0], src[1], src[2], src[4], src[5], src[6], src[8], src[9], src[10]};
    const float t[3] = {src[3], src[7], src[11]};
    float WR[9] = {}, Rn[9] = {}, tn[3] = {};
    for (int r = 0; r < 3; ++r)
        for (int c = 0; c < 3; ++c)
            for (int k = 0; k < 3; ++k) WR[r * 3 + c] += W[r * 3 + k] * R[k * 3 + c];
    for (int r = 0; r < 3; ++r)
        for (int c = 0; c < 3; ++c)
            for (int k = 0; k < 3; ++k) Rn[r * 3 + c] += WR[r * 3 + k] * C[k * 3 + c];
    for (int r = 0; r < 3; ++r)
        for (int k = 0; k < 3; ++k) tn[r] += W[r * 3 + k] * t[k];
    for (int r = 0; r < 3; ++r) {
        dst[4 * r + 0] = Rn[r * 3 + 0];
        dst[4 * r + 1] = Rn[r * 3 + 1];
        dst[4 * r + 2] = Rn[r * 3 + 2];
        dst[4 * r + 3] = tn[r] * tf.scale + tf.bias[r];
    }
    dst[12] = dst[13] = dst[14] = 0.0f;
    dst[15] = 1.0f;
}

bool load_nerf_synthetic(const std::string& path, HostDataset& out, std::string* e, const SceneTransform& tf) {
    namespace fs = std::filesystem;
    fs::path json_path(path);
    if (json_path.extension() != ".json") json_path /= "transforms_train.json";
    std::ifstream f(json_path, std::ios::binary);
    if (!f) return fail(e, "dataset: cannot open " + json_path.string());
    std::stringstream ss;
    ss << f.rdbuf();
    Json doc;
    std::string err;
    if (!json_parse(ss.str(), doc, &err)) return fail(e, "dataset: " + json_path.string() + ": " + err);
    const Json* angle  = doc.get("camera_angle_x");
    const Json* frames = doc.get("frames");
    if (!angle || angle->kind != Json::Number || !frames || frames->kind != Json::Array || frames->arr.empty()) return fail(e, "dataset: camera_angle_x and a non-empty frames array are required");
    const size_t n = frames->arr.size();
    out = HostDataset{};
    out.cameras_4x4.resize(n * 16);
    for (size_t i = 0; i < n; ++i) {
        const Json& fr = frames->arr[i];
        const Json* fp = fr.get("file_path");
        const Json* tm = fr.get("transform_matrix");
        if (!fp || fp->kind != Json::String || !tm || tm->kind != Json::Array || tm->arr.size() != 4) return fail(e, "dataset: frame " + std::to_string(i) + " lacks file_path or a 4x4 transform_matrix");
        float m[16];
        for (size_t r = 0; r < 4; ++r) {
            const Json* row = tm->at(r);
            if (!row || row->kind != Json::Array || row->arr.size() != 4) return fail(e, "dataset: frame " + std::to_string(i) + ": transform_matrix is not 4x4");
            for (size_t c = 0; c < 4; ++c) {
                if (row->arr[c].kind != Json::Number) return fail(e, "dataset: frame " + std::to_string(i) + ": non-numeric matrix entry");
                m[r * 4 + c] = (float)row->arr[c].num;
            }
        }
        transform_camera(tf, m, out.cameras_4x4.data() + i * 16);
        fs::path img = json_path.parent_path() / fp->str;
        if (!img.has_extension()) img.replace_extension(".png");
        Image im;
        if (!png_read_file(img.string(), im, &err)) return fail(e, "dataset: " + img.string() + ": " + err);
        if (i == 0) {
            out.width  = im.width;
            out.height = im.height;
            out.images_rgba8.reserve(n * (size_t)im.width * im.height * 4);
        } else if (im.width != out.width || im.height != out.height) {
            return fail(e, "dataset: " + img.string() + ": frame size differs from the first frame");
        }
        out.images_rgba8.insert(out.images_rgba8.end(), im.rgba.begin(), im.rgba.end());
    }
    out.count = (uint32_t)n;
    const float wf = (float)out.width, hf = (float)out.height;
    out.fx = 0.5f * wf / std::tan((float)angle->num * 0.5f);
    out.fy = out.fx;
    out.cx = 0.5f * (wf - 1.0f);
    out.cy = 0.5f * (hf - 1.0f);
    return true;
}

Metrics evaluate_rgba8(const HostDataset& d, uint32_t camera, const uint8_t* pred) {
    const size_t px = (size_t)d.width * d.height;
    const uint8_t* gt = d.images_rgba8.data() + (size_t)camera * px * 4;
    const float inv = 1.0f / 255.0f;
    double se = 0.0, luma = 0.0;
    for (size_t i = 0; i < px; ++i) {
        const float a = gt[4 * i + 3] * inv;
        double sq     = 0.0;
        float p[3];
        for (int c = 0; c < 3; ++c) {
            const float g = gt[4 * i + c] * inv * a + (1.0f - a);
            p[c]          = pred[4 * i + c] * inv;
            const double diff = (double)(p[c] - g);
            sq += diff * diff;
        }
        se += sq / 3.0;
        luma += (double)(0.2126f * p[0] + 0.7152f * p[1] + 0.0722f * p[2]);
    }
    const double mse = se / (double)px;
    Metrics m;
    m.psnr      = mse > 0.0 ? -10.0 * std::log10(mse) : std::numeric_limits<double>::infinity();
    m.pred_luma = luma / (double)px;
    return m;
}

}  // namespace nerf_host
