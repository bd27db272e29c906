// checkpoint.hpp — safetensors-like weight files (see checkpoint.cpp).
#pragma once

#include <stdint.h>

#include <string>
#include <utility>
#include <vector>

namespace nerf_ckpt {

struct Tensor {
    std::string name;
    std::vector<uint64_t> shape;
    float* data;  // host, count() floats
    uint64_t count() const {
        uint64_t n = 1;
        for (uint64_t s : shape) n *= s;
        return n;
    }
};

bool save(const char* path, const std::vector<Tensor>& tensors, const std::vector<std::pair<std::string, std::string>>& meta_strings, const std::vector<std::pair<std::string, uint64_t>>& meta_numbers);
// The "format" string of a file's __metadata__.
bool read_format(const char* path, std::string& format, std::string& err);
// Fills each tensor's data (shapes must match the file); err explains a failure.
bool load(const char* path, std::vector<Tensor>& tensors, std::string& err);

}  // namespace nerf_ckpt
