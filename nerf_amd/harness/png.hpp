// png.hpp — PNG reading (8-bit greyscale, grey+alpha, RGB, RGBA and
// palette images, any filter, non-interlaced) into RGBA8, and RGBA8 writing
// (stored deflate blocks), for the dataset loader and the render output of
// the host harness.  Formats: PNG (ISO/IEC 15948), zlib (RFC 1950), deflate
// (RFC 1951).
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace nerf_host {

struct Image {
    uint32_t width = 0, height = 0;
    std::vector<uint8_t> rgba;  // width * height * 4, row-major, top row first
};

// Decodes a PNG held in memory.  Returns false (and sets *error) for
// malformed data or unsupported variants (interlacing, 16-bit samples).
bool png_decode(const uint8_t* data, size_t size, Image& out, std::string* error);
bool png_read_file(const std::string& path, Image& out, std::string* error);

// Encodes RGBA8 as a PNG (filter 0 on every row, stored deflate blocks).
std::vector<uint8_t> png_encode_rgba(uint32_t width, uint32_t height, const uint8_t* rgba);
bool png_write_file(const std::string& path, uint32_t width, uint32_t height, const uint8_t* rgba);

// zlib stream -> bytes (inflate of stored, fixed and dynamic Huffman blocks).
bool zlib_inflate(const uint8_t* data, size_t size, std::vector<uint8_t>& out, std::string* error);

uint32_t crc32(const uint8_t* data, size_t size, uint32_t crc = 0u);
uint32_t adler32(const uint8_t* data, size_t size, uint32_t adler = 1u);

}  // namespace nerf_host
