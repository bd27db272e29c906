// json.hpp — a small JSON reader (RFC 8259 values: objects, arrays,
// numbers, strings with escapes, true/false/null) for dataset descriptions.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace nerf_host {

struct Json {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool b = false;
    double num = 0.0;
    std::string str;
    std::vector<Json> arr;
    std::map<std::string, Json> obj;

    const Json* get(const std::string& key) const {
        if (kind != Object) return nullptr;
        auto it = obj.find(key);
        return it == obj.end() ? nullptr : &it->second;
    }
    const Json* at(size_t i) const { return kind == Array && i < arr.size() ? &arr[i] : nullptr; }
};

// Parses `text`; returns false with a message for malformed input.
bool json_parse(const std::string& text, Json& out, std::string* error);

}  // namespace nerf_host
