// checkpoint.cpp — weight checkpoint files for nerf_save_network_weights /
// nerf_load_network_weights.
//
// Container format of the reference (backend-cuda.cu:2466-2525): a u64
// little-endian header length, a JSON header, then raw little-endian f32
// tensor data; each tensor entry is {"dtype": "F32", "shape": [rows, cols],
// "data_offsets": [begin, end]} relative to the end of the header, and
// "__metadata__" carries the format name and network dimensions as numbers.
// Tensor names follow :1223-1241 ("density.input.weight", "color.hidden.0.weight",
// ...), plus "encoding.hash_table" for the hash grid, which the reference lacks.
// The JSON writer and the small reader below are this file's own (the
// reference uses nlohmann/json, which is not used here).
#include "checkpoint.hpp"

#include <stdio.h>
#include <string.h>

#include <cctype>
#include <cstdlib>
#include <fstream>
#include <map>

namespace nerf_ckpt {

namespace {

// Minimal JSON value and recursive-descent reader (objects, arrays, strings,
// numbers, true/false/null).  Enough for the header of this format.
struct Json {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    double num = 0.0;
    std::string str;
    std::vector<Json> arr;
    std::map<std::string, Json> obj;
};

struct Reader {
    const char* p;
    const char* end;
    bool ok = true;

    void ws() {
        while (p < end && std::isspace((unsigned char)*p)) ++p;
    }
    bool eat(char c) {
        ws();
        if (p < end && *p == c) {
            ++p;
            return true;
        }
        return false;
    }
    std::string string() {
        std::string s;
        if (!eat('"')) {
            ok = false;
            return s;
        }
        while (p < end && *p != '"') {
            if (*p == '\\' && p + 1 < end) {
                ++p;
                switch (*p) {
                case 'n': s += '\n'; break;
                case 't': s += '\t'; break;
                case 'r': s += '\r'; break;
                case 'b': s += '\b'; break;
                case 'f': s += '\f'; break;
                case 'u':
                    if (end - p < 5) {
                        ok = false;
                        return s;
                    }
                    s += '?';  // non-ASCII escapes are not used by this format
                    p += 4;
                    break;
                default: s += *p;
                }
                ++p;
            } else {
                s += *p++;
            }
        }
        if (p >= end) ok = false;
        else ++p;
        return s;
    }
    Json value(int depth = 0) {
        Json v;
        ws();
        if (p >= end || depth > 32) {
            ok = false;
            return v;
        }
        if (*p == '{') {
            ++p;
            v.kind = Json::Object;
            if (eat('}')) return v;
            do {
                std::string k = string();
                if (!ok || !eat(':')) {
                    ok = false;
                    return v;
                }
                v.obj[k] = value(depth + 1);
                if (!ok) return v;
            } while (eat(','));
            if (!eat('}')) ok = false;
        } else if (*p == '[') {
            ++p;
            v.kind = Json::Array;
            if (eat(']')) return v;
            do {
                v.arr.push_back(value(depth + 1));
                if (!ok) return v;
            } while (eat(','));
            if (!eat(']')) ok = false;
        } else if (*p == '"') {
            v.kind = Json::String;
            v.str  = string();
        } else if (!strncmp(p, "true", 4) && end - p >= 4) {
            v.kind = Json::Bool;
            v.num  = 1.0;
            p += 4;
        } else if (!strncmp(p, "false", 5) && end - p >= 5) {
            v.kind = Json::Bool;
            p += 5;
        } else if (!strncmp(p, "null", 4) && end - p >= 4) {
            p += 4;
        } else {
            char* q      = nullptr;
            std::string tmp(p, (size_t)std::min<ptrdiff_t>(end - p, 64));
            const double d = strtod(tmp.c_str(), &q);
            if (q == tmp.c_str()) {
                ok = false;
                return v;
            }
            v.kind = Json::Number;
            v.num  = d;
            p += (q - tmp.c_str());
        }
        return v;
    }
};

}  // namespace

// The header is written as the reference's JSON library writes it: compact,
// object keys in byte order at every level (so a file saved here and one
// saved by the reference for the same weights are byte-identical); tensor
// data follows in the order of `tensors`.
bool save(const char* path, const std::vector<Tensor>& tensors, const std::vector<std::pair<std::string, std::string>>& meta_strings, const std::vector<std::pair<std::string, uint64_t>>& meta_numbers) {
    std::map<std::string, std::string> meta;  // key -> serialised value
    for (const auto& kv : meta_strings) meta[kv.first] = "\"" + kv.second + "\"";
    for (const auto& kv : meta_numbers) meta[kv.first] = std::to_string(kv.second);
    std::map<std::string, std::string> top;
    std::string m = "{";
    for (const auto& kv : meta) m += (m.size() > 1 ? "," : "") + std::string("\"") + kv.first + "\":" + kv.second;
    top["__metadata__"] = m + "}";
    uint64_t off = 0;
    for (const Tensor& t : tensors) {
        const uint64_t bytes = t.count() * sizeof(float);
        std::string e        = "{\"data_offsets\":[" + std::to_string(off) + "," + std::to_string(off + bytes) + "],\"dtype\":\"F32\",\"shape\":[";
        for (size_t i = 0; i < t.shape.size(); ++i) e += (i ? "," : "") + std::to_string(t.shape[i]);
        top[t.name] = e + "]}";
        off += bytes;
    }
    std::string h = "{";
    for (const auto& kv : top) h += (h.size() > 1 ? "," : "") + std::string("\"") + kv.first + "\":" + kv.second;
    h += "}";
    std::ofstream f(path, std::ios::binary | std::ios::trunc);
    if (!f) return false;
    const uint64_t hl = h.size();
    f.write((const char*)&hl, sizeof(hl));
    f.write(h.data(), (std::streamsize)h.size());
    for (const Tensor& t : tensors) f.write((const char*)t.data, (std::streamsize)(t.count() * sizeof(float)));
    return (bool)f;
}

bool read_format(const char* path, std::string& format, std::string& err) {
    std::ifstream f(path, std::ios::binary);
    if (!f) {
        err = "cannot open checkpoint";
        return false;
    }
    uint64_t hl = 0;
    f.read((char*)&hl, sizeof(hl));
    if (!f || hl == 0 || hl > (64ull << 20)) {
        err = "bad header length";
        return false;
    }
    std::string h(hl, '\0');
    f.read(h.data(), (std::streamsize)hl);
    if (!f) {
        err = "truncated header";
        return false;
    }
    Reader r{h.data(), h.data() + h.size()};
    const Json root = r.value();
    if (!r.ok || root.kind != Json::Object) {
        err = "header is not a JSON object";
        return false;
    }
    auto meta = root.obj.find("__metadata__");
    if (meta == root.obj.end() || meta->second.kind != Json::Object) {
        err = "no __metadata__";
        return false;
    }
    auto fmt = meta->second.obj.find("format");
    if (fmt == meta->second.obj.end() || fmt->second.kind != Json::String) {
        err = "no format in __metadata__";
        return false;
    }
    format = fmt->second.str;
    return true;
}

bool load(const char* path, std::vector<Tensor>& tensors, std::string& err) {
    std::ifstream f(path, std::ios::binary);
    if (!f) {
        err = "cannot open checkpoint";
        return false;
    }
    uint64_t hl = 0;
    f.read((char*)&hl, sizeof(hl));
    if (!f || hl == 0 || hl > (64ull << 20)) {
        err = "bad header length";
        return false;
    }
    std::string h(hl, '\0');
    f.read(h.data(), (std::streamsize)hl);
    if (!f) {
        err = "truncated header";
        return false;
    }
    Reader r{h.data(), h.data() + h.size()};
    const Json root = r.value();
    if (!r.ok || root.kind != Json::Object) {
        err = "header is not a JSON object";
        return false;
    }
    const uint64_t data_base = sizeof(uint64_t) + hl;
    for (Tensor& t : tensors) {
        auto it = root.obj.find(t.name);
        if (it == root.obj.end() || it->second.kind != Json::Object) {
            err = "missing tensor " + t.name;
            return false;
        }
        const Json& e = it->second;
        auto dt       = e.obj.find("dtype");
        auto sh       = e.obj.find("shape");
        auto dof      = e.obj.find("data_offsets");
        if (dt == e.obj.end() || dt->second.str != "F32" || sh == e.obj.end() || dof == e.obj.end() || dof->second.arr.size() != 2 || sh->second.arr.size() != t.shape.size()) {
            err = "bad entry for " + t.name;
            return false;
        }
        for (size_t i = 0; i < t.shape.size(); ++i)
            if ((uint64_t)sh->second.arr[i].num != t.shape[i]) {
                err = "shape mismatch for " + t.name;
                return false;
            }
        const uint64_t b = (uint64_t)dof->second.arr[0].num, en = (uint64_t)dof->second.arr[1].num;
        if (en - b != t.count() * sizeof(float)) {
            err = "size mismatch for " + t.name;
            return false;
        }
        f.seekg((std::streamoff)(data_base + b), std::ios::beg);
        f.read((char*)t.data, (std::streamsize)(en - b));
        if (!f) {
            err = "truncated data for " + t.name;
            return false;
        }
    }
    return true;
}

}  // namespace nerf_ckpt
