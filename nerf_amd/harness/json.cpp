// json.cpp — recursive-descent reader for json.hpp.
#include "json.hpp"

#include <cstdlib>
#include <cstring>

namespace nerf_host {
namespace {

struct Parser {
    const char* p;
    const char* end;
    std::string err;
    int depth = 0;

    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
    }
    bool fail(const char* m) {
        if (err.empty()) err = m;
        return false;
    }
    bool lit(const char* s, Json& v, Json::Kind k, bool b) {
        const size_t n = std::strlen(s);
        if ((size_t)(end - p) < n || std::memcmp(p, s, n) != 0) return fail("json: bad literal");
        p += n;
        v.kind = k;
        v.b    = b;
        return true;
    }
    static void utf8(std::string& o, uint32_t cp) {
        if (cp < 0x80) o += (char)cp;
        else if (cp < 0x800) o += (char)(0xC0 | (cp >> 6)), o += (char)(0x80 | (cp & 63));
        else if (cp < 0x10000) o += (char)(0xE0 | (cp >> 12)), o += (char)(0x80 | ((cp >> 6) & 63)), o += (char)(0x80 | (cp & 63));
        else o += (char)(0xF0 | (cp >> 18)), o += (char)(0x80 | ((cp >> 12) & 63)), o += (char)(0x80 | ((cp >> 6) & 63)), o += (char)(0x80 | (cp & 63));
    }
    bool hex4(uint32_t& v) {
        if (end - p < 4) return fail("json: short \\u escape");
        v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else return fail("json: bad \\u escape");
        }
        return true;
    }
    bool string(std::string& o) {
        if (p >= end || *p != '"') return fail("json: expected string");
        ++p;
        while (p < end && *p != '"') {
            const char c = *p++;
            if ((unsigned char)c < 0x20) return fail("json: control character in string");
            if (c != '\\') {
                o += c;
                continue;
            }
            if (p >= end) return fail("json: bad escape");
            const char e = *p++;
            switch (e) {
            case '"': o += '"'; break;
            case '\\': o += '\\'; break;
            case '/': o += '/'; break;
            case 'b': o += '\b'; break;
            case 'f': o += '\f'; break;
            case 'n': o += '\n'; break;
            case 'r': o += '\r'; break;
            case 't': o += '\t'; break;
            case 'u': {
                uint32_t cp;
                if (!hex4(cp)) return false;
                if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
                    uint32_t lo;
                    if (end - p < 6 || p[0] != '\\' || p[1] != 'u') return fail("json: lone surrogate");
                    p += 2;
                    if (!hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return fail("json: bad surrogate pair");
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                }
                utf8(o, cp);
                break;
            }
            default: return fail("json: bad escape");
            }
        }
        if (p >= end) return fail("json: unterminated string");
        ++p;
        return true;
    }
    bool number(Json& v) {
        const char* s = p;
        if (p < end && *p == '-') ++p;
        if (p >= end || !(*p >= '0' && *p <= '9')) return fail("json: bad number");
        while (p < end && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '+' || *p == '-')) ++p;
        std::string tok(s, p);
        char* stop = nullptr;
        v.num      = std::strtod(tok.c_str(), &stop);
        if (!stop || *stop != '\0') return fail("json: bad number");
        v.kind = Json::Number;
        return true;
    }
    bool value(Json& v) {
        if (++depth > 256) return fail("json: nested too deeply");
        ws();
        if (p >= end) return fail("json: unexpected end");
        bool ok = true;
        switch (*p) {
        case '{': {
            ++p;
            v.kind = Json::Object;
            ws();
            if (p < end && *p == '}') {
                ++p;
                break;
            }
            for (;;) {
                ws();
                std::string key;
                if (!string(key)) return false;
                ws();
                if (p >= end || *p != ':') return fail("json: expected ':'");
                ++p;
                Json item;
                if (!value(item)) return false;
                v.obj[key] = std::move(item);
                ws();
                if (p < end && *p == ',') {
                    ++p;
                    continue;
                }
                if (p < end && *p == '}') {
                    ++p;
                    break;
                }
                return fail("json: expected ',' or '}'");
            }
            break;
        }
        case '[': {
            ++p;
            v.kind = Json::Array;
            ws();
            if (p < end && *p == ']') {
                ++p;
                break;
            }
            for (;;) {
                Json item;
                if (!value(item)) return false;
                v.arr.push_back(std::move(item));
                ws();
                if (p < end && *p == ',') {
                    ++p;
                    continue;
                }
                if (p < end && *p == ']') {
                    ++p;
                    break;
                }
                return fail("json: expected ',' or ']'");
            }
            break;
        }
        case '"':
            v.kind = Json::String;
            ok     = string(v.str);
            break;
        case 't': ok = lit("true", v, Json::Bool, true); break;
        case 'f': ok = lit("false", v, Json::Bool, false); break;
        case 'n': ok = lit("null", v, Json::Null, false); break;
        default: ok = number(v); break;
        }
        --depth;
        return ok;
    }
};

}  // namespace

bool json_parse(const std::string& text, Json& out, std::string* error) {
    Parser ps{text.data(), text.data() + text.size(), {}};
    out = Json{};
    bool ok = ps.value(out);
    if (ok) {
        ps.ws();
        if (ps.p != ps.end) ok = ps.fail("json: trailing characters");
    }
    if (!ok && error) *error = ps.err;
    return ok;
}

}  // namespace nerf_host
