// png.cpp — see png.hpp.  Inflate follows RFC 1951 section 3.2 (block
// types, the fixed code, the code-length alphabet and its order, the
// length and distance base/extra tables); decoding uses a 10-bit lookup
// table with a canonical-code walk for longer codes.
#include "png.hpp"

#include <cstdio>
#include <cstring>

namespace nerf_host {
namespace {

struct BitReader {
    const uint8_t* p;
    size_t n, pos = 0;  // byte position
    uint32_t bitbuf = 0, bitcnt = 0;
    bool overrun = false;
    uint32_t bits(uint32_t k) {  // k <= 24, LSB first
        while (bitcnt < k) {
            uint32_t b = 0;
            if (pos < n) b = p[pos++];
            else overrun = true;
            bitbuf |= b << bitcnt;
            bitcnt += 8;
        }
        const uint32_t v = bitbuf & ((1u << k) - 1u);
        bitbuf >>= k;
        bitcnt -= k;
        return v;
    }
    uint32_t peek(uint32_t k) {
        while (bitcnt < k) {
            uint32_t b = 0;
            if (pos < n) b = p[pos++];
            else if (bitcnt >= 32u - 8u) break;
            bitbuf |= b << bitcnt;
            bitcnt += 8;
        }
        return bitbuf & ((1u << k) - 1u);
    }
    void drop(uint32_t k) {
        if (k > bitcnt) overrun = true;
        bitbuf >>= k;
        bitcnt = k > bitcnt ? 0u : bitcnt - k;
    }
    void align() {
        drop(bitcnt & 7u);
    }
};

constexpr uint32_t kMaxBits = 15, kFastBits = 10;

// Canonical Huffman code from code lengths (RFC 1951 3.2.2).
struct Huffman {
    uint16_t count[kMaxBits + 1] = {};
    std::vector<uint16_t> symbol;   // symbols ordered by (length, value)
    std::vector<uint16_t> fast;     // [code bits reversed, kFastBits] -> (len << 9) | symbol, 0 = slow path
    bool build(const uint8_t* lengths, uint32_t n) {
        std::memset(count, 0, sizeof(count));
        for (uint32_t i = 0; i < n; ++i) count[lengths[i]]++;
        count[0] = 0;
        int left = 1;
        for (uint32_t len = 1; len <= kMaxBits; ++len) {
            left <<= 1;
            left -= count[len];
            if (left < 0) return false;  // over-subscribed
        }
        uint16_t offs[kMaxBits + 2] = {};
        for (uint32_t len = 1; len <= kMaxBits; ++len) offs[len + 1] = offs[len] + count[len];
        symbol.assign(n, 0);
        for (uint32_t i = 0; i < n; ++i)
            if (lengths[i]) symbol[offs[lengths[i]]++] = (uint16_t)i;
        // Fast table: codes of up to kFastBits bits, indexed by their bits
        // in stream order (the code reversed).
        fast.assign(1u << kFastBits, 0);
        uint32_t code = 0, idx = 0;
        for (uint32_t len = 1; len <= kFastBits; ++len) {
            for (uint32_t k = 0; k < count[len]; ++k, ++idx, ++code) {
                uint32_t rev = 0;
                for (uint32_t b = 0; b < len; ++b) rev |= ((code >> b) & 1u) << (len - 1u - b);
                for (uint32_t fill = rev; fill < (1u << kFastBits); fill += 1u << len) fast[fill] = (uint16_t)((len << 9) | symbol[idx]);
            }
            code <<= 1;
        }
        return true;
    }
    int decode(BitReader& br) const {
        const uint32_t look = br.peek(kFastBits);
        const uint16_t e    = fast[look];
        if (e) {
            br.drop(e >> 9);
            return e & 511;
        }
        // Canonical walk, one bit at a time (codes longer than kFastBits).
        int code = 0, first = 0, index = 0;
        for (uint32_t len = 1; len <= kMaxBits; ++len) {
            code |= (int)br.bits(1);
            const int c = count[len];
            if (code - c < first) return symbol[index + (code - first)];
            index += c;
            first += c;
            first <<= 1;
            code <<= 1;
        }
        return -1;
    }
};

const uint16_t kLenBase[29]  = {3, 4, 5, 6, 7, 8, 9, 10, 11, 13, 15, 17, 19, 23, 27, 31, 35, 43, 51, 59, 67, 83, 99, 115, 131, 163, 195, 227, 258};
const uint8_t kLenExtra[29]  = {0, 0, 0, 0, 0, 0, 0, 0, 1, 1, 1, 1, 2, 2, 2, 2, 3, 3, 3, 3, 4, 4, 4, 4, 5, 5, 5, 5, 0};
const uint16_t kDistBase[30] = {1, 2, 3, 4, 5, 7, 9, 13, 17, 25, 33, 49, 65, 97, 129, 193, 257, 385, 513, 769, 1025, 1537, 2049, 3073, 4097, 6145, 8193, 12289, 16385, 24577};
const uint8_t kDistExtra[30] = {0, 0, 0, 0, 1, 1, 2, 2, 3, 3, 4, 4, 5, 5, 6, 6, 7, 7, 8, 8, 9, 9, 10, 10, 11, 11, 12, 12, 13, 13};
const uint8_t kClOrder[19]   = {16, 17, 18, 0, 8, 7, 9, 6, 10, 5, 11, 4, 12, 3, 13, 2, 14, 1, 15};

bool fail(std::string* e, const char* msg) {
    if (e) *e = msg;
    return false;
}

bool inflate_codes(BitReader& br, const Huffman& lit, const Huffman& dist, std::vector<uint8_t>& out, std::string* e) {
    for (;;) {
        const int sym = lit.decode(br);
        if (sym < 0 || br.overrun) return fail(e, "inflate: bad literal/length code");
        if (sym < 256) {
            out.push_back((uint8_t)sym);
        } else if (sym == 256) {
            return true;
        } else {
            const int li = sym - 257;
            if (li >= 29) return fail(e, "inflate: bad length symbol");
            const uint32_t len = kLenBase[li] + br.bits(kLenExtra[li]);
            const int ds       = dist.decode(br);
            if (ds < 0 || ds >= 30) return fail(e, "inflate: bad distance code");
            const uint32_t d = kDistBase[ds] + br.bits(kDistExtra[ds]);
            if (d > out.size()) return fail(e, "inflate: distance beyond the output");
            const size_t from = out.size() - d;
            for (uint32_t k = 0; k < len; ++k) out.push_back(out[from + k]);
        }
    }
}

}  // namespace

uint32_t crc32(const uint8_t* data, size_t size, uint32_t crc) {
    static uint32_t table[256];
    static bool ready = false;
    if (!ready) {
        for (uint32_t i = 0; i < 256; ++i) {
            uint32_t c = i;
            for (int k = 0; k < 8; ++k) c = (c & 1u) ? 0xEDB88320u ^ (c >> 1) : c >> 1;
            table[i] = c;
        }
        ready = true;
    }
    crc = ~crc;
    for (size_t i = 0; i < size; ++i) crc = table[(crc ^ data[i]) & 0xFFu] ^ (crc >> 8);
    return ~crc;
}

uint32_t adler32(const uint8_t* data, size_t size, uint32_t adler) {
    uint32_t a = adler & 0xFFFFu, b = adler >> 16;
    for (size_t i = 0; i < size; ++i) {
        a = (a + data[i]) % 65521u;
        b = (b + a) % 65521u;
    }
    return (b << 16) | a;
}

bool zlib_inflate(const uint8_t* data, size_t size, std::vector<uint8_t>& out, std::string* e) {
    if (size < 6) return fail(e, "zlib: stream too short");
    const uint8_t cmf = data[0], flg = data[1];
    if ((cmf & 15u) != 8u || ((cmf << 8) | flg) % 31u != 0u) return fail(e, "zlib: bad header");
    if (flg & 0x20u) return fail(e, "zlib: preset dictionary not supported");
    BitReader br{data + 2, size - 2};
    bool last = false;
    while (!last) {
        last              = br.bits(1) != 0u;
        const uint32_t bt = br.bits(2);
        if (bt == 0u) {
            br.align();
            // The bit buffer is byte-aligned and holds whole bytes: drain it.
            uint8_t hdr[4];
            for (int k = 0; k < 4; ++k) hdr[k] = (uint8_t)br.bits(8);
            const uint32_t len = hdr[0] | (hdr[1] << 8), nlen = hdr[2] | (hdr[3] << 8);
            if ((len ^ 0xFFFFu) != nlen) return fail(e, "inflate: stored block length check");
            for (uint32_t k = 0; k < len; ++k) out.push_back((uint8_t)br.bits(8));
        } else if (bt == 1u) {
            static Huffman lit, dist;
            static bool ready = false;
            if (!ready) {
                uint8_t l[288], d[30];
                for (int i = 0; i < 144; ++i) l[i] = 8;
                for (int i = 144; i < 256; ++i) l[i] = 9;
                for (int i = 256; i < 280; ++i) l[i] = 7;
                for (int i = 280; i < 288; ++i) l[i] = 8;
                for (int i = 0; i < 30; ++i) d[i] = 5;
                lit.build(l, 288);
                dist.build(d, 30);
                ready = true;
            }
            if (!inflate_codes(br, lit, dist, out, e)) return false;
        } else if (bt == 2u) {
            const uint32_t hlit = br.bits(5) + 257u, hdist = br.bits(5) + 1u, hclen = br.bits(4) + 4u;
            uint8_t cl[19] = {};
            for (uint32_t i = 0; i < hclen; ++i) cl[kClOrder[i]] = (uint8_t)br.bits(3);
            Huffman clh;
            if (!clh.build(cl, 19)) return fail(e, "inflate: bad code-length code");
            uint8_t lens[320] = {};
            uint32_t i = 0;
            while (i < hlit + hdist) {
                const int sym = clh.decode(br);
                if (sym < 0 || br.overrun) return fail(e, "inflate: bad code length");
                if (sym < 16) {
                    lens[i++] = (uint8_t)sym;
                } else {
                    uint32_t rep = 0;
                    uint8_t v    = 0;
                    if (sym == 16) {
                        if (i == 0) return fail(e, "inflate: repeat with no previous length");
                        v   = lens[i - 1];
                        rep = 3 + br.bits(2);
                    } else if (sym == 17) {
                        rep = 3 + br.bits(3);
                    } else {
                        rep = 11 + br.bits(7);
                    }
                    if (i + rep > hlit + hdist) return fail(e, "inflate: code lengths overflow");
                    while (rep--) lens[i++] = v;
                }
            }
            Huffman lit, dist;
            if (!lit.build(lens, hlit) || !dist.build(lens + hlit, hdist)) return fail(e, "inflate: bad dynamic code");
            if (!inflate_codes(br, lit, dist, out, e)) return false;
        } else {
            return fail(e, "inflate: reserved block type");
        }
        if (br.overrun) return fail(e, "inflate: truncated stream");
    }
    return true;
}

namespace {
uint32_t be32(const uint8_t* p) { return ((uint32_t)p[0] << 24) | ((uint32_t)p[1] << 16) | ((uint32_t)p[2] << 8) | p[3]; }
void put_be32(std::vector<uint8_t>& v, uint32_t x) {
    v.push_back((uint8_t)(x >> 24));
    v.push_back((uint8_t)(x >> 16));
    v.push_back((uint8_t)(x >> 8));
    v.push_back((uint8_t)x);
}
uint8_t paeth(int a, int b, int c) {
    const int p = a + b - c, pa = p > a ? p - a : a - p, pb = p > b ? p - b : b - p, pc = p > c ? p - c : c - p;
    return (uint8_t)(pa <= pb && pa <= pc ? a : (pb <= pc ? b : c));
}
}  // namespace

bool png_decode(const uint8_t* d, size_t n, Image& out, std::string* e) {
    static const uint8_t sig[8] = {0x89, 'P', 'N', 'G', 0x0D, 0x0A, 0x1A, 0x0A};
    if (n < 8 || std::memcmp(d, sig, 8) != 0) return fail(e, "png: bad signature");
    size_t pos = 8;
    uint32_t w = 0, h = 0, depth = 0, ctype = 0, interlace = 0;
    std::vector<uint8_t> idat, palette, trns;
    bool have_ihdr = false, ended = false;
    while (pos + 12 <= n && !ended) {
        const uint32_t len = be32(d + pos);
        if (pos + 12 + (size_t)len > n) return fail(e, "png: truncated chunk");
        const uint8_t* type = d + pos + 4;
        const uint8_t* body = d + pos + 8;
        if (crc32(type, 4 + (size_t)len) != be32(body + len)) return fail(e, "png: chunk CRC mismatch");
        if (!std::memcmp(type, "IHDR", 4)) {
            if (len != 13) return fail(e, "png: bad IHDR");
            w = be32(body), h = be32(body + 4), depth = body[8], ctype = body[9], interlace = body[12];
            if (body[10] != 0 || body[11] != 0) return fail(e, "png: unknown compression or filter method");
            have_ihdr = true;
        } else if (!std::memcmp(type, "PLTE", 4)) {
            palette.assign(body, body + len);
        } else if (!std::memcmp(type, "tRNS", 4)) {
            trns.assign(body, body + len);
        } else if (!std::memcmp(type, "IDAT", 4)) {
            idat.insert(idat.end(), body, body + len);
        } else if (!std::memcmp(type, "IEND", 4)) {
            ended = true;
        }
        pos += 12 + (size_t)len;
    }
    if (!have_ihdr || !ended) return fail(e, "png: missing IHDR or IEND");
    if (interlace != 0) return fail(e, "png: interlaced images are not supported");
    if (depth != 8) return fail(e, "png: only 8-bit samples are supported");
    uint32_t ch = 0;
    switch (ctype) {
    case 0: ch = 1; break;
    case 2: ch = 3; break;
    case 3: ch = 1; break;
    case 4: ch = 2; break;
    case 6: ch = 4; break;
    default: return fail(e, "png: bad colour type");
    }
    if (ctype == 3 && palette.empty()) return fail(e, "png: palette image without PLTE");
    if (w == 0 || h == 0 || (uint64_t)w * h > (1ull << 28)) return fail(e, "png: bad size");
    std::vector<uint8_t> raw;
    raw.reserve((size_t)h * (1 + (size_t)w * ch));
    if (!zlib_inflate(idat.data(), idat.size(), raw, e)) return false;
    const size_t stride = (size_t)w * ch;
    if (raw.size() < (size_t)h * (stride + 1)) return fail(e, "png: image data too short");
    std::vector<uint8_t> cur(stride), prev(stride, 0);
    out.width = w, out.height = h;
    out.rgba.assign((size_t)w * h * 4, 0);
    for (uint32_t y = 0; y < h; ++y) {
        const uint8_t* line = raw.data() + (size_t)y * (stride + 1);
        const uint8_t f     = line[0];
        for (size_t x = 0; x < stride; ++x) {
            const int a = x >= ch ? cur[x - ch] : 0, b = prev[x], c = x >= ch ? prev[x - ch] : 0;
            const uint8_t v = line[1 + x];
            switch (f) {
            case 0: cur[x] = v; break;
            case 1: cur[x] = (uint8_t)(v + a); break;
            case 2: cur[x] = (uint8_t)(v + b); break;
            case 3: cur[x] = (uint8_t)(v + ((a + b) >> 1)); break;
            case 4: cur[x] = (uint8_t)(v + paeth(a, b, c)); break;
            default: return fail(e, "png: bad filter type");
            }
        }
        uint8_t* o = out.rgba.data() + (size_t)y * w * 4;
        for (uint32_t x = 0; x < w; ++x) {
            uint8_t r, g, b, al = 255;
            switch (ctype) {
            case 0: r = g = b = cur[x]; if (trns.size() >= 2 && cur[x] == trns[1]) al = 0; break;
            case 2:
                r = cur[3 * x], g = cur[3 * x + 1], b = cur[3 * x + 2];
                if (trns.size() >= 6 && r == trns[1] && g == trns[3] && b == trns[5]) al = 0;
                break;
            case 3: {
                const uint32_t k = cur[x];
                if (3 * k + 2 >= palette.size()) return fail(e, "png: palette index out of range");
                r = palette[3 * k], g = palette[3 * k + 1], b = palette[3 * k + 2];
                if (k < trns.size()) al = trns[k];
                break;
            }
            case 4: r = g = b = cur[2 * x]; al = cur[2 * x + 1]; break;
            default: r = cur[4 * x], g = cur[4 * x + 1], b = cur[4 * x + 2], al = cur[4 * x + 3]; break;
            }
            o[4 * x] = r, o[4 * x + 1] = g, o[4 * x + 2] = b, o[4 * x + 3] = al;
        }
        std::swap(cur, prev);
    }
    return true;
}

bool png_read_file(const std::string& path, Image& out, std::string* e) {
    FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) return fail(e, "png: cannot open file");
    std::vector<uint8_t> buf;
    uint8_t chunk[1 << 16];
    size_t got;
    while ((got = std::fread(chunk, 1, sizeof(chunk), f)) > 0) buf.insert(buf.end(), chunk, chunk + got);
    std::fclose(f);
    return png_decode(buf.data(), buf.size(), out, e);
}

std::vector<uint8_t> png_encode_rgba(uint32_t w, uint32_t h, const uint8_t* rgba) {
    std::vector<uint8_t> raw;
    raw.reserve((size_t)h * (1 + (size_t)w * 4));
    for (uint32_t y = 0; y < h; ++y) {
        raw.push_back(0);
        raw.insert(raw.end(), rgba + (size_t)y * w * 4, rgba + (size_t)(y + 1) * w * 4);
    }
    std::vector<uint8_t> z = {0x78, 0x01};
    for (size_t off = 0; off < raw.size() || off == 0;) {
        const size_t len = raw.size() - off < 65535u ? raw.size() - off : 65535u;
        z.push_back(off + len >= raw.size() ? 1 : 0);
        z.push_back((uint8_t)len), z.push_back((uint8_t)(len >> 8));
        z.push_back((uint8_t)~len), z.push_back((uint8_t)(~len >> 8));
        z.insert(z.end(), raw.begin() + off, raw.begin() + off + len);
        off += len;
        if (len == 0) break;
    }
    const uint32_t ad = adler32(raw.data(), raw.size());
    put_be32(z, ad);
    std::vector<uint8_t> png = {0x89, 'P', 'N', 'G', 0x0D, 0x0A, 0x1A, 0x0A};
    auto chunk = [&](const char* type, const std::vector<uint8_t>& body) {
        put_be32(png, (uint32_t)body.size());
        const size_t at = png.size();
        png.insert(png.end(), type, type + 4);
        png.insert(png.end(), body.begin(), body.end());
        put_be32(png, crc32(png.data() + at, 4 + body.size()));
    };
    std::vector<uint8_t> ihdr;
    put_be32(ihdr, w);
    put_be32(ihdr, h);
    ihdr.push_back(8), ihdr.push_back(6), ihdr.push_back(0), ihdr.push_back(0), ihdr.push_back(0);
    chunk("IHDR", ihdr);
    chunk("IDAT", z);
    chunk("IEND", {});
    return png;
}

bool png_write_file(const std::string& path, uint32_t w, uint32_t h, const uint8_t* rgba) {
    const std::vector<uint8_t> png = png_encode_rgba(w, h, rgba);
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f) return false;
    const bool ok = std::fwrite(png.data(), 1, png.size(), f) == png.size();
    return std::fclose(f) == 0 && ok;
}

}  // namespace nerf_host
