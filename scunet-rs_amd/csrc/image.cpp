// image.cpp - the PNG codec of the command-line denoiser (the reference's src/image.rs,
// which delegates to the `png` crate). Host code only; zlib does the deflate stream.
//
// Decoding follows the PNG specification (ISO/IEC 15948): chunk framing with CRC-32
// checks, IHDR, the concatenated IDAT zlib stream, the five per-row filters and Adam7
// interlacing. Only what image.rs:26-31 accepts is converted: 8-bit gray, gray+alpha,
// RGB and RGBA (alpha dropped). Encoding writes one 8-bit non-interlaced image whose
// row filters are chosen per row by the smallest sum of absolute filtered bytes.
#include "../../include/scunet_image.h"

#include <zlib.h>

#include <algorithm>
#include <cerrno>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

thread_local std::string g_err;

int fail(const std::string& m) {
    g_err = m;
    return 1;
}

const uint8_t kSig[8] = {137, 80, 78, 71, 13, 10, 26, 10};

uint32_t be32(const uint8_t* p) {
    return (uint32_t(p[0]) << 24) | (uint32_t(p[1]) << 16) | (uint32_t(p[2]) << 8) | uint32_t(p[3]);
}

void put32(std::vector<uint8_t>& o, uint32_t v) {
    o.push_back(uint8_t(v >> 24));
    o.push_back(uint8_t(v >> 16));
    o.push_back(uint8_t(v >> 8));
    o.push_back(uint8_t(v));
}

// Adam7 passes: first column, first row, column step, row step.
const int kAdam7[7][4] = {{0, 0, 8, 8}, {4, 0, 8, 8}, {0, 4, 4, 8}, {2, 0, 4, 4},
                          {0, 2, 2, 4}, {1, 0, 2, 2}, {0, 1, 1, 2}};

inline int paeth(int a, int b, int c) {
    int p = a + b - c;
    int pa = std::abs(p - a), pb = std::abs(p - b), pc = std::abs(p - c);
    if (pa <= pb && pa <= pc) return a;
    return pb <= pc ? b : c;
}

// Undo one row's filter in place; `prev` is the reconstructed row above (zeros for the
// first row of a pass), `bpp` the bytes per pixel.
bool unfilter(int type, uint8_t* cur, const uint8_t* prev, size_t n, size_t bpp) {
    switch (type) {
    case 0: return true;
    case 1:
        for (size_t i = bpp; i < n; ++i) cur[i] = uint8_t(cur[i] + cur[i - bpp]);
        return true;
    case 2:
        for (size_t i = 0; i < n; ++i) cur[i] = uint8_t(cur[i] + prev[i]);
        return true;
    case 3:
        for (size_t i = 0; i < n; ++i) {
            int a = i >= bpp ? cur[i - bpp] : 0;
            cur[i] = uint8_t(cur[i] + ((a + prev[i]) >> 1));
        }
        return true;
    case 4:
        for (size_t i = 0; i < n; ++i) {
            int a = i >= bpp ? cur[i - bpp] : 0, c = i >= bpp ? prev[i - bpp] : 0;
            cur[i] = uint8_t(cur[i] + paeth(a, prev[i], c));
        }
        return true;
    default: return false;
    }
}

// Filter one row with `type` into out (n bytes); returns the sum of |signed byte|.
uint64_t filter_row(int type, const uint8_t* cur, const uint8_t* prev, size_t n, size_t bpp, uint8_t* out) {
    uint64_t s = 0;
    for (size_t i = 0; i < n; ++i) {
        int a = i >= bpp ? cur[i - bpp] : 0, b = prev[i], c = i >= bpp ? prev[i - bpp] : 0;
        int pred = type == 0 ? 0 : type == 1 ? a : type == 2 ? b : type == 3 ? ((a + b) >> 1) : paeth(a, b, c);
        uint8_t v = uint8_t(cur[i] - pred);
        out[i] = v;
        s += uint64_t(std::abs(int(int8_t(v))));
    }
    return s;
}

std::string chunk_name(const uint8_t* p) {
    std::string s;
    for (int i = 0; i < 4; ++i) s += (p[i] >= 32 && p[i] < 127) ? char(p[i]) : '?';
    return s;
}

bool read_file(const std::string& path, std::vector<uint8_t>& b) {
    FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) {
        g_err = path + ": " + std::strerror(errno);
        return false;
    }
    uint8_t buf[1 << 16];
    size_t n;
    while ((n = std::fread(buf, 1, sizeof buf, f)) > 0) b.insert(b.end(), buf, buf + n);
    bool bad = std::ferror(f) != 0;
    std::fclose(f);
    if (bad) {
        g_err = path + ": read error";
        return false;
    }
    return true;
}

int decode(const std::string& path, float** data, size_t* oc, size_t* oh, size_t* ow) {
    std::vector<uint8_t> b;
    if (!read_file(path, b)) return 1;
    if (b.size() < 8 || std::memcmp(b.data(), kSig, 8) != 0) return fail(path + ": not a PNG file (bad signature)");
    size_t pos = 8;
    bool have_ihdr = false, have_iend = false;
    uint32_t w = 0, h = 0;
    int depth = 0, ctype = 0, interlace = 0;
    std::vector<uint8_t> idat;
    while (pos < b.size()) {
        if (b.size() - pos < 12) return fail(path + ": truncated PNG (a chunk header runs past the end)");
        uint32_t len = be32(&b[pos]);
        const uint8_t* type = &b[pos + 4];
        std::string name = chunk_name(type);
        if (len > 0x7fffffffu || b.size() - pos - 12 < len)
            return fail(path + ": truncated PNG (chunk " + name + " runs past the end)");
        const uint8_t* body = type + 4;
        uint32_t crc = uint32_t(crc32(crc32(0L, Z_NULL, 0), type, len + 4));
        if (crc != be32(body + len)) return fail(path + ": CRC mismatch in chunk " + name);
        if (!have_ihdr) {
            if (name != "IHDR" || len != 13) return fail(path + ": the first chunk is " + name + ", not IHDR");
            w = be32(body);
            h = be32(body + 4);
            depth = body[8];
            ctype = body[9];
            interlace = body[12];
            if (w == 0 || h == 0 || w > 0x7fffffffu || h > 0x7fffffffu || body[10] != 0 || body[11] != 0 ||
                interlace > 1)
                return fail(path + ": invalid IHDR");
            have_ihdr = true;
        } else if (name == "IDAT") {
            idat.insert(idat.end(), body, body + len);
        } else if (name == "IEND") {
            have_iend = true;
            break;
        } else if (name == "IHDR") {
            return fail(path + ": a second IHDR chunk");
        } else if (!(type[0] & 0x20) && name != "PLTE") {
            return fail(path + ": unknown critical chunk " + name);
        }
        pos += size_t(len) + 12;
    }
    if (!have_ihdr) return fail(path + ": truncated PNG (no IHDR)");
    int spp;   // samples per pixel
    switch (ctype) {
    case 0: spp = 1; break;
    case 2: spp = 3; break;
    case 4: spp = 2; break;
    case 6: spp = 4; break;
    case 3: return fail(path + ": unsupported colour type Indexed");
    default: return fail(path + ": invalid colour type " + std::to_string(ctype));
    }
    if (depth != 8)
        return fail(path + ": " + std::to_string(depth) + "-bit samples; this reader takes 8-bit PNGs only");
    if (!have_iend) return fail(path + ": truncated PNG (no IEND)");
    if (idat.empty()) return fail(path + ": no image data (IDAT)");
    // 2^28 pixels: beyond what the network can run on one device (about 1.6 KB of device
    // memory per pixel), and a bound on what a header can make this reader allocate.
    if (uint64_t(w) * h > (uint64_t(1) << 28))
        return fail(path + ": image too large (" + std::to_string(w) + "x" + std::to_string(h) + ")");

    // The passes' geometry and the size of the filtered stream.
    struct Pass { size_t x0, y0, dx, dy, pw, ph; };
    std::vector<Pass> passes;
    if (interlace == 0) {
        passes.push_back({0, 0, 1, 1, w, h});
    } else {
        for (auto& a : kAdam7) {
            size_t pw = w > size_t(a[0]) ? (w - a[0] + a[2] - 1) / a[2] : 0;
            size_t ph = h > size_t(a[1]) ? (h - a[1] + a[3] - 1) / a[3] : 0;
            if (pw && ph) passes.push_back({size_t(a[0]), size_t(a[1]), size_t(a[2]), size_t(a[3]), pw, ph});
        }
    }
    size_t raw_n = 0;
    for (auto& p : passes) raw_n += p.ph * (1 + p.pw * spp);
    // deflate expands at most ~1032:1, so a stream this short cannot fill the image: refuse
    // before allocating for it.
    if (idat.size() * 1032 + 64 < raw_n)
        return fail(path + ": image data ends early (" + std::to_string(idat.size()) +
                    " compressed bytes for " + std::to_string(raw_n) + ")");
    std::vector<uint8_t> raw(raw_n);

    z_stream z;
    std::memset(&z, 0, sizeof z);
    if (inflateInit(&z) != Z_OK) return fail(path + ": zlib init failed");
    size_t in_off = 0, out_off = 0;
    int zr = Z_OK;
    while (out_off < raw_n) {
        size_t in_left = idat.size() - in_off, out_left = raw_n - out_off;
        z.next_in = idat.data() + in_off;
        z.avail_in = uInt(in_left < (1u << 30) ? in_left : (1u << 30));
        z.next_out = raw.data() + out_off;
        z.avail_out = uInt(out_left < (1u << 30) ? out_left : (1u << 30));
        uInt ai = z.avail_in, ao = z.avail_out;
        zr = inflate(&z, Z_NO_FLUSH);
        in_off += ai - z.avail_in;
        out_off += ao - z.avail_out;
        if (zr == Z_STREAM_END) break;
        if (zr != Z_OK && zr != Z_BUF_ERROR) break;
        if (zr == Z_BUF_ERROR && ai == z.avail_in && ao == z.avail_out) break;   // no progress
    }
    std::string zmsg = z.msg ? z.msg : "";
    inflateEnd(&z);
    if (zr == Z_DATA_ERROR || zr == Z_MEM_ERROR || zr == Z_STREAM_ERROR || zr == Z_NEED_DICT)
        return fail(path + ": corrupt image data (zlib: " + (zmsg.empty() ? std::to_string(zr) : zmsg) + ")");
    if (out_off < raw_n)
        return fail(path + ": image data ends early (" + std::to_string(out_off) + " of " + std::to_string(raw_n) +
                    " bytes)");

    // Unfilter every pass and place its pixels.
    std::vector<uint8_t> px(size_t(w) * h * spp);
    size_t off = 0;
    for (auto& p : passes) {
        size_t rb = p.pw * spp;
        std::vector<uint8_t> zero(rb, 0);
        const uint8_t* prev = zero.data();
        for (size_t r = 0; r < p.ph; ++r) {
            uint8_t* row = raw.data() + off;
            int ft = row[0];
            if (!unfilter(ft, row + 1, prev, rb, spp))
                return fail(path + ": invalid filter type " + std::to_string(ft) + " in row " + std::to_string(r));
            size_t y = p.y0 + r * p.dy;
            if (p.dx == 1) {
                std::memcpy(&px[y * w * spp], row + 1, rb);
            } else {
                for (size_t i = 0; i < p.pw; ++i)
                    std::memcpy(&px[(y * w + p.x0 + i * p.dx) * spp], row + 1 + i * spp, spp);
            }
            prev = row + 1;
            off += 1 + rb;
        }
    }

    size_t c = (ctype == 2 || ctype == 6) ? 3 : 1, plane = size_t(w) * h;
    float* out = static_cast<float*>(std::malloc(c * plane * sizeof(float)));
    if (!out) return fail(path + ": out of host memory");
    for (size_t i = 0; i < plane; ++i)
        for (size_t ch = 0; ch < c; ++ch) out[ch * plane + i] = float(px[i * spp + ch]) / 255.0f;
    *data = out;
    *oc = c;
    *oh = h;
    *ow = w;
    return 0;
}

// image.rs:58-64: clamp to [0, 1] (NaN passes through the clamp), scale, add one half and
// convert with saturation (NaN to 0), in float arithmetic with no fused multiply-add.
uint8_t quantize(float v) {
#pragma clang fp contract(off)
    v = v < 0.0f ? 0.0f : (v > 1.0f ? 1.0f : v);
    float s = v * 255.0f;
    s = s + 0.5f;
    if (!(s >= 0.0f)) return 0;
    return s >= 255.0f ? 255 : uint8_t(s);
}

void chunk(std::vector<uint8_t>& o, const char* type, const uint8_t* body, size_t n) {
    put32(o, uint32_t(n));
    size_t at = o.size();
    o.insert(o.end(), type, type + 4);
    if (n) o.insert(o.end(), body, body + n);
    put32(o, uint32_t(crc32(crc32(0L, Z_NULL, 0), &o[at], uInt(n + 4))));
}

int encode(const std::string& path, const float* data, size_t c, size_t h, size_t w) {
    if (c != 1 && c != 3) return fail("cannot write " + std::to_string(c) + " channels as PNG");
    if (h == 0 || w == 0 || h > 0x7fffffffu || w > 0x7fffffffu || uint64_t(w) * h > (uint64_t(1) << 34))
        return fail(path + ": cannot write a " + std::to_string(h) + "x" + std::to_string(w) + " image");
    size_t rb = w * c, plane = h * w;
    std::vector<uint8_t> cur(rb), prev(rb, 0), cand(rb), best(rb), raw;
    raw.reserve(h * (rb + 1));
    for (size_t y = 0; y < h; ++y) {
        for (size_t x = 0; x < w; ++x)
            for (size_t ch = 0; ch < c; ++ch) cur[x * c + ch] = quantize(data[ch * plane + y * w + x]);
        uint64_t best_s = UINT64_MAX;
        int best_t = 0;
        for (int t = 0; t < 5; ++t) {
            uint64_t s = filter_row(t, cur.data(), prev.data(), rb, c, cand.data());
            if (s < best_s) {
                best_s = s;
                best_t = t;
                best.swap(cand);
            }
        }
        raw.push_back(uint8_t(best_t));
        raw.insert(raw.end(), best.begin(), best.end());
        prev.swap(cur);
    }
    uLongf zn = compressBound(uLong(raw.size()));
    std::vector<uint8_t> z(zn);
    if (compress2(z.data(), &zn, raw.data(), uLong(raw.size()), 6) != Z_OK) return fail(path + ": zlib failed");

    std::vector<uint8_t> o(kSig, kSig + 8);
    uint8_t ihdr[13];
    std::vector<uint8_t> hb;
    put32(hb, uint32_t(w));
    put32(hb, uint32_t(h));
    std::memcpy(ihdr, hb.data(), 8);
    ihdr[8] = 8;                        // bit depth
    ihdr[9] = c == 3 ? 2 : 0;           // RGB or grayscale
    ihdr[10] = ihdr[11] = ihdr[12] = 0; // deflate, adaptive filtering, no interlace
    chunk(o, "IHDR", ihdr, 13);
    const size_t kIdat = size_t(1) << 20;
    for (size_t at = 0; at < zn; at += kIdat) chunk(o, "IDAT", z.data() + at, std::min(kIdat, size_t(zn) - at));
    chunk(o, "IEND", nullptr, 0);

    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f) return fail(path + ": " + std::strerror(errno));
    bool ok = std::fwrite(o.data(), 1, o.size(), f) == o.size();
    ok = (std::fclose(f) == 0) && ok;
    if (!ok) return fail(path + ": write error");
    return 0;
}

}  // namespace

extern "C" {

// No C++ exception leaves the C ABI: an allocation that fails (a header claiming a huge
// image, say) is reported like any other error.
int scunet_image_read(const char* path, float** data, size_t* c, size_t* h, size_t* w) {
    g_err.clear();
    if (!path || !data || !c || !h || !w) return fail("scunet_image_read: null argument");
    *data = nullptr;
    try {
        return decode(path, data, c, h, w);
    } catch (const std::bad_alloc&) {
        return fail(std::string(path) + ": out of host memory");
    } catch (const std::exception& e) {
        return fail(std::string(path) + ": " + e.what());
    }
}

void scunet_image_free(float* data) { std::free(data); }

int scunet_image_write(const char* path, const float* data, size_t c, size_t h, size_t w) {
    g_err.clear();
    if (!path || !data) return fail("scunet_image_write: null argument");
    try {
        return encode(path, data, c, h, w);
    } catch (const std::bad_alloc&) {
        return fail(std::string(path) + ": out of host memory");
    } catch (const std::exception& e) {
        return fail(std::string(path) + ": " + e.what());
    }
}

const char* scunet_image_error(void) { return g_err.c_str(); }

}  // extern "C"
