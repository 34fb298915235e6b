// image_io.cpp -- image decoding / encoding, box-filter resize lives in
// input_data.cpp, and Brown-Conrady undistortion
// (core/src/loaders/image_io.cpp of the reference, which decodes through
// CoreGraphics).  Decoders here: PNG (bit depth 1-16, grey / grey+alpha /
// RGB / RGBA / palette, non-interlaced and Adam7) through zlib, binary
// PPM/PGM, and JPEG (jpeg.cpp).  Output is float32 RGB in [0,1]; alpha is
// dropped.
#include <zlib.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <fstream>
#include <stdexcept>
#include <string>

#include "input_data.hpp"

namespace {

std::vector<uint8_t> read_file(const std::string &path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot open image: " + path);
    return std::vector<uint8_t>((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
}

uint32_t be32(const uint8_t *p) { return (uint32_t)p[0] << 24 | (uint32_t)p[1] << 16 | (uint32_t)p[2] << 8 | p[3]; }

int paeth(int a, int b, int c) {
    const int p = a + b - c, pa = std::abs(p - a), pb = std::abs(p - b), pc = std::abs(p - c);
    return (pa <= pb && pa <= pc) ? a : (pb <= pc ? b : c);
}

// Reverses the PNG scanline filters of one (sub)image in place; returns the
// number of bytes consumed.
size_t unfilter(uint8_t *data, size_t avail, int w, int h, int bpp_bits, std::vector<uint8_t> &out) {
    const size_t stride = ((size_t)w * bpp_bits + 7) / 8;
    const int bpp = std::max(1, bpp_bits / 8);
    if (avail < (stride + 1) * h) throw std::runtime_error("PNG: truncated image data");
    out.assign(stride * h, 0);
    for (int y = 0; y < h; ++y) {
        const uint8_t ft = data[y * (stride + 1)];
        const uint8_t *src = data + y * (stride + 1) + 1;
        uint8_t *row = out.data() + y * stride;
        const uint8_t *prev = y ? row - stride : nullptr;
        for (size_t i = 0; i < stride; ++i) {
            const int a = i >= (size_t)bpp ? row[i - bpp] : 0, b = prev ? prev[i] : 0;
            const int c = (prev && i >= (size_t)bpp) ? prev[i - bpp] : 0;
            int v = src[i];
            switch (ft) {
                case 0: break;
                case 1: v += a; break;
                case 2: v += b; break;
                case 3: v += (a + b) >> 1; break;
                case 4: v += paeth(a, b, c); break;
                default: throw std::runtime_error("PNG: bad filter type");
            }
            row[i] = (uint8_t)v;
        }
    }
    return (stride + 1) * h;
}

Image decode_png(const std::vector<uint8_t> &f, const std::string &path) {
    static const uint8_t sig[8] = {137, 80, 78, 71, 13, 10, 26, 10};
    if (f.size() < 33 || std::memcmp(f.data(), sig, 8) != 0) throw std::runtime_error("not a PNG: " + path);
    int w = 0, h = 0, depth = 0, ctype = 0, interlace = 0;
    std::vector<uint8_t> idat, palette;
    size_t p = 8;
    while (p + 12 <= f.size()) {
        const uint32_t len = be32(&f[p]);
        const char *type = (const char *)&f[p + 4];
        const uint8_t *d = &f[p + 8];
        if (p + 12 + (size_t)len > f.size()) throw std::runtime_error("PNG: truncated chunk in " + path);
        if (!std::memcmp(type, "IHDR", 4)) {
            w = (int)be32(d);
            h = (int)be32(d + 4);
            depth = d[8];
            ctype = d[9];
            interlace = d[12];
        } else if (!std::memcmp(type, "PLTE", 4)) {
            palette.assign(d, d + len);
        } else if (!std::memcmp(type, "IDAT", 4)) {
            idat.insert(idat.end(), d, d + len);
        } else if (!std::memcmp(type, "IEND", 4)) {
            break;
        }
        p += 12 + len;
    }
    const int chans = ctype == 0 ? 1 : ctype == 2 ? 3 : ctype == 3 ? 1 : ctype == 4 ? 2 : ctype == 6 ? 4 : 0;
    if (w <= 0 || h <= 0 || chans == 0 || !(depth == 1 || depth == 2 || depth == 4 || depth == 8 || depth == 16))
        throw std::runtime_error("PNG: unsupported header in " + path);
    const int bpp_bits = chans * depth;
    // inflate
    std::vector<uint8_t> raw;
    {
        z_stream zs{};
        if (inflateInit(&zs) != Z_OK) throw std::runtime_error("PNG: zlib init failed");
        zs.next_in = idat.data();
        zs.avail_in = (uInt)idat.size();
        uint8_t buf[1 << 16];
        int rc;
        do {
            zs.next_out = buf;
            zs.avail_out = sizeof(buf);
            rc = inflate(&zs, Z_NO_FLUSH);
            if (rc != Z_OK && rc != Z_STREAM_END) {
                inflateEnd(&zs);
                throw std::runtime_error("PNG: corrupt image data in " + path);
            }
            raw.insert(raw.end(), buf, buf + (sizeof(buf) - zs.avail_out));
        } while (rc != Z_STREAM_END);
        inflateEnd(&zs);
    }
    Image img;
    img.width = w;
    img.height = h;
    img.data.assign((size_t)w * h * 3, 0.0f);
    const float maxv = (float)((1 << depth) - 1);
    auto sample = [&](const uint8_t *row, int x, int ch) -> int {  // channel ch of pixel x in an unfiltered row
        if (depth == 8) return row[x * chans + ch];
        if (depth == 16) return (row[2 * (x * chans + ch)] << 8) | row[2 * (x * chans + ch) + 1];
        const int bit = (x * chans + ch) * depth;
        return (row[bit >> 3] >> (8 - depth - (bit & 7))) & ((1 << depth) - 1);
    };
    auto store = [&](const std::vector<uint8_t> &px, int sw, int sh, int ox, int oy, int dx, int dy) {
        const size_t stride = ((size_t)sw * bpp_bits + 7) / 8;
        for (int y = 0; y < sh; ++y) {
            const uint8_t *row = px.data() + y * stride;
            for (int x = 0; x < sw; ++x) {
                float *o = &img.data[((size_t)(oy + y * dy) * w + ox + x * dx) * 3];
                if (ctype == 3) {
                    const int idx = sample(row, x, 0);
                    if ((size_t)(3 * idx + 2) >= palette.size()) throw std::runtime_error("PNG: palette index");
                    for (int c = 0; c < 3; ++c) o[c] = palette[3 * idx + c] / 255.0f;
                } else if (chans <= 2) {
                    const float v = sample(row, x, 0) / maxv;
                    o[0] = o[1] = o[2] = v;
                } else {
                    for (int c = 0; c < 3; ++c) o[c] = sample(row, x, c) / maxv;
                }
            }
        }
    };
    std::vector<uint8_t> px;
    if (interlace == 0) {
        unfilter(raw.data(), raw.size(), w, h, bpp_bits, px);
        store(px, w, h, 0, 0, 1, 1);
    } else {
        static const int sx[7] = {0, 4, 0, 2, 0, 1, 0}, sy[7] = {0, 0, 4, 0, 2, 0, 1};
        static const int dx[7] = {8, 8, 4, 4, 2, 2, 1}, dy[7] = {8, 8, 8, 4, 4, 2, 2};
        size_t off = 0;
        for (int pass = 0; pass < 7; ++pass) {
            const int pw = (w - sx[pass] + dx[pass] - 1) / dx[pass], ph = (h - sy[pass] + dy[pass] - 1) / dy[pass];
            if (pw <= 0 || ph <= 0) continue;
            off += unfilter(raw.data() + off, raw.size() - off, pw, ph, bpp_bits, px);
            store(px, pw, ph, sx[pass], sy[pass], dx[pass], dy[pass]);
        }
    }
    return img;
}

Image decode_pnm(const std::vector<uint8_t> &f, const std::string &path) {
    size_t p = 2;
    auto next_int = [&]() {
        while (p < f.size()) {
            if (f[p] == '#') {
                while (p < f.size() && f[p] != '\n') ++p;
            } else if (std::isspace(f[p])) {
                ++p;
            } else {
                break;
            }
        }
        int v = 0;
        bool any = false;
        while (p < f.size() && std::isdigit(f[p])) {
            v = v * 10 + (f[p++] - '0');
            any = true;
        }
        if (!any) throw std::runtime_error("PNM: bad header in " + path);
        return v;
    };
    const bool rgb = f[1] == '6';
    const int w = next_int(), h = next_int(), maxv = next_int();
    ++p;  // single whitespace after maxval
    const int bytes = maxv > 255 ? 2 : 1, chans = rgb ? 3 : 1;
    if (w <= 0 || h <= 0 || maxv <= 0 || p + (size_t)w * h * chans * bytes > f.size())
        throw std::runtime_error("PNM: truncated " + path);
    Image img;
    img.width = w;
    img.height = h;
    img.data.resize((size_t)w * h * 3);
    for (size_t i = 0; i < (size_t)w * h; ++i)
        for (int c = 0; c < 3; ++c) {
            const size_t k = (i * chans + (rgb ? c : 0)) * bytes + p;
            const int v = bytes == 2 ? (f[k] << 8 | f[k + 1]) : f[k];
            img.data[3 * i + c] = (float)v / (float)maxv;
        }
    return img;
}

void put32(std::vector<uint8_t> &o, uint32_t v) {
    for (int s = 24; s >= 0; s -= 8) o.push_back((uint8_t)(v >> s));
}

void chunk(std::vector<uint8_t> &o, const char *type, const std::vector<uint8_t> &d) {
    put32(o, (uint32_t)d.size());
    const size_t at = o.size();
    o.insert(o.end(), type, type + 4);
    o.insert(o.end(), d.begin(), d.end());
    put32(o, (uint32_t)crc32(0, o.data() + at, (uInt)(d.size() + 4)));
}

// Inverse radial-tangential model by fixed-point iteration (20 steps).
void undistort_point(float xd, float yd, float k1, float k2, float p1, float p2, float k3, float &xu, float &yu) {
    xu = xd;
    yu = yd;
    for (int it = 0; it < 20; ++it) {
        const float r2 = xu * xu + yu * yu, radial = 1.0f + r2 * (k1 + r2 * (k2 + r2 * k3));
        const float tx = 2.0f * p1 * xu * yu + p2 * (r2 + 2.0f * xu * xu);
        const float ty = p1 * (r2 + 2.0f * yu * yu) + 2.0f * p2 * xu * yu;
        xu = (xd - tx) / radial;
        yu = (yd - ty) / radial;
    }
}

void distort_point(float x, float y, float k1, float k2, float p1, float p2, float k3, float &xd, float &yd) {
    const float r2 = x * x + y * y, radial = 1.0f + r2 * (k1 + r2 * (k2 + r2 * k3));
    xd = x * radial + 2.0f * p1 * x * y + p2 * (r2 + 2.0f * x * x);
    yd = y * radial + p1 * (r2 + 2.0f * y * y) + 2.0f * p2 * x * y;
}

}  // namespace

// jpeg.cpp
Image decode_jpeg(const std::vector<uint8_t> &f, const std::string &path);

Image imreadRGB(const std::string &path) {
    const std::vector<uint8_t> f = read_file(path);
    if (f.size() >= 8 && f[0] == 137 && f[1] == 'P' && f[2] == 'N' && f[3] == 'G') return decode_png(f, path);
    if (f.size() >= 2 && f[0] == 'P' && (f[1] == '6' || f[1] == '5')) return decode_pnm(f, path);
    if (f.size() >= 3 && f[0] == 0xFF && f[1] == 0xD8) return decode_jpeg(f, path);
    throw std::runtime_error("unrecognised image format: " + path);
}

void imwriteRGB(const std::string &path, const Image &img) {
    std::vector<uint8_t> raw;
    raw.reserve((size_t)(img.width * 3 + 1) * img.height);
    for (int y = 0; y < img.height; ++y) {
        raw.push_back(0);
        for (int x = 0; x < img.width * 3; ++x) {
            const float v = std::min(std::max(img.data[(size_t)y * img.width * 3 + x], 0.0f), 1.0f);
            raw.push_back((uint8_t)std::lround(v * 255.0f));
        }
    }
    uLongf zlen = compressBound((uLong)raw.size());
    std::vector<uint8_t> z(zlen);
    if (compress2(z.data(), &zlen, raw.data(), (uLong)raw.size(), 6) != Z_OK)
        throw std::runtime_error("PNG: compression failed");
    z.resize(zlen);
    std::vector<uint8_t> o = {137, 80, 78, 71, 13, 10, 26, 10};
    std::vector<uint8_t> ihdr;
    put32(ihdr, (uint32_t)img.width);
    put32(ihdr, (uint32_t)img.height);
    ihdr.insert(ihdr.end(), {8, 2, 0, 0, 0});
    chunk(o, "IHDR", ihdr);
    chunk(o, "IDAT", z);
    chunk(o, "IEND", {});
    std::ofstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot write " + path);
    f.write((const char *)o.data(), (std::streamsize)o.size());
}

// Brown-Conrady undistortion onto the same intrinsics, cropped to the
// largest axis-aligned rectangle without invalid border (image_io.cpp:
// 226-340): the crop edges are the innermost undistorted positions of the
// four image borders, sampled at 200 points each; pixels are resampled
// bilinearly from the distorted image.
UndistortResult undistortImage(const Image &src, float fx, float fy, float cx, float cy, float k1, float k2,
                               float p1, float p2, float k3) {
    const int w = src.width, h = src.height, ns = 200;
    float top = -1e9f, bottom = 1e9f, left = -1e9f, right = 1e9f;
    for (int i = 0; i < ns; ++i) {
        const float t = (float)i / (ns - 1);
        float xu, yu;
        undistort_point((t * w - cx) / fx, (0.0f - cy) / fy, k1, k2, p1, p2, k3, xu, yu);
        top = std::max(top, yu * fy + cy);
        undistort_point((t * w - cx) / fx, ((float)(h - 1) - cy) / fy, k1, k2, p1, p2, k3, xu, yu);
        bottom = std::min(bottom, yu * fy + cy);
        undistort_point((0.0f - cx) / fx, (t * h - cy) / fy, k1, k2, p1, p2, k3, xu, yu);
        left = std::max(left, xu * fx + cx);
        undistort_point(((float)(w - 1) - cx) / fx, (t * h - cy) / fy, k1, k2, p1, p2, k3, xu, yu);
        right = std::min(right, xu * fx + cx);
    }
    int rx = std::max(0, (int)std::ceil(left)), ry = std::max(0, (int)std::ceil(top));
    int rw = std::min(w, (int)std::floor(right)) - rx, rh = std::min(h, (int)std::floor(bottom)) - ry;
    if (rw <= 0 || rh <= 0) {
        rx = ry = 0;
        rw = w;
        rh = h;
    }
    UndistortResult r;
    r.image.width = rw;
    r.image.height = rh;
    r.image.data.resize((size_t)rw * rh * 3);
    for (int oy = 0; oy < rh; ++oy)
        for (int ox = 0; ox < rw; ++ox) {
            float xd, yd;
            distort_point(((float)(ox + rx) - cx) / fx, ((float)(oy + ry) - cy) / fy, k1, k2, p1, p2, k3, xd, yd);
            const float sx = xd * fx + cx, sy = yd * fy + cy;
            const float fx0 = std::floor(sx), fy0 = std::floor(sy);
            const int x0 = std::clamp((int)fx0, 0, w - 1), x1 = std::clamp((int)fx0 + 1, 0, w - 1);
            const int y0 = std::clamp((int)fy0, 0, h - 1), y1 = std::clamp((int)fy0 + 1, 0, h - 1);
            const float ax = sx - fx0, ay = sy - fy0;
            float *o = &r.image.data[((size_t)oy * rw + ox) * 3];
            for (int c = 0; c < 3; ++c) {
                const float t0 = src.data[((size_t)y0 * w + x0) * 3 + c] * (1 - ax) + src.data[((size_t)y0 * w + x1) * 3 + c] * ax;
                const float t1 = src.data[((size_t)y1 * w + x0) * 3 + c] * (1 - ax) + src.data[((size_t)y1 * w + x1) * 3 + c] * ax;
                o[c] = t0 * (1 - ay) + t1 * ay;
            }
        }
    r.fx = fx;
    r.fy = fy;
    r.cx = cx - rx;
    r.cy = cy - ry;
    r.width = rw;
    r.height = rh;
    return r;
}
