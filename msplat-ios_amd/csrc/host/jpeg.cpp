// jpeg.cpp -- JPEG decoding for the image loaders: baseline and extended
// sequential Huffman (SOF0 / SOF1) and progressive (SOF2) 8-bit JPEG after
// ITU-T T.81, with restart intervals and any sampling factors.  The
// reference decodes every image through CoreGraphics
// (core/src/loaders/image_io.cpp:12-58); the captures its loaders read
// (COLMAP, Nerfstudio, Polycam) ship JPEG.
//
// Steps: markers -> Huffman-coded scans into per-block coefficients (all
// scans of a progressive image refine the same coefficient store) ->
// dequantisation and the 8x8 inverse DCT (separable, in double) -> chroma
// upsampling (for 2:1 factors the triangular filter that libjpeg calls
// "fancy" upsampling: each output sample weights its nearer input 3:1, the
// usual decoder behaviour; other factors replicate) -> YCbCr to RGB
// (JFIF: R = Y + 1.402 Cr', G = Y - 0.34414 Cb' - 0.71414 Cr',
// B = Y + 1.772 Cb', in 16-bit fixed point).  Arithmetic coding, 12-bit samples, lossless and
// hierarchical modes and CMYK are refused.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "input_data.hpp"

namespace {

[[noreturn]] void fail(const std::string &path, const std::string &why) {
    throw std::runtime_error("JPEG " + path + ": " + why);
}

// Zig-zag scan position k -> natural (row-major) index in the 8x8 block.
constexpr uint8_t kZigZag[64] = {0,  1,  8,  16, 9,  2,  3,  10, 17, 24, 32, 25, 18, 11, 4,  5,
                                 12, 19, 26, 33, 40, 48, 41, 34, 27, 20, 13, 6,  7,  14, 21, 28,
                                 35, 42, 49, 56, 57, 50, 43, 36, 29, 22, 15, 23, 30, 37, 44, 51,
                                 58, 59, 52, 45, 38, 31, 39, 46, 53, 60, 61, 54, 47, 55, 62, 63};

// A Huffman table in canonical form (T.81 Annex C): for each code length L,
// codes mincode[L] .. maxcode[L] map to values starting at valptr[L]; a
// 9-bit lookup resolves short codes at once.
struct Huffman {
    bool defined = false;
    uint8_t vals[256] = {};
    int32_t maxcode[18] = {}, valptr[17] = {}, mincode[17] = {};
    uint16_t fast[512] = {};  // (length << 8 | value) + 1 for codes of <= 9 bits, 0 otherwise
    // Returns false, having written nothing, when the counts do not form a
    // prefix code: canonical assignment (T.81 C.2) must keep every code of
    // length L below 2^L.
    bool build(const uint8_t counts[16], const uint8_t *v, int nv) {
        int64_t room = 1;  // codes of the current length still unassigned
        for (int len = 1; len <= 16; ++len) {
            room = 2 * room - counts[len - 1];
            if (room < 0) return false;
        }
        std::memcpy(vals, v, (size_t)nv);
        int code = 0, k = 0;
        std::memset(fast, 0, sizeof(fast));
        for (int len = 1; len <= 16; ++len) {
            valptr[len] = k;
            mincode[len] = code;
            for (int i = 0; i < counts[len - 1]; ++i, ++k, ++code)
                if (len <= 9)
                    for (int f = code << (9 - len); f < (code + 1) << (9 - len); ++f)
                        fast[f] = (uint16_t)(((len << 8) | vals[k]) + 1);
            maxcode[len] = counts[len - 1] ? code - 1 : -1;
            code <<= 1;
        }
        maxcode[17] = 0x7fffffff;
        defined = true;
        return true;
    }
};

struct Component {
    int id = 0, h = 1, v = 1, tq = 0;
    int bw = 0, bh = 0;            // blocks per line / column covering the MCUs
    std::vector<int16_t> coef;     // bw * bh blocks of 64 coefficients (natural order)
    int td = 0, ta = 0, dc_pred = 0;
    std::vector<uint8_t> plane;    // samples, (bw * 8) x (bh * 8)
};

class BitReader {
public:
    BitReader(const uint8_t *d, size_t n, size_t pos) : d_(d), n_(n), pos_(pos) {}
    size_t pos() const { return pos_; }
    // bits are taken MSB first; after a marker only zeros are supplied
    int bits(int k) {
        fill(k);
        const int v = (int)((acc_ >> (cnt_ - k)) & ((1u << k) - 1u));
        cnt_ -= k;
        return v;
    }
    int bit() { return bits(1); }
    int peek9() {
        fill(9);
        return (int)((acc_ >> (cnt_ - 9)) & 511u);
    }
    void skip(int k) { cnt_ -= k; }
    // T.81 F.2.2.1 EXTEND of a k-bit magnitude
    int receive_extend(int k) {
        if (k == 0) return 0;
        const int v = bits(k);
        return v < (1 << (k - 1)) ? v - (1 << k) + 1 : v;
    }
    int decode(const Huffman &h, const std::string &path) {
        const int f = h.fast[peek9()];
        if (f) {
            skip((f - 1) >> 8);
            return (f - 1) & 255;
        }
        int code = bits(1), len = 1;
        while (code > h.maxcode[len]) {
            code = (code << 1) | bits(1);
            if (++len > 16) fail(path, "bad Huffman code");
        }
        return h.vals[h.valptr[len] + code - h.mincode[len]];
    }
    // expects RSTn at a restart interval boundary
    void restart(const std::string &path) {
        cnt_ = 0;
        acc_ = 0;
        marker_ = false;
        while (pos_ + 1 < n_ && !(d_[pos_] == 0xFF && d_[pos_ + 1] >= 0xD0 && d_[pos_ + 1] <= 0xD7)) ++pos_;
        if (pos_ + 1 >= n_) fail(path, "missing restart marker");
        pos_ += 2;
    }

private:
    void fill(int k) {
        while (cnt_ < k) {
            uint32_t b = 0;
            if (!marker_ && pos_ < n_) {
                b = d_[pos_];
                if (b == 0xFF) {
                    const uint8_t nx = pos_ + 1 < n_ ? d_[pos_ + 1] : 0;
                    if (nx == 0x00) {
                        pos_ += 2;
                    } else {
                        marker_ = true;  // leave the marker for the parser
                        b = 0;
                    }
                } else {
                    ++pos_;
                }
            }
            acc_ = (acc_ << 8) | b;
            cnt_ += 8;
        }
    }
    const uint8_t *d_;
    size_t n_, pos_;
    uint64_t acc_ = 0;
    int cnt_ = 0;
    bool marker_ = false;
};

// 8x8 inverse DCT (T.81 A.3.3) of dequantised coefficients, in double,
// level-shifted by 128, rounded and clamped to [0, 255].
struct Idct {
    double c[8][8];  // c[x][u] = C(u)/2 cos((2x + 1) u pi / 16)
    Idct() {
        for (int x = 0; x < 8; ++x)
            for (int u = 0; u < 8; ++u)
                c[x][u] = (u == 0 ? std::sqrt(0.5) : 1.0) * 0.5 * std::cos((2 * x + 1) * u * M_PI / 16.0);
    }
    void run(const int32_t in[64], uint8_t *out, int stride) const {
        double tmp[64];
        for (int v = 0; v < 8; ++v)  // rows of coefficients -> spatial x
            for (int x = 0; x < 8; ++x) {
                double s = 0.0;
                for (int u = 0; u < 8; ++u) s += c[x][u] * in[v * 8 + u];
                tmp[v * 8 + x] = s;
            }
        for (int x = 0; x < 8; ++x)
            for (int y = 0; y < 8; ++y) {
                double s = 0.0;
                for (int v = 0; v < 8; ++v) s += c[y][v] * tmp[v * 8 + x];
                const double p = std::floor(s + 128.5);
                out[y * stride + x] = (uint8_t)std::min(255.0, std::max(0.0, p));
            }
    }
};

class Decoder {
public:
    Decoder(const std::vector<uint8_t> &f, const std::string &path) : f_(f), path_(path) {}

    Image decode() {
        const uint8_t *d = f_.data();
        const size_t n = f_.size();
        if (n < 4 || d[0] != 0xFF || d[1] != 0xD8) fail(path_, "no SOI marker");
        size_t p = 2;
        bool frame = false, done = false;
        while (!done) {
            while (p < n && d[p] != 0xFF) ++p;  // skip fill / stray bytes
            while (p < n && d[p] == 0xFF) ++p;
            if (p >= n) break;
            const uint8_t m = d[p++];
            if (m == 0xD9) {
                done = true;
                break;
            }
            if (m >= 0xD0 && m <= 0xD7) continue;
            if (p + 2 > n) fail(path_, "truncated marker");
            const size_t len = (size_t)d[p] << 8 | d[p + 1];
            if (len < 2 || p + len > n) fail(path_, "truncated segment");
            const uint8_t *s = d + p + 2;
            const size_t sl = len - 2;
            switch (m) {
                case 0xC0: case 0xC1: case 0xC2:
                    read_frame(s, sl, m == 0xC2);
                    frame = true;
                    p += len;
                    break;
                case 0xC4: read_dht(s, sl); p += len; break;
                case 0xDB: read_dqt(s, sl); p += len; break;
                case 0xDD:
                    if (sl < 2) fail(path_, "bad DRI");
                    restart_ = s[0] << 8 | s[1];
                    p += len;
                    break;
                case 0xDA:
                    if (!frame) fail(path_, "scan before frame header");
                    p = scan(s, sl, p + len);
                    break;
                case 0xEE:  // Adobe: transform flag 0 means RGB components
                    if (sl >= 12 && std::memcmp(s, "Adobe", 5) == 0) adobe_transform_ = s[11];
                    p += len;
                    break;
                default:
                    if ((m >= 0xC3 && m <= 0xCF && m != 0xC4 && m != 0xC8 && m != 0xCC) || m == 0xDE)
                        fail(path_, "unsupported coding process (arithmetic, lossless or hierarchical)");
                    p += len;  // APPn, COM, DNL and the rest
            }
        }
        if (!frame || !scanned_) fail(path_, "no image data");
        return finish();
    }

private:
    void read_dqt(const uint8_t *s, size_t n) {
        size_t i = 0;
        while (i < n) {
            const int pq = s[i] >> 4, tq = s[i] & 15;
            if (tq > 3) fail(path_, "bad quantisation table id");
            ++i;
            if (i + (pq ? 128 : 64) > n) fail(path_, "truncated quantisation table");
            for (int k = 0; k < 64; ++k) {
                qt_[tq][kZigZag[k]] = pq ? (s[i + 2 * k] << 8 | s[i + 2 * k + 1]) : s[i + k];
            }
            i += pq ? 128 : 64;
        }
    }
    void read_dht(const uint8_t *s, size_t n) {
        size_t i = 0;
        while (i < n) {
            if (i + 17 > n) fail(path_, "truncated Huffman table");
            const int tc = s[i] >> 4, th = s[i] & 15;
            if (tc > 1 || th > 3) fail(path_, "bad Huffman table id");
            int total = 0;
            for (int k = 0; k < 16; ++k) total += s[i + 1 + k];
            if (total > 256 || i + 17 + total > n) fail(path_, "bad Huffman table");
            // 8-bit samples: DC difference categories 0..11, AC magnitude
            // sizes 0..10 (T.81 F.1.2.1, F.1.2.2; Table K.3 / K.5 ranges)
            for (int k = 0; k < total; ++k) {
                const int val = s[i + 17 + k];
                if (tc ? (val & 15) > 10 : val > 11) fail(path_, "bad Huffman value");
            }
            if (!(tc ? ac_[th] : dc_[th]).build(s + i + 1, s + i + 17, total))
                fail(path_, "Huffman code lengths do not form a prefix code");
            i += 17 + total;
        }
    }
    void read_frame(const uint8_t *s, size_t n, bool progressive) {
        if (n < 6) fail(path_, "bad frame header");
        if (s[0] != 8) fail(path_, "only 8-bit samples are supported");
        height_ = s[1] << 8 | s[2];
        width_ = s[3] << 8 | s[4];
        const int nc = s[5];
        if (width_ <= 0 || height_ <= 0) fail(path_, "bad image size (DNL is not supported)");
        if ((int64_t)width_ * height_ > (int64_t)1 << 28) fail(path_, "image larger than 2^28 pixels");
        if (nc != 1 && nc != 3) fail(path_, "only 1 or 3 components are supported");
        if (n < 6 + 3 * (size_t)nc) fail(path_, "bad frame header");
        progressive_ = progressive;
        comps_.assign(nc, Component());
        hmax_ = vmax_ = 1;
        for (int c = 0; c < nc; ++c) {
            Component &k = comps_[c];
            k.id = s[6 + 3 * c];
            k.h = s[7 + 3 * c] >> 4;
            k.v = s[7 + 3 * c] & 15;
            k.tq = s[8 + 3 * c];
            if (k.h < 1 || k.h > 4 || k.v < 1 || k.v > 4 || k.tq > 3) fail(path_, "bad component");
            hmax_ = std::max(hmax_, k.h);
            vmax_ = std::max(vmax_, k.v);
        }
        // Components are upsampled by whole factors; a frame whose largest
        // sampling factor is not a multiple of every component's is refused.
        for (const Component &k : comps_)
            if (hmax_ % k.h || vmax_ % k.v) fail(path_, "non-integral chroma sampling ratio");
        mcux_ = (width_ + 8 * hmax_ - 1) / (8 * hmax_);
        mcuy_ = (height_ + 8 * vmax_ - 1) / (8 * vmax_);
        for (Component &k : comps_) {
            k.bw = mcux_ * k.h;
            k.bh = mcuy_ * k.v;
            k.coef.assign((size_t)k.bw * k.bh * 64, 0);
        }
    }

    // One scan (T.81 B.2.3, G.1): returns the file position after its data.
    size_t scan(const uint8_t *s, size_t n, size_t data_pos) {
        if (n < 1) fail(path_, "bad scan header");
        const int ns = s[0];
        if (ns < 1 || ns > 4 || n < 4 + 2 * (size_t)ns) fail(path_, "bad scan header");
        std::vector<Component *> sc;
        for (int i = 0; i < ns; ++i) {
            const int id = s[1 + 2 * i];
            Component *k = nullptr;
            for (Component &c : comps_)
                if (c.id == id) k = &c;
            if (!k) fail(path_, "scan names an unknown component");
            k->td = s[2 + 2 * i] >> 4;
            k->ta = s[2 + 2 * i] & 15;
            if (k->td > 3 || k->ta > 3) fail(path_, "bad table selector");
            sc.push_back(k);
        }
        const int ss = s[1 + 2 * ns], se = s[2 + 2 * ns], ah = s[3 + 2 * ns] >> 4, al = s[3 + 2 * ns] & 15;
        if (progressive_) {
            if (ss > se || se > 63 || (ss == 0 && se != 0) || (ss > 0 && ns != 1) || al > 13)
                fail(path_, "bad progressive scan parameters");
        } else if (ss != 0 || se != 63 || ah != 0 || al != 0) {
            fail(path_, "bad sequential scan parameters");
        }
        for (Component *k : sc) {
            k->dc_pred = 0;
            if ((!progressive_ || (ss == 0 && ah == 0)) && !dc_[k->td].defined) fail(path_, "undefined DC table");
            if ((!progressive_ || ss > 0) && !ac_[k->ta].defined && !(progressive_ && ss == 0))
                fail(path_, "undefined AC table");
        }
        BitReader br(f_.data(), f_.size(), data_pos);
        eobrun_ = 0;
        // a single-component scan covers that component's blocks of the
        // image (not of the MCUs); an interleaved one walks the MCUs
        const bool single = ns == 1;
        int units_x, units_y;
        if (single) {
            units_x = (int)((std::ceil(width_ * sc[0]->h / (double)hmax_)) + 7) / 8;
            units_y = (int)((std::ceil(height_ * sc[0]->v / (double)vmax_)) + 7) / 8;
        } else {
            units_x = mcux_;
            units_y = mcuy_;
        }
        const int64_t units = (int64_t)units_x * units_y;
        for (int64_t u = 0; u < units; ++u) {
            if (restart_ && u > 0 && u % restart_ == 0) {
                br.restart(path_);
                for (Component *k : sc) k->dc_pred = 0;
                eobrun_ = 0;
            }
            const int ux = (int)(u % units_x), uy = (int)(u / units_x);
            if (single) {
                block(br, *sc[0], ux, uy, ss, se, ah, al);
            } else {
                for (Component *k : sc)
                    for (int by = 0; by < k->v; ++by)
                        for (int bx = 0; bx < k->h; ++bx) block(br, *k, ux * k->h + bx, uy * k->v + by, ss, se, ah, al);
            }
        }
        scanned_ = true;
        // continue after the scan's entropy-coded data: at the next marker
        // other than RSTn
        size_t q = std::max(br.pos(), data_pos);
        const uint8_t *d = f_.data();
        while (q + 1 < f_.size() && !(d[q] == 0xFF && d[q + 1] != 0x00 && !(d[q + 1] >= 0xD0 && d[q + 1] <= 0xD7)))
            ++q;
        return q;
    }

    void block(BitReader &br, Component &k, int bx, int by, int ss, int se, int ah, int al) {
        int16_t *c = &k.coef[((size_t)by * k.bw + bx) * 64];
        if (!progressive_) {
            const int t = br.decode(dc_[k.td], path_);
            k.dc_pred += br.receive_extend(t);
            c[0] = (int16_t)k.dc_pred;
            for (int i = 1; i < 64;) {
                const int rs = br.decode(ac_[k.ta], path_);
                const int r = rs >> 4, sz = rs & 15;
                if (sz == 0) {
                    if (r != 15) break;  // EOB
                    i += 16;
                    continue;
                }
                i += r;
                if (i > 63) fail(path_, "coefficient index out of range");
                c[kZigZag[i++]] = (int16_t)br.receive_extend(sz);
            }
            return;
        }
        if (ss == 0) {  // DC scans (G.1.2.1)
            if (ah == 0) {
                const int t = br.decode(dc_[k.td], path_);
                k.dc_pred += br.receive_extend(t);
                c[0] = (int16_t)(k.dc_pred * (1 << al));
            } else if (br.bit()) {
                c[0] = (int16_t)(c[0] | (1 << al));
            }
            return;
        }
        if (ah == 0) {  // AC first pass (G.1.2.2)
            if (eobrun_ > 0) {
                --eobrun_;
                return;
            }
            for (int i = ss; i <= se;) {
                const int rs = br.decode(ac_[k.ta], path_);
                const int r = rs >> 4, sz = rs & 15;
                if (sz == 0) {
                    if (r < 15) {
                        eobrun_ = (1 << r) - 1;
                        if (r) eobrun_ += br.bits(r);
                        break;
                    }
                    i += 16;
                    continue;
                }
                i += r;
                if (i > 63) fail(path_, "coefficient index out of range");
                c[kZigZag[i++]] = (int16_t)(br.receive_extend(sz) * (1 << al));
            }
            return;
        }
        // AC refinement (G.1.2.3): every nonzero coefficient in the band
        // gets a correction bit; new coefficients are +-1 << al
        const int p1 = 1 << al, m1 = -(1 << al);
        int i = ss;
        if (eobrun_ == 0) {
            for (; i <= se;) {
                const int rs = br.decode(ac_[k.ta], path_);
                int r = rs >> 4;
                const int sz = rs & 15;
                int val = 0;
                if (sz) {
                    if (sz != 1) fail(path_, "bad refinement value");
                    val = br.bit() ? p1 : m1;
                } else if (r != 15) {
                    eobrun_ = 1 << r;
                    if (r) eobrun_ += br.bits(r);
                    break;  // the rest of the band is refined below
                }
                // skip r zero coefficients (refining the nonzero ones
                // passed), then place val at the next zero one
                while (i <= se) {
                    int16_t &z = c[kZigZag[i]];
                    if (z != 0) {
                        if (br.bit() && (z & p1) == 0) z = (int16_t)(z >= 0 ? z + p1 : z + m1);
                    } else {
                        if (r == 0) {
                            if (val) z = (int16_t)val;
                            ++i;
                            break;
                        }
                        --r;
                    }
                    ++i;
                }
            }
        }
        if (eobrun_ > 0) {
            for (; i <= se; ++i) {
                int16_t &z = c[kZigZag[i]];
                if (z != 0 && br.bit() && (z & p1) == 0) z = (int16_t)(z >= 0 ? z + p1 : z + m1);
            }
            --eobrun_;
        }
    }

    Image finish() {
        const Idct idct;
        for (Component &k : comps_) {
            const int pw = k.bw * 8;
            k.plane.assign((size_t)pw * k.bh * 8, 0);
            const int *q = qt_[k.tq];
            int32_t blk[64];
            for (int by = 0; by < k.bh; ++by)
                for (int bx = 0; bx < k.bw; ++bx) {
                    const int16_t *c = &k.coef[((size_t)by * k.bw + bx) * 64];
                    for (int i = 0; i < 64; ++i) blk[i] = (int32_t)c[i] * q[i];
                    idct.run(blk, &k.plane[(size_t)by * 8 * pw + bx * 8], pw);
                }
            std::vector<int16_t>().swap(k.coef);
        }
        // full-resolution samples of every component
        const int nc = (int)comps_.size();
        std::vector<std::vector<uint8_t>> full(nc);
        for (int c = 0; c < nc; ++c) full[c] = upsample(comps_[c]);
        Image img;
        img.width = width_;
        img.height = height_;
        img.data.resize((size_t)width_ * height_ * 3);
        const size_t np = (size_t)width_ * height_;
        if (nc == 1) {
            for (size_t i = 0; i < np; ++i) img.data[3 * i] = img.data[3 * i + 1] = img.data[3 * i + 2] = full[0][i] / 255.0f;
            return img;
        }
        const bool rgb = adobe_transform_ == 0 || (comps_[0].id == 'R' && comps_[1].id == 'G' && comps_[2].id == 'B');
        for (size_t i = 0; i < np; ++i) {
            const int y = full[0][i], cb = full[1][i], cr = full[2][i];
            int r, g, b;
            if (rgb) {
                r = y, g = cb, b = cr;
            } else {
                // the JFIF constants in 16-bit fixed point, rounded half up
                const long cbp = cb - 128, crp = cr - 128;
                r = clamp8(y + ((91881L * crp + 32768L) >> 16));
                g = clamp8(y + ((-22554L * cbp - 46802L * crp + 32768L) >> 16));
                b = clamp8(y + ((116130L * cbp + 32768L) >> 16));
            }
            img.data[3 * i] = r / 255.0f;
            img.data[3 * i + 1] = g / 255.0f;
            img.data[3 * i + 2] = b / 255.0f;
        }
        return img;
    }

    static int clamp8(long v) { return (int)std::min(255L, std::max(0L, v)); }

    // The component's samples at image resolution.  For 2:1 factors the
    // triangular filter: horizontally out[2i] = (3 in[i] + in[i-1] + 1) / 4,
    // out[2i+1] = (3 in[i] + in[i+1] + 2) / 4 (edges replicate); for 2:1
    // in both directions the vertical 3:1 sum first, then horizontally
    // (3 cur + neighbour + 8 or + 7) / 16.  Other ratios replicate samples.
    std::vector<uint8_t> upsample(const Component &k) const {
        const int pw = k.bw * 8, ph = k.bh * 8;
        const int fx = hmax_ / k.h, fy = vmax_ / k.v;
        std::vector<uint8_t> out((size_t)width_ * height_);
        const int cw = (width_ * k.h + hmax_ - 1) / hmax_;  // the component's own width
        auto at = [&](int x, int y) -> int {
            x = std::min(std::max(x, 0), cw - 1);
            y = std::min(std::max(y, 0), ph - 1);
            return k.plane[(size_t)y * pw + x];
        };
        if (k.h == hmax_ && k.v == vmax_) {  // full resolution: ph >= height_, pw >= width_
            for (int y = 0; y < height_; ++y)
                std::memcpy(&out[(size_t)y * width_], &k.plane[(size_t)y * pw], (size_t)width_);
        } else if (fx == 2 && fy == 1) {
            for (int y = 0; y < height_; ++y)
                for (int x = 0; x < width_; ++x) {
                    const int i = x >> 1;
                    const int cur = at(i, y);
                    out[(size_t)y * width_ + x] =
                        (x & 1) ? (uint8_t)((3 * cur + at(i + 1 < cw ? i + 1 : i, y) + 2) >> 2)
                                : (uint8_t)((3 * cur + at(i > 0 ? i - 1 : i, y) + 1) >> 2);
                }
        } else if (fx == 2 && fy == 2) {
            const int chh = (height_ * k.v + vmax_ - 1) / vmax_;  // the component's own height
            auto col = [&](int i, int y, int near) {  // 3 * cur + nearer row (edges replicate)
                const int yn = std::min(std::max(near, 0), chh - 1);
                return 3 * at(i, y) + at(i, yn);
            };
            for (int y = 0; y < height_; ++y) {
                const int j = y >> 1;
                const int near = (y & 1) ? j + 1 : j - 1;
                for (int x = 0; x < width_; ++x) {
                    const int i = x >> 1;
                    const int cur = col(i, j, near);
                    int v;
                    if (x & 1)
                        v = (3 * cur + col(i + 1 < cw ? i + 1 : i, j, near) + 7) >> 4;
                    else
                        v = (3 * cur + col(i > 0 ? i - 1 : i, j, near) + 8) >> 4;
                    out[(size_t)y * width_ + x] = (uint8_t)v;
                }
            }
        } else {
            for (int y = 0; y < height_; ++y)
                for (int x = 0; x < width_; ++x) out[(size_t)y * width_ + x] = (uint8_t)at(x / fx, y / fy);
        }
        return out;
    }

    const std::vector<uint8_t> &f_;
    const std::string &path_;
    int qt_[4][64] = {};
    Huffman dc_[4], ac_[4];
    std::vector<Component> comps_;
    int width_ = 0, height_ = 0, hmax_ = 1, vmax_ = 1, mcux_ = 0, mcuy_ = 0;
    int restart_ = 0, eobrun_ = 0, adobe_transform_ = -1;
    bool progressive_ = false, scanned_ = false;
};

}  // namespace

Image decode_jpeg(const std::vector<uint8_t> &f, const std::string &path) { return Decoder(f, path).decode(); }
