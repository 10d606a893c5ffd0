// jpeg_decode.cpp — JPEG decoding of the dataset's target images.
//
// The reference decodes every image through CoreGraphics (imreadRGB,
// image_io.cpp:12-50); its own datasets are JPEG (COLMAP scenes such as
// mipnerf360's *.JPG).  This file decodes the JPEG process of ITU-T T.81 /
// ISO 10918-1 that such files use, written from the standard:
//   * baseline and extended sequential DCT (SOF0 / SOF1, 8-bit samples) and
//     progressive DCT (SOF2) with spectral selection and successive
//     approximation (T.81 G.1.2), Huffman entropy coding (T.81 F.2, G.1.2);
//   * 1 (grey) or 3 components with any sampling factors 1..4, restart
//     intervals (DRI / RSTn), 8- and 16-bit quantisation tables;
//   * 3-component images are YCbCr (JFIF) unless an Adobe APP14 segment says
//     the samples are RGB (transform 0).
// Pixels: the inverse DCT is the Loeffler-Ligtenberg-Moschytz factorisation
// (ICASSP 1989) in fixed point (rotation constants scaled by 2^13,
// two extra bits of precision between the column and the row pass, the
// results rounded and clamped to 0..255), chroma planes sampled at half the
// rate are interpolated with the triangular 3:1 filter (the "fancy"
// upsampling of the Independent JPEG Group's library, rounding biases
// alternating between neighbouring outputs), and YCbCr becomes RGB with the
// JFIF matrix (R = Y + 1.402 Cr', G = Y - 0.34414 Cb' - 0.71414 Cr',
// B = Y + 1.772 Cb') in 16-bit fixed point.  These are the methods of the
// libjpeg family that most decoders (Pillow among them) use by default, so
// the decoded samples agree with theirs; CoreGraphics' own decoder is closed
// and may differ in the last bit of a sample.  Arithmetic coding, 12-bit
// samples, lossless and hierarchical JPEG and CMYK are rejected with a clear
// error.
#include "jpeg_decode.hpp"

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

namespace msplat {

namespace {

[[noreturn]] void fail(const std::string& path, const std::string& what) {
    throw std::runtime_error(path + ": " + what);
}

std::vector<uint8_t> read_all(const std::string& path) {
    FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) throw std::runtime_error("cannot open image " + path);
    std::vector<uint8_t> buf;
    uint8_t tmp[1 << 16];
    size_t got;
    while ((got = std::fread(tmp, 1, sizeof(tmp), f)) > 0) buf.insert(buf.end(), tmp, tmp + got);
    std::fclose(f);
    return buf;
}

// Zig-zag scan position -> natural (row-major) coefficient index (T.81 A.3.6).
constexpr uint8_t kZigzag[64] = {
    0,  1,  8,  16, 9,  2,  3,  10, 17, 24, 32, 25, 18, 11, 4,  5,  12, 19, 26, 33, 40, 48,
    41, 34, 27, 20, 13, 6,  7,  14, 21, 28, 35, 42, 49, 56, 57, 50, 43, 36, 29, 22, 15, 23,
    30, 37, 44, 51, 58, 59, 52, 45, 38, 31, 39, 46, 53, 60, 61, 54, 47, 55, 62, 63};

// A Huffman table (T.81 C, F.2.2.3): codes of each length are consecutive;
// a 9-bit lookup decodes the short codes in one step.
struct Huffman {
    bool present = false;
    uint8_t sym[256] = {};
    int32_t maxcode[18] = {};     // largest code of each length, -1 if none
    int32_t valptr[17] = {};      // index in sym of the first code of each length
    int32_t mincode[17] = {};
    uint16_t fast[512] = {};      // (length << 8) | symbol, 0 if longer than 9 bits
};

void build_huffman(Huffman& h, const uint8_t counts[16], const uint8_t* syms, int nsym) {
    std::memcpy(h.sym, syms, (size_t)nsym);
    int code = 0, k = 0;
    std::fill(std::begin(h.fast), std::end(h.fast), (uint16_t)0);
    for (int len = 1; len <= 16; ++len) {
        h.valptr[len] = k;
        h.mincode[len] = code;
        for (int i = 0; i < counts[len - 1]; ++i, ++k, ++code) {
            if (len <= 9) {
                const int pad = 9 - len;
                for (int f = 0; f < (1 << pad); ++f)
                    h.fast[(code << pad) | f] = (uint16_t)((len << 8) | h.sym[k]);
            }
        }
        h.maxcode[len] = counts[len - 1] ? code - 1 : -1;
        code <<= 1;
    }
    h.maxcode[17] = 0x7FFFFFFF;
    h.present = true;
}

// Entropy-coded segment reader: bytes with 0xFF00 stuffing removed; a marker
// ends the data (zero bits are read past it, as T.81 F.2.2.5 allows for the
// padding of the last byte).
struct BitReader {
    const uint8_t* p;
    const uint8_t* end;
    uint64_t acc = 0;
    int nbits = 0;
    bool hit_marker = false;
    bool exhausted = false;   // the file ended inside the entropy-coded data

    void fill() {
        while (nbits <= 56) {
            uint32_t b = 0;
            if (!hit_marker && p >= end) exhausted = true;
            if (!hit_marker && p < end) {
                b = *p;
                if (b == 0xFF) {
                    const uint32_t nx = p + 1 < end ? p[1] : 0xD9;
                    if (nx == 0x00) {
                        p += 2;
                    } else {
                        hit_marker = true;   // leave the marker for the caller
                        b = 0;
                    }
                } else {
                    ++p;
                }
            }
            acc |= (uint64_t)b << (56 - nbits);
            nbits += 8;
        }
    }
    uint32_t peek(int n) {
        if (nbits < n) fill();
        return (uint32_t)(acc >> (64 - n));
    }
    void skip(int n) {
        acc <<= n;
        nbits -= n;
    }
    uint32_t bits(int n) {
        if (n == 0) return 0;
        const uint32_t v = peek(n);
        skip(n);
        return v;
    }
    int bit() { return (int)bits(1); }
    // The next marker after byte alignment (RSTn expected).
    void reset_at_marker() {
        acc = 0;
        nbits = 0;
        hit_marker = false;
    }
};

int decode_huff(BitReader& br, const Huffman& h, const std::string& path) {
    const uint32_t look = br.peek(9);
    const uint16_t f = h.fast[look];
    if (f) {
        br.skip(f >> 8);
        return f & 0xFF;
    }
    uint32_t code = br.peek(16);
    for (int len = 10; len <= 16; ++len) {
        const int32_t c = (int32_t)(code >> (16 - len));
        if (c <= h.maxcode[len]) {
            br.skip(len);
            return h.sym[h.valptr[len] + c - h.mincode[len]];
        }
    }
    fail(path, "corrupt JPEG data (bad Huffman code)");
}

// EXTEND (T.81 F.2.2.1): the s-bit magnitude category v as a signed value.
inline int extend(uint32_t v, int s) {
    return s == 0 ? 0 : ((int)v < (1 << (s - 1)) ? (int)v - (1 << s) + 1 : (int)v);
}

struct Component {
    int id = 0, h = 1, v = 1, tq = 0;
    int bw = 0, bh = 0;            // blocks per row / column in the MCU-padded grid
    int dw = 0, dh = 0;            // samples of the downsampled plane (ceil(W h / Hmax), ...)
    int td = 0, ta = 0;            // Huffman tables of the current scan
    int dc_pred = 0;
    std::vector<int16_t> coef;     // bw * bh blocks of 64 coefficients, natural order
};

// Loeffler-Ligtenberg-Moschytz 8-point IDCT in fixed point.
constexpr int CB = 13, P1 = 2;   // constant bits, extra bits between the passes
constexpr int32_t C0298 = 2446, C0390 = 3196, C0541 = 4433, C0765 = 6270, C0899 = 7373,
                  C1175 = 9633, C1501 = 12299, C1847 = 15137, C1961 = 16069, C2053 = 16819,
                  C2562 = 20995, C3072 = 25172;   // round(c * 2^13) of the rotation constants

// One 1-D transform of in[0..7] (stride s) into 8 values scaled by 2^CB,
// in 64-bit arithmetic (dequantised coefficients of 16-bit tables reach
// 2^27 before the constants multiply them).
inline void idct8(const int64_t* in, int s, int64_t* out) {
    int64_t z2 = in[2 * s], z3 = in[6 * s];
    int64_t z1 = (z2 + z3) * C0541;
    int64_t t2 = z1 - z3 * C1847;
    int64_t t3 = z1 + z2 * C0765;
    z2 = in[0];
    z3 = in[4 * s];
    int64_t t0 = (z2 + z3) * (1 << CB);
    int64_t t1 = (z2 - z3) * (1 << CB);
    const int64_t e10 = t0 + t3, e13 = t0 - t3, e11 = t1 + t2, e12 = t1 - t2;
    t0 = in[7 * s];
    t1 = in[5 * s];
    t2 = in[3 * s];
    t3 = in[1 * s];
    z1 = t0 + t3;
    z2 = t1 + t2;
    z3 = t0 + t2;
    int64_t z4 = t1 + t3;
    const int64_t z5 = (z3 + z4) * C1175;
    t0 *= C0298;
    t1 *= C2053;
    t2 *= C3072;
    t3 *= C1501;
    z1 *= -C0899;
    z2 *= -C2562;
    z3 = z3 * -C1961 + z5;
    z4 = z4 * -C0390 + z5;
    t0 += z1 + z3;
    t1 += z2 + z4;
    t2 += z2 + z3;
    t3 += z1 + z4;
    out[0] = e10 + t3;
    out[7] = e10 - t3;
    out[1] = e11 + t2;
    out[6] = e11 - t2;
    out[2] = e12 + t1;
    out[5] = e12 - t1;
    out[3] = e13 + t0;
    out[4] = e13 - t0;
}

// Dequantised block -> 8x8 samples (level-shifted by 128, clamped) into dst
// with row stride ds.
void idct_block(const int16_t* coef, const uint16_t* q, uint8_t* dst, int ds) {
    int64_t in[64], ws[64], tmp[8];
    for (int i = 0; i < 64; ++i) in[i] = (int64_t)coef[i] * (int64_t)q[i];
    for (int c = 0; c < 8; ++c) {   // columns: descale to 2^P1
        idct8(in + c, 8, tmp);
        for (int r = 0; r < 8; ++r) ws[r * 8 + c] = (tmp[r] + (1 << (CB - P1 - 1))) >> (CB - P1);
    }
    for (int r = 0; r < 8; ++r) {   // rows: the rounding half enters with the DC term
        int64_t row[8];
        for (int c = 0; c < 8; ++c) row[c] = ws[r * 8 + c];
        row[0] += 1 << (P1 + 2);
        idct8(row, 1, tmp);
        for (int c = 0; c < 8; ++c) {
            const int64_t v = (tmp[c] >> (CB + P1 + 3)) + 128;
            dst[r * ds + c] = (uint8_t)(v < 0 ? 0 : v > 255 ? 255 : v);
        }
    }
}

struct Decoder {
    std::string path;
    const uint8_t* data;
    size_t size;
    size_t pos = 0;
    int W = 0, H = 0, ncomp = 0, hmax = 1, vmax = 1, mcux = 0, mcuy = 0;
    bool progressive = false;
    int restart = 0;
    bool adobe = false;
    int adobe_transform = -1;
    bool jfif = false;
    uint16_t qt[4][64] = {};
    bool qt_ok[4] = {};
    Huffman hdc[4], hac[4];
    std::vector<Component> comp;
    int eobrun = 0;

    uint16_t u16(size_t at) const {
        if (at + 2 > size) fail(path, "truncated JPEG file");
        return (uint16_t)(data[at] << 8 | data[at + 1]);
    }

    void read_dqt(size_t at, size_t len) {
        size_t p = at, e = at + len;
        while (p < e) {
            const int pq = data[p] >> 4, tq = data[p] & 15;
            ++p;
            if (tq > 3 || pq > 1) fail(path, "bad quantisation table");
            if (p + (pq ? 128 : 64) > e) fail(path, "truncated quantisation table");
            for (int k = 0; k < 64; ++k) {
                const uint16_t v = pq ? (uint16_t)(data[p + 2 * k] << 8 | data[p + 2 * k + 1]) : data[p + k];
                qt[tq][kZigzag[k]] = v;
            }
            p += pq ? 128 : 64;
            qt_ok[tq] = true;
        }
    }

    void read_dht(size_t at, size_t len) {
        size_t p = at, e = at + len;
        while (p < e) {
            if (p + 17 > e) fail(path, "truncated Huffman table");
            const int tc = data[p] >> 4, th = data[p] & 15;
            if (tc > 1 || th > 3) fail(path, "bad Huffman table");
            uint8_t counts[16];
            int n = 0;
            for (int i = 0; i < 16; ++i) {
                counts[i] = data[p + 1 + i];
                n += counts[i];
            }
            if (n > 256 || p + 17 + n > e) fail(path, "bad Huffman table");
            build_huffman(tc ? hac[th] : hdc[th], counts, data + p + 17, n);
            p += 17 + n;
        }
    }

    void read_sof(size_t at, size_t len, int type) {
        if (type == 3 || type > 3) fail(path, "lossless / hierarchical / arithmetic-coded JPEG is not supported");
        if (len < 6) fail(path, "bad frame header");
        if (data[at] != 8) fail(path, "only 8-bit JPEG samples are supported");
        H = u16(at + 1);
        W = u16(at + 3);
        ncomp = data[at + 5];
        if (W <= 0 || H <= 0) fail(path, "JPEG without a size in its frame header is not supported");
        if (ncomp != 1 && ncomp != 3) fail(path, "JPEG with " + std::to_string(ncomp) + " components is not supported");
        if (len < 6 + 3 * (size_t)ncomp) fail(path, "bad frame header");
        progressive = type == 2;
        comp.assign(ncomp, Component{});
        for (int i = 0; i < ncomp; ++i) {
            Component& c = comp[i];
            c.id = data[at + 6 + 3 * i];
            c.h = data[at + 7 + 3 * i] >> 4;
            c.v = data[at + 7 + 3 * i] & 15;
            c.tq = data[at + 8 + 3 * i];
            if (c.h < 1 || c.h > 4 || c.v < 1 || c.v > 4 || c.tq > 3) fail(path, "bad component parameters");
            hmax = std::max(hmax, c.h);
            vmax = std::max(vmax, c.v);
        }
        if ((int64_t)W * H > (int64_t)1 << 30) fail(path, "image too large");
        mcux = (W + 8 * hmax - 1) / (8 * hmax);
        mcuy = (H + 8 * vmax - 1) / (8 * vmax);
        for (Component& c : comp) {
            c.bw = mcux * c.h;
            c.bh = mcuy * c.v;
            c.dw = (W * c.h + hmax - 1) / hmax;
            c.dh = (H * c.v + vmax - 1) / vmax;
            c.coef.assign((size_t)c.bw * c.bh * 64, 0);
        }
    }

    // Decoding of one block's coefficients in the current scan.
    void block_baseline(BitReader& br, Component& c, int16_t* blk) {
        const Huffman& dc = hdc[c.td];
        const Huffman& ac = hac[c.ta];
        if (!dc.present || !ac.present) fail(path, "scan uses an undefined Huffman table");
        const int s = decode_huff(br, dc, path);
        if (s > 11) fail(path, "corrupt JPEG data (DC category)");
        c.dc_pred += extend(br.bits(s), s);
        blk[0] = (int16_t)c.dc_pred;
        for (int k = 1; k < 64;) {
            const int rs = decode_huff(br, ac, path);
            const int r = rs >> 4, sz = rs & 15;
            if (sz == 0) {
                if (r != 15) break;   // EOB
                k += 16;
                continue;
            }
            k += r;
            if (k > 63) fail(path, "corrupt JPEG data (AC run)");
            blk[kZigzag[k]] = (int16_t)extend(br.bits(sz), sz);
            ++k;
        }
    }

    void block_dc_first(BitReader& br, Component& c, int16_t* blk, int al) {
        const Huffman& dc = hdc[c.td];
        if (!dc.present) fail(path, "scan uses an undefined Huffman table");
        const int s = decode_huff(br, dc, path);
        if (s > 11) fail(path, "corrupt JPEG data (DC category)");
        c.dc_pred += extend(br.bits(s), s);
        blk[0] = (int16_t)(c.dc_pred * (1 << al));
    }

    void block_dc_refine(BitReader& br, int16_t* blk, int al) {
        if (br.bit()) blk[0] = (int16_t)(blk[0] | (1 << al));
    }

    void block_ac_first(BitReader& br, Component& c, int16_t* blk, int ss, int se, int al) {
        if (eobrun > 0) {
            --eobrun;
            return;
        }
        const Huffman& ac = hac[c.ta];
        if (!ac.present) fail(path, "scan uses an undefined Huffman table");
        for (int k = ss; k <= se;) {
            const int rs = decode_huff(br, ac, path);
            const int r = rs >> 4, sz = rs & 15;
            if (sz == 0) {
                if (r < 15) {   // EOBr: this block and 2^r - 1 + bits more end here
                    eobrun = (1 << r) - 1 + (int)br.bits(r);
                    break;
                }
                k += 16;
                continue;
            }
            k += r;
            if (k > se) fail(path, "corrupt JPEG data (AC run)");
            blk[kZigzag[k]] = (int16_t)(extend(br.bits(sz), sz) * (1 << al));
            ++k;
        }
    }

    // Successive approximation of AC coefficients (T.81 G.1.2.3): nonzero
    // coefficients get a correction bit, new ones are +-1 << al.
    void block_ac_refine(BitReader& br, Component& c, int16_t* blk, int ss, int se, int al) {
        const int p1 = 1 << al, m1 = -1 * (1 << al);
        int k = ss;
        if (eobrun <= 0) {
            const Huffman& ac = hac[c.ta];
            if (!ac.present) fail(path, "scan uses an undefined Huffman table");
            for (; k <= se;) {
                const int rs = decode_huff(br, ac, path);
                int r = rs >> 4;
                const int sz = rs & 15;
                int val = 0;
                if (sz == 0) {
                    if (r < 15) {
                        eobrun = (1 << r) + (int)br.bits(r);
                        break;
                    }
                    // ZRL: sixteen zero-history coefficients are skipped
                } else {
                    if (sz != 1) fail(path, "corrupt JPEG data (refinement size)");
                    val = br.bit() ? p1 : m1;
                }
                for (; k <= se; ++k) {
                    int16_t& co = blk[kZigzag[k]];
                    if (co != 0) {
                        if (br.bit() && (co & p1) == 0) co = (int16_t)(co >= 0 ? co + p1 : co + m1);
                    } else {
                        if (r == 0) {
                            if (val) co = (int16_t)val;
                            ++k;
                            break;
                        }
                        --r;
                    }
                }
            }
        }
        if (eobrun > 0) {   // the rest of the band: correction bits of the nonzero ones
            for (; k <= se; ++k) {
                int16_t& co = blk[kZigzag[k]];
                if (co != 0 && br.bit() && (co & p1) == 0) co = (int16_t)(co >= 0 ? co + p1 : co + m1);
            }
            --eobrun;
        }
    }

    // One scan (SOS header at `at`); returns the position after its data.
    size_t scan(size_t at, size_t len) {
        const int ns = data[at];
        if (ns < 1 || ns > 4 || len < 4 + 2 * (size_t)ns) fail(path, "bad scan header");
        std::vector<Component*> sc;
        for (int i = 0; i < ns; ++i) {
            const int cid = data[at + 1 + 2 * i];
            Component* c = nullptr;
            for (Component& x : comp)
                if (x.id == cid) c = &x;
            if (!c) fail(path, "scan names an unknown component");
            c->td = data[at + 2 + 2 * i] >> 4;
            c->ta = data[at + 2 + 2 * i] & 15;
            if (c->td > 3 || c->ta > 3) fail(path, "bad scan header");
            sc.push_back(c);
        }
        const size_t q = at + 1 + 2 * ns;
        const int ss = data[q], se = data[q + 1], ah = data[q + 2] >> 4, al = data[q + 2] & 15;
        if (progressive) {
            if (ss > se || se > 63 || (ss == 0 && se != 0) || (ss > 0 && ns != 1) || al > 13)
                fail(path, "bad progressive scan parameters");
        } else if (ss != 0 || se != 63 || ah != 0 || al != 0) {
            fail(path, "bad sequential scan parameters");
        }
        for (Component* c : sc) c->dc_pred = 0;
        eobrun = 0;
        BitReader br{data + at + len, data + size};
        // Units of the scan: interleaved MCUs, or the component's own blocks
        // in raster order over its unpadded block grid (T.81 A.2.2-A.2.3).
        const bool inter = ns > 1;
        int64_t units;
        int ubw = 0, ubh = 0;
        if (inter) {
            units = (int64_t)mcux * mcuy;
        } else {
            ubw = (sc[0]->dw + 7) / 8;
            ubh = (sc[0]->dh + 7) / 8;
            units = (int64_t)ubw * ubh;
        }
        int since_rst = 0, next_rst = 0;
        for (int64_t u = 0; u < units; ++u) {
            if (restart && since_rst == restart) {
                // byte-align and expect RSTn
                const uint8_t* p = br.p;
                while (p + 1 < data + size && !(p[0] == 0xFF && p[1] >= 0xD0 && p[1] <= 0xD7)) ++p;
                if (p + 1 >= data + size) fail(path, "missing restart marker");
                if (p[1] != 0xD0 + next_rst) fail(path, "restart markers out of order");
                next_rst = (next_rst + 1) & 7;
                br.p = p + 2;
                br.reset_at_marker();
                for (Component* c : sc) c->dc_pred = 0;
                eobrun = 0;
                since_rst = 0;
            }
            ++since_rst;
            if (inter) {
                const int mx = (int)(u % mcux), my = (int)(u / mcux);
                for (Component* c : sc)
                    for (int by = 0; by < c->v; ++by)
                        for (int bx = 0; bx < c->h; ++bx) {
                            const int gx = mx * c->h + bx, gy = my * c->v + by;
                            unit(br, *c, &c->coef[((size_t)gy * c->bw + gx) * 64], ss, se, ah, al);
                        }
            } else {
                Component* c = sc[0];
                const int gx = (int)(u % ubw), gy = (int)(u / ubw);
                unit(br, *c, &c->coef[((size_t)gy * c->bw + gx) * 64], ss, se, ah, al);
            }
        }
        // the scan's data ends at the next marker other than RSTn; a file
        // that ends inside it is truncated (zeros were decoded past its end)
        if (br.exhausted) fail(path, "truncated JPEG data");
        const uint8_t* p = br.p;
        while (p + 1 < data + size && !(p[0] == 0xFF && p[1] != 0x00 && !(p[1] >= 0xD0 && p[1] <= 0xD7))) ++p;
        return (size_t)(p - data);
    }

    void unit(BitReader& br, Component& c, int16_t* blk, int ss, int se, int ah, int al) {
        if (!progressive) {
            block_baseline(br, c, blk);
        } else if (ss == 0) {
            if (ah == 0) block_dc_first(br, c, blk, al);
            else block_dc_refine(br, blk, al);
        } else if (ah == 0) {
            block_ac_first(br, c, blk, ss, se, al);
        } else {
            block_ac_refine(br, c, blk, ss, se, al);
        }
    }

    void parse() {
        if (size < 4 || data[0] != 0xFF || data[1] != 0xD8) fail(path, "not a JPEG file");
        pos = 2;
        bool frame = false, any_scan = false;
        while (true) {
            while (pos < size && data[pos] != 0xFF) ++pos;   // tolerate fill before a marker
            while (pos < size && data[pos] == 0xFF) ++pos;
            if (pos >= size) {
                if (any_scan) break;   // EOI missing after complete data
                fail(path, "truncated JPEG file");
            }
            const int m = data[pos++];
            if (m == 0xD9) break;                        // EOI
            if (m >= 0xD0 && m <= 0xD7) continue;        // stray RSTn
            if (m == 0x01) continue;                     // TEM
            const size_t len = u16(pos);
            if (len < 2 || pos + len > size) fail(path, "truncated JPEG segment");
            const size_t at = pos + 2, body = len - 2;
            if (m == 0xC0 || m == 0xC1 || m == 0xC2) {
                if (frame) fail(path, "more than one frame");
                read_sof(at, body, m - 0xC0);
                frame = true;
            } else if ((m >= 0xC3 && m <= 0xCF) && m != 0xC4 && m != 0xC8 && m != 0xCC) {
                fail(path, "lossless / hierarchical / arithmetic-coded JPEG is not supported");
            } else if (m == 0xC4) {
                read_dht(at, body);
            } else if (m == 0xCC) {
                fail(path, "arithmetic-coded JPEG is not supported");
            } else if (m == 0xDB) {
                read_dqt(at, body);
            } else if (m == 0xDD) {
                if (body < 2) fail(path, "bad restart interval");
                restart = u16(at);
            } else if (m == 0xDA) {
                if (!frame) fail(path, "scan before the frame header");
                pos = scan(at, body);
                any_scan = true;
                continue;
            } else if (m == 0xE0) {
                if (body >= 5 && std::memcmp(data + at, "JFIF\0", 5) == 0) jfif = true;
            } else if (m == 0xEE) {
                if (body >= 12 && std::memcmp(data + at, "Adobe", 5) == 0) {
                    adobe = true;
                    adobe_transform = data[at + 11];
                }
            }
            pos += len;
        }
        if (!frame || !any_scan) fail(path, "JPEG without image data");
        for (const Component& c : comp)
            if (!qt_ok[c.tq]) fail(path, "component uses an undefined quantisation table");
    }

    // The component's samples as a dw x dh plane.
    std::vector<uint8_t> plane(const Component& c) const {
        const int pw = c.bw * 8;
        std::vector<uint8_t> full((size_t)pw * c.bh * 8);
        for (int by = 0; by < c.bh; ++by)
            for (int bx = 0; bx < c.bw; ++bx)
                idct_block(&c.coef[((size_t)by * c.bw + bx) * 64], qt[c.tq],
                           &full[((size_t)by * 8) * pw + bx * 8], pw);
        std::vector<uint8_t> out((size_t)c.dw * c.dh);
        for (int y = 0; y < c.dh; ++y) std::memcpy(&out[(size_t)y * c.dw], &full[(size_t)y * pw], (size_t)c.dw);
        return out;
    }

    // The plane at full resolution (W x H): triangular interpolation for 2:1
    // horizontal and / or vertical ratios, replication otherwise.
    std::vector<uint8_t> upsample(const Component& c, const std::vector<uint8_t>& p) const {
        const int fx = hmax / c.h, fy = vmax / c.v;
        const bool exact = hmax % c.h == 0 && vmax % c.v == 0;
        if (!exact) fail(path, "non-integral chroma sampling ratio");
        const int dw = c.dw, dh = c.dh;
        if (fx == 1 && fy == 1) return p;
        std::vector<uint8_t> out((size_t)W * H);
        if ((fx == 2 || fx == 1) && (fy == 2 || fy == 1)) {
            const int ow = dw * fx;
            std::vector<uint8_t> row((size_t)ow);
            for (int oy = 0; oy < H; ++oy) {
                const int y = oy / fy;
                // vertical 3:1 sums (or the row itself times 4 without vertical interpolation)
                const int ny = fy == 2 ? (oy % 2 == 0 ? std::max(y - 1, 0) : std::min(y + 1, dh - 1)) : y;
                const uint8_t* r0 = &p[(size_t)y * dw];
                const uint8_t* r1 = &p[(size_t)ny * dw];
                if (fx == 2) {
                    if (fy == 2) {
                        // column sums 3 * this + other row, then 3:1 across columns; rounding
                        // biases 8 / 7 on the left / right output of each input column
                        auto cs = [&](int x) { return 3 * (int)r0[x] + (int)r1[x]; };
                        if (dw == 1) {
                            const int s = cs(0);
                            row[0] = (uint8_t)((4 * s + 8) >> 4);
                            row[1] = (uint8_t)((4 * s + 7) >> 4);
                        } else {
                            for (int x = 0; x < dw; ++x) {
                                const int s = cs(x);
                                row[2 * x] = (uint8_t)(x == 0 ? (4 * s + 8) >> 4 : (3 * s + cs(x - 1) + 8) >> 4);
                                row[2 * x + 1] =
                                    (uint8_t)(x == dw - 1 ? (4 * s + 7) >> 4 : (3 * s + cs(x + 1) + 7) >> 4);
                            }
                        }
                    } else {
                        // 3:1 across columns, biases 1 / 2; the image's edge columns are copied
                        for (int x = 0; x < dw; ++x) {
                            const int s = r0[x];
                            row[2 * x] = (uint8_t)(x == 0 ? s : (3 * s + r0[x - 1] + 1) >> 2);
                            row[2 * x + 1] = (uint8_t)(x == dw - 1 ? s : (3 * s + r0[x + 1] + 2) >> 2);
                        }
                    }
                } else {
                    // vertical 3:1 only, biases 1 (upper output row) / 2 (lower)
                    const int bias = oy % 2 == 0 ? 1 : 2;
                    for (int x = 0; x < dw; ++x) row[x] = (uint8_t)((3 * (int)r0[x] + (int)r1[x] + bias) >> 2);
                }
                std::memcpy(&out[(size_t)oy * W], row.data(), (size_t)W);
            }
            return out;
        }
        for (int oy = 0; oy < H; ++oy)
            for (int ox = 0; ox < W; ++ox) out[(size_t)oy * W + ox] = p[(size_t)(oy / fy) * dw + ox / fx];
        return out;
    }

    DecodedImage finish() {
        DecodedImage img;
        img.width = W;
        img.height = H;
        img.rgb.resize((size_t)W * H * 3);
        std::vector<std::vector<uint8_t>> full(ncomp);
        for (int i = 0; i < ncomp; ++i) full[i] = upsample(comp[i], plane(comp[i]));
        if (ncomp == 1) {
            for (size_t i = 0; i < (size_t)W * H; ++i) {
                const float v = full[0][i] / 255.0f;
                img.rgb[3 * i] = img.rgb[3 * i + 1] = img.rgb[3 * i + 2] = v;
            }
            return img;
        }
        // RGB samples: Adobe transform 0, or no JFIF marker and component
        // ids 'R', 'G', 'B'
        const bool rgb = (adobe && adobe_transform == 0) ||
                         (!jfif && !adobe && comp[0].id == 'R' && comp[1].id == 'G' && comp[2].id == 'B');
        if (rgb) {
            for (size_t i = 0; i < (size_t)W * H; ++i)
                for (int c = 0; c < 3; ++c) img.rgb[3 * i + c] = full[c][i] / 255.0f;
            return img;
        }
        // JFIF YCbCr -> RGB in 16-bit fixed point: f(x) = round(x 2^16)
        constexpr int32_t kCrR = 91881, kCbB = 116130, kCrG = 46802, kCbG = 22554, kHalf = 1 << 15;
        for (size_t i = 0; i < (size_t)W * H; ++i) {
            const int y = full[0][i], cb = (int)full[1][i] - 128, cr = (int)full[2][i] - 128;
            const int r = y + ((kCrR * cr + kHalf) >> 16);
            const int g = y + ((-kCbG * cb + kHalf - kCrG * cr) >> 16);
            const int b = y + ((kCbB * cb + kHalf) >> 16);
            img.rgb[3 * i] = std::min(std::max(r, 0), 255) / 255.0f;
            img.rgb[3 * i + 1] = std::min(std::max(g, 0), 255) / 255.0f;
            img.rgb[3 * i + 2] = std::min(std::max(b, 0), 255) / 255.0f;
        }
        return img;
    }
};

}  // namespace

bool is_jpeg_file(const std::string& path) {
    FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) return false;
    uint8_t sig[3] = {};
    const size_t n = std::fread(sig, 1, 3, f);
    std::fclose(f);
    return n == 3 && sig[0] == 0xFF && sig[1] == 0xD8 && sig[2] == 0xFF;
}

DecodedImage decode_jpeg(const std::string& path) {
    const std::vector<uint8_t> file = read_all(path);
    Decoder d;
    d.path = path;
    d.data = file.data();
    d.size = file.size();
    d.parse();
    return d.finish();
}

}  // namespace msplat
