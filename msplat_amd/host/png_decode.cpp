// png_decode.cpp — PNG image decoding for the dataset's target images.
//
// The reference decodes images with CoreGraphics (imreadRGB,
// image_io.cpp:12-50): the image is drawn into an 8-bit RGBX buffer and each
// channel becomes byte / 255 in fp32.  This file decodes PNG files with
// zlib (the only image library whose headers this platform ships) into the
// same float RGB: non-interlaced PNGs of every colour type (grey, RGB,
// palette, grey + alpha, RGBA) at bit depths 1-16.  16-bit samples keep their
// high byte; sub-byte grey levels are scaled to 0..255 as the PNG
// specification's sample depth scaling prescribes (v * 255 / (2^d - 1)).
// Transparency: the reference draws the image into a zero-filled context
// without alpha (kCGImageAlphaNoneSkipLast), i.e. source-over black, so a
// sample with alpha a (from the alpha channel or a tRNS chunk) becomes
// round(c * a / 255), and fully transparent pixels are black.
#include "png_decode.hpp"

#include <zlib.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <vector>

namespace msplat {

namespace {

uint32_t be32(const uint8_t* p) {
    return (uint32_t)p[0] << 24 | (uint32_t)p[1] << 16 | (uint32_t)p[2] << 8 | (uint32_t)p[3];
}

std::vector<uint8_t> read_file(const std::string& path) {
    FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) throw std::runtime_error("cannot open image " + path);
    std::vector<uint8_t> buf;
    uint8_t tmp[1 << 16];
    size_t got;
    while ((got = std::fread(tmp, 1, sizeof(tmp), f)) > 0) buf.insert(buf.end(), tmp, tmp + got);
    std::fclose(f);
    return buf;
}

int paeth(int a, int b, int c) {
    const int p = a + b - c;
    const int pa = p > a ? p - a : a - p, pb = p > b ? p - b : b - p, pc = p > c ? p - c : c - p;
    if (pa <= pb && pa <= pc) return a;
    return pb <= pc ? b : c;
}

}  // namespace

bool is_png_file(const std::string& path) {
    FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) return false;
    uint8_t sig[8] = {};
    const size_t n = std::fread(sig, 1, 8, f);
    std::fclose(f);
    static const uint8_t kSig[8] = {0x89, 'P', 'N', 'G', 0x0D, 0x0A, 0x1A, 0x0A};
    return n == 8 && std::memcmp(sig, kSig, 8) == 0;
}

DecodedImage decode_png(const std::string& path) {
    const std::vector<uint8_t> file = read_file(path);
    static const uint8_t kSig[8] = {0x89, 'P', 'N', 'G', 0x0D, 0x0A, 0x1A, 0x0A};
    if (file.size() < 8 || std::memcmp(file.data(), kSig, 8) != 0)
        throw std::runtime_error(path + ": not a PNG file");
    uint32_t W = 0, H = 0;
    int depth = 0, ctype = -1, interlace = 0;
    std::vector<uint8_t> palette, trns, idat;
    size_t pos = 8;
    bool seen_end = false;
    while (pos + 12 <= file.size()) {
        const uint32_t len = be32(&file[pos]);
        if (len > file.size() - pos - 12) throw std::runtime_error(path + ": truncated PNG chunk");
        const uint8_t* type = &file[pos + 4];
        const uint8_t* data = &file[pos + 8];
        if (std::memcmp(type, "IHDR", 4) == 0) {
            if (len < 13) throw std::runtime_error(path + ": bad IHDR");
            W = be32(data);
            H = be32(data + 4);
            depth = data[8];
            ctype = data[9];
            interlace = data[12];
        } else if (std::memcmp(type, "PLTE", 4) == 0) {
            palette.assign(data, data + len);
        } else if (std::memcmp(type, "tRNS", 4) == 0) {
            trns.assign(data, data + len);
        } else if (std::memcmp(type, "IDAT", 4) == 0) {
            idat.insert(idat.end(), data, data + len);
        } else if (std::memcmp(type, "IEND", 4) == 0) {
            seen_end = true;
            break;
        }
        pos += 12 + (size_t)len;
    }
    if (!seen_end || W == 0 || H == 0) throw std::runtime_error(path + ": incomplete PNG");
    if (interlace != 0) throw std::runtime_error(path + ": interlaced PNG is not supported");
    int channels;
    switch (ctype) {
        case 0: channels = 1; break;   // grey
        case 2: channels = 3; break;   // RGB
        case 3: channels = 1; break;   // palette index
        case 4: channels = 2; break;   // grey + alpha
        case 6: channels = 4; break;   // RGBA
        default: throw std::runtime_error(path + ": unknown PNG colour type");
    }
    const bool depth_ok = depth == 8 || depth == 16 ||
                          ((ctype == 0 || ctype == 3) && (depth == 1 || depth == 2 || depth == 4));
    if (!depth_ok || (ctype == 3 && depth == 16)) throw std::runtime_error(path + ": bad PNG bit depth");
    if (ctype == 3 && (palette.empty() || palette.size() % 3 != 0))
        throw std::runtime_error(path + ": palette image without PLTE");
    if ((uint64_t)W * H > (uint64_t)1 << 30) throw std::runtime_error(path + ": image too large");
    const size_t bits_per_px = (size_t)channels * depth;
    const size_t stride = (W * bits_per_px + 7) / 8;   // bytes per scanline (no filter byte)
    const size_t bpp = std::max<size_t>(1, bits_per_px / 8);
    std::vector<uint8_t> raw((stride + 1) * H);
    // zlib counts bytes in 32-bit fields: inflate in pieces of at most
    // UINT_MAX bytes of input and output (16-bit RGBA images reach 8 GiB)
    z_stream zs{};
    if (inflateInit(&zs) != Z_OK) throw std::runtime_error("zlib init failed");
    const size_t kPiece = 0xFFFFFFFFu;
    size_t in_left = idat.size(), out_left = raw.size();
    zs.next_in = idat.data();
    zs.next_out = raw.data();
    int zr = Z_OK;
    while (zr == Z_OK) {
        if (zs.avail_in == 0 && in_left > 0) {
            zs.avail_in = (uInt)std::min(in_left, kPiece);
            in_left -= zs.avail_in;
        }
        if (zs.avail_out == 0 && out_left > 0) {
            zs.avail_out = (uInt)std::min(out_left, kPiece);
            out_left -= zs.avail_out;
        }
        const uInt before_in = zs.avail_in, before_out = zs.avail_out;
        zr = inflate(&zs, in_left == 0 ? Z_FINISH : Z_NO_FLUSH);
        if (zr == Z_BUF_ERROR && (zs.avail_in != before_in || zs.avail_out != before_out)) zr = Z_OK;
        if (zr == Z_OK && zs.avail_out == 0 && out_left == 0) break;   // image data complete
        if (zr == Z_OK && zs.avail_in == 0 && in_left == 0 && zs.avail_out != 0) {
            zr = Z_DATA_ERROR;   // stream ended early
        }
    }
    const size_t produced = raw.size() - out_left - zs.avail_out;
    inflateEnd(&zs);
    if ((zr != Z_STREAM_END && zr != Z_OK) || produced != raw.size())
        throw std::runtime_error(path + ": corrupt PNG image data");
    // Undo the per-scanline filters in place.
    std::vector<uint8_t> prev(stride, 0);
    for (uint32_t y = 0; y < H; ++y) {
        uint8_t* row = &raw[(size_t)y * (stride + 1)];
        const int f = row[0];
        uint8_t* cur = row + 1;
        for (size_t i = 0; i < stride; ++i) {
            const int a = i >= bpp ? cur[i - bpp] : 0, b = prev[i], c = i >= bpp ? prev[i - bpp] : 0;
            int v = cur[i];
            switch (f) {
                case 0: break;
                case 1: v += a; break;
                case 2: v += b; break;
                case 3: v += (a + b) >> 1; break;
                case 4: v += paeth(a, b, c); break;
                default: throw std::runtime_error(path + ": bad PNG filter type");
            }
            cur[i] = (uint8_t)v;
        }
        std::memcpy(prev.data(), cur, stride);
    }
    // tRNS (PNG spec 11.3.2.1): palette alphas (entries past the chunk are
    // opaque), or one grey / RGB sample value, at the image's bit depth, that
    // marks fully transparent pixels
    const bool key_grey = ctype == 0 && trns.size() >= 2;
    const bool key_rgb = ctype == 2 && trns.size() >= 6;
    const uint32_t kg = key_grey ? ((uint32_t)trns[0] << 8 | trns[1]) : 0;
    const uint32_t kr = key_rgb ? ((uint32_t)trns[0] << 8 | trns[1]) : 0;
    const uint32_t kgn = key_rgb ? ((uint32_t)trns[2] << 8 | trns[3]) : 0;
    const uint32_t kb = key_rgb ? ((uint32_t)trns[4] << 8 | trns[5]) : 0;
    DecodedImage img;
    img.width = (int)W;
    img.height = (int)H;
    img.rgb.resize((size_t)W * H * 3);
    const int maxv = (1 << depth) - 1;
    for (uint32_t y = 0; y < H; ++y) {
        const uint8_t* cur = &raw[(size_t)y * (stride + 1) + 1];
        for (uint32_t x = 0; x < W; ++x) {
            uint8_t px[3];
            int alpha = 255;
            if (depth < 8) {   // grey or palette, packed from the high bits
                const size_t bit = (size_t)x * depth;
                const int v = (cur[bit / 8] >> (8 - depth - (int)(bit % 8))) & maxv;
                if (ctype == 3) {
                    if ((size_t)v * 3 + 2 >= palette.size()) throw std::runtime_error(path + ": palette index out of range");
                    for (int c = 0; c < 3; ++c) px[c] = palette[(size_t)v * 3 + c];
                    if ((size_t)v < trns.size()) alpha = trns[v];
                } else {
                    px[0] = px[1] = px[2] = (uint8_t)(v * 255 / maxv);
                    if (key_grey && (uint32_t)v == kg) alpha = 0;
                }
            } else {
                const size_t step = (size_t)channels * (depth / 8);
                const uint8_t* s = cur + (size_t)x * step;   // high byte first (16-bit)
                const size_t hb = depth / 8;
                // a whole sample at the image's depth (for the tRNS key)
                auto sample = [&](int c) -> uint32_t {
                    return hb == 2 ? ((uint32_t)s[2 * c] << 8 | s[2 * c + 1]) : s[c];
                };
                if (ctype == 3) {
                    const size_t v = s[0];
                    if (v * 3 + 2 >= palette.size()) throw std::runtime_error(path + ": palette index out of range");
                    for (int c = 0; c < 3; ++c) px[c] = palette[v * 3 + c];
                    if (v < trns.size()) alpha = trns[v];
                } else if (channels <= 2) {
                    px[0] = px[1] = px[2] = s[0];
                    if (channels == 2) alpha = s[hb];
                    else if (key_grey && sample(0) == kg) alpha = 0;
                } else {
                    for (int c = 0; c < 3; ++c) px[c] = s[c * hb];
                    if (channels == 4) alpha = s[3 * hb];
                    else if (key_rgb && sample(0) == kr && sample(1) == kgn && sample(2) == kb) alpha = 0;
                }
            }
            if (alpha != 255)   // source-over black, rounded to the nearest level
                for (int c = 0; c < 3; ++c) px[c] = (uint8_t)((px[c] * alpha + 127) / 255);
            float* o = &img.rgb[((size_t)y * W + x) * 3];
            for (int c = 0; c < 3; ++c) o[c] = px[c] / 255.0f;
        }
    }
    return img;
}

}  // namespace msplat
