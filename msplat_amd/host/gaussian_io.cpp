// gaussian_io.cpp — PLY / .splat scene files (core/src/loaders/
// save_gaussians.cpp).  Layouts and value conversions are documented in
// gaussian_io.hpp.
#include "gaussian_io.hpp"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <numeric>
#include <stdexcept>

namespace msplat {

namespace {

constexpr double SH_C0 = 0.28209479177387814;   // 1 / (2 sqrt(pi))
constexpr int64_t ROWS_PER_WRITE = 1 << 16;

void check_sizes(const HostGaussians& g) {
    const size_t n = (size_t)g.n;
    if (g.n < 0 || g.means.size() != 3 * n || g.scales.size() != 3 * n || g.quats.size() != 4 * n ||
        g.f_dc.size() != 3 * n || g.f_rest.size() != (size_t)g.rest_bases * 3 * n ||
        g.opacities.size() != n)
        throw std::runtime_error("gaussian arrays do not match the gaussian count");
}

float world_pos(const HostGaussians& g, const Crs& crs, int64_t i, int j) {
    const float m = g.means[3 * i + j];
    return crs.keep ? (m / crs.scale + crs.translation[j]) : m;
}

uint8_t to_byte(float v) { return v == v ? (uint8_t)v : (uint8_t)0; }
uint8_t to_byte(double v) { return v == v ? (uint8_t)v : (uint8_t)0; }

}  // namespace

void save_gaussian_ply(const std::string& path, const HostGaussians& g, const Crs& crs, int step) {
    check_sizes(g);
    std::ofstream o(path, std::ios::binary);
    if (!o.is_open()) throw std::runtime_error("Cannot open PLY file for writing: " + path);
    const int num_dc = 3, num_fr = g.rest_bases * 3;
    o << "ply\nformat binary_little_endian 1.0\n";
    o << "comment msplat v" << step << "\n";
    o << "element vertex " << g.n << "\n";
    o << "property float x\nproperty float y\nproperty float z\n";
    o << "property float nx\nproperty float ny\nproperty float nz\n";
    for (int i = 0; i < num_dc; ++i) o << "property float f_dc_" << i << "\n";
    for (int i = 0; i < num_fr; ++i) o << "property float f_rest_" << i << "\n";
    o << "property float opacity\n";
    o << "property float scale_0\nproperty float scale_1\nproperty float scale_2\n";
    o << "property float rot_0\nproperty float rot_1\nproperty float rot_2\nproperty float rot_3\n";
    o << "end_header\n";
    const int per_row = 3 + 3 + num_dc + num_fr + 1 + 3 + 4;
    std::vector<float> rows;
    for (int64_t r0 = 0; r0 < g.n; r0 += ROWS_PER_WRITE) {
        const int64_t r1 = std::min(g.n, r0 + ROWS_PER_WRITE);
        rows.assign((size_t)(r1 - r0) * per_row, 0.f);
        for (int64_t i = r0; i < r1; ++i) {
            float* row = rows.data() + (size_t)(i - r0) * per_row;
            int c = 0;
            for (int j = 0; j < 3; ++j) row[c++] = world_pos(g, crs, i, j);
            c += 3;   // normals stay zero
            for (int j = 0; j < num_dc; ++j) row[c++] = g.f_dc[3 * i + j];
            // [K-1, 3] -> [3, K-1]
            for (int ch = 0; ch < 3; ++ch)
                for (int b = 0; b < g.rest_bases; ++b)
                    row[c++] = g.f_rest[((size_t)i * g.rest_bases + b) * 3 + ch];
            row[c++] = g.opacities[i];
            for (int j = 0; j < 3; ++j) {
                const float s = g.scales[3 * i + j];
                row[c++] = crs.keep ? std::log(std::exp(s) / crs.scale) : s;
            }
            for (int j = 0; j < 4; ++j) row[c++] = g.quats[4 * i + j];
        }
        o.write(reinterpret_cast<const char*>(rows.data()), (std::streamsize)(rows.size() * 4));
    }
    if (!o) throw std::runtime_error("write failed: " + path);
}

void save_gaussian_splat(const std::string& path, const HostGaussians& g, const Crs& crs) {
    check_sizes(g);
    std::ofstream o(path, std::ios::binary);
    if (!o.is_open()) throw std::runtime_error("Cannot open .splat file for writing: " + path);
    std::vector<float> key((size_t)g.n);
    for (int64_t i = 0; i < g.n; ++i) {
        float s = std::exp(g.scales[3 * i]) + std::exp(g.scales[3 * i + 1]) +
                  std::exp(g.scales[3 * i + 2]);
        if (crs.keep) s /= crs.scale;
        key[i] = s / (1.0f + std::exp(-g.opacities[i]));
    }
    std::vector<int64_t> idx((size_t)g.n);
    std::iota(idx.begin(), idx.end(), (int64_t)0);
    std::stable_sort(idx.begin(), idx.end(), [&](int64_t a, int64_t b) { return key[a] > key[b]; });
    std::vector<uint8_t> buf;
    for (int64_t r0 = 0; r0 < g.n; r0 += ROWS_PER_WRITE) {
        const int64_t r1 = std::min(g.n, r0 + ROWS_PER_WRITE);
        buf.assign((size_t)(r1 - r0) * 32, 0);
        for (int64_t r = r0; r < r1; ++r) {
            const int64_t i = idx[r];
            uint8_t* p = buf.data() + (size_t)(r - r0) * 32;
            float m[3], sc[3];
            for (int j = 0; j < 3; ++j) {
                m[j] = world_pos(g, crs, i, j);
                const float e = std::exp(g.scales[3 * i + j]);
                sc[j] = crs.keep ? e / crs.scale : e;
            }
            std::memcpy(p, m, 12);
            std::memcpy(p + 12, sc, 12);
            for (int j = 0; j < 3; ++j)
                p[24 + j] = to_byte(std::clamp(((double)g.f_dc[3 * i + j] * SH_C0 + 0.5) * 255.0, 0.0, 255.0));
            const float sig = 1.0f / (1.0f + std::exp(-g.opacities[i]));
            p[27] = to_byte(std::clamp(sig * 255.0f, 0.0f, 255.0f));
            for (int j = 0; j < 4; ++j)
                p[28 + j] = to_byte(std::clamp(g.quats[4 * i + j] * 128.0f + 128.0f, 0.0f, 255.0f));
        }
        o.write(reinterpret_cast<const char*>(buf.data()), (std::streamsize)buf.size());
    }
    if (!o) throw std::runtime_error("write failed: " + path);
}

HostGaussians load_gaussian_ply(const std::string& path, const Crs& crs, int* step) {
    std::ifstream f(path, std::ios::binary);
    if (!f.is_open()) throw std::runtime_error("Cannot open PLY file: " + path);
    std::string line;
    std::getline(f, line);
    if (line.find("ply") == std::string::npos) throw std::runtime_error("Not a PLY file: " + path);
    std::getline(f, line);   // format line
    int64_t n = 0;
    int it = 0, num_dc = 0, num_fr = 0;
    bool ended = false;
    const std::string iter_prefix = "comment Generated by msplat at iteration ";
    const std::string vert_prefix = "element vertex ";
    while (std::getline(f, line)) {
        if (line == "end_header") { ended = true; break; }
        if (line.rfind(iter_prefix, 0) == 0) it = std::stoi(line.substr(iter_prefix.size()));
        if (line.rfind(vert_prefix, 0) == 0) n = std::stoll(line.substr(vert_prefix.size()));
        if (line.rfind("property float f_dc_", 0) == 0) ++num_dc;
        if (line.rfind("property float f_rest_", 0) == 0) ++num_fr;
    }
    if (!ended) throw std::runtime_error("PLY header has no end_header: " + path);
    if (n <= 0) throw std::runtime_error("PLY has no vertices");
    if (num_dc != 3) throw std::runtime_error("PLY must have three f_dc properties");
    if (num_fr % 3 != 0) throw std::runtime_error("PLY f_rest count is not a multiple of 3");
    HostGaussians g;
    g.n = n;
    g.rest_bases = num_fr / 3;
    g.means.resize(3 * n);
    g.scales.resize(3 * n);
    g.quats.resize(4 * n);
    g.f_dc.resize(3 * n);
    g.f_rest.resize((size_t)num_fr * n);
    g.opacities.resize(n);
    const int per_row = 3 + 3 + num_dc + num_fr + 1 + 3 + 4;
    std::vector<float> rows;
    for (int64_t r0 = 0; r0 < n; r0 += ROWS_PER_WRITE) {
        const int64_t r1 = std::min(n, r0 + ROWS_PER_WRITE);
        rows.resize((size_t)(r1 - r0) * per_row);
        f.read(reinterpret_cast<char*>(rows.data()), (std::streamsize)(rows.size() * 4));
        if (!f) throw std::runtime_error("PLY data is truncated: " + path);
        for (int64_t i = r0; i < r1; ++i) {
            const float* row = rows.data() + (size_t)(i - r0) * per_row;
            int c = 0;
            for (int j = 0; j < 3; ++j) g.means[3 * i + j] = row[c++];
            c += 3;   // normals
            for (int j = 0; j < 3; ++j) g.f_dc[3 * i + j] = row[c++];
            for (int ch = 0; ch < 3; ++ch)   // [3, K-1] -> [K-1, 3]
                for (int b = 0; b < g.rest_bases; ++b)
                    g.f_rest[((size_t)i * g.rest_bases + b) * 3 + ch] = row[c++];
            g.opacities[i] = row[c++];
            for (int j = 0; j < 3; ++j) g.scales[3 * i + j] = row[c++];
            for (int j = 0; j < 4; ++j) g.quats[4 * i + j] = row[c++];
        }
    }
    if (crs.keep) {
        for (int64_t i = 0; i < n; ++i)
            for (int j = 0; j < 3; ++j)
                g.means[3 * i + j] = (g.means[3 * i + j] - crs.translation[j]) * crs.scale;
        for (auto& s : g.scales) s = std::log(crs.scale * std::exp(s));
    }
    if (step) *step = it;
    return g;
}

}  // namespace msplat
