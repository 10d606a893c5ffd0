// dataset.cpp — COLMAP ingest, normalisation and initial gaussians (see
// dataset.hpp for the reference functions each part follows).
#include "dataset.hpp"

#include <sys/stat.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <fstream>
#include <random>
#include <sstream>
#include <stdexcept>
#include <unordered_map>

#include "mtensor.hpp"

namespace msplat {

namespace {

bool exists(const std::string& p) {
    struct stat st;
    return ::stat(p.c_str(), &st) == 0;
}

template <typename T>
T rd(std::ifstream& f, const std::string& what) {
    T v{};
    f.read(reinterpret_cast<char*>(&v), sizeof(T));
    if (!f) throw std::runtime_error(what + " is truncated");
    return v;
}

struct ColmapCamera {
    int width = 0, height = 0;
    float fx = 0, fy = 0, cx = 0, cy = 0, k1 = 0, k2 = 0, p1 = 0, p2 = 0;
};

struct ColmapImage {
    uint32_t cam = 0;
    double q[4] = {1, 0, 0, 0};   // w x y z, world to camera
    double t[3] = {0, 0, 0};
    std::string name;
};

// readCamerasBin (load_colmap.cpp:38-74); models SIMPLE_PINHOLE, PINHOLE,
// SIMPLE_RADIAL, RADIAL, OPENCV.
std::unordered_map<uint32_t, ColmapCamera> read_cameras(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f.is_open()) throw std::runtime_error("Cannot open " + path);
    const uint64_t n = rd<uint64_t>(f, path);
    std::unordered_map<uint32_t, ColmapCamera> out;
    for (uint64_t i = 0; i < n; ++i) {
        ColmapCamera c;
        const uint32_t id = rd<uint32_t>(f, path);
        const uint32_t model = rd<uint32_t>(f, path);
        c.width = (int)rd<uint64_t>(f, path);
        c.height = (int)rd<uint64_t>(f, path);
        auto d = [&]() { return (float)rd<double>(f, path); };
        switch (model) {
            case 0: c.fx = c.fy = d(); c.cx = d(); c.cy = d(); break;
            case 1: c.fx = d(); c.fy = d(); c.cx = d(); c.cy = d(); break;
            case 2: c.fx = c.fy = d(); c.cx = d(); c.cy = d(); c.k1 = d(); break;
            case 3: c.fx = c.fy = d(); c.cx = d(); c.cy = d(); c.k1 = d(); c.k2 = d(); break;
            case 4:
                c.fx = d(); c.fy = d(); c.cx = d(); c.cy = d();
                c.k1 = d(); c.k2 = d(); c.p1 = d(); c.p2 = d();
                break;
            default: throw std::runtime_error("Unsupported COLMAP camera model: " + std::to_string(model));
        }
        out[id] = c;
    }
    return out;
}

// readImagesBin (load_colmap.cpp:76-102): pose, camera id, name; the 2D
// points are skipped.
std::vector<ColmapImage> read_images(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f.is_open()) throw std::runtime_error("Cannot open " + path);
    const uint64_t n = rd<uint64_t>(f, path);
    std::vector<ColmapImage> out;
    for (uint64_t i = 0; i < n; ++i) {
        ColmapImage im;
        (void)rd<uint32_t>(f, path);   // image id
        for (double& v : im.q) v = rd<double>(f, path);
        for (double& v : im.t) v = rd<double>(f, path);
        im.cam = rd<uint32_t>(f, path);
        char ch;
        while (f.read(&ch, 1) && ch != '\0') im.name += ch;
        const uint64_t pts2d = rd<uint64_t>(f, path);
        f.seekg((std::streamoff)(pts2d * 24), std::ios::cur);
        if (!f) throw std::runtime_error(path + " is truncated");
        out.push_back(im);
    }
    return out;
}

// readColmapPoints (load_ply.cpp:163-205).
void read_points_bin(const std::string& path, std::vector<float>& xyz, std::vector<uint8_t>& rgb) {
    std::ifstream f(path, std::ios::binary);
    if (!f.is_open()) throw std::runtime_error("Cannot open points3D.bin: " + path);
    const uint64_t n = rd<uint64_t>(f, path);
    xyz.resize(n * 3);
    rgb.resize(n * 3);
    for (uint64_t i = 0; i < n; ++i) {
        (void)rd<uint64_t>(f, path);   // point id
        for (int k = 0; k < 3; ++k) xyz[3 * i + k] = (float)rd<double>(f, path);
        for (int k = 0; k < 3; ++k) rgb[3 * i + k] = rd<uint8_t>(f, path);
        (void)rd<double>(f, path);     // reprojection error
        const uint64_t track = rd<uint64_t>(f, path);
        f.seekg((std::streamoff)(track * 8), std::ios::cur);
        if (!f) throw std::runtime_error(path + " is truncated");
    }
}

// quatToRotMat + w2cToCamToWorld (load_colmap.cpp:9-18, 104-119).
void cam_to_world(const double quat[4], const double t[3], float out[16]) {
    double w = quat[0], x = quat[1], y = quat[2], z = quat[3];
    const double n = std::sqrt(w * w + x * x + y * y + z * z);
    w /= n; x /= n; y /= n; z /= n;
    const float R[9] = {(float)(1 - 2 * (y * y + z * z)), (float)(2 * (x * y - w * z)),
                        (float)(2 * (x * z + w * y)),     (float)(2 * (x * y + w * z)),
                        (float)(1 - 2 * (x * x + z * z)), (float)(2 * (y * z - w * x)),
                        (float)(2 * (x * z - w * y)),     (float)(2 * (y * z + w * x)),
                        (float)(1 - 2 * (x * x + y * y))};
    const float Ri[9] = {R[0], R[3], R[6], R[1], R[4], R[7], R[2], R[5], R[8]};
    const float Ti[3] = {-(Ri[0] * (float)t[0] + Ri[1] * (float)t[1] + Ri[2] * (float)t[2]),
                         -(Ri[3] * (float)t[0] + Ri[4] * (float)t[1] + Ri[5] * (float)t[2]),
                         -(Ri[6] * (float)t[0] + Ri[7] * (float)t[1] + Ri[8] * (float)t[2])};
    const float m[16] = {Ri[0], -Ri[1], -Ri[2], Ti[0], Ri[3], -Ri[4], -Ri[5], Ti[1],
                         Ri[6], -Ri[7], -Ri[8], Ti[2], 0.f,   0.f,    0.f,    1.f};
    std::memcpy(out, m, sizeof(m));
}

}  // namespace

void read_point_ply(const std::string& path, std::vector<float>& xyz, std::vector<uint8_t>& rgb) {
    std::ifstream f(path, std::ios::binary);
    if (!f.is_open()) throw std::runtime_error("Cannot open PLY file: " + path);
    std::string line;
    std::getline(f, line);
    if (line.find("ply") == std::string::npos) throw std::runtime_error("Not a PLY file: " + path);
    enum Ty { F32, F64, U8, U16, I32, UNK };
    struct Prop { std::string name; Ty ty; int off; };
    auto parse_ty = [](const std::string& t) {
        if (t == "float" || t == "float32") return F32;
        if (t == "double" || t == "float64") return F64;
        if (t == "uchar" || t == "uint8") return U8;
        if (t == "ushort" || t == "uint16") return U16;
        if (t == "int" || t == "int32") return I32;
        return UNK;
    };
    auto size_of = [](Ty t) { return t == F64 ? 8 : t == U8 ? 1 : t == U16 ? 2 : t == UNK ? 0 : 4; };
    bool binary = false, ascii = false;
    int64_t nv = 0;
    int vbytes = 0;
    std::vector<Prop> props;
    while (std::getline(f, line)) {
        if (line == "end_header") break;
        std::istringstream iss(line);
        std::string tok;
        iss >> tok;
        if (tok == "format") {
            std::string fmt;
            iss >> fmt;
            binary = fmt == "binary_little_endian";
            ascii = fmt == "ascii";
        } else if (tok == "element") {
            std::string name;
            iss >> name;
            if (name == "vertex") iss >> nv;
        } else if (tok == "property" && nv > 0) {
            std::string ts, name;
            iss >> ts >> name;
            const Ty t = parse_ty(ts);
            props.push_back({name, t, vbytes});
            vbytes += size_of(t);
        }
    }
    if (nv == 0) throw std::runtime_error("PLY has no vertices");
    if (!binary && !ascii)
        throw std::runtime_error("Unsupported PLY format (need ascii or binary_little_endian)");
    auto find = [&](const char* n) {
        for (size_t i = 0; i < props.size(); ++i)
            if (props[i].name == n) return (int)i;
        return -1;
    };
    const int ix = find("x"), iy = find("y"), iz = find("z");
    const int ir = find("red"), ig = find("green"), ib = find("blue");
    if (ix < 0 || iy < 0 || iz < 0) throw std::runtime_error("PLY missing x/y/z properties");
    const bool colour = ir >= 0 && ig >= 0 && ib >= 0;
    xyz.assign((size_t)nv * 3, 0.f);
    rgb.assign((size_t)nv * 3, 128);
    if (binary) {
        std::vector<char> buf(vbytes);
        auto as_float = [&](int pi) -> float {
            const Prop& p = props[pi];
            if (p.ty == F32) { float v; std::memcpy(&v, &buf[p.off], 4); return v; }
            if (p.ty == F64) { double v; std::memcpy(&v, &buf[p.off], 8); return (float)v; }
            return 0.f;
        };
        auto as_u8 = [&](int pi) -> uint8_t {
            const Prop& p = props[pi];
            if (p.ty == U8) return (uint8_t)buf[p.off];
            if (p.ty == U16) { uint16_t v; std::memcpy(&v, &buf[p.off], 2); return (uint8_t)(v >> 8); }
            if (p.ty == F32) { float v; std::memcpy(&v, &buf[p.off], 4); return (uint8_t)(v * 255.0f); }
            return 128;
        };
        for (int64_t i = 0; i < nv; ++i) {
            f.read(buf.data(), vbytes);
            if (!f) throw std::runtime_error("PLY data is truncated: " + path);
            xyz[3 * i] = as_float(ix);
            xyz[3 * i + 1] = as_float(iy);
            xyz[3 * i + 2] = as_float(iz);
            if (colour) {
                rgb[3 * i] = as_u8(ir);
                rgb[3 * i + 1] = as_u8(ig);
                rgb[3 * i + 2] = as_u8(ib);
            }
        }
    } else {
        for (int64_t i = 0; i < nv; ++i) {
            if (!std::getline(f, line)) throw std::runtime_error("PLY data is truncated: " + path);
            std::istringstream iss(line);
            std::vector<std::string> tk;
            std::string t;
            while (iss >> t) tk.push_back(t);
            if (tk.size() < props.size()) throw std::runtime_error("PLY row is short: " + path);
            xyz[3 * i] = std::stof(tk[ix]);
            xyz[3 * i + 1] = std::stof(tk[iy]);
            xyz[3 * i + 2] = std::stof(tk[iz]);
            if (colour) {
                const bool fl = props[ir].ty == F32 || props[ir].ty == F64;
                const int idx[3] = {ir, ig, ib};
                for (int k = 0; k < 3; ++k) {
                    const float v = std::stof(tk[idx[k]]);
                    rgb[3 * i + k] = fl ? (uint8_t)(v * 255.0f) : (uint8_t)v;
                }
            }
        }
    }
}

void auto_scale_and_center(Dataset& d) {
    if (d.cameras.empty()) return;
    float mean[3] = {0.f, 0.f, 0.f};
    for (auto& c : d.cameras) {
        mean[0] += c.camToWorld[3];
        mean[1] += c.camToWorld[7];
        mean[2] += c.camToWorld[11];
    }
    const int n = (int)d.cameras.size();
    for (float& m : mean) m /= n;
    for (int k = 0; k < 3; ++k) d.translation[k] = mean[k];
    for (auto& c : d.cameras) {
        c.camToWorld[3] -= mean[0];
        c.camToWorld[7] -= mean[1];
        c.camToWorld[11] -= mean[2];
    }
    float max_abs = 0.f;
    for (auto& c : d.cameras) {
        max_abs = std::max(max_abs, std::abs(c.camToWorld[3]));
        max_abs = std::max(max_abs, std::abs(c.camToWorld[7]));
        max_abs = std::max(max_abs, std::abs(c.camToWorld[11]));
    }
    d.scale = max_abs > 0 ? 1.0f / max_abs : 1.0f;
    for (auto& c : d.cameras) {
        c.camToWorld[3] *= d.scale;
        c.camToWorld[7] *= d.scale;
        c.camToWorld[11] *= d.scale;
    }
    const size_t np = d.xyz.size() / 3;
    for (size_t i = 0; i < np; ++i)
        for (int k = 0; k < 3; ++k) d.xyz[3 * i + k] = (d.xyz[3 * i + k] - mean[k]) * d.scale;
}

Dataset load_colmap(const std::string& root, const std::string& image_dir) {
    const std::string sparse = exists(root + "/cameras.bin") ? root : root + "/sparse/0";
    const std::string images = !image_dir.empty() ? image_dir
                               : exists(root + "/images") ? root + "/images"
                                                          : root;
    auto cams = read_cameras(sparse + "/cameras.bin");
    auto ims = read_images(sparse + "/images.bin");
    std::sort(ims.begin(), ims.end(),
              [](const ColmapImage& a, const ColmapImage& b) { return a.name < b.name; });
    Dataset d;
    for (const auto& im : ims) {
        auto it = cams.find(im.cam);
        if (it == cams.end()) continue;
        const ColmapCamera& cc = it->second;
        DatasetCamera c;
        c.width = cc.width; c.height = cc.height;
        c.fx = cc.fx; c.fy = cc.fy; c.cx = cc.cx; c.cy = cc.cy;
        c.k1 = cc.k1; c.k2 = cc.k2; c.p1 = cc.p1; c.p2 = cc.p2;
        c.filePath = images + "/" + im.name;
        cam_to_world(im.q, im.t, c.camToWorld);
        d.cameras.push_back(c);
    }
    if (exists(sparse + "/points3D.bin")) read_points_bin(sparse + "/points3D.bin", d.xyz, d.rgb);
    else if (exists(sparse + "/points3D.ply")) read_point_ply(sparse + "/points3D.ply", d.xyz, d.rgb);
    auto_scale_and_center(d);
    return d;
}

HostGaussians init_gaussians(const std::vector<float>& xyz, const std::vector<uint8_t>& rgb,
                             int sh_degree) {
    const int64_t n = (int64_t)(xyz.size() / 3);
    if (n < 4) throw std::runtime_error("the point cloud needs at least 4 points");
    if (rgb.size() != xyz.size()) throw std::runtime_error("one colour per point is needed");
    if (sh_degree < 0 || sh_degree > 4) throw std::runtime_error("SH degree must be 0..4");
    HostGaussians g;
    g.n = n;
    g.rest_bases = (sh_degree + 1) * (sh_degree + 1) - 1;
    g.means = xyz;
    // scales: log of the mean distance to the three nearest other points
    {
        MTensor pts = MTensor::empty({n, 3}, DType::Float32);
        MTensor dist = MTensor::empty({n}, DType::Float32);
        pts.copy_from_host(xyz.data(), xyz.size() * sizeof(float));
        check(msplat_hip_knn_mean_dist(pts.data<float>(), n, dist.data<float>()), "knn");
        std::vector<float> sc((size_t)n);
        dist.copy_to_host(sc.data(), sc.size() * sizeof(float));
        g.scales.resize((size_t)n * 3);
        for (int64_t i = 0; i < n; ++i) {
            const float v = std::log(sc[i]);
            g.scales[3 * i] = g.scales[3 * i + 1] = g.scales[3 * i + 2] = v;
        }
    }
    // random unit quaternions (model.cpp:76-89)
    {
        std::mt19937 rng(42);
        std::uniform_real_distribution<float> dist(0.0f, 1.0f);
        g.quats.resize((size_t)n * 4);
        for (int64_t i = 0; i < n; ++i) {
            const float u = dist(rng), v = dist(rng), w = dist(rng);
            g.quats[4 * i + 0] = std::sqrt(1 - u) * std::sin(2 * M_PI * v);
            g.quats[4 * i + 1] = std::sqrt(1 - u) * std::cos(2 * M_PI * v);
            g.quats[4 * i + 2] = std::sqrt(u) * std::sin(2 * M_PI * w);
            g.quats[4 * i + 3] = std::sqrt(u) * std::cos(2 * M_PI * w);
        }
    }
    const double C0 = 0.28209479177387814;
    g.f_dc.resize((size_t)n * 3);
    for (size_t i = 0; i < (size_t)n * 3; ++i) g.f_dc[i] = (float)((rgb[i] / 255.0 - 0.5) / C0);
    g.f_rest.assign((size_t)n * g.rest_bases * 3, 0.f);
    g.opacities.assign((size_t)n, std::log(0.1f / 0.9f));
    return g;
}

}  // namespace msplat
