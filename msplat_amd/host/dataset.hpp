// dataset.hpp — COLMAP dataset ingest on the host: cameras, poses and the
// sparse point cloud of a COLMAP reconstruction, normalised like the
// reference's input data, and the initial gaussians built from the cloud.
//
// Follows core/src/loaders/load_colmap.cpp (cameras.bin / images.bin /
// points3D.bin, or points3D.ply through readPly, load_ply.cpp:34-161),
// core/src/input_data.cpp:79-161 (autoScaleAndCenter, splitTrainTest) and
// Model::Model (model.cpp:43-117) for the initial gaussians.  Images are not
// decoded here (the reference decodes with CoreGraphics): each camera keeps
// the path of its image, and the caller supplies the pixels.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "gaussian_io.hpp"

namespace msplat {

// One camera of the dataset (input_data.hpp:20-38 without the image).
struct DatasetCamera {
    int width = 0, height = 0;
    float fx = 0, fy = 0, cx = 0, cy = 0;
    float k1 = 0, k2 = 0, p1 = 0, p2 = 0;
    float camToWorld[16] = {};   // row-major, OpenGL (Y up, Z back)
    std::string filePath;
};

struct Dataset {
    std::vector<DatasetCamera> cameras;
    std::vector<float> xyz;        // [n,3]
    std::vector<uint8_t> rgb;      // [n,3]
    float scale = 1.f;             // world = stored / scale + translation
    float translation[3] = {0.f, 0.f, 0.f};
};

// loadColmap (load_colmap.cpp:121-164): the sparse model under root or
// root/sparse/0; image_dir empty: root/images if it exists, else root.
// Cameras sorted by image file name, poses camera-to-world with the OpenGL
// axis flip, then autoScaleAndCenter.  Throws on missing or malformed files.
Dataset load_colmap(const std::string& root, const std::string& image_dir);

// autoScaleAndCenter (input_data.cpp:79-125).
void auto_scale_and_center(Dataset& d);

// Point cloud of a PLY file (readPly, load_ply.cpp:34-161): x, y, z and,
// when present, red, green, blue; binary little-endian or ascii.
void read_point_ply(const std::string& path, std::vector<float>& xyz, std::vector<uint8_t>& rgb);

// Initial gaussians of a point cloud (Model::Model, model.cpp:59-110):
// means = points; log-scales = log of the mean distance to the three
// nearest other points (repeated on the three axes; computed on the GPU by
// msplat_hip_knn_mean_dist); unit quaternions from mt19937(42) uniforms;
// f_dc = (rgb / 255 - 0.5) / C0; zero higher SH bands; opacity logit(0.1).
HostGaussians init_gaussians(const std::vector<float>& xyz, const std::vector<uint8_t>& rgb,
                             int sh_degree);

}  // namespace msplat
