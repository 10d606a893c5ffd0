// knn.hip — initial gaussian scales from the point cloud: for every point the
// mean Euclidean distance to its three nearest other points.
//
// The reference builds a nanoflann kd-tree and asks for the 4 nearest
// neighbours of each point (the point itself first), then averages
// sqrt(d) over neighbours 1..3 (PointsTensor::scales,
// core/include/kdtree_tensor.hpp:26-40; used by Model::Model, model.cpp:63-73).
// On the GPU the points are bucketed into a uniform grid (cell id by point,
// one stable radix sort by cell, cell ranges from the run edges) and one
// thread per point visits cells in Chebyshev rings around its own.  After
// ring r every point not yet seen is at least r*h - margin away (h: cell
// edge), so the search stops once the fourth-smallest squared distance is
// below that bound.  Squared distances are accumulated per axis like
// nanoflann's L2_Simple_Adaptor ((dx^2 + dy^2) + dz^2 in fp32) and the four
// smallest are kept sorted, so the result is the kd-tree's exactly.
#include "common.hpp"
#include "kernels.hpp"

namespace msp {

namespace {

__device__ __forceinline__ int cell_coord(float v, float lo, float inv_h, int dim) {
    const int c = (int)floorf((v - lo) * inv_h);
    return min(max(c, 0), dim - 1);
}

__global__ __launch_bounds__(256) void k_knn_cells(int64_t n, const float* __restrict__ xyz,
                                                   KnnGrid g, uint32_t* __restrict__ key,
                                                   uint32_t* __restrict__ val) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const int cx = cell_coord(xyz[3 * i], g.lo[0], g.inv_h, g.dim[0]);
    const int cy = cell_coord(xyz[3 * i + 1], g.lo[1], g.inv_h, g.dim[1]);
    const int cz = cell_coord(xyz[3 * i + 2], g.lo[2], g.inv_h, g.dim[2]);
    key[i] = (uint32_t)((cz * g.dim[1] + cy) * g.dim[0] + cx);
    val[i] = (uint32_t)i;
}

__device__ __forceinline__ void keep4(float d, float* b) {
    if (d < b[3]) {
        if (d < b[2]) {
            b[3] = b[2];
            if (d < b[1]) {
                b[2] = b[1];
                if (d < b[0]) { b[1] = b[0]; b[0] = d; }
                else b[1] = d;
            } else {
                b[2] = d;
            }
        } else {
            b[3] = d;
        }
    }
}

__global__ __launch_bounds__(256) void k_knn_search(int64_t n, const float* __restrict__ xyz,
                                                    KnnGrid g, const uint32_t* __restrict__ order,
                                                    const int* __restrict__ cstart,
                                                    const int* __restrict__ cend,
                                                    float* __restrict__ mean_dist) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float px = xyz[3 * i], py = xyz[3 * i + 1], pz = xyz[3 * i + 2];
    const int cx = cell_coord(px, g.lo[0], g.inv_h, g.dim[0]);
    const int cy = cell_coord(py, g.lo[1], g.inv_h, g.dim[1]);
    const int cz = cell_coord(pz, g.lo[2], g.inv_h, g.dim[2]);
    float b[4] = {INFINITY, INFINITY, INFINITY, INFINITY};
    const int rmax = max(g.dim[0], max(g.dim[1], g.dim[2]));
    for (int r = 0; r <= rmax; ++r) {
        const int z0 = max(cz - r, 0), z1 = min(cz + r, g.dim[2] - 1);
        const int y0 = max(cy - r, 0), y1 = min(cy + r, g.dim[1] - 1);
        const int x0 = max(cx - r, 0), x1 = min(cx + r, g.dim[0] - 1);
        auto visit = [&](int x, int y, int z) {
            const int c = (z * g.dim[1] + y) * g.dim[0] + x;
            const int e = cend[c];
            for (int s = cstart[c]; s < e; ++s) {
                const uint32_t j = order[s];
                const float dx = px - xyz[3 * j], dy = py - xyz[3 * j + 1], dz = pz - xyz[3 * j + 2];
                float d = 0.f;
                d += dx * dx;
                d += dy * dy;
                d += dz * dz;
                keep4(d, b);
            }
        };
        // the cells at Chebyshev distance exactly r (clamped to the grid)
        for (int z = z0; z <= z1; ++z) {
            const bool zs = z == cz - r || z == cz + r;
            for (int y = y0; y <= y1; ++y) {
                if (zs || y == cy - r || y == cy + r) {
                    for (int x = x0; x <= x1; ++x) visit(x, y, z);
                } else {
                    if (cx - r >= 0) visit(cx - r, y, z);
                    if (r > 0 && cx + r < g.dim[0]) visit(cx + r, y, z);
                }
            }
        }
        // unseen points lie beyond r*h (less a margin for the cell rounding)
        const float reach = fmaxf((float)r * g.h - g.margin, 0.f);
        if (b[3] <= reach * reach) break;
    }
    float sum = 0.f;
    sum += sqrtf(b[1]);
    sum += sqrtf(b[2]);
    sum += sqrtf(b[3]);
    mean_dist[i] = sum / 3;
}

inline unsigned blocks_for(int64_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace

void launch_knn_cells(hipStream_t s, int64_t n, const float* xyz, const KnnGrid& g,
                      uint32_t* key, uint32_t* val) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_knn_cells, dim3(blocks_for(n)), dim3(256), 0, s, n, xyz, g, key, val);
}

void launch_knn_search(hipStream_t s, int64_t n, const float* xyz, const KnnGrid& g,
                       const uint32_t* order, const int* cstart, const int* cend,
                       float* mean_dist) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_knn_search, dim3(blocks_for(n)), dim3(256), 0, s, n, xyz, g, order,
                       cstart, cend, mean_dist);
}

}  // namespace msp
