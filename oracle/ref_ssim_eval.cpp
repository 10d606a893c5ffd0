// Driver for the reference's ssim_eval (core/src/ssim.cpp:61-123): reads
// int32 H, W, window size, float sigma, then the render and the target
// ([H,W,3] fp32 each) from the file named by argv[1] and prints the SSIM as a
// hex float.  Test infrastructure: built into oracle/_ref/ only when
// /root/reference exists.
#include <cstdio>
#include <cstdint>
#include <vector>
#include "ssim.hpp"

int main(int argc, char** argv) {
    if (argc != 2) return 2;
    FILE* f = std::fopen(argv[1], "rb");
    if (!f) return 2;
    int32_t hdr[3];
    float sigma;
    if (std::fread(hdr, 4, 3, f) != 3 || std::fread(&sigma, 4, 1, f) != 1) return 2;
    const int64_t n = (int64_t)hdr[0] * hdr[1] * 3;
    MTensor img({hdr[0], hdr[1], 3}, DType::Float32), gt({hdr[0], hdr[1], 3}, DType::Float32);
    if (std::fread(img.data_ptr(), 4, n, f) != (size_t)n) return 2;
    if (std::fread(gt.data_ptr(), 4, n, f) != (size_t)n) return 2;
    std::fclose(f);
    std::printf("%a\n", (double)ssim_eval(img, gt, hdr[2], sigma));
    return 0;
}
