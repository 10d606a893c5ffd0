// png_decode.hpp — decoding of the dataset's PNG target images (zlib).
#pragma once

#include <string>
#include <vector>

namespace msplat {

// An RGB image, float32 HWC in [0, 1].
struct DecodedImage {
    int width = 0, height = 0;
    std::vector<float> rgb;
};

// True when the file starts with the PNG signature.
bool is_png_file(const std::string& path);

// Decodes a non-interlaced PNG into float RGB (each channel byte / 255, as the
// reference's imreadRGB, image_io.cpp:12-50); throws on unsupported or corrupt
// files.
DecodedImage decode_png(const std::string& path);

}  // namespace msplat
