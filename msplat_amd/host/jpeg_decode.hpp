// jpeg_decode.hpp — decoding of the dataset's JPEG target images.
#pragma once

#include <string>

#include "png_decode.hpp"   // DecodedImage

namespace msplat {

// True when the file starts with a JPEG start-of-image marker (FF D8 FF).
bool is_jpeg_file(const std::string& path);

// Decodes a baseline, extended-sequential or progressive Huffman-coded JPEG
// (8-bit, grey or three components) into float RGB (each channel byte / 255,
// as the reference's imreadRGB, image_io.cpp:12-50); throws on unsupported
// or corrupt files.
DecodedImage decode_jpeg(const std::string& path);

}  // namespace msplat
