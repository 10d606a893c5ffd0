// Driver for the reference's createSSIMWindow (core/src/ssim.cpp:7-24).
// Prints the 11x11 window taps as hex floats, one per line.  Test
// infrastructure: built into oracle/_ref/ only when /root/reference exists.
#include <cstdio>
#include "ssim.hpp"

int main() {
    std::vector<float> w = createSSIMWindow(11, 1.5f);
    for (float v : w) std::printf("%a\n", (double)v);
    return 0;
}
