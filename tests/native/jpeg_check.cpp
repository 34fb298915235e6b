// jpeg_check.cpp -- CPU harness for the JPEG decoder (csrc/host/jpeg.cpp):
// decodes each file named on the command line and prints one line per file,
// "ok W H" or "error <message>".  Built with AddressSanitizer by the tests,
// so an out-of-bounds access in the decoder ends the run with a report
// instead of passing silently.
#include <cstdio>
#include <fstream>
#include <iterator>
#include <stdexcept>
#include <string>
#include <vector>

#include "input_data.hpp"

Image decode_jpeg(const std::vector<uint8_t> &f, const std::string &path);

int main(int argc, char **argv) {
    for (int i = 1; i < argc; ++i) {
        std::ifstream in(argv[i], std::ios::binary);
        std::vector<uint8_t> f((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
        try {
            const Image img = decode_jpeg(f, argv[i]);
            std::printf("ok %d %d\n", img.width, img.height);
        } catch (const std::exception &e) {
            std::printf("error %s\n", e.what());
        }
    }
    return 0;
}
