// memh_reader.cpp -- prints what the reference's memh readers
// (hls/common/test_memh.hpp:54-76) return for a file, one decimal value per
// line.  Built by ref.mk against the reference checkout; used by the tests to
// pin the Python readers of golden_trace.py.
#include <cstdio>
#include <exception>
#include <string>

#include "test_memh.hpp"

int main(int argc, char** argv) {
    if (argc != 3) {
        std::fprintf(stderr, "usage: memh_reader i32|u32|i8 FILE\n");
        return 2;
    }
    namespace hc = tinyllama::hls_common;
    const std::string mode = argv[1];
    try {
        if (mode == "i32") {
            for (int32_t v : hc::read_scalar_memh_i32(argv[2])) std::printf("%d\n", (int)v);
        } else if (mode == "u32") {
            for (uint32_t v : hc::read_scalar_memh_u32(argv[2])) std::printf("%u\n", (unsigned)v);
        } else if (mode == "i8") {
            for (int8_t v : hc::read_scalar_memh_i8(argv[2])) std::printf("%d\n", (int)v);
        } else {
            return 2;
        }
    } catch (const std::exception& e) {
        std::fprintf(stderr, "%s\n", e.what());
        return 1;
    }
    return 0;
}
