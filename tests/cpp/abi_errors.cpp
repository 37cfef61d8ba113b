// CPU-side check of the C++ host's kernel-level API (yt::kernel::hip in
// include/yt/ytensor.hpp): argument errors are reported as exceptions before
// anything touches a GPU.
#include <cstdio>
#include <stdexcept>

#include "yt/ytensor.hpp"

int main() {
    int fails = 0;
    try {
        yt::kernel::hip::sgemm(nullptr, nullptr, nullptr, -1, 2, 2, 1.0f, 0.0f, 2, 1, 2, 1, 2, 1);
        std::puts("no exception for m = -1");
        fails++;
    } catch (const std::invalid_argument& e) {
        std::printf("ok: %s\n", e.what());
    }
    try {
        yt::kernel::hip::flash_attention(YTHIP_BF16, nullptr, nullptr, nullptr, nullptr, 4, 4, 128, 128, 0.f, 128, 2,
                                         128, 1, 128, 1, 128, 1);
        std::puts("no exception for csq = 2");
        fails++;
    } catch (const std::invalid_argument& e) {
        std::printf("ok: %s\n", e.what());
    }
    // m == 0 is the reference's no-op (sgemm.inl:594): no exception
    yt::kernel::hip::sgemm(nullptr, nullptr, nullptr, 0, 2, 2, 1.0f, 0.0f, 2, 1, 2, 1, 2, 1);
    std::printf("abi version %d\n", ythip_abi_version());
    return fails;
}
