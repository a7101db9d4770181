// TEST INFRASTRUCTURE ONLY: runs the library's routing launcher
// (launch_routing / launch_routing_shared of tau.rs_amd/csrc/routing.hip, as
// rewritten by prep.py) on the CPU emulator of wave_emu/hip/hip_runtime.h.
// usage: route_emu in.bin out.bin
//   in.bin:  int32 T, E, K, dtype (0 f32, 1 bf16 bits; | 0x100 raw weights), shared;
//            then T * (E + shared) logits (f32 or uint16)
//   out.bin: int32 status, then T * 2 * (K + shared) f32 routes
#include <cstdio>
#include <vector>

#include "kernels.hpp"

int main(int argc, char** argv) {
    if (argc != 3) return 2;
    FILE* f = std::fopen(argv[1], "rb");
    if (!f) return 2;
    int h[5];
    if (std::fread(h, sizeof(int), 5, f) != 5) return 2;
    const int T = h[0], E = h[1], K = h[2], dtype = h[3], shared = h[4];
    const size_t n = (size_t)T * (E + shared), bytes = (dtype & 1) ? 2 : 4;
    std::vector<unsigned char> logits(n * bytes);
    const size_t got = std::fread(logits.data(), 1, logits.size(), f);
    std::fclose(f);
    if (got != logits.size()) return 2;
    std::vector<float> routes((size_t)T * 2 * (K + shared), -7.0f);
    const int status = shared ? tau_amd::launch_routing_shared(logits.data(), dtype, routes.data(), T, E, K, nullptr)
                              : tau_amd::launch_routing(logits.data(), dtype, routes.data(), T, E, K, nullptr);
    FILE* o = std::fopen(argv[2], "wb");
    if (!o) return 2;
    std::fwrite(&status, 4, 1, o);
    std::fwrite(routes.data(), 4, routes.size(), o);
    std::fclose(o);
    return 0;
}
