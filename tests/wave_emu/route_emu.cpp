// TEST INFRASTRUCTURE ONLY: runs the library's routing kernels
// (route_kernel / route_shared_kernel of tau.rs_amd/csrc/dispatch.hpp) on the
// CPU, one 64-lane wavefront (four tokens) at a time, each lane a thread, with
// the wave intrinsics of wave_emu/hip/hip_runtime.h.
// usage: route_emu in.bin out.bin
//   in.bin:  int32 T, E, K, dtype (0 f32, 1 bf16 bits), normalize, shared;
//            then T * (E + shared) logits (f32 or uint16)
//   out.bin: T * 2 * (K + shared) f32 routes
#include <cstdio>
#include <thread>
#include <vector>

#include "dispatch.hpp"

using namespace tau_amd;

template <int EP, typename T>
static void run_wave(const T* logits, float* routes, int tokens, int E, int K, int normalize, int shared, int w) {
    emu::Wave wave;
    emu::wave = &wave;
    std::vector<std::thread> lanes;
    for (int l = 0; l < 64; ++l)
        lanes.emplace_back([=] {
            threadIdx.x = l;
            blockIdx.x = w;
            if (shared) route_shared_kernel<EP, T>(logits, routes, tokens, E, K, normalize);
            else route_kernel<EP, T>(logits, routes, tokens, E, K, normalize);
        });
    for (auto& t : lanes) t.join();
}

template <typename T>
static void run(const T* logits, float* routes, int tokens, int E, int K, int normalize, int shared) {
    const int ep = (E + 15) / 16;
    for (int w = 0; w < (tokens + 3) / 4; ++w) {
        if (ep <= 1) run_wave<1, T>(logits, routes, tokens, E, K, normalize, shared, w);
        else if (ep <= 2) run_wave<2, T>(logits, routes, tokens, E, K, normalize, shared, w);
        else if (ep <= 4) run_wave<4, T>(logits, routes, tokens, E, K, normalize, shared, w);
        else if (ep <= 8) run_wave<8, T>(logits, routes, tokens, E, K, normalize, shared, w);
        else if (ep <= 16) run_wave<16, T>(logits, routes, tokens, E, K, normalize, shared, w);
        else run_wave<32, T>(logits, routes, tokens, E, K, normalize, shared, w);
    }
}

int main(int argc, char** argv) {
    if (argc != 3) return 2;
    FILE* f = std::fopen(argv[1], "rb");
    if (!f) return 2;
    int h[6];
    if (std::fread(h, sizeof(int), 6, f) != 6) return 2;
    const int T = h[0], E = h[1], K = h[2], dtype = h[3], normalize = h[4], shared = h[5];
    const size_t n = (size_t)T * (E + shared);
    std::vector<float> lf(dtype ? 0 : n);
    std::vector<uint16_t> lb(dtype ? n : 0);
    const size_t got = dtype ? std::fread(lb.data(), 2, n, f) : std::fread(lf.data(), 4, n, f);
    std::fclose(f);
    if (got != n) return 2;
    std::vector<float> routes((size_t)T * 2 * (K + shared), -7.0f);
    if (dtype) run<uint16_t>(lb.data(), routes.data(), T, E, K, normalize, shared);
    else run<float>(lf.data(), routes.data(), T, E, K, normalize, shared);
    FILE* o = std::fopen(argv[2], "wb");
    if (!o) return 2;
    std::fwrite(routes.data(), 4, routes.size(), o);
    std::fclose(o);
    return 0;
}
