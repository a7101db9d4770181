// TEST INFRASTRUCTURE ONLY: runs the library's fused decode path
// (launch_decode_moe of tau.rs_amd/csrc/decode_moe.hip: routing, the decode
// projections and the combine; with -DTAU_DECODE_ONE_LAUNCH the one-launch
// layer of decode_layer.hip) on the CPU emulator of wave_emu/hip/hip_runtime.h.
// usage: decode_emu in.bin out.bin
//   in.bin:  int32 T, H, I, E, K, weight_layout, logits_dtype; then x [T,H] u16,
//            logits [T,E] (f32 or u16), gate_up [E,2I,H] u16, down [E,H,I] u16
//   out.bin: int32 status, capacity; routes [T,2K] f32; meta [2E+2], offsets [E+1],
//            slots [cap], tiles [cap/16] int32; activated [T*K,I], contributions
//            [T*K,H], output [T,H] u16
#include <cstdio>
#include <vector>

#include "kernels.hpp"

template <typename V>
static bool read(FILE* f, V& v) {
    return std::fread(v.data(), sizeof(v[0]), v.size(), f) == v.size();
}
template <typename V>
static void write(FILE* f, const V& v) {
    std::fwrite(v.data(), sizeof(v[0]), v.size(), f);
}

int main(int argc, char** argv) {
    if (argc != 3) return 2;
    FILE* f = std::fopen(argv[1], "rb");
    if (!f) return 2;
    int h[7];
    if (std::fread(h, sizeof(int), 7, f) != 7) return 2;
    const int T = h[0], H = h[1], I = h[2], E = h[3], K = h[4], layout = h[5], ldt = h[6];
    std::vector<uint16_t> x((size_t)T * H), gu((size_t)E * 2 * I * H), dn((size_t)E * H * I);
    std::vector<unsigned char> logits((size_t)T * E * ((ldt & 1) ? 2 : 4));
    if (!read(f, x) || !read(f, logits) || !read(f, gu) || !read(f, dn)) return 2;
    std::fclose(f);
    const int cap = (int)tau_amd::capacity_for(T, E, K, 16);
    std::vector<float> routes((size_t)T * 2 * K, -7.f);
    std::vector<int> meta(2 * E + 2, -7), offsets(E + 1, -7), slots(cap, -7), tiles(cap / 16, -7);
    std::vector<uint16_t> act((size_t)T * K * I, 0x7777), con((size_t)T * K * H, 0x7777), out((size_t)T * H, 0x7777);
    const int status = tau_amd::launch_decode_moe(x.data(), logits.data(), ldt, gu.data(), dn.data(), routes.data(),
                                                  meta.data(), offsets.data(), slots.data(), tiles.data(), act.data(),
                                                  con.data(), out.data(), T, H, I, E, K, cap, layout, nullptr,
                                                  nullptr, nullptr);
    FILE* o = std::fopen(argv[2], "wb");
    if (!o) return 2;
    std::fwrite(&status, 4, 1, o);
    std::fwrite(&cap, 4, 1, o);
    write(o, routes);
    write(o, meta);
    write(o, offsets);
    write(o, slots);
    write(o, tiles);
    write(o, act);
    write(o, con);
    write(o, out);
    std::fclose(o);
    return 0;
}
