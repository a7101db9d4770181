// TEST INFRASTRUCTURE ONLY: runs the library's whole routed layer through its
// C ABI (tau_launch_moe_prefill_ex of tau.rs_amd/csrc/moe.hip: routing,
// dispatch, the grouped gate_up and down projections, the combine) on the CPU
// emulator of wave_emu/hip/hip_runtime.h.
// usage: prefill_emu in.bin out.bin
//   in.bin:  int32 T, H, I, E, K, tile_rows, weight_layout, logits_dtype, shared; then
//            x [T,H] u16, logits [T,E'] (f32 or u16), gate_up [E',2I,H] u16, down [E',H,I] u16
//            with E' = E + shared.  shared = 1: the always-on shared expert is
//            folded in as expert E (tau_launch_moe_routing_shared_ex writes the
//            routes from the [T, E+1] logits, then tau_launch_moe_prefill_ex runs
//            from those routes with E+1 experts and K+1 picks)
//   out.bin: int32 status, capacity; routes [T,2K] f32; meta [2E+2], offsets [E+1],
//            slots [cap], tiles [cap/tile_rows] int32; activated [cap,I],
//            contributions [T*K,H], output [T,H] u16; int64 counts of the emulated
//            wave instructions: 16x16x32 MFMAs, 32x32x16 MFMAs, direct-to-LDS copies
// Every device buffer lives in one arena mapped at 0x7e0080000000, so the low
// 32 bits of every address have bit 31 set: a 64-bit address rebuilt from two
// 32-bit words with the low word sign-extended (the fault of the 128x128
// wave-tile build) then points outside the arena and the run fails.
#include <sys/mman.h>

#include <cstdio>
#include <cstring>
#include <vector>

#include "../../include/tau_moe.h"
#include "hip/hip_runtime.h"  // the emulator's instruction counts

static char* g_arena = nullptr;
static size_t g_used = 0;
constexpr size_t kArena = (size_t)1 << 30;

// A buffer of n elements in the arena, filled with `fill`.
template <typename T>
struct Buf {
    T* p = nullptr;
    size_t n = 0;
    Buf(size_t n_, T fill) : n(n_) {
        const size_t bytes = (n * sizeof(T) + 255) / 256 * 256;
        if (g_used + bytes > kArena) std::abort();
        p = (T*)(g_arena + g_used);
        g_used += bytes;
        for (size_t i = 0; i < n; ++i) p[i] = fill;
    }
    T* data() { return p; }
};

template <typename V>
static bool read(FILE* f, V& v) {
    return std::fread(v.data(), sizeof(v.data()[0]), v.n, f) == v.n;
}
template <typename V>
static void write(FILE* f, V& v) {
    std::fwrite(v.data(), sizeof(v.data()[0]), v.n, f);
}

int main(int argc, char** argv) {
    if (argc != 3) return 2;
    void* hint = (void*)0x7e0080000000ull;
    g_arena = (char*)mmap(hint, kArena, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_FIXED_NOREPLACE,
                          -1, 0);
    if (g_arena != hint) {
        std::fprintf(stderr, "could not map the arena at %p\n", hint);
        return 4;
    }
    FILE* f = std::fopen(argv[1], "rb");
    if (!f) return 2;
    int h[9];
    if (std::fread(h, sizeof(int), 9, f) != 9) return 2;
    const int T = h[0], H = h[1], I = h[2], E0 = h[3], K0 = h[4], M = h[5], layout = h[6], ldt = h[7];
    const int shared = h[8];
    const int E = E0 + shared, K = K0 + shared;  // the schedule's experts and picks
    Buf<uint16_t> x((size_t)T * H, 0), gu((size_t)E * 2 * I * H, 0), dn((size_t)E * H * I, 0);
    Buf<unsigned char> logits((size_t)T * E * ((ldt & 1) ? 2 : 4), 0);
    if (!read(f, x) || !read(f, logits) || !read(f, gu) || !read(f, dn)) return 2;
    std::fclose(f);
    size_t sz[7];
    if (tau_moe_workspace_bytes(T, H, I, E, K, M, sz)) return 3;
    const int cap = (int)tau_moe_prefill_capacity(T, E, K, M);
    Buf<float> routes(sz[0] / 4, -7.f);
    Buf<int> meta(sz[1] / 4, -7), offsets(sz[2] / 4, -7), slots(sz[3] / 4, -7), tiles(sz[4] / 4, -7);
    Buf<uint16_t> act(sz[5] / 2, 0x7777), con(sz[6] / 2, 0x7777), out((size_t)T * H, 0x7777);
    int status = 0;
    if (shared) status = tau_launch_moe_routing_shared_ex(logits.data(), ldt, routes.data(), T, E0, K0, nullptr);
    if (status == 0)
        status = tau_launch_moe_prefill_ex(x.data(), shared ? nullptr : logits.data(), ldt, gu.data(), dn.data(),
                                           routes.data(), meta.data(), offsets.data(), slots.data(), tiles.data(),
                                           act.data(), con.data(), out.data(), T, H, I, E, K, M, cap, layout,
                                           nullptr, nullptr, nullptr);
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
    const long long counts[3] = {emu::count_mfma16, emu::count_mfma32, emu::count_dma16};
    std::fwrite(counts, sizeof counts[0], 3, o);
    std::fclose(o);
    return 0;
}
