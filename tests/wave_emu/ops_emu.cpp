// TEST INFRASTRUCTURE ONLY: runs the library's router projection + routing
// (tau_launch_moe_router_route_ex, router.hip and routing.hip) and the fused
// residual add + centered RMSNorm (tau_launch_fused_residual_rms_norm and
// tau_launch_centered_rms_norm_configured, norm.hip) through their C ABI on the
// CPU emulator of wave_emu/hip/hip_runtime.h.
// usage: ops_emu in.bin out.bin
//   mode 0 in:  int32 0, T, H, E, K, has_bias; x [T,H] u16, weight [E,H] u16, bias [E] f32
//          out: int32 status; logits [T,E] f32; routes [T,2K] f32
//   mode 1 in:  int32 1, rows, columns, dtype (0 f32, 1 bf16), preferred_bytes; f32 epsilon;
//               input, branch [rows,columns], weight [columns] (4 or 2 bytes each)
//          out: int32 status; residual, output, norm(residual) [rows,columns]
// Buffers live in an arena mapped at 0x7e0080000000 (low address words with
// bit 31 set, as in prefill_emu).
#include <sys/mman.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "../../include/tau_moe.h"

static char* g_arena = nullptr;
static size_t g_used = 0;
constexpr size_t kArena = (size_t)1 << 30;

static void* take(size_t bytes) {
    bytes = (bytes + 255) / 256 * 256;
    if (g_used + bytes > kArena) std::abort();
    void* p = g_arena + g_used;
    g_used += bytes;
    return p;
}
static bool read(FILE* f, void* p, size_t bytes) { return std::fread(p, 1, bytes, f) == bytes; }

int main(int argc, char** argv) {
    if (argc != 3) return 2;
    void* hint = (void*)0x7e0080000000ull;
    g_arena = (char*)mmap(hint, kArena, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_FIXED_NOREPLACE,
                          -1, 0);
    if (g_arena != hint) return 4;
    FILE* f = std::fopen(argv[1], "rb");
    if (!f) return 2;
    int mode = -1;
    if (!read(f, &mode, 4)) return 2;
    FILE* o = nullptr;
    if (mode == 0) {
        int h[5];
        if (!read(f, h, sizeof h)) return 2;
        const int T = h[0], H = h[1], E = h[2], K = h[3], has_bias = h[4];
        void* x = take((size_t)T * H * 2);
        void* w = take((size_t)E * H * 2);
        float* bias = (float*)take((size_t)E * 4);
        if (!read(f, x, (size_t)T * H * 2) || !read(f, w, (size_t)E * H * 2) || !read(f, bias, (size_t)E * 4))
            return 2;
        float* logits = (float*)take((size_t)T * E * 4);
        float* routes = (float*)take((size_t)T * 2 * K * 4);
        std::memset(logits, 0x7f, (size_t)T * E * 4);
        std::memset(routes, 0x7f, (size_t)T * 2 * K * 4);
        const int status =
            tau_launch_moe_router_route_ex(x, w, has_bias ? bias : nullptr, logits, routes, T, H, E, K, nullptr);
        o = std::fopen(argv[2], "wb");
        if (!o) return 2;
        std::fwrite(&status, 4, 1, o);
        std::fwrite(logits, 4, (size_t)T * E, o);
        std::fwrite(routes, 4, (size_t)T * 2 * K, o);
    } else if (mode == 1) {
        int h[4];
        float eps = 0.f;
        if (!read(f, h, sizeof h) || !read(f, &eps, 4)) return 2;
        const int rows = h[0], cols = h[1], dtype = h[2], policy = h[3];
        const size_t es = dtype ? 2 : 4, n = (size_t)rows * cols;
        void* x = take(n * es);
        void* b = take(n * es);
        void* w = take((size_t)cols * es);
        if (!read(f, x, n * es) || !read(f, b, n * es) || !read(f, w, (size_t)cols * es)) return 2;
        void* res = take(n * es);
        void* y = take(n * es);
        void* alone = take(n * es);
        std::memset(res, 0x7f, n * es);
        std::memset(y, 0x7f, n * es);
        std::memset(alone, 0x7f, n * es);
        int status = tau_launch_fused_residual_rms_norm(x, b, w, res, y, rows, cols, eps, dtype, nullptr, policy);
        if (status == 0)
            status = tau_launch_centered_rms_norm_configured(res, w, alone, rows, cols, eps, dtype, nullptr, policy);
        o = std::fopen(argv[2], "wb");
        if (!o) return 2;
        std::fwrite(&status, 4, 1, o);
        std::fwrite(res, 1, n * es, o);
        std::fwrite(y, 1, n * es, o);
        std::fwrite(alone, 1, n * es, o);
    } else {
        return 2;
    }
    std::fclose(f);
    std::fclose(o);
    return 0;
}
