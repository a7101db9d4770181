// TEST INFRASTRUCTURE ONLY: calls one of the library's reference-compatible C
// ABI entry points (and the separate shared-expert path) on the CPU emulator
// of wave_emu/hip/hip_runtime.h, with buffers described by the input file.
// usage: abi_emu in.bin out.bin
//   in.bin:  int32 mode, nbuf, nint; int32 ints[nint]; then per buffer an int64
//            byte count and that many bytes (a zero count passes a null pointer)
//   out.bin: int32 status; then every buffer's bytes, in order
// Modes (ints in brackets; b<i> = buffer i):
//   0 tau_launch_moe_routing_fp32(b0, b1, [rows])
//   1 tau_launch_moe_prefill_dispatch(b0..b4, [tokens, capacity, tile_rows])
//   2 tau_launch_moe_prefill(b0..b13 = input, logits, gate_up, down, routes, meta,
//       offsets, slots, tiles, projected, activated, contributions, output,
//       receipts, [tokens, hidden, intermediate, capacity, tile m, n, k, warps, stages])
//   3 tau_launch_moe_prefill_gemm(b0..b6 = input, weights, routes, slots, tiles,
//       output, receipt, [tokens, capacity, n, k, down, tile m, n, k, warps, stages])
//   4 tau_launch_silu_and_mul(b0, b1, [rows, columns, dtype])
//   5 tau_launch_moe_shared_combine(b0..b4, [rows, width])
//   6 tau_launch_linear_bf16_fp32(b0, b1, b2, [rows, columns, inner])
//   7 tau_launch_moe_decode_gemm: b0..b(B-1) inputs, bB..b(2B-1) weights,
//       b(2B)..b(3B-1) outputs; the device pointer arrays are built here
//       [batches, columns, inner, profile backend, n, k, warps, stages]
//   8 tau_launch_fused_bf16_moe_decode(b0..b12, [hidden, intermediate, experts,
//       top_k, profile backend, n, k, warps, stages])
//   9 tau_launch_moe_shared_expert_ex(b0..b8 = input, gate_up_s, down_s,
//       gate_weight, routed, activated_ws, shared_ws, output, residual,
//       [tokens, hidden, shared_intermediate, weight_layout]); output = routed
//       when b7 is empty (the in-place form)
//  10 tau_moe_pack_weights(b0 src, b1 dst, [experts, rows, columns])
// Buffers live in an arena mapped at 0x7e0080000000 (low address words with
// bit 31 set).
#include <sys/mman.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "../../include/tau_moe.h"

static char* g_arena = nullptr;
static size_t g_used = 0;
constexpr size_t kArena = (size_t)1 << 31;

static char* take(size_t bytes) {
    bytes = (bytes + 255) / 256 * 256;
    if (g_used + bytes > kArena) std::abort();
    char* p = g_arena + g_used;
    g_used += bytes;
    return p;
}

int main(int argc, char** argv) {
    if (argc != 3) return 2;
    void* hint = (void*)0x7e0080000000ull;
    g_arena = (char*)mmap(hint, kArena, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_FIXED_NOREPLACE,
                          -1, 0);
    if (g_arena != hint) return 4;
    FILE* f = std::fopen(argv[1], "rb");
    if (!f) return 2;
    int hdr[3];
    if (std::fread(hdr, 4, 3, f) != 3) return 2;
    const int mode = hdr[0], nbuf = hdr[1], nint = hdr[2];
    std::vector<int> iv(nint);
    if (nint && std::fread(iv.data(), 4, nint, f) != (size_t)nint) return 2;
    std::vector<char*> b(nbuf, nullptr);
    std::vector<int64_t> sz(nbuf, 0);
    for (int i = 0; i < nbuf; ++i) {
        if (std::fread(&sz[i], 8, 1, f) != 1) return 2;
        if (sz[i] > 0) {
            b[i] = take((size_t)sz[i]);
            if (std::fread(b[i], 1, (size_t)sz[i], f) != (size_t)sz[i]) return 2;
        }
    }
    std::fclose(f);
    auto I = [&](int i) { return iv.at(i); };
    int status = -100;
    switch (mode) {
        case 0:
            status = tau_launch_moe_routing_fp32(b[0], (float*)b[1], I(0), nullptr);
            break;
        case 1:
            status = tau_launch_moe_prefill_dispatch((const float*)b[0], (int*)b[1], (int*)b[2], (int*)b[3],
                                                     (int*)b[4], I(0), I(1), I(2), nullptr);
            break;
        case 2: {
            const TauGemmTile t{I(4), I(5), I(6), I(7), I(8)};
            status = tau_launch_moe_prefill(b[0], b[1], b[2], b[3], (float*)b[4], (int*)b[5], (int*)b[6],
                                            (int*)b[7], (int*)b[8], b[9], b[10], b[11], b[12], I(0), I(1), I(2),
                                            I(3), &t, &t, (int*)b[13], nullptr);
            break;
        }
        case 3: {
            const TauGemmTile t{I(5), I(6), I(7), I(8), I(9)};
            status = tau_launch_moe_prefill_gemm(b[0], b[1], (const float*)b[2], (const int*)b[3],
                                                 (const int*)b[4], b[5], I(0), I(1), I(2), I(3), I(4), &t,
                                                 (int*)b[6], nullptr);
            break;
        }
        case 4:
            status = tau_launch_silu_and_mul(b[0], b[1], I(0), I(1), I(2), nullptr);
            break;
        case 5:
            status = tau_launch_moe_shared_combine(b[0], b[1], b[2], b[3], b[4], I(0), I(1), nullptr);
            break;
        case 6:
            status = tau_launch_linear_bf16_fp32(b[0], b[1], (float*)b[2], I(0), I(1), I(2), nullptr);
            break;
        case 7: {
            const int B = I(0);
            if (nbuf != 3 * B) return 2;
            void** ptrs = (void**)take(sizeof(void*) * 3 * B);  // device pointer arrays
            for (int i = 0; i < 3 * B; ++i) ptrs[i] = b[i];
            const TauDecodeProfile prof{I(3), I(4), I(5), I(6), I(7)};
            status = tau_launch_moe_decode_gemm(ptrs, ptrs + B, ptrs + 2 * B, B, I(1), I(2), &prof, nullptr,
                                                nullptr);
            break;
        }
        case 8: {
            const TauDecodeProfile prof{I(4), I(5), I(6), I(7), I(8)};
            status = tau_launch_fused_bf16_moe_decode(b[0], b[1], b[2], b[3], b[4], b[5], b[6], b[7], b[8], b[9],
                                                      b[10], b[11], b[12], I(0), I(1), I(2), I(3), &prof, &prof,
                                                      nullptr, nullptr);
            break;
        }
        case 9:
            status = tau_launch_moe_shared_expert_ex(b[0], b[1], b[2], b[3], b[4], b[5], b[6], b[7] ? b[7] : b[4],
                                                     I(0), I(1), I(2), I(3), b[8], nullptr);
            break;
        case 10:
            status = tau_moe_pack_weights(b[0], b[1], I(0), I(1), I(2), nullptr);
            break;
        default:
            return 2;
    }
    FILE* o = std::fopen(argv[2], "wb");
    if (!o) return 2;
    std::fwrite(&status, 4, 1, o);
    for (int i = 0; i < nbuf; ++i)
        if (sz[i] > 0) std::fwrite(b[i], 1, (size_t)sz[i], o);
    std::fclose(o);
    return 0;
}
