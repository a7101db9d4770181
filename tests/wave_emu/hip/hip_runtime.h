// TEST INFRASTRUCTURE ONLY (tests/test_route_emulated.py): a CPU stand-in for
// the HIP device environment, just large enough to compile the routing
// device code (tau.rs_amd/csrc/dispatch.hpp) for the host and run one
// 64-lane wavefront with one std::thread per lane.  Cross-lane operations
// (DPP moves, shuffles, ballots) exchange values through a shared array
// between two barrier phases, so every lane must reach them in the same order,
// as on the GPU, where routing runs them with every lane active.  DPP
// controls follow the CDNA ISA: quad_perm, row_shr, row_mirror,
// row_half_mirror and row_newbcast (lane n of each 16-lane row to all of it).
// Never part of the library build.
#pragma once
#include <barrier>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstring>

#define __device__
#define __host__
#define __global__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define __shared__

struct EmuDim3 {
    unsigned x = 0, y = 0, z = 0;
};
inline thread_local EmuDim3 threadIdx, blockIdx, blockDim, gridDim;

typedef int hipError_t;
typedef void* hipStream_t;
constexpr int hipSuccess = 0;
constexpr int hipErrorInvalidValue = 1;

inline float __uint_as_float(uint32_t u) { return __builtin_bit_cast(float, u); }
inline uint32_t __float_as_uint(float f) { return __builtin_bit_cast(uint32_t, f); }
inline int min(int a, int b) { return a < b ? a : b; }
inline int max(int a, int b) { return a > b ? a : b; }
inline long min(long a, long b) { return a < b ? a : b; }
inline int __popcll(unsigned long long v) { return __builtin_popcountll(v); }
inline int __ffsll(long long v) { return __builtin_ffsll(v); }

namespace emu {
struct Wave {
    std::barrier<> bar{64};
    uint64_t slot[64];
};
inline Wave* wave = nullptr;  // the running wavefront
inline int lane() { return (int)(threadIdx.x & 63); }

// Publishes v, waits for all lanes, returns lane src's value (or `fallback`
// when src < 0), then waits again so that the slots can be reused.
inline uint64_t exchange(uint64_t v, int src, uint64_t fallback) {
    wave->slot[lane()] = v;
    wave->bar.arrive_and_wait();
    const uint64_t r = src >= 0 ? wave->slot[src] : fallback;
    wave->bar.arrive_and_wait();
    return r;
}

// Source lane of DPP control `ctrl` for lane l, or -1 when it has none.
inline int dpp_source(int l, int ctrl) {
    const int row = l & ~15, r = l & 15;
    if (ctrl <= 0xff) {  // quad_perm
        const int q = l & ~3, i = l & 3;
        return q + ((ctrl >> (2 * i)) & 3);
    }
    if (ctrl >= 0x111 && ctrl <= 0x11f) {  // row_shr:n
        const int n = ctrl - 0x110;
        return r >= n ? row + r - n : -1;
    }
    if (ctrl == 0x140) return row + (15 - r);                     // row_mirror
    if (ctrl == 0x141) return row + (r & 8) + (7 - (r & 7));      // row_half_mirror
    if (ctrl >= 0x150 && ctrl <= 0x15f) return row + (ctrl - 0x150);  // row_newbcast:n
    __builtin_trap();
}
}  // namespace emu

inline int emu_update_dpp(int old, int src, int ctrl, int, int, bool) {
    const int s = emu::dpp_source(emu::lane(), ctrl);
    return (int)(uint32_t)emu::exchange((uint32_t)src, s, (uint32_t)old);
}
#define __builtin_amdgcn_update_dpp(old, src, ctrl, rm, bm, bc) emu_update_dpp(old, src, ctrl, rm, bm, bc)

template <typename T>
inline T __shfl(T v, int src, int width = 64) {
    uint64_t bits = 0;
    std::memcpy(&bits, &v, sizeof(T));
    const uint64_t r = emu::exchange(bits, ((src % width) + width) % width, 0);
    T out;
    std::memcpy(&out, &r, sizeof(T));
    return out;
}
template <typename T>
inline T __shfl_up(T v, unsigned d, int width = 64) {
    const int l = emu::lane();
    return __shfl(v, (int)l - (int)d >= 0 ? l - (int)d : l, width);
}
inline uint64_t __ballot(int pred) {
    uint64_t mask = 0;
    emu::wave->slot[emu::lane()] = pred ? 1 : 0;
    emu::wave->bar.arrive_and_wait();
    for (int i = 0; i < 64; ++i) mask |= emu::wave->slot[i] ? (1ull << i) : 0;
    emu::wave->bar.arrive_and_wait();
    return mask;
}
inline int __any(int pred) { return __ballot(pred) != 0; }
inline void __syncthreads() { emu::wave->bar.arrive_and_wait(); }
inline int emu_readlane(int v, int l) { return (int)emu::exchange((uint32_t)v, l, 0); }
#define __builtin_amdgcn_readlane(v, l) emu_readlane(v, l)
#define __builtin_amdgcn_readfirstlane(v) emu_readlane(v, 0)
