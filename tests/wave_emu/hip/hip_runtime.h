// TEST INFRASTRUCTURE ONLY (tests/test_route_emulated.py,
// tests/test_decode_emulated.py): a CPU stand-in for the HIP device
// environment, large enough to compile the library's routing and decode
// kernels for the host and run them.  A workgroup's work items are user-level
// contexts (own stacks, an x86-64 register switch) on one thread, switched at
// barriers; each 64-lane
// wavefront exchanges cross-lane values (DPP moves, shuffles, ballots, MFMA
// operands) through a shared array between two phases of a per-wave barrier,
// so every lane of a wave must reach them in the same order, as on the GPU,
// where these kernels run them with every lane active (a barrier that can
// never complete aborts with a message).  __syncthreads is a workgroup
// barrier; workgroups of a launch run one after another (the kernels emulated
// here never wait on each other).  DPP controls
// follow the CDNA ISA: quad_perm, row_shr, row_mirror, row_half_mirror and
// row_newbcast (lane n of each 16-lane row to all of it).  v_mfma_f32_16x16x32
// _bf16 is computed in f32 with K summed in order (the hardware's internal
// order is not modelled: results are compared to the oracle within tolerance,
// or between kernels that issue the same MFMA sequence).
// Sources with <<< >>> launches and __shared__ declarations are rewritten for
// this header by tests/wave_emu/prep.py.  Never part of the library build.
#pragma once

#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <memory>
#include <tuple>
#include <type_traits>
#include <vector>

#define __device__
#define __host__
#define __global__
#define __forceinline__ inline
#define __launch_bounds__(...)

struct EmuDim3 {
    unsigned x = 0, y = 0, z = 0;
    EmuDim3() = default;
    EmuDim3(unsigned x_, unsigned y_ = 1, unsigned z_ = 1) : x(x_), y(y_), z(z_) {}
};
typedef EmuDim3 dim3;
// The running work item's coordinates (set by the scheduler before it resumes a work item).
inline EmuDim3 threadIdx, blockIdx, blockDim, gridDim;

typedef int hipError_t;
typedef void* hipStream_t;
constexpr int hipSuccess = 0;
constexpr int hipErrorInvalidValue = 1;
constexpr int hipErrorInvalidSymbol = 13;
inline hipError_t hipGetLastError() { return hipSuccess; }
inline hipError_t hipGetDevice(int* d) {
    *d = 0;
    return hipSuccess;
}
inline hipError_t hipGetSymbolAddress(void** p, const void* symbol) {
    *p = const_cast<void*>(symbol);
    return hipSuccess;
}
#define HIP_SYMBOL(x) (&(x))
#define __align__(n) alignas(n)

inline float __uint_as_float(uint32_t u) { return __builtin_bit_cast(float, u); }
inline uint32_t __float_as_uint(float f) { return __builtin_bit_cast(uint32_t, f); }
inline int min(int a, int b) { return a < b ? a : b; }
inline int max(int a, int b) { return a > b ? a : b; }
inline long min(long a, long b) { return a < b ? a : b; }
inline int __popcll(unsigned long long v) { return __builtin_popcountll(v); }
inline int __ffsll(long long v) { return __builtin_ffsll(v); }
inline int atomicAdd(int* p, int v) {  // work items never run at the same time
    const int old = *p;
    *p = old + v;
    return old;
}

namespace emu {
// Work items are user-level contexts on one OS thread, switched at barriers
// (cooperative: a work item runs until it waits at a barrier or returns).
struct Barrier {
    int expected = 0, arrived = 0;
    unsigned generation = 0;
};
// x86-64 context switch: saves the callee-saved registers on the current
// stack, stores the stack pointer in *save, continues on the stack `next`
// (as left by a previous switch, or prepared by make_stack).
__attribute__((naked, noinline)) static void switch_stack(void** save, void* next) {
    asm volatile(
        "push %rbp\n\tpush %rbx\n\tpush %r12\n\tpush %r13\n\tpush %r14\n\tpush %r15\n\t"
        "mov %rsp, (%rdi)\n\tmov %rsi, %rsp\n\t"
        "pop %r15\n\tpop %r14\n\tpop %r13\n\tpop %r12\n\tpop %rbx\n\tpop %rbp\n\tret");
}
// A fresh stack whose first switch enters `entry` (which never returns).
inline void* make_stack(char* base, size_t size, void (*entry)()) {
    uintptr_t top = ((uintptr_t)base + size) & ~(uintptr_t)15;
    void** sp = (void**)top;
    *--sp = nullptr;          // entry's (unused) return address: rsp % 16 == 8 on entry
    *--sp = (void*)entry;     // popped by the switch's ret
    for (int i = 0; i < 6; ++i) *--sp = nullptr;  // rbp, rbx, r12-r15
    return sp;
}

struct Item {
    void* sp = nullptr;
    std::unique_ptr<char[]> stack;
    bool done = false;
    Barrier* waiting = nullptr;  // barrier it waits at
    unsigned gen = 0;            // the barrier's generation when it arrived
};
struct Wave {
    Barrier bar;
    uint64_t slot[64];
    uint32_t a[64][4], b[64][4];
};
struct Group {
    Barrier bar;
    std::vector<Wave> waves;
    std::vector<unsigned char> lds;
    std::vector<Item> items;
    void* scheduler_sp = nullptr;
    unsigned current = 0;
};
inline Group* group = nullptr;
inline const std::function<void()>* body = nullptr;
inline int lane() { return (int)(threadIdx.x & 63); }
inline Wave& wave() { return group->waves[threadIdx.x >> 6]; }
inline void* dynamic_lds() { return group->lds.data(); }

inline void arrive(Barrier& b) {
    Item& me = group->items[group->current];
    me.waiting = &b;
    me.gen = b.generation;
    if (++b.arrived == b.expected) {  // last arrival releases everyone
        b.arrived = 0;
        ++b.generation;
    }
    switch_stack(&me.sp, group->scheduler_sp);
}

// Publishes v, waits for the wave, returns lane src's value (or `fallback`
// when src < 0), then waits again so that the slots can be reused.
inline uint64_t exchange(uint64_t v, int src, uint64_t fallback) {
    Wave& w = wave();
    w.slot[lane()] = v;
    arrive(w.bar);
    const uint64_t r = src >= 0 ? w.slot[src] : fallback;
    arrive(w.bar);
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
    if (ctrl == 0x140) return row + (15 - r);                         // row_mirror
    if (ctrl == 0x141) return row + (r & 8) + (7 - (r & 7));          // row_half_mirror
    if (ctrl >= 0x150 && ctrl <= 0x15f) return row + (ctrl - 0x150);  // row_newbcast:n
    std::fprintf(stderr, "emulator: DPP control %#x not modelled\n", ctrl);
    std::abort();
}

inline void item_entry() {
    (*body)();
    Item& me = group->items[group->current];
    me.done = true;
    switch_stack(&me.sp, group->scheduler_sp);  // never resumed
    std::abort();
}

// Runs grid x block work items, workgroup by workgroup.
inline void launch(EmuDim3 grid, unsigned block, size_t lds, const std::function<void()>& fn) {
    constexpr size_t kStack = 128 * 1024;
    for (unsigned g = 0; g < grid.x * grid.y; ++g) {
        Group grp;
        grp.bar.expected = (int)block;
        grp.waves.resize((block + 63) / 64);
        for (auto& w : grp.waves) w.bar.expected = 64;
        grp.lds.assign(lds + 16, 0xA5);  // stale contents, as LDS holds whatever was there
        grp.items.resize(block);
        group = &grp;
        body = &fn;
        blockIdx = EmuDim3(g % grid.x, g / grid.x, 0);
        blockDim = EmuDim3(block);
        gridDim = grid;
        for (unsigned t = 0; t < block; ++t) {
            Item& it = grp.items[t];
            it.stack.reset(new char[kStack]);
            it.sp = make_stack(it.stack.get(), kStack, item_entry);
        }
        // Round-robin over runnable work items until all have returned.
        for (;;) {
            bool all_done = true, progressed = false;
            for (unsigned t = 0; t < block; ++t) {
                Item& it = grp.items[t];
                if (it.done) continue;
                all_done = false;
                if (it.waiting && it.waiting->generation == it.gen) continue;  // still blocked
                it.waiting = nullptr;
                grp.current = t;
                threadIdx.x = t;
                switch_stack(&grp.scheduler_sp, it.sp);
                progressed = true;
            }
            if (all_done) break;
            if (!progressed) {
                std::fprintf(stderr, "emulator: workgroup %u deadlocked at a barrier\n", g);
                std::abort();
            }
        }
    }
}
// A rewritten launch: config is (grid, block[, lds bytes[, stream]]).
template <typename F, typename G, typename B, typename... Rest>
inline void launch_with(F fn, G grid, B block, Rest... rest) {
    size_t lds = 0;
    if constexpr (sizeof...(Rest) >= 1) lds = (size_t)std::get<0>(std::tuple<Rest...>(rest...));
    if constexpr (std::is_same_v<G, EmuDim3>) launch(grid, (unsigned)block, lds, fn);
    else launch(EmuDim3((unsigned)grid), (unsigned)block, lds, fn);
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
template <typename T>
inline T __shfl_xor(T v, int m, int width = 64) {
    return __shfl(v, emu::lane() ^ m, width);
}
inline uint64_t __ballot(int pred) {
    emu::Wave& w = emu::wave();
    w.slot[emu::lane()] = pred ? 1 : 0;
    emu::arrive(w.bar);
    uint64_t mask = 0;
    for (int i = 0; i < 64; ++i) mask |= w.slot[i] ? (1ull << i) : 0;
    emu::arrive(w.bar);
    return mask;
}
inline int __any(int pred) { return __ballot(pred) != 0; }
inline void __syncthreads() { emu::arrive(emu::group->bar); }
// On the GPU a wave's lanes run in lockstep, so values a wave stores to LDS
// are visible to its other lanes' later loads; the emulator's lanes run apart
// between synchronisation points, and the kernels mark these places.
#define __builtin_amdgcn_wave_barrier() emu::arrive(emu::wave().bar)
inline int emu_readlane(int v, int l) { return (int)emu::exchange((uint32_t)v, l, 0); }
#define __builtin_amdgcn_readlane(v, l) emu_readlane(v, l)
#define __builtin_amdgcn_readfirstlane(v) emu_readlane(v, 0)

namespace emu {
// Wave-instruction counts since the process started (counted by lane 0):
// MFMAs of each shape and direct-to-LDS copies.
inline long long count_mfma16 = 0, count_mfma32 = 0, count_dma16 = 0;
}  // namespace emu

// v_mfma_f32_16x16x32_bf16: lane l holds A[l%16][8(l/16)..+8], B[8(l/16)..+8][l%16]
// and D[4(l/16)+q][l%16], q = 0..3.
typedef __bf16 emu_bf16x8 __attribute__((ext_vector_type(8)));
typedef float emu_f32x4 __attribute__((ext_vector_type(4)));
inline emu_f32x4 emu_mfma_16x16x32_bf16(emu_bf16x8 a, emu_bf16x8 b, emu_f32x4 c) {
    emu::Wave& w = emu::wave();
    const int l = emu::lane();
    if (l == 0) ++emu::count_mfma16;
    std::memcpy(w.a[l], &a, 16);
    std::memcpy(w.b[l], &b, 16);
    emu::arrive(w.bar);
    emu_f32x4 d = c;
    const int j = l % 16;
    for (int q = 0; q < 4; ++q) {
        const int i = 4 * (l / 16) + q;
        float acc = c[q];
        for (int k = 0; k < 32; ++k) {
            const int kq = k / 8, ke = k % 8;
            __bf16 av, bv;
            std::memcpy(&av, (const char*)w.a[kq * 16 + i] + 2 * ke, 2);
            std::memcpy(&bv, (const char*)w.b[kq * 16 + j] + 2 * ke, 2);
            acc += (float)av * (float)bv;
        }
        d[q] = acc;
    }
    emu::arrive(w.bar);
    return d;
}
#define __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, x, y, z) emu_mfma_16x16x32_bf16(a, b, c)

// v_mfma_f32_32x32x16_bf16: lane l holds A[l%32][8(l/32)..+8], B[8(l/32)..+8][l%32]
// and D[8(q/4) + 4(l/32) + q%4][l%32], q = 0..15.
typedef float emu_f32x16 __attribute__((ext_vector_type(16)));
inline emu_f32x16 emu_mfma_32x32x16_bf16(emu_bf16x8 a, emu_bf16x8 b, emu_f32x16 c) {
    emu::Wave& w = emu::wave();
    const int l = emu::lane();
    if (l == 0) ++emu::count_mfma32;
    std::memcpy(w.a[l], &a, 16);
    std::memcpy(w.b[l], &b, 16);
    emu::arrive(w.bar);
    emu_f32x16 d = c;
    const int j = l % 32;
    for (int q = 0; q < 16; ++q) {
        const int i = 8 * (q / 4) + 4 * (l / 32) + q % 4;
        float acc = c[q];
        for (int k = 0; k < 16; ++k) {
            const int kq = k / 8, ke = k % 8;
            __bf16 av, bv;
            std::memcpy(&av, (const char*)w.a[kq * 32 + i] + 2 * ke, 2);
            std::memcpy(&bv, (const char*)w.b[kq * 32 + j] + 2 * ke, 2);
            acc += (float)av * (float)bv;
        }
        d[q] = acc;
    }
    emu::arrive(w.bar);
    return d;
}
#define __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, x, y, z) emu_mfma_32x32x16_bf16(a, b, c)
#define __builtin_amdgcn_iglp_opt(x) ((void)0)
#define __builtin_amdgcn_sched_barrier(x) ((void)0)

namespace emu {
// global_load_lds_dwordx4: each lane copies 16 bytes from its source to the
// wave's LDS base (the first lane's destination) + 16 * lane.
inline void dma16(const uint16_t* src, uint16_t* lds) {
    uint16_t* base = __shfl(lds, 0);
    if (lane() == 0) ++count_dma16;
    std::memcpy(base + 8 * lane(), src, 16);
}
}  // namespace emu
