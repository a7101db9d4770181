// Router projection with the bias add fused, then routing (Router::logits and
// Router::reference_plan of crates/models/src/components/sparse_moe/
// routing.rs:91-93,125-231; the native routing of kernels/moe_routing.cu:15-52).
//
//   logits[t, e] = sum_h x[t, h] * W[e, h]  (+ bias[e])     f32, BF16 operands
//   routes[t]    = route_row(logits[t])                      ids + weights, [T, 2K]
//
// The projection is a skinny GEMM (E is 8..512): one workgroup per 16 tokens x
// 16*EB router rows, sixteen waves splitting K into sixteen slices, so every
// wave issues its whole slice's loads in one or two batches and the latency
// chain per wave stays short (a workgroup that owned all E rows would stream
// the full E*H*2 bytes itself).  Each wave runs v_mfma_f32_16x16x32_bf16 with
// 16 router rows as the A operand and the 16 tokens as the B operand; the
// sixteen K-slice partials are summed in LDS in slice order (deterministic),
// the bias is added once, and the f32 logits are written.  The routing kernel
// then routes them.  Needs H % 32 == 0 and 16-byte aligned x and W.
#include "kernels.hpp"

namespace tau_amd {
namespace {

constexpr int kRouterTokens = 16;
constexpr int kSlices = 16;  // waves per workgroup, one K slice each

__device__ __forceinline__ bf16x8 router_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// EB: 16-row router blocks per workgroup.
template <int EB>
__global__ __launch_bounds__(64 * kSlices) void router_logits_kernel(const uint16_t* x, const uint16_t* w,
                                                                     const float* bias, float* logits, int T, int H,
                                                                     int E) {
    __shared__ float part[kSlices][kRouterTokens][16 * EB];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t0 = blockIdx.x * kRouterTokens;
    const int e0 = blockIdx.y * 16 * EB;
    const int steps = H / 32, per = (steps + kSlices - 1) / kSlices;
    const int k_begin = min(steps, wave * per) * 32, k_end = min(steps, (wave + 1) * per) * 32;

    // Operand rows: token t0 + lane%16 and router row e0 + 16*b + lane%16 (clamped).
    const int kofs = (lane >> 4) * 8;
    const uint16_t* xrow = x + (size_t)min(t0 + (lane & 15), T - 1) * H + kofs;
    const uint16_t* wrow[EB];
#pragma unroll
    for (int b = 0; b < EB; ++b) wrow[b] = w + (size_t)min(e0 + 16 * b + (lane & 15), E - 1) * H + kofs;
    f32x4 acc[EB];
#pragma unroll
    for (int b = 0; b < EB; ++b)
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[b][q] = 0.f;

    // Batches of U K steps, all loads of a batch issued before its MFMAs.
    constexpr int U = 8 / EB;
    for (int kb = k_begin; kb < k_end; kb += 32 * U) {
        u32x4 xv[U], wv[EB][U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = min(kb + 32 * u, k_end - 32);  // clamped: the tail batch repeats a step, masked below
            xv[u] = *(const u32x4*)(xrow + k);
#pragma unroll
            for (int b = 0; b < EB; ++b) wv[b][u] = *(const u32x4*)(wrow[b] + k);
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (kb + 32 * u < k_end)
#pragma unroll
                for (int b = 0; b < EB; ++b)
                    acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(router_bf16x8(wv[b][u]), router_bf16x8(xv[u]),
                                                                     acc[b], 0, 0, 0);
    }

    // Value q of lane l: row e0 + 16*b + (l/16)*4 + q, token t0 + l%16.
#pragma unroll
    for (int b = 0; b < EB; ++b)
#pragma unroll
        for (int q = 0; q < 4; ++q) part[wave][lane & 15][16 * b + (lane >> 4) * 4 + q] = acc[b][q];
    __syncthreads();

    // Slice partials summed in slice order, then the bias; one (token, row) per thread.
    for (int j = threadIdx.x; j < kRouterTokens * 16 * EB; j += 64 * kSlices) {
        const int t = j / (16 * EB), e = j - t * (16 * EB);
        if (t0 + t >= T || e0 + e >= E) continue;
        float v = part[0][t][e];
#pragma unroll
        for (int sl = 1; sl < kSlices; ++sl) v = v + part[sl][t][e];
        if (bias) v = v + bias[e0 + e];
        logits[(size_t)(t0 + t) * E + e0 + e] = v;
    }
}

template <int EB>
int launch_router_logits_t(const uint16_t* x, const uint16_t* w, const float* bias, float* logits, int T, int H,
                           int E, hipStream_t s) {
    const dim3 grid((unsigned)((T + kRouterTokens - 1) / kRouterTokens), (unsigned)((E + 16 * EB - 1) / (16 * EB)));
    router_logits_kernel<EB><<<grid, 64 * kSlices, 0, s>>>(x, w, bias, logits, T, H, E);
    return (int)hipGetLastError();
}

}  // namespace

bool router_logits_supported(const void* x, const void* w, int hidden, int experts) {
    return hidden > 0 && hidden % 32 == 0 && ((uintptr_t)x % 16) == 0 && ((uintptr_t)w % 16) == 0 && experts > 0;
}

// Router blocks per workgroup: one at decode sizes (most workgroups), four once
// there are enough token groups to fill the GPU (x tiles re-read 4x less).
int launch_router_logits(const void* input, const void* weight, const float* bias, float* logits, int tokens,
                         int hidden, int experts, hipStream_t s) {
    if (!input || !weight || !logits || tokens <= 0 || !router_logits_supported(input, weight, hidden, experts))
        return kInvalid;
    const uint16_t* x = (const uint16_t*)input;
    const uint16_t* w = (const uint16_t*)weight;
    const long groups = (tokens + kRouterTokens - 1) / kRouterTokens;
    if (groups >= 128 && experts >= 64)
        return launch_router_logits_t<4>(x, w, bias, logits, tokens, hidden, experts, s);
    return launch_router_logits_t<1>(x, w, bias, logits, tokens, hidden, experts, s);
}

}  // namespace tau_amd
