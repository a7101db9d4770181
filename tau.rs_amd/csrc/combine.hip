// Rank-ordered combine of the weighted expert contributions.
//
// out[t, h] = bf16(sum_{r=0..K-1} f32(contributions[t*K + r, h])), the ranks
// added in order starting from zero (the reference's combine_ranked,
// crates/cuda-kernels/src/kernels/moe_dispatch.cuh:13-20, and the CPU loop of
// crates/models/src/components/sparse_moe/experts.rs:142-151); every element is
// NaN when the dispatch marked the plan invalid (moe_dispatch.cu:78-85).
// With a residual, out = bf16(f32(bf16(sum)) + f32(residual)): the layer's
// residual add (decoder.rs:96-116 of qwen3_5_common) fused, bit-identical to
// the separate BF16 add.  HBM-bound: each thread moves 16-byte vectors.
#include "kernels.hpp"

namespace tau_amd {
namespace {

// Ordered combine: out[t,h] = bf16(sum_r f32(contrib[t*K + r, h])), ranks in order
// (moe_dispatch.cuh:13-20); NaN everywhere when the plan was invalid.
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t* contributions, uint16_t* output,
                                                      const int* status, int T_, int H, int K,
                                                      const uint16_t* residual) {
    const int chunks = H / 8;
    const long idx = (long)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (long)T_ * chunks) return;
    const int t = (int)(idx / chunks), c = (int)(idx - (long)t * chunks);
    const bool invalid = status[0] != 0;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const uint16_t* base = contributions + (size_t)t * K * H + c * 8;
    for (int r = 0; r < K; ++r) {
        const u32x4 v = *(const u32x4*)(base + (size_t)r * H);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            acc[2 * q] += __uint_as_float(v[q] << 16);
            acc[2 * q + 1] += __uint_as_float(v[q] & 0xffff0000u);
        }
    }
    if (residual) {
        const u32x4 rv = *(const u32x4*)(residual + (size_t)t * H + c * 8);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            acc[2 * q] = round_bf16(acc[2 * q]) + __uint_as_float(rv[q] << 16);
            acc[2 * q + 1] = round_bf16(acc[2 * q + 1]) + __uint_as_float(rv[q] & 0xffff0000u);
        }
    }
    u32x4 o;
#pragma unroll
    for (int q = 0; q < 4; ++q)
        o[q] = invalid ? 0x7fc07fc0u : pack_bf16x2(acc[2 * q], acc[2 * q + 1]);
    *(u32x4*)(output + (size_t)t * H + c * 8) = o;
}

// Scalar combine for hidden sizes that are not multiples of eight.
__global__ __launch_bounds__(256) void combine_scalar_kernel(const uint16_t* contributions, uint16_t* output,
                                                             const int* status, int T_, int H, int K,
                                                             const uint16_t* residual) {
    const long idx = (long)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (long)T_ * H) return;
    const int t = (int)(idx / H), h = (int)(idx - (long)t * H);
    float acc = 0.f;
    for (int r = 0; r < K; ++r) acc += bf16_bits_to_float(contributions[((size_t)t * K + r) * H + h]);
    if (residual) acc = round_bf16(acc) + bf16_bits_to_float(residual[idx]);
    output[idx] = status[0] ? (uint16_t)0x7fc0 : float_to_bf16_bits(acc);
}

}  // namespace

int launch_combine(const void* contributions, void* output, const int* status, int tokens, int H, int K,
                   const void* residual, hipStream_t s) {
    if (!contributions || !output || !status || tokens <= 0 || H <= 0 || K <= 0) return kInvalid;
    if (H % 8 == 0) {
        const long n = (long)tokens * (H / 8);
        combine_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(
            (const uint16_t*)contributions, (uint16_t*)output, status, tokens, H, K, (const uint16_t*)residual);
    } else {
        const long n = (long)tokens * H;
        combine_scalar_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(
            (const uint16_t*)contributions, (uint16_t*)output, status, tokens, H, K, (const uint16_t*)residual);
    }
    return (int)hipGetLastError();
}

}  // namespace tau_amd
