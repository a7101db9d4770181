// Memory-bound MoE stages: packed SiLU·mul and the shared-expert gate/combine.
//
// silu_and_mul follows crates/cuda-kernels/src/kernels/silu_and_mul.cu:51-76 of
// the reference (packed [gate..., up...] rows, FP32 math, one final round);
// shared_combine follows moe_shared.cu:11-37 (FP32 dot x.w_s, sigmoid, then
// bf16(fma(gate, shared, routed))).  Both are HBM-bound: 128-bit accesses where
// the row width allows, one workgroup per token row for the gate.
#include "kernels.hpp"

namespace tau_amd {
namespace {

template <typename T>
__device__ __forceinline__ float ld(const T* p, long i);
template <>
__device__ __forceinline__ float ld<float>(const float* p, long i) { return p[i]; }
template <>
__device__ __forceinline__ float ld<uint16_t>(const uint16_t* p, long i) { return bf16_bits_to_float(p[i]); }

template <typename T>
__device__ __forceinline__ void st(T* p, long i, float v);
template <>
__device__ __forceinline__ void st<float>(float* p, long i, float v) { p[i] = v; }
template <>
__device__ __forceinline__ void st<uint16_t>(uint16_t* p, long i, float v) { p[i] = float_to_bf16_bits(v); }

template <typename T>
__global__ __launch_bounds__(256) void silu_and_mul_kernel(const T* in, T* out, int rows, int columns) {
    const long n = (long)rows * columns;
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
        const long r = i / columns;
        const int c = (int)(i - r * columns);
        const float g = ld<T>(in, r * 2 * columns + c);
        const float u = ld<T>(in, r * 2 * columns + columns + c);
        st<T>(out, i, silu(g) * u);
    }
}

// One workgroup per token: gate = sigmoid(sum_h x[h] * w[h]) in FP32, then
// out = bf16(fma(gate, shared, routed)).  A null weight means an ungated
// shared expert (gate = 1).
__global__ __launch_bounds__(256) void shared_combine_kernel(const uint16_t* x, const uint16_t* w,
                                                             const uint16_t* shared, const uint16_t* routed,
                                                             uint16_t* out, int width, const uint16_t* residual) {
    __shared__ float partial[4];
    const long row = (long)blockIdx.x * width;
    float gate = 1.0f;
    if (w) {
        float s = 0.f;
        for (int c = threadIdx.x; c < width; c += 256) s += bf16_bits_to_float(x[row + c]) * bf16_bits_to_float(w[c]);
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) s += __shfl_xor(s, d, 64);
        if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = s;
        __syncthreads();
        gate = sigmoid((partial[0] + partial[1]) + (partial[2] + partial[3]));
    }
    for (int c = threadIdx.x; c < width; c += 256) {
        float v = fmaf(gate, bf16_bits_to_float(shared[row + c]), bf16_bits_to_float(routed[row + c]));
        if (residual) v = round_bf16(v) + bf16_bits_to_float(residual[row + c]);  // fused residual add
        out[row + c] = float_to_bf16_bits(v);
    }
}

// Row-major W[e][rows][cols] -> frag16: 16-byte piece p of the output holds
// row 16*band + lane%16, columns 32*kc + 8*(lane/16) .. +8, where
// p = ((e*bands + band)*kchunks + kc)*64 + lane.  One thread per piece; the
// writes are fully coalesced, the reads are 16-byte segments of 16 rows.
__global__ void pack_frag16_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst, int rows,
                                   int cols, long pieces) {
    const int kchunks = cols / 32, bands = rows / 16;
    for (long p = blockIdx.x * (long)blockDim.x + threadIdx.x; p < pieces; p += (long)gridDim.x * blockDim.x) {
        const int lane = (int)(p & 63);
        const long f = p >> 6;
        const int kc = (int)(f % kchunks);
        const long eb = f / kchunks;
        const int band = (int)(eb % bands);
        const long e = eb / bands;
        const long row = (long)band * 16 + (lane & 15);
        const long col = (long)kc * 32 + (lane >> 4) * 8;
        *(u32x4*)(dst + p * 8) = *(const u32x4*)(src + (e * rows + row) * cols + col);
    }
}

// out[r, c] += bias[c] (f32, one add after the projection, as a Linear with bias).
__global__ void add_bias_kernel(float* __restrict__ out, const float* __restrict__ bias, long rows, int cols) {
    const long n = rows * cols;
    for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
        out[i] += bias[i % cols];
}

}  // namespace

int launch_add_bias(float* out, const float* bias, int rows, int cols, hipStream_t s) {
    if (!out || !bias || rows <= 0 || cols <= 0) return kInvalid;
    long blocks = ((long)rows * cols + 255) / 256;
    if (blocks > 65535L * 8) blocks = 65535L * 8;
    add_bias_kernel<<<(unsigned)blocks, 256, 0, s>>>(out, bias, rows, cols);
    return (int)hipGetLastError();
}

int launch_pack_frag16(const void* src, void* dst, int experts, int rows, int cols, hipStream_t s) {
    const long pieces = (long)experts * rows * cols / 8;
    long blocks = (pieces + 255) / 256;
    if (blocks > 65535L * 8) blocks = 65535L * 8;
    pack_frag16_kernel<<<(unsigned)blocks, 256, 0, s>>>((const uint16_t*)src, (uint16_t*)dst, rows, cols, pieces);
    return (int)hipGetLastError();
}

int launch_silu_and_mul(const void* in, void* out, int rows, int columns, int dtype, hipStream_t s) {
    if (!in || !out || rows <= 0 || columns <= 0 || (dtype != 0 && dtype != 1)) return kInvalid;
    const long n = (long)rows * columns;
    long blocks = (n + 255) / 256;
    if (blocks > 65535L * 8) blocks = 65535L * 8;
    if (dtype == 0)
        silu_and_mul_kernel<float><<<(unsigned)blocks, 256, 0, s>>>((const float*)in, (float*)out, rows, columns);
    else
        silu_and_mul_kernel<uint16_t>
            <<<(unsigned)blocks, 256, 0, s>>>((const uint16_t*)in, (uint16_t*)out, rows, columns);
    return (int)hipGetLastError();
}

int launch_shared_combine(const void* x, const void* w, const void* shared, const void* routed, void* out,
                          int rows, int width, const void* residual, hipStream_t s) {
    if (!x || !shared || !routed || !out || rows <= 0 || width <= 0) return kInvalid;
    shared_combine_kernel<<<rows, 256, 0, s>>>((const uint16_t*)x, (const uint16_t*)w, (const uint16_t*)shared,
                                               (const uint16_t*)routed, (uint16_t*)out, width,
                                               (const uint16_t*)residual);
    return (int)hipGetLastError();
}

}  // namespace tau_amd
