// Single-token decode entry points of the reference ABI.
//
// tau_launch_moe_decode_gemm replaces the reference's pointer-array decode
// projection (crates/cuda-kernels/src/kernels/moe_decode_gemm.cu:125-147) and
// tau_launch_fused_bf16_moe_decode its one-token pipeline
// (fused_bf16_moe_decode.cu:56-91): route -> per-rank gate_up GEMV (f32) ->
// BF16 store -> SiLU·mul -> per-rank down GEMV (f32) -> weighted BF16 store ->
// rank-ordered combine.  Every intermediate buffer the reference fills is
// filled here too, with the same rounding points.
//
// CDNA4 design: the GEMVs are weight-streaming waves; each wave owns 16 weight
// rows, loads them with 128-bit loads straight into the A operand of
// v_mfma_f32_16x16x32_bf16 and supplies the input vector as B column 0, so one
// MFMA retires a 16x32 slice of the dot products.  Experts are read from the
// device-side routing result, so no host readback or pointer rebuild is needed.
#include "kernels.hpp"

namespace tau_amd {
int launch_silu_and_mul(const void* in, void* out, int rows, int columns, int dtype, hipStream_t s);
}

using namespace tau_amd;

namespace {

constexpr int kExperts = 256, kTopK = 8;
constexpr int kGemvWaves = 4;

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ u32x4 chunk_or_zero(const uint16_t* row, int k, int K, bool ok) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (!ok) return v;
    if (k + 8 <= K && ((uintptr_t)(row + k) % 16) == 0) return *(const u32x4*)(row + k);
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
        const uint32_t lo = k + j < K ? row[k + j] : 0u;
        const uint32_t hi = k + j + 1 < K ? row[k + j + 1] : 0u;
        v[j / 2] = lo | (hi << 16);
    }
    return v;
}

// out[c] = sum_k W[c, k] * x[k] for 16 rows per wave.  x supplied as B column 0.
__device__ __forceinline__ void gemv16(const uint16_t* W, const uint16_t* x, float* out, int columns, int inner) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c0 = (blockIdx.x * kGemvWaves + wave) * 16;
    if (c0 >= columns) return;
    const int col = c0 + (lane & 15), kofs = (lane >> 4) * 8;
    const bool w_ok = col < columns;
    const bool x_ok = (lane & 15) == 0;
    const uint16_t* wrow = W + (long)(w_ok ? col : 0) * inner;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int kb = 0; kb < inner; kb += 32) {
        const u32x4 a = chunk_or_zero(wrow, kb + kofs, inner, w_ok);
        const u32x4 b = chunk_or_zero(x, kb + kofs, inner, x_ok);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), acc, 0, 0, 0);
    }
    // Column 0 of the 16x16 result lives in lanes 0, 16, 32, 48 (4 rows each).
    if ((lane & 15) == 0) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int c = c0 + (lane >> 4) * 4 + q;
            if (c < columns) out[c] = acc[q];
        }
    }
}

__global__ __launch_bounds__(64 * kGemvWaves) void ptr_gemv_kernel(const uint16_t* const* inputs,
                                                                   const uint16_t* const* weights,
                                                                   float* const* outputs, int columns, int inner,
                                                                   int* receipt) {
    if (receipt && blockIdx.x == 0 && threadIdx.x == 0) {
        int* r = receipt + blockIdx.y * 5;
        r[0] = 3; r[1] = 16 * kGemvWaves; r[2] = 32; r[3] = kGemvWaves; r[4] = 1;
    }
    gemv16(weights[blockIdx.y], inputs[blockIdx.y], outputs[blockIdx.y], columns, inner);
}

// Per-rank GEMV with the expert read from the device: out[r] = W[ids[r]] . x_r.
__global__ __launch_bounds__(64 * kGemvWaves) void rank_gemv_kernel(const uint16_t* x, long x_stride,
                                                                    const uint16_t* W, long w_stride,
                                                                    const int* ids, float* out, int columns,
                                                                    int inner, int* receipt) {
    const int r = blockIdx.y;
    if (receipt && blockIdx.x == 0 && threadIdx.x == 0) {
        int* q = receipt + r * 5;
        q[0] = 3; q[1] = 16 * kGemvWaves; q[2] = 32; q[3] = kGemvWaves; q[4] = 1;
    }
    gemv16(W + (long)ids[r] * w_stride, x + r * x_stride, out + (long)r * columns, columns, inner);
}

// Reads the packed route row; a malformed rank uses expert 0 with a NaN
// weight (fused_bf16_moe_decode.cu:18-43) so no out-of-range weight is read.
__global__ void prepare_kernel(const float* routes, int* ids, float* weights) {
    const int r = threadIdx.x;
    if (r >= kTopK) return;
    const float id = routes[r], w = routes[kTopK + r];
    const bool valid = __builtin_isfinite(id) && id >= 0.f && id < (float)kExperts && __builtin_isfinite(w);
    ids[r] = valid ? (int)id : 0;
    weights[r] = valid ? w : __builtin_nanf("");
}

// out[i] = bf16(in[i] * (weights ? weights[i / columns] : 1)).
__global__ __launch_bounds__(256) void weighted_store_kernel(const float* in, const float* weights, uint16_t* out,
                                                             int columns, long count) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i < count) out[i] = float_to_bf16_bits(weights ? in[i] * weights[i / columns] : in[i]);
}

// out[h] = bf16(sum_r f32(experts[r, h])), ranks in order.
__global__ __launch_bounds__(256) void rank_combine_kernel(const uint16_t* experts, uint16_t* out, int hidden) {
    const int h = blockIdx.x * 256 + threadIdx.x;
    if (h >= hidden) return;
    float s = 0.f;
    for (int r = 0; r < kTopK; ++r) s += bf16_bits_to_float(experts[(long)r * hidden + h]);
    out[h] = float_to_bf16_bits(s);
}

bool profile_ok(const TauDecodeProfile* c) {
    if (!c) return false;
    if (c->backend == 0) return c->n == 16 && c->k == 16 && c->warps == 1 && c->stages == 1;
    if (c->backend != 1 && c->backend != 2) return false;
    const bool n = c->n == 32 || c->n == 64 || c->n == 128;
    const bool k = c->k == 32 || c->k == 64 || c->k == 128;
    const bool w = c->warps == 1 || c->warps == 2 || c->warps == 4 || c->warps == 8;
    const bool s = c->stages == 1 || c->stages == 2;
    return n && k && w && s;
}

}  // namespace

extern "C" {

int tau_launch_moe_decode_gemm(const void* inputs, const void* weights, void* outputs, int batches, int columns,
                               int inner, const TauDecodeProfile* config, int* receipts, void* stream) {
    if (!inputs || !weights || !outputs || !profile_ok(config) || batches <= 0 || batches > 65535 ||
        columns <= 0 || inner <= 0)
        return kInvalid;
    dim3 grid((columns + 16 * kGemvWaves - 1) / (16 * kGemvWaves), batches);
    ptr_gemv_kernel<<<grid, 64 * kGemvWaves, 0, (hipStream_t)stream>>>(
        (const uint16_t* const*)inputs, (const uint16_t* const*)weights, (float* const*)outputs, columns, inner,
        receipts);
    return (int)hipGetLastError();
}

int tau_launch_fused_bf16_moe_decode(const void* input, const void* logits, const void* gate_up,
                                     const void* down, void* selected_ids, void* selected_weights,
                                     void* pointer_workspace, void* gate_up_output, void* activated_output,
                                     void* expert_output, void* gate_up_fp32, void* expert_fp32, void* output,
                                     int hidden, int intermediate, int num_experts, int top_k,
                                     const TauDecodeProfile* gate_up_config, const TauDecodeProfile* down_config,
                                     int* receipts, void* stream) {
    if (!input || !logits || !gate_up || !down || !selected_ids || !selected_weights || !pointer_workspace ||
        !gate_up_output || !activated_output || !expert_output || !gate_up_fp32 || !expert_fp32 || !output ||
        hidden <= 0 || intermediate <= 0 || !profile_ok(gate_up_config) || !profile_ok(down_config) ||
        num_experts != kExperts || top_k != kTopK)
        return -1;
    hipStream_t s = (hipStream_t)stream;
    float* routes = (float*)pointer_workspace;
    int code = launch_routing(logits, 1, routes, 1, kExperts, kTopK, s);
    if (code) return code;
    int* ids = (int*)selected_ids;
    float* wts = (float*)selected_weights;
    prepare_kernel<<<1, 64, 0, s>>>(routes, ids, wts);
    if ((code = (int)hipGetLastError())) return code;
    const int two_i = 2 * intermediate;
    dim3 g1((two_i + 16 * kGemvWaves - 1) / (16 * kGemvWaves), kTopK);
    rank_gemv_kernel<<<g1, 64 * kGemvWaves, 0, s>>>((const uint16_t*)input, 0, (const uint16_t*)gate_up,
                                                    (long)two_i * hidden, ids, (float*)gate_up_fp32, two_i,
                                                    hidden, receipts);
    if ((code = (int)hipGetLastError())) return code;
    const long n1 = (long)kTopK * two_i;
    weighted_store_kernel<<<(unsigned)((n1 + 255) / 256), 256, 0, s>>>((const float*)gate_up_fp32, nullptr,
                                                                      (uint16_t*)gate_up_output, two_i, n1);
    if ((code = (int)hipGetLastError())) return code;
    code = launch_silu_and_mul(gate_up_output, activated_output, kTopK, intermediate, 1, s);
    if (code) return code;
    dim3 g2((hidden + 16 * kGemvWaves - 1) / (16 * kGemvWaves), kTopK);
    rank_gemv_kernel<<<g2, 64 * kGemvWaves, 0, s>>>((const uint16_t*)activated_output, intermediate,
                                                    (const uint16_t*)down, (long)hidden * intermediate, ids,
                                                    (float*)expert_fp32, hidden, intermediate,
                                                    receipts ? receipts + kTopK * 5 : nullptr);
    if ((code = (int)hipGetLastError())) return code;
    const long n2 = (long)kTopK * hidden;
    weighted_store_kernel<<<(unsigned)((n2 + 255) / 256), 256, 0, s>>>((const float*)expert_fp32, wts,
                                                                      (uint16_t*)expert_output, hidden, n2);
    if ((code = (int)hipGetLastError())) return code;
    rank_combine_kernel<<<(hidden + 255) / 256, 256, 0, s>>>((const uint16_t*)expert_output, (uint16_t*)output,
                                                             hidden);
    return (int)hipGetLastError();
}

}  // extern "C"
