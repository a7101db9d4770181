// Centered RMSNorm and the fused residual add + centered RMSNorm that feeds the
// MoE block (the decoder layer's post-attention norm: forward_block of
// crates/models/src/qwen3_5_common/decoder.rs:95-116, CenteredRmsNorm of
// crates/models/src/components/rms_norm.rs:39-74,107-150, native kernels in
// crates/cuda-kernels/src/kernels/centered_rms_norm.cu:269-435).
//
//   residual[t, h] = input[t, h] + branch[t, h]      rounded in the storage dtype
//   inv_rms[t]     = 1 / sqrt(sum_h residual[t, h]^2 / H + eps)     (f32)
//   output[t, h]   = (residual[t, h] * inv_rms[t]) * (1 + weight[h]) rounded once
//
// The standalone norm is the same kernel with no branch (residual = input).
// One wave per row: each lane owns chunks of 16 bytes (8 BF16 or 4 FP32
// values) at chunk index v*64 + lane, sums its squares in chunk order, and the
// 64 lane sums are combined by an xor butterfly, after which every lane holds
// the same total bit for bit.  Rows whose chunks fit in registers keep the
// rounded residual there between the two passes; wider rows recompute it from
// the inputs (the same values).  16-byte accesses are used when every pointer
// and the row stride are 16-byte aligned; the scalar path reads and writes the
// same elements in the same order, so both produce identical bits.  HBM-bound:
// 2 reads + 2 writes of [T, H] per fused call, 1 + 1 standalone.
#include "kernels.hpp"

namespace tau_amd {
namespace {

constexpr int kNormRowsPerBlock = 4;  // one wave per row, 256 threads

template <typename T>
__device__ __forceinline__ float storage_round(float v) {
    if constexpr (sizeof(T) == 2) return round_bf16(v);
    else return v;
}

// The chunk's 16 bytes (n <= V valid values, zeros past them) in storage
// order, by one 16-byte load or by element loads.
template <typename T, bool VEC>
__device__ __forceinline__ u32x4 load_raw(const T* p, size_t base, int n) {
    constexpr int V = 16 / sizeof(T);
    if constexpr (VEC) {
        return *(const u32x4*)(p + base);
    } else {
        u32x4 raw = {0u, 0u, 0u, 0u};
        if constexpr (sizeof(T) == 2) {
#pragma unroll
            for (int q = 0; q < V; ++q) {
                const uint32_t h = q < n ? (uint32_t)((const uint16_t*)p)[base + q] : 0u;
                raw[q >> 1] |= (q & 1) ? h << 16 : h;
            }
        } else {
#pragma unroll
            for (int q = 0; q < V; ++q) raw[q] = q < n ? __float_as_uint(((const float*)p)[base + q]) : 0u;
        }
        return raw;
    }
}

// Packs V values (already representable in T) into the chunk's 16 bytes.
template <typename T>
__device__ __forceinline__ u32x4 pack_chunk(const float* v) {
    u32x4 raw;
    if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int q = 0; q < 4; ++q) raw[q] = pack_bf16x2(v[2 * q], v[2 * q + 1]);
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) raw[q] = __float_as_uint(v[q]);
    }
    return raw;
}

template <typename T>
__device__ __forceinline__ void unpack_chunk(u32x4 raw, float* v) {
    if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] = __uint_as_float(q & 1 ? raw[q >> 1] & 0xffff0000u : raw[q >> 1] << 16);
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = __uint_as_float(raw[q]);
    }
}

// Stores the n valid values of one chunk, rounded to T.
template <typename T, bool VEC>
__device__ __forceinline__ void store_chunk(T* p, size_t base, int n, const float* v) {
    constexpr int V = 16 / sizeof(T);
    if constexpr (VEC) {
        *(u32x4*)(p + base) = pack_chunk<T>(v);
    } else {
#pragma unroll
        for (int q = 0; q < V; ++q) {
            if (q < n) {
                if constexpr (sizeof(T) == 2) p[base + q] = float_to_bf16_bits(v[q]);
                else p[base + q] = v[q];
            }
        }
    }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// MAXV > 0: rows of at most MAXV chunks per lane keep the residual (and, up
// to 8 chunks, the weight) in registers between the passes; MAXV == 0: any
// width, the second pass reloads the inputs and recomputes the residual (the
// same values).  Loads are issued kG chunks at a time, all before the
// group's stores (outputs never overlap the inputs), so a row costs one or
// two memory round trips instead of one per chunk.
template <typename T, bool VEC, int MAXV>
__global__ __launch_bounds__(64 * kNormRowsPerBlock) void residual_norm_kernel(const T* input, const T* branch,
                                                                               const T* weight, T* residual_out,
                                                                               T* out, int rows, int H, float eps) {
    constexpr int V = 16 / sizeof(T);
    constexpr int kG = 4;                        // chunks per load group
    constexpr bool kKeepW = MAXV > 0 && MAXV <= 8;
    constexpr int KV = MAXV > 0 ? MAXV : 1;
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * kNormRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;  // the whole wave
    const size_t off = (size_t)row * H;
    const int chunks = (H + V - 1) / V;
    const int nv = (chunks + 63) / 64;
    const int groups = (nv + kG - 1) / kG;
    auto valid = [&](int v) { return v < nv && v * 64 + lane < chunks; };
    auto count = [&](int v) { return min(V, H - (v * 64 + lane) * V); };

    // Residual of chunk v from its raw input and branch, rounded in the storage dtype.
    auto residual = [&](u32x4 xr, u32x4 br, float* r) {
        unpack_chunk<T>(xr, r);
        if (branch) {
            float b[V];
            unpack_chunk<T>(br, b);
#pragma unroll
            for (int q = 0; q < V; ++q) r[q] = storage_round<T>(r[q] + b[q]);
        }
    };
    // Loads of one group: input, branch and (when wanted) weight chunks.
    auto load_group = [&](int v0, u32x4* xr, u32x4* br, u32x4* wr, bool want_w) {
#pragma unroll
        for (int g = 0; g < kG; ++g) {
            const int v = v0 + g;
            if (!valid(v)) continue;
            const int c = v * 64 + lane, n = count(v);
            xr[g] = load_raw<T, VEC>(input, off + (size_t)c * V, n);
            if (branch) br[g] = load_raw<T, VEC>(branch, off + (size_t)c * V, n);
            if (want_w) wr[g] = load_raw<T, VEC>(weight, (size_t)c * V, n);
        }
    };

    u32x4 keep[KV], wkeep[kKeepW ? KV : 1];
    float ss = 0.f;
    auto pass1_group = [&](int v0) {
        u32x4 xr[kG], br[kG], wr[kG];
        load_group(v0, xr, br, wr, kKeepW);
#pragma unroll
        for (int g = 0; g < kG; ++g) {
            const int v = v0 + g;
            if (!valid(v)) continue;
            const int c = v * 64 + lane, n = count(v);
            float r[V];
            residual(xr[g], br[g], r);
            if (residual_out) store_chunk<T, VEC>(residual_out, off + (size_t)c * V, n, r);
#pragma unroll
            for (int q = 0; q < V; ++q)
                if (q < n) ss += r[q] * r[q];
            if constexpr (MAXV > 0) {
                keep[min(v, KV - 1)] = pack_chunk<T>(r);
                if constexpr (kKeepW) wkeep[min(v, KV - 1)] = wr[g];
            }
        }
    };
    if constexpr (MAXV > 0) {
#pragma unroll
        for (int v0 = 0; v0 < MAXV; v0 += kG)
            if (v0 / kG < groups) pass1_group(v0);
    } else {
        for (int v0 = 0; v0 < nv; v0 += kG) pass1_group(v0);
    }

    const float total = wave_sum(ss);
    const float inv = 1.0f / sqrtf(total / (float)H + eps);

    auto pass2_group = [&](int v0) {
        u32x4 xr[kG], br[kG], wr[kG];
        if constexpr (MAXV == 0) {
            load_group(v0, xr, br, wr, true);
        } else if constexpr (!kKeepW) {
#pragma unroll
            for (int g = 0; g < kG; ++g)
                if (valid(v0 + g))
                    wr[g] = load_raw<T, VEC>(weight, (size_t)((v0 + g) * 64 + lane) * V, count(v0 + g));
        }
#pragma unroll
        for (int g = 0; g < kG; ++g) {
            const int v = v0 + g;
            if (!valid(v)) continue;
            const int c = v * 64 + lane, n = count(v);
            float r[V], w[V], o[V];
            if constexpr (MAXV > 0) unpack_chunk<T>(keep[min(v, KV - 1)], r);
            else residual(xr[g], br[g], r);
            if constexpr (kKeepW) unpack_chunk<T>(wkeep[min(v, KV - 1)], w);
            else unpack_chunk<T>(wr[g], w);
#pragma unroll
            for (int q = 0; q < V; ++q) o[q] = (r[q] * inv) * (1.0f + w[q]);
            store_chunk<T, VEC>(out, off + (size_t)c * V, n, o);
        }
    };
    if constexpr (MAXV > 0) {
#pragma unroll
        for (int v0 = 0; v0 < MAXV; v0 += kG)
            if (v0 / kG < groups) pass2_group(v0);
    } else {
        for (int v0 = 0; v0 < nv; v0 += kG) pass2_group(v0);
    }
}

template <typename T, bool VEC>
int launch_norm_typed(const T* input, const T* branch, const T* weight, T* residual_out, T* out, int rows, int H,
                      float eps, hipStream_t s) {
    constexpr int V = 16 / sizeof(T);
    const long chunks = ((long)H + V - 1) / V;
    const long nv = (chunks + 63) / 64;
    const unsigned grid = (unsigned)(((long)rows + kNormRowsPerBlock - 1) / kNormRowsPerBlock);
    const unsigned threads = 64 * kNormRowsPerBlock;
    if (nv <= 2)
        residual_norm_kernel<T, VEC, 2><<<grid, threads, 0, s>>>(input, branch, weight, residual_out, out, rows, H, eps);
    else if (nv <= 8)
        residual_norm_kernel<T, VEC, 8><<<grid, threads, 0, s>>>(input, branch, weight, residual_out, out, rows, H, eps);
    else if (nv <= 16)
        residual_norm_kernel<T, VEC, 16><<<grid, threads, 0, s>>>(input, branch, weight, residual_out, out, rows, H, eps);
    else
        residual_norm_kernel<T, VEC, 0><<<grid, threads, 0, s>>>(input, branch, weight, residual_out, out, rows, H, eps);
    return (int)hipGetLastError();
}

template <typename T>
int launch_norm_dtype(const void* input, const void* branch, const void* weight, void* residual_out, void* out,
                      int rows, int H, float eps, int preferred_bytes, hipStream_t s) {
    const uintptr_t align = (uintptr_t)input | (uintptr_t)branch | (uintptr_t)weight | (uintptr_t)residual_out |
                            (uintptr_t)out | (uintptr_t)((size_t)H * sizeof(T));
    const bool vec = preferred_bytes >= 16 && align % 16 == 0;
    const T* x = (const T*)input;
    const T* b = (const T*)branch;
    const T* w = (const T*)weight;
    T* r = (T*)residual_out;
    T* y = (T*)out;
    if (vec) return launch_norm_typed<T, true>(x, b, w, r, y, rows, H, eps, s);
    return launch_norm_typed<T, false>(x, b, w, r, y, rows, H, eps, s);
}

}  // namespace

int launch_residual_norm(const void* input, const void* branch, const void* weight, void* residual_out, void* out,
                         int rows, int columns, float eps, int dtype, int preferred_bytes, hipStream_t s) {
    if (!input || !weight || !out || rows <= 0 || columns <= 0 || !(eps > 0.0f) || !__builtin_isfinite(eps))
        return kInvalid;
    if ((branch == nullptr) != (residual_out == nullptr)) return kInvalid;
    if (preferred_bytes != 0 && preferred_bytes != 4 && preferred_bytes != 8 && preferred_bytes != 16)
        return kInvalid;
    if (dtype == 0)
        return launch_norm_dtype<float>(input, branch, weight, residual_out, out, rows, columns, eps, preferred_bytes, s);
    if (dtype == 1)
        return launch_norm_dtype<uint16_t>(input, branch, weight, residual_out, out, rows, columns, eps,
                                           preferred_bytes, s);
    return kInvalid;
}

}  // namespace tau_amd
