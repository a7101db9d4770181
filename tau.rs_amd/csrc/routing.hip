// Router softmax / top-k and stable expert-major dispatch for the MoE path.
//
// Semantics follow the reference's f32 CPU plan (tau.rs
// crates/models/src/components/sparse_moe/routing.rs:125-257): softmax over the
// E router logits in FP32, top-K by (probability descending, expert id
// ascending), weights renormalised by their rank-ordered sum, and every
// expert's assignment list in ascending token order.  The packed `routes`
// row [K ids as float, K weights] and the `meta` words follow the reference's
// native layout (crates/cuda-kernels/src/kernels/moe_routing.cu:15-52,
// moe_dispatch.cuh:9, moe_dispatch.cu:11-85), generalised from E=256/K=8.
//
// CDNA4 design: one 64-lane wavefront per token; each lane owns E/64 logits,
// ordering decisions use 64-bit (score, ~id) keys reduced with DPP/ds_swizzle
// shuffles, so a top-K costs K wave reductions and no shared memory.  Dispatch
// is one 1024-thread workgroup: 16 waves each own a contiguous assignment
// segment, count it, prefix the per-wave counts per expert, and scatter with
// ballot-derived in-wave ranks, so the permutation is deterministic and
// token-ascending without atomics on global memory.
#include "kernels.hpp"

namespace tau_amd {
namespace {

// Order-preserving map of an FP32 value onto uint32 (larger float -> larger key).
__device__ __forceinline__ uint32_t orderable(float v) {
    uint32_t u = __float_as_uint(v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        uint64_t o = __shfl_xor(v, d, 64);
        v = o > v ? o : v;
    }
    return v;
}

__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v = fmaxf(v, __shfl_xor(v, d, 64));
    return v;
}

__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
    return v;
}

template <typename T>
__device__ __forceinline__ float load_logit(const T* p, size_t i);
template <>
__device__ __forceinline__ float load_logit<float>(const float* p, size_t i) { return p[i]; }
template <>
__device__ __forceinline__ float load_logit<uint16_t>(const uint16_t* p, size_t i) {
    return bf16_bits_to_float(p[i]);
}

// Routes one token with the calling wave.  `row` points at the token's logits,
// `out` at its packed [2K] routes row.
template <int EP, typename T>
__device__ __forceinline__ void route_token(const T* row, float* out, int E, int K) {
    const int lane = threadIdx.x & 63;
    float d[EP], p[EP];
    bool finite = true;
    float maximum = -INFINITY;
#pragma unroll
    for (int j = 0; j < EP; ++j) {
        int e = j * 64 + lane;
        d[j] = e < E ? load_logit<T>(row, e) : -INFINITY;
        if (e < E) finite &= __builtin_isfinite(d[j]);
        maximum = fmaxf(maximum, d[j]);
    }
    if (!__all(finite)) {
        for (int i = lane; i < 2 * K; i += 64) out[i] = __builtin_nanf("");
        return;
    }
    maximum = wave_max_f32(maximum);
    float local = 0.f;
#pragma unroll
    for (int j = 0; j < EP; ++j) {
        int e = j * 64 + lane;
        // x - max, with -0 folded onto +0 so equal probabilities give equal keys.
        d[j] = (d[j] - maximum) + 0.0f;
        p[j] = e < E ? expf(d[j]) : 0.f;
        local += p[j];
    }
    const float denominator = wave_sum_f32(local);
#pragma unroll
    for (int j = 0; j < EP; ++j) p[j] = p[j] / denominator;

    // exp is monotone, so (x - max) orders experts exactly as their
    // probabilities do, ties included, without depending on exp rounding.
    uint32_t taken = 0;
    float selected_sum = 0.f;
    float my_weight = 0.f;
    int my_id = 0;
    for (int r = 0; r < K; ++r) {
        uint64_t best = 0;
#pragma unroll
        for (int j = 0; j < EP; ++j) {
            int e = j * 64 + lane;
            if (e < E && !(taken & (1u << j))) {
                uint64_t key = ((uint64_t)orderable(d[j]) << 32) | (uint32_t)(0xffffffffu - (uint32_t)e);
                best = key > best ? key : best;
            }
        }
        best = wave_max_u64(best);
        const int id = (int)(0xffffffffu - (uint32_t)(best & 0xffffffffu));
        const int owner = id & 63, slot = id >> 6;
        float mine = 0.f;
#pragma unroll
        for (int j = 0; j < EP; ++j)
            if (j == slot) mine = p[j];
        const float prob = __shfl(mine, owner, 64);
        if (lane == owner) taken |= 1u << slot;
        selected_sum += prob;  // rank order, as routing.rs:187-191
        if (lane == r) { my_id = id; my_weight = prob; }
    }
    if (lane < K) {
        out[lane] = (float)my_id;
        out[K + lane] = my_weight / selected_sum;
    }
}

template <int EP, typename T>
__global__ __launch_bounds__(256) void route_kernel(const T* logits, float* routes, int T_, int E, int K) {
    const int token = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (token >= T_) return;
    route_token<EP, T>(logits + (size_t)token * E, routes + (size_t)token * 2 * K, E, K);
}

// --------------------------------------------------------------------------
// Dispatch
// --------------------------------------------------------------------------

constexpr int kDispatchThreads = 1024;
constexpr int kDispatchWaves = kDispatchThreads / 64;

// Reads and validates one assignment (moe_dispatch.cu:23-33 of the reference):
// a finite integral id in [0,E), no duplicate among the token's earlier ranks,
// and a finite non-negative weight.  Returns the expert or -1.
__device__ __forceinline__ int assignment_expert(const float* routes, int a, int K, int E) {
    const int t = a / K, r = a - t * K;
    const float* row = routes + (size_t)t * 2 * K;
    const float id = row[r], w = row[K + r];
    bool valid = __builtin_isfinite(id) && id >= 0.f && id < (float)E && floorf(id) == id &&
                 __builtin_isfinite(w) && w >= 0.f;
    for (int q = 0; q < r && valid; ++q) valid = row[q] != id;
    return valid ? (int)id : -1;
}

// In-wave stable rank of this lane among active lanes holding the same expert.
// Returns the peer mask (lanes with the same expert).
__device__ __forceinline__ uint64_t match_expert(int e, bool active, int bits) {
    uint64_t peers = __ballot(active);
    for (int b = 0; b < bits; ++b) {
        const bool bit = (e >> b) & 1;
        const uint64_t m = __ballot(bit);
        peers &= bit ? m : ~m;
    }
    return peers;
}

struct DispatchArgs {
    const uint16_t* logits_bf16;  // fused routing (small T) or null
    const float* logits_f32;
    float* routes;
    int* meta;
    int* offsets;
    int* slots;
    int* tiles;
    int tokens, E, K, M;
    int capacity;
    int expert_bits;
};

// One workgroup builds counts, padded offsets, the stable permutation, the
// tile worklist and the status/padded-total words.  With `Fused`, the same
// workgroup first routes every token (used for decode-sized batches).
template <bool Fused, int EP>
__global__ __launch_bounds__(kDispatchThreads) void dispatch_kernel(DispatchArgs p) {
    extern __shared__ int lds[];
    int* wcount = lds;                                  // [16][E]
    int* total = lds + kDispatchWaves * p.E;             // [E]
    int* padded = total + p.E;                          // [E + 1] exclusive scan
    int* flag = padded + p.E + 1;                       // [1]
    int* scan_tmp = flag + 1;                           // [kDispatchThreads]
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int A = p.tokens * p.K;

    if constexpr (Fused) {
        for (int t = wave; t < p.tokens; t += kDispatchWaves) {
            if (p.logits_bf16)
                route_token<EP, uint16_t>(p.logits_bf16 + (size_t)t * p.E, p.routes + (size_t)t * 2 * p.K, p.E, p.K);
            else
                route_token<EP, float>(p.logits_f32 + (size_t)t * p.E, p.routes + (size_t)t * 2 * p.K, p.E, p.K);
        }
        __threadfence_block();
    }
    for (int i = tid; i < kDispatchWaves * p.E; i += kDispatchThreads) wcount[i] = 0;
    if (tid == 0) flag[0] = 0;
    __syncthreads();

    // Phase 1: per-wave counts over contiguous segments.
    const int seg = ((A + kDispatchWaves - 1) / kDispatchWaves + 63) / 64 * 64;
    const int begin = wave * seg, end = min(A, begin + seg);
    int* my = wcount + wave * p.E;
    bool bad = false;
    for (int a0 = begin; a0 < end; a0 += 64) {
        const int a = a0 + lane;
        int e = -1;
        if (a < end) {
            e = assignment_expert(p.routes, a, p.K, p.E);
            bad |= e < 0;
        }
        const bool active = e >= 0;
        const uint64_t peers = match_expert(e, active, p.expert_bits);
        if (active && (peers & lanemask_lt()) == 0) my[e] += __popcll(peers);
    }
    if (__any(bad) && lane == 0) flag[0] = 1;
    __syncthreads();

    // Phase 2: per-expert prefix over waves, then padded exclusive scan over experts.
    for (int e = tid; e < p.E; e += kDispatchThreads) {
        int run = 0;
        for (int w = 0; w < kDispatchWaves; ++w) {
            const int c = wcount[w * p.E + e];
            wcount[w * p.E + e] = run;
            run += c;
        }
        total[e] = run;
    }
    __syncthreads();
    {
        // Each thread owns a contiguous run of experts, then a block scan.
        const int per = (p.E + kDispatchThreads - 1) / kDispatchThreads;
        const int e0 = tid * per;
        int local = 0;
        for (int e = e0; e < min(p.E, e0 + per); ++e) local += (total[e] + p.M - 1) / p.M * p.M;
        scan_tmp[tid] = local;
        __syncthreads();
        for (int d = 1; d < kDispatchThreads; d <<= 1) {
            const int v = tid >= d ? scan_tmp[tid - d] : 0;
            __syncthreads();
            scan_tmp[tid] += v;
            __syncthreads();
        }
        int run = scan_tmp[tid] - local;
        for (int e = e0; e < min(p.E, e0 + per); ++e) {
            padded[e] = run;
            run += (total[e] + p.M - 1) / p.M * p.M;
        }
        if (tid == kDispatchThreads - 1) padded[p.E] = scan_tmp[tid];
    }
    __syncthreads();

    // Phase 3: stable scatter.  Wave w's cursor for expert e starts at
    // offsets[e] + (assignments of e in earlier segments).
    for (int a0 = begin; a0 < end; a0 += 64) {
        const int a = a0 + lane;
        int e = -1;
        if (a < end) e = assignment_expert(p.routes, a, p.K, p.E);
        const bool active = e >= 0;
        const uint64_t peers = match_expert(e, active, p.expert_bits);
        const int leader = peers ? __ffsll((unsigned long long)peers) - 1 : 0;
        int base = 0;
        if (active && lane == leader) base = my[e];
        base = __shfl(base, leader, 64);
        if (active) {
            const int rank = __popcll(peers & lanemask_lt());
            p.slots[padded[e] + base + rank] = a;
            if (lane == leader) my[e] = base + __popcll(peers);
        }
    }

    // Phase 4: metadata, tile worklist and padding sentinels.
    const int padded_total = padded[p.E];
    for (int e = tid; e < p.E; e += kDispatchThreads) {
        p.meta[e] = total[e];
        p.meta[p.E + e] = total[e];
        p.offsets[e] = padded[e];
    }
    if (tid == 0) {
        p.offsets[p.E] = padded_total;
        p.meta[2 * p.E] = flag[0];
        p.meta[2 * p.E + 1] = padded_total;
    }
    const int ntiles = p.capacity / p.M;
    for (int tile = tid; tile < ntiles; tile += kDispatchThreads) {
        const int row0 = tile * p.M;
        int e = -1;
        if (row0 < padded_total) {
            int lo = 0, hi = p.E - 1;  // last expert with padded[e] <= row0
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (padded[mid] <= row0) lo = mid; else hi = mid - 1;
            }
            e = lo;
        }
        p.tiles[tile] = e;
        const int valid_end = e >= 0 ? padded[e] + total[e] : 0;
        for (int row = max(row0, valid_end); row < row0 + p.M; ++row) p.slots[row] = A;
    }
}

// Ordered combine: out[t,h] = bf16(sum_r f32(contrib[t*K + r, h])), ranks in order
// (moe_dispatch.cuh:13-20); NaN everywhere when the plan was invalid.
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t* contributions, uint16_t* output,
                                                      const int* status, int T_, int H, int K) {
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
    u32x4 o;
#pragma unroll
    for (int q = 0; q < 4; ++q)
        o[q] = invalid ? 0x7fc07fc0u : pack_bf16x2(acc[2 * q], acc[2 * q + 1]);
    *(u32x4*)(output + (size_t)t * H + c * 8) = o;
}

// Scalar combine for hidden sizes that are not multiples of eight.
__global__ __launch_bounds__(256) void combine_scalar_kernel(const uint16_t* contributions, uint16_t* output,
                                                             const int* status, int T_, int H, int K) {
    const long idx = (long)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (long)T_ * H) return;
    const int t = (int)(idx / H), h = (int)(idx - (long)t * H);
    float acc = 0.f;
    for (int r = 0; r < K; ++r) acc += bf16_bits_to_float(contributions[((size_t)t * K + r) * H + h]);
    output[idx] = status[0] ? (uint16_t)0x7fc0 : float_to_bf16_bits(acc);
}

template <typename T>
int launch_route(const T* logits, float* routes, int tokens, int E, int K, hipStream_t s) {
    const int blocks = (tokens + 3) / 4;
    const int ep = (E + 63) / 64;
    if (ep <= 1) route_kernel<1, T><<<blocks, 256, 0, s>>>(logits, routes, tokens, E, K);
    else if (ep <= 2) route_kernel<2, T><<<blocks, 256, 0, s>>>(logits, routes, tokens, E, K);
    else if (ep <= 4) route_kernel<4, T><<<blocks, 256, 0, s>>>(logits, routes, tokens, E, K);
    else if (ep <= 8) route_kernel<8, T><<<blocks, 256, 0, s>>>(logits, routes, tokens, E, K);
    else route_kernel<16, T><<<blocks, 256, 0, s>>>(logits, routes, tokens, E, K);
    return (int)hipGetLastError();
}

size_t dispatch_lds_bytes(int E) {
    return sizeof(int) * ((size_t)kDispatchWaves * E + E + E + 1 + 1 + kDispatchThreads);
}

template <bool Fused>
int launch_dispatch_ep(DispatchArgs a, hipStream_t s) {
    const size_t lds = dispatch_lds_bytes(a.E);
    const int ep = (a.E + 63) / 64;
    if (ep <= 1) dispatch_kernel<Fused, 1><<<1, kDispatchThreads, lds, s>>>(a);
    else if (ep <= 2) dispatch_kernel<Fused, 2><<<1, kDispatchThreads, lds, s>>>(a);
    else if (ep <= 4) dispatch_kernel<Fused, 4><<<1, kDispatchThreads, lds, s>>>(a);
    else if (ep <= 8) dispatch_kernel<Fused, 8><<<1, kDispatchThreads, lds, s>>>(a);
    else dispatch_kernel<Fused, 16><<<1, kDispatchThreads, lds, s>>>(a);
    return (int)hipGetLastError();
}

}  // namespace

// Largest expert count the routing/dispatch kernels accept (16 logits per lane;
// the dispatch LDS footprint is (18 E + 1026) words, 75 KB at E = 1024).
constexpr int kMaxExperts = 1024;
constexpr int kMaxTopK = 32;
constexpr int kFusedRouteMaxTokens = 256;

int64_t capacity_for(int64_t tokens, int64_t E, int64_t K, int64_t M) {
    if (tokens <= 0 || E <= 0 || K <= 0 || M <= 0) return -1;
    const int64_t a = tokens * K;
    const int64_t bound = a + (a < E ? a : E) * (M - 1) + (M - 1);
    return bound / M * M;
}

int launch_routing(const void* logits, int logits_dtype, float* routes, int tokens, int E, int K,
                   hipStream_t s) {
    if (!logits || !routes || tokens <= 0 || E <= 0 || E > kMaxExperts || K <= 0 || K > E || K > kMaxTopK ||
        (logits_dtype != 0 && logits_dtype != 1))
        return kInvalid;
    if (logits_dtype == 1) return launch_route<uint16_t>((const uint16_t*)logits, routes, tokens, E, K, s);
    return launch_route<float>((const float*)logits, routes, tokens, E, K, s);
}

// Dispatch (and, with logits, routing first when the batch is small enough
// to route inside the dispatch workgroup).
int launch_dispatch(const void* logits, int logits_dtype, float* routes, int* meta, int* offsets, int* slots,
                    int* tiles, int tokens, int E, int K, int M, int capacity, hipStream_t s) {
    if (!routes || !meta || !offsets || !slots || !tiles || tokens <= 0 || E <= 0 || E > kMaxExperts || K <= 0 ||
        K > E || K > kMaxTopK || M <= 0 || capacity <= 0 || capacity % M)
        return kInvalid;
    if ((int64_t)tokens * K > (int64_t)1 << 30) return kInvalid;
    if ((int64_t)capacity < capacity_for(tokens, E, K, M)) return kInvalid;
    DispatchArgs a{};
    a.routes = routes;
    a.meta = meta;
    a.offsets = offsets;
    a.slots = slots;
    a.tiles = tiles;
    a.tokens = tokens;
    a.E = E;
    a.K = K;
    a.M = M;
    a.capacity = capacity;
    int bits = 0;
    while ((1 << bits) < E) ++bits;
    a.expert_bits = bits;
    if (logits) {
        if (logits_dtype != 0 && logits_dtype != 1) return kInvalid;
        if (tokens <= kFusedRouteMaxTokens) {
            if (logits_dtype == 1) a.logits_bf16 = (const uint16_t*)logits;
            else a.logits_f32 = (const float*)logits;
            return launch_dispatch_ep<true>(a, s);
        }
        int code = launch_routing(logits, logits_dtype, routes, tokens, E, K, s);
        if (code) return code;
    }
    return launch_dispatch_ep<false>(a, s);
}

int launch_combine(const void* contributions, void* output, const int* status, int tokens, int H, int K,
                   hipStream_t s) {
    if (!contributions || !output || !status || tokens <= 0 || H <= 0 || K <= 0) return kInvalid;
    if (H % 8 == 0) {
        const long n = (long)tokens * (H / 8);
        combine_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>((const uint16_t*)contributions,
                                                                  (uint16_t*)output, status, tokens, H, K);
    } else {
        const long n = (long)tokens * H;
        combine_scalar_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>((const uint16_t*)contributions,
                                                                         (uint16_t*)output, status, tokens, H, K);
    }
    return (int)hipGetLastError();
}

}  // namespace tau_amd
