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

// Wave-wide reductions built from DPP lane moves (no LDS traffic): butterfly
// inside each 16-lane row, then row_bcast:15 / row_bcast:31 carry the row
// results upward so lane 63 holds the full reduction, read back uniformly.
template <int Ctrl, int RowMask>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t identity, uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)identity, (int)v, Ctrl, RowMask, 0xf, false);
}

template <int Ctrl, int RowMask>
__device__ __forceinline__ float dpp_f32(float identity, float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(identity), __float_as_int(v), Ctrl, RowMask,
                                                      0xf, false));
}

constexpr int kQuadXor1 = 0xb1, kQuadXor2 = 0x4e, kRowHalfMirror = 0x141, kRowMirror = 0x140;
constexpr int kRowBcast15 = 0x142, kRowBcast31 = 0x143;

__device__ __forceinline__ float wave_max_f32(float v) {
    const float id = -INFINITY;
    v = fmaxf(v, dpp_f32<kQuadXor1, 0xf>(id, v));
    v = fmaxf(v, dpp_f32<kQuadXor2, 0xf>(id, v));
    v = fmaxf(v, dpp_f32<kRowHalfMirror, 0xf>(id, v));
    v = fmaxf(v, dpp_f32<kRowMirror, 0xf>(id, v));
    v = fmaxf(v, dpp_f32<kRowBcast15, 0xa>(id, v));
    v = fmaxf(v, dpp_f32<kRowBcast31, 0xc>(id, v));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ float wave_sum_f32(float v) {
    v += dpp_f32<kQuadXor1, 0xf>(0.f, v);
    v += dpp_f32<kQuadXor2, 0xf>(0.f, v);
    v += dpp_f32<kRowHalfMirror, 0xf>(0.f, v);
    v += dpp_f32<kRowMirror, 0xf>(0.f, v);
    v += dpp_f32<kRowBcast15, 0xa>(0.f, v);
    v += dpp_f32<kRowBcast31, 0xc>(0.f, v);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

template <int Ctrl, int RowMask>
__device__ __forceinline__ uint64_t max_step_u64(uint64_t v) {
    const uint32_t lo = dpp_u32<Ctrl, RowMask>(0u, (uint32_t)v);
    const uint32_t hi = dpp_u32<Ctrl, RowMask>(0u, (uint32_t)(v >> 32));
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    return o > v ? o : v;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    v = max_step_u64<kQuadXor1, 0xf>(v);
    v = max_step_u64<kQuadXor2, 0xf>(v);
    v = max_step_u64<kRowHalfMirror, 0xf>(v);
    v = max_step_u64<kRowMirror, 0xf>(v);
    v = max_step_u64<kRowBcast15, 0xa>(v);
    v = max_step_u64<kRowBcast31, 0xc>(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, 63);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), 63);
    return ((uint64_t)hi << 32) | lo;
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
        const float prob = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), owner));
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
    // No short-circuit: the earlier-rank loads are independent and issue together.
    for (int q = 0; q < r; ++q) valid &= row[q] != id;
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
    int* scratch;  // multi-workgroup: [chunks][E] counts, then bases; [chunks] flags
    int tokens, E, K, M;
    int capacity;
    int expert_bits;
    int chunk;     // assignments per workgroup chunk (multiple of 1024)
};

struct DispatchLds {
    int* wcount;    // [16][E] per-wave counts, then per-wave bases
    int* total;     // [E] counts of this workgroup's span
    int* padded;    // [E + 1] padded exclusive scan
    int* flag;      // [1]
    int* scan_tmp;  // [kDispatchThreads]
};

__device__ __forceinline__ DispatchLds dispatch_lds(int* lds, int E) {
    DispatchLds l;
    l.wcount = lds;
    l.total = lds + kDispatchWaves * E;
    l.padded = l.total + E;
    l.flag = l.padded + E + 1;
    l.scan_tmp = l.flag + 1;
    return l;
}

// Per-wave counts of [span_begin, span_end), each wave a contiguous segment;
// then per-expert exclusive prefix over waves (wcount becomes per-wave bases)
// and total[e] = count of e in the span.  Sets flag on any invalid route.
__device__ void span_counts(const DispatchArgs& p, const DispatchLds& l, int span_begin, int span_end) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    for (int i = tid; i < kDispatchWaves * p.E; i += kDispatchThreads) l.wcount[i] = 0;
    if (tid == 0) l.flag[0] = 0;
    __syncthreads();
    const int n = span_end - span_begin;
    const int seg = ((n + kDispatchWaves - 1) / kDispatchWaves + 63) / 64 * 64;
    const int begin = span_begin + wave * seg, end = min(span_end, begin + seg);
    int* my = l.wcount + wave * p.E;
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
    if (__any(bad) && lane == 0) l.flag[0] = 1;
    __syncthreads();
    for (int e = tid; e < p.E; e += kDispatchThreads) {
        int run = 0;
        for (int w = 0; w < kDispatchWaves; ++w) {
            const int c = l.wcount[w * p.E + e];
            l.wcount[w * p.E + e] = run;
            run += c;
        }
        l.total[e] = run;
    }
    __syncthreads();
}

// Stable scatter of the span: slot position = base[e] + per-wave base + in-wave rank.
__device__ void span_scatter(const DispatchArgs& p, const DispatchLds& l, int span_begin, int span_end,
                             const int* base /* [E], LDS or global */) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int n = span_end - span_begin;
    const int seg = ((n + kDispatchWaves - 1) / kDispatchWaves + 63) / 64 * 64;
    const int begin = span_begin + wave * seg, end = min(span_end, begin + seg);
    int* my = l.wcount + wave * p.E;
    for (int a0 = begin; a0 < end; a0 += 64) {
        const int a = a0 + lane;
        int e = -1;
        if (a < end) e = assignment_expert(p.routes, a, p.K, p.E);
        const bool active = e >= 0;
        const uint64_t peers = match_expert(e, active, p.expert_bits);
        const int leader = peers ? __ffsll((unsigned long long)peers) - 1 : 0;
        int off = 0;
        if (active && lane == leader) off = my[e];
        off = __shfl(off, leader, 64);
        if (active) {
            const int rank = __popcll(peers & lanemask_lt());
            p.slots[base[e] + off + rank] = a;
            if (lane == leader) my[e] = off + __popcll(peers);
        }
    }
}

// Padded exclusive scan of total[] over experts into padded[0..E].
__device__ void padded_scan(const DispatchArgs& p, const DispatchLds& l) {
    const int tid = threadIdx.x;
    const int per = (p.E + kDispatchThreads - 1) / kDispatchThreads;
    const int e0 = tid * per;
    int local = 0;
    for (int e = e0; e < min(p.E, e0 + per); ++e) local += (l.total[e] + p.M - 1) / p.M * p.M;
    l.scan_tmp[tid] = local;
    __syncthreads();
    for (int d = 1; d < kDispatchThreads; d <<= 1) {
        const int v = tid >= d ? l.scan_tmp[tid - d] : 0;
        __syncthreads();
        l.scan_tmp[tid] += v;
        __syncthreads();
    }
    int run = l.scan_tmp[tid] - local;
    for (int e = e0; e < min(p.E, e0 + per); ++e) {
        l.padded[e] = run;
        run += (l.total[e] + p.M - 1) / p.M * p.M;
    }
    if (tid == kDispatchThreads - 1) l.padded[p.E] = l.scan_tmp[tid];
    __syncthreads();
}

// Metadata words, offsets, the tile worklist and padding sentinels.
__device__ void finalize_plan(const DispatchArgs& p, const DispatchLds& l, int status) {
    const int tid = threadIdx.x;
    const int A = p.tokens * p.K;
    const int padded_total = l.padded[p.E];
    for (int e = tid; e < p.E; e += kDispatchThreads) {
        p.meta[e] = l.total[e];
        p.meta[p.E + e] = l.total[e];
        p.offsets[e] = l.padded[e];
    }
    if (tid == 0) {
        p.offsets[p.E] = padded_total;
        p.meta[2 * p.E] = status;
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
                if (l.padded[mid] <= row0) lo = mid; else hi = mid - 1;
            }
            e = lo;
        }
        p.tiles[tile] = e;
        const int valid_end = e >= 0 ? l.padded[e] + l.total[e] : 0;
        for (int row = max(row0, valid_end); row < row0 + p.M; ++row) p.slots[row] = A;
    }
}

// One workgroup builds the whole plan.  With `Fused`, the same workgroup
// first routes every token (decode-sized batches).
template <bool Fused, int EP>
__global__ __launch_bounds__(kDispatchThreads) void dispatch_single_kernel(DispatchArgs p) {
    extern __shared__ int lds[];
    const DispatchLds l = dispatch_lds(lds, p.E);
    const int wave = threadIdx.x >> 6;
    if constexpr (Fused) {
        for (int t = wave; t < p.tokens; t += kDispatchWaves) {
            if (p.logits_bf16)
                route_token<EP, uint16_t>(p.logits_bf16 + (size_t)t * p.E, p.routes + (size_t)t * 2 * p.K, p.E, p.K);
            else
                route_token<EP, float>(p.logits_f32 + (size_t)t * p.E, p.routes + (size_t)t * 2 * p.K, p.E, p.K);
        }
        __threadfence_block();
        __syncthreads();
    }
    const int A = p.tokens * p.K;
    span_counts(p, l, 0, A);
    const int status = l.flag[0];
    padded_scan(p, l);
    span_scatter(p, l, 0, A, l.padded);
    finalize_plan(p, l, status);
}

// Multi-workgroup plan, step 1: per-chunk expert counts and status.
__global__ __launch_bounds__(kDispatchThreads) void dispatch_hist_kernel(DispatchArgs p) {
    extern __shared__ int lds[];
    const DispatchLds l = dispatch_lds(lds, p.E);
    const int A = p.tokens * p.K, c = blockIdx.x;
    const int b = c * p.chunk, e_ = min(A, b + p.chunk);
    span_counts(p, l, b, e_);
    for (int e = threadIdx.x; e < p.E; e += kDispatchThreads) p.scratch[(size_t)c * p.E + e] = l.total[e];
    if (threadIdx.x == 0) p.scratch[(size_t)gridDim.x * p.E + c] = l.flag[0];
}

// Step 2 (one workgroup): chunk bases per expert, padded offsets, metadata.
__global__ __launch_bounds__(kDispatchThreads) void dispatch_plan_kernel(DispatchArgs p, int chunks) {
    extern __shared__ int lds[];
    const DispatchLds l = dispatch_lds(lds, p.E);
    int* cnt = l.scan_tmp + kDispatchThreads;  // [chunks][E]
    const int n = chunks * p.E;
    for (int i = threadIdx.x; i < n; i += kDispatchThreads) cnt[i] = p.scratch[i];
    __shared__ int status_word;
    if (threadIdx.x == 0) status_word = 0;
    __syncthreads();
    for (int c = threadIdx.x; c < chunks; c += kDispatchThreads)
        if (p.scratch[(size_t)chunks * p.E + c]) atomicOr(&status_word, 1);
    for (int e = threadIdx.x; e < p.E; e += kDispatchThreads) {
        int run = 0;
        for (int c = 0; c < chunks; ++c) {
            const int v = cnt[c * p.E + e];
            cnt[c * p.E + e] = run;
            run += v;
        }
        l.total[e] = run;
    }
    __syncthreads();
    padded_scan(p, l);
    for (int i = threadIdx.x; i < n; i += kDispatchThreads) p.scratch[i] = cnt[i] + l.padded[i % p.E];
    finalize_plan(p, l, status_word);
}

// Step 3: stable scatter of each chunk from its absolute bases.
__global__ __launch_bounds__(kDispatchThreads) void dispatch_scatter_kernel(DispatchArgs p) {
    extern __shared__ int lds[];
    const DispatchLds l = dispatch_lds(lds, p.E);
    const int A = p.tokens * p.K, c = blockIdx.x;
    const int b = c * p.chunk, e_ = min(A, b + p.chunk);
    span_counts(p, l, b, e_);
    span_scatter(p, l, b, e_, p.scratch + (size_t)c * p.E);
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
int launch_dispatch_single(DispatchArgs a, hipStream_t s) {
    const size_t lds = dispatch_lds_bytes(a.E);
    const int ep = (a.E + 63) / 64;
    if (ep <= 1) dispatch_single_kernel<Fused, 1><<<1, kDispatchThreads, lds, s>>>(a);
    else if (ep <= 2) dispatch_single_kernel<Fused, 2><<<1, kDispatchThreads, lds, s>>>(a);
    else if (ep <= 4) dispatch_single_kernel<Fused, 4><<<1, kDispatchThreads, lds, s>>>(a);
    else if (ep <= 8) dispatch_single_kernel<Fused, 8><<<1, kDispatchThreads, lds, s>>>(a);
    else dispatch_single_kernel<Fused, 16><<<1, kDispatchThreads, lds, s>>>(a);
    return (int)hipGetLastError();
}

}  // namespace

// Largest expert count the routing/dispatch kernels accept (8 logits per lane;
// the dispatch LDS footprint is (18 E + 1026) words, 41 KB at E = 512).
constexpr int kMaxExperts = 512;
constexpr int kMaxTopK = 32;
constexpr int kFusedRouteMaxTokens = 256;
constexpr int kDispatchChunk = 4096;  // assignments per workgroup in the multi-workgroup plan
constexpr int kPlanLdsWords = 4096;   // [chunks][E] counts staged by the plan workgroup

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
                    int* tiles, int tokens, int E, int K, int M, int capacity, void* scratch, size_t scratch_bytes,
                    hipStream_t s) {
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
    const int A = tokens * K;
    // Chunk so that the plan workgroup can stage all [chunks][E] counts in LDS.
    const int max_chunks = kPlanLdsWords / E;
    int chunk = kDispatchChunk;
    if ((A + chunk - 1) / chunk > max_chunks) chunk = ((A + max_chunks - 1) / max_chunks + 1023) / 1024 * 1024;
    const int chunks = (A + chunk - 1) / chunk;
    const bool multi = A > kDispatchChunk && scratch && E <= kPlanLdsWords &&
                       scratch_bytes >= sizeof(int) * ((size_t)chunks * E + chunks);
    if (logits) {
        if (logits_dtype != 0 && logits_dtype != 1) return kInvalid;
        if (tokens <= kFusedRouteMaxTokens && !multi) {
            if (logits_dtype == 1) a.logits_bf16 = (const uint16_t*)logits;
            else a.logits_f32 = (const float*)logits;
            return launch_dispatch_single<true>(a, s);
        }
        int code = launch_routing(logits, logits_dtype, routes, tokens, E, K, s);
        if (code) return code;
    }
    if (!multi) return launch_dispatch_single<false>(a, s);
    a.scratch = (int*)scratch;
    a.chunk = chunk;
    const size_t lds = dispatch_lds_bytes(E);
    dispatch_hist_kernel<<<chunks, kDispatchThreads, lds, s>>>(a);
    dispatch_plan_kernel<<<1, kDispatchThreads, lds + sizeof(int) * (size_t)chunks * E, s>>>(a, chunks);
    dispatch_scatter_kernel<<<chunks, kDispatchThreads, lds, s>>>(a);
    return (int)hipGetLastError();
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
