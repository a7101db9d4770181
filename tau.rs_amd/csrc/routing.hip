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
// CDNA4 design.
//  * Routing: one 16-lane DPP row per token, four tokens per wavefront.  Each
//    lane owns E/16 logits; the max and the K arg-max steps are row-local DPP
//    butterflies (quad_perm, row_half_mirror, row_mirror), so a top-K costs no
//    LDS or cross-lane memory traffic and the four tokens of a wave proceed
//    together.  The softmax is the reference's f32 one bit for bit: exp with
//    glibc expf's results (libm_expf.hpp), the denominator summed in expert
//    order (one DPP-broadcast add per expert), one division per expert.
//    Ordering keys are (probability, ~id) in 64 bits, so distinct logits whose
//    probabilities round equal tie to the lower id, as in the reference.
//  * Dispatch: a counting sort.  Every assignment's expert is staged in LDS,
//    16 waves each count a contiguous segment (ballot-derived peer masks, no
//    global atomics), counts are prefixed per expert over waves and over
//    workgroup chunks, and each assignment lands at
//    offset[e] + earlier-chunk count + earlier-wave count + in-wave rank, which
//    is the token-ascending order of the reference's CPU plan.  Small batches
//    run route + plan + scatter in one workgroup; large ones route over the
//    whole GPU, then histogram chunks, then scatter chunks (each chunk
//    workgroup recomputing the small plan from the chunk counts).
#include "dispatch.hpp"

namespace tau_amd {
namespace {

template <typename T>
int launch_route(const T* logits, float* routes, int tokens, int E, int K, int normalize, hipStream_t s) {
    const int blocks = (tokens + 3) / 4;
    const int ep = (E + 15) / 16;
    if (ep <= 1) route_kernel<1, T><<<blocks, 64, 0, s>>>(logits, routes, tokens, E, K, normalize);
    else if (ep <= 2) route_kernel<2, T><<<blocks, 64, 0, s>>>(logits, routes, tokens, E, K, normalize);
    else if (ep <= 4) route_kernel<4, T><<<blocks, 64, 0, s>>>(logits, routes, tokens, E, K, normalize);
    else if (ep <= 8) route_kernel<8, T><<<blocks, 64, 0, s>>>(logits, routes, tokens, E, K, normalize);
    else if (ep <= 16) route_kernel<16, T><<<blocks, 64, 0, s>>>(logits, routes, tokens, E, K, normalize);
    else route_kernel<32, T><<<blocks, 64, 0, s>>>(logits, routes, tokens, E, K, normalize);
    return (int)hipGetLastError();
}

template <template <int> class Launch>
int by_ep(int E, const DispatchArgs& a, unsigned grid, size_t lds, hipStream_t s) {
    const int ep = (E + 15) / 16;
    if (ep <= 1) return Launch<1>::go(a, grid, lds, s);
    if (ep <= 2) return Launch<2>::go(a, grid, lds, s);
    if (ep <= 4) return Launch<4>::go(a, grid, lds, s);
    if (ep <= 8) return Launch<8>::go(a, grid, lds, s);
    if (ep <= 16) return Launch<16>::go(a, grid, lds, s);
    return Launch<32>::go(a, grid, lds, s);
}

template <int EP>
struct SingleLaunch {
    static int go(const DispatchArgs& a, unsigned grid, size_t lds, hipStream_t s) {
        dispatch_single_kernel<EP><<<grid, kThreads, lds, s>>>(a);
        return (int)hipGetLastError();
    }
};

template <int EP>
struct HistLaunch {
    static int go(const DispatchArgs& a, unsigned grid, size_t lds, hipStream_t s) {
        dispatch_hist_kernel<EP><<<grid, kThreads, lds, s>>>(a);
        return (int)hipGetLastError();
    }
};

}  // namespace

// Largest expert count the routing/dispatch kernels accept (32 logits per
// lane of a 16-lane row; dispatch LDS (19 E + 5122) words, 59 KB at E = 512).
constexpr int kMaxExperts = 512;  // routed experts (16 lanes x 32 logits per token row)
constexpr int kMaxTopK = 32;

int64_t capacity_for(int64_t tokens, int64_t E, int64_t K, int64_t M) {
    if (tokens <= 0 || E <= 0 || K <= 0 || M <= 0) return -1;
    const int64_t a = tokens * K;
    const int64_t bound = a + (a < E ? a : E) * (M - 1) + (M - 1);
    return bound / M * M;
}

// logits_dtype: 0 = f32, 1 = BF16, optionally OR TAU_MOE_ROUTE_RAW_WEIGHTS.
bool logits_dtype_ok(int logits_dtype) {
    const int dtype = logits_dtype & ~TAU_MOE_ROUTE_RAW_WEIGHTS;
    return dtype == 0 || dtype == 1;
}

int launch_routing(const void* logits, int logits_dtype, float* routes, int tokens, int E, int K,
                   hipStream_t s) {
    if (!logits || !routes || tokens <= 0 || E <= 0 || E > kMaxExperts || K <= 0 || K > E || K > kMaxTopK ||
        !logits_dtype_ok(logits_dtype))
        return kInvalid;
    const int normalize = !(logits_dtype & TAU_MOE_ROUTE_RAW_WEIGHTS);
    if (logits_dtype & 1) return launch_route<uint16_t>((const uint16_t*)logits, routes, tokens, E, K, normalize, s);
    return launch_route<float>((const float*)logits, routes, tokens, E, K, normalize, s);
}

namespace {

template <typename T>
int launch_route_shared(const T* logits, float* routes, int tokens, int E, int K, int normalize, hipStream_t s) {
    const int blocks = (tokens + 3) / 4;
    const int ep = (E + 15) / 16;
    if (ep <= 1) route_shared_kernel<1, T><<<blocks, 64, 0, s>>>(logits, routes, tokens, E, K, normalize);
    else if (ep <= 2) route_shared_kernel<2, T><<<blocks, 64, 0, s>>>(logits, routes, tokens, E, K, normalize);
    else if (ep <= 4) route_shared_kernel<4, T><<<blocks, 64, 0, s>>>(logits, routes, tokens, E, K, normalize);
    else if (ep <= 8) route_shared_kernel<8, T><<<blocks, 64, 0, s>>>(logits, routes, tokens, E, K, normalize);
    else if (ep <= 16) route_shared_kernel<16, T><<<blocks, 64, 0, s>>>(logits, routes, tokens, E, K, normalize);
    else route_shared_kernel<32, T><<<blocks, 64, 0, s>>>(logits, routes, tokens, E, K, normalize);
    return (int)hipGetLastError();
}

}  // namespace

// Routing with the shared expert folded in (route_shared_kernel): logits
// [T, E+1], routes [T, 2(K+1)].
int launch_routing_shared(const void* logits, int logits_dtype, float* routes, int tokens, int E, int K,
                          hipStream_t s) {
    if (!logits || !routes || tokens <= 0 || E <= 0 || E > kMaxExperts || K <= 0 || K > E || K + 1 > kMaxTopK ||
        !logits_dtype_ok(logits_dtype))
        return kInvalid;
    const int normalize = !(logits_dtype & TAU_MOE_ROUTE_RAW_WEIGHTS);
    if (logits_dtype & 1)
        return launch_route_shared<uint16_t>((const uint16_t*)logits, routes, tokens, E, K, normalize, s);
    return launch_route_shared<float>((const float*)logits, routes, tokens, E, K, normalize, s);
}

// Dispatch; with logits, routing runs inside the plan kernels.  `scratch`
// (optional) enables the multi-workgroup plan for large batches.
int launch_dispatch(const void* logits, int logits_dtype, float* routes, int* meta, int* offsets, int* slots,
                    int* tiles, int tokens, int E, int K, int M, int capacity, void* scratch, size_t scratch_bytes,
                    hipStream_t s) {
    // From given routes one more expert is allowed: a shared expert folded in as expert E.
    if (!routes || !meta || !offsets || !slots || !tiles || tokens <= 0 || E <= 0 ||
        E > kMaxExperts + (logits ? 0 : 1) || K <= 0 || K > E || K > kMaxTopK || M <= 0 || capacity <= 0 ||
        capacity % M)
        return kInvalid;
    if ((int64_t)tokens * K > (int64_t)1 << 30) return kInvalid;
    if ((int64_t)capacity < capacity_for(tokens, E, K, M)) return kInvalid;
    if (logits && !logits_dtype_ok(logits_dtype)) return kInvalid;
    DispatchArgs a{};
    a.logits = logits;
    a.logits_bf16 = logits_dtype & 1;
    a.normalize = !(logits_dtype & TAU_MOE_ROUTE_RAW_WEIGHTS);
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
    const size_t lds = sizeof(int) * dispatch_lds_words(E);
    // Multi-workgroup chunks: at most 32 (each scatter workgroup sums the
    // [chunks][E] counts from scratch; 64 measured slower on the 4096-token
    // layer), each a whole number of 64-token routing passes that fits the
    // LDS expert stage.
    {
        const int max_chunks = 32;
        const int stage_tokens = std::max(1, kSpanLds / K);
        int ct = (tokens + max_chunks - 1) / max_chunks;
        ct = (ct + 63) / 64 * 64;
        if (ct > stage_tokens) ct = stage_tokens >= 64 ? stage_tokens / 64 * 64 : stage_tokens;
        a.chunk_tokens = ct;
    }
    const int chunks = (tokens + a.chunk_tokens - 1) / a.chunk_tokens;
    const bool multi = chunks > 1 && scratch && scratch_bytes >= sizeof(int) * ((size_t)chunks * E + chunks);
    if (!multi) {
        // Route separately (every CU) unless the batch is a few tokens, whose
        // routing the plan workgroup does faster than an extra launch.
        if (logits && ((int64_t)tokens * K > kSpanLds || tokens >= kSplitRouteTokens)) {
            const int code = launch_routing(logits, logits_dtype, routes, tokens, E, K, s);
            if (code) return code;
            a.logits = nullptr;
        }
        return by_ep<SingleLaunch>(E, a, 1, lds, s);
    }
    a.scratch = (int*)scratch;
    if (logits) {  // route over the whole GPU, then histogram chunks from the routes
        const int code = launch_routing(logits, logits_dtype, routes, tokens, E, K, s);
        if (code) return code;
        a.logits = nullptr;
    }
    int code = by_ep<HistLaunch>(E, a, chunks, lds, s);
    if (code) return code;
    dispatch_scatter_kernel<<<chunks, kThreads, lds, s>>>(a);
    return (int)hipGetLastError();
}

}  // namespace tau_amd
