// Device code of routing and dispatch, shared by the routing/dispatch
// launchers (routing.hip) and the fused decode path (decode_moe.hip), which
// runs the dispatch plan inside its own launch.  Design notes are at the top
// of routing.hip.
#pragma once
#include <algorithm>

#include "kernels.hpp"
#include "libm_expf.hpp"

namespace tau_amd {
namespace {

// ---------------------------------------------------------------------------
// Row (16-lane) DPP reductions; every lane of the row receives the result.
// ---------------------------------------------------------------------------
constexpr int kQuadXor1 = 0xb1, kQuadXor2 = 0x4e, kRowHalfMirror = 0x141, kRowMirror = 0x140;
constexpr int kRowShr1 = 0x111;  // lane i reads lane i-1 of its row (lane 0 of the row reads 0)

template <int Ctrl>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, Ctrl, 0xf, 0xf, false);
}
template <int Ctrl>
__device__ __forceinline__ float dppf(float v) {
    return __uint_as_float(dpp<Ctrl>(__float_as_uint(v)));
}

__device__ __forceinline__ float row_max(float v) {
    v = fmaxf(v, dppf<kQuadXor1>(v));
    v = fmaxf(v, dppf<kQuadXor2>(v));
    v = fmaxf(v, dppf<kRowHalfMirror>(v));
    v = fmaxf(v, dppf<kRowMirror>(v));
    return v;
}

__device__ __forceinline__ float row_sum(float v) {
    v += dppf<kQuadXor1>(v);
    v += dppf<kQuadXor2>(v);
    v += dppf<kRowHalfMirror>(v);
    v += dppf<kRowMirror>(v);
    return v;
}

// Sum of p[j] over the row's values in expert order e = 16 j + lane, one
// element at a time (((p_0 + p_1) + p_2) + ...): the sequential f32 sum of the
// reference's softmax denominator.  Each step is one v_add_f32 with a DPP
// row_newbcast operand (lane L of the row broadcast to all 16 lanes).
template <int L, int EP>
__device__ __forceinline__ float row_sum_in_order(const float (&p)[EP], float acc) {
    if constexpr (L == 16 * EP) {
        return acc;
    } else {
        return row_sum_in_order<L + 1, EP>(p, acc + dppf<0x150 + (L & 15)>(p[L >> 4]));
    }
}

__device__ __forceinline__ uint32_t row_or(uint32_t v) {
    v |= dpp<kQuadXor1>(v);
    v |= dpp<kQuadXor2>(v);
    v |= dpp<kRowHalfMirror>(v);
    v |= dpp<kRowMirror>(v);
    return v;
}

template <int Ctrl>
__device__ __forceinline__ uint64_t max_step(uint64_t v) {
    const uint64_t o = ((uint64_t)dpp<Ctrl>((uint32_t)(v >> 32)) << 32) | dpp<Ctrl>((uint32_t)v);
    return o > v ? o : v;
}

__device__ __forceinline__ uint64_t row_max_u64(uint64_t v) {
    v = max_step<kQuadXor1>(v);
    v = max_step<kQuadXor2>(v);
    v = max_step<kRowHalfMirror>(v);
    v = max_step<kRowMirror>(v);
    return v;
}

// Order-preserving map of an FP32 value onto uint32 (larger float -> larger key).
__device__ __forceinline__ uint32_t orderable(float v) {
    uint32_t u = __float_as_uint(v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Inverse of orderable().
__device__ __forceinline__ float from_orderable(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

template <typename T>
__device__ __forceinline__ float load_logit(const T* p, size_t i);
template <>
__device__ __forceinline__ float load_logit<float>(const float* p, size_t i) { return p[i]; }
template <>
__device__ __forceinline__ float load_logit<uint16_t>(const uint16_t* p, size_t i) {
    return bf16_bits_to_float(p[i]);
}

// Routes token `t` with the calling 16-lane row.  Writes the packed routes row
// and, when `eids` is non-null, the K selected experts (or -1 for every rank
// of a rejected row) at eids[0..K).  Returns true when the row was rejected.
// Rows with `active == false` take part in the DPP steps but write nothing.
// `normalize`: weights p / (rank-ordered sum of the K selected p), else the
// selected probabilities as they are (normalize_selected_weights of
// sparse_moe/config.rs:45, applied at routing.rs:198-202).
// Layout overrides (0 = default): `ldl` logits per row (E), `routes_stride`
// floats per routes row (2K) and `weights_ofs` offset of the weights in it (K).
template <int EP, typename T>
__device__ __forceinline__ bool route_row(const T* logits, int t, bool active, float* routes, int E, int K,
                                          int* eids, bool normalize, int ldl = 0, int routes_stride = 0,
                                          int weights_ofs = 0) {
    const int l16 = threadIdx.x & 15;
    const T* row = logits + (size_t)(active ? t : 0) * (ldl ? ldl : E);
    float d[EP], p[EP];  // logits; softmax probabilities
    uint32_t nonfinite = 0;
    float maximum = -INFINITY;
    // Unconditional loads (clamped index) so all EP loads are in flight at
    // once; a guarded load becomes a branch that waits for each in turn.
#pragma unroll
    for (int j = 0; j < EP; ++j) {
        const int e = j * 16 + l16;
        d[j] = load_logit<T>(row, e < E ? e : 0);
    }
#pragma unroll
    for (int j = 0; j < EP; ++j) {
        const bool in = j * 16 + l16 < E;
        nonfinite |= (uint32_t)(in && !__builtin_isfinite(d[j]));
        d[j] = in ? d[j] : -INFINITY;
        maximum = fmaxf(maximum, d[j]);
    }
    nonfinite = row_or(nonfinite);
    maximum = row_max(maximum);
    // Softmax as the reference's f32 CPU path computes it: numerators
    // exp(x - max) with glibc's expf bits, their sum in expert order, one
    // division each.  Experts are then ranked on these probabilities, so
    // distinct logits whose probabilities round equal tie to the lower id
    // exactly as routing.rs:239-257 does.
#pragma unroll
    for (int j = 0; j < EP; ++j) {
        const int e = j * 16 + l16;
        p[j] = e < E ? expf_glibc(d[j] - maximum) : 0.f;
    }
    const float denominator = row_sum_in_order<0, EP>(p, 0.f);
#pragma unroll
    for (int j = 0; j < EP; ++j) p[j] = p[j] / denominator;

    float selected_sum = 0.f;
    int my_id[2] = {0, 0};
    float my_p[2] = {0.f, 0.f};
    // Rank r's pick is published to lane r % 16 of the row (slot r / 16).
    auto publish = [&](int r, uint64_t best) {
        const int id = (int)(0xffffffffu - (uint32_t)best);
        const float prob = from_orderable((uint32_t)(best >> 32));  // the key is the probability
        selected_sum += prob;  // rank order, as routing.rs:187-191
        if (l16 == (r & 15)) {
            if (r < 16) { my_id[0] = id; my_p[0] = prob; }
            else { my_id[1] = id; my_p[1] = prob; }
        }
    };
    // pick(): the next expert of the row by (probability desc, id asc), as a
    // 64-bit key (orderable(probability), ~id) identical on all 16 lanes.
    // Up to 16 keys per lane: each lane sorts its keys once (bitonic network,
    // descending) and a pick is the row max of the lane heads; its owner
    // advances.  32 keys per lane: a strict '>' scan over the untaken 32-bit
    // values in slot order (the smallest id wins a tie within the lane).
    uint64_t key[EP <= 16 ? EP : 1];
    uint32_t ord[EP <= 16 ? 1 : EP];
    int h = 0;           // sorted form: keys this lane has given up
    uint32_t taken = 0;  // scan form: slots already picked
    if constexpr (EP <= 16) {
#pragma unroll
        for (int j = 0; j < EP; ++j) {
            const int e = j * 16 + l16;
            key[j] = e < E ? ((uint64_t)orderable(p[j]) << 32) | (0xffffffffu - (uint32_t)e) : 0;
        }
#pragma unroll
        for (int size = 2; size <= EP; size <<= 1)
#pragma unroll
            for (int stride = size / 2; stride > 0; stride >>= 1)
#pragma unroll
                for (int i = 0; i < EP; ++i) {
                    const int j = i ^ stride;
                    if (j > i) {
                        const uint64_t a = key[i], b = key[j];
                        const bool swap = (i & size) == 0 ? a < b : a > b;
                        key[i] = swap ? b : a;
                        key[j] = swap ? a : b;
                    }
                }
    } else {
#pragma unroll
        for (int j = 0; j < EP; ++j) ord[j] = j * 16 + l16 < E ? orderable(p[j]) : 0u;  // valid values are > 0
    }
    auto pick = [&]() -> uint64_t {
        if constexpr (EP <= 16) {
            // head = key[h] through a log2(EP)-level select tree; 0 once exhausted
            uint64_t t[EP];
#pragma unroll
            for (int i = 0; i < EP; ++i) t[i] = key[i];
#pragma unroll
            for (int w = EP / 2, b = 0; w >= 1; w /= 2, ++b)
#pragma unroll
                for (int i = 0; i < w; ++i) t[i] = ((h >> b) & 1) ? t[2 * i + 1] : t[2 * i];
            const uint64_t mine = h < EP ? t[0] : 0;
            const uint64_t best = row_max_u64(mine);
            h += mine == best;  // keys are distinct (ids differ): only the owner advances
            return best;
        } else {
            uint32_t bo = 0;
            int bj = 0;
#pragma unroll
            for (int j = 0; j < EP; ++j) {
                const uint32_t v = (taken >> j) & 1u ? 0u : ord[j];
                bj = v > bo ? j : bj;
                bo = v > bo ? v : bo;
            }
            const uint64_t mine = bo ? ((uint64_t)bo << 32) | (0xffffffffu - (uint32_t)(bj * 16 + l16)) : 0;
            const uint64_t best = row_max_u64(mine);
            taken |= (mine == best) ? 1u << bj : 0u;
            return best;
        }
    };
    if (K <= 16) {
        // Picks only record the winning key in lane r; probabilities are then
        // computed by all ranks at once and summed in rank order.
        uint64_t picked = 0;
        for (int r = 0; r < K; ++r) {
            const uint64_t best = pick();
            picked = l16 == r ? best : picked;
        }
        const bool ranked = l16 < K;
        const float prob = ranked ? from_orderable((uint32_t)(picked >> 32)) : 0.f;
        // Left fold p0 + p1 + ... + p(K-1), as the sequential loop of
        // routing.rs:187-191: lane r adds its p to lane r-1's partial.
        float partial = prob;
        for (int r = 1; r < K; ++r) {
            const float prev = __uint_as_float(
                (uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(partial), kRowShr1, 0xf, 0xf, false));
            partial = l16 == r ? prev + prob : partial;
        }
        selected_sum = __shfl(partial, (int)(threadIdx.x & ~15u) + K - 1, 64);
        my_id[0] = ranked ? (int)(0xffffffffu - (uint32_t)picked) : 0;
        my_p[0] = prob;
    } else {
        for (int r = 0; r < K; ++r) publish(r, pick());
    }
    if (active) {
        float* out = routes + (size_t)t * (routes_stride ? routes_stride : 2 * K);
        const int wofs = weights_ofs ? weights_ofs : K;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int rank = s * 16 + l16;
            if (rank < K) {
                out[rank] = nonfinite ? __builtin_nanf("") : (float)my_id[s];
                out[wofs + rank] = nonfinite ? __builtin_nanf("") : normalize ? my_p[s] / selected_sum : my_p[s];
                if (eids) eids[rank] = nonfinite ? -1 : my_id[s];
            }
        }
    }
    return nonfinite != 0;
}

// One wavefront (four tokens) per workgroup, so small batches still spread
// over every CU.
template <int EP, typename T>
__global__ __launch_bounds__(64) void route_kernel(const T* logits, float* routes, int T_, int E, int K,
                                                   int normalize) {
    const int t = blockIdx.x * 4 + (threadIdx.x >> 4);
    route_row<EP, T>(logits, t, t < T_, routes, E, K, nullptr, normalize != 0);
}

// Routing with an always-on shared expert folded in as expert E: logits rows
// hold E router logits then the shared gate logit x . w_s; ranks 0..K-1 are
// the routed top-K as route_kernel writes them, rank K is (id E, weight
// sigmoid(gate)), in rows of 2(K+1) floats.  A rejected routed row (or a
// non-finite gate, through its weight) invalidates the plan as before.
template <int EP, typename T>
__global__ __launch_bounds__(64) void route_shared_kernel(const T* logits, float* routes, int T_, int E, int K,
                                                          int normalize) {
    const int t = blockIdx.x * 4 + (threadIdx.x >> 4);
    const bool active = t < T_;
    const int K1 = K + 1;
    const bool bad = route_row<EP, T>(logits, t, active, routes, E, K, nullptr, normalize != 0, E + 1, 2 * K1, K1);
    if (active && (threadIdx.x & 15) == 0) {
        const float gate = load_logit<T>(logits, (size_t)t * (E + 1) + E);
        float* out = routes + (size_t)t * 2 * K1;
        out[K] = bad ? __builtin_nanf("") : (float)E;
        // sigmoid 1 / (1 + exp(-g)) with glibc's exp bits, as the f32 CPU path
        out[K1 + K] = bad ? __builtin_nanf("") : 1.0f / (1.0f + expf_glibc(-gate));
    }
}

// ---------------------------------------------------------------------------
// Dispatch
// ---------------------------------------------------------------------------
constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kSpanLds = 4096;      // assignments whose experts fit the LDS stage
constexpr int kSplitRouteTokens = 32;  // batches from this size route in their own launch

// Validates one externally supplied assignment (moe_dispatch.cu:23-33 of the
// reference): a finite integral id in [0,E), no duplicate among the token's
// earlier ranks, a finite non-negative weight.  Returns the expert or -1.
__device__ __forceinline__ int assignment_expert(const float* routes, int a, int K, int E) {
    const int t = a / K, r = a - t * K;
    const float* row = routes + (size_t)t * 2 * K;
    const float id = row[r], w = row[K + r];
    bool dup = false;
    for (int q0 = 0; q0 < r; q0 += 8) {  // earlier ranks, 8 loads in flight per batch
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = row[min(q0 + u, r)];  // clamped: unconditional loads
#pragma unroll
        for (int u = 0; u < 8; ++u) dup |= q0 + u < r && v[u] == id;
    }
    const bool valid = __builtin_isfinite(id) && id >= 0.f && id < (float)E && floorf(id) == id &&
                       __builtin_isfinite(w) && w >= 0.f && !dup;
    return valid ? (int)id : -1;
}

// Lanes of the wave holding the same expert (ballot over the id bits).
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
    const void* logits;  // routing input (null: routes given)
    int logits_bf16;
    int normalize;  // renormalise the selected weights (routing from logits only)
    float* routes;
    int* meta;
    int* offsets;
    int* slots;
    int* tiles;
    int* scratch;  // multi-workgroup: [chunks][E] counts -> bases; [chunks] flags
    int tokens, E, K, M;
    int capacity;
    int expert_bits;
    int chunk_tokens;  // tokens per workgroup chunk (multi-workgroup plan)
};

struct DispatchLds {
    int* wcount;    // [16][E] per-wave counts, then per-wave bases
    int* total;     // [E] counts of this workgroup's span
    int* padded;    // [E + 1] padded exclusive scan
    int* flag;      // [1]
    int* scan_tmp;  // [NT]
    int* eids;      // [kSpanLds] expert of each assignment of the span
    int* base;      // [E] multi-workgroup: this chunk's first slot per expert
};

template <int NT = kThreads>
__host__ __device__ inline size_t dispatch_lds_words(int E) {
    return (size_t)(NT / 64) * E + E + E + 1 + 1 + NT + kSpanLds + E;
}

template <int NT>
__device__ __forceinline__ DispatchLds dispatch_lds(int* lds, int E) {
    DispatchLds l;
    l.wcount = lds;
    l.total = lds + (NT / 64) * E;
    l.padded = l.total + E;
    l.flag = l.padded + E + 1;
    l.scan_tmp = l.flag + 1;
    l.eids = l.scan_tmp + NT;
    l.base = l.eids + kSpanLds;
    return l;
}

// Expert of assignment a of the span: from the LDS stage when it holds the span.
struct SpanExperts {
    const int* lds;  // null: read and validate routes in global memory
    int begin;
    __device__ __forceinline__ int get(const DispatchArgs& p, int a) const {
        return lds ? lds[a - begin] : assignment_expert(p.routes, a, p.K, p.E);
    }
};

// Stages the span's validated experts in LDS (span <= kSpanLds); sets flag on
// any invalid assignment.
template <int NT>
__device__ void stage_span(const DispatchArgs& p, const DispatchLds& l, int begin, int end) {
    bool bad = false;
    for (int a = begin + (int)threadIdx.x; a < end; a += NT) {
        const int e = assignment_expert(p.routes, a, p.K, p.E);
        l.eids[a - begin] = e;
        bad |= e < 0;
    }
    if (bad) l.flag[0] = 1;
}

// Per-wave counts of [begin, end) (each wave a contiguous segment), then the
// per-expert exclusive prefix over waves; total[e] = count of e in the span.
template <int NT>
__device__ void span_counts(const DispatchArgs& p, const DispatchLds& l, int begin_, int end_, SpanExperts src,
                            bool check) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int n = end_ - begin_;
    const int seg = ((n + (NT / 64) - 1) / (NT / 64) + 63) / 64 * 64;
    const int begin = begin_ + wave * seg, end = min(end_, begin + seg);
    int* my = l.wcount + wave * p.E;
    bool bad = false;
    for (int a0 = begin; a0 < end; a0 += 64) {
        const int a = a0 + lane;
        const int e = a < end ? src.get(p, a) : -1;
        if (check && a < end) bad |= e < 0;
        const bool active = e >= 0;
        const uint64_t peers = match_expert(e, active, p.expert_bits);
        if (active && (peers & lanemask_lt()) == 0) my[e] += __popcll(peers);
    }
    if (check && __any(bad) && lane == 0) l.flag[0] = 1;
    __syncthreads();
    for (int e = tid; e < p.E; e += NT) {
        int run = 0;
        for (int w = 0; w < (NT / 64); ++w) {
            const int c = l.wcount[w * p.E + e];
            l.wcount[w * p.E + e] = run;
            run += c;
        }
        l.total[e] = run;
    }
    __syncthreads();
}

// Stable scatter of the span: slot = base[e] + per-wave base + in-wave rank.
template <int NT>
__device__ void span_scatter(const DispatchArgs& p, const DispatchLds& l, int begin_, int end_, SpanExperts src,
                             const int* base) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int n = end_ - begin_;
    const int seg = ((n + (NT / 64) - 1) / (NT / 64) + 63) / 64 * 64;
    const int begin = begin_ + wave * seg, end = min(end_, begin + seg);
    int* my = l.wcount + wave * p.E;
    for (int a0 = begin; a0 < end; a0 += 64) {
        const int a = a0 + lane;
        const int e = a < end ? src.get(p, a) : -1;
        const bool active = e >= 0;
        const uint64_t peers = match_expert(e, active, p.expert_bits);
        const int leader = peers ? __ffsll((unsigned long long)peers) - 1 : 0;
        int off = 0;
        if (active && lane == leader) off = my[e];
        off = __shfl(off, leader, 64);
        if (active) {
            p.slots[base[e] + off + __popcll(peers & lanemask_lt())] = a;
            if (lane == leader) my[e] = off + __popcll(peers);
        }
    }
}

// Padded exclusive scan of total[] over experts into padded[0..E] (E <=
// NT: one expert per thread): shuffle scan within each wave, wave totals
// through LDS, one barrier.
template <int NT>
__device__ void padded_scan(const DispatchArgs& p, const DispatchLds& l) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int v = tid < p.E ? (l.total[tid] + p.M - 1) / p.M * p.M : 0;
    int x = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(x, d, 64);
        if (lane >= d) x += y;
    }
    if (lane == 63) l.scan_tmp[wave] = x;
    __syncthreads();
    int before = 0;
    for (int w = 0; w < wave; ++w) before += l.scan_tmp[w];
    const int exclusive = before + x - v;
    if (tid < p.E) l.padded[tid] = exclusive;
    if (tid == p.E - 1) l.padded[p.E] = exclusive + v;
    __syncthreads();
}

// Metadata words, offsets, the tile worklist and padding sentinels, from the
// plan in LDS (total = per-expert counts, padded = padded offsets).  Work is
// split over `parts` workgroups (the chunk workgroups of the multi-workgroup
// plan); part 0 writes the metadata words.
template <int NT>
__device__ void finalize_part(const DispatchArgs& p, const DispatchLds& l, int status, int part, int parts) {
    const int tid = threadIdx.x;
    const int A = p.tokens * p.K;
    const int padded_total = l.padded[p.E];
    if (part == 0) {
        for (int e = tid; e < p.E; e += NT) {
            p.meta[e] = l.total[e];
            p.meta[p.E + e] = l.total[e];
            p.offsets[e] = l.padded[e];
        }
        if (tid == 0) {
            p.offsets[p.E] = padded_total;
            p.meta[2 * p.E] = status;
            p.meta[2 * p.E + 1] = padded_total;
        }
    }
    // Tile worklist and padding sentinels straight from each expert's padded
    // range [padded[e], padded[e+1]).  This part's experts are e = part +
    // parts * j; wave w takes j = w, w + 16, ...: lane i first reads expert
    // j = w + 16 i's range from LDS (one read per lane), then the wave walks
    // its experts with readlane, its lanes storing 64 consecutive rows
    // (coalesced) per instruction.
    const int ntiles = p.capacity / p.M;
    {
        const int wave = tid >> 6, lane = tid & 63;
        const int nmine = part < p.E ? (p.E - part + parts - 1) / parts : 0;
        const int jl = wave + (NT / 64) * lane;
        int pb = 0, pe = 0, pt = 0;
        if (jl < nmine) {
            const int e = part + parts * jl;
            pb = l.padded[e];
            pe = l.padded[e + 1];
            pt = l.total[e];
        }
        const int count = wave < nmine ? (nmine - wave + (NT / 64) - 1) / (NT / 64) : 0;
        for (int i = 0; i < count; ++i) {
            const int e = part + parts * (wave + (NT / 64) * i);
            const int b = __builtin_amdgcn_readlane(pb, i), end = __builtin_amdgcn_readlane(pe, i);
            const int valid_end = b + __builtin_amdgcn_readlane(pt, i);
            for (int t = b / p.M + lane; t < end / p.M; t += 64) p.tiles[t] = e;
            for (int row = valid_end + lane; row < end; row += 64) p.slots[row] = A;
        }
    }
    const int stride = parts * NT, first = part * NT + tid;
    for (int t = padded_total / p.M + first; t < ntiles; t += stride) p.tiles[t] = -1;
    for (long row = (long)padded_total + first; row < p.capacity; row += stride) p.slots[row] = A;
}

// Routes tokens [t0, t1) with the workgroup (4 tokens per wave per pass),
// staging the experts of assignments [t0*K, t1*K) in l.eids.
template <int EP, int NT>
__device__ void route_span(const DispatchArgs& p, const DispatchLds& l, int t0, int t1) {
    const int row = threadIdx.x >> 4;  // 64 rows per workgroup
    bool bad = false;
    for (int tb = t0; tb < t1; tb += NT / 16) {
        const int t = tb + row;
        const bool active = t < t1;
        int* eids = l.eids + (size_t)(t - t0) * p.K;
        if (p.logits_bf16)
            bad |= route_row<EP, uint16_t>((const uint16_t*)p.logits, t, active, p.routes, p.E, p.K, eids,
                                                 p.normalize != 0) && active;
        else
            bad |= route_row<EP, float>((const float*)p.logits, t, active, p.routes, p.E, p.K, eids,
                                                 p.normalize != 0) && active;
    }
    if (bad) l.flag[0] = 1;
}

template <int NT>
__device__ void clear_counts(const DispatchArgs& p, const DispatchLds& l) {
    for (int i = threadIdx.x; i < (NT / 64) * p.E; i += NT) l.wcount[i] = 0;
    if (threadIdx.x == 0) l.flag[0] = 0;
    __syncthreads();
}

// One workgroup (NT) builds the whole plan (optionally routing first);
// `lds` holds dispatch_lds_words(E) words.
template <int EP, int NT>
__device__ void dispatch_single_body(const DispatchArgs& p, int* lds) {
    const DispatchLds l = dispatch_lds<NT>(lds, p.E);
    const int A = p.tokens * p.K;
    clear_counts<NT>(p, l);
    SpanExperts src{nullptr, 0};
    if (A <= kSpanLds) {
        if (p.logits) route_span<EP, NT>(p, l, 0, p.tokens);
        else stage_span<NT>(p, l, 0, A);
        src.lds = l.eids;
    }
    __syncthreads();
    span_counts<NT>(p, l, 0, A, src, src.lds == nullptr);
    const int status = l.flag[0];
    padded_scan<NT>(p, l);
    span_scatter<NT>(p, l, 0, A, src, l.padded);
    finalize_part<NT>(p, l, status, 0, 1);
}

template <int EP>
__global__ __launch_bounds__(kThreads) void dispatch_single_kernel(DispatchArgs p) {
    extern __shared__ int lds[];
    dispatch_single_body<EP, kThreads>(p, lds);
}

// Multi-workgroup plan, step 1: route (or stage) one chunk of tokens and
// publish its per-expert counts and status.
template <int EP>
__global__ __launch_bounds__(kThreads) void dispatch_hist_kernel(DispatchArgs p) {
    extern __shared__ int lds[];
    const DispatchLds l = dispatch_lds<kThreads>(lds, p.E);
    const int c = blockIdx.x;
    const int t0 = c * p.chunk_tokens, t1 = min(p.tokens, t0 + p.chunk_tokens);
    clear_counts<kThreads>(p, l);
    if (p.logits) route_span<EP, kThreads>(p, l, t0, t1);
    else stage_span<kThreads>(p, l, t0 * p.K, t1 * p.K);
    __syncthreads();
    span_counts<kThreads>(p, l, t0 * p.K, t1 * p.K, SpanExperts{l.eids, t0 * p.K}, false);
    for (int e = threadIdx.x; e < p.E; e += kThreads) p.scratch[(size_t)c * p.E + e] = l.total[e];
    if (threadIdx.x == 0) p.scratch[(size_t)gridDim.x * p.E + c] = l.flag[0];
}

// Step 2: every chunk workgroup recomputes the plan from the chunk counts
// (per-expert totals, its own chunk's prefix, the padded scan; a few KB from
// L2), writes its share of the tile worklist and sentinels, then scatters its
// chunk stably from the absolute per-expert bases.
__global__ __launch_bounds__(kThreads) void dispatch_scatter_kernel(DispatchArgs p) {
    extern __shared__ int lds[];
    const DispatchLds l = dispatch_lds<kThreads>(lds, p.E);
    const int c = blockIdx.x, chunks = gridDim.x;
    clear_counts<kThreads>(p, l);
    for (int e = threadIdx.x; e < p.E; e += kThreads) {
        int run = 0, before = 0;
        for (int q0 = 0; q0 < chunks; q0 += 8) {  // 8 independent loads in flight per batch
            int v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = p.scratch[(size_t)min(q0 + u, chunks - 1) * p.E + e];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int q = q0 + u;
                before = q == c ? run : before;
                run += q < chunks ? v[u] : 0;
            }
        }
        l.total[e] = run;
        l.base[e] = before;
    }
    for (int q = threadIdx.x; q < chunks; q += kThreads)
        if (p.scratch[(size_t)chunks * p.E + q]) l.flag[0] = 1;
    __syncthreads();
    const int status = l.flag[0];
    padded_scan<kThreads>(p, l);
    for (int e = threadIdx.x; e < p.E; e += kThreads) l.base[e] += l.padded[e];
    finalize_part<kThreads>(p, l, status, c, chunks);
    __syncthreads();
    const int b = c * p.chunk_tokens * p.K, e_ = min(p.tokens, (c + 1) * p.chunk_tokens) * p.K;
    stage_span<kThreads>(p, l, b, e_);  // routes were validated by the histogram step
    __syncthreads();
    const SpanExperts src{l.eids, b};
    span_counts<kThreads>(p, l, b, e_, src, false);
    span_scatter<kThreads>(p, l, b, e_, src, l.base);
}

}  // namespace
}  // namespace tau_amd
