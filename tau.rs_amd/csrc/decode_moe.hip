// Fused decode path of the MoE layer (small batches: T <= 64 tokens, E <= 256).
//
// Same results as the general path (routing -> dispatch -> grouped gate_up ->
// grouped down -> combine; moe_prefill.cu:15-38 of the reference), reordered so
// that the dispatch plan is off the critical path.  At decode sizes the layer is
// a weight stream (every expert's gate_up and down panels, ~1.2 GB for
// Qwen3-30B-A3B) and the plan kernels were pure latency in front of it:
//   1. routing over every CU (routes [T, 2K]);
//   2. gate_up: one wave per (expert, 32 output columns).  The wave issues its
//      first weight batch, then finds its expert's assignments by scanning the
//      routes (T*K ids, token order = the plan's stable order), and streams the
//      expert's panel through 16x16x32 MFMAs for those rows;
//      activated[a] = bf16(silu(bf16 g) * bf16 u) for assignment a = t*K + r;
//   3. down: the same row lists; contributions[a] = bf16(acc * w[a]).  One
//      extra workgroup of this launch builds the dispatch plan (meta, offsets,
//      slots, tiles) from the routes while the other waves stream weights;
//   4. the rank-ordered combine (reads the plan's status word).
// Per output element the MFMA sequence (K order, 16x16x32 shape) and the
// epilogue roundings are those of the streaming kernel of the general path, so
// the outputs are bit-identical to it.
#include "dispatch.hpp"

namespace tau_amd {

namespace {

__device__ __forceinline__ bf16x8 as_bf16x8_(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

struct DecodeArgs {
    const uint16_t* a;     // gate_up: x [T, lda]; down: activated [T*K, lda] (by assignment)
    const uint16_t* w;     // expert weights [E][N_w][k] (row-major or frag16)
    const float* routes;   // [T, 2K]
    void* out;             // gate_up: activated [T*K, ldo]; down: contributions [T*K, ldo]
    int tokens, K, E;
    int n, k;              // output columns, inner dimension
    int lda, ldo;
    long w_expert_stride;  // elements
    int w_up_offset;       // rows between gate row j and up row j (gate_up)
    int* receipt;          // optional 5 words
};

constexpr int kListRows = 64;  // assignments per expert the row list holds (T <= 64)

template <int NB, int U>
struct DecodeBatch {
    u32x4 g[NB][U];
    u32x4 u[NB][U];
    u32x4 x[U];
};

// EPI: kEpiSilu (gate_up, A rows = tokens) or kEpiScatterWeighted (down, A
// rows = assignments).  PLAN: the last workgroup builds the dispatch plan.
template <int EPI, int NB, int U, int W, int WL, bool PLAN>
__global__ __launch_bounds__(64 * W) void decode_gemm_kernel(DecodeArgs p, DispatchArgs plan) {
    if constexpr (PLAN) {
        if (blockIdx.x == gridDim.x - 1) {
            extern __shared__ int plan_lds[];
            static_assert(!PLAN || W == 4, "the plan workgroup runs with 256 threads");
            dispatch_single_body<1, 64 * W>(plan, plan_lds);  // from routes: no routing inside
            return;
        }
    }
    constexpr bool kSilu = EPI == kEpiSilu;
    constexpr int KS = WL == kWeightsFrag16 ? 16 : 1;  // weight elements per unit of k
    __shared__ int row_list[W][kListRows];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (p.receipt && blockIdx.x == 0 && threadIdx.x == 0) {
        p.receipt[0] = 16; p.receipt[1] = 16 * NB * (kSilu ? 2 : 1); p.receipt[2] = 32 * U;
        p.receipt[3] = W; p.receipt[4] = 2;
    }
    const int n_groups = (p.n + 16 * NB - 1) / (16 * NB);
    const int total = p.E * n_groups;
    const int groups = (total + W - 1) / W;
    const int per_xcd = (groups + kXcds - 1) / kXcds;
    const int group = xcd_remap(blockIdx.x, per_xcd);
    const int item = group * W + wave;
    if (group < 0 || group >= groups || item >= total) return;
    const int e = item / n_groups, ng = item - e * n_groups;

    // Weight stream pointers (as the general streaming kernel).
    const uint16_t* wexp = p.w + (long)e * p.w_expert_stride;
    const uint16_t* wg[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int col = ng * 16 * NB + b * 16 + (lane & 15);
        if constexpr (WL == kWeightsFrag16)
            wg[b] = wexp + (long)(col < p.n ? col >> 4 : 0) * 16 * p.k + lane * 8;
        else
            wg[b] = wexp + (long)(col < p.n ? col : 0) * p.k + (lane >> 4) * 8;
    }
    const long up = (long)p.w_up_offset * p.k;
    const int kofs = (lane >> 4) * 8;
    const uint16_t* xs = p.a;  // set per row group
    auto load = [&](DecodeBatch<NB, U>& t, int kb) {
#pragma unroll
        for (int q = 0; q < U; ++q) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                t.g[b][q] = *(const u32x4*)(wg[b] + (kb + q * 32) * KS);
                if constexpr (kSilu) t.u[b][q] = *(const u32x4*)(wg[b] + up + (kb + q * 32) * KS);
            }
            t.x[q] = *(const u32x4*)(xs + kb + q * 32);
        }
    };

    constexpr int KB = 32 * U;
    const int main_k = p.k / KB * KB;
    DecodeBatch<NB, U> b0, b1;
    // First weight batch in flight before the row scan (x is loaded again
    // once the rows are known).
    if (main_k > 0) load(b0, 0);

    // Row list: this expert's assignments in ascending order.  8 route loads
    // in flight per lane per pass (clamped indices, no branches).
    const int A = p.tokens * p.K;
    int* list = row_list[wave];
    list[lane] = -1;
    int n_rows = 0;
    const float fe = (float)e;
    for (int base = 0; base < A; base += 64 * 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int a = min(base + u * 64 + lane, A - 1);
            const int t = a / p.K;
            v[u] = p.routes[(size_t)t * 2 * p.K + (a - t * p.K)];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int a = base + u * 64 + lane;
            const bool hit = a < A && v[u] == fe;
            const uint64_t m = __ballot(hit);
            const int rank = n_rows + __popcll(m & lanemask_lt());
            if (hit && rank < kListRows) list[rank] = a;
            n_rows += __popcll(m);
        }
    }
    if (n_rows > kListRows) n_rows = kListRows;  // unreachable for T <= 64 (one rank per token and expert)
    // The list is read below by other lanes of this wave: the wave's LDS
    // stores come first (waves execute in order; this keeps the compiler from
    // moving the reads above them).
    __builtin_amdgcn_wave_barrier();

    for (int g0 = 0; g0 < n_rows; g0 += 16) {
        const int a_row = list[g0 + (lane & 15)];  // -1: padding lane
        const bool ok = g0 + (lane & 15) < n_rows && a_row >= 0;
        long x_row = 0;
        if (ok) x_row = kSilu ? a_row / p.K : a_row;
        xs = p.a + x_row * (long)p.lda + kofs;

        f32x4 acc_g[NB], acc_u[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int q = 0; q < 4; ++q) acc_g[b][q] = acc_u[b][q] = 0.f;
        auto mma = [&](DecodeBatch<NB, U>& t) {
#pragma unroll
            for (int q = 0; q < U; ++q) {
                u32x4 xv = t.x[q];
                if (!ok) xv = u32x4{0u, 0u, 0u, 0u};
                const bf16x8 xb = as_bf16x8_(xv);
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    acc_g[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8_(t.g[b][q]), xb, acc_g[b], 0, 0, 0);
                    if constexpr (kSilu)
                        acc_u[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8_(t.u[b][q]), xb, acc_u[b], 0, 0, 0);
                }
            }
        };
        int kb = 0;
        if (main_k > 0) {
            if (g0 == 0) {
                // the weights of b0 are in flight; fetch the now known x rows
#pragma unroll
                for (int q = 0; q < U; ++q) b0.x[q] = *(const u32x4*)(xs + q * 32);
            } else {
                load(b0, 0);
            }
            for (; kb + 2 * KB <= main_k; kb += 2 * KB) {
                load(b1, kb + KB);
                mma(b0);
                if (kb + 2 * KB < main_k) load(b0, kb + 2 * KB);
                mma(b1);
            }
            if (kb < main_k) {
                mma(b0);
                kb += KB;
            }
        }
        for (; kb < p.k; kb += 32) {  // K tail in 32-wide steps (k % 32 == 0 on this path)
            const u32x4 xv = ok ? *(const u32x4*)(xs + kb) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const u32x4 gv = *(const u32x4*)(wg[b] + kb * KS);
                acc_g[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8_(gv), as_bf16x8_(xv), acc_g[b], 0, 0, 0);
                if constexpr (kSilu) {
                    const u32x4 uv = *(const u32x4*)(wg[b] + up + kb * KS);
                    acc_u[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8_(uv), as_bf16x8_(xv), acc_u[b], 0, 0, 0);
                }
            }
        }

        // 16x16 accumulator: value q of lane l is column (l/16)*4 + q of the
        // block, row l%16 of the group.
        if (!ok) continue;
        float wt = 1.0f;
        if constexpr (!kSilu) {
            const int t = a_row / p.K;
            wt = p.routes[(size_t)t * 2 * p.K + p.K + (a_row - t * p.K)];
        }
        uint16_t* out = (uint16_t*)p.out + (long)a_row * p.ldo;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int oc = ng * 16 * NB + b * 16 + (lane >> 4) * 4;
            float v[4];
#pragma unroll
            for (int q = 0; q < 4; ++q)
                v[q] = kSilu ? silu(round_bf16(acc_g[b][q])) * round_bf16(acc_u[b][q]) : acc_g[b][q] * wt;
            if (oc + 3 < p.n) {
                u32x2 pk;
                pk[0] = pack_bf16x2(v[0], v[1]);
                pk[1] = pack_bf16x2(v[2], v[3]);
                *(u32x2*)(out + oc) = pk;
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    if (oc + q < p.n) out[oc + q] = float_to_bf16_bits(v[q]);
            }
        }
    }
}

template <int EPI, int NB, int U, int W, int WL, bool PLAN>
int launch_decode_gemm(const DecodeArgs& p, const DispatchArgs& plan, size_t plan_lds, hipStream_t s) {
    const long n_groups = (p.n + 16 * NB - 1) / (16 * NB);
    const long groups = ((long)p.E * n_groups + W - 1) / W;
    const long grid = (groups + kXcds - 1) / kXcds * kXcds + (PLAN ? 1 : 0);
    if (grid <= 0 || grid > 0x7fffffffL) return kInvalid;
    decode_gemm_kernel<EPI, NB, U, W, WL, PLAN><<<(unsigned)grid, 64 * W, PLAN ? plan_lds : 0, s>>>(p, plan);
    return (int)hipGetLastError();
}

}  // namespace

bool decode_path_supported(int tokens, int hidden, int intermediate, int experts, int top_k, int tile_rows,
                           int weight_layout) {
    return tile_rows == 16 && tokens >= 1 && tokens <= kListRows && experts <= 256 && top_k <= 32 &&
           hidden % 64 == 0 && intermediate % 64 == 0 &&
           (weight_layout == kWeightsRowMajor || weight_layout == kWeightsFrag16);
}

namespace {

// Plan arguments of the down launch's plan workgroup (built from the routes).
DispatchArgs decode_plan_args(float* routes, int* meta, int* offsets, int* slots, int* tiles, int tokens,
                              int experts, int top_k, int capacity) {
    DispatchArgs plan{};
    plan.routes = routes;
    plan.meta = meta;
    plan.offsets = offsets;
    plan.slots = slots;
    plan.tiles = tiles;
    plan.tokens = tokens;
    plan.E = experts;
    plan.K = top_k;
    plan.M = 16;
    plan.capacity = capacity;
    int bits = 0;
    while ((1 << bits) < experts) ++bits;
    plan.expert_bits = bits;
    return plan;
}

DecodeArgs decode_gate_up_args(const void* input, const void* gate_up, const float* routes, void* activated,
                               int tokens, int hidden, int intermediate, int experts, int top_k, int* receipt) {
    DecodeArgs g{};
    g.a = (const uint16_t*)input;
    g.w = (const uint16_t*)gate_up;
    g.routes = routes;
    g.out = activated;
    g.tokens = tokens;
    g.K = top_k;
    g.E = experts;
    g.n = intermediate;
    g.k = hidden;
    g.lda = hidden;
    g.ldo = intermediate;
    g.w_expert_stride = (long)2 * intermediate * hidden;
    g.w_up_offset = intermediate;
    g.receipt = receipt;
    return g;
}

DecodeArgs decode_down_args(const void* activated, const void* down, const float* routes, void* contributions,
                            int tokens, int hidden, int intermediate, int experts, int top_k, int* receipt) {
    DecodeArgs d{};
    d.a = (const uint16_t*)activated;
    d.w = (const uint16_t*)down;
    d.routes = routes;
    d.out = contributions;
    d.tokens = tokens;
    d.K = top_k;
    d.E = experts;
    d.n = hidden;
    d.k = intermediate;
    d.lda = intermediate;
    d.ldo = hidden;
    d.w_expert_stride = (long)hidden * intermediate;
    d.w_up_offset = 0;
    d.receipt = receipt;
    return d;
}

// Column blocks per wave and K batch depth measured on MI355X for these
// kernels (frag16 gate_up 2 x 16 columns, 8 x 32 K; down 4 x 16 columns,
// 4 x 32 K for K < 1024 (Qwen3-30B-A3B), 2 x 16 columns, 8 x 32 K for
// longer rows (Qwen3-235B-A22B)); the plan workgroup of the down launch
// has the same 256 threads as the GEMM workgroups.
int launch_decode_gate_up(const DecodeArgs& g, int weight_layout, hipStream_t s) {
    const DispatchArgs none{};
    if (weight_layout == kWeightsFrag16)
        return launch_decode_gemm<kEpiSilu, 2, 8, 4, kWeightsFrag16, false>(g, none, 0, s);
    return launch_decode_gemm<kEpiSilu, 1, 4, 4, kWeightsRowMajor, false>(g, none, 0, s);
}

int launch_decode_down(const DecodeArgs& d, const DispatchArgs& plan, int weight_layout, hipStream_t s) {
    const size_t plan_lds = sizeof(int) * dispatch_lds_words<256>(plan.E);
    if (weight_layout == kWeightsFrag16) {
        if (d.k < 1024)
            return launch_decode_gemm<kEpiScatterWeighted, 4, 4, 4, kWeightsFrag16, true>(d, plan, plan_lds, s);
        return launch_decode_gemm<kEpiScatterWeighted, 2, 8, 4, kWeightsFrag16, true>(d, plan, plan_lds, s);
    }
    return launch_decode_gemm<kEpiScatterWeighted, 4, 4, 4, kWeightsRowMajor, true>(d, plan, plan_lds, s);
}

}  // namespace

int launch_decode_moe(const void* input, const void* logits, int logits_dtype, const void* gate_up,
                      const void* down, float* routes, int* meta, int* offsets, int* slots, int* tiles,
                      void* activated, void* contributions, void* output, int tokens, int hidden,
                      int intermediate, int experts, int top_k, int capacity, int weight_layout,
                      const void* residual, int* receipts, hipStream_t s) {
    if (!decode_path_supported(tokens, hidden, intermediate, experts, top_k, 16, weight_layout)) return kInvalid;
    int code = 0;
#ifdef TAU_DECODE_ONE_LAUNCH
    code = launch_decode_layer(input, logits, logits_dtype, gate_up, down, routes, meta, offsets, slots, tiles,
                               activated, contributions, tokens, hidden, intermediate, experts, top_k, capacity,
                               weight_layout, receipts, s);
    if (code != kNotApplicable) {
        if (code) return code;
        return launch_combine(contributions, output, meta + 2 * experts, tokens, hidden, top_k, residual, s);
    }
    code = 0;
#endif
    if (logits) {  // otherwise the caller's routes (routing fused with the router projection)
        code = launch_routing(logits, logits_dtype, routes, tokens, experts, top_k, s);
        if (code) return code;
    }
    const DispatchArgs plan = decode_plan_args(routes, meta, offsets, slots, tiles, tokens, experts, top_k, capacity);
    const DecodeArgs g = decode_gate_up_args(input, gate_up, routes, activated, tokens, hidden, intermediate, experts,
                                             top_k, receipts);
    const DecodeArgs d = decode_down_args(activated, down, routes, contributions, tokens, hidden, intermediate,
                                          experts, top_k, receipts ? receipts + 5 : nullptr);
    code = launch_decode_gate_up(g, weight_layout, s);
    if (code) return code;
    code = launch_decode_down(d, plan, weight_layout, s);
    if (code) return code;
    return launch_combine(contributions, output, meta + 2 * experts, tokens, hidden, top_k, residual, s);
}

int launch_decode_projection(const void* a, const void* w, float* routes, int* meta, int* offsets, int* slots,
                             int* tiles, void* out, int tokens, int hidden, int intermediate, int experts, int top_k,
                             int capacity, int projection, int weight_layout, int* receipt, hipStream_t s) {
    if (!a || !w || !routes || !out || (projection != 0 && projection != 1) ||
        !decode_path_supported(tokens, hidden, intermediate, experts, top_k, 16, weight_layout))
        return kInvalid;
    if (projection == 0)
        return launch_decode_gate_up(decode_gate_up_args(a, w, routes, out, tokens, hidden, intermediate, experts,
                                                         top_k, receipt),
                                     weight_layout, s);
    if (!meta || !offsets || !slots || !tiles || capacity < capacity_for(tokens, experts, top_k, 16)) return kInvalid;
    return launch_decode_down(decode_down_args(a, w, routes, out, tokens, hidden, intermediate, experts, top_k, receipt),
                              decode_plan_args(routes, meta, offsets, slots, tiles, tokens, experts, top_k, capacity),
                              weight_layout, s);
}

}  // namespace tau_amd
