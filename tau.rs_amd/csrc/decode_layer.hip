// One-launch decode layer (T <= 64 tokens): routing, gate_up + SiLU·mul and
// down + route weight for one expert per workgroup, with the expert's
// activated rows kept in LDS between the two projections; then the
// rank-ordered combine as a second launch.
//
// The two-launch decode path (decode_moe.hip) streams gate_up's weights in one
// launch and down's in the next: the second launch cannot start streaming
// until the first has drained, and each launch ends in a partial round of
// workgroups.  Here each workgroup owns (expert e, split s): it routes every
// token itself (the routes are a few KB of L2 reads), collects e's
// assignments, streams e's whole gate_up panel into activated rows in LDS,
// then streams its share (1/S of the columns) of e's down panel.  With
// E * S workgroups, one per CU, every CU streams the same number of weight
// bytes (balanced whatever the routing), and the S workgroups of an expert run
// side by side on one XCD, so the gate_up panel they all read comes from HBM
// once.  The workgroups also write the dispatch plan the API returns (meta,
// offsets, slots, tiles; the two-launch path builds it in one extra
// workgroup): each counts every assignment (a 2K-entry LDS histogram), and
// split 0 of expert e writes e's share.
//
// Per output element the MFMA sequence (16x16x32 over K in order) and the
// epilogue roundings are those of the two-launch path, so results are
// bit-identical to it (and to the general path).
//
// Compiled in with -DTAU_DECODE_ONE_LAUNCH (off by default until measured).
#include "dispatch.hpp"

namespace tau_amd {

#ifdef TAU_DECODE_ONE_LAUNCH

namespace {

__device__ __forceinline__ bf16x8 as_bf16x8_l(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

constexpr int kLayerWaves = 4;  // one wave per SIMD: the gate_up stream holds ~400 registers
constexpr int kLayerThreads = 64 * kLayerWaves;
constexpr int kLayerMaxTokens = 64;
constexpr int kLayerMaxExperts = 256;

struct DecodeLayerArgs {
    const void* logits;
    int logits_bf16, normalize;
    const uint16_t* x;         // [T, H]
    const uint16_t* gate_up;   // [E][2I][H]
    const uint16_t* down;      // [E][H][I]
    uint16_t* activated;       // [T*K, I] by assignment (written by split 0)
    uint16_t* contributions;   // [T*K, H] by assignment
    int tokens, K, E, H, I;
    int splits;                // workgroups per expert (down columns split S ways)
    int* receipt;              // optional 10 words
};

template <int NB, int U, bool SILU>
struct LayerBatch {
    u32x4 g[NB][U];
    u32x4 u[NB][SILU ? U : 1];
    u32x4 x[U];
};

// Streams columns [col0, col0 + 16 NB) of one expert panel (k inner) against
// the assignment rows list[0..n_rows) in groups of 16, as the two-launch
// decode kernel does per wave.  A rows come from `a_of(row_index)` (a pointer
// to the row's first element; global x for gate_up, LDS activated for down).
// SILU: gate rows col, up rows col + up_rows; the result
// bf16(silu(bf16 g) * bf16 u) goes to store(row_index, col, packed pair...).
template <int NB, int U, int WL, bool SILU, typename ARow, typename Store>
__device__ __forceinline__ void stream_columns(const uint16_t* wexp, int n, int k, long up_rows, int col0,
                                               const int* list, int n_rows, ARow a_of, Store store,
                                               LayerBatch<NB, U, SILU>& b0, bool b0_loaded) {
    constexpr int KS = WL == kWeightsFrag16 ? 16 : 1;
    const int lane = threadIdx.x & 63;
    const uint16_t* wg[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int col = col0 + b * 16 + (lane & 15);
        if constexpr (WL == kWeightsFrag16)
            wg[b] = wexp + (long)(col < n ? col >> 4 : 0) * 16 * k + lane * 8;
        else
            wg[b] = wexp + (long)(col < n ? col : 0) * k + (lane >> 4) * 8;
    }
    const long up = up_rows * k;
    const int kofs = (lane >> 4) * 8;
    const uint16_t* xs = nullptr;
    auto load_w = [&](LayerBatch<NB, U, SILU>& t, int kb) {
#pragma unroll
        for (int q = 0; q < U; ++q)
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                t.g[b][q] = *(const u32x4*)(wg[b] + (kb + q * 32) * KS);
                if constexpr (SILU) t.u[b][q] = *(const u32x4*)(wg[b] + up + (kb + q * 32) * KS);
            }
    };
    auto load_x = [&](LayerBatch<NB, U, SILU>& t, int kb) {
#pragma unroll
        for (int q = 0; q < U; ++q) t.x[q] = *(const u32x4*)(xs + kb + q * 32);
    };
    constexpr int KB = 32 * U;
    const int main_k = k / KB * KB;
    if (main_k > 0 && !b0_loaded) load_w(b0, 0);
    LayerBatch<NB, U, SILU> b1;
    for (int g0 = 0; g0 < n_rows; g0 += 16) {
        const int ri = g0 + (lane & 15);
        const bool ok = ri < n_rows;
        xs = a_of(ok ? ri : 0) + kofs;
        f32x4 acc_g[NB], acc_u[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int q = 0; q < 4; ++q) acc_g[b][q] = acc_u[b][q] = 0.f;
        auto mma = [&](LayerBatch<NB, U, SILU>& t) {
#pragma unroll
            for (int q = 0; q < U; ++q) {
                u32x4 xv = t.x[q];
                if (!ok) xv = u32x4{0u, 0u, 0u, 0u};
                const bf16x8 xb = as_bf16x8_l(xv);
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    acc_g[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8_l(t.g[b][q]), xb, acc_g[b], 0, 0, 0);
                    if constexpr (SILU)
                        acc_u[b] =
                            __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8_l(t.u[b][q]), xb, acc_u[b], 0, 0, 0);
                }
            }
        };
        int kb = 0;
        if (main_k > 0) {
            if (g0 > 0) load_w(b0, 0);  // later row groups stream the panel again (from L2)
            load_x(b0, 0);
            for (; kb + 2 * KB <= main_k; kb += 2 * KB) {
                load_w(b1, kb + KB);
                load_x(b1, kb + KB);
                mma(b0);
                if (kb + 2 * KB < main_k) {
                    load_w(b0, kb + 2 * KB);
                    load_x(b0, kb + 2 * KB);
                }
                mma(b1);
            }
            if (kb < main_k) {
                mma(b0);
                kb += KB;
            }
        }
        for (; kb < k; kb += 32) {  // K tail in 32-wide steps (k % 32 == 0 on this path)
            const u32x4 xv = ok ? *(const u32x4*)(xs + kb) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const u32x4 gv = *(const u32x4*)(wg[b] + kb * KS);
                acc_g[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8_l(gv), as_bf16x8_l(xv), acc_g[b], 0, 0, 0);
                if constexpr (SILU) {
                    const u32x4 uv = *(const u32x4*)(wg[b] + up + kb * KS);
                    acc_u[b] =
                        __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8_l(uv), as_bf16x8_l(xv), acc_u[b], 0, 0, 0);
                }
            }
        }
        if (!ok) continue;
        // 16x16 accumulator: value q of lane l is column (l/16)*4 + q of the
        // block, row l%16 of the group.
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int oc = col0 + b * 16 + (lane >> 4) * 4;
            float v[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] = SILU ? silu(round_bf16(acc_g[b][q])) * round_bf16(acc_u[b][q]) : acc_g[b][q];
            store(ri, oc, v);
        }
    }
}

// All of one wave's column groups (col0 = first + g * stride, g < groups) as
// one continuous software pipeline when the expert has at most 16 rows (the
// usual decode case) and k is a whole number of batches: the next batch's
// loads are issued before the current batch's MFMAs also across group
// boundaries, so a wave (one per SIMD here) never waits for a group's first
// batch.  Otherwise the groups run one by one (stream_columns).  Same MFMA
// sequence per output element either way.
// Weight part of batch `step` (group step / spg, K batch step % spg): the
// gate (or only) rows when G, the up rows when UP.
template <int NB, int U, int WL, bool SILU, bool G = true, bool UP = true>
__device__ __forceinline__ void load_group_weights(LayerBatch<NB, U, SILU>& t, const uint16_t* wexp, int n, int k,
                                                   long up, int first, int stride, int spg, int step) {
    constexpr int KS = WL == kWeightsFrag16 ? 16 : 1;
    const int lane = threadIdx.x & 63;
    const int g = step / spg, kb = (step - g * spg) * 32 * U;
    const int col0 = first + g * stride;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int col = col0 + b * 16 + (lane & 15);
        const uint16_t* w = WL == kWeightsFrag16 ? wexp + (long)(col < n ? col >> 4 : 0) * 16 * k + lane * 8
                                                 : wexp + (long)(col < n ? col : 0) * k + (lane >> 4) * 8;
#pragma unroll
        for (int q = 0; q < U; ++q) {
            if constexpr (G) t.g[b][q] = *(const u32x4*)(w + (kb + q * 32) * KS);
            if constexpr (SILU && UP) t.u[b][q] = *(const u32x4*)(w + up + (kb + q * 32) * KS);
        }
    }
}

// b0: the caller may have issued the gate (or only) rows of batch 0 already
// (`b0_weights`), e.g. before the rows were known.
template <int NB, int U, int WL, bool SILU, typename ARow, typename Store>
__device__ __forceinline__ void stream_wave_groups(const uint16_t* wexp, int n, int k, long up_rows, int first,
                                                   int stride, int groups, const int* list, int n_rows, ARow a_of,
                                                   Store store, LayerBatch<NB, U, SILU>& b0, bool b0_weights) {
    constexpr int KB = 32 * U;
    LayerBatch<NB, U, SILU> b1;
    if (groups <= 0 || n_rows <= 0) return;
    if (n_rows > 16 || k % KB != 0) {
        for (int g = 0; g < groups; ++g) {  // (a gate-only preload of batch 0 is simply loaded again)
            LayerBatch<NB, U, SILU> t;
            stream_columns<NB, U, WL, SILU>(wexp, n, k, up_rows, first + g * stride, list, n_rows, a_of, store, t,
                                            false);
        }
        return;
    }
    const int lane = threadIdx.x & 63;
    const bool ok = (lane & 15) < n_rows;
    const uint16_t* xs = a_of(ok ? (lane & 15) : 0) + (lane >> 4) * 8;
    const long up = up_rows * k;
    const int spg = k / KB;  // batches per group
    const int total = groups * spg;
    auto load = [&](LayerBatch<NB, U, SILU>& t, int step, bool gate_loaded) {
        if (gate_loaded) load_group_weights<NB, U, WL, SILU, false, true>(t, wexp, n, k, up, first, stride, spg, step);
        else load_group_weights<NB, U, WL, SILU>(t, wexp, n, k, up, first, stride, spg, step);
        const int kb = (step % spg) * KB;
#pragma unroll
        for (int q = 0; q < U; ++q) t.x[q] = *(const u32x4*)(xs + kb + q * 32);
    };
    f32x4 acc_g[NB], acc_u[NB];
    auto mma = [&](LayerBatch<NB, U, SILU>& t, int step) {
        const int g = step / spg;
        if (step == g * spg) {
#pragma unroll
            for (int b = 0; b < NB; ++b)
#pragma unroll
                for (int q = 0; q < 4; ++q) acc_g[b][q] = acc_u[b][q] = 0.f;
        }
#pragma unroll
        for (int q = 0; q < U; ++q) {
            u32x4 xv = t.x[q];
            if (!ok) xv = u32x4{0u, 0u, 0u, 0u};
            const bf16x8 xb = as_bf16x8_l(xv);
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                acc_g[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8_l(t.g[b][q]), xb, acc_g[b], 0, 0, 0);
                if constexpr (SILU)
                    acc_u[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8_l(t.u[b][q]), xb, acc_u[b], 0, 0, 0);
            }
        }
        if (step == (g + 1) * spg - 1 && ok) {  // the group's last batch: epilogue
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int oc = first + g * stride + b * 16 + (lane >> 4) * 4;
                float v[4];
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    v[q] = SILU ? silu(round_bf16(acc_g[b][q])) * round_bf16(acc_u[b][q]) : acc_g[b][q];
                store(lane & 15, oc, v);
            }
        }
    };
    load(b0, 0, b0_weights);
    for (int step = 0; step < total; step += 2) {
        if (step + 1 < total) load(b1, step + 1, false);
        mma(b0, step);
        if (step + 2 < total) load(b0, step + 2, false);
        if (step + 1 < total) mma(b1, step + 1);
    }
}

// Byte offset of the activated rows in LDS (after the count, list, weights
// and routes), 16-byte aligned; the layout is spelled out in the kernel.
__host__ __device__ inline size_t layer_act_offset(int T, int K) {
    const size_t head = 4 * sizeof(int) + kLayerMaxTokens * (sizeof(int) + sizeof(float)) +
                        kLayerMaxExperts * sizeof(int) + (size_t)T * 2 * K * sizeof(float);
    return (head + 15) / 16 * 16;
}

// NBG/UG: gate_up column blocks per wave and K batch depth; NBD/UD: down's.
template <int EP, typename LT, int NBG, int UG, int NBD, int UD, int WL>
__global__ __launch_bounds__(kLayerThreads) void decode_layer_kernel(DecodeLayerArgs p, DispatchArgs plan) {
    extern __shared__ __attribute__((aligned(16))) unsigned char layer_lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int items = p.E * p.splits;
    const int per_xcd = (items + kXcds - 1) / kXcds;
    const int item = xcd_remap(blockIdx.x, per_xcd);  // the splits of an expert share an XCD
    if (item < 0 || item >= items) return;
    const int e = item / p.splits, s = item - e * p.splits;
    if (p.receipt && item == 0 && tid == 0) {
        p.receipt[0] = 16; p.receipt[1] = 32 * NBG; p.receipt[2] = 32 * UG; p.receipt[3] = kLayerWaves;
        p.receipt[4] = 1;
        p.receipt[5] = 16; p.receipt[6] = 16 * NBD; p.receipt[7] = 32 * UD; p.receipt[8] = kLayerWaves;
        p.receipt[9] = 1;
    }
    const int T = p.tokens, K = p.K, I = p.I, H = p.H;
    // LDS: [0] row count, [1] rejected-row flag, [2] padded offset of e,
    // [3] padded total; row list [64]; route weights [64]; per-expert counts
    // [256]; routes [T][2K] f32; activated [T][I] bf16 (16-byte aligned).
    int* n_rows_lds = (int*)layer_lds;
    int* list = n_rows_lds + 4;
    float* wts = (float*)(list + kLayerMaxTokens);
    int* counts = (int*)(wts + kLayerMaxTokens);
    float* routes = (float*)(counts + kLayerMaxExperts);
    uint16_t* act = (uint16_t*)(layer_lds + layer_act_offset(T, K));

    const uint16_t* wgu = p.gate_up + (long)e * 2 * I * H;
    const uint16_t* wdn = p.down + (long)e * H * I;
    const int ng_gu = (I + 16 * NBG - 1) / (16 * NBG);  // gate_up column groups, dealt to waves in turn
    const int cols_dn = H / p.splits;                    // this split's down columns
    const int ng_dn = (cols_dn + 16 * NBD - 1) / (16 * NBD);

    // The gate rows of this wave's first gate_up batch are requested before
    // routing, whose latency they then overlap.
    // (The launcher requires H to be a whole number of batches, so batch 0
    // exists; a wave without groups loads column 0's rows and drops them.)
    const int groups_gu = wave < ng_gu ? (ng_gu - wave + kLayerWaves - 1) / kLayerWaves : 0;
    LayerBatch<NBG, UG, true> bg;  // gate rows only: the up rows would not fit in registers beside routing
    load_group_weights<NBG, UG, WL, true, true, false>(bg, wgu, I, H, (long)I * H, wave * 16 * NBG,
                                                       kLayerWaves * 16 * NBG, H / (32 * UG), 0);
    // Route every token (four per wave per pass) into LDS.
    for (int i = tid; i < kLayerMaxExperts; i += kLayerThreads) counts[i] = 0;
    if (tid == 0) n_rows_lds[1] = 0;
    for (int t0 = 0; t0 < T; t0 += kLayerThreads / 16) {
        const int t = t0 + (tid >> 4);
        if (route_row<EP, LT>((const LT*)p.logits, t, t < T, routes, p.E, K, nullptr, p.normalize != 0) &&
            t < T)
            n_rows_lds[1] = 1;  // a rejected row (non-finite logits): the plan is invalid
    }
    __syncthreads();
    // The dispatch plan (what dispatch_single_body builds for the two-launch
    // path): every workgroup counts all assignments; split 0 of each expert
    // writes that expert's counts, offset, slots and tiles, item 0 the
    // routes, the status and padded total and the tail past the total.
    const int A = T * K;
    for (int a = tid; a < A; a += kLayerThreads) {
        const float id = routes[(a / K) * 2 * K + a % K];
        if (id == id) atomicAdd(&counts[(int)id], 1);  // NaN ids (rejected rows) count nowhere
    }
    __syncthreads();
    if (wave == 0) {  // padded exclusive offset of e and the padded total
        int before = 0, total = 0;
        for (int x = lane; x < p.E; x += 64) {
            const int pad = (counts[x] + 15) / 16 * 16;
            before += x < e ? pad : 0;
            total += pad;
        }
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) {
            before += __shfl_xor(before, d, 64);
            total += __shfl_xor(total, d, 64);
        }
        if (lane == 0) {
            n_rows_lds[2] = before;
            n_rows_lds[3] = total;
        }
    }
    // This expert's assignments in ascending order (the plan's stable order)
    // and their route weights; a rejected row's ids are NaN and match nothing.
    if (wave == 0) {
        int n = 0;
        const float fe = (float)e;
        for (int a0 = 0; a0 < A; a0 += 64) {
            const int a = a0 + lane;
            const int t = a / K, r = a - t * K;
            const bool hit = a < A && routes[t * 2 * K + r] == fe;
            const uint64_t m = __ballot(hit);
            const int rank = n + __popcll(m & lanemask_lt());
            if (hit && rank < kLayerMaxTokens) {
                list[rank] = a;
                wts[rank] = routes[t * 2 * K + K + r];
            }
            n += __popcll(m);
        }
        if (lane == 0) n_rows_lds[0] = n < kLayerMaxTokens ? n : kLayerMaxTokens;
    }
    __syncthreads();
    const int n_rows = n_rows_lds[0];
    if (s == 0) {
        const int off = n_rows_lds[2], cnt = counts[e], end = off + (cnt + 15) / 16 * 16;
        if (tid == 0) {
            plan.meta[e] = cnt;
            plan.meta[p.E + e] = cnt;
            plan.offsets[e] = off;
        }
        for (int r = tid; r < end - off; r += kLayerThreads) plan.slots[off + r] = r < cnt ? list[r] : A;
        for (int b = tid; b < (end - off) / 16; b += kLayerThreads) plan.tiles[off / 16 + b] = e;
    }
    if (item == 0) {
        const int total = n_rows_lds[3];
        if (tid == 0) {
            plan.offsets[p.E] = total;
            plan.meta[2 * p.E] = n_rows_lds[1];
            plan.meta[2 * p.E + 1] = total;
        }
        for (int i = tid; i < T * 2 * K; i += kLayerThreads) plan.routes[i] = routes[i];
        for (int b = total / 16 + tid; b < plan.capacity / 16; b += kLayerThreads) plan.tiles[b] = -1;
        for (int r = total + tid; r < plan.capacity; r += kLayerThreads) plan.slots[r] = A;
    }

    // gate_up + SiLU·mul into LDS (and, for split 0, the API's activated rows).
    const bool write_global = s == 0;
    {
        auto a_of = [&](int ri) -> const uint16_t* { return p.x + (long)(list[ri] / K) * H; };
        auto store = [&](int ri, int oc, const float* v) {
            u32x2 pk;
            pk[0] = pack_bf16x2(v[0], v[1]);
            pk[1] = pack_bf16x2(v[2], v[3]);
            if (oc + 3 < I) {
                *(u32x2*)(act + (long)ri * I + oc) = pk;
                if (write_global) *(u32x2*)(p.activated + (long)list[ri] * I + oc) = pk;
            }
        };
        stream_wave_groups<NBG, UG, WL, true>(wgu, I, H, I, wave * 16 * NBG, kLayerWaves * 16 * NBG, groups_gu,
                                              list, n_rows, a_of, store, bg, true);
    }
    __syncthreads();

    // down + route weight from the LDS rows, this split's columns.
    {
        auto a_of = [&](int ri) -> const uint16_t* { return act + (long)ri * I; };
        auto store = [&](int ri, int oc, const float* v) {
            const float w = wts[ri];
            u32x2 pk;
            pk[0] = pack_bf16x2(v[0] * w, v[1] * w);
            pk[1] = pack_bf16x2(v[2] * w, v[3] * w);
            if (oc + 3 < H) *(u32x2*)(p.contributions + (long)list[ri] * H + oc) = pk;
        };
        const int groups = wave < ng_dn ? (ng_dn - wave + kLayerWaves - 1) / kLayerWaves : 0;
        LayerBatch<NBD, UD, false> bd;
        stream_wave_groups<NBD, UD, WL, false>(wdn, H, I, 0, s * cols_dn + wave * 16 * NBD, kLayerWaves * 16 * NBD,
                                               groups, list, n_rows, a_of, store, bd, false);
    }
}

template <int EP, typename LT, int WL>
int launch_layer_ep(const DecodeLayerArgs& a, const DispatchArgs& plan, int grid, size_t lds, hipStream_t s) {
    if constexpr (WL == kWeightsFrag16) {
        if (a.I < 1024)
            decode_layer_kernel<EP, LT, 2, 8, 4, 4, WL><<<grid, kLayerThreads, lds, s>>>(a, plan);
        else
            decode_layer_kernel<EP, LT, 2, 8, 2, 8, WL><<<grid, kLayerThreads, lds, s>>>(a, plan);
    } else {
        decode_layer_kernel<EP, LT, 1, 4, 4, 4, WL><<<grid, kLayerThreads, lds, s>>>(a, plan);
    }
    return (int)hipGetLastError();
}

template <typename LT, int WL>
int launch_layer_lt(const DecodeLayerArgs& a, const DispatchArgs& plan, int grid, size_t lds, hipStream_t s) {
    const int ep = (a.E + 15) / 16;
    if (ep <= 1) return launch_layer_ep<1, LT, WL>(a, plan, grid, lds, s);
    if (ep <= 2) return launch_layer_ep<2, LT, WL>(a, plan, grid, lds, s);
    if (ep <= 4) return launch_layer_ep<4, LT, WL>(a, plan, grid, lds, s);
    if (ep <= 8) return launch_layer_ep<8, LT, WL>(a, plan, grid, lds, s);
    return launch_layer_ep<16, LT, WL>(a, plan, grid, lds, s);
}

}  // namespace

// The one-launch decode layer when it applies (routing from logits, E <= 256,
// T <= 64, the activated rows of T tokens in LDS), else kNotApplicable.
int launch_decode_layer(const void* input, const void* logits, int logits_dtype, const void* gate_up,
                        const void* down, float* routes, int* meta, int* offsets, int* slots, int* tiles,
                        void* activated, void* contributions, int tokens, int hidden, int intermediate, int experts,
                        int top_k, int capacity, int weight_layout, int* receipts, hipStream_t s) {
    if (!logits || tokens > kLayerMaxTokens || experts > 256 || top_k > 32) return kNotApplicable;
    // Splits per expert: about one workgroup per CU, each split's down
    // columns a whole number of 64-column groups.  Every split recomputes its
    // expert's whole gate_up (from L2 after the first), so splits stop at 4
    // (with fewer than 64 experts the grid then leaves CUs idle; the benchmark
    // layers have 128).
    int splits = 1;
    while (splits < 4 && experts * splits * 2 <= 256 && hidden % (64 * splits * 2) == 0) splits *= 2;
    const size_t lds = layer_act_offset(tokens, top_k) + (size_t)tokens * intermediate * 2;
    // Whole K batches for both projections (256 = the widest batch, 8 x 32).
    if (lds > 150 * 1024 || hidden % 256 || intermediate % 256) return kNotApplicable;

    DecodeLayerArgs a{};
    a.logits = logits;
    a.logits_bf16 = logits_dtype & 1;
    a.normalize = !(logits_dtype & TAU_MOE_ROUTE_RAW_WEIGHTS);
    a.x = (const uint16_t*)input;
    a.gate_up = (const uint16_t*)gate_up;
    a.down = (const uint16_t*)down;
    a.activated = (uint16_t*)activated;
    a.contributions = (uint16_t*)contributions;
    a.tokens = tokens;
    a.K = top_k;
    a.E = experts;
    a.H = hidden;
    a.I = intermediate;
    a.splits = splits;
    a.receipt = receipts;
    DispatchArgs plan{};
    plan.logits = logits;
    plan.logits_bf16 = a.logits_bf16;
    plan.normalize = a.normalize;
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
    const int items = experts * splits;
    const int grid = (items + kXcds - 1) / kXcds * kXcds;
    const bool bf = a.logits_bf16;
    if (weight_layout == kWeightsFrag16)
        return bf ? launch_layer_lt<uint16_t, kWeightsFrag16>(a, plan, grid, lds, s)
                  : launch_layer_lt<float, kWeightsFrag16>(a, plan, grid, lds, s);
    return bf ? launch_layer_lt<uint16_t, kWeightsRowMajor>(a, plan, grid, lds, s)
              : launch_layer_lt<float, kWeightsRowMajor>(a, plan, grid, lds, s);
}

#endif  // TAU_DECODE_ONE_LAUNCH

}  // namespace tau_amd
