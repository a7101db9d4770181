// Grouped expert GEMMs for the MoE path on CDNA4 (gfx950).
//
// Both projections compute out[row, n] = sum_k A[row, k] * W[e][n, k] with A
// and W K-contiguous ("NT"), BF16 operands and FP32 accumulators, over the
// expert-major row blocks produced by dispatch (tiles[m] = expert of the
// m-th M-row block).  The reference's grouped kernel and epilogues are
// crates/cuda-kernels/src/kernels/moe_gemm.cu:63-138 and
// linear_bf16_fp32.cu:47-98; the numerical contract kept here is:
//   gate_up : gu = bf16(acc), a = bf16(silu(g) * u)   (fused, no [cap,2I] pass)
//   down    : c[slot] = bf16(acc * w[slot])           (weight before the round)
//
// Two kernel families:
//  * lds_gemm   -- prefill.  BM x BN x 64 block tile, 4 waves, each wave a grid
//                  of 32x32x16 MFMAs; A/B panels staged through a double-
//                  buffered LDS (row stride 72 BF16 to spread banks) with the
//                  next K panel prefetched into registers during the MFMAs.
//                  Gate_up B panels hold BN/2 gate rows then the matching
//                  BN/2 up rows, so each lane owns (g, u) pairs for SiLU.
//  * stream_gemm -- decode / small groups.  One wave per (16-row block,
//                  16 output columns): expert weights are streamed from HBM
//                  straight into 16x16x32 MFMA A-operands with 128-bit loads
//                  (no LDS), several K steps in flight per wave.
// Work items are mapped XCD-major (consecutive items on one XCD's L2) and the
// number of live M blocks is read on the device from the dispatch metadata,
// so no host readback is needed and dead capacity costs one early exit.
#include "kernels.hpp"
#include "mfma_copy_plan.hpp"

#include <type_traits>

namespace tau_amd {

namespace {

template <bool Aligned>
__device__ __forceinline__ u32x4 load_chunk(const uint16_t* row, int k, int K, bool valid) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (!valid) return v;
    if constexpr (Aligned) {
        if (k < K) v = *(const u32x4*)(row + k);
    } else {
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
            uint32_t lo = k + j < K ? row[k + j] : 0u;
            uint32_t hi = k + j + 1 < K ? row[k + j + 1] : 0u;
            v[j / 2] = lo | (hi << 16);
        }
    }
    return v;
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ int live_blocks(const GemmArgs& p, int bm) {
    const int cap_blocks = (p.rows + bm - 1) / bm;
    if (!p.meta_total) return cap_blocks;
    const int used = (p.meta_total[0] + bm - 1) / bm;
    return used < cap_blocks ? used : cap_blocks;
}

// ---------------------------------------------------------------------------
// LDS-tiled MFMA kernel (prefill)
// ---------------------------------------------------------------------------
constexpr int kBK = 64;
constexpr int kLdsStride = kBK + 8;  // BF16 elements per staged row

template <int BM, int BN, int WM, int WN, int AM, int EPI, bool Aligned>
__global__ __launch_bounds__(64 * WM * WN) void lds_gemm(GemmArgs p) {
    constexpr int NT = 64 * WM * WN;
    constexpr int TM = BM / WM, TN = BN / WN;  // wave tile
    constexpr int MI = TM / 32, NI = TN / 32;   // 32x32 MFMA blocks per wave
    static_assert(MI >= 1 && NI >= 1, "wave tile too small");
    static_assert(EPI != kEpiSilu || NI % 2 == 0, "SiLU pairs gate/up blocks");
    constexpr int ACH = BM * (kBK / 8) / NT;     // 16-byte chunks per thread
    constexpr int BCH = BN * (kBK / 8) / NT;
    static_assert(ACH * NT == BM * kBK / 8 && BCH * NT == BN * kBK / 8, "tile/threads mismatch");
    constexpr int NOUT = EPI == kEpiSilu ? BN / 2 : BN;  // output columns per block

    __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * kLdsStride];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * kLdsStride];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    if (p.receipt && blockIdx.x == 0 && tid == 0) {
        p.receipt[0] = BM; p.receipt[1] = BN; p.receipt[2] = kBK; p.receipt[3] = WM * WN; p.receipt[4] = 2;
    }
    const int n_tiles = (p.n + NOUT - 1) / NOUT;
    const int live = live_blocks(p, BM);
    const int total = live * n_tiles;
    const int per_xcd = (total + kXcds - 1) / kXcds;
    const int item = xcd_remap(blockIdx.x, per_xcd);
    if (item < 0 || item >= total) return;
    const int m_tile = item / n_tiles, n_tile = item - m_tile * n_tiles;
    const int expert = p.tiles ? p.tiles[m_tile] : 0;
    const int row0 = m_tile * BM;
    const int c0 = n_tile * NOUT;

    if (expert < 0) {
        if constexpr (EPI == kEpiStoreBf16) {  // dead capacity reads as zeros
            uint16_t* out = (uint16_t*)p.out;
            for (int i = tid; i < BM * NOUT; i += NT) {
                const int r = row0 + i / NOUT, c = c0 + i % NOUT;
                if (r < p.rows && c < p.n) out[(size_t)r * p.ldo + c] = 0;
            }
        }
        return;
    }

    // Per-thread A/B chunk sources, fixed across K.
    const uint16_t* a_src[ACH];
    bool a_ok[ACH];
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
        const int c = tid + i * NT, r = c / (kBK / 8);
        const int row = row0 + r;
        bool ok = row < p.rows;
        long src_row = row;
        if constexpr (AM == kAGather) {
            const int slot = ok ? p.slots[row] : p.assignments;
            ok = slot >= 0 && slot < p.assignments;
            src_row = ok ? slot / p.topk : 0;
        }
        a_ok[i] = ok;
        a_src[i] = p.a + src_row * (long)p.lda;
    }
    const uint16_t* wexp = p.w + (long)expert * p.w_expert_stride;
    const uint16_t* b_src[BCH];
    bool b_ok[BCH];
#pragma unroll
    for (int i = 0; i < BCH; ++i) {
        const int c = tid + i * NT, r = c / (kBK / 8);
        long wrow;
        bool ok;
        if constexpr (EPI == kEpiSilu) {
            const int j = c0 + (r < BN / 2 ? r : r - BN / 2);
            ok = j < p.n;
            wrow = (r < BN / 2 ? j : j + p.w_up_offset);
        } else {
            const int j = c0 + r;
            ok = j < p.n;
            wrow = j;
        }
        b_ok[i] = ok;
        b_src[i] = wexp + (ok ? wrow : 0) * (long)p.k;
    }

    f32x16 acc[MI][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j)
#pragma unroll
            for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.f;

    u32x4 ra[ACH], rb[BCH];
    const int nk = (p.k + kBK - 1) / kBK;
    auto gload = [&](int kt) {
        const int kb = kt * kBK;
#pragma unroll
        for (int i = 0; i < ACH; ++i) {
            const int kc = ((tid + i * NT) % (kBK / 8)) * 8;
            ra[i] = load_chunk<Aligned>(a_src[i], kb + kc, p.k, a_ok[i]);
        }
#pragma unroll
        for (int i = 0; i < BCH; ++i) {
            const int kc = ((tid + i * NT) % (kBK / 8)) * 8;
            rb[i] = load_chunk<Aligned>(b_src[i], kb + kc, p.k, b_ok[i]);
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < ACH; ++i) {
            const int c = tid + i * NT;
            *(u32x4*)&As[buf][(c / (kBK / 8)) * kLdsStride + (c % (kBK / 8)) * 8] = ra[i];
        }
#pragma unroll
        for (int i = 0; i < BCH; ++i) {
            const int c = tid + i * NT;
            *(u32x4*)&Bs[buf][(c / (kBK / 8)) * kLdsStride + (c % (kBK / 8)) * 8] = rb[i];
        }
    };

    gload(0);
    sstore(0);
    __syncthreads();
    const int lrow = lane & 31, lk = (lane >> 5) * 8;
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) gload(kt + 1);
#pragma unroll
        for (int ks = 0; ks < kBK / 16; ++ks) {
            bf16x8 af[MI], bfr[NI];
#pragma unroll
            for (int i = 0; i < MI; ++i)
                af[i] = as_bf16x8(*(const u32x4*)&As[buf][(wm * TM + i * 32 + lrow) * kLdsStride + ks * 16 + lk]);
#pragma unroll
            for (int j = 0; j < NI; ++j) {
                int brow;
                if constexpr (EPI == kEpiSilu) {
                    // first NI/2 blocks: gate rows, last NI/2: matching up rows
                    const int jj = j < NI / 2 ? j : j - NI / 2;
                    brow = (j < NI / 2 ? 0 : BN / 2) + wn * (TN / 2) + jj * 32 + lrow;
                } else {
                    brow = wn * TN + j * 32 + lrow;
                }
                bfr[j] = as_bf16x8(*(const u32x4*)&Bs[buf][brow * kLdsStride + ks * 16 + lk]);
            }
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < NI; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) sstore(buf ^ 1);
        __syncthreads();
    }

    // Epilogue.  32x32 accumulator layout: value q of lane l sits at
    // row (q/4)*8 + (l/32)*4 + q%4, column l%32 of its block.
    const int lcol = lane & 31, lr4 = (lane >> 5) * 4;
#pragma unroll
    for (int i = 0; i < MI; ++i) {
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const int r = row0 + wm * TM + i * 32 + (q >> 2) * 8 + lr4 + (q & 3);
            if (r >= p.rows) continue;
            if constexpr (EPI == kEpiSilu) {
                uint16_t* out = (uint16_t*)p.out;
#pragma unroll
                for (int j = 0; j < NI / 2; ++j) {
                    const int c = c0 + wn * (TN / 2) + j * 32 + lcol;
                    if (c < p.n) {
                        const float g = round_bf16(acc[i][j][q]);
                        const float u = round_bf16(acc[i][j + NI / 2][q]);
                        out[(size_t)r * p.ldo + c] = float_to_bf16_bits(silu(g) * u);
                    }
                }
            } else if constexpr (EPI == kEpiStoreBf16) {
                uint16_t* out = (uint16_t*)p.out;
#pragma unroll
                for (int j = 0; j < NI; ++j) {
                    const int c = c0 + wn * TN + j * 32 + lcol;
                    if (c < p.n) out[(size_t)r * p.ldo + c] = float_to_bf16_bits(acc[i][j][q]);
                }
            } else if constexpr (EPI == kEpiStoreF32) {
                float* out = (float*)p.out;
#pragma unroll
                for (int j = 0; j < NI; ++j) {
                    const int c = c0 + wn * TN + j * 32 + lcol;
                    if (c < p.n) out[(size_t)r * p.ldo + c] = acc[i][j][q];
                }
            } else {  // kEpiScatterWeighted
                const int slot = p.slots[r];
                if (slot < 0 || slot >= p.assignments) continue;
                const int t = slot / p.topk, rk = slot - t * p.topk;
                const float wt = p.routes[(size_t)t * 2 * p.topk + p.topk + rk];
                uint16_t* out = (uint16_t*)p.out;
#pragma unroll
                for (int j = 0; j < NI; ++j) {
                    const int c = c0 + wn * TN + j * 32 + lcol;
                    if (c < p.n) out[(size_t)slot * p.ldo + c] = float_to_bf16_bits(acc[i][j][q] * wt);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Weight-streaming MFMA kernel (decode / small groups), 16-row blocks
// ---------------------------------------------------------------------------
constexpr int kStreamWaves = 4;
constexpr int kStreamUnroll = 4;  // K steps of 32 kept in flight per wave

template <int AM, int EPI, bool Aligned>
__global__ __launch_bounds__(64 * kStreamWaves) void stream_gemm(GemmArgs p) {
    constexpr bool kSilu = EPI == kEpiSilu;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (p.receipt && blockIdx.x == 0 && threadIdx.x == 0) {
        p.receipt[0] = 16; p.receipt[1] = kSilu ? 32 : 16; p.receipt[2] = 32 * kStreamUnroll;
        p.receipt[3] = kStreamWaves; p.receipt[4] = 1;
    }
    const int n_blocks = (p.n + 15) / 16;
    const int live = live_blocks(p, 16);
    const int total = live * n_blocks;
    const int groups = (total + kStreamWaves - 1) / kStreamWaves;  // items per WG = 4 waves
    const int per_xcd = (groups + kXcds - 1) / kXcds;
    const int group = xcd_remap(blockIdx.x, per_xcd);
    const int item = group * kStreamWaves + wave;
    if (group < 0 || group >= groups || item >= total) return;
    const int m_tile = item / n_blocks, nb = item - m_tile * n_blocks;
    const int expert = p.tiles ? p.tiles[m_tile] : 0;
    if (expert < 0) {
        if constexpr (EPI == kEpiStoreBf16) {
            uint16_t* out = (uint16_t*)p.out;
            for (int i = lane; i < 256; i += 64) {
                const int r = m_tile * 16 + i / 16, c = nb * 16 + i % 16;
                if (r < p.rows && c < p.n) out[(size_t)r * p.ldo + c] = 0;
            }
        }
        return;
    }
    const int row = m_tile * 16 + (lane & 15);
    const int kofs = (lane >> 4) * 8;
    // B operand: the 16 token rows of this block.
    bool x_ok = row < p.rows;
    long x_row = row;
    if constexpr (AM == kAGather) {
        const int slot = x_ok ? p.slots[row] : p.assignments;
        x_ok = slot >= 0 && slot < p.assignments;
        x_row = x_ok ? slot / p.topk : 0;
    }
    const uint16_t* xs = p.a + x_row * (long)p.lda;
    // A operand: 16 weight rows (output columns); gate and up for SiLU.
    const int wcol = nb * 16 + (lane & 15);
    const bool w_ok = wcol < p.n;
    const uint16_t* wexp = p.w + (long)expert * p.w_expert_stride;
    const uint16_t* wg = wexp + (long)(w_ok ? wcol : 0) * p.k;
    const uint16_t* wu = kSilu ? wg + (long)p.w_up_offset * p.k : nullptr;

    f32x4 acc_g = {0.f, 0.f, 0.f, 0.f}, acc_u = {0.f, 0.f, 0.f, 0.f};
    const int steps = (p.k + 31) / 32;
    int s = 0;
    for (; s + kStreamUnroll <= steps; s += kStreamUnroll) {
        u32x4 g[kStreamUnroll], u[kStreamUnroll], x[kStreamUnroll];
#pragma unroll
        for (int q = 0; q < kStreamUnroll; ++q) {
            const int kb = (s + q) * 32;
            g[q] = load_chunk<Aligned>(wg, kb + kofs, p.k, w_ok);
            if constexpr (kSilu) u[q] = load_chunk<Aligned>(wu, kb + kofs, p.k, w_ok);
            x[q] = load_chunk<Aligned>(xs, kb + kofs, p.k, x_ok);
        }
#pragma unroll
        for (int q = 0; q < kStreamUnroll; ++q) {
            acc_g = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(g[q]), as_bf16x8(x[q]), acc_g, 0, 0, 0);
            if constexpr (kSilu)
                acc_u = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(u[q]), as_bf16x8(x[q]), acc_u, 0, 0, 0);
        }
    }
    for (; s < steps; ++s) {
        const int kb = s * 32;
        const u32x4 g = load_chunk<Aligned>(wg, kb + kofs, p.k, w_ok);
        const u32x4 x = load_chunk<Aligned>(xs, kb + kofs, p.k, x_ok);
        acc_g = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(g), as_bf16x8(x), acc_g, 0, 0, 0);
        if constexpr (kSilu) {
            const u32x4 u = load_chunk<Aligned>(wu, kb + kofs, p.k, w_ok);
            acc_u = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(u), as_bf16x8(x), acc_u, 0, 0, 0);
        }
    }

    // 16x16 accumulator: value q of lane l is output column (l/16)*4 + q of the
    // block (A rows) for token row l%16 (B columns).
    const int orow = m_tile * 16 + (lane & 15);
    if (orow >= p.rows) return;
    const int oc = nb * 16 + (lane >> 4) * 4;
    float v[4];
    long out_row = orow;
    if constexpr (EPI == kEpiSilu) {
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = silu(round_bf16(acc_g[q])) * round_bf16(acc_u[q]);
    } else if constexpr (EPI == kEpiScatterWeighted) {
        const int slot = p.slots[orow];
        if (slot < 0 || slot >= p.assignments) return;
        const int t = slot / p.topk, rk = slot - t * p.topk;
        const float wt = p.routes[(size_t)t * 2 * p.topk + p.topk + rk];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = acc_g[q] * wt;
        out_row = slot;
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = acc_g[q];
    }
    if constexpr (EPI == kEpiStoreF32) {
        float* out = (float*)p.out + out_row * (long)p.ldo;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (oc + q < p.n) out[oc + q] = v[q];
    } else {
        uint16_t* out = (uint16_t*)p.out + out_row * (long)p.ldo;
        if (oc + 3 < p.n && (p.ldo % 4) == 0) {
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

// -DTAU_SPLIT_ROWS=32|64|128: 256-row dispatch blocks with at most that many
// live rows run in a second launch on the weight-streaming kernel (two 16-row
// groups), the 64x256 or the 128x128 MFMA tile (default off).
#ifdef TAU_SPLIT_ROWS
constexpr int kSplitRows = TAU_SPLIT_ROWS;
static_assert(kSplitRows == 32 || kSplitRows == 64 || kSplitRows == 128, "TAU_SPLIT_ROWS is 32, 64 or 128");
#else
constexpr int kSplitRows = 0;
#endif

// With -DTAU_M256_BIG_WAVES the 128x128 wave tiles skip the MFMAs of their
// 32-row fragments that hold only padding (-DTAU_BIG_WAVE_NO_SKIP keeps
// every MFMA, for comparison).
#ifdef TAU_BIG_WAVE_NO_SKIP
constexpr bool kBigWaveSkip = false;
#else
constexpr bool kBigWaveSkip = true;
#endif
// -DTAU_FRAG_SKIP: the shipped 256-row tile (64x64 wave tiles) skips padding
// per 32-row fragment instead of per wave (off by default).
#ifdef TAU_FRAG_SKIP
constexpr bool kFragSkip = true;
#else
constexpr bool kFragSkip = false;
#endif

// Pipelined weight-streaming kernel for 16-byte-aligned operands.  Each wave
// owns NB 16-column blocks (gate and up blocks for SiLU) of one 16-row block;
// loads carry no branches (invalid rows are clamped to a valid address and
// zeroed afterwards) and batches of U K-steps are double-buffered, so one
// batch is in flight while the previous one feeds the MFMAs.
template <int NB, int U, int RT>
struct StreamBatch {
    u32x4 x[RT][U];
    u32x4 g[NB][U];
    u32x4 u[NB][U];
};

// RT 16-row token groups share every weight fragment (rows per item = 16*RT).
template <int AM, int EPI, int NB, int U, int W, int RT, int WL = kWeightsRowMajor>
__global__ __launch_bounds__(64 * W) void stream_gemm_fast(GemmArgs p) {
    constexpr bool kSilu = EPI == kEpiSilu;
    constexpr int R = 16 * RT;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (p.receipt && blockIdx.x == 0 && threadIdx.x == 0) {
        p.receipt[0] = R; p.receipt[1] = 16 * NB * (kSilu ? 2 : 1); p.receipt[2] = 32 * U;
        p.receipt[3] = W; p.receipt[4] = 2;
    }
    const int n_groups = (p.n + 16 * NB - 1) / (16 * NB);
    // Small-block split (32 rows): the dispatch blocks are block_stride rows
    // apart and this kernel takes the blocks with at most R live rows.
    constexpr bool kStrided = kSplitRows == R;
    const int stride = kStrided && p.block_stride ? p.block_stride : R;
    const int live = live_blocks(p, stride);
    const int total = live * n_groups;
    const int groups = (total + W - 1) / W;
    const int per_xcd = (groups + kXcds - 1) / kXcds;
    const int group = xcd_remap(blockIdx.x, per_xcd);
    const int item = group * W + wave;
    if (group < 0 || group >= groups || item >= total) return;
    const int m_tile = item / n_groups, ng = item - m_tile * n_groups;
    const int row0 = m_tile * stride;
    if (kStrided && p.split_rows > 0) {
        // Padding is a suffix of an expert's block: the block has more than R
        // live rows iff row row0 + R holds an assignment (the MFMA tile's).
        const int probe = row0 + R;
        if (probe < p.rows && probe < row0 + stride && p.slots[probe] >= 0 && p.slots[probe] < p.assignments)
            return;
    }
    const int expert = p.tiles ? p.tiles[m_tile] : 0;
    if (expert < 0) {
        if constexpr (EPI == kEpiStoreBf16) {
            uint16_t* out = (uint16_t*)p.out;
            for (int i = lane; i < stride * 16 * NB; i += 64) {
                const int r = row0 + i / (16 * NB), c = ng * 16 * NB + i % (16 * NB);
                if (r < p.rows && c < p.n) out[(size_t)r * p.ldo + c] = 0;
            }
        }
        return;
    }
    if constexpr (kStrided && EPI != kEpiScatterWeighted) {
        // The block's rows past R are padding: zeros, as in the MFMA tile.
        uint16_t* out = (uint16_t*)p.out;
        for (int i = lane; i < (stride - R) * 16 * NB; i += 64) {
            const int r = row0 + R + i / (16 * NB), c = ng * 16 * NB + i % (16 * NB);
            if (r < p.rows && c < p.n) out[(size_t)r * p.ldo + c] = 0;
        }
    }
    const int kofs = (lane >> 4) * 8;
    bool x_ok[RT];
    const uint16_t* xs[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const int row = row0 + rt * 16 + (lane & 15);
        bool ok = row < p.rows;
        long x_row = ok ? row : 0;
        if constexpr (AM == kAGather) {
            const int slot = ok ? p.slots[row] : p.assignments;
            ok = slot >= 0 && slot < p.assignments;
            x_row = ok ? slot / p.topk : 0;
        }
        x_ok[rt] = ok;
        xs[rt] = p.a + x_row * (long)p.lda + kofs;
    }
    const uint16_t* wexp = p.w + (long)expert * p.w_expert_stride;
    const uint16_t* wg[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int col = ng * 16 * NB + b * 16 + (lane & 15);
        if constexpr (WL == kWeightsFrag16)  // 1 KB fragment per 32-wide K chunk, lanes in MFMA order
            wg[b] = wexp + (long)(col < p.n ? col >> 4 : 0) * 16 * p.k + lane * 8;
        else
            wg[b] = wexp + (long)(col < p.n ? col : 0) * p.k + kofs;
    }
    constexpr int KS = WL == kWeightsFrag16 ? 16 : 1;  // weight elements per unit of k
    const long up = (long)p.w_up_offset * p.k;

    f32x4 acc_g[NB][RT], acc_u[NB][RT];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int q = 0; q < 4; ++q) acc_g[b][rt][q] = acc_u[b][rt][q] = 0.f;

    auto load = [&](StreamBatch<NB, U, RT>& t, int kb) {
#pragma unroll
        for (int q = 0; q < U; ++q) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                t.g[b][q] = *(const u32x4*)(wg[b] + (kb + q * 32) * KS);
                if constexpr (kSilu) t.u[b][q] = *(const u32x4*)(wg[b] + up + (kb + q * 32) * KS);
            }
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) t.x[rt][q] = *(const u32x4*)(xs[rt] + kb + q * 32);
        }
    };
    auto mma = [&](StreamBatch<NB, U, RT>& t) {
#pragma unroll
        for (int q = 0; q < U; ++q) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                u32x4 xv = t.x[rt][q];
                if (!x_ok[rt]) xv = u32x4{0u, 0u, 0u, 0u};
                const bf16x8 xb = as_bf16x8(xv);
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    acc_g[b][rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(t.g[b][q]), xb, acc_g[b][rt], 0, 0, 0);
                    if constexpr (kSilu)
                        acc_u[b][rt] =
                            __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(t.u[b][q]), xb, acc_u[b][rt], 0, 0, 0);
                }
            }
        }
    };

    constexpr int KB = 32 * U;
    const int main_k = p.k / KB * KB;
    StreamBatch<NB, U, RT> b0, b1;
    int kb = 0;
    if (main_k > 0) {
        load(b0, 0);
        for (; kb + 2 * KB <= main_k; kb += 2 * KB) {
            load(b1, kb + KB);
            mma(b0);
            if (kb + 2 * KB < main_k) load(b0, kb + 2 * KB);
            mma(b1);
        }
        if (kb < main_k) {  // one batch left (already loaded into b0)
            mma(b0);
            kb += KB;
        }
    }
    // Tail (K not a multiple of 32*U): 8-element chunks, masked.
    for (; kb < p.k; kb += 32) {
        const bool in = kb + kofs < p.k;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            u32x4 xv = {0u, 0u, 0u, 0u};
            if (in && x_ok[rt]) xv = *(const u32x4*)(xs[rt] + kb);
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                u32x4 gv = {0u, 0u, 0u, 0u}, uv = {0u, 0u, 0u, 0u};
                if (in) {
                    gv = *(const u32x4*)(wg[b] + kb * KS);
                    if constexpr (kSilu) uv = *(const u32x4*)(wg[b] + up + kb * KS);
                }
                acc_g[b][rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(gv), as_bf16x8(xv), acc_g[b][rt], 0, 0, 0);
                if constexpr (kSilu)
                    acc_u[b][rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(uv), as_bf16x8(xv), acc_u[b][rt], 0, 0, 0);
            }
        }
    }

    // 16x16 accumulator: value q of lane l is column (l/16)*4 + q of the block,
    // token row l%16 of its group.
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const int orow = row0 + rt * 16 + (lane & 15);
        if (orow >= p.rows) continue;
        long out_row = orow;
        float wt = 1.0f;
        if constexpr (EPI == kEpiScatterWeighted) {
            const int slot = p.slots[orow];
            if (slot < 0 || slot >= p.assignments) continue;
            const int t = slot / p.topk, rk = slot - t * p.topk;
            wt = p.routes[(size_t)t * 2 * p.topk + p.topk + rk];
            out_row = slot;
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int oc = ng * 16 * NB + b * 16 + (lane >> 4) * 4;
            float v[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if constexpr (EPI == kEpiSilu)
                    v[q] = silu(round_bf16(acc_g[b][rt][q])) * round_bf16(acc_u[b][rt][q]);
                else if constexpr (EPI == kEpiScatterWeighted) v[q] = acc_g[b][rt][q] * wt;
                else v[q] = acc_g[b][rt][q];
            }
            if constexpr (EPI == kEpiStoreF32) {
                float* out = (float*)p.out + out_row * (long)p.ldo;
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    if (oc + q < p.n) out[oc + q] = v[q];
            } else {
                uint16_t* out = (uint16_t*)p.out + out_row * (long)p.ldo;
                if (oc + 3 < p.n && (p.ldo % 4) == 0) {
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
}

// ---------------------------------------------------------------------------
// Direct-to-LDS pipelined MFMA kernel (prefill, K a multiple of 64)
// ---------------------------------------------------------------------------
// Block tile BM x BN x 64; WM x WN waves, each owning a (BM/WM) x (BN/WN) grid
// of 32x32x16 MFMAs.  Operand panels move HBM -> LDS with direct-to-LDS loads
// (16 bytes per lane, no VGPR staging) into STAGES ring buffers.  A rows (and
// row-major weight rows) are 128 bytes with the 16-byte chunk index XOR-
// swizzled (swz below), so fragment reads spread over all banks; frag16
// weights are staged as whole 1 KB fragments, whose 16-lane read phases are
// 256 contiguous bytes.
// One barrier per K step: waiting on the oldest stage's loads, the barrier,
// then the next loads into the stage every wave has just finished with.
// The epilogue stages the BF16 tile in LDS and writes 16-byte row segments,
// scattered by slot for the down projection.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// One 16-byte-per-lane global -> LDS copy; the wave's 64 lanes fill 1 KB of
// LDS from `lds` on.  Issued as inline assembly so that the compiler's
// wait-count insertion does not track it: the builtin form makes every later
// LDS read wait for all outstanding copies (vmcnt(0)), including the ones for
// the stage after next, which serialises loads with MFMAs.  Completion is
// awaited explicitly with wait_vmcnt before the barrier that publishes a stage.
__device__ __forceinline__ void lds_dma16(const uint16_t* src, uint16_t* lds) {
    typedef __attribute__((address_space(3))) uint16_t* lds_u16;
    const uint32_t base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_u16)lds);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(base) : "memory", "m0");
}
// (hipcc warns that m0 is a reserved register in the clobber list.  These
// kernels have no m0 access of the compiler's own: in the generated code of
// grouped_gemm.hip every m0 write and read is inside these asm statements.)

// The same copy addressed as a wave-uniform 64-bit base (SGPR pair) plus a
// 32-bit per-lane byte offset: one VGPR per copy stream instead of two, and
// the K advance moves only the scalar base.  Used by the 128x128 wave tiles,
// whose 256 accumulators leave no room for 64-bit per-lane addresses.
__device__ __forceinline__ void lds_dma16_off(const uint16_t* base, uint32_t off_bytes, uint16_t* lds) {
    typedef __attribute__((address_space(3))) uint16_t* lds_u16;
    const uint32_t lbase = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_u16)lds);
    const uint64_t g = (uint64_t)(uintptr_t)base;
    // readfirstlane returns int: the words go back through uint32_t.
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane(address_hi(g));
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane(address_lo(g));
    const uint64_t gs = join_address(hi, lo);
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off_bytes), "s"(gs), "s"(lbase)
                 : "memory", "m0");
}

// Workgroup barrier without the memory fence of __syncthreads (which waits
// for every outstanding global load, in-flight LDS copies included).  Callers
// order LDS themselves: copies by wait_vmcnt, fragment reads are consumed by
// MFMAs (lgkmcnt) before the barrier that lets a stage be overwritten.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }


// IG >= 0 asks the compiler's instruction-group scheduler for strategy IG
// (__builtin_amdgcn_iglp_opt) in the K loop; 1 interleaves the fragment reads
// with the MFMAs of a single wave and was measured faster for the 256x256 and
// 128x128 tiles.
template <int BM, int BN, int WM, int WN, int STAGES, int AM, int EPI, int BK = 64, int WL = kWeightsRowMajor,
          int IG = -1>
__global__ __launch_bounds__(64 * WM * WN) void mfma_gemm(GemmArgs p) {
    constexpr int NT = 64 * WM * WN;
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int MI = TM / 32, NI = TN / 32;
    static_assert(MI >= 1 && NI >= 1, "wave tile too small");
    // 128x128 wave tiles (256 accumulators, kept in AGPRs): operands are
    // copied with 32-bit offsets from scalar bases and padding waves do not
    // leave the K loop early, so the accumulators stay put across it.
    constexpr bool kBigWave = TM * TN >= 128 * 128;
    static_assert(EPI != kEpiSilu || NI % 2 == 0, "SiLU pairs gate/up blocks");
    static_assert(EPI != kEpiStoreF32, "f32 outputs use lds_gemm");
    constexpr int CPR = BK / 8;                          // 16-byte chunks per staged row
    constexpr int RPI = 64 / CPR;                        // rows filled by one wave instruction
    constexpr int ACH = BM * CPR / NT, BCH = BN * CPR / NT;  // 16-byte chunks per thread per stage
    static_assert(ACH * NT == BM * CPR && BCH * NT == BN * CPR, "tile/threads mismatch");
    constexpr int L = ACH + BCH;                         // loads per thread per stage
    constexpr int NOUT = EPI == kEpiSilu ? BN / 2 : BN;
    constexpr int STAGE_ELEMS = (BM + BN) * BK;
    constexpr int CSTRIDE = NOUT + 8;                    // epilogue tile row stride (elements)
    constexpr int SMEM_ELEMS = STAGES * STAGE_ELEMS > BM * CSTRIDE ? STAGES * STAGE_ELEMS : BM * CSTRIDE;
    __shared__ __attribute__((aligned(1024))) uint16_t smem[SMEM_ELEMS];
    __shared__ long row_src[BM];   // gather: source row of A; down: destination slot (or -1)
    __shared__ float row_w[BM];    // down: route weight

    const int tid = threadIdx.x, lane = tid & 63;
    // Wave-uniform for the big wave tiles, which keeps the LDS stage addresses scalar.
    const int wave = kBigWave ? __builtin_amdgcn_readfirstlane(tid >> 6) : tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    if (p.receipt && blockIdx.x == 0 && tid == 0) {
        p.receipt[0] = BM; p.receipt[1] = BN; p.receipt[2] = BK; p.receipt[3] = WM * WN; p.receipt[4] = STAGES;
    }
    const int n_tiles = (p.n + NOUT - 1) / NOUT;
    // Rows between dispatch blocks: a kernel shorter than 256 rows may run the
    // small blocks of a 256-row dispatch (small-block split).
    constexpr bool kStrided = kSplitRows > 0 && BM < 256;
    const int stride = kStrided && p.block_stride ? p.block_stride : BM;
    const int live = live_blocks(p, stride);
    const int total = live * n_tiles;
    const int per_xcd = (total + kXcds - 1) / kXcds;
    const int item = xcd_remap(blockIdx.x, per_xcd);
    if (item < 0 || item >= total) return;
    const int m_tile = item / n_tiles, n_tile = item - m_tile * n_tiles;
    const int expert = p.tiles ? p.tiles[m_tile] : 0;
    const int row0 = m_tile * stride;
    const int c0 = n_tile * NOUT;
    if (kSplitRows > 0 && p.split_rows > 0) {
        // Padding is a suffix of an expert's block: the block has more than
        // split_rows live rows iff row row0 + split_rows holds an assignment.
        const int probe = row0 + p.split_rows;
        const bool big = probe < p.rows && probe < row0 + stride && p.slots[probe] >= 0 &&
                         p.slots[probe] < p.assignments;
        if (BM > p.split_rows ? !big : big) return;  // dead capacity goes to the shorter tile
    }
    if (expert < 0) {
        if constexpr (EPI == kEpiStoreBf16) {  // dead capacity reads as zeros
            uint16_t* out = (uint16_t*)p.out;
            for (int i = tid; i < stride * NOUT; i += NT) {
                const int r = row0 + i / NOUT, c = c0 + i % NOUT;
                if (r < p.rows && c < p.n) out[(size_t)r * p.ldo + c] = 0;
            }
        }
        return;
    }

    // Row table: A source rows (gather), destination slots and weights (down).
    for (int r = tid; r < BM; r += NT) {
        const int row = row0 + r;
        long src = -1;
        float w = 0.f;
        if (row < p.rows) {
            if constexpr (AM == kAGather || EPI == kEpiScatterWeighted) {
                const int slot = p.slots[row];
                if (slot >= 0 && slot < p.assignments) {
                    if constexpr (AM == kAGather) src = slot / p.topk;
                    else src = slot;
                    if constexpr (EPI == kEpiScatterWeighted) {
                        const int t = slot / p.topk, rk = slot - t * p.topk;
                        w = p.routes[(size_t)t * 2 * p.topk + p.topk + rk];
                    }
                }
            } else {
                src = row;
            }
        }
        row_src[r] = src;
        row_w[r] = w;
    }
    __syncthreads();

    // A wave whose rows are all padding (an expert's tail block) skips its
    // fragment reads and MFMAs; it still loads its share and joins barriers.
    bool wave_rows_live = true;
    if constexpr (AM == kAGather || EPI == kEpiScatterWeighted) {
        bool any = false;
        for (int j = lane; j < TM; j += 64) any |= row_src[wm * TM + j] >= 0;
        wave_rows_live = __any(any);
    }

    // A copies of 8-row groups that are all padding are skipped (padding rows
    // are a suffix of the tile, so the group's first row decides); their LDS
    // rows keep stale values, feed only padding rows of the product and are
    // replaced by zeros in the epilogue.  Safe with two stages, whose wait
    // drains every outstanding copy whatever their number.
    bool a_live[ACH];
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
        const int r = (i * (NT / 64) + wave) * RPI;
        a_live[i] = STAGES != 2 || !(AM == kAGather || EPI == kEpiScatterWeighted) || row_src[r] >= 0;
    }
    // Per-lane load sources.  Instruction i of wave w fills rows
    // [q*RPI, (q+1)*RPI) with q = i*(NT/64) + w; lane l supplies row
    // q*RPI + l/CPR into chunk slot l%CPR, i.e. global chunk slot ^ swz(row).
    const uint16_t* a_src[ACH];
    uint32_t a_off[ACH];  // the same as byte offsets from p.a (big wave tiles)
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
        int r, kchunk;
        row_copy_slot<NT, CPR>(i, wave, lane, r, kchunk);
        long src_row;
        if constexpr (AM == kAGather) {
            const long s_ = row_src[r];
            src_row = s_ >= 0 ? s_ : 0;  // padding rows read row 0; their outputs are dropped
        } else {
            src_row = row0 + r < p.rows ? row0 + r : 0;
        }
        a_src[i] = p.a + src_row * (long)p.lda + kchunk;
        a_off[i] = (uint32_t)((src_row * (long)p.lda + kchunk) * 2);
    }
    const uint16_t* wexp = p.w + (long)expert * p.w_expert_stride;
    // Row-major weights: staged like A (swizzled 128-byte rows).  Frag16
    // weights: instruction q copies one whole 1 KB fragment (16 rows x 32 of
    // K), so the B stage holds BN/16 bands x BK/32 fragments in global order.
    const uint16_t* b_src[BCH];
    uint32_t b_off[BCH];  // the same as byte offsets from wexp (big wave tiles)
#pragma unroll
    for (int i = 0; i < BCH; ++i) {
        const long e_off = b_copy_offset<NT, CPR, BN, BK, EPI == kEpiSilu, WL == kWeightsFrag16>(
            i, wave, lane, c0, p.n, p.w_up_offset, p.k);
        b_src[i] = wexp + e_off;
        b_off[i] = (uint32_t)(e_off * 2);
    }
    auto issue = [&](int kt, int stage) {
        uint16_t* As = smem + stage * STAGE_ELEMS;
        uint16_t* Bs = As + BM * BK;
        const int kb = kt * BK;
#pragma unroll
        for (int i = 0; i < ACH; ++i) {
            if (!a_live[i]) continue;
            if constexpr (kBigWave) lds_dma16_off(p.a + kb, a_off[i], As + (i * (NT / 64) + wave) * 512);
            else lds_dma16(a_src[i] + kb, As + (i * (NT / 64) + wave) * 512);
        }
#pragma unroll
        for (int i = 0; i < BCH; ++i) {
            const int kw = WL == kWeightsFrag16 ? kb * 16 : kb;
            if constexpr (kBigWave) lds_dma16_off(wexp + kw, b_off[i], Bs + (i * (NT / 64) + wave) * 512);
            else lds_dma16(b_src[i] + kw, Bs + (i * (NT / 64) + wave) * 512);
        }
    };

    f32x16 acc[MI][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j)
#pragma unroll
            for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.f;

    const int nk = p.k / BK;
#pragma unroll
    for (int s_ = 0; s_ < STAGES - 1; ++s_)
        if (s_ < nk) issue(s_, s_);

    const int lr = lane & 31, lh = lane >> 5;
    // Fragment reads of one 16-deep K step; the next step's reads are issued
    // before the current step's MFMAs so LDS latency hides under the MFMAs.
    auto frags = [&](const uint16_t* As, const uint16_t* Bs, int ks, bf16x8* af, bf16x8* bfr) {
        const int c = ks * 2 + lh;
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            const int r = wm * TM + i * 32 + lr;
            af[i] = as_bf16x8(*(const u32x4*)(As + r * BK + ((c ^ swz<CPR>(r)) * 8)));
        }
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            int r;
            if constexpr (EPI == kEpiSilu) {
                const int jj = j < NI / 2 ? j : j - NI / 2;
                r = (j < NI / 2 ? 0 : BN / 2) + wn * (TN / 2) + jj * 32 + lr;
            } else {
                r = wn * TN + j * 32 + lr;
            }
            if constexpr (WL == kWeightsFrag16) {
                // row r, K piece 2*ks + lh of the stage: fragment (r/16, piece/4),
                // 16-byte slot (piece%4)*16 + r%16.
                const int piece = ks * 2 + lh;
                bfr[j] = as_bf16x8(*(const u32x4*)(Bs + ((r >> 4) * (BK / 32) + (piece >> 2)) * 512 +
                                                   ((piece & 3) * 16 + (r & 15)) * 8));
            } else {
                bfr[j] = as_bf16x8(*(const u32x4*)(Bs + r * BK + ((c ^ swz<CPR>(r)) * 8)));
            }
        }
    };
    if constexpr (((kBigWave && kBigWaveSkip) || (kFragSkip && BM == 256)) &&
                  (AM == kAGather || EPI == kEpiScatterWeighted)) {
        // Padding is a suffix of the block, so the 32-row fragments holding
        // live rows are a prefix of the wave's MI.  The K loop runs with the
        // MFMAs and A fragment reads of that prefix only; the other fragments
        // keep zero accumulators (their rows are written as zeros or dropped).
        // The count is wave-uniform and chosen once, outside the K loop, so
        // the accumulators never move.
        static_assert(MI <= 4, "at most four 32-row fragments per wave");
        int nl = 0;
#pragma unroll
        for (int i = 0; i < MI; ++i) nl += row_src[wm * TM + i * 32] >= 0;
        nl = __builtin_amdgcn_readfirstlane(nl);
        auto k_loop = [&](auto nl_tag) {
            constexpr int NL = decltype(nl_tag)::value;
            for (int kt = 0; kt < nk; ++kt) {
                if (kt + STAGES - 2 < nk) wait_vmcnt<(STAGES - 2) * L>();
                else wait_vmcnt<0>();
                lds_barrier();
                if (kt + STAGES - 1 < nk) issue(kt + STAGES - 1, (kt + STAGES - 1) % STAGES);
                if constexpr (NL > 0) {
                    const uint16_t* As = smem + (kt % STAGES) * STAGE_ELEMS;
                    const uint16_t* Bs = As + BM * BK;
                    if constexpr (IG >= 0) __builtin_amdgcn_iglp_opt(IG);
                    bf16x8 af[2][MI], bfr[2][NI];
                    auto frags_nl = [&](int ks, bf16x8* a_, bf16x8* b_) {
                        bf16x8 a_all[MI];
                        frags(As, Bs, ks, a_all, b_);  // reads of fragments past NL are dead code
#pragma unroll
                        for (int i = 0; i < NL; ++i) a_[i] = a_all[i];
                    };
                    frags_nl(0, af[0], bfr[0]);
#pragma unroll
                    for (int ks = 0; ks < BK / 16; ++ks) {
                        if (ks + 1 < BK / 16) frags_nl(ks + 1, af[(ks + 1) & 1], bfr[(ks + 1) & 1]);
#pragma unroll
                        for (int i = 0; i < NL; ++i)
#pragma unroll
                            for (int j = 0; j < NI; ++j)
                                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ks & 1][i], bfr[ks & 1][j],
                                                                                    acc[i][j], 0, 0, 0);
                    }
                }
            }
        };
        switch (nl) {
            case 4: k_loop(std::integral_constant<int, MI < 4 ? MI : 4>{}); break;
            case 3: k_loop(std::integral_constant<int, MI < 3 ? MI : 3>{}); break;
            case 2: k_loop(std::integral_constant<int, MI < 2 ? MI : 2>{}); break;
            case 1: k_loop(std::integral_constant<int, 1>{}); break;
            default: k_loop(std::integral_constant<int, 0>{}); break;
        }
    } else {
        for (int kt = 0; kt < nk; ++kt) {
            // Tile kt's loads are done once at most the later-issued loads remain
            // (VMEM loads complete in order).
            if (kt + STAGES - 2 < nk) wait_vmcnt<(STAGES - 2) * L>();
            else wait_vmcnt<0>();
            lds_barrier();
            if (kt + STAGES - 1 < nk) issue(kt + STAGES - 1, (kt + STAGES - 1) % STAGES);
            const uint16_t* As = smem + (kt % STAGES) * STAGE_ELEMS;
            const uint16_t* Bs = As + BM * BK;
            if constexpr (!kBigWave) {
                if (!wave_rows_live) continue;
            }
            if constexpr (IG >= 0) __builtin_amdgcn_iglp_opt(IG);
            bf16x8 af[2][MI], bfr[2][NI];
            frags(As, Bs, 0, af[0], bfr[0]);
    #pragma unroll
            for (int ks = 0; ks < BK / 16; ++ks) {
                if (ks + 1 < BK / 16) frags(As, Bs, ks + 1, af[(ks + 1) & 1], bfr[(ks + 1) & 1]);
    #pragma unroll
                for (int i = 0; i < MI; ++i)
    #pragma unroll
                    for (int j = 0; j < NI; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ks & 1][i], bfr[ks & 1][j], acc[i][j], 0, 0, 0);
            }
        }
    }
    __syncthreads();  // stages are reused for the output tile

    // Epilogue 1: accumulators -> BF16 tile in LDS.  Value q of lane l sits at
    // row (q/4)*8 + (l/32)*4 + q%4, column l%32 of its 32x32 block.
    uint16_t* C = smem;
#pragma unroll
    for (int i = 0; i < MI; ++i) {
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const int r = wm * TM + i * 32 + (q >> 2) * 8 + lh * 4 + (q & 3);
            if constexpr (EPI == kEpiSilu) {
#pragma unroll
                for (int j = 0; j < NI / 2; ++j) {
                    const float g = round_bf16(acc[i][j][q]);
                    const float u = round_bf16(acc[i][j + NI / 2][q]);
                    C[r * CSTRIDE + wn * (TN / 2) + j * 32 + lr] = float_to_bf16_bits(silu(g) * u);
                }
            } else {
                const float w = EPI == kEpiScatterWeighted ? row_w[r] : 1.0f;
#pragma unroll
                for (int j = 0; j < NI; ++j) {
                    const float v = EPI == kEpiScatterWeighted ? acc[i][j][q] * w : acc[i][j][q];
                    C[r * CSTRIDE + wn * TN + j * 32 + lr] = float_to_bf16_bits(v);
                }
            }
        }
        // Big wave tiles: keep each row block's accumulator reads next to
        // their use (hoisting all 256 would exhaust the VGPRs).
        if constexpr (kBigWave) __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();

    // Epilogue 2: 16-byte row segments to global memory.
    constexpr int SEGS = NOUT / 8;
    uint16_t* out = (uint16_t*)p.out;
    const bool vec = (p.ldo % 8) == 0 && ((uintptr_t)p.out % 16) == 0;
    if constexpr (kStrided && EPI != kEpiScatterWeighted) {
        // A small block run by a kernel shorter than the dispatch block: the
        // block's rows past BM are padding and are written as zeros.
        for (int i = tid; i < (stride - BM) * SEGS; i += NT) {
            const int row = row0 + BM + i / SEGS, col = c0 + (i % SEGS) * 8;
            if (row >= p.rows || col >= p.n) continue;
            uint16_t* o = out + (long)row * p.ldo + col;
            if (vec && col + 8 <= p.n) *(u32x4*)o = u32x4{0u, 0u, 0u, 0u};
            else for (int e = 0; e < 8 && col + e < p.n; ++e) o[e] = 0;
        }
    }
    for (int i = tid; i < BM * SEGS; i += NT) {
        const int r = i / SEGS, sg = i - r * SEGS;
        const int row = row0 + r;
        if (row >= p.rows) continue;
        long dst;
        bool pad = false;  // gathered padding row: zero, as the reference's zero-filled A makes it
        if constexpr (EPI == kEpiScatterWeighted) {
            dst = row_src[r];
            if (dst < 0) continue;
        } else {
            dst = row;
            if constexpr (AM == kAGather) pad = row_src[r] < 0;
        }
        const int col = c0 + sg * 8;
        if (col >= p.n) continue;
        const uint16_t* src = C + r * CSTRIDE + sg * 8;
        uint16_t* o = out + dst * (long)p.ldo + col;
        if (vec && col + 8 <= p.n) {
            *(u32x4*)o = pad ? u32x4{0u, 0u, 0u, 0u} : *(const u32x4*)src;
        } else {
            for (int e = 0; e < 8 && col + e < p.n; ++e) o[e] = pad ? (uint16_t)0 : src[e];
        }
    }
}

template <int BM, int BN, int WM, int WN, int STAGES, int AM, int EPI, int BK = 64, int WL = kWeightsRowMajor,
          int IG = -1>
int launch_mfma(const GemmArgs& p, hipStream_t s) {
    constexpr int NOUT = EPI == kEpiSilu ? BN / 2 : BN;
    if constexpr ((BM / WM) * (BN / WN) >= 128 * 128) {
        // 32-bit operand offsets: the A rows and one expert's weights must
        // span less than 4 GiB.
        const long a_rows = AM == kAGather ? (long)p.assignments / p.topk : (long)p.rows;
        if (a_rows * (long)p.lda * 2 >= (1L << 32) || p.w_expert_stride * 2 >= (1L << 32)) return kInvalid;
    }
    const int stride = p.block_stride ? p.block_stride : BM;
    if (stride < BM || stride % BM) return kInvalid;
    const long m_blocks = (p.rows + stride - 1) / stride;
    const long n_tiles = (p.n + NOUT - 1) / NOUT;
    const long grid = (m_blocks * n_tiles + kXcds - 1) / kXcds * kXcds;
    if (grid <= 0 || grid > 0x7fffffffL) return kInvalid;
    mfma_gemm<BM, BN, WM, WN, STAGES, AM, EPI, BK, WL, IG><<<(unsigned)grid, 64 * WM * WN, 0, s>>>(p);
    return (int)hipGetLastError();
}

template <int BM, int BN, int WM, int WN, int AM, int EPI>
int launch_lds(const GemmArgs& p, bool aligned, hipStream_t s) {
    constexpr int NOUT = EPI == kEpiSilu ? BN / 2 : BN;
    const long m_blocks = (p.rows + BM - 1) / BM;
    const long n_tiles = (p.n + NOUT - 1) / NOUT;
    const long total = m_blocks * n_tiles;
    const long grid = (total + kXcds - 1) / kXcds * kXcds;
    if (grid <= 0 || grid > 0x7fffffffL) return kInvalid;
    if (aligned) lds_gemm<BM, BN, WM, WN, AM, EPI, true><<<(unsigned)grid, 64 * WM * WN, 0, s>>>(p);
    else lds_gemm<BM, BN, WM, WN, AM, EPI, false><<<(unsigned)grid, 64 * WM * WN, 0, s>>>(p);
    return (int)hipGetLastError();
}

// Weight-streaming launch.  Columns per wave (NB blocks of 16) and K steps per
// batch (U) were chosen by measurement on MI355X: SiLU gate_up streams two
// weight rows per output column and prefers NB=1; single-stream projections
// prefer NB=4.
template <int AM, int EPI, int RT, int WL>
int launch_stream(const GemmArgs& p, bool aligned, hipStream_t s) {
    // Row-major weights: SiLU streams two weight rows per column and prefers
    // one 16-column block per wave; single-stream projections prefer four.
    // Frag16 weights (1 KB contiguous fragments): two blocks per wave, eight
    // K steps per batch.
    constexpr int NB = WL == kWeightsFrag16 ? 2 : (EPI == kEpiSilu ? 1 : 4);
    constexpr int U = WL == kWeightsFrag16 ? 8 : 4;
    const int rows = p.block_stride ? p.block_stride : 16 * RT;  // rows between the row blocks
    const long m_blocks = (p.rows + rows - 1) / rows;
    if (!aligned) {
        if (RT != 1 || WL != kWeightsRowMajor) return kInvalid;
        const long n_blocks = (p.n + 15) / 16;
        const long groups = (m_blocks * n_blocks + kStreamWaves - 1) / kStreamWaves;
        const long grid = (groups + kXcds - 1) / kXcds * kXcds;
        stream_gemm<AM, EPI, false><<<(unsigned)grid, 64 * kStreamWaves, 0, s>>>(p);
        return (int)hipGetLastError();
    }
    const long n_blocks = (p.n + 16 * NB - 1) / (16 * NB);
    const long groups = (m_blocks * n_blocks + kStreamWaves - 1) / kStreamWaves;
    const long grid = (groups + kXcds - 1) / kXcds * kXcds;
    if (grid <= 0 || grid > 0x7fffffffL) return kInvalid;
    stream_gemm_fast<AM, EPI, NB, U, kStreamWaves, RT, WL><<<(unsigned)grid, 64 * kStreamWaves, 0, s>>>(p);
    return (int)hipGetLastError();
}

// Row block -> kernel.  Every kernel's row block must equal `bm`: dispatch
// built tiles[] (one expert per bm rows) and the kernels index it per block.
// 16/32: weight streaming; 64/128/256: direct-to-LDS
// MFMA tiles (64x256 with 4 waves, 128x128 with 4 waves, 256x256 with 16
// waves, wave tile 64x64), measured best on MI355X for the prefill shapes; shapes the MFMA
// kernel cannot take (K not a multiple of 64, unaligned rows, FP32 output)
// use the register-staged LDS kernel, which reads row-major weights only.
// 256x256 tiles: 4x4 waves of 64x64 (the measured default) or, built with
// -DTAU_M256_BIG_WAVES, 2x2 waves of 128x128 with AGPR accumulators.
#ifdef TAU_M256_BIG_WAVES
constexpr int kM256WavesM = 2, kM256WavesN = 2;
#else
constexpr int kM256WavesM = 4, kM256WavesN = 4;
#endif

template <int AM, int EPI, int WL>
int launch_by_rows(const GemmArgs& p, int bm, bool aligned, hipStream_t s) {
    const bool mfma_ok = aligned && p.k % 64 == 0 && EPI != kEpiStoreF32;
    if constexpr (EPI != kEpiStoreF32) {
        if (mfma_ok) {
            switch (bm) {
                case 64: return launch_mfma<64, 256, 1, 4, 2, AM, EPI, 64, WL>(p, s);
                case 128: return launch_mfma<128, 128, 2, 2, 2, AM, EPI, 64, WL, 1>(p, s);
                case 256: {
                    if constexpr (kSplitRows > 0) {
                        // Blocks with at most kSplitRows live rows (an expert's
                        // tail or a lightly routed expert) run on the shorter
                        // tile, the rest on the 256-row tile.
                        // The receipt keeps describing the 256-row tile.
                        GemmArgs big = p, small = p;
                        big.split_rows = small.split_rows = kSplitRows;
                        small.block_stride = 256;
                        small.receipt = nullptr;
                        const int code =
                            launch_mfma<256, 256, kM256WavesM, kM256WavesN, 2, AM, EPI, 64, WL, 1>(big, s);
                        if (code) return code;
                        if constexpr (kSplitRows == 32) return launch_stream<AM, EPI, 2, WL>(small, aligned, s);
                        else if constexpr (kSplitRows == 64)
                            return launch_mfma<64, 256, 1, 4, 2, AM, EPI, 64, WL>(small, s);
                        else return launch_mfma<128, 128, 2, 2, 2, AM, EPI, 64, WL, 1>(small, s);
                    }
                    return launch_mfma<256, 256, kM256WavesM, kM256WavesN, 2, AM, EPI, 64, WL, 1>(p, s);
                }
                default: break;
            }
        }
    }
    switch (bm) {
        case 16: return launch_stream<AM, EPI, 1, WL>(p, aligned, s);
        case 32:
            if (aligned) return launch_stream<AM, EPI, 2, WL>(p, aligned, s);
            break;
        default: break;
    }
    if constexpr (WL != kWeightsRowMajor) {
        return kInvalid;
    } else {
        switch (bm) {
            case 32: return launch_lds<32, 128, 1, 2, AM, EPI>(p, aligned, s);
            case 64: return launch_lds<64, 128, 2, 2, AM, EPI>(p, aligned, s);
            case 128: return launch_lds<128, 128, 2, 2, AM, EPI>(p, aligned, s);
            case 256: return launch_lds<256, 128, 4, 2, AM, EPI>(p, aligned, s);
            default: return kInvalid;
        }
    }
}

template <int AM, int EPI>
int launch_layout(const GemmArgs& p, int bm, bool aligned, hipStream_t s) {
    if (p.w_layout == kWeightsFrag16) {
        if constexpr (EPI == kEpiStoreF32) return kInvalid;
        else return launch_by_rows<AM, EPI, kWeightsFrag16>(p, bm, aligned, s);
    }
    return launch_by_rows<AM, EPI, kWeightsRowMajor>(p, bm, aligned, s);
}

}  // namespace

// Row-block sizes of the compiled kernels: 16 (weight streaming) and
// 32 (streaming, two row groups) and 64/128/256 (LDS-tiled MFMA).  Dispatch must
// pad experts to the same M.
bool gemm_rows_supported(int bm) { return bm == 16 || bm == 32 || bm == 64 || bm == 128 || bm == 256; }

int launch_grouped_gemm(const GemmArgs& p, int bm, int a_mode, int epilogue, hipStream_t s) {
    if (!p.a || !p.w || !p.out || p.rows <= 0 || p.n <= 0 || p.k <= 0 || p.lda < p.k || p.ldo < p.n)
        return kInvalid;
    if (!gemm_rows_supported(bm)) return kInvalid;
    if ((a_mode == kAGather || epilogue == kEpiScatterWeighted) && (!p.slots || p.topk <= 0)) return kInvalid;
    if (epilogue == kEpiScatterWeighted && !p.routes) return kInvalid;
    const bool aligned = p.k % 8 == 0 && p.lda % 8 == 0 && ((uintptr_t)p.a % 16) == 0 && ((uintptr_t)p.w % 16) == 0 &&
                         (p.w_expert_stride % 8) == 0;
    if (p.w_layout == kWeightsFrag16 &&
        (!aligned || p.k % 64 || p.n % 16 || p.w_up_offset % 16 || epilogue == kEpiStoreF32))
        return kInvalid;
    if (p.w_layout != kWeightsRowMajor && p.w_layout != kWeightsFrag16) return kInvalid;
    if (a_mode == kAGather) {
        switch (epilogue) {
            case kEpiSilu: return launch_layout<kAGather, kEpiSilu>(p, bm, aligned, s);
            case kEpiStoreBf16: return launch_layout<kAGather, kEpiStoreBf16>(p, bm, aligned, s);
            default: return kInvalid;
        }
    }
    switch (epilogue) {
        case kEpiSilu: return launch_layout<kADirect, kEpiSilu>(p, bm, aligned, s);
        case kEpiStoreBf16: return launch_layout<kADirect, kEpiStoreBf16>(p, bm, aligned, s);
        case kEpiScatterWeighted: return launch_layout<kADirect, kEpiScatterWeighted>(p, bm, aligned, s);
        case kEpiStoreF32: return launch_layout<kADirect, kEpiStoreF32>(p, bm, aligned, s);
        default: return kInvalid;
    }
}

}  // namespace tau_amd
