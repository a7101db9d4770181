/*
 * TEST INFRASTRUCTURE ONLY -- the parity oracle for the MoE expert-FFN path.
 *
 * This file is a CPU restatement of tau.rs's f32 sparse-MoE path
 * (SparseMoeBlock built with optimize_kernel=false on the CPU) plus a
 * "BF16 contract" mode that mirrors the rounding points of the reference's
 * native BF16 prefill kernels.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it, and only as the checker or the
 * timed CPU baseline.  The product library never links or calls it.
 *
 * Reference functions restated here (paths relative to the tau.rs root):
 *   routing      crates/models/src/components/sparse_moe/routing.rs:125-231
 *                (softmax_last_dim at :139-141, rank-order weight sum :187-191,
 *                 w = p / sum at :198-202, per-expert lists at :215-227)
 *   top-k        crates/models/src/components/sparse_moe/routing.rs:239-257
 *                (score descending, smaller expert id on equal scores)
 *   expert loop  crates/models/src/components/sparse_moe/experts.rs:97-152
 *   expert MLP   crates/models/src/components/mlp.rs:50-83,
 *                crates/models/src/components/mlp/projection.rs:123-142
 *   shared       crates/models/src/components/sparse_moe/shared_expert.rs:39-69,142-160
 *   dispatch     crates/cuda-kernels/src/kernels/moe_dispatch.cu:11-85
 *                (padded offsets, slot sentinel, tile worklist, status word),
 *                with the stable token-ascending order of routing.rs:215-227
 *   BF16 rounds  crates/cuda-kernels/src/kernels/moe_gemm.cu:119-137,
 *                linear_bf16_fp32.cu:74-98, silu_and_mul.cu:71-74,
 *                moe_dispatch.cuh:13-20, moe_shared.cu:17-36
 *
 * Third-party arithmetic the reference delegates (candle-core 0.11.0,
 * candle-nn 0.11.0, gemm 0.18/0.19) is not vendored; its published algorithm
 * is restated: softmax = max, exp(x-max), sum, divide; silu(v) = v/(1+exp(-v));
 * sigmoid(v) = 1/(1+exp(-v)); matmul = f32 dot products.  Summation order of
 * the dot products and of the softmax denominator is this file's own (8-lane
 * partial sums, then a fixed pairwise fold; the softmax sum is sequential):
 * bit patterns of f32 outputs are therefore pinned only to tolerance, while
 * expert ids and permutation order are exact.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORACLE_ACT_SILU 0
#define ORACLE_ACT_RELU 1

/* Round-to-nearest-even f32 -> bf16 -> f32, NaN kept quiet. */
static inline float bf16_round(float v) {
    uint32_t u;
    memcpy(&u, &v, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) {
        u = (u | 0x00400000u) & 0xffff0000u;
    } else {
        u += 0x7fffu + ((u >> 16) & 1u);
        u &= 0xffff0000u;
    }
    float r;
    memcpy(&r, &u, 4);
    return r;
}

float oracle_bf16_round(float v) { return bf16_round(v); }

void oracle_bf16_round_array(const float* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = bf16_round(in[i]);
}

static inline float act_apply(float v, int act) {
    if (act == ORACLE_ACT_RELU) return v > 0.f ? v : 0.f;
    return v / (1.0f + expf(-v));
}

void oracle_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

int oracle_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------ */
/* Routing: routing.rs:125-257                                          */
/* ------------------------------------------------------------------ */

/* Softmax of one row (candle_nn::ops::softmax_last_dim): max, exp(x - max),
 * sequential sum, divide. */
static void softmax_row(const float* logits, int E, float* p) {
    float maximum = -INFINITY;
    for (int e = 0; e < E; ++e) maximum = fmaxf(maximum, logits[e]);
    float sum = 0.f;
    for (int e = 0; e < E; ++e) {
        p[e] = expf(logits[e] - maximum);
        sum += p[e];
    }
    for (int e = 0; e < E; ++e) p[e] = p[e] / sum;
}

/* "a before b" in routing.rs:239-257's order: larger score, then smaller id. */
static inline int ranks_before(const float* s, int a, int b) {
    if (s[a] == s[b]) return a < b;
    return s[a] > s[b];
}

/* select_experts (routing.rs:239-257): rejects K == 0, K > E and non-finite
 * scores; returns the K best ids in rank order.  Returns 0 on success. */
int oracle_select_experts(const float* scores, int E, int K, int32_t* ids) {
    if (K <= 0 || K > E) return -1;
    for (int e = 0; e < E; ++e)
        if (!isfinite(scores[e])) return -1;
    /* Partial selection sort: K passes, each picks the best remaining id. */
    unsigned char* taken = (unsigned char*)calloc((size_t)E, 1);
    if (!taken) return -2;
    for (int r = 0; r < K; ++r) {
        int best = -1;
        for (int e = 0; e < E; ++e) {
            if (taken[e]) continue;
            if (best < 0 || ranks_before(scores, e, best)) best = e;
        }
        taken[best] = 1;
        ids[r] = best;
    }
    free(taken);
    return 0;
}

/* Router reference plan, routing half (routing.rs:125-231 with softmax
 * scores): per token, softmax over E, top-K, then w = p / sum(selected p)
 * summed in rank order when `normalize`.  Returns -1 - token for the first
 * token whose row is rejected by select_experts (non-finite logits); the
 * reference bails at that point. */
int oracle_route(const float* logits, int T, int E, int K, int normalize,
                 int32_t* ids, float* weights, float* probabilities /*[T,E] or NULL*/) {
    float* p = (float*)malloc(sizeof(float) * (size_t)E);
    if (!p) return -100000000;
    for (int t = 0; t < T; ++t) {
        softmax_row(logits + (size_t)t * E, E, p);
        if (probabilities) memcpy(probabilities + (size_t)t * E, p, sizeof(float) * (size_t)E);
        if (oracle_select_experts(p, E, K, ids + (size_t)t * K) != 0) {
            free(p);
            return -1 - t;
        }
        float sum = 0.f;
        for (int r = 0; r < K; ++r) sum += p[ids[(size_t)t * K + r]];
        for (int r = 0; r < K; ++r) {
            float w = p[ids[(size_t)t * K + r]];
            weights[(size_t)t * K + r] = normalize ? w / sum : w;
        }
    }
    free(p);
    return 0;
}

/* Router reference plan, grouping half (routing.rs:215-227): tokens are
 * visited in ascending order, so every expert's list is token-ascending.
 * counts[E]; offsets[E+1] exclusive prefix; slots[A] = t*K + r, expert-major. */
void oracle_plan(const int32_t* ids, int T, int K, int E,
                 int32_t* counts, int32_t* offsets, int32_t* slots) {
    memset(counts, 0, sizeof(int32_t) * (size_t)E);
    for (int64_t a = 0; a < (int64_t)T * K; ++a) counts[ids[a]]++;
    offsets[0] = 0;
    for (int e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + counts[e];
    int32_t* cursor = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
    memcpy(cursor, offsets, sizeof(int32_t) * (size_t)E);
    for (int t = 0; t < T; ++t)
        for (int r = 0; r < K; ++r) {
            int e = ids[(size_t)t * K + r];
            slots[cursor[e]++] = t * K + r;
        }
    free(cursor);
}

/* Capacity bound of the padded dispatch (crates/cuda-kernels/src/moe/prefill.rs:17-30,
 * generalised from E=256/K=8): all assignments plus a worst-case M-1 padding
 * rows for every expert that can be non-empty, rounded to a multiple of M. */
int64_t oracle_capacity(int64_t T, int64_t E, int64_t K, int64_t M) {
    if (T <= 0 || E <= 0 || K <= 0 || M <= 0) return -1;
    int64_t a = T * K;
    int64_t bound = a + (a < E ? a : E) * (M - 1) + (M - 1);
    return bound / M * M;
}

/* Padded device-layout dispatch (moe_dispatch.cu:11-85 semantics, stable
 * order).  meta[2E+2] = counts[E], cursors[E] (equal to counts after the
 * scatter), status, padded total.  offsets[E+1] padded to M.  slots[cap]:
 * assignment t*K+r in token-ascending order inside each expert, sentinel
 * T*K on padding rows.  tiles[cap/M]: expert of each M-row tile, -1 past
 * the padded total.  Invalid routes set status=1 and contribute nothing. */
int oracle_dispatch(const int32_t* ids, int T, int K, int E, int M, int64_t cap,
                    int32_t* meta, int32_t* offsets, int32_t* slots, int32_t* tiles) {
    int64_t A = (int64_t)T * K;
    memset(meta, 0, sizeof(int32_t) * (size_t)(2 * E + 2));
    for (int64_t i = 0; i < cap; ++i) slots[i] = (int32_t)A;
    for (int64_t i = 0; i < cap / M; ++i) tiles[i] = -1;
    for (int64_t a = 0; a < A; ++a) {
        int t = (int)(a / K), r = (int)(a % K);
        int e = ids[a];
        int valid = e >= 0 && e < E;
        for (int q = 0; q < r && valid; ++q) valid = ids[(size_t)t * K + q] != e;
        if (!valid) { meta[2 * E] = 1; continue; }
        meta[e]++;
    }
    int64_t end = 0;
    for (int e = 0; e < E; ++e) {
        offsets[e] = (int32_t)end;
        end += ((int64_t)meta[e] + M - 1) / M * M;
    }
    offsets[E] = (int32_t)end;
    meta[2 * E + 1] = (int32_t)end;
    if (end > cap) return -1;
    for (int e = 0; e < E; ++e)
        for (int64_t tile = offsets[e] / M; tile < offsets[e + 1] / M; ++tile) tiles[tile] = e;
    for (int64_t a = 0; a < A; ++a) {
        int t = (int)(a / K), r = (int)(a % K);
        int e = ids[a];
        int valid = e >= 0 && e < E;
        for (int q = 0; q < r && valid; ++q) valid = ids[(size_t)t * K + q] != e;
        if (!valid) continue;
        slots[offsets[e] + meta[E + e]++] = (int32_t)a;
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* Dense kernels                                                        */
/* ------------------------------------------------------------------ */

typedef float v8f __attribute__((vector_size(32)));

static inline v8f load8(const float* p) {
    v8f v;
    memcpy(&v, p, sizeof(v));
    return v;
}

static inline float hsum8(v8f v) {
    return ((v[0] + v[4]) + (v[2] + v[6])) + ((v[1] + v[5]) + (v[3] + v[7]));
}

/* C[i, j] = sum_k A[i, k] * B[j, k] for i < m, j < n, both operands K-contiguous
 * (row strides lda, ldb), C row stride ldc.  4x4 register blocks with 8-lane
 * partial sums; lane tails are added last in k order. */
static void gemm_nt(const float* A, int64_t lda, const float* B, int64_t ldb,
                    float* C, int64_t ldc, int m, int n, int k) {
    int k8 = k / 8 * 8;
    for (int i0 = 0; i0 < m; i0 += 4) {
        int mi = m - i0 < 4 ? m - i0 : 4;
        for (int j0 = 0; j0 < n; j0 += 4) {
            int nj = n - j0 < 4 ? n - j0 : 4;
            v8f acc[4][4];
            for (int a = 0; a < 4; ++a)
                for (int b = 0; b < 4; ++b) acc[a][b] = (v8f){0, 0, 0, 0, 0, 0, 0, 0};
            const float* ar[4];
            const float* br[4];
            for (int a = 0; a < 4; ++a) ar[a] = A + (int64_t)(i0 + (a < mi ? a : 0)) * lda;
            for (int b = 0; b < 4; ++b) br[b] = B + (int64_t)(j0 + (b < nj ? b : 0)) * ldb;
            for (int kk = 0; kk < k8; kk += 8) {
                v8f bv[4];
                for (int b = 0; b < 4; ++b) bv[b] = load8(br[b] + kk);
                for (int a = 0; a < 4; ++a) {
                    v8f av = load8(ar[a] + kk);
                    for (int b = 0; b < 4; ++b) acc[a][b] += av * bv[b];
                }
            }
            for (int a = 0; a < mi; ++a)
                for (int b = 0; b < nj; ++b) {
                    float s = hsum8(acc[a][b]);
                    for (int kk = k8; kk < k; ++kk) s += ar[a][kk] * br[b][kk];
                    C[(int64_t)(i0 + a) * ldc + j0 + b] = s;
                }
        }
    }
}

void oracle_linear_f32(const float* input, const float* weight, float* output,
                       int rows, int columns, int inner) {
    gemm_nt(input, inner, weight, inner, output, columns, rows, columns, inner);
}

/* One expert over its gathered rows.  f32 mode (bf16 == 0): mlp.rs:50-83 on
 * the CPU; gate = x Wg^T, up = x Wu^T, a = act(gate) * up, d = a Wd^T, c = d*w.
 * BF16 mode (bf16 == 1): gate_up rounded to BF16, a = bf16(silu(g) * u) in
 * f32, c = bf16(d * w) (moe_gemm.cu:119-137, silu_and_mul.cu:71-74,
 * linear_bf16_fp32.cu:176-206 weight-before-round). */
static void expert_rows(const float* xe, int n, int H, int I,
                        const float* gate_up, const float* down,
                        const float* w, int act, int bf16, float* c /*[n,H]*/) {
    float* gu = (float*)malloc(sizeof(float) * (size_t)n * 2 * I);
    float* a = (float*)malloc(sizeof(float) * (size_t)n * I);
    gemm_nt(xe, H, gate_up, H, gu, 2 * I, n, 2 * I, H);
    for (int i = 0; i < n; ++i)
        for (int j = 0; j < I; ++j) {
            float g = gu[(size_t)i * 2 * I + j], u = gu[(size_t)i * 2 * I + I + j];
            if (bf16) {
                g = bf16_round(g);
                u = bf16_round(u);
                a[(size_t)i * I + j] = bf16_round(act_apply(g, act) * u);
            } else {
                a[(size_t)i * I + j] = act_apply(g, act) * u;
            }
        }
    gemm_nt(a, I, down, I, c, H, n, H, I);
    for (int i = 0; i < n; ++i) {
        float wi = w ? w[i] : 1.0f;
        for (int h = 0; h < H; ++h) {
            float v = c[(size_t)i * H + h] * wi;
            c[(size_t)i * H + h] = bf16 ? bf16_round(v) : v;
        }
    }
    free(gu);
    free(a);
}

/* Routed experts (experts.rs:97-152).  Experts are visited in ascending order;
 * each gathers its token rows (token-ascending, routing.rs:215-227), computes
 * the weighted MLP and writes the assignment's staged row t*K + r; the output
 * is then summed over ranks 0..K-1 in f32 starting from zero and, in BF16
 * mode, rounded once.  gate_up [E,2I,H] (gate rows first), down [E,H,I].
 * Only tokens with token_mask[t] != 0 are computed when a mask is given
 * (tokens are independent, so a subset reproduces those rows exactly). */
int oracle_moe(const float* x, int T, int H, int I, int E, int K,
               const int32_t* ids, const float* weights,
               const float* gate_up, const float* down,
               int act, int bf16, const unsigned char* token_mask, float* out) {
    int64_t A = (int64_t)T * K;
    int32_t* counts = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
    int32_t* offsets = (int32_t*)malloc(sizeof(int32_t) * (size_t)(E + 1));
    int32_t* slots = (int32_t*)malloc(sizeof(int32_t) * (size_t)A);
    float* staged = (float*)calloc((size_t)A * H, sizeof(float));
    if (!counts || !offsets || !slots || !staged) return -1;
    oracle_plan(ids, T, K, E, counts, offsets, slots);
    /* Work items: (expert, row block) so that one hot expert still spreads. */
    const int RB = 64;
    int64_t items = 0;
    for (int e = 0; e < E; ++e) items += (counts[e] + RB - 1) / RB;
    int64_t* item_e = (int64_t*)malloc(sizeof(int64_t) * (size_t)(items + 1));
    int64_t* item_r = (int64_t*)malloc(sizeof(int64_t) * (size_t)(items + 1));
    int64_t q = 0;
    for (int e = 0; e < E; ++e)
        for (int r0 = 0; r0 < counts[e]; r0 += RB) { item_e[q] = e; item_r[q] = r0; ++q; }
    #pragma omp parallel for schedule(dynamic, 1)
    for (int64_t it = 0; it < items; ++it) {
        int e = (int)item_e[it];
        int r0 = (int)item_r[it];
        int rows = counts[e] - r0 < RB ? counts[e] - r0 : RB;
        const int32_t* sl = slots + offsets[e] + r0;
        int32_t* keep = (int32_t*)malloc(sizeof(int32_t) * (size_t)rows);
        int n = 0;
        for (int i = 0; i < rows; ++i)
            if (!token_mask || token_mask[sl[i] / K]) keep[n++] = sl[i];
        if (n) {
            float* xe = (float*)malloc(sizeof(float) * (size_t)n * H);
            float* we = (float*)malloc(sizeof(float) * (size_t)n);
            float* c = (float*)malloc(sizeof(float) * (size_t)n * H);
            for (int i = 0; i < n; ++i) {
                memcpy(xe + (size_t)i * H, x + (size_t)(keep[i] / K) * H, sizeof(float) * (size_t)H);
                we[i] = weights[keep[i]];
            }
            expert_rows(xe, n, H, I, gate_up + (size_t)e * 2 * I * H,
                        down + (size_t)e * H * I, we, act, bf16, c);
            for (int i = 0; i < n; ++i)
                memcpy(staged + (size_t)keep[i] * H, c + (size_t)i * H, sizeof(float) * (size_t)H);
            free(xe); free(we); free(c);
        }
        free(keep);
    }
    #pragma omp parallel for schedule(static)
    for (int t = 0; t < T; ++t) {
        if (token_mask && !token_mask[t]) continue;
        for (int h = 0; h < H; ++h) {
            float s = 0.f;
            for (int r = 0; r < K; ++r) s += staged[((size_t)t * K + r) * H + h];
            out[(size_t)t * H + h] = bf16 ? bf16_round(s) : s;
        }
    }
    free(item_e); free(item_r);
    free(counts); free(offsets); free(slots); free(staged);
    return 0;
}

/* Dense gated MLP over all rows (mlp.rs forward, used by the shared expert):
 * f32 mode act(x Wg^T) * (x Wu^T) then Wd; BF16 mode rounds gate_up, the
 * activation product and the down output once each. */
void oracle_dense_mlp(const float* x, int T, int H, int I,
                      const float* gate_up, const float* down, int act, int bf16,
                      float* out) {
    #pragma omp parallel for schedule(dynamic, 1)
    for (int t0 = 0; t0 < T; t0 += 32) {
        int n = T - t0 < 32 ? T - t0 : 32;
        expert_rows(x + (size_t)t0 * H, n, H, I, gate_up, down, NULL, act, bf16,
                    out + (size_t)t0 * H);
    }
}

/* The shared expert's gate, sigmoid(v) = 1 / (1 + exp(-v)) in f32
 * (candle's sigmoid op at shared_expert.rs:155), elementwise. */
void oracle_sigmoid(const float* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = 1.0f / (1.0f + expf(-in[i]));
}

/* Shared-expert combine, f32 CPU path (shared_expert.rs:68,142-159):
 * out = routed + shared * sigmoid(x . w_s), with the product and the sum
 * rounded separately.  gate_weight NULL means an ungated shared expert. */
void oracle_shared_combine_f32(const float* x, const float* gate_weight,
                               const float* shared, const float* routed,
                               float* out, int T, int H) {
    for (int t = 0; t < T; ++t) {
        float g = 1.0f;
        if (gate_weight) {
            float dot[1];
            gemm_nt(x + (size_t)t * H, H, gate_weight, H, dot, 1, 1, 1, H);
            g = 1.0f / (1.0f + expf(-dot[0]));
        }
        for (int h = 0; h < H; ++h) {
            float s = shared[(size_t)t * H + h];
            if (gate_weight) s = s * g;
            out[(size_t)t * H + h] = routed[(size_t)t * H + h] + s;
        }
    }
}

/* Shared-expert combine, BF16 contract (moe_shared.cu:17-36):
 * out = bf16(fma(sigmoid(x . w_s), shared, routed)), the dot in f32. */
void oracle_shared_combine_bf16(const float* x, const float* gate_weight,
                                const float* shared, const float* routed,
                                float* out, int T, int H) {
    for (int t = 0; t < T; ++t) {
        float dot[1];
        gemm_nt(x + (size_t)t * H, H, gate_weight, H, dot, 1, 1, 1, H);
        float g = 1.0f / (1.0f + expf(-dot[0]));
        for (int h = 0; h < H; ++h)
            out[(size_t)t * H + h] =
                bf16_round(fmaf(g, shared[(size_t)t * H + h], routed[(size_t)t * H + h]));
    }
}

/* silu_and_mul (silu_and_mul.cu:51-76): packed rows [gate..., up...];
 * out = (g / (1 + exp(-g))) * u in f32, rounded to BF16 once when bf16. */
void oracle_silu_and_mul(const float* in, float* out, int rows, int columns, int bf16) {
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < columns; ++c) {
            float g = in[(size_t)r * 2 * columns + c];
            float u = in[(size_t)r * 2 * columns + columns + c];
            float v = (g / (1.0f + expf(-g))) * u;
            out[(size_t)r * columns + c] = bf16 ? bf16_round(v) : v;
        }
}

/* Centered RMSNorm, the f32 CPU path of CenteredRmsNorm (rms_norm.rs:107-150;
 * normalize_in_f32 at :204-210): per row, sum of squares in f32 (each square
 * rounded, then a sequential sum), mean = sum / cols, inv = 1 / sqrt(mean + eps),
 * y = (x * inv) * (1 + w), rounded to BF16 when bf16.  With a branch, the row
 * is first input + branch rounded in the storage dtype (the unfused pair of
 * rms_norm.rs:66-74, a Candle add in that dtype), written to residual_out. */
void oracle_centered_rms_norm(const float* input, const float* branch, const float* weight,
                              float* residual_out, float* out, int rows, int cols, float eps, int bf16) {
    float* row = (float*)malloc(sizeof(float) * (size_t)cols);
    for (int r = 0; r < rows; ++r) {
        const size_t o = (size_t)r * cols;
        for (int c = 0; c < cols; ++c) {
            float v = input[o + c];
            if (branch) {
                v = v + branch[o + c];
                if (bf16) v = bf16_round(v);
            }
            row[c] = v;
            if (residual_out) residual_out[o + c] = v;
        }
        float ss = 0.0f;
        for (int c = 0; c < cols; ++c) {
            const float sq = row[c] * row[c];
            ss = ss + sq;
        }
        const float inv = 1.0f / sqrtf(ss / (float)cols + eps);
        for (int c = 0; c < cols; ++c) {
            const float y = (row[c] * inv) * (1.0f + weight[c]);
            out[o + c] = bf16 ? bf16_round(y) : y;
        }
    }
    free(row);
}
