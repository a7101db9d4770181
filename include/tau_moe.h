/*
 * tau_moe.h -- C ABI of libtau_moe_hip.so, the MI355X (gfx950) MoE expert-FFN
 * path: router softmax/top-k, stable expert-major dispatch, grouped gate_up
 * GEMM with fused SiLU·mul, grouped down GEMM with the route-weight epilogue,
 * and the rank-ordered combine.
 *
 * Conventions (all entry points):
 *   - device pointers, plain ints; `stream` is a hipStream_t passed as void*
 *     (NULL = the default stream);
 *   - launches are asynchronous on `stream`, never allocate, synchronise or
 *     read back, and keep no global state (callers may serialise on one
 *     workspace the way the reference's owners do with a mutex);
 *   - return 0 on successful enqueue, 1 (hipErrorInvalidValue, same value as
 *     the reference's cudaErrorInvalidValue) for rejected arguments, otherwise
 *     the hipGetLastError() code; the fused single-token decode returns -1 for
 *     argument errors as its reference counterpart does;
 *   - data errors (non-finite logits, malformed routes) never fail a launch:
 *     they set the plan's status word and every output element becomes NaN;
 *   - BF16 tensors are raw uint16 bit patterns; routes are f32 [T, 2K]
 *     (K expert ids stored as floats, then K weights, renormalised unless
 *     TAU_MOE_ROUTE_RAW_WEIGHTS is set); meta is int32 [2E+2] = counts[E],
 *     cursors[E], status, padded row total.
 *
 * Reference interfaces replaced (paths relative to the tau.rs root):
 *   crates/cuda-kernels/src/cuda_ffi.rs (declarations) and the CUDA
 *   definitions under crates/cuda-kernels/src/kernels/.  The reference entry
 *   points fix E = 256 and K = 8; the *_ex entry points take E and K.
 */
#ifndef TAU_MOE_H
#define TAU_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Expert weight layouts accepted by the *_ex entry points.
 *   ROW_MAJOR: W[e][n][k] as the reference stores it (gate_up [E,2I,H],
 *              down [E,H,I]).
 *   FRAG16:    the same values regrouped by tau_moe_pack_weights into 1 KB
 *              MFMA operand fragments: 16-byte piece p of expert e holds row
 *              16*b + (p%64)%16, columns 32*c + 8*((p%64)/16) .. +8, where
 *              p = (b*(k/32) + c)*64 + lane.  Needs n % 16 == 0 and
 *              k % 64 == 0; every weight stream then reads whole 1 KB
 *              contiguous fragments. */
#define TAU_MOE_WEIGHTS_ROW_MAJOR 0
#define TAU_MOE_WEIGHTS_FRAG16 1

/* repr(C) tile words of crates/cuda-kernels/src/moe/config.rs:12-20. */
typedef struct TauGemmTile { int m, n, k, warps, stages; } TauGemmTile;
/* repr(C) profile words of crates/cuda-kernels/src/moe/decode_config.rs:10-18. */
typedef struct TauDecodeProfile { int backend, n, k, warps, stages; } TauDecodeProfile;

/* ---------------- reference-compatible entry points (E=256, K=8) ---------------- */

/* Replaces tau_launch_moe_routing_fp32 (cuda_ffi.rs:81-86; moe_routing.cu:56-61).
 * logits: BF16 [rows, 256]; routes: f32 [rows, 16]. */
int tau_launch_moe_routing_fp32(const void* logits, float* routes, int rows, void* stream);

/* Replaces tau_launch_moe_prefill_dispatch (cuda_ffi.rs:33-43; moe_dispatch.cu:88-104).
 * meta [514], offsets [257], slots [capacity], tiles [capacity/tile_rows].
 * tile_rows in {16, 32, 64, 128, 256}; capacity >= tau_moe_prefill_capacity(...).
 * The permutation is stable (token-ascending inside each expert). */
int tau_launch_moe_prefill_dispatch(const float* routes, int* meta, int* offsets, int* slots, int* tiles,
                                    int tokens, int capacity, int tile_rows, void* stream);

/* Replaces tau_launch_moe_prefill_combine (moe_dispatch.cu:107-114).
 * contributions BF16 [rows*8, width] -> output BF16 [rows, width]. */
int tau_launch_moe_prefill_combine(const void* contributions, void* output, const int* meta, int rows,
                                   int width, void* stream);

/* Replaces tau_launch_moe_prefill_gemm (moe_gemm.cuh:18-20; moe_gemm.cu:185-200).
 * down == 0: output[row, :n] = bf16(x[slot/8] . W_e^T), zeros on padding rows.
 * down == 1: output[slot, :n] = bf16((input[row] . W_e^T) * w[slot]).
 * cfg->m selects the row block (it must equal the dispatch tile_rows); the
 * other words are validated against the reference catalog and the executed
 * CDNA4 tile is stamped into receipt[0..4] when receipt is non-null. */
int tau_launch_moe_prefill_gemm(const void* input, const void* weights, const float* routes, const int* slots,
                                const int* tiles, void* output, int tokens, int capacity, int n, int k, int down,
                                const TauGemmTile* cfg, int* receipt, void* stream);

/* Replaces tau_launch_moe_prefill (cuda_ffi.rs:45-67; moe_prefill.cu:15-38).
 * input BF16 [T,H], logits BF16 [T,256], gate_up BF16 [256,2I,H] (gate rows
 * first), down BF16 [256,H,I]; activated BF16 [capacity, I]; contributions
 * BF16 [T*8, H]; output BF16 [T, H].  `projected` is accepted but not written:
 * SiLU·mul is fused into the gate_up epilogue with the same rounding points. */
int tau_launch_moe_prefill(const void* input, const void* logits, const void* gate_up, const void* down,
                           float* routes, int* meta, int* offsets, int* slots, int* tiles, void* projected,
                           void* activated, void* contributions, void* output, int tokens, int hidden,
                           int intermediate, int capacity, const TauGemmTile* gate_up_config,
                           const TauGemmTile* down_config, int* receipts, void* stream);

/* Replaces tau_launch_silu_and_mul (cuda_ffi.rs:247-254; silu_and_mul.cu:81-132).
 * dtype 0 = f32, 1 = BF16; input [rows, 2*columns] -> output [rows, columns]. */
int tau_launch_silu_and_mul(const void* input, void* output, int rows, int columns, int dtype, void* stream);

/* Replaces tau_launch_moe_shared_combine (cuda_ffi.rs:70-79; moe_shared.cu:41-54).
 * output = bf16(fma(sigmoid(input . weight), shared, routed)); width <= 8192. */
int tau_launch_moe_shared_combine(const void* input, const void* weight, const void* shared, const void* routed,
                                  void* output, int rows, int width, void* stream);

/* Replaces tau_launch_linear_bf16_fp32 (cuda_ffi.rs:88-96; linear_bf16_fp32.cu:102-110).
 * output f32 [rows, columns] = input BF16 [rows, inner] . weight BF16 [columns, inner]^T. */
int tau_launch_linear_bf16_fp32(const void* input, const void* weight, float* output, int rows, int columns,
                                int inner, void* stream);

/* Replaces tau_launch_moe_decode_gemm (cuda_ffi.rs:20-30; moe_decode_gemm.cu:125-147).
 * Device pointer arrays: inputs[b] BF16 [inner], weights[b] BF16 [columns, inner],
 * outputs[b] f32 [columns]. */
int tau_launch_moe_decode_gemm(const void* inputs, const void* weights, void* outputs, int batches, int columns,
                               int inner, const TauDecodeProfile* config, int* receipts, void* stream);

/* Replaces tau_launch_fused_bf16_moe_decode (cuda_ffi.rs:266-288;
 * fused_bf16_moe_decode.cu:56-91): one token, routing through the rank-ordered
 * combine.  Buffers: selected_ids int32 [8], selected_weights f32 [8],
 * pointer_workspace >= 64 bytes, gate_up_output BF16 [8,2I], activated_output
 * BF16 [8,I], expert_output BF16 [8,H], gate_up_fp32 f32 [8,2I], expert_fp32
 * f32 [8,H], output BF16 [H].  Returns -1 for argument errors. */
int tau_launch_fused_bf16_moe_decode(const void* input, const void* logits, const void* gate_up,
                                     const void* down, void* selected_ids, void* selected_weights,
                                     void* pointer_workspace, void* gate_up_output, void* activated_output,
                                     void* expert_output, void* gate_up_fp32, void* expert_fp32, void* output,
                                     int hidden, int intermediate, int num_experts, int top_k,
                                     const TauDecodeProfile* gate_up_config, const TauDecodeProfile* down_config,
                                     int* receipts, void* stream);

/* ---------------- generalised entry points (any E <= 512, K <= 32; the layer
 * entry points take E + 1 <= 513 experts from given routes when a shared expert
 * is folded in) ---------------- */

/* Capacity of the padded dispatch, generalising moe_prefill_capacity_for_tile
 * (crates/cuda-kernels/src/moe/prefill.rs:17-30); -1 for invalid input. */
int64_t tau_moe_prefill_capacity(int tokens, int experts, int top_k, int tile_rows);

/* Row block chosen by the library for a routing shape: 16 selects the
 * weight-streaming decode kernels (16, 32), 64/128/256 the LDS-tiled MFMA kernels. */
int tau_moe_select_tile_rows(int tokens, int experts, int top_k, int hidden, int intermediate);

/* Workspace bytes for tau_launch_moe_prefill_ex, in argument order:
 * routes, meta, offsets, slots, tiles, activated, contributions. */
int tau_moe_workspace_bytes(int tokens, int hidden, int intermediate, int experts, int top_k, int tile_rows,
                            size_t out_bytes[7]);

/* Flag OR-ed into any logits_dtype argument: route weights are the selected
 * softmax probabilities as they are, not renormalised by their sum
 * (normalize_selected_weights = false; sparse_moe/config.rs:45,
 * sparse_moe/routing.rs:198-202).  Without it weights are renormalised. */
#define TAU_MOE_ROUTE_RAW_WEIGHTS 0x100

/* Router softmax/top-k; logits_dtype 0 = f32, 1 = BF16 (| TAU_MOE_ROUTE_RAW_WEIGHTS);
 * routes f32 [T, 2K].  Experts are ranked on their f32 softmax probabilities
 * (exp with glibc expf's results, the sum in expert order), larger first and
 * the lower id on equal probabilities, as routing.rs:125-257. */
int tau_launch_moe_routing_ex(const void* logits, int logits_dtype, float* routes, int tokens, int experts,
                              int top_k, void* stream);

/* Dispatch; when `logits` is non-null routing runs first (inside the dispatch
 * workgroup for tokens <= 256).  meta [2E+2], offsets [E+1]. */
int tau_launch_moe_prefill_dispatch_ex(const void* logits, int logits_dtype, float* routes, int* meta,
                                       int* offsets, int* slots, int* tiles, int tokens, int experts, int top_k,
                                       int tile_rows, int capacity, void* stream);

/* Rank-ordered combine: output[t] = bf16(sum_r contributions[t*K + r]); with a
 * residual (BF16 [T,H], may be NULL) output = bf16(f32(that) + residual), the
 * layer's residual add (qwen3_5_common/decoder.rs:96-116) fused. */
int tau_launch_moe_prefill_combine_ex(const void* contributions, void* output, const int* meta, int tokens,
                                      int hidden, int experts, int top_k, const void* residual, void* stream);

/* Whole routed path for any (E, K): routing, dispatch, gate_up+SiLU·mul,
 * down+weight, combine.  logits NULL: `routes` already holds the [T, 2K]
 * routes (tau_launch_moe_router_route_ex, or E+1 experts and K+1 picks from
 * tau_launch_moe_routing_shared_ex) and routing is skipped.  tile_rows from
 * tau_moe_select_tile_rows (or any of
 * 16/32/64/128/256); weight_layout TAU_MOE_WEIGHTS_* for both weight tensors;
 * residual (may be NULL) is added in the combine as above (pass it here only
 * when no shared expert follows); receipts (optional) receive 10 words,
 * gate_up then down. */
int tau_launch_moe_prefill_ex(const void* input, const void* logits, int logits_dtype, const void* gate_up,
                              const void* down, float* routes, int* meta, int* offsets, int* slots, int* tiles,
                              void* activated, void* contributions, void* output, int tokens, int hidden,
                              int intermediate, int experts, int top_k, int tile_rows, int capacity,
                              int weight_layout, const void* residual, int* receipts, void* stream);

/* One grouped projection over an existing dispatch (meta/slots/tiles from
 * tau_launch_moe_prefill_dispatch_ex with the same tile_rows):
 * projection 0: a = input x [T,H], w = gate_up [E,2I,H], out = activated [cap,I]
 *               (bf16(silu(bf16(g)) * bf16(u)));
 * projection 1: a = activated [cap,I], w = down [E,H,I], out = contributions
 *               [T*K,H] (bf16(acc * w_route) at each assignment's slot). */
int tau_launch_moe_grouped_gemm_ex(const void* a, const void* w, const float* routes, const int* slots,
                                   const int* tiles, const int* meta, void* out, int tokens, int hidden,
                                   int intermediate, int experts, int top_k, int tile_rows, int capacity,
                                   int projection, int weight_layout, int* receipt, void* stream);

/* One projection of the fused decode path (tokens <= 64, E <= 256,
 * tile_rows 16) from existing routes, exactly the launch that
 * tau_launch_moe_prefill_ex issues for it: projection 0 = gate_up + SiLU·mul
 * (a = x [T,H], w = gate_up, out = activated [T*K, I], rows by assignment
 * t*K + r); projection 1 = down + route weight (a = activated, w = down, out =
 * contributions [T*K, H]) whose extra workgroup builds meta/offsets/slots/tiles
 * (required for projection 1; capacity as for tile_rows 16).  The reference's
 * decode projections are `project` in moe_decode_gemm.cu:47-85 (launched per
 * expert from fused_bf16_moe_decode.cu:56-91); this entry point exists so that
 * a caller can time or run the decode projections apart. */
int tau_launch_moe_decode_projection_ex(const void* a, const void* w, float* routes, int* meta, int* offsets,
                                        int* slots, int* tiles, void* out, int tokens, int hidden, int intermediate,
                                        int experts, int top_k, int capacity, int projection, int weight_layout,
                                        int* receipt, void* stream);

/* Always-on shared expert (shared_expert.rs:39-69): dense gated MLP over all
 * tokens with gate_up_s BF16 [2Is,H], down_s BF16 [Is,H]^T = [H,Is], then
 * output = bf16(fma(sigmoid(x . gate_weight), shared, routed)) (gate_weight
 * may be NULL for an ungated expert).  activated_ws BF16 [T,Is], shared_ws
 * BF16 [T,H].  `output` may alias `routed`.  residual (BF16 [T,H], may be NULL):
 * output = bf16(f32(bf16(fma(...))) + residual), the fused residual add. */
int tau_launch_moe_shared_expert_ex(const void* input, const void* gate_up_s, const void* down_s,
                                    const void* gate_weight, const void* routed, void* activated_ws,
                                    void* shared_ws, void* output, int tokens, int hidden,
                                    int shared_intermediate, int weight_layout, const void* residual,
                                    void* stream);

/* Router projection (routing.rs:91-93, Router::logits; bias of config.rs:37-78):
 * logits f32 [T, E] = input BF16 [T, H] . weight BF16 [E, H]^T (+ bias f32 [E],
 * may be NULL), f32 accumulation, the bias added once after the projection.
 * Feeds the *_ex entry points with logits_dtype 0. */
int tau_launch_moe_router_ex(const void* input, const void* weight, const float* bias, float* logits, int tokens,
                             int hidden, int experts, void* stream);

/* Replaces tau_launch_fused_residual_rms_norm (cuda_ffi.rs:210-222;
 * centered_rms_norm.cu:545-565): the decoder layer's post-attention residual
 * add and centered RMSNorm in front of the MoE block (decoder.rs:103-116).
 * residual_output = input + branch rounded in the storage dtype;
 * output = (residual * 1/sqrt(mean(residual^2) + epsilon)) * (1 + weight), f32
 * arithmetic, rounded once.  input/branch/residual_output/output [rows, columns],
 * weight [columns]; dtype 0 = f32, 1 = BF16; epsilon > 0 and finite;
 * preferred_bytes 0, 4, 8 or 16 caps the access width (results do not depend
 * on it).  Inputs are not modified; the outputs must not overlap them (input
 * and branch may be the same buffer). */
int tau_launch_fused_residual_rms_norm(const void* input, const void* branch, const void* weight,
                                       void* residual_output, void* output, int rows, int columns, float epsilon,
                                       int dtype, void* stream, int preferred_bytes);

/* Replaces tau_launch_centered_rms_norm_configured (cuda_ffi.rs:231-241;
 * centered_rms_norm.cu:445-508): the same normalization without the add. */
int tau_launch_centered_rms_norm_configured(const void* input, const void* weight, void* output, int rows,
                                            int columns, float epsilon, int dtype, void* stream,
                                            int preferred_bytes);

/* Replaces tau_launch_centered_rms_norm (centered_rms_norm.cu:511-516): the
 * configured form with preferred_bytes = 16. */
int tau_launch_centered_rms_norm(const void* input, const void* weight, void* output, int rows, int columns,
                                 float epsilon, int dtype, void* stream);

/* Router projection and routing in one call, replacing Router::logits
 * followed by the routing kernel (sparse_moe/routing.rs:91-93,125-231;
 * moe_routing.cu:15-52 generalised to any E <= 512, K <= 32): logits f32
 * [T, E] = input BF16 [T, H] . weight BF16 [E, H]^T (+ bias f32 [E], may be
 * NULL), exactly as tau_launch_moe_router_ex, into `logits` (required), then
 * softmax / top-K / renormalised weights into routes [T, 2K] as
 * tau_launch_moe_routing_ex does from those logits.  Two launches (projection
 * with the bias fused; routing). */
int tau_launch_moe_router_route_ex(const void* input, const void* weight, const float* bias, float* logits,
                                   float* routes, int tokens, int hidden, int experts, int top_k, void* stream);

/* The always-on shared expert folded into the routed schedule (the
 * shared-expert branch of SparseMoeBlock::forward_routed, sparse_moe.rs:102-151,
 * and SharedExpert::combine, shared_expert.rs:39-69, run as one more expert):
 * logits f32/BF16 [T, E+1] hold the E router logits then the shared gate logit
 * x . w_s; routes [T, 2(K+1)] get the routed top-K at ranks 0..K-1 exactly as
 * tau_launch_moe_routing_ex writes them and (id E, weight sigmoid(gate)) at
 * rank K.  With expert E's weights appended to the banks (gate_up
 * [E+1, 2I, H], down [E+1, H, I]; requires the shared intermediate size = I),
 * tau_launch_moe_prefill_ex(logits = NULL, experts = E+1, top_k = K+1)
 * computes routed + sigmoid(x . w_s) * shared(x) in one grouped schedule
 * (contributions summed in f32 in rank order, rounded once). */
int tau_launch_moe_routing_shared_ex(const void* logits, int logits_dtype, float* routes, int tokens, int experts,
                                     int top_k, void* stream);

/* The same from hidden states: weight BF16 [E+1, H] = router rows then w_s,
 * bias f32 [E+1] (may be NULL; the shared gate has none, so bias[E] = 0),
 * logits f32 [T, E+1] (required), then the routing above. */
int tau_launch_moe_router_route_shared_ex(const void* input, const void* weight, const float* bias, float* logits,
                                          float* routes, int tokens, int hidden, int experts, int top_k,
                                          void* stream);

/* Load-time weight preparation (no reference counterpart: the reference's
 * kernels read its packed [E, n, k] storage directly, sparse_moe/experts.rs:
 * 50-90).  Writes the FRAG16 form of row-major src [experts, rows, columns]
 * into dst (same size, must not overlap).  rows % 16 == 0, columns % 64 == 0. */
int tau_moe_pack_weights(const void* src, void* dst, int experts, int rows, int columns, void* stream);

/* Library identification: gfx target the code objects were built for. */
const char* tau_moe_build_target(void);

#ifdef __cplusplus
}
#endif

#endif /* TAU_MOE_H */
