// extern "C" boundary of the MoE expert-FFN path (declared in include/tau_moe.h).
//
// Each entry point validates its arguments on the host, then enqueues the
// CDNA4 kernels on the caller's stream.  The composition mirrors the
// reference's stateless prefill composer (crates/cuda-kernels/src/kernels/
// moe_prefill.cu:15-38): routing -> dispatch -> gate_up -> down -> combine, with
// SiLU·mul folded into the gate_up epilogue and routing folded into the
// dispatch workgroup for decode-sized batches.
#include <climits>

#include "kernels.hpp"

namespace tau_amd {
int launch_silu_and_mul(const void* in, void* out, int rows, int columns, int dtype, hipStream_t s);
int launch_shared_combine(const void* x, const void* w, const void* shared, const void* routed, void* out,
                          int rows, int width, const void* residual, hipStream_t s);
bool router_logits_supported(const void* x, const void* w, int hidden, int experts);
int launch_router_logits(const void* input, const void* weight, const float* bias, float* logits, int tokens,
                         int hidden, int experts, hipStream_t s);
int launch_residual_norm(const void* input, const void* branch, const void* weight, void* residual_out, void* out,
                         int rows, int columns, float eps, int dtype, int preferred_bytes, hipStream_t s);
}  // namespace tau_amd

using namespace tau_amd;

namespace {

constexpr int kRefExperts = 256;
constexpr int kRefTopK = 8;
constexpr int kMaxTokens = 1 << 20;

inline hipStream_t as_stream(void* s) { return (hipStream_t)s; }

// The reference catalog of prefill tiles (crates/cuda-kernels/src/moe/config.rs:38-76).
bool reference_tile_ok(const TauGemmTile* c) {
    if (!c) return false;
    const bool m = c->m == 16 || c->m == 32 || c->m == 64 || c->m == 128 || c->m == 256;
    const bool n = c->n == 16 || c->n == 32 || c->n == 64 || c->n == 128;
    const bool k = c->k == 16 || c->k == 32 || c->k == 64 || c->k == 128;
    const bool w = c->warps == 1 || c->warps == 2 || c->warps == 4 || c->warps == 8;
    const bool s = c->stages == 1 || c->stages == 2;
    return m && n && k && w && s;
}

GemmArgs gate_up_args(const void* input, const void* gate_up, const float* routes, const int* slots,
                      const int* tiles, const int* meta_total, void* out, int tokens, int top_k, int capacity,
                      int hidden, int intermediate, int* receipt, int weight_layout) {
    GemmArgs g{};
    g.w_layout = weight_layout;
    g.a = (const uint16_t*)input;
    g.w = (const uint16_t*)gate_up;
    g.routes = routes;
    g.slots = slots;
    g.tiles = tiles;
    g.meta_total = meta_total;
    g.out = out;
    g.rows = capacity;
    g.assignments = tokens * top_k;
    g.topk = top_k;
    g.n = intermediate;
    g.k = hidden;
    g.lda = hidden;
    g.ldo = intermediate;
    g.w_expert_stride = (long)2 * intermediate * hidden;
    g.w_up_offset = intermediate;
    g.receipt = receipt;
    return g;
}

GemmArgs down_args(const void* activated, const void* down, const float* routes, const int* slots,
                   const int* tiles, const int* meta_total, void* contributions, int tokens, int top_k,
                   int capacity, int hidden, int intermediate, int* receipt, int weight_layout) {
    GemmArgs g{};
    g.w_layout = weight_layout;
    g.a = (const uint16_t*)activated;
    g.w = (const uint16_t*)down;
    g.routes = routes;
    g.slots = slots;
    g.tiles = tiles;
    g.meta_total = meta_total;
    g.out = contributions;
    g.rows = capacity;
    g.assignments = tokens * top_k;
    g.topk = top_k;
    g.n = hidden;
    g.k = intermediate;
    g.lda = intermediate;
    g.ldo = hidden;
    g.w_expert_stride = (long)hidden * intermediate;
    g.w_up_offset = 0;
    g.receipt = receipt;
    return g;
}

// Up to 512 routed experts, plus one when a shared expert is folded in as
// expert E (its routes come from tau_launch_moe_routing_shared_ex).
constexpr int kMaxLayerExperts = 513;

bool shape_ok(int tokens, int hidden, int intermediate, int experts, int top_k) {
    return tokens > 0 && tokens <= kMaxTokens && hidden > 0 && intermediate > 0 && intermediate <= INT_MAX / 2 &&
           experts > 0 && experts <= kMaxLayerExperts && top_k > 0 && top_k <= 32 && top_k <= experts &&
           (int64_t)tokens * top_k * hidden <= (int64_t)1 << 40;
}

// Frag16 weights need 16-row bands (gate, up and down rows) and K in whole
// 64-wide MFMA steps for every projection of the layer.
bool layout_ok(int weight_layout, int hidden, int intermediate) {
    if (weight_layout == TAU_MOE_WEIGHTS_ROW_MAJOR) return true;
    return weight_layout == TAU_MOE_WEIGHTS_FRAG16 && hidden % 64 == 0 && intermediate % 64 == 0;
}

}  // namespace

extern "C" {

int tau_launch_moe_router_route_ex(const void* input, const void* weight, const float* bias, float* logits,
                                   float* routes, int tokens, int hidden, int experts, int top_k, void* stream) {
    if (!routes || top_k <= 0 || top_k > 32 || top_k > experts) return kInvalid;
    const int code = tau_launch_moe_router_ex(input, weight, bias, logits, tokens, hidden, experts, stream);
    if (code) return code;
    return launch_routing(logits, 0, routes, tokens, experts, top_k, as_stream(stream));
}

int tau_launch_moe_routing_shared_ex(const void* logits, int logits_dtype, float* routes, int tokens, int experts,
                                     int top_k, void* stream) {
    if (tokens <= 0 || tokens > kMaxTokens) return kInvalid;
    return launch_routing_shared(logits, logits_dtype, routes, tokens, experts, top_k, as_stream(stream));
}

int tau_launch_moe_router_route_shared_ex(const void* input, const void* weight, const float* bias, float* logits,
                                          float* routes, int tokens, int hidden, int experts, int top_k,
                                          void* stream) {
    if (!routes || experts <= 0 || experts > 512 || top_k <= 0 || top_k + 1 > 32 || top_k > experts)
        return kInvalid;
    const int code = tau_launch_moe_router_ex(input, weight, bias, logits, tokens, hidden, experts + 1, stream);
    if (code) return code;
    return launch_routing_shared(logits, 0, routes, tokens, experts, top_k, as_stream(stream));
}

int tau_launch_moe_router_ex(const void* input, const void* weight, const float* bias, float* logits, int tokens,
                             int hidden, int experts, void* stream) {
    if (!input || !weight || !logits || tokens <= 0 || tokens > kMaxTokens || hidden <= 0 || experts <= 0 ||
        experts > kMaxLayerExperts)
        return kInvalid;
    if (router_logits_supported(input, weight, hidden, experts))  // skinny-GEMM kernel, bias fused
        return launch_router_logits(input, weight, bias, logits, tokens, hidden, experts, as_stream(stream));
    const int code = tau_launch_linear_bf16_fp32(input, weight, logits, tokens, experts, hidden, stream);
    if (code || !bias) return code;
    return launch_add_bias(logits, bias, tokens, experts, as_stream(stream));
}

int tau_moe_pack_weights(const void* src, void* dst, int experts, int rows, int columns, void* stream) {
    if (!src || !dst || src == dst || experts <= 0 || rows <= 0 || columns <= 0 || rows % 16 || columns % 64 ||
        (long)experts * rows * columns / 8 > INT_MAX)
        return kInvalid;
    return launch_pack_frag16(src, dst, experts, rows, columns, as_stream(stream));
}

const char* tau_moe_build_target(void) { return "gfx950"; }

int64_t tau_moe_prefill_capacity(int tokens, int experts, int top_k, int tile_rows) {
    if (tokens <= 0 || tokens > kMaxTokens || experts <= 0 || top_k <= 0 || top_k > experts ||
        !gemm_rows_supported(tile_rows))
        return -1;
    return capacity_for(tokens, experts, top_k, tile_rows);
}

int tau_moe_select_tile_rows(int tokens, int experts, int top_k, int hidden, int intermediate) {
    (void)hidden;
    (void)intermediate;
    if (tokens <= 0 || experts <= 0 || top_k <= 0) return 16;
    const double rows_per_expert = (double)tokens * top_k / experts;
    // Measured on MI355X over balanced (30B-A3B, 235B-A22B) and skewed (biased,
    // Zipf) routing, 128..8192 tokens: decode batches (<= 64 tokens, the fused
    // decode path) and <= 8 rows per expert stream weights in 16-row groups;
    // <= 16 rows, 32-row groups; <= 32 rows, 128-row MFMA tiles; beyond, 256-row
    // MFMA tiles (whose all-padding wave rows skip their MFMAs), which skewed
    // routing prefers from ~32 rows per expert on.
    if (tokens <= 64 || rows_per_expert <= 8.0) return 16;
    if (rows_per_expert <= 16.0) return 32;
    if (rows_per_expert <= 32.0) return 128;
    return 256;
}

int tau_moe_workspace_bytes(int tokens, int hidden, int intermediate, int experts, int top_k, int tile_rows,
                            size_t out_bytes[7]) {
    if (!out_bytes || !shape_ok(tokens, hidden, intermediate, experts, top_k) || !gemm_rows_supported(tile_rows))
        return kInvalid;
    const int64_t cap = capacity_for(tokens, experts, top_k, tile_rows);
    out_bytes[0] = sizeof(float) * (size_t)tokens * 2 * top_k;
    out_bytes[1] = sizeof(int) * (size_t)(2 * experts + 2);
    out_bytes[2] = sizeof(int) * (size_t)(experts + 1);
    out_bytes[3] = sizeof(int) * (size_t)cap;
    out_bytes[4] = sizeof(int) * (size_t)(cap / tile_rows);
    out_bytes[5] = 2 * (size_t)cap * intermediate;
    out_bytes[6] = 2 * (size_t)tokens * top_k * hidden;
    return 0;
}

int tau_launch_moe_routing_ex(const void* logits, int logits_dtype, float* routes, int tokens, int experts,
                              int top_k, void* stream) {
    if (tokens > kMaxTokens) return kInvalid;
    return launch_routing(logits, logits_dtype, routes, tokens, experts, top_k, as_stream(stream));
}

int tau_launch_moe_routing_fp32(const void* logits, float* routes, int rows, void* stream) {
    if (!logits || !routes || rows <= 0) return kInvalid;
    return tau_launch_moe_routing_ex(logits, 1, routes, rows, kRefExperts, kRefTopK, stream);
}

int tau_launch_moe_prefill_dispatch_ex(const void* logits, int logits_dtype, float* routes, int* meta,
                                       int* offsets, int* slots, int* tiles, int tokens, int experts, int top_k,
                                       int tile_rows, int capacity, void* stream) {
    if (tokens <= 0 || tokens > kMaxTokens || !gemm_rows_supported(tile_rows)) return kInvalid;
    return launch_dispatch(logits, logits_dtype, routes, meta, offsets, slots, tiles, tokens, experts, top_k,
                           tile_rows, capacity, nullptr, 0, as_stream(stream));
}

int tau_launch_moe_prefill_dispatch(const float* routes, int* meta, int* offsets, int* slots, int* tiles,
                                    int tokens, int capacity, int tile_rows, void* stream) {
    if (tokens <= 0 || tokens > 65535) return kInvalid;
    return tau_launch_moe_prefill_dispatch_ex(nullptr, 0, (float*)routes, meta, offsets, slots, tiles, tokens,
                                              kRefExperts, kRefTopK, tile_rows, capacity, stream);
}

int tau_launch_moe_prefill_combine_ex(const void* contributions, void* output, const int* meta, int tokens,
                                      int hidden, int experts, int top_k, const void* residual, void* stream) {
    if (!meta || experts <= 0 || top_k <= 0 || tokens > kMaxTokens) return kInvalid;
    return launch_combine(contributions, output, meta + 2 * experts, tokens, hidden, top_k, residual,
                          as_stream(stream));
}

int tau_launch_moe_prefill_combine(const void* contributions, void* output, const int* meta, int rows,
                                   int width, void* stream) {
    if (rows <= 0 || rows > 65535) return kInvalid;
    return tau_launch_moe_prefill_combine_ex(contributions, output, meta, rows, width, kRefExperts, kRefTopK, nullptr,
                                             stream);
}

int tau_launch_moe_prefill_gemm(const void* input, const void* weights, const float* routes, const int* slots,
                                const int* tiles, void* output, int tokens, int capacity, int n, int k, int down,
                                const TauGemmTile* cfg, int* receipt, void* stream) {
    if (!reference_tile_ok(cfg) || !input || !weights || !routes || !slots || !tiles || !output || tokens <= 0 ||
        tokens > 65535 || capacity <= 0 || n <= 0 || k <= 0 || (down != 0 && down != 1) || capacity % cfg->m)
        return kInvalid;
    GemmArgs g{};
    g.a = (const uint16_t*)input;
    g.w = (const uint16_t*)weights;
    g.routes = routes;
    g.slots = slots;
    g.tiles = tiles;
    g.meta_total = nullptr;
    g.out = output;
    g.rows = capacity;
    g.assignments = tokens * kRefTopK;
    g.topk = kRefTopK;
    g.n = n;
    g.k = k;
    g.lda = k;
    g.ldo = n;
    g.w_expert_stride = (long)n * k;
    g.receipt = receipt;
    if (down) return launch_grouped_gemm(g, cfg->m, kADirect, kEpiScatterWeighted, as_stream(stream));
    return launch_grouped_gemm(g, cfg->m, kAGather, kEpiStoreBf16, as_stream(stream));
}

int tau_launch_moe_prefill_ex(const void* input, const void* logits, int logits_dtype, const void* gate_up,
                              const void* down, float* routes, int* meta, int* offsets, int* slots, int* tiles,
                              void* activated, void* contributions, void* output, int tokens, int hidden,
                              int intermediate, int experts, int top_k, int tile_rows, int capacity,
                              int weight_layout, const void* residual, int* receipts, void* stream) {
    if (!input || !gate_up || !down || !routes || !meta || !offsets || !slots || !tiles || !activated ||
        !contributions || !output || !shape_ok(tokens, hidden, intermediate, experts, top_k) ||
        !layout_ok(weight_layout, hidden, intermediate) ||
        (logits && (!logits_dtype_ok(logits_dtype) || experts > 512)) ||
        !gemm_rows_supported(tile_rows) || capacity < capacity_for(tokens, experts, top_k, tile_rows) ||
        capacity % tile_rows)
        return kInvalid;
    hipStream_t s = as_stream(stream);
    if (decode_path_supported(tokens, hidden, intermediate, experts, top_k, tile_rows, weight_layout))
        return launch_decode_moe(input, logits, logits_dtype, gate_up, down, routes, meta, offsets, slots, tiles,
                                 activated, contributions, output, tokens, hidden, intermediate, experts, top_k,
                                 capacity, weight_layout, residual, receipts, s);
    // The contributions buffer is free until the down projection: it holds the
    // multi-workgroup dispatch's per-chunk counts.
    int code = launch_dispatch(logits, logits_dtype, routes, meta, offsets, slots, tiles, tokens, experts, top_k,
                               tile_rows, capacity, contributions, (size_t)2 * tokens * top_k * hidden, s);
    if (code) return code;
    const int* total = meta + 2 * experts + 1;
    GemmArgs g = gate_up_args(input, gate_up, routes, slots, tiles, total, activated, tokens, top_k, capacity,
                              hidden, intermediate, receipts, weight_layout);
    code = launch_grouped_gemm(g, tile_rows, kAGather, kEpiSilu, s);
    if (code) return code;
    GemmArgs d = down_args(activated, down, routes, slots, tiles, total, contributions, tokens, top_k, capacity,
                           hidden, intermediate, receipts ? receipts + 5 : nullptr, weight_layout);
    code = launch_grouped_gemm(d, tile_rows, kADirect, kEpiScatterWeighted, s);
    if (code) return code;
    return launch_combine(contributions, output, meta + 2 * experts, tokens, hidden, top_k, residual, s);
}

int tau_launch_moe_grouped_gemm_ex(const void* a, const void* w, const float* routes, const int* slots,
                                   const int* tiles, const int* meta, void* out, int tokens, int hidden,
                                   int intermediate, int experts, int top_k, int tile_rows, int capacity,
                                   int projection, int weight_layout, int* receipt, void* stream) {
    if (!a || !w || !routes || !slots || !tiles || !meta || !out ||
        !shape_ok(tokens, hidden, intermediate, experts, top_k) || !gemm_rows_supported(tile_rows) ||
        !layout_ok(weight_layout, hidden, intermediate) ||
        capacity < capacity_for(tokens, experts, top_k, tile_rows) || capacity % tile_rows ||
        (projection != 0 && projection != 1))
        return kInvalid;
    const int* total = meta + 2 * experts + 1;
    if (projection == 0) {
        GemmArgs g = gate_up_args(a, w, routes, slots, tiles, total, out, tokens, top_k, capacity, hidden,
                                  intermediate, receipt, weight_layout);
        return launch_grouped_gemm(g, tile_rows, kAGather, kEpiSilu, as_stream(stream));
    }
    GemmArgs d = down_args(a, w, routes, slots, tiles, total, out, tokens, top_k, capacity, hidden, intermediate,
                           receipt, weight_layout);
    return launch_grouped_gemm(d, tile_rows, kADirect, kEpiScatterWeighted, as_stream(stream));
}

int tau_launch_moe_decode_projection_ex(const void* a, const void* w, float* routes, int* meta, int* offsets,
                                        int* slots, int* tiles, void* out, int tokens, int hidden, int intermediate,
                                        int experts, int top_k, int capacity, int projection, int weight_layout,
                                        int* receipt, void* stream) {
    return launch_decode_projection(a, w, routes, meta, offsets, slots, tiles, out, tokens, hidden, intermediate,
                                    experts, top_k, capacity, projection, weight_layout, receipt, as_stream(stream));
}

int tau_launch_moe_prefill(const void* input, const void* logits, const void* gate_up, const void* down,
                           float* routes, int* meta, int* offsets, int* slots, int* tiles, void* projected,
                           void* activated, void* contributions, void* output, int tokens, int hidden,
                           int intermediate, int capacity, const TauGemmTile* gate_up_config,
                           const TauGemmTile* down_config, int* receipts, void* stream) {
    (void)projected;
    if (!reference_tile_ok(gate_up_config) || !reference_tile_ok(down_config) ||
        gate_up_config->m != down_config->m || tokens <= 0 || tokens > 65535)
        return kInvalid;
    return tau_launch_moe_prefill_ex(input, logits, 1, gate_up, down, routes, meta, offsets, slots, tiles,
                                     activated, contributions, output, tokens, hidden, intermediate, kRefExperts,
                                     kRefTopK, gate_up_config->m, capacity, TAU_MOE_WEIGHTS_ROW_MAJOR, nullptr,
                                     receipts, stream);
}

int tau_launch_silu_and_mul(const void* input, void* output, int rows, int columns, int dtype, void* stream) {
    return launch_silu_and_mul(input, output, rows, columns, dtype, as_stream(stream));
}

int tau_launch_moe_shared_combine(const void* input, const void* weight, const void* shared, const void* routed,
                                  void* output, int rows, int width, void* stream) {
    if (!weight || width > 8192) return kInvalid;
    return launch_shared_combine(input, weight, shared, routed, output, rows, width, nullptr, as_stream(stream));
}

int tau_launch_linear_bf16_fp32(const void* input, const void* weight, float* output, int rows, int columns,
                                int inner, void* stream) {
    if (!input || !weight || !output || rows <= 0 || columns <= 0 || inner <= 0) return kInvalid;
    GemmArgs g{};
    g.a = (const uint16_t*)input;
    g.w = (const uint16_t*)weight;
    g.out = output;
    g.rows = rows;
    g.n = columns;
    g.k = inner;
    g.lda = inner;
    g.ldo = columns;
    g.w_expert_stride = 0;
    const int bm = rows <= 16 ? 16 : (rows <= 64 ? 64 : 128);
    return launch_grouped_gemm(g, bm, kADirect, kEpiStoreF32, as_stream(stream));
}

int tau_launch_moe_shared_expert_ex(const void* input, const void* gate_up_s, const void* down_s,
                                    const void* gate_weight, const void* routed, void* activated_ws,
                                    void* shared_ws, void* output, int tokens, int hidden,
                                    int shared_intermediate, int weight_layout, const void* residual,
                                    void* stream) {
    if (!input || !gate_up_s || !down_s || !routed || !activated_ws || !shared_ws || !output || tokens <= 0 ||
        tokens > kMaxTokens || hidden <= 0 || shared_intermediate <= 0 ||
        !layout_ok(weight_layout, hidden, shared_intermediate))
        return kInvalid;
    hipStream_t s = as_stream(stream);
    // Row blocks of the dense shared GEMMs: weight streaming for decode sizes,
    // then 128-row MFMA tiles (256-row tiles leave too few workgroups for a
    // dense GEMM of a few thousand tokens: measured slower at 2048).
    const int bm = tokens <= 16 ? 16 : (tokens <= 64 ? 64 : 128);
    GemmArgs g = gate_up_args(input, gate_up_s, nullptr, nullptr, nullptr, nullptr, activated_ws, tokens, 1,
                              tokens, hidden, shared_intermediate, nullptr, weight_layout);
    int code = launch_grouped_gemm(g, bm, kADirect, kEpiSilu, s);
    if (code) return code;
    GemmArgs d{};
    d.w_layout = weight_layout;
    d.a = (const uint16_t*)activated_ws;
    d.w = (const uint16_t*)down_s;
    d.out = shared_ws;
    d.rows = tokens;
    d.n = hidden;
    d.k = shared_intermediate;
    d.lda = shared_intermediate;
    d.ldo = hidden;
    code = launch_grouped_gemm(d, bm, kADirect, kEpiStoreBf16, s);
    if (code) return code;
    return launch_shared_combine(input, gate_weight, shared_ws, routed, output, tokens, hidden, residual, s);
}

int tau_launch_fused_residual_rms_norm(const void* input, const void* branch, const void* weight,
                                       void* residual_output, void* output, int rows, int columns, float epsilon,
                                       int dtype, void* stream, int preferred_bytes) {
    if (!branch || !residual_output) return kInvalid;
    return launch_residual_norm(input, branch, weight, residual_output, output, rows, columns, epsilon, dtype,
                                preferred_bytes, as_stream(stream));
}

int tau_launch_centered_rms_norm_configured(const void* input, const void* weight, void* output, int rows,
                                            int columns, float epsilon, int dtype, void* stream,
                                            int preferred_bytes) {
    return launch_residual_norm(input, nullptr, weight, nullptr, output, rows, columns, epsilon, dtype,
                                preferred_bytes, as_stream(stream));
}

int tau_launch_centered_rms_norm(const void* input, const void* weight, void* output, int rows, int columns,
                                 float epsilon, int dtype, void* stream) {
    return tau_launch_centered_rms_norm_configured(input, weight, output, rows, columns, epsilon, dtype, stream, 16);
}

}  // extern "C"
