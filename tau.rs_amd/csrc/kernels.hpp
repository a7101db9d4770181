// Internal launcher interface shared by the library's translation units.
#pragma once
#include "common.hpp"

namespace tau_amd {

enum AMode { kAGather = 0, kADirect = 1 };
enum Epilogue { kEpiSilu = 0, kEpiStoreBf16 = 1, kEpiScatterWeighted = 2, kEpiStoreF32 = 3 };
// Expert weight layouts.  Row-major: W[e][n][k].  Frag16: each 16-row x 32-wide
// K block is one contiguous 1 KB MFMA operand fragment, 16-byte piece p holding
// row 16*nb + p%16, columns 32*kc + 8*(p/16) .. +8; blocks run K-fastest, so a
// 16-row band of one expert is 16*K contiguous elements.
enum WeightLayout { kWeightsRowMajor = 0, kWeightsFrag16 = 1 };

struct GemmArgs {
    const uint16_t* a;        // gather: x [T,lda]; direct: rows [rows,lda]
    const uint16_t* w;        // expert weights [E][N_w][K] (N_w = 2I for gate_up)
    const float* routes;      // [T, 2*topk] (scatter epilogue)
    const int* slots;         // [cap] assignment per row (gather / scatter)
    const int* tiles;         // [cap/BM] expert per row block, or null (single group)
    const int* meta_total;    // padded row total on the device, or null
    void* out;                // activated / projected / contributions / f32 output
    int rows;                 // capacity (grouped) or row count (dense)
    int assignments;          // T * topk; slot sentinel value
    int topk;
    int n;                    // output columns (I for gate_up-silu, N otherwise)
    int k;                    // inner dimension
    int lda;                  // A row stride (elements)
    int ldo;                  // output row stride (elements)
    long w_expert_stride;     // elements between experts
    int w_up_offset;          // rows between gate row j and up row j (I)
    int w_layout;             // WeightLayout of w
    int* receipt;             // optional 5 words stamped by the executed kernel
    // Small-block split (0 = off): the dispatch's row blocks are `block_stride`
    // rows apart (0 = the kernel's own BM); with split_rows > 0 a kernel whose
    // BM exceeds split_rows skips blocks with at most split_rows live rows and
    // a kernel with BM == split_rows takes only those.
    int block_stride;
    int split_rows;
};

int launch_grouped_gemm(const GemmArgs& p, int bm, int a_mode, int epilogue, hipStream_t s);
int launch_pack_frag16(const void* src, void* dst, int experts, int rows, int cols, hipStream_t s);
int launch_add_bias(float* out, const float* bias, int rows, int cols, hipStream_t s);
bool gemm_rows_supported(int bm);

int64_t capacity_for(int64_t tokens, int64_t E, int64_t K, int64_t M);
int launch_routing_shared(const void* logits, int logits_dtype, float* routes, int tokens, int E, int K,
                          hipStream_t s);
// logits_dtype 0 (f32) or 1 (BF16), optionally OR TAU_MOE_ROUTE_RAW_WEIGHTS.
bool logits_dtype_ok(int logits_dtype);
int launch_routing(const void* logits, int logits_dtype, float* routes, int tokens, int E, int K,
                   hipStream_t s);
int launch_dispatch(const void* logits, int logits_dtype, float* routes, int* meta, int* offsets, int* slots,
                    int* tiles, int tokens, int E, int K, int M, int capacity, void* scratch, size_t scratch_bytes,
                    hipStream_t s);
int launch_combine(const void* contributions, void* output, const int* status, int tokens, int H, int K,
                   const void* residual, hipStream_t s);

// Fused decode path (decode_moe.hip): same outputs as routing + dispatch +
// grouped GEMMs + combine with 16-row blocks, the plan built off the critical
// path.  Activated/contributions rows are indexed by assignment t*K + r.
bool decode_path_supported(int tokens, int hidden, int intermediate, int experts, int top_k, int tile_rows,
                           int weight_layout);
// Returned by optional paths that do not apply to a shape (the caller falls back).
constexpr int kNotApplicable = -2;
int launch_decode_layer(const void* input, const void* logits, int logits_dtype, const void* gate_up,
                        const void* down, float* routes, int* meta, int* offsets, int* slots, int* tiles,
                        void* activated, void* contributions, int tokens, int hidden, int intermediate, int experts,
                        int top_k, int capacity, int weight_layout, int* receipts, hipStream_t s);
int launch_decode_projection(const void* a, const void* w, float* routes, int* meta, int* offsets, int* slots,
                             int* tiles, void* out, int tokens, int hidden, int intermediate, int experts, int top_k,
                             int capacity, int projection, int weight_layout, int* receipt, hipStream_t s);
int launch_decode_moe(const void* input, const void* logits, int logits_dtype, const void* gate_up,
                      const void* down, float* routes, int* meta, int* offsets, int* slots, int* tiles,
                      void* activated, void* contributions, void* output, int tokens, int hidden,
                      int intermediate, int experts, int top_k, int capacity, int weight_layout,
                      const void* residual, int* receipts, hipStream_t s);

}  // namespace tau_amd
