// gx_internal.hpp - shared definitions of the gfx950 quantized-product library.
//
// Weight layout on the device ("R64").  A matrix's rows are cut into tiles of
// 64 rows (the last tile padded with zero rows).  Within a tile every per-row
// byte stream is cut into 16-byte chunks, and chunk j of the 64 rows is stored
// as one contiguous kilobyte: chunk j of row r of tile t lives at
//     plane + ((t * chunks_per_row + j) * 64 + r) * 16.
// A wavefront whose lanes are 64 consecutive rows therefore reads 1 KiB of
// contiguous memory with one 16-byte load per lane, and a lane that owns a row
// walks that row's chunks 1 KiB apart.  The byte count equals the GGUF
// layout's, apart from the padding rows and scale chunks.
//
//   Q4_0:  plane 0 = the 16 nibble bytes of each block (chunk j = block j),
//          plane 1 = the fp16 block scales, 8 blocks per chunk.
//   Q6_K:  plane 0 = per superblock 13 chunks: ql (8), qh (4), scales (1),
//          plane 1 = the fp16 superblock scales, 8 superblocks per chunk.
//   F32:   row-major floats, unchanged.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/golem_hip.h"

namespace gx {

constexpr int kTileRows = 64;
constexpr int kChunk = 16;
constexpr int kQ4Block = 32;      // nn/quant.go:50
constexpr int kQ4BlockBytes = 18; // nn/quant.go:52
constexpr int kSuper = 256;       // nn/quant.go:54
constexpr int kQ6BlockBytes = 210;// nn/quant.go:56
constexpr int kQ6Chunks = 13;     // ql 8 + qh 4 + scales 1
// The blocks of one stretch: a row's products are summed within a stretch
// first, then the stretch sums in order (the canonical order every Q4_0
// kernel here follows).  Eight blocks is also one scale chunk.
constexpr int kStretch = 8;

// The fp16 copy of a Q8_0 activation (q16) is laid out in the operand order
// of v_mfma_f32_32x32x16_f16: tokens in groups of 32, and for group G, block
// b and k-half h (inputs 32b + 16h .. + 15) one 1 KiB panel in which lane
// 32g + li of a wavefront finds, at 16 bytes per lane, token 32G + li's inputs
// 32b + 16h + 8g .. + 7.  The buffer holds ceil(M/32)*32 tokens; tokens past
// M are zero.
__host__ __device__ inline size_t q16_offset(int t, int k, int blocks) {
    const int G = t >> 5, li = t & 31, b = k >> 5, j = k & 31;
    const int h = j >> 4, g = (j >> 3) & 1, e = j & 7;
    return ((((size_t)G * blocks + b) * 2 + h) * 64 + 32 * g + li) * 8 + e;
}

int fail(int code, const char *fmt, ...);
int succeed();  // clears the thread's error message; GX_OK
int check_launch(const char *what);

}  // namespace gx

struct gx_ctx {
    int device;
    hipStream_t stream;
    hipEvent_t t0, t1;
    int cu_count;
    float *gelu_table;  // golem's 65536-entry GELU table, built on the device at init
    float *argmax_v;    // the greedy pick's part maxima [kArgmaxRows][kArgmaxParts]
    int32_t *argmax_i;  // and their indices
    uint8_t *scratch;   // this device's copy of the no-alloc entry points' static scratch (gx_api.hip)
    float *route_scale;     // the many-position router's norm scales [kRouteScaleMax]
    struct gx_rows *rows;   // the coalesced MatVecRows products (gx_api.hip)
};


constexpr int kArgmaxParts = 128;  // workgroups per row of the greedy pick
constexpr int kArgmaxRows = 64;    // rows per launch pair
constexpr int kRouteMaxPos = 4;    // positions routed by the few-position router kernel
constexpr int kRouteScaleMax = 4096;  // positions of one many-position router pass

struct gx_weight {
    gx_ctx *ctx;
    int quant, rows, cols, count;
    int tiles;           // ceil(rows / 64)
    int blocks;          // Q4_0: cols/32; Q6_K: cols/256; F32: cols
    int dchunks;         // ceil(blocks / 8)
    size_t plane0_bytes; // per matrix
    size_t matrix_bytes; // per matrix, both planes
    uint8_t *dev;
};

#define GX_HIP(expr)                                                                          \
    do {                                                                                      \
        hipError_t e_ = (expr);                                                               \
        if (e_ != hipSuccess)                                                                 \
            return gx::fail(GX_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(e_));       \
    } while (0)

#define GX_CHECK(cond, ...)                                                                   \
    do {                                                                                      \
        if (!(cond))                                                                          \
            return gx::fail(GX_ERR_INVALID, __VA_ARGS__);                                     \
    } while (0)

// ---- launchers implemented in the kernel files ---------------------------
namespace gx {
int launch_repack(gx_ctx *ctx, const uint8_t *src, gx_weight *w);
int launch_rows(gx_ctx *ctx, const gx_weight *w, int expert, const int32_t *ids, int n, float *out);
int launch_quantize_q8_0(gx_ctx *ctx, const float *x, int ldx, int M, int K, int8_t *q, float *scales,
                         int32_t *qsum, float *corr, uint16_t *q16);
int launch_quantize_q8_k(gx_ctx *ctx, const float *x, int ldx, int M, int K, int8_t *q, float *kscales,
                         int16_t *bsums);
// form: -1 the product's own choice, 0 the SGPR-activation kernel, 1 the
// one-column LDS kernel (M = 1).  dots: null, or the per-block integers
// [M][row_end - row_start][K/32] of the kernel that runs.
int launch_q4_0_matvec(gx_ctx *ctx, const gx_weight *w, const uint8_t *mat, const int8_t *q, const float *scales,
                       const int32_t *qsum, int M, int row_start, int row_end, const float *bias, float *y,
                       int ldy, int32_t *dots, int form);
int launch_q4_0_gemm(gx_ctx *ctx, const gx_weight *w, const uint8_t *mat, const int8_t *q, const float *scales,
                     int M, int row_start, int row_end, const float *bias, float *y, int ldy, int32_t *dots);
int launch_q4_0_gemm_swiglu(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const float *scales, int M,
                            int8_t *mq, float *ms, int32_t *mqs);
// The Q|K|V product of a batch with the head norms, RoPE and the fp16
// query and cache stores of qwen_qk_rope in its epilogue (rows: the query,
// key and value heads stacked, hd 64 or 128).
struct QkvRopeArgs {
    const int32_t *positions;
    const float *q_norm, *k_norm, *rope_cos, *rope_sin;
    float eps;
    uint16_t *qh, *kcache, *vcache;
    int context, heads, kv_heads, hd;
    const int32_t *slots;
    int nslots;
};
int launch_q4_0_gemm_qkv_rope(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const float *scales, int M,
                              const QkvRopeArgs &a);
// The expert-grouped product: work items {expert, first, count <= 32, 0}
// over the units sorted by expert (gx_moe.hip's sort); dots as above, by
// output (unit) row.
int launch_q4_0_gemm_grouped(gx_ctx *ctx, const gx_weight *w, const int32_t *work, int max_items,
                             const int32_t *sorted, int act_div, const int8_t *q, const float *scales, float *y,
                             int ldy, int32_t *dots);
int launch_q4_0_gemm_f16(gx_ctx *ctx, const gx_weight *w, const uint8_t *mat, const uint16_t *q16,
                         const float *scales, int M, int row_start, int row_end, const float *bias, float *y, int ldy,
                         int32_t *dots);
int launch_q4_0_matvec_units(gx_ctx *ctx, const gx_weight *w, const int32_t *unit_expert, int units, int act_div,
                              const int8_t *q, const float *scales, const int32_t *qsum, float *y, int ldy,
                              int32_t *dots);
int launch_q4_0_matvec_swiglu(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const float *scales,
                               const int32_t *qsum, int M, int8_t *mq, float *ms, int32_t *mqs);
int launch_q4_0_matvec_fused(gx_ctx *ctx, const gx_weight *w, int epi, int row_start, int row_end, float *y,
                              const float *x, const float *add, const float *gain, float eps, float *x_out,
                              int8_t *q, float *scales, int32_t *qsum, int32_t *dots);
int launch_q6_k_matvec(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const float *kscales,
                       const int16_t *bsums, int M, int row_start, int row_end, const float *bias, float *y,
                       int ldy, int32_t *dots);
int moe_workspace_bytes(int M, int k, int D, int F, int E, size_t *bytes);
int launch_gelu_table(gx_ctx *ctx, float *table);
int launch_geglu_quant(gx_ctx *ctx, const float *gu, int ldgu, int M, int ffn, int8_t *q, float *scales,
                       int32_t *qsum);
int launch_moe_join(gx_ctx *ctx, float *shared, int lds_, float *experts, int lde, const float *resid, int ldr,
                    const float *post1, const float *post2, const float *post, int M, int K, float eps, float *out,
                    int ldo);
int launch_moe_route(gx_ctx *ctx, const gx_weight *router, const float *router_scale, const float *resid, int ldr,
                     int M, int k, float eps, float *logits, int32_t *ids, float *weights);
int launch_moe_experts(gx_ctx *ctx, const gx_weight *gate_up, const gx_weight *down, const float *down_scale,
                       const float *x, int ldx, int M, int k, const int32_t *ids, const float *weights, float *out,
                       int ldo, uint8_t *ws, const float *gelu_table);
int launch_moe_block_dots(gx_ctx *ctx, const gx_weight *gate_up, const gx_weight *down, const float *x, int ldx,
                          int M, int k, const int32_t *ids, const int8_t *mid_q, const float *mid_scales,
                          const int32_t *mid_qsum, uint8_t *ws, int32_t *dots_gate_up, int32_t *dots_down);
int launch_qwen_norm_quant(gx_ctx *ctx, float *x, int ldx, const float *add, int lda, const float *gain, int M, int K,
                           float eps, float *out, int ldo, int8_t *q, float *scales, int32_t *qsum);
int launch_qwen_qk_rope(gx_ctx *ctx, const float *qkv, int ldqkv, int M, int heads, int kv_heads, int hd,
                        const int32_t *positions, const float *q_norm, const float *k_norm, const float *rope_cos,
                        const float *rope_sin, float eps, uint16_t *qh, uint16_t *kcache, uint16_t *vcache,
                        int context, const int32_t *slots, int nslots);
size_t qwen_attention_workspace(int M, int heads, int max_pos);
int launch_qwen_rope_attention(gx_ctx *ctx, const float *qkv, int ldqkv, int M, int heads, int kv_heads, int hd,
                               int max_pos, const int32_t *positions, const float *q_norm, const float *k_norm,
                               const float *rope_cos, const float *rope_sin, float eps, uint16_t *kcache,
                               uint16_t *vcache, int context, float scale, int8_t *q, float *scales, int32_t *qsum,
                               const int32_t *slots, int nslots, int parallel);
int launch_qwen_attention(gx_ctx *ctx, const uint16_t *qh, int M, int heads, int kv_heads, int hd, int max_pos,
                          const int32_t *positions, const uint16_t *kcache, const uint16_t *vcache, int context,
                          float scale, int8_t *q, float *scales, int32_t *qsum, uint8_t *workspace,
                          const int32_t *slots, int nslots, int parallel, float *heads_f);
int launch_qwen_swiglu_quant(gx_ctx *ctx, const float *gu, int ldgu, int M, int ffn, int group, int8_t *q,
                             float *scales, int32_t *qsum);
int launch_argmax(gx_ctx *ctx, const float *x, int ldx, int M, int n, int32_t *out, int32_t *history,
                  int history_len, int32_t *pos, int32_t *positions, int32_t *row_tokens = nullptr,
                  int32_t *row_positions = nullptr);
int launch_f32_matvec(gx_ctx *ctx, const gx_weight *w, const float *x, int ldx, int M, int row_start, int row_end,
                      float *y, int ldy);
}  // namespace gx
