// gx_gemm.hip - the Q4_0 x Q8_0 product for a batch of tokens (prefill) on
// int8 MFMA.
//
// golem reads a prompt through the same MatVecBatch as a single token, with
// the batch as the inner loop (nn/matrix.go:67-81, nn/pack_q4_0.go:159-221).
// Here the batch is a real dense contraction: v_mfma_i32_32x32x32_i8 takes one
// Q4_0 block (32 inputs) of 32 rows against the same block of 32 tokens and
// returns the exact per-block integers; the fp32 scales are applied to them
// per block in the canonical order of the matrix-vector kernel
// (gx_q4_0.hip), stretch by stretch, so a token's result is bit-identical
// whether it came through this kernel or that one.
//
// Tile: a workgroup of four wavefronts owns 64 rows (one R64 tile) x 64
// tokens; each wavefront one 32x32 quarter.  The weights' nibbles are widened
// to signed int8 in registers (n - 8); the activations are already int8.
// The block scales of the tile's rows and tokens for one stretch are staged
// in LDS as floats, double-buffered, one barrier per stretch.
#include "gx_device.hpp"
#include "gx_internal.hpp"

namespace gx {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// Nibbles 0..15 in each byte -> (n - 8) as int8: n + 120 stays below 256
// without a carry, and flipping the top bit subtracts 128.
__device__ __forceinline__ uint32_t widen_nibbles(uint32_t n) { return (n + 0x78787878u) ^ 0x80808080u; }

template <bool DOTS>
__global__ __launch_bounds__(256) void q4_0_gemm_kernel(const uint8_t *__restrict__ W, size_t plane0_bytes, int B,
                                                        int DC, const int8_t *__restrict__ q,
                                                        const float *__restrict__ scales, int K, int M,
                                                        int row_base, int row_start, int row_end,
                                                        const float *__restrict__ bias, float *__restrict__ y,
                                                        int ldy, int32_t *__restrict__ dots) {
    __shared__ float sdw[2][kStretch][64];
    __shared__ float sda[2][kStretch][64];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wv = tid >> 6;
    const int n0 = row_base + blockIdx.x * 64;
    const int m0 = blockIdx.y * 64;
    const int nw = 32 * (wv & 1), mw = 32 * (wv >> 1);
    const int li = lane & 31, g = lane >> 5;

    const int arow = n0 + nw + li;
    const uint8_t *a_src = W + ((size_t)(arow >> 6) * B * kTileRows + (arow & 63)) * kChunk;
    const int bm = m0 + mw + li;
    const bool bvalid = bm < M;
    const int8_t *b_src = q + (size_t)(bvalid ? bm : 0) * K + 16 * g;

    float acc[16], tot[16];
#pragma unroll
    for (int e = 0; e < 16; e++)
        acc[e] = 0.0f, tot[e] = 0.0f;

    const int S = (B + kStretch - 1) / kStretch;
    const int nrows = row_end - row_start;
    for (int s = 0; s < S; s++) {
        const int buf = s & 1;
        const int b0 = s * kStretch;
        const int nb = min(kStretch, B - b0);
        if (!DOTS) {
            if (tid < 64) {
                const int n = n0 + tid;
                const uint4 dch = *(const uint4 *)(W + plane0_bytes +
                                                   (((size_t)(n >> 6) * DC + s) * kTileRows + (n & 63)) * kChunk);
#pragma unroll
                for (int j = 0; j < kStretch; j++)
                    sdw[buf][j][tid] = chunk_half(dch, j);
            } else if (tid < 128) {
                const int m = m0 + tid - 64;
#pragma unroll
                for (int j = 0; j < kStretch; j++)
                    sda[buf][j][tid - 64] = (m < M && j < nb) ? scales[(size_t)m * B + b0 + j] : 0.0f;
            }
            __syncthreads();
        }
        for (int j = 0; j < nb; j++) {
            const int b = b0 + j;
            const uint4 wq = *(const uint4 *)(a_src + (size_t)b * kTileRows * kChunk);
            const uint32_t sh = 4 * g;
            v4i A;
            A.x = (int)widen_nibbles((wq.x >> sh) & 0x0F0F0F0Fu);
            A.y = (int)widen_nibbles((wq.y >> sh) & 0x0F0F0F0Fu);
            A.z = (int)widen_nibbles((wq.z >> sh) & 0x0F0F0F0Fu);
            A.w = (int)widen_nibbles((wq.w >> sh) & 0x0F0F0F0Fu);
            v4i Bv = {0, 0, 0, 0};
            if (bvalid)
                Bv = *(const v4i *)(b_src + (size_t)b * kQ4Block);
            v16i C = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
            C = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, Bv, C, 0, 0, 0);
            if (DOTS) {
                if (bvalid) {
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        const int n = n0 + nw + 8 * (e >> 2) + 4 * g + (e & 3);
                        if (n >= row_start && n < row_end)
                            dots[((size_t)bm * nrows + (n - row_start)) * B + b] = C[e];
                    }
                }
            } else {
                const float da = sda[buf][j][mw + li];
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const float dw = sdw[buf][j][nw + 8 * (e >> 2) + 4 * g + (e & 3)];
                    const float sc = dw * da;
                    acc[e] = fmaf((float)C[e], sc, acc[e]);
                }
            }
        }
        if (!DOTS) {
#pragma unroll
            for (int e = 0; e < 16; e++) {
                tot[e] = tot[e] + acc[e];
                acc[e] = 0.0f;
            }
        }
    }
    if (DOTS || !bvalid)
        return;
#pragma unroll
    for (int e = 0; e < 16; e++) {
        const int n = n0 + nw + 8 * (e >> 2) + 4 * g + (e & 3);
        if (n >= row_start && n < row_end) {
            float v = tot[e];
            if (bias)
                v = v + bias[n];
            y[(size_t)bm * ldy + n] = v;
        }
    }
}

}  // namespace

int launch_q4_0_gemm(gx_ctx *ctx, const gx_weight *w, const uint8_t *mat, const int8_t *q, const float *scales,
                     const int32_t *qsum, int M, int row_start, int row_end, const float *bias, float *y, int ldy,
                     int32_t *dots) {
    (void)qsum;  // the widened weights are signed: no recentring term
    const int row_base = (row_start / 64) * 64;
    dim3 grid((row_end - row_base + 63) / 64, (M + 63) / 64);
    if (dots)
        q4_0_gemm_kernel<true><<<grid, 256, 0, ctx->stream>>>(mat, w->plane0_bytes, w->blocks, w->dchunks, q, scales,
                                                              w->cols, M, row_base, row_start, row_end, bias, y, ldy,
                                                              dots);
    else
        q4_0_gemm_kernel<false><<<grid, 256, 0, ctx->stream>>>(mat, w->plane0_bytes, w->blocks, w->dchunks, q,
                                                               scales, w->cols, M, row_base, row_start, row_end,
                                                               bias, y, ldy, dots);
    return check_launch("q4_0_gemm");
}

}  // namespace gx
