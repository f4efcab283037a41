// gx_q6_k.hip - the Q6_K x Q8_K matrix-vector product (the logit head).
//
// golem's matVecQ6_KRows / dotQ6_KGo (nn/dot_q6_k.go:19-54, :77-103), bit for
// bit: per superblock the exact integer sum - 32*shift, then
//   t_b   = (float(isum_b) * d_b) * kscale_b       two fp32 products
//   total = ((0 + t_0) + t_1) + ...                 in superblock order
// (-ffp-contract=off keeps the products and sums unfused, as Go's amd64
// compiler leaves them).  Up to eight activation columns share one read of
// the weights, the role of dotQ6_Kx2 (nn/dot_q6_k_x2_amd64.s:64-154), and
// give each column exactly its one-column result.
//
// Decomposition as the Q4_0 kernel: a workgroup owns one 64-row tile, each
// wavefront whole superblocks, a lane one row.  The activation of a
// superblock is uniform across the wavefront and is read into SGPRs with
// scalar loads; the superblock terms meet in LDS and one wavefront adds them
// in order.
#include "gx_device.hpp"
#include "gx_internal.hpp"

namespace gx {
namespace {

template <int NC>
__global__ __launch_bounds__(1024) void q6_k_matvec_kernel(
    const uint8_t *__restrict__ W, size_t plane0_bytes, int B, int DC, const int8_t *__restrict__ q,
    const float *__restrict__ kscales, const int16_t *__restrict__ bsums, int K, int tile0, int row_start,
    int row_end, const float *__restrict__ bias, float *__restrict__ y, int ldy, int32_t *__restrict__ dots) {
    extern __shared__ float part[];  // [B][NC][64]
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nwaves = blockDim.x >> 6;
    const int tile = tile0 + blockIdx.x;
    const int row = tile * kTileRows + lane;
    const uint8_t *d_row = W + plane0_bytes + ((size_t)tile * DC * kTileRows + lane) * kChunk;

    for (int s = wave; s < B; s += nwaves) {
        const uint8_t *base = W + (((size_t)tile * B + s) * kQ6Chunks * kTileRows + lane) * kChunk;
        uint32_t ql[32], qh[16];
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const uint4 v = load_stream(base + (size_t)c * kTileRows * kChunk);
            ql[4 * c] = v.x, ql[4 * c + 1] = v.y, ql[4 * c + 2] = v.z, ql[4 * c + 3] = v.w;
        }
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint4 v = load_stream(base + (size_t)(8 + c) * kTileRows * kChunk);
            qh[4 * c] = v.x, qh[4 * c + 1] = v.y, qh[4 * c + 2] = v.z, qh[4 * c + 3] = v.w;
        }
        const uint4 sc = load_stream(base + (size_t)12 * kTileRows * kChunk);
        const float d = half_bits_to_float(*(const uint16_t *)(d_row + (size_t)(s >> 3) * kTileRows * kChunk +
                                                              (size_t)(s & 7) * 2));
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const uint32_t *a = (const uint32_t *)(q + (size_t)c * K + (size_t)s * kSuper);
            const uint32_t *bs = (const uint32_t *)(bsums + (size_t)c * (K / 16) + (size_t)s * 16);
            const int32_t isum = q6_k_block_isum(ql, qh, sc, a, bs);
            if (dots) {
                if (row >= row_start && row < row_end)
                    dots[((size_t)c * (row_end - row_start) + (row - row_start)) * B + s] = isum;
            } else {
                const float t0 = (float)isum * d;
                part[(s * NC + c) * kTileRows + lane] = t0 * kscales[(size_t)c * B + s];
            }
        }
    }
    if (dots)
        return;
    __syncthreads();
    if (wave == 0 && row >= row_start && row < row_end) {
#pragma unroll
        for (int c = 0; c < NC; c++) {
            float total = 0.0f;
            for (int s = 0; s < B; s++)
                total = total + part[(s * NC + c) * kTileRows + lane];
            if (bias)
                total = total + bias[row];
            y[(size_t)c * ldy + row] = total;
        }
    }
}

template <int NC>
int launch_nc(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const float *kscales, const int16_t *bsums,
              int row_start, int row_end, const float *bias, float *y, int ldy, int32_t *dots) {
    const int B = w->blocks;
    const int waves = min(B, 16);
    const size_t lds = dots ? 0 : (size_t)B * NC * kTileRows * sizeof(float);
    GX_CHECK(lds <= 64 * 1024, "gx: a %d-input Q6_K row is wider than this kernel's LDS", w->cols);
    const int tile0 = row_start / kTileRows;
    const int grid = (row_end + kTileRows - 1) / kTileRows - tile0;
    q6_k_matvec_kernel<NC><<<grid, 64 * waves, lds, ctx->stream>>>(w->dev, w->plane0_bytes, B, w->dchunks, q,
                                                                   kscales, bsums, w->cols, tile0, row_start,
                                                                   row_end, bias, y, ldy, dots);
    return check_launch("q6_k_matvec");
}

}  // namespace

int launch_q6_k_matvec(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const float *kscales,
                       const int16_t *bsums, int M, int row_start, int row_end, const float *bias, float *y,
                       int ldy, int32_t *dots) {
    const int K = w->cols, B = w->blocks;
    const size_t nrows = (size_t)(row_end - row_start);
    int c = 0;
    while (c < M) {
        const int left = M - c;
        const int8_t *qc = q + (size_t)c * K;
        const float *kc = kscales ? kscales + (size_t)c * B : nullptr;
        const int16_t *bc = bsums + (size_t)c * (K / 16);
        float *yc = y ? y + (size_t)c * ldy : nullptr;
        int32_t *dc = dots ? dots + (size_t)c * nrows * B : nullptr;
        int rc;
        if (left >= 8) {
            rc = launch_nc<8>(ctx, w, qc, kc, bc, row_start, row_end, bias, yc, ldy, dc);
            c += 8;
        } else if (left >= 4) {
            rc = launch_nc<4>(ctx, w, qc, kc, bc, row_start, row_end, bias, yc, ldy, dc);
            c += 4;
        } else if (left >= 2) {
            rc = launch_nc<2>(ctx, w, qc, kc, bc, row_start, row_end, bias, yc, ldy, dc);
            c += 2;
        } else {
            rc = launch_nc<1>(ctx, w, qc, kc, bc, row_start, row_end, bias, yc, ldy, dc);
            c += 1;
        }
        if (rc)
            return rc;
    }
    return GX_OK;
}

}  // namespace gx
