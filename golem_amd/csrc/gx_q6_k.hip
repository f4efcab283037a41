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
// Decomposition as the Q4_0 kernel: a workgroup owns RW rows, a lane one
// (row, superblock-slot) pair; the superblock terms meet in LDS and one lane
// per row adds them in order.
#include "gx_device.hpp"
#include "gx_internal.hpp"

namespace gx {
namespace {

template <int RW, int NC>
__global__ __launch_bounds__(1024) void q6_k_matvec_kernel(
    const uint8_t *__restrict__ W, size_t plane0_bytes, int B, int DC, const int8_t *__restrict__ q,
    const float *__restrict__ kscales, const int16_t *__restrict__ bsums, int K, int row_base, int row_start,
    int row_end, const float *__restrict__ bias, float *__restrict__ y, int ldy, int nslots,
    int32_t *__restrict__ dots, int M) {
    extern __shared__ float part[];  // [B][NC][RW]
    const int tid = threadIdx.x;
    const int r = tid % RW, slot = tid / RW;
    const int row = row_base + blockIdx.x * RW + r;
    const int tile = row >> 6, rr = row & 63;
    const uint8_t *d_row = W + plane0_bytes + ((size_t)tile * DC * kTileRows + rr) * kChunk;

    if (slot < nslots) {
        for (int s = slot; s < B; s += nslots) {
            const uint8_t *base = W + (((size_t)tile * B + s) * kQ6Chunks * kTileRows + rr) * kChunk;
            uint32_t ql[32], qh[16];
#pragma unroll
            for (int c = 0; c < 8; c++) {
                const uint4 v = *(const uint4 *)(base + (size_t)c * kTileRows * kChunk);
                ql[4 * c] = v.x, ql[4 * c + 1] = v.y, ql[4 * c + 2] = v.z, ql[4 * c + 3] = v.w;
            }
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const uint4 v = *(const uint4 *)(base + (size_t)(8 + c) * kTileRows * kChunk);
                qh[4 * c] = v.x, qh[4 * c + 1] = v.y, qh[4 * c + 2] = v.z, qh[4 * c + 3] = v.w;
            }
            const uint4 sc = *(const uint4 *)(base + (size_t)12 * kTileRows * kChunk);
            const uint4 dch = *(const uint4 *)(d_row + (size_t)(s >> 3) * kTileRows * kChunk);
            const float d = chunk_half(dch, s & 7);
#pragma unroll
            for (int c = 0; c < NC; c++) {
                const int4 *a = (const int4 *)(q + (size_t)c * K + (size_t)s * kSuper);
                int4 av[16];
#pragma unroll
                for (int i = 0; i < 16; i++)
                    av[i] = a[i];
                const int4 *bsp = (const int4 *)(bsums + (size_t)c * (K / 16) + (size_t)s * 16);
                const int32_t isum = q6_k_block_isum(ql, qh, sc, av, bsp[0], bsp[1]);
                if (dots) {
                    if (row >= row_start && row < row_end)
                        dots[((size_t)c * (row_end - row_start) + (row - row_start)) * B + s] = isum;
                } else {
                    const float t0 = (float)isum * d;
                    part[(s * NC + c) * RW + r] = t0 * kscales[(size_t)c * B + s];
                }
            }
        }
    }
    if (dots)
        return;
    __syncthreads();
    if (slot == 0 && row >= row_start && row < row_end) {
#pragma unroll
        for (int c = 0; c < NC; c++) {
            float total = 0.0f;
            for (int s = 0; s < B; s++)
                total = total + part[(s * NC + c) * RW + r];
            if (bias)
                total = total + bias[row];
            y[(size_t)c * ldy + row] = total;
        }
    }
}

template <int RW, int NC>
int launch_rw(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const float *kscales, const int16_t *bsums,
              int row_start, int row_end, const float *bias, float *y, int ldy, int32_t *dots) {
    const int B = w->blocks;
    const int nslots = min(B, 1024 / RW);
    const int threads = ((RW * nslots + 63) / 64) * 64;
    const size_t lds = dots ? 0 : (size_t)B * NC * RW * sizeof(float);
    GX_CHECK(lds <= 64 * 1024, "gx: a %d-input Q6_K row is wider than this kernel's LDS", w->cols);
    const int row_base = (row_start / RW) * RW;
    const int grid = (row_end - row_base + RW - 1) / RW;
    q6_k_matvec_kernel<RW, NC><<<grid, threads, lds, ctx->stream>>>(w->dev, w->plane0_bytes, B, w->dchunks, q,
                                                                     kscales, bsums, w->cols, row_base, row_start,
                                                                     row_end, bias, y, ldy, nslots, dots, NC);
    return check_launch("q6_k_matvec");
}

template <int NC>
int launch_nc(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const float *kscales, const int16_t *bsums,
              int row_start, int row_end, const float *bias, float *y, int ldy, int32_t *dots) {
    const int rows = row_end - row_start;
    const int want = 2 * ctx->cu_count;
    if (rows / 32 >= want)
        return launch_rw<32, NC>(ctx, w, q, kscales, bsums, row_start, row_end, bias, y, ldy, dots);
    if (rows / 16 >= want)
        return launch_rw<16, NC>(ctx, w, q, kscales, bsums, row_start, row_end, bias, y, ldy, dots);
    return launch_rw<8, NC>(ctx, w, q, kscales, bsums, row_start, row_end, bias, y, ldy, dots);
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
