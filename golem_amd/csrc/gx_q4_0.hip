// gx_q4_0.hip - the Q4_0 x Q8_0 matrix-vector product (decode, M <= 8).
//
// This is golem's matVecPackedQ4_0Rows / matVecQ4_0Rows (nn/pack_q4_0.go:
// 159-221, nn/dot_q4_0.go:168-270) rebuilt for a bandwidth-bound GPU kernel.
//
// Canonical order.  Every Q4_0 kernel in this library (this one and the
// MFMA product) computes a row's value the same way, so that a column's
// result does not depend on how many columns were in the batch:
//   isum_b = sum_j (n_j - 8) * q_j                      exact int32
//   s_b    = d_w[b] * d_a[b]                             one fp32 product
//   P_s    = fma(float(isum_b), s_b, P_s) for the blocks b of stretch s,
//            in order, starting from +0 (a stretch is 8 blocks)
//   y      = ((0 + P_0) + P_1) + ...  (+ bias)
// golem sums the same integers with an unsigned nibble and a cancelling
// correction term (nn/dot_q4_0.go:64-66); the two agree to rounding.
//
// Decomposition.  A workgroup owns RW consecutive rows and all stretches of
// them; a lane is one (row, stretch-slot) pair.  Lanes of one slot read RW
// consecutive rows' 16-byte chunks, which are contiguous in the R64 layout.
// The stretch sums meet in LDS and one lane per row adds them in order.
#include "gx_device.hpp"
#include "gx_internal.hpp"

namespace gx {
namespace {

template <int RW, int NC>
__global__ __launch_bounds__(1024) void q4_0_matvec_kernel(
    const uint8_t *__restrict__ W, size_t plane0_bytes, int B, int DC, const int8_t *__restrict__ q,
    const float *__restrict__ scales, const int32_t *__restrict__ qsum, int K, int row_base, int row_start,
    int row_end, const float *__restrict__ bias, float *__restrict__ y, int ldy, int nslots) {
    extern __shared__ float part[];  // [S][NC][RW]
    const int S = (B + kStretch - 1) / kStretch;
    const int tid = threadIdx.x;
    const int r = tid % RW, slot = tid / RW;
    const int row = row_base + blockIdx.x * RW + r;
    const int tile = row >> 6, rr = row & 63;
    const uint8_t *qs_row = W + ((size_t)tile * B * kTileRows + rr) * kChunk;
    const uint8_t *d_row = W + plane0_bytes + ((size_t)tile * DC * kTileRows + rr) * kChunk;

    if (slot < nslots) {
        for (int s = slot; s < S; s += nslots) {
            const int b0 = s * kStretch;
            const int nb = min(kStretch, B - b0);
            uint4 wq[kStretch];
#pragma unroll
            for (int j = 0; j < kStretch; j++)
                if (j < nb)
                    wq[j] = *(const uint4 *)(qs_row + (size_t)(b0 + j) * kTileRows * kChunk);
            const uint4 dch = *(const uint4 *)(d_row + (size_t)s * kTileRows * kChunk);
            float p[NC];
#pragma unroll
            for (int c = 0; c < NC; c++)
                p[c] = 0.0f;
#pragma unroll
            for (int j = 0; j < kStretch; j++) {
                if (j < nb) {
                    const float dw = chunk_half(dch, j);
                    const int b = b0 + j;
#pragma unroll
                    for (int c = 0; c < NC; c++) {
                        const int4 *a = (const int4 *)(q + (size_t)c * K + (size_t)b * kQ4Block);
                        const int32_t isum = q4_0_block_isum(wq[j], a[0], a[1], qsum[(size_t)c * B + b]);
                        const float sc = dw * scales[(size_t)c * B + b];
                        p[c] = fmaf((float)isum, sc, p[c]);
                    }
                }
            }
#pragma unroll
            for (int c = 0; c < NC; c++)
                part[(s * NC + c) * RW + r] = p[c];
        }
    }
    __syncthreads();
    if (slot == 0 && row >= row_start && row < row_end) {
#pragma unroll
        for (int c = 0; c < NC; c++) {
            float acc = 0.0f;
            for (int s = 0; s < S; s++)
                acc = acc + part[(s * NC + c) * RW + r];
            if (bias)
                acc = acc + bias[row];
            y[(size_t)c * ldy + row] = acc;
        }
    }
}

// The per-block integers of the kernel above, for the parity tests: one
// thread per (m, row, block), through the same q4_0_block_isum.
__global__ void q4_0_block_dots_kernel(const uint8_t *__restrict__ W, int B, const int8_t *__restrict__ q,
                                       const int32_t *__restrict__ qsum, int K, int M, int row_start, int nrows,
                                       int32_t *__restrict__ out) {
    const size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= (size_t)M * nrows * B)
        return;
    const int b = (int)(id % B);
    const int r = (int)((id / B) % nrows);
    const int m = (int)(id / ((size_t)B * nrows));
    const int row = row_start + r;
    const int tile = row >> 6, rr = row & 63;
    const uint4 w = *(const uint4 *)(W + (((size_t)tile * B + b) * kTileRows + rr) * kChunk);
    const int4 *a = (const int4 *)(q + (size_t)m * K + (size_t)b * kQ4Block);
    out[id] = q4_0_block_isum(w, a[0], a[1], qsum[(size_t)m * B + b]);
}

template <int RW, int NC>
int launch_rw(gx_ctx *ctx, const gx_weight *w, const uint8_t *mat, const int8_t *q, const float *scales,
              const int32_t *qsum, int row_start, int row_end, const float *bias, float *y, int ldy) {
    const int B = w->blocks;
    const int S = (B + kStretch - 1) / kStretch;
    const int nslots = min(S, 1024 / RW);
    const int threads = ((RW * nslots + 63) / 64) * 64;
    const size_t lds = (size_t)S * NC * RW * sizeof(float);
    GX_CHECK(lds <= 64 * 1024, "gx: a %d-input Q4_0 row is wider than this kernel's LDS", w->cols);
    const int row_base = (row_start / RW) * RW;
    const int grid = (row_end - row_base + RW - 1) / RW;
    q4_0_matvec_kernel<RW, NC><<<grid, threads, lds, ctx->stream>>>(mat, w->plane0_bytes, B, w->dchunks, q, scales,
                                                                     qsum, w->cols, row_base, row_start, row_end,
                                                                     bias, y, ldy, nslots);
    return check_launch("q4_0_matvec");
}

template <int NC>
int launch_nc(gx_ctx *ctx, const gx_weight *w, const uint8_t *mat, const int8_t *q, const float *scales,
              const int32_t *qsum, int row_start, int row_end, const float *bias, float *y, int ldy) {
    // Rows per workgroup: the widest that still gives every CU about two
    // workgroups; narrower tiles spread a small matrix over more CUs.
    const int rows = row_end - row_start;
    const int want = 2 * ctx->cu_count;
    if (rows / 32 >= want)
        return launch_rw<32, NC>(ctx, w, mat, q, scales, qsum, row_start, row_end, bias, y, ldy);
    if (rows / 16 >= want)
        return launch_rw<16, NC>(ctx, w, mat, q, scales, qsum, row_start, row_end, bias, y, ldy);
    return launch_rw<8, NC>(ctx, w, mat, q, scales, qsum, row_start, row_end, bias, y, ldy);
}

}  // namespace

int launch_q4_0_matvec(gx_ctx *ctx, const gx_weight *w, const uint8_t *mat, const int8_t *q, const float *scales,
                       const int32_t *qsum, int M, int row_start, int row_end, const float *bias, float *y,
                       int ldy) {
    // Columns in groups of 8, 4, 2, 1, each group reading the weights once;
    // the per-column arithmetic is the same whatever the group.
    int c = 0;
    const int K = w->cols, B = w->blocks;
    while (c < M) {
        const int left = M - c;
        const int8_t *qc = q + (size_t)c * K;
        const float *sc = scales + (size_t)c * B;
        const int32_t *qs = qsum + (size_t)c * B;
        float *yc = y + (size_t)c * ldy;
        int rc;
        if (left >= 8) {
            rc = launch_nc<8>(ctx, w, mat, qc, sc, qs, row_start, row_end, bias, yc, ldy);
            c += 8;
        } else if (left >= 4) {
            rc = launch_nc<4>(ctx, w, mat, qc, sc, qs, row_start, row_end, bias, yc, ldy);
            c += 4;
        } else if (left >= 2) {
            rc = launch_nc<2>(ctx, w, mat, qc, sc, qs, row_start, row_end, bias, yc, ldy);
            c += 2;
        } else {
            rc = launch_nc<1>(ctx, w, mat, qc, sc, qs, row_start, row_end, bias, yc, ldy);
            c += 1;
        }
        if (rc)
            return rc;
    }
    return GX_OK;
}

int launch_q4_0_block_dots_matvec(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const int32_t *qsum, int M,
                                  int row_start, int row_end, int32_t *out) {
    const int nrows = row_end - row_start;
    const size_t total = (size_t)M * nrows * w->blocks;
    const int threads = 256;
    q4_0_block_dots_kernel<<<(unsigned)((total + threads - 1) / threads), threads, 0, ctx->stream>>>(
        w->dev, w->blocks, q, qsum, w->cols, M, row_start, nrows, out);
    return check_launch("q4_0_block_dots");
}

}  // namespace gx
