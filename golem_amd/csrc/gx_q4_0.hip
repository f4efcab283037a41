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
// Decomposition.  A workgroup owns one 64-row tile of the R64 layout; each
// wavefront takes whole stretches, and a lane is one row of the tile.  The
// wavefront's 16-byte loads of a stretch's chunks are 1 KiB contiguous, and
// the activation of a stretch is the same for all 64 lanes, so it is read
// with scalar loads into SGPRs and fed to v_dot4 from there: the vector
// memory path carries weights only.  The stretch sums meet in LDS and one
// wavefront adds them in order.
#include "gx_device.hpp"
#include "gx_internal.hpp"

namespace gx {
namespace {

// With UNITS, blockIdx.y is a unit of a mixture-of-experts batch: unit u
// multiplies expert unit_expert[u] of a stack (matrices matrix_bytes apart)
// by activation row u / act_div, into output row u.
template <int NC, bool UNITS>
__global__ __launch_bounds__(1024) void q4_0_matvec_kernel(
    const uint8_t *__restrict__ W, size_t plane0_bytes, int B, int DC, const int8_t *__restrict__ q,
    const float *__restrict__ scales, const int32_t *__restrict__ qsum, int K, int tile0, int row_start,
    int row_end, const float *__restrict__ bias, float *__restrict__ y, int ldy,
    const int32_t *__restrict__ unit_expert, size_t matrix_bytes, int act_div, int experts) {
    extern __shared__ float part[];  // [S][NC][64]
    const int S = (B + kStretch - 1) / kStretch;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nwaves = blockDim.x >> 6;
    const int tile = tile0 + blockIdx.x;
    if (UNITS) {
        const int u = blockIdx.y;
        const int e = unit_expert[u];
        if (e < 0 || e >= experts) {  // an id out of range reads nothing and yields NaN
            const int row = tile * kTileRows + lane;
            if (threadIdx.x < 64 && row < row_end)
                y[(size_t)u * ldy + row] = __builtin_nanf("");
            return;
        }
        W += (size_t)e * matrix_bytes;
        const int a = u / act_div;
        q += (size_t)a * K;
        scales += (size_t)a * B;
        qsum += (size_t)a * B;
        y += (size_t)u * ldy;
    }
    const uint8_t *qs_row = W + ((size_t)tile * B * kTileRows + lane) * kChunk;
    const uint8_t *d_row = W + plane0_bytes + ((size_t)tile * DC * kTileRows + lane) * kChunk;

    for (int s = wave; s < S; s += nwaves) {
        const int b0 = s * kStretch;
        const int nb = min(kStretch, B - b0);
        // Unconditional loads: past the last block a load repeats the last
        // block (in bounds) and its product is skipped, so the compiler issues
        // all nine loads back to back instead of one per guarded branch.
        uint4 wq[kStretch];
#pragma unroll
        for (int j = 0; j < kStretch; j++)
            wq[j] = load_stream(qs_row + (size_t)min(b0 + j, B - 1) * kTileRows * kChunk);
        const uint4 dch = *(const uint4 *)(d_row + (size_t)s * kTileRows * kChunk);
        float p[NC];
#pragma unroll
        for (int c = 0; c < NC; c++)
            p[c] = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; c++) {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                // Four blocks' activation at a time, loaded before any use.
                int4 a0[4], a1[4];
                int32_t qs[4];
                float sa[4];
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    const int b = min(b0 + 4 * h + jj, B - 1);
                    const int4 *a = (const int4 *)(q + (size_t)c * K + (size_t)b * kQ4Block);
                    a0[jj] = a[0];
                    a1[jj] = a[1];
                    qs[jj] = qsum[(size_t)c * B + b];
                    sa[jj] = scales[(size_t)c * B + b];
                }
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    const int j = 4 * h + jj;
                    if (j < nb) {
                        const int32_t isum = q4_0_block_isum(wq[j], a0[jj], a1[jj], qs[jj]);
                        const float sc = chunk_half(dch, j) * sa[jj];
                        p[c] = fmaf((float)isum, sc, p[c]);
                    }
                }
            }
        }
#pragma unroll
        for (int c = 0; c < NC; c++)
            part[(s * NC + c) * kTileRows + lane] = p[c];
    }
    __syncthreads();
    const int row = tile * kTileRows + lane;
    if (wave == 0 && row >= row_start && row < row_end) {
#pragma unroll
        for (int c = 0; c < NC; c++) {
            float acc = 0.0f;
            for (int s = 0; s < S; s++)
                acc = acc + part[(s * NC + c) * kTileRows + lane];
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

template <int NC>
int launch_nc(gx_ctx *ctx, const gx_weight *w, const uint8_t *mat, const int8_t *q, const float *scales,
              const int32_t *qsum, int row_start, int row_end, const float *bias, float *y, int ldy) {
    const int B = w->blocks;
    const int S = (B + kStretch - 1) / kStretch;
    const int waves = min(S, 16);
    const size_t lds = (size_t)S * NC * kTileRows * sizeof(float);
    GX_CHECK(lds <= 64 * 1024, "gx: a %d-input Q4_0 row is wider than this kernel's LDS", w->cols);
    const int tile0 = row_start / kTileRows;
    const int grid = (row_end + kTileRows - 1) / kTileRows - tile0;
    q4_0_matvec_kernel<NC, false><<<grid, 64 * waves, lds, ctx->stream>>>(
        mat, w->plane0_bytes, B, w->dchunks, q, scales, qsum, w->cols, tile0, row_start, row_end, bias, y, ldy,
        nullptr, 0, 1, 0);
    return check_launch("q4_0_matvec");
}

}  // namespace

int launch_q4_0_matvec(gx_ctx *ctx, const gx_weight *w, const uint8_t *mat, const int8_t *q, const float *scales,
                       const int32_t *qsum, int M, int row_start, int row_end, const float *bias, float *y,
                       int ldy) {
    // Columns in groups of 8, 4, 2, 1, each group reading the weights once;
    // the per-column arithmetic is the same whatever the group.  Very wide
    // rows keep the group narrow enough for the stretch sums to fit in LDS.
    int c = 0;
    const int K = w->cols, B = w->blocks;
    const size_t per_column = (size_t)((B + kStretch - 1) / kStretch) * kTileRows * sizeof(float);
    const int widest = per_column * 8 <= 64 * 1024 ? 8 : per_column * 4 <= 64 * 1024 ? 4
                     : per_column * 2 <= 64 * 1024 ? 2 : 1;
    while (c < M) {
        const int left = M - c;
        const int8_t *qc = q + (size_t)c * K;
        const float *sc = scales + (size_t)c * B;
        const int32_t *qs = qsum + (size_t)c * B;
        float *yc = y + (size_t)c * ldy;
        int rc;
        if (left >= 8 && widest >= 8) {
            rc = launch_nc<8>(ctx, w, mat, qc, sc, qs, row_start, row_end, bias, yc, ldy);
            c += 8;
        } else if (left >= 4 && widest >= 4) {
            rc = launch_nc<4>(ctx, w, mat, qc, sc, qs, row_start, row_end, bias, yc, ldy);
            c += 4;
        } else if (left >= 2 && widest >= 2) {
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

int launch_q4_0_matvec_units(gx_ctx *ctx, const gx_weight *w, const int32_t *unit_expert, int units, int act_div,
                              const int8_t *q, const float *scales, const int32_t *qsum, float *y, int ldy) {
    const int B = w->blocks;
    const int S = (B + kStretch - 1) / kStretch;
    const int waves = min(S, 16);
    const size_t lds = (size_t)S * kTileRows * sizeof(float);
    GX_CHECK(lds <= 64 * 1024, "gx: a %d-input Q4_0 row is wider than this kernel's LDS", w->cols);
    dim3 grid(w->tiles, units);
    q4_0_matvec_kernel<1, true><<<grid, 64 * waves, lds, ctx->stream>>>(
        w->dev, w->plane0_bytes, B, w->dchunks, q, scales, qsum, w->cols, 0, 0, w->rows, nullptr, y, ldy,
        unit_expert, w->matrix_bytes, act_div, w->count);
    return check_launch("q4_0_matvec_units");
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
