// gx_f32.hip - float32 matrix-vector product in golem's generic DotF32 order.
//
// Matrix.rows' F32 case (nn/matrix.go:113-120) calls DotF32 (nn/dot_f32.go:
// 13-33) per (row, column): four accumulators take the elements i = 4t + j in
// turn, mul then add, the elements past the last whole four go to the first,
// and the result is (s0 + s1) + (s2 + s3).  Each accumulator is a serial
// chain, so four lanes run the four chains of one dot and meet through two
// shuffles in exactly that final order.  This is the router of golem's MoE
// (gemma/moe.go:48), whose logits decide the experts; reproducing the order
// makes the selection identical, not merely close.
#include "gx_device.hpp"
#include "gx_internal.hpp"

namespace gx {
namespace {

__global__ __launch_bounds__(256) void f32_matvec_kernel(const float *__restrict__ W, int cols,
                                                         const float *__restrict__ x, int ldx, int M, int row_start,
                                                         int nrows, float *__restrict__ y, int ldy) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t dot = gid >> 2;
    const int j = (int)(gid & 3);
    const bool live = dot < (size_t)M * nrows;
    const int m = live ? (int)(dot / nrows) : 0;
    const int row = live ? row_start + (int)(dot % nrows) : row_start;
    const float *a = W + (size_t)row * cols;
    const float *b = x + (size_t)m * ldx;
    float s = 0.0f;
    if (live) {
        const int whole = cols & ~3;
        for (int i = j; i < whole; i += 4) {
            const float p = a[i] * b[i];
            s = s + p;
        }
        if (j == 0)
            for (int i = whole; i < cols; i++) {
                const float p = a[i] * b[i];
                s = s + p;
            }
    }
    // (s0 + s1) + (s2 + s3): pairs first, then the two pair sums.
    const float pair = s + __shfl_xor(s, 1, 4);
    const float other = __shfl_xor(pair, 2, 4);
    if (live && j == 0)
        y[(size_t)m * ldy + row] = pair + other;
}

}  // namespace

int launch_f32_matvec(gx_ctx *ctx, const gx_weight *w, const float *x, int ldx, int M, int row_start, int row_end,
                      float *y, int ldy) {
    const int nrows = row_end - row_start;
    const size_t lanes = (size_t)M * nrows * 4;
    const int threads = 256;
    f32_matvec_kernel<<<(unsigned)((lanes + threads - 1) / threads), threads, 0, ctx->stream>>>(
        (const float *)w->dev, w->cols, x, ldx, M, row_start, nrows, y, ldy);
    return check_launch("f32_matvec");
}

}  // namespace gx
