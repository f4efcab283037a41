// gx_quant.hip - the activation quantisers of nn.Batch on the device.
//
// Q8_0 (Batch.quantizeBlock, nn/batch.go:109-143) and Q8_K (Batch.QuantizeK,
// nn/batch.go:159-213), bit for bit: IEEE division for the scale and its
// inverse (the inverse is 127/peak, a division, not 1/scale), golem's
// round-half-even (nearestInt), the Q8_0 scale rounded through fp16, and the
// Q8_K extreme taken as the first element of largest magnitude.
#include "gx_device.hpp"
#include "gx_internal.hpp"

namespace gx {
namespace {

// One lane per element, 32 lanes per block: a wavefront quantises two blocks.
// x is [M][ldx]; q [M][K], scales/qsum/corr [M][K/32]; q16 in panel order
// (q16_offset), over Mp = ceil(M/32)*32 tokens, the ones past M zero.
__global__ __launch_bounds__(256) void quantize_q8_0_kernel(const float *__restrict__ x, int ldx, int M, int Mp,
                                                            int K, int8_t *__restrict__ q,
                                                            float *__restrict__ scales, int32_t *__restrict__ qsum,
                                                            float *__restrict__ corr, uint16_t *__restrict__ q16) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    // M*K and Mp*K are multiples of 32 and blocks are 256 threads, so a
    // 32-lane group is wholly inside or wholly outside each range.
    if (gid >= (size_t)(q16 ? Mp : M) * K)
        return;
    const int m = (int)(gid / K), k = (int)(gid % K);
    const size_t o16 = q16 ? q16_offset(m, k, K >> 5) : 0;
    if (m >= M) {  // padding tokens of the fp16 copy
        q16[o16] = 0;
        return;
    }
    const float v = x[(size_t)m * ldx + k];
    float peak = fabsf(v);
#pragma unroll
    for (int off = 16; off > 0; off >>= 1)
        peak = fmaxf(peak, __shfl_xor(peak, off, 32));
    const int block = k >> 5;
    const size_t index = (size_t)m * (K >> 5) + block;
    if (peak == 0.0f) {
        q[gid] = 0;
        if (q16)
            q16[o16] = 0;
        if ((k & 31) == 0) {
            scales[index] = 0.0f;
            qsum[index] = 0;
            if (corr)
                corr[index] = 0.0f;
        }
        return;
    }
    const float scale = __fdiv_rn(peak, 127.0f);
    const float inverse = __fdiv_rn(127.0f, peak);
    const float stored = half_bits_to_float(float_to_half_bits(scale));
    const float prod = v * inverse;
    int32_t n = nearest_int(prod);
    n = n > 127 ? 127 : (n < -128 ? -128 : n);
    q[gid] = (int8_t)n;
    if (q16)  // the same integer as fp16 (exact: |n| <= 128)
        q16[o16] = float_to_half_bits((float)n);
    int32_t sum = n;
#pragma unroll
    for (int off = 16; off > 0; off >>= 1)
        sum += __shfl_xor(sum, off, 32);
    if ((k & 31) == 0) {
        scales[index] = stored;
        qsum[index] = sum;
        if (corr) {
            const float eight_scale = 8.0f * stored;
            corr[index] = eight_scale * (float)sum;
        }
    }
}

// One wavefront per 256-element superblock, four consecutive elements per
// lane.  x is [M][ldx]; q [M][K], kscales [M][K/256], bsums [M][K/16].
__global__ __launch_bounds__(256) void quantize_q8_k_kernel(const float *__restrict__ x, int ldx, int M, int K,
                                                            int8_t *__restrict__ q, float *__restrict__ kscales,
                                                            int16_t *__restrict__ bsums) {
    const int lane = threadIdx.x & 63;
    const size_t sb = (size_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int nsb = K / kSuper;
    if (sb >= (size_t)M * nsb)
        return;
    const int m = (int)(sb / nsb), b = (int)(sb % nsb);
    const float4 v4 = *(const float4 *)(x + (size_t)m * ldx + (size_t)b * kSuper + 4 * lane);
    const float v[4] = {v4.x, v4.y, v4.z, v4.w};
    int32_t gsum;
    float ks;
    const uint32_t packed = q8_k_wave(v, lane, &gsum, &ks);
    *(uint32_t *)(q + (size_t)m * K + (size_t)b * kSuper + 4 * lane) = packed;
    if ((lane & 3) == 0)
        bsums[(size_t)m * (K / 16) + (size_t)b * 16 + (lane >> 2)] = (int16_t)gsum;
    if (lane == 0)
        kscales[(size_t)m * nsb + b] = ks;
}

}  // namespace

int launch_quantize_q8_0(gx_ctx *ctx, const float *x, int ldx, int M, int K, int8_t *q, float *scales, int32_t *qsum,
                         float *corr, uint16_t *q16) {
    const int Mp = (M + 31) / 32 * 32;
    const size_t total = (size_t)(q16 ? Mp : M) * K;
    const int threads = 256;
    quantize_q8_0_kernel<<<(unsigned)((total + threads - 1) / threads), threads, 0, ctx->stream>>>(
        x, ldx, M, Mp, K, q, scales, qsum, corr, q16);
    return check_launch("quantize_q8_0");
}

int launch_quantize_q8_k(gx_ctx *ctx, const float *x, int ldx, int M, int K, int8_t *q, float *kscales,
                         int16_t *bsums) {
    GX_CHECK(ldx % 4 == 0, "gx: the Q8_K quantiser needs ldx a multiple of 4");
    const size_t sbs = (size_t)M * (K / kSuper);
    const int per_block = 4;  // wavefronts per 256-thread block
    quantize_q8_k_kernel<<<(unsigned)((sbs + per_block - 1) / per_block), 64 * per_block, 0, ctx->stream>>>(
        x, ldx, M, K, q, kscales, bsums);
    return check_launch("quantize_q8_k");
}

}  // namespace gx
