// gx_layout.hip - repacking GGUF blocks into the R64 device layout, and
// expanding single rows back to floats (Matrix.Row).
#include "gx_device.hpp"
#include "gx_internal.hpp"

namespace gx {
namespace {

// One thread per (matrix, row, block): the 18-byte Q4_0 block
// (nn/dot_q4_0.go:3-13, scale first) is split into its 16 nibble bytes (plane
// 0, chunk = block) and its fp16 scale (plane 1, 8 blocks per chunk).
__global__ void repack_q4_0_kernel(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, int rows, int blocks,
                                   int dchunks, size_t plane0_bytes, size_t matrix_bytes, int count) {
    const size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t per_matrix = (size_t)rows * blocks;
    if (id >= per_matrix * count)
        return;
    const int e = (int)(id / per_matrix);
    const size_t rb = id % per_matrix;
    const int row = (int)(rb / blocks), b = (int)(rb % blocks);
    const uint8_t *s = src + ((size_t)e * per_matrix + rb) * kQ4BlockBytes;
    uint8_t *m = dst + (size_t)e * matrix_bytes;
    const int tile = row >> 6, r = row & 63;
    uint8_t *qs = m + (((size_t)tile * blocks + b) * kTileRows + r) * kChunk;
#pragma unroll
    for (int j = 0; j < 16; j++)
        qs[j] = s[2 + j];
    uint8_t *d = m + plane0_bytes + (((size_t)tile * dchunks + (b >> 3)) * kTileRows + r) * kChunk + (b & 7) * 2;
    d[0] = s[0];
    d[1] = s[1];
}

// One thread per (matrix, row, superblock): the 210-byte Q6_K superblock
// (ql 128 | qh 64 | scales 16 | fp16 d, nn/dequant_q6_k.go:3-15) becomes 13
// chunks of plane 0 and one fp16 of plane 1.
__global__ void repack_q6_k_kernel(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, int rows, int blocks,
                                   int dchunks, size_t plane0_bytes, size_t matrix_bytes, int count) {
    const size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t per_matrix = (size_t)rows * blocks;
    if (id >= per_matrix * count)
        return;
    const int e = (int)(id / per_matrix);
    const size_t rb = id % per_matrix;
    const int row = (int)(rb / blocks), b = (int)(rb % blocks);
    const uint8_t *s = src + ((size_t)e * per_matrix + rb) * kQ6BlockBytes;
    uint8_t *m = dst + (size_t)e * matrix_bytes;
    const int tile = row >> 6, r = row & 63;
    for (int c = 0; c < kQ6Chunks; c++) {
        uint8_t *o = m + ((((size_t)tile * blocks + b) * kQ6Chunks + c) * kTileRows + r) * kChunk;
        for (int j = 0; j < 16; j++)
            o[j] = s[c * 16 + j];
    }
    uint8_t *d = m + plane0_bytes + (((size_t)tile * dchunks + (b >> 3)) * kTileRows + r) * kChunk + (b & 7) * 2;
    d[0] = s[208];
    d[1] = s[209];
}

// Matrix.Row for Q4_0 (dequantizeQ4_0Row, nn/matrix.go:175-190): one thread
// per (output row, block); float(n - 8) * scale, one rounding.
__global__ void rows_q4_0_kernel(const uint8_t *__restrict__ m, int rows, int blocks, int dchunks,
                                 size_t plane0_bytes, const int32_t *__restrict__ ids, int n,
                                 float *__restrict__ out) {
    const int id = blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= n * blocks)
        return;
    const int i = id / blocks, b = id % blocks;
    const int row = ids[i];
    if (row < 0 || row >= rows) {  // an id out of range reads nothing and yields NaN
        for (int j = 0; j < kQ4Block; j++)
            out[(size_t)i * blocks * kQ4Block + (size_t)b * kQ4Block + j] = __builtin_nanf("");
        return;
    }
    const int tile = row >> 6, r = row & 63;
    const uint4 w = *(const uint4 *)(m + (((size_t)tile * blocks + b) * kTileRows + r) * kChunk);
    const uint4 dc = *(const uint4 *)(m + plane0_bytes + (((size_t)tile * dchunks + (b >> 3)) * kTileRows + r) * kChunk);
    const float scale = chunk_half(dc, b & 7);
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
    float *dst = out + (size_t)i * blocks * kQ4Block + (size_t)b * kQ4Block;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const uint32_t byte = (words[j >> 2] >> (8 * (j & 3))) & 0xFF;
        dst[j] = (float)((int32_t)(byte & 0x0F) - 8) * scale;
        dst[j + 16] = (float)((int32_t)(byte >> 4) - 8) * scale;
    }
}

// Matrix.Row for Q6_K (DequantizeQ6_K, nn/dequant_q6_k.go:18-51): one thread
// per (output row, superblock, i in 0..63), writing the four values of one
// (half, i) position: (d * scale) * float(q - 32), two roundings.
__global__ void rows_q6_k_kernel(const uint8_t *__restrict__ m, int rows, int blocks, int dchunks,
                                 size_t plane0_bytes, const int32_t *__restrict__ ids, int n,
                                 float *__restrict__ out) {
    const int id = blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= n * blocks * 64)
        return;
    const int pos = id & 63;
    const int b = (id >> 6) % blocks, i_out = (id >> 6) / blocks;
    const int half = pos >> 5, i = pos & 31;
    const int row = ids[i_out];
    if (row < 0 || row >= rows) {
        float *dst = out + (size_t)i_out * blocks * kSuper + (size_t)b * kSuper + half * 128;
        dst[i] = dst[i + 32] = dst[i + 64] = dst[i + 96] = __builtin_nanf("");
        return;
    }
    const int tile = row >> 6, r = row & 63;
    const uint8_t *base = m + (((size_t)tile * blocks + b) * kQ6Chunks * kTileRows + r) * kChunk;
    auto byte_at = [&](int off) -> uint32_t {  // byte `off` of the 208-byte superblock body
        return base[(size_t)(off >> 4) * kTileRows * kChunk + (off & 15)];
    };
    const uint8_t *dptr = m + plane0_bytes + (((size_t)tile * dchunks + (b >> 3)) * kTileRows + r) * kChunk + (b & 7) * 2;
    const float d = half_bits_to_float((uint32_t)dptr[0] | ((uint32_t)dptr[1] << 8));
    const uint32_t l0 = byte_at(half * 64 + i), l1 = byte_at(half * 64 + i + 32), h = byte_at(128 + half * 32 + i);
    const int group = i / 16;
    const int8_t s0 = (int8_t)byte_at(192 + half * 8 + group + 0);
    const int8_t s1 = (int8_t)byte_at(192 + half * 8 + group + 2);
    const int8_t s2 = (int8_t)byte_at(192 + half * 8 + group + 4);
    const int8_t s3 = (int8_t)byte_at(192 + half * 8 + group + 6);
    const int32_t q1 = (int32_t)(l0 & 0x0F) | (int32_t)((h >> 0) & 3) << 4;
    const int32_t q2 = (int32_t)(l1 & 0x0F) | (int32_t)((h >> 2) & 3) << 4;
    const int32_t q3 = (int32_t)(l0 >> 4) | (int32_t)((h >> 4) & 3) << 4;
    const int32_t q4 = (int32_t)(l1 >> 4) | (int32_t)((h >> 6) & 3) << 4;
    float *dst = out + (size_t)i_out * blocks * kSuper + (size_t)b * kSuper + half * 128;
    dst[i + 0] = d * (float)s0 * (float)(q1 - 32);
    dst[i + 32] = d * (float)s1 * (float)(q2 - 32);
    dst[i + 64] = d * (float)s2 * (float)(q3 - 32);
    dst[i + 96] = d * (float)s3 * (float)(q4 - 32);
}

__global__ void rows_f32_kernel(const float *__restrict__ m, int rows, int cols, const int32_t *__restrict__ ids,
                                int n, float *__restrict__ out) {
    const size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= (size_t)n * cols)
        return;
    const int i = (int)(id / cols), c = (int)(id % cols);
    const int row = ids[i];
    out[id] = (row < 0 || row >= rows) ? __builtin_nanf("") : m[(size_t)row * cols + c];
}

}  // namespace

int launch_repack(gx_ctx *ctx, const uint8_t *src, gx_weight *w) {
    const size_t n = (size_t)w->rows * w->blocks * w->count;
    const int threads = 256;
    const unsigned grid = (unsigned)((n + threads - 1) / threads);
    if (w->quant == GX_Q4_0)
        repack_q4_0_kernel<<<grid, threads, 0, ctx->stream>>>(src, w->dev, w->rows, w->blocks, w->dchunks,
                                                               w->plane0_bytes, w->matrix_bytes, w->count);
    else
        repack_q6_k_kernel<<<grid, threads, 0, ctx->stream>>>(src, w->dev, w->rows, w->blocks, w->dchunks,
                                                               w->plane0_bytes, w->matrix_bytes, w->count);
    return check_launch("repack");
}

int launch_rows(gx_ctx *ctx, const gx_weight *w, int expert, const int32_t *ids, int n, float *out) {
    const uint8_t *m = w->dev + (size_t)expert * w->matrix_bytes;
    const int threads = 256;
    if (w->quant == GX_Q4_0) {
        const int total = n * w->blocks;
        rows_q4_0_kernel<<<(total + threads - 1) / threads, threads, 0, ctx->stream>>>(
            m, w->rows, w->blocks, w->dchunks, w->plane0_bytes, ids, n, out);
    } else if (w->quant == GX_Q6_K) {
        const int total = n * w->blocks * 64;
        rows_q6_k_kernel<<<(total + threads - 1) / threads, threads, 0, ctx->stream>>>(
            m, w->rows, w->blocks, w->dchunks, w->plane0_bytes, ids, n, out);
    } else {
        const size_t total = (size_t)n * w->cols;
        rows_f32_kernel<<<(unsigned)((total + threads - 1) / threads), threads, 0, ctx->stream>>>(
            (const float *)m, w->rows, w->cols, ids, n, out);
    }
    return check_launch("rows");
}

}  // namespace gx
