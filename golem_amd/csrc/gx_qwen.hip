// gx_qwen.hip - the pieces of golem's Qwen3 dense block (qwen/) that sit
// between the quantised products, on the device.
//
// A block for M consecutive positions (qwen/block.go:32-102) runs as
//   norm_quant      x += add (the previous half's residual); RMSNormPlain(x,
//                   gain); Q8_0 of the result          (block.go:45-52, 59-68)
//   Q|K|V product   one Q4_0 matrix, the three stacked by rows
//   qk_rope         per head: RMSNormPlain(head, q_norm / k_norm), RoPE,
//                   the query rounded through fp16, the key and value stored
//                   into the layer's fp16 cache       (attention.go:57-84,
//                                                      cache.go:52-60)
//   attention       per (position, head): scale * DotF32(query, key) over the
//                   visible prefix, SoftmaxInPlace, probabilities rounded
//                   through fp16, Axpy of the values in position order, Q8_0
//                   of the head                       (attention.go:96-124)
//   O product, norm_quant (x += attention), Gate|Up product (stacked),
//   swiglu_quant    silu(gate) * up with ggml's expf, Q8_0 (block.go:82-90,
//                   nn/swiglu.go:31-82)
//   Down product; its residual add opens the next block's norm_quant.
// argmax_kernel is the greedy pick over logits (ties to the lower id).
//
// The per-head RMSNormPlain sums its 128 squares left to right in float64, as
// golem does; the width-wide one uses the fixed tree of gx_device.hpp.
#include "gx_device.hpp"
#include "gx_internal.hpp"

namespace gx {
namespace {

constexpr int kQNormThreads = 1024;

// One position per workgroup: x (and add) [M][ld], gain [K].  out, when given,
// receives the normed floats [M][ldo]; q/scales/qsum receive its Q8_0 form.
// RMSNormPlain's float64 sum is the tree of gx_device.hpp (512 partials,
// partial t = elements t, t+512, ... in order, halved pairwise), here with
// the partials held by threads 0..511.
__global__ __launch_bounds__(kQNormThreads) void qwen_norm_quant_kernel(float *__restrict__ x, int ldx,
                                                                        const float *__restrict__ add, int lda,
                                                                        const float *__restrict__ gain, int K,
                                                                        float eps, float *__restrict__ out, int ldo,
                                                                        int8_t *__restrict__ q,
                                                                        float *__restrict__ scales,
                                                                        int32_t *__restrict__ qsum) {
    extern __shared__ float xs[];  // K floats, then the K gains
    float *gl = xs + K;
    __shared__ double red[512];
    __shared__ float scale_sh;
    const int tid = threadIdx.x, t = blockIdx.x;
    float *xr = x + (size_t)t * ldx;
    const float *ar = add ? add + (size_t)t * lda : nullptr;
#pragma unroll 4
    for (int i = tid; i < K; i += kQNormThreads) {
        const float v = xr[i];
        const float a = ar ? ar[i] : 0.0f;
        gl[i] = gain[i];
        xs[i] = ar ? v + a : v;
    }
    __syncthreads();
    if (ar)  // the residual, written back
        for (int i = tid; i < K; i += kQNormThreads)
            xr[i] = xs[i];
    if (tid < 512) {
        double part = 0.0;
        for (int i = tid; i < K; i += 512) {
            const float v = xs[i];
            const float sq = v * v;
            part += (double)sq;
        }
        red[tid] = part;
    }
    __syncthreads();
    double s = 0.0;
    if (tid < 256)
        s = red[tid] + red[tid + 256];  // w = 256
    __syncthreads();
    if (tid < 256)
        red[tid] = s;
    __syncthreads();
    if (tid < 128)
        s = s + red[tid + 128];
    __syncthreads();
    if (tid < 128)
        red[tid] = s;
    __syncthreads();
    if (tid < 64) {
        s = s + red[tid + 64];
        for (int w = 32; w > 0; w >>= 1) {
            const double o = __shfl_down(s, w, 64);
            if (tid < w)
                s = s + o;
        }
        if (tid == 0)
            scale_sh = norm_scale(s, K, eps);
    }
    __syncthreads();
    const float sc = scale_sh;
    // Element i = j*1024 + tid: a 32-lane group covers one Q8_0 block.
    const int B = K >> 5;
    for (int base = 0; base < K; base += kQNormThreads) {
        const int i = base + tid;
        if (i < K) {  // K % 32 == 0: whole groups in or out
            const float v = xs[i] * sc;
            const float nv = v * gl[i];
            if (out)
                out[(size_t)t * ldo + i] = nv;
            if (q) {
                float stored;
                int32_t sm;
                const int32_t n = q8_0_lane(nv, &stored, &sm);
                q[(size_t)t * K + i] = (int8_t)n;
                if ((i & 31) == 0) {
                    scales[(size_t)t * B + (i >> 5)] = stored;
                    qsum[(size_t)t * B + (i >> 5)] = sm;
                }
            }
        }
    }
}

// RMSNormPlain of one head of hd floats held two per lane (lane owns i and
// i + 64), the float64 sum taken left to right by lane 0 from LDS.
__device__ __forceinline__ float head_norm_scale(const float *h, int hd, float eps) {
    double s = 0.0;
    for (int i = 0; i < hd; i++) {
        const float v = h[i];
        const float sq = v * v;
        s += (double)sq;
    }
    const float mean = (float)(s / (double)hd);
    return (float)(1.0 / sqrt((double)(mean + eps)));
}

constexpr int kHeadMax = 256;  // head_dim limit (two values per lane)

// grid (M, heads + kv_heads), one wavefront.  qkv [M][ldqkv] holds each
// position's Q rows, then K rows, then V rows.  rope_cos/sin are [context][hd/2].
// Query heads: normed, rotated, rounded to fp16 into qh [M][heads*hd].  Key-
// value heads: the key normed and rotated, both rounded to fp16 into the
// layer's caches at [pos][kvh][hd].
__global__ __launch_bounds__(64) void qwen_qk_rope_kernel(const float *__restrict__ qkv, int ldqkv, int heads,
                                                          int kv_heads, int hd, const int32_t *__restrict__ positions,
                                                          const float *__restrict__ q_norm,
                                                          const float *__restrict__ k_norm,
                                                          const float *__restrict__ rope_cos,
                                                          const float *__restrict__ rope_sin, float eps,
                                                          uint16_t *__restrict__ qh, uint16_t *__restrict__ kcache,
                                                          uint16_t *__restrict__ vcache) {
    __shared__ float h[kHeadMax];
    __shared__ float sc_sh;
    const int lane = threadIdx.x, t = blockIdx.x, u = blockIdx.y;
    const int pos = positions[t];
    const int half = hd >> 1;
    const bool is_q = u < heads;
    const int col = is_q ? u * hd : heads * hd + (u - heads) * hd;
    const float *src = qkv + (size_t)t * ldqkv + col;
    for (int i = lane; i < hd; i += 64)
        h[i] = src[i];
    __syncthreads();
    if (lane == 0)
        sc_sh = head_norm_scale(h, hd, eps);
    __syncthreads();
    const float sc = sc_sh;
    const float *gain = is_q ? q_norm : k_norm;
    // normed, then rotated in pairs (i, i + half): RoPETable.Apply, nn/rope.go:62-73
    for (int i = lane; i < half; i += 64) {
        const float re0 = h[i], im0 = h[i + half];
        const float re = (re0 * sc) * gain[i], im = (im0 * sc) * gain[i + half];
        const float c = rope_cos[(size_t)pos * half + i], s = rope_sin[(size_t)pos * half + i];
        const float a = re * c - im * s;
        const float b = re * s + im * c;
        if (is_q) {
            qh[(size_t)t * heads * hd + u * hd + i] = (uint16_t)float_to_half_bits(a);
            qh[(size_t)t * heads * hd + u * hd + i + half] = (uint16_t)float_to_half_bits(b);
        } else {
            const size_t o = ((size_t)pos * kv_heads + (u - heads)) * hd;
            kcache[o + i] = (uint16_t)float_to_half_bits(a);
            kcache[o + i + half] = (uint16_t)float_to_half_bits(b);
        }
    }
    if (!is_q) {
        const float *vsrc = qkv + (size_t)t * ldqkv + (heads + kv_heads) * hd + (u - heads) * hd;
        const size_t o = ((size_t)pos * kv_heads + (u - heads)) * hd;
        for (int i = lane; i < hd; i += 64)
            vcache[o + i] = (uint16_t)float_to_half_bits(vsrc[i]);
    }
}

// grid (M, kv_heads), 256 threads: position t's G = heads / kv_heads query
// heads that read key-value head kvh, against the layer's cache over
// positions 0 .. positions[t] (n of them).  Per query head, in golem's order:
// scores (scale * DotF32), SoftmaxInPlace (max; exp in float64; the sum taken
// position by position by one thread; the division), probabilities rounded
// to fp16, then dst = sum over positions in order of Axpy(value, probability)
// -- G * hd independent chains, two per thread.  The key and value rows are
// read once for the G heads.  Values pass through LDS in chunks of kAttnChunk
// positions, fetched two chunks ahead.  The heads' outputs are quantised
// (Q8_0) into q/scales/qsum at columns (kvh*G + g)*hd of a [M][heads*hd] batch.
constexpr int kAttnThreads = 256;
constexpr int kAttnChunk = 32;   // positions per value chunk
constexpr int kAttnDepth = 3;    // value chunks in LDS (two in flight)

template <int G, int HD>
__global__ __launch_bounds__(kAttnThreads) void qwen_attention_kernel(const uint16_t *__restrict__ qh, int kv_heads,
                                                                      const int32_t *__restrict__ positions,
                                                                      const uint16_t *__restrict__ kcache,
                                                                      const uint16_t *__restrict__ vcache,
                                                                      float scale, int sstride,
                                                                      int8_t *__restrict__ q,
                                                                      float *__restrict__ scales,
                                                                      int32_t *__restrict__ qsum) {
    constexpr int hd = HD;
    extern __shared__ float lds[];
    float *query = lds;                                  // [G][hd]
    float *scores = query + G * kHeadMax;                // [G][sstride]
    uint16_t *vbuf = (uint16_t *)(scores + G * sstride); // [kAttnDepth][kAttnChunk][hd]
    __shared__ float red[kAttnThreads / 64][G];
    __shared__ float total[G];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int t = blockIdx.x, kvh = blockIdx.y;
    const int heads = G * kv_heads, width = heads * hd;
    const int n = positions[t] + 1;
    for (int c = tid; c < G * hd; c += kAttnThreads) {
        const int g = c / hd, i = c - g * hd;
        query[g * kHeadMax + i] = half_bits_to_float(qh[(size_t)t * width + (kvh * G + g) * hd + i]);
    }
    __syncthreads();

    // Scores: a thread per position; the key row is read once for the G heads.
    float mx[G];
#pragma unroll
    for (int g = 0; g < G; g++)
        mx[g] = -INFINITY;
    for (int p = tid; p < n; p += kAttnThreads) {
        const uint16_t *key = kcache + ((size_t)p * kv_heads + kvh) * hd;
        float s[G][4];
#pragma unroll
        for (int g = 0; g < G; g++)
            s[g][0] = s[g][1] = s[g][2] = s[g][3] = 0.0f;
        v4u_stream kr[hd / 8];  // the whole key row first
#pragma unroll
        for (int i = 0; i < hd; i += 8)
            kr[i / 8] = *(const v4u_stream *)(key + i);
#pragma unroll
        for (int i = 0; i < hd; i += 8) {
            const v4u_stream kw = kr[i / 8];
            const uint32_t w4[4] = {kw.x, kw.y, kw.z, kw.w};
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float kv = half_bits_to_float((w4[j >> 1] >> (16 * (j & 1))) & 0xFFFFu);
#pragma unroll
                for (int g = 0; g < G; g++) {
                    const float pr = query[g * kHeadMax + i + j] * kv;
                    s[g][j & 3] = s[g][j & 3] + pr;
                }
            }
        }
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float dot = (s[g][0] + s[g][1]) + (s[g][2] + s[g][3]);
            const float sc = scale * dot;
            scores[g * sstride + p] = sc;
            mx[g] = fmaxf(mx[g], sc);
        }
    }
#pragma unroll
    for (int g = 0; g < G; g++) {
        for (int off = 32; off > 0; off >>= 1)
            mx[g] = fmaxf(mx[g], __shfl_xor(mx[g], off, 64));
        if (lane == 0)
            red[wave][g] = mx[g];
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; g++) {
        float m = red[0][g];
        for (int w = 1; w < kAttnThreads / 64; w++)
            m = fmaxf(m, red[w][g]);
        for (int p = tid; p < n; p += kAttnThreads)
            scores[g * sstride + p] = (float)exp((double)(scores[g * sstride + p] - m));
    }
    __syncthreads();
    if (tid < G) {  // SoftmaxInPlace's sum, position by position (read 16 at a time)
        const float *e = scores + tid * sstride;
        float sum = 0.0f;
        int p = 0;
        for (; p + 16 <= n; p += 16) {
            float v[16];
#pragma unroll
            for (int j = 0; j < 16; j++)
                v[j] = e[p + j];
#pragma unroll
            for (int j = 0; j < 16; j++)
                sum += v[j];
        }
        for (; p < n; p++)
            sum += e[p];
        total[tid] = sum;
    }

    // Value chunks: chunk k holds positions k*kAttnChunk ..; thread tid carries
    // hd*kAttnChunk/(8*256) 16-byte pieces of a chunk.
    const int pieces = hd * kAttnChunk / 8;  // uint4 per chunk
    const int chunks = (n + kAttnChunk - 1) / kAttnChunk;
    v4u_stream stage[2][2];  // up to two pieces per thread (hd <= 128), two chunks ahead
#define GX_ATTN_FETCH(k, slot)                                                                                       \
    do {                                                                                                             \
        _Pragma("unroll") for (int r = 0; r < 2; r++) {                                                            \
            const int pc = tid + r * kAttnThreads;                                                                   \
            if (pc < pieces) {                                                                                       \
                const int pp = (k) * kAttnChunk + pc / (hd / 8);                                                     \
                const int col = (pc % (hd / 8)) * 8;                                                                 \
                stage[slot][r] = *(const v4u_stream *)(vcache + ((size_t)min(pp, n - 1) * kv_heads + kvh) * hd + col); \
            }                                                                                                        \
        }                                                                                                            \
    } while (0)
#define GX_ATTN_PUT(k, slot)                                                                                         \
    do {                                                                                                             \
        uint16_t *vb = vbuf + (size_t)((k) % kAttnDepth) * kAttnChunk * hd;                                          \
        _Pragma("unroll") for (int r = 0; r < 2; r++) {                                                            \
            const int pc = tid + r * kAttnThreads;                                                                   \
            if (pc < pieces)                                                                                         \
                *(v4u_stream *)(vb + (pc / (hd / 8)) * hd + (pc % (hd / 8)) * 8) = stage[slot][r];                  \
        }                                                                                                            \
    } while (0)
    GX_ATTN_FETCH(0, 0);
    if (chunks > 1)
        GX_ATTN_FETCH(1, 1);
    GX_ATTN_PUT(0, 0);
    __syncthreads();
    // probabilities, rounded through fp16 (SoftmaxInPlace's division)
#pragma unroll
    for (int g = 0; g < G; g++)
        for (int p = tid; p < n; p += kAttnThreads)
            scores[g * sstride + p] = half_bits_to_float(float_to_half_bits(scores[g * sstride + p] / total[g]));
    if (chunks > 1)
        GX_ATTN_PUT(1, 1);
    __syncthreads();

    const int c0 = tid, c1 = tid + kAttnThreads;  // chains (head, element)
    // a thread without a chain computes on head G - 1 (in bounds) and stores nothing
    const int g0 = min(c0 / hd, G - 1), i0 = c0 - (c0 / hd) * hd;
    const int g1 = min(c1 / hd, G - 1), i1 = c1 - (c1 / hd) * hd;
    float d0 = 0.0f, d1 = 0.0f;
#define GX_ATTN_CHUNK(k, slot)                                                                                       \
    do {                                                                                                             \
        if ((k) + 2 < chunks)                                                                                        \
            GX_ATTN_FETCH((k) + 2, slot);                                                                            \
        const uint16_t *vb = vbuf + (size_t)((k) % kAttnDepth) * kAttnChunk * hd;                                    \
        const int p0 = (k) * kAttnChunk, pn = min(kAttnChunk, n - p0);                                               \
        if (pn == kAttnChunk) { /* a whole chunk: reads first, then the two chains in order */                       \
            for (int jb = 0; jb < kAttnChunk; jb += 8) {                                                             \
                float a0[8], v0[8], a1[8], v1[8];                                                                    \
                _Pragma("unroll") for (int j = 0; j < 8; j++) {                                                      \
                    a0[j] = scores[g0 * sstride + p0 + jb + j];                                                      \
                    v0[j] = half_bits_to_float(vb[(jb + j) * hd + i0]);                                              \
                    a1[j] = scores[g1 * sstride + p0 + jb + j];                                                      \
                    v1[j] = half_bits_to_float(vb[(jb + j) * hd + i1]);                                              \
                }                                                                                                    \
                _Pragma("unroll") for (int j = 0; j < 8; j++) {                                                      \
                    const float m0 = a0[j] * v0[j];                                                                  \
                    d0 = d0 + m0;                                                                                    \
                    const float m1 = a1[j] * v1[j];                                                                  \
                    d1 = d1 + m1;                                                                                    \
                }                                                                                                    \
            }                                                                                                        \
        } else {                                                                                                     \
            for (int j = 0; j < pn; j++) {                                                                           \
                const float m0 = scores[g0 * sstride + p0 + j] * half_bits_to_float(vb[j * hd + i0]);                \
                d0 = d0 + m0;                                                                                        \
                const float m1 = scores[g1 * sstride + p0 + j] * half_bits_to_float(vb[j * hd + i1]);                \
                d1 = d1 + m1;                                                                                        \
            }                                                                                                        \
        }                                                                                                            \
        if ((k) + 2 < chunks) /* chunk k + 2 into the buffer chunk k - 1 used */                                     \
            GX_ATTN_PUT((k) + 2, slot);                                                                              \
        __syncthreads();                                                                                             \
    } while (0)
    // Chunk k's registers are slot k & 1; the loop runs two chunks a pass so
    // that the slot is a constant.
    for (int k = 0; k < chunks; k += 2) {
        GX_ATTN_CHUNK(k, 0);
        if (k + 1 < chunks)
            GX_ATTN_CHUNK(k + 1, 1);
    }
#undef GX_ATTN_CHUNK
#undef GX_ATTN_FETCH
#undef GX_ATTN_PUT
    // Q8_0 of the heads: consecutive chains are consecutive elements of one
    // head (hd % 32 == 0), so a 32-lane group is one block.
    const int B = width >> 5;
    for (int r = 0; r < 2; r++) {
        const int c = r == 0 ? c0 : c1;
        if (r * kAttnThreads < G * hd) {  // uniform
            if (c < G * hd) {             // whole 32-lane groups
                float stored;
                int32_t sm;
                const int32_t nq = q8_0_lane(r == 0 ? d0 : d1, &stored, &sm);
                const int col = (kvh * G + c / hd) * hd + (c % hd);
                q[(size_t)t * width + col] = (int8_t)nq;
                if ((col & 31) == 0) {
                    scales[(size_t)t * B + (col >> 5)] = stored;
                    qsum[(size_t)t * B + (col >> 5)] = sm;
                }
            }
        }
    }
}

// expf (ggml_v_expf one value at a time), nn/swiglu.go:31-74.
__device__ __forceinline__ float ggml_expf(float x) {
    const float shift = 0x1.8p23f;
    const float log2e = 0x1.715476p+0f;
    const float ln2hi = 0x1.62e4p-1f;
    const float ln2lo = 0x1.7f7d1cp-20f;
    const float c0 = 0x1.ffffecp-1f;
    const float c1 = 0x1.fffdb6p-2f;
    const float c2 = 0x1.555e66p-3f;
    const float c3 = 0x1.573e2ep-5f;
    const float c4 = 0x1.0e4020p-7f;
    const float z = x * log2e + shift;
    const float n = z - shift;
    if (n > 126.0f || n < -126.0f)
        return (float)exp((double)x);
    const float b = x - n * ln2hi - n * ln2lo;
    const float k = __uint_as_float((__float_as_uint(z) << 23) + __float_as_uint(1.0f));
    const float u = b * b;
    const float j = ((c4 * b + c3) * u + (c2 * b + c1)) * u + c0 * b;
    return j * k + k;
}

// grid (ceil(ffn/256), M): gu [M][ldgu] holds each position's gate then up
// (ffn each).  mid = silu(gate) * up (SwiGLURange, nn/swiglu.go:77-82), Q8_0.
__global__ __launch_bounds__(256) void qwen_swiglu_quant_kernel(const float *__restrict__ gu, int ldgu, int ffn,
                                                                int8_t *__restrict__ q, float *__restrict__ scales,
                                                                int32_t *__restrict__ qsum) {
    const int t = blockIdx.y;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= ffn)
        return;  // ffn % 32 == 0: whole groups
    const float g = gu[(size_t)t * ldgu + i];
    const float u = gu[(size_t)t * ldgu + ffn + i];
    const float e = ggml_expf(-g);
    const float den = 1.0f + e;
    const float sl = g / den;
    const float v = sl * u;
    float stored;
    int32_t s;
    const int32_t n = q8_0_lane(v, &stored, &s);
    q[(size_t)t * ffn + i] = (int8_t)n;
    if ((i & 31) == 0) {
        scales[(size_t)t * (ffn >> 5) + (i >> 5)] = stored;
        qsum[(size_t)t * (ffn >> 5) + (i >> 5)] = s;
    }
}

// One row per workgroup: the index of the largest value, the lower index on
// ties (NaN never wins).  Each thread scans a strided set of float4s, then the
// workgroup reduces (value, index) pairs.
constexpr int kArgmaxThreads = 1024;
__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(const float *__restrict__ x, int ldx, int n,
                                                                int32_t *__restrict__ out) {
    __shared__ float bv_sh[kArgmaxThreads];
    __shared__ int bi_sh[kArgmaxThreads];
    const int tid = threadIdx.x;
    const float *r = x + (size_t)blockIdx.x * ldx;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    auto take = [&](float v, int i) {
        if (v > bv || (bi == 0x7fffffff && v == v)) {  // scanned in rising order: equal values keep the first
            bv = v;
            bi = i;
        }
    };
    const bool vec = ((uintptr_t)r & 15) == 0;
    const int n4 = vec ? n / 4 : 0;
#pragma unroll 4
    for (int q = tid; q < n4; q += kArgmaxThreads) {
        const float4 v = *(const float4 *)(r + 4 * q);
        take(v.x, 4 * q);
        take(v.y, 4 * q + 1);
        take(v.z, 4 * q + 2);
        take(v.w, 4 * q + 3);
    }
    for (int i = 4 * n4 + tid; i < n; i += kArgmaxThreads)
        take(r[i], i);
    bv_sh[tid] = bv;
    bi_sh[tid] = bi;
    __syncthreads();
    for (int w = kArgmaxThreads / 2; w > 0; w >>= 1) {
        if (tid < w) {
            const float ov = bv_sh[tid + w];
            const int oi = bi_sh[tid + w];
            if (oi != 0x7fffffff && (bi_sh[tid] == 0x7fffffff || ov > bv_sh[tid] ||
                                     (ov == bv_sh[tid] && oi < bi_sh[tid]))) {
                bv_sh[tid] = ov;
                bi_sh[tid] = oi;
            }
        }
        __syncthreads();
    }
    if (tid == 0)
        out[blockIdx.x] = bi_sh[0] == 0x7fffffff ? 0 : bi_sh[0];
}

}  // namespace

int launch_qwen_norm_quant(gx_ctx *ctx, float *x, int ldx, const float *add, int lda, const float *gain, int M, int K,
                           float eps, float *out, int ldo, int8_t *q, float *scales, int32_t *qsum) {
    const size_t lds = 2 * sizeof(float) * (size_t)K;
    GX_CHECK(lds <= 64 * 1024, "gx: a norm over %d values does not fit the LDS", K);
    qwen_norm_quant_kernel<<<M, kQNormThreads, lds, ctx->stream>>>(x, ldx, add, lda, gain, K, eps, out, ldo, q,
                                                                   scales, qsum);
    return check_launch("qwen_norm_quant");
}

int launch_qwen_qk_rope(gx_ctx *ctx, const float *qkv, int ldqkv, int M, int heads, int kv_heads, int hd,
                        const int32_t *positions, const float *q_norm, const float *k_norm, const float *rope_cos,
                        const float *rope_sin, float eps, uint16_t *qh, uint16_t *kcache, uint16_t *vcache) {
    GX_CHECK(hd <= kHeadMax && hd % 2 == 0, "gx: head width %d unsupported (even, at most %d)", hd, kHeadMax);
    qwen_qk_rope_kernel<<<dim3((unsigned)M, (unsigned)(heads + kv_heads)), 64, 0, ctx->stream>>>(
        qkv, ldqkv, heads, kv_heads, hd, positions, q_norm, k_norm, rope_cos, rope_sin, eps, qh, kcache, vcache);
    return check_launch("qwen_qk_rope");
}

int launch_qwen_attention(gx_ctx *ctx, const uint16_t *qh, int M, int heads, int kv_heads, int hd, int max_pos,
                          const int32_t *positions, const uint16_t *kcache, const uint16_t *vcache, float scale,
                          int8_t *q, float *scales, int32_t *qsum) {
    const int G = heads / kv_heads;
    GX_CHECK(hd <= 128 && hd % 32 == 0, "gx: attention supports head widths that are multiples of 32 up to 128");
    GX_CHECK(G == 1 || G == 2 || G == 4 || G == 8, "gx: %d query heads per key-value head unsupported", G);
    GX_CHECK(G * hd <= 2 * kAttnThreads, "gx: %d query heads of %d per key-value head exceed the kernel's %d chains", G,
             hd, 2 * kAttnThreads);
    const int sstride = max_pos + 1;
    const size_t lds = sizeof(float) * ((size_t)G * kHeadMax + (size_t)G * sstride) +
                       sizeof(uint16_t) * (size_t)kAttnDepth * kAttnChunk * hd;
    GX_CHECK(lds <= 64 * 1024, "gx: attention over %d positions with %d heads per group does not fit the LDS",
             max_pos + 1, G);
    const dim3 grid((unsigned)M, (unsigned)kv_heads);
#define GX_ATTN_LAUNCH(GG, HH)                                                                                       \
    qwen_attention_kernel<GG, HH><<<grid, kAttnThreads, lds, ctx->stream>>>(qh, kv_heads, positions, kcache, vcache,  \
                                                                            scale, sstride, q, scales, qsum)
#define GX_ATTN_LAUNCH_HD(GG)                                                                                        \
    do {                                                                                                             \
        if (hd == 32)                                                                                                \
            GX_ATTN_LAUNCH(GG, 32);                                                                                  \
        else if (hd == 64)                                                                                           \
            GX_ATTN_LAUNCH(GG, 64);                                                                                  \
        else if (hd == 96)                                                                                           \
            GX_ATTN_LAUNCH(GG, 96);                                                                                  \
        else                                                                                                         \
            GX_ATTN_LAUNCH(GG, 128);                                                                                 \
    } while (0)
    if (G == 1)
        GX_ATTN_LAUNCH_HD(1);
    else if (G == 2)
        GX_ATTN_LAUNCH_HD(2);
    else if (G == 4)
        GX_ATTN_LAUNCH_HD(4);
    else
        GX_ATTN_LAUNCH_HD(8);
#undef GX_ATTN_LAUNCH_HD
#undef GX_ATTN_LAUNCH
    return check_launch("qwen_attention");
}

int launch_qwen_swiglu_quant(gx_ctx *ctx, const float *gu, int ldgu, int M, int ffn, int8_t *q, float *scales,
                             int32_t *qsum) {
    qwen_swiglu_quant_kernel<<<dim3((unsigned)((ffn + 255) / 256), (unsigned)M), 256, 0, ctx->stream>>>(
        gu, ldgu, ffn, q, scales, qsum);
    return check_launch("qwen_swiglu_quant");
}

int launch_argmax(gx_ctx *ctx, const float *x, int ldx, int M, int n, int32_t *out) {
    argmax_kernel<<<M, kArgmaxThreads, 0, ctx->stream>>>(x, ldx, n, out);
    return check_launch("argmax");
}

}  // namespace gx
