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

constexpr int kQNormThreads = 256;

// One position per workgroup: x (and add) [M][ld], gain [K].  out, when given,
// receives the normed floats [M][ldo]; q/scales/qsum receive its Q8_0 form.
__global__ __launch_bounds__(kQNormThreads) void qwen_norm_quant_kernel(float *__restrict__ x, int ldx,
                                                                        const float *__restrict__ add, int lda,
                                                                        const float *__restrict__ gain, int K,
                                                                        float eps, float *__restrict__ out, int ldo,
                                                                        int8_t *__restrict__ q,
                                                                        float *__restrict__ scales,
                                                                        int32_t *__restrict__ qsum) {
    extern __shared__ float xs[];  // K floats
    __shared__ double red[kQNormThreads];
    __shared__ float scale_sh;
    const int tid = threadIdx.x, t = blockIdx.x;
    float *xr = x + (size_t)t * ldx;
    for (int i = tid; i < K; i += kQNormThreads) {
        float v = xr[i];
        if (add) {
            v = v + add[(size_t)t * lda + i];
            xr[i] = v;
        }
        xs[i] = v;
    }
    __syncthreads();
    double p0, p1;
    norm_partials(xs, K, p0, p1);
    const double sum = norm_tree(p0, p1, red);
    if (tid == 0)
        scale_sh = norm_scale(sum, K, eps);
    __syncthreads();
    const float sc = scale_sh;
    // Element i = j*256 + tid: a 32-lane group covers one Q8_0 block.
    const int B = K >> 5;
    for (int base = 0; base < K; base += kQNormThreads) {
        const int i = base + tid;
        if (i < K) {  // K % 32 == 0: whole groups in or out
            const float v = xs[i] * sc;
            const float nv = v * gain[i];
            if (out)
                out[(size_t)t * ldo + i] = nv;
            if (q) {
                float stored;
                int32_t s;
                const int32_t n = q8_0_lane(nv, &stored, &s);
                q[(size_t)t * K + i] = (int8_t)n;
                if ((i & 31) == 0) {
                    scales[(size_t)t * B + (i >> 5)] = stored;
                    qsum[(size_t)t * B + (i >> 5)] = s;
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

constexpr int kAttnMaxCtx = 8192;

// grid (M, heads), one wavefront: position t's query head h against the
// layer's cache over positions 0 .. positions[t].  scores: LDS, one per
// visible position.  The head's output is quantised (Q8_0, 32-lane groups)
// into q/scales/qsum at columns h*hd of a [M][heads*hd] batch.
__global__ __launch_bounds__(64) void qwen_attention_kernel(const uint16_t *__restrict__ qh, int heads, int kv_heads,
                                                            int hd, const int32_t *__restrict__ positions,
                                                            const uint16_t *__restrict__ kcache,
                                                            const uint16_t *__restrict__ vcache, float scale,
                                                            int8_t *__restrict__ q, float *__restrict__ scales,
                                                            int32_t *__restrict__ qsum) {
    extern __shared__ float scores[];  // n
    __shared__ float query[kHeadMax];
    __shared__ float total_sh;
    const int lane = threadIdx.x, t = blockIdx.x, h = blockIdx.y;
    const int n = positions[t] + 1;
    const int kvh = h / (heads / kv_heads);
    const int width = heads * hd;
    for (int i = lane; i < hd; i += 64)
        query[i] = half_bits_to_float(qh[(size_t)t * width + h * hd + i]);
    __syncthreads();

    // Scores: a lane per visible position, DotF32's four chains
    // (nn/dot_f32.go:13-33), scaled.
    float mx = -INFINITY;
    for (int p = lane; p < n; p += 64) {
        const uint16_t *key = kcache + ((size_t)p * kv_heads + kvh) * hd;
        float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
        for (int i = 0; i + 3 < hd; i += 4) {
            const uint2 kw = *(const uint2 *)(key + i);
            const float p0 = query[i] * half_bits_to_float(kw.x & 0xFFFFu);
            const float p1 = query[i + 1] * half_bits_to_float(kw.x >> 16);
            const float p2 = query[i + 2] * half_bits_to_float(kw.y & 0xFFFFu);
            const float p3 = query[i + 3] * half_bits_to_float(kw.y >> 16);
            s0 = s0 + p0;
            s1 = s1 + p1;
            s2 = s2 + p2;
            s3 = s3 + p3;
        }
        const float dot = (s0 + s1) + (s2 + s3);
        const float sc = scale * dot;
        scores[p] = sc;
        mx = fmaxf(mx, sc);
    }
    for (int off = 32; off > 0; off >>= 1)
        mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    // SoftmaxInPlace (nn/ops.go:59-75): exp in float64, the sum in position
    // order (one lane), then the division; each probability rounded to fp16.
    for (int p = lane; p < n; p += 64)
        scores[p] = (float)exp((double)(scores[p] - mx));
    __syncthreads();
    if (lane == 0) {
        float sum = 0.0f;
        for (int p = 0; p < n; p++)
            sum += scores[p];
        total_sh = sum;
    }
    __syncthreads();
    const float total = total_sh;
    for (int p = lane; p < n; p += 64)
        scores[p] = half_bits_to_float(float_to_half_bits(scores[p] / total));
    __syncthreads();

    // dst = sum over positions, in order, of Axpy(value, probability)
    // (nn/kernel.go:221-233): lane owns elements lane and lane + 64.
    float d0 = 0.0f, d1 = 0.0f;
    const int i0 = lane, i1 = lane + 64;
    for (int p = 0; p < n; p++) {
        const uint16_t *val = vcache + ((size_t)p * kv_heads + kvh) * hd;
        const float a = scores[p];
        if (i0 < hd) {
            const float m = a * half_bits_to_float(val[i0]);
            d0 = d0 + m;
        }
        if (i1 < hd) {
            const float m = a * half_bits_to_float(val[i1]);
            d1 = d1 + m;
        }
    }
    // Q8_0 of the head (hd % 32 == 0): two 32-lane groups per pass.
    const int B = width >> 5;
    for (int k = 0; k < 2; k++) {
        const int i = k == 0 ? i0 : i1;
        if (k * 64 < hd) {  // uniform
            float stored;
            int32_t s;
            const int32_t nq = q8_0_lane(k == 0 ? d0 : d1, &stored, &s);
            const int c = h * hd + i;
            q[(size_t)t * width + c] = (int8_t)nq;
            if ((i & 31) == 0) {
                scales[(size_t)t * B + (c >> 5)] = stored;
                qsum[(size_t)t * B + (c >> 5)] = s;
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
// ties (NaN never wins).
__global__ __launch_bounds__(256) void argmax_kernel(const float *__restrict__ x, int ldx, int n,
                                                     int32_t *__restrict__ out) {
    __shared__ float bv_sh[256];
    __shared__ int bi_sh[256];
    const int tid = threadIdx.x;
    const float *r = x + (size_t)blockIdx.x * ldx;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int i = tid; i < n; i += 256) {
        const float v = r[i];
        if (v > bv || (bi == 0x7fffffff && v == v)) {  // indices rise: equal values keep the first
            bv = v;
            bi = i;
        }
    }
    bv_sh[tid] = bv;
    bi_sh[tid] = bi;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
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
    const size_t lds = sizeof(float) * (size_t)K;
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
    GX_CHECK(hd <= 128 && hd % 32 == 0, "gx: attention supports head widths that are multiples of 32 up to 128");
    GX_CHECK(max_pos + 1 <= kAttnMaxCtx, "gx: attention context %d exceeds %d", max_pos + 1, kAttnMaxCtx);
    const size_t lds = sizeof(float) * (size_t)(max_pos + 1);
    qwen_attention_kernel<<<dim3((unsigned)M, (unsigned)heads), 64, lds, ctx->stream>>>(
        qh, heads, kv_heads, hd, positions, kcache, vcache, scale, q, scales, qsum);
    return check_launch("qwen_attention");
}

int launch_qwen_swiglu_quant(gx_ctx *ctx, const float *gu, int ldgu, int M, int ffn, int8_t *q, float *scales,
                             int32_t *qsum) {
    qwen_swiglu_quant_kernel<<<dim3((unsigned)((ffn + 255) / 256), (unsigned)M), 256, 0, ctx->stream>>>(
        gu, ldgu, ffn, q, scales, qsum);
    return check_launch("qwen_swiglu_quant");
}

int launch_argmax(gx_ctx *ctx, const float *x, int ldx, int M, int n, int32_t *out) {
    argmax_kernel<<<M, 256, 0, ctx->stream>>>(x, ldx, n, out);
    return check_launch("argmax");
}

}  // namespace gx
