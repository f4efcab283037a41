// gx_moe.hip - the expert branch of golem's mixture of experts on the device.
//
// ExpertFFN (gemma/moe.go:112-180) for M positions:
//   Route (gemma/moe.go:34-53): x = RMSNormPlain(resid) * (1/sqrt(Dim)) *
//     RouterScale, router logits = DotF32(router row, x) in golem's generic
//     order, chooseExperts (moe.go:62-88): top_k by repeated argmax (strict >,
//     ties to the lower index), weights exp(l - top) in float64, renormalised.
//   Units (position t, slot k): gate_up = GateUp[id] . Q8_0(x_t) (2*ffn rows,
//     gate first), mid = GELUTable(gate) * up, quantised to Q8_0,
//     partial = Down[id] . mid (moe.go:137-162).
//   out_t = sum_k (w_k * DownScale[id]) * partial_k, golem's generic Axpy in
//     slot order (moe.go:165-179, nn/kernel.go:221-233).
// Few positions (decode) run each unit as a matrix-vector product; more
// positions are sorted by expert (a stable counting sort, so the order does
// not depend on scheduling) and each expert's units go through the MFMA
// product as one ragged batch.  Both compute a unit's rows in the same
// canonical order, so a position's result does not depend on the batch.
#include "gx_device.hpp"
#include "gx_internal.hpp"

namespace gx {
namespace {

// golem's GELU table (nn/gelu_table.go:25-38): for every fp16 input,
// fp16(float32(geluTanh(float64(input)))), held as float.
__global__ void gelu_table_kernel(float *__restrict__ table) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= 65536)
        return;
    const double x = (double)half_bits_to_float((uint32_t)i);
    const double sqrt2_over_pi = 0.79788456080286535587989211986876;
    const double coef_a = 0.044715;
    const double inner = sqrt2_over_pi * x * (1.0 + coef_a * x * x);
    const double g = 0.5 * x * (1.0 + tanh(inner));
    table[i] = half_bits_to_float(float_to_half_bits((float)g));
}

// The router.
//
// Logits: DotF32 (nn/dot_f32.go:13-33) is four serial chains -- chain c adds
// the products of elements c, c+4, c+8, ... in order -- that meet as
// (s0 + s1) + (s2 + s3).  A lane runs one chain in that order, so the logits
// are golem's bits.  RMSNormPlain (nn/ops.go:195-214) squares in float32 and
// sums in float64, here in a fixed tree: 512 partial sums, partial t holding
// elements t, t+512, t+1024, ... in order, then halved pairwise (t + w for
// w = 256 .. 1).  golem sums left to right; the two float64 sums differ by a
// few units in the 53rd bit, below the float32 rounding of the mean except in
// rare ties.  The normalised input is (x * scale) * ((1/sqrt(D)) *
// RouterScale[i]), as Route forms it (gemma/moe.go:34-53).
//
//   moe_logits_one_kernel: one workgroup per (expert, position); the row and
//     the position's input sit in LDS, every load issued at once.  Few
//     positions (decode), where the cost is latency.
//   moe_logits_kernel<EW>: EW experts x 64/EW positions per workgroup; rows and
//     inputs pass through LDS a 64-input chunk at a time, fetched from a ring
//     of registers kLogitsDepth chunks ahead.  Many positions.
constexpr int kLogitsThreads = 256;
constexpr int kLogitsChunk = 64;     // inputs per chunk
constexpr int kLogitsChunkPad = 68;  // chunk row stride in LDS (bank spread)
constexpr int kLogitsDepth = 8;      // chunks fetched ahead
constexpr int kLogitsOneMaxD = 7168; // row + input in LDS: 57 KB
constexpr int kLogitsOneF4 = kLogitsOneMaxD / 4 / kLogitsThreads;

__global__ __launch_bounds__(kLogitsThreads) void moe_logits_one_kernel(const float *__restrict__ router, int D,
                                                                        int E, const float *__restrict__ router_scale,
                                                                        const float *__restrict__ resid, int ldr,
                                                                        float eps, float *__restrict__ logits) {
    extern __shared__ float lds[];
    float *row = lds, *xr = lds + D;
    __shared__ double red[kLogitsThreads];
    __shared__ float scale_sh;
    const int tid = threadIdx.x, e = blockIdx.x, t = blockIdx.y;
    const float *rg = router + (size_t)e * D;
    const float *xg = resid + (size_t)t * ldr;
    const int n4 = D / 4;
    // Clamped indices and clamped stores (a thread past the end stores the
    // last piece's own value again): every load is issued before the first
    // wait, with no branch for a load to sink into.
    float4 rv[kLogitsOneF4 + 1], xv[kLogitsOneF4 + 1], sv[kLogitsOneF4 + 1];
#pragma unroll
    for (int f = 0; f <= kLogitsOneF4; f++) {
        const int q = min(tid + f * kLogitsThreads, n4 - 1);
        rv[f] = *(const float4 *)(rg + 4 * q);
        xv[f] = *(const float4 *)(xg + 4 * q);
        sv[f] = router_scale ? *(const float4 *)(router_scale + 4 * q) : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
    }
#pragma unroll
    for (int f = 0; f <= kLogitsOneF4; f++) {
        const int q = min(tid + f * kLogitsThreads, n4 - 1);
        *(float4 *)(row + 4 * q) = rv[f];
        *(float4 *)(xr + 4 * q) = xv[f];
    }
    __syncthreads();
    double p0, p1;
    norm_partials(xr, D, p0, p1);
    const double sum = norm_tree(p0, p1, red);
    if (tid == 0)
        scale_sh = norm_scale(sum, D, eps);
    __syncthreads();
    const float sc = scale_sh;
    const float inv_sqrt_dim = (float)(1.0 / sqrt((double)D));
    // x * scale * ((1/sqrt(D)) * RouterScale[i]), from the registers
#pragma unroll
    for (int f = 0; f <= kLogitsOneF4; f++) {
        const int q = min(tid + f * kLogitsThreads, n4 - 1);
        const float x4[4] = {xv[f].x, xv[f].y, xv[f].z, xv[f].w}, s4[4] = {sv[f].x, sv[f].y, sv[f].z, sv[f].w};
        float o4[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float normed = x4[c] * sc;
            const float factor = inv_sqrt_dim * s4[c];
            o4[c] = normed * factor;
        }
        *(float4 *)(xr + 4 * q) = make_float4(o4[0], o4[1], o4[2], o4[3]);
    }
    __syncthreads();
    if (tid < 64) {
        const int c = tid & 3;
        float acc = 0.0f;
        if (tid < 4) {
            for (int i0 = c; i0 < D; i0 += 64) {  // D % 64 == 0: 16 steps per pass
                float a[16], b[16];
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    a[j] = row[i0 + 4 * j];
                    b[j] = xr[i0 + 4 * j];
                }
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    const float prod = a[j] * b[j];
                    acc = acc + prod;
                }
            }
        }
        const float s1 = __shfl_down(acc, 1, 64), s2 = __shfl_down(acc, 2, 64), s3 = __shfl_down(acc, 3, 64);
        if (tid == 0)
            logits[(size_t)t * E + e] = (acc + s1) + (s2 + s3);
    }
}

template <int EW>
__global__ __launch_bounds__(kLogitsThreads) void moe_logits_kernel(const float *__restrict__ router, int D, int E,
                                                                    const float *__restrict__ router_scale,
                                                                    const float *__restrict__ resid, int ldr, int M,
                                                                    float eps, float *__restrict__ logits) {
    constexpr int P = 64 / EW;                       // positions per workgroup
    constexpr int XF4 = P * 16 / kLogitsThreads;     // input float4 per thread per chunk
    constexpr int RT = EW * 16;                      // threads holding a row float4 per chunk
    constexpr int BUF = (EW + P) * kLogitsChunkPad;  // a chunk in LDS: rows, then inputs
    __shared__ float buf[2 * BUF];
    __shared__ float scale[P];
    __shared__ double red[kLogitsThreads];
    const int tid = threadIdx.x;
    const int e0 = blockIdx.x * EW, t0 = blockIdx.y * P;

    // The norm's scale for each position, the workgroup together.
    for (int p = 0; p < P && t0 + p < M; p++) {
        double p0, p1;
        norm_partials(resid + (size_t)(t0 + p) * ldr, D, p0, p1);
        const double sum = norm_tree(p0, p1, red);
        if (tid == 0)
            scale[p] = norm_scale(sum, D, eps);
        __syncthreads();
    }

    const float inv_sqrt_dim = (float)(1.0 / sqrt((double)D));
    const int re = (tid % RT) >> 4, rq = tid & 15;  // this thread's row float4 of a chunk
    const float *rsrc = router + (size_t)min(e0 + re, E - 1) * D + 4 * rq;
    float xs[kLogitsDepth][XF4 * 4], rs[kLogitsDepth][4];
    const int c = tid & 3, e = (tid >> 2) % EW, p = (tid >> 2) / EW;  // lane = (p, e, c)
    float acc = 0.0f;
    const int chunks = D / kLogitsChunk;

#define GX_LOGITS_FETCH(k, slot)                                                                                     \
    do {                                                                                                             \
        for (int f = 0; f < XF4; f++) {                                                                              \
            const int idx = tid + f * kLogitsThreads;                                                                \
            const int tt = min(t0 + (idx >> 4), M - 1);                                                              \
            const float4 v = *(const float4 *)(resid + (size_t)tt * ldr + (k) * kLogitsChunk + 4 * (idx & 15));     \
            xs[slot][4 * f + 0] = v.x;                                                                               \
            xs[slot][4 * f + 1] = v.y;                                                                               \
            xs[slot][4 * f + 2] = v.z;                                                                               \
            xs[slot][4 * f + 3] = v.w;                                                                               \
        }                                                                                                            \
        const float4 r = *(const float4 *)(rsrc + (k) * kLogitsChunk);                                               \
        rs[slot][0] = r.x;                                                                                           \
        rs[slot][1] = r.y;                                                                                           \
        rs[slot][2] = r.z;                                                                                           \
        rs[slot][3] = r.w;                                                                                           \
    } while (0)

#define GX_LOGITS_PUT(k, slot)                                                                                       \
    do {                                                                                                             \
        float *b = buf + ((k) & 1) * BUF;                                                                            \
        if (tid < RT)                                                                                                \
            for (int j = 0; j < 4; j++)                                                                              \
                b[re * kLogitsChunkPad + 4 * rq + j] = rs[slot][j];                                                  \
        float *bx = b + EW * kLogitsChunkPad;                                                                        \
        for (int f = 0; f < XF4; f++) {                                                                              \
            const int idx = tid + f * kLogitsThreads;                                                                \
            const int pp = idx >> 4, q = idx & 15;                                                                   \
            const float sc = scale[pp];                                                                              \
            const int i0 = (k) * kLogitsChunk + 4 * q;                                                               \
            for (int j = 0; j < 4; j++) {                                                                            \
                const float normed = xs[slot][4 * f + j] * sc;                                                       \
                const float factor = inv_sqrt_dim * (router_scale ? router_scale[i0 + j] : 1.0f);                    \
                bx[pp * kLogitsChunkPad + 4 * q + j] = normed * factor;                                              \
            }                                                                                                        \
        }                                                                                                            \
    } while (0)

#pragma unroll
    for (int u = 0; u < kLogitsDepth; u++)
        if (u < chunks)
            GX_LOGITS_FETCH(u, u);
    GX_LOGITS_PUT(0, 0);
    if (kLogitsDepth < chunks)
        GX_LOGITS_FETCH(kLogitsDepth, 0);
    __syncthreads();
    for (int kb = 0; kb < chunks; kb += kLogitsDepth) {
#pragma unroll
        for (int u = 0; u < kLogitsDepth; u++) {
            const int k = kb + u;
            if (k < chunks) {
                const float *b = buf + (k & 1) * BUF;
                const float *rk = b + e * kLogitsChunkPad + c;
                const float *xr = b + EW * kLogitsChunkPad + p * kLogitsChunkPad + c;
                float av[16], bv[16];
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    av[j] = rk[4 * j];
                    bv[j] = xr[4 * j];
                }
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    const float prod = av[j] * bv[j];
                    acc = acc + prod;
                }
                // chunk k + 1 into the other buffer (last read at chunk k - 1);
                // its ring slot then takes chunk k + 1 + depth
                const int nu = (u + 1) % kLogitsDepth;  // a constant once unrolled
                if (k + 1 < chunks) {
                    GX_LOGITS_PUT(k + 1, nu);
                    if (k + 1 + kLogitsDepth < chunks)
                        GX_LOGITS_FETCH(k + 1 + kLogitsDepth, nu);
                }
                __syncthreads();
            }
        }
    }
#undef GX_LOGITS_FETCH
#undef GX_LOGITS_PUT
    const float s1 = __shfl_down(acc, 1, 64), s2 = __shfl_down(acc, 2, 64), s3 = __shfl_down(acc, 3, 64);
    if (c == 0 && t0 + p < M && e0 + e < E)
        logits[(size_t)(t0 + p) * E + e0 + e] = (acc + s1) + (s2 + s3);
}

// chooseExperts (gemma/moe.go:62-88) for one position per wavefront: k rounds
// of argmax over the logits not yet chosen.  golem scans in index order and
// replaces its best on a strictly greater logit, so ties go to the lower
// index and a NaN is taken only when it is the first logit not yet chosen
// (no comparison with it is ever true); the wavefront reduction keeps exactly
// that rule.  Weights: exp(l - top) in float64, rounded to float32, summed in
// slot order, divided by the sum.
constexpr int kTopkMaxPerLane = 16;  // E <= 1024
constexpr int kTopkMax = 64;         // k <= 64

__global__ __launch_bounds__(64) void moe_topk_kernel(const float *__restrict__ logits, int E, int k,
                                                      int32_t *__restrict__ ids, float *__restrict__ weights) {
    __shared__ float chosen_l[kTopkMax];
    __shared__ float wv[kTopkMax];
    __shared__ float lg[64 * kTopkMaxPerLane];
    const int t = blockIdx.x, lane = threadIdx.x;
    const float *lgg = logits + (size_t)t * E;
    float v[kTopkMaxPerLane];
    unsigned taken = 0;  // bit j: logit lane + 64 j is chosen or absent
#pragma unroll
    for (int j = 0; j < kTopkMaxPerLane; j++) {
        const int e = lane + 64 * j;
        v[j] = lgg[min(e, E - 1)];
        lg[e] = v[j];
        taken |= (e >= E ? 1u : 0u) << j;
    }
    __syncthreads();
    // A NaN logit is taken only as the first logit not yet chosen; without
    // any, a round is a plain argmax (greater value, then lower index).
    bool nan_here = false;
#pragma unroll
    for (int j = 0; j < kTopkMaxPerLane; j++)
        nan_here |= lane + 64 * j < E && v[j] != v[j];
    const bool any_nan = __any(nan_here);
    for (int round = 0; round < k; round++) {
        int best = 0x7fffffff;
        if (any_nan) {
            int first = 0x7fffffff;
            const unsigned open = ~taken & ((1u << kTopkMaxPerLane) - 1);
            if (open)
                first = lane + 64 * __builtin_ctz(open);
            for (int w = 32; w > 0; w >>= 1)
                first = min(first, __shfl_xor(first, w, 64));
            if (lg[first] != lg[first])
                best = first;
        }
        if (best == 0x7fffffff) {
            // largest non-NaN value not yet chosen, lowest index among equals
            float bv = 0.0f;
            int bi = 0x7fffffff;
#pragma unroll
            for (int j = 0; j < kTopkMaxPerLane; j++) {
                const int e = lane + 64 * j;
                if (((taken >> j) & 1u) || v[j] != v[j])
                    continue;
                if (bi == 0x7fffffff || v[j] > bv) {  // e rises with j: equal values keep the lower index
                    bv = v[j];
                    bi = e;
                }
            }
            for (int w = 32; w > 0; w >>= 1) {
                const float ov = __shfl_xor(bv, w, 64);
                const int oi = __shfl_xor(bi, w, 64);
                if (oi != 0x7fffffff && (bi == 0x7fffffff || ov > bv || (ov == bv && oi < bi))) {
                    bv = ov;
                    bi = oi;
                }
            }
            best = bi;
        }
        if ((best & 63) == lane)
            taken |= 1u << (best >> 6);
        if (lane == 0) {
            ids[(size_t)t * k + round] = best;
            chosen_l[round] = lg[best];
        }
    }
    __syncthreads();
    // exp(l - top) in float64 for every slot at once; the sum in slot order.
    if (lane < k)
        wv[lane] = (float)exp((double)(chosen_l[lane] - chosen_l[0]));
    __syncthreads();
    float total = 0.0f;
    for (int j = 0; j < k; j++)
        total += wv[j];
    if (lane < k)
        weights[(size_t)t * k + lane] = wv[lane] / total;
}

// mid = GELUTable(gate) * up for one unit per workgroup row, then its Q8_0
// form (Batch.quantizeBlock): gate_up is [U][ld] with each row's F gates then
// its F ups, mid_q [U][F].
__global__ __launch_bounds__(256) void moe_gelu_mul_quant_kernel(const float *__restrict__ gate_up, int ld, int F,
                                                                  int U, const float *__restrict__ table,
                                                                  int8_t *__restrict__ q, float *__restrict__ scales,
                                                                  int32_t *__restrict__ qsum) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (size_t)U * F)
        return;  // U*F is a multiple of 32: whole 32-lane groups drop out
    const int u = (int)(gid / F), i = (int)(gid % F);
    const float gate = gate_up[(size_t)u * ld + i];
    const float up = gate_up[(size_t)u * ld + F + i];
    // GELUTable (nn/gelu_table.go:40-52)
    float gl;
    if (gate <= -10.0f)
        gl = 0.0f;
    else if (gate >= 10.0f)
        gl = gate;
    else
        gl = table[float_to_half_bits(gate)];
    const float v = gl * up;
    // quantizeBlock (nn/batch.go:109-143), as gx_quant.hip's kernel
    float peak = fabsf(v);
#pragma unroll
    for (int off = 16; off > 0; off >>= 1)
        peak = fmaxf(peak, __shfl_xor(peak, off, 32));
    const size_t index = (size_t)u * (F >> 5) + (i >> 5);
    if (peak == 0.0f) {
        q[gid] = 0;
        if ((i & 31) == 0) {
            scales[index] = 0.0f;
            qsum[index] = 0;
        }
        return;
    }
    const float scale = __fdiv_rn(peak, 127.0f);
    const float inverse = __fdiv_rn(127.0f, peak);
    const float prod = v * inverse;
    int32_t n = nearest_int(prod);
    n = n > 127 ? 127 : (n < -128 ? -128 : n);
    q[gid] = (int8_t)n;
    int32_t sum = n;
#pragma unroll
    for (int off = 16; off > 0; off >>= 1)
        sum += __shfl_xor(sum, off, 32);
    if ((i & 31) == 0) {
        scales[index] = half_bits_to_float(float_to_half_bits(scale));
        qsum[index] = sum;
    }
}

// The join of moeHalf (gemma/block.go:195-205), one position per workgroup:
// shared = RMSNormPlain(shared, post1) and experts = RMSNormPlain(experts,
// post2), both written back (golem's buffers hold them so afterwards);
// combined = shared + experts; RMSNormPlain(combined, post); out = resid +
// combined.  Each norm is a float64 sum of squares in the order of the other
// residual norms, then (v * scale) * gain in float32.
constexpr int kJoinThreads = 1024;
__global__ __launch_bounds__(kJoinThreads) void moe_join_kernel(float *__restrict__ shared, int lds_,
                                                               float *__restrict__ experts, int lde,
                                                               const float *__restrict__ resid, int ldr,
                                                               const float *__restrict__ post1,
                                                               const float *__restrict__ post2,
                                                               const float *__restrict__ post, int K, float eps,
                                                               float *__restrict__ out, int ldo) {
    extern __shared__ float join[];  // shared, experts: K floats each
    float *sh = join, *ex = join + K;
    __shared__ double red[512];
    __shared__ double total;
    const int tid = threadIdx.x, t = blockIdx.x;
    float *sr = shared + (size_t)t * lds_, *er = experts + (size_t)t * lde;
    for (int i = tid; i < K; i += kJoinThreads) {
        sh[i] = sr[i];
        ex[i] = er[i];
    }
    __syncthreads();
    const float s1 = norm_scale(block_sum_squares(sh, K, red, &total), K, eps);
    const float s2 = norm_scale(block_sum_squares(ex, K, red, &total), K, eps);
    for (int i = tid; i < K; i += kJoinThreads) {
        const float a = sh[i] * s1 * post1[i], b = ex[i] * s2 * post2[i];
        sr[i] = a;
        er[i] = b;
        sh[i] = a + b;  // combined, in place of the shared values
    }
    __syncthreads();
    const float s3 = norm_scale(block_sum_squares(sh, K, red, &total), K, eps);
    const float *rr = resid + (size_t)t * ldr;
    float *orow = out + (size_t)t * ldo;
    for (int i = tid; i < K; i += kJoinThreads)
        orow[i] = rr[i] + sh[i] * s3 * post[i];
}

// The expert sum: out[t][i] = 0, then out += (w_k * DownScale[id_k]) *
// partial_k for k in slot order, each step a rounded product then a rounded
// sum (golem's generic Axpy).
__global__ void moe_reduce_kernel(const float *__restrict__ partial, int D, int M, int k,
                                  const int32_t *__restrict__ ids, const float *__restrict__ weights,
                                  const float *__restrict__ down_scale, float *__restrict__ out, int ldo) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (size_t)M * D)
        return;
    const int t = (int)(gid / D), i = (int)(gid % D);
    float acc = 0.0f;
    for (int j = 0; j < k; j++) {
        const int u = t * k + j;
        const float a = weights[u] * (down_scale ? down_scale[ids[u]] : 1.0f);
        const float p = a * partial[(size_t)u * D + i];
        acc = acc + p;
    }
    out[(size_t)t * ldo + i] = acc;
}

// Stable counting sort of the U = M*k units by expert, in one workgroup, and
// the work list of the grouped product.  Units with an id outside [0, E) are
// left out of every group (their partial sums stay NaN).
//   sorted[0..U): units, expert by expert, each expert's in unit order
//   work[item] = {expert, first, count, 0}, items of up to `tile` units,
//   expert by expert; the items past the last are {0, 0, 0, 0}.
constexpr int kSortThreads = 1024;
__global__ __launch_bounds__(kSortThreads) void moe_sort_kernel(const int32_t *__restrict__ ids, int U, int E,
                                                                int tile, int max_items,
                                                                int32_t *__restrict__ sorted,
                                                                int32_t *__restrict__ work) {
    extern __shared__ int32_t sh[];  // counts[E], offsets[E], placed[E], chunk ids[kSortThreads]
    int32_t *counts = sh, *offsets = sh + E, *placed = sh + 2 * E, *chunk = sh + 3 * E;
    const int tid = threadIdx.x;
    for (int e = tid; e < E; e += kSortThreads)
        counts[e] = 0, placed[e] = 0;
    for (int i = tid; i < max_items; i += kSortThreads) {
        work[4 * i] = 0, work[4 * i + 1] = 0, work[4 * i + 2] = 0, work[4 * i + 3] = 0;
    }
    __syncthreads();
    for (int u = tid; u < U; u += kSortThreads) {
        const int e = ids[u];
        if (e >= 0 && e < E)
            atomicAdd(&counts[e], 1);
    }
    __syncthreads();
    if (tid == 0) {
        int acc = 0, item = 0;
        for (int e = 0; e < E; e++) {
            offsets[e] = acc;
            for (int f = 0; f < counts[e]; f += tile) {
                if (item < max_items) {
                    work[4 * item] = e;
                    work[4 * item + 1] = acc + f;
                    work[4 * item + 2] = min(tile, counts[e] - f);
                }
                item++;
            }
            acc += counts[e];
        }
    }
    __syncthreads();
    // Units in chunks of kSortThreads, in order: a unit's place is its
    // expert's offset, plus the units of that expert in earlier chunks, plus
    // those before it in this chunk.
    for (int base = 0; base < U; base += kSortThreads) {
        const int u = base + tid;
        const int e = u < U ? ids[u] : -1;
        chunk[tid] = e;
        __syncthreads();
        if (e >= 0 && e < E) {
            int before = 0;
            for (int j = 0; j < tid; j++)
                before += chunk[j] == e;
            sorted[offsets[e] + placed[e] + before] = u;
        }
        __syncthreads();
        if (e >= 0 && e < E)
            atomicAdd(&placed[e], 1);
        __syncthreads();
    }
}

__global__ void fill_nan_kernel(float *__restrict__ p, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n)
        p[i] = __builtin_nanf("");
}

constexpr size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// Workspace layout for M positions, k slots, width D, expert width F.
struct MoeSpace {
    size_t xq, xs, xqs, gu, mq, ms, mqs, part, sorted, work, total;
    int units, max_items;
};

MoeSpace moe_space(int M, int k, int D, int F, int E) {
    MoeSpace s{};
    const size_t U = (size_t)M * k;
    s.units = (int)U;
    s.max_items = E + (int)((U + 127) / 128);
    size_t at = 0;
    auto take = [&](size_t bytes) {
        const size_t here = at;
        at += align256(bytes);
        return here;
    };
    s.xq = take((size_t)M * D);
    s.xs = take((size_t)M * (D / 32) * 4);
    s.xqs = take((size_t)M * (D / 32) * 4);
    s.gu = take(U * 2 * F * 4);
    s.mq = take(U * F);
    s.ms = take(U * (F / 32) * 4);
    s.mqs = take(U * (F / 32) * 4);
    s.part = take(U * D * 4);
    s.sorted = take(U * 4);
    s.work = take((size_t)s.max_items * 16);
    s.total = at;
    return s;
}

}  // namespace

int moe_workspace_bytes(int M, int k, int D, int F, int E, size_t *bytes) {
    *bytes = moe_space(M, k, D, F, E).total;
    return GX_OK;
}

int launch_geglu_quant(gx_ctx *ctx, const float *gu, int ldgu, int M, int ffn, int8_t *q, float *scales,
                       int32_t *qsum) {
    const size_t n = (size_t)M * ffn;
    if (n == 0)
        return GX_OK;
    moe_gelu_mul_quant_kernel<<<(unsigned)((n + 255) / 256), 256, 0, ctx->stream>>>(gu, ldgu, ffn, M,
                                                                                    ctx->gelu_table, q, scales,
                                                                                    qsum);
    return check_launch("geglu_quant");
}

int launch_moe_join(gx_ctx *ctx, float *shared, int lds_, float *experts, int lde, const float *resid, int ldr,
                    const float *post1, const float *post2, const float *post, int M, int K, float eps, float *out,
                    int ldo) {
    if (M == 0)
        return GX_OK;
    const size_t lds = 2 * (size_t)K * sizeof(float);
    GX_CHECK(lds <= 64 * 1024, "gx: a %d-wide residual does not fit the join's LDS", K);
    moe_join_kernel<<<M, kJoinThreads, lds, ctx->stream>>>(shared, lds_, experts, lde, resid, ldr, post1, post2,
                                                           post, K, eps, out, ldo);
    return check_launch("moe_join");
}

int launch_gelu_table(gx_ctx *ctx, float *table) {
    gelu_table_kernel<<<256, 256, 0, ctx->stream>>>(table);
    return check_launch("gelu_table");
}

int launch_moe_route(gx_ctx *ctx, const gx_weight *router, const float *router_scale, const float *resid, int ldr,
                     int M, int k, float eps, float *logits, int32_t *ids, float *weights) {
    const int D = router->cols, E = router->rows;
    GX_CHECK(D % kLogitsChunk == 0, "gx: the router's width %d is not a multiple of %d", D, kLogitsChunk);
    GX_CHECK(E <= 64 * kTopkMaxPerLane, "gx: %d experts exceed the router's limit of %d", E, 64 * kTopkMaxPerLane);
    GX_CHECK(k <= kTopkMax, "gx: top_k %d exceeds %d", k, kTopkMax);
    GX_CHECK(((uintptr_t)resid & 15) == 0 && ldr % 4 == 0, "gx: resid must be 16-byte aligned with ldr %% 4 == 0");
    const float *rw = (const float *)router->dev;
    if (M <= 4 && D <= kLogitsOneMaxD) {
        const size_t lds = 2 * sizeof(float) * (size_t)D;
        moe_logits_one_kernel<<<dim3((unsigned)E, (unsigned)M), kLogitsThreads, lds, ctx->stream>>>(
            rw, D, E, router_scale, resid, ldr, eps, logits);
    } else {
        constexpr int EW = 4, P = 64 / EW;
        const dim3 grid((unsigned)((E + EW - 1) / EW), (unsigned)((M + P - 1) / P));
        moe_logits_kernel<EW><<<grid, kLogitsThreads, 0, ctx->stream>>>(rw, D, E, router_scale, resid, ldr, M, eps,
                                                                         logits);
    }
    if (int rc = check_launch("moe_logits"))
        return rc;
    moe_topk_kernel<<<M, 64, 0, ctx->stream>>>(logits, E, k, ids, weights);
    return check_launch("moe_topk");
}

int launch_moe_experts(gx_ctx *ctx, const gx_weight *gate_up, const gx_weight *down, const float *down_scale,
                       const float *x, int ldx, int M, int k, const int32_t *ids, const float *weights, float *out,
                       int ldo, uint8_t *ws, const float *gelu_table) {
    const int D = gate_up->cols, F = down->cols, E = gate_up->count;
    const MoeSpace s = moe_space(M, k, D, F, E);
    const int U = s.units;
    int8_t *xq = (int8_t *)(ws + s.xq);
    float *xs = (float *)(ws + s.xs);
    int32_t *xqs = (int32_t *)(ws + s.xqs);
    float *gu = (float *)(ws + s.gu);
    int8_t *mq = (int8_t *)(ws + s.mq);
    float *ms = (float *)(ws + s.ms);
    int32_t *mqs = (int32_t *)(ws + s.mqs);
    float *part = (float *)(ws + s.part);
    int32_t *sorted = (int32_t *)(ws + s.sorted);
    int32_t *work = (int32_t *)(ws + s.work);

    // Each position's input, quantised once for its k units (moe.go:119-125).
    if (int rc = launch_quantize_q8_0(ctx, x, ldx, M, D, xq, xs, xqs, nullptr, nullptr))
        return rc;
    const bool grouped = M > 4;
    if (grouped) {
        // A unit whose expert id is out of range is in no group: its sums
        // stay NaN, and so does its position's output.
        const size_t n = (size_t)U * 2 * F;
        fill_nan_kernel<<<(unsigned)((n + 255) / 256), 256, 0, ctx->stream>>>(gu, n);
        const size_t np = (size_t)U * D;
        fill_nan_kernel<<<(unsigned)((np + 255) / 256), 256, 0, ctx->stream>>>(part, np);
        const size_t lds = (size_t)(3 * E + kSortThreads) * sizeof(int32_t);
        GX_CHECK(lds <= 64 * 1024, "gx: %d experts do not fit the sort's LDS", E);
        moe_sort_kernel<<<1, kSortThreads, lds, ctx->stream>>>(ids, U, E, 128, s.max_items, sorted, work);
        if (int rc = check_launch("moe_sort"))
            return rc;
        if (int rc = launch_q4_0_gemm_grouped(ctx, gate_up, work, s.max_items, sorted, k, xq, xs, gu, 2 * F))
            return rc;
    } else {
        if (int rc = launch_q4_0_matvec_units(ctx, gate_up, ids, U, k, xq, xs, xqs, gu, 2 * F, nullptr))
            return rc;
    }
    const size_t n = (size_t)U * F;
    moe_gelu_mul_quant_kernel<<<(unsigned)((n + 255) / 256), 256, 0, ctx->stream>>>(gu, 2 * F, F, U, gelu_table,
                                                                                    mq, ms, mqs);
    if (int rc = check_launch("moe_gelu_mul_quant"))
        return rc;
    if (grouped) {
        if (int rc = launch_q4_0_gemm_grouped(ctx, down, work, s.max_items, sorted, 1, mq, ms, part, D))
            return rc;
    } else {
        if (int rc = launch_q4_0_matvec_units(ctx, down, ids, U, 1, mq, ms, mqs, part, D, nullptr))
            return rc;
    }
    const size_t no = (size_t)M * D;
    moe_reduce_kernel<<<(unsigned)((no + 255) / 256), 256, 0, ctx->stream>>>(part, D, M, k, ids, weights,
                                                                             down_scale, out, ldo);
    return check_launch("moe_reduce");
}

}  // namespace gx
