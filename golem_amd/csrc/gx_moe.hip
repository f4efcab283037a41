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

constexpr int kRouteThreads = 512;

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

// Route for one position per workgroup.
__global__ __launch_bounds__(kRouteThreads) void moe_route_kernel(const float *__restrict__ router, int D, int E,
                                                                  const float *__restrict__ router_scale,
                                                                  const float *__restrict__ resid, int ldr, int k,
                                                                  float eps, float *__restrict__ logits,
                                                                  int32_t *__restrict__ ids,
                                                                  float *__restrict__ weights) {
    extern __shared__ float xr[];  // D floats, then E logits
    __shared__ double part[kRouteThreads];
    __shared__ float chains[kRouteThreads];
    const int tid = threadIdx.x;
    const int t = blockIdx.x;
    const float *x = resid + (size_t)t * ldr;
    float *lg = xr + D;

    // RMSNormPlain (nn/ops.go:195-214): float32 squares summed in float64.
    // The sum is taken in a fixed tree (each thread its elements in order,
    // then pairwise), not golem's left-to-right loop; the two float64 sums
    // differ by at most a few units in the 53rd bit, below the float32
    // rounding of the mean except in rare ties.
    double s = 0.0;
    for (int i = tid; i < D; i += kRouteThreads) {
        const float v = x[i];
        const float sq = v * v;
        s += (double)sq;
    }
    part[tid] = s;
    __syncthreads();
    for (int w = kRouteThreads / 2; w > 0; w >>= 1) {
        if (tid < w)
            part[tid] = part[tid] + part[tid + w];
        __syncthreads();
    }
    const float mean = (float)(part[0] / (double)D);
    const float scale = (float)(1.0 / sqrt((double)(mean + eps)));
    const float inv_sqrt_dim = (float)(1.0 / sqrt((double)D));
    for (int i = tid; i < D; i += kRouteThreads) {
        const float normed = x[i] * scale;
        const float factor = inv_sqrt_dim * (router_scale ? router_scale[i] : 1.0f);
        xr[i] = normed * factor;
    }
    __syncthreads();

    // DotF32 (nn/dot_f32.go:13-33) for every expert: four lanes per expert
    // run the four accumulators, elements past the last four go to the
    // first, result (s0 + s1) + (s2 + s3).
    const int whole = D & ~3;
    for (int base = 0; base < 4 * E; base += kRouteThreads) {
        const int id = base + tid;
        const int e = id >> 2, c = id & 3;
        float acc = 0.0f;
        if (e < E) {
            const float *row = router + (size_t)e * D;
            for (int i = c; i < whole; i += 4) {
                const float p = row[i] * xr[i];
                acc = acc + p;
            }
            if (c == 0)
                for (int i = whole; i < D; i++) {
                    const float p = row[i] * xr[i];
                    acc = acc + p;
                }
        }
        chains[tid] = acc;
        __syncthreads();
        if (e < E && c == 0) {
            const float v = (chains[tid] + chains[tid + 1]) + (chains[tid + 2] + chains[tid + 3]);
            lg[e] = v;
            logits[(size_t)t * E + e] = v;
        }
        __syncthreads();
    }

    // chooseExperts (gemma/moe.go:62-88).
    if (tid == 0) {
        int32_t chosen[64];
        for (int j = 0; j < k; j++) {
            int best = -1;
            for (int e = 0; e < E; e++) {
                bool taken = false;
                for (int i = 0; i < j; i++)
                    taken |= chosen[i] == e;
                if (taken)
                    continue;
                if (best < 0 || lg[e] > lg[best])
                    best = e;
            }
            chosen[j] = best;
            ids[(size_t)t * k + j] = best;
        }
        const float top = lg[chosen[0]];
        float total = 0.0f;
        float wv[64];
        for (int j = 0; j < k; j++) {
            wv[j] = (float)exp((double)(lg[chosen[j]] - top));
            total += wv[j];
        }
        for (int j = 0; j < k; j++)
            weights[(size_t)t * k + j] = wv[j] / total;
    }
}

// mid = GELUTable(gate) * up for one unit per workgroup row, then its Q8_0
// form (Batch.quantizeBlock): gate_up is [U][2F], mid_q [U][F].
__global__ __launch_bounds__(256) void moe_gelu_mul_quant_kernel(const float *__restrict__ gate_up, int F, int U,
                                                                  const float *__restrict__ table,
                                                                  int8_t *__restrict__ q, float *__restrict__ scales,
                                                                  int32_t *__restrict__ qsum) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (size_t)U * F)
        return;  // U*F is a multiple of 32: whole 32-lane groups drop out
    const int u = (int)(gid / F), i = (int)(gid % F);
    const float gate = gate_up[(size_t)u * 2 * F + i];
    const float up = gate_up[(size_t)u * 2 * F + F + i];
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

int launch_gelu_table(gx_ctx *ctx, float *table) {
    gelu_table_kernel<<<256, 256, 0, ctx->stream>>>(table);
    return check_launch("gelu_table");
}

int launch_moe_route(gx_ctx *ctx, const gx_weight *router, const float *router_scale, const float *resid, int ldr,
                     int M, int k, float eps, float *logits, int32_t *ids, float *weights) {
    const int D = router->cols, E = router->rows;
    const size_t lds = (size_t)(D + E) * sizeof(float);
    GX_CHECK(lds <= 64 * 1024, "gx: a router of %d x %d does not fit this kernel's LDS", E, D);
    moe_route_kernel<<<M, kRouteThreads, lds, ctx->stream>>>((const float *)router->dev, D, E, router_scale, resid,
                                                             ldr, k, eps, logits, ids, weights);
    return check_launch("moe_route");
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
        if (int rc = launch_q4_0_matvec_units(ctx, gate_up, ids, U, k, xq, xs, xqs, gu, 2 * F))
            return rc;
    }
    const size_t n = (size_t)U * F;
    moe_gelu_mul_quant_kernel<<<(unsigned)((n + 255) / 256), 256, 0, ctx->stream>>>(gu, F, U, gelu_table, mq, ms,
                                                                                    mqs);
    if (int rc = check_launch("moe_gelu_mul_quant"))
        return rc;
    if (grouped) {
        if (int rc = launch_q4_0_gemm_grouped(ctx, down, work, s.max_items, sorted, 1, mq, ms, part, D))
            return rc;
    } else {
        if (int rc = launch_q4_0_matvec_units(ctx, down, ids, U, 1, mq, ms, mqs, part, D))
            return rc;
    }
    const size_t no = (size_t)M * D;
    moe_reduce_kernel<<<(unsigned)((no + 255) / 256), 256, 0, ctx->stream>>>(part, D, M, k, ids, weights,
                                                                             down_scale, out, ldo);
    return check_launch("moe_reduce");
}

}  // namespace gx
