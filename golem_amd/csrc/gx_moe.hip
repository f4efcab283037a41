// gx_moe.hip - the expert branch of golem's mixture of experts on the device.
//
// ExpertFFN (gemma/moe.go:112-180) for M positions:
//   Route (gemma/moe.go:34-53): x = RMSNormPlain(resid) * (1/sqrt(Dim)) *
//     RouterScale, router logits = DotF32(router row, x) in the order golem
//     runs it on x86 (dotF32AVX2), chooseExperts (moe.go:62-88): top_k by
//     repeated argmax (strict >,
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

// The router.
//
// Logits: DotF32 on an amd64 host with AVX2 (nn/dot_f32.go:18-20) is
// dotF32AVX2 (nn/dot_f32_amd64.s:43-113): 32 chains -- lane j of its four
// eight-lane registers adds the product of element 32g + j of every group of
// 32, each product rounded before the add -- then lanes j + 8 onto j and j +
// 24 onto j + 16, those two, lanes j + 4, pairs (0, 2) and (1, 3), and the
// last two (dot_f32_avx2_combine).  A lane runs one chain, so the logits are
// golem's x86 bits, from chains of D/32 steps where the generic form's four
// chains take D/4.  (The router's width is a multiple of 64: no eights, no
// tail.)  RMSNormPlain (nn/ops.go:195-214) squares in float32 and
// sums in float64, here in a fixed tree: 512 partial sums, partial t holding
// elements t, t+512, t+1024, ... in order, then halved pairwise (t + w for
// w = 256 .. 1).  golem sums left to right; the two float64 sums differ by a
// few units in the 53rd bit, below the float32 rounding of the mean except in
// rare ties.  The normalised input is (x * scale) * ((1/sqrt(D)) *
// RouterScale[i]), as Route forms it (gemma/moe.go:34-53).
//
//   moe_route_one_kernel: one workgroup per (expert, position) for few
//     positions (decode), where the cost is latency: the row and the input
//     are read with every load issued at once, the products are formed by
//     all threads into LDS, and 32 lanes run the chains.  The choice is a
//     second launch (moe_topk_kernel): handing the logits to the position's
//     last workgroup inside the launch (a release count per logit, an
//     acquire, the logits read back at device scope) cost more than the
//     launch (config 4 decode 24.6 -> 22.7 us).
//   moe_norm_scale_kernel + moe_logits_kernel: the norm scales once per
//     position, then 8 experts x 16 positions per workgroup, a lane one
//     chain of four positions' logits; rows and inputs pass through LDS 256
//     inputs at a time.  Many positions; the choosing is moe_topk_kernel.
constexpr int kLogitsThreads = 256;
constexpr int kLogitsChunk = 64;     // the router's width is a multiple of this
constexpr int kLogitsOneMaxD = 7168; // input + products in LDS: 57 KB
constexpr int kLogitsOneF4 = kLogitsOneMaxD / 4 / kLogitsThreads;
constexpr int kTopkMaxPerLane = 16;  // E <= 1024
constexpr int kTopkMax = 64;         // k <= 64
constexpr int kUnitMaxPos = 4;       // positions whose units run as matrix-vector products
constexpr int kGroupTok = 32;        // units of a grouped product's work item (its token tile)

// dotF32AVX2's end (nn/dot_f32_amd64.s:79-99) over the 32 chains held by the
// lanes of an aligned 32-lane group (chain j in lane j): Y0 + Y1 and Y2 + Y3
// lane by lane, then their sum, then lanes j and j + 4, then (0, 2) and
// (1, 3), then the two.  The result is in the group's first lane.
__device__ __forceinline__ float dot_f32_avx2_combine(float acc) {
    const float t = acc + __shfl_down(acc, 8, 32);   // lanes 0..7: Y0 + Y1; 16..23: Y2 + Y3
    const float v = t + __shfl_down(t, 16, 32);      // lanes 0..7: (Y0 + Y1) + (Y2 + Y3)
    const float w = v + __shfl_down(v, 4, 32);       // lanes 0..3
    const float x = w + __shfl_down(w, 2, 32);       // lanes 0..1
    return x + __shfl_down(x, 1, 32);                // lane 0
}

// chooseExperts (gemma/moe.go:62-88) for one position, by a whole workgroup
// of at least 64 threads.  golem takes k rounds of an argmax that scans in
// index order and replaces its best only on a strictly greater logit.
// Without a NaN the rounds take the logits by value, largest first and
// equal values lower index first, so logit i is taken in round
//     r = #{j : l_j > l_i} + #{j < i : l_j == l_i},
// which every thread computes for its logit at once, one unsigned compare a
// logit, on keys that order (value, -index) as one 64-bit integer
// (rank_key).  A NaN is taken only as the first logit not yet chosen (no
// comparison with it is ever true); with any NaN present wavefront 0 runs
// the rounds as golem does.  Weights: exp(l - top) in float64 of the float32
// difference, rounded to float32 (exp_neg: bit for bit that, on every
// difference this can be, <= 0 or NaN), summed in slot order, divided by the
// sum -- in wavefront 0's registers, the sum's terms by shuffles.
//
// The caller stages the logits in LDS first (stage_logits): lg holds them
// as floats and comp their keys, both padded to a multiple of 32 (keys 0,
// below every logit's), and any_nan says whether one is a NaN.

// The order of a non-NaN float as an unsigned integer (-0 taken as +0, as
// golem's comparisons take it), above it the index reversed: a larger key
// is a larger logit, or an equal one at a lower index.
__device__ __forceinline__ uint64_t rank_key(float v, int i) {
    const uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
    const uint32_t key = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)key << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)i);
}

// Logits [0, E) from `src` (read by `load`) into lg and comp; returns, in
// every thread, whether any is a NaN (the barrier that publishes them).
template <typename Load>
__device__ __forceinline__ bool stage_logits(int E, float *lg, uint64_t *comp, Load &&load) {
    const int E32 = (E + 31) & ~31;
    bool nan_here = false;
    for (int i = threadIdx.x; i < E32; i += blockDim.x) {
        const float v = i < E ? load(i) : -__builtin_inff();
        lg[i] = v;
        comp[i] = i < E ? rank_key(v, i) : 0;
        nan_here |= v != v;
    }
    return __syncthreads_or(nan_here);
}

__device__ void choose_experts(const float *lg, const uint64_t *comp, bool any_nan, int E, int k, float *sel_l,
                               int32_t *sel_i, int32_t *__restrict__ ids, float *__restrict__ weights) {
    const int tid = threadIdx.x, nt = blockDim.x;
    if (!any_nan) {
        // Two threads a logit when the workgroup has them (adjacent lanes,
        // each half of the keys), their counts added by a lane swap.
        const int E32 = (E + 31) & ~31;
        const int split = nt >= 2 * E32 ? 2 : 1;
        const int span = E32 / split, per = nt / split;
        for (int i0 = 0; i0 < E; i0 += per) {  // the same trip count in every thread
            const int i = i0 + tid / split, h = tid % split;
            const uint64_t c = comp[min(i, E - 1)];
            const uint64_t *cj = comp + h * span;
            int r = 0;
            for (int j = 0; j < span; j += 16) {
                uint64_t w[16];  // 16 keys in flight at once
#pragma unroll
                for (int u = 0; u < 16; u++)
                    w[u] = cj[j + u];
#pragma unroll
                for (int u = 0; u < 16; u++)
                    r += (int)(w[u] > c);
            }
            if (split == 2)
                r += __shfl_xor(r, 1, 64);
            if (i < E && h == 0 && r < k) {
                sel_l[r] = lg[i];
                sel_i[r] = i;
            }
        }
    } else if (tid < 64) {
        const int lane = tid;
        float v[kTopkMaxPerLane];
        unsigned taken = 0;  // bit j: logit lane + 64 j is chosen or absent
#pragma unroll
        for (int j = 0; j < kTopkMaxPerLane; j++) {
            const int e = lane + 64 * j;
            v[j] = lg[min(e, E - 1)];
            taken |= (e >= E ? 1u : 0u) << j;
        }
        for (int round = 0; round < k; round++) {
            // the first logit not yet chosen wins the round if it is a NaN
            int first = 0x7fffffff;
            const unsigned open = ~taken & ((1u << kTopkMaxPerLane) - 1);
            if (open)
                first = lane + 64 * __builtin_ctz(open);
            for (int w = 32; w > 0; w >>= 1)
                first = min(first, __shfl_xor(first, w, 64));
            int best = lg[first] != lg[first] ? first : 0x7fffffff;
            if (best == 0x7fffffff) {
                // otherwise the largest non-NaN logit not yet chosen, the
                // lowest index among equals
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
                sel_i[round] = best;
                sel_l[round] = lg[best];
            }
        }
    }
    __syncthreads();
    if (tid < 64) {
        const float e = exp_neg(sel_l[min(tid, k - 1)] - sel_l[0]);
        float total = 0.0f;
        for (int j = 0; j < k; j++)
            total += __shfl(e, j, 64);
        if (tid < k) {
            ids[tid] = sel_i[tid];
            weights[tid] = e / total;
        }
    }
}

__global__ __launch_bounds__(kLogitsThreads) void moe_route_one_kernel(
    const float *__restrict__ router, int D, int E, const float *__restrict__ router_scale,
    const float *__restrict__ resid, int ldr, float eps, float *__restrict__ logits) {
    // LDS: the input [D], then the products [D] in element order
    extern __shared__ __align__(16) float lds[];
    __shared__ double red[kLogitsThreads];
    __shared__ float scale_sh;
    const int tid = threadIdx.x, e = blockIdx.x, t = blockIdx.y;
    float *xr = lds;
    float *P = lds + D;
    const float *rg = router + (size_t)e * D;
    const float *xg = resid + (size_t)t * ldr;
    const int n4 = D / 4;
    // Clamped indices: every load is issued before the first wait, with no
    // branch for a load to sink into.
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
        const int q = tid + f * kLogitsThreads;
        if (q < n4)
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
    // The products row[i] * ((x[i] * scale) * ((1/sqrt(D)) * RouterScale[i])),
    // in element order.
#pragma unroll
    for (int f = 0; f <= kLogitsOneF4; f++) {
        const int q = tid + f * kLogitsThreads;
        const float x4[4] = {xv[f].x, xv[f].y, xv[f].z, xv[f].w}, s4[4] = {sv[f].x, sv[f].y, sv[f].z, sv[f].w};
        const float r4[4] = {rv[f].x, rv[f].y, rv[f].z, rv[f].w};
        if (q < n4) {
            float4 pv;
            float *pp = (float *)&pv;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const float normed = x4[c] * sc;
                const float factor = inv_sqrt_dim * s4[c];
                const float xn = normed * factor;
                pp[c] = r4[c] * xn;
            }
            *(float4 *)(P + 4 * q) = pv;
        }
    }
    __syncthreads();
    if (tid < 64) {
        // chain tid (lanes 0..31): products tid, tid + 32, ... in order, eight
        // read ahead of the dependent adds
        float acc = 0.0f;
        const int steps = D / 32;
        const float *pc = P + (tid & 31);
        float a[8];
#pragma unroll
        for (int u = 0; u < 8; u++)
            a[u] = pc[32 * min(u, steps - 1)];
        for (int g = 0; g < steps; g += 8) {
            float b[8];
#pragma unroll
            for (int u = 0; u < 8; u++)
                b[u] = pc[32 * min(g + 8 + u, steps - 1)];
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (g + u < steps)
                    acc = acc + a[u];
#pragma unroll
            for (int u = 0; u < 8; u++)
                a[u] = b[u];
        }
        const float logit = dot_f32_avx2_combine(acc);
        if (tid == 0)
            logits[(size_t)t * E + e] = logit;
    }
}

// Many positions: the norm scales first, one wavefront a position
// (moe_norm_scale_kernel, every load of a position in flight at once), then
// the logits.
//
// RMSNormPlain's scale of one position with exactly the sums of
// norm_partials + norm_tree: lane l holds partials l + 64 m (m < 8),
// partial t summing elements t, t + 512, ... in order; then the same
// pairwise halving (t + 256, t + 128, t + 64 within the lane, then across
// lanes).
constexpr int kNormRounds = 8;  // 512-element rounds of loads in flight at once

__global__ __launch_bounds__(256) void moe_norm_scale_kernel(const float *__restrict__ resid, int ldr, int M, int D,
                                                             float eps, float *__restrict__ scale) {
    const int l = threadIdx.x & 63, t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= M)
        return;  // whole wavefronts
    const float *x = resid + (size_t)t * ldr;
    double p[8];
#pragma unroll
    for (int m = 0; m < 8; m++)
        p[m] = 0.0;
    for (int base = 0; base < D; base += 512 * kNormRounds) {
        float v[kNormRounds][8];
#pragma unroll
        for (int u = 0; u < kNormRounds; u++)
#pragma unroll
            for (int m = 0; m < 8; m++)
                v[u][m] = x[min(base + 512 * u + l + 64 * m, D - 1)];
#pragma unroll
        for (int u = 0; u < kNormRounds; u++)
#pragma unroll
            for (int m = 0; m < 8; m++) {
                const float a = base + 512 * u + l + 64 * m < D ? v[u][m] : 0.0f;
                const float sq = a * a;
                p[m] += (double)sq;
            }
    }
    double q[4], r[2];
#pragma unroll
    for (int m = 0; m < 4; m++)
        q[m] = p[m] + p[m + 4];
#pragma unroll
    for (int m = 0; m < 2; m++)
        r[m] = q[m] + q[m + 2];
    double s = r[0] + r[1];
    for (int w = 32; w > 0; w >>= 1) {
        const double o = __shfl_down(s, w, 64);
        if (l < w)
            s = s + o;
    }
    if (l == 0)
        scale[t] = norm_scale(s, D, eps);
}

// The logits: EW experts x P positions a workgroup (32 EW G threads), a lane
// one of the 32 chains of P / G logits (lane = chain j + 32 (expert + EW
// group)): group g holds positions g, g + G, ... so that each router element
// read from LDS serves P / G positions.  Rows and inputs pass through LDS CH
// at a time, double buffered (the next chunk's global loads are in flight
// while this one is summed); chain j adds the products of the chunk's
// elements j, j + 32, ... in order, and a logit's 32 lanes meet as
// dotF32AVX2 ends.
constexpr int kLgEW = 8;

template <int P, int G, int CH>
__global__ __launch_bounds__(32 * kLgEW * G) void moe_logits_kernel(const float *__restrict__ router, int D, int E,
                                                                   const float *__restrict__ router_scale,
                                                                   const float *__restrict__ resid, int ldr, int M,
                                                                   const float *__restrict__ scales,
                                                                   float *__restrict__ logits) {
    constexpr int NT = 32 * kLgEW * G, Q = CH / 4, PG = P / G;  // threads; float4s of a row's chunk
    constexpr int RF = (kLgEW * Q + NT - 1) / NT, XF = (P * Q + NT - 1) / NT;  // staged float4s a thread
    static_assert(CH % 32 == 0 && P % G == 0, "whole groups of 32 a chunk, whole position groups");
    __shared__ __align__(16) float Rs[2][kLgEW][CH];
    __shared__ __align__(16) float Xs[2][P][CH];
    const int tid = threadIdx.x;
    const int e0 = blockIdx.x * kLgEW, t0 = blockIdx.y * P;
    const int j = tid & 31, e = (tid >> 5) % kLgEW, g = tid / (32 * kLgEW);  // this lane's chains
    const float inv_sqrt_dim = (float)(1.0 / sqrt((double)D));

    // This thread's staging: row piece idx = tid + NT f (expert idx / Q,
    // float4 idx % Q of the chunk), input piece likewise (position idx / Q);
    // past D the pieces are zero.
    float4 rv[RF], xv[XF], sv[XF];
    float sc[XF];
#pragma unroll
    for (int f = 0; f < XF; f++)
        sc[f] = scales[min(t0 + min((tid + NT * f) / Q, P - 1), M - 1)];
    auto fetch = [&](int k) {
        const int i0 = k * CH;
#pragma unroll
        for (int f = 0; f < RF; f++) {
            const int idx = tid + NT * f, i = i0 + 4 * (idx % Q);
            const float *rsrc = router + (size_t)min(e0 + min(idx / Q, kLgEW - 1), E - 1) * D;
            rv[f] = i < D ? *(const float4 *)(rsrc + i) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (int f = 0; f < XF; f++) {
            const int idx = tid + NT * f, i = i0 + 4 * (idx % Q);
            const float *xr = resid + (size_t)min(t0 + min(idx / Q, P - 1), M - 1) * ldr;
            xv[f] = i < D ? *(const float4 *)(xr + i) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            sv[f] = router_scale && i < D ? *(const float4 *)(router_scale + i) : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
        }
    };
    auto put = [&](int buf) {
#pragma unroll
        for (int f = 0; f < RF; f++) {
            const int idx = tid + NT * f;
            if (idx < kLgEW * Q)
                *(float4 *)&Rs[buf][idx / Q][4 * (idx % Q)] = rv[f];
        }
#pragma unroll
        for (int f = 0; f < XF; f++) {
            const int idx = tid + NT * f;
            if (idx < P * Q) {
                const float x4[4] = {xv[f].x, xv[f].y, xv[f].z, xv[f].w}, s4[4] = {sv[f].x, sv[f].y, sv[f].z, sv[f].w};
                float4 o;
                float *op = (float *)&o;
#pragma unroll
                for (int cc = 0; cc < 4; cc++) {
                    const float normed = x4[cc] * sc[f];
                    const float factor = inv_sqrt_dim * s4[cc];
                    op[cc] = normed * factor;
                }
                *(float4 *)&Xs[buf][idx / Q][4 * (idx % Q)] = o;
            }
        }
    };

    const int chunks = (D + CH - 1) / CH;
    fetch(0);
    put(0);
    __syncthreads();
    float acc[PG];
#pragma unroll
    for (int c = 0; c < PG; c++)
        acc[c] = 0.0f;
    for (int k = 0; k < chunks; k++) {
        const int buf = k & 1;
        if (k + 1 < chunks)
            fetch(k + 1);
        const float *rr = Rs[buf][e] + j;
        const float *xx = Xs[buf][g] + j;
        // the chunk's steps in order; past D the products are +0, which
        // leave a sum that starts from +0 unchanged
#pragma unroll
        for (int s = 0; s < CH / 32; s++) {
            const float r = rr[32 * s];
#pragma unroll
            for (int c = 0; c < PG; c++) {
                const float prod = r * xx[G * CH * c + 32 * s];
                acc[c] = acc[c] + prod;
            }
        }
        if (k + 1 < chunks)
            put(buf ^ 1);  // the other buffer was last read in chunk k - 1
        __syncthreads();
    }
#pragma unroll
    for (int c = 0; c < PG; c++) {
        const int p = g + G * c;
        const float logit = dot_f32_avx2_combine(acc[c]);
        if (j == 0 && t0 + p < M && e0 + e < E)
            logits[(size_t)(t0 + p) * E + e0 + e] = logit;
    }
}

// chooseExperts for many positions: one workgroup a position.
__global__ __launch_bounds__(256) void moe_topk_kernel(const float *__restrict__ logits, int E, int k,
                                                       int32_t *__restrict__ ids, float *__restrict__ weights) {
    __shared__ __align__(16) float lg[64 * kTopkMaxPerLane];
    __shared__ __align__(16) uint64_t comp[64 * kTopkMaxPerLane];
    __shared__ float sel_l[kTopkMax];
    __shared__ int32_t sel_i[kTopkMax];
    const int t = blockIdx.x;
    const float *lt = logits + (size_t)t * E;
    const bool any_nan = stage_logits(E, lg, comp, [&](int i) { return lt[i]; });
    choose_experts(lg, comp, any_nan, E, k, sel_l, sel_i, ids + (size_t)t * k, weights + (size_t)t * k);
}

// mid = GELUTable(gate) * up for the 32 values of one Q8_0 block, one value a
// lane on lanes 0..31 (all of them active), then the block's Q8_0
// (Batch.quantizeBlock, nn/batch.go:109-143, as gx_quant.hip's kernel):
// lane l writes q[l]; lane 0 the scale (through fp16) and the sum of q.
// golem's GELU table (nn/gelu_table.go:25-38): for every fp16 input,
// fp16(float32(geluTanh(float64(input)))), held as float.
// GELUTable (nn/gelu_table.go:40-52): 0 at or below -10, the input at or
// above 10, the table at the input's fp16 bits between -- read from the
// table, or (table null) the table's entry computed in place by the
// table's own arithmetic, which saves a dependent global load.
__device__ __forceinline__ float gelu_entry(uint32_t h) {
    const double x = (double)half_bits_to_float(h);
    const double sqrt2_over_pi = 0.79788456080286535587989211986876;
    const double coef_a = 0.044715;
    const double inner = sqrt2_over_pi * x * (1.0 + coef_a * x * x);
    const double g = 0.5 * x * (1.0 + tanh(inner));
    return half_bits_to_float(float_to_half_bits((float)g));
}

__global__ void gelu_table_kernel(float *__restrict__ table) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < 65536)
        table[i] = gelu_entry((uint32_t)i);
}

__device__ __forceinline__ void gelu_mul_q8_0(float gate, float up, const float *__restrict__ table, int8_t *q,
                                              float *scale_out, int32_t *qsum_out) {
    const int l = threadIdx.x & 31;
    float gl;
    if (gate <= -10.0f)
        gl = 0.0f;
    else if (gate >= 10.0f)
        gl = gate;
    else
        gl = table ? table[float_to_half_bits(gate)] : gelu_entry(float_to_half_bits(gate));
    const float v = gl * up;
    float peak = fabsf(v);
#pragma unroll
    for (int off = 16; off > 0; off >>= 1)
        peak = fmaxf(peak, __shfl_xor(peak, off, 32));
    if (peak == 0.0f) {
        q[l] = 0;
        if (l == 0) {
            *scale_out = 0.0f;
            *qsum_out = 0;
        }
        return;
    }
    const float scale = __fdiv_rn(peak, 127.0f);
    const float inverse = __fdiv_rn(127.0f, peak);
    const float prod = v * inverse;
    int32_t n = nearest_int(prod);
    n = n > 127 ? 127 : (n < -128 ? -128 : n);
    q[l] = (int8_t)n;
    int32_t sum = n;
#pragma unroll
    for (int off = 16; off > 0; off >>= 1)
        sum += __shfl_xor(sum, off, 32);
    if (l == 0) {
        *scale_out = half_bits_to_float(float_to_half_bits(scale));
        *qsum_out = sum;
    }
}

// mid = GELUTable(gate) * up for one unit per workgroup row, then its Q8_0
// form: gate_up is [U][ld] with each row's F gates then its F ups, mid_q
// [U][F].  (The grouped path; few positions fuse this into the product.)
__global__ __launch_bounds__(256) void moe_gelu_mul_quant_kernel(const float *__restrict__ gate_up, int ld, int F,
                                                                  int U, const float *__restrict__ table,
                                                                  int8_t *__restrict__ q, float *__restrict__ scales,
                                                                  int32_t *__restrict__ qsum) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (size_t)U * F)
        return;  // U*F is a multiple of 32: whole 32-lane groups drop out
    const int u = (int)(gid / F), i = (int)(gid % F);
    const size_t index = (size_t)u * (F >> 5) + (i >> 5);
    gelu_mul_q8_0(gate_up[(size_t)u * ld + i], gate_up[(size_t)u * ld + F + i], table, q + (gid & ~(size_t)31),
                  scales + index, qsum + index);
}

// The same, four values a lane (eight lanes a Q8_0 block, q8_0_quad's
// arithmetic, which is gelu_mul_q8_0's): for 16-byte aligned rows.
__global__ __launch_bounds__(256) void moe_gelu_mul_quant4_kernel(const float *__restrict__ gate_up, int ld, int F,
                                                                   int U, const float *__restrict__ table,
                                                                   int8_t *__restrict__ q,
                                                                   float *__restrict__ scales,
                                                                   int32_t *__restrict__ qsum) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int F4 = F / 4;
    if (gid >= (size_t)U * F4)
        return;  // U*F/4 is a multiple of 8: whole 8-lane groups drop out
    const int u = (int)(gid / F4), i = 4 * (int)(gid % F4);
    const float4 g4 = *(const float4 *)(gate_up + (size_t)u * ld + i);
    const float4 u4 = *(const float4 *)(gate_up + (size_t)u * ld + F + i);
    const float gate[4] = {g4.x, g4.y, g4.z, g4.w}, up[4] = {u4.x, u4.y, u4.z, u4.w};
    float v[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        float gl;
        if (gate[c] <= -10.0f)
            gl = 0.0f;
        else if (gate[c] >= 10.0f)
            gl = gate[c];
        else
            gl = table[float_to_half_bits(gate[c])];
        v[c] = gl * up[c];
    }
    float stored;
    int32_t sum;
    const uint32_t packed = q8_0_quad(v, &stored, &sum);
    *(uint32_t *)(q + (size_t)u * F + i) = packed;
    if ((gid & 7) == 0) {
        const size_t index = (size_t)u * (F >> 5) + (i >> 5);
        scales[index] = stored;
        qsum[index] = sum;
    }
}

// ---- few positions: the units as matrix-vector products ---------------------
//
// Two kernels after the router, each reading its expert matrices once per
// unit (moe.go:127-163):
//   moe_gate_up_kernel: unit u = blockIdx.y (position u / k, expert ids[u]).
//     Its position's input is quantised to Q8_0 by each wavefront for the
//     stretch it multiplies (q8_0_quad: the separate quantiser's values) and
//     moved to SGPRs, as in the fused norm products.  A workgroup owns gate
//     rows 32h .. 32h+31 (lanes 0..31) and the same up rows F + 32h ..
//     (lanes 32..63), each lane reading its row where the R64 layout keeps it,
//     so that its 32 results are one Q8_0 block of mid: GELUTable(gate) * up
//     and the block's Q8_0 are its epilogue.
//   moe_down_reduce_kernel: position t = blockIdx.y; a workgroup owns 16 rows
//     (a quarter of an R64 tile) of all k units' down products, and sums them
//     with the routing weights in slot order -- golem's Axpy (out = 0, out +=
//     (w_j * DownScale[id_j]) * value_j, a rounded product then a rounded sum)
//     -- so no partial leaves the workgroup.
// A unit's row value is the canonical one of every Q4_0 kernel here (block
// products fma'd within a stretch from +0, stretch sums in order from +0).
// An id outside [0, E) reads nothing: its unit's value is NaN, and so is its
// position's output.
//
// DOTS: the same kernels writing each (unit, row, block) integer, gate_up
// into dots[u][row][b] for its 2F rows in golem's order, down into
// dots[t*k + j][row][b]; they then store no output.

template <bool DOTS>
__global__ __launch_bounds__(1024) void moe_gate_up_kernel(
    const uint8_t *__restrict__ W, size_t plane0_bytes, size_t matrix_bytes, int B, int DC, int F, int experts,
    const float *__restrict__ x, int ldx, int k, const int32_t *__restrict__ ids, const float *__restrict__ table,
    int8_t *__restrict__ mq, float *__restrict__ ms, int32_t *__restrict__ mqs, int32_t *__restrict__ dots) {
    extern __shared__ float part[];  // [S][64]
    const int K = B * kQ4Block, S = (B + kStretch - 1) / kStretch;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nwaves = blockDim.x >> 6;
    const int h = blockIdx.x, u = blockIdx.y;
    const int e = ids[u];
    const size_t mb = (size_t)u * (F / kQ4Block) + h;  // the mid block this workgroup makes
    if (e < 0 || e >= experts) {
        if (!DOTS && threadIdx.x < 32) {
            mq[mb * kQ4Block + threadIdx.x] = 0;
            if (threadIdx.x == 0) {
                ms[mb] = __builtin_nanf("");
                mqs[mb] = 0;
            }
        }
        return;
    }
    W += (size_t)e * matrix_bytes;
    const float *xa = x + (size_t)(u / k) * ldx;
    const int rowg = lane < 32 ? 32 * h + lane : F + 32 * h + (lane - 32);  // golem's row of this lane
    const int tile = rowg >> 6, rin = rowg & 63;
    const uint8_t *qs_row = W + ((size_t)tile * B * kTileRows + rin) * kChunk;
    const uint8_t *d_row = W + plane0_bytes + ((size_t)tile * DC * kTileRows + rin) * kChunk;

    for (int s = wave; s < S; s += nwaves) {
        const int b0 = s * kStretch;
        const int nb = min(kStretch, B - b0);
        // The stretch's inputs first (values 32 b0 + 4 lane .. + 3; past the
        // row the last four again, never used), then its weights.
        float v[4];
        const int i0 = min(b0 * kQ4Block + 4 * lane, K - 4);
#pragma unroll
        for (int c = 0; c < 4; c++)
            v[c] = xa[i0 + c];
        uint4 wq[kStretch];
#pragma unroll
        for (int j = 0; j < kStretch; j++)
            wq[j] = load_stream(qs_row + (size_t)min(b0 + j, B - 1) * kTileRows * kChunk);
        const uint4 dch = *(const uint4 *)(d_row + (size_t)s * kTileRows * kChunk);
        float bstored;
        int32_t bsum;
        const uint32_t aq = q8_0_quad(v, &bstored, &bsum);
        float p = 0.0f;
#pragma unroll
        for (int j = 0; j < kStretch; j++) {
            if (j < nb) {
                int4 a0, a1;
                a0.x = __builtin_amdgcn_readlane((int)aq, 8 * j + 0);
                a0.y = __builtin_amdgcn_readlane((int)aq, 8 * j + 1);
                a0.z = __builtin_amdgcn_readlane((int)aq, 8 * j + 2);
                a0.w = __builtin_amdgcn_readlane((int)aq, 8 * j + 3);
                a1.x = __builtin_amdgcn_readlane((int)aq, 8 * j + 4);
                a1.y = __builtin_amdgcn_readlane((int)aq, 8 * j + 5);
                a1.z = __builtin_amdgcn_readlane((int)aq, 8 * j + 6);
                a1.w = __builtin_amdgcn_readlane((int)aq, 8 * j + 7);
                const int32_t qs = __builtin_amdgcn_readlane(bsum, 8 * j);
                const float sa = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bstored), 8 * j));
                const int32_t isum = q4_0_block_isum(wq[j], a0, a1, qs);
                const float scl = chunk_half(dch, j) * sa;
                p = fmaf((float)isum, scl, p);
                if (DOTS)
                    dots[((size_t)u * 2 * F + rowg) * B + b0 + j] = isum;
            }
        }
        part[s * kTileRows + lane] = p;
    }
    __syncthreads();
    if (!DOTS && wave == 0) {
        float acc = 0.0f;
        for (int s0 = 0; s0 < S; s0 += 8) {
            float pv[8];  // eight stretch sums in flight at once, added in order
#pragma unroll
            for (int u = 0; u < 8; u++)
                pv[u] = part[min(s0 + u, S - 1) * kTileRows + lane];
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (s0 + u < S)
                    acc = acc + pv[u];
        }
        const float up = __shfl_down(acc, 32, 64);
        if (lane < 32)
            gelu_mul_q8_0(acc, up, table, mq + mb * kQ4Block, ms + mb, mqs + mb);
    }
}

constexpr int kDownRows = 16;   // rows of a down workgroup
constexpr int kDownActRegs = 4; // staged 16-byte activation pieces per thread

__host__ __device__ inline size_t down_part_bytes(int pairs) { return ((size_t)pairs * kDownRows * 4 + 15) & ~(size_t)15; }

template <bool DOTS>
__global__ __launch_bounds__(1024) void moe_down_reduce_kernel(
    const uint8_t *__restrict__ W, size_t plane0_bytes, size_t matrix_bytes, int B, int DC, int experts,
    const int8_t *__restrict__ mq, const float *__restrict__ ms, const int32_t *__restrict__ mqs, int k,
    const int32_t *__restrict__ ids, const float *__restrict__ weights, const float *__restrict__ down_scale,
    float *__restrict__ out, int ldo, int D, int32_t *__restrict__ dots) {
    // LDS: the pairs' stretch sums [k*S][16] floats, then the position's k
    // activations: q [k][F] int8, scales [k][B] float, sums [k][B] int32.
    extern __shared__ __align__(16) uint8_t lds_raw[];
    const int F = B * kQ4Block, S = (B + kStretch - 1) / kStretch, P = k * S;
    float *part = (float *)lds_raw;
    int8_t *qa = (int8_t *)(lds_raw + down_part_bytes(P));
    float *sa = (float *)(qa + (size_t)k * F);
    int32_t *qsa = (int32_t *)(sa + (size_t)k * B);
    const int tid = threadIdx.x, nt = blockDim.x;
    const int lane = tid & 63, wave = tid >> 6, nwaves = nt >> 6;
    const int t = blockIdx.y;
    const int tile = blockIdx.x >> 2, r = (blockIdx.x & 3) * kDownRows + (lane & 15);
    const int row = tile * kTileRows + r;
    const int32_t *idt = ids + (size_t)t * k;
    // The routing factors w_j * DownScale[id_j]: lane j of wavefront 0 loads
    // slot j's id and weight ahead of everything, its scale behind the
    // weights (so that no wait for it holds them up), and forms the factor
    // once the products are done; the sum reads it from that lane.
    int e_reg = 0;
    float w_reg = 0.0f;
    if (!DOTS && wave == 0 && lane < k) {
        e_reg = idt[lane];
        w_reg = weights[(size_t)t * k + lane];
    }

    // The activations: every load in flight together (indices past the end
    // clamped, the values never stored), then into LDS below.
    const int n16 = k * F / 16, nb = k * B;
    const int4 *qsrc = (const int4 *)(mq + (size_t)t * k * F);
    const float *ssrc = ms + (size_t)t * k * B;
    const int32_t *qssrc = mqs + (size_t)t * k * B;
    int4 qv[kDownActRegs];
    float sv[kDownActRegs];
    int32_t qsv[kDownActRegs];
#pragma unroll
    for (int a = 0; a < kDownActRegs; a++)
        qv[a] = qsrc[min(tid + a * nt, n16 - 1)];
#pragma unroll
    for (int a = 0; a < kDownActRegs; a++) {
        sv[a] = ssrc[min(tid + a * nt, nb - 1)];
        qsv[a] = qssrc[min(tid + a * nt, nb - 1)];
    }
    // This lane's pair p = j * S + s (slot j, stretch s): pairs wave * 4 +
    // lane / 16, then nwaves * 4 further on.
    int p = wave * 4 + (lane >> 4);
    uint4 wq[kStretch], dch;
    bool bad = false;
    auto load_pair = [&](int pp) {
        const int pc = min(pp, P - 1);
        const int j = pc / S, s = pc - j * S;
        const int e = idt[j];
        bad = e < 0 || e >= experts;
        const uint8_t *We = W + (size_t)(bad ? 0 : e) * matrix_bytes;
        const uint8_t *qs_row = We + ((size_t)tile * B * kTileRows + r) * kChunk;
        const uint8_t *d_row = We + plane0_bytes + ((size_t)tile * DC * kTileRows + r) * kChunk;
#pragma unroll
        for (int jj = 0; jj < kStretch; jj++)
            wq[jj] = load_stream(qs_row + (size_t)min(s * kStretch + jj, B - 1) * kTileRows * kChunk);
        dch = *(const uint4 *)(d_row + (size_t)s * kTileRows * kChunk);
    };
    load_pair(p);
    float ds_reg = 1.0f;
    if (!DOTS && wave == 0 && lane < k && down_scale)
        ds_reg = e_reg >= 0 && e_reg < experts ? down_scale[e_reg] : __builtin_nanf("");
#pragma unroll
    for (int a = 0; a < kDownActRegs; a++) {
        const int i = tid + a * nt;
        if (i < n16)
            ((int4 *)qa)[i] = qv[a];
        if (i < nb) {
            sa[i] = sv[a];
            qsa[i] = qsv[a];
        }
    }
    lds_barrier();

    for (int base = wave * 4;;) {
        if (p < P) {
            const int j = p / S, s = p - j * S;
            const int b0 = s * kStretch;
            const int n = min(kStretch, B - b0);
            const int8_t *aj = qa + (size_t)j * F;
            float acc = 0.0f;
#pragma unroll
            for (int jj = 0; jj < kStretch; jj++) {
                if (jj < n) {
                    const int b = b0 + jj;
                    const int4 *ap = (const int4 *)(aj + (size_t)b * kQ4Block);
                    const int32_t isum = q4_0_block_isum(wq[jj], ap[0], ap[1], qsa[j * B + b]);
                    const float scl = chunk_half(dch, jj) * sa[j * B + b];
                    acc = fmaf((float)isum, scl, acc);
                    if (DOTS && !bad)
                        dots[(((size_t)t * k + j) * D + row) * B + b] = isum;
                }
            }
            part[p * kDownRows + (lane & 15)] = bad ? __builtin_nanf("") : acc;
        }
        base += nwaves * 4;
        if (base >= P)
            break;
        p += nwaves * 4;
        load_pair(p);
    }
    const float a_reg = w_reg * ds_reg;  // slot `lane`'s factor (lanes < k of wavefront 0)
    lds_barrier();

    if (!DOTS && wave == 0 && lane < kDownRows) {
        // The pairs' sums in order, eight in flight at once: each slot's
        // stretch sums from +0, then o += factor * value, slot by slot.
        float o = 0.0f, v = 0.0f;
        int s = 0, j = 0;  // the same in every lane
        for (int p0 = 0; p0 < P; p0 += 8) {
            float pv[8];
#pragma unroll
            for (int u = 0; u < 8; u++)
                pv[u] = part[min(p0 + u, P - 1) * kDownRows + lane];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                if (p0 + u < P) {
                    v = v + pv[u];
                    if (++s == S) {
                        const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a_reg), j));
                        const float pr = a * v;
                        o = o + pr;
                        v = 0.0f;
                        s = 0;
                        j++;
                    }
                }
            }
        }
        out[(size_t)t * ldo + row] = o;
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
__global__ void moe_reduce_kernel(const float *__restrict__ partial, int D, int M, int k, int E,
                                  const int32_t *__restrict__ ids, const float *__restrict__ weights,
                                  const float *__restrict__ down_scale, float *__restrict__ out, int ldo) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (size_t)M * D)
        return;
    const int t = (int)(gid / D), i = (int)(gid % D);
    float acc = 0.0f;
    for (int j = 0; j < k; j++) {
        const int u = t * k + j;
        const int e = ids[u];
        if (e < 0 || e >= E) {  // in no group: its partial row was never written
            acc = __builtin_nanf("");
            continue;
        }
        const float a = weights[u] * (down_scale ? down_scale[e] : 1.0f);
        const float p = a * partial[(size_t)u * D + i];
        acc = acc + p;
    }
    out[(size_t)t * ldo + i] = acc;
}

// The same, four outputs a thread (16-byte aligned rows).
__global__ __launch_bounds__(256) void moe_reduce4_kernel(const float *__restrict__ partial, int D, int M, int k,
                                                          int E, const int32_t *__restrict__ ids,
                                                          const float *__restrict__ weights,
                                                          const float *__restrict__ down_scale,
                                                          float *__restrict__ out, int ldo) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int D4 = D / 4;
    if (gid >= (size_t)M * D4)
        return;
    const int t = (int)(gid / D4), i = 4 * (int)(gid % D4);
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int j = 0; j < k; j++) {
        const int u = t * k + j;
        const int e = ids[u];
        if (e < 0 || e >= E) {  // in no group: its partial row was never written
#pragma unroll
            for (int c = 0; c < 4; c++)
                acc[c] = __builtin_nanf("");
            continue;
        }
        const float a = weights[u] * (down_scale ? down_scale[e] : 1.0f);
        const float4 p4 = *(const float4 *)(partial + (size_t)u * D + i);
        const float pv[4] = {p4.x, p4.y, p4.z, p4.w};
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float p = a * pv[c];
            acc[c] = acc[c] + p;
        }
    }
    *(float4 *)(out + (size_t)t * ldo + i) = make_float4(acc[0], acc[1], acc[2], acc[3]);
}

// ---- F32 expert stacks ------------------------------------------------------
//
// golem's ExpertStack carries any nn.Quant (gemma/weights.go:59-72).  With F32
// stacks, Matrix.rows' F32 case (nn/matrix.go:113-120) multiplies the Batch's
// floats in DotF32's generic order, so the position's input and mid enter
// unquantised (the Batch's Q8_0 form, which QuantizeColumnRange also fills,
// is never read by an F32 matrix): gate|up = DotF32(GateUp[e] row, x_t),
// GELUTable(gate) * up in place of the gate, partial = DotF32(Down[e] row,
// mid), then the same weighted sum.  Four lanes a dot, as f32_matvec_kernel.
// A unit whose id is out of range writes nothing; the sum makes its
// position's output NaN.
__global__ __launch_bounds__(256) void moe_f32_units_kernel(const float *__restrict__ W, size_t matrix_floats,
                                                            int rows, int cols, const float *__restrict__ x, int ldx,
                                                            int act_div, int U, const int32_t *__restrict__ ids,
                                                            int E, float *__restrict__ y, int ldy) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t dot = gid >> 2;
    const int j = (int)(gid & 3);
    const bool in = dot < (size_t)U * rows;
    const int u = in ? (int)(dot / rows) : 0;
    const int row = in ? (int)(dot % rows) : 0;
    const int e = ids[u];
    const bool live = in && e >= 0 && e < E;
    const float *a = W + (size_t)(live ? e : 0) * matrix_floats + (size_t)row * cols;
    const float *b = x + (size_t)(u / act_div) * ldx;
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
    // (s0 + s1) + (s2 + s3)
    const float pair = s + __shfl_xor(s, 1, 4);
    const float other = __shfl_xor(pair, 2, 4);
    if (live && j == 0)
        y[(size_t)u * ldy + row] = pair + other;
}

// mid = GELUTable(gate) * up, in place of the gate: gu [U][ld], gate then up.
__global__ __launch_bounds__(256) void moe_gelu_mul_f32_kernel(float *__restrict__ gu, int ld, int F, int U,
                                                               const float *__restrict__ table) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (size_t)U * F)
        return;
    const int u = (int)(gid / F), i = (int)(gid % F);
    float *row = gu + (size_t)u * ld;
    const float gate = row[i];
    float gl;
    if (gate <= -10.0f)
        gl = 0.0f;
    else if (gate >= 10.0f)
        gl = gate;
    else
        gl = table[float_to_half_bits(gate)];
    row[i] = gl * row[F + i];
}

// Stable counting sort of the U = M*k units by expert, in one workgroup, and
// the work list of the grouped product.  Units with an id outside [0, E) are
// left out of every group (the sum gives their positions NaN).
//   sorted[0..U): units, expert by expert, each expert's in unit order
//   work[item] = {expert, first, count, 0}, items of up to `tile` units,
//   expert by expert; the items past the last are {0, 0, 0, 0}.
// Counts per expert first (their exclusive scan is each expert's first
// place), then the units kSortThreads at a time: a unit's place is its
// expert's first place, plus that expert's units in earlier chunks (a
// running count), in earlier wavefronts of this chunk (per-wavefront counts
// summed in wavefront order), and in lower lanes of its own wavefront (its
// rank, from a ballot match).  The experts' totals are counted with LDS
// atomics, which are order-free, and the wavefront counts written by one lane
// each, so the places do not depend on scheduling.
constexpr int kSortThreads = 1024;
constexpr int kSortWaves = kSortThreads / 64;
constexpr int kSortHeld = 4;  // ids a thread keeps in registers (U <= 4096 read once)

// Exclusive prefix sums of a and b over the workgroup's threads in thread
// order (kSortThreads threads); tmp: 2 * kSortWaves ints of LDS.
__device__ __forceinline__ void scan2_exclusive(int a, int b, int &ea, int &eb, int *tmp) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int ia = a, ib = b;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int ua = __shfl_up(ia, d, 64), ub = __shfl_up(ib, d, 64);
        if (lane >= d) {
            ia += ua;
            ib += ub;
        }
    }
    if (lane == 63) {
        tmp[wave] = ia;
        tmp[kSortWaves + wave] = ib;
    }
    __syncthreads();
    int wa = 0, wb = 0;
    for (int w = 0; w < wave; w++) {
        wa += tmp[w];
        wb += tmp[kSortWaves + w];
    }
    ea = wa + ia - a;
    eb = wb + ib - b;
    __syncthreads();
}

// This lane's rank among the lower lanes of its wavefront that hold the same
// expert e, and in count how many lanes hold it (for valid lanes; every lane
// of the wavefront calls it): a ballot on each of e's nb low bits keeps the
// lanes that agree with it on that bit.
__device__ __forceinline__ int wave_match_rank(int e, bool valid, int nb, int &count) {
    uint64_t peers = __ballot(valid);
    for (int b = 0; b < nb; b++) {
        const bool bit = (e >> b) & 1;
        const uint64_t set = __ballot(bit);
        peers &= bit ? set : ~set;
    }
    count = __popcll(peers);
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(peers >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)peers, 0u));
}

__global__ __launch_bounds__(kSortThreads) void moe_sort_kernel(const int32_t *__restrict__ ids, int U, int E,
                                                                int tile, int max_items,
                                                                int32_t *__restrict__ sorted,
                                                                int32_t *__restrict__ work) {
    // LDS: first[E], run[E], cnt[kSortWaves][E]
    extern __shared__ __align__(16) int32_t sh[];
    __shared__ int32_t tmp[2 * kSortWaves];
    int32_t *first = sh, *run = first + E, *cnt = run + E;
    const int tid = threadIdx.x, wave = tid >> 6;
    const int nb = E > 1 ? 32 - __clz(E - 1) : 0;
    for (int e = tid; e < E; e += kSortThreads)
        run[e] = 0;
    for (int i = tid; i < 4 * max_items; i += kSortThreads)
        work[i] = 0;
    __syncthreads();
    // This thread's first kSortHeld ids stay in registers for the placing
    // below (read once).
    int held[kSortHeld];
#pragma unroll
    for (int h = 0; h < kSortHeld; h++)
        held[h] = tid + h * kSortThreads < U ? ids[tid + h * kSortThreads] : -1;
#pragma unroll
    for (int h = 0; h < kSortHeld; h++)
        if (held[h] >= 0 && held[h] < E)
            atomicAdd(&run[held[h]], 1);
    for (int u = tid + kSortHeld * kSortThreads; u < U; u += kSortThreads) {
        const int e = ids[u];
        if (e >= 0 && e < E)
            atomicAdd(&run[e], 1);
    }
    __syncthreads();
    // Each expert's first place and first item (E <= kSortThreads).
    {
        const int c = tid < E ? run[tid] : 0;
        const int ni = (c + tile - 1) / tile;
        int fp, fi;
        scan2_exclusive(c, ni, fp, fi, tmp);
        if (tid < E) {
            first[tid] = fp;
            for (int f = 0; f < ni && fi + f < max_items; f++) {
                work[4 * (fi + f)] = tid;
                work[4 * (fi + f) + 1] = fp + f * tile;
                work[4 * (fi + f) + 2] = min(tile, c - f * tile);
            }
            run[tid] = 0;
        }
    }
    for (int base = 0, h = 0; base < U; base += kSortThreads, h++) {
        const int u = base + tid;
        int e = -1;
#pragma unroll
        for (int hh = 0; hh < kSortHeld; hh++)
            if (hh == h)
                e = held[hh];
        if (h >= kSortHeld)
            e = u < U ? ids[u] : -1;
        const bool valid = e >= 0 && e < E;
        if (!valid)
            e = -1;
        for (int i = tid; i < kSortWaves * E; i += kSortThreads)
            cnt[i] = 0;
        // this unit's rank among the lanes below it with the same expert;
        // the highest of them writes the wavefront's count of the expert
        int count;
        const int r = wave_match_rank(e, valid, nb, count);
        __syncthreads();
        if (valid && r == count - 1)
            cnt[wave * E + e] = count;
        __syncthreads();
        // per expert: the running count before each wavefront of the chunk
        for (int x = tid; x < E; x += kSortThreads) {
            int acc = run[x];
            for (int w = 0; w < kSortWaves; w++) {
                const int c = cnt[w * E + x];
                cnt[w * E + x] = acc;
                acc += c;
            }
            run[x] = acc;
        }
        __syncthreads();
        if (valid)
            sorted[first[e] + cnt[wave * E + e] + r] = u;
        __syncthreads();
    }
}

// The same stable counting sort in one pass, for at most kSortSmallC chunks
// of kSortThreads units over at most kSortThreads / 8 experts (a prompt's
// units at a time), run by workgroup 0 of moe_sort_quant_kernel.  Unit
// u = tid + kSortThreads c belongs to group g = kSortWaves c + wave (its
// wavefront's 64 units of chunk c, groups in unit order).  Its rank among
// the group's lower lanes with the same expert comes from wave_match_rank,
// and the highest such lane writes the group's count of the expert, so no
// counter is shared.  Thread t = j E + e (j < 8) then prefixes expert e's
// counts over its 2C groups from j 2C (group-major counters: consecutive
// banks across a wavefront) and records their sum; after a barrier it adds
// the lower j's sums while wavefront 0 scans the experts' totals into their
// first places and work items.  A unit's place first[e] + (earlier groups'
// count) + rank is the one the chunked kernel above gives it: units of an
// expert in unit order.
constexpr int kSortSmallC = 4;
constexpr int kSortSmallCounters = kSortSmallC * kSortWaves * (kSortThreads / 8);

__host__ __device__ inline bool sort_small_fits(int U, int E) {
    return U <= kSortSmallC * kSortThreads && E <= kSortThreads / 8;
}

// LDS ints sort_small uses for E experts.
__host__ __device__ inline int sort_small_lds_ints(int E) { return kSortSmallCounters + 9 * E; }

__device__ __forceinline__ void sort_small(const int32_t *__restrict__ ids, int U, int E, int tile, int max_items,
                                           int32_t *__restrict__ sorted, int32_t *__restrict__ work, int32_t *sh) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int C = (U + kSortThreads - 1) / kSortThreads, G = C * kSortWaves, per = G / 8;
    int32_t *cnt = sh;                        // [G][E]: group counts, then places within the expert
    int32_t *part = sh + kSortSmallCounters;  // [8][E]: each j's sum of counts
    int32_t *first = part + 8 * E;            // [E]
    int raw[kSortSmallC];
#pragma unroll
    for (int c = 0; c < kSortSmallC; c++) {
        const int u = tid + kSortThreads * c;
        raw[c] = c < C && u < U ? ids[u] : -1;
    }
    // the clearing overlaps the loads above
    for (int i = tid; i < G * E; i += kSortThreads)
        cnt[i] = 0;
    for (int i = tid; i < 4 * max_items; i += kSortThreads)
        work[i] = 0;
    const int nb = E > 1 ? 32 - __clz(E - 1) : 0;
    int ev[kSortSmallC], rank[kSortSmallC], count[kSortSmallC];
#pragma unroll
    for (int c = 0; c < kSortSmallC; c++) {
        ev[c] = raw[c] >= 0 && raw[c] < E ? raw[c] : -1;
        rank[c] = 0;
        count[c] = 0;
        if (c < C)  // uniform: every lane of the wavefront takes part in the match
            rank[c] = wave_match_rank(ev[c], ev[c] >= 0, nb, count[c]);
    }
    __syncthreads();  // the clearing before the counts
#pragma unroll
    for (int c = 0; c < kSortSmallC; c++)
        if (c < C && ev[c] >= 0 && rank[c] == count[c] - 1)
            cnt[(kSortWaves * c + wave) * E + ev[c]] = count[c];
    __syncthreads();
    const int e8 = tid % E, j8 = tid / E;  // j8 < 8: thread t = j E + e walks expert e's groups from j 2C
    int excl[2 * kSortSmallC];
    if (j8 < 8) {
        int v[2 * kSortSmallC];
#pragma unroll
        for (int i = 0; i < 2 * kSortSmallC; i++)
            v[i] = i < per ? cnt[(j8 * per + i) * E + e8] : 0;
        int run = 0;
#pragma unroll
        for (int i = 0; i < 2 * kSortSmallC; i++) {
            excl[i] = run;
            run += v[i];
        }
        part[j8 * E + e8] = run;
    }
    __syncthreads();
    if (j8 < 8) {
        int before = 0;
        for (int jj = 0; jj < j8; jj++)
            before += part[jj * E + e8];
#pragma unroll
        for (int i = 0; i < 2 * kSortSmallC; i++)
            if (i < per)
                cnt[(j8 * per + i) * E + e8] = before + excl[i];
    }
    if (wave == 0) {
        // experts 2 lane and 2 lane + 1 (E <= 128): totals, then their first
        // places and first items by an inclusive scan over the lanes
        const int ea = 2 * lane, eb = ea + 1;
        int ta = 0, tb = 0;
#pragma unroll
        for (int jj = 0; jj < 8; jj++) {
            ta += ea < E ? part[jj * E + ea] : 0;
            tb += eb < E ? part[jj * E + eb] : 0;
        }
        const int na = (ta + tile - 1) / tile, nb2 = (tb + tile - 1) / tile;
        int ic = ta + tb, in = na + nb2;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int uc = __shfl_up(ic, d, 64), un = __shfl_up(in, d, 64);
            if (lane >= d) {
                ic += uc;
                in += un;
            }
        }
        const int fa = ic - ta - tb, fia = in - na - nb2;
        auto items = [&](int e, int fp, int fi, int ce, int ni) {
            first[e] = fp;
            for (int f = 0; f < ni && fi + f < max_items; f++) {
                work[4 * (fi + f)] = e;
                work[4 * (fi + f) + 1] = fp + f * tile;
                work[4 * (fi + f) + 2] = min(tile, ce - f * tile);
            }
        };
        if (ea < E)
            items(ea, fa, fia, ta, na);
        if (eb < E)
            items(eb, fa + ta, fia + na, tb, nb2);
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < kSortSmallC; c++) {
        const int e = ev[c];
        if (c < C && e >= 0)
            sorted[first[e] + cnt[(kSortWaves * c + wave) * E + e] + rank[c]] = tid + kSortThreads * c;
    }
}

// The grouped path's first launch: workgroup 0 sorts the units (sort_small),
// the others quantise each position's input to Q8_0 for its k units, four
// values a thread (eight threads a block: q8_0_quad, Batch.quantizeBlock's
// bits), as quantize_q8_0_kernel does one value a thread.
__global__ __launch_bounds__(kSortThreads) void moe_sort_quant_kernel(
    const int32_t *__restrict__ ids, int U, int E, int tile, int max_items, int32_t *__restrict__ sorted,
    int32_t *__restrict__ work, const float *__restrict__ x, int ldx, int M, int D, int8_t *__restrict__ q,
    float *__restrict__ scales, int32_t *__restrict__ qsum) {
    extern __shared__ __align__(16) int32_t sort_sh[];
    if (blockIdx.x == 0) {
        sort_small(ids, U, E, tile, max_items, sorted, work, sort_sh);
        return;
    }
    const size_t i4 = (size_t)(blockIdx.x - 1) * kSortThreads + threadIdx.x;
    const int n4 = D / 4;
    if (i4 >= (size_t)M * n4)  // whole eight-lane groups: D % 32 == 0
        return;
    const int m = (int)(i4 / n4), c4 = (int)(i4 - (size_t)m * n4);
    const float4 xv = *(const float4 *)(x + (size_t)m * ldx + 4 * c4);
    const float v[4] = {xv.x, xv.y, xv.z, xv.w};
    float stored;
    int32_t sm;
    const uint32_t packed = q8_0_quad(v, &stored, &sm);
    *(uint32_t *)(q + (size_t)m * D + 4 * c4) = packed;
    if ((c4 & 7) == 0) {
        const size_t b = (size_t)m * (D >> 5) + (c4 >> 3);
        scales[b] = stored;
        qsum[b] = sm;
    }
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
    s.max_items = E + (int)((U + kGroupTok - 1) / kGroupTok);
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
    if (((uintptr_t)gu & 15) == 0 && ldgu % 4 == 0)
        moe_gelu_mul_quant4_kernel<<<(unsigned)((n / 4 + 255) / 256), 256, 0, ctx->stream>>>(
            gu, ldgu, ffn, M, ctx->gelu_table, q, scales, qsum);
    else
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
    if (M <= kRouteMaxPos && D <= kLogitsOneMaxD) {
        const size_t lds = sizeof(float) * 2 * (size_t)D;
        GX_CHECK(lds <= 64 * 1024, "gx: the router's %d inputs do not fit the few-position kernel", D);
        moe_route_one_kernel<<<dim3((unsigned)E, (unsigned)M), kLogitsThreads, lds, ctx->stream>>>(
            rw, D, E, router_scale, resid, ldr, eps, logits);
        if (int rc = check_launch("moe_route_one"))
            return rc;
        moe_topk_kernel<<<M, E <= 64 ? 64 : E <= 128 ? 128 : 256, 0, ctx->stream>>>(logits, E, k, ids, weights);
        return check_launch("moe_topk");
    }
    // Positions in runs of at most kRouteScaleMax (the context's scales).
    for (int m0 = 0; m0 < M; m0 += kRouteScaleMax) {
        const int m = min(kRouteScaleMax, M - m0);
        const float *rr = resid + (size_t)m0 * ldr;
        moe_norm_scale_kernel<<<(unsigned)((m + 3) / 4), 256, 0, ctx->stream>>>(rr, ldr, m, D, eps, ctx->route_scale);
        if (int rc = check_launch("moe_norm_scale"))
            return rc;
        constexpr int P = 16, G = 4, CH = 256;
        const dim3 grid((unsigned)((E + kLgEW - 1) / kLgEW), (unsigned)((m + P - 1) / P));
        moe_logits_kernel<P, G, CH><<<grid, 32 * kLgEW * G, 0, ctx->stream>>>(rw, D, E, router_scale, rr, ldr, m,
                                                                        ctx->route_scale, logits + (size_t)m0 * E);
        if (int rc = check_launch("moe_logits"))
            return rc;
    }
    moe_topk_kernel<<<M, E <= 64 ? 64 : E <= 128 ? 128 : 256, 0, ctx->stream>>>(logits, E, k, ids, weights);
    return check_launch("moe_topk");
}

namespace {

// The few-position kernels' launch shapes (gate_up: one stretch a wavefront
// or more; down: four pairs a wavefront, at most 16 wavefronts).
struct UnitShape {
    int gu_waves, dn_waves;
    size_t gu_lds, dn_lds;
};

int unit_shape(const gx_weight *gate_up, const gx_weight *down, int k, UnitShape *sh) {
    const int Sg = (gate_up->blocks + kStretch - 1) / kStretch;
    sh->gu_waves = min(Sg, 16);
    sh->gu_lds = (size_t)Sg * kTileRows * sizeof(float);
    const int B = down->blocks, F = down->cols, Sd = (B + kStretch - 1) / kStretch, pairs = k * Sd;
    sh->dn_waves = min((pairs + 3) / 4, 16);
    const int nt = 64 * sh->dn_waves;
    sh->dn_lds = down_part_bytes(pairs) + (size_t)k * F + (size_t)k * B * 8;
    GX_CHECK(sh->gu_lds <= 64 * 1024, "gx: a %d-input expert row is wider than the gate_up kernel's LDS",
             gate_up->cols);
    GX_CHECK(sh->dn_lds <= 64 * 1024 && k * F / 16 <= kDownActRegs * nt && k * B <= kDownActRegs * nt,
             "gx: %d units of %d-input down rows do not fit the down kernel", k, F);
    GX_CHECK(down->rows % kDownRows == 0, "gx: %d down rows are not a multiple of %d", down->rows, kDownRows);
    return GX_OK;
}

}  // namespace

namespace {

// The sort and the input's Q8_0 in one launch, when the units fit the
// one-pass sort and the input is whole float4s; false: nothing launched.
bool launch_sort_quant(gx_ctx *ctx, const int32_t *ids, int U, int E, const MoeSpace &s, int32_t *sorted,
                       int32_t *work, const float *x, int ldx, int M, int D, int8_t *xq, float *xs, int32_t *xqs) {
    if (!sort_small_fits(U, E) || ((uintptr_t)x & 15) != 0 || ldx % 4 != 0 || D % 32 != 0)
        return false;
    const size_t lds = (size_t)sort_small_lds_ints(E) * sizeof(int32_t);
    const size_t n4 = (size_t)M * D / 4;
    const unsigned grid = 1 + (unsigned)((n4 + kSortThreads - 1) / kSortThreads);
    moe_sort_quant_kernel<<<grid, kSortThreads, lds, ctx->stream>>>(ids, U, E, kGroupTok, s.max_items, sorted, work,
                                                                   x, ldx, M, D, xq, xs, xqs);
    return true;
}

int launch_sort(gx_ctx *ctx, const int32_t *ids, int U, int E, const MoeSpace &s, int32_t *sorted, int32_t *work) {
    const size_t lds = (size_t)(2 + kSortWaves) * E * sizeof(int32_t);
    GX_CHECK(E <= kSortThreads && lds <= 64 * 1024, "gx: %d experts do not fit the sort's LDS", E);
    moe_sort_kernel<<<1, kSortThreads, lds, ctx->stream>>>(ids, U, E, kGroupTok, s.max_items, sorted, work);
    return check_launch("moe_sort");
}

}  // namespace

int launch_moe_experts(gx_ctx *ctx, const gx_weight *gate_up, const gx_weight *down, const float *down_scale,
                       const float *x, int ldx, int M, int k, const int32_t *ids, const float *weights, float *out,
                       int ldo, uint8_t *ws, const float *gelu_table) {
    const int D = gate_up->cols, F = down->cols, E = gate_up->count;
    const MoeSpace s = moe_space(M, k, D, F, E);
    const int U = s.units;
    if (gate_up->quant == GX_F32) {
        // F32 stacks (both): DotF32 products of the unquantised input and mid
        float *gu = (float *)(ws + s.gu);
        float *part = (float *)(ws + s.part);
        const size_t g_lanes = (size_t)U * 2 * F * 4, d_lanes = (size_t)U * D * 4, nm = (size_t)U * F;
        moe_f32_units_kernel<<<(unsigned)((g_lanes + 255) / 256), 256, 0, ctx->stream>>>(
            (const float *)gate_up->dev, gate_up->matrix_bytes / 4, 2 * F, D, x, ldx, k, U, ids, E, gu, 2 * F);
        if (int rc = check_launch("moe_f32_gate_up"))
            return rc;
        moe_gelu_mul_f32_kernel<<<(unsigned)((nm + 255) / 256), 256, 0, ctx->stream>>>(gu, 2 * F, F, U, gelu_table);
        if (int rc = check_launch("moe_gelu_mul_f32"))
            return rc;
        moe_f32_units_kernel<<<(unsigned)((d_lanes + 255) / 256), 256, 0, ctx->stream>>>(
            (const float *)down->dev, down->matrix_bytes / 4, D, F, gu, 2 * F, 1, U, ids, E, part, D);
        if (int rc = check_launch("moe_f32_down"))
            return rc;
        const size_t no = (size_t)M * D;
        moe_reduce_kernel<<<(unsigned)((no + 255) / 256), 256, 0, ctx->stream>>>(part, D, M, k, E, ids, weights,
                                                                                 down_scale, out, ldo);
        return check_launch("moe_reduce");
    }
    int8_t *mq = (int8_t *)(ws + s.mq);
    float *ms = (float *)(ws + s.ms);
    int32_t *mqs = (int32_t *)(ws + s.mqs);

    if (M <= kUnitMaxPos) {
        // Few positions: two kernels, each unit a matrix-vector product.
        UnitShape sh;
        if (int rc = unit_shape(gate_up, down, k, &sh))
            return rc;
        moe_gate_up_kernel<false><<<dim3((unsigned)(F / kQ4Block), (unsigned)U), 64 * sh.gu_waves, sh.gu_lds,
                                    ctx->stream>>>(gate_up->dev, gate_up->plane0_bytes, gate_up->matrix_bytes,
                                                   gate_up->blocks, gate_up->dchunks, F, E, x, ldx, k, ids, gelu_table,
                                                   mq, ms, mqs, nullptr);
        if (int rc = check_launch("moe_gate_up"))
            return rc;
        moe_down_reduce_kernel<false><<<dim3((unsigned)(D / kDownRows), (unsigned)M), 64 * sh.dn_waves, sh.dn_lds,
                                        ctx->stream>>>(down->dev, down->plane0_bytes, down->matrix_bytes,
                                                       down->blocks, down->dchunks, E, mq, ms, mqs, k, ids, weights,
                                                       down_scale, out, ldo, D, nullptr);
        return check_launch("moe_down_reduce");
    }

    int8_t *xq = (int8_t *)(ws + s.xq);
    float *xs = (float *)(ws + s.xs);
    int32_t *xqs = (int32_t *)(ws + s.xqs);
    float *gu = (float *)(ws + s.gu);
    float *part = (float *)(ws + s.part);
    int32_t *sorted = (int32_t *)(ws + s.sorted);
    int32_t *work = (int32_t *)(ws + s.work);
    // Each position's input, quantised once for its k units (moe.go:119-125),
    // and the units sorted by expert.  A unit whose expert id is out of range
    // is in no group: its rows are never written, and the sum makes its
    // position's output NaN.
    if (launch_sort_quant(ctx, ids, U, E, s, sorted, work, x, ldx, M, D, xq, xs, xqs)) {
        if (int rc = check_launch("moe_sort_quant"))
            return rc;
    } else {
        if (int rc = launch_quantize_q8_0(ctx, x, ldx, M, D, xq, xs, xqs, nullptr, nullptr))
            return rc;
        if (int rc = launch_sort(ctx, ids, U, E, s, sorted, work))
            return rc;
    }
    if (int rc = launch_q4_0_gemm_grouped(ctx, gate_up, work, s.max_items, sorted, k, xq, xs, gu, 2 * F, nullptr))
        return rc;
    const size_t nm4 = (size_t)U * F / 4;  // gu is the workspace's (aligned), F a multiple of 32
    moe_gelu_mul_quant4_kernel<<<(unsigned)((nm4 + 255) / 256), 256, 0, ctx->stream>>>(gu, 2 * F, F, U, gelu_table,
                                                                                       mq, ms, mqs);
    if (int rc = check_launch("moe_gelu_mul_quant"))
        return rc;
    if (int rc = launch_q4_0_gemm_grouped(ctx, down, work, s.max_items, sorted, 1, mq, ms, part, D, nullptr))
        return rc;
    if (((uintptr_t)out & 15) == 0 && ldo % 4 == 0) {
        const size_t no4 = (size_t)M * D / 4;
        moe_reduce4_kernel<<<(unsigned)((no4 + 255) / 256), 256, 0, ctx->stream>>>(part, D, M, k, E, ids, weights,
                                                                                   down_scale, out, ldo);
    } else {
        const size_t no = (size_t)M * D;
        moe_reduce_kernel<<<(unsigned)((no + 255) / 256), 256, 0, ctx->stream>>>(part, D, M, k, E, ids, weights,
                                                                                 down_scale, out, ldo);
    }
    return check_launch("moe_reduce");
}

int launch_moe_block_dots(gx_ctx *ctx, const gx_weight *gate_up, const gx_weight *down, const float *x, int ldx,
                          int M, int k, const int32_t *ids, const int8_t *mid_q, const float *mid_scales,
                          const int32_t *mid_qsum, uint8_t *ws, int32_t *dots_gate_up, int32_t *dots_down) {
    const int D = gate_up->cols, F = down->cols, E = gate_up->count;
    if (M <= kUnitMaxPos) {
        UnitShape sh;
        if (int rc = unit_shape(gate_up, down, k, &sh))
            return rc;
        if (dots_gate_up) {
            moe_gate_up_kernel<true><<<dim3((unsigned)(F / kQ4Block), (unsigned)(M * k)), 64 * sh.gu_waves,
                                       sh.gu_lds, ctx->stream>>>(gate_up->dev, gate_up->plane0_bytes,
                                                                 gate_up->matrix_bytes, gate_up->blocks,
                                                                 gate_up->dchunks, F, E, x, ldx, k, ids,
                                                                 ctx->gelu_table, nullptr, nullptr, nullptr,
                                                                 dots_gate_up);
            if (int rc = check_launch("moe_gate_up dots"))
                return rc;
        }
        if (dots_down) {
            moe_down_reduce_kernel<true><<<dim3((unsigned)(D / kDownRows), (unsigned)M), 64 * sh.dn_waves,
                                           sh.dn_lds, ctx->stream>>>(down->dev, down->plane0_bytes,
                                                                     down->matrix_bytes, down->blocks, down->dchunks,
                                                                     E, mid_q, mid_scales, mid_qsum, k, ids, nullptr,
                                                                     nullptr, nullptr, 0, D, dots_down);
            if (int rc = check_launch("moe_down_reduce dots"))
                return rc;
        }
        return GX_OK;
    }
    // More positions: the grouped products over the same sort as the product's.
    const MoeSpace s = moe_space(M, k, D, F, E);
    int8_t *xq = (int8_t *)(ws + s.xq);
    float *xs = (float *)(ws + s.xs);
    int32_t *xqs = (int32_t *)(ws + s.xqs);
    int32_t *sorted = (int32_t *)(ws + s.sorted);
    int32_t *work = (int32_t *)(ws + s.work);
    if (int rc = launch_sort(ctx, ids, s.units, E, s, sorted, work))
        return rc;
    if (dots_gate_up) {
        if (int rc = launch_quantize_q8_0(ctx, x, ldx, M, D, xq, xs, xqs, nullptr, nullptr))
            return rc;
        if (int rc = launch_q4_0_gemm_grouped(ctx, gate_up, work, s.max_items, sorted, k, xq, xs, nullptr, 0,
                                              dots_gate_up))
            return rc;
    }
    if (dots_down) {
        if (int rc = launch_q4_0_gemm_grouped(ctx, down, work, s.max_items, sorted, 1, mid_q, mid_scales, nullptr, 0,
                                              dots_down))
            return rc;
    }
    return GX_OK;
}

}  // namespace gx
