// gx_device.hpp - device helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gx {

// fp16 -> fp32, exact (v_cvt_f32_f16; fp16 denormals are kept on gfx950).
// The widening golem's halfToFloat does by hand (nn/dot_q4_0.go:21-43).
__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    return __half2float(__ushort_as_half((unsigned short)(h & 0xFFFFu)));
}

// fp32 -> fp16 bits, round to nearest even (v_cvt_f16_f32), golem's
// floatToHalf (nn/half.go:8-38) on finite inputs.
__device__ __forceinline__ uint32_t float_to_half_bits(float f) {
    return (uint32_t)__half_as_ushort(__float2half_rn(f));
}

// A workgroup barrier that orders LDS only: it waits for this wavefront's
// LDS operations (lgkmcnt), not for its global loads or stores in flight
// (__syncthreads' fence waits for those too once a global store precedes
// it).  Global memory written before it is not made visible by it.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// An LDS pointer, for the direct global-to-LDS loads.
typedef __attribute__((address_space(3))) void *lds_ptr;

// Wait until at most N vector-memory operations of this wavefront are in
// flight (expcnt and lgkmcnt unconstrained).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// The j-th of the eight fp16 values packed in a 16-byte chunk.
__device__ __forceinline__ float chunk_half(const uint4 &c, int j) {
    const uint32_t word = (j >> 1) == 0 ? c.x : (j >> 1) == 1 ? c.y : (j >> 1) == 2 ? c.z : c.w;
    return half_bits_to_float((j & 1) ? (word >> 16) : word);
}

// A 16-byte load of weights that are streamed once per product: the
// non-temporal hint keeps them from displacing the activations and outputs
// in the caches (global_load ... nt).
typedef unsigned v4u_stream __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_stream(const uint8_t *p) {
    const v4u_stream v = __builtin_nontemporal_load((const v4u_stream *)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// golem's nearestInt (nn/batch.go:221-224): round half to even by adding
// 1.5*2^23 and reading the low mantissa bits.
__device__ __forceinline__ int32_t nearest_int(float f) {
    const float s = f + 12582912.0f;
    return (int32_t)(__float_as_uint(s) & 0x007fffffu) - 0x00400000;
}

// (float)exp((double)d) for d <= 0 (a softmax's s - max, as SoftmaxInPlace
// takes it, nn/ops.go:59-73), as straight-line float64 arithmetic so that
// several exponentials interleave: n = rint(d 64 / ln2), r = d - n ln2 / 64
// (ln2 / 64 split hi + lo, the first product exact: hi has 42 significant
// bits and |n| < 2^14), e^r - 1 by Horner's rule on the Taylor series to r^5
// (|r| <= ln2 / 128), then 2^(j/64) (1 + (e^r - 1)) with j = n mod 64 from a
// table of the 64 float64 values 2^(j/64), correctly rounded, as one fma,
// scaled by 2^(n div 64) and rounded to float.  Below -110 (under float's
// least subnormal) and at -inf the result is +0; a NaN stays NaN.  Over every
// float in [-110, 0] it equals (float)exp((double)d) of a correctly rounded
// float64 exp, bit for bit (checked exhaustively on the host against the C
// library; a Taylor series to r^4 is not enough: 9 floats differ); the same
// steps in C are the oracle's orc_exp_neg.  Twelve float64 operations and a
// table read, where the series to r^13 without a table took twenty-one.
__constant__ double kExp2Sixtyfourths[64] = {
    0x1p+0, 0x1.02c9a3e778061p+0, 0x1.059b0d3158574p+0, 0x1.0874518759bc8p+0,
    0x1.0b5586cf9890fp+0, 0x1.0e3ec32d3d1a2p+0, 0x1.11301d0125b51p+0, 0x1.1429aaea92dep+0,
    0x1.172b83c7d517bp+0, 0x1.1a35beb6fcb75p+0, 0x1.1d4873168b9aap+0, 0x1.2063b88628cd6p+0,
    0x1.2387a6e756238p+0, 0x1.26b4565e27cddp+0, 0x1.29e9df51fdee1p+0, 0x1.2d285a6e4030bp+0,
    0x1.306fe0a31b715p+0, 0x1.33c08b26416ffp+0, 0x1.371a7373aa9cbp+0, 0x1.3a7db34e59ff7p+0,
    0x1.3dea64c123422p+0, 0x1.4160a21f72e2ap+0, 0x1.44e086061892dp+0, 0x1.486a2b5c13cdp+0,
    0x1.4bfdad5362a27p+0, 0x1.4f9b2769d2ca7p+0, 0x1.5342b569d4f82p+0, 0x1.56f4736b527dap+0,
    0x1.5ab07dd485429p+0, 0x1.5e76f15ad2148p+0, 0x1.6247eb03a5585p+0, 0x1.6623882552225p+0,
    0x1.6a09e667f3bcdp+0, 0x1.6dfb23c651a2fp+0, 0x1.71f75e8ec5f74p+0, 0x1.75feb564267c9p+0,
    0x1.7a11473eb0187p+0, 0x1.7e2f336cf4e62p+0, 0x1.82589994cce13p+0, 0x1.868d99b4492edp+0,
    0x1.8ace5422aa0dbp+0, 0x1.8f1ae99157736p+0, 0x1.93737b0cdc5e5p+0, 0x1.97d829fde4e5p+0,
    0x1.9c49182a3f09p+0, 0x1.a0c667b5de565p+0, 0x1.a5503b23e255dp+0, 0x1.a9e6b5579fdbfp+0,
    0x1.ae89f995ad3adp+0, 0x1.b33a2b84f15fbp+0, 0x1.b7f76f2fb5e47p+0, 0x1.bcc1e904bc1d2p+0,
    0x1.c199bdd85529cp+0, 0x1.c67f12e57d14bp+0, 0x1.cb720dcef9069p+0, 0x1.d072d4a07897cp+0,
    0x1.d5818dcfba487p+0, 0x1.da9e603db3285p+0, 0x1.dfc97337b9b5fp+0, 0x1.e502ee78b3ff6p+0,
    0x1.ea4afa2a490dap+0, 0x1.efa1bee615a27p+0, 0x1.f50765b6e454p+0, 0x1.fa7c1819e90d8p+0
};

__device__ __forceinline__ float exp_neg(float df) {
    const double d = (double)df;
    const double n = __builtin_rint(d * 0x1.71547652b82fep+6);
    double r = __builtin_fma(-n, 0x1.62e42fefa38p-7, d);
    r = __builtin_fma(-n, 0x1.ef358p-51, r);
    double p = 1.0 / 120.0;
    p = __builtin_fma(p, r, 1.0 / 24.0);
    p = __builtin_fma(p, r, 1.0 / 6.0);
    p = __builtin_fma(p, r, 0.5);
    p = __builtin_fma(p, r, 1.0);
    p = p * r;
    const int ni = (int)n;
    const double t = kExp2Sixtyfourths[ni & 63];
    const float out = (float)__builtin_ldexp(__builtin_fma(t, p, t), ni >> 6);
    return d < -110.0 ? 0.0f : out;
}

// exp_neg of N values: N independent float64 chains side by side, each
// value's bits exp_neg's.
template <int N>
__device__ __forceinline__ void exp_neg_n(const float *df, float *out) {
#pragma unroll
    for (int i = 0; i < N; i++)
        out[i] = exp_neg(df[i]);
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

// A lane's neighbour's value through DPP, for wavefront reductions without an
// LDS round trip: CTRL 0xB1 = quad_perm [1,0,3,2] (lane l ^ 1), 0x4E =
// quad_perm [2,3,0,1] (l ^ 2), 0x141 = row_half_mirror (7 - l within 8
// lanes), 0x140 = row_mirror (15 - l within 16 lanes).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// The pairwise sum of a wavefront's 64 values, every lane getting the same
// bits: lane l adds lane l ^ 1's value, then l ^ 2's, l ^ 4's, l ^ 8's, l ^
// 16's and l ^ 32's (each step a commutative add of two equal-structured
// partial sums), i.e. ((v0 + v1) + (v2 + v3)) + ... as a balanced tree in lane
// order.  Once a quad (eight, sixteen lanes) holds equal values, the mirror
// permutations pick a lane of the partner group, which holds the same value
// as lane l ^ 4 (l ^ 8); rows are combined through readlane.
__device__ __forceinline__ float wave_pairwise_sum(float v) {
    v = v + dpp_f32<0xB1>(v);
    v = v + dpp_f32<0x4E>(v);
    v = v + dpp_f32<0x141>(v);
    v = v + dpp_f32<0x140>(v);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (r0 + r1) + (r2 + r3);
}

// The maximum of a wavefront's 64 values (fmaxf: NaNs ignored), in every lane.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f32<0xB1>(v));
    v = fmaxf(v, dpp_f32<0x4E>(v));
    v = fmaxf(v, dpp_f32<0x141>(v));
    v = fmaxf(v, dpp_f32<0x140>(v));
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

template <int CTRL>
__device__ __forceinline__ int32_t dpp_i32(int32_t v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

// The maximum and the integer sum over each aligned group of 8 lanes
// (lane l with l ^ 1, l ^ 2, then the other quad of the eight), every lane
// of the group getting the result.  Order-free: max and integer addition
// are exact in any order.
__device__ __forceinline__ float group8_max(float v) {
    v = fmaxf(v, dpp_f32<0xB1>(v));
    v = fmaxf(v, dpp_f32<0x4E>(v));
    return fmaxf(v, dpp_f32<0x141>(v));
}
__device__ __forceinline__ int32_t group8_sum(int32_t v) {
    v += dpp_i32<0xB1>(v);
    v += dpp_i32<0x4E>(v);
    return v + dpp_i32<0x141>(v);
}

// The same over each aligned group of 32 lanes (a wavefront's halves): rows
// of 16 through DPP, the two rows of a half through readlane.
__device__ __forceinline__ float group32_max(float v) {
    v = group8_max(v);
    v = fmaxf(v, dpp_f32<0x140>(v));
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (__lane_id() < 32) ? fmaxf(r0, r1) : fmaxf(r2, r3);
}
__device__ __forceinline__ int32_t group32_sum(int32_t v) {
    v = group8_sum(v);
    v += dpp_i32<0x140>(v);
    const int32_t r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
    const int32_t r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
    return (__lane_id() < 32) ? r0 + r1 : r2 + r3;
}

// Q8_0 (Batch.quantizeBlock, nn/batch.go:109-143) of a 32-value block held
// four values a lane by eight consecutive lanes (lanes 8k .. 8k+7 of a
// wavefront, values in order): the same arithmetic as q8_0_lane.  Returns the
// lane's four int8 packed in order; the block's fp16-rounded scale and sum of
// q come back in *stored and *sum (valid in all eight lanes).
__device__ __forceinline__ uint32_t q8_0_quad(const float v[4], float *stored, int32_t *sum) {
    float peak = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    peak = group8_max(peak);
    if (peak == 0.0f) {
        *stored = 0.0f;
        *sum = 0;
        return 0u;
    }
    const float scale = __fdiv_rn(peak, 127.0f);
    const float inverse = __fdiv_rn(127.0f, peak);
    *stored = half_bits_to_float(float_to_half_bits(scale));
    uint32_t packed = 0;
    int32_t s = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float prod = v[k] * inverse;
        int32_t n = nearest_int(prod);
        n = n > 127 ? 127 : (n < -128 ? -128 : n);
        s += n;
        packed |= ((uint32_t)n & 0xFFu) << (8 * k);
    }
    *sum = group8_sum(s);
    return packed;
}

// Four signed byte products added to c (v_dot4_i32_i8).
__device__ __forceinline__ int32_t dot4(uint32_t a, uint32_t b, int32_t c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// The signed integer dot of one Q4_0 block against 32 int8 activations:
// sum_j (n_j - 8) * q_j.  The nibble order is golem's (nn/dot_q4_0.go:5-8):
// the low nibble of byte j is weight j, the high nibble weight j+16.  The
// unsigned nibbles meet the activations in v_dot4 and the recentring is the
// single term -8 * sum(q).
__device__ __forceinline__ int32_t q4_0_block_isum(const uint4 &w, const int4 &a0, const int4 &a1, int32_t qsum) {
    int32_t s = -8 * qsum;
    s = dot4(w.x & 0x0F0F0F0Fu, (uint32_t)a0.x, s);
    s = dot4(w.y & 0x0F0F0F0Fu, (uint32_t)a0.y, s);
    s = dot4(w.z & 0x0F0F0F0Fu, (uint32_t)a0.z, s);
    s = dot4(w.w & 0x0F0F0F0Fu, (uint32_t)a0.w, s);
    s = dot4((w.x >> 4) & 0x0F0F0F0Fu, (uint32_t)a1.x, s);
    s = dot4((w.y >> 4) & 0x0F0F0F0Fu, (uint32_t)a1.y, s);
    s = dot4((w.z >> 4) & 0x0F0F0F0Fu, (uint32_t)a1.z, s);
    s = dot4((w.w >> 4) & 0x0F0F0F0Fu, (uint32_t)a1.w, s);
    return s;
}

// The integer of one Q6_K superblock against a Q8_K activation, golem's
// sum - 32*shift (nn/dot_q6_k.go:31-51), restated group by group:
// sum_g sc[g] * (sum_{k in g} q6_k * a_k - 32 * bsum[g]).  The 6-bit values
// are assembled four bytes at a time from the ql/qh chunks.
//   ql: 32 dwords (128 bytes), qh: 16 dwords (64 bytes), sc: 16 int8 (per
//   lane); a: 64 dwords (256 int8), bsum: 8 dwords (16 int16), both read
//   where they lie, so a wavefront-uniform activation becomes scalar loads.
__device__ __forceinline__ int32_t q6_k_block_isum(const uint32_t *ql, const uint32_t *qh, const uint4 &sc,
                                                   const uint32_t *__restrict__ A, const uint32_t *__restrict__ bs) {
    const uint32_t scw[4] = {sc.x, sc.y, sc.z, sc.w};
    int32_t isum = 0;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        int32_t g[8];
#pragma unroll
        for (int i = 0; i < 8; i++)
            g[i] = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t L = ql[16 * h + k], L2 = ql[16 * h + 8 + k], H = qh[8 * h + k];
            const uint32_t qa = (L & 0x0F0F0F0Fu) | ((H << 4) & 0x30303030u);
            const uint32_t qb = (L2 & 0x0F0F0F0Fu) | ((H << 2) & 0x30303030u);
            const uint32_t qc = ((L >> 4) & 0x0F0F0F0Fu) | (H & 0x30303030u);
            const uint32_t qd = ((L2 >> 4) & 0x0F0F0F0Fu) | ((H >> 2) & 0x30303030u);
            const int grp = k >> 2;
            g[0 + grp] = dot4(qa, A[32 * h + k], g[0 + grp]);
            g[2 + grp] = dot4(qb, A[32 * h + 8 + k], g[2 + grp]);
            g[4 + grp] = dot4(qc, A[32 * h + 16 + k], g[4 + grp]);
            g[6 + grp] = dot4(qd, A[32 * h + 24 + k], g[6 + grp]);
        }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int gi = 8 * h + i;
            const int32_t s = (int32_t)(int8_t)(scw[gi >> 2] >> (8 * (gi & 3)));
            const int32_t b = (int32_t)(int16_t)(bs[gi >> 1] >> (16 * (gi & 1)));  // bsum pairs as words
            isum += s * (g[i] - 32 * b);
        }
    }
    return isum;
}

// ---- RMSNormPlain's float64 sum (nn/ops.go:195-214) over 256 threads ------
//
// The squares are float32 products summed in float64 in a fixed tree: 512
// partial sums, partial t holding elements t, t+512, t+1024, ... in order,
// then halved pairwise (t + w for w = 256 .. 1).  golem sums left to right;
// the two float64 sums differ by a few units in the 53rd bit, below the
// float32 rounding of the mean except in rare ties.
// Partial sums t and t + 256 of the norm's tree (this thread's pair), over
// x[0, D) with x in LDS or global memory.  Elements are read 8 per partial
// at a time; past D they read as element D - 1 and add 0.0, which leaves a
// non-negative double unchanged.
__device__ __forceinline__ void norm_partials(const float *x, int D, double &p0, double &p1) {
    const int tid = threadIdx.x;
    p0 = 0.0;
    p1 = 0.0;
    for (int base = 0; base < D; base += 8 * 512) {
        float v0[8], v1[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            v0[u] = x[min(base + tid + 512 * u, D - 1)];
            v1[u] = x[min(base + tid + 256 + 512 * u, D - 1)];
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const float a = base + tid + 512 * u < D ? v0[u] : 0.0f;
            const float b = base + tid + 256 + 512 * u < D ? v1[u] : 0.0f;
            const float sa = a * a, sb = b * b;
            p0 += (double)sa;
            p1 += (double)sb;
        }
    }
}

// The rest of the tree (w = 256 .. 1) across a 256-thread workgroup; the
// result is valid in thread 0.  `red` is 256 doubles of LDS.
__device__ __forceinline__ double norm_tree(double p0, double p1, double *red) {
    const int tid = threadIdx.x;
    double s = p0 + p1;  // w = 256
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
    }
    return s;
}

// x (+ add) of K values staged for a fused pre-norm: each value into xs
// (LDS) and, when x_out is given, x_out; partial t of the tree (t < 512)
// into red[t] (LDS).  Eight elements of a partial are loaded at a time, so a
// thread waits for one round trip per 4096 values.
__device__ __forceinline__ void norm_stage(const float *x, const float *add, int K, float *xs, float *x_out,
                                           double *red) {
    for (int pt = threadIdx.x; pt < 512; pt += blockDim.x) {
        double acc = 0.0;
        for (int base = 0; base < K; base += 8 * 512) {
            float v[8], a[8];
#pragma unroll
            for (int u = 0; u < 8; u++)
                v[u] = x[min(base + pt + 512 * u, K - 1)];
            if (add) {
#pragma unroll
                for (int u = 0; u < 8; u++)
                    a[u] = add[min(base + pt + 512 * u, K - 1)];
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int i = base + pt + 512 * u;
                if (i < K) {
                    const float s = add ? v[u] + a[u] : v[u];
                    xs[i] = s;
                    if (x_out)
                        x_out[i] = s;
                    const float sq = s * s;
                    acc += (double)sq;
                }
            }
        }
        red[pt] = acc;
    }
}

// The tree over red[512] (LDS) by one wavefront: lane l pairs partials
// l + 64 m itself (t + 256, then t + 128, then t + 64), then the shuffle
// tree across lanes.  The sum is valid in lane 0.
__device__ __forceinline__ double norm_tree_wave(const double *red) {
    const int l = threadIdx.x & 63;
    const double a = red[l] + red[l + 256], b = red[l + 64] + red[l + 320];
    const double c = red[l + 128] + red[l + 384], d = red[l + 192] + red[l + 448];
    double s = (a + c) + (b + d);
    for (int w = 32; w > 0; w >>= 1) {
        const double o = __shfl_down(s, w, 64);
        if (l < w)
            s = s + o;
    }
    return s;
}

__device__ __forceinline__ float norm_scale(double sum, int D, float eps) {
    const float mean = (float)(sum / (double)D);
    return (float)(1.0 / sqrt((double)(mean + eps)));
}

// The float64 sum of squares of K floats in LDS, by a workgroup of at least
// 512 threads, in the order every whole-row RMSNormPlain here uses: 512
// strided partials, then a pairwise tree down to one.  red: 512 doubles of
// LDS; the sum comes back in every thread through *bcast (LDS).
__device__ __forceinline__ double block_sum_squares(const float *xs, int K, double *red, double *bcast) {
    const int tid = threadIdx.x;
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
        s = red[tid] + red[tid + 256];
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
            *bcast = s;
    }
    __syncthreads();
    return *bcast;
}


// The minimum of an integer over a wavefront, in every lane.
__device__ __forceinline__ int32_t wave_min_i32(int32_t v) {
    v = min(v, dpp_i32<0xB1>(v));
    v = min(v, dpp_i32<0x4E>(v));
    v = min(v, dpp_i32<0x141>(v));
    v = min(v, dpp_i32<0x140>(v));
    const int32_t r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
    const int32_t r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
    return min(min(r0, r1), min(r2, r3));
}

// Batch.QuantizeK of one 256-element superblock by one wavefront
// (nn/batch.go:159-213), lane l holding elements 4l .. 4l+3: extreme = the
// signed value of the first element of largest magnitude, inverse =
// -128 / extreme, q = min(127, nearestInt(x * inverse)), kscale =
// 1 / inverse; a superblock of zeros gives zeros.  Returns the lane's four q
// packed in a dword; *gsum receives the sum of its 16-element group in every
// lane of the group's quad (lanes 4g .. 4g+3), *kscale the superblock's
// scale (every lane).  NaNs never win the magnitude comparison, as in
// golem's loop.
__device__ __forceinline__ uint32_t q8_k_wave(const float v[4], int lane, int32_t *gsum, float *kscale) {
    float peak = 0.0f;
    int at = 256;  // the lane's first element of its largest magnitude
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float a = fabsf(v[i]);
        if (a > peak) {
            peak = a;
            at = 4 * lane + i;
        }
    }
    const float top = wave_max(peak);
    if (top == 0.0f) {
        *gsum = 0;
        *kscale = 0.0f;
        return 0u;
    }
    // the lowest index of the largest magnitude: every lane's own first
    // occurrence, the lowest of those that reach the wavefront's maximum
    const int first = wave_min_i32(peak == top ? at : 256);
    const float mine = (first & 3) == 0 ? v[0] : (first & 3) == 1 ? v[1] : (first & 3) == 2 ? v[2] : v[3];
    const float extreme = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), first >> 2));
    const float inverse = __fdiv_rn(-128.0f, extreme);
    uint32_t packed = 0;
    int32_t sum = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float prod = v[i] * inverse;
        int32_t n = nearest_int(prod);
        n = n > 127 ? 127 : n;
        packed |= ((uint32_t)(uint8_t)(int8_t)n) << (8 * i);
        sum += n;
    }
    sum += dpp_i32<0xB1>(sum);
    sum += dpp_i32<0x4E>(sum);
    *gsum = sum;
    *kscale = __fdiv_rn(1.0f, inverse);
    return packed;
}

// Q8_0 of one element per lane of a 32-lane group (Batch.quantizeBlock,
// nn/batch.go:109-143): returns q; the group's fp16-rounded scale and sum of
// q come back in *stored and *sum (valid in every lane).
__device__ __forceinline__ int32_t q8_0_lane(float v, float *stored, int32_t *sum) {
    const float peak = group32_max(fabsf(v));
    if (peak == 0.0f) {
        *stored = 0.0f;
        *sum = 0;
        return 0;
    }
    const float scale = __fdiv_rn(peak, 127.0f);
    const float inverse = __fdiv_rn(127.0f, peak);
    *stored = half_bits_to_float(float_to_half_bits(scale));
    const float prod = v * inverse;
    int32_t n = nearest_int(prod);
    n = n > 127 ? 127 : (n < -128 ? -128 : n);
    *sum = group32_sum(n);
    return n;
}

}  // namespace gx
