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
// argmax_part_kernel + argmax_final_kernel are the greedy pick over logits
// (ties to the lower id).
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
// partial t = elements t, t+512, ... in order, halved pairwise): threads
// 0..511 stage x (+ add) and their partials (norm_stage) while threads
// 512..1023 stage the gains, wavefront 0 takes the tree (norm_tree_wave) --
// two barriers -- and the Q8_0 goes four values a lane, a block per eight
// lanes (q8_0_quad).  (Against a five-barrier tree and one value a lane:
// 6.3 -> 4.9 us at 8 positions of 2560.)
__global__ __launch_bounds__(kQNormThreads) void qwen_norm_quant_kernel(float *__restrict__ x, int ldx,
                                                                        const float *__restrict__ add, int lda,
                                                                        const float *__restrict__ gain, int K,
                                                                        float eps, float *__restrict__ out, int ldo,
                                                                        int8_t *__restrict__ q,
                                                                        float *__restrict__ scales,
                                                                        int32_t *__restrict__ qsum) {
    extern __shared__ __align__(16) float xs[];  // K floats, then the K gains
    float *gl = xs + K;
    __shared__ double red[512];
    __shared__ float scale_sh;
    const int tid = threadIdx.x, t = blockIdx.x;
    float *xr = x + (size_t)t * ldx;
    const float *ar = add ? add + (size_t)t * lda : nullptr;
    if (tid < 512) {
        norm_stage(xr, ar, K, xs, ar ? xr : nullptr, red);  // x + add written back as the residual
    } else {
        for (int i = tid - 512; i < K; i += kQNormThreads - 512)
            gl[i] = gain[i];
    }
    __syncthreads();
    if (tid < 64) {
        const double total = norm_tree_wave(red);
        if (tid == 0)
            scale_sh = norm_scale(total, K, eps);
    }
    __syncthreads();
    const float sc = scale_sh;
    const int B = K >> 5;
    for (int i4 = tid; i4 < K / 4; i4 += kQNormThreads) {  // K % 32 == 0: whole eight-lane groups in or out
        const float4 xv = ((const float4 *)xs)[i4];
        const float4 gv = ((const float4 *)gl)[i4];
        float nv[4];
        nv[0] = (xv.x * sc) * gv.x;
        nv[1] = (xv.y * sc) * gv.y;
        nv[2] = (xv.z * sc) * gv.z;
        nv[3] = (xv.w * sc) * gv.w;
        if (out) {
            float *o = out + (size_t)t * ldo + 4 * i4;
#pragma unroll
            for (int k = 0; k < 4; k++)
                o[k] = nv[k];
        }
        if (q) {
            float stored;
            int32_t sm;
            const uint32_t packed = q8_0_quad(nv, &stored, &sm);
            ((uint32_t *)(q + (size_t)t * K))[i4] = packed;
            if ((i4 & 7) == 0) {
                scales[(size_t)t * B + (i4 >> 3)] = stored;
                qsum[(size_t)t * B + (i4 >> 3)] = sm;
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
// layer's caches of `context` positions: the key in 16-byte pieces,
// [kvh][hd/8][pos][8] (a wavefront reading piece i of 64 consecutive
// positions reads 1 KiB in one run), the value at [kvh][hd][pos].
__device__ __forceinline__ void kcache_put(uint16_t *kt, int context, int e, uint16_t v) {
    kt[(size_t)(e >> 3) * context * 8 + (e & 7)] = v;
}

__global__ __launch_bounds__(64) void qwen_qk_rope_kernel(const float *__restrict__ qkv, int ldqkv, int heads,
                                                          int kv_heads, int hd, const int32_t *__restrict__ positions,
                                                          const float *__restrict__ q_norm,
                                                          const float *__restrict__ k_norm,
                                                          const float *__restrict__ rope_cos,
                                                          const float *__restrict__ rope_sin, float eps,
                                                          uint16_t *__restrict__ qh, uint16_t *__restrict__ kcache,
                                                          uint16_t *__restrict__ vcache, int context,
                                                          const int32_t *__restrict__ slots, int nslots) {
    __shared__ float h[kHeadMax];
    __shared__ float sc_sh;
    const int lane = threadIdx.x, t = blockIdx.x, u = blockIdx.y;
    const int pos = positions[t];
    // A position past the cache, or a slot that names no conversation, has
    // no place: nothing is stored, and the query is NaN, which the attention
    // and everything after carry to the output.
    const bool placed = pos >= 0 && pos < context && (!slots || (slots[t] >= 0 && slots[t] < nslots));
    if (!placed) {
        if (u < heads)
            for (int i = lane; i < hd; i += 64)
                qh[(size_t)t * heads * hd + u * hd + i] = 0x7E00;
        return;
    }
    if (slots) {  // the token's own conversation: its slot of the caches
        const size_t at = (size_t)slots[t] * kv_heads * hd * context;
        kcache += at;
        vcache += at;
    }
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
            // [kvh][hd/8][context][8]: piece e/8 of a key at position pos
            uint16_t *kt = kcache + (size_t)(u - heads) * hd * context + (size_t)pos * 8;
            kcache_put(kt, context, i, (uint16_t)float_to_half_bits(a));
            kcache_put(kt, context, i + half, (uint16_t)float_to_half_bits(b));
        }
    }
    if (!is_q) {
        const float *vsrc = qkv + (size_t)t * ldqkv + (heads + kv_heads) * hd + (u - heads) * hd;
        uint16_t *vt = vcache + (size_t)(u - heads) * hd * context + pos;
        for (int i = lane; i < hd; i += 64)
            vt[(size_t)i * context] = (uint16_t)float_to_half_bits(vsrc[i]);
    }
}

// The same for a batch: grid (ceil(M / kQkTok), heads + kv_heads), 256
// threads, kQkTok tokens of one head a workgroup.  The tokens' heads and the
// norm's gains are staged in LDS (a key-value head's value rows are loaded
// at the same time, into registers, for later); the 64 float64 sums of
// squares run side by side, one lane a token, each left to right as
// head_norm_scale takes it, while every thread's rotation-table loads --
// which wait only on the positions -- are in flight; then the rotation,
// each output element from the same operations as the one-token kernel, and
// the fp16 stores laid out so that consecutive lanes take consecutive tokens
// where the destination runs over positions: a key's 16-byte pieces (a
// wavefront writes a piece of 64 positions, 1 KiB) and a value's elements
// (128 bytes of one element row); a query's 16-byte pieces run along its
// head.  The same bits as qwen_qk_rope_kernel.
constexpr int kQkTok = 64;

template <int HD>
__global__ __launch_bounds__(256) void qwen_qk_rope_tile_kernel(
    const float *__restrict__ qkv, int ldqkv, int M, int heads, int kv_heads, const int32_t *__restrict__ positions,
    const float *__restrict__ q_norm, const float *__restrict__ k_norm, const float *__restrict__ rope_cos,
    const float *__restrict__ rope_sin, float eps, uint16_t *__restrict__ qh, uint16_t *__restrict__ kcache,
    uint16_t *__restrict__ vcache, int context, const int32_t *__restrict__ slots, int nslots) {
    constexpr int half = HD / 2, P = HD / 8;    // rotation pairs; 16-byte pieces a head
    constexpr int kItems = kQkTok * P / 256;    // (token, piece) items a thread
    constexpr int kRows4 = kQkTok * HD / 4 / 256;  // float4s of a head tile a thread
    static_assert(kItems * 256 == kQkTok * P && kRows4 * 256 * 4 == kQkTok * HD, "whole items");
    __shared__ float hs[kQkTok][HD + 1];      // +1: a lane a token reads down a column without conflicts
    __shared__ float gs[HD];
    __shared__ float scs[kQkTok];
    __shared__ int pos_s[kQkTok];
    __shared__ int place_s[kQkTok];           // placed: 1; no place: 0; past the batch: -1
    __shared__ int slot_s[kQkTok];
    const int tid = threadIdx.x, t0 = blockIdx.x * kQkTok, u = blockIdx.y;
    const bool is_q = u < heads;
    const int col = is_q ? u * HD : heads * HD + (u - heads) * HD;
    const float *gain = is_q ? q_norm : k_norm;
    if (tid < kQkTok) {
        const int t = t0 + tid;
        int pl = -1, pos = 0, sl = 0;
        if (t < M) {
            pos = positions[t];
            sl = slots ? slots[t] : 0;
            pl = pos >= 0 && pos < context && (!slots || (sl >= 0 && sl < nslots)) ? 1 : 0;
        }
        pos_s[tid] = pos;
        place_s[tid] = pl;
        slot_s[tid] = sl;
    }
    if (tid < HD)
        gs[tid] = gain[tid];
    // the heads, a float4 a thread at a time (rows past the batch repeat the
    // last); a key-value head's value rows into registers alongside
    const int vcol = (heads + kv_heads) * HD + (u - heads) * HD;
    float4 vv[kRows4];
#pragma unroll
    for (int r = 0; r < kRows4; r++) {
        const int idx = tid + 256 * r;
        const int tk = idx / (HD / 4), c4 = idx - tk * (HD / 4);
        const float *row = qkv + (size_t)min(t0 + tk, M - 1) * ldqkv;
        const float4 v = *(const float4 *)(row + col + 4 * c4);
        if (!is_q)
            vv[r] = *(const float4 *)(row + vcol + 4 * c4);
        hs[tk][4 * c4] = v.x;
        hs[tk][4 * c4 + 1] = v.y;
        hs[tk][4 * c4 + 2] = v.z;
        hs[tk][4 * c4 + 3] = v.w;
    }
    __syncthreads();
    // (token, piece) items: queries with the piece fastest (a query's pieces
    // are contiguous), keys with the token fastest (a piece's positions are).
    // Their rotation tables go out now, while the norms' sums run.
    float4 c0[kItems], c1[kItems], s0[kItems], s1[kItems];
#pragma unroll
    for (int it = 0; it < kItems; it++) {
        const int idx = tid + 256 * it;
        const int tk = is_q ? idx / P : idx % kQkTok, pc = is_q ? idx % P : idx / kQkTok;
        if (place_s[tk] > 0) {
            const int pos = pos_s[tk];
            const int j0 = 8 * pc < half ? 8 * pc : 8 * pc - half;
            c0[it] = *(const float4 *)(rope_cos + (size_t)pos * half + j0);
            c1[it] = *(const float4 *)(rope_cos + (size_t)pos * half + j0 + 4);
            s0[it] = *(const float4 *)(rope_sin + (size_t)pos * half + j0);
            s1[it] = *(const float4 *)(rope_sin + (size_t)pos * half + j0 + 4);
        }
    }
    if (tid < kQkTok) {
        // head_norm_scale's sum, left to right, sixteen values read ahead
        const float *hr = hs[tid];
        double acc = 0.0;
        for (int i0 = 0; i0 < HD; i0 += 16) {
            float v[16];
#pragma unroll
            for (int i = 0; i < 16; i++)
                v[i] = hr[i0 + i];
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const float sq = v[i] * v[i];
                acc += (double)sq;
            }
        }
        const float mean = (float)(acc / (double)HD);
        scs[tid] = (float)(1.0 / sqrt((double)(mean + eps)));
    }
    __syncthreads();
    // Element e of a rotated head: pair j = e % half, a = re c - im s (e <
    // half), b = re s + im c (e >= half), re = x_j sc g_j, im = x_{j+half}
    // sc g_{j+half}: RoPETable.Apply, nn/rope.go:62-73.  A piece's eight
    // elements share one side, so their pairs are eight consecutive j.
#pragma unroll
    for (int it = 0; it < kItems; it++) {
        const int idx = tid + 256 * it;
        const int tk = is_q ? idx / P : idx % kQkTok, pc = is_q ? idx % P : idx / kQkTok;
        const int pl = place_s[tk];
        if (pl < 0)
            continue;
        const int pos = pos_s[tk];
        uint32_t w[4] = {0x7E007E00u, 0x7E007E00u, 0x7E007E00u, 0x7E007E00u};  // no place: a NaN query
        if (pl) {
            const bool lo = 8 * pc < half;
            const int j0 = lo ? 8 * pc : 8 * pc - half;
            const float cs[8] = {c0[it].x, c0[it].y, c0[it].z, c0[it].w, c1[it].x, c1[it].y, c1[it].z, c1[it].w};
            const float sn[8] = {s0[it].x, s0[it].y, s0[it].z, s0[it].w, s1[it].x, s1[it].y, s1[it].z, s1[it].w};
            const float sc = scs[tk];
            uint32_t hb[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int j = j0 + k;
                const float re = (hs[tk][j] * sc) * gs[j], im = (hs[tk][j + half] * sc) * gs[j + half];
                const float v = lo ? re * cs[k] - im * sn[k] : re * sn[k] + im * cs[k];
                hb[k] = float_to_half_bits(v);
            }
#pragma unroll
            for (int k = 0; k < 4; k++)
                w[k] = hb[2 * k] | (hb[2 * k + 1] << 16);
        }
        const v4u_stream o = {w[0], w[1], w[2], w[3]};
        if (is_q) {
            *(v4u_stream *)(qh + (size_t)(t0 + tk) * heads * HD + u * HD + 8 * pc) = o;
        } else if (pl) {
            uint16_t *kt = kcache + (size_t)slot_s[tk] * kv_heads * HD * context + (size_t)(u - heads) * HD * context;
            *(v4u_stream *)(kt + ((size_t)pc * context + pos) * 8) = o;
        }
    }
    if (is_q)
        return;
    // the values: from the registers into the staging rows, then a lane a
    // token down each element row
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kRows4; r++) {
        const int idx = tid + 256 * r;
        const int tk = idx / (HD / 4), c4 = idx - tk * (HD / 4);
        hs[tk][4 * c4] = vv[r].x;
        hs[tk][4 * c4 + 1] = vv[r].y;
        hs[tk][4 * c4 + 2] = vv[r].z;
        hs[tk][4 * c4 + 3] = vv[r].w;
    }
    __syncthreads();
    for (int idx = tid; idx < kQkTok * HD; idx += 256) {
        const int tk = idx % kQkTok, d = idx / kQkTok;
        if (place_s[tk] > 0) {
            uint16_t *vt = vcache + (size_t)slot_s[tk] * kv_heads * HD * context + (size_t)(u - heads) * HD * context;
            vt[(size_t)d * context + pos_s[tk]] = (uint16_t)float_to_half_bits(hs[tk][d]);
        }
    }
}

// The attention proper runs as three passes over a workspace: scores
// sc [M][heads][S] floats and probabilities prob [M][heads][S] fp16, where S
// is the deepest visible prefix rounded up to 64.
//   scores   a lane per cached position: scale * DotF32(query, key) in
//            DotF32's four-chain order
//   softmax  a wavefront per (position, head): SoftmaxInPlace's maximum,
//            exp in float64, the sum taken position by position, the
//            division, the probability rounded through fp16
//   values   Axpy in position order, a lane per (position, head, element),
//            the value cache ([kv_heads][hd][context], positions contiguous)
//            staged through LDS; Q8_0 of the heads
// The query, keys, values and probabilities are all fp16 values, so each
// product of two of them is exact in float32: a fused multiply-add then
// rounds exactly as golem's multiply-then-add does (its one rounding is the
// addition's), and the kernels use v_fma_mix, which takes the fp16 operands
// as they are stored.

__device__ __forceinline__ float half_lo(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xFFFFu));
}
__device__ __forceinline__ float half_hi(uint32_t w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16)); }

// lo/hi(a) * lo/hi(b) + c for fp16 pairs a and b, as one v_fma_mix: written
// out so that a key row reused for several heads stays in its packed form
// (the compiler would otherwise widen it to 128 floats once and run out of
// registers).
__device__ __forceinline__ float fma_mix_lo(uint32_t a, uint32_t b, float c) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,1,0]" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}
__device__ __forceinline__ float fma_mix_hi(uint32_t a, uint32_t b, float c) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,1,0] op_sel_hi:[1,1,0]" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

constexpr int kTile = 64;  // positions per scores wavefront
typedef float v4f_lds __attribute__((ext_vector_type(4)));

// grid (S/64 position tiles, heads/GH head groups, ceil(M/TT) token tiles),
// one wavefront.  Lane = cached position p; its key row is held in registers
// for the GH heads (of one key-value head) of the TT tokens.  Their TT x GH
// queries are staged in LDS first, every load in flight at once, and read
// back as broadcasts (all lanes one address).  (Read as scalar loads, one
// query after another, each dot product waited for its own query; with the
// tile maxima reduced here as well, config 3's 512-token prompt spent 65 us
// a layer in this pass, now 43.)
template <int HD>
__global__ __launch_bounds__(64) void attn_scores_kernel(const uint16_t *__restrict__ qh, int M, int heads, int G,
                                                         int GH, int TT, const int32_t *__restrict__ positions, int limit,
                                                         const uint16_t *__restrict__ kcache, int context,
                                                         float scale, int S, float *__restrict__ sc,
                                                         const int32_t *__restrict__ slots, int nslots, int kv_heads) {
    extern __shared__ __align__(16) uint32_t qst[];  // [TT][GH][HD / 2] fp16 pairs
    const int lane = threadIdx.x, tile = blockIdx.x;
    const int h0 = blockIdx.y * GH, t0 = blockIdx.z * TT;
    const int kvh = h0 / G;
    if (slots)  // with slots, a token tile is one token (TT = 1); reads stay inside the caches
        kcache += (size_t)min(max(slots[t0], 0), nslots - 1) * kv_heads * HD * context;
    const int tn = min(TT, M - t0);
    int last = -1;
    for (int tt = 0; tt < tn; tt++)
        last = max(last, min(positions[t0 + tt], limit - 1));
    if (tile * kTile > last)
        return;  // the whole wavefront: nothing visible here
    // The queries: 16-byte pieces c = (tt * GH + j) * HD / 8 + i, token rows
    // past the batch clamped to its last (never used).
    {
        constexpr int kPer = HD / 8;  // pieces a query
        const int pieces = TT * GH * kPer;
        for (int c0 = 0; c0 < pieces; c0 += 8 * 64) {
            v4u_stream v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int c = min(c0 + u * 64 + lane, pieces - 1);
                const int qi = c / kPer, i = c - qi * kPer;
                const int tt = qi / GH, j = qi - tt * GH;
                v[u] = ((const v4u_stream *)(qh + ((size_t)min(t0 + tt, M - 1) * heads + h0 + j) * HD))[i];
            }
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (c0 + u * 64 + lane < pieces)
                    ((v4u_stream *)qst)[c0 + u * 64 + lane] = v[u];
        }
    }
    const int p = tile * kTile + lane;
    const v4u_stream *kr = (const v4u_stream *)(kcache + (size_t)kvh * HD * context) + min(p, last);
    v4u_stream k[HD / 8];
#pragma unroll
    for (int i = 0; i < HD / 8; i++)
        k[i] = kr[(size_t)i * context];
    __syncthreads();
    for (int tt = 0; tt < tn; tt++) {
        const int t = t0 + tt;
        const int n = min(positions[t] + 1, limit);
        if (tile * kTile >= n)
            continue;
        for (int j = 0; j < GH; j++) {
            const int h = h0 + j;
            const uint32_t *q = qst + (tt * GH + j) * (HD / 2);
            float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;  // elements 4i, 4i+1, 4i+2, 4i+3
#pragma unroll
            for (int i = 0; i < HD / 8; i++) {
                const uint32_t kw[4] = {k[i].x, k[i].y, k[i].z, k[i].w};
#pragma unroll
                for (int w = 0; w < 4; w += 2) {
                    const uint32_t qa = q[4 * i + w], qb = q[4 * i + w + 1];
                    s0 = __builtin_fmaf(half_lo(qa), half_lo(kw[w]), s0);
                    s1 = __builtin_fmaf(half_hi(qa), half_hi(kw[w]), s1);
                    s2 = __builtin_fmaf(half_lo(qb), half_lo(kw[w + 1]), s2);
                    s3 = __builtin_fmaf(half_hi(qb), half_hi(kw[w + 1]), s3);
                }
            }
            const float v = scale * ((s0 + s1) + (s2 + s3));
            const size_t row = (size_t)t * heads + h;
            if (p < n)
                sc[row * S + p] = v;
        }
    }
}

constexpr int kSoftChunk = 2048;  // exponentials per pass through LDS

// Sum e[0 .. n) into `total` one value at a time, in order: two register sets
// of 16, the next set's LDS reads under this set's additions.  e is 16-byte
// aligned and readable to e[n + 15] (the reads of a set may pass n; those
// values are never added).
__device__ __forceinline__ float serial_sum(const float *e, int n, float total) {
    const v4f_lds *e4 = (const v4f_lds *)e;
    v4f_lds a[4], b[4];
#pragma unroll
    for (int u = 0; u < 4; u++)
        a[u] = e4[u];
    int j = 0;
    for (; j + 32 <= n; j += 32) {
#pragma unroll
        for (int u = 0; u < 4; u++)
            b[u] = e4[(j + 16) / 4 + u];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            total += a[u].x;
            total += a[u].y;
            total += a[u].z;
            total += a[u].w;
        }
#pragma unroll
        for (int u = 0; u < 4; u++)
            a[u] = e4[(j + 32) / 4 + u];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            total += b[u].x;
            total += b[u].y;
            total += b[u].z;
            total += b[u].w;
        }
    }
    if (j + 16 <= n) {  // a holds e[j .. j + 16)
#pragma unroll
        for (int u = 0; u < 4; u++) {
            total += a[u].x;
            total += a[u].y;
            total += a[u].z;
            total += a[u].w;
        }
        j += 16;
    }
    for (; j < n; j++)
        total += e[j];
    return total;
}

// grid (ceil(heads / kSoftRows), M), a wavefront per (position t, head h):
// SoftmaxInPlace (nn/ops.go:59-73) of the row's scores, then RoundHalf of
// each probability.  The wavefronts of a workgroup share nothing (each has
// its own `cap` + 16 floats of LDS, cap = min(kSoftChunk, S)), so a CU holds
// twice as many rows at once as with one-wavefront workgroups: the row's
// total is a serial chain on one lane, and more rows in flight cover it.
// (Config 3's 512-token prompt: 25 us a layer with one row a workgroup.)
constexpr int kSoftRows = 4;
__global__ __launch_bounds__(64 * kSoftRows) void attn_softmax_kernel(int heads, const int32_t *__restrict__ positions,
                                                                      int limit, int S, int cap,
                                                                      float *__restrict__ sc,
                                                                      uint16_t *__restrict__ prob) {
    extern __shared__ __align__(16) float esh[];  // [kSoftRows][cap + 16]: serial_sum reads to n + 15
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int h = blockIdx.x * kSoftRows + w, t = blockIdx.y;
    if (h >= heads)
        return;  // the whole wavefront; no workgroup barrier follows
    float *e = esh + w * (cap + 16);
    const size_t row = (size_t)t * heads + h;
    const int n = min(positions[t] + 1, limit);
    float *s = sc + row * S;
    // The maximum is exact in any order; it is taken here, once a row, from
    // the scores themselves.  (Each scores wavefront reducing its tile's
    // maximum across its lanes, one dot product after another, was a chain
    // of six cross-lane round trips per product: most of the scores pass.)
    float m = -INFINITY;
    for (int j = lane; j < n; j += 64)
        m = fmaxf(m, s[j]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
        m = fmaxf(m, __shfl_xor(m, off, 64));
    float total = 0.0f;  // lane 0's
    for (int c0 = 0; c0 < n; c0 += cap) {
        const int cn = min(cap, n - c0);
        for (int j = lane; j < cn; j += 64) {
            const float v = (float)exp((double)(s[c0 + j] - m));
            e[j] = v;
            if (n > cap)
                s[c0 + j] = v;  // kept for the division
        }
        // one wavefront: its LDS accesses complete in order; the wait keeps
        // the compiler from moving lane 0's reads above the stores
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (lane == 0)
            total = serial_sum(e, cn, total);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    total = __shfl(total, 0, 64);
    uint16_t *pr = prob + row * S;
    if (n <= cap) {
        for (int j = lane; j < n; j += 64)
            pr[j] = (uint16_t)float_to_half_bits(__fdiv_rn(e[j], total));
    } else {
        for (int j = lane; j < n; j += 64)
            pr[j] = (uint16_t)float_to_half_bits(__fdiv_rn(s[j], total));
    }
}

constexpr int kValSlice = 32;    // elements of a head per workgroup: one Q8_0 block
constexpr int kValChunk = 768;   // positions per pass through LDS
constexpr int kValStride = kValChunk + 8;  // LDS row stride in halves (16 bytes of padding)
constexpr int kValRegs = 24;     // value pieces a thread holds in flight

// grid (kv_heads * hd/32 slices, ceil(M/TT) token tiles), NT = TT*G*32
// threads.  Thread (tt, g, d): chain of element d of the slice for query
// head kvh*G + g of token t0 + tt, over positions 0 .. positions[t] in order:
// acc = fma(p, v, acc) (Axpy, nn/kernel.go:221-233).  The slice's value rows
// (32 rows of positions) and the TT*G probability rows pass through LDS a
// chunk of kValChunk positions at a time; a 32-lane group's chains are one
// Q8_0 block of the head outputs.
template <int NT>
__global__ __launch_bounds__(NT) void attn_values_kernel(int M, int heads, int G, int hd,
                                                         const int32_t *__restrict__ positions, int limit,
                                                         const uint16_t *__restrict__ vcache, int context,
                                                         int kv_heads, int S, const uint16_t *__restrict__ prob,
                                                         int8_t *__restrict__ q, float *__restrict__ scales,
                                                         int32_t *__restrict__ qsum, const int32_t *__restrict__ slots,
                                                         int nslots) {
    constexpr int rows = NT / kValSlice;  // (tt, g) pairs
    __shared__ __align__(16) uint16_t vs[kValSlice * kValStride];
    __shared__ __align__(16) uint16_t ps[rows * kValStride];
    const int tid = threadIdx.x;
    const int slices = hd / kValSlice, TT = rows / G;
    const int kvh = blockIdx.x / slices, d0 = (blockIdx.x - kvh * slices) * kValSlice;
    const int t0 = blockIdx.y * TT, tn = min(TT, M - t0);
    const int dd = tid % kValSlice, hg = tid / kValSlice;
    const int tt = hg / G, g = hg - tt * G;
    const bool live = tt < tn;
    const int n = live ? min(positions[t0 + tt] + 1, limit) : 0;
    int nmax = 0;
    for (int i = 0; i < tn; i++)
        nmax = max(nmax, min(positions[t0 + i] + 1, limit));
    if (slots)  // with slots, a token tile is one token (TT = 1); reads stay inside the caches
        vcache += (size_t)min(max(slots[t0], 0), nslots - 1) * kv_heads * hd * context;
    const uint16_t *vrow = vcache + ((size_t)kvh * hd + d0) * context;
    float acc = 0.0f;
    for (int c0 = 0; c0 < nmax; c0 += kValChunk) {
        const int groups = (min(kValChunk, nmax - c0) + 7) / 8;  // 8-position pieces of a row
        const int pieces = kValSlice * groups;
        __syncthreads();  // the previous chunk's chains are done with the buffers
        for (int base = 0; base < pieces; base += NT * kValRegs) {
            v4u_stream r[kValRegs];
#pragma unroll
            for (int u = 0; u < kValRegs; u++) {
                const int i = min(base + tid + u * NT, pieces - 1);
                const int rr = i / groups, c = i - rr * groups;
                r[u] = *(const v4u_stream *)(vrow + (size_t)rr * context + c0 + 8 * c);
            }
#pragma unroll
            for (int u = 0; u < kValRegs; u++) {
                const int i = base + tid + u * NT;
                if (i < pieces) {
                    const int rr = i / groups, c = i - rr * groups;
                    *(v4u_stream *)(vs + rr * kValStride + 8 * c) = r[u];
                }
            }
        }
        for (int i = tid; i < rows * groups; i += NT) {
            const int rr = i / groups, c = i - rr * groups;
            const int ttr = rr / G, hr = kvh * G + (rr - ttr * G);
            v4u_stream v = {0u, 0u, 0u, 0u};
            if (ttr < tn)
                v = *(const v4u_stream *)(prob + ((size_t)(t0 + ttr) * heads + hr) * S + c0 + 8 * c);
            *(v4u_stream *)(ps + rr * kValStride + 8 * c) = v;
        }
        __syncthreads();
        const int ln = min(kValChunk, n - c0);  // this chain's positions in the chunk
        const uint16_t *vr = vs + dd * kValStride, *pr = ps + hg * kValStride;
        int j = 0;
#pragma unroll 4
        for (; j + 8 <= ln; j += 8) {
            const v4u_stream vv = *(const v4u_stream *)(vr + j);
            const v4u_stream pp = *(const v4u_stream *)(pr + j);
            acc = __builtin_fmaf(half_lo(pp.x), half_lo(vv.x), acc);
            acc = __builtin_fmaf(half_hi(pp.x), half_hi(vv.x), acc);
            acc = __builtin_fmaf(half_lo(pp.y), half_lo(vv.y), acc);
            acc = __builtin_fmaf(half_hi(pp.y), half_hi(vv.y), acc);
            acc = __builtin_fmaf(half_lo(pp.z), half_lo(vv.z), acc);
            acc = __builtin_fmaf(half_hi(pp.z), half_hi(vv.z), acc);
            acc = __builtin_fmaf(half_lo(pp.w), half_lo(vv.w), acc);
            acc = __builtin_fmaf(half_hi(pp.w), half_hi(vv.w), acc);
        }
        for (; j < ln; j++)
            acc = __builtin_fmaf((float)__builtin_bit_cast(_Float16, pr[j]),
                                 (float)__builtin_bit_cast(_Float16, vr[j]), acc);
    }
    float stored;
    int32_t sm;
    const int32_t nq = q8_0_lane(acc, &stored, &sm);
    if (live) {
        const int width = heads * hd, B = width >> 5;
        const int t = t0 + tt, col = (kvh * G + g) * hd + d0 + dd;
        q[(size_t)t * width + col] = (int8_t)nq;
        if (dd == 0) {
            scales[(size_t)t * B + (col >> 5)] = stored;
            qsum[(size_t)t * B + (col >> 5)] = sm;
        }
    }
}

// The same value chains for a prompt's tokens.  A wavefront owns 64 value
// elements (lane d) of one head g for TC tokens.  Per chunk of kSpChunk
// positions the workgroup stages the slice's value rows (TT = TGW*TC tokens
// of the group's G heads share them) and its TT*G probability rows in LDS;
// a wavefront's probabilities are uniform, read one step ahead as broadcasts
// (all lanes one address).  (Read as wavefront-wide vector loads of one
// address straight from the workspace, one step ahead did not cover their
// latency: 64 us a layer at config 3's 512-token prompt.)
// Each lane runs TC chains, one a token, each in position order with its own
// accumulator: attn_values_kernel's fma order, so the same bits.  (That
// kernel staged the probabilities in LDS too and read them per lane: at 512
// tokens its LDS traffic and its two tokens a workgroup set the time.)
constexpr int kSpDims = 64;     // value elements a wavefront
constexpr int kSpChunk = 512;   // positions a pass through LDS
constexpr int kSpStride = kSpChunk + 8;

template <int TC, int G, int TGW>
__global__ __launch_bounds__(64 * TGW * G) void attn_values_sp_kernel(int M, int heads, int hd,
                                                                      const int32_t *__restrict__ positions,
                                                                      int limit, const uint16_t *__restrict__ vcache,
                                                                      int context, int kv_heads, int S,
                                                                      const uint16_t *__restrict__ prob,
                                                                      int8_t *__restrict__ q,
                                                                      float *__restrict__ scales,
                                                                      int32_t *__restrict__ qsum) {
    constexpr int NT = 64 * TGW * G, TT = TGW * TC;
    extern __shared__ __align__(16) uint16_t vs[];  // [kSpDims][kSpStride], then ps [TT * G][kSpStride]
    uint16_t *ps = vs + kSpDims * kSpStride;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tg = wave / G, g = wave - tg * G;
    const int slices = hd / kSpDims;
    const int kvh = blockIdx.x / slices, d0 = (blockIdx.x - kvh * slices) * kSpDims;
    const int t0 = blockIdx.y * TT, tn = min(TT, M - t0);
    int n[TC];
#pragma unroll
    for (int c = 0; c < TC; c++) {
        const int tt = tg * TC + c;
        n[c] = tt < tn ? min(positions[t0 + tt] + 1, limit) : 0;
    }
    int nmax = 0;
    for (int i = 0; i < tn; i++)
        nmax = max(nmax, min(positions[t0 + i] + 1, limit));
    const uint16_t *vrow = vcache + ((size_t)kvh * hd + d0) * context;
    float acc[TC];
#pragma unroll
    for (int c = 0; c < TC; c++)
        acc[c] = 0.0f;
    for (int c0 = 0; c0 < nmax; c0 += kSpChunk) {
        const int groups = (min(kSpChunk, nmax - c0) + 7) / 8;  // 8-position pieces of a row
        const int pieces = kSpDims * groups;
        __syncthreads();  // the previous chunk's chains are done with the rows
        for (int base = 0; base < pieces; base += NT * 4) {
            v4u_stream r[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int i = min(base + tid + u * NT, pieces - 1);
                const int rr = i / groups, c = i - rr * groups;
                r[u] = *(const v4u_stream *)(vrow + (size_t)rr * context + c0 + 8 * c);
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int i = base + tid + u * NT;
                if (i < pieces) {
                    const int rr = i / groups, c = i - rr * groups;
                    *(v4u_stream *)(vs + rr * kSpStride + 8 * c) = r[u];
                }
            }
        }
        {
            // probability row pr = token tt * G + head gg (tokens past the
            // batch read its last token's row; positions past a token's
            // prefix are staged and never used)
            const int ppieces = TT * G * groups;
            for (int base = 0; base < ppieces; base += NT * 4) {
                v4u_stream r[4];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int i = min(base + tid + u * NT, ppieces - 1);
                    const int pr = i / groups, c = i - pr * groups;
                    const int tt = pr / G, gg = pr - tt * G;
                    r[u] = *(const v4u_stream *)(prob + ((size_t)(t0 + min(tt, tn - 1)) * heads + kvh * G + gg) * S +
                                                 c0 + 8 * c);
                }
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int i = base + tid + u * NT;
                    if (i < ppieces) {
                        const int pr = i / groups, c = i - pr * groups;
                        *(v4u_stream *)(ps + pr * kSpStride + 8 * c) = r[u];
                    }
                }
            }
        }
        __syncthreads();
        const uint16_t *vr = vs + lane * kSpStride;
        int ln[TC], lmin = kSpChunk;
        const uint16_t *prl[TC];  // this wavefront's probability rows in LDS
#pragma unroll
        for (int c = 0; c < TC; c++) {
            ln[c] = min(kSpChunk, n[c] - c0);
            lmin = min(lmin, ln[c]);
            prl[c] = ps + ((tg * TC + c) * G + g) * kSpStride;
        }
        // 16 positions a step, every chain whole; the probabilities come
        // from LDS as broadcasts, one step ahead.
        int j = 0;
        v4u_stream pa[TC][2], pb[TC][2];
#define GX_SP_LOAD(DST, JJ)                                                                                          \
    do {                                                                                                             \
        _Pragma("unroll") for (int c = 0; c < TC; c++) {                                                            \
            _Pragma("unroll") for (int u = 0; u < 2; u++)                                                           \
                DST[c][u] = *(const v4u_stream *)(prl[c] + (JJ) + 8 * u);                                          \
        }                                                                                                            \
    } while (0)
#define GX_SP_STEP(SRC, JJ)                                                                                          \
    do {                                                                                                             \
        _Pragma("unroll") for (int u = 0; u < 2; u++) {                                                             \
            const v4u_stream vv = *(const v4u_stream *)(vr + (JJ) + 8 * u);                                          \
            _Pragma("unroll") for (int c = 0; c < TC; c++) {                                                        \
                const v4u_stream pp = SRC[c][u];                                                                     \
                float a = acc[c];                                                                                    \
                a = fma_mix_lo(pp.x, vv.x, a);                                                                       \
                a = fma_mix_hi(pp.x, vv.x, a);                                                                       \
                a = fma_mix_lo(pp.y, vv.y, a);                                                                       \
                a = fma_mix_hi(pp.y, vv.y, a);                                                                       \
                a = fma_mix_lo(pp.z, vv.z, a);                                                                       \
                a = fma_mix_hi(pp.z, vv.z, a);                                                                       \
                a = fma_mix_lo(pp.w, vv.w, a);                                                                       \
                a = fma_mix_hi(pp.w, vv.w, a);                                                                       \
                acc[c] = a;                                                                                          \
            }                                                                                                        \
        }                                                                                                            \
    } while (0)
        if (16 <= lmin)
            GX_SP_LOAD(pa, 0);
        while (j + 16 <= lmin) {
            if (j + 32 <= lmin)
                GX_SP_LOAD(pb, j + 16);
            GX_SP_STEP(pa, j);
            j += 16;
            if (j + 16 > lmin)
                break;
            if (j + 32 <= lmin)
                GX_SP_LOAD(pa, j + 16);
            GX_SP_STEP(pb, j);
            j += 16;
        }
#undef GX_SP_STEP
#undef GX_SP_LOAD
        // the chains' tails, 24 positions a round (three 8-position pieces
        // of every chain requested together), position by position within
        int lmax = 0;
#pragma unroll
        for (int c = 0; c < TC; c++)
            lmax = max(lmax, ln[c]);
        for (; j < lmax; j += 24) {
            v4u_stream pt[TC][3];
#pragma unroll
            for (int c = 0; c < TC; c++)
#pragma unroll
                for (int u = 0; u < 3; u++)  // past the prefix: read, never used
                    pt[c][u] = *(const v4u_stream *)(prl[c] + min(j + 8 * u, kSpChunk - 8));
#pragma unroll
            for (int u = 0; u < 3; u++) {
                const int jp = j + 8 * u;
                const v4u_stream vv = *(const v4u_stream *)(vr + min(jp, kSpChunk - 8));
                const uint32_t vw[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
                for (int c = 0; c < TC; c++) {
                    const uint32_t pw[4] = {pt[c][u].x, pt[c][u].y, pt[c][u].z, pt[c][u].w};
#pragma unroll
                    for (int e = 0; e < 8; e++)
                        if (jp + e < ln[c])
                            acc[c] = (e & 1) ? fma_mix_hi(pw[e >> 1], vw[e >> 1], acc[c])
                                             : fma_mix_lo(pw[e >> 1], vw[e >> 1], acc[c]);
                }
            }
        }
    }
    const int width = heads * hd, B = width >> 5;
#pragma unroll
    for (int c = 0; c < TC; c++) {
        float stored;
        int32_t sm;
        const int32_t nq = q8_0_lane(acc[c], &stored, &sm);  // a Q8_0 block a 32-lane half
        const int tt = tg * TC + c;
        if (tt < tn) {
            const int t = t0 + tt, col = (kvh * G + g) * hd + d0 + lane;
            q[(size_t)t * width + col] = (int8_t)nq;
            if ((lane & 31) == 0) {
                scales[(size_t)t * B + (col >> 5)] = stored;
                qsum[(size_t)t * B + (col >> 5)] = sm;
            }
        }
    }
}

// Decode attention in one kernel (M <= 4 positions, or one position per
// conversation, prefixes of at most kDecodeMax positions): grid
// (heads / G * hd/32 slices, M), 512 threads.  A workgroup computes, for G
// query heads of key-value head kvh (G = 1, or the whole group of heads that
// share kvh), the scores over the whole prefix (a thread per position, its key
// rows in registers, the queries in LDS), the softmax and the probabilities,
// then the 32 value chains of its slice for each head -- the same arithmetic,
// in the same order, as the three passes above.  Its slice of the value rows
// and its key rows are loaded first, so that the loads overlap; the slices'
// workgroups repeat the scores and softmax of their heads.
constexpr int kDecodeMax = 768;
constexpr int kDecodeThreads = 512;
constexpr int kDecodeStride = kDecodeMax + 8;  // value and probability rows, in halves
constexpr int kDecodeRegs = kValSlice * (kDecodeMax / 8) / kDecodeThreads;  // value pieces per thread
constexpr int kDecodeRows = (kDecodeMax + kDecodeThreads - 1) / kDecodeThreads;  // positions per thread
constexpr int kScoreStride = kDecodeMax + 20;  // score rows 20 banks apart (conflict-free serial sums), read to n + 15

//
// FUSE (one position, M = 1): the kernel also does qwen_qk_rope_kernel's work
// for that position.  Every workgroup stages its G query heads and its key
// head from the Q|K|V product, takes each head's norm (head_norm_scale, a
// lane per head) and rotates it with the same expressions, so the fp16 query
// and key are qwen_qk_rope_kernel's bit for bit; the query goes straight to
// LDS.  The new key and value are stored to the caches (the key by the
// head's first slice, each slice its 32 value elements) for later
// positions, and this position's own score and value term use the computed
// copies, never the cache entries being written.
struct QkRope {
    const float *qkv;
    int ldqkv;
    const float *q_norm, *k_norm, *rope_cos, *rope_sin;
    float eps;
    uint16_t *kcache, *vcache;  // the caches the position is stored into
};

template <int HD, int G, bool FUSE>
__global__ __launch_bounds__(kDecodeThreads) void attn_decode_kernel(
    const uint16_t *__restrict__ qh, int heads, int kv_heads, const int32_t *__restrict__ positions, int limit,
    const uint16_t *kcache, const uint16_t *vcache, int context, float scale,
    int8_t *__restrict__ q, float *__restrict__ scales, int32_t *__restrict__ qsum,
    const int32_t *__restrict__ slots, int nslots, QkRope fz) {
    // LDS: region A holds the scores [G][kScoreStride] floats, later the value
    // slice [32][kDecodeStride] halves; then the probabilities [G][kDecodeStride]
    // halves and the queries [G][HD] halves.
    // (+128 bytes: the chains' last reads may pass the end of the rows)
    __shared__ __align__(16) uint8_t lds[kValSlice * kDecodeStride * 2 + G * kDecodeStride * 2 + G * HD * 2 + 128];
    static_assert(G * kScoreStride * 4 + 64 <= kValSlice * kDecodeStride * 2, "scores fit region A");
    __shared__ float red[kDecodeThreads / 64][G];
    __shared__ float total[G];
    float *sc = (float *)lds;
    uint16_t *vs = (uint16_t *)lds;
    uint16_t *ps = (uint16_t *)(lds + kValSlice * kDecodeStride * 2);
    uint32_t *ql = (uint32_t *)(lds + kValSlice * kDecodeStride * 2 + G * kDecodeStride * 2);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    constexpr int slices = HD / kValSlice;
    // Workgroup b: key-value head b % kv_heads (so that the workgroups of one
    // key-value head share an XCD's L2), and within it query heads
    // h0 .. h0 + G - 1 and value slice d0.
    const int group = heads / kv_heads;  // query heads per key-value head
    const int kvh = blockIdx.x % kv_heads, rb = blockIdx.x / kv_heads;
    const int hl = rb / slices, d0 = (rb - hl * slices) * kValSlice;
    const int h0 = kvh * group + hl * G;
    const bool first = hl == 0;  // the head group that stores the position (FUSE)
    const int t = blockIdx.y;
    const int pos = positions[t];
    const int n = min(max(pos, 0) + 1, limit);
    // FUSE: a position outside the cache has no place in it: it stores
    // nothing, its query is NaN, and the rotation tables are read at the
    // cache's last position instead (in bounds).  One past max_pos but inside
    // the cache is stored and attends positions 0 .. max_pos, as
    // qwen_qk_rope_kernel and this kernel without FUSE do.
    const int rpos = min(max(pos, 0), context - 1);
    const int groups = (n + 7) / 8, pieces = kValSlice * groups;
    bool store = pos >= 0 && pos < context;  // FUSE: the position has a place and is stored
    if (slots) {  // the token's own conversation; reads stay inside the caches
        const size_t at = (size_t)min(max(slots[t], 0), nslots - 1) * kv_heads * HD * context;
        kcache += at;
        vcache += at;
        if (FUSE) {
            store = store && slots[t] >= 0 && slots[t] < nslots;
            fz.kcache += at;
            fz.vcache += at;
        }
    }

    // FUSE (G = 1): wavefront 0 alone prepares the position -- its query head
    // and key head (fp32, from the Q|K|V row, four values a lane), the
    // slice's value elements, and the norm gains and rotation of the HD pairs
    // (i, i + HD/2), two a lane -- with these loads issued before its cache
    // reads, while the other wavefronts go straight to theirs.
    static_assert(!FUSE || G == 1, "the fused prologue serves one query head per workgroup");
    constexpr int kHalf = HD / 2;
    float4 hx = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float nv = 0.0f, rg0[2], rg1[2], rc[2], rs[2];
    if (FUSE && wave == 0) {
        const float *row = fz.qkv + (size_t)t * fz.ldqkv;
        const int e = min(4 * lane, 2 * HD - 4);  // query elements, then key elements
        hx = *(const float4 *)(row + (e < HD ? h0 * HD + e : heads * HD + kvh * HD + (e - HD)));
        nv = row[(heads + kv_heads) * HD + kvh * HD + d0 + (lane & (kValSlice - 1))];
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int i = min(lane + 64 * r, HD - 1);  // pair i: head i / (HD/2)
            const int w = i / kHalf, j = i - w * kHalf;
            const float *gain = w == 0 ? fz.q_norm : fz.k_norm;
            rg0[r] = gain[j];
            rg1[r] = gain[j + kHalf];
            rc[r] = fz.rope_cos[(size_t)rpos * kHalf + j];
            rs[r] = fz.rope_sin[(size_t)rpos * kHalf + j];
        }
    }

    // The G queries (adjacent heads of the row) first, then the key pieces of
    // this thread's positions, then the value slice (32 rows of positions,
    // 16 bytes = 8 positions a piece): the queries can be stored while the
    // rest is in flight.
    const uint32_t *qg = (const uint32_t *)(qh + ((size_t)t * heads + h0) * HD);
    const uint32_t qr = FUSE ? 0u : qg[min(tid, G * HD / 2 - 1)];
    v4u_stream k[kDecodeRows][HD / 8];
    const v4u_stream *kbase = (const v4u_stream *)(kcache + (size_t)kvh * HD * context);
#pragma unroll
    for (int r = 0; r < kDecodeRows; r++) {
        const int p = min(tid + r * kDecodeThreads, n - 1);
#pragma unroll
        for (int i = 0; i < HD / 8; i++)
            k[r][i] = kbase[(size_t)i * context + p];
    }
    const uint16_t *vrow = vcache + ((size_t)kvh * HD + d0) * context;
    v4u_stream vr[kDecodeRegs];
#pragma unroll
    for (int u = 0; u < kDecodeRegs; u++) {
        const int i = min(tid + u * kDecodeThreads, pieces - 1);
        const int rr = i / groups, c = i - rr * groups;
        vr[u] = *(const v4u_stream *)(vrow + (size_t)rr * context + 8 * c);
    }
    static_assert(G * HD / 2 <= kDecodeThreads, "one query dword per thread");
    // FUSE: the new key, fp16, at the end of region A (scores use its front)
    uint16_t *nk = (uint16_t *)(lds + kValSlice * kDecodeStride * 2 - HD * 2);
    if (FUSE) {
        static_assert(G * kScoreStride * 4 + 64 <= kValSlice * kDecodeStride * 2 - HD * 2, "scores clear the key");
        static_assert(2 * HD * 12 <= kValSlice * kDecodeStride * 2 - HD * 2, "staged heads fit region A");
        __shared__ float hs[2];
        if (wave == 0) {
            // The two heads and their squares (float32, widened) in region A;
            // lanes 0 and 1 then add a head's squares in order in float64:
            // head_norm_scale's sum, bit for bit, with its reads in flight.
            float *hh = (float *)lds;
            double *sq = (double *)(lds + 2 * HD * 4);
            if (4 * lane < 2 * HD) {
                *(float4 *)(hh + 4 * lane) = hx;
                const float x4[4] = {hx.x, hx.y, hx.z, hx.w};
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const float v = x4[k];
                    const float sqf = v * v;
                    sq[4 * lane + k] = (double)sqf;
                }
            }
            if (lane < 2) {
                const double *sh = sq + lane * HD;
                double acc = 0.0;
#pragma unroll 16
                for (int i = 0; i < HD; i++)
                    acc += sh[i];
                const float mean = (float)(acc / (double)HD);
                hs[lane] = (float)(1.0 / sqrt((double)(mean + fz.eps)));
            }
            // normed, then rotated in pairs (i, i + HD/2): RoPETable.Apply,
            // nn/rope.go:62-73, as qwen_qk_rope_kernel
            uint16_t *qlh = (uint16_t *)ql;
#pragma unroll
            for (int r = 0; r < 2; r++) {
                const int i = lane + 64 * r;
                if (i >= HD)
                    break;
                const int w = i / kHalf, j = i - w * kHalf;
                const float sc = hs[w];
                const float re0 = hh[w * HD + j], im0 = hh[w * HD + j + kHalf];
                const float re = (re0 * sc) * rg0[r], im = (im0 * sc) * rg1[r];
                const float c = rc[r], sn = rs[r];
                const float a = re * c - im * sn;
                const float b = re * sn + im * c;
                uint16_t ha = (uint16_t)float_to_half_bits(a), hb = (uint16_t)float_to_half_bits(b);
                if (w == 0) {
                    if (!store)  // no conversation: the query is NaN
                        ha = hb = 0x7E00;
                    qlh[j] = ha;
                    qlh[j + kHalf] = hb;
                } else {
                    nk[j] = ha;
                    nk[j + kHalf] = hb;
                    if (store && first && d0 == 0) {
                        uint16_t *kt = fz.kcache + (size_t)kvh * HD * context + (size_t)pos * 8;
                        kcache_put(kt, context, j, ha);
                        kcache_put(kt, context, j + kHalf, hb);
                    }
                }
            }
            if (store && first && lane < kValSlice)
                fz.vcache[((size_t)kvh * HD + d0 + lane) * context + pos] = (uint16_t)float_to_half_bits(nv);
        }
        __syncthreads();
        // this position's key from the copy, not the cache entry being written
        if (pos == n - 1) {
#pragma unroll
            for (int r = 0; r < kDecodeRows; r++)
                if (tid + r * kDecodeThreads == pos) {
#pragma unroll
                    for (int i = 0; i < HD / 8; i++)
                        k[r][i] = ((const v4u_stream *)nk)[i];
                }
        }
    } else {
        if (tid < G * HD / 2)
            ql[tid] = qr;
        __syncthreads();
    }

    // scores, DotF32's four chains: element e of a head goes to chain e % 4
    float mx[G];
#pragma unroll
    for (int g = 0; g < G; g++)
        mx[g] = -INFINITY;
#pragma unroll
    for (int r = 0; r < kDecodeRows; r++) {
        const int p = tid + r * kDecodeThreads;
        if (r * kDecodeThreads + wave * 64 >= n)
            break;  // the wavefront's positions are all past the prefix
#pragma unroll
        for (int g = 0; g < G; g++) {
            const v4u_stream *qv = (const v4u_stream *)(ql + g * HD / 2);
            float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll
            for (int i = 0; i < HD / 8; i++) {
                const v4u_stream qq = qv[i], kk = k[r][i];
                s0 = fma_mix_lo(qq.x, kk.x, s0);
                s1 = fma_mix_hi(qq.x, kk.x, s1);
                s2 = fma_mix_lo(qq.y, kk.y, s2);
                s3 = fma_mix_hi(qq.y, kk.y, s3);
                s0 = fma_mix_lo(qq.z, kk.z, s0);
                s1 = fma_mix_hi(qq.z, kk.z, s1);
                s2 = fma_mix_lo(qq.w, kk.w, s2);
                s3 = fma_mix_hi(qq.w, kk.w, s3);
            }
            const float v = scale * ((s0 + s1) + (s2 + s3));
            if (p < n) {
                sc[g * kScoreStride + p] = v;
                mx[g] = fmaxf(mx[g], v);
            }
        }
    }
#pragma unroll
    for (int g = 0; g < G; g++) {
#pragma unroll
        for (int off = 32; off > 0; off >>= 1)
            mx[g] = fmaxf(mx[g], __shfl_xor(mx[g], off, 64));
        if (lane == 0)
            red[wave][g] = mx[g];
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; g++) {
        float m = red[0][g];
#pragma unroll
        for (int w = 1; w < kDecodeThreads / 64; w++)
            m = fmaxf(m, red[w][g]);
        for (int p = tid; p < n; p += kDecodeThreads)
            sc[g * kScoreStride + p] = (float)exp((double)(sc[g * kScoreStride + p] - m));
    }
    __syncthreads();
    if (tid < G)
        total[tid] = serial_sum(sc + tid * kScoreStride, n, 0.0f);
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; g++)
        for (int p = tid; p < groups * 8; p += kDecodeThreads)
            ps[g * kDecodeStride + p] =
                p < n ? (uint16_t)float_to_half_bits(__fdiv_rn(sc[g * kScoreStride + p], total[g])) : (uint16_t)0;
    __syncthreads();  // the scores are dead: region A takes the value slice
#pragma unroll
    for (int u = 0; u < kDecodeRegs; u++) {
        const int i = tid + u * kDecodeThreads;
        if (i < pieces) {
            const int rr = i / groups, c = i - rr * groups;
            *(v4u_stream *)(vs + rr * kDecodeStride + 8 * c) = vr[u];
        }
    }
    if (FUSE && pos == n - 1) {
        __syncthreads();  // the staged pieces first, then this position's values over them
        if (tid < kValSlice)
            vs[tid * kDecodeStride + pos] = (uint16_t)float_to_half_bits(nv);
    }
    __syncthreads();
    if (tid < G * kValSlice) {
        const int dd = tid % kValSlice, g = tid / kValSlice;
        const uint16_t *vrr = vs + dd * kDecodeStride, *pr = ps + g * kDecodeStride;
        float acc = 0.0f;
        // 32 positions a set, the next set's LDS reads under this set's fmas
        // (a set may read past n, inside the LDS array; those are not used)
        v4u_stream av[4], ap[4], bv[4], bp[4];
#define GX_DEC_LOAD(sv, sp, at)                                                                                      \
    _Pragma("unroll") for (int u = 0; u < 4; u++) {                                                                  \
        sv[u] = *(const v4u_stream *)(vrr + (at) + 8 * u);                                                           \
        sp[u] = *(const v4u_stream *)(pr + (at) + 8 * u);                                                            \
    }
#define GX_DEC_FMA(sv, sp)                                                                                           \
    _Pragma("unroll") for (int u = 0; u < 4; u++) {                                                                  \
        acc = __builtin_fmaf(half_lo(sp[u].x), half_lo(sv[u].x), acc);                                               \
        acc = __builtin_fmaf(half_hi(sp[u].x), half_hi(sv[u].x), acc);                                               \
        acc = __builtin_fmaf(half_lo(sp[u].y), half_lo(sv[u].y), acc);                                               \
        acc = __builtin_fmaf(half_hi(sp[u].y), half_hi(sv[u].y), acc);                                               \
        acc = __builtin_fmaf(half_lo(sp[u].z), half_lo(sv[u].z), acc);                                               \
        acc = __builtin_fmaf(half_hi(sp[u].z), half_hi(sv[u].z), acc);                                               \
        acc = __builtin_fmaf(half_lo(sp[u].w), half_lo(sv[u].w), acc);                                               \
        acc = __builtin_fmaf(half_hi(sp[u].w), half_hi(sv[u].w), acc);                                               \
    }
        int j = 0;
        GX_DEC_LOAD(av, ap, 0);
        for (; j + 64 <= n; j += 64) {
            GX_DEC_LOAD(bv, bp, j + 32);
            GX_DEC_FMA(av, ap);
            GX_DEC_LOAD(av, ap, j + 64);
            GX_DEC_FMA(bv, bp);
        }
        if (j + 32 <= n) {  // av holds positions j .. j + 32
            GX_DEC_FMA(av, ap);
            j += 32;
        }
#undef GX_DEC_FMA
#undef GX_DEC_LOAD
        for (; j + 8 <= n; j += 8) {
            const v4u_stream vv = *(const v4u_stream *)(vrr + j);
            const v4u_stream pp = *(const v4u_stream *)(pr + j);
            acc = __builtin_fmaf(half_lo(pp.x), half_lo(vv.x), acc);
            acc = __builtin_fmaf(half_hi(pp.x), half_hi(vv.x), acc);
            acc = __builtin_fmaf(half_lo(pp.y), half_lo(vv.y), acc);
            acc = __builtin_fmaf(half_hi(pp.y), half_hi(vv.y), acc);
            acc = __builtin_fmaf(half_lo(pp.z), half_lo(vv.z), acc);
            acc = __builtin_fmaf(half_hi(pp.z), half_hi(vv.z), acc);
            acc = __builtin_fmaf(half_lo(pp.w), half_lo(vv.w), acc);
            acc = __builtin_fmaf(half_hi(pp.w), half_hi(vv.w), acc);
        }
        for (; j < n; j++)
            acc = __builtin_fmaf((float)__builtin_bit_cast(_Float16, pr[j]),
                                 (float)__builtin_bit_cast(_Float16, vrr[j]), acc);
        float stored;
        int32_t sm;
        const int32_t nq = q8_0_lane(acc, &stored, &sm);
        const int width = heads * HD, B = width >> 5;
        const int col = (h0 + g) * HD + d0 + dd;
        q[(size_t)t * width + col] = (int8_t)nq;
        if (dd == 0) {
            scales[(size_t)t * B + (col >> 5)] = stored;
            qsum[(size_t)t * B + (col >> 5)] = sm;
        }
    }
}


// ---- decode attention, sums in a parallel order -----------------------------
//
// The decode step's default attention (M <= 4 positions, or one position per
// conversation, prefixes of at most kDecodeMax): grid (heads * hd/VW, M), a
// workgroup per (query head, VW-element value slice, token), 1024 threads.
// The same scores, maximum, float64 exponentials, division and fp16 rounding
// of each probability as golem's SoftmaxInPlace and Axpy (qwen/attention.go:
// 96-114, nn/ops.go:59-73), with the two serial sums taken in a fixed parallel
// order that does not depend on the launch's extent (so that a step replayed
// from a graph launched for the whole cache equals the same step launched for
// its own prefix) nor on the workgroup's shape:
//   total  = ((0 + B_0) + B_1) + ...   B_b the pairwise sum of block b's 64
//            exponentials (lane = p % 64; lane l adds l ^ 1, then l ^ 2, ...,
//            l ^ 32: wave_pairwise_sum), zeros past the prefix;
//   out[d] = ((0 + R_0) + R_1) + ...   R_r the fma chain of run r's 32
//            probability * value products in position order, from +0.
// The reordered total moves a probability on an fp16 rounding boundary by one
// step now and then (head values within a few 1e-5 of RMS of golem's), the
// reordered value sums by about 1e-7.
//
// Loads: the whole extent's key rows (a lane per position: a wavefront reads
// 1 KiB of a key piece) and the value slice (its VW rows are contiguous: each
// wavefront load reads a 1 KiB run, staged through LDS) are requested before
// the token's position (itself a load) is known; positions past the prefix
// are read and left out of every sum.  With FUSE, wavefront 0 first runs the
// prologue (head norms, RoPE, the position's cache store) on loads it issues
// ahead of its share of the cache loads.  Barriers wait for LDS only, so the
// prologue's stores and the cache loads stay in flight across them.
// VW: kValSlice (a head's 32-element slice, the long form, extents up to
// kDecodeMax) or HD (the whole head, one workgroup a query head, extents up
// to kParShortMax: a quarter of the workgroups, for the lock-step
// conversations' short prefixes).  ROWS: key rows a cache thread scores.
constexpr int kParThreads = 1024;
constexpr int kParBlock = 64;      // positions a block of the softmax total
constexpr int kParRun = 32;        // positions a run of the value sums
constexpr int kParShortMax = 128;  // the extents the whole-head form holds
constexpr int kParMaxRuns = kDecodeMax / kParRun;      // 24
constexpr int kParMaxBlocks = kDecodeMax / kParBlock;  // 12

template <int VW, bool FUSE>
struct ParShape {
    static constexpr int kCap = VW == kValSlice ? kDecodeMax : kParShortMax;  // positions the form holds
    static constexpr int kStride = kCap + 8;               // halves a staged value row (rows 4 banks apart)
    static constexpr int kPieces = kCap / 8;               // 16-byte pieces a staged row
    static constexpr int kVLoads = VW * kPieces / kParThreads;  // value pieces a thread stages
    static constexpr int kSlots = kParThreads / VW;        // run slots
    static constexpr int kRunsPer = (kCap / kParRun + kSlots - 1) / kSlots;  // runs a thread sums
    static constexpr int kW0 = FUSE ? 1 : 0;               // wavefronts out of the cache work
    static constexpr int kCT = kParThreads - 64 * kW0;     // cache threads
    static constexpr int kMaxRows = (kCap + kCT - 1) / kCT;  // key rows a cache thread may score
};

template <int HD, bool FUSE, int ROWS, int VW>
__global__ __launch_bounds__(kParThreads) void attn_par_kernel(
    const uint16_t *__restrict__ qh, int heads, int kv_heads, const int32_t *__restrict__ positions, int limit,
    const uint16_t *kcache, const uint16_t *vcache, int context, float scale,
    int8_t *__restrict__ q, float *__restrict__ scales, int32_t *__restrict__ qsum,
    const int32_t *__restrict__ slots, int nslots, QkRope fz, float *__restrict__ heads_f) {
    using Sh = ParShape<VW, FUSE>;
    constexpr int kCT = Sh::kCT, kCWaves = kCT / 64, kHalf = HD / 2;
    static_assert(VW * Sh::kPieces % kParThreads == 0 && kParThreads % VW == 0, "whole pieces and run slots");
    static_assert(Sh::kRunsPer * Sh::kSlots * kParRun >= Sh::kCap, "the runs are covered");
    static_assert(ROWS == 1 || ROWS == Sh::kMaxRows, "one key row a thread, or as many as the form holds");
    __shared__ __align__(16) uint32_t ql[HD / 2];                 // the query, fp16 pairs
    __shared__ __align__(16) uint16_t nk[HD];                    // FUSE: this position's key
    __shared__ __align__(16) uint16_t nvl[VW];                   // FUSE: this position's values of the slice
    __shared__ __align__(16) uint16_t vs[VW * Sh::kStride];      // the value slice, fp16
    __shared__ __align__(16) uint16_t ps[Sh::kCap];              // probabilities, fp16
    __shared__ float redm[kParThreads / 64];
    __shared__ float bsum[kParMaxBlocks];
    __shared__ float vpart[Sh::kCap / kParRun][VW + 1];
    __shared__ __align__(16) float hh[2 * HD];                   // FUSE: the query and key heads, fp32
    __shared__ __align__(16) double sq[2 * HD];                  // and their squares
    __shared__ float hs[2];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    constexpr int slices = HD / VW;
    const int group = heads / kv_heads;
    const int kvh = blockIdx.x % kv_heads, rb = blockIdx.x / kv_heads;
    const int hl = rb / slices, d0 = (rb - hl * slices) * VW;
    const int h0 = kvh * group + hl;
    const bool first = hl == 0;  // the query head whose workgroups store the position (FUSE)
    const int t = blockIdx.y;
    if (hl >= group)  // a grid wider than the heads: nothing of this workgroup's exists
        return;
    const int *pos_src = positions + t;
    const int32_t *slot_src = slots ? slots + t : nullptr;
    // FUSE, wavefront 0: the Q|K|V row's query and key heads, this position's
    // values of the slice and the norm gains first (no initial values: a
    // value for the other wavefronts would make wavefront 0 wait here)
    constexpr int kNv = (VW + 63) / 64;
    float4 hx;
    float nv[kNv], rg0[2], rg1[2], rc[2], rs[2];
    if (FUSE && wave == 0) {
        const float *row = fz.qkv + (size_t)t * fz.ldqkv;
        const int e = min(4 * lane, 2 * HD - 4);  // query elements, then key elements
        hx = *(const float4 *)(row + (e < HD ? h0 * HD + e : heads * HD + kvh * HD + (e - HD)));
#pragma unroll
        for (int r = 0; r < kNv; r++)
            nv[r] = row[(heads + kv_heads) * HD + kvh * HD + d0 + ((lane + 64 * r) % VW)];
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int i = min(lane + 64 * r, HD - 1);
            const int w = i / kHalf, j = i - w * kHalf;
            const float *gain = w == 0 ? fz.q_norm : fz.k_norm;
            rg0[r] = gain[j];
            rg1[r] = gain[j + kHalf];
        }
    }
    // without FUSE the query comes first: one dword a thread
    const uint32_t qr = FUSE ? 0u : ((const uint32_t *)(qh + ((size_t)t * heads + h0) * HD))[min(tid, HD / 2 - 1)];
    // a conversation's own caches: the slot decides the addresses
    size_t at = 0;
    if (slots)
        at = (size_t)min(max(*slot_src, 0), nslots - 1) * kv_heads * HD * context;
    // the key rows of the cache threads' positions ct + kCT r
    v4u_stream k[ROWS][HD / 8];
    const bool cw = !(FUSE && wave == 0);                       // a cache wavefront
    const int ct = tid - 64 * Sh::kW0, cwave = wave - Sh::kW0;  // its thread and wavefront among them
    if (cw) {
        const v4u_stream *kbase = (const v4u_stream *)(kcache + at + (size_t)kvh * HD * context);
#pragma unroll
        for (int r = 0; r < ROWS; r++) {
            if (r == 0 || r * kCT + cwave * 64 < limit) {
                const int p = min(ct + r * kCT, limit - 1);
#pragma unroll
                for (int i = 0; i < HD / 8; i++)
                    k[r][i] = kbase[(size_t)i * context + p];
            }
        }
    }
    // the value slice: VW contiguous rows, 16-byte pieces of the extent (with
    // FUSE, wavefront 0 issues its share after the rotation tables: loads
    // return in order, and the prologue waits for the tables)
    const uint16_t *vslice = vcache + at + ((size_t)kvh * HD + d0) * context;
    const int lastp = (limit - 1) >> 3;
    v4u_stream vr[Sh::kVLoads];
    auto load_values = [&]() {
#pragma unroll
        for (int c = 0; c < Sh::kVLoads; c++) {
            const int j = tid + kParThreads * c, row = j / Sh::kPieces, col = j - row * Sh::kPieces;
            vr[c] = *(const v4u_stream *)(vslice + (size_t)row * context + 8 * min(col, lastp));
        }
    };
    if (cw)
        load_values();
    const int pos = *pos_src;
    const int n = min(max(pos, 0) + 1, limit);
    const int rpos = min(max(pos, 0), context - 1);  // outside the cache: the tables' last row, nothing stored
    bool store = pos >= 0 && pos < context;
    if (FUSE && slots) {
        store = store && *slot_src >= 0 && *slot_src < nslots;
        fz.kcache += at;
        fz.vcache += at;
    }
    if (FUSE && wave == 0) {
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int i = min(lane + 64 * r, HD - 1);
            const int j = i % kHalf;
            rc[r] = fz.rope_cos[(size_t)rpos * kHalf + j];
            rs[r] = fz.rope_sin[(size_t)rpos * kHalf + j];
        }
        load_values();
    }
    if (FUSE) {
        if (wave == 0) {
            // the two heads' norms: the squares in parallel, each head's
            // float64 sum in order in one lane (head_norm_scale's, bit for bit)
            if (4 * lane < 2 * HD) {
                *(float4 *)(hh + 4 * lane) = hx;
                const float x4[4] = {hx.x, hx.y, hx.z, hx.w};
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const float v = x4[c];
                    const float sqf = v * v;
                    sq[4 * lane + c] = (double)sqf;
                }
            }
            if (lane < 2) {
                const double *sh = sq + lane * HD;
                double acc = 0.0;
#pragma unroll 16
                for (int i = 0; i < HD; i++)
                    acc += sh[i];
                const float mean = (float)(acc / (double)HD);
                hs[lane] = (float)(1.0 / sqrt((double)(mean + fz.eps)));
            }
            uint16_t *qlh = (uint16_t *)ql;
#pragma unroll
            for (int r = 0; r < 2; r++) {
                const int i = lane + 64 * r;
                if (i >= HD)
                    break;
                const int w = i / kHalf, j = i - w * kHalf;
                const float sc = hs[w];
                const float re0 = hh[w * HD + j], im0 = hh[w * HD + j + kHalf];
                const float re = (re0 * sc) * rg0[r], im = (im0 * sc) * rg1[r];
                const float c = rc[r], sn = rs[r];
                const float a = re * c - im * sn;
                const float b = re * sn + im * c;
                uint16_t ha = (uint16_t)float_to_half_bits(a), hb = (uint16_t)float_to_half_bits(b);
                if (w == 0) {
                    if (!store)  // no place in the cache: the query is NaN
                        ha = hb = 0x7E00;
                    qlh[j] = ha;
                    qlh[j + kHalf] = hb;
                } else {
                    nk[j] = ha;
                    nk[j + kHalf] = hb;
                    if (store && first && d0 == 0) {
                        uint16_t *kt = fz.kcache + (size_t)kvh * HD * context + (size_t)pos * 8;
                        kcache_put(kt, context, j, ha);
                        kcache_put(kt, context, j + kHalf, hb);
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < kNv; r++) {
                const int l = lane + 64 * r;
                if (l < VW) {
                    asm volatile("" : "+v"(nv[r]));  // converted here, not hoisted up to its load
                    const uint16_t vb = (uint16_t)float_to_half_bits(nv[r]);
                    nvl[l] = vb;
                    if (store && first)
                        fz.vcache[((size_t)kvh * HD + d0 + l) * context + pos] = vb;
                }
            }
        }
    } else {
        if (tid < HD / 2)
            ql[tid] = qr;
    }
    lds_barrier();
    if (FUSE && pos == n - 1 && cw) {  // this position's key from the copy, not the cache entry being written
#pragma unroll
        for (int r = 0; r < ROWS; r++)
            if (ct + r * kCT == pos) {
#pragma unroll
                for (int i = 0; i < HD / 8; i++)
                    k[r][i] = ((const v4u_stream *)nk)[i];
            }
    }

    // scores (DotF32's four chains: element e of the head goes to chain e % 4)
    // and their maximum
    float s[ROWS];
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
        s[r] = -INFINITY;
        if (!cw || r * kCT + cwave * 64 >= n)
            continue;
        const int p = ct + r * kCT;
        const v4u_stream *qv = (const v4u_stream *)ql;
        float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll
        for (int i = 0; i < HD / 8; i++) {
            const v4u_stream qq = qv[i], kk = k[r][i];
            s0 = fma_mix_lo(qq.x, kk.x, s0);
            s1 = fma_mix_hi(qq.x, kk.x, s1);
            s2 = fma_mix_lo(qq.y, kk.y, s2);
            s3 = fma_mix_hi(qq.y, kk.y, s3);
            s0 = fma_mix_lo(qq.z, kk.z, s0);
            s1 = fma_mix_hi(qq.z, kk.z, s1);
            s2 = fma_mix_lo(qq.w, kk.w, s2);
            s3 = fma_mix_hi(qq.w, kk.w, s3);
        }
        const float v = scale * ((s0 + s1) + (s2 + s3));
        if (p < n) {
            s[r] = v;
            mx = fmaxf(mx, v);
        }
    }
    mx = wave_max(mx);
    if (lane == 0)
        redm[wave] = mx;
    lds_barrier();
    float m = redm[0];
#pragma unroll
    for (int w = 1; w < kParThreads / 64; w++)
        m = fmaxf(m, redm[w]);
    // exponentials (exp_neg: SoftmaxInPlace's float64 exp rounded to float,
    // bit for bit); each 64-position block's
    // pairwise sum (a cache wavefront's lanes are one block's positions)
    float e[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
        e[r] = cw && ct + r * kCT < n ? exp_neg(s[r] - m) : 0.0f;
        if (cw && r * kCT + cwave * 64 < n) {
            const float b = wave_pairwise_sum(e[r]);
            if (lane == 0)
                bsum[cwave + kCWaves * r] = b;
        }
    }
    lds_barrier();
    // the total, blocks in order; the probabilities, rounded through fp16,
    // zeros past the prefix to the end of the last run
    const int nblocks = (n + kParBlock - 1) / kParBlock, nruns = (n + kParRun - 1) / kParRun;
    float total = 0.0f;
    for (int b = 0; b < nblocks; b++)
        total = total + bsum[b];
    if (cw) {
#pragma unroll
        for (int r = 0; r < ROWS; r++) {
            const int p = ct + r * kCT;
            if (p < n)
                ps[p] = (uint16_t)float_to_half_bits(__fdiv_rn(e[r], total));
            else if (p < nruns * kParRun)
                ps[p] = 0;
        }
    }
    // the value slice into LDS (with FUSE this position's values from the
    // copy, not the cache entries being written)
#pragma unroll
    for (int c = 0; c < Sh::kVLoads; c++) {
        const int j = tid + kParThreads * c, row = j / Sh::kPieces, col = j - row * Sh::kPieces;
        v4u_stream vv = vr[c];
        if (FUSE && pos == n - 1 && col == (pos >> 3)) {
            const int e8 = pos & 7;
            uint32_t wd[4] = {vv.x, vv.y, vv.z, vv.w};
            const uint32_t nb = nvl[row];
#pragma unroll
            for (int h = 0; h < 4; h++) {
                if (e8 == 2 * h)
                    wd[h] = (wd[h] & 0xFFFF0000u) | nb;
                if (e8 == 2 * h + 1)
                    wd[h] = (wd[h] & 0x0000FFFFu) | (nb << 16);
            }
            vv.x = wd[0];
            vv.y = wd[1];
            vv.z = wd[2];
            vv.w = wd[3];
        }
        *(v4u_stream *)(&vs[row * Sh::kStride + 8 * col]) = vv;
    }
    lds_barrier();

    // the runs' fma chains: whole 8-position pieces, then the piece the prefix
    // ends in, position by position (nothing past the prefix is read)
    const int dd = tid % VW, js = tid / VW;  // the thread's element and run slot
#pragma unroll
    for (int i = 0; i < Sh::kRunsPer; i++) {
        const int r = js + Sh::kSlots * i;
        if (r >= nruns)
            break;
        const int whole = min((n - r * kParRun) >> 3, kParRun / 8);
        const uint16_t *vrow = vs + dd * Sh::kStride + r * kParRun;
        const uint16_t *prow = ps + r * kParRun;
        float acc = 0.0f;
#pragma unroll
        for (int u = 0; u < kParRun / 8; u++) {
            if (u < whole) {
                const v4u_stream vv = *(const v4u_stream *)(vrow + 8 * u);
                const v4u_stream pp = *(const v4u_stream *)(prow + 8 * u);
                acc = fma_mix_lo(pp.x, vv.x, acc);
                acc = fma_mix_hi(pp.x, vv.x, acc);
                acc = fma_mix_lo(pp.y, vv.y, acc);
                acc = fma_mix_hi(pp.y, vv.y, acc);
                acc = fma_mix_lo(pp.z, vv.z, acc);
                acc = fma_mix_hi(pp.z, vv.z, acc);
                acc = fma_mix_lo(pp.w, vv.w, acc);
                acc = fma_mix_hi(pp.w, vv.w, acc);
            }
        }
        const int p0 = r * kParRun + 8 * whole;
        if (whole < kParRun / 8 && p0 < n) {
            const v4u_stream vv = *(const v4u_stream *)(vrow + 8 * whole);
            const v4u_stream pp = *(const v4u_stream *)(prow + 8 * whole);
            const uint32_t vw[4] = {vv.x, vv.y, vv.z, vv.w}, pw[4] = {pp.x, pp.y, pp.z, pp.w};
            for (int c = 0; c < n - p0; c++)
                acc = (c & 1) ? fma_mix_hi(pw[c >> 1], vw[c >> 1], acc) : fma_mix_lo(pw[c >> 1], vw[c >> 1], acc);
        }
        vpart[r][dd] = acc;
    }
    lds_barrier();
    // runs in order, then the slice's Q8_0 blocks (a 32-lane group a block)
    if (tid < VW) {
        float o = 0.0f;
        for (int r = 0; r < nruns; r++)
            o = o + vpart[r][tid];
        float stored;
        int32_t sm;
        const int32_t nq = q8_0_lane(o, &stored, &sm);
        const int width = heads * HD, B = width >> 5;
        const int col = h0 * HD + d0 + tid;
        if (heads_f)  // the head outputs themselves, for parity checks
            heads_f[(size_t)t * width + col] = o;
        if (q) {
            q[(size_t)t * width + col] = (int8_t)nq;
            if ((tid & 31) == 0) {
                scales[(size_t)t * B + (col >> 5)] = stored;
                qsum[(size_t)t * B + (col >> 5)] = sm;
            }
        }
    }
}

// ---- prompt attention on the matrix cores -----------------------------------
//
// The parallel form for a prompt (M > 4 tokens of one conversation, prefixes
// of at most kPmMax): grid (ceil(M / 32), heads), a workgroup per (query head,
// 32-token tile), eight wavefronts.  Per token, over its positions 0 .. pos:
//   scores  s_p = scale * (q . k_p): v_mfma_f32_32x32x16_f16 over the head
//           (fp16 operands, exact products, fp32 sums in the matrix core's
//           order), 32 tokens x 32 positions a tile, into LDS;
//   maximum, exponentials (exp_neg: the float64 exp of the float
//           difference, as SoftmaxInPlace), total and fp16 probabilities as the
//           decode's parallel order takes them: the total is ((0 + B_0) +
//           B_1) + ..., B_b the pairwise sum (wave_pairwise_sum) of 64-position
//           block b;
//   values  out[d] = sum_p prob_p * v_p[d]: the same MFMA, the probabilities
//           as the 32 x 16 operand (tokens x positions), the value rows as
//           the 16 x 32 one (positions x head elements); the positions in two
//           halves (a wavefront each), the first half's sum plus the second's.
// Positions past a token's own are +0 probabilities; value elements past the
// tile's last position are zeroed before they enter the product, so a cache
// entry not yet written (any bits) never reaches a sum.  The matrix cores'
// order of the two dot products is the only difference from the decode
// form: the head values are golem's within float rounding (checked at 1e-4 of
// RMS, as the decode's parallel order).
constexpr int kPmTok = 32;       // tokens a workgroup: one MFMA tile of rows
constexpr int kPmWaves = 8;
constexpr int kPmThreads = 64 * kPmWaves;
constexpr int kPmMax = 1024;     // positions the form holds (scores in LDS)
constexpr int kPmPre = 4;        // value pieces a lane keeps in flight

typedef _Float16 pm_v8h __attribute__((ext_vector_type(8)));
typedef float pm_v16f __attribute__((ext_vector_type(16)));

__host__ __device__ inline int pm_stride(int limit) { return ((limit + 63) & ~63) + 4; }  // floats a score row

template <int HD>
__global__ __launch_bounds__(kPmThreads, 4) void attn_prompt_mfma_kernel(
    const uint16_t *__restrict__ qh, int M, int heads, int kv_heads, const int32_t *__restrict__ positions,
    int limit, const uint16_t *__restrict__ kcache, const uint16_t *__restrict__ vcache, int context, float scale,
    int8_t *__restrict__ q, float *__restrict__ scales, int32_t *__restrict__ qsum, float *__restrict__ heads_f) {
    static_assert(HD % 32 == 0, "whole 32-element head blocks");
    constexpr int KS = HD / 16;  // the head in MFMA k-steps
    extern __shared__ __align__(16) float sl[];  // [kPmTok][stride]: scores, then exponentials
    __shared__ int nrow[kPmTok];
    __shared__ float mrow[kPmTok], trow[kPmTok];
    __shared__ float bsum[kPmTok][kPmMax / 64];
    __shared__ __align__(16) uint16_t qs[kPmTok][HD + 8];  // the tile's queries (+8: rows 4 banks apart)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, li = lane & 31, g = lane >> 5;
    // the second half of the heads takes the token tiles in reverse order:
    // workgroups L and L + grid / 2, which tend to share a CU, then hold
    // tiles i and n - 1 - i (light with heavy) rather than the same tile
    const int h = blockIdx.y;
    const int tile = 2 * blockIdx.y >= gridDim.y ? gridDim.x - 1 - blockIdx.x : blockIdx.x;
    const int t0 = tile * kPmTok;
    const int kvh = h / (heads / kv_heads);
    const int stride = pm_stride(limit);

    // the tile's queries into LDS (read back as the operands: token t0 + li,
    // elements 16 s + 8 g .., in registers they would crowd out the keys)
    for (int i = tid; i < kPmTok * (HD / 8); i += kPmThreads) {
        const int tk = i / (HD / 8), c = i - tk * (HD / 8);
        *(v4u_stream *)&qs[tk][8 * c] =
            *(const v4u_stream *)(qh + ((size_t)min(t0 + tk, M - 1) * heads + h) * HD + 8 * c);
    }
    if (tid < kPmTok)
        nrow[tid] = t0 + tid < M ? min(max(positions[t0 + tid], 0) + 1, limit) : 0;
    lds_barrier();
    int nmax = 0;
#pragma unroll 8
    for (int r = 0; r < kPmTok; r++)
        nmax = max(nmax, nrow[r]);
    const int np = (nmax + 63) & ~63;  // whole 64-position blocks

    // scores: wavefront w takes the 32-position tiles w, w + 4, ...; key
    // pieces past nmax repeat the last one (in bounds, never used)
    // (the next tile's keys are requested before this one's products: all
    // of a tile's loads in flight at once)
    // (32-bit byte offsets from one uniform base: an address a piece
    // costs one register, not two)
    const char *kb = (const char *)(kcache + (size_t)kvh * HD * context);
    auto kload = [&](int j, pm_v8h *bk) {
        const int p = min(32 * j + li, nmax - 1);
#pragma unroll
        for (int s = 0; s < KS; s++)
            bk[s] = *(const pm_v8h *)(kb + (uint32_t)(((2 * s + g) * context + p) * 16));
    };
    pm_v8h bk[KS];
    kload(wave, bk);
    for (int j = wave; j < np / 32; j += kPmWaves) {
        pm_v8h cur[KS];
#pragma unroll
        for (int s = 0; s < KS; s++)
            cur[s] = bk[s];
        if (j + kPmWaves < np / 32)
            kload(j + kPmWaves, bk);
        pm_v16f acc = {};
#pragma unroll
        for (int s = 0; s < KS; s++) {
            const pm_v8h aq = *(const pm_v8h *)&qs[li][16 * s + 8 * g];
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(aq, cur[s], acc, 0, 0, 0);
        }
#pragma unroll
        for (int e = 0; e < 16; e++)
            sl[(8 * (e >> 2) + 4 * g + (e & 3)) * stride + 32 * j + li] = scale * acc[e];
    }
    lds_barrier();

    // The values: wavefront w takes head block db = w % 4 (elements 32 db ..
    // 32 db + 31) over half hf = w / 4 of the k-steps (16 positions each);
    // its first kPmPre value pieces go out now, to land while the softmax
    // runs (its barriers wait for LDS only): lane (li, g) holds positions
    // 16 i + 8 g .. + 7 of element 32 db + li.
    const int db = wave & 3, hf = wave >> 2;
    const bool pv = db < HD / 32;
    const int nsteps = np / 16, half = (nsteps + 1) / 2;
    const int i_lo = hf ? half : 0, i_hi = hf ? nsteps : half;
    const uint16_t *vrow = vcache + ((size_t)kvh * HD + 32 * db + li) * context;
    auto vload = [&](int i) -> v4u_stream {
        return *(const v4u_stream *)(vrow + min(16 * i + 8 * g, context - 8));  // a multiple of 8, as the context is
    };
    v4u_stream vr[kPmPre];
    if (pv) {
#pragma unroll
        for (int u = 0; u < kPmPre; u++)
            vr[u] = vload(min(i_lo + u, i_hi - 1));
    }

    // each token's maximum over its own positions: a wavefront a token, lane
    // l holding positions 64 b + l
    for (int r = wave; r < kPmTok; r += kPmWaves) {
        const int n = nrow[r];
        const float *row = sl + r * stride;
        const int nbr = (n + 63) >> 6;
        float m = -INFINITY;
        for (int b0 = 0; b0 < nbr; b0 += 4) {  // four reads in flight
            float v[4];
#pragma unroll
            for (int u = 0; u < 4; u++)
                v[u] = row[64 * min(b0 + u, nbr - 1) + lane];
#pragma unroll
            for (int u = 0; u < 4; u++)
                m = 64 * (b0 + u) + lane < n ? fmaxf(m, v[u]) : m;
        }
        m = wave_max(m);
        if (lane == 0)
            mrow[r] = m;
    }
    lds_barrier();
    // exponentials in place and each 64-position block's pairwise sum, a
    // wavefront a token, four blocks at once (independent float64 chains,
    // every lane computing; positions past the token's own become +0)
    for (int r = wave; r < kPmTok; r += kPmWaves) {
        const int n = nrow[r], nbr = (n + 63) >> 6;
        const float m = mrow[r];
        float *row = sl + r * stride;
        for (int b0 = 0; b0 < nbr; b0 += 4) {
            float d[4], ev[4];
#pragma unroll
            for (int u = 0; u < 4; u++)
                d[u] = row[64 * min(b0 + u, nbr - 1) + lane] - m;
            exp_neg_n<4>(d, ev);
#pragma unroll
            for (int u = 0; u < 4; u++)
                ev[u] = 64 * (b0 + u) + lane < n ? ev[u] : 0.0f;
            float bs[4];
#pragma unroll
            for (int u = 0; u < 4; u++)
                bs[u] = wave_pairwise_sum(ev[u]);
#pragma unroll
            for (int u = 0; u < 4; u++) {
                if (b0 + u < nbr) {
                    row[64 * (b0 + u) + lane] = ev[u];
                    if (lane == 0)
                        bsum[r][b0 + u] = bs[u];
                }
            }
        }
    }
    lds_barrier();
    if (tid < kPmTok) {
        float total = 0.0f;
        const int nbr = (nrow[tid] + 63) >> 6;
        for (int b = 0; b < nbr; b++)
            total = total + bsum[tid][b];
        trow[tid] = total;
    }
    lds_barrier();
    // the probabilities fp16(e / total) in place (+0 past the token's own
    // positions): sixteen lanes a token, 128 positions a step; a step's
    // halves overwrite floats of its own or an earlier step, already read (a
    // wavefront's LDS accesses keep their order)
    {
        const int r = tid >> 4, sub = tid & 15;
        const float tot = trow[r];
        const int n = nrow[r];
        float *row = sl + r * stride;
        uint16_t *hrow = (uint16_t *)row;
        for (int c = 0; 128 * c < np; c++) {
            const int p0 = 128 * c + 8 * sub;
            if (p0 < np) {
                const float4 e0 = *(const float4 *)(row + p0), e1 = *(const float4 *)(row + p0 + 4);
                const float ev[8] = {e0.x, e0.y, e0.z, e0.w, e1.x, e1.y, e1.z, e1.w};
                uint32_t hv[8];
#pragma unroll
                for (int k = 0; k < 8; k++)
                    hv[k] = p0 + k < n ? float_to_half_bits(__fdiv_rn(ev[k], tot)) : 0u;
                *(v4u_stream *)(hrow + p0) = (v4u_stream){hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16),
                                                          hv[4] | (hv[5] << 16), hv[6] | (hv[7] << 16)};
            }
        }
    }
    lds_barrier();

    // values: the probabilities as the row operand, the value pieces as the
    // column operand; piece i + kPmPre is requested as piece i is used
    const uint16_t *pr = (const uint16_t *)(sl + li * stride) + 8 * g;
    pm_v16f acc = {};
    if (pv) {
        for (int i0 = i_lo; i0 < i_hi; i0 += kPmPre) {
#pragma unroll
            for (int u = 0; u < kPmPre; u++) {
                const int i = i0 + u;
                if (i < i_hi) {
                    v4u_stream vv = vr[u];
                    if (i + kPmPre < i_hi)
                        vr[u] = vload(i + kPmPre);
                    const int p0 = 16 * i + 8 * g;
                    if (p0 + 8 > nmax) {  // the piece the tile's positions end in, or past them: zeros from nmax
#pragma unroll
                        for (int k = 0; k < 4; k++) {
                            const uint32_t keep = (p0 + 2 * k < nmax ? 0x0000FFFFu : 0u) |
                                                  (p0 + 2 * k + 1 < nmax ? 0xFFFF0000u : 0u);
                            vv[k] &= keep;
                        }
                    }
                    const pm_v8h ap = *(const pm_v8h *)(pr + 16 * i);
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ap, __builtin_bit_cast(pm_v8h, vv), acc, 0, 0, 0);
                }
            }
        }
    }
    // the two halves' sums added, first half first: the second half's
    // wavefronts leave theirs in LDS (the probabilities are spent)
    lds_barrier();
    float *part = sl + db * 16 * 64 + lane;
    if (pv && hf) {
#pragma unroll
        for (int e = 0; e < 16; e++)
            part[64 * e] = acc[e];
    }
    lds_barrier();
    // the first half's wavefronts add the second's and lay the tile's head
    // floats out token by token: acc[e] is token 8 (e / 4) + 4 g + e % 4,
    // head element 32 db + li
    constexpr int OS = HD + 4;  // floats a staged output row
    float *ot = sl + 4 * 16 * 64;
    if (pv && !hf) {
#pragma unroll
        for (int e = 0; e < 16; e++)
            ot[(8 * (e >> 2) + 4 * g + (e & 3)) * OS + 32 * db + li] = acc[e] + part[64 * e];
    }
    lds_barrier();
    // then every thread: four consecutive values of a token, eight lanes a
    // Q8_0 block
    const int width = heads * HD, B = width >> 5;
    for (int i4 = tid; i4 < kPmTok * (HD / 4); i4 += kPmThreads) {
        const int tk = i4 / (HD / 4), c4 = i4 - tk * (HD / 4), t = t0 + tk;
        const float4 o = *(const float4 *)(ot + tk * OS + 4 * c4);
        const float v[4] = {o.x, o.y, o.z, o.w};
        float stored;
        int32_t sm;
        const uint32_t packed = q8_0_quad(v, &stored, &sm);
        if (t < M) {
            const int col = h * HD + 4 * c4;
            if (heads_f)
                *(float4 *)(heads_f + (size_t)t * width + col) = o;
            if (q) {
                *(uint32_t *)(q + (size_t)t * width + col) = packed;
                if ((c4 & 7) == 0) {
                    scales[(size_t)t * B + (col >> 5)] = stored;
                    qsum[(size_t)t * B + (col >> 5)] = sm;
                }
            }
        }
    }
}

int launch_prompt_mfma(gx_ctx *ctx, const uint16_t *qh, int M, int heads, int kv_heads, int hd, int limit,
                       const int32_t *positions, const uint16_t *kcache, const uint16_t *vcache, int context,
                       float scale, int8_t *q, float *scales, int32_t *qsum, float *heads_f) {
    // the scores; later the second half's value sums, 4 x 16 x 64 floats
    // the scores, later the half sums [4][16][64] and the output tile [32][hd + 4]
    const size_t lds =
        sizeof(float) * std::max((size_t)kPmTok * pm_stride(limit), (size_t)4 * 16 * 64 + (size_t)kPmTok * (hd + 4));
    const dim3 grid((unsigned)((M + kPmTok - 1) / kPmTok), (unsigned)heads);
#define GX_PM(HH)                                                                                                    \
    attn_prompt_mfma_kernel<HH><<<grid, kPmThreads, lds, ctx->stream>>>(                                             \
        qh, M, heads, kv_heads, positions, limit, kcache, vcache, context, scale, q, scales, qsum, heads_f)
    if (hd == 32)
        GX_PM(32);
    else if (hd == 64)
        GX_PM(64);
    else if (hd == 96)
        GX_PM(96);
    else
        GX_PM(128);
#undef GX_PM
    return check_launch("qwen_attention prompt mfma");
}

// grid (ceil(ffn/256), M): gu [M][ldgu] holds each position's gate then up
// (ffn each), or gates and ups interleaved by 32 (group 32).  mid =
// silu(gate) * up (SwiGLURange, nn/swiglu.go:77-82), Q8_0.
__global__ __launch_bounds__(256) void qwen_swiglu_quant_kernel(const float *__restrict__ gu, int ldgu, int ffn,
                                                                int group, int8_t *__restrict__ q,
                                                                float *__restrict__ scales,
                                                                int32_t *__restrict__ qsum) {
    const int t = blockIdx.y;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= ffn)
        return;  // ffn % 32 == 0: whole groups
    // group 0: gate [ffn] then up [ffn]; group 32: 32 gates then their 32 ups
    const size_t gi = group ? (size_t)(i >> 5) * 64 + (i & 31) : (size_t)i;
    const size_t ui = group ? gi + 32 : (size_t)ffn + i;
    const float g = gu[(size_t)t * ldgu + gi];
    const float u = gu[(size_t)t * ldgu + ui];
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

// Greedy choice in two launches: kArgmaxParts workgroups per row each take
// a contiguous part and leave the part's largest value and the lowest index
// holding it (none if the part is all NaN); one wavefront per row then merges
// the parts.  "Larger value, else lower index" is a total order, so the
// result is the index of the largest non-NaN value, the lower index on ties,
// whatever the split.  golem's Argmax (gemma/model.go:288-296,
// qwen/model_test.go:118-126) starts from index 0 and moves only to a value
// greater than the current best, so a NaN anywhere but at index 0 never wins,
// and a NaN at index 0 wins outright (nothing compares greater): the merge
// returns 0 when x[0] is NaN, and 0 when every value is NaN.
constexpr int kArgmaxThreads = 256;
constexpr int kNone = 0x7fffffff;

__device__ __forceinline__ void argmax_merge(float &bv, int &bi, float ov, int oi) {
    if (oi != kNone && (bi == kNone || ov > bv || (ov == bv && oi < bi))) {
        bv = ov;
        bi = oi;
    }
}

// grid (kArgmaxParts, M)
__global__ __launch_bounds__(kArgmaxThreads) void argmax_part_kernel(const float *__restrict__ x, int ldx, int n,
                                                                     float *__restrict__ part_v,
                                                                     int32_t *__restrict__ part_i) {
    __shared__ float bv_sh[kArgmaxThreads / 64];
    __shared__ int bi_sh[kArgmaxThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *r = x + (size_t)blockIdx.y * ldx;
    const int chunk = ((n + kArgmaxParts - 1) / kArgmaxParts + 3) & ~3;
    const int lo = min(n, (int)blockIdx.x * chunk), hi = min(n, lo + chunk);
    float bv = -INFINITY;
    int bi = kNone;
    auto take = [&](float v, int i) {
        if (v > bv || (bi == kNone && v == v)) {  // rising order: equal values keep the first
            bv = v;
            bi = i;
        }
    };
    if (((uintptr_t)r & 15) == 0) {
        const int q0 = lo / 4, q1 = hi / 4;  // lo is a multiple of 4
#pragma unroll 4
        for (int q = q0 + tid; q < q1; q += kArgmaxThreads) {
            const float4 v = *(const float4 *)(r + 4 * q);
            take(v.x, 4 * q);
            take(v.y, 4 * q + 1);
            take(v.z, 4 * q + 2);
            take(v.w, 4 * q + 3);
        }
        for (int i = 4 * q1 + tid; i < hi; i += kArgmaxThreads)
            take(r[i], i);
    } else {
        for (int i = lo + tid; i < hi; i += kArgmaxThreads)
            take(r[i], i);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        argmax_merge(bv, bi, ov, oi);
    }
    if (lane == 0) {
        bv_sh[wave] = bv;
        bi_sh[wave] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < kArgmaxThreads / 64; w++)
            argmax_merge(bv, bi, bv_sh[w], bi_sh[w]);
        part_v[(size_t)blockIdx.y * kArgmaxParts + blockIdx.x] = bv;
        part_i[(size_t)blockIdx.y * kArgmaxParts + blockIdx.x] = bi;
    }
}

// grid (M), one wavefront.  With `history` (M = 1, a captured decode step):
// also, while *pos + 1 < history_len, history[*pos + 1] = id, *pos += 1 and
// positions[0] = the new *pos; at the history's end the counter stops there,
// so a step replayed past the end never addresses past it.  With
// `row_tokens` (a lock-step step of M conversations): row_tokens[m] = id and
// row_positions[m] += 1, each row's next input.
__global__ __launch_bounds__(64) void argmax_final_kernel(const float *__restrict__ x, int ldx,
                                                          const float *__restrict__ part_v,
                                                          const int32_t *__restrict__ part_i,
                                                          int32_t *__restrict__ out, int32_t *__restrict__ history,
                                                          int history_len, int32_t *__restrict__ pos,
                                                          int32_t *__restrict__ positions,
                                                          int32_t *__restrict__ row_tokens,
                                                          int32_t *__restrict__ row_positions) {
    const int lane = threadIdx.x;
    float bv = -INFINITY;
    int bi = kNone;
    for (int p = lane; p < kArgmaxParts; p += 64)
        argmax_merge(bv, bi, part_v[(size_t)blockIdx.x * kArgmaxParts + p],
                     part_i[(size_t)blockIdx.x * kArgmaxParts + p]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        argmax_merge(bv, bi, ov, oi);
    }
    if (lane == 0) {
        const float x0 = x[(size_t)blockIdx.x * ldx];
        const int id = (bi == kNone || x0 != x0) ? 0 : bi;
        out[blockIdx.x] = id;
        if (row_tokens) {
            row_tokens[blockIdx.x] = id;
            row_positions[blockIdx.x] += 1;
        }
        if (history) {
            const int next = pos[0] + 1;
            if (next < history_len) {
                history[next] = id;
                pos[0] = next;
                positions[0] = next;
            }
        }
    }
}

// The parallel-order decode attention (attn_par_kernel): the whole-head form
// (VW = HD, a workgroup a query head) for extents of at most kParShortMax
// positions with whole-wavefront head widths, else 32-element slices; one key
// row a cache thread when the extent fits the cache threads (half the key
// registers), else as many as kDecodeMax needs.
template <bool FUSE>
int launch_par(gx_ctx *ctx, const uint16_t *qh, int M, int heads, int kv_heads, int hd, int limit,
               const int32_t *positions, const uint16_t *kcache, const uint16_t *vcache, int context, float scale,
               int8_t *q, float *scales, int32_t *qsum, const int32_t *slots, int nslots, const QkRope &fz,
               float *heads_f) {
#define GX_PAR(HH, RR, VV)                                                                                           \
    attn_par_kernel<HH, FUSE, RR, VV><<<dim3((unsigned)(heads * (HH / VV)), (unsigned)M), kParThreads, 0,            \
                                        ctx->stream>>>(qh, heads, kv_heads, positions, limit, kcache, vcache,       \
                                                       context, scale, q, scales, qsum, slots, nslots, fz, heads_f)
#define GX_PAR_R(HH, SHORT)                                                                                          \
    do {                                                                                                             \
        if (SHORT && limit <= kParShortMax)                                                                          \
            GX_PAR(HH, 1, (SHORT ? HH : kValSlice));                                                                 \
        else if (limit <= ParShape<kValSlice, FUSE>::kCT)                                                            \
            GX_PAR(HH, 1, kValSlice);                                                                                \
        else                                                                                                         \
            GX_PAR(HH, (ParShape<kValSlice, FUSE>::kMaxRows), kValSlice);                                            \
    } while (0)
    if (hd == 32)
        GX_PAR_R(32, false);
    else if (hd == 64)
        GX_PAR_R(64, true);
    else if (hd == 96)
        GX_PAR_R(96, false);
    else
        GX_PAR_R(128, true);
#undef GX_PAR_R
#undef GX_PAR
    return check_launch("qwen_attention parallel");
}

}  // namespace

int launch_qwen_norm_quant(gx_ctx *ctx, float *x, int ldx, const float *add, int lda, const float *gain, int M, int K,
                           float eps, float *out, int ldo, int8_t *q, float *scales, int32_t *qsum) {
    const size_t lds = 2 * sizeof(float) * (size_t)K;
    GX_CHECK(lds <= 160 * 1024, "gx: a norm over %d values does not fit the LDS", K);
    qwen_norm_quant_kernel<<<M, kQNormThreads, lds, ctx->stream>>>(x, ldx, add, lda, gain, K, eps, out, ldo, q,
                                                                   scales, qsum);
    return check_launch("qwen_norm_quant");
}

int launch_qwen_qk_rope(gx_ctx *ctx, const float *qkv, int ldqkv, int M, int heads, int kv_heads, int hd,
                        const int32_t *positions, const float *q_norm, const float *k_norm, const float *rope_cos,
                        const float *rope_sin, float eps, uint16_t *qh, uint16_t *kcache, uint16_t *vcache,
                        int context, const int32_t *slots, int nslots) {
    GX_CHECK(hd <= kHeadMax && hd % 8 == 0, "gx: head width %d unsupported (a multiple of 8, at most %d)", hd,
             kHeadMax);
    // A batch (and a head width the tiled kernel is built for, operands it
    // can read 16 bytes at a time): 64 tokens of a head a workgroup.
    const bool aligned =
        (((uintptr_t)qkv | (uintptr_t)rope_cos | (uintptr_t)rope_sin | (uintptr_t)qh | (uintptr_t)kcache) & 15) == 0 &&
        ldqkv % 4 == 0;
    if (M >= 32 && (hd == 64 || hd == 128) && aligned) {
        const dim3 grid((unsigned)((M + kQkTok - 1) / kQkTok), (unsigned)(heads + kv_heads));
        if (hd == 64)
            qwen_qk_rope_tile_kernel<64><<<grid, 256, 0, ctx->stream>>>(qkv, ldqkv, M, heads, kv_heads, positions,
                                                                         q_norm, k_norm, rope_cos, rope_sin, eps, qh,
                                                                         kcache, vcache, context, slots, nslots);
        else
            qwen_qk_rope_tile_kernel<128><<<grid, 256, 0, ctx->stream>>>(qkv, ldqkv, M, heads, kv_heads, positions,
                                                                          q_norm, k_norm, rope_cos, rope_sin, eps, qh,
                                                                          kcache, vcache, context, slots, nslots);
        return check_launch("qwen_qk_rope tiles");
    }
    qwen_qk_rope_kernel<<<dim3((unsigned)M, (unsigned)(heads + kv_heads)), 64, 0, ctx->stream>>>(
        qkv, ldqkv, heads, kv_heads, hd, positions, q_norm, k_norm, rope_cos, rope_sin, eps, qh, kcache, vcache,
        context, slots, nslots);
    return check_launch("qwen_qk_rope");
}

size_t qwen_attention_workspace(int M, int heads, int max_pos) {
    const size_t S = ((size_t)max_pos + kTile) / kTile * kTile;
    const size_t rows = (size_t)M * heads;
    auto up = [](size_t b) { return (b + 255) / 256 * 256; };
    return up(rows * S * sizeof(float)) + up(rows * S * sizeof(uint16_t));
}

int launch_qwen_attention(gx_ctx *ctx, const uint16_t *qh, int M, int heads, int kv_heads, int hd, int max_pos,
                          const int32_t *positions, const uint16_t *kcache, const uint16_t *vcache, int context,
                          float scale, int8_t *q, float *scales, int32_t *qsum, uint8_t *workspace,
                          const int32_t *slots, int nslots, int parallel, float *heads_f) {
    const int G = heads / kv_heads;
    GX_CHECK(hd == 32 || hd == 64 || hd == 96 || hd == 128, "gx: attention supports head widths 32, 64, 96 and 128");
    GX_CHECK(G == 1 || G == 2 || G == 4 || G == 8, "gx: %d query heads per key-value head unsupported", G);
    const int S = (max_pos + kTile) / kTile * kTile;
    const int limit = max_pos + 1;  // positions beyond max_pos are read as max_pos
    const size_t rows = (size_t)M * heads;
    auto up = [](size_t b) { return (b + 255) / 256 * 256; };
    float *sc = (float *)workspace;
    uint16_t *prob = (uint16_t *)(workspace + up(rows * S * sizeof(float)));

    // One workgroup per token: a few tokens of one conversation, or tokens of
    // several conversations (slots), whose caches share nothing.
    if (parallel && (M <= 4 || slots) && limit <= kDecodeMax)
        return launch_par<false>(ctx, qh, M, heads, kv_heads, hd, limit, positions, kcache, vcache, context, scale,
                                 q, scales, qsum, slots, nslots, QkRope{}, heads_f);
    // A prompt of one conversation in the parallel order: the matrix cores.
    if (parallel && !slots && limit <= kPmMax)
        return launch_prompt_mfma(ctx, qh, M, heads, kv_heads, hd, limit, positions, kcache, vcache, context, scale,
                                  q, scales, qsum, heads_f);
    if ((M <= 4 || slots) && limit <= kDecodeMax) {
// One query head per workgroup when that fills at most two workgroups per CU
// (128 workgroups for config 3's decode rather than 32): the scores,
// exponentials and divisions a workgroup repeats for its value slice shrink
// by the group size; the key rows are read by more workgroups, from the L2
// their key-value head's workgroups share.  Larger batches keep a group of
// query heads per workgroup.
#define GX_DECODE(HH, GG)                                                                                            \
    attn_decode_kernel<HH, GG, false><<<dim3((unsigned)(heads / GG * (HH / kValSlice)), (unsigned)M), kDecodeThreads,\
                                        0, ctx->stream>>>(qh, heads, kv_heads, positions, limit, kcache, vcache,      \
                                                          context, scale, q, scales, qsum, slots, nslots, QkRope{})
#define GX_DECODE_G(HH)                                                                                              \
    do {                                                                                                             \
        if ((size_t)M * heads * (HH / kValSlice) <= 2 * (size_t)ctx->cu_count || G == 1)                             \
            GX_DECODE(HH, 1);                                                                                        \
        else if (G == 2)                                                                                             \
            GX_DECODE(HH, 2);                                                                                        \
        else if (G == 4)                                                                                             \
            GX_DECODE(HH, 4);                                                                                        \
        else                                                                                                         \
            GX_DECODE(HH, 8);                                                                                        \
    } while (0)
        if (hd == 32)
            GX_DECODE_G(32);
        else if (hd == 64)
            GX_DECODE_G(64);
        else if (hd == 96)
            GX_DECODE_G(96);
        else
            GX_DECODE_G(128);
#undef GX_DECODE_G
#undef GX_DECODE
        return check_launch("qwen_attention decode");
    }
    // Scores: decode spreads the heads of a group over wavefronts (the key
    // rows are re-read from L2); a batch shares each key row among the group's
    // heads and 8 tokens.
    const int GH = M <= 4 ? 1 : G, TT = M <= 4 || slots ? 1 : 8;
    const dim3 sgrid((unsigned)(S / kTile), (unsigned)(heads / GH), (unsigned)((M + TT - 1) / TT));
#define GX_SCORES(HH)                                                                                                \
    attn_scores_kernel<HH><<<sgrid, 64, (size_t)TT * GH * HH * 2, ctx->stream>>>(                               \
        qh, M, heads, G, GH, TT, positions, limit, kcache, context, scale, S, sc, slots, nslots, kv_heads)
    if (hd == 32)
        GX_SCORES(32);
    else if (hd == 64)
        GX_SCORES(64);
    else if (hd == 96)
        GX_SCORES(96);
    else
        GX_SCORES(128);
#undef GX_SCORES
    if (int rc = check_launch("qwen_attention scores"))
        return rc;
    {
        const int cap = min(kSoftChunk, S);
        attn_softmax_kernel<<<dim3((unsigned)((heads + kSoftRows - 1) / kSoftRows), (unsigned)M), 64 * kSoftRows,
                              (size_t)kSoftRows * (cap + 16) * sizeof(float), ctx->stream>>>(heads, positions, limit, S,
                                                                                             cap, sc, prob);
    }
    if (int rc = check_launch("qwen_attention softmax"))
        return rc;
    // Values for a prompt (head widths of whole 64-element wavefronts): the
    // probabilities as wavefront-wide operands, 16 wavefronts a workgroup,
    // four tokens a wavefront.  Config 3's 512-token prefill: 106 -> 64 us a
    // layer (counters: the VALU ~11 % busy, a third of the wave cycles
    // waiting -- every probability reaches all 64 lanes of a wavefront).
    if (M > 4 && !slots && G <= 4 && hd % kSpDims == 0) {
        constexpr int kTC = 4;
#define GX_VSP(GG)                                                                                                   \
    do {                                                                                                             \
        constexpr int TGW = 16 / GG, TT = TGW * kTC;                                                                 \
        const size_t lds = (size_t)(kSpDims + TT * GG) * kSpStride * sizeof(uint16_t);                               \
        attn_values_sp_kernel<kTC, GG, TGW><<<dim3((unsigned)(kv_heads * (hd / kSpDims)),                            \
                                                   (unsigned)((M + TT - 1) / TT)),                                   \
                                              64 * TGW * GG, lds, ctx->stream>>>(M, heads, hd, positions, limit,     \
                                                                                 vcache, context, kv_heads, S, prob, \
                                                                                 q, scales, qsum);                   \
    } while (0)
        if (G == 1)
            GX_VSP(1);
        else if (G == 2)
            GX_VSP(2);
        else
            GX_VSP(4);
#undef GX_VSP
        return check_launch("qwen_attention values");
    }
    // Values: TT tokens of G heads per workgroup, 32 chains each (NT <= 256).
    int NT = G * kValSlice;
    while (NT < 128 && NT * 2 <= G * kValSlice * M)
        NT *= 2;
    if (M > 4 && NT < 256)
        NT *= 2;
    if (slots)  // a token tile is one token: its cache is its own
        NT = G * kValSlice;
    const int TT2 = NT / (G * kValSlice);
    const dim3 vgrid((unsigned)(kv_heads * (hd / kValSlice)), (unsigned)((M + TT2 - 1) / TT2));
#define GX_VALUES(N)                                                                                                 \
    attn_values_kernel<N><<<vgrid, N, 0, ctx->stream>>>(M, heads, G, hd, positions, limit, vcache, context,         \
                                                        kv_heads, S, prob, q, scales, qsum, slots, nslots)
    if (NT == 32)
        GX_VALUES(32);
    else if (NT == 64)
        GX_VALUES(64);
    else if (NT == 128)
        GX_VALUES(128);
    else
        GX_VALUES(256);
#undef GX_VALUES
    return check_launch("qwen_attention values");
}

int launch_qwen_rope_attention(gx_ctx *ctx, const float *qkv, int ldqkv, int M, int heads, int kv_heads, int hd,
                               int max_pos, const int32_t *positions, const float *q_norm, const float *k_norm,
                               const float *rope_cos, const float *rope_sin, float eps, uint16_t *kcache,
                               uint16_t *vcache, int context, float scale, int8_t *q, float *scales, int32_t *qsum,
                               const int32_t *slots, int nslots, int parallel) {
    const int G = heads / kv_heads;
    GX_CHECK(hd == 32 || hd == 64 || hd == 96 || hd == 128, "gx: attention supports head widths 32, 64, 96 and 128");
    GX_CHECK(G == 1 || G == 2 || G == 4 || G == 8, "gx: %d query heads per key-value head unsupported", G);
    const int limit = max_pos + 1;
    GX_CHECK(limit <= kDecodeMax, "gx: the fused attention reads at most %d positions, not %d", kDecodeMax, limit);
    const QkRope fz{qkv, ldqkv, q_norm, k_norm, rope_cos, rope_sin, eps, kcache, vcache};
    if (parallel)
        return launch_par<true>(ctx, nullptr, M, heads, kv_heads, hd, limit, positions, kcache, vcache, context,
                                scale, q, scales, qsum, slots, nslots, fz, nullptr);
#define GX_FUSED(HH)                                                                                                 \
    attn_decode_kernel<HH, 1, true><<<dim3((unsigned)(heads * (HH / kValSlice)), (unsigned)M), kDecodeThreads, 0,             \
                                      ctx->stream>>>(nullptr, heads, kv_heads, positions, limit, kcache, vcache,     \
                                                     context, scale, q, scales, qsum, slots, nslots, fz)
    if (hd == 32)
        GX_FUSED(32);
    else if (hd == 64)
        GX_FUSED(64);
    else if (hd == 96)
        GX_FUSED(96);
    else
        GX_FUSED(128);
#undef GX_FUSED
    return check_launch("qwen_rope_attention");
}

int launch_qwen_swiglu_quant(gx_ctx *ctx, const float *gu, int ldgu, int M, int ffn, int group, int8_t *q,
                             float *scales, int32_t *qsum) {
    qwen_swiglu_quant_kernel<<<dim3((unsigned)((ffn + 255) / 256), (unsigned)M), 256, 0, ctx->stream>>>(
        gu, ldgu, ffn, group, q, scales, qsum);
    return check_launch("qwen_swiglu_quant");
}

int launch_argmax(gx_ctx *ctx, const float *x, int ldx, int M, int n, int32_t *out, int32_t *history,
                  int history_len, int32_t *pos, int32_t *positions, int32_t *row_tokens, int32_t *row_positions) {
    for (int m0 = 0; m0 < M; m0 += kArgmaxRows) {
        const int rows = min(kArgmaxRows, M - m0);
        argmax_part_kernel<<<dim3(kArgmaxParts, (unsigned)rows), kArgmaxThreads, 0, ctx->stream>>>(
            x + (size_t)m0 * ldx, ldx, n, ctx->argmax_v, ctx->argmax_i);
        argmax_final_kernel<<<rows, 64, 0, ctx->stream>>>(x + (size_t)m0 * ldx, ldx, ctx->argmax_v, ctx->argmax_i,
                                                          out + m0, history, history_len, pos, positions,
                                                          row_tokens ? row_tokens + m0 : nullptr,
                                                          row_positions ? row_positions + m0 : nullptr);
        if (int rc = check_launch("argmax"))
            return rc;
    }
    return GX_OK;
}

}  // namespace gx
