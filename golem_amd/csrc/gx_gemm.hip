// gx_gemm.hip - the Q4_0 x Q8_0 product for a batch of tokens (prefill) on
// int8 MFMA.
//
// golem reads a prompt through the same MatVecBatch as a single token, with
// the batch as the inner loop (nn/matrix.go:67-81, nn/pack_q4_0.go:159-221).
// Here the batch is a real dense contraction: v_mfma_i32_32x32x32_i8 takes one
// Q4_0 block (32 inputs) of 32 rows against the same block of 32 tokens and
// returns the exact per-block integers; the fp32 scales are applied to them
// per block in the canonical order of the matrix-vector kernel
// (gx_q4_0.hip), stretch by stretch, so a token's result is bit-identical
// whether it came through this kernel or that one.
//
// The per-block epilogue is what bounds this product: every output element
// needs float(isum) * (d_w * d_a) added to its sum, per block.  The scale
// product d_w[i] * d_a[j] of a 32x32 tile is an outer product of two fp16
// vectors (golem stores d_a, the Q8_0 scale, already rounded through fp16),
// so it comes from the matrix core too: v_mfma_f32_32x32x8_f16 with the two
// vectors in k = 0 and zeros elsewhere gives every product exactly (an
// 11-bit by 11-bit product fits fp32; the int8 kernel puts them in k = 0 and
// k = 4 and takes 2 d_w d_a against half the integer).  The vector ALU is
// left with one conversion (a subtraction) and one fma per element per
// block.
//
// Two kernels: the int8 one below (loads straight into LDS, every Q4_0
// product of more than a few tokens, dense or grouped by expert) and an fp16
// one for callers that hold the activation's fp16 copy.  The weights'
// nibbles are widened to signed int8 (n - 8) in registers as they are read.
#include <type_traits>

#include "gx_device.hpp"
#include "gx_internal.hpp"

namespace gx {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));

// A 32x32x8 f16 operand holding the fp16 bits `h` at k = 0 (lanes 0..31,
// element 0) and zeros everywhere else.
__device__ __forceinline__ v4h k0_operand(uint32_t h, bool first_half) {
    const uint2 bits = make_uint2(first_half ? (h & 0xFFFFu) : 0u, 0u);
    return __builtin_bit_cast(v4h, bits);
}

// The same operand in both halves of the wavefront (k = 0 and k = 4): the
// outer product then holds every d_w[i] * d_a[j] twice, 2 d_w d_a, exactly.
// `h` has its upper 16 bits clear (a u16 LDS read, or a VOP1 fp16 result).
__device__ __forceinline__ v4h k04_operand(uint32_t h) {
    return __builtin_bit_cast(v4h, make_uint2(h, 0u));
}

// {fp16(f), +0} as one dword, in one instruction.  Exact for a value that fp16
// holds, whatever the rounding (the Q8_0 activation scales are fp16 values).
__device__ __forceinline__ uint32_t half2_bits_rtz(float f) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(f, 0.0f));
}


// Blocks a pipeline stage holds (half a stretch).
constexpr int kStage = 4;

// A mixture-of-experts product runs grouped: workgroup row y of the grid is
// work item y, {expert, first, count}, covering units sorted[first ..
// first + count) of one expert (count 0: nothing to do).  Unit u reads
// activation row u / act_div and writes output row u.
struct Groups {
    const int32_t *work;
    const int32_t *sorted;
    int act_div;
    size_t matrix_bytes;
};

// ---- the fp16 product ------------------------------------------------------
//
// The same contraction with the per-block integers taken by
// v_mfma_f32_32x32x16_f16 from integer-valued fp16 operands: the weights
// (n - 8) and the Q8_0 values q, both exact in fp16.  Every product and every
// partial sum is an integer below 2^24 in magnitude, so the fp32 result is
// the exact per-block integer, already a float: the epilogue is one fma per
// element per block, where the int8 kernel needs a conversion and an fma.
//
// Tile: a workgroup owns 64 rows (one R64 tile) x 32*NWT tokens; wavefront w
// owns the 64 rows x token group w (32 tokens): two 32x32 MFMA tiles sharing
// the activation operand.  The rows' nibbles are widened to fp16 once per
// workgroup into LDS, four blocks per stage, double buffered: the next
// stage's nibbles are in flight while this one's MFMAs run.  Each wavefront
// reads its activation operands straight from the panel-ordered fp16 copy
// (q16_offset): one contiguous 1 KiB per operand, one block ahead.
constexpr int kFStage = 4;   // blocks per stage
constexpr int kFWRow = 40;   // halves per staged weight row (32 + pad: 80-byte rows)

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

// Four nibbles (one per byte, values 0..15) -> four fp16 values n - 8, as two
// dwords.  0x64 above a byte makes the fp16 1024 + n; subtracting 1032 is
// exact.
__device__ __forceinline__ void nibbles_to_f16(uint32_t n, uint32_t &lo, uint32_t &hi) {
    const uint32_t a = __builtin_amdgcn_perm(0x64646464u, n, 0x04010400u);
    const uint32_t b = __builtin_amdgcn_perm(0x64646464u, n, 0x04030402u);
    const v2h bias = {(_Float16)1032.0f, (_Float16)1032.0f};
    lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(v2h, a) - bias);
    hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(v2h, b) - bias);
}

// One block row of nibbles (16 bytes) -> its 32 fp16 weights in golem's
// order in LDS: [0,16) from the low nibbles of bytes 0..15, [16,32) from the
// high nibbles.
__device__ __forceinline__ void widen_row(const v4u &w, uint16_t *row) {
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
    uint32_t out[16];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        nibbles_to_f16(words[k] & 0x0F0F0F0Fu, out[2 * k], out[2 * k + 1]);
        nibbles_to_f16((words[k] >> 4) & 0x0F0F0F0Fu, out[8 + 2 * k], out[8 + 2 * k + 1]);
    }
#pragma unroll
    for (int k = 0; k < 4; k++)
        *(v4u *)(row + 8 * k) = (v4u){out[4 * k], out[4 * k + 1], out[4 * k + 2], out[4 * k + 3]};
}

template <int NWT, bool DOTS>
__global__ __launch_bounds__(64 * NWT) void q4_0_gemm_f16_kernel(
    const uint8_t *__restrict__ W, size_t plane0_bytes, int B, int DC, const uint16_t *__restrict__ q16,
    const float *__restrict__ scales, int M, int tile0, int row_start, int row_end, const float *__restrict__ bias,
    float *__restrict__ y, int ldy, int32_t *__restrict__ dots) {
    constexpr int NT = 64 * NWT;
    constexpr int RW = (kFStage * kTileRows + NT - 1) / NT;  // 16-byte nibble chunks per thread per stage
    __shared__ __attribute__((aligned(16))) uint16_t wl[2][kFStage][kTileRows][kFWRow];
    __shared__ uint16_t dwl[2][kFStage][kTileRows];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wv = tid >> 6, li = lane & 31, g = lane >> 5;
    const int tile = tile0 + blockIdx.x;
    const int n0 = tile * kTileRows;
    const int Gn = (M + 31) / 32;
    const int G = blockIdx.y * NWT + wv;  // this wavefront's token group
    const int Gc = min(G, Gn - 1);
    const int t = 32 * G + li;            // this lane's token
    const float *srow = scales ? scales + (size_t)min(t, M - 1) * B : nullptr;
    const uint16_t *panel = q16 + (size_t)Gc * B * 1024 + 8 * lane;  // + (2b + h) * 512
    const int S = (B + kFStage - 1) / kFStage;
    const int nrows = row_end - row_start;

    // Stage h's nibbles: chunk c (block c / 64, row c % 64) for c = tid + NT i;
    // clamped past the last block (never used).  Scales: rows tid < 64, the
    // 8 bytes of the row's scale chunk that hold the stage's 4 blocks.
    v4u raw[RW];
    uint2 sraw = make_uint2(0, 0);
    auto fetch_w = [&](int h, v4u (&r)[RW], uint2 &sr) {
#pragma unroll
        for (int i = 0; i < RW; i++) {
            const int c = min(tid + NT * i, kFStage * kTileRows - 1);
            const int b = min(h * kFStage + (c >> 6), B - 1);
            r[i] = *(const v4u *)(W + (((size_t)tile * B + b) * kTileRows + (c & 63)) * kChunk);
        }
        if (!DOTS && tid < kTileRows) {
            const int b0 = h * kFStage;
            sr = *(const uint2 *)(W + plane0_bytes + (((size_t)tile * DC + (b0 >> 3)) * kTileRows + tid) * kChunk +
                                  2 * (b0 & 7));
        }
    };
    auto commit_w = [&](int buf, const v4u (&r)[RW], const uint2 &sr) {
#pragma unroll
        for (int i = 0; i < RW; i++) {
            const int c = tid + NT * i;
            if (c < kFStage * kTileRows)
                widen_row(r[i], wl[buf][c >> 6][c & 63]);
        }
        if (!DOTS && tid < kTileRows) {
            dwl[buf][0][tid] = (uint16_t)(sr.x & 0xFFFFu);
            dwl[buf][1][tid] = (uint16_t)(sr.x >> 16);
            dwl[buf][2][tid] = (uint16_t)(sr.y & 0xFFFFu);
            dwl[buf][3][tid] = (uint16_t)(sr.y >> 16);
        }
    };

    v16f acc0, acc1, tot0, tot1;
#pragma unroll
    for (int e = 0; e < 16; e++)
        acc0[e] = acc1[e] = tot0[e] = tot1[e] = 0.0f;
    const v16f zero_f = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

    // Activation operands a stage ahead, in two register sets that alternate
    // by stage (the stage loop is unrolled by two, so each set's registers are
    // fixed): slot j of a set holds block 4s + j's two panels and scale
    // (clamped past the last block; never used there).
    v8h PA0[kFStage], PA1[kFStage], PB0[kFStage], PB1[kFStage];
    float dA[kFStage], dB[kFStage];
#define GX_F16_LOAD_SET(P0, P1, DS, s)                                                                               \
    do {                                                                                                             \
        for (int j = 0; j < kFStage; j++) {                                                                          \
            const int bn = min((s) * kFStage + j, B - 1);                                                            \
            P0[j] = *(const v8h *)(panel + (size_t)(2 * bn) * 512);                                                  \
            P1[j] = *(const v8h *)(panel + (size_t)(2 * bn + 1) * 512);                                              \
            DS[j] = DOTS ? 0.0f : srow[bn];                                                                          \
        }                                                                                                            \
    } while (0)

// One stage, software-pipelined across the two row tiles: tile 0's MFMAs for
// block j, then tile 1's fmas for block j - 1 (results of the previous
// block's MFMAs), then tile 1's MFMAs for block j, then tile 0's fmas for
// block j -- each batch of fmas runs while an independent batch of MFMAs is
// in the matrix core.  `pend` is the block whose tile-1 fmas are pending (-1:
// none).
#define GX_F16_FMA(D, SC, ACC, TOT, bb)                                                                              \
    do {                                                                                                             \
        for (int e = 0; e < 16; e++)                                                                                 \
            ACC[e] = fmaf(D[e], SC[e], ACC[e]);                                                                      \
        if (((bb) & (kStretch - 1)) == kStretch - 1 || (bb) == B - 1) { /* a stretch ends */                         \
            for (int e = 0; e < 16; e++) {                                                                           \
                TOT[e] = TOT[e] + ACC[e];                                                                            \
                ACC[e] = 0.0f;                                                                                       \
            }                                                                                                        \
        }                                                                                                            \
    } while (0)

#define GX_F16_DOTS(D, roff, bb)                                                                                     \
    do {                                                                                                             \
        if (t < M) {                                                                                                 \
            for (int e = 0; e < 16; e++) {                                                                           \
                const int n = n0 + (roff) + 8 * (e >> 2) + 4 * g + (e & 3);                                          \
                if (n >= row_start && n < row_end)                                                                   \
                    dots[((size_t)t * nrows + (n - row_start)) * B + (bb)] = (int32_t)D[e];                          \
            }                                                                                                        \
        }                                                                                                            \
    } while (0)

#define GX_F16_STAGE(P0, P1, DS, h)                                                                                  \
    do {                                                                                                             \
        const int buf = (h) & 1;                                                                                     \
        const int nb = min(kFStage, B - (h) * kFStage);                                                              \
        for (int j = 0; j < kFStage; j++) {                                                                          \
            if (j < nb) {                                                                                            \
                const int b = (h) * kFStage + j;                                                                     \
                const v4h Bs = k0_operand(float_to_half_bits(DS[j]), g == 0);                                        \
                {                                                                                                    \
                    const v8h A00 = *(const v8h *)&wl[buf][j][li][8 * g];                                            \
                    const v8h A01 = *(const v8h *)&wl[buf][j][li][16 + 8 * g];                                       \
                    D0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(A00, P0[j], zero_f, 0, 0, 0);                         \
                    D0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(A01, P1[j], D0, 0, 0, 0);                            \
                    if (!DOTS)                                                                                       \
                        S0 = __builtin_amdgcn_mfma_f32_32x32x8f16(k0_operand(dwl[buf][j][li], g == 0), Bs, zero_f,  \
                                                                  0, 0, 0);                                          \
                }                                                                                                    \
                if (!DOTS && pend >= 0)                                                                              \
                    GX_F16_FMA(D1, S1, acc1, tot1, pend);                                                            \
                {                                                                                                    \
                    const v8h A10 = *(const v8h *)&wl[buf][j][32 + li][8 * g];                                       \
                    const v8h A11 = *(const v8h *)&wl[buf][j][32 + li][16 + 8 * g];                                  \
                    D1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(A10, P0[j], zero_f, 0, 0, 0);                         \
                    D1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(A11, P1[j], D1, 0, 0, 0);                            \
                    if (!DOTS)                                                                                       \
                        S1 = __builtin_amdgcn_mfma_f32_32x32x8f16(k0_operand(dwl[buf][j][32 + li], g == 0), Bs,     \
                                                                  zero_f, 0, 0, 0);                                  \
                }                                                                                                    \
                if (DOTS) {                                                                                          \
                    GX_F16_DOTS(D0, 0, b);                                                                           \
                    GX_F16_DOTS(D1, 32, b);                                                                          \
                } else {                                                                                             \
                    GX_F16_FMA(D0, S0, acc0, tot0, b);                                                               \
                }                                                                                                    \
                pend = b;                                                                                            \
            }                                                                                                        \
        }                                                                                                            \
    } while (0)

    v16f D0 = zero_f, D1 = zero_f, S0 = zero_f, S1 = zero_f;
    int pend = -1;
    fetch_w(0, raw, sraw);
    GX_F16_LOAD_SET(PA0, PA1, dA, 0);
    commit_w(0, raw, sraw);
    __syncthreads();
    for (int h = 0; h < S; h += 2) {  // set A holds stage h
        if (h + 1 < S) {  // in flight during this stage's arithmetic
            fetch_w(h + 1, raw, sraw);
            GX_F16_LOAD_SET(PB0, PB1, dB, h + 1);
        }
        GX_F16_STAGE(PA0, PA1, dA, h);
        if (h + 1 >= S)
            break;
        commit_w((h + 1) & 1, raw, sraw);
        __syncthreads();
        if (h + 2 < S) {
            fetch_w(h + 2, raw, sraw);
            GX_F16_LOAD_SET(PA0, PA1, dA, h + 2);
        }
        GX_F16_STAGE(PB0, PB1, dB, h + 1);
        if (h + 2 < S) {
            commit_w(h & 1, raw, sraw);
            __syncthreads();
        }
    }
    if (!DOTS && pend >= 0)  // the last block's tile-1 fmas
        GX_F16_FMA(D1, S1, acc1, tot1, pend);
#undef GX_F16_LOAD_SET
#undef GX_F16_STAGE
#undef GX_F16_FMA
#undef GX_F16_DOTS
    if (DOTS || t >= M)
        return;
#pragma unroll
    for (int e = 0; e < 16; e++) {
        const int r = 8 * (e >> 2) + 4 * g + (e & 3);
        const int na = n0 + r, nb2 = n0 + 32 + r;
        if (na >= row_start && na < row_end)
            y[(size_t)t * ldy + na] = bias ? tot0[e] + bias[na] : tot0[e];
        if (nb2 >= row_start && nb2 < row_end)
            y[(size_t)t * ldy + nb2] = bias ? tot1[e] + bias[nb2] : tot1[e];
    }
}


// ---- the int8 product, loads straight into LDS -------------------------
//
// The kernel for the Q4_0 x Q8_0 product of a batch.  Every stage's operands come in by direct
// global-to-LDS loads (global_load_lds_dwordx4 / _dword): no registers stage
// them, and the stages live in an LDS ring of kRing slots (four for the
// 64-token form, three for the 32-token one), all but one in flight while one
// is multiplied.  A workgroup owns 128 rows (two R64 tiles) x 64 tokens; each
// of its eight wavefronts one 32x32 MFMA tile (rows 32*(w&3), tokens
// 32*(w>>2)), at four wavefronts per SIMD (two workgroups per CU).  Per stage
// (4 blocks) each wavefront issues exactly kLoads loads, so `s_waitcnt
// vmcnt((kRing - 2) kLoads)` before the stage's barrier means "this stage has
// landed" for every wavefront; the barrier is the bare s_barrier (the fence of
// __syncthreads would wait for every load in flight).  Slot layout (bytes):
//   [0, 8192)       nibbles  [block 4][row 128][16]
//   [8192, 16384)   int8     [block 4][half 2][token 64][16]
//   [16384, 17408)  act. scales (fp32) [block 4][token 64]
//   [17408, 18432)  weight scales (fp16) [row 128][block 4]
constexpr int kDmaTok = 64;
// LDS slots of the ring (stages in flight + 1).  The 64-token form takes
// four (two workgroups a CU still fit: 2 x 72 KiB): config 2 at M = 2048
// 180 -> 177 us; the 32-token form keeps three, which keep three
// workgroups a CU (four slots: M = 512 50 -> 55 us, config 4's prefill
// 181 -> 189 us).
#ifndef GX_DMA_RING64
#define GX_DMA_RING64 4
#endif
#ifndef GX_DMA_RING32
#define GX_DMA_RING32 3
#endif
// The integer products run on a biased chain.  The weights enter the MFMA as
// 16 * (n - 8) (the nibble in a byte's high half, its top bit flipped), and
// each block's MFMA adds its 16 * isum to the previous block's output; a
// stretch's chain starts from the bits of 1.5 * 2^18.  Read as fp32, every
// output is then 1.5 * 2^18 plus half the stretch's running isum, exactly:
// the ulp in [2^18, 2^19) is 1/32, and the running sum of a stretch is at
// most 8 blocks * 32 * 8 * 128 = 2^18 in magnitude, 2^22 ulps either side of
// the middle of the binade, whose ends (bits 0x48800000 and 0x49000000) are
// exactly 2^18 and 2^19.  The difference of two consecutive outputs is half
// the block's isum as an fp32 -- one full-rate subtraction instead of a
// conversion -- and the scale outer product is 2 d_w d_a (k04_operand), so
// fma(isum / 2, 2 d_w d_a, acc) is golem's fma(isum, d_w d_a, acc) bit for
// bit: the two products are the same real number, rounded once.
constexpr int kChainBias = 0x48C00000;  // 393216.0f

// One block's operands from LDS (nibbles, activations, weight scale,
// activation scale), issued without a wait.  Written out so that the
// compiler sees no LDS load: it would otherwise make each one wait for every
// load-to-LDS in flight, the next stages' included.  The caller waits
// (lgkmcnt) before it uses the four registers.
//
// Lane (row or token l % 32, half g = l / 32) reads 8 bytes of its row's
// nibble chunk, bytes 8g .. 8g + 7, and takes both nibbles of each: its MFMA
// slots are k = 16 + 8g .. 16 + 8g + 7 (the high nibbles) then k = 8g ..
// 8g + 7 (the low ones), and its activation operand holds the same k in the
// same order: bytes 8g .. 8g + 7 of the block's second half (OA1), then of
// its first half (OA0).  The integer sum does not depend on the order of k;
// a lane widening a whole half-chunk's one nibble needed two instructions a
// dword for the low half, and this takes six for the lane's sixteen.
template <int OW, int OA1, int OA0, int OD, int OS>
__device__ __forceinline__ void lds_read_block(uint32_t aw, uint32_t aa, uint32_t ad, uint32_t as, uint2 &rw,
                                               uint2 &ra1, uint2 &ra0, uint32_t &rdw, float &rda) {
    asm volatile(
        "ds_read_b64 %0, %5 offset:%9\n\t"
        "ds_read_b64 %1, %6 offset:%10\n\t"
        "ds_read_b64 %2, %6 offset:%11\n\t"
        "ds_read_u16 %3, %7 offset:%12\n\t"
        "ds_read_b32 %4, %8 offset:%13"
        : "=&v"(rw), "=&v"(ra1), "=&v"(ra0), "=&v"(rdw), "=&v"(rda)
        : "v"(aw), "v"(aa), "v"(ad), "v"(as), "i"(OW), "i"(OA1), "i"(OA0), "i"(OD), "i"(OS));
}

template <int J, int N, typename F>
__device__ __forceinline__ void unroll(F &&f) {  // f(integral_constant<int, J>) for J in [J, N)
    if constexpr (J < N) {
        f(std::integral_constant<int, J>{});
        unroll<J + 1, N>(f);
    }
}


// The two tile shapes of the direct-to-LDS product.  Both: a workgroup owns
// 128 rows (two R64 tiles), a wavefront one 32x32 MFMA tile (rows 32*(w&3),
// tokens 32*(w>>2)).
//   TOK 64: eight wavefronts; three loads a wavefront a stage.  Slot bytes:
//     [0, 8192) nibbles [block 4][row 128][16]
//     [8192, 16384) int8 [block 4][half 2][token 64][16]
//     [16384, 17408) act. scales (fp32) [block 4][token 64]
//     [17408, 18432) weight scales (fp16) [row 128][block 4]
//   TOK 32: four wavefronts (for batches of few tokens: an expert's share of
//     a prompt); five loads a wavefront a stage -- two of nibbles, one of
//     int8, two dwords of scales (the last of wavefronts 2 and 3 a dummy, so
//     that every wavefront issues the same count).  Slot bytes:
//     [0, 8192) nibbles [block 4][row 128][16]
//     [8192, 12288) int8 [block 4][half 2][token 32][16]
//     [12288, 12800) act. scales (fp32) [block 4][token 32]
//     [12800, 13824) weight scales (fp16) [row 128][block 4]
//     [13824, 14080) the dummy dwords
template <int TOK>
struct DmaShape;
template <>
struct DmaShape<64> {
    static constexpr int kWaves = 8, kLoads = 3, kSlot = 18432, kOcc = 4;  // two workgroups a CU
    static constexpr int kRing = GX_DMA_RING64;
    static constexpr int kAct = 8192, kActScale = 16384, kWScale = 17408;
};
template <>
struct DmaShape<32> {
    static constexpr int kWaves = 4, kLoads = 5, kSlot = 14336, kOcc = 3;  // three workgroups a CU (LDS)
    static constexpr int kRing = GX_DMA_RING32;
    static constexpr int kAct = 8192, kActScale = 12288, kWScale = 12800, kDummy = 13824;
};

// EPI 2's epilogue (see the kernel): 4 wavefronts, wavefront rg holding
// rows 32 rg .. of the workgroup's 128 for tokens first + li.  Element e of
// a rotated head: pair j = e % half, a = re c - im s (e < half), b = re s +
// im c, re = x_j sc g_j, im = x_{j+half} sc g_{j+half} (RoPETable.Apply,
// nn/rope.go:62-73; qwen/attention.go:57-84, qwen/cache.go:52-60).
constexpr int kQkvStride = 129;  // a token's staged row: a lane a token reads down a column without conflicts

__device__ __forceinline__ void qkv_rope_epilogue(const v16f &tot, uint8_t *lds, const QkvRopeArgs &qr, int T0,
                                                  int rg, int li, int g, int first, int count) {
    const int tid = threadIdx.x;
    const int hd = qr.hd, half = hd >> 1, P = hd >> 3, hpw = 128 / hd;  // pieces a head; heads a workgroup
    const int nheads = qr.heads + 2 * qr.kv_heads;
    const int h0 = T0 * kTileRows / hd;  // the workgroup's first head
    float *hs = (float *)lds;                       // [32 tokens][kQkvStride]
    float *gs = hs + 32 * kQkvStride;               // [128]: each row's gain
    float *scs = gs + 128;                          // [2][32] norm scales
    int *pos_s = (int *)(scs + 64), *place_s = pos_s + 32, *slot_s = place_s + 32;
    __syncthreads();  // every wavefront is past its last operand reads
#pragma unroll
    for (int e = 0; e < 16; e++)
        hs[li * kQkvStride + 32 * rg + 8 * (e >> 2) + 4 * g + (e & 3)] = tot[e];
    // section of head k of the workgroup: 0 query, 1 key, 2 value, 3 none
    auto section = [&](int k) -> int {
        const int hg = h0 + k;
        return hg < qr.heads ? 0 : hg < qr.heads + qr.kv_heads ? 1 : hg < nheads ? 2 : 3;
    };
    if (tid < 32) {
        int pl = -1, pos = 0, sl = 0;
        if (tid < count) {
            const int t = first + tid;
            pos = qr.positions[t];
            sl = qr.slots ? qr.slots[t] : 0;
            pl = pos >= 0 && pos < qr.context && (!qr.slots || (sl >= 0 && sl < qr.nslots)) ? 1 : 0;
        }
        pos_s[tid] = pos;
        place_s[tid] = pl;
        slot_s[tid] = sl;
    } else if (tid >= 64 && tid < 192) {
        const int r = tid - 64, sec = section(r / hd);
        gs[r] = sec == 0 ? qr.q_norm[r % hd] : sec == 1 ? qr.k_norm[r % hd] : 0.0f;
    }
    __syncthreads();
    // (head, token, piece) items of the query and key heads, two a thread:
    // a query's pieces fastest (contiguous in qh), a key's tokens fastest
    // (a piece's positions are contiguous in the cache).  Their rotation
    // tables go out now, while the norms' sums run.
    float4 c0[2], c1[2], s0[2], s1[2];
    int ik[2], itk[2], ipc[2], isec[2];
#pragma unroll
    for (int it = 0; it < 2; it++) {
        const int idx = tid + 256 * it, k = idx / (32 * P), rem = idx - k * 32 * P;
        const int sec = section(k);
        const int tk = sec == 0 ? rem / P : rem & 31, pc = sec == 0 ? rem % P : rem >> 5;
        ik[it] = k, itk[it] = tk, ipc[it] = pc, isec[it] = sec;
        if (sec <= 1 && place_s[tk] > 0) {
            const int pos = pos_s[tk];
            const int j0 = 8 * pc < half ? 8 * pc : 8 * pc - half;
            c0[it] = *(const float4 *)(qr.rope_cos + (size_t)pos * half + j0);
            c1[it] = *(const float4 *)(qr.rope_cos + (size_t)pos * half + j0 + 4);
            s0[it] = *(const float4 *)(qr.rope_sin + (size_t)pos * half + j0);
            s1[it] = *(const float4 *)(qr.rope_sin + (size_t)pos * half + j0 + 4);
        }
    }
    if (tid < 32 * hpw) {
        // head_norm_scale's sum, left to right, sixteen values read ahead
        const int k = tid >> 5, tk = tid & 31;
        if (section(k) <= 1 && tk < count) {
            const float *hr = hs + tk * kQkvStride + k * hd;
            double acc = 0.0;
            for (int i0 = 0; i0 < hd; i0 += 16) {
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
            const float mean = (float)(acc / (double)hd);
            scs[tid] = (float)(1.0 / sqrt((double)(mean + qr.eps)));
        }
    }
    __syncthreads();
#pragma unroll
    for (int it = 0; it < 2; it++) {
        const int k = ik[it], tk = itk[it], pc = ipc[it], sec = isec[it];
        const int pl = place_s[tk];
        if (sec > 1 || pl < 0)
            continue;
        const int pos = pos_s[tk], hg = h0 + k;
        uint32_t w[4] = {0x7E007E00u, 0x7E007E00u, 0x7E007E00u, 0x7E007E00u};  // no place: a NaN query
        if (pl) {
            const bool lo = 8 * pc < half;
            const int j0 = lo ? 8 * pc : 8 * pc - half;
            const float cs[8] = {c0[it].x, c0[it].y, c0[it].z, c0[it].w, c1[it].x, c1[it].y, c1[it].z, c1[it].w};
            const float sn[8] = {s0[it].x, s0[it].y, s0[it].z, s0[it].w, s1[it].x, s1[it].y, s1[it].z, s1[it].w};
            const float sc = scs[k * 32 + tk];
            const float *hr = hs + tk * kQkvStride + k * hd;
            const float *gr = gs + k * hd;
            uint32_t hb[8];
#pragma unroll
            for (int kk = 0; kk < 8; kk++) {
                const int j = j0 + kk;
                const float re = (hr[j] * sc) * gr[j], im = (hr[j + half] * sc) * gr[j + half];
                const float v = lo ? re * cs[kk] - im * sn[kk] : re * sn[kk] + im * cs[kk];
                hb[kk] = float_to_half_bits(v);
            }
#pragma unroll
            for (int kk = 0; kk < 4; kk++)
                w[kk] = hb[2 * kk] | (hb[2 * kk + 1] << 16);
        }
        const v4u_stream o = {w[0], w[1], w[2], w[3]};
        if (sec == 0) {
            *(v4u_stream *)(qr.qh + (size_t)(first + tk) * qr.heads * hd + (size_t)hg * hd + 8 * pc) = o;
        } else if (pl) {
            uint16_t *kt = qr.kcache + (size_t)slot_s[tk] * qr.kv_heads * hd * qr.context +
                           (size_t)(hg - qr.heads) * hd * qr.context;
            *(v4u_stream *)(kt + ((size_t)pc * qr.context + pos) * 8) = o;
        }
    }
    // the value heads: a lane a token down each element row
    for (int k = 0; k < hpw; k++) {
        if (section(k) != 2)
            continue;
        const int kvh = h0 + k - qr.heads - qr.kv_heads;
        for (int idx = tid; idx < 32 * hd; idx += 256) {
            const int tk = idx & 31, d = idx >> 5;
            if (place_s[tk] > 0) {
                uint16_t *vt = qr.vcache + (size_t)slot_s[tk] * qr.kv_heads * hd * qr.context +
                               (size_t)kvh * hd * qr.context;
                vt[(size_t)d * qr.context + pos_s[tk]] = (uint16_t)float_to_half_bits(hs[tk * kQkvStride + k * hd + d]);
            }
        }
    }
}

// GROUPED: blockIdx.y is an item of the expert work list (grp.work[item] =
// {expert, first, count <= TOK, 0}; count 0 past the last item): the item's
// tokens are units sorted[first ..], token t reading activation row
// sorted[first + t] / act_div and writing output row sorted[first + t], all
// against expert grp.work[item].x of the stack (matrices matrix_bytes
// apart).  Otherwise tokens TOK * blockIdx.y .. of the batch.
//
// DOTS: the same kernel, also writing every block's integer (the chain
// difference x below) to dots[out row][n - row_start][b]; the scales are then
// not needed, and their loads read the activation instead (in bounds).
//
// EPI 1 (dense, whole matrix): the rows are gate and up interleaved by 32 (a
// tile's rows 0..31 gate, 32..63 up, for the same 32 outputs), and the
// product ends in silu(gate) * up and its Q8_0 (qwen_swiglu_quant_kernel's
// arithmetic, element for element) into mq / ms / mqs [M][rows / 2]: the
// wavefront of a tile's up rows passes its sums through LDS to the
// wavefront of the gate rows, whose lane pair (l, l + 32) holds one token's
// 32 outputs, one Q8_0 block.
//
// EPI 2 (dense, whole matrix, TOK 32): the rows are the query, key and value
// heads stacked (hd = 64 or 128 rows a head, so a workgroup's 128 rows are
// whole heads), and the product ends in qwen_qk_rope_tile_kernel's work for
// its heads and 32 tokens, bit for bit: the sums staged in LDS by token, a
// query or key head's RMSNormPlain (float64, left to right, a lane a token),
// RoPE with golem's tables, fp16, the query into qr.qh and the key and value
// into the caches -- without the [M][rows] float round trip.
template <int TOK, bool GROUPED, bool DOTS, int EPI = 0>
__global__ __launch_bounds__(64 * DmaShape<TOK>::kWaves, DmaShape<TOK>::kOcc) void q4_0_gemm_dma_kernel(
    const uint8_t *__restrict__ W, size_t plane0_bytes, int B, int DC, const int8_t *__restrict__ q,
    const float *__restrict__ scales, int K, int M, int tiles, int tile0, int row_start, int row_end,
    const float *__restrict__ bias, float *__restrict__ y, int ldy, int32_t *__restrict__ dots, Groups grp,
    int xcd_pairs, int8_t *__restrict__ mq, float *__restrict__ ms, int32_t *__restrict__ mqs, QkvRopeArgs qr) {
    using Sh = DmaShape<TOK>;
    constexpr int kSlotB = Sh::kSlot;
    // Software-pipelined blocks (one block's MFMAs ahead of the previous
    // block's epilogue) need ~30 more registers: the 32-token form, at three
    // workgroups a CU by its LDS, has them; the 64-token form would lose its
    // fourth wavefront a SIMD.
    constexpr bool kPipe = TOK == 32;
    constexpr int kRing = Sh::kRing;
    __shared__ __align__(16) uint8_t ring_lds[kRing * kSlotB];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    // The workgroup's row pair bx and token group by.  With xcd_pairs > 0 the
    // grid is one-dimensional in the dispatcher's XCD order (workgroup i runs
    // on XCD i % 8): XCD x takes row pairs [x P / 8, (x + 1) P / 8) of the P
    // and every token group, token group by token group, so that its L2
    // holds its rows' weights while the tokens stream past once.  (A 2-D
    // grid deals every XCD all row pairs: each L2 refetches the whole matrix
    // many times over.)
    int bx = blockIdx.x, by = blockIdx.y;
    if (!GROUPED && xcd_pairs > 0) {
        const int x = blockIdx.x & 7, local = blockIdx.x >> 3;
        const int lo = x * xcd_pairs / 8, n = (x + 1) * xcd_pairs / 8 - lo;
        if (local >= n * ((M + TOK - 1) / TOK))
            return;  // this XCD's share is done: the whole workgroup
        by = local / n;
        bx = lo + (local - by * n);
    }
    const int T0 = tile0 + 2 * bx;                // the workgroup's first R64 tile
    const int rg = wv & 3, tg = wv >> 2;          // this wavefront's 32 rows and 32 tokens
    const int li = lane & 31, g = lane >> 5;
    int first, count;
    if (GROUPED) {
        const int4 item = ((const int4 *)grp.work)[by];
        count = item.z;
        if (count <= 0)
            return;  // past the last item: the whole workgroup
        W += (size_t)item.x * grp.matrix_bytes;
        first = item.y;
    } else {
        first = by * TOK;
        count = min(TOK, M - first);
    }
    // token t's activation row and output row
    auto arow = [&](int t) -> int { return GROUPED ? grp.sorted[first + t] / grp.act_div : first + t; };
    auto orow = [&](int t) -> int { return GROUPED ? grp.sorted[first + t] : first + t; };
    // Stages, two to a stretch.  An odd count gets one more stage: the second
    // half of the last stretch, all of whose blocks lie past the row, with
    // weight scales 0 from the plane's padding.
    const int Hp = ((B + kStage - 1) / kStage + 1) & ~1;

    // This lane's sources, fixed for the product.  Loads past the matrix, the
    // batch or the second tile read in-bounds neighbours; their values are
    // never used (weight scale 0, or not stored).
    auto wpair_src = [&](int pidx) -> const uint8_t * {  // weight-scale pair pidx of the 256
        const int r = pidx >> 1;
        const int dt = min(T0 + (r >> 6), tiles - 1);
        return W + plane0_bytes + ((size_t)dt * DC * kTileRows + (r & 63)) * kChunk + 4 * (pidx & 1);
    };
    const uint8_t *wsrc0, *wsrc1 = nullptr, *ssrc, *ssrc2 = nullptr;
    const int8_t *asrc;
    int wj, wh;
    if constexpr (TOK == 64) {
        wj = wv & 3, wh = wv >> 2;                // nibble load: block wj, rows 64*wh + lane
        wsrc0 = W + ((size_t)min(T0 + wh, tiles - 1) * B * kTileRows + lane) * kChunk;
        const int ag = wv & 1;                    // activation load: block wv >> 1, half ag, token lane
        asrc = q + (size_t)arow(min(lane, count - 1)) * K + 16 * ag;
        // The third load is a dword for every wavefront: waves 0..3 an
        // activation scale (block wv, token lane), waves 4..7 a pair of
        // weight scales (pair 64 * (wv - 4) + lane).
        if (wv < 4)
            ssrc = DOTS ? (const uint8_t *)(q + (size_t)arow(min(lane, count - 1)) * K)
                        : (const uint8_t *)(scales + (size_t)arow(min(lane, count - 1)) * B);
        else
            ssrc = wpair_src(64 * (wv - 4) + lane);
    } else {
        wj = wv, wh = 0;                          // nibble loads: block wv, rows lane and 64 + lane
        wsrc0 = W + ((size_t)min(T0, tiles - 1) * B * kTileRows + lane) * kChunk;
        wsrc1 = W + ((size_t)min(T0 + 1, tiles - 1) * B * kTileRows + lane) * kChunk;
        asrc = q + (size_t)arow(min(li, count - 1)) * K + 16 * g;  // block wv, half g, token li
        // Dword A: waves 0, 1 activation scale idx = 64 wv + lane (block
        // idx / 32, token idx % 32); waves 2, 3 weight-scale pair 64 (wv - 2)
        // + lane.  Dword B: waves 0, 1 pair 128 + 64 wv + lane; waves 2, 3 a
        // dummy (the pair of lane again, into the dummy dwords).
        if (wv < 2) {
            const int t = (64 * wv + lane) & 31;
            ssrc = DOTS ? (const uint8_t *)(q + (size_t)arow(min(t, count - 1)) * K)
                        : (const uint8_t *)(scales + (size_t)arow(min(t, count - 1)) * B);
            ssrc2 = wpair_src(128 + 64 * wv + lane);
        } else {
            ssrc = wpair_src(64 * (wv - 2) + lane);
            ssrc2 = ssrc;
        }
    }

    auto ring = [&](auto slot_tag) -> uint8_t * { return ring_lds + decltype(slot_tag)::value * kSlotB; };
    auto issue = [&](auto slot_tag, int h) {
        h = min(h, Hp - 1);  // past the last stage: the last stage again, into the free slot
        uint8_t *slot = ring(slot_tag);
        const int b0 = h * kStage;
        const size_t woff = (size_t)min(b0 + wj, B - 1) * kTileRows * kChunk;
        const size_t pair_off = (size_t)(b0 >> 3) * kTileRows * kChunk + 8 * ((b0 >> 2) & 1);
        if constexpr (TOK == 64) {
            __builtin_amdgcn_global_load_lds(wsrc0 + woff, (lds_ptr)(slot + (wj * 128 + 64 * wh) * 16), 16, 0, 0);
            __builtin_amdgcn_global_load_lds(asrc + (size_t)min(b0 + (wv >> 1), B - 1) * kQ4Block,
                                             (lds_ptr)(slot + Sh::kAct + wv * 1024), 16, 0, 0);
            const size_t soff = wv < 4 ? (size_t)min(b0 + wv, B - 1) * 4 : pair_off;
            __builtin_amdgcn_global_load_lds(ssrc + soff, (lds_ptr)(slot + Sh::kActScale + wv * 256), 4, 0, 0);
        } else {
            __builtin_amdgcn_global_load_lds(wsrc0 + woff, (lds_ptr)(slot + (wj * 128) * 16), 16, 0, 0);
            __builtin_amdgcn_global_load_lds(wsrc1 + woff, (lds_ptr)(slot + (wj * 128 + 64) * 16), 16, 0, 0);
            __builtin_amdgcn_global_load_lds(asrc + (size_t)min(b0 + wv, B - 1) * kQ4Block,
                                             (lds_ptr)(slot + Sh::kAct + wv * 1024), 16, 0, 0);
            if (wv < 2) {
                const int blk = (64 * wv + lane) >> 5;
                __builtin_amdgcn_global_load_lds(ssrc + (size_t)min(b0 + blk, B - 1) * 4,
                                                 (lds_ptr)(slot + Sh::kActScale + wv * 256), 4, 0, 0);
                __builtin_amdgcn_global_load_lds(ssrc2 + pair_off, (lds_ptr)(slot + Sh::kWScale + 512 + wv * 256),
                                                 4, 0, 0);
            } else {
                __builtin_amdgcn_global_load_lds(ssrc + pair_off, (lds_ptr)(slot + Sh::kWScale + (wv - 2) * 256),
                                                 4, 0, 0);
                __builtin_amdgcn_global_load_lds(ssrc2 + pair_off, (lds_ptr)(slot + Sh::kDummy), 4, 0, 0);
            }
        }
    };

    v16f acc, tot;
    v16i chain;
#pragma unroll
    for (int e = 0; e < 16; e++)
        tot[e] = 0.0f;
    const v16f zero_f = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    // This lane's LDS read addresses in slot 0 (the slot, block and half go
    // in the reads' immediate offsets).
    const uint32_t lds_base = (uint32_t)(uintptr_t)(lds_ptr)ring_lds;
    const uint32_t lds_w = lds_base + (32 * rg + li) * 16 + 8 * g;
    const uint32_t lds_a = lds_base + Sh::kAct + (32 * tg + li) * 16 + 8 * g;
    const uint32_t lds_dw = lds_base + Sh::kWScale + (32 * rg + li) * 8;
    const uint32_t lds_da = lds_base + Sh::kActScale + (32 * tg + li) * 4;

    // One stage: four blocks.  kFirst marks a stretch's first stage, whose
    // first block starts the chain from the bias and the stretch sum from
    // its product (x * s == fma(x, s, 0) but for the sign of a zero, which
    // the total's 0 + P cannot show).
    auto stage = [&](auto slot_tag, auto first_tag, int h) {
        constexpr int kSlot = decltype(slot_tag)::value;
        constexpr bool kFirst = decltype(first_tag)::value;
        wait_vmcnt<(kRing - 2) * Sh::kLoads>();  // stage h has landed (stages h + 1 .. may be in flight)
        __builtin_amdgcn_s_barrier();
        // into the slot stage h - 1 used; every wavefront is past it
        issue(std::integral_constant<int, (kSlot + kRing - 1) % kRing>{}, h + kRing - 1);
        constexpr int so = kSlot * kSlotB;
        // The operands of block j + 1 are read while block j is multiplied.
        uint2 wq_n, Bh_n, Bl_n;
        uint32_t dwh_n;
        float da_n;
        auto read = [&](auto j_tag) {
            constexpr int j = decltype(j_tag)::value;
            lds_read_block<so + j * 2048, so + (2 * j + 1) * TOK * 16, so + 2 * j * TOK * 16, so + 2 * j,
                           so + j * TOK * 4>(lds_w, lds_a, lds_dw, lds_da, wq_n, Bh_n, Bl_n, dwh_n, da_n);
        };
        read(std::integral_constant<int, 0>{});
        // front(j): block j's operands land, block j + 1's reads go out, and
        // block j's two MFMAs are issued; back(j): block j's chain
        // differences and fmas.
        v16f Sr[kStage];
        v16i Nr[kStage];
        auto front = [&](auto j_tag) {
            constexpr int j = decltype(j_tag)::value;
            // the previous block's work stays above this block's wait
            __builtin_amdgcn_sched_barrier(0);
            // the reads land; the registers pass through the wait so that
            // nothing touches them before it
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(wq_n), "+v"(Bh_n), "+v"(Bl_n), "+v"(dwh_n), "+v"(da_n));
            const uint2 wq = wq_n;
            const v4i Bv = {(int)Bh_n.x, (int)Bh_n.y, (int)Bl_n.x, (int)Bl_n.y};
            const uint32_t dwh = dwh_n;
            const float da = da_n;
            if constexpr (j + 1 < kStage)
                read(std::integral_constant<int, j + 1>{});
            // The scale outer product goes to the matrix core first: it does
            // not wait for the chain, and the integer MFMA queues behind it
            // while the nibbles are widened.  (Issued after the integer MFMA,
            // the compiler put the first chain difference ahead of it, so
            // the scales waited for the integers: two MFMA latencies a
            // block.)
            // a block past the row has weight scale 0 (the padding is zero):
            // fma(x, 0, acc) == acc
            Sr[j] = __builtin_amdgcn_mfma_f32_32x32x8f16(k04_operand(dwh), k04_operand(half2_bits_rtz(da)), zero_f, 0,
                                                          0, 0);
            // 16 (n - 8) in every byte: the high nibbles in place, the low
            // ones shifted up, the top bit flipped
            v4i A;
            A.x = (int)((wq.x & 0xF0F0F0F0u) ^ 0x80808080u);
            A.y = (int)((wq.y & 0xF0F0F0F0u) ^ 0x80808080u);
            A.z = (int)(((wq.x << 4) & 0xF0F0F0F0u) ^ 0x80808080u);
            A.w = (int)(((wq.y << 4) & 0xF0F0F0F0u) ^ 0x80808080u);
            v16i prev;
            if constexpr (kFirst && j == 0) {
                // written afresh each stretch (a resident copy would cost 16
                // registers and a wavefront per SIMD)
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    int bias;
                    asm volatile("v_mov_b32 %0, %1" : "=v"(bias) : "i"(kChainBias));
                    prev[e] = bias;
                }
            } else if constexpr (j == 0) {
                prev = chain;
            } else {
                prev = Nr[j - 1];
            }
            Nr[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, Bv, prev, 0, 0, 0);
        };
        auto back = [&](auto j_tag) {
            constexpr int j = decltype(j_tag)::value;
            constexpr bool start = kFirst && j == 0;
#pragma unroll
            for (int e = 0; e < 16; e++) {
                // half the block's isum, exactly (a stretch's first block
                // subtracts the bias as a literal: its MFMA then runs in
                // place, with no copy of the bias kept for the difference)
                int pb;
                if constexpr (start)
                    pb = kChainBias;
                else if constexpr (j == 0)
                    pb = chain[e];
                else
                    pb = Nr[j - 1][e];
                const float x = __int_as_float(Nr[j][e]) - __int_as_float(pb);
                acc[e] = start ? x * Sr[j][e] : fmaf(x, Sr[j][e], acc[e]);
                if constexpr (DOTS) {
                    const int b = h * kStage + j, tt = 32 * tg + li;
                    const int n = T0 * kTileRows + 32 * rg + 8 * (e >> 2) + 4 * g + (e & 3);
                    if (b < B && tt < count && n >= row_start && n < row_end)
                        dots[((size_t)orow(tt) * (row_end - row_start) + (n - row_start)) * B + b] = (int)(2.0f * x);
                }
            }
        };
        if constexpr (kPipe) {
            // block j + 1's MFMAs go out before block j's differences, which
            // then run while the matrix core works on them
            front(std::integral_constant<int, 0>{});
            unroll<0, kStage>([&](auto j_tag) {
                constexpr int j = decltype(j_tag)::value;
                if constexpr (j + 1 < kStage)
                    front(std::integral_constant<int, j + 1>{});
                __builtin_amdgcn_sched_barrier(0);
                back(j_tag);
            });
        } else {
            unroll<0, kStage>([&](auto j_tag) {
                front(j_tag);
                __builtin_amdgcn_sched_barrier(0);
                back(j_tag);
            });
        }
        chain = Nr[kStage - 1];
        // the stage's sums are complete here, not sunk past the next barrier
#pragma unroll
        for (int e = 0; e < 16; e++)
            asm volatile("" : "+v"(acc[e]));
    };

    auto fold = [&]() {  // a stretch is two stages
#pragma unroll
        for (int e = 0; e < 16; e++)
            tot[e] = tot[e] + acc[e];
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;
    if constexpr (kRing == 3) {
        issue(S0{}, 0);
        issue(S1{}, 1);
        for (int h = 0;; h += 6) {  // three stretches: the ring comes round to slot 0
            stage(S0{}, std::true_type{}, h);
            stage(S1{}, std::false_type{}, h + 1);
            fold();
            if (h + 2 >= Hp)
                break;
            stage(S2{}, std::true_type{}, h + 2);
            stage(S0{}, std::false_type{}, h + 3);
            fold();
            if (h + 4 >= Hp)
                break;
            stage(S1{}, std::true_type{}, h + 4);
            stage(S2{}, std::false_type{}, h + 5);
            fold();
            if (h + 6 >= Hp)
                break;
        }
    } else {
        using S3 = std::integral_constant<int, 3>;
        issue(S0{}, 0);
        issue(S1{}, 1);
        issue(S2{}, 2);
        for (int h = 0;; h += 4) {  // two stretches: the ring comes round to slot 0
            stage(S0{}, std::true_type{}, h);
            stage(S1{}, std::false_type{}, h + 1);
            fold();
            if (h + 2 >= Hp)
                break;
            stage(S2{}, std::true_type{}, h + 2);
            stage(S3{}, std::false_type{}, h + 3);
            fold();
            if (h + 4 >= Hp)
                break;
        }
    }
    wait_vmcnt<0>();  // the trailing loads land before the workgroup ends
    const int t = 32 * tg + li;
    if constexpr (EPI == 1) {
        __syncthreads();  // every wavefront is past its last operand reads
        float *xch = (float *)ring_lds;  // [wavefront pair][lane][17]
        const int pair = wv >> 1;
        if (rg & 1) {
#pragma unroll
            for (int e = 0; e < 16; e++)
                xch[(pair * 64 + lane) * 17 + e] = tot[e];
        }
        __syncthreads();
        const int tile = T0 + (rg >> 1);
        if (!(rg & 1) && tile * kTileRows < row_end) {
            const int F = row_end >> 1;  // outputs a token
            float v[16];
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const float gt = tot[e], u = xch[(pair * 64 + lane) * 17 + e];
                const float ex = ggml_expf(-gt);
                const float den = 1.0f + ex;
                const float sl = gt / den;
                v[e] = sl * u;
            }
            float peak = fabsf(v[0]);
#pragma unroll
            for (int e = 1; e < 16; e++)
                peak = fmaxf(peak, fabsf(v[e]));
            peak = fmaxf(peak, __shfl_xor(peak, 32, 64));  // the token's other 16 outputs
            int32_t n[16];
            float stored = 0.0f;
            if (peak == 0.0f) {
#pragma unroll
                for (int e = 0; e < 16; e++)
                    n[e] = 0;
            } else {
                const float scale = __fdiv_rn(peak, 127.0f);
                const float inverse = __fdiv_rn(127.0f, peak);
                stored = half_bits_to_float(float_to_half_bits(scale));
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int32_t k = nearest_int(v[e] * inverse);
                    n[e] = k > 127 ? 127 : (k < -128 ? -128 : k);
                }
            }
            int32_t sum = 0;
#pragma unroll
            for (int e = 0; e < 16; e++)
                sum += n[e];
            sum += __shfl_xor(sum, 32, 64);
            if (t < count) {
                const int row = orow(t);
                // element e is output 8 (e / 4) + 4 g + e % 4 of the tile's 32
#pragma unroll
                for (int e4 = 0; e4 < 4; e4++) {
                    const uint32_t w = (uint32_t)(n[4 * e4] & 0xFF) | ((uint32_t)(n[4 * e4 + 1] & 0xFF) << 8) |
                                       ((uint32_t)(n[4 * e4 + 2] & 0xFF) << 16) |
                                       ((uint32_t)(n[4 * e4 + 3] & 0xFF) << 24);
                    *(uint32_t *)(mq + (size_t)row * F + tile * 32 + 8 * e4 + 4 * g) = w;
                }
                if (g == 0) {
                    ms[(size_t)row * (F >> 5) + tile] = stored;
                    mqs[(size_t)row * (F >> 5) + tile] = sum;
                }
            }
        }
    } else if constexpr (EPI == 2) {
        static_assert(TOK == 32 && !GROUPED && !DOTS, "the Q|K|V epilogue is a dense 32-token form");
        qkv_rope_epilogue(tot, ring_lds, qr, T0, rg, li, g, first, count);
    } else if (!DOTS && t < count) {
        float *yr = y + (size_t)orow(t) * ldy;
        const int nb = T0 * kTileRows + 32 * rg;  // the wavefront's first row
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int n = nb + 8 * (e >> 2) + 4 * g + (e & 3);
            if (n >= row_start && n < row_end)
                yr[n] = bias ? tot[e] + bias[n] : tot[e];
        }
    }
}

}  // namespace

namespace {
// The dense product's grid and launch (EPI 0: y = the product; EPI 1: the
// SwiGLU + Q8_0 epilogue into mq / ms / mqs).
template <int EPI>
int launch_dense(gx_ctx *ctx, const gx_weight *w, const uint8_t *mat, const int8_t *q, const float *scales, int M,
                 int row_start, int row_end, const float *bias, float *y, int ldy, int32_t *dots, int8_t *mq,
                 float *ms, int32_t *mqs) {
    // the widened weights are signed: no recentring term, so no qsum
    const int tile0 = row_start / kTileRows;
    const int tiles = (row_end + kTileRows - 1) / kTileRows - tile0;
    const Groups none{nullptr, nullptr, 1, 0};
    const int pairs = (tiles + 1) / 2;
    // Up to 1024 tokens, 32-token workgroups: twice as many of them to fill
    // the CUs (config 2's 9728 x 2560 in a graph over rotating copies: M = 64
    // 25.0 -> 20.1 us, M = 512 62.0 -> 56.1 us; M = 2048 195 against 198 us
    // keeps 64), unless the 64-token form has a thousand workgroups anyway
    // (config 3's Gate|Up, 19456 rows, at a 512-token prompt: the prefill
    // 9.93 -> 9.80 ms).  Between 256 and 512 of them, though, some CUs take
    // two 32-token workgroups to the others' one, where the 64-token form
    // fits in one round (config 3's O and Down, 2560 rows, at a 512-token
    // prompt: 35.1 -> 33.1 and 71.0 -> 63.6 us).  The per-token arithmetic
    // is the same either way.
    const int w32 = pairs * ((M + 31) / 32);
    const int tok = (M <= 1024 && pairs * ((M + kDmaTok - 1) / kDmaTok) < 1000 && (w32 <= 256 || w32 > 512))
                        ? 32
                        : kDmaTok;
    const int groups = (M + tok - 1) / tok;
    // XCD order for matrices of at least eight row pairs (every XCD some).
    const int xp = pairs >= 8 ? pairs : 0;
    const dim3 grid = xp ? dim3((unsigned)(8 * ((pairs + 7) / 8) * groups)) : dim3((unsigned)pairs, (unsigned)groups);
#define GX_DMA_LAUNCH(TK, NT, DD)                                                                                   \
    q4_0_gemm_dma_kernel<TK, false, DD, EPI><<<grid, NT, 0, ctx->stream>>>(                                         \
        mat, w->plane0_bytes, w->blocks, w->dchunks, q, scales, w->cols, M, w->tiles, tile0, row_start, row_end,     \
        bias, y, ldy, DD ? dots : nullptr, none, xp, mq, ms, mqs, QkvRopeArgs{})
    if constexpr (EPI == 1) {
        if (tok == 32)
            GX_DMA_LAUNCH(32, 256, false);
        else
            GX_DMA_LAUNCH(64, 512, false);
    } else {
        if (tok == 32 && dots)
            GX_DMA_LAUNCH(32, 256, true);
        else if (tok == 32)
            GX_DMA_LAUNCH(32, 256, false);
        else if (dots)
            GX_DMA_LAUNCH(64, 512, true);
        else
            GX_DMA_LAUNCH(64, 512, false);
    }
#undef GX_DMA_LAUNCH
    return check_launch("q4_0_gemm");
}
}  // namespace

int launch_q4_0_gemm(gx_ctx *ctx, const gx_weight *w, const uint8_t *mat, const int8_t *q, const float *scales,
                     int M, int row_start, int row_end, const float *bias, float *y, int ldy, int32_t *dots) {
    return launch_dense<0>(ctx, w, mat, q, scales, M, row_start, row_end, bias, y, ldy, dots, nullptr, nullptr,
                           nullptr);
}

int launch_q4_0_gemm_swiglu(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const float *scales, int M,
                            int8_t *mq, float *ms, int32_t *mqs) {
    return launch_dense<1>(ctx, w, w->dev, q, scales, M, 0, w->rows, nullptr, nullptr, 0, nullptr, mq, ms, mqs);
}

int launch_q4_0_gemm_qkv_rope(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const float *scales, int M,
                              const QkvRopeArgs &a) {
    // the 32-token form always (its epilogue's shape), in XCD order
    const int pairs = (w->tiles + 1) / 2, groups = (M + 31) / 32;
    const Groups none{nullptr, nullptr, 1, 0};
    const int xp = pairs >= 8 ? pairs : 0;
    const dim3 grid = xp ? dim3((unsigned)(8 * ((pairs + 7) / 8) * groups)) : dim3((unsigned)pairs, (unsigned)groups);
    q4_0_gemm_dma_kernel<32, false, false, 2><<<grid, 256, 0, ctx->stream>>>(
        w->dev, w->plane0_bytes, w->blocks, w->dchunks, q, scales, w->cols, M, w->tiles, 0, 0, w->rows, nullptr,
        nullptr, 0, nullptr, none, xp, nullptr, nullptr, nullptr, a);
    return check_launch("q4_0_gemm qkv_rope");
}

int launch_q4_0_gemm_grouped(gx_ctx *ctx, const gx_weight *w, const int32_t *work, int max_items,
                             const int32_t *sorted, int act_div, const int8_t *q, const float *scales, float *y,
                             int ldy, int32_t *dots) {
    // Items of at most kGroupTok units (the sort's tile), 32 tokens a workgroup.
    const dim3 grid((unsigned)((w->tiles + 1) / 2), (unsigned)max_items);
    const Groups grp{work, sorted, act_div, w->matrix_bytes};
    if (dots)
        q4_0_gemm_dma_kernel<32, true, true><<<grid, 256, 0, ctx->stream>>>(
            w->dev, w->plane0_bytes, w->blocks, w->dchunks, q, scales, w->cols, 0, w->tiles, 0, 0, w->rows, nullptr,
            y, ldy, dots, grp, 0, nullptr, nullptr, nullptr, QkvRopeArgs{});
    else
        q4_0_gemm_dma_kernel<32, true, false><<<grid, 256, 0, ctx->stream>>>(
            w->dev, w->plane0_bytes, w->blocks, w->dchunks, q, scales, w->cols, 0, w->tiles, 0, 0, w->rows, nullptr,
            y, ldy, nullptr, grp, 0, nullptr, nullptr, nullptr, QkvRopeArgs{});
    return check_launch("q4_0_gemm_grouped");
}
}  // namespace gx

namespace gx {

int launch_q4_0_gemm_f16(gx_ctx *ctx, const gx_weight *w, const uint8_t *mat, const uint16_t *q16,
                         const float *scales, int M, int row_start, int row_end, const float *bias, float *y, int ldy,
                         int32_t *dots) {
    const int tile0 = row_start / kTileRows;
    const unsigned tiles = (unsigned)((row_end + kTileRows - 1) / kTileRows - tile0);
    const int groups = (M + 31) / 32;
    // Token groups per workgroup: wider workgroups share the widening of the
    // weights among more tokens; narrower ones keep more workgroups in flight.
    const int nwt = groups <= 32 ? 2 : 4;
    const dim3 grid(tiles, (unsigned)((groups + nwt - 1) / nwt));
#define GX_F16_LAUNCH(N)                                                                                             \
    do {                                                                                                             \
        if (dots)                                                                                                    \
            q4_0_gemm_f16_kernel<N, true><<<grid, 64 * N, 0, ctx->stream>>>(                                         \
                mat, w->plane0_bytes, w->blocks, w->dchunks, q16, scales, M, tile0, row_start, row_end, bias, y, ldy, \
                dots);                                                                                               \
        else                                                                                                         \
            q4_0_gemm_f16_kernel<N, false><<<grid, 64 * N, 0, ctx->stream>>>(                                        \
                mat, w->plane0_bytes, w->blocks, w->dchunks, q16, scales, M, tile0, row_start, row_end, bias, y, ldy, \
                dots);                                                                                               \
    } while (0)
    if (nwt == 2)
        GX_F16_LAUNCH(2);
    else
        GX_F16_LAUNCH(4);
#undef GX_F16_LAUNCH
    return check_launch("q4_0_gemm_f16");
}

}  // namespace gx
