// gx_q4_0.hip - the Q4_0 x Q8_0 matrix-vector product (decode, M <= 8).
//
// This is golem's matVecPackedQ4_0Rows / matVecQ4_0Rows (nn/pack_q4_0.go:
// 159-221, nn/dot_q4_0.go:168-270) rebuilt for a bandwidth-bound GPU kernel.
//
// Canonical order.  Every Q4_0 kernel in this library (these and the MFMA
// products) computes a row's value the same way, so that a column's result
// does not depend on how many columns were in the batch or which kernel ran:
//   isum_b = sum_j (n_j - 8) * q_j                      exact int32
//   s_b    = d_w[b] * d_a[b]                             one fp32 product
//   P_s    = fma(float(isum_b), s_b, P_s) for the blocks b of stretch s,
//            in order, starting from +0 (a stretch is 8 blocks)
//   y      = ((0 + P_0) + P_1) + ...  (+ bias)
// golem sums the same integers with an unsigned nibble and a cancelling
// correction term (nn/dot_q4_0.go:64-66); the two agree to rounding.
//
// Five kernels:
//   q4_0_matvec_kernel<NC, UNITS>  a workgroup owns one 64-row tile, a
//       wavefront whole stretches, a lane one row.  The stretch's activation
//       is the same for all 64 lanes, so it is read with scalar loads into
//       SGPRs and fed to v_dot4 from there.  NC columns (8, 4, 2, 1) share
//       one weight read; UNITS runs one expert of a stack per unit (MoE).
//   q4_0_matvec_lds_kernel<R, IT>  one column (M = 1) of a matrix with few
//       tiles: a workgroup owns R rows (a quarter tile) and all their
//       stretches, lane l being row l % R and stretch slot l / R, so that
//       four times as many workgroups pull weights with no cross-workgroup
//       sum.  The stretches of a wavefront differ, so the activation is
//       staged in LDS first.
//   q4_0_matvec_fused_kernel<EPI, DB>  one position whose activation the
//       product makes itself: x + add, RMSNormPlain(gain, eps) and Q8_0 (a
//       block's pre-norm, qwen/block.go:45-52, 59-68), each wavefront
//       quantising the stretch it multiplies into SGPRs; EPI 1 applies
//       SwiGLU to a tile of gate and up rows interleaved by 32 and writes the
//       Q8_0 block of its 32 outputs (qwen/block.go:82-90, nn/swiglu.go:
//       77-82).
//   q4_0_matvec_cols_kernel<R, NC>  2..8 columns: every column's
//       activation staged in LDS at once, on whole, half or quarter tiles.
//   q4_0_matvec_fused_lds_kernel<R>  the same pre-norm product without the
//       SwiGLU epilogue on sub-tiles of R rows (lanes as in the LDS kernel),
//       for a matrix whose whole tiles would leave most CUs idle.
//
// The norm's prologue is norm_stage + norm_tree_wave (gx_device.hpp): two
// barriers where a tree halved through LDS took five (Q|K|V 6.82 -> 6.56 us,
// Gate|Up 11.11 -> 10.78 us in a graph of launches over rotating copies).
//
// Where the weight loads go out.  Measured on the box (a HIP graph of
// launches over rotating weight copies, config 3's shapes): issuing every
// weight load at a kernel's start, ahead of its prologue, is slower, not
// faster -- Gate|Up with the norm 11.0 -> 15.7 us: a workgroup dispatched
// late finds its activation loads queued behind the weight streams of the
// workgroups dispatched before it.  So each kernel fetches what its prologue
// needs first and the weights after the prologue's loads have landed.
//
// Per-block integer export: each kernel is compiled twice from the same
// source, DOTS false for the product and DOTS true for the parity checks,
// which also writes the isum of every (column, row, block) it computes to
// dots[c][r - row_start][b] and stores no output row.  (A run-time switch
// instead -- one uniform branch per block -- cost the product 0.2-0.5 us a
// launch on the box.)
#include "gx_device.hpp"
#include "gx_internal.hpp"

namespace gx {
namespace {

// With UNITS, blockIdx.y is a unit of a mixture-of-experts batch: unit u
// multiplies expert unit_expert[u] of a stack (matrices matrix_bytes apart)
// by activation row u / act_div, into output row u.
template <int NC, bool UNITS, bool DOTS>
__global__ __launch_bounds__(1024) void q4_0_matvec_kernel(
    const uint8_t *__restrict__ W, size_t plane0_bytes, int B, int DC, const int8_t *__restrict__ q,
    const float *__restrict__ scales, const int32_t *__restrict__ qsum, int K, int tile0, int row_start,
    int row_end, const float *__restrict__ bias, float *__restrict__ y, int ldy,
    const int32_t *__restrict__ unit_expert, size_t matrix_bytes, int act_div, int experts,
    int32_t *__restrict__ dots) {
    extern __shared__ float part[];  // [S][NC][64]
    const int S = (B + kStretch - 1) / kStretch;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nwaves = blockDim.x >> 6;
    const int tile = tile0 + blockIdx.x;
    const int nrows = row_end - row_start;
    if (UNITS) {
        const int u = blockIdx.y;
        const int e = unit_expert[u];
        if (e < 0 || e >= experts) {  // an id out of range reads nothing and yields NaN
            const int row = tile * kTileRows + lane;
            if (threadIdx.x < 64 && row < row_end)
                y[(size_t)u * ldy + row] = __builtin_nanf("");
            return;
        }
        W += (size_t)e * matrix_bytes;
        const int a = u / act_div;
        q += (size_t)a * K;
        scales += (size_t)a * B;
        qsum += (size_t)a * B;
        y += (size_t)u * ldy;
        if (DOTS)
            dots += (size_t)u * nrows * B;
    }
    const uint8_t *qs_row = W + ((size_t)tile * B * kTileRows + lane) * kChunk;
    const uint8_t *d_row = W + plane0_bytes + ((size_t)tile * DC * kTileRows + lane) * kChunk;

    for (int s = wave; s < S; s += nwaves) {
        const int b0 = s * kStretch;
        const int nb = min(kStretch, B - b0);
        // Unconditional loads: past the last block a load repeats the last
        // block (in bounds) and its product is skipped, so the compiler issues
        // all nine loads back to back instead of one per guarded branch.
        uint4 wq[kStretch];
#pragma unroll
        for (int j = 0; j < kStretch; j++)
            wq[j] = load_stream(qs_row + (size_t)min(b0 + j, B - 1) * kTileRows * kChunk);
        const uint4 dch = *(const uint4 *)(d_row + (size_t)s * kTileRows * kChunk);
        float p[NC];
#pragma unroll
        for (int c = 0; c < NC; c++)
            p[c] = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; c++) {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                // Four blocks' activation at a time, loaded before any use.
                int4 a0[4], a1[4];
                int32_t qs[4];
                float sa[4];
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    const int b = min(b0 + 4 * h + jj, B - 1);
                    const int4 *a = (const int4 *)(q + (size_t)c * K + (size_t)b * kQ4Block);
                    a0[jj] = a[0];
                    a1[jj] = a[1];
                    qs[jj] = qsum[(size_t)c * B + b];
                    sa[jj] = scales[(size_t)c * B + b];
                }
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    const int j = 4 * h + jj;
                    if (j < nb) {
                        const int32_t isum = q4_0_block_isum(wq[j], a0[jj], a1[jj], qs[jj]);
                        const float sc = chunk_half(dch, j) * sa[jj];
                        p[c] = fmaf((float)isum, sc, p[c]);
                        if (DOTS) {
                            const int row = tile * kTileRows + lane;
                            if (row >= row_start && row < row_end)
                                dots[((size_t)c * nrows + (row - row_start)) * B + b0 + j] = isum;
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int c = 0; c < NC; c++)
            part[(s * NC + c) * kTileRows + lane] = p[c];
    }
    __syncthreads();
    const int row = tile * kTileRows + lane;
    if (wave == 0 && row >= row_start && row < row_end) {
#pragma unroll
        for (int c = 0; c < NC; c++) {
            float acc = 0.0f;
            for (int s = 0; s < S; s++)
                acc = acc + part[(s * NC + c) * kTileRows + lane];
            if (bias)
                acc = acc + bias[row];
            if (!DOTS)
                y[(size_t)c * ldy + row] = acc;
        }
    }
}

// ---- one column, activation in LDS ------------------------------------------

constexpr int kActRegs = 4;  // staged 16-byte activation pieces per thread

// LDS layout (bytes): part [S*R] floats, q [K] int8, scales [B], qsum [B].
__host__ __device__ inline size_t lds_part_bytes(int S, int R) { return ((size_t)S * R * 4 + 15) & ~(size_t)15; }
__host__ __device__ inline size_t lds_act_bytes(int K, int B) { return ((size_t)K + (size_t)B * 8 + 15) & ~(size_t)15; }

// IT stretches a lane (IT = 2 when one pass of at most 16 wavefronts does
// not cover the row).
template <int R, int IT, bool DOTS>
__global__ __launch_bounds__(1024) void q4_0_matvec_lds_kernel(
    const uint8_t *__restrict__ W, size_t plane0_bytes, int B, int DC, const int8_t *__restrict__ q,
    const float *__restrict__ scales, const int32_t *__restrict__ qsum, int group0, int row_start, int row_end,
    const float *__restrict__ bias, float *__restrict__ y, int32_t *__restrict__ dots) {
    constexpr int kSlots = kTileRows / R;  // stretch slots per wavefront
    extern __shared__ __align__(16) uint8_t lds_raw[];
    const int K = B * kQ4Block;
    const int S = (B + kStretch - 1) / kStretch;
    float *part = (float *)lds_raw;
    int8_t *qa = (int8_t *)(lds_raw + lds_part_bytes(S, R));
    float *sa = (float *)(qa + K);
    int32_t *qsa = (int32_t *)(sa + B);
    const int tid = threadIdx.x, nt = blockDim.x;
    const int lane = tid & 63, wave = tid >> 6, nwaves = nt >> 6;
    const int g = group0 + blockIdx.x;
    const int tile = g / kSlots, r = (g - tile * kSlots) * R + lane % R;
    const int row = tile * kTileRows + r;
    const bool in_range = row >= row_start && row < row_end;

    // The activation: every load in flight together (indices past the end
    // clamped, the values never stored), then into LDS.
    {
        const int n16 = K / 16;
        int4 qv[kActRegs];
        float sv[kActRegs];
        int32_t qsv[kActRegs];
#pragma unroll
        for (int k = 0; k < kActRegs; k++)
            qv[k] = ((const int4 *)q)[min(tid + k * nt, n16 - 1)];
#pragma unroll
        for (int k = 0; k < kActRegs; k++) {
            sv[k] = scales[min(tid + k * nt, B - 1)];
            qsv[k] = qsum[min(tid + k * nt, B - 1)];
        }
#pragma unroll
        for (int k = 0; k < kActRegs; k++) {
            const int i = tid + k * nt;
            if (i < n16)
                ((int4 *)qa)[i] = qv[k];
            if (i < B) {
                sa[i] = sv[k];
                qsa[i] = qsv[k];
            }
        }
    }
    // The weights: IT stretches, 8 nibble chunks and one scale chunk each
    // (past the last block: the last one again).
    const uint8_t *qs_row = W + ((size_t)tile * B * kTileRows + r) * kChunk;
    const uint8_t *d_row = W + plane0_bytes + ((size_t)tile * DC * kTileRows + r) * kChunk;
    int st[IT];
    uint4 wq[IT][kStretch], dch[IT];
#pragma unroll
    for (int it = 0; it < IT; it++) {
        st[it] = it * nwaves * kSlots + wave * kSlots + lane / R;
        const int sc = min(st[it], S - 1);
#pragma unroll
        for (int j = 0; j < kStretch; j++)
            wq[it][j] = load_stream(qs_row + (size_t)min(sc * kStretch + j, B - 1) * kTileRows * kChunk);
        dch[it] = *(const uint4 *)(d_row + (size_t)sc * kTileRows * kChunk);
    }
    lds_barrier();

    // Each lane's stretches, summed from +0 in block order.
#pragma unroll
    for (int it = 0; it < IT; it++) {
        const int s = st[it];
        if (s < S) {
            const int b0 = s * kStretch;
            const int nb = min(kStretch, B - b0);
            float p = 0.0f;
#pragma unroll
            for (int j = 0; j < kStretch; j++) {
                if (j < nb) {
                    const int b = b0 + j;
                    const int4 *ap = (const int4 *)(qa + (size_t)b * kQ4Block);
                    const int32_t isum = q4_0_block_isum(wq[it][j], ap[0], ap[1], qsa[b]);
                    const float scl = chunk_half(dch[it], j) * sa[b];
                    p = fmaf((float)isum, scl, p);
                    if (DOTS && in_range)
                        dots[(size_t)(row - row_start) * B + b] = isum;
                }
            }
            part[s * R + lane % R] = p;
        }
    }
    lds_barrier();

    // The stretch sums in stretch order from 0: the one-tile kernel's sum,
    // bit for bit.
    if (!DOTS && wave == 0 && lane < R && in_range) {
        float acc = 0.0f;
        for (int t = 0; t < S; t++)
            acc = acc + part[t * R + lane];
        y[row] = bias ? acc + bias[row] : acc;
    }
}

// NC columns (2 <= M <= 8 as the product groups them) on tiles of R rows:
// the whole activation of the NC columns is staged in LDS first (one round
// trip; the whole-tile kernel's per-block scalar loads, NC of them in a row
// per stretch, were a chain of cache round trips), and the R-row shape
// spreads a matrix of few tiles over more CUs (golem's lock-step slots read
// O and Down, 40 tiles each, at M = 8).  Lane l is row l % R and stretch
// slot l / R; it sums its stretch for every column from +0 in block order,
// and thread (c, r) then adds column c's stretch sums of row r in order:
// each column is the one-column kernels' bit for bit.
constexpr int kColRegs = 8;  // staged 16-byte activation pieces per thread per pass

__host__ __device__ inline size_t cols_lds_bytes(int S, int R, int NC, int K, int B) {
    return lds_part_bytes(S * NC, R) + lds_act_bytes(NC * K, NC * B);
}

// EPI 1 (R = 64, every row): the rows are gate and up interleaved by 32 as
// for q4_0_matvec_fused_kernel<1>; wavefront w takes column c = w (then
// w + nwaves ..): lane l sums its row, and the tile's 32 outputs
// silu(gate) * up go to their Q8_0 block in mq/ms/mqs [NC][rows / 2], the
// fused kernel's epilogue bit for bit.
template <int R, int NC, bool DOTS, int EPI = 0>
__global__ __launch_bounds__(1024) void q4_0_matvec_cols_kernel(
    const uint8_t *__restrict__ W, size_t plane0_bytes, int B, int DC, const int8_t *__restrict__ q,
    const float *__restrict__ scales, const int32_t *__restrict__ qsum, int group0, int row_start, int row_end,
    const float *__restrict__ bias, float *__restrict__ y, int ldy, int32_t *__restrict__ dots,
    int8_t *__restrict__ mq = nullptr, float *__restrict__ ms = nullptr, int32_t *__restrict__ mqs = nullptr) {
    static_assert(EPI == 0 || R == kTileRows, "the SwiGLU epilogue takes whole tiles");
    constexpr int kSlots = kTileRows / R;
    extern __shared__ __align__(16) uint8_t lds_raw[];
    const int K = B * kQ4Block;
    const int S = (B + kStretch - 1) / kStretch;
    float *part = (float *)lds_raw;  // [S][NC][R]
    int8_t *qa = (int8_t *)(lds_raw + lds_part_bytes(S * NC, R));  // [NC][K]
    float *sa = (float *)(qa + (size_t)NC * K);                     // [NC][B]
    int32_t *qsa = (int32_t *)(sa + NC * B);                         // [NC][B]
    const int tid = threadIdx.x, nt = blockDim.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int g = group0 + blockIdx.x;
    const int tile = g / kSlots, r = (g - tile * kSlots) * R + lane % R;
    const int row = tile * kTileRows + r;
    const bool in_range = row >= row_start && row < row_end;
    const int st = wave * kSlots + lane / R;  // this lane's stretch

    // The activation of the NC columns first (rows q[c] are consecutive),
    // every load of a pass in flight together, into LDS; then the weights.
    // (Weights first was slower: the activation's loads queue behind them --
    // one column, Down 6.50 -> 7.38 us, O 4.42 -> 4.70 us.)
    const int n16 = NC * K / 16, nb = NC * B;
    for (int base = 0; base < max(n16, nb); base += kColRegs * nt) {
        int4 qv[kColRegs];
        float sv[kColRegs];
        int32_t qsv[kColRegs];
#pragma unroll
        for (int k = 0; k < kColRegs; k++) {
            const int i = base + tid + k * nt;
            qv[k] = ((const int4 *)q)[min(i, n16 - 1)];
            sv[k] = scales[min(i, nb - 1)];
            qsv[k] = qsum[min(i, nb - 1)];
        }
#pragma unroll
        for (int k = 0; k < kColRegs; k++) {
            const int i = base + tid + k * nt;
            if (i < n16)
                ((int4 *)qa)[i] = qv[k];
            if (i < nb) {
                sa[i] = sv[k];
                qsa[i] = qsv[k];
            }
        }
    }
    const uint8_t *qs_row = W + ((size_t)tile * B * kTileRows + r) * kChunk;
    const uint8_t *d_row = W + plane0_bytes + ((size_t)tile * DC * kTileRows + r) * kChunk;
    uint4 wq[kStretch], dch;
    if (wave * kSlots < S) {  // wavefronts past the last stretch load nothing
        const int sc = min(st, S - 1);
#pragma unroll
        for (int j = 0; j < kStretch; j++)
            wq[j] = load_stream(qs_row + (size_t)min(sc * kStretch + j, B - 1) * kTileRows * kChunk);
        dch = *(const uint4 *)(d_row + (size_t)sc * kTileRows * kChunk);
    }
    lds_barrier();

    if (st < S) {
        const int b0 = st * kStretch;
        const int nbk = min(kStretch, B - b0);
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const int8_t *qc = qa + (size_t)c * K;
            float p = 0.0f;
#pragma unroll
            for (int j = 0; j < kStretch; j++) {
                if (j < nbk) {
                    const int b = b0 + j;
                    const int4 *ap = (const int4 *)(qc + (size_t)b * kQ4Block);
                    const int32_t isum = q4_0_block_isum(wq[j], ap[0], ap[1], qsa[c * B + b]);
                    const float scl = chunk_half(dch, j) * sa[c * B + b];
                    p = fmaf((float)isum, scl, p);
                    if (DOTS && in_range)
                        dots[((size_t)c * (row_end - row_start) + (row - row_start)) * B + b] = isum;
                }
            }
            part[(st * NC + c) * R + lane % R] = p;
        }
    }
    lds_barrier();
    if (!DOTS && EPI == 1) {
        const int F = row_end / 2;  // the SwiGLU's width: gate and up rows in equal number
        for (int c = wave; c < NC; c += nt >> 6) {
            float acc = 0.0f;
            for (int t = 0; t < S; t++)
                acc = acc + part[(t * NC + c) * kTileRows + lane];
            // lane l < 32: gate 32 * tile + l; lane l + 32: its up
            const float u = __shfl_down(acc, 32, 64);
            const float gt = acc;
            const float ex = ggml_expf(-gt);
            const float den = 1.0f + ex;
            const float sl = gt / den;
            const float v = sl * u;
            float stored;
            int32_t sm;
            const int32_t nq = q8_0_lane(v, &stored, &sm);
            if (lane < 32) {
                mq[(size_t)c * F + (size_t)tile * 32 + lane] = (int8_t)nq;
                if (lane == 0) {
                    ms[(size_t)c * (F / kQ4Block) + tile] = stored;
                    mqs[(size_t)c * (F / kQ4Block) + tile] = sm;
                }
            }
        }
    } else if (!DOTS) {
        for (int pr = tid; pr < NC * R; pr += nt) {
            const int c = pr / R, rr = pr - c * R;
            const int orow = tile * kTileRows + (g - tile * kSlots) * R + rr;
            if (orow >= row_start && orow < row_end) {
                float acc = 0.0f;
                for (int t = 0; t < S; t++)
                    acc = acc + part[(t * NC + c) * R + rr];
                if (bias)
                    acc = acc + bias[orow];
                y[(size_t)c * ldy + orow] = acc;
            }
        }
    }
}

// ---- few columns on the matrix cores ---------------------------------------
//
// 2..16 columns (lock-step decode of several conversations, short batches):
// the per-block integers come from v_mfma_i32_16x16x32_i8, 16 weight rows
// against the same block of 16 columns, instead of from per-lane dot
// products -- the multi-column kernel above spends ~25 vector instructions
// per (row, column, block) and is VALU-bound from about 4 columns on
// (config 3's Gate|Up at 8 columns: 28 MB in 26.8 us).
//
// Operands (one 16x16x32 MFMA a block): lane l holds row/column l % 16 and
// inputs 8 (l / 16) .. 8 (l / 16) + 7 of the block.  A Q4_0 chunk holds
// inputs 0..15 in the low nibbles of bytes 0..15 and 16..31 in the high
// ones, so lane group k = l / 16 reads bytes 8 (k & 1) .. + 7 of its row's
// chunk and takes the low (k < 2) or high nibbles, widened in place to
// 16 (n - 8) as a signed byte.  The accumulators chain through a stretch
// from the bits of kMfmaChainBias: read as fp32, each output is that bias plus
// the stretch's running isum exactly (the ulp in [2^19, 2^20) is 1/16 and a
// stretch's running sum is at most 8 * 32 * 8 * 128 = 2^18 in magnitude),
// so the block's isum is the difference of two consecutive outputs, one
// full-rate subtraction.  The scale product d_w * d_a of the tile is an
// outer product of two fp16 vectors, exact in fp32: v_mfma_f32_16x16x16f16
// with the two vectors at input 0 and zeros elsewhere.  The vector ALU is
// left with one subtraction and one fma per output per block, in the
// canonical order, so a column's values are those of every other kernel
// bit for bit.
//
// Work: a workgroup owns RG row groups of 16 rows (R = 16 RG rows of one
// tile); a unit is (row group, stretch), and wavefront w takes units w,
// w + nwaves, ...  Each unit's stretch sum P_s for its 16 rows x 16 columns
// goes to LDS part[s][c][r]; the sums over s in order follow a barrier.
//   EPI 0: y[c][row] for rows [row_start, row_end), columns c < M.
//   EPI 1 (RG = 4, whole tiles of gate and up interleaved by 32): the
//          SwiGLU and Q8_0 epilogue of q4_0_matvec_cols_kernel<64, NC, .., 1>
//          per column.
typedef int v4i_mf __attribute__((ext_vector_type(4)));
typedef float v4f_mf __attribute__((ext_vector_type(4)));
typedef _Float16 v4h_mf __attribute__((ext_vector_type(4)));
typedef unsigned v2u_mf __attribute__((ext_vector_type(2)));
constexpr int kMfmaChainBias = 0x49400000;  // 1.5 * 2^19 as fp32 bits
constexpr int kMfmaCols = 16;
constexpr size_t kLdsMax = 160 * 1024;  // a gfx950 workgroup's LDS

template <int RG, int EPI, bool DOTS>
__global__ __launch_bounds__(1024) void q4_0_mfma_cols_kernel(
    const uint8_t *__restrict__ W, size_t plane0_bytes, int B, int DC, const int8_t *__restrict__ q,
    const float *__restrict__ scales, int M, int group0, int row_start, int row_end,
    const float *__restrict__ bias, float *__restrict__ y, int ldy, int32_t *__restrict__ dots,
    int8_t *__restrict__ mq, float *__restrict__ ms, int32_t *__restrict__ mqs) {
    constexpr int R = 16 * RG, kSlots = kTileRows / R;
    static_assert(EPI == 0 || RG == 4, "the SwiGLU epilogue takes whole tiles");
    extern __shared__ __align__(16) float part[];  // [S][M][R]
    const int K = B * kQ4Block;
    const int S = (B + kStretch - 1) / kStretch;
    const int tid = threadIdx.x, nt = blockDim.x;
    const int lane = tid & 63, wave = tid >> 6, nw = nt >> 6;
    const int g = group0 + blockIdx.x;
    const int tile = g / kSlots, r0 = (g - tile * kSlots) * R;  // the group's first row within its tile
    const int i = lane & 15, kb = lane >> 4;
    const uint32_t wsh = kb < 2 ? 4u : 0u;  // low nibbles move up into the byte's high half
    const bool col_ok = i < M;
    const int8_t *qcol = q + (size_t)min(i, M - 1) * K + 8 * kb;
    const float *scol = scales + (size_t)min(i, M - 1) * B;

    for (int u = wave; u < RG * S; u += nw) {
        const int rg = u / S, s = u - rg * S;
        const int b0 = s * kStretch, nbk = min(kStretch, B - b0);
        const int rl = r0 + 16 * rg + i;  // lane's row (as the A operand's row) within the tile
        const uint8_t *wp = W + ((size_t)(tile * B + b0) * kTileRows + rl) * kChunk + 8 * (kb & 1);
        // the unit's loads: the columns' inputs first, then the weights
        long av[kStretch];
        v2u_mf wv[kStretch];
        float da[kStretch];
        uint4 dch = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
        for (int j = 0; j < kStretch; j++) {
            av[j] = 0;
            da[j] = 0.0f;
            if (j < nbk && col_ok)
                av[j] = *(const long *)(qcol + (size_t)(b0 + j) * kQ4Block);
            if (j < nbk && col_ok && kb == 0)
                da[j] = scol[b0 + j];
        }
#pragma unroll
        for (int j = 0; j < kStretch; j++)
            if (j < nbk)
                wv[j] = __builtin_nontemporal_load((const v2u_mf *)(wp + (size_t)j * kTileRows * kChunk));
        if (kb == 0)
            dch = *(const uint4 *)(W + plane0_bytes + ((size_t)(tile * DC + s) * kTileRows + rl) * kChunk);

        v4i_mf prev;
#pragma unroll
        for (int e = 0; e < 4; e++)
            prev[e] = kMfmaChainBias;
        const v4f_mf zero = {0.0f, 0.0f, 0.0f, 0.0f};
        v4f_mf p = zero;
#pragma unroll
        for (int j = 0; j < kStretch; j++) {
            if (j < nbk) {
                const uint32_t lo = ((wv[j].x << wsh) & 0xF0F0F0F0u) ^ 0x80808080u;
                const uint32_t hi = ((wv[j].y << wsh) & 0xF0F0F0F0u) ^ 0x80808080u;
                const long A = (long)(((unsigned long)hi << 32) | lo);
                const v4i_mf next = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, av[j], prev, 0, 0, 0);
                const uint32_t dw = ((j >> 1) == 0 ? dch.x : (j >> 1) == 1 ? dch.y : (j >> 1) == 2 ? dch.z : dch.w);
                const uint32_t dwh = (j & 1) ? (dw >> 16) : (dw & 0xFFFFu);
                const v4h_mf wa = __builtin_bit_cast(v4h_mf, make_uint2(dwh, 0u));
                const v4h_mf ca = __builtin_bit_cast(v4h_mf, make_uint2(float_to_half_bits(da[j]), 0u));
                const v4f_mf sc = __builtin_amdgcn_mfma_f32_16x16x16f16(wa, ca, zero, 0, 0, 0);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float x = __int_as_float(next[e]) - __int_as_float(prev[e]);  // the block's isum
                    p[e] = fmaf(x, sc[e], p[e]);
                    if (DOTS) {
                        const int row = tile * kTileRows + r0 + 16 * rg + 4 * kb + e;
                        if (col_ok && row >= row_start && row < row_end)
                            dots[((size_t)i * (row_end - row_start) + (row - row_start)) * B + b0 + j] = (int)x;
                    }
                }
                prev = next;
            }
        }
        if (col_ok)
            *(float4 *)&part[((size_t)s * M + i) * R + 16 * rg + 4 * kb] = make_float4(p[0], p[1], p[2], p[3]);
    }
    if (DOTS)
        return;
    lds_barrier();
    if (EPI == 1) {
        const int F = row_end / 2;  // the SwiGLU's width: gate and up rows in equal number
        for (int c = wave; c < M; c += nw) {
            float acc = 0.0f;
            for (int t = 0; t < S; t++)
                acc = acc + part[((size_t)t * M + c) * kTileRows + lane];
            // lane l < 32: gate 32 * tile + l; lane l + 32: its up
            const float u = __shfl_down(acc, 32, 64);
            const float gt = acc;
            const float ex = ggml_expf(-gt);
            const float den = 1.0f + ex;
            const float sl = gt / den;
            const float v = sl * u;
            float stored;
            int32_t sm;
            const int32_t nq = q8_0_lane(v, &stored, &sm);
            if (lane < 32) {
                mq[(size_t)c * F + (size_t)tile * 32 + lane] = (int8_t)nq;
                if (lane == 0) {
                    ms[(size_t)c * (F / kQ4Block) + tile] = stored;
                    mqs[(size_t)c * (F / kQ4Block) + tile] = sm;
                }
            }
        }
    } else {
        for (int pr = tid; pr < M * R; pr += nt) {
            const int c = pr / R, rr = pr - c * R;
            const int orow = tile * kTileRows + r0 + rr;
            if (orow >= row_start && orow < row_end) {
                float acc = 0.0f;
                for (int t = 0; t < S; t++)
                    acc = acc + part[((size_t)t * M + c) * R + rr];
                if (bias)
                    acc = acc + bias[orow];
                y[(size_t)c * ldy + orow] = acc;
            }
        }
    }
}

// The same product with the columns' inputs and scales staged in LDS once
// per workgroup (16-byte loads, every load of a pass in flight together).
// Reading the B operands straight from global memory (q4_0_mfma_cols_kernel)
// costs a scattered 8-byte load per lane and block and the whole activation
// again for every 16 rows: at config 3's shapes and 8 columns that traffic,
// not the weights', set the time (Q|K|V 8.1 us, of which the weights' loads
// alone 4.7).  Rows of the staged activation are K + 16 bytes apart and its
// scales B + 1 floats apart, so that the 16 columns x 4 lane groups of a
// B-operand read fall in distinct LDS banks.  The stretch sums then reuse
// the activation's LDS (after a barrier).  This form (16 rows a workgroup)
// serves rows of 17 to 48 stretches: wavefront w takes stretches w, w + 16,
// .. (SW of them at most), their weights all requested into registers
// before the barrier; rows of at most 16 stretches take the form below,
// whose weights arrive through LDS.
__host__ __device__ inline size_t mfma_lds_act_bytes(int M, int K, int B) {
    return (((size_t)M * (K + 16) + 15) & ~(size_t)15) + (size_t)M * (B + 1) * sizeof(float);
}

template <int SW, bool DOTS>
__global__ __launch_bounds__(1024) void q4_0_mfma_cols_lds_kernel(
    const uint8_t *__restrict__ W, size_t plane0_bytes, int B, int DC, const int8_t *__restrict__ q,
    const float *__restrict__ scales, int M, int group0, int row_start, int row_end,
    const float *__restrict__ bias, float *__restrict__ y, int ldy, int32_t *__restrict__ dots) {
    constexpr int RG = 1, R = 16, kSlots = kTileRows / R;
    extern __shared__ __align__(16) uint8_t lds_raw[];
    const int K = B * kQ4Block, ldq = K + 16, lds_b = B + 1;
    const int S = (B + kStretch - 1) / kStretch;
    int8_t *qa = (int8_t *)lds_raw;                                                 // [M][K + 16]
    float *sa = (float *)(lds_raw + (((size_t)M * ldq + 15) & ~(size_t)15));       // [M][B + 1]
    float *part = (float *)lds_raw;                                                 // [S][M][R], after the barrier
    const int tid = threadIdx.x, nt = blockDim.x;
    const int lane = tid & 63, wave = tid >> 6, nw = nt >> 6;
    const int g = group0 + blockIdx.x;
    const int tile = g / kSlots, r0 = (g - tile * kSlots) * R;
    const int i = lane & 15, kb = lane >> 4;
    const uint32_t wsh = kb < 2 ? 4u : 0u;
    const bool col_ok = i < M;

    // The columns' inputs and scales into LDS, every load of a pass in
    // flight together, and only then this wavefront's weights.  (Weights
    // requested before the staging loads have landed are slower: config 3's
    // Down at 8 columns 12.2 -> 13.8 us, Gate|Up 16.0 -> 19.2 us.)
    const int n16 = K / 16, p16 = M * n16, nb = M * B;
    for (int base = 0; base < max(p16, nb); base += kColRegs * nt) {
        int4 qv[kColRegs];
        float sv[kColRegs];
#pragma unroll
        for (int k = 0; k < kColRegs; k++) {
            const int e = base + tid + k * nt;
            qv[k] = ((const int4 *)q)[min(e, p16 - 1)];
            sv[k] = scales[min(e, nb - 1)];
        }
#pragma unroll
        for (int k = 0; k < kColRegs; k++) {
            const int e = base + tid + k * nt;
            if (e < p16) {
                const int c = e / n16;
                *(int4 *)(qa + (size_t)c * ldq + (size_t)(e - c * n16) * 16) = qv[k];
            }
            if (e < nb) {
                const int c = e / B;
                sa[c * lds_b + (e - c * B)] = sv[k];
            }
        }
    }
    // this wavefront's stretches wave, wave + nw, .. (SW of them at most) of
    // the RG row groups, every load in flight together
    v2u_mf wv[SW][RG][kStretch];
    uint4 dch[SW][RG];
#pragma unroll
    for (int k = 0; k < SW; k++) {
        const int s = wave + k * nw, b0 = s * kStretch, nbk = min(kStretch, B - b0);
#pragma unroll
        for (int rg = 0; rg < RG; rg++) {
            const int rl = r0 + 16 * rg + i;
            const uint8_t *wp = W + ((size_t)(tile * B + b0) * kTileRows + rl) * kChunk + 8 * (kb & 1);
#pragma unroll
            for (int j = 0; j < kStretch; j++)
                if (j < nbk)
                    wv[k][rg][j] = __builtin_nontemporal_load((const v2u_mf *)(wp + (size_t)j * kTileRows * kChunk));
            dch[k][rg] = make_uint4(0u, 0u, 0u, 0u);
            if (kb == 0 && s < S)
                dch[k][rg] = *(const uint4 *)(W + plane0_bytes + ((size_t)(tile * DC + s) * kTileRows + rl) * kChunk);
        }
    }
    lds_barrier();

    const v4f_mf zero = {0.0f, 0.0f, 0.0f, 0.0f};
    v4f_mf p[SW][RG];
    const int8_t *qrow = qa + (size_t)min(i, M - 1) * ldq + 8 * kb;
    const float *srow = sa + min(i, M - 1) * lds_b;
    // stretch by stretch: the first one's blocks are multiplied while the
    // later stretches' weights still arrive (interleaving the stretches'
    // blocks instead, for independent MFMA chains, waits for every stretch
    // first: config 3's Down at 8 columns 12.2 -> 14.0 us)
#pragma unroll
    for (int k = 0; k < SW; k++) {
        const int s = wave + k * nw, b0 = s * kStretch, nbk = min(kStretch, B - b0);  // nbk <= 0 past the row
        v4i_mf prev[RG];
#pragma unroll
        for (int rg = 0; rg < RG; rg++) {
            p[k][rg] = zero;
#pragma unroll
            for (int e = 0; e < 4; e++)
                prev[rg][e] = kMfmaChainBias;
        }
#pragma unroll
        for (int j = 0; j < kStretch; j++) {
            if (j < nbk) {
                const int b = b0 + j;
                const long bop = col_ok ? *(const long *)(qrow + (size_t)b * kQ4Block) : 0;
                const float da = (col_ok && kb == 0) ? srow[b] : 0.0f;
                const v4h_mf ca = __builtin_bit_cast(v4h_mf, make_uint2(float_to_half_bits(da), 0u));
#pragma unroll
                for (int rg = 0; rg < RG; rg++) {
                    const uint32_t lo = ((wv[k][rg][j].x << wsh) & 0xF0F0F0F0u) ^ 0x80808080u;
                    const uint32_t hi = ((wv[k][rg][j].y << wsh) & 0xF0F0F0F0u) ^ 0x80808080u;
                    const long A = (long)(((unsigned long)hi << 32) | lo);
                    const v4i_mf next = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, bop, prev[rg], 0, 0, 0);
                    const uint4 &dc = dch[k][rg];
                    const uint32_t dw = (j >> 1) == 0 ? dc.x : (j >> 1) == 1 ? dc.y : (j >> 1) == 2 ? dc.z : dc.w;
                    const uint32_t dwh = (j & 1) ? (dw >> 16) : (dw & 0xFFFFu);
                    const v4h_mf wa = __builtin_bit_cast(v4h_mf, make_uint2(dwh, 0u));
                    const v4f_mf sc = __builtin_amdgcn_mfma_f32_16x16x16f16(wa, ca, zero, 0, 0, 0);
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float x = __int_as_float(next[e]) - __int_as_float(prev[rg][e]);  // the block's isum
                        p[k][rg][e] = fmaf(x, sc[e], p[k][rg][e]);
                        if (DOTS) {
                            const int row = tile * kTileRows + r0 + 16 * rg + 4 * kb + e;
                            if (col_ok && row >= row_start && row < row_end)
                                dots[((size_t)i * (row_end - row_start) + (row - row_start)) * B + b] = (int)x;
                        }
                    }
                    prev[rg] = next;
                }
            }
        }
    }
    if (DOTS)
        return;
    lds_barrier();  // every wavefront is done with the staged activation
    if (col_ok) {
#pragma unroll
        for (int k = 0; k < SW; k++) {
            const int s = wave + k * nw;
            if (s < S) {
#pragma unroll
                for (int rg = 0; rg < RG; rg++)
                    *(float4 *)&part[((size_t)s * M + i) * R + 16 * rg + 4 * kb] =
                        make_float4(p[k][rg][0], p[k][rg][1], p[k][rg][2], p[k][rg][3]);
            }
        }
    }
    lds_barrier();
    for (int pr = tid; pr < M * R; pr += nt) {
        const int c = pr / R, rr = pr - c * R;
        const int orow = tile * kTileRows + r0 + rr;
        if (orow >= row_start && orow < row_end) {
            float acc = 0.0f;
            for (int t = 0; t < S; t++)
                acc = acc + part[((size_t)t * M + c) * R + rr];
            if (bias)
                acc = acc + bias[orow];
            y[(size_t)c * ldy + orow] = acc;
        }
    }
}

// The LDS-staged product with the weights arriving in LDS too: each
// wavefront's row groups go global -> LDS as whole 16-byte chunks (lane l:
// row l % 16 of the group, blocks l / 16 and 4 + l / 16 of the stretch), two
// row groups in flight in a ring of two 2 KiB slots, and the A operands are
// read back in the MFMA's layout (8 bytes a lane).  Against 8-byte loads
// straight into registers this halves the weights' load instructions and
// frees the registers that held them (64 for four row groups).  The compute
// phase reads LDS through inline asm only: the compiler would otherwise make
// every LDS read wait for all global-to-LDS loads in flight.
constexpr int kMfmaSlotB = 2048;  // one row group's stretch: 16 rows x 8 blocks x 16 bytes

template <int OFF>
__device__ __forceinline__ void ds_read_u64(uint32_t addr, v2u_mf &r) {
    asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
}
template <int OFF>
__device__ __forceinline__ void ds_read_f32(uint32_t addr, float &r) {
    asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
}

__host__ __device__ inline size_t mfma_dma_ring_offset(int M, int K, int B) {
    return (mfma_lds_act_bytes(M, K, B) + 15) & ~(size_t)15;
}

template <int RG, int EPI, bool DOTS>
__global__ __launch_bounds__(1024) void q4_0_mfma_cols_dma_kernel(
    const uint8_t *__restrict__ W, size_t plane0_bytes, int B, int DC, const int8_t *__restrict__ q,
    const float *__restrict__ scales, int M, int group0, int row_start, int row_end,
    const float *__restrict__ bias, float *__restrict__ y, int ldy, int32_t *__restrict__ dots,
    int8_t *__restrict__ mq, float *__restrict__ ms, int32_t *__restrict__ mqs) {
    constexpr int R = 16 * RG, kSlots = kTileRows / R;
    static_assert(EPI == 0 || RG == 4, "the SwiGLU epilogue takes whole tiles");
    extern __shared__ __align__(16) uint8_t lds_raw[];
    const int K = B * kQ4Block, ldq = K + 16, lds_b = B + 1;
    const int S = (B + kStretch - 1) / kStretch;
    int8_t *qa = (int8_t *)lds_raw;                                                 // [M][K + 16]
    float *sa = (float *)(lds_raw + (((size_t)M * ldq + 15) & ~(size_t)15));       // [M][B + 1]
    float *part = (float *)lds_raw;                                                 // [S][M][R], after the barrier
    const int tid = threadIdx.x, nt = blockDim.x;
    const int lane = tid & 63, wave = tid >> 6;
    uint8_t *ring = lds_raw + mfma_dma_ring_offset(M, K, B) + (size_t)wave * 2 * kMfmaSlotB;
    const int g = group0 + blockIdx.x;
    const int tile = g / kSlots, r0 = (g - tile * kSlots) * R;
    const int i = lane & 15, kb = lane >> 4;
    const uint32_t wsh = kb < 2 ? 4u : 0u;
    const bool col_ok = i < M;
    const int s = wave, b0 = s * kStretch, nbk = min(kStretch, B - b0);

    // the columns' inputs and scales into LDS, every load of a pass in flight
    const int n16 = K / 16, p16 = M * n16, nb = M * B;
    for (int base = 0; base < max(p16, nb); base += kColRegs * nt) {
        int4 qv[kColRegs];
        float sv[kColRegs];
#pragma unroll
        for (int k = 0; k < kColRegs; k++) {
            const int e = base + tid + k * nt;
            qv[k] = ((const int4 *)q)[min(e, p16 - 1)];
            sv[k] = scales[min(e, nb - 1)];
        }
#pragma unroll
        for (int k = 0; k < kColRegs; k++) {
            const int e = base + tid + k * nt;
            if (e < p16) {
                const int c = e / n16;
                *(int4 *)(qa + (size_t)c * ldq + (size_t)(e - c * n16) * 16) = qv[k];
            }
            if (e < nb) {
                const int c = e / B;
                sa[c * lds_b + (e - c * B)] = sv[k];
            }
        }
    }
    // the row groups' weight scales, then their chunks (two groups in flight)
    uint4 dch[RG];
#pragma unroll
    for (int rg = 0; rg < RG; rg++) {
        dch[rg] = make_uint4(0u, 0u, 0u, 0u);
        if (kb == 0)
            dch[rg] = *(const uint4 *)(W + plane0_bytes + ((size_t)(tile * DC + s) * kTileRows + r0 + 16 * rg + i) *
                                                             kChunk);
    }
    const uint8_t *wsrc = W + ((size_t)tile * B * kTileRows + r0 + i) * kChunk;
#define GX_MFMA_ISSUE(RGI, SLOT)                                                                                     \
    do {                                                                                                             \
        _Pragma("unroll") for (int h = 0; h < 2; h++) {                                                              \
            const int b = min(b0 + 4 * h + kb, B - 1);                                                               \
            __builtin_amdgcn_global_load_lds(wsrc + ((size_t)b * kTileRows + 16 * (RGI)) * kChunk,                   \
                                             (lds_ptr)(ring + (SLOT) * kMfmaSlotB + h * 1024), 16, 0, 0);            \
        }                                                                                                            \
    } while (0)
    GX_MFMA_ISSUE(0, 0);
    if (RG > 1)
        GX_MFMA_ISSUE(1, 1);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this thread's staging stores
    __builtin_amdgcn_s_barrier();

    // the stretch's B operands and activation scales (asm reads, no wait on
    // the weights in flight)
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_ptr)lds_raw;
    const uint32_t qaddr = lds0 + (uint32_t)(min(i, M - 1) * ldq + 8 * kb + b0 * kQ4Block);
    const uint32_t saddr = (uint32_t)(uintptr_t)(lds_ptr)sa + (uint32_t)((min(i, M - 1) * lds_b + b0) * 4);
    v2u_mf bq[kStretch];
    float das[kStretch];
    ds_read_u64<0 * kQ4Block>(qaddr, bq[0]);
    ds_read_u64<1 * kQ4Block>(qaddr, bq[1]);
    ds_read_u64<2 * kQ4Block>(qaddr, bq[2]);
    ds_read_u64<3 * kQ4Block>(qaddr, bq[3]);
    ds_read_u64<4 * kQ4Block>(qaddr, bq[4]);
    ds_read_u64<5 * kQ4Block>(qaddr, bq[5]);
    ds_read_u64<6 * kQ4Block>(qaddr, bq[6]);
    ds_read_u64<7 * kQ4Block>(qaddr, bq[7]);
    ds_read_f32<0>(saddr, das[0]);
    ds_read_f32<4>(saddr, das[1]);
    ds_read_f32<8>(saddr, das[2]);
    ds_read_f32<12>(saddr, das[3]);
    ds_read_f32<16>(saddr, das[4]);
    ds_read_f32<20>(saddr, das[5]);
    ds_read_f32<24>(saddr, das[6]);
    ds_read_f32<28>(saddr, das[7]);
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(bq[0]), "+v"(bq[1]), "+v"(bq[2]), "+v"(bq[3]), "+v"(bq[4]), "+v"(bq[5]), "+v"(bq[6]),
                   "+v"(bq[7]), "+v"(das[0]), "+v"(das[1]), "+v"(das[2]), "+v"(das[3]), "+v"(das[4]), "+v"(das[5]),
                   "+v"(das[6]), "+v"(das[7]));
    v4h_mf ca[kStretch];
    long bop[kStretch];
#pragma unroll
    for (int j = 0; j < kStretch; j++) {
        bop[j] = col_ok ? (long)(((unsigned long)bq[j].y << 32) | bq[j].x) : 0;
        ca[j] = __builtin_bit_cast(v4h_mf, make_uint2(col_ok && kb == 0 ? float_to_half_bits(das[j]) : 0u, 0u));
    }

    const v4f_mf zero = {0.0f, 0.0f, 0.0f, 0.0f};
    v4f_mf p[RG];
    const uint32_t abase = (uint32_t)(uintptr_t)(lds_ptr)ring + (uint32_t)(i * 16 + 8 * (kb & 1));
#pragma unroll
    for (int rg = 0; rg < RG; rg++) {
        if (rg + 1 < RG)
            wait_vmcnt<2>();  // this group's chunks have landed (the next group's may be in flight)
        else
            wait_vmcnt<0>();
        v2u_mf wa[kStretch];
        const uint32_t aslot = abase + (uint32_t)((rg & 1) * kMfmaSlotB);
        ds_read_u64<0 * 256>(aslot, wa[0]);
        ds_read_u64<1 * 256>(aslot, wa[1]);
        ds_read_u64<2 * 256>(aslot, wa[2]);
        ds_read_u64<3 * 256>(aslot, wa[3]);
        ds_read_u64<1024 + 0 * 256>(aslot, wa[4]);
        ds_read_u64<1024 + 1 * 256>(aslot, wa[5]);
        ds_read_u64<1024 + 2 * 256>(aslot, wa[6]);
        ds_read_u64<1024 + 3 * 256>(aslot, wa[7]);
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(wa[0]), "+v"(wa[1]), "+v"(wa[2]), "+v"(wa[3]), "+v"(wa[4]), "+v"(wa[5]), "+v"(wa[6]),
                       "+v"(wa[7]));
        if (rg + 2 < RG)
            GX_MFMA_ISSUE(rg + 2, rg & 1);  // into the slot just read
        v4i_mf prev;
#pragma unroll
        for (int e = 0; e < 4; e++)
            prev[e] = kMfmaChainBias;
        p[rg] = zero;
#pragma unroll
        for (int j = 0; j < kStretch; j++) {
            if (j < nbk) {
                const uint32_t lo = ((wa[j].x << wsh) & 0xF0F0F0F0u) ^ 0x80808080u;
                const uint32_t hi = ((wa[j].y << wsh) & 0xF0F0F0F0u) ^ 0x80808080u;
                const long A = (long)(((unsigned long)hi << 32) | lo);
                const v4i_mf next = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, bop[j], prev, 0, 0, 0);
                const uint4 &dc = dch[rg];
                const uint32_t dw = (j >> 1) == 0 ? dc.x : (j >> 1) == 1 ? dc.y : (j >> 1) == 2 ? dc.z : dc.w;
                const uint32_t dwh = (j & 1) ? (dw >> 16) : (dw & 0xFFFFu);
                const v4h_mf wh = __builtin_bit_cast(v4h_mf, make_uint2(dwh, 0u));
                const v4f_mf sc = __builtin_amdgcn_mfma_f32_16x16x16f16(wh, ca[j], zero, 0, 0, 0);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float x = __int_as_float(next[e]) - __int_as_float(prev[e]);  // the block's isum
                    p[rg][e] = fmaf(x, sc[e], p[rg][e]);
                    if (DOTS) {
                        const int row = tile * kTileRows + r0 + 16 * rg + 4 * kb + e;
                        if (col_ok && row >= row_start && row < row_end)
                            dots[((size_t)i * (row_end - row_start) + (row - row_start)) * B + b0 + j] = (int)x;
                    }
                }
                prev = next;
            }
        }
    }
#undef GX_MFMA_ISSUE
    if (DOTS)
        return;
    lds_barrier();  // every wavefront is done with the staged activation
    if (col_ok) {
#pragma unroll
        for (int rg = 0; rg < RG; rg++)
            *(float4 *)&part[((size_t)s * M + i) * R + 16 * rg + 4 * kb] =
                make_float4(p[rg][0], p[rg][1], p[rg][2], p[rg][3]);
    }
    lds_barrier();
    if (EPI == 1) {
        const int F = row_end / 2;
        for (int c = wave; c < M; c += nt >> 6) {
            float acc = 0.0f;
            for (int t = 0; t < S; t++)
                acc = acc + part[((size_t)t * M + c) * kTileRows + lane];
            // lane l < 32: gate 32 * tile + l; lane l + 32: its up
            const float u = __shfl_down(acc, 32, 64);
            const float gt = acc;
            const float ex = ggml_expf(-gt);
            const float den = 1.0f + ex;
            const float sl = gt / den;
            const float v = sl * u;
            float stored;
            int32_t sm;
            const int32_t nq = q8_0_lane(v, &stored, &sm);
            if (lane < 32) {
                mq[(size_t)c * F + (size_t)tile * 32 + lane] = (int8_t)nq;
                if (lane == 0) {
                    ms[(size_t)c * (F / kQ4Block) + tile] = stored;
                    mqs[(size_t)c * (F / kQ4Block) + tile] = sm;
                }
            }
        }
    } else {
        for (int pr = tid; pr < M * R; pr += nt) {
            const int c = pr / R, rr = pr - c * R;
            const int orow = tile * kTileRows + r0 + rr;
            if (orow >= row_start && orow < row_end) {
                float acc = 0.0f;
                for (int t = 0; t < S; t++)
                    acc = acc + part[((size_t)t * M + c) * R + rr];
                if (bias)
                    acc = acc + bias[orow];
                y[(size_t)c * ldy + orow] = acc;
            }
        }
    }
}

// One position (M = 1) whose activation is produced by the product itself:
// x (+ add) -> RMSNormPlain(gain, eps) -> Q8_0, a block's pre-norm
// (qwen/block.go:45-52, 59-68), so that the norm needs no kernel of its own.
// Every workgroup stages x + add in LDS and computes the norm's float64 sum
// of squares with the same 512-partial tree as the separate norm kernel;
// workgroup 0 writes x + add to x_out.  Each wavefront quantises the 256
// values of the stretch it multiplies (four a lane, a Q8_0 block per eight
// lanes) and moves them to SGPRs with readlane, which is where the plain
// kernel's activation sits.  The values, and so the products, are the
// separate kernels' bit for bit.
//   EPI 0: y[row] for rows [row_start, row_end).
//   EPI 1: the rows are gate and up interleaved by 32 (tile t holds gate rows
//          32t .. 32t+31, then the same up rows): the tile's 32 outputs
//          silu(gate) * up (SwiGLURange, nn/swiglu.go:77-82) go straight to
//          their Q8_0 block t in q/scales/qsum, the down projection's input.

// DB: two stretch slots a wavefront (double-buffered); without it a
// wavefront has one slot and half the registers, so that two workgroups fit
// a CU.
template <int EPI, bool DB, bool DOTS>
__global__ __launch_bounds__(1024) void q4_0_matvec_fused_kernel(
    const uint8_t *__restrict__ W, size_t plane0_bytes, int B, int DC, int K, int tile0, int row_start, int row_end,
    float *__restrict__ y, const float *__restrict__ x, const float *__restrict__ add,
    const float *__restrict__ gain, float eps, float *__restrict__ x_out, int8_t *__restrict__ q,
    float *__restrict__ scales, int32_t *__restrict__ qsum, int32_t *__restrict__ dots) {
    extern __shared__ __align__(16) float lds[];  // part [S][64], then xs [K]
    __shared__ double red[512];
    __shared__ float scale_sh;
    const int S = (B + kStretch - 1) / kStretch;
    float *part = lds;
    float *xs = lds + S * kTileRows;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nwaves = blockDim.x >> 6;
    const int tile = tile0 + blockIdx.x;
    const int row = tile * kTileRows + lane;
    const bool in_range = row >= row_start && row < row_end;
    const uint8_t *qs_row = W + ((size_t)tile * B * kTileRows + lane) * kChunk;
    const uint8_t *d_row = W + plane0_bytes + ((size_t)tile * DC * kTileRows + lane) * kChunk;

    // x (+ add) into LDS and the norm's partials (norm_stage), then its tree
    // in wavefront 0: two barriers.
    norm_stage(x, add, K, xs, blockIdx.x == 0 ? x_out : nullptr, red);
    __syncthreads();
    if (wave == 0) {
        const double total = norm_tree_wave(red);
        if (tid == 0)
            scale_sh = norm_scale(total, K, eps);
    }
    // A wavefront's slot k is stretch wave + k*nwaves; every wavefront runs
    // the same number of slots (a slot past S loads stretch S - 1 again and
    // computes nothing), two register sets, a slot's loads issued a slot
    // ahead under one uniform condition, so the wait counts stay exact.
    const int slots = DB ? (S + nwaves - 1) / nwaves : 1;
    uint4 wa[kStretch], wb[DB ? kStretch : 1], da, db;
    float4 ga, gb;
#define GX_FU_LOAD(wq, dch, gq, st)                                                                                  \
    do {                                                                                                             \
        const int sc_ = min((st), S - 1);                                                                            \
        _Pragma("unroll") for (int j = 0; j < kStretch; j++)                                                         \
            wq[j] = load_stream(qs_row + (size_t)min(sc_ * kStretch + j, B - 1) * kTileRows * kChunk);               \
        dch = *(const uint4 *)(d_row + (size_t)sc_ * kTileRows * kChunk);                                            \
        gq = *(const float4 *)(gain + min(sc_ * kStretch * kQ4Block + 4 * lane, K - 4));                             \
    } while (0)
    __syncthreads();
    const float sc = scale_sh;
    // The weights go out only now: with them in flight the norm's LDS steps
    // and barriers above ran measurably slower (Gate|Up 12.1 -> 10.5 us);
    // the quantisation below still overlaps their latency.
    GX_FU_LOAD(wa, da, ga, wave);
    if (DB && slots > 1)
        GX_FU_LOAD(wb, db, gb, wave + nwaves);

    // The stretch's activation (values b0*32 + 4*lane .. + 3), its Q8_0 in
    // SGPRs, and the product of the 64 rows with it.
#define GX_FU_STRETCH(wq, dch, gq, st)                                                                               \
    do {                                                                                                             \
        const int b0 = (st) * kStretch;                                                                              \
        const int nb = min(kStretch, B - b0);                                                                        \
        const float4 xq = *(const float4 *)(xs + min(b0 * kQ4Block + 4 * lane, K - 4));                              \
        const float xa[4] = {xq.x, xq.y, xq.z, xq.w}, gg[4] = {gq.x, gq.y, gq.z, gq.w};                              \
        float v[4];                                                                                                  \
        _Pragma("unroll") for (int k = 0; k < 4; k++) {                                                              \
            const float nv = xa[k] * sc;                                                                             \
            v[k] = nv * gg[k];                                                                                       \
        }                                                                                                            \
        float bstored;                                                                                               \
        int32_t bsum;                                                                                                \
        const uint32_t aq = q8_0_quad(v, &bstored, &bsum);                                                           \
        float p = 0.0f;                                                                                              \
        _Pragma("unroll") for (int j = 0; j < kStretch; j++) {                                                       \
            if (j < nb) {                                                                                            \
                int4 a0, a1;                                                                                         \
                a0.x = __builtin_amdgcn_readlane((int)aq, 8 * j + 0);                                                \
                a0.y = __builtin_amdgcn_readlane((int)aq, 8 * j + 1);                                                \
                a0.z = __builtin_amdgcn_readlane((int)aq, 8 * j + 2);                                                \
                a0.w = __builtin_amdgcn_readlane((int)aq, 8 * j + 3);                                                \
                a1.x = __builtin_amdgcn_readlane((int)aq, 8 * j + 4);                                                \
                a1.y = __builtin_amdgcn_readlane((int)aq, 8 * j + 5);                                                \
                a1.z = __builtin_amdgcn_readlane((int)aq, 8 * j + 6);                                                \
                a1.w = __builtin_amdgcn_readlane((int)aq, 8 * j + 7);                                                \
                const int32_t qs = __builtin_amdgcn_readlane(bsum, 8 * j);                                           \
                const float sa = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bstored), 8 * j));          \
                const int32_t isum = q4_0_block_isum(wq[j], a0, a1, qs);                                             \
                const float scl = chunk_half(dch, j) * sa;                                                           \
                p = fmaf((float)isum, scl, p);                                                                       \
                if (DOTS && in_range)                                                                                \
                    dots[(size_t)(row - row_start) * B + b0 + j] = isum;                                             \
            }                                                                                                        \
        }                                                                                                            \
        part[(st) * kTileRows + lane] = p;                                                                           \
    } while (0)
    if (DB) {
        for (int k = 0; k < slots; k += 2) {
            const int s = wave + k * nwaves;
            if (s < S)
                GX_FU_STRETCH(wa, da, ga, s);
            if (k + 2 < slots)
                GX_FU_LOAD(wa, da, ga, s + 2 * nwaves);
            if (k + 1 < slots && s + nwaves < S)
                GX_FU_STRETCH(wb, db, gb, s + nwaves);
            if (k + 3 < slots)
                GX_FU_LOAD(wb, db, gb, s + 3 * nwaves);
        }
    } else if (wave < S) {
        GX_FU_STRETCH(wa, da, ga, wave);
    }
#undef GX_FU_STRETCH
#undef GX_FU_LOAD
    __syncthreads();
    if (wave == 0) {
        float acc = 0.0f;
        for (int s = 0; s < S; s++)
            acc = acc + part[s * kTileRows + lane];
        if (EPI == 0) {
            if (!DOTS && in_range)
                y[row] = acc;
        } else {
            // lane l < 32: gate 32*tile + l; lane l + 32: its up
            const float u = __shfl_down(acc, 32, 64);
            const float g = acc;
            const float ex = ggml_expf(-g);
            const float den = 1.0f + ex;
            const float sl = g / den;
            const float v = sl * u;
            float stored;
            int32_t sm;
            const int32_t nq = q8_0_lane(v, &stored, &sm);
            if (lane < 32) {
                q[(size_t)tile * 32 + lane] = (int8_t)nq;
                if (lane == 0) {
                    scales[tile] = stored;
                    qsum[tile] = sm;
                }
            }
        }
    }
}

// The fused pre-norm product (EPI 0) on sub-tiles of R rows, so that a matrix
// of few tiles spreads its weights over more CUs: a CU fetches only a few
// tens of GB/s, so Q|K|V's 96 whole tiles on 96 of 256 CUs wait on their
// CUs, not on HBM.  Each workgroup makes the whole activation (x + add, the
// norm, Q8_0 of every block, four values a thread from its own float4) into
// LDS and then multiplies as q4_0_matvec_lds_kernel does: lane l is row
// l % R and stretch slot l / R.  Values, and so products, are the whole-tile
// kernel's bit for bit.
template <int R, bool DOTS>
__global__ __launch_bounds__(1024) void q4_0_matvec_fused_lds_kernel(
    const uint8_t *__restrict__ W, size_t plane0_bytes, int B, int DC, int group0, int row_start, int row_end,
    float *__restrict__ y, const float *__restrict__ x, const float *__restrict__ add,
    const float *__restrict__ gain, float eps, float *__restrict__ x_out, int32_t *__restrict__ dots) {
    constexpr int kSlots = kTileRows / R;
    extern __shared__ __align__(16) uint8_t lds_raw[];
    __shared__ double red[512];
    __shared__ float scale_sh;
    const int K = B * kQ4Block;
    const int S = (B + kStretch - 1) / kStretch;
    float *part = (float *)lds_raw;
    float *xs = (float *)(lds_raw + lds_part_bytes(S, R));
    int8_t *qa = (int8_t *)(xs + K);
    float *sa = (float *)(qa + K);
    int32_t *qsa = (int32_t *)(sa + B);
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int g = group0 + blockIdx.x;
    const int tile = g / kSlots, r = (g - tile * kSlots) * R + lane % R;
    const int row = tile * kTileRows + r;
    const bool in_range = row >= row_start && row < row_end;

    // x (+ add) into LDS and the norm's partials, then its tree in
    // wavefront 0 (as q4_0_matvec_fused_kernel)
    const int n4 = K / 4;
    const float4 gv = ((const float4 *)gain)[min(tid, n4 - 1)];
    norm_stage(x, add, K, xs, blockIdx.x == 0 ? x_out : nullptr, red);
    __syncthreads();
    if (wave == 0) {
        const double total = norm_tree_wave(red);
        if (tid == 0)
            scale_sh = norm_scale(total, K, eps);
    }
    __syncthreads();
    const float sc = scale_sh;
    // The weights go out now, behind the activation's loads.
    const uint8_t *qs_row = W + ((size_t)tile * B * kTileRows + r) * kChunk;
    const uint8_t *d_row = W + plane0_bytes + ((size_t)tile * DC * kTileRows + r) * kChunk;
    const int st = wave * kSlots + lane / R;
    uint4 wq[kStretch], dch;
    if (wave * kSlots < S) {  // wavefronts past the last stretch load nothing
        const int s = min(st, S - 1);
#pragma unroll
        for (int j = 0; j < kStretch; j++)
            wq[j] = load_stream(qs_row + (size_t)min(s * kStretch + j, B - 1) * kTileRows * kChunk);
        dch = *(const uint4 *)(d_row + (size_t)s * kTileRows * kChunk);
    }
    // Q8_0: thread i quantises values 4i .. 4i+3, eight threads a block.
    {
        const float4 xv = ((const float4 *)xs)[min(tid, n4 - 1)];
        const float xa[4] = {xv.x, xv.y, xv.z, xv.w}, ga[4] = {gv.x, gv.y, gv.z, gv.w};
        float v[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float nv = xa[k] * sc;
            v[k] = nv * ga[k];
        }
        float bstored;
        int32_t bsum;
        const uint32_t aq = q8_0_quad(v, &bstored, &bsum);
        if (tid < n4) {
            ((uint32_t *)qa)[tid] = aq;
            if ((tid & 7) == 0) {
                sa[tid >> 3] = bstored;
                qsa[tid >> 3] = bsum;
            }
        }
    }
    lds_barrier();

    // The lane's stretch, from +0 in block order.
    if (st < S) {
        const int b0 = st * kStretch;
        const int nb = min(kStretch, B - b0);
        float p = 0.0f;
#pragma unroll
        for (int j = 0; j < kStretch; j++) {
            if (j < nb) {
                const int b = b0 + j;
                const int4 *ap = (const int4 *)(qa + (size_t)b * kQ4Block);
                const int32_t isum = q4_0_block_isum(wq[j], ap[0], ap[1], qsa[b]);
                const float scl = chunk_half(dch, j) * sa[b];
                p = fmaf((float)isum, scl, p);
                if (DOTS && in_range)
                    dots[(size_t)(row - row_start) * B + b] = isum;
            }
        }
        part[st * R + lane % R] = p;
    }
    lds_barrier();
    if (!DOTS && wave == 0 && lane < R && in_range) {
        float acc = 0.0f;
        for (int t = 0; t < S; t++)
            acc = acc + part[t * R + lane];
        y[row] = acc;
    }
}

template <int NC>
int launch_nc(gx_ctx *ctx, const gx_weight *w, const uint8_t *mat, const int8_t *q, const float *scales,
              const int32_t *qsum, int row_start, int row_end, const float *bias, float *y, int ldy,
              int32_t *dots) {
    const int B = w->blocks;
    const int S = (B + kStretch - 1) / kStretch;
    const int waves = min(S, 16);
    const size_t lds = (size_t)S * NC * kTileRows * sizeof(float);
    GX_CHECK(lds <= 64 * 1024, "gx: a %d-input Q4_0 row is wider than this kernel's LDS", w->cols);
    const int tile0 = row_start / kTileRows;
    const int grid = (row_end + kTileRows - 1) / kTileRows - tile0;
    if (dots)
        q4_0_matvec_kernel<NC, false, true><<<grid, 64 * waves, lds, ctx->stream>>>(
            mat, w->plane0_bytes, B, w->dchunks, q, scales, qsum, w->cols, tile0, row_start, row_end, bias, y, ldy,
            nullptr, 0, 1, 0, dots);
    else
        q4_0_matvec_kernel<NC, false, false><<<grid, 64 * waves, lds, ctx->stream>>>(
            mat, w->plane0_bytes, B, w->dchunks, q, scales, qsum, w->cols, tile0, row_start, row_end, bias, y, ldy,
            nullptr, 0, 1, 0, nullptr);
    return check_launch("q4_0_matvec");
}

// The one-column LDS kernel runs a quarter tile a workgroup, its
// wavefronts covering the row's stretches in one pass (IT = 1) or two.
constexpr int kLdsRows = 16;

bool lds_fits(const gx_weight *w, int *it, int *waves, size_t *lds) {
    const int B = w->blocks, K = w->cols, S = (B + kStretch - 1) / kStretch;
    constexpr int slots = kTileRows / kLdsRows;
    for (int IT = 1; IT <= 2; IT++) {
        const int wv = (S + slots * IT - 1) / (slots * IT);
        const int nt = 64 * wv;
        const size_t bytes = lds_part_bytes(S, kLdsRows) + lds_act_bytes(K, B);
        if (wv <= 16 && K / 16 <= kActRegs * nt && B <= kActRegs * nt && bytes <= 64 * 1024) {
            *it = IT;
            *waves = wv;
            *lds = bytes;
            return true;
        }
    }
    return false;
}

// The multi-column kernel's shape for NC columns: whole tiles when they
// give enough workgroups to keep most CUs fetching, else half or quarter
// tiles; every stretch in one pass of at most 16 wavefronts; LDS within
// 64 KiB.
bool cols_shape(const gx_ctx *ctx, const gx_weight *w, int tiles, int NC, int *R, int *waves, size_t *lds) {
    const int B = w->blocks, K = w->cols, S = (B + kStretch - 1) / kStretch;
    const int want = ctx->cu_count * 3 / 5;
    const int rs[3] = {64, 32, 16};
    for (int i = 0; i < 3; i++) {
        const int r = rs[i], slots = kTileRows / r;
        const int wv = (S + slots - 1) / slots;
        const size_t bytes = cols_lds_bytes(S, r, NC, K, B);
        if (wv > 16 || bytes > 64 * 1024)
            continue;
        if (tiles * slots >= want || r == 16) {
            *R = r;
            *waves = wv;
            *lds = bytes;
            return true;
        }
    }
    return false;
}

template <int NC>
int launch_cols(gx_ctx *ctx, const gx_weight *w, const uint8_t *mat, const int8_t *q, const float *scales,
                const int32_t *qsum, int R, int waves, size_t lds, int row_start, int row_end, const float *bias,
                float *y, int ldy, int32_t *dots) {
    const int tile0 = row_start / kTileRows;
    const int tiles = (row_end + kTileRows - 1) / kTileRows - tile0;
    const int slots = kTileRows / R;
    const unsigned grid = (unsigned)(tiles * slots), threads = (unsigned)(64 * waves);
#define GX_COLS(RR, DD)                                                                                              \
    q4_0_matvec_cols_kernel<RR, NC, DD><<<grid, threads, lds, ctx->stream>>>(                                        \
        mat, w->plane0_bytes, w->blocks, w->dchunks, q, scales, qsum, tile0 * slots, row_start, row_end, bias, y,    \
        ldy, dots)
    if (R == 64 && dots)
        GX_COLS(64, true);
    else if (R == 64)
        GX_COLS(64, false);
    else if (R == 32 && dots)
        GX_COLS(32, true);
    else if (R == 32)
        GX_COLS(32, false);
    else if (dots)
        GX_COLS(16, true);
    else
        GX_COLS(16, false);
#undef GX_COLS
    return check_launch("q4_0_matvec_cols");
}

template <int NC>
int launch_cols_swiglu(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const float *scales, const int32_t *qsum,
                       int waves, size_t lds, int8_t *mq, float *ms, int32_t *mqs) {
    q4_0_matvec_cols_kernel<kTileRows, NC, false, 1><<<w->tiles, 64 * waves, lds, ctx->stream>>>(
        w->dev, w->plane0_bytes, w->blocks, w->dchunks, q, scales, qsum, 0, 0, w->rows, nullptr, nullptr, 0, nullptr,
        mq, ms, mqs);
    return check_launch("q4_0_matvec_cols_swiglu");
}

// The few-column MFMA product: R = 16 rows a workgroup (EPI 0) or whole
// tiles (EPI 1), a wavefront a (row group, stretch) unit at a time.
size_t mfma_cols_lds(const gx_weight *w, int M, int R) {
    const int S = (w->blocks + kStretch - 1) / kStretch;
    return (size_t)S * M * R * sizeof(float);
}

int launch_mfma_cols(gx_ctx *ctx, const gx_weight *w, const uint8_t *mat, const int8_t *q, const float *scales, int M,
                     int row_start, int row_end, const float *bias, float *y, int ldy, int32_t *dots) {
    const int B = w->blocks, S = (B + kStretch - 1) / kStretch;
    const int tile0 = row_start / kTileRows;
    const int tiles = (row_end + kTileRows - 1) / kTileRows - tile0;
    // One stretch a wavefront: the form with the weights through LDS, 32-row
    // workgroups for a matrix of 64 tiles or more (config 3 at 8 columns,
    // graph of launches over rotating copies: Q|K|V 8.1 -> 6.6 us, Gate|Up
    // 17.6 -> 13.7, O 6.7 -> 6.4).
    if (S <= 16) {
        const int RG = tiles >= 64 ? 2 : 1;
        const size_t bytes = std::max(mfma_dma_ring_offset(M, w->cols, B) + (size_t)S * 2 * kMfmaSlotB,
                                      mfma_cols_lds(w, M, 16 * RG));
        if (bytes <= kLdsMax) {
            const int slots = kTileRows / (16 * RG);
            const unsigned grid = (unsigned)(tiles * slots), threads = (unsigned)(64 * S);
#define GX_MD(RR, DD)                                                                                                \
    q4_0_mfma_cols_dma_kernel<RR, 0, DD><<<grid, threads, bytes, ctx->stream>>>(                                     \
        mat, w->plane0_bytes, B, w->dchunks, q, scales, M, tile0 * slots, row_start, row_end, bias, y, ldy, dots,    \
        nullptr, nullptr, nullptr)
            if (RG == 2 && dots)
                GX_MD(2, true);
            else if (RG == 2)
                GX_MD(2, false);
            else if (dots)
                GX_MD(1, true);
            else
                GX_MD(1, false);
#undef GX_MD
            return check_launch("q4_0_mfma_cols_dma");
        }
    }
    // Up to three stretches a wavefront: weights into registers (config 3's
    // Down at 8 columns 13.7 -> 12.2 us against the unstaged form).
    const int SW = (S + 15) / 16;
    const size_t staged = std::max(mfma_lds_act_bytes(M, w->cols, B), mfma_cols_lds(w, M, 16));
    if (SW <= 3 && staged <= kLdsMax) {
        const unsigned grid = (unsigned)(tiles * 4), threads = (unsigned)(64 * min(S, 16));
#define GX_MF(SS, DD)                                                                                                \
    q4_0_mfma_cols_lds_kernel<SS, DD><<<grid, threads, staged, ctx->stream>>>(                                       \
        mat, w->plane0_bytes, B, w->dchunks, q, scales, M, tile0 * 4, row_start, row_end, bias, y, ldy, dots)
        if (SW <= 2 && dots)
            GX_MF(2, true);
        else if (SW <= 2)
            GX_MF(2, false);
        else if (dots)
            GX_MF(3, true);
        else
            GX_MF(3, false);
#undef GX_MF
        return check_launch("q4_0_mfma_cols_lds");
    }
    constexpr int kSlots = kTileRows / 16;
    const unsigned grid = (unsigned)(tiles * kSlots), threads = (unsigned)(64 * min(S, 16));
    const size_t lds = mfma_cols_lds(w, M, 16);
    if (dots)
        q4_0_mfma_cols_kernel<1, 0, true><<<grid, threads, lds, ctx->stream>>>(
            mat, w->plane0_bytes, w->blocks, w->dchunks, q, scales, M, tile0 * kSlots, row_start, row_end, bias, y,
            ldy, dots, nullptr, nullptr, nullptr);
    else
        q4_0_mfma_cols_kernel<1, 0, false><<<grid, threads, lds, ctx->stream>>>(
            mat, w->plane0_bytes, w->blocks, w->dchunks, q, scales, M, tile0 * kSlots, row_start, row_end, bias, y,
            ldy, nullptr, nullptr, nullptr, nullptr);
    return check_launch("q4_0_mfma_cols");
}

}  // namespace

int launch_q4_0_matvec(gx_ctx *ctx, const gx_weight *w, const uint8_t *mat, const int8_t *q, const float *scales,
                       const int32_t *qsum, int M, int row_start, int row_end, const float *bias, float *y,
                       int ldy, int32_t *dots, int form) {
    const int tile0 = row_start / kTileRows;
    const int tiles = (row_end + kTileRows - 1) / kTileRows - tile0;
    // One column of a matrix with few tiles (at most a quarter as many as
    // CUs), or when asked (form 1): quarter tiles.  Measured in a graph of
    // launches over rotating copies: O 2560 x 4096 5.7 -> 4.5 us, Down
    // 2560 x 9728 9.8 -> 6.8 us; with 152 tiles (config 0) the whole-tile
    // kernel stays ahead (5.4 against 6.1 us).
    if (M == 1 && form != 0 && (form == 1 || tiles * 4 <= ctx->cu_count)) {
        int IT, waves;
        size_t lds;
        if (lds_fits(w, &IT, &waves, &lds)) {
            constexpr int slots = kTileRows / kLdsRows;
            const unsigned grid = (unsigned)(tiles * slots), threads = (unsigned)(64 * waves);
#define GX_LDS(II, DD)                                                                                               \
    q4_0_matvec_lds_kernel<kLdsRows, II, DD><<<grid, threads, lds, ctx->stream>>>(                                   \
        mat, w->plane0_bytes, w->blocks, w->dchunks, q, scales, qsum, tile0 * slots, row_start, row_end, bias, y, dots)
            if (IT == 1 && !dots)
                GX_LDS(1, false);
            else if (IT == 1)
                GX_LDS(1, true);
            else if (!dots)
                GX_LDS(2, false);
            else
                GX_LDS(2, true);
#undef GX_LDS
            return check_launch("q4_0_matvec_lds");
        }
        GX_CHECK(form != 1, "gx: a %d-input Q4_0 row does not fit the one-column kernel", w->cols);
    }
    const int K = w->cols, B = w->blocks;
    const size_t nrows = (size_t)(row_end - row_start);
    // Two to eight columns (or form 2): the LDS-staged kernel, columns in
    // groups of 8, 4, 2, 1 as its LDS allows, each group reading the weights
    // once.  Measured at config 3's shapes and M = 8 (eight lock-step
    // conversations, kernel trace), against the whole-tile kernel: Down
    // 2 x 21.6 -> 2 x 11.7 us, O 17.7 -> 12.4, Q|K|V 15.8 -> 13.7, Gate|Up
    // 27.8 -> 28.7 (whole tiles either way).
    // 2..16 columns (or form 3): the per-block integers on the matrix cores.
    if (((M >= 2 && form < 0) || form == 3) && M <= kMfmaCols && mfma_cols_lds(w, M, 16) <= 64 * 1024)
        return launch_mfma_cols(ctx, w, mat, q, scales, M, row_start, row_end, bias, y, ldy, dots);
    GX_CHECK(form != 3, "gx: %d columns of %d inputs do not fit the few-column MFMA kernel", M, w->cols);
    if ((M >= 2 && form != 0) || form == 2) {
        int c = 0;
        while (c < M) {
            const int left = M - c;
            int NC = 0, R = 0, waves = 0;
            size_t lds = 0;
            const int widths[4] = {8, 4, 2, 1};
            for (int i = 0; i < 4 && NC == 0; i++)
                if (widths[i] <= left && cols_shape(ctx, w, tiles, widths[i], &R, &waves, &lds))
                    NC = widths[i];
            if (NC == 0)
                break;  // too wide for the LDS: the whole-tile kernel below
            const int8_t *qc = q + (size_t)c * K;
            const float *sc = scales + (size_t)c * B;
            const int32_t *qs = qsum + (size_t)c * B;
            float *yc = y ? y + (size_t)c * ldy : nullptr;
            int32_t *dc = dots ? dots + (size_t)c * nrows * B : nullptr;
            int rc;
            if (NC == 8)
                rc = launch_cols<8>(ctx, w, mat, qc, sc, qs, R, waves, lds, row_start, row_end, bias, yc, ldy, dc);
            else if (NC == 4)
                rc = launch_cols<4>(ctx, w, mat, qc, sc, qs, R, waves, lds, row_start, row_end, bias, yc, ldy, dc);
            else if (NC == 2)
                rc = launch_cols<2>(ctx, w, mat, qc, sc, qs, R, waves, lds, row_start, row_end, bias, yc, ldy, dc);
            else
                rc = launch_cols<1>(ctx, w, mat, qc, sc, qs, R, waves, lds, row_start, row_end, bias, yc, ldy, dc);
            if (rc)
                return rc;
            c += NC;
        }
        if (c == M)
            return GX_OK;
        GX_CHECK(form != 2, "gx: a %d-input Q4_0 row does not fit the multi-column kernel", w->cols);
        q += (size_t)c * K;
        scales += (size_t)c * B;
        qsum += (size_t)c * B;
        if (y)
            y += (size_t)c * ldy;
        if (dots)
            dots += (size_t)c * nrows * B;
        M -= c;
    }
    // Columns in groups of 8, 4, 2, 1 on whole tiles with the activation in
    // scalar registers, each group reading the weights once; the per-column
    // arithmetic is the same whatever the group.  Very wide rows keep the
    // group narrow enough for the stretch sums to fit in LDS.
    int c = 0;
    const size_t per_column = (size_t)((B + kStretch - 1) / kStretch) * kTileRows * sizeof(float);
    const int widest = per_column * 8 <= 64 * 1024 ? 8 : per_column * 4 <= 64 * 1024 ? 4
                     : per_column * 2 <= 64 * 1024 ? 2 : 1;
    while (c < M) {
        const int left = M - c;
        const int8_t *qc = q + (size_t)c * K;
        const float *sc = scales + (size_t)c * B;
        const int32_t *qs = qsum + (size_t)c * B;
        float *yc = y ? y + (size_t)c * ldy : nullptr;
        int32_t *dc = dots ? dots + (size_t)c * nrows * B : nullptr;
        int rc;
        if (left >= 8 && widest >= 8) {
            rc = launch_nc<8>(ctx, w, mat, qc, sc, qs, row_start, row_end, bias, yc, ldy, dc);
            c += 8;
        } else if (left >= 4 && widest >= 4) {
            rc = launch_nc<4>(ctx, w, mat, qc, sc, qs, row_start, row_end, bias, yc, ldy, dc);
            c += 4;
        } else if (left >= 2 && widest >= 2) {
            rc = launch_nc<2>(ctx, w, mat, qc, sc, qs, row_start, row_end, bias, yc, ldy, dc);
            c += 2;
        } else {
            rc = launch_nc<1>(ctx, w, mat, qc, sc, qs, row_start, row_end, bias, yc, ldy, dc);
            c += 1;
        }
        if (rc)
            return rc;
    }
    return GX_OK;
}

int launch_q4_0_matvec_swiglu(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const float *scales,
                               const int32_t *qsum, int M, int8_t *mq, float *ms, int32_t *mqs) {
    const int K = w->cols, B = w->blocks, S = (B + kStretch - 1) / kStretch, F = w->rows / 2;
    const size_t ringed = std::max(mfma_dma_ring_offset(M, K, B) + (size_t)S * 2 * kMfmaSlotB,
                                   mfma_cols_lds(w, M, kTileRows));
    if (M <= kMfmaCols && S <= 16 && ringed <= kLdsMax) {
        // (config 3's Gate|Up at 8 columns: 22.0 us with the weights in
        // registers, 17.0 through LDS)
        q4_0_mfma_cols_dma_kernel<4, 1, false><<<w->tiles, 64 * S, ringed, ctx->stream>>>(
            w->dev, w->plane0_bytes, B, w->dchunks, q, scales, M, 0, 0, w->rows, nullptr, nullptr, 0, nullptr, mq, ms,
            mqs);
        return check_launch("q4_0_mfma_cols_dma_swiglu");
    }
    if (M <= kMfmaCols && mfma_cols_lds(w, M, kTileRows) <= 64 * 1024) {
        q4_0_mfma_cols_kernel<4, 1, false><<<w->tiles, 64 * min(4 * S, 16), mfma_cols_lds(w, M, kTileRows),
                                              ctx->stream>>>(w->dev, w->plane0_bytes, B, w->dchunks, q, scales, M,
                                                             0, 0, w->rows, nullptr, nullptr, 0, nullptr, mq, ms,
                                                             mqs);
        return check_launch("q4_0_mfma_cols_swiglu");
    }
    GX_CHECK(S <= 16, "gx: a %d-input row is too wide for the multi-column SwiGLU product", K);
    int c = 0;
    while (c < M) {
        const int left = M - c;
        const int widths[4] = {8, 4, 2, 1};
        int NC = 0;
        size_t lds = 0;
        for (int i = 0; i < 4 && NC == 0; i++) {
            const size_t bytes = cols_lds_bytes(S, kTileRows, widths[i], K, B);
            if (widths[i] <= left && bytes <= 64 * 1024) {
                NC = widths[i];
                lds = bytes;
            }
        }
        GX_CHECK(NC > 0, "gx: a %d-input row does not fit the multi-column SwiGLU product", K);
        const int8_t *qc = q + (size_t)c * K;
        const float *sc = scales + (size_t)c * B;
        const int32_t *qs = qsum + (size_t)c * B;
        int8_t *mqc = mq + (size_t)c * F;
        float *msc = ms + (size_t)c * (F / kQ4Block);
        int32_t *mqsc = mqs + (size_t)c * (F / kQ4Block);
        int rc;
        if (NC == 8)
            rc = launch_cols_swiglu<8>(ctx, w, qc, sc, qs, S, lds, mqc, msc, mqsc);
        else if (NC == 4)
            rc = launch_cols_swiglu<4>(ctx, w, qc, sc, qs, S, lds, mqc, msc, mqsc);
        else if (NC == 2)
            rc = launch_cols_swiglu<2>(ctx, w, qc, sc, qs, S, lds, mqc, msc, mqsc);
        else
            rc = launch_cols_swiglu<1>(ctx, w, qc, sc, qs, S, lds, mqc, msc, mqsc);
        if (rc)
            return rc;
        c += NC;
    }
    return GX_OK;
}

int launch_q4_0_matvec_units(gx_ctx *ctx, const gx_weight *w, const int32_t *unit_expert, int units, int act_div,
                              const int8_t *q, const float *scales, const int32_t *qsum, float *y, int ldy,
                              int32_t *dots) {
    const int B = w->blocks;
    const int S = (B + kStretch - 1) / kStretch;
    const int waves = min(S, 16);
    const size_t lds = (size_t)S * kTileRows * sizeof(float);
    GX_CHECK(lds <= 64 * 1024, "gx: a %d-input Q4_0 row is wider than this kernel's LDS", w->cols);
    dim3 grid(w->tiles, units);
    if (dots)
        q4_0_matvec_kernel<1, true, true><<<grid, 64 * waves, lds, ctx->stream>>>(
            w->dev, w->plane0_bytes, B, w->dchunks, q, scales, qsum, w->cols, 0, 0, w->rows, nullptr, y, ldy,
            unit_expert, w->matrix_bytes, act_div, w->count, dots);
    else
        q4_0_matvec_kernel<1, true, false><<<grid, 64 * waves, lds, ctx->stream>>>(
            w->dev, w->plane0_bytes, B, w->dchunks, q, scales, qsum, w->cols, 0, 0, w->rows, nullptr, y, ldy,
            unit_expert, w->matrix_bytes, act_div, w->count, nullptr);
    return check_launch("q4_0_matvec_units");
}

int launch_q4_0_matvec_fused(gx_ctx *ctx, const gx_weight *w, int epi, int row_start, int row_end, float *y,
                              const float *x, const float *add, const float *gain, float eps, float *x_out,
                              int8_t *q, float *scales, int32_t *qsum, int32_t *dots) {
    const int B = w->blocks, K = w->cols;
    const int S = (B + kStretch - 1) / kStretch;
    const int tile0 = row_start / kTileRows;
    const int grid = (row_end + kTileRows - 1) / kTileRows - tile0;
    // Without the SwiGLU epilogue, a matrix whose whole tiles would fill at
    // most half the CUs runs on half tiles (measured in a graph of launches
    // over rotating copies, config 3's Q|K|V: 6.56 -> 6.29 us; quarter tiles
    // 6.97, eighth tiles 9.8: every workgroup makes the whole activation).
    {
        constexpr int R = 32, slots = kTileRows / R;
        const int waves = max((K / 4 + 63) / 64, (S + slots - 1) / slots);
        const size_t lds = lds_part_bytes(S, R) + (size_t)K * sizeof(float) + lds_act_bytes(K, B);
        if (epi == 0 && grid * slots <= ctx->cu_count && waves <= 16 && lds <= 56 * 1024 &&
            ((uintptr_t)w->dev & 15) == 0 && ((uintptr_t)gain & 15) == 0) {
            if (dots)
                q4_0_matvec_fused_lds_kernel<R, true><<<grid * slots, 64 * waves, lds, ctx->stream>>>(
                    w->dev, w->plane0_bytes, B, w->dchunks, tile0 * slots, row_start, row_end, y, x, add, gain, eps,
                    x_out, dots);
            else
                q4_0_matvec_fused_lds_kernel<R, false><<<grid * slots, 64 * waves, lds, ctx->stream>>>(
                    w->dev, w->plane0_bytes, B, w->dchunks, tile0 * slots, row_start, row_end, y, x, add, gain, eps,
                    x_out, nullptr);
            return check_launch("q4_0_matvec_fused_lds");
        }
    }
    const int waves = min(S, 16);
    const size_t lds = ((size_t)S * kTileRows + K) * sizeof(float);
    GX_CHECK(lds <= 56 * 1024, "gx: a %d-input Q4_0 row is wider than this kernel's LDS", K);
#define GX_FUSED(E, D, DD)                                                                                           \
    q4_0_matvec_fused_kernel<E, D, DD><<<grid, 64 * waves, lds, ctx->stream>>>(                                      \
        w->dev, w->plane0_bytes, B, w->dchunks, K, tile0, row_start, row_end, y, x, add, gain, eps, x_out, q, scales, \
        qsum, dots)
#define GX_FUSED_D(E, D)                                                                                             \
    do {                                                                                                             \
        if (dots)                                                                                                    \
            GX_FUSED(E, D, true);                                                                                    \
        else                                                                                                         \
            GX_FUSED(E, D, false);                                                                                   \
    } while (0)
    const bool db = S > waves;
    if (epi == 0 && !db)
        GX_FUSED_D(0, false);
    else if (epi == 0)
        GX_FUSED_D(0, true);
    else if (!db)
        GX_FUSED_D(1, false);
    else
        GX_FUSED_D(1, true);
#undef GX_FUSED_D
#undef GX_FUSED
    return check_launch("q4_0_matvec_fused");
}

}  // namespace gx
