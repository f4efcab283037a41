/*
 * oracle.c - CPU restatement of golem's generic (portable) Go arithmetic for
 * the quantized linear-layer path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in golem_amd/ links, loads or calls this
 * file.  It is the checker the GPU path is compared against: pytest, the smoke
 * check and bench.py's cpu_baseline leg are its only users.
 *
 * Float semantics.  golem is compiled by gc for amd64 at GOAMD64=v1: float32
 * operations are SSE scalar operations, each rounded to float32, evaluated
 * left to right, with no fused multiply-add.  This file is built with
 * `gcc -O2 -ffp-contract=off` and no -march, which gives exactly that
 * (FLT_EVAL_METHOD == 0 on x86-64).  Every expression below keeps the
 * parenthesisation golem's source implies.
 *
 * Layouts follow golem's nn.Batch (nn/batch.go:17-45):
 *   Q      int8   [block][column][32]   (interleaved by column, stride = Stride)
 *   Scales float  [block][column]
 *   Corr   float  [block][column]
 *   QK     int8   [column][width]
 *   KScales float [column][width/256]
 *   BSums  int16  [column][width/16]
 * Outputs ys are [column][ldy] float32 (golem's ys[c][r]).
 *
 * Citations are file:line in ThiraSoft/golem.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define QUANT_BLOCK 32         /* nn/quant.go:50 */
#define Q4_0_BLOCK_BYTES 18    /* nn/quant.go:52 */
#define SUPER_BLOCK 256        /* nn/quant.go:54 */
#define Q6_K_BLOCK_BYTES 210   /* nn/quant.go:56 */
#define PACKED_ROWS 8          /* nn/pack_q4_0.go:41 */
#define PACKED_BLOCK_BYTES 144 /* nn/pack_q4_0.go:44 */
#define K_TILE 2048            /* nn/dot_q4_0.go:148 */
#define ROW_TILE_BYTES (24 * 1024) /* nn/dot_q4_0.go:150 */
#define MAX_ROW_TILE 64        /* nn/dot_q4_0.go:151 */
#define MAX_GROUP_TILE 8       /* nn/pack_q4_0.go:152 */

enum { ORC_F32 = 0, ORC_BF16 = 1, ORC_Q4_0 = 2, ORC_Q6_K = 3 }; /* nn/quant.go:12-17 */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint16_t le16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline int imin(int a, int b) { return a < b ? a : b; }
static inline int imax(int a, int b) { return a > b ? a : b; }

/* ---- fp16 ------------------------------------------------------------- */

/* halfToFloat, nn/dot_q4_0.go:21-43: exact widening, subnormals normalised by
 * hand, infinities and NaNs kept. */
float orc_half_to_float(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    uint32_t exponent = (h >> 10) & 0x1F;
    uint32_t mantissa = h & 0x03FF;
    if (exponent == 0) {
        if (mantissa == 0)
            return u2f(sign);
        uint32_t e = 127 - 15 + 1;
        while ((mantissa & 0x0400) == 0) {
            mantissa <<= 1;
            e--;
        }
        mantissa &= 0x03FF;
        return u2f(sign | e << 23 | mantissa << 13);
    }
    if (exponent == 0x1F)
        return u2f(sign | 0xFFu << 23 | mantissa << 13);
    return u2f(sign | (exponent + 127 - 15) << 23 | mantissa << 13);
}

/* floatToHalf, nn/half.go:8-38: round to nearest even, NaN -> 0x7E00 with
 * sign, overflow -> infinity, subnormals rounded. */
uint16_t orc_float_to_half(float f)
{
    uint32_t bits = f2u(f);
    uint16_t sign = (uint16_t)((bits >> 16) & 0x8000);
    int32_t exponent = (int32_t)((bits >> 23) & 0xFF) - 127 + 15;
    uint32_t mantissa = bits & 0x7FFFFF;

    if ((bits & 0x7FFFFFFF) == 0)
        return sign;
    if (exponent >= 0x1F) {
        if ((bits & 0x7F800000) == 0x7F800000 && mantissa != 0)
            return sign | 0x7E00;
        return sign | 0x7C00;
    }
    if (exponent <= 0) {
        if (exponent < -10)
            return sign;
        mantissa |= 0x800000;
        uint32_t shift = (uint32_t)(14 - exponent);
        uint16_t half = (uint16_t)(mantissa >> shift);
        uint32_t remainder = mantissa & ((1u << shift) - 1);
        if (remainder > (1u << (shift - 1)) || (remainder == (1u << (shift - 1)) && (half & 1) == 1))
            half++;
        return sign | half;
    }
    uint16_t half = (uint16_t)((uint32_t)exponent << 10 | (mantissa >> 13));
    uint32_t remainder = mantissa & 0x1FFF;
    if (remainder > 0x1000 || (remainder == 0x1000 && (half & 1) == 1))
        half++;
    return sign | half;
}

/* RoundHalf, nn/half.go:48 */
float orc_round_half(float v) { return orc_half_to_float(orc_float_to_half(v)); }

/* RoundHalf over n values in place (the cache entries and queries of a
 * head, qwen/attention.go:67, qwen/cache.go:52-60). */
void orc_round_half_n(float *x, int n)
{
    for (int i = 0; i < n; i++)
        x[i] = orc_round_half(x[i]);
}

/* nearestInt, nn/batch.go:221-224: adding 1.5*2^23 leaves the rounded
 * integer in the low mantissa bits (valid for |f| < 2^22). */
int32_t orc_nearest_int(float f)
{
    const float magic = 12582912.0f;
    float s = f + magic;
    return (int32_t)(f2u(s) & 0x007fffff) - 0x00400000;
}

/* ---- activation quantisers -------------------------------------------- */

/* Batch.quantizeBlock, nn/batch.go:109-143.  F is [size][width] row-major
 * (golem's b.F[column]). */
static void quantize_block(const float *F, int width, int stride, int8_t *Q,
                           float *Scales, float *Corr, int block, int column)
{
    const float *values = F + (size_t)column * width + (size_t)block * QUANT_BLOCK;
    size_t index = (size_t)block * stride + column;
    int8_t *q = Q + index * QUANT_BLOCK;

    float peak = 0;
    for (int i = 0; i < QUANT_BLOCK; i++) {
        float a = fabsf(values[i]);
        if (a > peak)
            peak = a;
    }
    if (peak == 0) {
        Scales[index] = 0;
        Corr[index] = 0;
        memset(q, 0, QUANT_BLOCK);
        return;
    }
    float scale = peak / 127;
    float inverse = 127 / peak;
    Scales[index] = orc_half_to_float(orc_float_to_half(scale));

    int32_t sum = 0;
    for (int i = 0; i < QUANT_BLOCK; i++) {
        int32_t n = orc_nearest_int(values[i] * inverse);
        if (n > 127)
            n = 127;
        else if (n < -128)
            n = -128;
        q[i] = (int8_t)n;
        sum += n;
    }
    Corr[index] = 8 * Scales[index] * (float)sum;
}

/* Batch.QuantizeRange, nn/batch.go:74-85 (Quantize = QuantizeRange(0, Width),
 * :69).  Returns -1 for the panic on a range that is not block aligned. */
int orc_quantize_range(const float *F, int width, int size, int stride, int8_t *Q,
                       float *Scales, float *Corr, int first, int last)
{
    if (first % QUANT_BLOCK != 0 || last % QUANT_BLOCK != 0)
        return -1;
    for (int block = first / QUANT_BLOCK; block < last / QUANT_BLOCK; block++)
        for (int c = 0; c < size; c++)
            quantize_block(F, width, stride, Q, Scales, Corr, block, c);
    return 0;
}

/* Batch.QuantizeColumnRange, nn/batch.go:91-103 (without the BF16 rounding,
 * which only bfloat16 weights ask for). */
void orc_quantize_column_range(const float *F, int width, int stride, int8_t *Q,
                               float *Scales, float *Corr, int column, int first, int last)
{
    for (int block = first / QUANT_BLOCK; block < last / QUANT_BLOCK; block++)
        quantize_block(F, width, stride, Q, Scales, Corr, block, column);
}

/* Batch.QuantizeK, nn/batch.go:159-213.  Returns -1 for the panic on a width
 * that is not a whole number of superblocks. */
int orc_quantize_k(const float *F, int width, int size, int8_t *QK, float *KScales, int16_t *BSums)
{
    if (width % SUPER_BLOCK != 0)
        return -1;
    int nsb = width / SUPER_BLOCK;
    for (int c = 0; c < size; c++) {
        int8_t *q = QK + (size_t)c * width;
        float *scales = KScales + (size_t)c * nsb;
        int16_t *sums = BSums + (size_t)c * (width / 16);
        for (int block = 0; block < nsb; block++) {
            const float *values = F + (size_t)c * width + (size_t)block * SUPER_BLOCK;
            int8_t *into = q + (size_t)block * SUPER_BLOCK;
            float peak = 0, extreme = 0;
            for (int i = 0; i < SUPER_BLOCK; i++) {
                float a = values[i];
                if (a < 0)
                    a = -a;
                if (a > peak) {
                    peak = a;
                    extreme = values[i];
                }
            }
            if (peak == 0) {
                scales[block] = 0;
                memset(into, 0, SUPER_BLOCK);
                memset(sums + block * (SUPER_BLOCK / 16), 0, sizeof(int16_t) * (SUPER_BLOCK / 16));
                continue;
            }
            float inverse = -128 / extreme;
            for (int i = 0; i < SUPER_BLOCK; i++) {
                int32_t n = orc_nearest_int(values[i] * inverse);
                if (n > 127)
                    n = 127;
                into[i] = (int8_t)n;
            }
            scales[block] = 1 / inverse;
            for (int g = 0; g < SUPER_BLOCK / 16; g++) {
                int32_t sum = 0;
                for (int i = 0; i < 16; i++)
                    sum += into[g * 16 + i];
                sums[block * (SUPER_BLOCK / 16) + g] = (int16_t)sum;
            }
        }
    }
    return 0;
}

/* ---- Q4_0, row layout ------------------------------------------------- */

/* The per-block integer of dotQ4_0Go (nn/dot_q4_0.go:58-63): unsigned nibbles,
 * low nibble of byte j is weight j, high nibble is weight j+16. */
static inline int32_t q4_0_block_acc(const uint8_t *nibbles, const int8_t *q)
{
    int32_t accumulator = 0;
    for (int j = 0; j < QUANT_BLOCK / 2; j++) {
        uint8_t byte_value = nibbles[j];
        int32_t low = byte_value & 0x0F;
        int32_t high = byte_value >> 4;
        accumulator += low * (int32_t)q[j] + high * (int32_t)q[j + 16];
    }
    return accumulator;
}

/* The same integer, exported for the tests. */
int32_t orc_q4_0_acc(const uint8_t *nibbles, const int8_t *q) { return q4_0_block_acc(nibbles, q); }

/* dotQ4_0Go, nn/dot_q4_0.go:49-70: one row against one column over n inputs
 * beginning at block `first`; adds into state[0] (sum) and state[8]
 * (correction). */
void orc_dot_q4_0_go(const uint8_t *w, const int8_t *Q, const float *Scales, const float *Corr,
                     int stride, int first, int column, int n, float *state)
{
    float sum = 0, correction = 0;
    for (int step = 0; step < n / QUANT_BLOCK; step++) {
        const uint8_t *bytes = w + (size_t)step * Q4_0_BLOCK_BYTES;
        float scale = orc_half_to_float(le16(bytes));
        size_t index = (size_t)(first + step) * stride + column;
        const int8_t *q = Q + index * QUANT_BLOCK;
        int32_t accumulator = q4_0_block_acc(bytes + 2, q);
        sum += (float)accumulator * scale * Scales[index];
        correction += scale * Corr[index];
    }
    state[0] += sum;
    state[8] += correction;
}

/* fold, nn/dot_q4_0.go:108-114 */
float orc_fold(const float *lanes, float correction)
{
    float h0 = lanes[0] + lanes[4];
    float h1 = lanes[1] + lanes[5];
    float h2 = lanes[2] + lanes[6];
    float h3 = lanes[3] + lanes[7];
    return (h0 + h2) + (h1 + h3) - correction;
}

/* matVecQ4_0Rows with the generic kernels of nn/dot_q4_0_generic.go:5-37,
 * nn/dot_q4_0.go:168-270.  The x4/x8 generic forms call dotQ4_0Go once per
 * column into a fresh state and add it (dot_q4_0.go:74-96), so every
 * (row, column) is: for each k-stretch of kTile inputs, state += stretch sums;
 * then fold.  The row/column tiling only changes the visiting order, not the
 * arithmetic, so it is restated as the per-(row, column) sequence. */
void orc_mat_vec_q4_0_rows(const uint8_t *w, const int8_t *Q, const float *Scales, const float *Corr,
                           int stride, int size, int inputs, float *ys, int ldy, int start, int end)
{
    size_t row_bytes = (size_t)(inputs / QUANT_BLOCK) * Q4_0_BLOCK_BYTES;
    int steps = inputs <= K_TILE ? inputs : K_TILE;
    for (int c = 0; c < size; c++) {
        for (int r = start; r < end; r++) {
            float state[9] = {0};
            for (int k = 0; k < inputs; k += steps) {
                int block = k / QUANT_BLOCK, n = imin(steps, inputs - k);
                orc_dot_q4_0_go(w + r * row_bytes + (size_t)block * Q4_0_BLOCK_BYTES, Q, Scales, Corr,
                                stride, block, c, n, state);
            }
            ys[(size_t)c * ldy + r] = orc_fold(state, state[8]);
        }
    }
}

/* dequantizeQ4_0Row, nn/matrix.go:175-190 */
void orc_dequantize_q4_0_row(const uint8_t *w, int n, float *out)
{
    for (int b = 0; b < n / QUANT_BLOCK; b++) {
        const uint8_t *block = w + (size_t)b * Q4_0_BLOCK_BYTES;
        float scale = orc_half_to_float(le16(block));
        const uint8_t *nibbles = block + 2;
        float *dst = out + (size_t)b * QUANT_BLOCK;
        for (int j = 0; j < QUANT_BLOCK / 2; j++) {
            uint8_t byte_value = nibbles[j];
            dst[j] = (float)((int32_t)(byte_value & 0x0F) - 8) * scale;
            dst[j + 16] = (float)((int32_t)(byte_value >> 4) - 8) * scale;
        }
    }
}

/* ---- Q4_0, eight-row packed layout ------------------------------------ */

static const int low_rows[4] = {0, 1, 4, 5};  /* nn/pack_q4_0.go:54 */
static const int high_rows[4] = {2, 3, 6, 7}; /* nn/pack_q4_0.go:55 */

/* PackedQ4_0Bytes, nn/pack_q4_0.go:65-67 */
size_t orc_packed_q4_0_bytes(int rows, int cols)
{
    return (size_t)(rows / PACKED_ROWS) * (cols / QUANT_BLOCK) * PACKED_BLOCK_BYTES;
}

/* PackQ4_0, nn/pack_q4_0.go:77-110 */
int orc_pack_q4_0(const uint8_t *w, int rows, int cols, uint8_t *out)
{
    if (cols % QUANT_BLOCK != 0)
        return -1;
    int blocks = cols / QUANT_BLOCK;
    size_t row_bytes = (size_t)blocks * Q4_0_BLOCK_BYTES;
    for (int group = 0; group < rows / PACKED_ROWS; group++) {
        int base = group * PACKED_ROWS;
        uint8_t *into = out + (size_t)group * blocks * PACKED_BLOCK_BYTES;
        uint8_t spread[PACKED_ROWS][QUANT_BLOCK];
        for (int b = 0; b < blocks; b++) {
            uint8_t *dst = into + (size_t)b * PACKED_BLOCK_BYTES;
            for (int r = 0; r < PACKED_ROWS; r++) {
                const uint8_t *src = w + (size_t)(base + r) * row_bytes + (size_t)b * Q4_0_BLOCK_BYTES;
                dst[r * 2] = src[0];
                dst[r * 2 + 1] = src[1];
                for (int j = 0; j < QUANT_BLOCK / 2; j++) {
                    spread[r][j] = src[2 + j] & 0x0F;
                    spread[r][j + 16] = src[2 + j] >> 4;
                }
            }
            uint8_t *nibbles = dst + 16;
            for (int g = 0; g < 4; g++) {
                uint8_t *chunk = nibbles + g * 32;
                for (int s = 0; s < 4; s++) {
                    const uint8_t *low = spread[low_rows[s]], *high = spread[high_rows[s]];
                    for (int j = 0; j < 8; j++)
                        chunk[s * 8 + j] = (uint8_t)(low[g * 8 + j] | high[g * 8 + j] << 4);
                }
            }
        }
    }
    return 0;
}

/* dotPackedQ4_0Go, nn/pack_q4_0.go:120-146: eight rows against one column,
 * accumulated into state[0..7]. */
void orc_dot_packed_q4_0_go(const uint8_t *w, const int8_t *Q, const float *Scales, const float *Corr,
                            int stride, int block, int column, int n, float *state)
{
    for (int step = 0; step < n / QUANT_BLOCK; step++) {
        const uint8_t *group = w + (size_t)step * PACKED_BLOCK_BYTES;
        size_t index = (size_t)(block + step) * stride + column;
        const int8_t *q = Q + index * QUANT_BLOCK;
        float activation = Scales[index], correction = Corr[index];

        int32_t sums[PACKED_ROWS] = {0};
        const uint8_t *nibbles = group + 16;
        for (int g = 0; g < 4; g++) {
            const uint8_t *chunk = nibbles + g * 32;
            for (int s = 0; s < 4; s++) {
                for (int j = 0; j < 8; j++) {
                    int32_t value = q[g * 8 + j];
                    uint8_t byte_value = chunk[s * 8 + j];
                    sums[low_rows[s]] += (int32_t)(byte_value & 0x0F) * value;
                    sums[high_rows[s]] += (int32_t)(byte_value >> 4) * value;
                }
            }
        }
        for (int r = 0; r < PACKED_ROWS; r++) {
            float scale = orc_half_to_float(le16(group + r * 2));
            state[r] += (float)sums[r] * (scale * activation);
            state[r] -= scale * correction;
        }
    }
}

/* matVecPackedQ4_0Rows with the generic kernels of nn/pack_q4_0_generic.go:
 * 5-20, nn/pack_q4_0.go:159-221.  The generic form clears the state at the
 * first stretch and then accumulates straight into it, so each (row, column)
 * is one serial pass over the blocks.  Only rows in [start, end) are
 * written. */
void orc_mat_vec_packed_q4_0_rows(const uint8_t *w, const int8_t *Q, const float *Scales, const float *Corr,
                                  int stride, int size, int inputs, float *ys, int ldy, int start, int end)
{
    size_t group_bytes = (size_t)(inputs / QUANT_BLOCK) * PACKED_BLOCK_BYTES;
    int first = start / PACKED_ROWS, last = (end + PACKED_ROWS - 1) / PACKED_ROWS;
    int steps = imin(K_TILE, inputs);
    for (int g = first; g < last; g++) {
        for (int c = 0; c < size; c++) {
            float state[PACKED_ROWS] = {0};
            for (int k = 0; k < inputs; k += steps) {
                int block = k / QUANT_BLOCK, n = imin(steps, inputs - k);
                orc_dot_packed_q4_0_go(w + g * group_bytes + (size_t)block * PACKED_BLOCK_BYTES, Q, Scales,
                                       Corr, stride, block, c, n, state);
            }
            int row = g * PACKED_ROWS;
            for (int r = 0; r < PACKED_ROWS; r++)
                if (row + r >= start && row + r < end)
                    ys[(size_t)c * ldy + row + r] = state[r];
        }
    }
}

/* ---- Q6_K --------------------------------------------------------------- */

/* The per-superblock integer of dotQ6_KGo, nn/dot_q6_k.go:31-51:
 * sum - 32*shift. */
int32_t orc_q6_k_block_isum(const uint8_t *block, const int8_t *activations, const int16_t *group_sums)
{
    const uint8_t *low = block, *high = block + 128, *block_scales = block + 192;
    int32_t sum = 0;
    for (int half = 0; half < 2; half++) {
        const uint8_t *l = low + half * 64, *h = high + half * 32;
        const int8_t *s = (const int8_t *)block_scales + half * 8;
        const int8_t *a = activations + half * 128;
        for (int i = 0; i < 32; i++) {
            int group = i / 16;
            sum += (int32_t)s[group + 0] * ((int32_t)(l[i] & 0x0F) | (int32_t)(h[i] & 3) << 4) * (int32_t)a[i];
            sum += (int32_t)s[group + 2] * ((int32_t)(l[i + 32] & 0x0F) | (int32_t)((h[i] >> 2) & 3) << 4) *
                   (int32_t)a[i + 32];
            sum += (int32_t)s[group + 4] * ((int32_t)(l[i] >> 4) | (int32_t)((h[i] >> 4) & 3) << 4) *
                   (int32_t)a[i + 64];
            sum += (int32_t)s[group + 6] * ((int32_t)(l[i + 32] >> 4) | (int32_t)((h[i] >> 6) & 3) << 4) *
                   (int32_t)a[i + 96];
        }
    }
    int32_t shift = 0;
    for (int g = 0; g < SUPER_BLOCK / 16; g++)
        shift += (int32_t)(int8_t)block_scales[g] * (int32_t)group_sums[g];
    return sum - 32 * shift;
}

/* dotQ6_KGo, nn/dot_q6_k.go:19-54 */
float orc_dot_q6_k_go(const uint8_t *w, const int8_t *q, const int16_t *bsums, const float *scales, int n)
{
    float total = 0;
    for (int b = 0; b < n / SUPER_BLOCK; b++) {
        const uint8_t *block = w + (size_t)b * Q6_K_BLOCK_BYTES;
        float super_scale = orc_half_to_float(le16(block + 208));
        int32_t isum = orc_q6_k_block_isum(block, q + (size_t)b * SUPER_BLOCK, bsums + b * (SUPER_BLOCK / 16));
        total += (float)isum * super_scale * scales[b];
    }
    return total;
}

/* matVecQ6_KRows, nn/dot_q6_k.go:77-103, with the generic dotQ6_Kx2 that
 * declines (nn/dot_q6_k_x2_generic.go:7): one column at a time. */
void orc_mat_vec_q6_k_rows(const uint8_t *w, const int8_t *QK, const float *KScales, const int16_t *BSums,
                           int width, int size, int inputs, float *ys, int ldy, int start, int end)
{
    size_t stride = (size_t)(inputs / SUPER_BLOCK) * Q6_K_BLOCK_BYTES;
    for (int r = start; r < end; r++)
        for (int c = 0; c < size; c++)
            ys[(size_t)c * ldy + r] = orc_dot_q6_k_go(w + r * stride, QK + (size_t)c * width,
                                                     BSums + (size_t)c * (width / 16),
                                                     KScales + (size_t)c * (width / SUPER_BLOCK), inputs);
}

/* DequantizeQ6_K, nn/dequant_q6_k.go:18-51 */
void orc_dequantize_q6_k(const uint8_t *w, int n, float *out)
{
    for (int b = 0; b < n / SUPER_BLOCK; b++) {
        const uint8_t *block = w + (size_t)b * Q6_K_BLOCK_BYTES;
        const uint8_t *low = block, *high = block + 128;
        const int8_t *scales = (const int8_t *)(block + 192);
        float super_scale = orc_half_to_float(le16(block + 208));
        float *dst = out + (size_t)b * SUPER_BLOCK;
        for (int half = 0; half < 2; half++) {
            const uint8_t *l = low + half * 64, *h = high + half * 32;
            const int8_t *s = scales + half * 8;
            float *d = dst + half * 128;
            for (int i = 0; i < 32; i++) {
                int group = i / 16;
                int32_t q1 = (int32_t)(l[i] & 0x0F) | (int32_t)((h[i] >> 0) & 3) << 4;
                int32_t q2 = (int32_t)(l[i + 32] & 0x0F) | (int32_t)((h[i] >> 2) & 3) << 4;
                int32_t q3 = (int32_t)(l[i] >> 4) | (int32_t)((h[i] >> 4) & 3) << 4;
                int32_t q4 = (int32_t)(l[i + 32] >> 4) | (int32_t)((h[i] >> 6) & 3) << 4;
                d[i + 0] = super_scale * (float)s[group + 0] * (float)(q1 - 32);
                d[i + 32] = super_scale * (float)s[group + 2] * (float)(q2 - 32);
                d[i + 64] = super_scale * (float)s[group + 4] * (float)(q3 - 32);
                d[i + 96] = super_scale * (float)s[group + 6] * (float)(q4 - 32);
            }
        }
    }
}

/* ---- float32 ------------------------------------------------------------ */

/* DotF32 generic form, nn/dot_f32.go:13-33 */
float orc_dot_f32(const float *a, const float *b, int n)
{
    if (n == 0)
        return 0;
    float s0 = 0, s1 = 0, s2 = 0, s3 = 0;
    int i = 0;
    for (; i + 3 < n; i += 4) {
        s0 += a[i] * b[i];
        s1 += a[i + 1] * b[i + 1];
        s2 += a[i + 2] * b[i + 2];
        s3 += a[i + 3] * b[i + 3];
    }
    for (; i < n; i++)
        s0 += a[i] * b[i];
    return (s0 + s1) + (s2 + s3);
}

/* Matrix.rows, nn/matrix.go:94-131: packed prefix and row-layout tail for
 * Q4_0, Q6_K, F32 through DotF32, then the bias for rows in [start, end).
 * packed may be NULL (no Repack). */
int orc_matrix_rows(int quant, const uint8_t *data, const uint8_t *packed, int rows, int cols, const float *bias,
                    int bias_len, const float *F, const int8_t *Q, const float *Scales, const float *Corr,
                    const int8_t *QK, const float *KScales, const int16_t *BSums, int stride, int size, float *ys,
                    int ldy, int start, int end)
{
    switch (quant) {
    case ORC_Q4_0: {
        int packed_rows = rows / PACKED_ROWS * PACKED_ROWS;
        if (packed != NULL && start < packed_rows) {
            orc_mat_vec_packed_q4_0_rows(packed, Q, Scales, Corr, stride, size, cols, ys, ldy, start,
                                         imin(end, packed_rows));
            if (end > packed_rows)
                orc_mat_vec_q4_0_rows(data, Q, Scales, Corr, stride, size, cols, ys, ldy, packed_rows, end);
        } else {
            orc_mat_vec_q4_0_rows(data, Q, Scales, Corr, stride, size, cols, ys, ldy, start, end);
        }
        break;
    }
    case ORC_F32: {
        const float *weights = (const float *)data;
        for (int r = start; r < end; r++)
            for (int c = 0; c < size; c++)
                ys[(size_t)c * ldy + r] = orc_dot_f32(weights + (size_t)r * cols, F + (size_t)c * cols, cols);
        break;
    }
    case ORC_Q6_K:
        if (QK == NULL)
            return -1; /* MatVecQ6_K's panic, nn/dot_q6_k.go:69 */
        orc_mat_vec_q6_k_rows(data, QK, KScales, BSums, cols, size, cols, ys, ldy, start, end);
        break;
    default:
        return -2; /* nn/matrix.go:124 */
    }
    for (int c = 0; c < size; c++)
        for (int i = start; i < end && i < bias_len; i++)
            ys[(size_t)c * ldy + i] += bias[i];
    return 0;
}

/* RMSNormPlain, nn/ops.go:195-214: squares in float32 summed in float64, mean
 * and reciprocal root in float32. gain may be NULL. */
void orc_rms_norm_plain(float *x, int n, const float *gain, float eps)
{
    double sum = 0;
    for (int i = 0; i < n; i++)
        sum += (double)(x[i] * x[i]);
    float mean = (float)(sum / (double)n);
    float scale = (float)(1 / sqrt((double)(mean + eps)));
    if (gain == NULL) {
        for (int i = 0; i < n; i++)
            x[i] = x[i] * scale;
        return;
    }
    for (int i = 0; i < n; i++)
        x[i] = x[i] * scale * gain[i];
}

/* geluTanh and buildGELUTable, nn/gelu_table.go:25-38 */
static double gelu_tanh(double x)
{
    const double sqrt2_over_pi = 0.79788456080286535587989211986876;
    const double coef_a = 0.044715;
    return 0.5 * x * (1 + tanh(sqrt2_over_pi * x * (1 + coef_a * x * x)));
}

void orc_gelu_table_build(float *table)
{
    for (int i = 0; i < 1 << 16; i++) {
        float in = orc_half_to_float((uint16_t)i);
        float out = (float)gelu_tanh((double)in);
        table[i] = orc_half_to_float(orc_float_to_half(out));
    }
}

static float gelu_table_storage[1 << 16];
static int gelu_table_ready = 0;

/* GELUTable, nn/gelu_table.go:40-52 */
void orc_gelu_table(float *x, int n)
{
    if (!gelu_table_ready) {
        orc_gelu_table_build(gelu_table_storage);
        gelu_table_ready = 1;
    }
    for (int i = 0; i < n; i++) {
        float v = x[i];
        if (v <= -10)
            x[i] = 0;
        else if (v >= 10)
            ;
        else
            x[i] = gelu_table_storage[orc_float_to_half(v)];
    }
}

/* expf (ggml_v_expf one value at a time), nn/swiglu.go:31-74 */
float orc_expf(float x)
{
    const float shift = 0x1.8p23f;
    const float log2e = 0x1.715476p+0f;
    const float ln2hi = 0x1.62e4p-1f;
    const float ln2lo = 0x1.7f7d1cp-20f;
    const float c0 = 0x1.ffffecp-1f;
    const float c1 = 0x1.fffdb6p-2f;
    const float c2 = 0x1.555e66p-3f;
    const float c3 = 0x1.573e2ep-5f;
    const float c4 = 0x1.0e4020p-7f;

    float z = x * log2e + shift;
    float n = z - shift;
    if (n > 126 || n < -126)
        return (float)exp((double)x);
    float b = x - n * ln2hi - n * ln2lo;
    float k = u2f((f2u(z) << 23) + f2u(1.0f));
    float u = b * b;
    float j = ((c4 * b + c3) * u + (c2 * b + c1)) * u + c0 * b;
    return j * k + k;
}

/* SwiGLURange, nn/swiglu.go:77-82 */
void orc_swiglu_range(float *gate, const float *up, int start, int end)
{
    for (int i = start; i < end; i++) {
        float g = gate[i];
        gate[i] = g / (1 + orc_expf(-g)) * up[i];
    }
}

/* SoftmaxInPlace, nn/ops.go:59-75 */
void orc_softmax_in_place(float *x, int n)
{
    float max = -INFINITY;
    for (int i = 0; i < n; i++)
        if (x[i] > max)
            max = x[i];
    float sum = 0;
    for (int i = 0; i < n; i++) {
        float e = (float)exp((double)(x[i] - max));
        x[i] = e;
        sum += e;
    }
    for (int i = 0; i < n; i++)
        x[i] /= sum;
}

/* Axpy generic form, nn/kernel.go:221-233: dst += a*src. */
void orc_axpy(float *dst, const float *src, int n, float a)
{
    for (int i = 0; i < n; i++)
        dst[i] += a * src[i];
}

/* ---- the Qwen3 decoder (qwen/) ------------------------------------------- */

/* RoPETable.Prepare, nn/rope.go:33-59, without frequency factors:
 * theta_i = position * base^(-2i/dims) in float64, cos and sin rounded to
 * float32.  (glibc's pow, cos and sin stand in for Go's math package; they
 * agree to about one unit in the last place of a float64, which rounds to the
 * same float32 except in rare ties.) */
void orc_rope_prepare(int dims, int position, double base, float *cos_out, float *sin_out)
{
    int half = dims / 2;
    for (int i = 0; i < half; i++) {
        double theta = (double)position * pow(base, -2 * (double)i / (double)dims);
        cos_out[i] = (float)cos(theta);
        sin_out[i] = (float)sin(theta);
    }
}

/* RoPETable.Apply, nn/rope.go:62-73: element i pairs with i + dims/2 (NeoX). */
void orc_rope_apply(float *vec, int dims, const float *c, const float *s)
{
    int half = dims / 2;
    for (int i = 0; i < half; i++) {
        float re = vec[i], im = vec[i + half];
        vec[i] = re * c[i] - im * s[i];
        vec[i + half] = re * s[i] + im * c[i];
    }
}

/* The device's exp_neg (golem_amd/csrc/gx_device.hpp): (float)exp((double)d)
 * for d <= 0 as straight-line float64 arithmetic -- n = rint(d 64 / ln2), r =
 * d - n ln2 / 64 (hi + lo), e^r - 1 as the Taylor series to r^5, times the
 * table value 2^(j/64) (j = n mod 64) in one fma, times 2^(n div 64),
 * rounded to float; +0 below -110.  Test infrastructure: tests check it
 * against the C library's exp over floats of [-110, 0] (it is the
 * exponential of SoftmaxInPlace, nn/ops.go:59-73, which golem takes in
 * float64). */
static const double orc_exp2_64[64] = {
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

float orc_exp_neg(float df) {
    const double d = (double)df;
    const double n = rint(d * 0x1.71547652b82fep+6);
    double r = fma(-n, 0x1.62e42fefa38p-7, d);
    r = fma(-n, 0x1.ef358p-51, r);
    double p = 1.0 / 120.0;
    p = fma(p, r, 1.0 / 24.0);
    p = fma(p, r, 1.0 / 6.0);
    p = fma(p, r, 0.5);
    p = fma(p, r, 1.0);
    p = p * r;
    const int ni = isnan(n) ? 0 : (int)n;
    const double t = orc_exp2_64[ni & 63];
    const float out = (float)ldexp(fma(t, p, t), ni >> 6);
    return d < -110.0 ? 0.0f : out;
}

/* Many at once (test helper): out[i] = orc_exp_neg(x[i]) and the count of
 * i where it differs from (float)exp((double)x[i]) in bits. */
long orc_exp_neg_check(const float *x, long n, float *out) {
    long bad = 0;
    for (long i = 0; i < n; i++) {
        const float a = orc_exp_neg(x[i]), b = (float)exp((double)x[i]);
        uint32_t ua, ub;
        memcpy(&ua, &a, 4);
        memcpy(&ub, &b, 4);
        bad += ua != ub;
        if (out)
            out[i] = a;
    }
    return bad;
}

/* One query head of one position, qwen/attention.go:96-124: against the first
 * n positions of a layer cache (K, V as [position][kvheads][hd] floats, already
 * rounded through fp16), scores = scale * DotF32(query, key), SoftmaxInPlace,
 * every probability rounded through fp16, then dst = sum over positions in
 * order of Axpy(value, probability) from zero.  scores holds n floats. */
void orc_attend(const float *query, const float *K, const float *V, int kvheads, int hd, int kv, int n, float scale,
                float *scores, float *dst)
{
    for (int p = 0; p < n; p++)
        scores[p] = scale * orc_dot_f32(query, K + ((size_t)p * kvheads + kv) * hd, hd);
    orc_softmax_in_place(scores, n);
    for (int p = 0; p < n; p++)
        scores[p] = orc_round_half(scores[p]);
    for (int i = 0; i < hd; i++)
        dst[i] = 0;
    for (int p = 0; p < n; p++)
        orc_axpy(dst, V + ((size_t)p * kvheads + kv) * hd, hd, scores[p]);
}

/* The decode attention in this build's parallel order -- NOT golem's: the
 * device's default decode attention (golem_amd/csrc/gx_qwen.hip,
 * attn_par_kernel), restated so that the kernel can be checked bit for bit;
 * golem's own order is orc_attend.
 * golem's scores, maximum, float64 exponentials, division and fp16 rounding
 * of each probability (qwen/attention.go:96-114, nn/ops.go:59-73), with the
 * two sums taken in a fixed parallel order:
 *   total  = ((0 + B_0) + B_1) + ... over blocks of 64 positions, B_b the
 *            pairwise sum of the block's exponentials (zeros past n): lane
 *            l = p % 64 holds e_p, then every lane adds lane l ^ 1's value,
 *            then l ^ 2's, ..., then l ^ 32's; B_b is lane 0's result;
 *   dst[d] = ((0 + R_0) + R_1) + ... over runs of 32 positions, R_r the
 *            chain acc = fma(prob_p, value_p[d], acc) from 0 over the run's
 *            positions below n in order.
 * The maximum ignores NaN scores as fmaxf does.  scores holds n floats and
 * is left holding the fp16-rounded probabilities. */
void orc_attend_parallel(const float *query, const float *K, const float *V, int kvheads, int hd, int kv, int n,
                      float scale, float *scores, float *dst)
{
    float m = -INFINITY;
    for (int p = 0; p < n; p++) {
        scores[p] = scale * orc_dot_f32(query, K + ((size_t)p * kvheads + kv) * hd, hd);
        m = fmaxf(m, scores[p]);
    }
    for (int p = 0; p < n; p++)
        scores[p] = (float)exp((double)(scores[p] - m));
    float total = 0;
    for (int b = 0; b * 64 < n; b++) {
        float lanes[64], next[64];
        for (int l = 0; l < 64; l++)
            lanes[l] = b * 64 + l < n ? scores[b * 64 + l] : 0.0f;
        for (int off = 1; off < 64; off <<= 1) {
            for (int l = 0; l < 64; l++)
                next[l] = lanes[l] + lanes[l ^ off];
            memcpy(lanes, next, sizeof(lanes));
        }
        total = total + lanes[0];
    }
    for (int p = 0; p < n; p++)
        scores[p] = orc_round_half(scores[p] / total);
    for (int d = 0; d < hd; d++) {
        float o = 0;
        for (int r = 0; r * 32 < n; r++) {
            float acc = 0;
            for (int p = r * 32; p < r * 32 + 32 && p < n; p++)
                acc = fmaf(scores[p], V[((size_t)p * kvheads + kv) * hd + d], acc);
            o = o + acc;
        }
        dst[d] = o;
    }
}

/* ---- mixture of experts ------------------------------------------------- */

/* chooseExperts, gemma/moe.go:62-88: repeated argmax (strict >, ties to the
 * lower index), softmax over the chosen in float64 exp, renormalised. */
void orc_choose_experts(const float *logits, int experts, int used, int32_t *ids, float *weights)
{
    for (int k = 0; k < used; k++) {
        int32_t best = -1;
        for (int e = 0; e < experts; e++) {
            int taken = 0;
            for (int j = 0; j < k; j++)
                if (ids[j] == e)
                    taken = 1;
            if (taken)
                continue;
            if (best < 0 || logits[e] > logits[best])
                best = e;
        }
        ids[k] = best;
    }
    float top = logits[ids[0]];
    float total = 0;
    for (int k = 0; k < used; k++) {
        weights[k] = (float)exp((double)(logits[ids[k]] - top));
        total += weights[k];
    }
    for (int k = 0; k < used; k++)
        weights[k] /= total;
}

/* DotF32 as it runs on an amd64 host with AVX2 (nn/dot_f32.go:18-20):
 * dotF32AVX2's order (nn/dot_f32_amd64.s:43-113).  Four registers of eight
 * lanes, lane j of register r adding the product of element 32g + 8r + j of
 * every whole group of 32 (each product rounded, then added: nothing fused);
 * then Y0 + Y1 and Y2 + Y3, then their sum; then the remaining whole groups
 * of eight into those eight lanes; then lanes j and j + 4, then pairs 0,2 and
 * 1,3, then the two; then the remaining elements one at a time. */
float orc_dot_f32_avx2(const float *a, const float *b, int n)
{
    if (n == 0)
        return 0;
    float y[32] = {0};
    int i = 0;
    for (; i + 32 <= n; i += 32)
        for (int j = 0; j < 32; j++) {
            float p = a[i + j] * b[i + j];
            y[j] = y[j] + p;
        }
    float v[8];
    for (int j = 0; j < 8; j++) {
        float y01 = y[j] + y[j + 8];
        float y23 = y[j + 16] + y[j + 24];
        v[j] = y01 + y23;
    }
    for (; i + 8 <= n; i += 8)
        for (int j = 0; j < 8; j++) {
            float p = a[i + j] * b[i + j];
            v[j] = v[j] + p;
        }
    float w[4];
    for (int j = 0; j < 4; j++)
        w[j] = v[j] + v[j + 4];
    float x0 = w[0] + w[2], x1 = w[1] + w[3];
    float s = x0 + x1;
    for (; i < n; i++) {
        float p = a[i] * b[i];
        s = s + p;
    }
    return s;
}

/* Route, gemma/moe.go:34-53, for one position: RMSNormPlain without a gain,
 * times (1/sqrt(Dim)) * RouterScale[i], then the F32 router rows through
 * DotF32 (Matrix.rows F32 case, nn/matrix.go:113-120) in the order golem
 * runs it on x86 (orc_dot_f32_avx2), then chooseExperts.
 * router_scale may be NULL (all ones).  logits receives `experts` values. */
void orc_route_one(const float *resid, int dim, const float *router /*[experts][dim]*/, const float *router_scale,
                   int experts, int used, float eps, float *scratch /*dim*/, float *logits, int32_t *ids,
                   float *weights)
{
    float scale = (float)(1 / sqrt((double)dim));
    memcpy(scratch, resid, sizeof(float) * dim);
    orc_rms_norm_plain(scratch, dim, NULL, eps);
    for (int i = 0; i < dim; i++)
        scratch[i] *= scale * (router_scale ? router_scale[i] : 1.0f);
    for (int e = 0; e < experts; e++)
        logits[e] = orc_dot_f32_avx2(router + (size_t)e * dim, scratch, dim);
    orc_choose_experts(logits, experts, used, ids, weights);
}

/* One (position, expert) unit of ExpertFFN, gemma/moe.go:119-162, on the row
 * layout (ExpertStack.At, gemma/weights.go:67-72; never repacked), both
 * products through Matrix.rows (MatVecRows, nn/matrix.go:87-131) of the
 * stack's format:
 *   x (dim floats) is quantised to Q8_0 as one contiguous column
 *     (moe.go:119-125),
 *   gate_up = GateUp[id] . x (2*ffn rows, gate first then up, moe.go:142-147),
 *   gate = GELUTable(gate); mid = gate * up (moe.go:149-152); mid quantised,
 *   partial = Down[id] . mid (dim rows, moe.go:154-156).
 * quant is ORC_Q4_0 (the configs' stacks: Q8_0 products) or ORC_F32 (golem's
 * own test stacks, gemma/moe_test.go:21-56: DotF32 of each row with the
 * floats; the Q8_0 forms are made but unread).  gate_up_w is one expert's
 * 2*ffn x dim rows, down_w its dim x ffn rows. */
void orc_expert_unit(int quant, const uint8_t *gate_up_w, const uint8_t *down_w, const float *x, int dim, int ffn,
                     float *partial)
{
    int8_t *q = malloc(dim);
    float *sc = malloc(sizeof(float) * (dim / 32)), *co = malloc(sizeof(float) * (dim / 32));
    float *gu = malloc(sizeof(float) * 2 * ffn);
    float *mid = malloc(sizeof(float) * ffn);
    int8_t *mq = malloc(ffn);
    float *msc = malloc(sizeof(float) * (ffn / 32)), *mco = malloc(sizeof(float) * (ffn / 32));

    orc_quantize_column_range(x, dim, 1, q, sc, co, 0, 0, dim);
    orc_matrix_rows(quant, gate_up_w, NULL, 2 * ffn, dim, NULL, 0, x, q, sc, co, NULL, NULL, NULL, 1, 1, gu, 2 * ffn,
                    0, 2 * ffn);
    orc_gelu_table(gu, ffn);
    for (int i = 0; i < ffn; i++)
        mid[i] = gu[i] * gu[ffn + i];
    orc_quantize_column_range(mid, ffn, 1, mq, msc, mco, 0, 0, ffn);
    orc_matrix_rows(quant, down_w, NULL, dim, ffn, NULL, 0, mid, mq, msc, mco, NULL, NULL, NULL, 1, 1, partial, dim, 0,
                    dim);

    free(q); free(sc); free(co); free(gu); free(mid); free(mq); free(msc); free(mco);
}

/* ExpertFFN's reduction, gemma/moe.go:165-179: out = sum_k Axpy(partial_k,
 * weight_k * DownScale[id]) with the generic Axpy; down_scale may be NULL
 * (all ones). */
void orc_expert_reduce(const float *partials /*[used][dim]*/, const int32_t *ids, const float *weights,
                       const float *down_scale, int used, int dim, float *out)
{
    for (int i = 0; i < dim; i++)
        out[i] = 0;
    for (int k = 0; k < used; k++) {
        float a = weights[k] * (down_scale ? down_scale[ids[k]] : 1.0f);
        orc_axpy(out, partials + (size_t)k * dim, dim, a);
    }
}
