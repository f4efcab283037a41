/*
 * golem_hip.h - C ABI of the MI355X (gfx950) quantized linear-layer path.
 *
 * This is the boundary a cgo shim binds to replace golem's nn.Matrix /
 * nn.Batch products (ThiraSoft/golem, package nn).  Every entry point takes
 * plain pointers and sizes; no HIP or torch types cross it.  Pointers named
 * "device" must point into device memory of the context's GPU (hipMalloc,
 * gx_alloc, or a torch tensor's storage); "host" pointers are ordinary memory.
 *
 * Errors.  Every call returns GX_OK (0) or a status code, and leaves a message
 * for gx_last_error() (thread-local).  Misuse that golem answers with a panic
 * ("nn: ...") is GX_ERR_INVALID with the same wording, so a shim can panic
 * with it unchanged.  Nothing falls back to a CPU path: a GPU failure is an
 * error, never silent zeros.
 *
 * Streams.  All work of a context is enqueued on one stream (the null stream
 * unless gx_set_stream chose another); calls return once it is enqueued.
 * gx_sync waits for it.  A context is not meant to be driven by several host
 * threads at once: golem serialises its parallel sections with a mutex
 * (nn/parallel.go:163-191) and a shim does the same.  The row-slice products
 * (gx_matvec_rows_*) are the exception: they take the context's lock
 * themselves, for golem's pool workers.
 *
 * Layouts on the device.
 *   Q8_0 activations (golem's Batch.Q/Scales/Corr, nn/batch.go:17-27), one
 *   token per row rather than golem's column interleave:
 *     q      int8    [M][K]
 *     scales float   [M][K/32]   the fp16-rounded scale, held as float
 *     qsum   int32   [M][K/32]   sum of the block's 32 q values
 *     corr   float   [M][K/32]   (8*scale)*float(qsum), golem's Corr (optional)
 *     q16    fp16    the same q values as fp16 (optional; exact), in the
 *                    operand order of the fp16 MFMA: ceil(M/32)*32*K values;
 *                    token t's input k sits at q16_offset below; tokens past
 *                    M are zero
 *   Q8_K activations (Batch.QK/KScales/BSums, nn/batch.go:29-32), same layout
 *   as golem's:
 *     q      int8    [M][K]
 *     kscales float  [M][K/256]
 *     bsums  int16   [M][K/16]
 *   Outputs y are float [M][ldy]; a product over rows [row_start, row_end)
 *   writes y[m*ldy + r] for r in that range and nothing else.
 *   Weights are repacked on upload into a 64-row interleaved layout (see
 *   gx_weight_upload); callers never address them directly.
 */
#ifndef GOLEM_HIP_H
#define GOLEM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    GX_OK = 0,
    GX_ERR_INVALID = 1,     /* misuse: golem panics with the same message */
    GX_ERR_HIP = 2,         /* the HIP runtime reported an error */
    GX_ERR_UNSUPPORTED = 3, /* a format or shape this build has no kernel for */
    GX_ERR_NOMEM = 4        /* a device allocation failed */
};

/* Weight formats: the values of golem's nn.Quant (nn/quant.go:12-17). */
enum { GX_F32 = 0, GX_BF16 = 1, GX_Q4_0 = 2, GX_Q6_K = 3 };

typedef struct gx_ctx gx_ctx;
typedef struct gx_weight gx_weight;

/* ---- context --------------------------------------------------------- */

/* The message of the last failing call on this thread ("" if none). */
const char *gx_last_error(void);

/* Opens a context on one GPU.  No counterpart in golem (it has no device);
 * the shim calls it once where golem builds its worker pool
 * (nn/parallel.go:59-72). */
int gx_init(int device, gx_ctx **out);
int gx_free(gx_ctx *ctx);

/* Chooses the stream (a hipStream_t, or NULL for the null stream) the
 * context enqueues on. */
int gx_set_stream(gx_ctx *ctx, void *stream);
/* Waits for everything enqueued on the context's stream. */
int gx_sync(gx_ctx *ctx);

/* Device memory for callers with no HIP runtime of their own (the cgo shim):
 * allocate, free, and synchronous copies. */
int gx_alloc(gx_ctx *ctx, size_t bytes, void **device);
int gx_dealloc(gx_ctx *ctx, void *device);
int gx_upload(gx_ctx *ctx, void *device, const void *host, size_t bytes);
int gx_download(gx_ctx *ctx, void *host, const void *device, size_t bytes);

/* Timing on the context's stream: gx_timer_start records an event,
 * gx_timer_stop records another, waits for it and returns the milliseconds
 * between the two. */
int gx_timer_start(gx_ctx *ctx);
int gx_timer_stop(gx_ctx *ctx, float *ms);

/* ---- weights (nn.Matrix) -------------------------------------------- */

/* Uploads one matrix of `rows` outputs by `cols` inputs, given in the GGUF
 * block layout golem's Matrix.Data holds (nn/matrix.go:23-31): Q4_0 rows of
 * cols/32 blocks of 18 bytes (nn/dot_q4_0.go:3-13), Q6_K rows of cols/256
 * superblocks of 210 bytes (nn/dequant_q6_k.go:3-15), F32 row-major floats.
 * `data` is host memory, or device memory when on_device is non-zero.  The
 * quantized formats are repacked on the device into a 64-row interleaved
 * layout of the same bytes (the role of Matrix.Repack, nn/matrix.go:40-46);
 * the matrix stays resident until gx_weight_free.  Replaces Matrix{Data,
 * Quant, Rows, Cols} plus Repack (nn/matrix.go:23-46).
 * Errors as golem: cols not a multiple of 32 for Q4_0 (nn/dot_q4_0.go:119),
 * of 256 for Q6_K (nn/dot_q6_k.go:66). */
int gx_weight_upload(gx_ctx *ctx, const void *data, size_t bytes, int on_device, int quant, int rows, int cols,
                     gx_weight **out);

/* Uploads `count` matrices of the same shape stored back to back, as golem's
 * gemma.ExpertStack (gemma/weights.go:59-72); expert i is the i-th matrix. */
int gx_weight_upload_stack(gx_ctx *ctx, const void *data, size_t bytes, int on_device, int quant, int rows,
                           int cols, int count, gx_weight **out);

int gx_weight_free(gx_weight *w);

/* Shape and the device bytes the resident copy occupies. */
int gx_weight_info(const gx_weight *w, int *quant, int *rows, int *cols, int *count, size_t *device_bytes);

/* Matrix.Row (nn/matrix.go:135-160): expands rows ids[0..n) of expert
 * `expert` (0 for a single matrix) into out[n][cols] (device floats).  The
 * embedding lookup of qwen/model.go:107-109 is this with n tokens. */
int gx_weight_rows(gx_ctx *ctx, const gx_weight *w, int expert, const int32_t *ids_device, int n, float *out);

/* ---- activations (nn.Batch) ------------------------------------------ */

/* Batch.Quantize / QuantizeRange / QuantizeColumnRange (nn/batch.go:69-143)
 * for M activations of K floats at x[m*ldx ...] (device).  corr and q16 may
 * be NULL; q16 (uint16 storage of fp16, ceil(M/32)*32*K values) is what the
 * fp16-MFMA batch product reads.  In q16, token t's input k is at
 *   ((((t/32)*(K/32) + k/32)*2 + (k%32)/16)*64 + 32*((k%16)/8) + t%32)*8 + k%8:
 * tokens in groups of 32, and per group, block and half-block one 1 KiB
 * panel holding each lane's 8 operand values contiguously.  K must be a
 * multiple of 32 (nn/batch.go:49-51). */
int gx_quantize_q8_0(gx_ctx *ctx, const float *x, int ldx, int M, int K, int8_t *q, float *scales, int32_t *qsum,
                     float *corr, uint16_t *q16);

/* Batch.QuantizeK (nn/batch.go:159-213).  K must be a multiple of 256
 * (nn/batch.go:160-162). */
int gx_quantize_q8_k(gx_ctx *ctx, const float *x, int ldx, int M, int K, int8_t *q, float *kscales,
                     int16_t *bsums);

/* ---- products (Matrix.MatVec / MatVecBatch / MatVecRows) ------------ */

/* y[m][r] = W[r] . x[m] (+ bias[r]) for the M activations of a Q8_0 batch and
 * rows r in [row_start, row_end) of a Q4_0 matrix: Matrix.MatVecBatch and
 * MatVecRows for Q4_0 (nn/matrix.go:78-104), and MatVecQ4_0
 * (nn/dot_q4_0.go:117-124) when the range is all rows.  bias is NULL or
 * rows floats (device).  One column runs a bandwidth-bound matrix-vector
 * kernel (activation in scalar registers, or in LDS on quarter tiles for a
 * matrix of few tiles); 2..16 columns the few-column int8-MFMA kernel
 * (16 rows against 16 columns a block); larger M a tiled product on int8
 * MFMA.  q16 may be NULL and is not read: the fp16-MFMA form is slower at
 * every M and runs only as gx_q4_0_block_dots path 2.  All of them sum every
 * row's blocks in the same order
 * from the same exact per-block integers, so a column's result does not
 * depend on M or on the kernel. */
int gx_matmul_q4_0(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const float *scales, const int32_t *qsum,
                   const uint16_t *q16, int M, int row_start, int row_end, const float *bias, float *y, int ldy);

/* The same product with one expert of a stack (gemma's
 * ExpertStack.At(expert).MatVecRows, gemma/moe.go:151-161). */
int gx_matmul_q4_0_expert(gx_ctx *ctx, const gx_weight *w, int expert, const int8_t *q, const float *scales,
                          const int32_t *qsum, const uint16_t *q16, int M, int row_start, int row_end, float *y,
                          int ldy);

/* y[m][r] = W[r] . x[m] (+ bias[r]) for a Q6_K matrix and a Q8_K batch:
 * MatVecQ6_K and matVecQ6_KRows (nn/dot_q6_k.go:64-103), which include the
 * two-column dotQ6_Kx2 (nn/dot_q6_k_amd64.go:14-20): one weight read serves
 * all M <= 8 columns.  Bit-identical to golem's dotQ6_KGo. */
int gx_matmul_q6_k(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const float *kscales, const int16_t *bsums,
                   int M, int row_start, int row_end, const float *bias, float *y, int ldy);

/* Matrix.MatVecRows for golem's fine-grained callers (nn/matrix.go:84-92):
 * its engines call it on 32-row slices from pool workers (qwen/block.go:
 * 82-90, qwen/attention.go:57-84), which as one product each would be
 * thousands of launches a token.  Here the first call for a (matrix,
 * activation q, generation, M) computes every row of the product once on the
 * device (gx_matmul_q4_0 / gx_matmul_q6_k) and copies it to pinned host
 * memory; every call, that one included, then copies rows [row_start,
 * row_end) of each column into ys[m * ldys + r] (host floats; ys holds full
 * columns, ldys >= row_end), as MatVecRows fills ys[c][start:end].
 * `generation` names the activation's contents: the caller changes it
 * whenever q changes (after each Batch.Quantize* of the batch).  Calls may
 * come from several threads at once: they serialise on the context's lock
 * and share one product per key; the bias stays with the caller, as
 * Matrix.rows adds it (nn/matrix.go:126-130).  The 16 most recent products
 * are kept (device + pinned host copies, allocated once per size);
 * gx_weight_free forgets a matrix's.  q4_0 takes the Q8_0 form, q6_k the
 * Q8_K form, as the products do. */
int gx_matvec_rows_q4_0(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const float *scales, const int32_t *qsum,
                        int M, uint64_t generation, int row_start, int row_end, float *ys, int ldys);
int gx_matvec_rows_q6_k(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const float *kscales, const int16_t *bsums,
                        int M, uint64_t generation, int row_start, int row_end, float *ys, int ldys);
/* Products computed and slices served so far by the two calls above (for
 * checks).  No counterpart in golem. */
int gx_matvec_rows_stats(gx_ctx *ctx, uint64_t *products, uint64_t *served);

/* y[m][r] = DotF32(W[r], x[m]) for an F32 matrix (Matrix.rows' F32 case,
 * nn/matrix.go:113-120), in the generic DotF32 order (nn/dot_f32.go:13-33):
 * four interleaved accumulators, then (s0+s1)+(s2+s3). */
int gx_matmul_f32(gx_ctx *ctx, const gx_weight *w, const float *x, int ldx, int M, int row_start, int row_end,
                  float *y, int ldy);

/* ---- per-block integers (parity instrumentation) --------------------- */

/* The signed per-block integer each product uses, sum_j (n_j - 8) * q_j, for
 * every (m, r, block): out[m][r - row_start][K/32] (device int32), exported
 * by the very kernel that computes the product (its per-block integer
 * output switched on; nothing else changes).  path 0: the matrix-vector
 * kernel with the activation in scalar registers (M <= 8 as the product
 * groups the columns, 8/4/2/1 a launch, and any larger M the same way);
 * path 1: the int8-MFMA product (the direct-to-LDS kernel every M > 8
 * product without q16 runs); path 2: the fp16-MFMA product (needs q16);
 * path 3: the one-column matrix-vector kernel with the activation in LDS
 * (M = 1, the whole/half/quarter-tile shape the product picks for this
 * matrix); path 4: the multi-column matrix-vector kernel with the
 * activations in LDS (2..8 columns a launch, in the column groups and tile
 * shape it picks); path 5: the few-column int8-MFMA kernel (what products of
 * 2 <= M <= 16 run).  golem's dotQ4_0Go accumulator
 * (nn/dot_q4_0.go:58-63) is this plus 8*qsum.  No counterpart in golem:
 * parity instrumentation. */
int gx_q4_0_block_dots(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const float *scales, const int32_t *qsum,
                       const uint16_t *q16, int M, int row_start, int row_end, int path, int32_t *out);

/* The per-block integers of the fused one-position products
 * (gx_norm_matmul_q4_0 when swiglu is 0, gx_norm_swiglu_q4_0 when it is 1),
 * from the same kernel: x + add is normed (RMSNormPlain(gain, eps)) and
 * quantised to Q8_0 inside it, and out[r - row_start][K/32] receives each
 * block's sum_j (n_j - 8) * q_j against that Q8_0 form.  swiglu 1 needs
 * every row and writes the SwiGLU Q8_0 into q/scales/qsum as
 * gx_norm_swiglu_q4_0 does.  No counterpart in golem: parity
 * instrumentation. */
int gx_q4_0_fused_block_dots(gx_ctx *ctx, const gx_weight *w, int swiglu, const float *x, const float *add,
                             const float *gain, float eps, int row_start, int row_end, int8_t *q, float *scales,
                             int32_t *qsum, int32_t *out);

/* The per-block integers of the expert products gx_moe_experts runs, from
 * those kernels with their integer output switched on: for M <= 4 the
 * fused matrix-vector kernels, for more positions the grouped int8-MFMA
 * product over the same sort by expert.  dots_gate_up [M*top_k][2*ffn][dim/32]
 * receives, for unit u (position u / top_k, expert ids[u]), each gate|up
 * row's block sums against Q8_0(x[u / top_k]); dots_down [M*top_k][dim]
 * [ffn/32] each down row's block sums against the unit's Q8_0 input given in
 * mid_q [M*top_k][ffn], mid_scales and mid_qsum [M*top_k][ffn/32].  Either
 * output may be NULL (then its inputs may be too).  More than 4 positions
 * need gx_moe_experts' workspace (it may be NULL otherwise).  A unit whose
 * id is out of range writes nothing.  No counterpart in golem: parity
 * instrumentation. */
int gx_moe_block_dots(gx_ctx *ctx, const gx_weight *gate_up, const gx_weight *down, const float *x, int ldx, int M,
                      int top_k, const int32_t *ids, const int8_t *mid_q, const float *mid_scales,
                      const int32_t *mid_qsum, void *workspace, size_t workspace_bytes, int32_t *dots_gate_up,
                      int32_t *dots_down);

/* dotQ6_KGo's per-superblock integer sum - 32*shift (nn/dot_q6_k.go:31-51)
 * for every (m, r, superblock): out[m][r - row_start][K/256]. */
int gx_q6_k_block_dots(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const int16_t *bsums, int M,
                       int row_start, int row_end, int32_t *out);

/* ---- mixture of experts (gemma.ExpertFFN) ---------------------------- */

/* golem's GELU table (nn/gelu_table.go:19-38), built on the device when the
 * context opens: out receives 65536 floats (device), entry i for the fp16
 * input with bits i. */
int gx_gelu_table(gx_ctx *ctx, float *out);

/* The device workspace gx_moe_experts needs for M positions of top_k
 * experts, model width dim, expert width ffn, and `experts` experts. */
int gx_moe_workspace_bytes(int M, int top_k, int dim, int ffn, int experts, size_t *bytes);

/* Route (gemma/moe.go:34-53) and chooseExperts (:62-88) for M positions:
 * resid[m*ldr ...] (device floats, dim = router->cols) is normalised by
 * RMSNormPlain without a gain (eps), scaled by (1/sqrt(dim)) *
 * router_scale[i] (router_scale may be NULL: ones), and multiplied by the F32
 * router (experts x dim) in DotF32's generic order.  Outputs (device):
 * logits [M][experts], ids [M][top_k], weights [M][top_k].  For M <= 4 this
 * is one kernel launch, whose last workgroup per position chooses the
 * experts; it keeps a counter per position in the context, so calls on one
 * context are ordered on its stream (as all calls on a context are). */
int gx_moe_route(gx_ctx *ctx, const gx_weight *router, const float *router_scale, const float *resid, int ldr, int M,
                 int top_k, float eps, float *logits, int32_t *ids, float *weights);

/* The expert units and their weighted sum of ExpertFFN (gemma/moe.go:
 * 112-180): for every position m and slot k, expert e = ids[m][k] of the
 * stacks gate_up (2*ffn x dim per expert, gate rows first, as the fused
 * tensor of gemma/README.md:276-278) and down (dim x ffn) computes
 * Down[e] . Q8_0(GELUTable(gate) * up) with gate|up = GateUp[e] . Q8_0(x[m]);
 * out[m] = sum_k (weights[m][k] * down_scale[e]) * that (down_scale may be
 * NULL: ones).  Few positions (M <= 4) run as two kernels: gate|up with
 * the input's Q8_0, GELU * up and the mid's Q8_0 fused, then down with the
 * weighted sum fused.  More are sorted by expert and run as ragged MFMA
 * batches, one per expert.  F32 stacks (both gate_up and down F32, as
 * golem's own MoE test holds them) take the input and mid unquantised into
 * DotF32 products (nn/matrix.go:113-120), bit for bit.  The
 * workspace (device, 256-byte aligned, gx_moe_workspace_bytes) is the
 * scratch golem keeps in its Scratch; no call allocates.  An id out of range
 * makes its position's output NaN. */
int gx_moe_experts(gx_ctx *ctx, const gx_weight *gate_up, const gx_weight *down, const float *down_scale,
                   const float *x, int ldx, int M, int top_k, const int32_t *ids, const float *weights, float *out,
                   int ldo, void *workspace, size_t workspace_bytes);

/* gx_moe_experts without the workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid allocation).  No counterpart in golem.  Its
 * scratch is a fixed 16 MiB of device memory the library holds on every GPU
 * it runs on until the process ends; a call whose workspace
 * (gx_moe_workspace_bytes) would exceed it is refused with GX_ERR_INVALID,
 * before any work is queued.  The call allocates nothing and queues the same
 * kernels as gx_moe_experts, so the outputs are the same bit for bit.  All
 * calls on one GPU share that scratch, which keeps the last call's contents:
 * calls that overlap on one GPU (several streams, several contexts, or
 * several host threads) race; order them on one stream. */
int gx_moe_experts_noalloc(gx_ctx *ctx, const gx_weight *gate_up, const gx_weight *down, const float *down_scale,
                           const float *x, int ldx, int M, int top_k, const int32_t *ids, const float *weights,
                           float *out, int ldo);

/* The shared expert's activation (gemma/block.go:163-174, the dense feed
 * forward's): gu [M][ldgu] holds each position's ffn gates then its ffn ups;
 * q/scales/qsum receive Q8_0(GELUTable(gate) * up) [M][ffn] (nn/gelu_table.go
 * :40-52, the table of gx_gelu_table).  ffn a multiple of 32. */
int gx_geglu_quant(gx_ctx *ctx, const float *gu, int ldgu, int M, int ffn, int8_t *q, float *scales,
                   int32_t *qsum);

/* The join of moeHalf (gemma/block.go:195-205) for M positions of width K:
 * shared[m] = RMSNormPlain(shared[m], post1) and experts[m] =
 * RMSNormPlain(experts[m], post2), both written back in place; then
 * out[m] = resid[m] + RMSNormPlain(shared[m] + experts[m], post).  All device
 * floats; out may be resid. */
int gx_moe_join(gx_ctx *ctx, float *shared, int lds, float *experts, int lde, const float *resid, int ldr,
                const float *post1, const float *post2, const float *post, int M, int K, float eps, float *out,
                int ldo);

/* ---- the Qwen3 dense block around the products (qwen/) --------------- */

/* x[m] += add[m] (add may be NULL: no residual), then RMSNormPlain(x[m], gain,
 * eps) (nn/ops.go:195-214) into out[m] (optional) and its Q8_0 form into
 * q/scales/qsum (optional): the two pre-norms of Block (qwen/block.go:45-52,
 * 59-68, the residual of the previous half folded in) and the final norm
 * (qwen/model.go:167-171).  x, add, out: device floats [M][ld*]; gain: K
 * device floats; K a multiple of 32. */
int gx_norm_quant(gx_ctx *ctx, float *x, int ldx, const float *add, int lda, const float *gain, int M, int K,
                  float eps, float *out, int ldo, int8_t *q, float *scales, int32_t *qsum);

/* The head-by-head part of Attention's projections (qwen/attention.go:57-84)
 * for M positions: qkv[m] holds the Q (heads*head_dim), K and V
 * (kv_heads*head_dim each) projections of position m.  Query heads are
 * normed by q_norm, rotated (NeoX pairs, RoPETable.Apply, nn/rope.go:62-73)
 * by rope_cos/rope_sin[positions[m]] ([context][head_dim/2] floats: golem's
 * RoPETable.Prepare values) and rounded to fp16 into qh [M][heads*head_dim];
 * key heads are normed by k_norm and rotated, and key and value are stored
 * rounded to fp16 into the layer's caches (LayerCache.Store,
 * qwen/cache.go:52-60), a cache of `context` positions: element e of the key
 * at kcache[kv_head][e / 8][positions[m]][e % 8] (16-byte pieces, a piece of
 * consecutive positions contiguous), the value transposed at
 * vcache[kv_head][e][positions[m]] (a value row holds one element of a head
 * over all positions).  positions[m] < context; head_dim a multiple of 8.
 * All device pointers; positions: M int32.
 * Slots (qwen/slots.go, qwen/place.go): with `slots` (M device int32) the
 * caches hold nslots conversations of `context` positions one after another
 * ([slot][kv_head]... of the layouts above) and position m belongs to
 * conversation slots[m] -- golem's Place{Cache: Slot(slots[m]), Pos}.  A slot
 * out of range stores nothing and leaves the position's query NaN.  NULL:
 * one conversation.  A position outside [0, context) is treated as such a
 * slot: nothing stored, query NaN. */
int gx_qwen_qk_rope(gx_ctx *ctx, const float *qkv, int ldqkv, int M, int heads, int kv_heads, int head_dim,
                    const int32_t *positions, const float *q_norm, const float *k_norm, const float *rope_cos,
                    const float *rope_sin, float eps, uint16_t *qh, uint16_t *kcache, uint16_t *vcache, int context,
                    const int32_t *slots, int nslots);

/* The Q|K|V product of M positions followed by gx_qwen_qk_rope, the same
 * values bit for bit: golem's Attention from its three products through the
 * cache stores (qwen/attention.go:34-84, qwen/cache.go:52-60), with
 * Matrix.MatMul's product (nn/matrix.go) on the Q4_0 matrix w whose rows are
 * the heads query heads, then the kv_heads key heads, then the kv_heads
 * value heads, head_dim rows each (golem's three matrices stacked by rows).
 * q / scales / qsum: the activation's Q8_0 form (gx_quantize_q8_0; q 16-byte
 * aligned).  qh, the caches, positions, slots and the rest as for
 * gx_qwen_qk_rope.  More than 16 positions at head widths 64 and 128 run as
 * one kernel (the heads' norms, RoPE and stores in the product's epilogue,
 * no float Q|K|V row written); otherwise qkv ([M][w->rows] floats, device)
 * receives the product, which then goes through gx_qwen_qk_rope -- qkv may
 * be NULL only when the single kernel applies.  No reference counterpart
 * as one call: it replaces the pair gx_matmul_q4_0 + gx_qwen_qk_rope. */
int gx_qwen_qkv_rope(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const float *scales, const int32_t *qsum,
                     int M, int heads, int kv_heads, int head_dim, const int32_t *positions, const float *q_norm,
                     const float *k_norm, const float *rope_cos, const float *rope_sin, float eps, uint16_t *qh,
                     uint16_t *kcache, uint16_t *vcache, int context, const int32_t *slots, int nslots,
                     float *qkv);

/* Device bytes of the workspace gx_qwen_attention needs for M positions of
 * `heads` query heads whose positions are at most max_pos. */
int gx_qwen_attention_workspace_bytes(int M, int heads, int max_pos, size_t *bytes);

/* The attention proper (qwen/attention.go:86-124) for M positions: every
 * query head of position m against the layer's cache (the layouts of
 * gx_qwen_qk_rope; context a multiple of 8 above max_pos) over positions
 * 0 .. positions[m] (max_pos bounds them all): scores (1/sqrt(head_dim)) *
 * DotF32, SoftmaxInPlace, probabilities rounded to fp16, values summed by
 * Axpy in position order; the heads' outputs [M][heads*head_dim] quantised to
 * Q8_0 into q/scales/qsum for the output projection.  workspace: 256-byte
 * aligned device memory of gx_qwen_attention_workspace_bytes.  slots /
 * nslots as for gx_qwen_qk_rope: position m reads only conversation
 * slots[m]'s cache (ForwardMixed, qwen/model.go:131-172). */
int gx_qwen_attention(gx_ctx *ctx, const uint16_t *qh, int M, int heads, int kv_heads, int head_dim, int max_pos,
                      const int32_t *positions, const uint16_t *kcache, const uint16_t *vcache, int context,
                      int8_t *q, float *scales, int32_t *qsum, void *workspace, size_t workspace_bytes,
                      const int32_t *slots, int nslots);

/* gx_qwen_qk_rope followed by gx_qwen_attention for ONE position
 * (qwen/attention.go:57-124 at batch 1, the decode step), in one kernel: the
 * head norms and RoPE of the Q|K|V row qkv (ldqkv as for gx_qwen_qk_rope),
 * the key and value stored into the caches at positions[0], and the
 * attention over positions 0 .. positions[0] (max_pos bounds it; at most 767),
 * quantised to Q8_0 into q/scales/qsum.  The caches and q/scales/qsum come
 * out bit for bit as the two calls leave them (the fp16 query is not written
 * anywhere).  slots / nslots as for gx_qwen_qk_rope, with one position.
 * A position outside [0, context) stores nothing and its query is NaN (the
 * rotation tables are then read at context - 1), so a replayed step whose
 * counter has reached the end of the context stays inside the caches; one
 * past max_pos but inside the cache is stored and attends positions
 * 0 .. max_pos, as the two calls do. */
int gx_qwen_rope_attention(gx_ctx *ctx, const float *qkv, int ldqkv, int heads, int kv_heads, int head_dim,
                           int max_pos, const int32_t *positions, const float *q_norm, const float *k_norm,
                           const float *rope_cos, const float *rope_sin, float eps, uint16_t *kcache,
                           uint16_t *vcache, int context, int8_t *q, float *scales, int32_t *qsum,
                           const int32_t *slots, int nslots);

/* gx_qwen_attention and gx_qwen_rope_attention with their two serial sums
 * taken in parallel, for decode steps (M <= 4 positions of one conversation,
 * or one position per conversation with slots; prefixes of at most 768):
 * SoftmaxInPlace's total (nn/ops.go:59-73) as a tree over the positions, and
 * each head element's Axpy over the positions (nn/kernel.go:221-233) as 16
 * runs of consecutive positions added in run order.  The scores, maximum,
 * exponentials, division and fp16 probabilities are golem's; only the order
 * of those two sums differs, so the head outputs are golem's within float
 * rounding -- within 1e-4 of RMS against the oracle, since a probability
 * that sits on an fp16 rounding boundary moves one fp16 step when the total
 * does by an ulp -- and their Q8_0 form matches golem's except where a value
 * sits on a rounding boundary.  Every
 * thread of a workgroup takes a share of both sums, where golem's order
 * leaves them to one lane per head and one per head element.  Same
 * arguments, caches and outputs as the serial forms; the caches come out bit
 * for bit the same.  A prompt (M > 4 tokens of one conversation, prefixes
 * of at most 1024) runs on the matrix cores instead: the scores and the
 * value sums are fp16 MFMA products (exact products, fp32 sums in the
 * matrix core's order), the maximum, exponentials, total and fp16
 * probabilities as above; the head outputs stay within 1e-4 of RMS of
 * golem's.  Longer prompts and batches with slots take the serial kernels. */
int gx_qwen_attention_parallel(gx_ctx *ctx, const uint16_t *qh, int M, int heads, int kv_heads, int head_dim,
                               int max_pos, const int32_t *positions, const uint16_t *kcache,
                               const uint16_t *vcache, int context, int8_t *q, float *scales, int32_t *qsum,
                               void *workspace, size_t workspace_bytes, const int32_t *slots, int nslots);
int gx_qwen_rope_attention_parallel(gx_ctx *ctx, const float *qkv, int ldqkv, int heads, int kv_heads,
                                    int head_dim, int max_pos, const int32_t *positions, const float *q_norm,
                                    const float *k_norm, const float *rope_cos, const float *rope_sin, float eps,
                                    uint16_t *kcache, uint16_t *vcache, int context, int8_t *q, float *scales,
                                    int32_t *qsum, const int32_t *slots, int nslots);

/* gx_qwen_rope_attention (parallel 0) or _parallel (parallel 1) for M tokens
 * of M different conversations at once: token t's Q|K|V row qkv[t*ldqkv],
 * position positions[t] of conversation slots[t] (slots required), its
 * Q8_0 heads at row t of q/scales/qsum -- the lock-step decode of several
 * conversations (qwen/place.go:33-41, one token a slot, as the server's
 * batch of slots).  Each token's values are those of the one-token call bit
 * for bit.  Two tokens of one conversation in one call are not allowed: a
 * token would not see the other's new cache entry. */
int gx_qwen_rope_attention_slots(gx_ctx *ctx, const float *qkv, int ldqkv, int M, int heads, int kv_heads,
                                 int head_dim, int max_pos, const int32_t *positions, const float *q_norm,
                                 const float *k_norm, const float *rope_cos, const float *rope_sin, float eps,
                                 uint16_t *kcache, uint16_t *vcache, int context, int8_t *q, float *scales,
                                 int32_t *qsum, const int32_t *slots, int nslots, int parallel);

/* The head outputs of gx_qwen_attention_parallel before their Q8_0, out
 * [M][heads*head_dim] (device floats): a decode step (M <= 4, prefixes to
 * 768) or a prompt (prefixes to 1024).  No counterpart in golem: parity
 * instrumentation for the parallel order. */
int gx_qwen_attention_heads(gx_ctx *ctx, const uint16_t *qh, int M, int heads, int kv_heads, int head_dim,
                            int max_pos, const int32_t *positions, const uint16_t *kcache, const uint16_t *vcache,
                            int context, float *out);

/* One position's RMSNormPlain + Q8_0 fused into the Q4_0 product that reads
 * it (M = 1): y[row] for rows [row_start, row_end) of w times
 * Q8_0(RMSNormPlain(x + add, gain, eps)), bit for bit gx_norm_quant followed
 * by gx_matmul_q4_0 (qwen/block.go:45-56, 59-72: a block's pre-norm and the
 * projection after it).  add may be NULL; x_out, when given, receives x + add
 * (the residual) and must not alias x or add.  x, add, gain (16-byte
 * aligned), x_out: device floats [w->cols]; y: device floats [w->rows]. */
int gx_norm_matmul_q4_0(gx_ctx *ctx, const gx_weight *w, const float *x, const float *add, const float *gain,
                        float eps, float *x_out, int row_start, int row_end, float *y);

/* The FFN's first half for one position (M = 1), fused: RMSNormPlain + Q8_0
 * of x + add as gx_norm_matmul_q4_0, the Gate and Up products of w, whose
 * rows are gate and up interleaved by 32 (rows 64k .. 64k+31 are gate rows
 * 32k .. 32k+31, the next 32 the same up rows), and silu(gate) * up with its
 * Q8_0 into q/scales/qsum [w->rows / 2] -- bit for bit gx_norm_quant,
 * gx_matmul_q4_0 and gx_swiglu_quant (group 32) (qwen/block.go:59-90,
 * nn/swiglu.go:77-82). */
int gx_norm_swiglu_q4_0(gx_ctx *ctx, const gx_weight *w, const float *x, const float *add, const float *gain,
                        float eps, float *x_out, int8_t *q, float *scales, int32_t *qsum);

/* gx_matmul_q4_0 over every row of a Gate|Up matrix whose gate and up rows
 * are interleaved by 32 (rows 64k .. 64k+31 gate rows 32k .., the next 32
 * the same up rows), then silu(gate) * up and its Q8_0 into mid_q
 * [M][rows/2], mid_scales and mid_qsum [M][rows/64] -- bit for bit
 * gx_matmul_q4_0 followed by gx_swiglu_quant (group 32) (qwen/block.go:
 * 82-90, nn/swiglu.go:77-82), in one kernel: 1 to 16 positions on the
 * matrix-vector kernels (golem's lock-step slots, short batches), more on
 * the int8 batch product with the same epilogue (a prompt).  No counterpart
 * in golem as one call. */
int gx_matmul_swiglu_q4_0(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const float *scales,
                          const int32_t *qsum, int M, int8_t *mid_q, float *mid_scales, int32_t *mid_qsum);

/* SwiGLURange (nn/swiglu.go:77-82) and the Q8_0 of the result: gu[m] holds
 * position m's gate (ffn floats) then up (ffn floats) when group is 0, or
 * gates and ups interleaved by 32 (32 gates, then their 32 ups, ...) when
 * group is 32; q/scales/qsum receive Q8_0(silu(gate) * up) [M][ffn].  ffn a
 * multiple of 32. */
int gx_swiglu_quant(gx_ctx *ctx, const float *gu, int ldgu, int M, int ffn, int group, int8_t *q, float *scales,
                    int32_t *qsum);

/* Greedy choice: ids[m] = the index of the largest of x[m][0..n), the lower
 * index on ties, by golem's rule (gemma/model.go:288-296,
 * qwen/model_test.go:118-126: start at index 0, move only to a greater
 * value): a NaN never wins except at index 0, where it wins outright, so the
 * pick is 0 when x[m][0] is NaN.
 * Workspace: the pick keeps its per-row partial results in scratch memory of
 * the context (allocated by gx_init).  Every gx_argmax / gx_argmax_step of one
 * context, including those recorded in a captured graph and replayed, must
 * therefore be ordered on one stream; two of them in flight at once on
 * different streams race on that scratch. */
int gx_argmax(gx_ctx *ctx, const float *x, int ldx, int M, int n, int32_t *ids);

/* One greedy step of a decode loop kept on the device (what golem's
 * generation loop does on the host after Logits, qwen/model.go): ids[0] =
 * gx_argmax of x[0..n); then, while *pos + 1 < history_len,
 * history[*pos + 1] = ids[0], *pos += 1 and positions[0] = the new *pos, so
 * that a captured decode step reads its next token and position from the
 * device.  At the history's end the counter stops (only ids[0] is written):
 * a step replayed past the end of the context never addresses past the
 * history, and gx_qwen_rope_attention stores nothing for a position outside
 * its cache.  pos, positions, history, ids: device int32.  The same workspace
 * rule as gx_argmax. */
int gx_argmax_step(gx_ctx *ctx, const float *x, int n, int32_t *ids, int32_t *history, int history_len,
                   int32_t *pos, int32_t *positions);

/* The greedy step of M conversations decoded in lock step (the server's
 * batch of slots, cmd/golem-server/runner.go:233-297, with the pick on the
 * device): ids[m] = gx_argmax of row m of x, then tokens[m] = ids[m] and
 * positions[m] += 1 -- row m's input to the next step -- in the same launch,
 * so a captured lock-step step needs no other work between replays.
 * tokens, positions, ids: device int32 [M].  The same workspace rule as
 * gx_argmax. */
int gx_argmax_slots_step(gx_ctx *ctx, const float *x, int ldx, int M, int n, int32_t *ids, int32_t *tokens,
                         int32_t *positions);

/* ---- calibration (measurement only) ----------------------------------- */

/* No counterpart in golem; no product calls these.  They give the
 * measurements beside the products their floors and ceilings on this GPU:
 * gx_calib_empty launches an empty kernel of `workgroups` workgroups (the
 * per-dispatch floor); gx_calib_read reads `bytes` (16-byte aligned, a
 * multiple of 16) with 16-byte non-temporal loads, each of `workgroups`
 * 512-thread workgroups a contiguous share (moving a product's bytes alone at
 * its grid), `sink` one word per workgroup, practically never written;
 * gx_calib_valu runs 8 * iters independent v_fmac_f32 per lane in 256-thread
 * workgroups (the VALU issue rate at saturation, for reading the SQ counters
 * of the products against). */
int gx_calib_empty(gx_ctx *ctx, int workgroups);
int gx_calib_read(gx_ctx *ctx, const void *src, size_t bytes, int workgroups, uint32_t *sink);
int gx_calib_valu(gx_ctx *ctx, int workgroups, int iters, float *sink);

/* ---- GGUF checkpoints (host only; no GPU needed) ----------------------- */

/* An opened GGUF file: mapped whole, read in place (tensors/gguf.go:33-41,
 * tensors/mmap.go).  Tensor data pointers point into the mapping and stay
 * valid until gx_gguf_close; gx_weight_upload(on_device = 0) takes them
 * directly.  Tensor types are ggml's numbers (0 F32, 1 F16, 2 Q4_0, 8 Q8_0,
 * 14 Q6_K, 30 BF16); metadata value types are GGUF's (0 uint8 ... 12
 * float64, 8 string, 9 array). */
typedef struct gx_gguf gx_gguf;

/* OpenGGUF (tensors/gguf.go:164-175): maps the file and reads the header,
 * metadata and tensor table, with golem's checks and messages ("not a GGUF
 * file", "GGUF version N, only 2 and 3 are read", "truncated at byte N",
 * "tensor \"x\" has N dimensions", "unsupported ggml type", a row that does not
 * divide into blocks, an alignment that is not a power of two, a tensor past
 * the end of the file), each prefixed with the path. */
int gx_gguf_open(const char *path, gx_gguf **out);
/* Close (tensors/gguf.go:314): unmaps; every pointer into the file dies. */
int gx_gguf_close(gx_gguf *g);

/* The tensor table (GGUF.Tensors): count, the name of entry i (file order,
 * a repeated name keeping its last entry), and Get (tensors/gguf.go:305):
 * type, dimensions (shape[0] is the row length), shape[4] (0 past ndims),
 * the data in the mapping and its size.  Any output may be NULL. */
int gx_gguf_tensor_count(const gx_gguf *g, int *count);
int gx_gguf_tensor_name(const gx_gguf *g, int index, const char **name);
int gx_gguf_tensor(const gx_gguf *g, const char *name, int *ggml_type, int *ndims, int64_t *shape,
                   const void **data, size_t *bytes);

/* The metadata (GGUF.Meta) and its typed accessors (tensors/gguf_meta.go):
 * String :18, Bool :30, Float32 :42 (float32 or float64), Uint32 :79 (any
 * integer width, converted as Go converts), Uint32Slice :88 and BoolSlice
 * (an array, or a scalar as an array of one), Strings (an array of strings;
 * string `index` of it when s is not NULL).  The *_s forms write at most
 * cap values and always the full count. */
int gx_gguf_meta_count(const gx_gguf *g, int *count);
int gx_gguf_meta_key(const gx_gguf *g, int index, const char **key, int *type);
int gx_gguf_meta_string(const gx_gguf *g, const char *key, const char **s, size_t *len);
int gx_gguf_meta_bool(const gx_gguf *g, const char *key, int *out);
int gx_gguf_meta_f32(const gx_gguf *g, const char *key, float *out);
int gx_gguf_meta_u32(const gx_gguf *g, const char *key, uint32_t *out);
int gx_gguf_meta_u32s(const gx_gguf *g, const char *key, uint32_t *out, size_t cap, size_t *count);
int gx_gguf_meta_bools(const gx_gguf *g, const char *key, uint8_t *out, size_t cap, size_t *count);
int gx_gguf_meta_strings(const gx_gguf *g, const char *key, size_t index, const char **s, size_t *len,
                         size_t *count);

#ifdef __cplusplus
}
#endif

#endif /* GOLEM_HIP_H */
