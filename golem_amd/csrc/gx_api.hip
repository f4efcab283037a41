// gx_api.hip - the C ABI of include/golem_hip.h: contexts, resident weights,
// argument checking, and dispatch to the kernels.
//
// Misuse is reported with golem's own panic messages (nn/dot_q4_0.go:119,
// nn/dot_q6_k.go:66-70, nn/batch.go:49-51, :75-77, :160-162,
// nn/matrix.go:124, :137) so a shim can panic with them unchanged.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <string>

#include "gx_internal.hpp"

namespace {
thread_local std::string g_error;

// The scratch of the entry points that allocate nothing (gx_moe_experts_noalloc):
// device memory of fixed size that the library holds on every GPU it runs
// on until the process ends.  Host code never passes `scratch` itself to a
// kernel -- on the host the name is only a stand-in -- but the address
// hipGetSymbolAddress gives for it on the context's device, kept in the
// context at gx_init.  Every call on one GPU shares it: calls that overlap
// on one GPU race, and each call finds what the last one left there.
constexpr size_t kScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];
}

namespace gx {

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

int succeed() {
    g_error.clear();
    return GX_OK;
}

int check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return fail(GX_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
    return GX_OK;
}

}  // namespace gx

static int ok() {
    g_error.clear();
    return GX_OK;
}

static int use(gx_ctx *ctx) {
    GX_CHECK(ctx != nullptr, "gx: no context");
    GX_HIP(hipSetDevice(ctx->device));
    return GX_OK;
}

// The coalesced MatVecRows products (gx_matvec_rows_*): golem's engines call
// MatVecRows on small row slices from pool workers (qwen/block.go:82-90,
// qwen/attention.go:57-84, gemma/moe.go:151-161).  The first call of a
// (matrix, activation, generation, M) computes every row once on the device
// and copies the product to pinned host memory; every call then copies its
// own rows from there.  A few products are kept, least recently used out.
struct gx_rows_entry {
    const gx_weight *w = nullptr;
    const void *act = nullptr;
    uint64_t generation = 0;
    int M = 0;
    bool valid = false;
    uint64_t last_use = 0;
    float *dev = nullptr;   // [M][rows], device
    float *host = nullptr;  // its copy, pinned host memory
    size_t cap = 0;         // floats each holds
};
constexpr int kRowsEntries = 16;
struct gx_rows {
    std::mutex mu;
    gx_rows_entry e[kRowsEntries];
    uint64_t clock = 0, products = 0, served = 0;
};

static void rows_release(gx_rows *r) {
    if (r == nullptr)
        return;
    for (gx_rows_entry &e : r->e) {
        (void)hipFree(e.dev);
        (void)hipHostFree(e.host);
    }
    delete r;
}

// Serves rows [row_start, row_end) of every column of w's product with an
// activation named by (act, generation, M); `product` writes the whole
// product into a device buffer of M x rows floats.
template <typename F>
static int rows_serve(gx_ctx *ctx, const gx_weight *w, const void *act, uint64_t generation, int M, int row_start,
                      int row_end, float *ys, int ldys, F &&product) {
    gx_rows *r = ctx->rows;
    std::lock_guard<std::mutex> lock(r->mu);
    gx_rows_entry *hit = nullptr;
    for (gx_rows_entry &e : r->e)
        if (e.valid && e.w == w && e.act == act && e.generation == generation && e.M == M)
            hit = &e;
    if (hit == nullptr) {
        hit = &r->e[0];
        for (gx_rows_entry &e : r->e)
            if (!e.valid || e.last_use < hit->last_use)
                hit = &e;
        hit->valid = false;
        const size_t need = (size_t)M * w->rows;
        if (hit->cap < need) {
            (void)hipFree(hit->dev);
            (void)hipHostFree(hit->host);
            hit->dev = nullptr;
            hit->host = nullptr;
            hit->cap = 0;
            GX_HIP(hipMalloc(&hit->dev, need * sizeof(float)));
            GX_HIP(hipHostMalloc(&hit->host, need * sizeof(float), hipHostMallocDefault));
            hit->cap = need;
        }
        if (int rc = product(hit->dev))
            return rc;
        GX_HIP(hipMemcpyAsync(hit->host, hit->dev, need * sizeof(float), hipMemcpyDeviceToHost, ctx->stream));
        GX_HIP(hipStreamSynchronize(ctx->stream));
        hit->w = w;
        hit->act = act;
        hit->generation = generation;
        hit->M = M;
        hit->valid = true;
        r->products++;
    }
    hit->last_use = ++r->clock;
    const int n = row_end - row_start;
    for (int m = 0; m < M && n > 0; m++)
        memcpy(ys + (size_t)m * ldys + row_start, hit->host + (size_t)m * w->rows + row_start, (size_t)n * sizeof(float));
    r->served++;
    return GX_OK;
}

static int rows_check(const gx_weight *w, int quant, int M, int row_start, int row_end, const float *ys, int ldys) {
    GX_CHECK(w != nullptr, "gx: no weights");
    GX_CHECK(w->quant == quant, "gx: the matrix is not %s", quant == GX_Q4_0 ? "Q4_0" : "Q6_K");
    GX_CHECK(w->count == 1, "gx: a row-slice product takes a single matrix");
    GX_CHECK(M >= 1, "gx: M must be at least 1, not %d", M);
    GX_CHECK(row_start >= 0 && row_start <= row_end && row_end <= w->rows,
             "nn: rows [%d, %d) outside a %d-row matrix", row_start, row_end, w->rows);
    GX_CHECK(ys != nullptr && ldys >= row_end, "gx: ys must hold rows up to %d a column (ldys %d)", row_end, ldys);
    return GX_OK;
}

extern "C" {

const char *gx_last_error(void) { return g_error.c_str(); }

int gx_init(int device, gx_ctx **out) {
    GX_CHECK(out != nullptr, "gx: no place for the context");
    int n = 0;
    GX_HIP(hipGetDeviceCount(&n));
    GX_CHECK(device >= 0 && device < n, "gx: device %d out of %d", device, n);
    GX_HIP(hipSetDevice(device));
    gx_ctx *ctx = new gx_ctx();
    ctx->device = device;
    ctx->stream = nullptr;
    hipDeviceProp_t prop;
    hipError_t e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) {
        delete ctx;
        return gx::fail(GX_ERR_HIP, "hipGetDeviceProperties: %s", hipGetErrorString(e));
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        delete ctx;
        return gx::fail(GX_ERR_UNSUPPORTED, "gx: built for gfx950, device %d is %s", device, prop.gcnArchName);
    }
    ctx->cu_count = prop.multiProcessorCount;
    if (hipEventCreate(&ctx->t0) != hipSuccess || hipEventCreate(&ctx->t1) != hipSuccess) {
        delete ctx;
        return gx::fail(GX_ERR_HIP, "hipEventCreate failed");
    }
    ctx->gelu_table = nullptr;
    ctx->argmax_v = nullptr;
    ctx->argmax_i = nullptr;
    ctx->scratch = nullptr;
    ctx->route_scale = nullptr;
    ctx->rows = new gx_rows();
    auto undo = [ctx]() {
        rows_release(ctx->rows);
        (void)hipFree(ctx->route_scale);
        (void)hipFree(ctx->gelu_table);
        (void)hipFree(ctx->argmax_v);
        (void)hipFree(ctx->argmax_i);
        (void)hipEventDestroy(ctx->t0);
        (void)hipEventDestroy(ctx->t1);
        delete ctx;
    };
    if (hipMalloc(&ctx->gelu_table, 65536 * sizeof(float)) != hipSuccess) {
        undo();
        return gx::fail(GX_ERR_NOMEM, "gx: cannot allocate the GELU table");
    }
    if (hipMalloc(&ctx->argmax_v, kArgmaxRows * kArgmaxParts * sizeof(float)) != hipSuccess ||
        hipMalloc(&ctx->argmax_i, kArgmaxRows * kArgmaxParts * sizeof(int32_t)) != hipSuccess) {
        undo();
        return gx::fail(GX_ERR_NOMEM, "gx: cannot allocate the greedy pick's workspace");
    }
    if (hipMalloc(&ctx->route_scale, kRouteScaleMax * sizeof(float)) != hipSuccess) {
        undo();
        return gx::fail(GX_ERR_NOMEM, "gx: cannot allocate the router's scales");
    }
    {
        // this device's address of the static scratch (the device is current)
        void *sp = nullptr;
        const hipError_t e = hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch));
        if (e != hipSuccess || sp == nullptr) {
            undo();
            return gx::fail(GX_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        }
        ctx->scratch = (uint8_t *)sp;
    }
    if (int rc = gx::launch_gelu_table(ctx, ctx->gelu_table)) {
        undo();
        return rc;
    }
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) {
        undo();
        return gx::fail(GX_ERR_HIP, "gx: building the GELU table failed");
    }
    *out = ctx;
    return ok();
}

int gx_free(gx_ctx *ctx) {
    if (ctx == nullptr)
        return ok();
    (void)hipSetDevice(ctx->device);
    (void)hipEventDestroy(ctx->t0);
    (void)hipEventDestroy(ctx->t1);
    (void)hipFree(ctx->gelu_table);
    (void)hipFree(ctx->argmax_v);
    (void)hipFree(ctx->argmax_i);
    (void)hipFree(ctx->route_scale);
    rows_release(ctx->rows);
    delete ctx;
    return ok();
}

int gx_set_stream(gx_ctx *ctx, void *stream) {
    if (int rc = use(ctx))
        return rc;
    ctx->stream = (hipStream_t)stream;
    return ok();
}

int gx_sync(gx_ctx *ctx) {
    if (int rc = use(ctx))
        return rc;
    GX_HIP(hipStreamSynchronize(ctx->stream));
    return ok();
}

int gx_alloc(gx_ctx *ctx, size_t bytes, void **device) {
    if (int rc = use(ctx))
        return rc;
    GX_CHECK(device != nullptr, "gx: no place for the pointer");
    if (hipMalloc(device, bytes == 0 ? 1 : bytes) != hipSuccess)
        return gx::fail(GX_ERR_NOMEM, "gx: cannot allocate %zu bytes", bytes);
    return ok();
}

int gx_dealloc(gx_ctx *ctx, void *device) {
    if (int rc = use(ctx))
        return rc;
    GX_HIP(hipFree(device));
    return ok();
}

int gx_upload(gx_ctx *ctx, void *device, const void *host, size_t bytes) {
    if (int rc = use(ctx))
        return rc;
    GX_HIP(hipMemcpyAsync(device, host, bytes, hipMemcpyHostToDevice, ctx->stream));
    GX_HIP(hipStreamSynchronize(ctx->stream));
    return ok();
}

int gx_download(gx_ctx *ctx, void *host, const void *device, size_t bytes) {
    if (int rc = use(ctx))
        return rc;
    GX_HIP(hipMemcpyAsync(host, device, bytes, hipMemcpyDeviceToHost, ctx->stream));
    GX_HIP(hipStreamSynchronize(ctx->stream));
    return ok();
}

int gx_timer_start(gx_ctx *ctx) {
    if (int rc = use(ctx))
        return rc;
    GX_HIP(hipEventRecord(ctx->t0, ctx->stream));
    return ok();
}

int gx_timer_stop(gx_ctx *ctx, float *ms) {
    if (int rc = use(ctx))
        return rc;
    GX_CHECK(ms != nullptr, "gx: no place for the time");
    GX_HIP(hipEventRecord(ctx->t1, ctx->stream));
    GX_HIP(hipEventSynchronize(ctx->t1));
    GX_HIP(hipEventElapsedTime(ms, ctx->t0, ctx->t1));
    return ok();
}

// ---- weights -------------------------------------------------------------

static int weight_upload(gx_ctx *ctx, const void *data, size_t bytes, int on_device, int quant, int rows, int cols,
                         int count, gx_weight **out) {
    if (int rc = use(ctx))
        return rc;
    GX_CHECK(out != nullptr && data != nullptr, "gx: no weights");
    GX_CHECK(rows > 0 && cols > 0 && count > 0, "nn: a matrix needs rows and columns");
    size_t src_row = 0;
    gx_weight w{};
    w.ctx = ctx;
    w.quant = quant;
    w.rows = rows;
    w.cols = cols;
    w.count = count;
    w.tiles = (rows + gx::kTileRows - 1) / gx::kTileRows;
    switch (quant) {
    case GX_Q4_0:
        GX_CHECK(cols % gx::kQ4Block == 0, "nn: Q4_0 rows must be a multiple of the block size");
        w.blocks = cols / gx::kQ4Block;
        w.dchunks = (w.blocks + 7) / 8;
        w.plane0_bytes = (size_t)w.tiles * w.blocks * gx::kTileRows * gx::kChunk;
        w.matrix_bytes = w.plane0_bytes + (size_t)w.tiles * w.dchunks * gx::kTileRows * gx::kChunk;
        src_row = (size_t)w.blocks * gx::kQ4BlockBytes;
        break;
    case GX_Q6_K:
        GX_CHECK(cols % gx::kSuper == 0, "nn: Q6_K rows must be a multiple of the superblock size");
        w.blocks = cols / gx::kSuper;
        w.dchunks = (w.blocks + 7) / 8;
        w.plane0_bytes = (size_t)w.tiles * w.blocks * gx::kQ6Chunks * gx::kTileRows * gx::kChunk;
        w.matrix_bytes = w.plane0_bytes + (size_t)w.tiles * w.dchunks * gx::kTileRows * gx::kChunk;
        src_row = (size_t)w.blocks * gx::kQ6BlockBytes;
        break;
    case GX_F32:
        w.blocks = cols;
        w.plane0_bytes = (size_t)rows * cols * 4;
        w.matrix_bytes = w.plane0_bytes;
        src_row = (size_t)cols * 4;
        break;
    default:
        return gx::fail(GX_ERR_UNSUPPORTED, "nn: quant %d is not a matrix format this build multiplies", quant);
    }
    const size_t need = src_row * rows * count;
    GX_CHECK(bytes >= need, "gx: %zu bytes given, a %dx%d matrix (x%d) needs %zu", bytes, rows, cols, count, need);

    gx_weight *wp = new gx_weight(w);
    if (hipMalloc(&wp->dev, wp->matrix_bytes * count) != hipSuccess) {
        delete wp;
        return gx::fail(GX_ERR_NOMEM, "gx: cannot allocate %zu bytes for weights", w.matrix_bytes * count);
    }
    int rc = GX_OK;
    if (quant == GX_F32) {
        hipError_t e = hipMemcpyAsync(wp->dev, data, need, on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice,
                                      ctx->stream);
        if (e != hipSuccess)
            rc = gx::fail(GX_ERR_HIP, "weight copy: %s", hipGetErrorString(e));
    } else {
        // Stage the GGUF bytes on the device and repack them there.
        const uint8_t *src = (const uint8_t *)data;
        uint8_t *staged = nullptr;
        if (!on_device) {
            if (hipMalloc(&staged, need) != hipSuccess) {
                (void)hipFree(wp->dev);
                delete wp;
                return gx::fail(GX_ERR_NOMEM, "gx: cannot allocate %zu bytes to stage weights", need);
            }
            hipError_t e = hipMemcpyAsync(staged, data, need, hipMemcpyHostToDevice, ctx->stream);
            if (e != hipSuccess)
                rc = gx::fail(GX_ERR_HIP, "weight copy: %s", hipGetErrorString(e));
            src = staged;
        }
        if (rc == GX_OK) {
            hipError_t e = hipMemsetAsync(wp->dev, 0, wp->matrix_bytes * count, ctx->stream);
            if (e != hipSuccess)
                rc = gx::fail(GX_ERR_HIP, "weight clear: %s", hipGetErrorString(e));
        }
        if (rc == GX_OK)
            rc = gx::launch_repack(ctx, src, wp);
        if (staged) {
            hipError_t e = hipStreamSynchronize(ctx->stream);
            if (e != hipSuccess && rc == GX_OK)
                rc = gx::fail(GX_ERR_HIP, "weight repack: %s", hipGetErrorString(e));
            (void)hipFree(staged);
        }
    }
    if (rc == GX_OK) {
        hipError_t e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess)
            rc = gx::fail(GX_ERR_HIP, "weight upload: %s", hipGetErrorString(e));
    }
    if (rc != GX_OK) {
        (void)hipFree(wp->dev);
        delete wp;
        return rc;
    }
    *out = wp;
    return ok();
}

int gx_weight_upload(gx_ctx *ctx, const void *data, size_t bytes, int on_device, int quant, int rows, int cols,
                     gx_weight **out) {
    return weight_upload(ctx, data, bytes, on_device, quant, rows, cols, 1, out);
}

int gx_weight_upload_stack(gx_ctx *ctx, const void *data, size_t bytes, int on_device, int quant, int rows,
                           int cols, int count, gx_weight **out) {
    return weight_upload(ctx, data, bytes, on_device, quant, rows, cols, count, out);
}

int gx_weight_free(gx_weight *w) {
    if (w == nullptr)
        return ok();
    (void)hipSetDevice(w->ctx->device);
    {  // a later matrix at the same address must not find this one's products
        std::lock_guard<std::mutex> lock(w->ctx->rows->mu);
        for (gx_rows_entry &e : w->ctx->rows->e)
            if (e.w == w)
                e.valid = false;
    }
    (void)hipFree(w->dev);
    delete w;
    return ok();
}

int gx_weight_info(const gx_weight *w, int *quant, int *rows, int *cols, int *count, size_t *device_bytes) {
    GX_CHECK(w != nullptr, "gx: no weights");
    if (quant)
        *quant = w->quant;
    if (rows)
        *rows = w->rows;
    if (cols)
        *cols = w->cols;
    if (count)
        *count = w->count;
    if (device_bytes)
        *device_bytes = w->matrix_bytes * w->count;
    return ok();
}

int gx_weight_rows(gx_ctx *ctx, const gx_weight *w, int expert, const int32_t *ids, int n, float *out) {
    if (int rc = use(ctx))
        return rc;
    GX_CHECK(w != nullptr && ids != nullptr && out != nullptr, "gx: missing argument");
    GX_CHECK(expert >= 0 && expert < w->count, "gx: expert %d out of %d", expert, w->count);
    GX_CHECK(n >= 0, "gx: negative row count");
    if (n == 0)
        return ok();
    if (int rc = gx::launch_rows(ctx, w, expert, ids, n, out))
        return rc;
    return ok();
}

// ---- activations ---------------------------------------------------------

int gx_quantize_q8_0(gx_ctx *ctx, const float *x, int ldx, int M, int K, int8_t *q, float *scales, int32_t *qsum,
                     float *corr, uint16_t *q16) {
    if (int rc = use(ctx))
        return rc;
    GX_CHECK(K % gx::kQ4Block == 0 && K > 0, "nn: activation length must be a multiple of the block size");
    GX_CHECK(M >= 0 && ldx >= K, "gx: bad batch shape M=%d ldx=%d K=%d", M, ldx, K);
    GX_CHECK(x && q && scales && qsum, "gx: missing argument");
    if (M == 0)
        return ok();
    if (int rc = gx::launch_quantize_q8_0(ctx, x, ldx, M, K, q, scales, qsum, corr, q16))
        return rc;
    return ok();
}

int gx_quantize_q8_k(gx_ctx *ctx, const float *x, int ldx, int M, int K, int8_t *q, float *kscales,
                     int16_t *bsums) {
    if (int rc = use(ctx))
        return rc;
    GX_CHECK(K % gx::kSuper == 0 && K > 0, "nn: the Q8_K form needs a multiple of the superblock size");
    GX_CHECK(M >= 0 && ldx >= K, "gx: bad batch shape M=%d ldx=%d K=%d", M, ldx, K);
    GX_CHECK(x && q && kscales && bsums, "gx: missing argument");
    GX_CHECK(((uintptr_t)x & 15) == 0 && ldx % 4 == 0 && ((uintptr_t)q & 3) == 0,
             "gx: the Q8_K quantiser needs x 16-byte aligned, ldx a multiple of 4 and q 4-byte aligned");
    if (M == 0)
        return ok();
    if (int rc = gx::launch_quantize_q8_k(ctx, x, ldx, M, K, q, kscales, bsums))
        return rc;
    return ok();
}

// ---- products ------------------------------------------------------------

static int check_product(const gx_weight *w, int quant, int M, int row_start, int row_end, const void *y, int ldy) {
    GX_CHECK(w != nullptr, "gx: no weights");
    GX_CHECK(w->quant == quant, "gx: a %s product was asked of a matrix of quant %d",
             quant == GX_Q4_0 ? "Q4_0" : quant == GX_Q6_K ? "Q6_K" : "F32", w->quant);
    GX_CHECK(M >= 0, "gx: negative batch");
    GX_CHECK(row_start >= 0 && row_start <= row_end && row_end <= w->rows, "nn: rows [%d,%d) out of %d", row_start,
             row_end, w->rows);
    GX_CHECK(y != nullptr || M == 0, "gx: no output");
    GX_CHECK(ldy >= row_end || M <= 1, "gx: ldy %d shorter than row %d", ldy, row_end);
    return GX_OK;
}

static int q4_0_product(gx_ctx *ctx, const gx_weight *w, int expert, const int8_t *q, const float *scales,
                        const int32_t *qsum, const uint16_t *q16, int M, int row_start, int row_end,
                        const float *bias, float *y, int ldy) {
    if (int rc = use(ctx))
        return rc;
    if (int rc = check_product(w, GX_Q4_0, M, row_start, row_end, y, ldy))
        return rc;
    GX_CHECK(expert >= 0 && expert < w->count, "gx: expert %d out of %d", expert, w->count);
    GX_CHECK(q && scales && qsum, "nn: a Q4_0 product needs the activation in its Q8_0 form");
    GX_CHECK(((uintptr_t)q & 15) == 0, "gx: q must be 16-byte aligned");
    if (M == 0 || row_start == row_end)
        return ok();
    const uint8_t *mat = w->dev + (size_t)expert * w->matrix_bytes;
    GX_CHECK(((uintptr_t)q16 & 15) == 0, "gx: q16 must be 16-byte aligned");
    // Every batch runs on int8 MFMA, q16 or not: the fp16-MFMA kernel is
    // slower at every M measured (config 2, M = 64 / 512 / 2048: 34.5 / 96.9
    // / 269.8 us against 16.7 / 55.5 / 186.0) and moves 2.6x its bytes; it
    // stays reachable for the parity checks (gx_q4_0_block_dots path 2).
    int rc;
    if (M <= 16)
        rc = gx::launch_q4_0_matvec(ctx, w, mat, q, scales, qsum, M, row_start, row_end, bias, y, ldy, nullptr, -1);
    else
        rc = gx::launch_q4_0_gemm(ctx, w, mat, q, scales, M, row_start, row_end, bias, y, ldy, nullptr);
    if (rc)
        return rc;
    return ok();
}

int gx_matmul_q4_0(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const float *scales, const int32_t *qsum,
                   const uint16_t *q16, int M, int row_start, int row_end, const float *bias, float *y, int ldy) {
    return q4_0_product(ctx, w, 0, q, scales, qsum, q16, M, row_start, row_end, bias, y, ldy);
}

int gx_norm_matmul_q4_0(gx_ctx *ctx, const gx_weight *w, const float *x, const float *add, const float *gain,
                        float eps, float *x_out, int row_start, int row_end, float *y) {
    if (int rc = use(ctx))
        return rc;
    if (int rc = check_product(w, GX_Q4_0, 1, row_start, row_end, y, row_end))
        return rc;
    GX_CHECK(w->count == 1, "gx: a fused product takes a single matrix");
    GX_CHECK(x && gain, "gx: missing argument");
    GX_CHECK(((uintptr_t)gain & 15) == 0, "gx: gain must be 16-byte aligned");
    GX_CHECK(x_out == nullptr || (x_out != x && x_out != add),
             "gx: x_out must not alias x or add (other workgroups still read them)");
    if (row_start == row_end)
        return ok();
    if (int rc = gx::launch_q4_0_matvec_fused(ctx, w, 0, row_start, row_end, y, x, add, gain, eps, x_out, nullptr,
                                              nullptr, nullptr, nullptr))
        return rc;
    return ok();
}

int gx_norm_swiglu_q4_0(gx_ctx *ctx, const gx_weight *w, const float *x, const float *add, const float *gain,
                        float eps, float *x_out, int8_t *q, float *scales, int32_t *qsum) {
    if (int rc = use(ctx))
        return rc;
    if (int rc = check_product(w, GX_Q4_0, 1, 0, w ? w->rows : 0, q, 0))
        return rc;
    GX_CHECK(w->count == 1, "gx: a fused product takes a single matrix");
    GX_CHECK(w->rows % 64 == 0, "gx: gate and up interleaved by 32 need a multiple of 64 rows, not %d", w->rows);
    GX_CHECK(x && gain && scales && qsum, "gx: missing argument");
    GX_CHECK(((uintptr_t)gain & 15) == 0, "gx: gain must be 16-byte aligned");
    GX_CHECK(x_out == nullptr || (x_out != x && x_out != add),
             "gx: x_out must not alias x or add (other workgroups still read them)");
    if (int rc = gx::launch_q4_0_matvec_fused(ctx, w, 1, 0, w->rows, nullptr, x, add, gain, eps, x_out, q, scales,
                                              qsum, nullptr))
        return rc;
    return ok();
}

int gx_q4_0_fused_block_dots(gx_ctx *ctx, const gx_weight *w, int swiglu, const float *x, const float *add,
                             const float *gain, float eps, int row_start, int row_end, int8_t *q, float *scales,
                             int32_t *qsum, int32_t *out) {
    if (int rc = use(ctx))
        return rc;
    if (int rc = check_product(w, GX_Q4_0, 1, row_start, row_end, out, row_end))
        return rc;
    GX_CHECK(w->count == 1, "gx: a fused product takes a single matrix");
    GX_CHECK(x && gain && out, "gx: missing argument");
    GX_CHECK(((uintptr_t)gain & 15) == 0, "gx: gain must be 16-byte aligned");
    GX_CHECK(swiglu == 0 || (row_start == 0 && row_end == w->rows && w->rows % 64 == 0 && q && scales && qsum),
             "gx: the SwiGLU form takes every row (a multiple of 64) and its Q8_0 outputs");
    if (row_start == row_end)
        return ok();
    if (int rc = gx::launch_q4_0_matvec_fused(ctx, w, swiglu ? 1 : 0, row_start, row_end, nullptr, x, add, gain, eps,
                                              nullptr, q, scales, qsum, out))
        return rc;
    return ok();
}

int gx_matmul_q4_0_expert(gx_ctx *ctx, const gx_weight *w, int expert, const int8_t *q, const float *scales,
                          const int32_t *qsum, const uint16_t *q16, int M, int row_start, int row_end, float *y,
                          int ldy) {
    return q4_0_product(ctx, w, expert, q, scales, qsum, q16, M, row_start, row_end, nullptr, y, ldy);
}

int gx_matmul_q6_k(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const float *kscales, const int16_t *bsums,
                   int M, int row_start, int row_end, const float *bias, float *y, int ldy) {
    if (int rc = use(ctx))
        return rc;
    if (int rc = check_product(w, GX_Q6_K, M, row_start, row_end, y, ldy))
        return rc;
    GX_CHECK(q && kscales && bsums, "nn: a Q6_K product needs the activation in its Q8_K form");
    GX_CHECK(((uintptr_t)q & 15) == 0 && ((uintptr_t)bsums & 15) == 0, "gx: q and bsums must be 16-byte aligned");
    if (M == 0 || row_start == row_end)
        return ok();
    if (int rc = gx::launch_q6_k_matvec(ctx, w, q, kscales, bsums, M, row_start, row_end, bias, y, ldy, nullptr))
        return rc;
    return ok();
}

int gx_matmul_swiglu_q4_0(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const float *scales,
                          const int32_t *qsum, int M, int8_t *mid_q, float *mid_scales, int32_t *mid_qsum) {
    if (int rc = use(ctx))
        return rc;
    if (int rc = check_product(w, GX_Q4_0, M, 0, w ? w->rows : 0, mid_q, w ? w->rows : 0))
        return rc;
    GX_CHECK(w->count == 1, "gx: a SwiGLU product takes a single matrix");
    GX_CHECK(w->rows % 64 == 0,
             "gx: the SwiGLU form needs gate and up rows interleaved by 32 (rows a multiple of 64, not %d)", w->rows);
    GX_CHECK(M >= 0, "gx: %d columns", M);
    GX_CHECK(q && scales && qsum && mid_q && mid_scales && mid_qsum, "gx: missing argument");
    GX_CHECK(((uintptr_t)q & 15) == 0, "gx: q must be 16-byte aligned");
    if (M == 0)
        return ok();
    // 1..16 columns on the matrix-vector kernels, more on the int8 batch
    // product with the same epilogue
    if (int rc = M <= 16 ? gx::launch_q4_0_matvec_swiglu(ctx, w, q, scales, qsum, M, mid_q, mid_scales, mid_qsum)
                         : gx::launch_q4_0_gemm_swiglu(ctx, w, q, scales, M, mid_q, mid_scales, mid_qsum))
        return rc;
    return ok();
}

int gx_matvec_rows_q4_0(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const float *scales, const int32_t *qsum,
                        int M, uint64_t generation, int row_start, int row_end, float *ys, int ldys) {
    if (int rc = use(ctx))
        return rc;
    if (int rc = rows_check(w, GX_Q4_0, M, row_start, row_end, ys, ldys))
        return rc;
    GX_CHECK(w->ctx == ctx, "gx: the matrix belongs to another context");
    if (int rc = rows_serve(ctx, w, q, generation, M, row_start, row_end, ys, ldys, [&](float *dev) {
            return q4_0_product(ctx, w, 0, q, scales, qsum, nullptr, M, 0, w->rows, nullptr, dev, w->rows);
        }))
        return rc;
    return ok();
}

int gx_matvec_rows_q6_k(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const float *kscales, const int16_t *bsums,
                        int M, uint64_t generation, int row_start, int row_end, float *ys, int ldys) {
    if (int rc = use(ctx))
        return rc;
    if (int rc = rows_check(w, GX_Q6_K, M, row_start, row_end, ys, ldys))
        return rc;
    GX_CHECK(w->ctx == ctx, "gx: the matrix belongs to another context");
    if (int rc = rows_serve(ctx, w, q, generation, M, row_start, row_end, ys, ldys, [&](float *dev) {
            return gx_matmul_q6_k(ctx, w, q, kscales, bsums, M, 0, w->rows, nullptr, dev, w->rows);
        }))
        return rc;
    return ok();
}

int gx_matvec_rows_stats(gx_ctx *ctx, uint64_t *products, uint64_t *served) {
    GX_CHECK(ctx != nullptr, "gx: no context");
    std::lock_guard<std::mutex> lock(ctx->rows->mu);
    if (products)
        *products = ctx->rows->products;
    if (served)
        *served = ctx->rows->served;
    return ok();
}

int gx_matmul_f32(gx_ctx *ctx, const gx_weight *w, const float *x, int ldx, int M, int row_start, int row_end,
                  float *y, int ldy) {
    if (int rc = use(ctx))
        return rc;
    if (int rc = check_product(w, GX_F32, M, row_start, row_end, y, ldy))
        return rc;
    GX_CHECK(x != nullptr && ldx >= w->cols, "gx: bad activation");
    if (M == 0 || row_start == row_end)
        return ok();
    if (int rc = gx::launch_f32_matvec(ctx, w, x, ldx, M, row_start, row_end, y, ldy))
        return rc;
    return ok();
}

int gx_q4_0_block_dots(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const float *scales, const int32_t *qsum,
                       const uint16_t *q16, int M, int row_start, int row_end, int path, int32_t *out) {
    if (int rc = use(ctx))
        return rc;
    if (int rc = check_product(w, GX_Q4_0, M, row_start, row_end, out, row_end))
        return rc;
    GX_CHECK(q && qsum && scales, "gx: missing activation");
    GX_CHECK(((uintptr_t)q & 15) == 0, "gx: q must be 16-byte aligned");
    GX_CHECK(path >= 0 && path <= 5,
             "gx: path must be 0 (matrix-vector), 1 (int8 MFMA), 2 (fp16 MFMA), 3 (one-column matrix-vector), 4 "
             "(multi-column matrix-vector) or 5 (few-column MFMA)");
    GX_CHECK(path != 2 || (q16 && ((uintptr_t)q16 & 15) == 0), "gx: path 2 needs a 16-byte aligned q16");
    GX_CHECK(path != 3 || M == 1, "gx: path 3 takes one column, not %d", M);
    if (M == 0 || row_start == row_end)
        return ok();
    int rc;
    if (path == 0 || path >= 3)
        rc = gx::launch_q4_0_matvec(ctx, w, w->dev, q, scales, qsum, M, row_start, row_end, nullptr, nullptr, 0, out,
                                    path == 0 ? 0 : path - 2);
    else if (path == 1)
        rc = gx::launch_q4_0_gemm(ctx, w, w->dev, q, scales, M, row_start, row_end, nullptr, nullptr, 0, out);
    else
        rc = gx::launch_q4_0_gemm_f16(ctx, w, w->dev, q16, nullptr, M, row_start, row_end, nullptr, nullptr, 0, out);
    if (rc)
        return rc;
    return ok();
}

int gx_moe_block_dots(gx_ctx *ctx, const gx_weight *gate_up, const gx_weight *down, const float *x, int ldx, int M,
                      int top_k, const int32_t *ids, const int8_t *mid_q, const float *mid_scales,
                      const int32_t *mid_qsum, void *workspace, size_t workspace_bytes, int32_t *dots_gate_up,
                      int32_t *dots_down) {
    if (int rc = use(ctx))
        return rc;
    GX_CHECK(gate_up && down && gate_up->quant == GX_Q4_0 && down->quant == GX_Q4_0,
             "gx: the expert stacks are Q4_0 matrices");
    GX_CHECK(gate_up->count == down->count, "gx: %d gate_up experts but %d down experts", gate_up->count, down->count);
    GX_CHECK(gate_up->rows == 2 * down->cols && down->rows == gate_up->cols,
             "gx: gate_up is %dx%d and down %dx%d: want 2F x D and D x F", gate_up->rows, gate_up->cols, down->rows,
             down->cols);
    GX_CHECK(top_k > 0 && top_k <= gate_up->count, "gx: top_k %d out of range", top_k);
    GX_CHECK(M >= 0, "gx: bad batch shape");
    GX_CHECK(ids && (!dots_gate_up || (x && ldx >= gate_up->cols)) &&
                 (!dots_down || (mid_q && mid_scales && mid_qsum)),
             "gx: missing argument");
    if (M > 4) {
        size_t need = 0;
        gx::moe_workspace_bytes(M, top_k, gate_up->cols, down->cols, gate_up->count, &need);
        GX_CHECK(workspace && ((uintptr_t)workspace & 255) == 0 && workspace_bytes >= need,
                 "gx: more than 4 positions need the experts' workspace (%zu bytes, 256-byte aligned)", need);
    }
    if (M == 0)
        return ok();
    if (int rc = gx::launch_moe_block_dots(ctx, gate_up, down, x, ldx, M, top_k, ids, mid_q, mid_scales, mid_qsum,
                                           (uint8_t *)workspace, dots_gate_up, dots_down))
        return rc;
    return ok();
}

int gx_q6_k_block_dots(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const int16_t *bsums, int M, int row_start,
                       int row_end, int32_t *out) {
    if (int rc = use(ctx))
        return rc;
    if (int rc = check_product(w, GX_Q6_K, M, row_start, row_end, out, row_end))
        return rc;
    GX_CHECK(q && bsums, "gx: missing activation");
    GX_CHECK(((uintptr_t)q & 15) == 0 && ((uintptr_t)bsums & 15) == 0, "gx: q and bsums must be 16-byte aligned");
    if (M == 0 || row_start == row_end)
        return ok();
    if (int rc = gx::launch_q6_k_matvec(ctx, w, q, nullptr, bsums, M, row_start, row_end, nullptr, nullptr, 0, out))
        return rc;
    return ok();
}

// ---- mixture of experts --------------------------------------------------

int gx_gelu_table(gx_ctx *ctx, float *out) {
    if (int rc = use(ctx))
        return rc;
    GX_CHECK(out != nullptr, "gx: no output");
    GX_HIP(hipMemcpyAsync(out, ctx->gelu_table, 65536 * sizeof(float), hipMemcpyDeviceToDevice, ctx->stream));
    return ok();
}

int gx_moe_workspace_bytes(int M, int top_k, int dim, int ffn, int experts, size_t *bytes) {
    GX_CHECK(bytes != nullptr, "gx: no place for the size");
    GX_CHECK(M >= 0 && top_k > 0 && dim > 0 && ffn > 0 && experts > 0, "gx: bad mixture shape");
    return gx::moe_workspace_bytes(M, top_k, dim, ffn, experts, bytes) == GX_OK ? ok() : GX_ERR_INVALID;
}

int gx_moe_route(gx_ctx *ctx, const gx_weight *router, const float *router_scale, const float *resid, int ldr, int M,
                 int top_k, float eps, float *logits, int32_t *ids, float *weights) {
    if (int rc = use(ctx))
        return rc;
    GX_CHECK(router != nullptr && router->quant == GX_F32 && router->count == 1, "gx: the router is an F32 matrix");
    GX_CHECK(top_k > 0 && top_k <= router->rows && top_k <= 64, "gx: top_k %d out of range for %d experts", top_k,
             router->rows);
    GX_CHECK(M >= 0 && ldr >= router->cols, "gx: bad residual shape");
    GX_CHECK(resid && logits && ids && weights, "gx: missing argument");
    if (M == 0)
        return ok();
    if (int rc = gx::launch_moe_route(ctx, router, router_scale, resid, ldr, M, top_k, eps, logits, ids, weights))
        return rc;
    return ok();
}

int gx_norm_quant(gx_ctx *ctx, float *x, int ldx, const float *add, int lda, const float *gain, int M, int K,
                  float eps, float *out, int ldo, int8_t *q, float *scales, int32_t *qsum) {
    if (int rc = use(ctx))
        return rc;
    GX_CHECK(K > 0 && K % 32 == 0, "nn: activation length must be a multiple of the block size");
    GX_CHECK(M >= 0 && ldx >= K && (!add || lda >= K) && (!out || ldo >= K), "gx: bad batch shape");
    GX_CHECK(x && gain && (out || q) && (!q || (scales && qsum)), "gx: missing argument");
    GX_CHECK(((uintptr_t)q & 3) == 0, "gx: q must be 4-byte aligned");
    if (M == 0)
        return ok();
    if (int rc = gx::launch_qwen_norm_quant(ctx, x, ldx, add, lda, gain, M, K, eps, out, ldo, q, scales, qsum))
        return rc;
    return ok();
}

int gx_qwen_qk_rope(gx_ctx *ctx, const float *qkv, int ldqkv, int M, int heads, int kv_heads, int head_dim,
                    const int32_t *positions, const float *q_norm, const float *k_norm, const float *rope_cos,
                    const float *rope_sin, float eps, uint16_t *qh, uint16_t *kcache, uint16_t *vcache, int context,
                    const int32_t *slots, int nslots) {
    if (int rc = use(ctx))
        return rc;
    GX_CHECK(heads > 0 && kv_heads > 0 && heads % kv_heads == 0, "gx: %d query heads over %d key-value heads", heads,
             kv_heads);
    GX_CHECK(M >= 0 && ldqkv >= (heads + 2 * kv_heads) * head_dim && context > 0, "gx: bad batch shape");
    GX_CHECK(qkv && positions && q_norm && k_norm && rope_cos && rope_sin && qh && kcache && vcache,
             "gx: missing argument");
    GX_CHECK(!slots || nslots > 0, "gx: %d slots", nslots);
    if (M == 0)
        return ok();
    if (int rc = gx::launch_qwen_qk_rope(ctx, qkv, ldqkv, M, heads, kv_heads, head_dim, positions, q_norm, k_norm,
                                         rope_cos, rope_sin, eps, qh, kcache, vcache, context, slots, nslots))
        return rc;
    return ok();
}

int gx_qwen_qkv_rope(gx_ctx *ctx, const gx_weight *w, const int8_t *q, const float *scales, const int32_t *qsum,
                     int M, int heads, int kv_heads, int head_dim, const int32_t *positions, const float *q_norm,
                     const float *k_norm, const float *rope_cos, const float *rope_sin, float eps, uint16_t *qh,
                     uint16_t *kcache, uint16_t *vcache, int context, const int32_t *slots, int nslots,
                     float *qkv) {
    if (int rc = use(ctx))
        return rc;
    GX_CHECK(w != nullptr && w->quant == GX_Q4_0 && w->count == 1, "gx: the Q|K|V product takes one Q4_0 matrix");
    GX_CHECK(heads > 0 && kv_heads > 0 && heads % kv_heads == 0, "gx: %d query heads over %d key-value heads", heads,
             kv_heads);
    GX_CHECK(head_dim > 0 && w->rows == (heads + 2 * kv_heads) * head_dim,
             "gx: %d rows are not %d query and 2 x %d key-value heads of %d", w->rows, heads, kv_heads, head_dim);
    GX_CHECK(M >= 0 && context > 0, "gx: bad batch shape");
    GX_CHECK(q && scales && qsum && positions && q_norm && k_norm && rope_cos && rope_sin && qh && kcache && vcache,
             "gx: missing argument");
    GX_CHECK(((uintptr_t)q & 15) == 0, "gx: q must be 16-byte aligned");
    GX_CHECK(!slots || nslots > 0, "gx: %d slots", nslots);
    if (M == 0)
        return ok();
    // (the epilogue stores the queries and keys 16 bytes at a time)
    const bool fused = M > 16 && (head_dim == 64 || head_dim == 128) &&
                       (((uintptr_t)rope_cos | (uintptr_t)rope_sin | (uintptr_t)qh | (uintptr_t)kcache) & 15) == 0;
    if (fused) {
        const gx::QkvRopeArgs a{positions, q_norm, k_norm, rope_cos, rope_sin, eps,  qh,
                                kcache,    vcache, context, heads, kv_heads, head_dim, slots, nslots};
        if (int rc = gx::launch_q4_0_gemm_qkv_rope(ctx, w, q, scales, M, a))
            return rc;
        return ok();
    }
    GX_CHECK(qkv != nullptr, "gx: %d positions of head width %d need the qkv buffer (the product, then the heads)", M,
             head_dim);
    if (int rc = q4_0_product(ctx, w, 0, q, scales, qsum, nullptr, M, 0, w->rows, nullptr, qkv, w->rows))
        return rc;
    if (int rc = gx::launch_qwen_qk_rope(ctx, qkv, w->rows, M, heads, kv_heads, head_dim, positions, q_norm, k_norm,
                                         rope_cos, rope_sin, eps, qh, kcache, vcache, context, slots, nslots))
        return rc;
    return ok();
}

static int rope_attention(gx_ctx *ctx, const float *qkv, int ldqkv, int M, int heads, int kv_heads, int head_dim,
                          int max_pos, const int32_t *positions, const float *q_norm, const float *k_norm,
                          const float *rope_cos, const float *rope_sin, float eps, uint16_t *kcache, uint16_t *vcache,
                          int context, int8_t *q, float *scales, int32_t *qsum, const int32_t *slots, int nslots,
                          int parallel) {
    if (int rc = use(ctx))
        return rc;
    GX_CHECK(heads > 0 && kv_heads > 0 && heads % kv_heads == 0, "gx: %d query heads over %d key-value heads", heads,
             kv_heads);
    GX_CHECK(ldqkv >= (heads + 2 * kv_heads) * head_dim && max_pos >= 0, "gx: bad batch shape");
    GX_CHECK(context % 8 == 0 && max_pos < context, "gx: a cache of %d positions (a multiple of 8) cannot hold %d",
             context, max_pos);
    GX_CHECK(qkv && positions && q_norm && k_norm && rope_cos && rope_sin && kcache && vcache && q && scales && qsum,
             "gx: missing argument");
    GX_CHECK(((uintptr_t)vcache & 15) == 0, "gx: the value cache must be 16-byte aligned");
    GX_CHECK(!slots || nslots > 0, "gx: %d slots", nslots);
    GX_CHECK(M == 1 || (M > 1 && slots), "gx: %d tokens of one conversation: the fused attention takes one token, "
             "or one token per conversation", M);
    if (M == 0)
        return ok();
    const float scale = (float)(1.0 / sqrt((double)head_dim));
    if (int rc = gx::launch_qwen_rope_attention(ctx, qkv, ldqkv, M, heads, kv_heads, head_dim, max_pos, positions, q_norm,
                                                k_norm, rope_cos, rope_sin, eps, kcache, vcache, context, scale, q,
                                                scales, qsum, slots, nslots, parallel))
        return rc;
    return ok();
}

int gx_qwen_rope_attention(gx_ctx *ctx, const float *qkv, int ldqkv, int heads, int kv_heads, int head_dim,
                           int max_pos, const int32_t *positions, const float *q_norm, const float *k_norm,
                           const float *rope_cos, const float *rope_sin, float eps, uint16_t *kcache,
                           uint16_t *vcache, int context, int8_t *q, float *scales, int32_t *qsum,
                           const int32_t *slots, int nslots) {
    return rope_attention(ctx, qkv, ldqkv, 1, heads, kv_heads, head_dim, max_pos, positions, q_norm, k_norm, rope_cos,
                          rope_sin, eps, kcache, vcache, context, q, scales, qsum, slots, nslots, 0);
}

int gx_qwen_rope_attention_parallel(gx_ctx *ctx, const float *qkv, int ldqkv, int heads, int kv_heads,
                                    int head_dim, int max_pos, const int32_t *positions, const float *q_norm,
                                    const float *k_norm, const float *rope_cos, const float *rope_sin, float eps,
                                    uint16_t *kcache, uint16_t *vcache, int context, int8_t *q, float *scales,
                                    int32_t *qsum, const int32_t *slots, int nslots) {
    return rope_attention(ctx, qkv, ldqkv, 1, heads, kv_heads, head_dim, max_pos, positions, q_norm, k_norm, rope_cos,
                          rope_sin, eps, kcache, vcache, context, q, scales, qsum, slots, nslots, 1);
}

int gx_qwen_rope_attention_slots(gx_ctx *ctx, const float *qkv, int ldqkv, int M, int heads, int kv_heads,
                                 int head_dim, int max_pos, const int32_t *positions, const float *q_norm,
                                 const float *k_norm, const float *rope_cos, const float *rope_sin, float eps,
                                 uint16_t *kcache, uint16_t *vcache, int context, int8_t *q, float *scales,
                                 int32_t *qsum, const int32_t *slots, int nslots, int parallel) {
    GX_CHECK(slots != nullptr, "gx: the fused attention of several tokens needs their conversations (slots)");
    GX_CHECK(M >= 0, "gx: bad batch shape");
    return rope_attention(ctx, qkv, ldqkv, M, heads, kv_heads, head_dim, max_pos, positions, q_norm, k_norm, rope_cos,
                          rope_sin, eps, kcache, vcache, context, q, scales, qsum, slots, nslots, parallel ? 1 : 0);
}

int gx_qwen_attention_workspace_bytes(int M, int heads, int max_pos, size_t *bytes) {
    GX_CHECK(M >= 0 && heads > 0 && max_pos >= 0 && bytes, "gx: bad attention shape");
    *bytes = gx::qwen_attention_workspace(M, heads, max_pos);
    return ok();
}

static int attention(gx_ctx *ctx, const uint16_t *qh, int M, int heads, int kv_heads, int head_dim, int max_pos,
                     const int32_t *positions, const uint16_t *kcache, const uint16_t *vcache, int context, int8_t *q,
                     float *scales, int32_t *qsum, void *workspace, size_t workspace_bytes, const int32_t *slots,
                     int nslots, int parallel) {
    if (int rc = use(ctx))
        return rc;
    GX_CHECK(heads > 0 && kv_heads > 0 && heads % kv_heads == 0, "gx: %d query heads over %d key-value heads", heads,
             kv_heads);
    GX_CHECK(M >= 0 && max_pos >= 0, "gx: bad batch shape");
    GX_CHECK(context % 8 == 0 && max_pos < context, "gx: a cache of %d positions (a multiple of 8) cannot hold %d",
             context, max_pos);
    GX_CHECK(qh && positions && kcache && vcache && q && scales && qsum && workspace, "gx: missing argument");
    GX_CHECK(((uintptr_t)vcache & 15) == 0, "gx: the value cache must be 16-byte aligned");
    GX_CHECK(((uintptr_t)workspace & 255) == 0, "gx: the workspace must be 256-byte aligned");
    GX_CHECK(!slots || nslots > 0, "gx: %d slots", nslots);
    if (M == 0)
        return ok();
    const size_t need = gx::qwen_attention_workspace(M, heads, max_pos);
    GX_CHECK(workspace_bytes >= need, "gx: the workspace holds %zu bytes, %zu needed", workspace_bytes, need);
    // llama.cpp's 1/sqrt(head_dim), taken in float64 and rounded (qwen/attention.go:90-93)
    const float scale = (float)(1.0 / sqrt((double)head_dim));
    if (int rc = gx::launch_qwen_attention(ctx, qh, M, heads, kv_heads, head_dim, max_pos, positions, kcache, vcache,
                                           context, scale, q, scales, qsum, (uint8_t *)workspace, slots,
                                           nslots, parallel, nullptr))
        return rc;
    return ok();
}

int gx_qwen_attention(gx_ctx *ctx, const uint16_t *qh, int M, int heads, int kv_heads, int head_dim, int max_pos,
                      const int32_t *positions, const uint16_t *kcache, const uint16_t *vcache, int context,
                      int8_t *q, float *scales, int32_t *qsum, void *workspace, size_t workspace_bytes,
                      const int32_t *slots, int nslots) {
    return attention(ctx, qh, M, heads, kv_heads, head_dim, max_pos, positions, kcache, vcache, context, q, scales,
                     qsum, workspace, workspace_bytes, slots, nslots, 0);
}

int gx_qwen_attention_heads(gx_ctx *ctx, const uint16_t *qh, int M, int heads, int kv_heads, int head_dim,
                            int max_pos, const int32_t *positions, const uint16_t *kcache, const uint16_t *vcache,
                            int context, float *out) {
    if (int rc = use(ctx))
        return rc;
    GX_CHECK(heads > 0 && kv_heads > 0 && heads % kv_heads == 0, "gx: %d query heads over %d key-value heads", heads,
             kv_heads);
    GX_CHECK(M > 0 && max_pos >= 0 && max_pos < (M <= 4 ? 768 : 1024),
             "gx: the head outputs are for a decode step (M <= 4, prefixes to 768) or a prompt (prefixes to 1024)");
    GX_CHECK(head_dim == 32 || head_dim == 64 || head_dim == 96 || head_dim == 128,
             "gx: attention supports head widths 32, 64, 96 and 128");
    GX_CHECK(context % 8 == 0 && max_pos < context, "gx: a cache of %d positions (a multiple of 8) cannot hold %d",
             context, max_pos);
    GX_CHECK(qh && positions && kcache && vcache && out, "gx: missing argument");
    GX_CHECK(((uintptr_t)vcache & 15) == 0, "gx: the value cache must be 16-byte aligned");
    const float scale = (float)(1.0 / sqrt((double)head_dim));
    if (int rc = gx::launch_qwen_attention(ctx, qh, M, heads, kv_heads, head_dim, max_pos, positions, kcache, vcache,
                                           context, scale, nullptr, nullptr, nullptr, nullptr, nullptr, 0, 1, out))
        return rc;
    return ok();
}

int gx_qwen_attention_parallel(gx_ctx *ctx, const uint16_t *qh, int M, int heads, int kv_heads, int head_dim,
                               int max_pos, const int32_t *positions, const uint16_t *kcache,
                               const uint16_t *vcache, int context, int8_t *q, float *scales, int32_t *qsum,
                               void *workspace, size_t workspace_bytes, const int32_t *slots, int nslots) {
    return attention(ctx, qh, M, heads, kv_heads, head_dim, max_pos, positions, kcache, vcache, context, q, scales,
                     qsum, workspace, workspace_bytes, slots, nslots, 1);
}

int gx_swiglu_quant(gx_ctx *ctx, const float *gu, int ldgu, int M, int ffn, int group, int8_t *q, float *scales,
                    int32_t *qsum) {
    if (int rc = use(ctx))
        return rc;
    GX_CHECK(ffn > 0 && ffn % 32 == 0, "nn: activation length must be a multiple of the block size");
    GX_CHECK(M >= 0 && ldgu >= 2 * ffn, "gx: bad batch shape");
    GX_CHECK(group == 0 || group == 32, "gx: gate and up come in halves (0) or by 32 (32), not by %d", group);
    GX_CHECK(gu && q && scales && qsum, "gx: missing argument");
    if (M == 0)
        return ok();
    if (int rc = gx::launch_qwen_swiglu_quant(ctx, gu, ldgu, M, ffn, group, q, scales, qsum))
        return rc;
    return ok();
}

int gx_geglu_quant(gx_ctx *ctx, const float *gu, int ldgu, int M, int ffn, int8_t *q, float *scales,
                   int32_t *qsum) {
    if (int rc = use(ctx))
        return rc;
    GX_CHECK(ffn > 0 && ffn % 32 == 0, "nn: activation length must be a multiple of the block size");
    GX_CHECK(M >= 0 && ldgu >= 2 * ffn, "gx: bad batch shape");
    GX_CHECK(gu && q && scales && qsum, "gx: missing argument");
    if (int rc = gx::launch_geglu_quant(ctx, gu, ldgu, M, ffn, q, scales, qsum))
        return rc;
    return ok();
}

int gx_moe_join(gx_ctx *ctx, float *shared, int lds, float *experts, int lde, const float *resid, int ldr,
                const float *post1, const float *post2, const float *post, int M, int K, float eps, float *out,
                int ldo) {
    if (int rc = use(ctx))
        return rc;
    GX_CHECK(K > 0 && M >= 0 && lds >= K && lde >= K && ldr >= K && ldo >= K, "gx: bad shape");
    GX_CHECK(shared && experts && resid && post1 && post2 && post && out, "gx: missing argument");
    GX_CHECK(shared != experts, "gx: the two branches must be separate buffers");
    if (int rc = gx::launch_moe_join(ctx, shared, lds, experts, lde, resid, ldr, post1, post2, post, M, K, eps, out,
                                     ldo))
        return rc;
    return ok();
}

int gx_argmax(gx_ctx *ctx, const float *x, int ldx, int M, int n, int32_t *ids) {
    if (int rc = use(ctx))
        return rc;
    GX_CHECK(M >= 0 && n > 0 && ldx >= n, "gx: bad shape");
    GX_CHECK(x && ids, "gx: missing argument");
    if (M == 0)
        return ok();
    if (int rc = gx::launch_argmax(ctx, x, ldx, M, n, ids, nullptr, 0, nullptr, nullptr))
        return rc;
    return ok();
}

int gx_argmax_step(gx_ctx *ctx, const float *x, int n, int32_t *ids, int32_t *history, int history_len,
                   int32_t *pos, int32_t *positions) {
    if (int rc = use(ctx))
        return rc;
    GX_CHECK(n > 0 && history_len > 0, "gx: bad shape");
    GX_CHECK(x && ids && history && pos && positions, "gx: missing argument");
    if (int rc = gx::launch_argmax(ctx, x, n, 1, n, ids, history, history_len, pos, positions))
        return rc;
    return ok();
}

int gx_argmax_slots_step(gx_ctx *ctx, const float *x, int ldx, int M, int n, int32_t *ids, int32_t *tokens,
                         int32_t *positions) {
    if (int rc = use(ctx))
        return rc;
    GX_CHECK(M >= 0 && n > 0 && ldx >= n, "gx: bad shape");
    GX_CHECK(x && ids && tokens && positions, "gx: missing argument");
    if (M == 0)
        return ok();
    if (int rc = gx::launch_argmax(ctx, x, ldx, M, n, ids, nullptr, 0, nullptr, nullptr, tokens, positions))
        return rc;
    return ok();
}

static int moe_experts(gx_ctx *ctx, const gx_weight *gate_up, const gx_weight *down, const float *down_scale,
                       const float *x, int ldx, int M, int top_k, const int32_t *ids, const float *weights, float *out,
                       int ldo, void *workspace, size_t workspace_bytes, bool noalloc) {
    if (int rc = use(ctx))
        return rc;
    GX_CHECK(gate_up && down && gate_up->quant == down->quant &&
                 (gate_up->quant == GX_Q4_0 || gate_up->quant == GX_F32),
             "gx: the expert stacks are Q4_0 matrices or F32 matrices, both the same");
    GX_CHECK(gate_up->count == down->count, "gx: %d gate_up experts but %d down experts", gate_up->count, down->count);
    GX_CHECK(gate_up->rows == 2 * down->cols && down->rows == gate_up->cols,
             "gx: gate_up is %dx%d and down %dx%d: want 2F x D and D x F", gate_up->rows, gate_up->cols, down->rows,
             down->cols);
    GX_CHECK(top_k > 0 && top_k <= gate_up->count, "gx: top_k %d out of range", top_k);
    GX_CHECK(M >= 0 && ldx >= gate_up->cols && ldo >= gate_up->cols, "gx: bad batch shape");
    GX_CHECK(x && ids && weights && out && workspace, "gx: missing argument");
    GX_CHECK(((uintptr_t)workspace & 255) == 0, "gx: the workspace must be 256-byte aligned");
    size_t need = 0;
    gx::moe_workspace_bytes(M, top_k, gate_up->cols, down->cols, gate_up->count, &need);
    if (noalloc)
        GX_CHECK(need <= workspace_bytes,
                 "gx: %d positions of %d experts need %zu bytes of scratch; gx_moe_experts_noalloc holds %zu (use "
                 "gx_moe_experts with a workspace, or fewer positions a call)",
                 M, top_k, need, workspace_bytes);
    GX_CHECK(workspace_bytes >= need, "gx: the workspace holds %zu bytes, %zu needed", workspace_bytes, need);
    if (M == 0)
        return ok();
    if (int rc = gx::launch_moe_experts(ctx, gate_up, down, down_scale, x, ldx, M, top_k, ids, weights, out, ldo,
                                        (uint8_t *)workspace, ctx->gelu_table))
        return rc;
    return ok();
}

int gx_moe_experts(gx_ctx *ctx, const gx_weight *gate_up, const gx_weight *down, const float *down_scale,
                   const float *x, int ldx, int M, int top_k, const int32_t *ids, const float *weights, float *out,
                   int ldo, void *workspace, size_t workspace_bytes) {
    return moe_experts(ctx, gate_up, down, down_scale, x, ldx, M, top_k, ids, weights, out, ldo, workspace,
                       workspace_bytes, false);
}

int gx_moe_experts_noalloc(gx_ctx *ctx, const gx_weight *gate_up, const gx_weight *down, const float *down_scale,
                           const float *x, int ldx, int M, int top_k, const int32_t *ids, const float *weights,
                           float *out, int ldo) {
    if (int rc = use(ctx))
        return rc;
    // the scratch's address on this device (from gx_init), never the symbol
    return moe_experts(ctx, gate_up, down, down_scale, x, ldx, M, top_k, ids, weights, out, ldo, ctx->scratch,
                       kScratchBytes, true);
}

}  // extern "C"
