// gx_calib.hip - calibration kernels for the measurements beside the
// products: no counterpart in golem, and no product calls them.
//
//   calib_empty_kernel   does nothing: the per-dispatch floor of a launch of
//                        a given grid, in a stream or a replayed graph.
//   calib_read_kernel    a plain streaming read of `bytes` with 16-byte
//                        non-temporal loads (as the products read weights),
//                        each workgroup a contiguous share: what moving a
//                        product's bytes alone costs at its grid.
//   calib_valu_kernel    independent chains of v_fmac_f32 (no memory): the
//                        VALU issue rate the SQ counters report at
//                        saturation, to read SQ_ACTIVE_INST_VALU and
//                        SQ_INSTS_VALU of the products against.
#include "gx_device.hpp"
#include "gx_internal.hpp"

namespace gx {
namespace {

__global__ __launch_bounds__(64) void calib_empty_kernel() {}

// grid: workgroups of 512 threads; workgroup b reads chunks b, b + grid, ...
// of 16 bytes per thread, XORs them, and writes one word (so the loads stay).
__global__ __launch_bounds__(512) void calib_read_kernel(const uint8_t *__restrict__ src, size_t chunks,
                                                         uint32_t *__restrict__ sink) {
    const size_t per = (chunks + gridDim.x - 1) / gridDim.x;  // 16-byte chunks a workgroup
    const size_t c0 = (size_t)blockIdx.x * per, c1 = min(c0 + per, chunks);
    uint32_t acc = 0;
#pragma unroll 16
    for (size_t c = c0 + threadIdx.x; c < c1; c += blockDim.x) {
        const uint4 v = load_stream(src + c * 16);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9E3779B9u)  // (practically never) keeps the loads
        sink[blockIdx.x] = acc;
}

// Eight independent fma chains a lane, `iters` steps each: 8 * iters
// v_fmac_f32 per lane, no loads.
__global__ __launch_bounds__(256) void calib_valu_kernel(int iters, float *__restrict__ sink) {
    float a[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
        a[i] = (float)(threadIdx.x + i);
    const float m = 1.0000001f, c = 1e-7f;
    for (int k = 0; k < iters; k++) {
#pragma unroll
        for (int i = 0; i < 8; i++)
            a[i] = __builtin_fmaf(a[i], m, c);
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++)
        s += a[i];
    if (s == 1234.5f)
        sink[blockIdx.x] = s;
}

}  // namespace
}  // namespace gx

extern "C" {

int gx_calib_empty(gx_ctx *ctx, int workgroups) {
    GX_CHECK(ctx && workgroups > 0, "gx: calibration needs a context and a grid");
    gx::calib_empty_kernel<<<workgroups, 64, 0, ctx->stream>>>();
    return gx::check_launch("calib_empty");
}

int gx_calib_read(gx_ctx *ctx, const void *src, size_t bytes, int workgroups, uint32_t *sink) {
    GX_CHECK(ctx && src && sink && workgroups > 0, "gx: calibration needs a context, a buffer, a sink and a grid");
    GX_CHECK(((uintptr_t)src & 15) == 0 && bytes % 16 == 0, "gx: the read takes whole 16-byte chunks");
    gx::calib_read_kernel<<<workgroups, 512, 0, ctx->stream>>>((const uint8_t *)src, bytes / 16, sink);
    return gx::check_launch("calib_read");
}

int gx_calib_valu(gx_ctx *ctx, int workgroups, int iters, float *sink) {
    GX_CHECK(ctx && sink && workgroups > 0 && iters > 0, "gx: calibration needs a context, a sink and a grid");
    gx::calib_valu_kernel<<<workgroups, 256, 0, ctx->stream>>>(iters, sink);
    return gx::check_launch("calib_valu");
}

}  // extern "C"
