// Runtime half of the boundary: context, device memory, copies, timing, the
// host Q2_0 codec, the GGUF <-> device-plane repack and the synthetic-data
// generators.  Replaces MetalContext (LLM/src/Metal/MetalContext.swift).
#include "gd_internal.h"

#include <stdarg.h>
#include <string.h>
#include <mutex>

static std::mutex g_err_mu;
static std::string g_err;   // last gd_ctx_create failure (no context yet)

int gd_fail(gd_ctx *ctx, int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (ctx) {
        ctx->err = buf;
    } else {
        std::lock_guard<std::mutex> lk(g_err_mu);
        g_err = buf;
    }
    return code;
}

int gd_hip_fail(gd_ctx *ctx, hipError_t e, const char *what) {
    int code = GD_EHIP;
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) code = GD_ENOMEM;
    if (e == hipErrorNoDevice || e == hipErrorInvalidDevice) code = GD_ENODEV;
    return gd_fail(ctx, code, "%s: %s", what, hipGetErrorString(e));
}

extern "C" int gd_device_count(int *n) {
    if (!n) return GD_EINVAL;
    int c = 0;
    if (hipGetDeviceCount(&c) != hipSuccess) c = 0;
    *n = c;
    return GD_OK;
}

extern "C" int gd_ctx_create(int device, gd_ctx **out) {
    if (!out) return GD_EINVAL;
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0)
        return gd_fail(nullptr, GD_ENODEV, "no HIP device (%s)",
                       e == hipSuccess ? "count 0" : hipGetErrorString(e));
    if (device < 0 || device >= n)
        return gd_fail(nullptr, GD_ENODEV, "device %d out of range [0,%d)", device, n);
    gd_ctx *c = new gd_ctx();
    c->device = device;
    if ((e = hipSetDevice(device)) != hipSuccess ||
        (e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking)) != hipSuccess ||
        (e = hipEventCreate(&c->ev_start)) != hipSuccess ||
        (e = hipEventCreate(&c->ev_stop)) != hipSuccess) {
        gd_fail(nullptr, GD_EHIP, "context setup: %s", hipGetErrorString(e));
        gd_ctx_destroy(c);
        return GD_EHIP;
    }
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, device) == hipSuccess) c->num_cus = p.multiProcessorCount;
    // A failed lookup leaves prefill_scratch null: only gd_gdn_prefill_noalloc
    // needs it, and it reports the failure then.
    (void)gd_prefill_scratch_attach(c);
    c->err.clear();
    *out = c;
    return GD_OK;
}

extern "C" void gd_ctx_destroy(gd_ctx *ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    if (ctx->ev_start) (void)hipEventDestroy(ctx->ev_start);
    if (ctx->ev_stop) (void)hipEventDestroy(ctx->ev_stop);
    if (ctx->ws) (void)hipFree(ctx->ws);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

extern "C" const char *gd_last_error(const gd_ctx *ctx) {
    if (ctx) return ctx->err.c_str();
    std::lock_guard<std::mutex> lk(g_err_mu);
    static thread_local std::string copy;
    copy = g_err;
    return copy.c_str();
}

int gd_ctx_workspace(gd_ctx *ctx, size_t bytes, void **out) {
    if (ctx->ws_bytes < bytes) {
        if (ctx->ws) {
            GD_HIP(ctx, hipStreamSynchronize(ctx->stream));
            GD_HIP(ctx, hipFree(ctx->ws));
            ctx->ws = nullptr;
            ctx->ws_bytes = 0;
        }
        hipError_t e = hipMalloc(&ctx->ws, bytes);
        if (e != hipSuccess) {
            ctx->ws = nullptr;
            return gd_fail(ctx, GD_ENOMEM, "workspace (%zu bytes): %s", bytes, hipGetErrorString(e));
        }
        ctx->ws_bytes = bytes;
    }
    *out = ctx->ws;
    return GD_OK;
}

extern "C" int gd_alloc(gd_ctx *ctx, size_t bytes, void **dptr) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, dptr != nullptr, "gd_alloc: null out pointer");
    *dptr = nullptr;
    if (bytes == 0) bytes = 256;
    GD_HIP(ctx, hipSetDevice(ctx->device));
    hipError_t e = hipMalloc(dptr, bytes);
    if (e != hipSuccess) {
        *dptr = nullptr;
        return gd_fail(ctx, GD_ENOMEM, "gd_alloc(%zu bytes): %s", bytes, hipGetErrorString(e));
    }
    return GD_OK;
}

extern "C" int gd_free(gd_ctx *ctx, void *dptr) {
    GD_CHECK_CTX(ctx);
    if (!dptr) return GD_OK;
    // Work enqueued on the stream may still read the buffer.
    GD_HIP(ctx, hipStreamSynchronize(ctx->stream));
    GD_HIP(ctx, hipFree(dptr));
    return GD_OK;
}

extern "C" int gd_upload(gd_ctx *ctx, void *dst, const void *src, size_t bytes) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, (dst && src) || bytes == 0, "gd_upload: null pointer");
    if (!bytes) return GD_OK;
    GD_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    GD_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return GD_OK;
}

extern "C" int gd_download(gd_ctx *ctx, void *dst, const void *src, size_t bytes) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, (dst && src) || bytes == 0, "gd_download: null pointer");
    if (!bytes) return GD_OK;
    GD_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    GD_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return GD_OK;
}

extern "C" int gd_copy(gd_ctx *ctx, void *dst, const void *src, size_t bytes) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, (dst && src) || bytes == 0, "gd_copy: null pointer");
    if (!bytes) return GD_OK;
    GD_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
    return GD_OK;
}

__global__ void gd_fill_u32_kernel(uint32_t *dst, uint32_t v, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) dst[i] = v;
}

extern "C" int gd_fill_u32(gd_ctx *ctx, void *dst, uint32_t value, size_t count) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, dst || count == 0, "gd_fill_u32: null pointer");
    if (!count) return GD_OK;
    unsigned blocks = (unsigned)std::min<size_t>((count + 255) / 256, 65536);
    hipLaunchKernelGGL(gd_fill_u32_kernel, dim3(blocks), dim3(256), 0, ctx->stream,
                       (uint32_t *)dst, value, count);
    GD_LAUNCHED(ctx, "gd_fill_u32");
    return GD_OK;
}

__global__ void gd_cast_kernel(const void *src, int st, void *dst, int dt, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) {
        const float v = st == GD_F32 ? ((const float *)src)[i] : gd_h2f(((const uint16_t *)src)[i]);
        if (dt == GD_F32) ((float *)dst)[i] = v;
        else ((uint16_t *)dst)[i] = gd_f2h(v);
    }
}

extern "C" int gd_cast(gd_ctx *ctx, const void *src, int src_dtype, void *dst, int dst_dtype,
                       size_t n) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, (src && dst) || n == 0, "gd_cast: null pointer");
    GD_REQUIRE(ctx, (src_dtype == GD_F32 || src_dtype == GD_F16) &&
                        (dst_dtype == GD_F32 || dst_dtype == GD_F16),
               "gd_cast: bad dtypes %d -> %d", src_dtype, dst_dtype);
    if (!n) return GD_OK;
    unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 65536);
    hipLaunchKernelGGL(gd_cast_kernel, dim3(blocks), dim3(256), 0, ctx->stream, src, src_dtype,
                       dst, dst_dtype, n);
    GD_LAUNCHED(ctx, "gd_cast");
    return GD_OK;
}

extern "C" int gd_sync(gd_ctx *ctx) {
    GD_CHECK_CTX(ctx);
    GD_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return GD_OK;
}

extern "C" int gd_timer_start(gd_ctx *ctx) {
    GD_CHECK_CTX(ctx);
    GD_HIP(ctx, hipEventRecord(ctx->ev_start, ctx->stream));
    return GD_OK;
}

extern "C" int gd_timer_stop(gd_ctx *ctx, float *ms) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, ms != nullptr, "gd_timer_stop: null out pointer");
    GD_HIP(ctx, hipEventRecord(ctx->ev_stop, ctx->stream));
    GD_HIP(ctx, hipEventSynchronize(ctx->ev_stop));
    GD_HIP(ctx, hipEventElapsedTime(ms, ctx->ev_start, ctx->ev_stop));
    return GD_OK;
}

// ------------------------------------------------------------ graph capture

struct gd_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

extern "C" int gd_graph_begin(gd_ctx *ctx) {
    GD_CHECK_CTX(ctx);
    GD_HIP(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    return GD_OK;
}

extern "C" int gd_graph_end(gd_ctx *ctx, gd_graph **out) {
    GD_CHECK_CTX(ctx);
    if (out) *out = nullptr;
    hipGraph_t graph = nullptr;
    const hipError_t e = hipStreamEndCapture(ctx->stream, &graph);
    if (e != hipSuccess) {
        if (graph) (void)hipGraphDestroy(graph);
        return gd_hip_fail(ctx, e, "gd_graph_end: hipStreamEndCapture");
    }
    if (!out) {
        (void)hipGraphDestroy(graph);
        return gd_fail(ctx, GD_EINVAL, "gd_graph_end: null out pointer (capture discarded)");
    }
    gd_graph *g = new gd_graph();
    g->graph = graph;
    const hipError_t ei = hipGraphInstantiate(&g->exec, graph, nullptr, nullptr, 0);
    if (ei != hipSuccess) {
        (void)hipGraphDestroy(graph);
        delete g;
        return gd_hip_fail(ctx, ei, "gd_graph_end: hipGraphInstantiate");
    }
    *out = g;
    return GD_OK;
}

extern "C" int gd_graph_launch(gd_ctx *ctx, gd_graph *g) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, g && g->exec, "gd_graph_launch: null graph");
    GD_HIP(ctx, hipGraphLaunch(g->exec, ctx->stream));
    return GD_OK;
}

extern "C" void gd_graph_destroy(gd_graph *g) {
    if (!g) return;
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    delete g;
}

// ---------------------------------------------------------------- host codec

extern "C" int gd_q2_0_pack(const uint8_t *codes, const uint16_t *scales, size_t n,
                            uint8_t *blocks) {
    if (!codes || !scales || !blocks || n % GD_Q2_0_QK) return GD_EINVAL;
    const size_t nb = n / GD_Q2_0_QK;
    for (size_t b = 0; b < nb; b++) {
        uint8_t *p = blocks + b * GD_Q2_0_BLOCK_BYTES;
        const uint16_t d = scales[b];
        p[0] = (uint8_t)(d & 0xff);          // f16 scale first, little-endian
        p[1] = (uint8_t)(d >> 8);
        const uint8_t *c = codes + b * GD_Q2_0_QK;
        for (int j = 0; j < 32; j++) {
            if ((c[4 * j] | c[4 * j + 1] | c[4 * j + 2] | c[4 * j + 3]) > 3) return GD_EINVAL;
            p[2 + j] = (uint8_t)(c[4 * j] | (c[4 * j + 1] << 2) |
                                 (c[4 * j + 2] << 4) | (c[4 * j + 3] << 6));
        }
    }
    return GD_OK;
}

extern "C" int gd_q2_0_unpack(const uint8_t *blocks, size_t n, uint8_t *codes,
                              uint16_t *scales) {
    if (!blocks || n % GD_Q2_0_QK || (!codes && !scales)) return GD_EINVAL;
    const size_t nb = n / GD_Q2_0_QK;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *p = blocks + b * GD_Q2_0_BLOCK_BYTES;
        if (scales) scales[b] = (uint16_t)(p[0] | (p[1] << 8));
        if (codes) {
            uint8_t *c = codes + b * GD_Q2_0_QK;
            for (int j = 0; j < GD_Q2_0_QK; j++)
                c[j] = (uint8_t)((p[2 + (j >> 2)] >> ((j & 3) << 1)) & 3);
        }
    }
    return GD_OK;
}

// ------------------------------------------------------- device planes / repack

extern "C" int gd_q2w_alloc(gd_ctx *ctx, int64_t K, int64_t R, gd_q2w *w) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, w && K > 0 && R > 0 && K % GD_Q2_0_QK == 0,
               "gd_q2w_alloc: K=%lld must be a positive multiple of 128, R=%lld > 0",
               (long long)K, (long long)R);
    w->codes = w->scales = nullptr;
    w->K = K; w->R = R;
    const size_t cb = gd_q2_codes_bytes(K, R), sb = gd_q2_scales_count(K, R) * 2;
    int rc = gd_alloc(ctx, cb, &w->codes);
    if (rc) return rc;
    rc = gd_alloc(ctx, sb, &w->scales);
    if (rc) { gd_free(ctx, w->codes); w->codes = nullptr; return rc; }
    // Padding rows and blocks must read as zero weights.
    if ((rc = gd_fill_u32(ctx, w->codes, 0u, cb / 4)) ||
        (rc = gd_fill_u32(ctx, w->scales, 0u, sb / 4))) {
        gd_q2w_free(ctx, w);
        return rc;
    }
    return GD_OK;
}

extern "C" int gd_q2w_free(gd_ctx *ctx, gd_q2w *w) {
    GD_CHECK_CTX(ctx);
    if (!w) return GD_OK;
    int rc = gd_free(ctx, w->codes);
    int rc2 = gd_free(ctx, w->scales);
    w->codes = w->scales = nullptr;
    return rc ? rc : rc2;
}

// One thread per 34-byte GGUF block (row-major order) of rows [row0, ...).  The GGUF side is only
// 2-byte aligned, so it is read as 17 halfwords; the code dwords go, nibble-
// interleaved, to their two 16-byte slots of the row group's tile, the scale
// to its slot.
__global__ void gd_repack_kernel(const uint16_t *src, uint8_t *codes, uint16_t *scales,
                                 int64_t nblk, int64_t row0, int64_t nblocks) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const int64_t row = row0 + b / nblk, blk = b % nblk;
    const int64_t steps = (nblk + 3) / 4, bgroups = (nblk + 15) / 16;
    const uint16_t *p = src + b * (GD_Q2_0_BLOCK_BYTES / 2);
    scales[gd_q2_scale_idx(row, blk, bgroups)] = p[0];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        u32x4 v;
#pragma unroll
        for (int j = 0; j < 4; j++)
            v[j] = gd_q2_to_dev((uint32_t)p[1 + 8 * h + 2 * j] | ((uint32_t)p[2 + 8 * h + 2 * j] << 16));
        *(u32x4 *)(codes + gd_q2_code_off(row, blk, h, steps)) = v;
    }
}

// Inverse of gd_repack_kernel for rows [row0, row0 + nrows).
__global__ void gd_export_kernel(const uint8_t *codes, const uint16_t *scales, uint16_t *dst,
                                 int64_t nblk, int64_t row0, int64_t nblocks) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const int64_t row = row0 + b / nblk, blk = b % nblk;
    const int64_t steps = (nblk + 3) / 4, bgroups = (nblk + 15) / 16;
    uint16_t *p = dst + b * (GD_Q2_0_BLOCK_BYTES / 2);
    p[0] = scales[gd_q2_scale_idx(row, blk, bgroups)];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const u32x4 v = *(const u32x4 *)(codes + gd_q2_code_off(row, blk, h, steps));
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t g = gd_q2_from_dev(v[j]);
            p[1 + 8 * h + 2 * j] = (uint16_t)(g & 0xffff);
            p[2 + 8 * h + 2 * j] = (uint16_t)(g >> 16);
        }
    }
}

static int check_q2w(gd_ctx *ctx, const gd_q2w *w, const char *who) {
    GD_REQUIRE(ctx, w && w->codes && w->scales, "%s: null weight planes", who);
    GD_REQUIRE(ctx, w->K > 0 && w->K % GD_Q2_0_QK == 0 && w->R > 0,
               "%s: K=%lld must be a positive multiple of 128, R=%lld > 0", who,
               (long long)w->K, (long long)w->R);
    GD_REQUIRE(ctx, ((uintptr_t)w->codes & 255) == 0 && ((uintptr_t)w->scales & 7) == 0,
               "%s: codes plane must be 256-byte aligned, scales 8-byte aligned", who);
    return GD_OK;
}
int gd_check_q2w(gd_ctx *ctx, const gd_q2w *w, const char *who) { return check_q2w(ctx, w, who); }

extern "C" int gd_q2_0_repack_rows(gd_ctx *ctx, const void *gguf, uint64_t woff, int64_t row0,
                                   int64_t nrows, gd_q2w *w) {
    GD_CHECK_CTX(ctx);
    int rc = check_q2w(ctx, w, "gd_q2_0_repack_rows");
    if (rc) return rc;
    GD_REQUIRE(ctx, gguf && woff % 2 == 0, "gd_q2_0_repack_rows: null source or odd offset");
    GD_REQUIRE(ctx, row0 >= 0 && nrows >= 0 && row0 + nrows <= w->R,
               "gd_q2_0_repack_rows: rows [%lld, %lld) outside [0, %lld)", (long long)row0,
               (long long)(row0 + nrows), (long long)w->R);
    const int64_t nblk = w->K / GD_Q2_0_QK, nb = nrows * nblk;
    if (!nb) return GD_OK;
    hipLaunchKernelGGL(gd_repack_kernel, dim3(gd_blocks(nb, 256)), dim3(256), 0, ctx->stream,
                       (const uint16_t *)((const uint8_t *)gguf + woff), (uint8_t *)w->codes,
                       (uint16_t *)w->scales, nblk, row0, nb);
    GD_LAUNCHED(ctx, "gd_repack_kernel");
    return GD_OK;
}

extern "C" int gd_q2_0_repack(gd_ctx *ctx, const void *gguf, uint64_t woff, gd_q2w *w) {
    GD_CHECK_CTX(ctx);
    int rc = check_q2w(ctx, w, "gd_q2_0_repack");
    if (rc) return rc;
    return gd_q2_0_repack_rows(ctx, gguf, woff, 0, w->R, w);
}

extern "C" int gd_q2_0_export_rows(gd_ctx *ctx, const gd_q2w *w, int64_t row0, int64_t nrows,
                                   void *gguf_out) {
    GD_CHECK_CTX(ctx);
    int rc = check_q2w(ctx, w, "gd_q2_0_export_rows");
    if (rc) return rc;
    GD_REQUIRE(ctx, gguf_out && ((uintptr_t)gguf_out & 1) == 0, "gd_q2_0_export_rows: bad output");
    GD_REQUIRE(ctx, row0 >= 0 && nrows >= 0 && row0 + nrows <= w->R,
               "gd_q2_0_export_rows: rows [%lld, %lld) outside [0, %lld)", (long long)row0,
               (long long)(row0 + nrows), (long long)w->R);
    const int64_t nblk = w->K / GD_Q2_0_QK, nb = nrows * nblk;
    if (!nb) return GD_OK;
    hipLaunchKernelGGL(gd_export_kernel, dim3(gd_blocks(nb, 256)), dim3(256), 0, ctx->stream,
                       (const uint8_t *)w->codes, (const uint16_t *)w->scales,
                       (uint16_t *)gguf_out, nblk, row0, nb);
    GD_LAUNCHED(ctx, "gd_export_kernel");
    return GD_OK;
}

extern "C" int gd_q2_0_export(gd_ctx *ctx, const gd_q2w *w, void *gguf_out) {
    GD_CHECK_CTX(ctx);
    int rc = check_q2w(ctx, w, "gd_q2_0_export");
    if (rc) return rc;
    return gd_q2_0_export_rows(ctx, w, 0, w->R, gguf_out);
}

extern "C" int gd_q2_0_upload(gd_ctx *ctx, const void *host_blocks, int64_t K, int64_t R,
                              gd_q2w *w) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, host_blocks && w, "gd_q2_0_upload: null pointer");
    int rc = gd_q2w_alloc(ctx, K, R, w);
    if (rc) return rc;
    const size_t bytes = (size_t)(R * (K / GD_Q2_0_QK) * GD_Q2_0_BLOCK_BYTES);
    void *staging = nullptr;
    if ((rc = gd_alloc(ctx, bytes, &staging)) ||
        (rc = gd_upload(ctx, staging, host_blocks, bytes)) ||
        (rc = gd_q2_0_repack(ctx, staging, 0, w)) ||
        (rc = gd_free(ctx, staging))) {
        gd_free(ctx, staging);
        gd_q2w_free(ctx, w);
        return rc;
    }
    return GD_OK;
}

// ------------------------------------------------------------ synthetic data

#define GD_RAND_RUN 64   // consecutive stream elements per thread

__device__ __forceinline__ uint32_t lcg_bits(uint64_t s) { return (uint32_t)(s >> 33); }

// lo + span*u with two roundings (no FMA contraction), as the host stream.
__device__ __forceinline__ float lerp_unfused(float lo, float span, float u) {
#pragma clang fp contract(off)
    return lo + span * u;
}

__global__ void gd_rand_uniform_kernel(float *out, size_t n, uint64_t s0, float lo, float span) {
    const size_t i0 = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * GD_RAND_RUN;
    if (i0 >= n) return;
    uint64_t s = gd_lcg_skip(s0, i0);
    const size_t end = i0 + GD_RAND_RUN < n ? i0 + GD_RAND_RUN : n;
    for (size_t i = i0; i < end; i++) {
        s = s * GD_LCG_A + GD_LCG_C;
        const float u = (float)lcg_bits(s) * 0x1p-31f;
        out[i] = lerp_unfused(lo, span, u);
    }
}

__global__ void gd_rand_normal_kernel(void *out, int dtype, size_t n, uint64_t s0, float mean,
                                      float sd) {
    // Each thread owns GD_RAND_RUN/2 Box-Muller pairs: elements [i0, i0+RUN).
    const size_t i0 = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * GD_RAND_RUN;
    if (i0 >= n) return;
    uint64_t s = gd_lcg_skip(s0, i0);
    for (size_t i = i0; i < i0 + GD_RAND_RUN && i < n; i += 2) {
        s = s * GD_LCG_A + GD_LCG_C;
        const uint32_t b1 = lcg_bits(s);
        s = s * GD_LCG_A + GD_LCG_C;
        const uint32_t b2 = lcg_bits(s);
        const float u1 = (float)((uint64_t)b1 + 1) * 0x1p-31f;   // (0, 1]
        const float u2 = (float)b2 * 0x1p-31f;                   // [0, 1)
        const float r = sqrtf(-2.0f * logf(u1));
        const float a = 6.283185307179586f * u2;
        const float z0 = mean + sd * (r * cosf(a));
        const float z1 = mean + sd * (r * sinf(a));
        if (dtype == GD_F32) {
            ((float *)out)[i] = z0;
            if (i + 1 < n) ((float *)out)[i + 1] = z1;
        } else {
            ((uint16_t *)out)[i] = gd_f2h(z0);
            if (i + 1 < n) ((uint16_t *)out)[i + 1] = gd_f2h(z1);
        }
    }
}

// Codes: one thread per 64 weights (16 code bytes, half a block) of the
// flattened [R][K] matrix; weight e uses element e of stream s0.
__global__ void gd_rand_codes_kernel(uint8_t *codes, int64_t K, size_t nweights, uint64_t s0) {
    const size_t e0 = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 64;
    if (e0 >= nweights) return;
    uint64_t s = gd_lcg_skip(s0, e0);
    const int64_t row = (int64_t)(e0 / (size_t)K), k0 = (int64_t)(e0 % (size_t)K);
    u32x4 v;
#pragma unroll
    for (int w = 0; w < 4; w++) {
        uint32_t word = 0;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            s = s * GD_LCG_A + GD_LCG_C;
            const uint32_t c = (uint32_t)(((uint64_t)lcg_bits(s) * 3u) >> 31);
            word |= c << gd_q2_bitpos(j);
        }
        v[w] = word;
    }
    *(u32x4 *)(codes + gd_q2_code_off(row, k0 >> 7, (int)((k0 >> 6) & 1), gd_q2_steps(K))) = v;
}

// Scales: element i of the stream is block i of the flattened [R][K/128] grid.
__global__ void gd_rand_scales_kernel(uint16_t *scales, int64_t nblk, size_t n, uint64_t s0,
                                      float lo, float span) {
    const size_t i0 = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * GD_RAND_RUN;
    if (i0 >= n) return;
    uint64_t s = gd_lcg_skip(s0, i0);
    const int64_t bgroups = (nblk + 15) / 16;
    for (size_t i = i0; i < i0 + GD_RAND_RUN && i < n; i++) {
        s = s * GD_LCG_A + GD_LCG_C;
        const float u = (float)lcg_bits(s) * 0x1p-31f;
        const int64_t row = (int64_t)(i / (size_t)nblk), blk = (int64_t)(i % (size_t)nblk);
        scales[gd_q2_scale_idx(row, blk, bgroups)] = gd_f2h(lerp_unfused(lo, span, u));
    }
}

static inline uint64_t stream_start(uint64_t seed) { return seed + GD_LCG_SEED_MIX; }

extern "C" int gd_rand_uniform(gd_ctx *ctx, float *out, size_t n, uint64_t seed, float lo,
                               float hi) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, out || n == 0, "gd_rand_uniform: null output");
    if (!n) return GD_OK;
    const size_t threads = (n + GD_RAND_RUN - 1) / GD_RAND_RUN;
    hipLaunchKernelGGL(gd_rand_uniform_kernel, dim3(gd_blocks(threads, 256)), dim3(256), 0,
                       ctx->stream, out, n, stream_start(seed), lo, hi - lo);
    GD_LAUNCHED(ctx, "gd_rand_uniform");
    return GD_OK;
}

extern "C" int gd_rand_normal(gd_ctx *ctx, void *out, int dtype, size_t n, uint64_t seed,
                              float mean, float sd) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, out || n == 0, "gd_rand_normal: null output");
    GD_REQUIRE(ctx, dtype == GD_F32 || dtype == GD_F16, "gd_rand_normal: bad dtype %d", dtype);
    if (!n) return GD_OK;
    const size_t threads = (n + GD_RAND_RUN - 1) / GD_RAND_RUN;
    hipLaunchKernelGGL(gd_rand_normal_kernel, dim3(gd_blocks(threads, 256)), dim3(256), 0,
                       ctx->stream, out, dtype, n, stream_start(seed), mean, sd);
    GD_LAUNCHED(ctx, "gd_rand_normal");
    return GD_OK;
}

extern "C" int gd_rand_q2w(gd_ctx *ctx, gd_q2w *w, uint64_t seed, float lo, float hi) {
    GD_CHECK_CTX(ctx);
    int rc = check_q2w(ctx, w, "gd_rand_q2w");
    if (rc) return rc;
    const size_t nw = (size_t)(w->R * w->K);       // multiple of 128
    hipLaunchKernelGGL(gd_rand_codes_kernel, dim3(gd_blocks(nw / 64, 256)), dim3(256), 0,
                       ctx->stream, (uint8_t *)w->codes, w->K, nw, stream_start(seed));
    GD_LAUNCHED(ctx, "gd_rand_codes");
    const size_t ns = nw / GD_Q2_0_QK;
    const size_t threads = (ns + GD_RAND_RUN - 1) / GD_RAND_RUN;
    hipLaunchKernelGGL(gd_rand_scales_kernel, dim3(gd_blocks(threads, 256)), dim3(256), 0,
                       ctx->stream, (uint16_t *)w->scales, w->K / GD_Q2_0_QK, ns,
                       stream_start(seed + 1), lo, hi - lo);
    GD_LAUNCHED(ctx, "gd_rand_scales");
    return GD_OK;
}
