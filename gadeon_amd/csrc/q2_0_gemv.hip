// Q2_0 GEMV entry point and row dequant.
//
// Reference: q2_0_gemv (LLM/metal/Kernels.metal:30-119) and the CPU oracle
// Q2_0.matvec (LLM/src/SIMD/Quant.swift:36-77), both computing per block
// d * (sum over codes of code*x - sum x) = d * sum((code-1)*x) in f32.  The
// kernel itself runs on the matrix cores (q2_0_gemv_mfma.hip); this file
// checks arguments and holds the row dequant used for token embeddings
// (MetalEnc.dequantRow / embedBatch).
#include "gd_internal.h"

namespace {

// out[n][k] = (code-1)*d of row ids[n], one thread per 16 weights (one code
// dword).  Exact: an f16 times -1/0/1/2.
__global__ void q2_0_dequant_rows_kernel(const uint8_t *__restrict__ codes,
                                         const uint16_t *__restrict__ scales,
                                         const int32_t *__restrict__ ids, float *__restrict__ out,
                                         int K, int R, int64_t n) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;   // dword index
    const int dpr = K >> 4;                                              // dwords per row
    if (e >= n * dpr) return;
    const int64_t tok = e / dpr;
    const int w = (int)(e % dpr);
    const int row = ids[tok];
    f32x4 *dst = (f32x4 *)(out + tok * K + 16 * w);
    if (row < 0 || row >= R) {                     // out-of-vocabulary id -> zeros
#pragma unroll
        for (int i = 0; i < 4; i++) dst[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        return;
    }
    const int blk = w >> 3, h = (w >> 2) & 1;       // 8 dwords per block, 4 per half
    const uint32_t word = *(const uint32_t *)(codes + gd_q2_code_off(row, blk, h, gd_q2_steps(K)) +
                                              4 * (w & 3));
    const float d = gd_h2f(scales[gd_q2_scale_idx(row, blk, gd_q2_bgroups(K))]);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        f32x4 v;
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] = (float)((int)((word >> gd_q2_bitpos(4 * i + j)) & 3u) - 1) * d;
        dst[i] = v;
    }
}

}  // namespace

int gd_check_q2w(gd_ctx *ctx, const gd_q2w *w, const char *who);

extern "C" int gd_q2_0_dequant_rows(gd_ctx *ctx, const gd_q2w *w, const int32_t *ids, int64_t n,
                                    float *out) {
    GD_CHECK_CTX(ctx);
    int rc = gd_check_q2w(ctx, w, "gd_q2_0_dequant_rows");
    if (rc) return rc;
    GD_REQUIRE(ctx, ids && out && n >= 0, "gd_q2_0_dequant_rows: bad arguments");
    GD_REQUIRE(ctx, ((uintptr_t)out & 15) == 0, "gd_q2_0_dequant_rows: out must be 16-byte aligned");
    GD_REQUIRE(ctx, w->K <= (1 << 24) && w->R < (1LL << 31), "gd_q2_0_dequant_rows: too large");
    if (!n) return GD_OK;
    const int64_t total = n * (w->K >> 4);
    hipLaunchKernelGGL(q2_0_dequant_rows_kernel, dim3(gd_blocks(total, 256)), dim3(256), 0,
                       ctx->stream, (const uint8_t *)w->codes, (const uint16_t *)w->scales, ids,
                       out, (int)w->K, (int)w->R, n);
    GD_LAUNCHED(ctx, "q2_0_dequant_rows");
    return GD_OK;
}

extern "C" int gd_q2_0_gemv(gd_ctx *ctx, const gd_q2w *w, const void *x, int x_dtype,
                            float *y) {
    GD_CHECK_CTX(ctx);
    int rc = gd_check_q2w(ctx, w, "gd_q2_0_gemv");
    if (rc) return rc;
    GD_REQUIRE(ctx, x && y, "gd_q2_0_gemv: null x or y");
    GD_REQUIRE(ctx, x_dtype == GD_F32 || x_dtype == GD_F16, "gd_q2_0_gemv: bad x dtype %d",
               x_dtype);
    GD_REQUIRE(ctx, ((uintptr_t)x & 15) == 0, "gd_q2_0_gemv: x must be 16-byte aligned");
    GD_REQUIRE(ctx, w->K <= 65536 && w->R < (1LL << 30),
               "gd_q2_0_gemv: K=%lld (at most 65536) or R=%lld too large", (long long)w->K,
               (long long)w->R);
    return gd_gemv_mfma(ctx, w, x, x_dtype, y, 1);
}

extern "C" int gd_q2_0_gemv_split(gd_ctx *ctx, const gd_q2w *w, const void *x, int x_dtype,
                                  float *y, int ksplit, int *nsplit) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, ksplit >= 1 && ksplit <= 4 && nsplit, "gd_q2_0_gemv_split: ksplit %d not 1..4",
               ksplit);
    int rc = gd_check_q2w(ctx, w, "gd_q2_0_gemv_split");
    if (rc) return rc;
    GD_REQUIRE(ctx, x && y, "gd_q2_0_gemv_split: null x or y");
    GD_REQUIRE(ctx, x_dtype == GD_F32 || x_dtype == GD_F16, "gd_q2_0_gemv_split: bad x dtype %d",
               x_dtype);
    GD_REQUIRE(ctx, ((uintptr_t)x & 15) == 0, "gd_q2_0_gemv_split: x must be 16-byte aligned");
    GD_REQUIRE(ctx, w->K <= 65536 && w->R < (1LL << 30),
               "gd_q2_0_gemv_split: K=%lld (at most 65536) or R=%lld too large", (long long)w->K,
               (long long)w->R);
    const int steps = (int)((w->K / 128 + 3) / 4);
    const int ks = (steps + ksplit - 1) / ksplit;
    *nsplit = (steps + ks - 1) / ks;
    return gd_gemv_mfma(ctx, w, x, x_dtype, y, ksplit);
}

// g[i] = w[i % 128] * silu(z[i]): the gate of the gated head norm.
__global__ void k_head_gate(const float *z, const float *w, float *g, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) g[i] = w[i & 127] * gd_silu(z[i]);
}

extern "C" int gd_q2_0_gemv_gated(gd_ctx *ctx, const gd_q2w *w, const float *o, const float *z,
                                  const float *w_norm, float eps, const float *bias, float *y) {
    GD_CHECK_CTX(ctx);
    int rc = gd_check_q2w(ctx, w, "gd_q2_0_gemv_gated");
    if (rc) return rc;
    GD_REQUIRE(ctx, o && z && w_norm && y, "gd_q2_0_gemv_gated: null o, z, w_norm or y");
    GD_REQUIRE(ctx, (((uintptr_t)o | (uintptr_t)z | (uintptr_t)w_norm) & 15) == 0,
               "gd_q2_0_gemv_gated: o, z and w_norm must be 16-byte aligned");
    GD_REQUIRE(ctx, w->K <= 30720 && w->R < (1LL << 30),
               "gd_q2_0_gemv_gated: K=%lld (at most 30720) or R=%lld too large", (long long)w->K,
               (long long)w->R);
    float *g = nullptr;
    if ((rc = gd_ctx_workspace(ctx, (size_t)w->K * 4, (void **)&g))) return rc;
    hipLaunchKernelGGL(k_head_gate, dim3(gd_blocks(w->K, 256)), dim3(256), 0, ctx->stream, z,
                       w_norm, g, (int)w->K);
    GD_LAUNCHED(ctx, "k_head_gate");
    return gd_gemv_mfma_gated(ctx, w, o, g, eps, y, bias, nullptr, nullptr, 0, 0);
}

extern "C" int gd_q2_0_gemv_norm(gd_ctx *ctx, const gd_q2w *w, const float *h,
                                 const float *delta, int nd, int64_t delta_stride,
                                 const float *w_norm, float eps, float *hout, float *y,
                                 uint16_t *glu_out) {
    GD_CHECK_CTX(ctx);
    int rc = gd_check_q2w(ctx, w, "gd_q2_0_gemv_norm");
    if (rc) return rc;
    GD_REQUIRE(ctx, h && w_norm && (y || glu_out), "gd_q2_0_gemv_norm: null h, w_norm or y");
    GD_REQUIRE(ctx, !glu_out || w->R % 32 == 0,
               "gd_q2_0_gemv_norm: SwiGLU needs R = 2 ff rows with ff a multiple of 16");
    GD_REQUIRE(ctx, hout != h, "gd_q2_0_gemv_norm: hout must not alias h");
    if (!delta) nd = 0;
    GD_REQUIRE(ctx, nd >= 0 && nd <= 8 && (nd <= 1 || (delta_stride >= w->K &&
                                                      delta_stride % 4 == 0 &&
                                                      delta_stride * nd < (1LL << 28))),
               "gd_q2_0_gemv_norm: nd=%d partials with stride %lld", nd, (long long)delta_stride);
    GD_REQUIRE(ctx, ((uintptr_t)h & 15) == 0 && ((uintptr_t)delta & 15) == 0 &&
                        ((uintptr_t)w_norm & 15) == 0 && ((uintptr_t)hout & 15) == 0,
               "gd_q2_0_gemv_norm: h, delta, w_norm, hout must be 16-byte aligned");
    GD_REQUIRE(ctx, w->K <= 15744 && w->R < (1LL << 30),
               "gd_q2_0_gemv_norm: K=%lld (at most 15744) or R=%lld too large",
               (long long)w->K, (long long)w->R);
    return gd_gemv_mfma_norm(ctx, w, h, delta, nd, (int)delta_stride, w_norm, eps, hout, y,
                             glu_out);
}
