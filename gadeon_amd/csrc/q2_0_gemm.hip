// Q2_0 ternary GEMM for prefill: Y[t][r] = sum_k X[t][k] W[r][k].
//
// Reference: q2_0_gemm_mm_h (LLM/metal/Kernels.metal:372-466; dq_q2_0_h
// :231-243), which dequantizes a 64x32 weight tile to half in threadgroup
// memory, stages X as half (:428) and accumulates 8x8 simdgroup products in
// f32.  The CPU oracle is T calls of Q2_0.matvec (Quant.swift:36-77).
//
// MI355X design:
//   * Workgroup tile 128 tokens x 128 weight rows, 4 waves of 64x64, each a
//     2x2 grid of v_mfma_f32_32x32x16_f16 (fp16 operands, f32 accumulate).
//   * Per K-slice of 64: X is staged to LDS as f16 (rounded if it arrives as
//     f32, exactly where the reference rounds), and the weight codes are
//     dequantized to (code-1)*d in f16 -- exact, as in dq_q2_0_h -- straight
//     into LDS.  Both tiles are double-buffered so the next slice's global
//     loads overlap this slice's MFMAs.
//   * LDS rows are padded by 16 bytes so the ds_read_b128 operand fetches of
//     8-lane groups hit distinct banks.
#include "gd_internal.h"

namespace {

constexpr int BT = 128;          // tokens per workgroup tile
constexpr int BR = 128;          // weight rows per workgroup tile
constexpr int BK = 64;           // K per LDS stage
constexpr int LDSW = BK + 8;     // padded row length in halves
constexpr int THREADS = 256;

// Eight codes (bits 0..15 of `u`) -> four f16x2 of (code-1)*d, in K order.
// 0x6400 | c is the f16 value 1024 + c; subtracting 1025 leaves c - 1 exactly,
// and the product with d is exact (a small integer times an f16).
__device__ __forceinline__ void dequant8(uint32_t u, f16x2 d2, uint32_t *out) {
    const f16x2 off = {(f16)-1025.0f, (f16)-1025.0f};
#pragma unroll
    for (int m = 0; m < 4; m++) {
        const uint32_t lo = (u >> (4 * m)) & 3u;
        const uint32_t hi = (u >> (4 * m + 2)) & 3u;
        const uint32_t bits = lo | (hi << 16) | 0x64006400u;
        f16x2 v = __builtin_bit_cast(f16x2, bits) + off;
        v = v * d2;
        out[m] = __builtin_bit_cast(uint32_t, v);
    }
}

template <int XT, int YT>
__global__ __launch_bounds__(THREADS) void q2_0_gemm_kernel(
        const uint8_t *__restrict__ codes, const uint16_t *__restrict__ scales,
        const void *__restrict__ Xv, void *__restrict__ Yv, int T, int K, int R) {
    __shared__ __attribute__((aligned(16))) f16 Xs[2][BT * LDSW];
    __shared__ __attribute__((aligned(16))) f16 Ws[2][BR * LDSW];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int t0 = blockIdx.y * BT;
    const int r0 = blockIdx.x * BR;
    const int wr = wave & 1;         // token half of the tile
    const int wc = wave >> 1;        // weight-row half
    const int nblk = K >> 7;
    const int csteps = (nblk + 3) >> 2;
    const int bgroups = (nblk + 15) >> 4;

    // Global -> register staging for one K-slice.
    u32x4 xr[4];                     // X: 4 x 8 halves per thread (f16 path)
    f32x4 xf[8];                     // X: 4 x 8 floats per thread (f32 path)
    uint32_t wc2[2];                 // 32 codes per thread
    uint16_t wd;                     // their block scale

    const int wrow = tid >> 1;       // weight row within the tile
    const int wpart = tid & 1;       // which 32 codes of the 64-code slice

    // Tile rows past T (tokens) or R (weight rows) re-read the last valid row:
    // their outputs are never stored and no valid output depends on them, so
    // the loads need no branch and all of them issue together.
    auto load_slice = [&](int k0) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int seg = tid + THREADS * i;
            const int row = seg >> 3, col = (seg & 7) * 8;
            const int t = min(t0 + row, T - 1);
            if (XT == 0) {
                xr[i] = *(const u32x4 *)((const f16 *)Xv + (size_t)t * K + k0 + col);
            } else {
                const f32x4 *p = (const f32x4 *)((const float *)Xv + (size_t)t * K + k0 + col);
                xf[2 * i] = p[0];
                xf[2 * i + 1] = p[1];
            }
        }
        // Codes k0 .. k0+63 of a row are one 16-byte slot of its tile
        // (half (k0/64)%2 of block k0/128); this thread takes 8 bytes of it.
        const int r = min(r0 + wrow, R - 1);
        const u32x2 v = *(const u32x2 *)(codes + gd_q2_code_off(r, k0 >> 7, (k0 >> 6) & 1, csteps) +
                                         8 * wpart);
        wc2[0] = v[0];
        wc2[1] = v[1];
        wd = scales[gd_q2_scale_idx(r, k0 >> 7, bgroups)];
    };

    auto store_slice = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int seg = tid + THREADS * i;
            const int row = seg >> 3, col = (seg & 7) * 8;
            u32x4 v;
            if (XT == 0) {
                v = xr[i];
            } else {
                f16x8 h;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    h[e] = (f16)xf[2 * i][e];
                    h[4 + e] = (f16)xf[2 * i + 1][e];
                }
                v = __builtin_bit_cast(u32x4, h);
            }
            *(u32x4 *)&Xs[buf][row * LDSW + col] = v;
        }
        const f16 d = __builtin_bit_cast(f16, wd);
        const f16x2 d2 = {d, d};
        uint32_t out[16];
        dequant8(wc2[0] & 0xffffu, d2, out);
        dequant8(wc2[0] >> 16, d2, out + 4);
        dequant8(wc2[1] & 0xffffu, d2, out + 8);
        dequant8(wc2[1] >> 16, d2, out + 12);
        u32x4 *dst = (u32x4 *)&Ws[buf][wrow * LDSW + 32 * wpart];
#pragma unroll
        for (int i = 0; i < 4; i++)
            dst[i] = u32x4{out[4 * i], out[4 * i + 1], out[4 * i + 2], out[4 * i + 3]};
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[a][b][v] = 0.f;

    const int nslices = K / BK;
    load_slice(0);
    store_slice(0);
    __syncthreads();

    const int li = lane & 31, lh = lane >> 5;
    for (int s = 0; s < nslices; s++) {
        const int buf = s & 1;
        if (s + 1 < nslices) load_slice((s + 1) * BK);
#pragma unroll
        for (int ks = 0; ks < BK / 16; ks++) {
            f16x8 a[2], b[2];
#pragma unroll
            for (int m = 0; m < 2; m++)
                a[m] = *(const f16x8 *)&Xs[buf][(wr * 64 + m * 32 + li) * LDSW + ks * 16 + 8 * lh];
#pragma unroll
            for (int n = 0; n < 2; n++)
                b[n] = *(const f16x8 *)&Ws[buf][(wc * 64 + n * 32 + li) * LDSW + ks * 16 + 8 * lh];
#pragma unroll
            for (int m = 0; m < 2; m++)
#pragma unroll
                for (int n = 0; n < 2; n++)
                    acc[m][n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[m], b[n], acc[m][n], 0, 0, 0);
        }
        if (s + 1 < nslices) store_slice(buf ^ 1);
        __syncthreads();
    }

    // D layout of the 32x32 MFMA: lane holds column li (weight row) and rows
    // 8*(v/4) + 4*lh + (v%4) (tokens) for v < 16.
#pragma unroll
    for (int m = 0; m < 2; m++)
#pragma unroll
        for (int n = 0; n < 2; n++) {
            const int r = r0 + wc * 64 + n * 32 + li;
            if (r >= R) continue;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int t = t0 + wr * 64 + m * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
                if (t < T) {
                    if (YT == 0) ((float *)Yv)[(size_t)t * R + r] = acc[m][n][v];
                    else ((uint16_t *)Yv)[(size_t)t * R + r] = gd_f2h(acc[m][n][v]);
                }
            }
        }
}

}  // namespace

int gd_check_q2w(gd_ctx *ctx, const gd_q2w *w, const char *who);

extern "C" int gd_q2_0_gemm(gd_ctx *ctx, const gd_q2w *w, int64_t T, const void *X,
                            int x_dtype, void *Y, int y_dtype) {
    GD_CHECK_CTX(ctx);
    int rc = gd_check_q2w(ctx, w, "gd_q2_0_gemm");
    if (rc) return rc;
    GD_REQUIRE(ctx, X && Y, "gd_q2_0_gemm: null X or Y");
    GD_REQUIRE(ctx, T > 0 && T < (1 << 30), "gd_q2_0_gemm: T=%lld out of range", (long long)T);
    GD_REQUIRE(ctx, (x_dtype == GD_F32 || x_dtype == GD_F16) &&
                        (y_dtype == GD_F32 || y_dtype == GD_F16),
               "gd_q2_0_gemm: bad dtypes x=%d y=%d", x_dtype, y_dtype);
    GD_REQUIRE(ctx, ((uintptr_t)X & 15) == 0, "gd_q2_0_gemm: X must be 16-byte aligned");
    GD_REQUIRE(ctx, w->K <= (1 << 24) && w->R < (1LL << 31) && (size_t)T * w->R < (1ULL << 62),
               "gd_q2_0_gemm: shape too large");
    const int K = (int)w->K, R = (int)w->R;
    dim3 grid(gd_blocks(R, BR), gd_blocks(T, BT));
    auto *c = (const uint8_t *)w->codes;
    auto *s = (const uint16_t *)w->scales;
    if (x_dtype == GD_F16 && y_dtype == GD_F32)
        hipLaunchKernelGGL((q2_0_gemm_kernel<0, 0>), grid, dim3(THREADS), 0, ctx->stream, c, s, X,
                           Y, (int)T, K, R);
    else if (x_dtype == GD_F16)
        hipLaunchKernelGGL((q2_0_gemm_kernel<0, 1>), grid, dim3(THREADS), 0, ctx->stream, c, s, X,
                           Y, (int)T, K, R);
    else if (y_dtype == GD_F32)
        hipLaunchKernelGGL((q2_0_gemm_kernel<1, 0>), grid, dim3(THREADS), 0, ctx->stream, c, s, X,
                           Y, (int)T, K, R);
    else
        hipLaunchKernelGGL((q2_0_gemm_kernel<1, 1>), grid, dim3(THREADS), 0, ctx->stream, c, s, X,
                           Y, (int)T, K, R);
    GD_LAUNCHED(ctx, "q2_0_gemm");
    return GD_OK;
}
