// Q2_0 ternary GEMV for decode: y[r] = sum_k W[r,k] x[k].
//
// Reference: q2_0_gemv (LLM/metal/Kernels.metal:30-119) and the CPU oracle
// Q2_0.matvec (LLM/src/SIMD/Quant.swift:36-77), both computing per block
// d * (sum over codes of code*x - sum x) = d * sum((code-1)*x) in f32.
//
// MI355X design (not a translation of the simdgroup kernel):
//   * Weights stream from the codes plane [R][K/4] with one 128-bit load per
//     lane: 16 bytes = 64 codes = half a Q2_0 block.  16 consecutive lanes
//     cover 256 contiguous bytes of one row, so a wave load is four fully
//     coalesced 256-byte segments.
//   * Lane l always owns the same K-chunks (l%16 + 16s), so its 64 x values
//     are loaded once per chunk step and reused for all the rows the lane
//     visits (G row groups of 4 rows).
//   * Unpack without a lookup: codes k and k+8 of a code dword w, shifted so
//     they land on bits 6-7 (or 8-9) of each 16-bit half and masked, form a
//     pair of f16 bit patterns whose values are exactly c*2^-18 (or c*2^-16):
//     f16 subnormals.  Each pair feeds v_dot2_f32_f16 against the matching x
//     pair into one of two buckets, recombined exactly by powers of two:
//     sum(code*x) = 2^18 * A + 2^16 * B.  Four shifts, eight masks and eight
//     dot2 per 16 weights.
//   * The K-reduction is a 16-lane butterfly (wave shuffles) and, when waves
//     split K, one LDS pass.
#include "gd_internal.h"

namespace {

constexpr int GEMV_THREADS = 256;   // 4 waves

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c,
                                  false);
}

// x pair for codes (16q + k, 16q + k + 8) of a 64-code chunk whose x values
// are the 32 dwords xd[] (two f16 per dword, ascending).
__device__ __forceinline__ uint32_t xpair(const uint32_t *xd, int q, int k) {
    const uint32_t a = xd[8 * q + (k >> 1)];
    const uint32_t b = xd[8 * q + 4 + (k >> 1)];
    return (k & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
}

// sum_j code_j * x_j over the 64 codes of one chunk, as 2^-24-scaled buckets.
// XS = 1: x given as one f16 set; XS = 2: x = hi + lo, two f16 sets.
template <int XS>
__device__ __forceinline__ float chunk_dot(const u32x4 &cw, const uint32_t (*xp)[8][4]) {
    // Codes are moved to bits 6-7 (value c*2^-18, bucket A) or bits 8-9
    // (c*2^-16, bucket B) of each f16 half: v_dot2_f32_f16 keeps f32-level
    // precision for those subnormals, but loses two bits per step further
    // down (measured: code at bit 0 -> 6e-5 relative error per product).
    constexpr uint32_t MA = 0x00C000C0u, MB = 0x03000300u;
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const uint32_t w = cw[q];
        const uint32_t l8 = w << 8, l4 = w << 4, u4 = w >> 4, u8 = w >> 8;
        const uint32_t t0 = l8 & MB, t1 = l4 & MA, t2 = l4 & MB, t3 = w & MA;
        const uint32_t t4 = w & MB, t5 = u4 & MA, t6 = u4 & MB, t7 = u8 & MA;
#pragma unroll
        for (int h = 0; h < XS; h++) {
            b = dot2(t0, xp[h][0][q], b);
            a = dot2(t1, xp[h][1][q], a);
            b = dot2(t2, xp[h][2][q], b);
            a = dot2(t3, xp[h][3][q], a);
            b = dot2(t4, xp[h][4][q], b);
            a = dot2(t5, xp[h][5][q], a);
            b = dot2(t6, xp[h][6][q], b);
            a = dot2(t7, xp[h][7][q], a);
        }
    }
    return fmaf(a, 4.0f, b) * 0x1p16f;    // 2^18 a + 2^16 b
}

// x for codes 64c .. 64c+63 of chunk c, as the pairs (16q+k, 16q+k+8), plus
// their f32 sum.  XT 0: f16 x.  XT 1: f32 x split exactly into hi + lo f16.
template <int XT, int XS>
__device__ __forceinline__ float load_x_chunk(const void *__restrict__ xv, int c,
                                              uint32_t (&xp)[XS][8][4]) {
    float sx = 0.f;
    if (XT == 0) {
        const u32x4 *xs = (const u32x4 *)xv + 8 * c;
        uint32_t xd[32];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const u32x4 t = xs[i];
            xd[4 * i] = t[0]; xd[4 * i + 1] = t[1];
            xd[4 * i + 2] = t[2]; xd[4 * i + 3] = t[3];
        }
#pragma unroll
        for (int i = 0; i < 32; i++) sx = dot2(xd[i], 0x3C003C00u, sx);
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int k = 0; k < 8; k++) xp[0][k][q] = xpair(xd, q, k);
    } else {
        const f32x4 *xs = (const f32x4 *)xv + 16 * c;
        uint32_t hi[32], lo[32];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const f32x4 t = xs[i];
#pragma unroll
            for (int e = 0; e < 4; e += 2) {
                const float x0 = t[e], x1 = t[e + 1];
                sx += x0;
                sx += x1;
                const f16 h0 = (f16)x0, h1 = (f16)x1;
                const f16 l0 = (f16)(x0 - (float)h0), l1 = (f16)(x1 - (float)h1);
                hi[2 * i + e / 2] = (uint32_t)__builtin_bit_cast(uint16_t, h0) |
                                    ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
                lo[2 * i + e / 2] = (uint32_t)__builtin_bit_cast(uint16_t, l0) |
                                    ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
            }
        }
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int k = 0; k < 8; k++) {
                xp[0][k][q] = xpair(hi, q, k);
                xp[XS - 1][k][q] = xpair(lo, q, k);
            }
    }
    return sx;
}

// One chunk step for G row groups: all G weight loads issue before any decode.
template <int XS, int G>
__device__ __forceinline__ void rows_step(const u32x4 *__restrict__ codes,
                                          const uint16_t *__restrict__ scales, int row0,
                                          int slot, int c, int cpr, int nblk, int R,
                                          const uint32_t (&xp)[XS][8][4], float sx,
                                          float (&acc)[G]) {
    // Rows past R read row R-1 (in bounds) and are zeroed by their scale, so
    // the loads carry no branch and all 2G of them are in flight together.
    u32x4 cw[G];
    uint16_t dh[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
        const int r = min(row0 + 4 * g + slot, R - 1);
        cw[g] = __builtin_nontemporal_load(codes + (size_t)r * cpr + c);
        dh[g] = scales[(size_t)r * nblk + (c >> 1)];
    }
#pragma unroll
    for (int g = 0; g < G; g++) {
        const float d = row0 + 4 * g + slot < R ? gd_h2f(dh[g]) : 0.f;
        const float cx = chunk_dot<XS>(cw[g], xp);
        acc[g] = fmaf(d, cx - sx, acc[g]);
    }
}

template <int G>
__device__ __forceinline__ void reduce16(float (&acc)[G]) {
#pragma unroll
    for (int g = 0; g < G; g++) {
        float v = acc[g];
        v += __shfl_xor(v, 1, 64);
        v += __shfl_xor(v, 2, 64);
        v += __shfl_xor(v, 4, 64);
        v += __shfl_xor(v, 8, 64);
        acc[g] = v;
    }
}

// Row-streaming GEMV: every wave owns whole rows (row sets of 4G rows, one
// row per 16-lane slot) and walks the row sets grid-stride.  When K fits one
// chunk step (K <= 1024) the lane's x chunk is loaded once and stays in
// registers for every row the wave visits.
template <int XT, int G>
__global__ __launch_bounds__(GEMV_THREADS) void q2_0_gemv_rows_kernel(
        const u32x4 *__restrict__ codes, const uint16_t *__restrict__ scales,
        const void *__restrict__ xv, float *__restrict__ y, int K, int R) {
    constexpr int XS = XT == 0 ? 1 : 2;
    const int lane = threadIdx.x & 63;
    const int cl = lane & 15, slot = lane >> 4;
    const int cpr = K >> 6, nblk = K >> 7;
    const int steps = (cpr + 15) >> 4;
    const int nsets = (R + 4 * G - 1) / (4 * G);
    const int wave_id = blockIdx.x * (GEMV_THREADS / 64) + (threadIdx.x >> 6);
    const int nwaves = gridDim.x * (GEMV_THREADS / 64);

    uint32_t xp[XS][8][4];
    float sx = 0.f;
    const bool one_step = steps == 1;
    if (one_step && cl < cpr) sx = load_x_chunk<XT, XS>(xv, cl, xp);

    for (int set = wave_id; set < nsets; set += nwaves) {
        const int row0 = set * 4 * G;
        float acc[G];
#pragma unroll
        for (int g = 0; g < G; g++) acc[g] = 0.f;
        for (int s = 0; s < steps; s++) {
            const int c = cl + 16 * s;
            if (c < cpr) {
                if (!one_step) sx = load_x_chunk<XT, XS>(xv, c, xp);
                rows_step<XS, G>(codes, scales, row0, slot, c, cpr, nblk, R, xp, sx, acc);
            }
        }
        reduce16<G>(acc);
        if (cl == 0) {
#pragma unroll
            for (int g = 0; g < G; g++) {
                const int r = row0 + 4 * g + slot;
                if (r < R) y[r] = acc[g];
            }
        }
    }
}

// K-split GEMV for few rows and long K: the four waves of a workgroup share
// one row set of 4G rows and take interleaved chunk steps; partial sums meet
// once in LDS.
template <int XT, int G>
__global__ __launch_bounds__(GEMV_THREADS) void q2_0_gemv_ksplit_kernel(
        const u32x4 *__restrict__ codes, const uint16_t *__restrict__ scales,
        const void *__restrict__ xv, float *__restrict__ y, int K, int R) {
    constexpr int XS = XT == 0 ? 1 : 2;
    constexpr int KW = GEMV_THREADS / 64;
    __shared__ float red[KW][4 * G];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int cl = lane & 15, slot = lane >> 4;
    const int row0 = blockIdx.x * 4 * G;
    const int cpr = K >> 6, nblk = K >> 7;
    const int steps = (cpr + 15) >> 4;

    float acc[G];
#pragma unroll
    for (int g = 0; g < G; g++) acc[g] = 0.f;
    for (int s = wave; s < steps; s += KW) {
        const int c = cl + 16 * s;
        if (c < cpr) {
            uint32_t xp[XS][8][4];
            const float sx = load_x_chunk<XT, XS>(xv, c, xp);
            rows_step<XS, G>(codes, scales, row0, slot, c, cpr, nblk, R, xp, sx, acc);
        }
    }
    reduce16<G>(acc);
    if (cl == 0) {
#pragma unroll
        for (int g = 0; g < G; g++) red[wave][4 * g + slot] = acc[g];
    }
    __syncthreads();
    if (wave == 0 && lane < 4 * G) {
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < KW; w++) v += red[w][lane];
        const int r = row0 + 4 * (lane >> 2) + (lane & 3);
        if (r < R) y[r] = v;
    }
}

// Row dequant (token embedding): out[n][k] = (code-1)*d of row ids[n], one
// thread per 16 weights (one code dword).  Exact: an f16 times -1/0/1/2.
__global__ void q2_0_dequant_rows_kernel(const uint32_t *__restrict__ codes,
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
    const uint32_t word = codes[(size_t)row * dpr + w];
    const float d = gd_h2f(scales[(size_t)row * (K >> 7) + (w >> 3)]);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        f32x4 v;
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] = (float)((int)((word >> (2 * (4 * i + j))) & 3u) - 1) * d;
        dst[i] = v;
    }
}

}  // namespace

int gd_check_q2w(gd_ctx *ctx, const gd_q2w *w, const char *who);
int gd_gemv_mfma(gd_ctx *ctx, const gd_q2w *w, const void *x, float *y);

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
                       ctx->stream, (const uint32_t *)w->codes, (const uint16_t *)w->scales, ids,
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
    GD_REQUIRE(ctx, w->K <= (1 << 24) && w->R < (1LL << 31),
               "gd_q2_0_gemv: K=%lld or R=%lld too large", (long long)w->K, (long long)w->R);
    const int K = (int)w->K, R = (int)w->R;
    // f16 x runs on the matrix cores (q2_0_gemv_mfma.hip); f32 x keeps the
    // exact hi+lo split on the VALU kernels below.
    if (x_dtype == GD_F16 && gd_gemv_mfma(ctx, w, x, y) == GD_OK) return GD_OK;
    const int steps = ((K >> 6) + 15) >> 4;
    const auto *c = (const u32x4 *)w->codes;
    const auto *s = (const uint16_t *)w->scales;
    const int cus = ctx->num_cus > 0 ? ctx->num_cus : 256;
    // Enough row sets to give every CU several waves -> stream whole rows;
    // otherwise split K across the waves of a workgroup.
    const bool rows = steps == 1 || (R + 31) / 32 >= 8 * cus;
    if (rows) {
        const bool big = (R + 31) / 32 >= 8 * cus;
        const int G = big ? 8 : 2;
        const int nsets = (R + 4 * G - 1) / (4 * G);
        const unsigned grid = (unsigned)std::min<int64_t>((nsets + 3) / 4, (int64_t)cus * 8);
#define GD_ROWS(XT, G_) \
    hipLaunchKernelGGL((q2_0_gemv_rows_kernel<XT, G_>), dim3(grid), dim3(GEMV_THREADS), 0, \
                       ctx->stream, c, s, x, y, K, R)
        if (x_dtype == GD_F16) { if (big) GD_ROWS(0, 8); else GD_ROWS(0, 2); }
        else { if (big) GD_ROWS(1, 8); else GD_ROWS(1, 2); }
#undef GD_ROWS
    } else {
        const unsigned grid = gd_blocks(R, 16);
        if (x_dtype == GD_F16)
            hipLaunchKernelGGL((q2_0_gemv_ksplit_kernel<0, 4>), dim3(grid), dim3(GEMV_THREADS), 0,
                               ctx->stream, c, s, x, y, K, R);
        else
            hipLaunchKernelGGL((q2_0_gemv_ksplit_kernel<1, 4>), dim3(grid), dim3(GEMV_THREADS), 0,
                               ctx->stream, c, s, x, y, K, R);
    }
    GD_LAUNCHED(ctx, "q2_0_gemv");
    return GD_OK;
}
