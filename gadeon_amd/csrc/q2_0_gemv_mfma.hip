// Q2_0 GEMV on the matrix cores: y[r] = sum_k W[r,k] x[k] for f16 x.
//
// Same result as q2_0_gemv (Kernels.metal:30-119) and Q2_0.matvec
// (Quant.swift:36-77): per block d * (sum(code*x) - sum(x)), f32 throughout.
//
// MI355X design.  v_mfma_f32_16x16x32_f16 multiplies 16 weight rows by 32
// K-values per instruction; the VALU only unpacks codes:
//   * A operand: lane (row l%16, K-group l/16) holds one Q2_0 block (32 code
//     bytes) of its row; block 4s + kgroup at chunk step s, so a row's four
//     consecutive blocks (one 128-byte line) stream per step.  Codes k and
//     k+8 of a code dword are shifted onto bits 8-9 of the two f16 halves and
//     masked: the halves are exactly c * 2^-16 (f16 subnormals, which the
//     matrix cores take at full precision), 15 VALU ops per 16 weights.
//   * B operand: the single x column is placed in output column (block % 16):
//     lane (column j, K-group) holds x only when j is its block's slot, else
//     zeros.  Sixteen consecutive blocks therefore accumulate in sixteen
//     different output columns, and each column is scaled by its own block
//     scale d once per 16 blocks ("drain"), where sum(x) of the block is
//     subtracted as well.  x is staged once per workgroup in LDS, already
//     permuted into the (k, k+8) pair order of the unpack, with a zero block
//     for the non-matching lanes.
//   * Work: mode A gives each wave G row groups (16 rows each) over all of K,
//     grid-stride; mode B (few rows, long K) lets the four waves of a
//     workgroup split K and meet in LDS.
#include "gd_internal.h"

namespace {

constexpr int MT = 256;

__device__ __forceinline__ void unpack_dword(uint32_t w, uint32_t (&t)[8]) {
    constexpr uint32_t M = 0x03000300u;
    t[0] = (w << 8) & M;
    t[1] = (w << 6) & M;
    t[2] = (w << 4) & M;
    t[3] = (w << 2) & M;
    t[4] = w & M;
    t[5] = (w >> 2) & M;
    t[6] = (w >> 4) & M;
    t[7] = (w >> 6) & M;
}

__device__ __forceinline__ f16x8 as_f16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    return __builtin_bit_cast(f16x8, u32x4{a, b, c, d});
}

template <int G, bool KSPLIT>
__global__ __launch_bounds__(MT) void q2_0_gemv_mfma_kernel(
        const uint32_t *__restrict__ codes, const uint16_t *__restrict__ scales,
        const uint16_t *__restrict__ x, float *__restrict__ y, int K, int R, int nsets) {
    extern __shared__ uint32_t lds[];
    const int nblk = K >> 7;
    uint32_t *xp = lds;                                   // [(nblk + 1)][64] x pairs
    float *sx = (float *)(lds + (nblk + 1) * 64);         // [nblk] block sums of x
    __shared__ float red[KSPLIT ? 4 : 1][16 * G];

    auto stage_x = [&]() {
    // Stage x: pair p = 8i + k of block b holds (x[b,16i+k], x[b,16i+k+8]).
    // Thread (b, i) loads the 16 x values 16i..16i+15 of block b (two 16-byte
    // loads), forms its 8 pairs in registers and writes them as 32 bytes; the
    // block sums come from an 8-lane shuffle reduction.
    for (int e = threadIdx.x; e < (nblk + 1) * 8; e += MT) {
        const int b = e >> 3, i = e & 7;
        u32x4 lo = u32x4{0u, 0u, 0u, 0u}, hi = lo;
        if (b < nblk) {
            const u32x4 *src = (const u32x4 *)(x + (size_t)b * 128 + 16 * i);
            lo = src[0];                      // x[16i .. 16i+7]
            hi = src[1];                      // x[16i+8 .. 16i+15]
        }
        u32x4 p0, p1;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            // pair k: (lo half k, hi half k); halves k of a u32x4 are dword k/2.
            const uint32_t a = lo[k >> 1], c = hi[k >> 1];
            const uint32_t a2 = lo[2 + (k >> 1)], c2 = hi[2 + (k >> 1)];
            p0[k] = (k & 1) ? ((a >> 16) | (c & 0xffff0000u)) : ((a & 0xffffu) | (c << 16));
            p1[k] = (k & 1) ? ((a2 >> 16) | (c2 & 0xffff0000u)) : ((a2 & 0xffffu) | (c2 << 16));
        }
        u32x4 *dst = (u32x4 *)(xp + b * 64 + 8 * i);
        dst[0] = p0;
        dst[1] = p1;
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            s += gd_h2f((uint16_t)(lo[k] & 0xffff)) + gd_h2f((uint16_t)(lo[k] >> 16));
            s += gd_h2f((uint16_t)(hi[k] & 0xffff)) + gd_h2f((uint16_t)(hi[k] >> 16));
        }
        s += __shfl_xor(s, 1, 64);
        s += __shfl_xor(s, 2, 64);
        s += __shfl_xor(s, 4, 64);
        if (i == 0 && b < nblk) sx[b] = s;
    }
    __syncthreads();
    };

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, kg = lane >> 4;
    const int steps = (nblk + 3) >> 2;
    const int dpr = K >> 4;                               // code dwords per row

    // Work items are (row set, chunk step) pairs walked in order, so the code
    // loads of the next item are always in flight while this one computes.
    int set0, set_stride, s_begin, s_end;
    if (KSPLIT) {                // the workgroup walks sets; its waves split the steps
        set0 = blockIdx.x;       // (the host guarantees steps >= 4: no empty wave)
        set_stride = gridDim.x;
        s_begin = steps * wave / 4;
        s_end = steps * (wave + 1) / 4;
    } else {                     // each wave walks its own sets grid-stride
        set0 = blockIdx.x * 4 + wave;
        set_stride = gridDim.x * 4;
        s_begin = 0;
        s_end = steps;
    }
    const int nsteps = s_end - s_begin;
    const int my_sets = set0 < nsets ? (nsets - 1 - set0) / set_stride + 1 : 0;
    const int nitems = my_sets * nsteps;

    auto load_codes = [&](int item, u32x4 (&cw)[G][2]) {
        const int set = set0 + (item / nsteps) * set_stride;
        const int s = s_begin + item % nsteps;
        const int blk_c = min(4 * s + kg, nblk - 1);
#pragma unroll
        for (int g = 0; g < G; g++) {
            const int row = min(set * 16 * G + 16 * g + col, R - 1);
            const u32x4 *p = (const u32x4 *)(codes + (size_t)row * dpr + (size_t)blk_c * 8);
            cw[g][0] = __builtin_nontemporal_load(p);
            cw[g][1] = __builtin_nontemporal_load(p + 1);
        }
    };

    f32x4 C[G], D[G];
    float yp[G][4];
#pragma unroll
    for (int g = 0; g < G; g++) {
        C[g] = f32x4{0.f, 0.f, 0.f, 0.f};
        D[g] = C[g];
#pragma unroll
        for (int v = 0; v < 4; v++) yp[g][v] = 0.f;
    }
    u32x4 cn[G][2];
    if (nitems > 0) load_codes(0, cn);        // first weights in flight during the staging
    stage_x();
    int dlo = s_begin;                                    // first step since the last drain
    for (int item = 0; item < nitems; item++) {
        u32x4 cw[G][2];
#pragma unroll
        for (int g = 0; g < G; g++) { cw[g][0] = cn[g][0]; cw[g][1] = cn[g][1]; }
        if (item + 1 < nitems) load_codes(item + 1, cn);
        const int set = set0 + (item / nsteps) * set_stride;
        const int s = s_begin + item % nsteps;
        const int row_base = set * 16 * G;
        const int blk = 4 * s + kg;
        const bool match = col == (blk & 15) && blk < nblk;
        const u32x4 *src = (const u32x4 *)(xp + (match ? blk : nblk) * 64);
        f16x8 Bm[16];
#pragma unroll
        for (int m = 0; m < 16; m++) Bm[m] = __builtin_bit_cast(f16x8, src[m]);
        // 2G independent accumulator chains, interleaved, so consecutive
        // MFMAs do not wait on each other's results.
#pragma unroll
        for (int i = 0; i < 8; i++) {
#pragma unroll
            for (int g = 0; g < G; g++) {
                uint32_t t[8];
                unpack_dword(cw[g][i >> 2][i & 3], t);
                C[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_f16x8(t[0], t[1], t[2], t[3]),
                                                              Bm[2 * i], C[g], 0, 0, 0);
                D[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_f16x8(t[4], t[5], t[6], t[7]),
                                                              Bm[2 * i + 1], D[g], 0, 0, 0);
            }
        }
        const bool set_end = s + 1 == s_end;
        if (((s + 1) & 3) == 0 || set_end) {
            // Drain: column `col` holds block 16*(dlo/4) + col of the steps
            // [dlo, s]; rows 4*kg + v of each row group.
            const int bj = 16 * (dlo >> 2) + col;
            const bool valid = bj >= 4 * dlo && bj < 4 * (s + 1) && bj < nblk;
            const int bjc = min(bj, nblk - 1);
            const float sxj = sx[bjc];
#pragma unroll
            for (int g = 0; g < G; g++) {
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int row = min(row_base + 16 * g + 4 * kg + v, R - 1);
                    const float d = gd_h2f(scales[(size_t)row * nblk + bjc]);
                    // The codes entered the MFMA as c * 2^-16.
                    const float cx = (C[g][v] + D[g][v]) * 0x1p16f;
                    yp[g][v] += valid ? d * (cx - sxj) : 0.f;
                }
                C[g] = f32x4{0.f, 0.f, 0.f, 0.f};
                D[g] = C[g];
            }
            dlo = set_end ? s_begin : s + 1;
        }
        if (set_end) {
            // Sum the 16 block columns of every row; with a K split, the four
            // waves (which reach every set end together) meet in LDS.
#pragma unroll
            for (int g = 0; g < G; g++)
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    float a = yp[g][v];
                    a += __shfl_xor(a, 1, 64);
                    a += __shfl_xor(a, 2, 64);
                    a += __shfl_xor(a, 4, 64);
                    a += __shfl_xor(a, 8, 64);
                    const int row = row_base + 16 * g + 4 * kg + v;
                    if (KSPLIT) {
                        if (col == 0) red[wave][16 * g + 4 * kg + v] = a;
                    } else if (col == 0 && row < R) {
                        y[row] = a;
                    }
                    yp[g][v] = 0.f;
                }
            if (KSPLIT) {
                __syncthreads();
                if (threadIdx.x < 16 * G) {
                    const int row = row_base + threadIdx.x;
                    if (row < R)
                        y[row] = red[0][threadIdx.x] + red[1][threadIdx.x] + red[2][threadIdx.x] +
                                 red[3][threadIdx.x];
                }
                __syncthreads();
            }
        }
    }
}

}  // namespace

// f16-x GEMV on the matrix cores; returns GD_EINVAL (without launching) for
// shapes it does not take, so the caller can use the VALU kernels instead.
int gd_gemv_mfma(gd_ctx *ctx, const gd_q2w *w, const void *x, float *y) {
    const int64_t K = w->K, R = w->R;
    if (K > 65536 || R >= (1LL << 31)) return GD_EINVAL;
    const int nblk = (int)(K >> 7);
    const size_t lds = (size_t)(nblk + 1) * 64 * 4 + (size_t)nblk * 4;
    const int64_t ngroups = (R + 15) / 16;
    const int cus = ctx->num_cus > 0 ? ctx->num_cus : 256;
    auto *c = (const uint32_t *)w->codes;
    auto *s = (const uint16_t *)w->scales;
    auto *xx = (const uint16_t *)x;
    const int steps = (nblk + 3) / 4;
    // Variant: rows per wave (G row groups of 16) and whether the four waves
    // of a workgroup split K.  Measured on MI355X, one row group per wave is
    // fastest at every shape (more waves in flight beats reusing x across
    // row groups); the K split pays when there are fewer than 16 row groups
    // per CU.  GADEON_GEMV_VARIANT (A1, A2, A4, B1, B2, B4) overrides it.
    static const char *forced = getenv("GADEON_GEMV_VARIANT");
    char mode = 'A';
    int G = 1;
    if (forced && (forced[0] == 'A' || forced[0] == 'B') && forced[1] >= '1' && forced[1] <= '4') {
        mode = forced[0];
        G = forced[1] - '0';
        if (G == 3) G = 2;
    } else if (ngroups < 16LL * cus && steps >= 4) {
        mode = 'B';
    }
    if (mode == 'B' && steps < 4) mode = 'A';
    const int nsets = (int)((ngroups + G - 1) / G);
    unsigned grid;
    if (mode == 'A') grid = (unsigned)std::min<int64_t>((nsets + 3) / 4, (int64_t)cus * 8);
    else grid = (unsigned)std::min<int64_t>(nsets, (int64_t)cus * 8);
#define GD_MF(G_, KS) \
    hipLaunchKernelGGL((q2_0_gemv_mfma_kernel<G_, KS>), dim3(grid), dim3(MT), lds, ctx->stream, \
                       c, s, xx, y, (int)K, (int)R, nsets)
    if (mode == 'A') {
        if (G == 4) GD_MF(4, false);
        else if (G == 2) GD_MF(2, false);
        else GD_MF(1, false);
    } else {
        if (G == 4) GD_MF(4, true);
        else if (G == 2) GD_MF(2, true);
        else GD_MF(1, true);
    }
#undef GD_MF
    GD_LAUNCHED(ctx, "q2_0_gemv_mfma");
    return GD_OK;
}
