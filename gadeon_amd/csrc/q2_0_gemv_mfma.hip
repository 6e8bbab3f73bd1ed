// Q2_0 GEMV on the matrix cores: y[r] = sum_k W[r,k] x[k].
//
// Same result as q2_0_gemv (Kernels.metal:30-119) and Q2_0.matvec
// (Quant.swift:36-77): per block d * (sum(code*x) - sum(x)), f32 throughout.
//
// MI355X design.  v_mfma_f32_16x16x32_f16 multiplies 16 weight rows by 32
// K-values per instruction; the VALU only unpacks codes:
//   * A operand: the weights are stored in 2 KiB tiles (16 rows x 512 K) in
//     the order the 64 lanes need them: lane (row l%16, K-group l/16) reads
//     one Q2_0 block (32 code bytes) of its row as two 16-byte loads, at
//     lane*16 and 1024 + lane*16, so every load instruction of a wave is one
//     contiguous 1 KiB.  Codes k and k+8 of a code dword are shifted onto bits
//     8-9 of the two f16 halves and masked: the halves are exactly c * 2^-16
//     (f16 subnormals, which the matrix cores take at full precision), 15
//     VALU ops per 16 weights.
//   * B operand: the single x column is placed in output column (block % 16):
//     lane (column j, K-group) holds x only when j is its block's slot, else
//     zeros.  Sixteen consecutive blocks therefore accumulate in sixteen
//     different output columns, and each column is scaled by its own block
//     scale d once per 16 blocks ("drain"), where sum(x) of the block is
//     subtracted as well.  x is staged once per workgroup in LDS, already
//     permuted into the (k, k+8) pair order of the unpack, with a zero block
//     for the non-matching lanes.  f32 x is split exactly enough into
//     hi = f16(x) and lo = f16((x - hi) * 2^11), two B operands accumulated
//     apart and recombined in f32 at the drain.
//   * Work split.  A "set" is one 16-row group; an "item" is one tile (one
//     chunk step of 512 K of one set).  Every workgroup gets the same number
//     of consecutive sets, and its four waves split the workgroup's items
//     into four equal contiguous ranges, so no wave waits on a longer one.
//     A set that one wave covers whole is written by that wave; a set cut by
//     a range boundary is summed in LDS after one barrier, in wave order (the
//     result does not depend on timing).
//   * Latency.  Each wave keeps the next P tiles in flight (a register ring),
//     and the four scales of a drain (one 8-byte load) are fetched with the
//     first tile of its group, so no load waits in the loop.
#include "gd_internal.h"

namespace {

constexpr int MT = 256;
constexpr int P = 2;

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

// Pairs (x[16i+k], x[16i+k+8]), k = 0..7, of 16 consecutive f16 values held
// as lo = x[16i..16i+7], hi = x[16i+8..16i+15].
__device__ __forceinline__ void make_pairs(const u32x4 &lo, const u32x4 &hi, u32x4 &p0,
                                           u32x4 &p1) {
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t l0 = lo[k >> 1], h0 = hi[k >> 1];
        const uint32_t l1 = lo[2 + (k >> 1)], h1 = hi[2 + (k >> 1)];
        p0[k] = (k & 1) ? ((l0 >> 16) | (h0 & 0xffff0000u)) : ((l0 & 0xffffu) | (h0 << 16));
        p1[k] = (k & 1) ? ((l1 >> 16) | (h1 & 0xffff0000u)) : ((l1 & 0xffffu) | (h1 << 16));
    }
}

__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
    return (uint32_t)gd_f2h(a) | ((uint32_t)gd_f2h(b) << 16);
}

// Position of an item inside the workgroup's item space (set-major).
struct Cursor {
    int set, s;
    __device__ void next(int steps) {
        if (++s == steps) { s = 0; ++set; }
    }
};

// XT: 0 = f16 x, 1 = f32 x (hi + lo split).
template <int XT>
__global__ __launch_bounds__(MT) void q2_0_gemv_mfma_kernel(
        const uint8_t *__restrict__ codes, const uint16_t *__restrict__ scales,
        const void *__restrict__ xv, float *__restrict__ y, int K, int R, int nsets,
        int sets_per_wg) {
    extern __shared__ uint32_t lds[];
    const int nblk = K >> 7;
    const int xstride = (nblk + 1) * 64;                   // dwords per x plane
    uint32_t *xp = lds;                                    // [(nblk + 1)][64] x pairs (hi)
    uint32_t *xq = lds + xstride;                          // lo plane (f32 x only)
    float *sx = (float *)(lds + (XT ? 2 : 1) * xstride);   // [nblk] block sums of x
    __shared__ float red[4][2][16];                        // partial sums of cut sets

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, kg = lane >> 4;
    const int steps = (nblk + 3) >> 2;
    const int bgroups = (nblk + 15) >> 4;

    const int set_lo = blockIdx.x * sets_per_wg;
    const int nset_wg = min(sets_per_wg, nsets - set_lo);
    const int total = nset_wg * steps;
    const int a = total * wave / 4, b = total * (wave + 1) / 4;
    const int nitems = b - a;

    // Loads of item `ld`: its tile, and at a group start (the first step of
    // 4, or the wave's first item) the scales its drain will use: rows
    // 4*kg .. 4*kg+3 of block 16*(s/4) + col.
    auto load = [&](const Cursor &ld, bool first, u32x4 (&cw)[2], u32x2 &sc) {
        const size_t set = (size_t)(set_lo + ld.set);
        const u32x4 *t = (const u32x4 *)(codes + ((set * steps + ld.s) << 11)) + lane;
        cw[0] = __builtin_nontemporal_load(t);
        cw[1] = __builtin_nontemporal_load(t + 64);
        if ((ld.s & 3) == 0 || first)
            sc = *(const u32x2 *)(scales + (((set * bgroups + (ld.s >> 2)) * 16 + col) * 16 + 4 * kg));
    };

    u32x4 ring[P][2];
    u32x2 rsc[P];
    Cursor ld{a / steps, a % steps};
#pragma unroll
    for (int p = 0; p < P; p++) {
        if (p < nitems) load(ld, p == 0, ring[p], rsc[p]);
        ld.next(steps);
    }

    // Stage x (all threads, while the first tiles are in flight): pair
    // p = 8i + k of block b holds (x[b,16i+k], x[b,16i+k+8]).  Thread (b, i)
    // loads x[16i .. 16i+15] of block b, forms its 8 pairs in registers and
    // writes them as 32 bytes; block sums come from an 8-lane shuffle sum.
    for (int e = threadIdx.x; e < (nblk + 1) * 8; e += MT) {
        const int bb = e >> 3, i = e & 7;
        float sum = 0.f;
        u32x4 p0, p1;
        if (XT == 0) {
            u32x4 lo = u32x4{0u, 0u, 0u, 0u}, hi = lo;
            if (bb < nblk) {
                const u32x4 *src = (const u32x4 *)((const uint16_t *)xv + (size_t)bb * 128 + 16 * i);
                lo = src[0];
                hi = src[1];
            }
            make_pairs(lo, hi, p0, p1);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                sum += gd_h2f((uint16_t)(lo[k] & 0xffff)) + gd_h2f((uint16_t)(lo[k] >> 16));
                sum += gd_h2f((uint16_t)(hi[k] & 0xffff)) + gd_h2f((uint16_t)(hi[k] >> 16));
            }
        } else {
            f32x4 f[4] = {};
            if (bb < nblk) {
                const f32x4 *src = (const f32x4 *)((const float *)xv + (size_t)bb * 128 + 16 * i);
#pragma unroll
                for (int q = 0; q < 4; q++) f[q] = src[q];
            }
            u32x4 hl, hh, ll, lh;                 // hi/lo halves of x[0..7], x[8..15]
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float x0 = f[q >> 1][2 * (q & 1)], x1 = f[q >> 1][2 * (q & 1) + 1];
                const float y0 = f[2 + (q >> 1)][2 * (q & 1)], y1 = f[2 + (q >> 1)][2 * (q & 1) + 1];
                const float hx0 = (float)(f16)x0, hx1 = (float)(f16)x1;
                const float hy0 = (float)(f16)y0, hy1 = (float)(f16)y1;
                hl[q] = pack_h2(x0, x1);
                hh[q] = pack_h2(y0, y1);
                ll[q] = pack_h2((x0 - hx0) * 0x1p11f, (x1 - hx1) * 0x1p11f);
                lh[q] = pack_h2((y0 - hy0) * 0x1p11f, (y1 - hy1) * 0x1p11f);
                sum += (x0 + x1) + (y0 + y1);
            }
            u32x4 q0, q1;
            make_pairs(hl, hh, p0, p1);
            make_pairs(ll, lh, q0, q1);
            u32x4 *dq = (u32x4 *)(xq + bb * 64 + 8 * i);
            dq[0] = q0;
            dq[1] = q1;
        }
        u32x4 *dst = (u32x4 *)(xp + bb * 64 + 8 * i);
        dst[0] = p0;
        dst[1] = p1;
        sum += __shfl_xor(sum, 1, 64);
        sum += __shfl_xor(sum, 2, 64);
        sum += __shfl_xor(sum, 4, 64);
        if (i == 0 && bb < nblk) sx[bb] = sum;
    }
    __syncthreads();

    f32x4 C = f32x4{0.f, 0.f, 0.f, 0.f}, D = C, C2 = C, D2 = C;
    float yp[4] = {0.f, 0.f, 0.f, 0.f}, dsc[4] = {0.f, 0.f, 0.f, 0.f};
    Cursor cur{a / steps, a % steps};
    int dlo = cur.s;                                      // first step of the open group
    for (int base = 0; base < nitems; base += P) {
#pragma unroll
        for (int p = 0; p < P; p++) {
            const int item = base + p;
            if (item >= nitems) break;
            const u32x4 cw0 = ring[p][0], cw1 = ring[p][1];
            const u32x2 sc = rsc[p];
            if (item + P < nitems) load(ld, false, ring[p], rsc[p]);
            ld.next(steps);
            const int s = cur.s;
            if ((s & 3) == 0 || item == 0) {
                dlo = s;
                dsc[0] = gd_h2f((uint16_t)(sc[0] & 0xffff));
                dsc[1] = gd_h2f((uint16_t)(sc[0] >> 16));
                dsc[2] = gd_h2f((uint16_t)(sc[1] & 0xffff));
                dsc[3] = gd_h2f((uint16_t)(sc[1] >> 16));
            }
            const int blk = 4 * s + kg;
            const bool match = col == (blk & 15) && blk < nblk;
            const int xoff = (match ? blk : nblk) * 64;
            const u32x4 *src = (const u32x4 *)(xp + xoff);
            const u32x4 *srq = (const u32x4 *)(xq + xoff);
            // Independent accumulator chains, interleaved, so consecutive
            // MFMAs do not wait on each other's results.
#pragma unroll
            for (int i = 0; i < 8; i++) {
                uint32_t t[8];
                unpack_dword(i < 4 ? cw0[i] : cw1[i - 4], t);
                const f16x8 a0 = as_f16x8(t[0], t[1], t[2], t[3]);
                const f16x8 a1 = as_f16x8(t[4], t[5], t[6], t[7]);
                C = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        a0, __builtin_bit_cast(f16x8, src[2 * i]), C, 0, 0, 0);
                D = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        a1, __builtin_bit_cast(f16x8, src[2 * i + 1]), D, 0, 0, 0);
                if (XT) {
                    C2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            a0, __builtin_bit_cast(f16x8, srq[2 * i]), C2, 0, 0, 0);
                    D2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            a1, __builtin_bit_cast(f16x8, srq[2 * i + 1]), D2, 0, 0, 0);
                }
            }
            const bool set_end = s + 1 == steps;
            const bool range_end = item + 1 == nitems;
            if (((s + 1) & 3) == 0 || set_end || range_end) {
                // Drain: column `col` holds block 16*(dlo/4) + col of the
                // steps [dlo, s]; rows 4*kg + v.
                const int bj = 16 * (dlo >> 2) + col;
                const bool valid = bj >= 4 * dlo && bj < 4 * (s + 1) && bj < nblk;
                const float sxj = sx[min(bj, nblk - 1)];
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    // The codes entered the MFMA as c * 2^-16 (and lo as x * 2^11).
                    float cx = (C[v] + D[v]) * 0x1p16f;
                    if (XT) cx += (C2[v] + D2[v]) * 0x1p5f;
                    yp[v] += valid ? dsc[v] * (cx - sxj) : 0.f;
                }
                C = f32x4{0.f, 0.f, 0.f, 0.f};
                D = C;
                C2 = C;
                D2 = C;
            }
            if (set_end || range_end) {
                // Sum the 16 block columns of every row.  A set this wave
                // covers whole goes straight to y; a cut one to LDS (slot 0
                // if it began before this wave's range, else slot 1).
                const int set_first = cur.set * steps;          // item index of s = 0
                const bool whole = set_first >= a && set_first + steps <= b;
                const int slot = set_first < a ? 0 : 1;
                const int row_base = (set_lo + cur.set) * 16;
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    float acc = yp[v];
                    acc += __shfl_xor(acc, 1, 64);
                    acc += __shfl_xor(acc, 2, 64);
                    acc += __shfl_xor(acc, 4, 64);
                    acc += __shfl_xor(acc, 8, 64);
                    const int r = 4 * kg + v;
                    if (col == 0) {
                        if (!whole) red[wave][slot][r] = acc;
                        else if (row_base + r < R) y[row_base + r] = acc;
                    }
                    yp[v] = 0.f;
                }
            }
            cur.next(steps);
        }
    }
    __syncthreads();
    // Cut sets: one per range boundary strictly inside a set (the same set
    // may hold several boundaries; the first of them sums it).
    if (threadIdx.x < 3 * 16) {
        const int bi = threadIdx.x / 16 + 1, r = threadIdx.x % 16;
        const int bnd = total * bi / 4;
        const int j = bnd / steps;
        const int prev = total * (bi - 1) / 4;
        const bool first_in_set = bi == 1 || prev <= j * steps;
        if (bnd % steps != 0 && first_in_set) {
            float acc = 0.f;
            for (int w = 0; w < 4; w++) {
                const int wa = total * w / 4, wb = total * (w + 1) / 4;
                const bool overlap = wa < wb && wa < (j + 1) * steps && wb > j * steps;
                const bool whole = wa <= j * steps && wb >= (j + 1) * steps;
                if (overlap && !whole) acc += red[w][j * steps < wa ? 0 : 1][r];
            }
            const int row = (set_lo + j) * 16 + r;
            if (row < R) y[row] = acc;
        }
    }
}

template <int XT>
int occupancy_wgs(size_t lds) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, q2_0_gemv_mfma_kernel<XT>, MT, lds) !=
                hipSuccess ||
        n < 1)
        n = 1;
    return n;
}

}  // namespace

// GEMV on the matrix cores for f16 or f32 x (the caller has checked w, x, y).
int gd_gemv_mfma(gd_ctx *ctx, const gd_q2w *w, const void *x, int x_dtype, float *y) {
    const int64_t K = w->K, R = w->R;
    const int XT = x_dtype == GD_F32 ? 1 : 0;
    const int nblk = (int)(K >> 7);
    const size_t lds = (size_t)(nblk + 1) * 64 * 4 * (XT ? 2 : 1) + (size_t)nblk * 4;
    GD_REQUIRE(ctx, lds <= 160 * 1024 - 512,
               "gd_q2_0_gemv: K=%lld too long for LDS staging of %s x", (long long)K,
               XT ? "f32" : "f16");
    const int cus = ctx->num_cus > 0 ? ctx->num_cus : 256;
    const int steps = (nblk + 3) / 4;
    const int64_t nsets = (R + 15) / 16;
    // Every resident workgroup gets the same number of sets.  The LDS
    // footprint depends on K, so the occupancy is looked up per shape.
    static int occ_memo[2][513];                          // by x type and nblk; 0 = unknown
    int &occ = occ_memo[XT][nblk];
    if (occ == 0) occ = XT ? occupancy_wgs<1>(lds) : occupancy_wgs<0>(lds);
    const int64_t max_wgs = (int64_t)cus * occ;
    const int64_t per = (nsets + max_wgs - 1) / max_wgs;
    GD_REQUIRE(ctx, per * steps * 4 < (1LL << 31), "gd_q2_0_gemv: R=%lld too large",
               (long long)R);
    const unsigned grid = (unsigned)((nsets + per - 1) / per);
    auto *c = (const uint8_t *)w->codes;
    auto *s = (const uint16_t *)w->scales;
    if (XT)
        hipLaunchKernelGGL(q2_0_gemv_mfma_kernel<1>, dim3(grid), dim3(MT), lds, ctx->stream, c, s,
                           x, y, (int)K, (int)R, (int)nsets, (int)per);
    else
        hipLaunchKernelGGL(q2_0_gemv_mfma_kernel<0>, dim3(grid), dim3(MT), lds, ctx->stream, c, s,
                           x, y, (int)K, (int)R, (int)nsets, (int)per);
    GD_LAUNCHED(ctx, "q2_0_gemv_mfma");
    return GD_OK;
}
