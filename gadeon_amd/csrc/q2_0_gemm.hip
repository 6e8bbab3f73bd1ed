// Q2_0 ternary GEMM for prefill: Y[t][r] = sum_k X[t][k] W[r][k].
//
// Reference: q2_0_gemm_mm_h (LLM/metal/Kernels.metal:372-466; dq_q2_0_h
// :231-243), which dequantizes a 64x32 weight tile to half in threadgroup
// memory, stages X as half (:428) and accumulates 8x8 simdgroup products in
// f32.  The CPU oracle is T calls of Q2_0.matvec (Quant.swift:36-77).
//
// MI355X design:
//   * v_mfma_f32_32x32x16_f16 (fp16 operands, f32 accumulate): the fastest
//     f16 MFMA shape on gfx950.  A = X (tokens), B = W (weight rows).
//   * X is the heavy operand (16 bits per element against 2 for W): one X
//     tile of MT*32 tokens is shared by the workgroup's NW waves, each of
//     which owns NT*32 weight rows.
//   * Every operand reaches LDS by direct buffer->LDS loads into a two-stage
//     ring of 128-K blocks (X, each wave's codes and row scales); the next
//     block's loads go out right after the barrier that opens this one.
//   * Each lane expands the 2-bit codes of its own B operand in registers to
//     (code-1)*d in f16 -- exact, as in dq_q2_0_h -- by the hardware fp4 ->
//     f16 conversion and one fused multiply-add per two weights.  To make a
//     lane's codes one masked code dword, the K order inside each 64-K slice
//     is permuted: lane half h, step s, element e carries K = 32h + 8s + e,
//     for X and W alike (a sum over K does not care).
//   * Short-R shapes split K into f32 partials that the caller sums, so that
//     every CU gets work; a cost model picks the tile and the split.
#include "gd_internal.h"

#include <cstdlib>
#include <type_traits>
#include <cstdio>

namespace {

constexpr int BK = 64;           // K per LDS stage (half a Q2_0 block)
#ifndef GD_GEMM_PD
#define GD_GEMM_PD 2
#endif
constexpr int PD = GD_GEMM_PD;   // K-steps of A/B prefetch in the inner loop

// Eight codes (c in the low two bits of the nibbles of v, in K order: the
// device order after one mask) -> eight f16 of (code-1)*d.  Each nibble is
// the e2m1 value c/2, so the fp4 -> f16 conversion with scale 2 gives c
// exactly, two per instruction, and the fused c*d - d rounds once to the
// exact (c-1)*d, as dq_q2_0_h's half product is exact.
__device__ __forceinline__ f16x8 dequant8(uint32_t v, f16x2 d2, f16x2 nd2) {
    const f16x2 c0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(v, 2.0f, 0);
    const f16x2 c1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(v, 2.0f, 1);
    const f16x2 c2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(v, 2.0f, 2);
    const f16x2 c3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(v, 2.0f, 3);
    u32x4 r;
    r[0] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(c0, d2, nd2));
    r[1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(c1, d2, nd2));
    r[2] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(c2, d2, nd2));
    r[3] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(c3, d2, nd2));
    return __builtin_bit_cast(f16x8, r);
}

// LDS position of 16-byte chunk c (0..7) of X tile row r: rows are 128
// bytes, unpadded, with the chunk index XOR-swizzled by the row so that the
// 16 (or 8) lanes served together by a ds_read_b128 of an A fragment (rows
// r..r+15, one chunk index) land on distinct banks.
__device__ __forceinline__ uint32_t xswz(int r) {
    return (uint32_t)(((r >> 1) & 7) ^ ((r & 1) << 2));
}

// Direct loads from a buffer into LDS (lds_base is the same for the wave;
// the data is in LDS once the wave's vmcnt has drained).  16 bytes: lane
// l's bytes land at lds_base + 16 l.  2 bytes: lane l writes a dword, the
// value zero-extended, at lds_base + 4 l (measured on gfx950).
__device__ __forceinline__ void lds_load16(__amdgpu_buffer_rsrc_t r, const void *lds_base,
                                           uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
            r, (__attribute__((address_space(3))) void *)lds_base, 16, voff, soff, 0, 0);
}
__device__ __forceinline__ void lds_load2(__amdgpu_buffer_rsrc_t r, const void *lds_base,
                                          uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
            r, (__attribute__((address_space(3))) void *)lds_base, 2, voff, soff, 0, 0);
}

// LDS of one pipeline stage (one 128-K block): X as two 64-K planes of BT
// rows x 128 bytes, then per wave and weight fragment the codes of 32 rows
// (lanes 0..31: first half of the block, 32..63: second half, 16 bytes a
// row) and the 32 row scales (one dword each, the f16 in its low half; the
// upper 32 dwords repeat them).
template <int MT, int NT, int NW, int EX> struct Stage {
    static constexpr int BT = MT * 32;
    static constexpr int XPLANE = BT * 128;
    static constexpr int NF = NW * NT + EX;               // weight fragments
    static constexpr int X = 0, C = 2 * XPLANE, S = C + NF * 1024;
    static constexpr int BYTES = S + NF * 256;
};

// MT x 32 tokens by NW * NT * 32 weight rows per workgroup of NW waves (the
// waves share the workgroup's X tile, so more waves load less X per MFMA);
// blocks (128 K)
// [z * bps, min((z+1) * bps, K/128)) of K for split z.  X is f16.  YT: 0 =
// f32, 1 = f16.  With nz > 1 the output is f32 partials at Y + z * T * R.
// glu_ff > 0 (one split): W is [gate; up] with glu_ff rows each and the
// output is SwiGLU, Yv[t][r] = f16(silu(gate_r . x_t) * (up_r . x_t)) for
// the columns glu_r0 <= r < glu_end of this launch (Yv has glu_ff columns):
// lanes 0..15 of a wave's fragment take gate rows g .. g+15 and lanes
// 16..31 up rows glu_ff + g .., so one shuffle pairs them; each wave holds
// NT such fragments.  EX = 1 (SwiGLU, one split, 4 x 2 x 8 tiles only): the
// workgroup also holds a seventeenth fragment after its NW * NT, whose 32
// MFMAs per block the waves share (wave w: token tile w % 4, the K-steps of
// parity w / 4; waves 4..7 hand their sums to waves 0..3 at the end), so
// that ff = 17408 = 64 x 272 columns fill one round of 256 workgroups.
// Two waves per SIMD, except the four-wave tiles of 8 fragments a wave
// ((8,1) and (4,2) with NW = 4), whose 128 accumulators and operands do not
// fit two waves' registers: one wave per SIMD, as the planner's tile times
// assume.
// Tail (tail_nz > 0; plain f32 output, one split, no EX): the units above
// cover the rows below tail_r0 (whole row tiles); the workgroups past them
// (8 per blocks) take the rows tail_r0 .. R-1 (fewer than a tile's), one per
// token tile and K split of tail_bps blocks, and write f32 partials
// tailY[z][t][r - tail_r0], so that a short remainder of rows does not cost
// a whole extra round of full-K units.
template <int MT, int NT, int NW, int YT, int EX = 0>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(NW == 4 && MT * NT == 8 ? 1 : 2))) void q2_0_gemm_kernel(
        const uint8_t *__restrict__ codes, const uint16_t *__restrict__ scales,
        const void *__restrict__ Xv, void *__restrict__ Yv, int T, int K, int R, int bps,
        int nrt, int nz, int per, int glu_ff, int glu_r0, int glu_end, float *__restrict__ tailY,
        int tail_r0, int tail_nz, int tail_bps) {
    static_assert(!EX || (MT == 4 && NT == 2 && NW == 8 && YT == 0), "EX: 4 x 2 x 8 SwiGLU tiles");
    using St = Stage<MT, NT, NW, EX>;
    constexpr int BT = St::BT;
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * St::BYTES];

    // Workgroup b runs on XCD b % 8.  Units (token tile, K split, row tile)
    // are numbered token-tile-major and dealt to XCDs in contiguous runs of
    // `per`, so each XCD's L2 holds one or two token tiles of X rather than
    // all of it.
    const int main_grid = 8 * per;
    const bool tail = (int)blockIdx.x >= main_grid;
    int rt, z, tt;
    if (!tail) {
        const int u = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
        if (u >= (int)((T + BT - 1) / BT) * nz * nrt) return;
        rt = u % nrt;
        z = (u / nrt) % nz;
        tt = u / (nrt * nz);
    } else {
        const int tu = (int)blockIdx.x - main_grid;
        rt = 0;
        z = tu % tail_nz;
        tt = tu / tail_nz;
    }
    // Output rows of this unit start at row0 (tail: tail_r0), in rows of ldy
    // values (tail: its own narrow partial planes).
    const int row0 = tail ? tail_r0 : 0, ldy = tail ? R - tail_r0 : R;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 31, lh = lane >> 5;
    const int t0 = tt * BT;
    // This wave's first row (SwiGLU: first gate row, 16 per fragment).
    const int rw = glu_ff ? glu_r0 + rt * (16 * St::NF) + wave * (16 * NT)
                          : row0 + rt * (St::NF * 32) + wave * (NT * 32);
    // EX: the extra fragment's first gate row, and this wave's share of it.
    // (SwiGLU: 16 gate rows and their up rows; plain: 32 rows.)
    const int xr = glu_ff ? glu_r0 + rt * (16 * St::NF) + 16 * NW * NT : rt * (St::NF * 32) + 32 * NW * NT;
    const int xm = wave & 3, xpar = wave >> 2;
    const int nblk = K >> 7;
    const int csteps = (nblk + 3) >> 2;
    const int bgroups = (nblk + 15) >> 4;
    const int b_begin = z * (tail ? tail_bps : bps);
    const int b_end = min(b_begin + (tail ? tail_bps : bps), nblk);

    // Buffer resources: X from token t0, codes and scales from this wave's
    // first 16-row group.  Tokens past T and row groups past R lie beyond
    // the resource and load as zeros; their outputs are never stored.
    const __amdgpu_buffer_rsrc_t xrs =
            gd_rsrc((const char *)Xv + (size_t)t0 * K * 2, (uint32_t)min(BT, T - t0) * K * 2);
    const int g0 = rw >> 4, rgroups = (R + 15) >> 4;
    const uint32_t gvalid = (uint32_t)max(0, min(glu_ff ? (glu_ff >> 4) + NT : 2 * NT, rgroups - g0));
    const __amdgpu_buffer_rsrc_t crs =
            gd_rsrc(codes + ((size_t)g0 * csteps << 11), gvalid * (uint32_t)csteps * 2048u);
    const __amdgpu_buffer_rsrc_t srs =
            gd_rsrc(scales + (size_t)g0 * bgroups * 256, gvalid * (uint32_t)bgroups * 512u);
    // EX: the extra fragment's gate and up row groups (its loads are wave 0's).
    const int gx = xr >> 4;
    const uint32_t gvx = EX ? (uint32_t)max(0, min(glu_ff ? (glu_ff >> 4) + 1 : 2, rgroups - gx)) : 0u;
    const __amdgpu_buffer_rsrc_t xcrs = gd_rsrc(codes + ((size_t)gx * csteps << 11), gvx * (uint32_t)csteps * 2048u);
    const __amdgpu_buffer_rsrc_t xsrs = gd_rsrc(scales + (size_t)gx * bgroups * 256, gvx * (uint32_t)bgroups * 512u);

    // X loads: 1 KB chunks q = wave + NW i of a stage (plane q / (BT/8), rows
    // 8 (q % (BT/8)) ..); lane l fills physical chunk l%8 of row l/8, which
    // holds logical chunk (l%8) ^ xswz(row): the swizzle is applied by
    // choosing each lane's source.
    constexpr int XCH = BT / (4 * NW);                    // chunks per wave
    static_assert(XCH * 4 * NW == BT, "X chunks must split evenly over the waves");
    uint32_t xvo[XCH];
#pragma unroll
    for (int i = 0; i < XCH; i++) {
        const int q = wave + NW * i, p = q / (BT / 8), r = 8 * (q % (BT / 8)) + (lane >> 3);
        const int c = (lane & 7) ^ (int)xswz(r);
        xvo[i] = (uint32_t)(r * K + 64 * p + 8 * c) * 2;
    }
    // Code and scale loads of fragment n: row group relative to g0 (SwiGLU:
    // lanes 16..31 of each half read the up rows), block half lh.
    uint32_t cvo[NT], svo[NT];
#pragma unroll
    for (int n = 0; n < NT; n++) {
        const int g = glu_ff ? n + ((li >> 4) ? (glu_ff >> 4) : 0) : 2 * n + (li >> 4);
        cvo[n] = ((uint32_t)(g * csteps) << 11) + ((uint32_t)lh << 10) + ((li & 15) << 4);
        svo[n] = ((uint32_t)g * bgroups * 256 + (li & 15)) * 2;
    }
    const int gxu = (li >> 4) ? (glu_ff ? glu_ff >> 4 : 1) : 0;   // EX: second row group
    const uint32_t xcvo = ((uint32_t)(gxu * csteps) << 11) + ((uint32_t)lh << 10) + ((li & 15) << 4);
    const uint32_t xsvo = ((uint32_t)gxu * bgroups * 256 + (li & 15)) * 2;
    // Issue every load of block blk into stage st.
    auto issue = [&](int blk, int st) {
        uint8_t *base = lds + st * St::BYTES;
        const uint32_t xk = (uint32_t)blk * 256;          // bytes of K before the block
#pragma unroll
        for (int i = 0; i < XCH; i++)
            lds_load16(xrs, base + St::X + (wave + NW * i) * 1024, xvo[i], xk);
        const uint32_t cs = ((uint32_t)(blk >> 2) << 11) + ((uint32_t)(blk & 3) << 8);
        const uint32_t ss = ((uint32_t)(blk >> 4) * 256 + (blk & 15) * 16) * 2;
#pragma unroll
        for (int n = 0; n < NT; n++) {
            lds_load16(crs, base + St::C + (wave * NT + n) * 1024, cvo[n], cs);
            lds_load2(srs, base + St::S + (wave * NT + n) * 256, svo[n], ss);
        }
        if (EX && wave == 0) {
            lds_load16(xcrs, base + St::C + NW * NT * 1024, xcvo, cs);
            lds_load2(xsrs, base + St::S + NW * NT * 256, xsvo, ss);
        }
    };

    // A-fragment reads: row m*32 + li, chunk 4*lh + ks.
    uint32_t alds[4];
#pragma unroll
    for (int ks = 0; ks < 4; ks++) alds[ks] = (uint32_t)li * 128 + (((4 * lh + ks) ^ xswz(li)) << 4);

    f32x16 acc[MT][NT];
#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
        for (int n = 0; n < NT; n++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[m][n][v] = 0.f;
    f32x16 accx;                                          // EX: this wave's share
#pragma unroll
    for (int v = 0; v < 16; v++) accx[v] = 0.f;

    // One block from stage st: eight K-steps of 16 (two 64-K halves).  The
    // A fragments of step j + PD are read and the B fragments of step j + 1
    // built before step j's MFMAs issue, across the halves, so an MFMA only
    // waits on an LDS read issued PD steps earlier.  EX: on the even steps j
    // the wave also multiplies token tile xm by the extra fragment at K-step
    // j + xpar, its A fragment and code dword read two steps ahead (by
    // address: xm and xpar are not constants).
    auto compute = [&](int st) {
        // EX reads A one step ahead (not PD): the extra fragment's registers
        // would not fit beside a third A slot.
        constexpr int PD = ::PD;
        const uint8_t *base = lds + st * St::BYTES;
        f16x2 d2[NT], nd2[NT];
        u32x2 cw[2][NT];
#pragma unroll
        for (int n = 0; n < NT; n++) {
            const f16 d = *(const f16 *)(base + St::S + (wave * NT + n) * 256 + 4 * li);
            d2[n] = f16x2{d, d};
            nd2[n] = -d2[n];
#pragma unroll
            for (int h = 0; h < 2; h++)
                cw[h][n] = *(const u32x2 *)(base + St::C + (wave * NT + n) * 1024 + (h * 32 + li) * 16 + 8 * lh);
        }
        f16x2 dx2, ndx2;
        f16x8 ax;
        uint32_t wx = 0;
        if constexpr (EX) {
            const f16 d = *(const f16 *)(base + St::S + NW * NT * 256 + 4 * li);
            dx2 = f16x2{d, d};
            ndx2 = -dx2;
        }
        // The A fragment and code dword of the extra fragment's K-step j +
        // xpar (j even: the plane and the code dword do not depend on xpar).
        auto read_ax = [&](int j) {
            const uint32_t ka = (uint32_t)li * 128 + (((4 * lh + (j & 3) + xpar) ^ xswz(li)) << 4);
            ax = *(const f16x8 *)(base + St::X + (j >> 2) * St::XPLANE + ka + xm * 4096);
            wx = *(const uint32_t *)(base + St::C + NW * NT * 1024 + ((j >> 2) * 32 + li) * 16 + 8 * lh +
                                     4 * ((j & 3) >> 1));
        };
        f16x8 a[PD + 1][MT], b[2][NT];
        auto read_a = [&](int j, int slot) {
            const uint8_t *xb = base + St::X + (j >> 2) * St::XPLANE;
#pragma unroll
            for (int m = 0; m < MT; m++) a[slot][m] = *(const f16x8 *)(xb + alds[j & 3] + m * 4096);
        };
        auto build_b = [&](int j, int slot) {
            const int h = j >> 2, ks = j & 3;
#pragma unroll
            for (int n = 0; n < NT; n++) {
                // Codes 0..7 of the dword for even ks, 8..15 for odd.
                const uint32_t w = cw[h][n][ks >> 1];
                b[slot][n] = dequant8((ks & 1 ? w >> 2 : w) & 0x33333333u, d2[n], nd2[n]);
            }
        };
#pragma unroll
        for (int j = 0; j < PD; j++) read_a(j, j);
        build_b(0, 0);
        if constexpr (EX) read_ax(0);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            // Issue priority falls as the wave advances through the block
            // (3, 3, 2, 2, 1, 1, 0, 0): a wave that lags the other wave of its
            // SIMD takes the issue slots first, so both reach the barrier
            // together instead of the older running ahead.
            switch (j) {
                case 0: __builtin_amdgcn_s_setprio(3); break;
                case 2: __builtin_amdgcn_s_setprio(2); break;
                case 4: __builtin_amdgcn_s_setprio(1); break;
                case 6: __builtin_amdgcn_s_setprio(0); break;
                default: break;
            }
            // The reads go out PD steps ahead; the fence keeps the compiler
            // from sinking them next to their use, where the MFMA would
            // wait for the LDS round trip.
            if (j + PD < 8) read_a(j + PD, (j + PD) % (PD + 1));
            __builtin_amdgcn_sched_barrier(0);
            if (j + 1 < 8) build_b(j + 1, (j + 1) & 1);
            const int cur = j % (PD + 1);
#pragma unroll
            for (int m = 0; m < MT; m++)
#pragma unroll
                for (int n = 0; n < NT; n++)
                    acc[m][n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[cur][m], b[j & 1][n], acc[m][n], 0, 0, 0);
            if constexpr (EX) {
                if ((j & 1) == 0) {
                    const f16x8 bx = dequant8((wx >> (2 * xpar)) & 0x33333333u, dx2, ndx2);
                    accx = __builtin_amdgcn_mfma_f32_32x32x16_f16(ax, bx, accx, 0, 0, 0);
                    if (j + 2 < 8) read_ax(j + 2);
                }
            }
        }
    };

    // Two stages: the loads of block b+1 go out right after the barrier that
    // opens block b (every wave is then done with block b-1, whose stage
    // they overwrite), so they have a whole block of MFMAs to land.  The
    // wait before the barrier covers only this thread's own direct loads;
    // the barrier makes every thread's visible.
    issue(b_begin, 0);
    int st = 0;
    for (int blk = b_begin; blk < b_end; blk++) {
        __builtin_amdgcn_s_waitcnt(0x0F70);               // vmcnt(0); lgkm and exp not waited
        __syncthreads();
        if (blk + 1 < b_end) issue(blk + 1, st ^ 1);
        compute(st);
        st ^= 1;
    }

    // D layout of the 32x32 MFMA: lane holds column li (weight row) and rows
    // 8*(v/4) + 4*lh + (v%4) (tokens) for v < 16.  Stores go through a
    // buffer resource over this token tile's output rows: a lane's base
    // offset is computed once, each value adds a constant multiple of the
    // row pitch, and tokens past T fall outside the resource (the store is
    // dropped; the whole offset is in the vector operand, which the bounds
    // check covers).
    const int rows_t = min(BT, T - t0);
    if (glu_ff && nz > 1) {
        // K split: f32 partials P[z][t][2 n] of this launch's n = glu_end -
        // glu_r0 columns, gate column c at c, its up partner at n + c (lane
        // li < 16 holds gate rows, li >= 16 the up rows); q2_0_glu_reduce
        // sums them and applies the SwiGLU.
        const int ncol = glu_end - glu_r0;
        const __amdgpu_buffer_rsrc_t prs = gd_rsrc(
                (float *)Yv + ((size_t)z * T + t0) * 2 * ncol, (uint32_t)rows_t * 2u * ncol * 4u);
#pragma unroll
        for (int n = 0; n < NT; n++) {
            const int c = rw + 16 * n + (li & 15) - glu_r0;
            if (c >= ncol) continue;
            const uint32_t pbase = ((uint32_t)(4 * lh) * 2u * ncol + (li < 16 ? c : ncol + c)) * 4u;
#pragma unroll
            for (int m = 0; m < MT; m++)
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const uint32_t po = (uint32_t)(m * 32 + 8 * (v >> 2) + (v & 3)) * 2u * ncol * 4u;
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[m][n][v]), prs,
                                                          pbase + po, 0, 0);
                }
        }
        return;
    }
    if (glu_ff) {
        // Lane li < 16 holds gate row g = rw + li, lane li + 16 the matching
        // up row: each half finishes eight of a fragment's sixteen tokens
        // (the first half v < 8, the second v >= 8), trading one shuffle
        // per pair of values.
        const bool gl = li < 16;
        const __amdgpu_buffer_rsrc_t ors =
                gd_rsrc((uint16_t *)Yv + (size_t)t0 * glu_ff, (uint32_t)rows_t * glu_ff * 2u);
        // One 32 x 32 accumulator tile: token tile m, this lane's gate row g.
        auto glu_tile = [&](const f32x16 &t, int m, int g) {
            const uint32_t obase = ((uint32_t)(4 * lh + (gl ? 0 : 16)) * glu_ff + g) * 2u;
            if (g < glu_end) {
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    // Both elements first, then a select: a lane-dependent
                    // index would compile to a 16-way select chain.
                    const float lo = t[q], hi = t[8 + q];
                    const float other = __shfl_xor(gl ? hi : lo, 16, 64);
                    const float mine = gl ? lo : hi;
                    const float gate = gl ? mine : other, up = gl ? other : mine;
                    const float sg = gate * __builtin_amdgcn_rcpf(1.0f + __expf(-gate));
                    const uint32_t so = (uint32_t)(m * 32 + 8 * (q >> 2) + (q & 3)) * glu_ff * 2u;
                    __builtin_amdgcn_raw_buffer_store_b16(gd_f2h(sg * up), ors, obase + so, 0, 0);
                }
            }
        };
#pragma unroll
        for (int n = 0; n < NT; n++)
#pragma unroll
            for (int m = 0; m < MT; m++) glu_tile(acc[m][n], m, rw + 16 * n + (li & 15));
        if constexpr (EX) {
            // Waves 4..7 hand their share of the extra fragment to waves 0..3
            // (same token tile, the other K-steps) through LDS.
            __syncthreads();                              // every wave is done with the stages
            float *xl = (float *)lds;
            if (xpar) {
#pragma unroll
                for (int v = 0; v < 16; v++) xl[(xm * 16 + v) * 64 + lane] = accx[v];
            }
            __syncthreads();
            if (!xpar) {
#pragma unroll
                for (int v = 0; v < 16; v++) accx[v] += xl[(xm * 16 + v) * 64 + lane];
                glu_tile(accx, xm, xr + (li & 15));
            }
        }
        return;
    }
    constexpr uint32_t ESZ = YT ? 2 : 4;
    uint8_t *ybuf = tail ? (uint8_t *)tailY : (uint8_t *)Yv;
    const __amdgpu_buffer_rsrc_t yrs =
            gd_rsrc(ybuf + ((size_t)z * T * ldy + (size_t)t0 * ldy) * ESZ, (uint32_t)rows_t * ldy * ESZ);
#pragma unroll
    for (int n = 0; n < NT; n++) {
        const int r = rw + n * 32 + li;
        if (r >= R) continue;
        const uint32_t ybase = ((uint32_t)(4 * lh) * ldy + (r - row0)) * ESZ;
#pragma unroll
        for (int m = 0; m < MT; m++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const uint32_t so = (uint32_t)(m * 32 + 8 * (v >> 2) + (v & 3)) * ldy * ESZ;
                if (YT == 0)
                    // __float_as_uint: hipcc turns a __builtin_bit_cast of a
                    // vector element into element 0 of the vector.
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[m][n][v]), yrs, ybase + so, 0, 0);
                else
                    __builtin_amdgcn_raw_buffer_store_b16(gd_f2h(acc[m][n][v]), yrs, ybase + so, 0, 0);
                // Store fragment by fragment: without the fence the compiler
                // converts every accumulator up front and the extra VGPRs
                // halve the occupancy of the whole kernel.
                if (v == 15) __builtin_amdgcn_sched_barrier(0);
            }
    }
    if constexpr (EX) {
        // The extra fragment (rows xr .. xr + 31): waves 4..7 hand their
        // share to waves 0..3 (same token tile, the other K-steps), which
        // store it like the others (f32 out or split partials).
        __syncthreads();                                  // every wave is done with the stages
        float *xl = (float *)lds;
        if (xpar) {
#pragma unroll
            for (int v = 0; v < 16; v++) xl[(xm * 16 + v) * 64 + lane] = accx[v];
        }
        __syncthreads();
        const int r = xr + li;
        if (!xpar && r < R) {
            const uint32_t ybase = ((uint32_t)(4 * lh) * R + r) * ESZ;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const float val = accx[v] + xl[(xm * 16 + v) * 64 + lane];
                const uint32_t so = (uint32_t)(xm * 32 + 8 * (v >> 2) + (v & 3)) * R * ESZ;
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(val), yrs, ybase + so, 0, 0);
            }
        }
    }
}

// Y[i] = sum_z P[z][i] (n elements, 4 per thread).
template <int YT>
__global__ __launch_bounds__(256) void q2_0_gemm_reduce(const float *__restrict__ P,
                                                        void *__restrict__ Y, size_t n, int nz) {
    const size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= n) return;
    f32x4 a = *(const f32x4 *)(P + i);
    for (int z = 1; z < nz; z++) a += *(const f32x4 *)(P + (size_t)z * n + i);
    if (YT == 0) {
        *(f32x4 *)((float *)Y + i) = a;
    } else {
        uint16_t *o = (uint16_t *)Y + i;
        o[0] = gd_f2h(a[0]);
        o[1] = gd_f2h(a[1]);
        o[2] = gd_f2h(a[2]);
        o[3] = gd_f2h(a[3]);
    }
}

typedef void (*gemm_fn)(const uint8_t *, const uint16_t *, const void *, void *, int, int, int,
                        int, int, int, int, int, int, int, float *, int, int, int);

template <int MT, int NT, int NW>
gemm_fn pick(int yt) {
    return yt ? q2_0_gemm_kernel<MT, NT, NW, 1> : q2_0_gemm_kernel<MT, NT, NW, 0>;
}

// The kernel for a tile of MT x 32 tokens by NW x NT x 32 rows (f32 X is
// converted to f16 first, see gemm_run).  Every tile's two LDS stages fit
// the 160 KB of a CU.
gemm_fn kernel_for(int mt, int nt, int nw, int yt) {
    if (nw == 4) {
        if (mt == 8 && nt == 1) return pick<8, 1, 4>(yt);
        if (mt == 4 && nt == 2) return pick<4, 2, 4>(yt);
        if (mt == 4 && nt == 1) return pick<4, 1, 4>(yt);
        if (mt == 2 && nt == 2) return pick<2, 2, 4>(yt);
        if (mt == 2 && nt == 1) return pick<2, 1, 4>(yt);
        if (mt == 1 && nt == 1) return pick<1, 1, 4>(yt);
    } else if (nw == 8) {
        if (mt == 4 && nt == 2) return pick<4, 2, 8>(yt);
        if (mt == 4 && nt == 1) return pick<4, 1, 8>(yt);
        if (mt == 2 && nt == 2) return pick<2, 2, 8>(yt);
        if (mt == 2 && nt == 1) return pick<2, 1, 8>(yt);
    }
    return nullptr;
}

// X16[i] = f16(X[i]) (round to nearest even), 4 per thread.
__global__ __launch_bounds__(256) void gemm_x_to_f16(const float *__restrict__ X,
                                                     uint16_t *__restrict__ X16, size_t n) {
    const size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= n) return;
    const f32x4 v = *(const f32x4 *)(X + i);
    const uint32_t lo = (uint32_t)gd_f2h(v[0]) | ((uint32_t)gd_f2h(v[1]) << 16);
    const uint32_t hi = (uint32_t)gd_f2h(v[2]) | ((uint32_t)gd_f2h(v[3]) << 16);
    *(u32x2 *)(X16 + i) = u32x2{lo, hi};
}

// SwiGLU of K-split partials: out[t][r0 + c] = f16(silu(sum_z P[z][t][c]) *
// sum_z P[z][t][n + c]) for c < n, partials summed in z order.  Thread per
// (t, c).
__global__ __launch_bounds__(256) void q2_0_glu_reduce(const float *__restrict__ P,
                                                       uint16_t *__restrict__ out, int T, int n,
                                                       int nz, int ff, int r0) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)T * n) return;
    const int t = (int)(i / n), c = (int)(i % n);
    float g = 0.f, u = 0.f;
    for (int z = 0; z < nz; z++) {
        const float *row = P + ((int64_t)z * T + t) * 2 * n;
        g += row[c];
        u += row[n + c];
    }
    const float sg = g * __builtin_amdgcn_rcpf(1.0f + __expf(-g));
    out[(int64_t)t * ff + r0 + c] = gd_f2h(sg * u);
}

}  // namespace

int gd_check_q2w(gd_ctx *ctx, const gd_q2w *w, const char *who);

namespace {

// Measured per-CU times of every tile (us per 128-K block of a round with
// k = 1, 2, 3 resident workgroups; `occ` of them fit on a CU).
struct Shape { int mt, nt, nw, occ; double t[3]; };
constexpr Shape SHAPES[9] = {{1, 1, 4, 3, {0.660, 1.000, 1.390}},
                             {2, 1, 4, 3, {0.600, 1.016, 1.571}}, {4, 1, 4, 2, {1.124, 1.762, 0}},
                             {2, 2, 4, 3, {1.133, 1.866, 2.701}}, {4, 2, 4, 1, {1.807, 0, 0}},
                             {2, 1, 8, 2, {0.978, 1.760, 0}},     {4, 1, 8, 1, {1.524, 0, 0}},
                             {2, 2, 8, 1, {1.763, 0, 0}},         {4, 2, 8, 1, {2.497, 0, 0}}};

constexpr double CS = 0.162;                            // us per MB of split partials

// Time of `units` workgroups of tile sh dealt evenly over the CUs, each
// running bps blocks: the busiest CU runs ceil(units / CUs) of them, occ at
// a time.
double round_cost(const Shape &sh, int64_t units, int cus, int bps) {
    const int64_t n = (units + cus - 1) / cus;
    const int64_t q = n / sh.occ, r = n % sh.occ;
    return bps * (q * sh.t[sh.occ - 1] + (r ? sh.t[r - 1] : 0.0));
}

}  // namespace

// Tile shape, waves per workgroup and K split for a T x K x R product, from
// a cost model fitted to MI355X timings of every plan on the stack's six
// prefill shapes, after a table of measured plans for the stack's own shapes:
//   * a tile (mt, nt, waves) runs up to `occ` workgroups per CU (its LDS:
//     two stages of one 128-K block; its registers);
//   * units are dealt evenly, so the busiest CU runs n = ceil(units / CUs)
//     of them, occ at a time; a round with k resident workgroups costs T[k-1]
//     per 128-K block of the split (a CU shared by more workgroups finishes
//     more of them per us, each one more slowly);
//   * split partials cost (2s+1) f32 passes over T x R (CS us per MB).
// The plan depends on the shape and the CU count alone (no process-wide
// override); gd_q2_0_gemm_plan runs a plan the caller chooses.
gd_gemm_plan gd_gemm_choose(gd_ctx *ctx, int64_t T, int64_t K, int64_t R, int x_dtype) {
    (void)x_dtype;
    const int nblk = (int)(K / 128);
    auto nz_of = [&](int s) {
        const int bps = (nblk + s - 1) / s;
        return (nblk + bps - 1) / bps;
    };
    const int cus = ctx->num_cus > 0 ? ctx->num_cus : 256;
    // Measured plans for the config-4 stack's prefill shapes and the 17408-row
    // gate|up at T = 512 on a full MI355X (the fastest of 29-41 forced plans,
    // min of repeated sweeps); the cost model below mispredicts the 2 x 1 x 4
    // tile several per CU.
    struct Tuned { int64_t K, R; gd_gemm_plan p; };
    static constexpr Tuned TUNED[] = {
            {5120, 17408, {2, 1, 1, 4}},     // gate|up, 17408 rows: 98.6 us (105.6)
            {5120, 8224, {2, 1, 1, 4}},      // GDN in_proj: 54.0 us (the model's pick 57.4)
            {5120, 12288, {2, 1, 1, 4}},     // attention in_proj: 63.2 (67.5)
            {2048, 5120, {2, 1, 1, 8}},      // GDN out_proj: 18.7 (19.5)
            {5120, 5120, {4, 1, 3, 8}},      // attention out_proj: 36.0 (36.5)
            {17408, 5120, {4, 1, 3, 8}},     // FFN down: 88.3 (89.8)
    };
    if (T == 512 && cus == 256)
        for (const Tuned &t : TUNED)
            if (t.K == K && t.R == R) return gd_gemm_plan{t.p.mt, t.p.nt, nz_of(t.p.split), t.p.nw};
    gd_gemm_plan best{4, 1, 1};
    double best_cost = 1e30;
    // The 17-fragment (4, 2, 8) tile (gd_q2_0_gemm_plan17) is not a
    // candidate: where it fills a round that 512-row tiles leave nearly
    // empty (the GDN in_proj, R = 8224 = 16 x 512 + 32), the extra K split
    // it needs costs more than the fuller round saves (pp512 1.1% slower).
    for (const Shape &sh : SHAPES) {
        const int64_t tiles = ((T + sh.mt * 32 - 1) / (sh.mt * 32)) *
                              ((R + sh.nw * sh.nt * 32 - 1) / (sh.nw * sh.nt * 32));
        for (int s = 1; s <= 8; s++) {
            const int bps = (nblk + s - 1) / s, nz = (nblk + bps - 1) / bps;
            if (nz < s) break;                            // no more distinct splits
            double cost = round_cost(sh, tiles * nz, cus, bps);
            if (nz > 1) cost += CS * (2.0 * nz + 1) * (double)T * R * 4 / 1e6;
            if (cost < best_cost) {
                best_cost = cost;
                best = gd_gemm_plan{sh.mt, sh.nt, nz, sh.nw};
            }
        }
    }
    return best;
}

// Launch one plan on f16 X.  plan.split > 1 requires y_dtype f32 and Y sized
// split * T * R (partials, summed by the caller).
int gd_gemm_launch(gd_ctx *ctx, const gd_q2w *w, int64_t T, const void *X, int x_dtype, void *Y,
                   int y_dtype, const gd_gemm_plan &p) {
    const int K = (int)w->K, R = (int)w->R;
    const int nblk = K / 128;
    const int bps = (nblk + p.split - 1) / p.split;     // blocks (128 K) per split
    const int nz = (nblk + bps - 1) / bps;
    const int yt = p.split > 1 ? 0 : (y_dtype == GD_F16);
    gemm_fn f = p.ex ? (p.mt == 4 && p.nt == 2 && p.nw == 8 && yt == 0 ? q2_0_gemm_kernel<4, 2, 8, 0, 1>
                                                                      : nullptr)
                     : kernel_for(p.mt, p.nt, p.nw, yt);
    GD_REQUIRE(ctx, f && x_dtype == GD_F16 && (p.split == 1 || y_dtype == GD_F32) && nz == p.split &&
                        R < (1 << 22),
               "gd_q2_0_gemm: bad plan %d,%d,%d,%d%s", p.mt, p.nt, p.split, p.nw, p.ex ? " (+1)" : "");
    const int nrt = gd_blocks(R, (p.nw * p.nt + p.ex) * 32);
    const int64_t units = (int64_t)gd_blocks(T, p.mt * 32) * nz * nrt;
    const int per = (int)((units + 7) / 8);
    hipLaunchKernelGGL(f, dim3(8 * per), dim3(64 * p.nw), 0, ctx->stream, (const uint8_t *)w->codes,
                       (const uint16_t *)w->scales, X, Y, (int)T, K, R, bps, nrt, nz, per, 0, 0, 0,
                       (float *)nullptr, 0, 0, 0);
    GD_LAUNCHED(ctx, "q2_0_gemm");
    return GD_OK;
}

// gd_gemm_launch of an unsplit plain plan over the rows below r0 = R rounded
// down to the plan's row tiles, with rows r0 .. R-1 as tail units of the same
// launch: K split into *tail_nz (in: at most; out: the count made) f32
// partials tailY[z][t][r - r0], which the caller sums; Y's rows from r0 on
// are not written.  When R is a few rows past whole tiles, the units of those
// rows would otherwise run the whole K as an extra round on a few CUs.
int gd_gemm_launch_tail(gd_ctx *ctx, const gd_q2w *w, int64_t T, const void *X, float *Y,
                        const gd_gemm_plan &p, float *tailY, int *tail_nz, int *tail_r0) {
    const int K = (int)w->K, R = (int)w->R, nblk = K / 128;
    const int rows = p.nw * p.nt * 32, r0 = R / rows * rows;
    gemm_fn f = kernel_for(p.mt, p.nt, p.nw, 0);
    GD_REQUIRE(ctx, f && p.split == 1 && !p.ex && r0 < R && tailY && tail_nz && *tail_nz >= 1 &&
                        R < (1 << 22),
               "gd_gemm_launch_tail: bad plan %d,%d,%d,%d for R=%d", p.mt, p.nt, p.split, p.nw, R);
    const int tbps = (nblk + *tail_nz - 1) / *tail_nz;
    const int tnz = (nblk + tbps - 1) / tbps;
    const int ttiles = (int)gd_blocks(T, p.mt * 32), nrt = r0 / rows;
    const int per = (int)(((int64_t)ttiles * nrt + 7) / 8);
    hipLaunchKernelGGL(f, dim3(8 * per + ttiles * tnz), dim3(64 * p.nw), 0, ctx->stream,
                       (const uint8_t *)w->codes, (const uint16_t *)w->scales, X, (void *)Y, (int)T, K,
                       R, nblk, nrt, 1, per, 0, 0, 0, tailY, r0, tnz, tbps);
    GD_LAUNCHED(ctx, "q2_0_gemm_tail");
    *tail_nz = tnz;
    *tail_r0 = r0;
    return GD_OK;
}

// SwiGLU GEMM: w holds [gate; up] (R = 2 * ff rows), X f16 [T][K], out f16
// [T][ff] = silu(gate . x) * (up . x).  A tile of NW waves with NT fragments
// each covers 16 NW NT output columns.  The columns run as one launch, or as
// two: the largest whole rounds of one tile (the big tiles are the fastest
// per FLOP, but ff = 17408 = 17 * 2^10 never fills whole rounds of them) and
// the rest with another, whose K may be split (gate/up partials in the
// context workspace, then q2_0_glu_reduce) -- whichever the cost model (the
// GEMM planner's measured tile times, the partials' round trip, ~2 us per
// extra launch) finds cheaper.  tile17: 1 forces the 17-fragment tile, 0
// keeps the plan off it, -1 lets the cost model choose.
int gd_gemm_glu(gd_ctx *ctx, const gd_q2w *w, int64_t T, const void *X, uint16_t *out,
                int tile17) {
    const int K = (int)w->K, R = (int)w->R, ff = R / 2;
    GD_REQUIRE(ctx, R % 32 == 0 && T > 0 && K % 128 == 0 && R < (1 << 22), "gd_gemm_glu: R=%d "
               "must hold two halves of 16-row groups (and be below 4194304)", R);
    const int nblk = K / 128;
    // A wave's code resource spans the gate rows from its own on plus the up
    // rows (ff/16 + NT row groups, NT <= 2) as a 32-bit byte range.
    GD_REQUIRE(ctx, (uint64_t)(R / 32 + 2) * (uint64_t)((nblk + 3) / 4) * 2048u < (1ULL << 32),
               "gd_gemm_glu: K=%d R=%d spans 4 GiB of codes in one buffer resource", K, R);
    const int cus = ctx->num_cus > 0 ? ctx->num_cus : 256;
    auto cols = [](const Shape &sh) { return 16 * sh.nw * sh.nt; };
    auto tiles_t = [&](const Shape &sh) { return (T + sh.mt * 32 - 1) / (sh.mt * 32); };
    // One launch of tile sh over ncols columns, K split into nz parts (the
    // partials' round trip and the reduce launch added).
    auto cost = [&](const Shape &sh, int ncols, int nz) {
        const int bps = (nblk + nz - 1) / nz;
        double c = round_cost(sh, tiles_t(sh) * ((ncols + cols(sh) - 1) / cols(sh)) * nz, cus, bps);
        if (nz > 1) c += CS * (2.0 * nz + 1) * (double)T * 2 * ncols * 4 / 1e6 + 2.0;
        return c;
    };
    auto splits = [&](int s) {                          // distinct K splits only
        const int bps = (nblk + s - 1) / s;
        return (nblk + bps - 1) / bps;
    };
    struct Part { const Shape *sh; int r0, r1, nz; };
    Part parts[2] = {{nullptr, 0, ff, 1}, {nullptr, ff, ff, 1}};
    double best = 1e30;
    // The (4, 2, 8) tile with a seventeenth fragment: 272 columns a
    // workgroup in one launch (ff = 17408 at T = 512: one round of 256).
    // Its blocks cost the plain tile's by the fragment count.
    const Shape &t428 = SHAPES[8];
    const int xcols = 16 * (t428.nw * t428.nt + 1);
    const double cost_ex =
            round_cost(t428, tiles_t(t428) * ((ff + xcols - 1) / xcols), cus, nblk) * 17.0 / 16.0;
    for (const Shape &a : SHAPES) {
        const double c1 = cost(a, ff, 1);
        if (c1 < best) { best = c1; parts[0] = {&a, 0, ff, 1}; parts[1] = {nullptr, ff, ff, 1}; }
        // Whole rounds of a: rounds * CUs * occ units of tiles_t(a) token tiles each.
        const int64_t per_round = (int64_t)cus * a.occ;
        if (per_round % tiles_t(a)) continue;
        const int64_t colt = per_round / tiles_t(a) * cols(a);   // columns per round
        const int main_cols = (int)(ff / colt * colt);
        if (main_cols == 0 || main_cols == ff) continue;
        for (const Shape &b : SHAPES)
            for (int s = 1; s <= 8; s *= 2) {
                const int nz = splits(s);
                if (nz < s) break;
                const double c2 = cost(a, main_cols, 1) + cost(b, ff - main_cols, nz) + 2.0;
                if (c2 < best) {
                    best = c2;
                    parts[0] = {&a, 0, main_cols, 1};
                    parts[1] = {&b, main_cols, ff, nz};
                }
            }
    }
    if (tile17 == 1 || (tile17 < 0 && cost_ex < best)) {
        const int nrt = gd_blocks(ff, xcols);
        const int64_t units = tiles_t(t428) * nrt;
        const int per = (int)((units + 7) / 8);
        hipLaunchKernelGGL((q2_0_gemm_kernel<4, 2, 8, 0, 1>), dim3(8 * per), dim3(64 * 8), 0,
                           ctx->stream, (const uint8_t *)w->codes, (const uint16_t *)w->scales, X,
                           (void *)out, (int)T, K, R, nblk, nrt, 1, per, ff, 0, ff, (float *)nullptr, 0, 0,
                           0);
        GD_LAUNCHED(ctx, "q2_0_gemm_glu");
        return GD_OK;
    }
    GD_REQUIRE(ctx, parts[0].sh, "gd_gemm_glu: no tile for ff=%d", ff);
    for (const Part &pt : parts) {
        if (!pt.sh || pt.r1 <= pt.r0) continue;
        const int ncol = pt.r1 - pt.r0;
        const int bps = (nblk + pt.nz - 1) / pt.nz;
        void *dst = out;
        if (pt.nz > 1) {
            int rc = gd_ctx_workspace(ctx, (size_t)pt.nz * T * 2 * ncol * 4, &dst);
            if (rc) return rc;
        }
        gemm_fn f = kernel_for(pt.sh->mt, pt.sh->nt, pt.sh->nw, 0);
        const int nrt = gd_blocks(ncol, cols(*pt.sh));
        const int64_t units = tiles_t(*pt.sh) * pt.nz * nrt;
        const int per = (int)((units + 7) / 8);
        hipLaunchKernelGGL(f, dim3(8 * per), dim3(64 * pt.sh->nw), 0, ctx->stream,
                           (const uint8_t *)w->codes, (const uint16_t *)w->scales, X, dst, (int)T,
                           K, R, bps, nrt, pt.nz, per, ff, pt.r0, pt.r1, (float *)nullptr, 0, 0, 0);
        GD_LAUNCHED(ctx, "q2_0_gemm_glu");
        if (pt.nz > 1) {
            hipLaunchKernelGGL(q2_0_glu_reduce, dim3(gd_blocks(T * ncol, 256)), dim3(256), 0,
                               ctx->stream, (const float *)dst, out, (int)T, ncol, pt.nz, ff, pt.r0);
            GD_LAUNCHED(ctx, "q2_0_glu_reduce");
        }
    }
    return GD_OK;
}

namespace {

// Checks shared by both entry points, then the plan (split partials summed
// into Y through the context workspace).
int gemm_run(gd_ctx *ctx, const gd_q2w *w, int64_t T, const void *X, int x_dtype, void *Y,
             int y_dtype, const gd_gemm_plan *forced) {
    GD_CHECK_CTX(ctx);
    int rc = gd_check_q2w(ctx, w, "gd_q2_0_gemm");
    if (rc) return rc;
    GD_REQUIRE(ctx, X && Y, "gd_q2_0_gemm: null X or Y");
    GD_REQUIRE(ctx, T > 0 && T < (1 << 30), "gd_q2_0_gemm: T=%lld out of range", (long long)T);
    GD_REQUIRE(ctx, (x_dtype == GD_F32 || x_dtype == GD_F16) &&
                        (y_dtype == GD_F32 || y_dtype == GD_F16),
               "gd_q2_0_gemm: bad dtypes x=%d y=%d", x_dtype, y_dtype);
    GD_REQUIRE(ctx, ((uintptr_t)X & 15) == 0, "gd_q2_0_gemm: X must be 16-byte aligned");
    // Buffer offsets are 32-bit: a 256-token tile of X or of the output and
    // a wave's code rows must stay below 4 GiB.
    GD_REQUIRE(ctx, w->K <= (1 << 22) && w->R < (1LL << 22) && (size_t)T * w->R < (1ULL << 62),
               "gd_q2_0_gemm: shape too large (K and R at most 4194304)");
    gd_gemm_plan p;
    if (forced) {
        GD_REQUIRE(ctx, kernel_for(forced->mt, forced->nt, forced->nw, 0) && forced->split >= 1 &&
                            forced->split <= 16,
                   "gd_q2_0_gemm_plan: no kernel for mt=%d nt=%d split=%d nw=%d", forced->mt,
                   forced->nt, forced->split, forced->nw);
        p = *forced;
        const int nblk = (int)(w->K / 128);
        const int bps = (nblk + p.split - 1) / p.split;
        p.split = (nblk + bps - 1) / bps;               // splits that hold blocks
    } else {
        p = gd_gemm_choose(ctx, T, w->K, w->R, x_dtype);
    }
    const size_t n = (size_t)T * w->R;
    // Partials are summed 4 at a time: odd-sized outputs run unsplit.
    if (n % 4) p.split = 1;
    // The 17-fragment tile writes f32 only: unsplit with f16 Y (also where
    // the line above just forced it unsplit), the plain tile.
    if (p.ex && p.split == 1 && y_dtype == GD_F16) p.ex = 0;
    // Workspace: f16 X (f32 X is rounded to f16 once, as the reference
    // stages it, Kernels.metal:428), then the split partials.
    const size_t nx = (size_t)T * w->K;
    const size_t xbytes = x_dtype == GD_F32 ? (nx * 2 + 255) / 256 * 256 : 0;
    const size_t pbytes = p.split > 1 ? n * p.split * 4 : 0;
    uint8_t *ws = nullptr;
    if (xbytes + pbytes) {
        rc = gd_ctx_workspace(ctx, xbytes + pbytes, (void **)&ws);
        if (rc) return rc;
    }
    if (xbytes) {
        hipLaunchKernelGGL(gemm_x_to_f16, dim3((unsigned)gd_blocks((int64_t)(nx / 4), 256)), dim3(256),
                           0, ctx->stream, (const float *)X, (uint16_t *)ws, nx);
        GD_LAUNCHED(ctx, "gemm_x_to_f16");
        X = ws;
    }
    if (p.split == 1) return gd_gemm_launch(ctx, w, T, X, GD_F16, Y, y_dtype, p);
    void *part = ws + xbytes;
    rc = gd_gemm_launch(ctx, w, T, X, GD_F16, part, GD_F32, p);
    if (rc) return rc;
    const unsigned blocks = (unsigned)gd_blocks((int64_t)(n / 4), 256);
    if (y_dtype == GD_F32)
        hipLaunchKernelGGL(q2_0_gemm_reduce<0>, dim3(blocks), dim3(256), 0, ctx->stream,
                           (const float *)part, Y, n, p.split);
    else
        hipLaunchKernelGGL(q2_0_gemm_reduce<1>, dim3(blocks), dim3(256), 0, ctx->stream,
                           (const float *)part, Y, n, p.split);
    GD_LAUNCHED(ctx, "q2_0_gemm_reduce");
    return GD_OK;
}

}  // namespace

extern "C" int gd_q2_0_gemm(gd_ctx *ctx, const gd_q2w *w, int64_t T, const void *X,
                            int x_dtype, void *Y, int y_dtype) {
    return gemm_run(ctx, w, T, X, x_dtype, Y, y_dtype, nullptr);
}

extern "C" int gd_q2_0_gemm_plan(gd_ctx *ctx, const gd_q2w *w, int64_t T, const void *X,
                                 int x_dtype, void *Y, int y_dtype, int mt, int nt, int split,
                                 int nw) {
    const gd_gemm_plan p{mt, nt, split, nw};
    return gemm_run(ctx, w, T, X, x_dtype, Y, y_dtype, &p);
}

extern "C" int gd_q2_0_gemm_plan17(gd_ctx *ctx, const gd_q2w *w, int64_t T, const void *X,
                                   int x_dtype, void *Y, int y_dtype, int split) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, split > 1 || y_dtype == GD_F32,
               "gd_q2_0_gemm_plan17: f16 Y needs a K split (the tile writes f32)");
    const gd_gemm_plan p{4, 2, split, 8, 1};
    return gemm_run(ctx, w, T, X, x_dtype, Y, y_dtype, &p);
}

extern "C" int gd_q2_0_gemm_plan_tail(gd_ctx *ctx, const gd_q2w *w, int64_t T, const void *X,
                                     float *Y, int mt, int nt, int nw, int tail_split,
                                     float *tailY, int *tail_nz, int *tail_r0) {
    GD_CHECK_CTX(ctx);
    int rc = gd_check_q2w(ctx, w, "gd_q2_0_gemm_plan_tail");
    if (rc) return rc;
    GD_REQUIRE(ctx, X && Y && tailY && tail_nz && tail_r0 && ((uintptr_t)X & 15) == 0,
               "gd_q2_0_gemm_plan_tail: null or misaligned pointer");
    GD_REQUIRE(ctx, T > 0 && T < (1 << 30) && w->K <= (1 << 22) && tail_split >= 1 && tail_split <= 16,
               "gd_q2_0_gemm_plan_tail: T=%lld K=%lld split=%d out of range", (long long)T,
               (long long)w->K, tail_split);
    *tail_nz = tail_split;
    return gd_gemm_launch_tail(ctx, w, T, X, Y, gd_gemm_plan{mt, nt, 1, nw}, tailY, tail_nz, tail_r0);
}

extern "C" int gd_q2_0_gemm_swiglu(gd_ctx *ctx, const gd_q2w *w, int64_t T, const void *X,
                                   uint16_t *out) {
    GD_CHECK_CTX(ctx);
    int rc = gd_check_q2w(ctx, w, "gd_q2_0_gemm_swiglu");
    if (rc) return rc;
    GD_REQUIRE(ctx, X && out, "gd_q2_0_gemm_swiglu: null X or out");
    GD_REQUIRE(ctx, T > 0 && T < (1 << 30), "gd_q2_0_gemm_swiglu: T=%lld out of range",
               (long long)T);
    GD_REQUIRE(ctx, ((uintptr_t)X & 15) == 0, "gd_q2_0_gemm_swiglu: X must be 16-byte aligned");
    GD_REQUIRE(ctx, w->R % 32 == 0, "gd_q2_0_gemm_swiglu: R=%lld is not 2 ff with ff a multiple "
               "of 16", (long long)w->R);
    GD_REQUIRE(ctx, w->K <= (1 << 22) && w->R < (1LL << 22) && (size_t)T * w->R < (1ULL << 62),
               "gd_q2_0_gemm_swiglu: shape too large (K and R at most 4194304)");
    return gd_gemm_glu(ctx, w, T, X, out, -1);
}

extern "C" int gd_q2_0_gemm_swiglu_plan(gd_ctx *ctx, const gd_q2w *w, int64_t T, const void *X,
                                        uint16_t *out, int tile17) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, tile17 == 0 || tile17 == 1, "gd_q2_0_gemm_swiglu_plan: tile17=%d not 0 or 1",
               tile17);
    int rc = gd_check_q2w(ctx, w, "gd_q2_0_gemm_swiglu_plan");
    if (rc) return rc;
    GD_REQUIRE(ctx, X && out, "gd_q2_0_gemm_swiglu_plan: null X or out");
    GD_REQUIRE(ctx, T > 0 && T < (1 << 30), "gd_q2_0_gemm_swiglu_plan: T=%lld out of range",
               (long long)T);
    GD_REQUIRE(ctx, ((uintptr_t)X & 15) == 0, "gd_q2_0_gemm_swiglu_plan: X must be 16-byte aligned");
    GD_REQUIRE(ctx, w->R % 32 == 0, "gd_q2_0_gemm_swiglu_plan: R=%lld is not 2 ff with ff a "
               "multiple of 16", (long long)w->R);
    GD_REQUIRE(ctx, w->K <= (1 << 22) && w->R < (1LL << 22) && (size_t)T * w->R < (1ULL << 62),
               "gd_q2_0_gemm_swiglu_plan: shape too large (K and R at most 4194304)");
    return gd_gemm_glu(ctx, w, T, X, out, tile17);
}
