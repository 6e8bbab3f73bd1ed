// Q2_0 GEMV on the matrix cores: y[r] = sum_k W[r,k] x[k].
//
// Same result as q2_0_gemv (Kernels.metal:30-119) and Q2_0.matvec
// (Quant.swift:36-77): per block d * (sum(code*x) - sum(x)), f32 throughout.
//
// MI355X design.  v_mfma_f32_4x4x4f16 (16 independent 4x4x4 products per
// instruction) does the multiply-adds; the VALU only unpacks codes.
//   * A operand: the weights are stored in 2 KiB tiles (16 rows x 512 K) in
//     the order the 64 lanes need them: lane l holds one Q2_0 block (32 code
//     bytes) of row l%16, block l/16 of the step, read as two 16-byte loads
//     at lane*16 and 1024 + lane*16, so every load instruction of a wave is
//     one contiguous 1 KiB.  As a 4x4x4 lane, l is row l%4 of MFMA block
//     l/4: MFMA block m covers rows 4*(m%4) .. 4*(m%4)+3 of Q2 block m/4.
//     Codes k and k+8 of a code dword land in the two f16 halves of an
//     operand dword by a mask alone (codes 2, 3, 4 sit at bits 4, 6, 8), or
//     by a mask after one of two shared shifts (w << 4 for codes 0, 1; w >> 6
//     for 5, 6, 7): ten VALU ops per 16 weights.  A half is then exactly
//     c * 2^(p-24) for bit position p (an f16 subnormal), and the x it meets
//     is staged pre-scaled by 2^(8-p), so every product is c * x * 2^-16.
//     Positions below 4 are not used: the matrix cores lose precision on
//     those subnormals (measured), while 4, 6 and 8 stay within about 1e-6
//     of the exact sum.  A block whose x would overflow f16 after the x16
//     pre-scale is staged scaled down by a power of two 2^-e, undone later.
//   * B operand: every lane reads the staged x of its own Q2 block, so the
//     four output columns of an MFMA block hold the same products and
//     column 0 is used (the lanes of one block read one LDS address, which
//     the LDS broadcasts).  x is staged once per workgroup in LDS, already
//     permuted into the (k, k+8) pair order of the unpack and pre-scaled,
//     with zero blocks past the last one for a short final step.  f32 x is
//     split into hi = f16(x) and lo = f16((x - hi) * 2^11), two B operands
//     accumulated apart and recombined in f32.
//   * Work split.  A "set" is one 16-row group; an "item" is one tile (one
//     chunk step of 512 K of one set).  Every workgroup gets the same number
//     of consecutive sets (and, with a K split, one range of steps).  Its
//     waves take the workgroup's items one at a time from an LDS counter, so
//     a wave whose loads come back late simply takes fewer items (with a
//     fixed share per wave, the workgroup waited about 3 us for its slowest
//     wave).  An item's products are scaled by their block scales d, sum(x)
//     of each block is subtracted, and the item's 16 row partials go to LDS;
//     after one barrier each row is summed over its steps in step order, so
//     the result does not depend on which wave took which item.
//   * Latency.  Each wave keeps the next P tiles in flight (a register ring),
//     each with the four scales its item needs (one 8-byte load).  Tiles,
//     scales and x are read with bounds-checked buffer loads: a load past
//     the end returns zeros without a memory access, so every load in the
//     main loop is unconditional and the compiler waits only for the tile an
//     item needs.  x is requested before the tiles (loads return in order).
#include "gd_internal.h"

namespace {

constexpr int XB = 68;    // LDS dwords per staged x block
// Dynamic LDS available beside the kernel's few static words.
constexpr size_t LDS_BYTES = 160 * 1024 - 2048;

// LDS bytes of the x staging: the x planes (two for f32 x), then the block
// sums and exponents of x.
size_t xlds_bytes(int nblk, bool hl) {
    return (size_t)(nblk + 5) * XB * 4 * (hl ? 2 : 1) + (size_t)((nblk + 1) & ~1) * 8;
}

// Operand dword m holds codes (m, m+8) of w at bit position POS[m] of its
// two f16 halves; the x pair it meets is pre-scaled by XSCALE[m] = 2^(8-POS[m]).
__device__ __forceinline__ void unpack_dword(uint32_t w, uint32_t (&t)[8]) {
    constexpr uint32_t M4 = 0x00300030u, M6 = 0x00C000C0u, M8 = 0x03000300u;
    const uint32_t u = w << 4, v = w >> 6;
    t[0] = u & M4;     // code 0 at bit 4
    t[1] = u & M6;     // code 1 at bit 6
    t[2] = w & M4;     // code 2 at bit 4
    t[3] = w & M6;     // code 3 at bit 6
    t[4] = w & M8;     // code 4 at bit 8
    t[5] = v & M4;     // code 5 at bit 4
    t[6] = v & M6;     // code 6 at bit 6
    t[7] = v & M8;     // code 7 at bit 8
}
__device__ constexpr float XSCALE[8] = {16.f, 4.f, 16.f, 4.f, 1.f, 16.f, 4.f, 1.f};

__device__ __forceinline__ f16x8 as_f16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    return __builtin_bit_cast(f16x8, u32x4{a, b, c, d});
}

// Two f32 -> two f16 (RNE) in one dword.
__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
    return (uint32_t)gd_f2h(a) | ((uint32_t)gd_f2h(b) << 16);
}

// Buffer resource over `bytes` bytes at p (raw: no stride).  Loads at an
// offset past the end return zeros without touching memory, which keeps
// every load of the main loop unconditional.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes,
                                             0x00020000);
}
constexpr int CP_NT = 2;   // cache policy: non-temporal (streamed once)

// x values of one staging entry (16 consecutive elements of one block).
// XT = 0: f16 x; 1: f32 x; 2: f32 residual h (+ delta) normalized in the
// staging (x = f16(rmsnorm(h + delta) * w)), then used as f16 x.
template <int XT> struct XChunk;
template <> struct XChunk<0> { u32x4 lo, hi; };
template <> struct XChunk<1> { f32x4 f[4]; };
template <> struct XChunk<2> { f32x4 f[4], d[4], w[4]; };

// SwiGLU output: with pair_sets > 0, W is [gate; up] with pair_sets sets
// (16 rows) in each half, a workgroup takes gate sets k .. and the matching
// up sets pair_sets + k .., and out[r] = f16(silu(gate_r . x) * (up_r . x))
// replaces y.
struct GluOut {
    uint16_t *out;
    int pair_sets;
};

// Fused input of the XT = 2 variant.
struct NormIn {
    const float *delta;      // nd partials delta + z * dstride added to h first
    const float *w;          // norm weight [K]
    float *hout;             // h + delta, written by workgroup 0 (null: not kept)
    float eps;
    int nd;                  // partials in delta (0: none)
    int dstride;             // floats between partials
};

// Waves per workgroup (all share one staged copy of x) and tiles in flight
// per wave.  Measured on the decode shapes: 16 waves and 2 tiles beat 4 or 8
// waves and 3 or 4 tiles everywhere.
constexpr int NW = 16, P = 2;

// XT: 0 = f16 x, 1 = f32 x (hi + lo split), 2 = normalized residual (see
// XChunk).  KBP: item partials kept per Q2 block (4 per row) in LDS, summed
// with the rest of the row at the end; otherwise summed across the block
// lanes first (needs 4x less LDS, for very long K).
template <int XT, bool KBP>
__global__ __launch_bounds__(64 * NW) void q2_0_gemv_mfma_kernel(
        const uint8_t *__restrict__ codes, const uint16_t *__restrict__ scales,
        const void *__restrict__ xv, float *__restrict__ y, int K, int R, int nsets,
        int sets_per_wg, int ksteps, NormIn nin, GluOut glu) {
    constexpr int MT = 64 * NW;
    constexpr bool HL = XT == 1;                          // x carried as f16 hi + lo
    // The dynamic LDS holds 16-byte operands, so it must start 16-byte
    // aligned after the static words (a 4-byte offset made every b128 LDS
    // access of the kernel misaligned and the GEMV several times slower).
    extern __shared__ __align__(16) uint32_t lds[];
    const int nblk = K >> 7;
    // LDS: x planes, block b at dword XB*b (64 pair dwords + 4 of padding, so
    // the blocks one load instruction reads start on different banks), then
    // zero blocks for the blocks of a short last step past K; per-block sum
    // and exponent of x (nblk rounded up to even, so that what follows is
    // 16-byte aligned); the row partials of every item.
    const int xstride = (nblk + 5) * XB;                   // dwords per x plane
    uint32_t *xp = lds;                                    // hi (or f16) pairs
    uint32_t *xq = lds + xstride;                          // lo plane (f32 x only)
    float *sx = (float *)(lds + (HL ? 2 : 1) * xstride);   // [nblk] block sums of x
    float *ex = sx + ((nblk + 1) & ~1);                    // [nblk] 2^(16+e_b)
    float *part = ex + ((nblk + 1) & ~1);                  // [items][4 blocks if KBP][16 rows]
    __shared__ __align__(16) int next_item;                // next item to take

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // Lane l holds row l%16 of Q2 block l/16 of a step (the tile order); as
    // a 4x4x4 MFMA lane it is row / column j = l%4 of MFMA block l/4, which
    // covers rows 4*rq .. 4*rq+3 (rq = l/4 % 4) of Q2 block kb = l/16.
    const int j = lane & 3, rq = (lane >> 2) & 3, kb = lane >> 4;
    const int steps = (nblk + 3) >> 2;
    const int bgroups = (nblk + 15) >> 4;

    // K split z = blockIdx.y: steps [s0, s1) of every set; its rows go to
    // y + z * R.  Item i is step s0 + i % L of set i / L (set-major).
    const int s0 = blockIdx.y * ksteps, s1 = min(steps, s0 + ksteps), L = s1 - s0;
    y += (size_t)blockIdx.y * R;
    // Sets of this workgroup, numbered c = 0 .. nset_wg-1 in LDS and in the
    // item space; set c is set set_lo + c of W.  With SwiGLU, nsets counts
    // gate sets, c < npair are gate sets and the rest their up sets, set
    // set_lo + pair_sets + c - npair of W.
    const int set_lo = blockIdx.x * sets_per_wg;
    const int npair = min(sets_per_wg, nsets - set_lo);
    const int nset_wg = glu.pair_sets ? 2 * npair : npair;
    const int wsets = glu.pair_sets ? glu.pair_sets + npair : npair;   // sets spanned in W
    const int total = nset_wg * L;                         // items of the workgroup
    // Item i is set i / L, step s0 + i % L: the quotient by multiply-high
    // (exact for i < 2^16 and L <= 128, which the host guarantees).
    const uint32_t Lmag = L == 1 ? 0u : (uint32_t)((0x100000000ull + L - 1) / L);
    auto set_of = [&](int it) { return L == 1 ? it : (int)__umulhi((uint32_t)it, Lmag); };

    // Staging entry e = (block e/8, chunk e%8): its x loads are issued before
    // the tile prefetch, so waiting for them leaves the tiles in flight.
    const int nstage = (nblk + 5) * 8;
    // Entries past the last x block (the zero blocks, and threads with no
    // entry) read past the end of x: zeros, without a memory access.
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(xv, (uint32_t)K * (XT ? 4u : 2u));
    const __amdgpu_buffer_rsrc_t drs =
            make_rsrc(nin.delta, nin.nd ? (uint32_t)((nin.nd - 1) * nin.dstride + K) * 4u : 0u);
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(nin.w, XT == 2 ? (uint32_t)K * 4u : 0u);
    auto load_x = [&](int e) {
        const int off = e < nblk * 8 ? (e >> 3) * 128 + 16 * (e & 7) : K;   // element offset
        XChunk<XT> c;
        if constexpr (XT == 0) {
            c.lo = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, off * 2, 0, 0));
            c.hi = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, off * 2 + 16, 0, 0));
        } else {
#pragma unroll
            for (int q = 0; q < 4; q++)
                c.f[q] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, off * 4 + 16 * q, 0, 0));
            if constexpr (XT == 2) {
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    c.d[q] = f32x4{0.f, 0.f, 0.f, 0.f};
                    // Entries past K (off == K) must read zeros: at z * dstride
                    // + K lies the next partial.
                    for (int z = 0; z < nin.nd; z++)
                        c.d[q] += __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                drs, off < K ? (uint32_t)((z * nin.dstride + off) * 4 + 16 * q)
                                             : 0xfffff000u, 0, 0));
                    c.w[q] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(wrs, off * 4 + 16 * q, 0, 0));
                }
            }
        }
        return c;
    };
    XChunk<XT> xc = load_x(threadIdx.x);
    // Keep the x loads ahead of the tile prefetch in the instruction stream:
    // loads complete in issue order, so x issued after the tiles would only
    // arrive behind them.
    __builtin_amdgcn_sched_barrier(0);

    // Tiles of the workgroup's sets: (set, s) is tile set * steps + s.  Loads
    // for items past the workgroup's last return zeros (they get an offset
    // beyond the resource).
    const __amdgpu_buffer_rsrc_t trs =
            make_rsrc(codes + (size_t)set_lo * steps * 2048, (uint32_t)wsets * steps * 2048u);
    const __amdgpu_buffer_rsrc_t srs =
            make_rsrc(scales + (size_t)set_lo * bgroups * 256, (uint32_t)wsets * bgroups * 512u);
    // Loads of item `it`: its tile, and for the lanes of column 0 the scales
    // of rows 4*rq .. 4*rq+3 of their block 4*s + kb (the other lanes load
    // nothing).
    // The address arithmetic has no branch (the compiler's wait counting is
    // exact only over straight-line loads): an item past the last gets the
    // offset 0xfffff000, beyond every resource.
    const int up_shift = glu.pair_sets ? glu.pair_sets - npair : 0;
    auto pick = [](uint32_t off, uint32_t dead) { return (off & ~dead) | (dead & 0xfffff000u); };
    auto load = [&](int it, u32x4 (&cw)[2], u32x2 &sc) {
        const int c = set_of(it), s = s0 + (it - c * L);
        const int ps = c + (c >= npair ? up_shift : 0);
        const uint32_t dead = (uint32_t)((total - 1 - it) >> 31);      // all ones past the end
        const uint32_t off = pick((uint32_t)(ps * steps + s) * 2048u + lane * 16, dead);
        cw[0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(trs, off, 0, CP_NT));
        cw[1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(trs, off + 1024, 0, CP_NT));
        const uint32_t si = (uint32_t)((ps * bgroups + (s >> 2)) * 16 + 4 * (s & 3) + kb) * 32 + 8 * rq;
        const uint32_t other = (uint32_t)-(int)(j != 0);
        sc = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(srs, pick(si, dead | other), 0, 0));
    };

    // Ring slot p starts with item p * NW + wave; each later item is taken
    // from the workgroup counter when a slot frees up.  One tile goes out
    // before the staging, the rest of the ring after it, so x (needed first)
    // does not queue behind the whole grid's prefetch.
    u32x4 ring[P][2];
    u32x2 rsc[P];
    int rit[P];
#pragma unroll
    for (int p = 0; p < P; p++) rit[p] = p * NW + wave;
    if (threadIdx.x == 0) next_item = NW * P;
    load(rit[0], ring[0], rsc[0]);

    // Stage x: pair p = 8i + k of block b holds (x[b,16i+k], x[b,16i+k+8]) *
    // XSCALE[k] * 2^-e_b.  Thread (b, i) forms the 8 pairs of x[16i ..
    // 16i+15] in registers and writes them as 32 bytes; the block's sum and
    // max|x| come from 8-lane shuffles.  e_b = 0 unless max|x| >= 2048.
    auto stage = [&](const int e, const XChunk<XT> &xc) {
        const int bb = e >> 3, i = e & 7;
        float sum = 0.f, amax = 0.f;
        f32x4 f[4];
        if constexpr (XT == 0) {
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const uint32_t d = q < 4 ? xc.lo[q] : xc.hi[q - 4];
                f[q >> 1][2 * (q & 1)] = gd_h2f((uint16_t)(d & 0xffff));
                f[q >> 1][2 * (q & 1) + 1] = gd_h2f((uint16_t)(d >> 16));
            }
        } else {
#pragma unroll
            for (int q = 0; q < 4; q++) f[q] = xc.f[q];
        }
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                sum += f[q][j];
                amax = fmaxf(amax, fabsf(f[q][j]));
            }
        sum += __shfl_xor(sum, 1, 64);
        sum += __shfl_xor(sum, 2, 64);
        sum += __shfl_xor(sum, 4, 64);
        amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
        amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
        amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
        // amax < 2^(E-126) for f32 exponent field E; amax * 16 * 2^-eb < 2^15.
        const int eb = min(111, max(0, (int)((__float_as_uint(amax) >> 23) & 0xff) - 137));
        const float down = __uint_as_float((uint32_t)(127 - eb) << 23);    // 2^-eb
        u32x4 p0, p1, q0, q1;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            // pair k = (x[16i+k], x[16i+k+8]) = (f[k/4][k%4], f[2+k/4][k%4])
            const float xa = f[k >> 2][k & 3] * down, xb = f[2 + (k >> 2)][k & 3] * down;
            const float ha = (float)(f16)xa, hb = (float)(f16)xb;
            const uint32_t hp = pack_h2(ha * XSCALE[k], hb * XSCALE[k]);
            if (k < 4) p0[k] = hp; else p1[k - 4] = hp;
            if (HL) {
                const uint32_t lp = pack_h2((xa - ha) * (0x1p11f * XSCALE[k]),
                                            (xb - hb) * (0x1p11f * XSCALE[k]));
                if (k < 4) q0[k] = lp; else q1[k - 4] = lp;
            }
        }
        if (e < nstage) {
            u32x4 *dst = (u32x4 *)(xp + bb * XB + 8 * i);
            dst[0] = p0;
            dst[1] = p1;
            if (HL) {
                u32x4 *dq = (u32x4 *)(xq + bb * XB + 8 * i);
                dq[0] = q0;
                dq[1] = q1;
            }
            if (i == 0 && bb < nblk) {
                sx[bb] = sum;
                ex[bb] = __uint_as_float((uint32_t)(127 + 16 + eb) << 23);   // 2^(16+eb)
            }
        }
    };
    // The first entry is straight-line code after the tile prefetch, so its
    // wait for x leaves the tiles in flight; further entries (K long enough
    // that (K/128 + 5) * 8 > threads) follow in a loop.
    if constexpr (XT == 2) {
        // x = f16(rmsnorm(h + delta) * w), as a separate add + norm kernel
        // followed by an f16 GEMV would form it; one entry per thread (the
        // host checks), entries past K load zeros.  Workgroup 0 keeps h +
        // delta for the next residual add.
        __shared__ float ssr[NW];
        float ss = 0.f;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            xc.f[q] += xc.d[q];
            ss += xc.f[q][0] * xc.f[q][0] + xc.f[q][1] * xc.f[q][1] +
                  xc.f[q][2] * xc.f[q][2] + xc.f[q][3] * xc.f[q][3];
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
        if (lane == 0) ssr[wave] = ss;
        if (blockIdx.x == 0 && nin.hout && threadIdx.x < nblk * 8) {
            float *ho = nin.hout + (threadIdx.x >> 3) * 128 + 16 * (threadIdx.x & 7);
#pragma unroll
            for (int q = 0; q < 4; q++) *(f32x4 *)(ho + 4 * q) = xc.f[q];
        }
        __syncthreads();
        float tot = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) tot += ssr[w];
        const float rs = 1.0f / sqrtf(tot / (float)K + nin.eps);
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int c = 0; c < 4; c++) xc.f[q][c] = (float)(f16)(xc.f[q][c] * rs * xc.w[q][c]);
    }
    stage(threadIdx.x, xc);
    if constexpr (XT != 2)
        for (int e = threadIdx.x + MT; e < nstage; e += MT) stage(e, load_x(e));
#pragma unroll
    for (int p = 1; p < P; p++) load(rit[p], ring[p], rsc[p]);
    __syncthreads();

    // One item (set c, step s): the four Q2 blocks 4s .. 4s+3 of 16 rows.
    // Every lane reads x of its own block kb, so the four columns of an
    // MFMA block hold the same products (only column 0 is used; a lane
    // group of one kb reads one address, which the LDS broadcasts).
    // Accumulator chains: f16 x uses two, f32 x two for hi and two for lo.
    auto step = [&](const int it, u32x4 (&tile)[2], u32x2 &sc) {
        const int c = set_of(it), s = s0 + (it - c * L);
        // MFMA block mb = lane/4 multiplies rows 4*rq .. 4*rq+3 of Q2 block
        // 4s + kb by four K values.  Blocks past the last (a short final
        // step) read zero-staged x and give zero products.
        const int blk = 4 * s + kb;
        const u32x4 *src = (const u32x4 *)(xp + blk * XB);
        const u32x4 *srq = (const u32x4 *)(xq + blk * XB);
        f32x4 acc[4];
#pragma unroll
        for (int d = 0; d < 8; d++) {
            uint32_t t[8];
            unpack_dword(tile[d >> 2][d & 3], t);
#pragma unroll
            for (int q = 0; q < 2; q++) {
                // Pairs 4q .. 4q+3 of chunk d: two MFMAs of four K values.
                const u32x4 bx = src[2 * d + q];
                const f16x4 a0 = __builtin_bit_cast(f16x4, u32x2{t[4 * q], t[4 * q + 1]});
                const f16x4 a1 = __builtin_bit_cast(f16x4, u32x2{t[4 * q + 2], t[4 * q + 3]});
                const f32x4 z{0.f, 0.f, 0.f, 0.f};
                // The first product of a chain starts it from zero.
                const bool first = d == 0 && q == 0;
                acc[0] = __builtin_amdgcn_mfma_f32_4x4x4f16(
                        a0, __builtin_bit_cast(f16x4, u32x2{bx[0], bx[1]}), first ? z : acc[0], 0, 0, 0);
                acc[1] = __builtin_amdgcn_mfma_f32_4x4x4f16(
                        a1, __builtin_bit_cast(f16x4, u32x2{bx[2], bx[3]}), first ? z : acc[1], 0, 0, 0);
                if (HL) {
                    const u32x4 bq = srq[2 * d + q];
                    acc[2] = __builtin_amdgcn_mfma_f32_4x4x4f16(
                            a0, __builtin_bit_cast(f16x4, u32x2{bq[0], bq[1]}), first ? z : acc[2], 0, 0, 0);
                    acc[3] = __builtin_amdgcn_mfma_f32_4x4x4f16(
                            a1, __builtin_bit_cast(f16x4, u32x2{bq[2], bq[3]}), first ? z : acc[3], 0, 0, 0);
                }
            }
        }
        // Lane (j, rq, kb) has rows 4*rq + v of block 4s + kb; every product
        // entered as c * x * 2^(-16-e_b) (lo with x 2^11).
        const bool live = blk < nblk;
        const int bj = min(blk, nblk - 1);
        const float sxj = sx[bj], exj = ex[bj];
        const float dsc[4] = {gd_h2f((uint16_t)(sc[0] & 0xffff)), gd_h2f((uint16_t)(sc[0] >> 16)),
                              gd_h2f((uint16_t)(sc[1] & 0xffff)), gd_h2f((uint16_t)(sc[1] >> 16))};
        f32x4 r;
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const float cx = HL ? (acc[0][v] + acc[1][v]) + (acc[2][v] + acc[3][v]) * 0x1p-11f
                                : acc[0][v] + acc[1][v];
            r[v] = live ? dsc[v] * (cx * exj - sxj) : 0.f;
        }
        if constexpr (KBP) {
            if (j == 0) *(f32x4 *)(part + (it * 4 + kb) * 16 + 4 * rq) = r;
        } else {
            // Sum the item's four blocks (lanes kb = 0 .. 3).
#pragma unroll
            for (int v = 0; v < 4; v++) {
                r[v] += __shfl_xor(r[v], 16, 64);
                r[v] += __shfl_xor(r[v], 32, 64);
            }
            if (j == 0 && kb == 0) *(f32x4 *)(part + it * 16 + 4 * rq) = r;
        }
    };
    // Items are consumed in the order they were taken and a wave's items
    // only grow, so once slot 0 is past the last item the wave is done.  The
    // loop has no other exit and every refill is issued (past the end: no
    // memory access), so each item waits only for its own loads.
    while (rit[0] < total) {
#pragma unroll
        for (int p = 0; p < P; p++) {
            int g = 0;
            if (lane == 0) g = atomicAdd(&next_item, 1);
            if (rit[p] < total) step(rit[p], ring[p], rsc[p]);
            rit[p] = __builtin_amdgcn_readfirstlane(g);
            load(rit[p], ring[p], rsc[p]);
        }
    }
    __syncthreads();
    // Rows: four adjacent threads per row, thread q summing its share of
    // the row's partials (KBP: block q of every step; else steps q, q+4,
    // ...), then the four added in lane order: the same order every time.
    constexpr int PI = KBP ? 4 : 1;                      // partials per item and row
    auto quarter = [&](int c, int r, int q) {
        const float *pp = part + c * L * PI * 16 + r;
        float acc = 0.f;
        if constexpr (KBP)
            for (int i = 0; i < L; i++) acc += pp[(i * 4 + q) * 16];
        else
            for (int i = q; i < L; i += 4) acc += pp[i * 16];
        return acc;
    };
    // Quad lanes by DPP quad_perm (1,0,3,2) then (2,3,0,1): each lane adds
    // its neighbour's value, so the four hold the same sum.
    auto combine = [](float a) {
        a += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(a), 0xB1, 0xF, 0xF, false));
        return a + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(a), 0x4E, 0xF, 0xF, false));
    };
    const int nrow = (glu.pair_sets ? npair : nset_wg) * 16;
    for (int base = 0; base < nrow * 4; base += MT) {   // uniform trip count: shuffles stay whole
        const int i = (base + threadIdx.x) >> 2, q = threadIdx.x & 3;
        const bool ok = i < nrow;
        const int c = ok ? i >> 4 : 0, r = i & 15;
        if (glu.pair_sets) {
            const float g = combine(ok ? quarter(c, r, q) : 0.f);
            const float u = combine(ok ? quarter(npair + c, r, q) : 0.f);
            if (ok && q == 0) glu.out[set_lo * 16 + i] = gd_f2h(gd_silu(g) * u);
        } else {
            const float v = combine(ok ? quarter(c, r, q) : 0.f);
            if (ok && q == 0 && set_lo * 16 + i < R) y[set_lo * 16 + i] = v;
        }
    }
}

// Work split of a GEMV: `per` consecutive sets per workgroup, K cut into nz
// splits of ksteps steps (split z writes y + z * R).  One 16-wave workgroup
// per CU: two fit, but two per CU, each with half the sets, measured 5-20%
// slower on every decode shape.
struct Split { int64_t per, grid; int ksteps, nz; bool kbp; };

// Item partial bytes: per Q2 block (KBP) or per row.
constexpr size_t PART_KBP = 256, PART_ROW = 64;

// lds_free: LDS beside the x staging, which holds the partials of every
// item of the workgroup's sets (rows_per_set sets of W per set counted).
// Per-block partials unless not even one set's fit.
Split plan(int64_t nsets, int steps, int ksplit, int64_t cus, size_t lds_free, int rows_per_set) {
    Split sp;
    sp.ksteps = (steps + ksplit - 1) / ksplit;
    sp.nz = (steps + sp.ksteps - 1) / sp.ksteps;
    const size_t per_set = (size_t)sp.ksteps * rows_per_set;
    sp.kbp = PART_KBP * per_set <= lds_free;
    const int64_t cap = std::max<int64_t>(
            1, std::min<int64_t>(256, (int64_t)(lds_free / ((sp.kbp ? PART_KBP : PART_ROW) * per_set))));
    // Every resident workgroup gets the same number of sets.
    sp.per = std::min(cap, (nsets * sp.nz + cus - 1) / cus);
    sp.grid = (nsets + sp.per - 1) / sp.per;
    return sp;
}

template <int XT>
int launch(gd_ctx *ctx, const gd_q2w *w, const void *x, float *y, size_t xlds,
           const NormIn &nin = NormIn{nullptr, nullptr, nullptr, 0.f, 0, 0}, int ksplit = 1,
           const GluOut &glu = GluOut{nullptr, 0}) {
    const int64_t K = w->K, R = w->R;
    const int nblk = (int)(K >> 7), steps = (nblk + 3) / 4;
    const int cus = ctx->num_cus > 0 ? ctx->num_cus : 256;
    // SwiGLU: split over gate sets, each bringing its up set along.
    const int64_t nsets = glu.pair_sets ? glu.pair_sets : (R + 15) / 16;
    const int rows_per_set = glu.pair_sets ? 2 : 1;
    const Split sp = plan(nsets, steps, glu.pair_sets ? 1 : ksplit, cus, LDS_BYTES - xlds,
                          rows_per_set);
    const size_t lds = xlds + (size_t)sp.per * rows_per_set * sp.ksteps * (sp.kbp ? PART_KBP : PART_ROW);
    // Items of a workgroup stay below 2^16 and a split below 128 steps (the
    // kernel's quotient by multiply-high).
    GD_REQUIRE(ctx, lds <= LDS_BYTES && sp.grid < (1LL << 31) && sp.ksteps <= 128 &&
                        sp.per * rows_per_set * sp.ksteps < (1 << 16),
               "gd_q2_0_gemv: K=%lld R=%lld does not fit", (long long)K, (long long)R);
    auto kern = sp.kbp ? q2_0_gemv_mfma_kernel<XT, true> : q2_0_gemv_mfma_kernel<XT, false>;
    hipLaunchKernelGGL(kern, dim3((unsigned)sp.grid, sp.nz), dim3(64 * NW), lds, ctx->stream,
                       (const uint8_t *)w->codes, (const uint16_t *)w->scales, x, y, (int)K, (int)R,
                       (int)nsets, (int)sp.per, sp.ksteps, nin, glu);
    GD_LAUNCHED(ctx, "q2_0_gemv_mfma");
    return GD_OK;
}

}  // namespace

// GEMV on the matrix cores for f16 or f32 x (the caller has checked w, x, y).
// ksplit > 1 cuts K into that many splits whose partial rows go to y + z * R
// (the caller sums them; gd_gemv_ksplit says how many there are).
int gd_gemv_mfma(gd_ctx *ctx, const gd_q2w *w, const void *x, int x_dtype, float *y,
                 int ksplit) {
    const int64_t K = w->K;
    const int XT = x_dtype == GD_F32 ? 1 : 0;
    const int nblk = (int)(K >> 7);
    const size_t xlds = xlds_bytes(nblk, XT);
    GD_REQUIRE(ctx, xlds + (size_t)64 * ((nblk + 3) / 4) <= LDS_BYTES,
               "gd_q2_0_gemv: K=%lld too long for LDS staging of %s x", (long long)K,
               XT ? "f32" : "f16");
    const NormIn none{nullptr, nullptr, nullptr, 0.f, 0, 0};
    return XT ? launch<1>(ctx, w, x, y, xlds, none, ksplit) : launch<0>(ctx, w, x, y, xlds, none, ksplit);
}

// K splits (1..4) for an f16-x GEMV whose partial rows the consumer can sum:
// the count that minimizes the tiles streamed by the busiest CU (the
// workgroups hold whole sets, so a short R leaves CUs idle unless K is
// split), plus a small charge per extra partial.  Returns the number of
// splits the launch will actually make.
int gd_gemv_ksplit(gd_ctx *ctx, int64_t K, int64_t R) {
    const int nblk = (int)(K >> 7), steps = (nblk + 3) / 4;
    const size_t xlds = xlds_bytes(nblk, false);
    if (K % 128 || xlds + (size_t)64 * steps > LDS_BYTES) return 1;
    const int cus = ctx->num_cus > 0 ? ctx->num_cus : 256;
    const int64_t nsets = (R + 15) / 16;
    int best = 1;
    double best_cost = 1e30;
    for (int z = 1; z <= 4; z++) {
        const Split sp = plan(nsets, steps, z, cus, LDS_BYTES - xlds, 1);
        // Items of the busiest workgroup (~0.2 us each), plus what each
        // extra partial costs the consumer that sums it (~0.6-0.9 us
        // measured on the fused-input GEMV: four items).
        const double cost = (double)((sp.grid * sp.nz + cus - 1) / cus) * sp.per * sp.ksteps +
                            4.0 * (sp.nz - 1);
        if (cost < best_cost - 1e-9) {
            best_cost = cost;
            best = sp.nz;
        }
    }
    return best;
}

// GEMV of x = f16(rmsnorm(h + delta) * normw): the residual add and norm
// that precede a decode projection, fused into its x staging (the caller has
// checked w and the pointers; K <= 15744 so that one thread stages one
// entry).  delta holds nd partials dstride floats apart (nd = 0: none);
// hout (if not null) receives h + delta; it must not alias h.
int gd_gemv_mfma_norm(gd_ctx *ctx, const gd_q2w *w, const float *h, const float *delta, int nd,
                      int dstride, const float *normw, float eps, float *hout, float *y,
                      uint16_t *glu_out) {
    const int nblk = (int)(w->K >> 7);
    const size_t xlds = xlds_bytes(nblk, false);
    GD_REQUIRE(ctx, (nblk + 5) * 8 <= 1024, "gd_gemv_norm: K=%lld too long (at most 15744)",
               (long long)w->K);
    GD_REQUIRE(ctx, !glu_out || w->R % 32 == 0, "gd_gemv_norm: SwiGLU needs R = 2 x 16k rows");
    const GluOut glu{glu_out, glu_out ? (int)(w->R / 32) : 0};
    return launch<2>(ctx, w, h, y, xlds, NormIn{delta, normw, hout, eps, delta ? nd : 0, dstride}, 1,
                     glu);
}
