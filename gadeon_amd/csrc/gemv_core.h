// The Q2_0 GEMV on the matrix cores as a device function (gemv::run), the
// body of the GEMV kernel in q2_0_gemv_mfma.hip.
//
// Same result as q2_0_gemv (Kernels.metal:30-119) and Q2_0.matvec
// (Quant.swift:36-77): per block d * (sum(code*x) - sum(x)), accumulated in
// f32 (the precision of each body is below).
//
// MI355X design.  Two item bodies share the work split below.
//   * Tiles.  The weights are stored in 2 KiB tiles (16 rows x 512 K) in the
//     order the 64 lanes need them: lane l holds one Q2_0 block (32 code
//     bytes) of row l%16, block l/16 of the step, read as two 16-byte loads
//     at lane*16 and 1024 + lane*16, so every load instruction of a wave is
//     one contiguous 1 KiB.
//   * fp4 body (F4, every K whose staging fits LDS: up to about 30K).
//     v_mfma_scale_f32_16x16x128_f8f6f4 with fp4 (e2m1) weights and e4m3 x.
//     A lane of that MFMA holds row l%16 and K 32*(l/16) .. +31, which the
//     tile order makes one Q2 block per lane group: a code c in the low two
//     bits of a nibble is the e2m1 value c/2, so 16 codes become two operand
//     dwords by w & 0x33333333 and (w >> 2) & 0x33333333 (three VALU ops per
//     16 weights; an A scale of 2 restores c).  x is staged per workgroup as
//     e4m3 pieces, x = 2^e (p0 + p1/16 + p2/256 [+ p3/4096]) with e per Q2
//     block: three pieces hold an f16 value exactly (four give f32 x about
//     20 bits).  B column 4q + j carries piece j of block q and is zero
//     elsewhere, so one MFMA's 16 columns hold the four blocks' piece sums
//     apart; the piece scales 2^(e - 4j) ride in the E8M0 B scales.  Four
//     MFMAs cover an item; a quad of lanes then adds the pieces and applies
//     d (sum c x - sum x) per block.  Precision: the matrix cores add each
//     group of 8 products aligned to the largest, keeping about 13 bits
//     below it (measured), so a small x beside a much larger one in the same
//     group of 8 loses low bits: relDiff against the f64 oracle is about
//     4e-6 for N(0,1) x and 1.7e-4 with every 97th element 3000x larger.
//   * f16 body (longer K).  v_mfma_f32_4x4x4f16 (16 independent 4x4x4
//     products per instruction); as a 4x4x4 lane, l is row l%4 of MFMA
//     block l/4: MFMA block m covers rows 4*(m%4) .. 4*(m%4)+3 of Q2 block
//     m/4.  Codes k and k+8 of a code dword land in the two f16 halves of an
//     operand dword by a mask alone (codes 2, 3, 4 sit at bits 4, 6, 8), or
//     by a mask after one of two shared shifts (w << 4 for codes 0, 1; w >> 6
//     for 5, 6, 7): ten VALU ops per 16 weights.  A half is then exactly
//     c * 2^(p-24) for bit position p (an f16 subnormal), and the x it meets
//     is staged pre-scaled by 2^(8-p), so every product is c * x * 2^-16.
//     Positions below 4 are not used: the matrix cores lose precision on
//     those subnormals (measured), while 4, 6 and 8 stay within about 1e-6
//     of the exact sum.  A block whose x would overflow f16 after the x16
//     pre-scale is staged scaled down by a power of two 2^-e, undone later.
//     Every lane reads the staged x of its own Q2 block, so the four output
//     columns of an MFMA block hold the same products and column 0 is used.
//     f32 x is split into hi = f16(x) and lo = f16((x - hi) * 2^11), two B
//     operands accumulated apart and recombined in f32.
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
#pragma once

#include "gd_internal.h"

namespace gemv {

constexpr int XB = 68;    // LDS dwords per staged x block
// Dynamic LDS available beside a kernel's few static words.
constexpr size_t LDS_BYTES = 160 * 1024 - 2048;
// Waves per workgroup (all share one staged copy of x) and tiles in flight
// per wave.  Measured on the decode shapes: 16 waves and 2 tiles beat 4 or 8
// waves and 3 or 4 tiles everywhere.
constexpr int NW = 16, P = 2;
constexpr int CP_NT = 2;     // cache policy: non-temporal (streamed once)
// Residual partials of the fused input that a kernel loads as one group
// with h and w (the stack's split-K projections leave one or two); the
// kernel is instantiated for 0 .. ND_UNROLL of them.
constexpr int ND_UNROLL = 2;

// LDS bytes of the x staging: the x planes (two for f32 x), then the block
// sums and exponents of x.
__host__ __device__ inline size_t xlds_bytes(int nblk, bool hl) {
    return (size_t)(nblk + 5) * XB * 4 * (hl ? 2 : 1) + (size_t)((nblk + 1) & ~1) * 8;
}

// The fp4 variant (F4) stages x as e4m3 pieces: per Q2 block, 8 chunks of 16
// elements x 4 piece slots of 16 bytes, then 64 bytes of padding (the block
// stride, 576 = 64 mod 256, puts the four blocks of a step on different LDS
// banks); the block sums and scale exponents follow.
constexpr int F4_BLK = 576;
__host__ __device__ inline size_t xlds_bytes_f4(int nblk) {
    return (size_t)(nblk + 5) * F4_BLK + (size_t)((nblk + 1) & ~1) * 8;
}
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef short s16x2 __attribute__((ext_vector_type(2)));

// Operand dword m holds codes (PA[m], PA[m] + 4) of w (the device order:
// code i < 8 at bit 4i, 8 + i at 4i + 2, so codes a and a + 4 share a
// position in the two halves) at bit position POS[m] of its two f16 halves;
// the x pair it meets is pre-scaled by XSCALE[m] = 2^(8-POS[m]).
__device__ __forceinline__ void unpack_dword(uint32_t w, uint32_t (&t)[8]) {
    constexpr uint32_t M4 = 0x00300030u, M6 = 0x00C000C0u, M8 = 0x03000300u;
    const uint32_t u = w << 4, v = w >> 6;
    t[0] = u & M4;     // codes 0, 4 at bit 4
    t[1] = u & M6;     // codes 8, 12 at bit 6
    t[2] = w & M4;     // codes 1, 5 at bit 4
    t[3] = w & M6;     // codes 9, 13 at bit 6
    t[4] = w & M8;     // codes 2, 6 at bit 8
    t[5] = v & M4;     // codes 10, 14 at bit 4
    t[6] = v & M6;     // codes 3, 7 at bit 6
    t[7] = v & M8;     // codes 11, 15 at bit 8
}
__device__ constexpr int PA[8] = {0, 8, 1, 9, 2, 10, 3, 11};
__device__ constexpr float XSCALE[8] = {16.f, 4.f, 16.f, 4.f, 1.f, 16.f, 4.f, 1.f};

// Two f32 -> two f16 (RNE) in one dword.
__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
    return (uint32_t)gd_f2h(a) | ((uint32_t)gd_f2h(b) << 16);
}

// x values of one staging unit (4 NQ consecutive elements of one block).
// XT = 0: f16 x; 1: f32 x; 2: f32 residual h (+ delta partials) and the
// norm weight w, staged as x = (h + delta) * w at f32 precision (the row sums
// are scaled by 1/rms(h + delta)); 3: f32 o and the gate g (= w silu(z)) of
// a gated head norm, staged as x = f16(o rs g) with rs the 1/rms of o over
// its 128-element block (one head).
template <int XT, int NQ> struct XChunk;
template <int NQ> struct XChunk<0, NQ> { u32x4 h[NQ / 2]; };
template <int NQ> struct XChunk<1, NQ> { f32x4 f[NQ]; };
template <int NQ> struct XChunk<2, NQ> { f32x4 f[NQ], w[NQ], d[ND_UNROLL][NQ]; };
template <int NQ> struct XChunk<3, NQ> { f32x4 f[NQ], g[NQ]; };

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

// XT = 3 side task: advance the conv ring of channels 0 .. n-1, ring rows j
// at ring + j * stride (j < 3): row 0 <- row 1, row 1 <- row 2, row 2 <-
// src (the step that read the old rows has run before this launch).  Each
// workgroup takes a run of channels (ring null: none).
struct RingAdv {
    float *ring;
    const float *src;
    int n, stride;
};

// One GEMV: W (codes, scales) [R][K], x, y; the work split (sets per
// workgroup `per`, K split into nz ranges of ksteps steps, gx workgroups per
// range: workgroup (bx, bz) takes sets bx * per .. of range bz).  lmag[0] and
// lmag[1]: ceil(2^32 / L) for the steps L of a range before the last and of
// the last (0 where L <= 1), the item -> set quotient by multiply-high.
struct Task {
    const uint8_t *codes;
    const uint16_t *scales;
    const void *x;
    float *y;
    const float *bias;       // added to the rows of K range 0 (null: none)
    int K, R, nsets, per, ksteps, nz, gx;
    uint32_t lmag[2];
    NormIn nin;
    GluOut glu;
    RingAdv ring;
};

// ceil(2^32 / L) for 1 < L <= 128 (0 otherwise): with it, i / L is
// umulhi(i, magic) exactly for i < 2^16.
__host__ __device__ inline uint32_t item_magic(int L) {
    return L <= 1 ? 0u : (uint32_t)((0x100000000ull + (unsigned)L - 1) / (unsigned)L);
}

// op over the 8 lanes of each aligned group of 8, every lane getting the
// result: the two quad exchanges leave each quad's value in all its lanes,
// so the half-row mirror (lane i takes lane 7 - i, in the other quad) adds
// the other quad's value as an exchange with lane i ^ 4 would.
template <class Op> __device__ __forceinline__ float group8(float v, Op op) {
    v = op(v, gd_dpp<GD_DPP_XOR1>(v));
    v = op(v, gd_dpp<GD_DPP_XOR2>(v));
    return op(v, gd_dpp<GD_DPP_HALF_MIRROR>(v));
}
// op over the G (8 or 16) lanes of each aligned group: for 16, the row
// mirror then pairs each lane with one in the other half-row, whose lanes
// all hold that half's value.
template <int G, class Op> __device__ __forceinline__ float group(float v, Op op) {
    static_assert(G == 8 || G == 16, "lane groups of 8 or 16");
    v = group8(v, op);
    if constexpr (G == 16) v = op(v, gd_dpp<GD_DPP_MIRROR>(v));
    return v;
}

// The register ring of a wave: P tiles with their scales and item numbers.
struct Ring {
    u32x4 t[P][2];
    u32x2 sc[P];
    int it[P];
};

// Buffer resource over `bytes` bytes at p (raw: no stride).  Loads at an
// offset past the end return zeros without touching memory, which keeps
// every load of the main loop unconditional.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes,
                                             0x00020000);
}

// What one workgroup does of task t.
struct Geo {
    int s0, L, set_lo, npair, nset_wg, wsets, total, steps, bgroups, up_shift;
    uint32_t Lmag;
    int bz;
};

__device__ __forceinline__ Geo geometry(const Task &t, int bx, int bz) {
    Geo g;
    const int nblk = t.K >> 7;
    g.steps = (nblk + 3) >> 2;
    g.bgroups = (nblk + 15) >> 4;
    g.bz = bz;
    // K split z = bz: steps [s0, s1) of every set.  Item i is step s0 + i % L
    // of set i / L (set-major).
    g.s0 = g.bz * t.ksteps;
    const int s1 = min(g.steps, g.s0 + t.ksteps);
    g.L = max(0, s1 - g.s0);
    // Sets of this workgroup, numbered c = 0 .. nset_wg-1 in LDS and in the
    // item space; set c is set set_lo + c of W.  With SwiGLU, nsets counts
    // gate sets, c < npair are gate sets and the rest their up sets, set
    // set_lo + pair_sets + c - npair of W.
    g.set_lo = bx * t.per;
    g.npair = g.bz < t.nz ? max(0, min(t.per, t.nsets - g.set_lo)) : 0;
    g.nset_wg = t.glu.pair_sets ? 2 * g.npair : g.npair;
    g.wsets = t.glu.pair_sets ? t.glu.pair_sets + g.npair : g.npair;   // sets spanned in W
    g.total = g.nset_wg * g.L;                                         // items
    g.up_shift = t.glu.pair_sets ? t.glu.pair_sets - g.npair : 0;
    // Item i is set i / L: the quotient by multiply-high (exact for i < 2^16
    // and L <= 128, which the host guarantees), the magic from the host.
    g.Lmag = t.lmag[g.bz == t.nz - 1 ? 1 : 0];
    return g;
}

__device__ __forceinline__ int set_of(const Geo &g, int it) {
    return g.L <= 1 ? it : (int)__umulhi((uint32_t)it, g.Lmag);
}

// Loads of item `it`: its tile, and for the lanes of column 0 the scales of
// rows 4*rq .. 4*rq+3 of their block 4*s + kb (the other lanes load
// nothing).  The address arithmetic has no branch (the compiler's wait
// counting is exact only over straight-line loads): an item past the last
// gets the offset 0xfffff000, beyond every resource.
// F4: the loading lanes are those of piece 0 (lane % 4 == 0); lane l takes
// rows 4*(l/16) .. +3 of block 4s + (l/4) % 4.
template <bool F4>
__device__ __forceinline__ void issue(const Task &t, const Geo &g, int it, u32x4 (&cw)[2],
                                      u32x2 &sc) {
    const int lane = threadIdx.x & 63;
    const int j = lane & 3, rq = F4 ? lane >> 4 : (lane >> 2) & 3, kb = F4 ? (lane >> 2) & 3 : lane >> 4;
    const __amdgpu_buffer_rsrc_t trs =
            make_rsrc(t.codes + (size_t)g.set_lo * g.steps * 2048, (uint32_t)g.wsets * g.steps * 2048u);
    const __amdgpu_buffer_rsrc_t srs =
            make_rsrc(t.scales + (size_t)g.set_lo * g.bgroups * 256, (uint32_t)g.wsets * g.bgroups * 512u);
    auto pick = [](uint32_t off, uint32_t dead) { return (off & ~dead) | (dead & 0xfffff000u); };
    const int c = set_of(g, it), s = g.s0 + (it - c * g.L);
    const int ps = c + (c >= g.npair ? g.up_shift : 0);
    const uint32_t dead = (uint32_t)((g.total - 1 - it) >> 31);      // all ones past the end
    const uint32_t off = pick((uint32_t)(ps * g.steps + s) * 2048u + lane * 16, dead);
    cw[0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(trs, off, 0, CP_NT));
    cw[1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(trs, off + 1024, 0, CP_NT));
    const uint32_t si = (uint32_t)((ps * g.bgroups + (s >> 2)) * 16 + 4 * (s & 3) + kb) * 32 + 8 * rq;
    const uint32_t other = (uint32_t)-(int)(j != 0);
    sc = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(srs, pick(si, dead | other), 0, 0));
}

// Runs task t's share of workgroup (bx, bz).  lds: the dynamic LDS (x staging,
// then the item partials).  XT: 0 = f16 x, 1 = f32 x (hi + lo split), 2 =
// normalized residual (see XChunk).  KBP: item partials kept per Q2 block (4
// per row) in LDS, summed with the rest of the row at the end; otherwise
// summed across the block lanes first (needs 4x less LDS, for very long K).
// SE: x elements a thread stages (16, or 8 with the fp4 body: twice the
// threads share the staging, for K up to (1024/16 - 5) blocks).
// All 64 * NW threads of the workgroup must call it.
template <int XT, bool KBP, bool F4, int ND = 0, int SE = 16>
__device__ void run(const Task &t, int bx, int bz, uint32_t *lds) {
    static_assert(ND >= 0 && ND <= ND_UNROLL && (XT == 2 || ND == 0), "partials: fused input only");
    static_assert(SE == 16 || (SE == 8 && F4), "half-entry staging: fp4 body only");
    static_assert(XT != 3 || (F4 && SE == 16), "gated head norm: fp4 body, 16 a thread");
    constexpr int NQ = SE / 4;                            // f32x4 of x per staging unit
    constexpr int UPB = 128 / SE;                         // staging units per block
    constexpr int MT = 64 * NW;
    // x at f32 precision: f32 x, and the fused input's h' * w (whose 1/rms
    // scales the row sums instead).
    constexpr bool XF = XT == 1 || XT == 2;               // (XT = 3 stages f16 values)
    constexpr bool HL = XF && !F4;                        // x carried as f16 hi + lo
    constexpr int NJ = XF ? 4 : 3;                        // F4: e4m3 pieces of x
    __shared__ __align__(16) int next_item;               // next item to take
    __shared__ float ssr[NW];                             // XT = 2: per-wave sums of h'^2
    const Geo g = geometry(t, bx, bz);
    const int K = t.K, R = t.R;
    const int nblk = K >> 7;
    // LDS: x planes, block b at dword XB*b (64 pair dwords + 4 of padding, so
    // the blocks one load instruction reads start on different banks), then
    // zero blocks for the blocks of a short last step past K; per-block sum
    // and exponent of x (nblk rounded up to even, so that what follows is
    // 16-byte aligned); the row partials of every item.  F4: the e4m3 piece
    // blocks (F4_BLK bytes each) in place of the planes.
    const int xstride = (nblk + 5) * XB;                   // dwords per x plane
    uint32_t *xp = lds;                                    // hi (or f16) pairs
    uint32_t *xq = lds + xstride;                          // lo plane (f32 x only)
    float *sx = (float *)(lds + (F4 ? (nblk + 5) * (F4_BLK / 4) : (HL ? 2 : 1) * xstride));
    float *ex = sx + ((nblk + 1) & ~1);                    // [nblk] 2^(16+e_b); F4: E8M0 byte
    float *part = ex + ((nblk + 1) & ~1);                  // [items][4 blocks if KBP][16 rows]
    uint8_t *xsb = (uint8_t *)lds;                         // F4 piece blocks

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // Lane l holds row l%16 of Q2 block l/16 of a step (the tile order); as
    // a 4x4x4 MFMA lane it is row / column j = l%4 of MFMA block l/4, which
    // covers rows 4*rq .. 4*rq+3 (rq = l/4 % 4) of Q2 block kb = l/16.
    const int j = lane & 3, rq = (lane >> 2) & 3, kb = lane >> 4;
    float *y = t.y + (size_t)g.bz * R;
    const int L = g.L, s0 = g.s0, set_lo = g.set_lo, npair = g.npair, total = g.total;
    // x blocks of this workgroup's K range (all of x unless K is split):
    // blocks xb0 .. xb0 + nbx - 1, staged from LDS block 0.
    const int xb0 = 4 * s0, nbx = max(0, min(nblk, 4 * (s0 + L)) - xb0);

    // Staging unit e = (block e/UPB, elements SE (e%UPB) ..): its x loads are
    // issued before the tile prefetch, so waiting for them leaves the tiles
    // in flight.
    const int nstage = (nbx + 5) * UPB;
    // Entries past the last x block (the zero blocks, and threads with no
    // entry) read past the end of x: zeros, without a memory access.
    const NormIn &nin = t.nin;
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(t.x, (uint32_t)K * (XT ? 4u : 2u));
    const __amdgpu_buffer_rsrc_t drs =
            make_rsrc(nin.delta, nin.nd ? (uint32_t)((nin.nd - 1) * nin.dstride + K) * 4u : 0u);
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(nin.w, XT == 2 ? (uint32_t)K * 4u : 0u);
    const __amdgpu_buffer_rsrc_t grs = make_rsrc(nin.delta, XT == 3 ? (uint32_t)K * 4u : 0u);
    // Element offset of staging unit e (K: a unit past the last x block).
    auto entry_off = [&](int e) { return e < nbx * UPB ? (xb0 + e / UPB) * 128 + SE * (e % UPB) : K; };
    // Dwords 4q .. 4q+3 of partial z of the entry at off; entries past K
    // (off == K) must read zeros (at z * dstride + K lies the next partial),
    // and so does a partial past nd: an offset outside the resource.
    auto dload = [&](int off, int z, int q, bool live) {
        return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                drs, live && off < K ? (uint32_t)((z * nin.dstride + off) * 4 + 16 * q) : 0xfffff000u,
                0, 0));
    };
    // Issues the loads of entry e only (no arithmetic, so that every load of
    // the entry is in flight before the first wait).
    auto load_x = [&](int e) {
        const int off = entry_off(e);
        XChunk<XT, NQ> c;
        if constexpr (XT == 0) {
#pragma unroll
            for (int q = 0; q < NQ / 2; q++)
                c.h[q] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, off * 2 + 16 * q, 0, 0));
        } else {
#pragma unroll
            for (int q = 0; q < NQ; q++)
                c.f[q] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, off * 4 + 16 * q, 0, 0));
            if constexpr (XT == 2) {
                // The first ND partials are loaded here, unconditionally and in
                // flight with h and w (summing them as they arrive, in a loop
                // over nd, waited for each load before issuing the next).
                // Partials past ND are loaded where they are summed.
#pragma unroll
                for (int z = 0; z < ND; z++)
#pragma unroll
                    for (int q = 0; q < NQ; q++) c.d[z][q] = dload(off, z, q, true);
#pragma unroll
                for (int q = 0; q < NQ; q++)
                    c.w[q] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(wrs, off * 4 + 16 * q, 0, 0));
            }
            if constexpr (XT == 3) {
#pragma unroll
                for (int q = 0; q < NQ; q++)
                    c.g[q] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(grs, off * 4 + 16 * q, 0, 0));
            }
        }
        return c;
    };
    // Waves with no staging entry issue no x loads: a load instruction
    // costs the CU's texture path about as much with every lane past the
    // end (zeros, no memory access) as with live lanes (measured: eight
    // such b128 loads per thread added about 1 us to a launch).
    // Every use of xc below is under the same wave-uniform condition, so the
    // idle waves' copy stays undefined and the branch joins without copies
    // (a zero-initialized copy made the loading waves wait for x there).
    const bool xwave = wave * 64 < nstage;
    // The bias of this thread's row in the first pass of the row sums at the
    // end (K range 0 only), requested with x so its latency is hidden.
    const __amdgpu_buffer_rsrc_t brs = make_rsrc(t.bias, t.bias && g.bz == 0 ? (uint32_t)R * 4u : 0u);
    auto bias_at = [&](int row) {
        return __builtin_amdgcn_raw_buffer_load_b32(brs, (uint32_t)row * 4u, 0, 0);
    };
    // Ring slot p starts with item p * NW + wave; each later item is taken
    // from the workgroup counter when a slot frees up.  One tile goes out
    // before the staging, the rest of the ring after it, so x (needed first)
    // does not queue behind the whole grid's prefetch.
    Ring rg;
#pragma unroll
    for (int p = 0; p < P; p++) rg.it[p] = p * NW + wave;
    uint32_t b0;
    // After x (loads complete in issue order, so x issued after the tiles
    // would only arrive behind them): the bias and the first tile.
    auto head = [&]() {
        b0 = bias_at(set_lo * 16 + (threadIdx.x >> 2));
        __builtin_amdgcn_sched_barrier(0);
        issue<F4>(t, g, rg.it[0], rg.t[0], rg.sc[0]);
        __builtin_amdgcn_sched_barrier(0);
    };
    // Every use of xc below is under the same wave-uniform condition, so the
    // idle waves' copy stays undefined and the branch joins without copies
    // (a zero-initialized copy made the loading waves wait for x there).
    // The bias and first tile are requested inside each branch, so that
    // work on x the compiler moves up into the loading branch still comes
    // after them.
    XChunk<XT, NQ> xc;
    if (xwave) {
        xc = load_x(threadIdx.x);
        __builtin_amdgcn_sched_barrier(0);
        head();
    } else {
        head();
    }
    if (threadIdx.x == 0) next_item = NW * P;
    // XT = 3: this workgroup's share of the conv ring advance, loaded now
    // (without a branch: channels outside the share read outside the
    // resources) and stored at the end.
    int rch = -1;
    float rv[3] = {0.f, 0.f, 0.f};
    if constexpr (XT == 3) {
        const RingAdv &ra = t.ring;
        const int nwg = t.gx * t.nz, share = (ra.n + nwg - 1) / nwg;
        const int c = (bz * t.gx + bx) * share + (int)threadIdx.x;
        const bool mine = ra.ring && (int)threadIdx.x < share && c < ra.n;
        const __amdgpu_buffer_rsrc_t rrs = make_rsrc(ra.ring, ra.ring ? (uint32_t)(3 * ra.stride) * 4u : 0u);
        const __amdgpu_buffer_rsrc_t srs = make_rsrc(ra.src, ra.ring ? (uint32_t)ra.n * 4u : 0u);
        const uint32_t o = mine ? (uint32_t)c * 4u : 0xfffff000u;
        rv[0] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rrs, mine ? o + (uint32_t)ra.stride * 4u : o, 0, 0));
        rv[1] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rrs, mine ? o + (uint32_t)ra.stride * 8u : o, 0, 0));
        rv[2] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(srs, o, 0, 0));
        rch = mine ? c : -1;
    }

    // Stage x: pair p = 8i + k of block b holds (x[b,16i+PA[k]], x[b,16i+PA[k]+4]) *
    // XSCALE[k] * 2^-e_b.  Thread (b, i) forms the 8 pairs of x[16i ..
    // 16i+15] in registers and writes them as 32 bytes; the block's sum and
    // max|x| come from 8-lane shuffles.  e_b = 0 unless max|x| >= 2048.
    auto stage = [&](const int e, const XChunk<XT, NQ> &xc) {
        // Block bb, 16-element chunk i, half hf8 of it (SE = 8).
        const int bb = e / UPB, sub = e % UPB;
        const int i = SE == 16 ? sub : sub >> 1, hf8 = SE == 16 ? 0 : sub & 1;
        float sum = 0.f, amax = 0.f;
        f32x4 f[NQ];
        if constexpr (XT == 3) {
            // The gated head norm (GDN.swift:113-115): the block's sum of
            // squares over its lane group, then each o rs g rounded to f16
            // as the f16 path stages it.
            float ssu = 0.f;
#pragma unroll
            for (int q = 0; q < NQ; q++)
#pragma unroll
                for (int j = 0; j < 4; j++) ssu += xc.f[q][j] * xc.f[q][j];
            const float ssb = group<UPB>(ssu, [](float a, float b) { return a + b; });
            const float rsh = 1.0f / sqrtf(ssb / 128.0f + nin.eps);
#pragma unroll
            for (int q = 0; q < NQ; q++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    f[q][j] = gd_h2f(gd_f2h(xc.f[q][j] * rsh * xc.g[q][j]));
        } else if constexpr (XT == 0) {
#pragma unroll
            for (int q = 0; q < 2 * NQ; q++) {
                const uint32_t d = xc.h[q >> 2][q & 3];
                f[q >> 1][2 * (q & 1)] = gd_h2f((uint16_t)(d & 0xffff));
                f[q >> 1][2 * (q & 1) + 1] = gd_h2f((uint16_t)(d >> 16));
            }
        } else {
#pragma unroll
            for (int q = 0; q < NQ; q++) f[q] = xc.f[q];
        }
#pragma unroll
        for (int q = 0; q < NQ; q++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                sum += f[q][j];
                amax = fmaxf(amax, fabsf(f[q][j]));
            }
        sum = group<UPB>(sum, [](float a, float b) { return a + b; });
        amax = group<UPB>(amax, [](float a, float b) { return fmaxf(a, b); });
        if constexpr (F4) {
            // x = 2^e (p0 + p1/16 + p2/256 [+ p3/4096]), e4m3 pieces with
            // max|x| 2^-e in [128, 256): p0 = e4m3(x 2^-e), each later piece
            // the e4m3 of 16 times what is left.  Piece j of the chunk goes
            // to slot j as 16 bytes in element order (the order the masked
            // code dwords give the weights).  The block's sum is that of the
            // pieces, so d (sum c x - sum x) cancels where c = 1.
            const int fe = (int)((__float_as_uint(amax) >> 23) & 0xff) - 127;
            const int eb = amax > 0.f ? min(120, max(-114, fe - 7)) : 0;
            // Piece jj is e4m3(r / 2^(eb - 4 jj)) of what the earlier pieces
            // leave, r, and leaves r - piece * 2^(eb - 4 jj) (exact): the
            // scaled conversions (which divide by, and multiply back by, the
            // power of two of their f32 scale; measured) do the scaling, so
            // r stays in x's own units.
            float sj[4];
#pragma unroll
            for (int jj = 0; jj < 4; jj++) sj[jj] = __uint_as_float((uint32_t)(127 + eb - 4 * jj) << 23);
            float tsum = 0.f;      // f32 x: what the pieces leave out
            u32x4 pc[4];
#pragma unroll
            for (int dw = 0; dw < NQ; dw++) {
                uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
                for (int hf = 0; hf < 2; hf++) {
                    // Bytes 2hf, 2hf+1 of dword dw: elements 4dw + 2hf, +1.
                    float a = f[dw][2 * hf], b = f[dw][2 * hf + 1];
#pragma unroll
                    for (int jj = 0; jj < NJ; jj++) {
                        const s16x2 o = __builtin_bit_cast(s16x2, w[jj]);
                        w[jj] = __builtin_bit_cast(uint32_t,
                                                   hf ? __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(o, a, b, sj[jj], true)
                                                      : __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(o, a, b, sj[jj], false));
                        // f16 x: three pieces hold it exactly (bar elements
                        // 2^-14 of the block's max), so the last needs no
                        // remainder.
                        if (XF || jj < NJ - 1) {
                            const f32x2 pv = hf ? __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w[jj], sj[jj], true)
                                                : __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w[jj], sj[jj], false);
                            a -= pv[0];
                            b -= pv[1];
                        }
                    }
                    if (XF) tsum += a + b;
                }
#pragma unroll
                for (int jj = 0; jj < 4; jj++) pc[jj][dw] = w[jj];
            }
            if (XF) {
                tsum = group<UPB>(tsum, [](float a, float b) { return a + b; });
            }
            if (e < nstage) {
                uint8_t *dst = xsb + bb * F4_BLK + 64 * i;
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    if constexpr (SE == 16) *(u32x4 *)(dst + 16 * jj) = pc[jj];
                    else *(u32x2 *)(dst + 16 * jj + 8 * hf8) = u32x2{pc[jj][0], pc[jj][1]};
                }
                if (i == 7 && hf8 == 0) {   // the padding: read as zeros by the idle lanes
                    u32x4 *pad = (u32x4 *)(xsb + bb * F4_BLK + 512);
#pragma unroll
                    for (int jj = 0; jj < 4; jj++) pad[jj] = u32x4{0u, 0u, 0u, 0u};
                }
                if (sub == 0 && bb < nbx) {
                    // sum of the pieces: sum x less what they leave out
                    sx[bb] = XF ? sum - tsum : sum;
                    ((int *)ex)[bb] = 127 + eb;
                }
            }
            return;
        }
        // amax < 2^(E-126) for f32 exponent field E; amax * 16 * 2^-eb < 2^15.
        const int eb = min(111, max(0, (int)((__float_as_uint(amax) >> 23) & 0xff) - 137));
        const float down = __uint_as_float((uint32_t)(127 - eb) << 23);    // 2^-eb
        u32x4 p0, p1, q0, q1;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            // pair k = (x[16i + PA[k]], x[16i + PA[k] + 4])
            const int ea = PA[k], eb = PA[k] + 4;
            const float xa = f[ea >> 2][ea & 3] * down, xb = f[eb >> 2][eb & 3] * down;
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
            if (i == 0 && bb < nbx) {
                sx[bb] = sum;
                ex[bb] = __uint_as_float((uint32_t)(127 + 16 + eb) << 23);   // 2^(16+eb)
            }
        }
    };
    // The first unit is straight-line code after the tile prefetch, so its
    // wait for x leaves the tiles in flight; further units (K long enough
    // that (K/128 + 5) * 128/SE > threads) follow in a loop.
    if constexpr (XT == 2) {
        // RMSNorm(h') * w with h' = h + delta: x = h' * w is staged as it is
        // (f32, four pieces) and the row sums are scaled by 1/rms(h') at the
        // end, so no barrier for the sum of squares stands between the x
        // loads and the staging: each wave's share goes to ssr here and is
        // read after the staging barrier.  One unit per thread (the host
        // checks), units past K load zeros.  Workgroup 0 keeps h' for the
        // next residual add.
        float ss = 0.f;
        if (xwave) {
            const int xoff = entry_off(threadIdx.x);
#pragma unroll
            for (int q = 0; q < NQ; q++) {
                // h + ((0 + p0) + p1 ...), the partials in order.
                f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int z = 0; z < ND; z++) d += xc.d[z][q];
                for (int z = ND; z < nin.nd; z++) d += dload(xoff, z, q, true);
                xc.f[q] += d;
                ss += xc.f[q][0] * xc.f[q][0] + xc.f[q][1] * xc.f[q][1] +
                      xc.f[q][2] * xc.f[q][2] + xc.f[q][3] * xc.f[q][3];
            }
            ss = gd_wave_sum(ss);
        }
        if (lane == 0) ssr[wave] = ss;
        if (bx == 0 && bz == 0 && nin.hout && threadIdx.x < nbx * UPB) {
            const uint32_t ho = (uint32_t)entry_off(threadIdx.x) * 4u;
            const __amdgpu_buffer_rsrc_t hrs = make_rsrc(nin.hout, (uint32_t)K * 4u);
#pragma unroll
            for (int q = 0; q < NQ; q++)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, xc.f[q]), hrs,
                                                       ho + 16 * q, 0, 0);
        }
        if (xwave) {
#pragma unroll
            for (int q = 0; q < NQ; q++) xc.f[q] *= xc.w[q];
        }
    }
    if (xwave) stage(threadIdx.x, xc);
    if constexpr (XT != 2)
        for (int e = threadIdx.x + MT; e < nstage; e += MT) stage(e, load_x(e));
#pragma unroll
    for (int p = 1; p < P; p++) issue<F4>(t, g, rg.it[p], rg.t[p], rg.sc[p]);
    __syncthreads();

    // One item (set c, step s): the four Q2 blocks 4s .. 4s+3 of 16 rows.
    // Every lane reads x of its own block kb, so the four columns of an
    // MFMA block hold the same products (only column 0 is used; a lane
    // group of one kb reads one address, which the LDS broadcasts).
    // Accumulator chains: f16 x uses two, f32 x two for hi and two for lo.
    auto step = [&](const int it, u32x4 (&tile)[2], u32x2 &sc) {
        const int c = set_of(g, it), s = s0 + (it - c * L);
        if constexpr (F4) {
            // v_mfma_scale_f32_16x16x128_f8f6f4, A = fp4 weights, B = e4m3 x.
            // A lane l holds row l%16 and K 32*(l/16) .. +31 of an MFMA,
            // which this tile order makes Q2 block l/16 of the step: MFMA m
            // takes code dwords 2m, 2m+1 (codes 32m .. 32m+31 of the block,
            // in order: the device order interleaves a dword's two halves by
            // nibble), each c in the low two bits of a nibble, i.e. the e2m1
            // value c/2 (scale 2 restores c).  B column n =
            // 4q + jp holds piece jp of block q's x and is zero elsewhere,
            // so C[row][4q + jp] sums block q alone.  B lane l (column l%16)
            // holds K 16*(l/16) .. +15 in bytes 0-15 and 64 + 16*(l/16) ..
            // +15 in bytes 16-31: its data is chunk 2m + (l/16)%2 of block
            // q, in the low half for q < 2 and the high half for q >= 2, and
            // only where q%2 == (l/16)/2; the other half (and lanes jp >= NJ)
            // read a zero region placed on other banks.  The B scale of lane
            // l (column l%16, K block l/16) is 2^(e_q - 4 jp) where l/16 is q.
            const int q = (lane >> 2) & 3, jp = lane & 3, G = lane >> 4;
            const int blk = 4 * (s - s0) + q;           // staged (local) block
            const bool act = (q & 1) == (G >> 1) && jp < NJ;
            const uint32_t zb = (uint32_t)((nbx + 3) * F4_BLK + 255) & ~255u;
            const uint32_t dat = (uint32_t)(blk * F4_BLK + ((G & 1) * 4 + jp) * 16);
            const uint32_t zer = zb + (uint32_t)((((q + (G & 1)) & 3) * 64) + jp * 16);
            const uint32_t alo = act && q < 2 ? dat : zer, ahi = act && q >= 2 ? dat : zer;
            const int bj = min(blk, nbx - 1);
            const int ev = ((const int *)ex)[bj];
            const int sb = G == q ? ev - 4 * jp : 127;
            constexpr uint32_t M = 0x33333333u;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int m = 0; m < 4; m++) {
                const uint32_t w0 = tile[m >> 1][2 * (m & 1)], w1 = tile[m >> 1][2 * (m & 1) + 1];
                const i32x8 a = {(int)(w0 & M), (int)((w0 >> 2) & M), (int)(w1 & M),
                                 (int)((w1 >> 2) & M), 0, 0, 0, 0};
                const u32x4 lo = *(const u32x4 *)(xsb + alo + m * 128);
                const u32x4 hi = *(const u32x4 *)(xsb + ahi + m * 128);
                const i32x8 b = {(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
                                 (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
                acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, acc, 4, 0, 0, 128, 0, sb);
            }
            // Lane l holds rows 4G + v, column l%16: sum the pieces (the
            // quad), then d (x . c - sum x) for block q.
            auto quad = [](float v) {
                v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));
                return v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false));
            };
            const bool live = blk < nbx;
            const float sxq = sx[bj];
            const float dsc[4] = {gd_h2f((uint16_t)(sc[0] & 0xffff)), gd_h2f((uint16_t)(sc[0] >> 16)),
                                  gd_h2f((uint16_t)(sc[1] & 0xffff)), gd_h2f((uint16_t)(sc[1] >> 16))};
            f32x4 r;
#pragma unroll
            for (int v = 0; v < 4; v++) r[v] = quad(acc[v]);   // every lane: DPP reads its quad
#pragma unroll
            for (int v = 0; v < 4; v++) r[v] = live ? dsc[v] * (r[v] - sxq) : 0.f;
            if constexpr (KBP) {
                if (jp == 0) *(f32x4 *)(part + (it * 4 + q) * 16 + 4 * G) = r;
            } else {
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    r[v] += __shfl_xor(r[v], 4, 64);
                    r[v] += __shfl_xor(r[v], 8, 64);
                }
                if (lane == 16 * G) *(f32x4 *)(part + it * 16 + 4 * G) = r;
            }
            return;
        }
        // MFMA block mb = lane/4 multiplies rows 4*rq .. 4*rq+3 of Q2 block
        // 4s + kb by four K values.  Blocks past the last (a short final
        // step) read zero-staged x and give zero products.
        const int blk = 4 * (s - s0) + kb;               // staged (local) block
        const u32x4 *src = (const u32x4 *)(xp + blk * XB);
        const u32x4 *srq = (const u32x4 *)(xq + blk * XB);
        f32x4 acc[4];
#pragma unroll
        for (int d = 0; d < 8; d++) {
            uint32_t tt[8];
            unpack_dword(tile[d >> 2][d & 3], tt);
#pragma unroll
            for (int q = 0; q < 2; q++) {
                // Pairs 4q .. 4q+3 of chunk d: two MFMAs of four K values.
                const u32x4 bx = src[2 * d + q];
                const f16x4 a0 = __builtin_bit_cast(f16x4, u32x2{tt[4 * q], tt[4 * q + 1]});
                const f16x4 a1 = __builtin_bit_cast(f16x4, u32x2{tt[4 * q + 2], tt[4 * q + 3]});
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
        const bool live = blk < nbx;
        const int bj = min(blk, nbx - 1);
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
    while (rg.it[0] < total) {
#pragma unroll
        for (int p = 0; p < P; p++) {
            int gi = 0;
            if (lane == 0) gi = atomicAdd(&next_item, 1);
            if (rg.it[p] < total) step(rg.it[p], rg.t[p], rg.sc[p]);
            rg.it[p] = __builtin_amdgcn_readfirstlane(gi);
            issue<F4>(t, g, rg.it[p], rg.t[p], rg.sc[p]);
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
    const GluOut &glu = t.glu;
    // XT = 2: the row sums of W (h' * w) times 1/rms(h'), the sum of squares
    // added over the waves in wave order.
    float rs = 1.f;
    if constexpr (XT == 2) {
        float tot = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) tot += ssr[w];
        rs = 1.0f / sqrtf(tot / (float)K + nin.eps);
    }
    const __amdgpu_buffer_rsrc_t yrs = make_rsrc(y, (uint32_t)R * 4u);
    const __amdgpu_buffer_rsrc_t ors = make_rsrc(glu.out, glu.pair_sets ? (uint32_t)glu.pair_sets * 32u : 0u);
    const int nrow = (glu.pair_sets ? npair : g.nset_wg) * 16;
    for (int base = 0; base < nrow * 4; base += MT) {   // uniform trip count: shuffles stay whole
        const int i = (base + threadIdx.x) >> 2, q = threadIdx.x & 3;
        const bool ok = i < nrow;
        const int c = ok ? i >> 4 : 0, r = i & 15;
        if (glu.pair_sets) {
            const float gv = rs * combine(ok ? quarter(c, r, q) : 0.f);
            const float u = rs * combine(ok ? quarter(npair + c, r, q) : 0.f);
            if (ok && q == 0)
                __builtin_amdgcn_raw_buffer_store_b16(gd_f2h(gd_silu(gv) * u), ors,
                                                      (uint32_t)(set_lo * 16 + i) * 2u, 0, 0);
        } else {
            // Rows past R read bias zero (outside the resource).
            const uint32_t bv = base == 0 ? b0 : bias_at(set_lo * 16 + i);
            const float v = rs * combine(ok ? quarter(c, r, q) : 0.f) + __uint_as_float(bv);
            if (ok && q == 0 && set_lo * 16 + i < R)
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), yrs,
                                                      (uint32_t)(set_lo * 16 + i) * 4u, 0, 0);
        }
    }
    if constexpr (XT == 3) {
        if (rch >= 0) {
            float *rg0 = t.ring.ring;
            rg0[rch] = rv[0];
            rg0[t.ring.stride + rch] = rv[1];
            rg0[2 * t.ring.stride + rch] = rv[2];
        }
    }
}

}  // namespace gemv
