// Chunked (WY / UT) Gated DeltaNet prefill on the matrix cores.
//
// The reference runs prefill as a token-serial scan (gdn_scan_batch2,
// LLM/metal/Kernels.metal:1570-1625; GDN.step, LLM/src/SIMD/GDN.swift:71-109).
// Unrolling that recurrence over a chunk of L tokens with state S0 gives the
// closed form of LLM/src/CoreML/MtpRollback.swift:3-12:
//   S_m = e^{G_m} S0 + sum_{s<=m} e^{G_m - G_s} k_s delta_s^T,  G = inclusive
// cumulative sum of g inside the chunk.  Writing delta for all L tokens at once:
//   A[t][s] = beta_t e^{G_t - G_s} (k_t . k_s)        (s < t, else 0)
//   T = (I + A)^-1                                   (unit lower triangular)
//   W = T diag(beta e^G) K,  U = T diag(beta) V,  delta = U - W S0
//   O = qScale (diag(e^G) Q S0) + P delta,  P[t][s] = qScale e^{G_t-G_s} (q_t . k_s), s <= t
//   S_L = e^{G_L} S0 + K^T diag(e^{G_L - G}) delta
// Every exponent is a difference G_t - G_s <= 0 (or G <= 0), so no factor
// exceeds 1 and nothing overflows however long the decay runs.
//
// MI355X design.  Every product above runs on v_mfma_f32_16x16x32_f16 with
// f32 accumulation.  Operands that are f32 -- S, delta, T, beta e^G k,
// beta v, P, and q, k, v themselves when they arrive as f32 -- are split into
// hi = f16(x) and lo = f16(x - hi) and multiplied as hi*hi + hi*lo + lo*hi
// (about 22 significant bits), so the result tracks the f32 recurrence of the
// reference's prefill scan.  f16 q, k, v (BASELINE's prefill inputs) are used
// as they are.
//   gdn_prep  (value head, chunk): K K^T and Q K^T on the matrix cores give A
//             and P; I + A is inverted in 16 x 16 blocks (diagonal blocks by
//             forward substitution, one wave each, then the blocks below in
//             levels of block products, all 256 threads); then W = T X and
//             U = T Y (the UT transform) on the matrix cores.  The chunks are
//             independent.
//   gdn_scan  (value head, 16 columns of S): walks the chunks in order:
//             delta = U - W S, S <- e^{G_L} S + K^T (e^{G_L-G} delta) on one
//             group of four waves (the serial chain, S in its registers),
//             O = qScale e^G (Q S) + P delta one chunk behind on a second
//             group, off the chain.  Value columns of S are independent,
//             which is what splits the serial part across workgroups.
// Workspace per (head, chunk) unit, CP = max(32, C) rows (rows past the
// chunk's tokens are zero): W hi/lo [CP][128] f16, U [CP][128] f32, P hi/lo
// [CP][CP] f16, K^T (hi, and lo for f32 k) [128][CP] f16, G [CP] f32.
#include "gd_internal.h"

namespace {

constexpr int DK = 128;          // key size handled
constexpr int DV = 128;          // value size handled
constexpr int NCOL = 16;         // value columns of S per scan workgroup
constexpr int PADK = DK + 8;     // LDS row of 128 f16 plus 16 bytes (bank spread)

__device__ __forceinline__ f32x4 mfma(const f16x8 &a, const f16x8 &b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// x = hi + lo, hi = f16(x), lo = f16(x - hi).
__device__ __forceinline__ void split8(const float (&x)[8], f16x8 &hi, f16x8 &lo) {
#pragma unroll
    for (int e = 0; e < 8; e++) {
        hi[e] = (f16)x[e];
        lo[e] = (f16)(x[e] - (float)hi[e]);
    }
}

// hi*hi + hi*lo + lo*hi, accumulated into c.
__device__ __forceinline__ f32x4 mfma3(const f16x8 &ah, const f16x8 &al, const f16x8 &bh,
                                       const f16x8 &bl, f32x4 c) {
    c = mfma(ah, bh, c);
    c = mfma(ah, bl, c);
    return mfma(al, bh, c);
}

// Eight consecutive activations as loaded (f16 or f32), converted by cvt8:
// keeping them raw lets a prefetch stay in flight until the values are used.
template <typename IO> struct Raw8;
template <> struct Raw8<uint16_t> { u32x4 v; };
template <> struct Raw8<float> { f32x4 a, b; };
template <typename IO>
__device__ __forceinline__ Raw8<IO> load_raw8(const void *base, int64_t idx) {
    Raw8<IO> r;
    if constexpr (sizeof(IO) == 2) {
        r.v = *(const u32x4 *)((const uint16_t *)base + idx);
    } else {
        const f32x4 *p = (const f32x4 *)((const float *)base + idx);
        r.a = p[0];
        r.b = p[1];
    }
    return r;
}
// As f16, zero when !ok.
template <typename IO>
__device__ __forceinline__ f16x8 cvt8(const Raw8<IO> &r, bool ok) {
    f16x8 h;
    if constexpr (sizeof(IO) == 2) {
        h = __builtin_bit_cast(f16x8, ok ? r.v : u32x4{0, 0, 0, 0});
    } else {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            h[e] = ok ? (f16)r.a[e] : (f16)0.0f;
            h[4 + e] = ok ? (f16)r.b[e] : (f16)0.0f;
        }
    }
    return h;
}

// hi/lo split of the eight f32 values of a raw load (zeros when !ok).
template <typename IO>
__device__ __forceinline__ void split_raw8(const Raw8<IO> &r, bool ok, f16x8 &hi, f16x8 &lo) {
    float x[8];
    if constexpr (sizeof(IO) == 4) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            x[e] = ok ? r.a[e] : 0.f;
            x[4 + e] = ok ? r.b[e] : 0.f;
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; e++) x[e] = 0.f;      // not used for f16 inputs
    }
    split8(x, hi, lo);
}

struct Work {
    f16 *Wh, *Wl;     // [u][CP][DK]
    float *U;         // [u][CP][DV]
    f16 *Ph, *Pl;     // [u][CP][CP]
    f16 *KT;          // [u][DK][CP]
    f16 *KTl;         // [u][DK][CP], f32 k only: k - f16(k)
    float *G;         // [u][CP]
    f16 *Qh, *Ql;     // [u][CP][DK], f32 q only: q split as prep forms it, for the scan
};

struct PrepArgs {
    const void *q, *k, *v;
    int64_t q_stride, k_stride, v_stride;
    const float *g, *beta;
    Work w;
    int64_t T;
    int nV, nK, C, nchunks;
    float qScale;
};

template <int CP, typename IO>
__global__ __launch_bounds__(256) void gdn_prep(PrepArgs a) {
    // f32 q, k, v: hi/lo pairs.  The lo halves of K and Q are needed only
    // until A and P are formed, so they share the space of Xh and Xl, which
    // are first written after that (and X, Y are then formed from the f32
    // inputs themselves, re-read from L2).
    constexpr bool HL = sizeof(IO) == 4;
    __shared__ __attribute__((aligned(16))) f16 Ks[CP][PADK];
    __shared__ __attribute__((aligned(16))) f16 QVs[CP][PADK];     // Q, later V
    __shared__ __attribute__((aligned(16))) f16 Xh[DK][CP + 8], Xl[DK][CP + 8];
    __shared__ __attribute__((aligned(16))) f16 Yh[DV][CP + 8], Yl[DV][CP + 8];
    static_assert(sizeof(Xh) >= sizeof(Ks), "K lo must fit where Xh lives");
    f16 (*Kl)[PADK] = reinterpret_cast<f16 (*)[PADK]>(&Xh[0][0]);
    f16 (*Ql)[PADK] = reinterpret_cast<f16 (*)[PADK]>(&Xl[0][0]);
    __shared__ __attribute__((aligned(16))) float Af[CP][CP + 4];
    __shared__ __attribute__((aligned(16))) float Tf[CP][CP + 4];
    __shared__ __attribute__((aligned(16))) float Ms[(CP / 16 - 1) * 256];   // block products
    __shared__ float Gs[CP], Bs[CP], BEs[CP];               // G, beta, beta e^G

    // Workgroup b runs on XCD b % 8.  When the units divide by 8, XCD x takes
    // the contiguous units x * units/8 .., so a head's chunks are written into
    // the L2 of the XCD whose scan workgroups read them (the scan deals each
    // head's column slices to one XCD in the same order).
    const int units = (int)gridDim.x;
    const int ub = units % 8 == 0 ? (int)((blockIdx.x & 7) * (units >> 3) + (blockIdx.x >> 3))
                                  : (int)blockIdx.x;
    const int hv = ub / a.nchunks, c = ub % a.nchunks;
    const int hk = hv % a.nK;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t t0 = (int64_t)c * a.C;
    const int L = (int)min((int64_t)a.C, a.T - t0);
    const int64_t u = (int64_t)hv * a.nchunks + c;
    const int lr = lane & 15, kg = lane >> 4;

    // Rows of K and Q (and V, kept in registers until Q is done): thread e
    // handles 8 consecutive elements of row e / 16.
    // Every load goes out before any is converted (rows past the chunk read
    // token 0 and are zeroed at conversion): loads under a branch, converted
    // on arrival, waited for one by one.
    constexpr int NE = CP * DK / 8 / 256;                   // entries per thread
    f16x8 vreg[NE];
    Raw8<IO> rk[NE], rq[NE], rv[NE];
#pragma unroll
    for (int n = 0; n < NE; n++) {
        const int e = tid + 256 * n, t = e >> 4, i8 = (e & 15) * 8;
        const int64_t tok = t0 + (t < L ? t : 0);
        rk[n] = load_raw8<IO>(a.k, tok * a.k_stride + (int64_t)hk * DK + i8);
        rq[n] = load_raw8<IO>(a.q, tok * a.q_stride + (int64_t)hk * DK + i8);
        rv[n] = load_raw8<IO>(a.v, tok * a.v_stride + (int64_t)hv * DV + i8);
    }
#pragma unroll
    for (int n = 0; n < NE; n++) {
        const int e = tid + 256 * n, t = e >> 4, i8 = (e & 15) * 8;
        const bool ok = t < L;
        if constexpr (HL) {
            f16x8 h, l;
            split_raw8<IO>(rk[n], ok, h, l);
            *(f16x8 *)&Ks[t][i8] = h;
            *(f16x8 *)&Kl[t][i8] = l;
            split_raw8<IO>(rq[n], ok, h, l);
            *(f16x8 *)&QVs[t][i8] = h;
            *(f16x8 *)&Ql[t][i8] = l;
            // The scan's output pass reads this split instead of splitting
            // q again at every chunk (rows past the chunk: zeros).
            const size_t qi = ((size_t)u * CP + t) * DK + i8;
            *(f16x8 *)&a.w.Qh[qi] = h;
            *(f16x8 *)&a.w.Ql[qi] = l;
        } else {
            *(f16x8 *)&Ks[t][i8] = cvt8<IO>(rk[n], ok);
            *(f16x8 *)&QVs[t][i8] = cvt8<IO>(rq[n], ok);
            vreg[n] = cvt8<IO>(rv[n], ok);
        }
    }
    if (wave == 0) {
        // Inclusive cumulative gate inside the chunk (wave prefix sum); rows
        // past L keep G[L-1] and get beta = 0.
        float gv = lane < L ? a.g[(t0 + lane) * a.nV + hv] : 0.f;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const float o = __shfl_up(gv, off, 64);
            if (lane >= off) gv += o;
        }
        if (lane < CP) {
            const float bt = lane < L ? a.beta[(t0 + lane) * a.nV + hv] : 0.f;
            Gs[lane] = gv;
            Bs[lane] = bt;
            BEs[lane] = bt * __expf(gv);
        }
    }
    __syncthreads();

    // K K^T -> A (s < t) and Q K^T -> P (s <= t), lower tiles on the matrix
    // cores; P's upper tiles are written as zeros.
    constexpr int NB = CP / 16;
    // Unrolled: a wave's tiles are independent, so their LDS reads, MFMA
    // chains and stores can overlap.
#pragma unroll
    for (int tile = wave; tile < 2 * NB * NB; tile += 4) {
        const bool isP = tile >= NB * NB;
        const int tt = isP ? tile - NB * NB : tile;
        const int ti = tt / NB, si = tt % NB;
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
        if (si <= ti) {
#pragma unroll
            for (int k0 = 0; k0 < DK; k0 += 32) {
                const f16x8 av = isP ? *(const f16x8 *)&QVs[ti * 16 + lr][k0 + kg * 8]
                                     : *(const f16x8 *)&Ks[ti * 16 + lr][k0 + kg * 8];
                const f16x8 bv = *(const f16x8 *)&Ks[si * 16 + lr][k0 + kg * 8];
                if constexpr (HL) {
                    const f16x8 al = isP ? *(const f16x8 *)&Ql[ti * 16 + lr][k0 + kg * 8]
                                         : *(const f16x8 *)&Kl[ti * 16 + lr][k0 + kg * 8];
                    const f16x8 bl = *(const f16x8 *)&Kl[si * 16 + lr][k0 + kg * 8];
                    acc = mfma3(av, al, bv, bl, acc);
                } else {
                    acc = mfma(av, bv, acc);
                }
            }
        }
        const int s = si * 16 + lr;
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int t = ti * 16 + kg * 4 + v;
            const float dec = __expf(Gs[t] - Gs[s]);          // factor in (0, 1]
            if (!isP) {
                Af[t][s] = (s < t && t < L) ? Bs[t] * dec * acc[v] : 0.f;
            } else {
                const float p = (s <= t && t < L) ? a.qScale * dec * acc[v] : 0.f;
                const f16 ph = (f16)p;
                const size_t pi = ((size_t)u * CP + t) * CP + s;
                a.w.Ph[pi] = ph;
                a.w.Pl[pi] = (f16)(p - (float)ph);
            }
        }
    }
    __syncthreads();
    // V replaces Q (f16 inputs; f32 ones are re-read for Y below).
    if constexpr (!HL) {
#pragma unroll
        for (int n = 0; n < NE; n++) {
            const int e = tid + 256 * n, t = e >> 4, i8 = (e & 15) * 8;
            *(f16x8 *)&QVs[t][i8] = vreg[n];
        }
    }
    __syncthreads();

    // T = (I + A)^-1 in 16 x 16 blocks (A is strictly lower triangular).
    // Diagonal blocks first, wave w inverting block w by forward
    // substitution with lane s < 16 holding its column s: T[t][s] =
    // -sum_{m<t} A[t][m] T[m][s] (T[m][s] = 0 for m < s, T[s][s] = 1);
    // blocks above the diagonal are zero.
    if (wave < NB && lane < 16) {
        const int b0 = wave * 16, s = lane;
        float Tc[16];
#pragma unroll
        for (int m = 0; m < 16; m++) Tc[m] = m == s ? 1.f : 0.f;
#pragma unroll
        for (int t = 1; t < 16; t++) {
            float acc = 0.f;
#pragma unroll
            for (int m = 0; m < t; m++) acc = fmaf(Af[b0 + t][b0 + m], Tc[m], acc);
            Tc[t] = t == s ? 1.f : -acc;
        }
#pragma unroll
        for (int m = 0; m < 16; m++) Tf[b0 + m][b0 + s] = Tc[m];
    }
    for (int e = tid; e < CP * CP; e += 256) {
        const int r = e / CP, cc = e % CP;
        if ((cc >> 4) > (r >> 4)) Tf[r][cc] = 0.f;
    }
    __syncthreads();
    // Blocks below the diagonal by distance d = i - j, each level from the
    // ones before it: T_ij = -T_ii (sum_{k=j}^{i-1} A_ik T_kj).  Thread e
    // takes element (r, cc) of block i = d + e / 256.
    for (int d = 1; d < NB; d++) {
        for (int e = tid; e < (NB - d) * 256; e += 256) {
            const int i = d + (e >> 8), j = i - d, r = (e >> 4) & 15, cc = e & 15;
            float m = 0.f;
            for (int k = j; k < i; k++)
#pragma unroll
                for (int q = 0; q < 16; q++)
                    m = fmaf(Af[i * 16 + r][k * 16 + q], Tf[k * 16 + q][j * 16 + cc], m);
            Ms[e] = m;
        }
        __syncthreads();
        for (int e = tid; e < (NB - d) * 256; e += 256) {
            const int i = d + (e >> 8), j = i - d, r = (e >> 4) & 15, cc = e & 15;
            const float *mb = Ms + (e & ~255);
            float t = 0.f;
#pragma unroll
            for (int q = 0; q < 16; q++) t = fmaf(Tf[i * 16 + r][i * 16 + q], mb[q * 16 + cc], t);
            Tf[i * 16 + r][j * 16 + cc] = -t;
        }
        __syncthreads();
    }
    // X^T = (diag(beta e^G) K)^T and Y^T = (diag(beta) V)^T, split, as the
    // B operands of T X and T Y, and K^T to the workspace for the scan's
    // state update (its A operand): entry (8 tokens s .. s+7, i), lanes
    // along i so that the row reads of K and V hit distinct banks.
    // f32 inputs: k and v come from global memory (the chunk was read moments
    // ago, so from L2), every load of an entry issued before any is used, at
    // clamped rows (rows past the chunk are zeroed on use).
    for (int e = tid; e < DK * (CP / 8); e += 256) {
        const int s8 = (e / DK) * 8, i = e % DK;
        float xv[8], yv[8];
        f16x8 kv, kl;
        if constexpr (HL) {
            float kf[8], vf[8];
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const int64_t tok = t0 + (s8 + q < L ? s8 + q : 0);
                kf[q] = ((const float *)a.k)[tok * a.k_stride + (int64_t)hk * DK + i];
                vf[q] = ((const float *)a.v)[tok * a.v_stride + (int64_t)hv * DV + i];
            }
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const int s = s8 + q;
                const float kk = s < L ? kf[q] : 0.f, vv = s < L ? vf[q] : 0.f;
                kv[q] = (f16)kk;
                kl[q] = (f16)(kk - (float)kv[q]);
                xv[q] = BEs[s] * kk;
                yv[q] = Bs[s] * vv;
            }
        } else {
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const int s = s8 + q;
                kv[q] = Ks[s][i];
                xv[q] = BEs[s] * (float)kv[q];
                yv[q] = Bs[s] * (float)QVs[s][i];
            }
        }
        f16x8 h, l;
        split8(xv, h, l);
        *(f16x8 *)&Xh[i][s8] = h;
        *(f16x8 *)&Xl[i][s8] = l;
        split8(yv, h, l);
        *(f16x8 *)&Yh[i][s8] = h;
        *(f16x8 *)&Yl[i][s8] = l;
        *(f16x8 *)&a.w.KT[((size_t)u * DK + i) * CP + s8] = kv;
        if constexpr (HL) *(f16x8 *)&a.w.KTl[((size_t)u * DK + i) * CP + s8] = kl;
    }
    if (tid < CP) a.w.G[(size_t)u * CP + tid] = Gs[tid];
    __syncthreads();

    // W = T X, U = T Y: wave w takes row block rb (of CP/16) for all 16
    // column tiles of W and U; T's rows are split once and reused.
    for (int rb = wave; rb < NB; rb += 4) {
        f16x8 th[CP / 32], tl[CP / 32];
#pragma unroll
        for (int ks = 0; ks < CP / 32; ks++) {
            float tv[8];
#pragma unroll
            for (int q = 0; q < 8; q++) tv[q] = Tf[rb * 16 + lr][ks * 32 + kg * 8 + q];
            split8(tv, th[ks], tl[ks]);
        }
        for (int ct = 0; ct < 16; ct++) {
            const bool isU = ct >= 8;
            const int ci = (ct & 7) * 16 + lr;          // column (key or value index)
            f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < CP / 32; ks++) {
                const int s0 = ks * 32 + kg * 8;
                const f16x8 bh = isU ? *(const f16x8 *)&Yh[ci][s0] : *(const f16x8 *)&Xh[ci][s0];
                const f16x8 bl = isU ? *(const f16x8 *)&Yl[ci][s0] : *(const f16x8 *)&Xl[ci][s0];
                acc = mfma3(th[ks], tl[ks], bh, bl, acc);
            }
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int t = rb * 16 + kg * 4 + v;
                const size_t idx = ((size_t)u * CP + t) * DK + ci;
                if (isU) {
                    a.w.U[idx] = acc[v];
                } else {
                    const f16 h = (f16)acc[v];
                    a.w.Wh[idx] = h;
                    a.w.Wl[idx] = (f16)(acc[v] - (float)h);
                }
            }
        }
    }
}

struct ScanArgs {
    const void *q;
    int64_t q_stride;
    Work w;
    float *S;
    void *o;
    int64_t o_stride;
    int64_t T;
    int nV, nK, C, nchunks;
    float qScale;
};

// The scan's workgroup is two groups of four waves.  The chain group walks the
// recurrence: per chunk delta = U - W S, then S <- e^{G_L} S + K^T (e^{G_L-G}
// delta), which is all the next chunk waits for.  The output group computes O
// = qScale e^G (Q S) + P delta one chunk behind, beside the chain: Q S while
// the chain updates S, P delta while it forms the next delta.  The split of S
// (hi/lo, the B operand of W S and Q S), delta and G are double-buffered in
// LDS by chunk parity, so neither group overwrites what the other still reads.
constexpr int SCAN_THREADS = 512;     // chain group: threads 0..255, output group 256..511

// The chain group's operands of one chunk, all independent of S, loaded one
// phase ahead of their use: W, U and G after delta, K^T after the update.
template <int CP, typename IO>
struct ChainRegs {
    float g;                              // G[tid] (tid < CP)
    f16x8 wh[DK / 32], wl[DK / 32];       // W rows 16*wave + lr
    float uv[NCOL / 16][4];               // U rows 16*wave + 4*kg + v, this lane's column
    f16x8 ka[2][CP / 32];                 // K^T rows 32*wave + 16*rt + lr
    f16x8 kal[sizeof(IO) == 4 ? 2 : 1][CP / 32];   // their lo halves (f32 k)
};

// The output group's operands of one chunk: Q and P.  f16 q is loaded raw
// (converted at use); f32 q as the hi/lo split prep stored.
template <int CP, typename IO>
struct OutRegs {
    Raw8<IO> qr[sizeof(IO) == 4 ? 1 : DK / 32];   // f16: Q row 16*wave + lr (row 0 past the chunk)
    f16x8 qh[sizeof(IO) == 4 ? DK / 32 : 1], ql[sizeof(IO) == 4 ? DK / 32 : 1];   // f32: the split
    f16x8 ph[CP / 32], pl[CP / 32];       // P row 16*wave + lr
};

template <int CP, typename IO, typename OT>
__global__ __launch_bounds__(SCAN_THREADS) void gdn_scan(ScanArgs a) {
    __shared__ __attribute__((aligned(16))) f16 Sh[2][NCOL][PADK], Sl[2][NCOL][PADK];  // S^T split
    __shared__ __attribute__((aligned(16))) f16 Dh[2][NCOL][CP + 8], Dl[2][NCOL][CP + 8];  // delta^T
    __shared__ __attribute__((aligned(16))) f16 Eh[NCOL][CP + 8], El[NCOL][CP + 8];  // decayed
    __shared__ float Gs[2][CP];

    constexpr int NCB = DV / NCOL;
    static_assert(NCB % 8 == 0, "the grid must split evenly over the 8 XCDs");
    static_assert(NCOL == 16, "one 16-column MFMA tile per lane group");
    // Workgroup b runs on XCD b % 8.  The NCB column slices of one head read
    // the same chunk operands (W, P, K^T, Q), so they are dealt to one XCD:
    // unit u = (b % 8) * (grid / 8) + b / 8, head u / NCB, so each chunk is
    // fetched into one L2 once instead of into every L2.
    const int u = (int)((blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3));
    const int hv = u / NCB, j0 = (u % NCB) * NCOL;
    const int hk = hv % a.nK;
    const int tid = threadIdx.x & 255, lane = tid & 63, wave = tid >> 6;
    // A wave's role as a scalar: the group branches below are jumps, so no
    // wave ever steps through another group's barriers with its lanes off.
    const int wbase = __builtin_amdgcn_readfirstlane((int)threadIdx.x);
    const bool chain = wbase < 256;
    const int lr = lane & 15, kg = lane >> 4;
    // A wave owns 16 chunk rows (with CP = 64 every wave does: a constant, so
    // no load below sits in a branch, which keeps the compiler's wait counts
    // exact).
    const bool rows = CP / 16 >= 4 || wave < CP / 16;
    const int tb = wave * 16;
    float *Sg = a.S + (size_t)hv * DK * DV;
    auto unit = [&](int c) { return (size_t)hv * a.nchunks + min(c, a.nchunks - 1); };

    // Chain group: S entries (rows 32*wave + 16*rt + 4*kg + v, column lr)
    // live in registers, as the state update's accumulators lay them out.
    // A group's operands for chunk c + 1 are loaded as soon as chunk c has
    // used them: W, U and G after delta, K^T after the update, P after
    // P delta, Q after Q S.  (Two register sets, loading two chunks ahead,
    // measured slower.)
    float st[2][4];
    auto loadW = [&](int c, ChainRegs<CP, IO> &k) {
        const size_t un = unit(c);
        k.g = a.w.G[un * CP + min(tid, CP - 1)];        // used by tid < CP
        if (rows) {
#pragma unroll
            for (int ks = 0; ks < DK / 32; ks++) {
                const size_t wi = (un * CP + tb + lr) * DK + ks * 32 + kg * 8;
                k.wh[ks] = *(const f16x8 *)&a.w.Wh[wi];
                k.wl[ks] = *(const f16x8 *)&a.w.Wl[wi];
            }
#pragma unroll
            for (int ct = 0; ct < NCOL / 16; ct++)
#pragma unroll
                for (int v = 0; v < 4; v++)
                    k.uv[ct][v] = a.w.U[(un * CP + tb + kg * 4 + v) * DV + j0 + ct * 16 + lr];
        }
    };
    auto loadK = [&](int c, ChainRegs<CP, IO> &k) {
        const size_t un = unit(c);
#pragma unroll
        for (int rt = 0; rt < 2; rt++)
#pragma unroll
            for (int ks = 0; ks < CP / 32; ks++) {
                const size_t ki = (un * DK + wave * 32 + rt * 16 + lr) * CP + ks * 32 + kg * 8;
                k.ka[rt][ks] = *(const f16x8 *)&a.w.KT[ki];
                if constexpr (sizeof(IO) == 4) k.kal[rt][ks] = *(const f16x8 *)&a.w.KTl[ki];
            }
    };
    // Split this lane's S entries into the hi/lo planes of buffer b.
    auto split_own = [&](int b) {
#pragma unroll
        for (int rt = 0; rt < 2; rt++) {
            const int i = wave * 32 + rt * 16 + kg * 4;
            f16 h[4], l[4];
#pragma unroll
            for (int v = 0; v < 4; v++) {
                h[v] = (f16)st[rt][v];
                l[v] = (f16)(st[rt][v] - (float)h[v]);
            }
            *(f16x4 *)&Sh[b][lr][i] = f16x4{h[0], h[1], h[2], h[3]};
            *(f16x4 *)&Sl[b][lr][i] = f16x4{l[0], l[1], l[2], l[3]};
        }
    };
    // One chunk of the chain: its two barriers, delta, the state update.
    auto chain_chunk = [&](int c, ChainRegs<CP, IO> &k) {
        const int b = c & 1;
        __syncthreads();
        // delta = U - W S (rows 16*wave ..), then delta^T and its decayed
        // copy e^{G_L - G_t} delta^T, split, to LDS.
        const float gl = Gs[b][CP - 1];                 // G of the chunk's last token
        if (rows) {
            const int j = lr;
            f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < DK / 32; ks++) {
                const int i0 = ks * 32 + kg * 8;
                acc = mfma3(k.wh[ks], k.wl[ks], *(const f16x8 *)&Sh[b][j][i0],
                            *(const f16x8 *)&Sl[b][j][i0], acc);
            }
            f16 dh[4], dl[4], eh[4], el[4];
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int t = tb + kg * 4 + v;
                const float d = k.uv[0][v] - acc[v];
                const float ed = expf(gl - Gs[b][t]) * d;
                dh[v] = (f16)d;
                dl[v] = (f16)(d - (float)dh[v]);
                eh[v] = (f16)ed;
                el[v] = (f16)(ed - (float)eh[v]);
            }
            const int tq = tb + kg * 4;
            *(f16x4 *)&Dh[b][j][tq] = f16x4{dh[0], dh[1], dh[2], dh[3]};
            *(f16x4 *)&Dl[b][j][tq] = f16x4{dl[0], dl[1], dl[2], dl[3]};
            *(f16x4 *)&Eh[j][tq] = f16x4{eh[0], eh[1], eh[2], eh[3]};
            *(f16x4 *)&El[j][tq] = f16x4{el[0], el[1], el[2], el[3]};
        }
        loadW(c + 1, k);
        __syncthreads();
        // S <- e^{G_L} S + K^T (e^{G_L - G} delta): rows 32*wave .. +31,
        // then its split into the other buffer and chunk c+1's G.
        const float decay = expf(gl);
#pragma unroll
        for (int rt = 0; rt < 2; rt++) {
            const int j = lr;
            f32x4 acc;
#pragma unroll
            for (int v = 0; v < 4; v++) acc[v] = decay * st[rt][v];
#pragma unroll
            for (int ks = 0; ks < CP / 32; ks++) {
                const int s0 = ks * 32 + kg * 8;
                if constexpr (sizeof(IO) == 4) {
                    acc = mfma3(k.ka[rt][ks], k.kal[rt][ks], *(const f16x8 *)&Eh[j][s0],
                                *(const f16x8 *)&El[j][s0], acc);
                } else {
                    acc = mfma(k.ka[rt][ks], *(const f16x8 *)&Eh[j][s0], acc);
                    acc = mfma(k.ka[rt][ks], *(const f16x8 *)&El[j][s0], acc);
                }
            }
#pragma unroll
            for (int v = 0; v < 4; v++) st[rt][v] = acc[v];
        }
        split_own(b ^ 1);
        if (tid < CP) Gs[b ^ 1][tid] = k.g;                // chunk c + 1's G
        loadK(c + 1, k);
    };

    // Output group.
    f32x4 oacc = f32x4{0.f, 0.f, 0.f, 0.f};
    auto loadQ = [&](int c, OutRegs<CP, IO> &o) {
        c = min(c, a.nchunks - 1);
        const int64_t t0 = (int64_t)c * a.C;
        const int L = (int)min((int64_t)a.C, a.T - t0);
        if (rows) {
            const int tr = tb + lr;
            const bool rok = tr < L;
            if constexpr (sizeof(IO) == 4) {
                const size_t un = unit(c);
#pragma unroll
                for (int ks = 0; ks < DK / 32; ks++) {
                    const size_t qi = (un * CP + tr) * DK + ks * 32 + kg * 8;
                    o.qh[ks] = *(const f16x8 *)&a.w.Qh[qi];
                    o.ql[ks] = *(const f16x8 *)&a.w.Ql[qi];
                }
            } else {
#pragma unroll
                for (int ks = 0; ks < DK / 32; ks++)
                    o.qr[ks] = load_raw8<IO>(a.q, (t0 + (rok ? tr : 0)) * a.q_stride +
                                                      (int64_t)hk * DK + ks * 32 + kg * 8);
            }
        }
    };
    auto loadP = [&](int c, OutRegs<CP, IO> &o) {
        const size_t un = unit(c);
        if (rows) {
#pragma unroll
            for (int ks = 0; ks < CP / 32; ks++) {
                const size_t pi = (un * CP + tb + lr) * CP + ks * 32 + kg * 8;
                o.ph[ks] = *(const f16x8 *)&a.w.Ph[pi];
                o.pl[ks] = *(const f16x8 *)&a.w.Pl[pi];
            }
        }
    };
    // O of chunk c, first part: qScale e^{G_t} (Q S_c) into oacc.
    auto out_qs = [&](int c, const OutRegs<CP, IO> &o) {
        const int b = c & 1;
        const int64_t t0 = (int64_t)c * a.C;
        const int L = (int)min((int64_t)a.C, a.T - t0);
        if (rows) {
            const int j = lr;
            f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < DK / 32; ks++) {
                const int i0 = ks * 32 + kg * 8;
                if constexpr (sizeof(IO) == 4) {
                    acc = mfma3(o.qh[ks], o.ql[ks], *(const f16x8 *)&Sh[b][j][i0],
                                *(const f16x8 *)&Sl[b][j][i0], acc);
                } else {
                    const f16x8 qa = cvt8<IO>(o.qr[ks], tb + lr < L);
                    acc = mfma(qa, *(const f16x8 *)&Sh[b][j][i0], acc);
                    acc = mfma(qa, *(const f16x8 *)&Sl[b][j][i0], acc);
                }
            }
#pragma unroll
            for (int v = 0; v < 4; v++) acc[v] *= a.qScale * expf(Gs[b][tb + kg * 4 + v]);
            oacc = acc;
        }
    };
    // Second part: + P delta_c, then the chunk's output rows (rows t >= L
    // lie past the bounds-checked resource: their stores are dropped).
    auto out_pd = [&](int c, const OutRegs<CP, IO> &o) {
        const int b = c & 1;
        const int64_t t0 = (int64_t)c * a.C;
        const int L = (int)min((int64_t)a.C, a.T - t0);
        const __amdgpu_buffer_rsrc_t ors = gd_rsrc((OT *)a.o + t0 * a.o_stride,
                                                   (uint32_t)L * (uint32_t)a.o_stride * sizeof(OT));
        const uint32_t obase = (uint32_t)hv * DV + j0;
        if (rows) {
            const int j = lr;
            f32x4 acc = oacc;
#pragma unroll
            for (int ks = 0; ks < CP / 32; ks++) {
                const int s0 = ks * 32 + kg * 8;
                acc = mfma3(o.ph[ks], o.pl[ks], *(const f16x8 *)&Dh[b][j][s0],
                            *(const f16x8 *)&Dl[b][j][s0], acc);
            }
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const uint32_t oo =
                        ((uint32_t)(tb + kg * 4 + v) * (uint32_t)a.o_stride + obase + j) * sizeof(OT);
                if constexpr (sizeof(OT) == 4)
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[v]), ors, oo, 0, 0);
                else
                    __builtin_amdgcn_raw_buffer_store_b16(gd_f2h(acc[v]), ors, oo, 0, 0);
            }
        }
    };
    // One chunk of the output group: its two barriers, P delta of chunk
    // c - 1, Q S of chunk c.
    auto out_chunk = [&](int c, OutRegs<CP, IO> &o) {
        __syncthreads();
        if (c > 0) {
            out_pd(c - 1, o);
            loadP(c, o);
        }
        __syncthreads();
        out_qs(c, o);
        loadQ(c + 1, o);
    };

    // Each group runs its own loop over the chunks (one merged loop would join
    // the groups' load streams at every phase, and the compiler's wait counts
    // would then wait for loads a group does not need).  Both loops pass the
    // same barriers: two per chunk and one after the last, 2 * nchunks + 1.
    if (chain) {
        ChainRegs<CP, IO> k;
        // Prologue: S_0 into registers, its split into buffer 0, G of chunk 0.
#pragma unroll
        for (int rt = 0; rt < 2; rt++)
#pragma unroll
            for (int v = 0; v < 4; v++)
                st[rt][v] = Sg[(size_t)(wave * 32 + rt * 16 + kg * 4 + v) * DV + j0 + lr];
        loadW(0, k);
        loadK(0, k);
        split_own(0);
        if (tid < CP) Gs[0][tid] = k.g;
        for (int c = 0; c < a.nchunks; c++) chain_chunk(c, k);
        __syncthreads();
#pragma unroll
        for (int rt = 0; rt < 2; rt++)
#pragma unroll
            for (int v = 0; v < 4; v++)
                Sg[(size_t)(wave * 32 + rt * 16 + kg * 4 + v) * DV + j0 + lr] = st[rt][v];
    } else {
        OutRegs<CP, IO> o;
        loadQ(0, o);
        loadP(0, o);
        for (int c = 0; c < a.nchunks; c++) out_chunk(c, o);
        __syncthreads();
        out_pd(a.nchunks - 1, o);
    }
}

template <int CP>
int launch(gd_ctx *ctx, const PrepArgs &pa, const ScanArgs &sa, int io_dtype, int o_dtype) {
    const unsigned units = (unsigned)(pa.nV * pa.nchunks);
    if (io_dtype == GD_F32)
        hipLaunchKernelGGL((gdn_prep<CP, float>), dim3(units), dim3(256), 0, ctx->stream, pa);
    else
        hipLaunchKernelGGL((gdn_prep<CP, uint16_t>), dim3(units), dim3(256), 0, ctx->stream, pa);
    GD_LAUNCHED(ctx, "gdn_prep");
    const dim3 grid((unsigned)(sa.nV * (DV / NCOL)));
#define GD_SCAN(IO, OT) \
    hipLaunchKernelGGL((gdn_scan<CP, IO, OT>), grid, dim3(SCAN_THREADS), 0, ctx->stream, sa)
    if (io_dtype == GD_F32) { if (o_dtype == GD_F32) GD_SCAN(float, float); else GD_SCAN(float, uint16_t); }
    else { if (o_dtype == GD_F32) GD_SCAN(uint16_t, float); else GD_SCAN(uint16_t, uint16_t); }
#undef GD_SCAN
    GD_LAUNCHED(ctx, "gdn_scan");
    return GD_OK;
}

}  // namespace

int gd_ctx_workspace(gd_ctx *ctx, size_t bytes, void **out);

namespace {

// Checks the arguments; *bytes receives the scratch the call needs (0 for T = 0).
int prefill_check(gd_ctx *ctx, const char *fn, int64_t T, int nV, int nK, int dk, int dv,
                  const void *q, int64_t q_stride, const void *k, int64_t k_stride,
                  const void *v, int64_t v_stride, int io_dtype, const float *g,
                  const float *beta, float *S, void *o, int64_t o_stride, int o_dtype, int C,
                  size_t *bytes) {
    GD_REQUIRE(ctx, q && k && v && g && beta && S && o, "%s: null pointer", fn);
    GD_REQUIRE(ctx, dk == DK && dv == DV, "%s: dk=%d dv=%d (takes 128/128)", fn, dk, dv);
    GD_REQUIRE(ctx, C == 16 || C == 32 || C == 64, "%s: chunk %d not 16/32/64", fn, C);
    GD_REQUIRE(ctx, nV > 0 && nK > 0 && T >= 0, "%s: nV=%d nK=%d T=%lld", fn, nV, nK,
               (long long)T);
    GD_REQUIRE(ctx, io_dtype == GD_F32 || io_dtype == GD_F16, "%s: bad io dtype", fn);
    GD_REQUIRE(ctx, o_dtype == GD_F32 || o_dtype == GD_F16, "%s: bad o dtype", fn);
    GD_REQUIRE(ctx, q_stride >= (int64_t)nK * dk && k_stride >= (int64_t)nK * dk &&
                        v_stride >= (int64_t)nV * dv && o_stride >= (int64_t)nV * dv,
               "%s: strides smaller than a token row", fn);
    // A chunk's output rows are stored through one 32-bit buffer range.
    GD_REQUIRE(ctx, o_stride <= (1 << 24), "%s: o_stride %lld above 2^24", fn,
               (long long)o_stride);
    // Rows are read 8 elements at a time.
    const int vec = io_dtype == GD_F16 ? 8 : 4;
    const int esz = io_dtype == GD_F16 ? 2 : 4;
    GD_REQUIRE(ctx, q_stride % 8 == 0 && k_stride % 8 == 0 && v_stride % 8 == 0 &&
                        ((uintptr_t)q % (vec * esz)) == 0 && ((uintptr_t)k % (vec * esz)) == 0 &&
                        ((uintptr_t)v % (vec * esz)) == 0,
               "%s: q/k/v rows must be 8-element strided and %d-byte aligned", fn, vec * esz);
    *bytes = 0;
    if (T == 0) return GD_OK;
    const size_t units = (size_t)nV * (size_t)((T + C - 1) / C);
    const size_t CP = C < 32 ? 32 : C;
    const size_t nkt = io_dtype == GD_F32 ? 2 : 1;
    // Wh, Wl; U; Ph, Pl; K^T (hi, lo); G; Q (hi, lo: f32 io) -- the layout
    // prefill_run carves.
    *bytes = units * (2 * CP * DK * 2 + CP * DV * 4 + 2 * CP * CP * 2 + nkt * DK * CP * 2 +
                      CP * 4 + (nkt - 1) * 2 * CP * DK * 2);
    return GD_OK;
}

// Launches prep + scan with their per-(head, chunk) operands in ws (at least
// the bytes prefill_check computed).  Every byte of ws the scan reads is
// written by prep in the same call, so ws needs no clearing.
int prefill_run(gd_ctx *ctx, void *ws, int64_t T, int nV, int nK, const void *q,
                int64_t q_stride, const void *k, int64_t k_stride, const void *v,
                int64_t v_stride, int io_dtype, const float *g, const float *beta, float *S,
                void *o, int64_t o_stride, int o_dtype, float qScale, int C) {
    const int nchunks = (int)((T + C - 1) / C);
    const int CP = C < 32 ? 32 : C;
    const size_t units = (size_t)nV * nchunks;
    const size_t wbytes = units * CP * DK * 2;          // each of Wh, Wl
    const size_t ubytes = units * CP * DV * 4;
    const size_t pbytes = units * CP * CP * 2;          // each of Ph, Pl
    const size_t kbytes = units * DK * CP * 2;          // K^T hi; lo too for f32 k
    const size_t nkt = io_dtype == GD_F32 ? 2 : 1;
    uint8_t *p = (uint8_t *)ws;
    Work w;
    w.Wh = (f16 *)p;            p += wbytes;
    w.Wl = (f16 *)p;            p += wbytes;
    w.U = (float *)p;           p += ubytes;
    w.Ph = (f16 *)p;            p += pbytes;
    w.Pl = (f16 *)p;            p += pbytes;
    w.KT = (f16 *)p;            p += kbytes;
    w.KTl = nkt == 2 ? (f16 *)p : nullptr;
    p += (nkt - 1) * kbytes;
    w.G = (float *)p;           p += units * CP * 4;
    w.Qh = nkt == 2 ? (f16 *)p : nullptr;
    p += (nkt - 1) * wbytes;
    w.Ql = nkt == 2 ? (f16 *)p : nullptr;

    PrepArgs pa{q, k, v, q_stride, k_stride, v_stride, g, beta, w, T, nV, nK, C, nchunks, qScale};
    ScanArgs sa{q, q_stride, w, S, o, o_stride, T, nV, nK, C, nchunks, qScale};
    return CP == 64 ? launch<64>(ctx, pa, sa, io_dtype, o_dtype)
                    : launch<32>(ctx, pa, sa, io_dtype, o_dtype);
}

// Scratch of gd_gdn_prefill_noalloc: a file-scope device array, so the entry
// needs no allocation.  Each device holds its own copy until the process
// ends; host code reaches it only through the address hipGetSymbolAddress
// returns for the current device (kept per context), never through the
// array's name.  Every call on a device shares it.
constexpr size_t PREFILL_SCRATCH_BYTES = GD_GDN_PREFILL_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[PREFILL_SCRATCH_BYTES];

}  // namespace

int gd_prefill_scratch_attach(gd_ctx *ctx) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) {
        ctx->prefill_scratch = nullptr;
        return gd_hip_fail(ctx, e, "prefill scratch: hipGetSymbolAddress");
    }
    ctx->prefill_scratch = p;
    return GD_OK;
}

extern "C" int gd_gdn_prefill(gd_ctx *ctx, int64_t T, int nV, int nK, int dk, int dv,
                              const void *q, int64_t q_stride, const void *k, int64_t k_stride,
                              const void *v, int64_t v_stride, int io_dtype, const float *g,
                              const float *beta, float *S, void *o, int64_t o_stride,
                              int o_dtype, float qScale, int C) {
    GD_CHECK_CTX(ctx);
    size_t bytes = 0;
    int rc = prefill_check(ctx, "gd_gdn_prefill", T, nV, nK, dk, dv, q, q_stride, k, k_stride, v,
                           v_stride, io_dtype, g, beta, S, o, o_stride, o_dtype, C, &bytes);
    if (rc || T == 0) return rc;
    void *ws = nullptr;
    if ((rc = gd_ctx_workspace(ctx, bytes, &ws))) return rc;
    return prefill_run(ctx, ws, T, nV, nK, q, q_stride, k, k_stride, v, v_stride, io_dtype, g,
                       beta, S, o, o_stride, o_dtype, qScale, C);
}

extern "C" int gd_gdn_prefill_noalloc(gd_ctx *ctx, int64_t T, int nV, int nK, int dk, int dv,
                                      const void *q, int64_t q_stride, const void *k,
                                      int64_t k_stride, const void *v, int64_t v_stride,
                                      int io_dtype, const float *g, const float *beta, float *S,
                                      void *o, int64_t o_stride, int o_dtype, float qScale,
                                      int C) {
    GD_CHECK_CTX(ctx);
    size_t bytes = 0;
    int rc = prefill_check(ctx, "gd_gdn_prefill_noalloc", T, nV, nK, dk, dv, q, q_stride, k,
                           k_stride, v, v_stride, io_dtype, g, beta, S, o, o_stride, o_dtype, C,
                           &bytes);
    if (rc || T == 0) return rc;
    GD_REQUIRE(ctx, bytes <= PREFILL_SCRATCH_BYTES,
               "gd_gdn_prefill_noalloc: needs %zu bytes of scratch for nV=%d x %lld chunks of "
               "%d, above its fixed %zu (GD_GDN_PREFILL_SCRATCH_BYTES); split T or use "
               "gd_gdn_prefill", bytes, nV, (long long)((T + C - 1) / C), C,
               PREFILL_SCRATCH_BYTES);
    GD_REQUIRE(ctx, ctx->prefill_scratch != nullptr,
               "gd_gdn_prefill_noalloc: the scratch array's device address could not be "
               "looked up when the context was created");
    return prefill_run(ctx, ctx->prefill_scratch, T, nV, nK, q, q_stride, k, k_stride, v,
                       v_stride, io_dtype, g, beta, S, o, o_stride, o_dtype, qScale, C);
}

extern "C" int gd_gdn_scan_batch(gd_ctx *ctx, const float *convOutN, int keyDim, int valueDim,
                                 int convDim, const float *gN, const float *betaN, float *S,
                                 float *oN, int nV, int nK, int dS, float qScale, int64_t N) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, convOutN && gN && betaN && S && oN, "gd_gdn_scan_batch: null pointer");
    GD_REQUIRE(ctx, keyDim == nK * dS && valueDim == nV * dS && convDim >= 2 * keyDim + valueDim,
               "gd_gdn_scan_batch: keyDim/valueDim/convDim inconsistent with nK, nV, dS");
    // The chunked prefill holds 128 x 128 states; other sizes take the
    // token-serial scan, as MetalEnc.gdnScanBatch falls back to
    // gdn_scan_batch where gdn_scan_batch2 does not fit (MetalEnc.swift:760-777).
    if (dS != 128)
        return gd_gdn_scan_batch_serial(ctx, convOutN, keyDim, valueDim, convDim, gN, betaN, S,
                                        oN, nV, nK, dS, qScale, N);
    return gd_gdn_prefill(ctx, N, nV, nK, dS, dS, convOutN, convDim, convOutN + keyDim, convDim,
                          convOutN + 2 * keyDim, convDim, GD_F32, gN, betaN, S, oN, valueDim,
                          GD_F32, qScale, 64);
}
