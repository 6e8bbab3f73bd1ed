/*
 * gd_oracle.c -- CPU restatement of the reference's Q2_0 + Gated DeltaNet
 * path.  TEST INFRASTRUCTURE ONLY: called by tests/ (as the parity checker)
 * and by bench.py's cpu_baseline leg; the product library never uses it.
 *
 * The reference is Swift (LLM/src/SIMD); it cannot be compiled on Linux, so
 * this file restates it in C, function by function, with the same f32
 * operation order where the order is the reference's.  Built with -O2 and no
 * -ffast-math so the order is kept.
 */
#define _GNU_SOURCE
#include "gd_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ LCG */

#define LCG_A 6364136223846793005ULL
#define LCG_C 1442695040888963407ULL
#define LCG_MIX 0x9E3779B97F4A7C15ULL

/* The LCG of MetalSelfTest.fill (MetalSelfTest.swift:12-21): s = seed + MIX;
 * per element s = s*A + C; bits = UInt32(s >> 33).  Those bits carry 31
 * significant bits, so the reference's Float(bits) / Float(UInt32.max) spans
 * only [0, 0.5) (its fill lands in [-1, 0)); these streams scale by 2^-31 so
 * u covers [0, 1).  Float(bits) * 2^-31 is exact scaling of a rounded value. */
void or_lcg_uniform(float *out, size_t n, uint64_t seed, float lo, float hi) {
    uint64_t s = seed + LCG_MIX;
    const float span = hi - lo;
    for (size_t i = 0; i < n; i++) {
        s = s * LCG_A + LCG_C;
        const float u = (float)(uint32_t)(s >> 33) * 0x1p-31f;
        out[i] = lo + span * u;
    }
}

/* Box-Muller over consecutive pairs of the same stream. */
static void normal_stream(size_t n, uint64_t seed, float mean, float sd, float *f,
                          uint16_t *h) {
    uint64_t s = seed + LCG_MIX;
    for (size_t i = 0; i < n; i += 2) {
        s = s * LCG_A + LCG_C;
        const uint32_t b1 = (uint32_t)(s >> 33);
        s = s * LCG_A + LCG_C;
        const uint32_t b2 = (uint32_t)(s >> 33);
        const float u1 = (float)((uint64_t)b1 + 1) * 0x1p-31f;
        const float u2 = (float)b2 * 0x1p-31f;
        const float r = sqrtf(-2.0f * logf(u1));
        const float a = 6.283185307179586f * u2;
        const float z0 = mean + sd * (r * cosf(a));
        const float z1 = mean + sd * (r * sinf(a));
        if (f) {
            f[i] = z0;
            if (i + 1 < n) f[i + 1] = z1;
        } else {
            h[i] = or_f2h(z0);
            if (i + 1 < n) h[i + 1] = or_f2h(z1);
        }
    }
}

void or_lcg_normal(float *out, size_t n, uint64_t seed, float mean, float sd) {
    normal_stream(n, seed, mean, sd, out, NULL);
}

void or_lcg_normal_f16(uint16_t *out, size_t n, uint64_t seed, float mean, float sd) {
    normal_stream(n, seed, mean, sd, NULL, out);
}

void or_lcg_q2_0(uint8_t *blocks, int64_t K, int64_t R, uint64_t seed, float lo, float hi) {
    const int64_t nb = K / 128;
    uint64_t s = seed + LCG_MIX;                 /* codes stream */
    uint64_t t = seed + 1 + LCG_MIX;             /* scales stream */
    const float span = hi - lo;
    for (int64_t r = 0; r < R; r++) {
        for (int64_t b = 0; b < nb; b++) {
            uint8_t *p = blocks + (r * nb + b) * 34;
            t = t * LCG_A + LCG_C;
            const float u = (float)(uint32_t)(t >> 33) * 0x1p-31f;
            const uint16_t d = or_f2h(lo + span * u);
            p[0] = (uint8_t)(d & 0xff);
            p[1] = (uint8_t)(d >> 8);
            memset(p + 2, 0, 32);
            for (int j = 0; j < 128; j++) {
                s = s * LCG_A + LCG_C;
                const uint32_t c = (uint32_t)(((uint64_t)(uint32_t)(s >> 33) * 3u) >> 31);
                p[2 + (j >> 2)] |= (uint8_t)(c << ((j & 3) * 2));
            }
        }
    }
}

/* ------------------------------------------------------------------ f16 */

float or_h2f(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    const int e = (h >> 10) & 0x1f;
    const uint32_t m = h & 0x3ff;
    float v;
    if (e == 0) v = ldexpf((float)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexpf((float)(m | 0x400), e - 25);
    uint32_t bits;
    memcpy(&bits, &v, 4);
    bits |= sign;
    memcpy(&v, &bits, 4);
    return v;
}

uint16_t or_f2h(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
    const uint32_t ax = x & 0x7fffffff;
    if (ax >= 0x7f800000) return (uint16_t)(sign | (ax > 0x7f800000 ? 0x7e00 : 0x7c00));
    if (ax >= 0x477ff000) return (uint16_t)(sign | 0x7c00);      /* rounds past 65504 */
    if (ax < 0x33000001) return sign;                           /* < half of min subnormal */
    int e = (int)(ax >> 23) - 127;
    uint32_t m = (ax & 0x7fffff) | 0x800000;
    int shift;                     /* bits dropped from the 24-bit significand */
    uint32_t base;
    if (e < -14) {                 /* subnormal result */
        shift = 13 + (-14 - e);
        base = 0;
    } else {
        shift = 13;
        base = (uint32_t)(e + 15) << 10;
        m &= 0x7fffff;             /* implicit bit carried through base */
    }
    uint32_t q = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1))) q++;
    return (uint16_t)(sign | (base + q));   /* a mantissa carry bumps the exponent */
}

/* ----------------------------------------------------------------- Q2_0 */

/* Quant.swift:15-30 */
void or_q2_0_dequant(const uint8_t *blocks, size_t n, float *out) {
    const size_t nb = n / 128;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *p = blocks + b * 34;
        const float d = or_h2f((uint16_t)(p[0] | (p[1] << 8)));
        for (int j = 0; j < 128; j++) {
            const int code = (p[2 + (j >> 2)] >> ((j & 3) << 1)) & 3;
            out[b * 128 + j] = (float)(code - 1) * d;
        }
    }
}

struct mv_job {
    const uint8_t *w;
    int64_t K, m0, m1;
    const float *x;
    float *out;
};

/* x with its bits cleared unless `bit` is set: adding it to a sum is the same
 * as adding x under `if (bit)`, since the sums below start at +0 and so are
 * never -0 (s + (+0) == s exactly for every other s). */
static inline float masked(float x, uint32_t bit) {
    uint32_t u;
    memcpy(&u, &x, 4);
    u &= 0u - bit;
    memcpy(&x, &u, 4);
    return x;
}

/* Quant.swift:53-73, one row: per block lo/hi/sy sums in weight order, then
 * acc += d * (lo + 2*hi - sy).  The conditional adds of the reference
 * (`if code & 1 { lo += x }`) are written as adds of masked values, which give
 * the same sums without a data-dependent branch per weight. */
static void *mv_rows(void *arg) {
    const struct mv_job *j = (const struct mv_job *)arg;
    const int64_t nblk = j->K / 128, rowBytes = nblk * 34;
    for (int64_t m = j->m0; m < j->m1; m++) {
        float acc = 0;
        const uint8_t *p = j->w + m * rowBytes;
        int64_t k = 0;
        for (int64_t b = 0; b < nblk; b++) {
            const float d = or_h2f((uint16_t)(p[0] | (p[1] << 8)));
            const uint8_t *qs = p + 2;
            float lo = 0, hi = 0, sy = 0;
            for (int jj = 0; jj < 128; jj++) {
                const uint32_t code = (qs[jj >> 2] >> ((jj & 3) << 1)) & 3;
                const float xv = j->x[k + jj];
                sy += xv;
                lo += masked(xv, code & 1);
                hi += masked(xv, code >> 1);
            }
            acc += d * (lo + 2 * hi - sy);
            p += 34;
            k += 128;
        }
        j->out[m] = acc;
    }
    return NULL;
}

static void run_jobs(void *(*fn)(void *), void *jobs, size_t job_size, int n) {
    pthread_t tid[256];
    if (n == 1) { fn(jobs); return; }
    for (int t = 0; t < n; t++) pthread_create(&tid[t], NULL, fn, (char *)jobs + t * job_size);
    for (int t = 0; t < n; t++) pthread_join(tid[t], NULL);
}

void or_q2_0_matvec(const uint8_t *w, int64_t K, int64_t M, const float *x, float *out,
                    int threads) {
    if (threads < 1) threads = 1;
    if (threads > M) threads = (int)(M > 0 ? M : 1);
    struct mv_job jobs[256];
    if (threads > 256) threads = 256;
    for (int t = 0; t < threads; t++) {
        jobs[t].w = w; jobs[t].K = K; jobs[t].x = x; jobs[t].out = out;
        jobs[t].m0 = M * t / threads;
        jobs[t].m1 = M * (t + 1) / threads;
    }
    run_jobs(mv_rows, jobs, sizeof jobs[0], threads);
}

/* ---- the same mat-vec for T tokens at once ---------------------------------
 * The reference CPU engine has no batched Q2_0 kernel: prefill is T separate
 * Q2_0.matvec calls (BonsaiEngine.swift:33-37).  or_q2_0_matmat computes
 * exactly those T results: each token's lo/hi/sy/acc sums are formed in
 * mv_rows's order, and only the lanes of a vector hold different tokens.  A
 * thread takes a range of rows and walks them block by block for one tile of
 * MM_TT tokens, so the tile's x slice of a block stays in L1. */
#define MM_TT 16
typedef float mm_vf __attribute__((vector_size(MM_TT * 4)));
typedef uint32_t mm_vu __attribute__((vector_size(MM_TT * 4)));

struct mm_job {
    const uint8_t *w;
    int64_t K, m0, m1, T, Tp;
    const float *xt;       /* [Tp/MM_TT][K][MM_TT], zero padded */
    float *acc;            /* [m1-m0][MM_TT] scratch */
    float *out;            /* [T][M] */
    int64_t M;
};

__attribute__((target_clones("avx512f", "avx2", "default")))
static void *mm_rows(void *arg) {
    const struct mm_job *j = (const struct mm_job *)arg;
    const int64_t nblk = j->K / 128, rowBytes = nblk * 34, nr = j->m1 - j->m0;
    for (int64_t t0 = 0; t0 < j->Tp; t0 += MM_TT) {
        const float *xt = j->xt + t0 * j->K;
        mm_vf *acc = (mm_vf *)j->acc;
        for (int64_t r = 0; r < nr; r++) acc[r] = (mm_vf){0};
        for (int64_t b = 0; b < nblk; b++) {
            const mm_vf *xb = (const mm_vf *)(xt + b * 128 * MM_TT);
            for (int64_t r = 0; r < nr; r++) {
                const uint8_t *p = j->w + (j->m0 + r) * rowBytes + b * 34;
                const float d = or_h2f((uint16_t)(p[0] | (p[1] << 8)));
                const uint8_t *qs = p + 2;
                mm_vf lo = {0}, hi = {0}, sy = {0};
                for (int jj = 0; jj < 128; jj++) {
                    const uint32_t code = (qs[jj >> 2] >> ((jj & 3) << 1)) & 3;
                    const mm_vf xv = xb[jj];
                    const mm_vu m1 = (mm_vu){0} - (code & 1), m2 = (mm_vu){0} - (code >> 1);
                    sy += xv;
                    lo += (mm_vf)((mm_vu)xv & m1);
                    hi += (mm_vf)((mm_vu)xv & m2);
                }
                acc[r] += d * (lo + 2 * hi - sy);
            }
        }
        for (int64_t r = 0; r < nr; r++)
            for (int t = 0; t < MM_TT && t0 + t < j->T; t++)
                j->out[(t0 + t) * j->M + j->m0 + r] = acc[r][t];
    }
    return NULL;
}

void or_q2_0_matmat(const uint8_t *w, int64_t K, int64_t M, int64_t T, const float *X,
                    float *out, int threads) {
    if (T <= 0 || M <= 0) return;
    if (threads < 1) threads = 1;
    if (threads > M) threads = (int)M;
    if (threads > 256) threads = 256;
    const int64_t Tp = (T + MM_TT - 1) / MM_TT * MM_TT;
    float *xt = (float *)aligned_alloc(64, (size_t)(Tp * K * 4));
    for (int64_t t0 = 0; t0 < Tp; t0 += MM_TT)
        for (int64_t k = 0; k < K; k++)
            for (int t = 0; t < MM_TT; t++)
                xt[t0 * K + k * MM_TT + t] = t0 + t < T ? X[(t0 + t) * K + k] : 0.0f;
    struct mm_job jobs[256];
    float *acc = (float *)aligned_alloc(64, (size_t)(M * MM_TT * 4));
    for (int t = 0; t < threads; t++) {
        const int64_t m0 = M * t / threads, m1 = M * (t + 1) / threads;
        struct mm_job jb = {w, K, m0, m1, T, Tp, xt, acc + m0 * MM_TT, out, M};
        jobs[t] = jb;
    }
    run_jobs(mm_rows, jobs, sizeof jobs[0], threads);
    free(acc);
    free(xt);
}

void or_q2_0_matvec_f64(const uint8_t *w, int64_t K, int64_t M, const double *x, double *out) {
    const int64_t nblk = K / 128;
    for (int64_t m = 0; m < M; m++) {
        double acc = 0;
        for (int64_t b = 0; b < nblk; b++) {
            const uint8_t *p = w + (m * nblk + b) * 34;
            const double d = (double)or_h2f((uint16_t)(p[0] | (p[1] << 8)));
            for (int j = 0; j < 128; j++) {
                const int code = (p[2 + (j >> 2)] >> ((j & 3) * 2)) & 3;
                acc += (double)(code - 1) * d * x[b * 128 + j];
            }
        }
        out[m] = acc;
    }
}

/* ----------------------------------------------------------- primitives */

float or_silu(float x) { return x / (1 + expf(-x)); }            /* Kernels.swift:5 */
float or_sigmoid(float x) { return 1 / (1 + expf(-x)); }         /* Kernels.swift:6 */
float or_softplus(float x) {                                      /* Kernels.swift:7-10 */
    return fmaxf(x, 0) + log1pf(expf(-fabsf(x)));
}

void or_rmsnorm(const float *x, const float *w, float *y, int64_t n, float eps) {
    float ss = 0;
    for (int64_t i = 0; i < n; i++) ss += x[i] * x[i];
    const float scale = 1 / sqrtf(ss / (float)n + eps);
    for (int64_t i = 0; i < n; i++) y[i] = x[i] * scale * w[i];
}

void or_rmsnorm_rows(float *x, int d, int64_t rows, const float *w, float eps) {
    for (int64_t r = 0; r < rows; r++) {
        float *p = x + r * d;
        float ss = 0;
        for (int i = 0; i < d; i++) ss += p[i] * p[i];
        const float s = 1 / sqrtf(ss / (float)d + eps);
        for (int i = 0; i < d; i++) p[i] = p[i] * s * w[i];
    }
}

void or_l2norm_rows(float *x, int d, int64_t rows, float eps) {
    for (int64_t r = 0; r < rows; r++) {
        float *p = x + r * d;
        float ss = 0;
        for (int i = 0; i < d; i++) ss += p[i] * p[i];
        const float s = 1 / sqrtf(ss + eps);
        for (int i = 0; i < d; i++) p[i] *= s;
    }
}

void or_softmax(float *x, int n) {
    float mx = -3.402823466e38f;
    for (int i = 0; i < n; i++) mx = fmaxf(mx, x[i]);
    float s = 0;
    for (int i = 0; i < n; i++) { const float e = expf(x[i] - mx); x[i] = e; s += e; }
    const float inv = 1 / s;
    for (int i = 0; i < n; i++) x[i] *= inv;
}

void or_rope_neox(float *x, int headDim, int nHead, int nRot, float base, int pos) {
    const int half = nRot / 2;
    for (int h = 0; h < nHead; h++) {
        float *p = x + h * headDim;
        for (int i = 0; i < half; i++) {
            const float freq = powf(base, -2 * (float)i / (float)nRot);
            const float ang = (float)pos * freq;
            const float c = cosf(ang), s = sinf(ang);
            const float a = p[i], b = p[i + half];
            p[i] = a * c - b * s;
            p[i + half] = a * s + b * c;
        }
    }
}

/* ------------------------------------------------------------------ GDN */

void or_gdn_gate(const float *bPre, const float *aPre, const float *dt, const float *aNeg,
                 float *beta, float *g, int nV, int64_t count) {
    for (int64_t i = 0; i < count; i++) {
        const int h = (int)(i % nV);
        beta[i] = or_sigmoid(bPre[i]);
        g[i] = or_softplus(aPre[i] + dt[h]) * aNeg[h];
    }
}

void or_gdn_conv(const float *qkvMix, float *cs, const float *cw, float *out, int convDim,
                 int kc) {
    for (int c = 0; c < convDim; c++) {
        float acc = 0;
        for (int j = 0; j < kc - 1; j++) acc += cs[j * convDim + c] * cw[c * kc + j];
        acc += qkvMix[c] * cw[c * kc + (kc - 1)];
        out[c] = or_silu(acc);
    }
    if (kc >= 2) {
        for (int j = 0; j < kc - 2; j++)
            for (int c = 0; c < convDim; c++) cs[j * convDim + c] = cs[(j + 1) * convDim + c];
        for (int c = 0; c < convDim; c++) cs[(kc - 2) * convDim + c] = qkvMix[c];
    }
}

/* GDN.swift:78-109 */
void or_gdn_scan(const float *q, const float *k, const float *v, const float *g,
                 const float *beta, float *S, float *o, int nV, int nK, int dS, float qScale) {
    float *sk = (float *)malloc(sizeof(float) * dS);
    float *d = (float *)malloc(sizeof(float) * dS);
    for (int hv = 0; hv < nV; hv++) {
        const int hk = hv % nK;
        const float *qh = q + hk * dS, *kh = k + hk * dS;
        const int voff = hv * dS;
        float *Sh = S + (int64_t)hv * dS * dS;
        const float gamma = expf(g[hv]), b = beta[hv];
        for (int j = 0; j < dS; j++) sk[j] = 0;
        for (int i = 0; i < dS; i++) {
            const float ki = kh[i];
            float *row = Sh + (int64_t)i * dS;
            for (int j = 0; j < dS; j++) {
                const float s = row[j] * gamma;
                row[j] = s;
                sk[j] += s * ki;
            }
        }
        for (int j = 0; j < dS; j++) d[j] = b * (v[voff + j] - sk[j]);
        for (int j = 0; j < dS; j++) o[voff + j] = 0;
        for (int i = 0; i < dS; i++) {
            const float ki = kh[i];
            const float qi = qh[i] * qScale;
            float *row = Sh + (int64_t)i * dS;
            for (int j = 0; j < dS; j++) {
                row[j] += ki * d[j];
                o[voff + j] += row[j] * qi;
            }
        }
    }
    free(sk);
    free(d);
}

void or_gdn_scan_f64(const double *q, const double *k, const double *v, const double *g,
                     const double *beta, double *S, double *o, int nV, int nK, int dS,
                     double qScale) {
    for (int hv = 0; hv < nV; hv++) {
        const int hk = hv % nK;
        const double *qh = q + hk * dS, *kh = k + hk * dS;
        double *Sh = S + (int64_t)hv * dS * dS;
        const double gamma = exp(g[hv]);
        for (int64_t e = 0; e < (int64_t)dS * dS; e++) Sh[e] *= gamma;
        for (int j = 0; j < dS; j++) {
            double sk = 0;
            for (int i = 0; i < dS; i++) sk += Sh[(int64_t)i * dS + j] * kh[i];
            const double dj = beta[hv] * (v[hv * dS + j] - sk);
            double acc = 0;
            for (int i = 0; i < dS; i++) {
                Sh[(int64_t)i * dS + j] += kh[i] * dj;
                acc += Sh[(int64_t)i * dS + j] * qh[i];
            }
            o[hv * dS + j] = acc * qScale;
        }
    }
}

/* The chunk identity in double, written with explicit matrices so that it is
 * independent of the sequential code it is checked against:
 *   A = tril(diag(beta) (K K^T o Gamma), -1), T = (I + A)^-1 (by forward
 *   substitution), delta = T diag(beta) (V - diag(e^G) K S0),
 *   O = qScale (diag(e^G) Q S0 + tril(Q K^T o Gamma) delta),
 *   S = e^{G_L} S0 + K^T diag(e^{G_L - G}) delta. */
void or_gdn_chunked_f64(int64_t T, int nV, int nK, int dk, int dv, const double *q,
                        const double *k, const double *v, const double *g, const double *beta,
                        double *S, double *o, double qScale, int C) {
    double *G = (double *)malloc(sizeof(double) * C);
    double *A = (double *)malloc(sizeof(double) * C * C);
    double *Tm = (double *)malloc(sizeof(double) * C * C);
    double *R = (double *)malloc(sizeof(double) * C * dv);      /* rhs / delta */
    double *D = (double *)malloc(sizeof(double) * C * dv);
    for (int hv = 0; hv < nV; hv++) {
        const int hk = hv % nK;
        double *Sh = S + (int64_t)hv * dk * dv;
        for (int64_t t0 = 0; t0 < T; t0 += C) {
            const int L = (int)(T - t0 < C ? T - t0 : C);
#define Q_(t, i) q[((t0 + (t)) * nK + hk) * dk + (i)]
#define K_(t, i) k[((t0 + (t)) * nK + hk) * dk + (i)]
#define V_(t, j) v[((t0 + (t)) * nV + hv) * dv + (j)]
            double acc = 0;
            for (int t = 0; t < L; t++) { acc += g[(t0 + t) * nV + hv]; G[t] = acc; }
            for (int t = 0; t < L; t++)
                for (int s = 0; s < L; s++) {
                    double kk = 0;
                    if (s < t) for (int i = 0; i < dk; i++) kk += K_(t, i) * K_(s, i);
                    A[t * C + s] = s < t ? beta[(t0 + t) * nV + hv] * exp(G[t] - G[s]) * kk : 0;
                }
            for (int s = 0; s < L; s++) {
                for (int t = 0; t < L; t++) Tm[t * C + s] = t == s ? 1 : 0;
                for (int t = s + 1; t < L; t++) {
                    double a2 = 0;
                    for (int m = s; m < t; m++) a2 += A[t * C + m] * Tm[m * C + s];
                    Tm[t * C + s] = -a2;
                }
            }
            /* rhs = diag(beta) (V - diag(e^G) K S0) */
            for (int t = 0; t < L; t++)
                for (int j = 0; j < dv; j++) {
                    double ks = 0;
                    for (int i = 0; i < dk; i++) ks += K_(t, i) * Sh[(int64_t)i * dv + j];
                    R[t * dv + j] = beta[(t0 + t) * nV + hv] * (V_(t, j) - exp(G[t]) * ks);
                }
            for (int t = 0; t < L; t++)
                for (int j = 0; j < dv; j++) {
                    double dd = 0;
                    for (int s = 0; s <= t; s++) dd += Tm[t * C + s] * R[s * dv + j];
                    D[t * dv + j] = dd;
                }
            for (int t = 0; t < L; t++)
                for (int j = 0; j < dv; j++) {
                    double qs = 0, pd = 0;
                    for (int i = 0; i < dk; i++) qs += Q_(t, i) * Sh[(int64_t)i * dv + j];
                    for (int s = 0; s <= t; s++) {
                        double qk = 0;
                        for (int i = 0; i < dk; i++) qk += Q_(t, i) * K_(s, i);
                        pd += exp(G[t] - G[s]) * qk * D[s * dv + j];
                    }
                    o[((t0 + t) * nV + hv) * dv + j] = qScale * (exp(G[t]) * qs + pd);
                }
            const double gl = G[L - 1];
            for (int i = 0; i < dk; i++)
                for (int j = 0; j < dv; j++) {
                    double a3 = 0;
                    for (int s = 0; s < L; s++) a3 += K_(s, i) * exp(gl - G[s]) * D[s * dv + j];
                    Sh[(int64_t)i * dv + j] = exp(gl) * Sh[(int64_t)i * dv + j] + a3;
                }
#undef Q_
#undef K_
#undef V_
        }
    }
    free(G); free(A); free(Tm); free(R); free(D);
}

/* MtpRollback.swift:20-60 */
void or_mtp_state_after(int m, int H, int DK, int DV, int C, const float *s0, const float *delta,
                        const float *k, const float *gcum, float *out) {
    for (int h = 0; h < H; h++) {
        const float *gc = gcum + h * C, *kh = k + h * C * DK, *dh = delta + h * C * DV;
        const float *sh = s0 + h * DK * DV;
        float *oh = out + h * DK * DV;
        const float gLast = gc[m - 1];
        const float eM = expf(gLast);
        for (int i = 0; i < DK; i++)
            for (int j = 0; j < DV; j++) oh[i * DV + j] = eM * sh[i * DV + j];
        for (int t = 0; t < m; t++) {
            const float w = expf(gLast - gc[t]);
            for (int i = 0; i < DK; i++) {
                const float wk = w * kh[t * DK + i];
                for (int j = 0; j < DV; j++) oh[i * DV + j] += wk * dh[t * DV + j];
            }
        }
    }
}

/* --------------------------------------------------- threaded decode batch */

struct dec_job {
    int b0, b1, nV, nK, dS;
    float *q, *k;
    const float *v, *g, *beta;
    float *S, *o;
    float qScale, eps;
};

static void *dec_rows(void *arg) {
    const struct dec_job *j = (const struct dec_job *)arg;
    for (int b = j->b0; b < j->b1; b++) {
        float *qb = j->q + (int64_t)b * j->nK * j->dS, *kb = j->k + (int64_t)b * j->nK * j->dS;
        or_l2norm_rows(qb, j->dS, j->nK, j->eps);
        or_l2norm_rows(kb, j->dS, j->nK, j->eps);
        or_gdn_scan(qb, kb, j->v + (int64_t)b * j->nV * j->dS, j->g + (int64_t)b * j->nV,
                    j->beta + (int64_t)b * j->nV, j->S + (int64_t)b * j->nV * j->dS * j->dS,
                    j->o + (int64_t)b * j->nV * j->dS, j->nV, j->nK, j->dS, j->qScale);
    }
    return NULL;
}

void or_gdn_decode_batch(int B, int nV, int nK, int dS, float *q, float *k, const float *v,
                         const float *g, const float *beta, float *S, float *o, float qScale,
                         float eps, int threads) {
    if (threads < 1) threads = 1;
    if (threads > B) threads = B;
    if (threads > 256) threads = 256;
    struct dec_job jobs[256];
    pthread_t tid[256];
    for (int t = 0; t < threads; t++) {
        struct dec_job j = {B * t / threads, B * (t + 1) / threads, nV, nK, dS, q, k, v, g,
                            beta, S, o, qScale, eps};
        jobs[t] = j;
    }
    if (threads == 1) { dec_rows(&jobs[0]); return; }
    for (int t = 0; t < threads; t++) pthread_create(&tid[t], NULL, dec_rows, &jobs[t]);
    for (int t = 0; t < threads; t++) pthread_join(tid[t], NULL);
}
