// Chunked (WY / UT) Gated DeltaNet prefill.
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
// Kernels:
//   gdn_chunk_prep  (value head, chunk)   -> W, U, P, G into a workspace; the
//                                            chunks are independent.
//   gdn_chunk_scan  (value head, columns) -> walks the chunks in order with a
//                                            slice of S resident in LDS:
//                                            delta, O, S update.
// Value columns of S are independent (column j needs only S[:, j]), which
// is what splits the serial part across workgroups.
#include "gd_internal.h"


namespace {

constexpr int CMAX = 64;         // largest chunk
constexpr int DK = 128;          // key size handled
constexpr int DV = 128;          // value size handled
constexpr int SCAN_COLS = 8;     // value columns per scan workgroup

template <typename T> __device__ __forceinline__ float ldx(const void *p, int64_t i);
template <> __device__ __forceinline__ float ldx<float>(const void *p, int64_t i) {
    return ((const float *)p)[i];
}
template <> __device__ __forceinline__ float ldx<uint16_t>(const void *p, int64_t i) {
    return gd_h2f(((const uint16_t *)p)[i]);
}

struct PrepArgs {
    const void *q, *k, *v;
    int64_t q_stride, k_stride, v_stride;
    const float *g, *beta;
    float *W, *U, *P, *G;        // workspace
    int64_t T;
    int nV, nK, C, nchunks;
    float qScale;
};

// Workspace layout per (head, chunk) unit u = hv * nchunks + c:
//   W[u][C][DK], U[u][C][DV], P[u][C][C], G[u][C]

template <typename IO>
__global__ __launch_bounds__(256) void gdn_chunk_prep(PrepArgs a) {
    __shared__ float Ks[CMAX][DK + 1];
    __shared__ float QVs[CMAX][DK + 1];      // Q, later V
    __shared__ float As[CMAX][CMAX + 1];
    __shared__ float Ts[CMAX][CMAX + 1];
    __shared__ float Gs[CMAX], Bs[CMAX];

    const int hv = blockIdx.x / a.nchunks, c = blockIdx.x % a.nchunks;
    const int hk = hv % a.nK;
    const int tid = threadIdx.x;
    const int C = a.C;
    const int64_t t0 = (int64_t)c * C;
    const int L = (int)((a.T - t0) < C ? (a.T - t0) : C);
    const int64_t u = (int64_t)hv * a.nchunks + c;

    for (int e = tid; e < C * DK; e += 256) {
        const int t = e / DK, i = e % DK;
        float kv = 0.f, qv = 0.f;
        if (t < L) {
            kv = ldx<IO>(a.k, (t0 + t) * a.k_stride + (int64_t)hk * DK + i);
            qv = ldx<IO>(a.q, (t0 + t) * a.q_stride + (int64_t)hk * DK + i);
        }
        Ks[t][i] = kv;
        QVs[t][i] = qv;
    }
    if (tid < 64) {
        // Inclusive cumulative gate inside the chunk (one wave, serial adds in
        // token order, as the token-serial recurrence multiplies them).
        if (tid == 0) {
            float acc = 0.f;
            for (int t = 0; t < C; t++) {
                if (t < L) acc += a.g[(t0 + t) * a.nV + hv];
                Gs[t] = acc;
                Bs[t] = t < L ? a.beta[(t0 + t) * a.nV + hv] : 0.f;
            }
        }
    }
    __syncthreads();
    if (tid < C) a.G[u * C + tid] = Gs[tid];

    // A (strictly lower) and P (lower incl. diagonal).
    for (int e = tid; e < C * C; e += 256) {
        const int t = e / C, s = e % C;
        float av = 0.f, pv = 0.f;
        if (s <= t && t < L) {
            float kk = 0.f, qk = 0.f;
            for (int i = 0; i < DK; i++) {
                kk = fmaf(Ks[t][i], Ks[s][i], kk);
                qk = fmaf(QVs[t][i], Ks[s][i], qk);
            }
            const float dec = expf(Gs[t] - Gs[s]);
            if (s < t) av = Bs[t] * dec * kk;
            pv = a.qScale * dec * qk;
        }
        As[t][s] = av;
        a.P[u * C * C + e] = pv;
    }
    __syncthreads();

    // T = (I + A)^-1, one column per thread: column s depends only on its own
    // earlier entries, T[t][s] = -sum_{m=s}^{t-1} A[t][m] T[m][s].
    if (tid < C) {
        const int s = tid;
        for (int t = 0; t < C; t++) Ts[t][s] = (t == s) ? 1.f : 0.f;
        for (int t = s + 1; t < C; t++) {
            float acc = 0.f;
            for (int m = s; m < t; m++) acc = fmaf(As[t][m], Ts[m][s], acc);
            Ts[t][s] = -acc;
        }
    }
    // V replaces Q.
    __syncthreads();
    for (int e = tid; e < C * DV; e += 256) {
        const int t = e / DV, j = e % DV;
        QVs[t][j] = t < L ? ldx<IO>(a.v, (t0 + t) * a.v_stride + (int64_t)hv * DV + j) : 0.f;
    }
    __syncthreads();

    // W = T diag(beta e^G) K and U = T diag(beta) V.
    const int col = tid & 127;
    for (int t = tid >> 7; t < C; t += 2) {
        float w = 0.f, uu = 0.f;
        for (int s = 0; s <= t; s++) {
            const float ts = Ts[t][s] * Bs[s];
            w = fmaf(ts * expf(Gs[s]), Ks[s][col], w);
            uu = fmaf(ts, QVs[s][col], uu);
        }
        a.W[(u * C + t) * DK + col] = w;
        a.U[(u * C + t) * DV + col] = uu;
    }
}

struct ScanArgs {
    const void *q, *k;
    int64_t q_stride, k_stride;
    const float *W, *U, *P, *G;
    float *S;
    void *o;
    int64_t o_stride;
    int64_t T;
    int nV, nK, C, nchunks;
    float qScale;
};

template <typename IO, typename OT>
__global__ __launch_bounds__(256) void gdn_chunk_scan(ScanArgs a) {
    __shared__ float Ws[CMAX][DK + 1];
    __shared__ float Qs[CMAX][DK + 1];
    __shared__ float Ks[CMAX][DK + 1];
    __shared__ float Ps[CMAX][CMAX + 1];
    __shared__ float Ss[DK][SCAN_COLS];
    __shared__ float Ds[CMAX][SCAN_COLS];
    __shared__ float Gs[CMAX];

    const int ncb = DV / SCAN_COLS;
    const int hv = blockIdx.x / ncb, cb = blockIdx.x % ncb;
    const int hk = hv % a.nK;
    const int tid = threadIdx.x;
    const int C = a.C;
    float *Sh = a.S + (int64_t)hv * DK * DV;
    const int j0 = cb * SCAN_COLS;

    for (int e = tid; e < DK * SCAN_COLS; e += 256) {
        const int i = e / SCAN_COLS, jj = e % SCAN_COLS;
        Ss[i][jj] = Sh[(int64_t)i * DV + j0 + jj];
    }

    for (int c = 0; c < a.nchunks; c++) {
        const int64_t t0 = (int64_t)c * C;
        const int L = (int)((a.T - t0) < C ? (a.T - t0) : C);
        const int64_t u = (int64_t)hv * a.nchunks + c;
        __syncthreads();
        for (int e = tid; e < C * DK; e += 256) {
            const int t = e / DK, i = e % DK;
            Ws[t][i] = a.W[(u * C + t) * DK + i];
            float qv = 0.f, kv = 0.f;
            if (t < L) {
                qv = ldx<IO>(a.q, (t0 + t) * a.q_stride + (int64_t)hk * DK + i);
                kv = ldx<IO>(a.k, (t0 + t) * a.k_stride + (int64_t)hk * DK + i);
            }
            Qs[t][i] = qv;
            Ks[t][i] = kv;
        }
        for (int e = tid; e < C * C; e += 256) Ps[e / C][e % C] = a.P[u * C * C + e];
        if (tid < C) Gs[tid] = a.G[u * C + tid];
        __syncthreads();

        // delta = U - W S
        for (int e = tid; e < C * SCAN_COLS; e += 256) {
            const int t = e / SCAN_COLS, jj = e % SCAN_COLS;
            float acc = 0.f;
            for (int i = 0; i < DK; i++) acc = fmaf(Ws[t][i], Ss[i][jj], acc);
            Ds[t][jj] = t < L ? a.U[(u * C + t) * DV + j0 + jj] - acc : 0.f;
        }
        __syncthreads();
        // O = qScale e^G (Q S) + P delta
        for (int e = tid; e < C * SCAN_COLS; e += 256) {
            const int t = e / SCAN_COLS, jj = e % SCAN_COLS;
            if (t >= L) continue;
            float qs = 0.f, pd = 0.f;
            for (int i = 0; i < DK; i++) qs = fmaf(Qs[t][i], Ss[i][jj], qs);
            for (int s = 0; s <= t; s++) pd = fmaf(Ps[t][s], Ds[s][jj], pd);
            const float ov = a.qScale * expf(Gs[t]) * qs + pd;
            const int64_t oi = (t0 + t) * a.o_stride + (int64_t)hv * DV + j0 + jj;
            if (sizeof(OT) == 4) ((float *)a.o)[oi] = ov;
            else ((uint16_t *)a.o)[oi] = gd_f2h(ov);
        }
        __syncthreads();
        // S = e^{G_L} S + K^T diag(e^{G_L - G}) delta
        const float gl = Gs[L - 1];
        for (int e = tid; e < DK * SCAN_COLS; e += 256) {
            const int i = e / SCAN_COLS, jj = e % SCAN_COLS;
            float acc = 0.f;
            for (int s = 0; s < L; s++) acc = fmaf(Ks[s][i] * expf(gl - Gs[s]), Ds[s][jj], acc);
            Ss[i][jj] = expf(gl) * Ss[i][jj] + acc;
        }
    }
    __syncthreads();
    for (int e = tid; e < DK * SCAN_COLS; e += 256) {
        const int i = e / SCAN_COLS, jj = e % SCAN_COLS;
        Sh[(int64_t)i * DV + j0 + jj] = Ss[i][jj];
    }
}

}  // namespace

int gd_ctx_workspace(gd_ctx *ctx, size_t bytes, void **out);

extern "C" int gd_gdn_prefill(gd_ctx *ctx, int64_t T, int nV, int nK, int dk, int dv,
                              const void *q, int64_t q_stride, const void *k, int64_t k_stride,
                              const void *v, int64_t v_stride, int io_dtype, const float *g,
                              const float *beta, float *S, void *o, int64_t o_stride,
                              int o_dtype, float qScale, int C) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, q && k && v && g && beta && S && o, "gd_gdn_prefill: null pointer");
    GD_REQUIRE(ctx, dk == DK && dv == DV, "gd_gdn_prefill: dk=%d dv=%d (takes 128/128)", dk, dv);
    GD_REQUIRE(ctx, C == 16 || C == 32 || C == 64, "gd_gdn_prefill: chunk %d not 16/32/64", C);
    GD_REQUIRE(ctx, nV > 0 && nK > 0 && T >= 0, "gd_gdn_prefill: nV=%d nK=%d T=%lld", nV, nK,
               (long long)T);
    GD_REQUIRE(ctx, io_dtype == GD_F32 || io_dtype == GD_F16, "gd_gdn_prefill: bad io dtype");
    GD_REQUIRE(ctx, o_dtype == GD_F32 || o_dtype == GD_F16, "gd_gdn_prefill: bad o dtype");
    GD_REQUIRE(ctx, q_stride >= (int64_t)nK * dk && k_stride >= (int64_t)nK * dk &&
                        v_stride >= (int64_t)nV * dv && o_stride >= (int64_t)nV * dv,
               "gd_gdn_prefill: strides smaller than a token row");
    if (T == 0) return GD_OK;
    const int nchunks = (int)((T + C - 1) / C);
    const size_t units = (size_t)nV * nchunks;
    const size_t floats = units * ((size_t)C * DK + (size_t)C * DV + (size_t)C * C + C);
    void *ws = nullptr;
    int rc = gd_ctx_workspace(ctx, floats * 4, &ws);
    if (rc) return rc;
    float *W = (float *)ws;
    float *U = W + units * C * DK;
    float *P = U + units * C * DV;
    float *G = P + units * C * C;

    PrepArgs pa{q, k, v, q_stride, k_stride, v_stride, g, beta, W, U, P, G, T, nV, nK, C,
                nchunks, qScale};
    if (io_dtype == GD_F32)
        hipLaunchKernelGGL(gdn_chunk_prep<float>, dim3((unsigned)units), dim3(256), 0,
                           ctx->stream, pa);
    else
        hipLaunchKernelGGL(gdn_chunk_prep<uint16_t>, dim3((unsigned)units), dim3(256), 0,
                           ctx->stream, pa);
    GD_LAUNCHED(ctx, "gdn_chunk_prep");

    ScanArgs sa{q, k, q_stride, k_stride, W, U, P, G, S, o, o_stride, T, nV, nK, C, nchunks,
                qScale};
    dim3 grid((unsigned)(nV * (DV / SCAN_COLS)));
#define GD_SCAN(IO, OT) \
    hipLaunchKernelGGL((gdn_chunk_scan<IO, OT>), grid, dim3(256), 0, ctx->stream, sa)
    if (io_dtype == GD_F32) { if (o_dtype == GD_F32) GD_SCAN(float, float); else GD_SCAN(float, uint16_t); }
    else { if (o_dtype == GD_F32) GD_SCAN(uint16_t, float); else GD_SCAN(uint16_t, uint16_t); }
#undef GD_SCAN
    GD_LAUNCHED(ctx, "gdn_chunk_scan");
    return GD_OK;
}

extern "C" int gd_gdn_scan_batch(gd_ctx *ctx, const float *convOutN, int keyDim, int valueDim,
                                 int convDim, const float *gN, const float *betaN, float *S,
                                 float *oN, int nV, int nK, int dS, float qScale, int64_t N) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, convOutN && gN && betaN && S && oN, "gd_gdn_scan_batch: null pointer");
    GD_REQUIRE(ctx, keyDim == nK * dS && valueDim == nV * dS && convDim >= 2 * keyDim + valueDim,
               "gd_gdn_scan_batch: keyDim/valueDim/convDim inconsistent with nK, nV, dS");
    return gd_gdn_prefill(ctx, N, nV, nK, dS, dS, convOutN, convDim, convOutN + keyDim, convDim,
                          convOutN + 2 * keyDim, convDim, GD_F32, gN, betaN, S, oN, valueDim,
                          GD_F32, qScale, 64);
}

