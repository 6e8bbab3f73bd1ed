// Gated DeltaNet glue and the per-token recurrence.
//
// Reference: GDN.step (LLM/src/SIMD/GDN.swift:20-120), the Metal kernels
// gdn_gate / gdn_conv / l2norm_rows / rmsnorm_rows / gdn_scan
// (LLM/metal/Kernels.metal:751-809, 1118-1243) and their MetalEnc hosts
// (LLM/src/Metal/MetalEnc.swift:213-272, 572-653).
//
// The fused decode step keeps one value column per lane: column j of the
// state, S[:, j], is all a lane needs (sk_j, delta_j, o_j are per-column), so
// a head's 64 KB state is read once and written once with no cross-lane
// reduction inside a wave; four waves split the key rows and meet once in LDS
// per reduction.  L2 normalization of q and k is folded into scalars:
// S^T k_hat = rk * S^T k and k_hat delta^T = k (rk * delta)^T.
#include "gd_internal.h"

// ------------------------------------------------------------------- gates

__global__ void gd_gate_kernel(const float *bPre, const float *aPre, const float *dt,
                               const float *aNeg, float *beta, float *g, int nV, int64_t count) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    const int h = (int)(i % nV);
    beta[i] = gd_sigmoid(bPre[i]);
    g[i] = gd_softplus(aPre[i] + dt[h]) * aNeg[h];
}

extern "C" int gd_gdn_gate(gd_ctx *ctx, const float *bPre, const float *aPre, const float *dt,
                           const float *aNeg, float *beta, float *g, int nV, int64_t count) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, bPre && aPre && dt && aNeg && beta && g, "gd_gdn_gate: null pointer");
    GD_REQUIRE(ctx, nV > 0 && count >= 0, "gd_gdn_gate: nV=%d count=%lld", nV, (long long)count);
    if (!count) return GD_OK;
    hipLaunchKernelGGL(gd_gate_kernel, dim3(gd_blocks(count, 256)), dim3(256), 0, ctx->stream,
                       bPre, aPre, dt, aNeg, beta, g, nV, count);
    GD_LAUNCHED(ctx, "gdn_gate");
    return GD_OK;
}

// ------------------------------------------------------------ causal conv

// One thread per channel; the ring stays in registers across the N tokens.
// window = [ring[0..dConv-2], x]; out = silu(sum window[j] * cw[c*dConv + j]).
template <int KC>
__global__ void gd_conv_kernel(const float *x, float *ring, const float *cw, float *out,
                               int convDim, int64_t N) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= convDim) return;
    float w[KC], r[KC];
#pragma unroll
    for (int j = 0; j < KC; j++) w[j] = cw[(int64_t)c * KC + j];
#pragma unroll
    for (int j = 0; j + 1 < KC; j++) r[j] = ring[(int64_t)j * convDim + c];
    for (int64_t n = 0; n < N; n++) {
        const float cur = x[n * convDim + c];
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j + 1 < KC; j++) acc += r[j] * w[j];
        acc += cur * w[KC - 1];
        out[n * convDim + c] = gd_silu(acc);
#pragma unroll
        for (int j = 0; j + 2 < KC; j++) r[j] = r[j + 1];
        if (KC >= 2) r[KC - 2] = cur;
    }
#pragma unroll
    for (int j = 0; j + 1 < KC; j++) ring[(int64_t)j * convDim + c] = r[j];
}

extern "C" int gd_gdn_conv(gd_ctx *ctx, const float *qkvMix, float *convState, const float *cw,
                           float *out, int convDim, int dConv, int64_t N) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, qkvMix && cw && out && (convState || dConv == 1), "gd_gdn_conv: null pointer");
    GD_REQUIRE(ctx, convDim > 0 && N >= 0, "gd_gdn_conv: convDim=%d N=%lld", convDim, (long long)N);
    GD_REQUIRE(ctx, dConv >= 1 && dConv <= 8, "gd_gdn_conv: dConv=%d not in [1,8]", dConv);
    if (!N) return GD_OK;
    dim3 g(gd_blocks(convDim, 256)), b(256);
    switch (dConv) {
#define GD_CONV_CASE(KC) \
    case KC: hipLaunchKernelGGL(gd_conv_kernel<KC>, g, b, 0, ctx->stream, qkvMix, convState, cw, \
                                out, convDim, N); break;
        GD_CONV_CASE(1) GD_CONV_CASE(2) GD_CONV_CASE(3) GD_CONV_CASE(4)
        GD_CONV_CASE(5) GD_CONV_CASE(6) GD_CONV_CASE(7) GD_CONV_CASE(8)
#undef GD_CONV_CASE
    }
    GD_LAUNCHED(ctx, "gdn_conv");
    return GD_OK;
}

// ------------------------------------------------------------------- norms

// One 64-lane wave per row.
__global__ void gd_l2norm_kernel(float *x, int d, int rowsPerTok, int64_t tokStride,
                                 int64_t rows, float eps) {
    const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int lane = threadIdx.x & 63;
    float *r = x + (row / rowsPerTok) * tokStride + (row % rowsPerTok) * d;
    float ss = 0.0f;
    for (int i = lane; i < d; i += 64) ss += r[i] * r[i];
    ss = gd_wave_sum(ss);
    const float s = 1.0f / sqrtf(ss + eps);
    for (int i = lane; i < d; i += 64) r[i] *= s;
}

extern "C" int gd_l2norm_rows(gd_ctx *ctx, float *x, int d, int rowsPerTok, int64_t tokStride,
                              int64_t tokens, float eps) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, x && d > 0 && rowsPerTok > 0 && tokens >= 0 &&
                        tokStride >= (int64_t)rowsPerTok * d,
               "gd_l2norm_rows: bad arguments");
    const int64_t rows = (int64_t)rowsPerTok * tokens;
    if (!rows) return GD_OK;
    hipLaunchKernelGGL(gd_l2norm_kernel, dim3(gd_blocks(rows, 4)), dim3(256), 0, ctx->stream, x,
                       d, rowsPerTok, tokStride, rows, eps);
    GD_LAUNCHED(ctx, "l2norm_rows");
    return GD_OK;
}

__global__ void gd_rmsnorm_rows_kernel(float *x, int d, int64_t rows, const float *w, float eps) {
    const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int lane = threadIdx.x & 63;
    float *r = x + row * d;
    float ss = 0.0f;
    for (int i = lane; i < d; i += 64) ss += r[i] * r[i];
    ss = gd_wave_sum(ss);
    const float s = 1.0f / sqrtf(ss / (float)d + eps);
    for (int i = lane; i < d; i += 64) r[i] = r[i] * s * w[i];
}

extern "C" int gd_rmsnorm_rows(gd_ctx *ctx, float *x, int d, int64_t rows, const float *w,
                               float eps) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, x && w && d > 0 && rows >= 0, "gd_rmsnorm_rows: bad arguments");
    if (!rows) return GD_OK;
    hipLaunchKernelGGL(gd_rmsnorm_rows_kernel, dim3(gd_blocks(rows, 4)), dim3(256), 0,
                       ctx->stream, x, d, rows, w, eps);
    GD_LAUNCHED(ctx, "rmsnorm_rows");
    return GD_OK;
}

// One 256-thread block per row of length n (the hidden size).
template <int YT>
__global__ void gd_rmsnorm_kernel(const float *x, const float *w, void *y, int64_t n, float eps) {
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    const float *xr = x + row * n;
    float ss = 0.0f;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) ss += xr[i] * xr[i];
    ss = gd_block_sum(ss, red);
    const float s = 1.0f / sqrtf(ss / (float)n + eps);
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
        const float v = xr[i] * s * w[i];
        if (YT == GD_F32) ((float *)y)[row * n + i] = v;
        else ((uint16_t *)y)[row * n + i] = gd_f2h(v);
    }
}

extern "C" int gd_rmsnorm(gd_ctx *ctx, const float *x, const float *w, void *y, int y_dtype,
                          int64_t n, int64_t rows, float eps) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, x && w && y && n > 0 && rows >= 0, "gd_rmsnorm: bad arguments");
    GD_REQUIRE(ctx, y_dtype == GD_F32 || y_dtype == GD_F16, "gd_rmsnorm: bad dtype");
    GD_REQUIRE(ctx, rows < (1LL << 31), "gd_rmsnorm: too many rows");
    if (!rows) return GD_OK;
    if (y_dtype == GD_F32)
        hipLaunchKernelGGL(gd_rmsnorm_kernel<GD_F32>, dim3((unsigned)rows), dim3(256), 0,
                           ctx->stream, x, w, y, n, eps);
    else
        hipLaunchKernelGGL(gd_rmsnorm_kernel<GD_F16>, dim3((unsigned)rows), dim3(256), 0,
                           ctx->stream, x, w, y, n, eps);
    GD_LAUNCHED(ctx, "rmsnorm");
    return GD_OK;
}

// ------------------------------------------------------------- elementwise

template <int OP>
__global__ void gd_elementwise_kernel(float *a, const float *b, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (OP == 0) a[i] = gd_silu(a[i]) * b[i];
    else if (OP == 1) a[i] = a[i] * gd_silu(b[i]);
    else a[i] += b[i];
}

template <int OP>
static int elementwise(gd_ctx *ctx, float *a, const float *b, int64_t n, const char *name) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, a && b && n >= 0, "%s: bad arguments", name);
    if (!n) return GD_OK;
    hipLaunchKernelGGL(gd_elementwise_kernel<OP>, dim3(gd_blocks(n, 256)), dim3(256), 0,
                       ctx->stream, a, b, n);
    GD_LAUNCHED(ctx, name);
    return GD_OK;
}

extern "C" int gd_silu_mul(gd_ctx *ctx, float *a, const float *b, int64_t n) {
    return elementwise<0>(ctx, a, b, n, "silu_mul");
}
extern "C" int gd_mul_silu(gd_ctx *ctx, float *a, const float *b, int64_t n) {
    return elementwise<1>(ctx, a, b, n, "mul_silu");
}
extern "C" int gd_add(gd_ctx *ctx, float *x, const float *y, int64_t n) {
    return elementwise<2>(ctx, x, y, n, "add_inplace");
}

// -------------------------------------------------- fused state-carry decode

namespace {

constexpr int DEC_DS = 128;      // state size handled by the fused kernel
constexpr int DEC_COLS = 64;     // value columns per workgroup (one per lane)
constexpr int DEC_ROWS = 32;     // key rows per wave (4 waves)

template <typename T> __device__ __forceinline__ float ld(const T *p, int64_t i);
template <> __device__ __forceinline__ float ld<float>(const float *p, int64_t i) { return p[i]; }
template <> __device__ __forceinline__ float ld<uint16_t>(const uint16_t *p, int64_t i) {
    return gd_h2f(p[i]);
}
template <typename T> __device__ __forceinline__ void st(T *p, int64_t i, float v);
template <> __device__ __forceinline__ void st<float>(float *p, int64_t i, float v) { p[i] = v; }
template <> __device__ __forceinline__ void st<uint16_t>(uint16_t *p, int64_t i, float v) {
    p[i] = gd_f2h(v);
}

// Grid: (dS/64 column blocks, nV heads, B sequences); 256 threads.
// NORM: L2-normalize q,k.  GATE: beta/g from pre-activations with dt/aNeg.
template <typename IO, bool NORM, bool GATE>
__global__ __launch_bounds__(256) void gd_decode_kernel(
        const IO *__restrict__ q, const IO *__restrict__ k, const IO *__restrict__ v,
        const float *__restrict__ g_in, const float *__restrict__ beta_in,
        const float *__restrict__ dt, const float *__restrict__ aNeg, float *__restrict__ S,
        IO *__restrict__ o, int nV, int nK, float qScale, float eps) {
    __shared__ float kq[2][DEC_DS];
    __shared__ float red[4][DEC_COLS];
    __shared__ float scal[2];

    const int jb = blockIdx.x, hv = blockIdx.y, b = blockIdx.z;
    const int hk = hv % nK;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = jb * DEC_COLS + lane;

    const int64_t qk_off = ((int64_t)b * nK + hk) * DEC_DS;
    const int64_t v_off = ((int64_t)b * nV + hv) * DEC_DS;
    const int64_t gb = (int64_t)b * nV + hv;
    float *Sh = S + ((int64_t)b * nV + hv) * DEC_DS * DEC_DS;

    // Issue the state loads first: they are the bandwidth.
    float s[DEC_ROWS];
#pragma unroll
    for (int r = 0; r < DEC_ROWS; r++) s[r] = Sh[(int64_t)(wave * DEC_ROWS + r) * DEC_DS + j];

    if (tid < DEC_DS) kq[0][tid] = ld(k, qk_off + tid);
    else kq[1][tid - DEC_DS] = ld(q, qk_off + tid - DEC_DS);
    float beta, gam;
    if (GATE) {
        beta = gd_sigmoid(beta_in[gb]);
        gam = expf(gd_softplus(g_in[gb] + dt[hv]) * aNeg[hv]);
    } else {
        beta = beta_in[gb];
        gam = expf(g_in[gb]);
    }
    const float vj = ld(v, v_off + j);
    __syncthreads();
    float rk = 1.0f, rq = 1.0f;
    if (NORM) {
        // Waves 0/1 reduce |k|^2 and |q|^2 (2 elements per lane).
        if (wave < 2) {
            const float a = kq[wave][lane], c = kq[wave][lane + 64];
            const float ss = gd_wave_sum(a * a + c * c);
            if (lane == 0) scal[wave] = 1.0f / sqrtf(ss + eps);
        }
        __syncthreads();
        rk = scal[0];
        rq = scal[1];
    }

    // Decay and this wave's part of S^T k.
    float sk = 0.0f;
#pragma unroll
    for (int r = 0; r < DEC_ROWS; r++) {
        s[r] *= gam;
        sk = fmaf(s[r], kq[0][wave * DEC_ROWS + r], sk);
    }
    red[wave][lane] = sk;
    __syncthreads();
    sk = (red[0][lane] + red[1][lane] + red[2][lane] + red[3][lane]) * rk;
    const float delta = beta * (vj - sk) * rk;   // rk folds k_hat into the update
    __syncthreads();                              // red[] is reused below

    float acc = 0.0f;
#pragma unroll
    for (int r = 0; r < DEC_ROWS; r++) {
        const int i = wave * DEC_ROWS + r;
        s[r] = fmaf(kq[0][i], delta, s[r]);
        acc = fmaf(s[r], kq[1][i], acc);
        Sh[(int64_t)i * DEC_DS + j] = s[r];
    }
    red[wave][lane] = acc;
    __syncthreads();
    if (wave == 0) {
        const float oj = (red[0][lane] + red[1][lane] + red[2][lane] + red[3][lane]) * rq * qScale;
        st(o, v_off + j, oj);
    }
}

// General-dS single-token scan for shapes the fused kernel does not take: one
// thread per (value head, column), as gdn_scan (Kernels.metal:1206-1243).
__global__ void gd_scan_generic_kernel(const float *q, const float *k, const float *v,
                                       const float *g, const float *beta, float *S, float *o,
                                       int nV, int nK, int dS, float qScale) {
    const int gid = blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= nV * dS) return;
    const int hv = gid / dS, j = gid % dS, hk = hv % nK;
    const float *qh = q + (int64_t)hk * dS, *kh = k + (int64_t)hk * dS;
    float *Sh = S + (int64_t)hv * dS * dS;
    const float gam = expf(g[hv]), b = beta[hv];
    float sk = 0.0f;
    for (int i = 0; i < dS; i++) {
        const float x = Sh[(int64_t)i * dS + j] * gam;
        Sh[(int64_t)i * dS + j] = x;
        sk += x * kh[i];
    }
    const float d = b * (v[(int64_t)hv * dS + j] - sk);
    float acc = 0.0f;
    for (int i = 0; i < dS; i++) {
        const float x = Sh[(int64_t)i * dS + j] + kh[i] * d;
        Sh[(int64_t)i * dS + j] = x;
        acc += x * qh[i];
    }
    o[(int64_t)hv * dS + j] = acc * qScale;
}

// N tokens of the scan for state sizes the chunked prefill does not take
// (dS != 128): gdn_scan_batch (Kernels.metal:1525-1565), which
// MetalEnc.gdnScanBatch dispatches for any dS (MetalEnc.swift:741-778).  One
// workgroup per value head, thread j owning value column j of S (dS <= 1024),
// tokens in order; q and k of the token are staged once per workgroup in
// LDS (the column walks read them at every row), S stays in device memory
// as in the reference (a head's dS x dS f32 exceeds LDS beyond 181).
__global__ __launch_bounds__(1024) void gd_scan_batch_serial_kernel(
        const float *convOutN, const float *gN, const float *betaN, float *S, float *oN, int nV,
        int nK, int dS, float qScale, int64_t N, int convDim, int keyDim, int valueDim) {
    extern __shared__ float qk[];                 // [2][dS]: q, k of the token
    const int hv = blockIdx.x, j = threadIdx.x, hk = hv % nK;
    float *Sh = S + (int64_t)hv * dS * dS;
    for (int64_t n = 0; n < N; n++) {
        const float *row = convOutN + n * convDim;
        __syncthreads();                          // the previous token's reads are done
        for (int i = threadIdx.x; i < dS; i += blockDim.x) {
            qk[i] = row[(int64_t)hk * dS + i];
            qk[dS + i] = row[keyDim + (int64_t)hk * dS + i];
        }
        __syncthreads();
        if (j >= dS) continue;
        const float gam = expf(gN[n * nV + hv]), b = betaN[n * nV + hv];
        const float *k = qk + dS, *q = qk;
        float sk = 0.0f;
        for (int i = 0; i < dS; i++) {
            const float x = Sh[(int64_t)i * dS + j] * gam;
            Sh[(int64_t)i * dS + j] = x;
            sk += x * k[i];
        }
        const float d = b * (row[2 * (int64_t)keyDim + (int64_t)hv * dS + j] - sk);
        float acc = 0.0f;
        for (int i = 0; i < dS; i++) {
            const float x = Sh[(int64_t)i * dS + j] + k[i] * d;
            Sh[(int64_t)i * dS + j] = x;
            acc += x * q[i];
        }
        oN[n * valueDim + (int64_t)hv * dS + j] = acc * qScale;
    }
}

}  // namespace

// Token-serial gdnScanBatch for any dS up to 1024 (the caller has checked
// the pointers and the dimensions).
int gd_gdn_scan_batch_serial(gd_ctx *ctx, const float *convOutN, int keyDim, int valueDim,
                             int convDim, const float *gN, const float *betaN, float *S,
                             float *oN, int nV, int nK, int dS, float qScale, int64_t N) {
    GD_REQUIRE(ctx, dS > 0 && dS <= 1024 && nV > 0 && nK > 0 && nV <= 65535,
               "gd_gdn_scan_batch: dS=%d nV=%d nK=%d (the token-serial scan takes dS <= 1024)",
               dS, nV, nK);
    if (N <= 0) return GD_OK;
    const int threads = (dS + 63) / 64 * 64;
    hipLaunchKernelGGL(gd_scan_batch_serial_kernel, dim3(nV), dim3(threads),
                       (size_t)2 * dS * sizeof(float), ctx->stream, convOutN, gN, betaN, S, oN,
                       nV, nK, dS, qScale, N, convDim, keyDim, valueDim);
    GD_LAUNCHED(ctx, "gdn_scan_batch");
    return GD_OK;
}

extern "C" int gd_gdn_decode(gd_ctx *ctx, int B, int nV, int nK, int dS, const void *q,
                             const void *k, const void *v, int io_dtype, const float *g_in,
                             const float *beta_in, const float *dt, const float *aNeg, float *S,
                             void *o, float qScale, float eps) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, q && k && v && g_in && beta_in && S && o, "gd_gdn_decode: null pointer");
    GD_REQUIRE(ctx, (dt == nullptr) == (aNeg == nullptr),
               "gd_gdn_decode: dt and aNeg must both be given or both be NULL");
    GD_REQUIRE(ctx, B > 0 && nV > 0 && nK > 0 && B <= 65535 && nV <= 65535,
               "gd_gdn_decode: B=%d nV=%d nK=%d", B, nV, nK);
    GD_REQUIRE(ctx, dS == DEC_DS, "gd_gdn_decode: dS=%d (the fused step takes 128)", dS);
    GD_REQUIRE(ctx, io_dtype == GD_F32 || io_dtype == GD_F16, "gd_gdn_decode: bad dtype");
    dim3 grid(DEC_DS / DEC_COLS, nV, B), blk(256);
    const bool gate = dt != nullptr;
#define GD_DEC(IO, G) \
    hipLaunchKernelGGL((gd_decode_kernel<IO, true, G>), grid, blk, 0, ctx->stream, \
                       (const IO *)q, (const IO *)k, (const IO *)v, g_in, beta_in, dt, aNeg, S, \
                       (IO *)o, nV, nK, qScale, eps)
    if (io_dtype == GD_F32) { if (gate) GD_DEC(float, true); else GD_DEC(float, false); }
    else { if (gate) GD_DEC(uint16_t, true); else GD_DEC(uint16_t, false); }
#undef GD_DEC
    GD_LAUNCHED(ctx, "gdn_decode");
    return GD_OK;
}

extern "C" int gd_gdn_scan(gd_ctx *ctx, const float *q, const float *k, const float *v,
                           const float *g, const float *beta, float *S, float *o, int nV, int nK,
                           int dS, float qScale) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, q && k && v && g && beta && S && o, "gd_gdn_scan: null pointer");
    GD_REQUIRE(ctx, nV > 0 && nK > 0 && dS > 0, "gd_gdn_scan: nV=%d nK=%d dS=%d", nV, nK, dS);
    if (dS == DEC_DS && nV <= 65535) {
        dim3 grid(DEC_DS / DEC_COLS, nV, 1);
        hipLaunchKernelGGL((gd_decode_kernel<float, false, false>), grid, dim3(256), 0,
                           ctx->stream, q, k, v, g, beta, nullptr, nullptr, S, o, nV, nK, qScale,
                           0.0f);
    } else {
        hipLaunchKernelGGL(gd_scan_generic_kernel, dim3(gd_blocks((int64_t)nV * dS, 256)),
                           dim3(256), 0, ctx->stream, q, k, v, g, beta, S, o, nV, nK, dS, qScale);
    }
    GD_LAUNCHED(ctx, "gdn_scan");
    return GD_OK;
}
