// A Bonsai-shape stack (random-init, or loaded from a GGUF file): the qwen35
// hybrid has Gated DeltaNet layers with a gated full-attention layer every
// `attn_interval`-th; the dense qwen3 lineage (cfg.dense) has plain ungated
// attention in every layer (Model.swift:1-69).  Each layer is followed by a
// SwiGLU FFN, all linears Q2_0.  It is the HIP counterpart of the reference's GPU engine
// (MetalEngine.extend / decode, LLM/src/Metal/MetalEngine.swift:183-296,
// 367-451, 657-796) and follows the op order of the CPU oracle
// BonsaiEngine.forward (LLM/src/SIMD/BonsaiEngine.swift:155-178), GDN.step
// (GDN.swift:20-120) and Attn.step (Attention.swift:72-139).
//
// MI355X layout choices:
//   * Projections that read the same input are stored as one Q2_0 matrix and
//     run as one GEMM/GEMV: GDN [qkv | z | beta | alpha], attention
//     [q|gate | k | v] (dense: [q | k | v]), FFN [gate | up].  Rows of a Q2_0 plane are
//     contiguous, so each original tensor is a row range of the fused one.
//   * Activations feeding a Q2_0 GEMM/GEMV are written as f16 by the kernel
//     that produces them (the reference stages GEMM inputs as half,
//     Kernels.metal:428); the residual stream and every recurrent state are f32.
//   * The attention KV cache is f16 in pages of `kv_block` positions reached
//     through a page table (MetalKVPool.swift); positions are read from device
//     memory so a decode step can be replayed as a captured HIP graph.
#include "gd_internal.h"

#include <utility>

#include <atomic>
#include <cmath>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

namespace {

constexpr int HD = 128;   // d_state handled by the fused GDN kernels

// ------------------------------------------------------------------ kernels

// beta = sigmoid(bPre), g = softplus(aPre + dt) * aNeg, reading the pre-
// activations out of the fused projection rows (GDN.swift:39-42).

// Causal depthwise conv (dConv = 4) + silu over N tokens of the strided qkv
// rows, ring in registers (GDN.swift:44-62).
__global__ void k_conv4(const float *proj, int64_t stride, float *ring, const float *cw,
                        float *out, int convDim, int N) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= convDim) return;
    const float w0 = cw[c * 4], w1 = cw[c * 4 + 1], w2 = cw[c * 4 + 2], w3 = cw[c * 4 + 3];
    float r0 = ring[c], r1 = ring[convDim + c], r2 = ring[2 * convDim + c];
    for (int n = 0; n < N; n++) {
        const float cur = proj[(int64_t)n * stride + c];
        float acc = 0.0f;
        acc += r0 * w0;
        acc += r1 * w1;
        acc += r2 * w2;
        acc += cur * w3;
        out[(int64_t)n * convDim + c] = gd_silu(acc);
        r0 = r1; r1 = r2; r2 = cur;
    }
    ring[c] = r0; ring[convDim + c] = r1; ring[2 * convDim + c] = r2;
}

// The GDN layer's prefill front end in one launch: causal conv + silu of
// every conv channel (Kernels.metal:1490-1520), the L2 norm of each q and k
// head row (Kernels.swift:41-52), the gates beta = sigmoid(b) and
// g = softplus(a + dt) * aNeg (GDN.swift:39-42), and the advance of the conv
// ring.  Wave task (row r of 128 channels, CT tokens n0 ..): lane l holds
// channels 128r + l and 128r + 64 + l and slides a window over the token
// rows n0-3 .. n0+CT-1.  Only the wave of the first tokens of a row reads the ring
// (earlier tokens than 0), so it alone writes the new ring, after its reads.
// The row-0 waves also compute the gates of their tokens.
constexpr int CT = 4;                        // tokens per wave task
// Sum of the NP split-K partials of proj[idx] (pstride floats apart), in split order.
template <int NP>
__device__ __forceinline__ float psum(const float *proj, int64_t pstride, int64_t idx) {
    float a = proj[idx];
#pragma unroll
    for (int p = 1; p < NP; p++) a += proj[p * pstride + idx];
    return a;
}
static_assert(CT >= 3, "only the first task of a row may reach back into the ring");
// Tail partials of the gate columns the prefill front end sums (at most).
constexpr int TAIL_MAX = 8;
// proj holds NP split-K partials of the in_proj output, pstride floats
// apart, summed as they are read.  tailp (if not null): the gate columns
// (off_b .. and off_a .., at or past tail_c0) are tail_np partials
// tailp[z][n][col - tail_c0] instead, tail_ps floats apart, rows of tail_ld.
template <int NP>
__global__ __launch_bounds__(256) void k_gdn_conv_prefill(
        const float *proj, int64_t stride, int64_t pstride, float *ring, const float *cw, float *out,
        int convDim, int nqk_rows, int N, float eps, int off_b, int off_a, const float *dt,
        const float *aNeg, float *beta, float *g, int nV, const float *tailp, int tail_c0,
        int tail_ld, int tail_np, int64_t tail_ps) {
    const int nrows = convDim / HD;
    const int64_t task = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int ngroups = (N + CT - 1) / CT;
    if (task >= (int64_t)nrows * ngroups) return;
    const int r = (int)(task % nrows), n0 = (int)(task / nrows) * CT;
    const int lane = threadIdx.x & 63;
    const int c[2] = {r * HD + lane, r * HD + 64 + lane};
    // Every load of both channels goes out before any value is used: the
    // weights, then both candidates of every window slot at clamped,
    // in-range addresses (the value is selected afterwards; loads under a
    // branch each waited for the one before).
    float w[2][4], win[2][CT + 3], pr[2][CT + 3], rr[2][3];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const f32x4 wv = *(const f32x4 *)(cw + (int64_t)c[h] * 4);
        w[h][0] = wv[0]; w[h][1] = wv[1]; w[h][2] = wv[2]; w[h][3] = wv[3];
#pragma unroll
        for (int j = 0; j < CT + 3; j++)
            pr[h][j] = psum<NP>(proj, pstride, (int64_t)min(max(n0 - 3 + j, 0), N - 1) * stride + c[h]);
#pragma unroll
        for (int j = 0; j < 3; j++) rr[h][j] = ring[(int64_t)j * convDim + c[h]];
    }
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int j = 0; j < CT + 3; j++) {
            const int m = n0 - 3 + j;            // token of window slot j
            win[h][j] = m < 0 ? rr[h][3 + m < 0 ? 0 : 3 + m] : m < N ? pr[h][j] : 0.f;
        }
    const bool norm = r < nqk_rows;
#pragma unroll
    for (int t = 0; t < CT; t++) {
        float v[2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            float acc = 0.0f;
            acc += win[h][t] * w[h][0];
            acc += win[h][t + 1] * w[h][1];
            acc += win[h][t + 2] * w[h][2];
            acc += win[h][t + 3] * w[h][3];
            v[h] = gd_silu(acc);
        }
        if (norm) {                              // wave-uniform
            float ss = 0.0f;
            ss += v[0] * v[0];
            ss += v[1] * v[1];
            ss = gd_wave_sum(ss);
            const float sc = 1.0f / sqrtf(ss + eps);
            v[0] *= sc;
            v[1] *= sc;
        }
        if (n0 + t < N) {
            out[(int64_t)(n0 + t) * convDim + c[0]] = v[0];
            out[(int64_t)(n0 + t) * convDim + c[1]] = v[1];
        }
    }
    if (n0 == 0) {
        // New ring: the inputs of tokens N-3 .. N-1, the old ring where those
        // precede token 0 (in win: slot j holds token j - 3).
#pragma unroll
        for (int h = 0; h < 2; h++) {
            float nr[3];
#pragma unroll
            for (int j = 0; j < 3; j++) {
                const int m = N - 3 + j;
                nr[j] = m < 0 ? win[h][3 + m] : psum<NP>(proj, pstride, (int64_t)m * stride + c[h]);
            }
#pragma unroll
            for (int j = 0; j < 3; j++) ring[(int64_t)j * convDim + c[h]] = nr[j];
        }
    }
    if (r == 0) {
        // Gate input column col of token n, its partials added in split order.
        // Up to TAIL_MAX partials, every load issued before the first add
        // (a loop to a runtime count waited for each load in turn).
        auto gin = [&](int n, int col) {
            if (tailp) {
                const float *tp = tailp + (int64_t)n * tail_ld + (col - tail_c0);
                float v[TAIL_MAX];
#pragma unroll
                for (int p = 0; p < TAIL_MAX; p++) v[p] = tp[(int64_t)min(p, tail_np - 1) * tail_ps];
                float a = v[0];
#pragma unroll
                for (int p = 1; p < TAIL_MAX; p++) a += p < tail_np ? v[p] : 0.f;
                return a;
            }
            return psum<NP>(proj, pstride, (int64_t)n * stride + col);
        };
        for (int i = lane; i < CT * nV; i += 64) {
            const int n = n0 + i / nV, hh = i % nV;
            if (n >= N) break;
            beta[(int64_t)n * nV + hh] = gd_sigmoid(gin(n, off_b + hh));
            g[(int64_t)n * nV + hh] = gd_softplus(gin(n, off_a + hh) + dt[hh]) * aNeg[hh];
        }
    }
}

// o <- rmsnorm_d(o) * w * silu(z), written as f16 for the out projection
// (GDN.swift:113-115).  One wave per (token, value head).
// Decode step of one recurrent layer for one value head, when every value
// head has its own q/k head (nK == nV, so no two workgroups touch the same
// conv channel): causal conv + SiLU of the head's q, k and v channels
// (advancing their conv ring), gate, L2 norms of q and k, the delta-rule
// state update, and the gated RMS norm of the output into f16.  The same
// arithmetic as k_conv4 + gd_gdn_decode (GATE, NORM) + k_onorm_silu, in one
// launch (GDN.swift:71-109, BonsaiEngine.swift:98-139).  16 waves: lane l of
// wave w owns value columns l and l + 64 and key rows 8w .. 8w+7, so each
// thread streams 16 state values and four waves per SIMD hide the latency.
constexpr int GS_W = 16, GS_R = HD / GS_W;       // waves, key rows per wave
constexpr int GS_COLS = 4;                       // k_gdn_step_cols: workgroups per head
__global__ __launch_bounds__(64 * GS_W) void k_gdn_step(
        const float *proj, float *ring, const float *cw, const float *dt, const float *aNeg,
        float *S, const float *onw, uint16_t *out, int convDim, int keyDim, int off_z, int off_b,
        int off_a, float qScale, float eps) {
    __shared__ float kq[2][HD];                  // k, q after conv + SiLU
    __shared__ float vs[HD];
    __shared__ float red[GS_W][2][64];           // S^T k partials
    __shared__ float red2[GS_W][2][64];          // readout partials
    __shared__ float gate[2];                    // beta, gamma
    __shared__ float nsq[4];                     // |q|^2, |k|^2 halves
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    float *Sh = S + (int64_t)h * HD * HD;
    // The gated norm's inputs (wave 0, at the end) are requested first, so
    // they are in registers by then.
    const float *zr = proj + off_z + h * HD;
    const float zv0 = wave == 0 ? zr[lane] : 0.f, zv1 = wave == 0 ? zr[lane + 64] : 0.f;
    const float nw0 = wave == 0 ? onw[lane] : 0.f, nw1 = wave == 0 ? onw[lane + 64] : 0.f;
    // State loads first: they are the bandwidth.
    float s0[GS_R], s1[GS_R];
#pragma unroll
    for (int r = 0; r < GS_R; r++) {
        s0[r] = Sh[(int64_t)(wave * GS_R + r) * HD + lane];
        s1[r] = Sh[(int64_t)(wave * GS_R + r) * HD + lane + 64];
    }
    auto conv = [&](int c) {
        const float w0 = cw[c * 4], w1 = cw[c * 4 + 1], w2 = cw[c * 4 + 2], w3 = cw[c * 4 + 3];
        const float r0 = ring[c], r1 = ring[convDim + c], r2 = ring[2 * convDim + c];
        const float cur = proj[c];
        float acc = 0.0f;
        acc += r0 * w0;
        acc += r1 * w1;
        acc += r2 * w2;
        acc += cur * w3;
        ring[c] = r1;
        ring[convDim + c] = r2;
        ring[2 * convDim + c] = cur;
        return gd_silu(acc);
    };
    // Threads 0..127: q channel tid; 128..255: k channel tid - 128;
    // 256..383: v channel tid - 256.
    if (tid < 3 * HD) {
        const int part = tid / HD, i = tid % HD;
        const float y = conv(part * keyDim + h * HD + i);
        if (part < 2) kq[1 - part][i] = y;
        else vs[i] = y;
        if (wave < 4) {       // q (waves 0, 1) and k (2, 3): this half's sum of squares
            const float ss = gd_wave_sum(y * y);
            if (lane == 0) nsq[wave] = ss;
        }
    } else if (tid == 3 * HD) {
        gate[0] = gd_sigmoid(proj[off_b + h]);
        gate[1] = expf(gd_softplus(proj[off_a + h] + dt[h]) * aNeg[h]);
    }
    __syncthreads();
    const float rk = 1.0f / sqrtf((nsq[2] + nsq[3]) + eps);
    const float beta = gate[0], gam = gate[1];
    float sk0 = 0.0f, sk1 = 0.0f;
#pragma unroll
    for (int r = 0; r < GS_R; r++) {
        const float kv = kq[0][wave * GS_R + r];
        s0[r] *= gam;
        s1[r] *= gam;
        sk0 = fmaf(s0[r], kv, sk0);
        sk1 = fmaf(s1[r], kv, sk1);
    }
    red[wave][0][lane] = sk0;
    red[wave][1][lane] = sk1;
    __syncthreads();
    sk0 = 0.0f;
    sk1 = 0.0f;
#pragma unroll
    for (int w = 0; w < GS_W; w++) {
        sk0 += red[w][0][lane];
        sk1 += red[w][1][lane];
    }
    sk0 *= rk;
    sk1 *= rk;
    const float d0 = beta * (vs[lane] - sk0) * rk, d1 = beta * (vs[lane + 64] - sk1) * rk;
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int r = 0; r < GS_R; r++) {
        const int i = wave * GS_R + r;
        const float kv = kq[0][i], qv = kq[1][i];
        s0[r] = fmaf(kv, d0, s0[r]);
        s1[r] = fmaf(kv, d1, s1[r]);
        a0 = fmaf(s0[r], qv, a0);
        a1 = fmaf(s1[r], qv, a1);
        Sh[(int64_t)i * HD + lane] = s0[r];
        Sh[(int64_t)i * HD + lane + 64] = s1[r];
    }
    red2[wave][0][lane] = a0;
    red2[wave][1][lane] = a1;
    __syncthreads();
    if (wave == 0) {
        float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
        for (int w = 0; w < GS_W; w++) {
            o0 += red2[w][0][lane];
            o1 += red2[w][1][lane];
        }
        const float rq = 1.0f / sqrtf((nsq[0] + nsq[1]) + eps);
        o0 *= rq * qScale;
        o1 *= rq * qScale;
        const float ss = gd_wave_sum(o0 * o0 + o1 * o1);
        const float sc = 1.0f / sqrtf(ss / (float)HD + eps);
        out[h * HD + lane] = gd_f2h(o0 * sc * nw0 * gd_silu(zv0));
        out[h * HD + lane + 64] = gd_f2h(o1 * sc * nw1 * gd_silu(zv1));
    }
}

// k_gdn_step's state update split over NS workgroups per value head, each
// owning 128/NS value columns of the head's state, so the state streams
// through NS times as many CUs.  Every workgroup forms the head's q and k
// (conv + SiLU, the same per-channel arithmetic and the same per-wave norm
// sums) and its own columns' v, and leaves the rest to its neighbours: the
// conv ring is read here and advanced by the out_proj launch that follows
// (gd_gemv_mfma_gated's side task), and the output goes out as f32 o (times
// 1/|q| and qScale) with the gate g = onw * silu(z) of each column, for that
// launch's x staging to apply the gated head norm (o * rs * g).
// Thread (rg, col): rows 8 rg .. 8 rg + 7 of column col, so the S^T k and
// readout sums run over the same row groups in the same order as
// k_gdn_step's waves: o is bit-identical to its pre-norm output.
template <int NS>
__global__ __launch_bounds__(16 * (HD / NS)) void k_gdn_step_cols(
        const float *proj, const float *ring, const float *cw, const float *dt, const float *aNeg,
        float *S, const float *onw, float *o_out, float *g_out, int convDim, int keyDim, int off_z,
        int off_b, int off_a, float qScale, float eps) {
    constexpr int NC = HD / NS;                  // value columns of this workgroup
    static_assert(16 * NC >= 2 * HD + NC + 1, "threads for the q/k/v conv and the gates");
    __shared__ float kq[2][HD];                  // k, q after conv + SiLU
    __shared__ float vs[NC];
    __shared__ float red[16][NC];                // S^T k partials by row group
    __shared__ float red2[16][NC];               // readout partials
    __shared__ float gate[2];                    // beta, gamma
    __shared__ float nsq[4];                     // |q|^2, |k|^2 halves
    const int h = blockIdx.x, c0 = blockIdx.y * NC, tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = tid % NC, rg = tid / NC;
    float *Sh = S + (int64_t)h * HD * HD;
    // The gate of this column (row group 0 writes it with o).
    const float zc = rg == 0 ? proj[off_z + h * HD + c0 + col] : 0.f;
    const float wc = rg == 0 ? onw[c0 + col] : 0.f;
    // State loads first: they are the bandwidth.
    float sv[8];
#pragma unroll
    for (int r = 0; r < 8; r++) sv[r] = Sh[(int64_t)(8 * rg + r) * HD + c0 + col];
    auto conv = [&](int c) {
        const float w0 = cw[c * 4], w1 = cw[c * 4 + 1], w2 = cw[c * 4 + 2], w3 = cw[c * 4 + 3];
        const float r0 = ring[c], r1 = ring[convDim + c], r2 = ring[2 * convDim + c];
        const float cur = proj[c];
        float acc = 0.0f;
        acc += r0 * w0;
        acc += r1 * w1;
        acc += r2 * w2;
        acc += cur * w3;
        return gd_silu(acc);
    };
    // Threads 0..127: q channel tid; 128..255: k channel tid - 128; then
    // this workgroup's NC v channels, then the gates.
    if (tid < 2 * HD) {
        const int part = tid / HD, i = tid % HD;
        const float y = conv(part * keyDim + h * HD + i);
        kq[1 - part][i] = y;
        const float ss = gd_wave_sum(y * y);      // waves 0, 1: q; 2, 3: k
        if (lane == 0) nsq[wave] = ss;
    } else if (tid < 2 * HD + NC) {
        vs[tid - 2 * HD] = conv(2 * keyDim + h * HD + c0 + tid - 2 * HD);
    } else if (tid == 2 * HD + NC) {
        gate[0] = gd_sigmoid(proj[off_b + h]);
        gate[1] = expf(gd_softplus(proj[off_a + h] + dt[h]) * aNeg[h]);
    }
    __syncthreads();
    const float rk = 1.0f / sqrtf((nsq[2] + nsq[3]) + eps);
    const float beta = gate[0], gam = gate[1];
    float sk = 0.0f;
#pragma unroll
    for (int r = 0; r < 8; r++) {
        sv[r] *= gam;
        sk = fmaf(sv[r], kq[0][8 * rg + r], sk);
    }
    red[rg][col] = sk;
    __syncthreads();
    sk = 0.0f;
#pragma unroll
    for (int g = 0; g < 16; g++) sk += red[g][col];
    sk *= rk;
    const float d = beta * (vs[col] - sk) * rk;
    float a = 0.0f;
#pragma unroll
    for (int r = 0; r < 8; r++) {
        const int i = 8 * rg + r;
        sv[r] = fmaf(kq[0][i], d, sv[r]);
        a = fmaf(sv[r], kq[1][i], a);
        Sh[(int64_t)i * HD + c0 + col] = sv[r];
    }
    red2[rg][col] = a;
    __syncthreads();
    if (rg == 0) {
        float o = 0.0f;
#pragma unroll
        for (int g = 0; g < 16; g++) o += red2[g][col];
        const float rq = 1.0f / sqrtf((nsq[0] + nsq[1]) + eps);
        o_out[h * HD + c0 + col] = o * (rq * qScale);
        g_out[h * HD + c0 + col] = wc * gd_silu(zc);
    }
}

// proj holds NP split-K partials of the in_proj output, pstride floats
// apart, summed here in split order (as q2_0_gemm_reduce sums them).
template <int NP>
__global__ void k_onorm_silu(const float *o, const float *proj, int64_t stride, int64_t pstride,
                             int off_z, const float *w, uint16_t *out, int nV, int N, float eps) {
    const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= N * nV) return;
    const int lane = threadIdx.x & 63;
    const int n = row / nV, h = row % nV;
    const float *r = o + (int64_t)row * HD;
    const float a = r[lane], b = r[lane + 64];
    const float ss = gd_wave_sum(a * a + b * b);
    const float s = 1.0f / sqrtf(ss / (float)HD + eps);
    const float *z = proj + (int64_t)n * stride + off_z + h * HD;
    float z0 = z[lane], z1 = z[lane + 64];
#pragma unroll
    for (int p = 1; p < NP; p++) {
        z0 += z[p * pstride + lane];
        z1 += z[p * pstride + lane + 64];
    }
    uint16_t *dst = out + (int64_t)row * HD;
    dst[lane] = gd_f2h(a * s * w[lane] * gd_silu(z0));
    dst[lane + 64] = gd_f2h(b * s * w[lane + 64] * gd_silu(z1));
}

// Greedy pick: index of the first maximum (BonsaiEngine.argmax, :187-191).
// Pass 1: per-block (max, first index) pairs; pass 2 (one block) reduces them.
__device__ __forceinline__ void argmax_merge(float &best, int &idx, float ob, int oi) {
    if (ob > best || (ob == best && oi < idx)) { best = ob; idx = oi; }
}

__device__ void argmax_block(float best, int idx, float *bv, int *bi, float *ob, int *oi) {
    for (int o = 32; o >= 1; o >>= 1)
        argmax_merge(best, idx, __shfl_xor(best, o, 64), __shfl_xor(idx, o, 64));
    if ((threadIdx.x & 63) == 0) { bv[threadIdx.x >> 6] = best; bi[threadIdx.x >> 6] = idx; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < (int)(blockDim.x >> 6); w++) argmax_merge(best, idx, bv[w], bi[w]);
        *ob = best;
        *oi = idx;
    }
}

constexpr int AMAX_BLOCKS = 128;
__global__ __launch_bounds__(256) void k_argmax_part(const float *v, int n, float *pv, int *pi) {
    __shared__ float bv[4];
    __shared__ int bi[4];
    float best = -INFINITY;
    int idx = 0x7fffffff;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += AMAX_BLOCKS * 256)
        argmax_merge(best, idx, v[i], i);
    argmax_block(best, idx, bv, bi, pv + blockIdx.x, pi + blockIdx.x);
}

// The pick goes to *out and to picks[*pos] (the pick made at that position),
// then the position advances by n.
__global__ __launch_bounds__(128) void k_argmax_final(const float *pv, const int *pi,
                                                      int32_t *out, int32_t *picks,
                                                      int32_t *pos, int n) {
    __shared__ float bv[2];
    __shared__ int bi[2];
    __shared__ float fb;
    __shared__ int fi;
    argmax_block(pv[threadIdx.x], pi[threadIdx.x], bv, bi, &fb, &fi);
    if (threadIdx.x == 0) {
        *out = fi;
        picks[*pos] = fi;
        *pos += n;
    }
}

// x += y over rows of n, then y16 = rmsnorm(x) * w as f16 (the residual add
// and the following norm, BonsaiEngine.swift:169-171).  One block per row.
// x += sum of the nsplit partials y + z * ystride (split-K GEMM output),
// then out = f16(rmsnorm(x) * w).  y may be null (norm only).
__global__ __launch_bounds__(1024) void k_add_rmsnorm(float *x, const float *y, const float *w,
                                                      uint16_t *out, int n, float eps,
                                                      int nsplit, int64_t ystride) {
    // Thread t holds elements 4t + 4096 k (k < 4, n <= 16384) in registers
    // between the sum and the normalization, so h is read and written once.
    __shared__ float red[16];
    const int64_t row = blockIdx.x;
    float *xr = x + row * n;
    const float *yr = y ? y + row * n : nullptr;
    float ss = 0.f;
    f32x4 v[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int i = threadIdx.x * 4 + k * 4096;
        if (i < n) {
            f32x4 a = *(const f32x4 *)(xr + i);
            if (yr) {
                for (int z = 0; z < nsplit; z++) a += *(const f32x4 *)(yr + z * ystride + i);
                *(f32x4 *)(xr + i) = a;
            }
            ss += a[0] * a[0] + a[1] * a[1] + a[2] * a[2] + a[3] * a[3];
            v[k] = a;
        }
    }
    ss = gd_block_sum(ss, red);
    const float s = 1.0f / sqrtf(ss / (float)n + eps);
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int i = threadIdx.x * 4 + k * 4096;
        if (i < n) {
            const f32x4 a = v[k];
            const f32x4 ww = *(const f32x4 *)(w + i);
            const uint32_t lo = (uint32_t)gd_f2h(a[0] * s * ww[0]) | ((uint32_t)gd_f2h(a[1] * s * ww[1]) << 16);
            const uint32_t hi = (uint32_t)gd_f2h(a[2] * s * ww[2]) | ((uint32_t)gd_f2h(a[3] * s * ww[3]) << 16);
            *(u32x2 *)(out + row * n + i) = u32x2{lo, hi};   // n % 4 == 0: 8-byte aligned
        }
    }
}

}  // namespace

// --------------------------------------------------------------- host side

struct StackLayer {
    bool rec = false;
    float *attn_norm = nullptr, *post_norm = nullptr;
    gd_q2w in_proj{}, out_proj{}, gate_up{}, down{};
    // GDN
    float *conv_w = nullptr, *dt = nullptr, *a_neg = nullptr, *ssm_norm = nullptr;
    float *conv_state = nullptr, *rec_state = nullptr;
    // attention
    float *q_norm = nullptr, *k_norm = nullptr;
    int att = -1;                // attention ordinal: this layer's K and V pools in KvPool
};

// Paged KV memory of a stack (MetalKVPool, MetalKVPool.swift:1-120, on one
// device allocation per pool): per attention layer one K and one V pool of
// `cap` physical pages of kv_block positions x kv_dim halves.  One logical
// -> physical page table serves every attention layer, since they append in
// lockstep.  A page is held by the live table and by bookmarks (`refs`); a
// completed page is never written again, so a bookmark shares it and copies
// only a partially filled tail page, and a restore gives the live table its
// own copy of that tail (MetalKVPool.snapshot / restore, :95-120).  When no
// page is free the pools double (a device copy of the pages so far), so
// memory follows the context in use and what bookmarks hold.  Bookmarks own a
// reference to the pool: it outlives the stack while any of them lives.
struct KvPool {
    gd_ctx *ctx = nullptr;
    int block = 0;                     // positions per page
    size_t page_elems = 0;             // halves per page
    int cap = 0;                       // physical pages per pool
    std::vector<uint16_t *> k, v;      // [attention layers] pools of cap pages
    std::vector<int> refs;             // [cap] holders of each page
    std::vector<int32_t> free;         // pages with no holder (popped from the back)
    uint64_t generation = 0;           // bumped whenever the pools move

    ~KvPool() {
        for (uint16_t *p : k) if (p) gd_free(ctx, p);
        for (uint16_t *p : v) if (p) gd_free(ctx, p);
    }
    // Capacity at least `want` pages (doubling), the held pages copied over.
    int grow(int want) {
        const int ncap = std::max(want, 2 * cap);
        std::vector<uint16_t *> nk(k.size(), nullptr), nv(v.size(), nullptr);
        const size_t bytes = (size_t)ncap * page_elems * 2, old = (size_t)cap * page_elems * 2;
        int rc = GD_OK;
        for (size_t a = 0; rc == GD_OK && a < k.size(); a++) {
            if ((rc = gd_alloc(ctx, bytes, (void **)&nk[a])) == GD_OK)
                rc = gd_alloc(ctx, bytes, (void **)&nv[a]);
            if (rc == GD_OK && old && (rc = gd_copy(ctx, nk[a], k[a], old)) == GD_OK)
                rc = gd_copy(ctx, nv[a], v[a], old);
        }
        if (rc == GD_OK) rc = gd_sync(ctx);
        if (rc) {
            for (uint16_t *p : nk) if (p) gd_free(ctx, p);
            for (uint16_t *p : nv) if (p) gd_free(ctx, p);
            return rc;
        }
        for (size_t a = 0; a < k.size(); a++) {
            if (k[a]) gd_free(ctx, k[a]);
            if (v[a]) gd_free(ctx, v[a]);
            k[a] = nk[a];
            v[a] = nv[a];
        }
        refs.resize(ncap, 0);
        for (int p = ncap - 1; p >= cap; p--) free.push_back(p);   // low pages first
        cap = ncap;
        generation++;
        return GD_OK;
    }
    // A free page, held once (the pools grow when none is free).
    int take(int32_t *page) {
        if (free.empty()) {
            const int rc = grow(cap + 1);
            if (rc) return rc;
        }
        *page = free.back();
        free.pop_back();
        refs[*page] = 1;
        return GD_OK;
    }
    void hold(int32_t p) { refs[p]++; }
    void drop(int32_t p) {
        if (--refs[p] == 0) free.push_back(p);
    }
    int held() const { return cap - (int)free.size(); }
    // Page dst of this pool <- page src of `from` (every attention layer's K and V).
    int copy_page(int32_t dst, const KvPool &from, int32_t src) {
        const size_t b = page_elems * 2;
        int rc = GD_OK;
        for (size_t a = 0; rc == GD_OK && a < k.size(); a++) {
            if ((rc = gd_copy(ctx, k[a] + (size_t)dst * page_elems, from.k[a] + (size_t)src * page_elems,
                              b)) == GD_OK)
                rc = gd_copy(ctx, v[a] + (size_t)dst * page_elems, from.v[a] + (size_t)src * page_elems, b);
        }
        return rc;
    }
};

// K splits of the GDN in_proj's tail rows (the gate columns past its whole
// row tiles, gd_gemm_launch_tail): 40 blocks of K at the stack's width make
// 5-block units, short enough to hide beside the full-K units.
constexpr int TAIL_SPLITS = 8;

struct gd_stack {
    gd_ctx *ctx = nullptr;
    gd_stack_config c{};
    int keyDim = 0, valDim = 0, convDim = 0, rp_rec = 0, rp_att = 0, max_pages = 0;
    std::vector<StackLayer> L;
    gd_q2w embd{};
    gd_q2w head{};               // lm_head: a copy of embd when tied (Model.swift:145)
    float *out_norm = nullptr;
    int32_t *page_table = nullptr;       // device: physical page of each logical page
    std::shared_ptr<KvPool> kv;
    std::vector<int32_t> live;           // the table's mapped entries (host copy)
    // scratch
    float *x = nullptr, *proj = nullptr, *conv_out = nullptr, *o32 = nullptr, *contrib = nullptr;
    float *beta = nullptr, *g = nullptr, *q32 = nullptr, *gate32 = nullptr, *logits = nullptr;
    float *attn_part = nullptr, *amax_v = nullptr;
    float *rope_tab = nullptr;           // [max_ctx][n_rot/2] (cos, sin), gd_rope_table
    int *amax_i = nullptr;
    uint16_t *xn16 = nullptr, *a16 = nullptr;
    int32_t *ids = nullptr, *dtok = nullptr;
    // dpos[0]: the next position; dpos[1]: the rope shift (rope position =
    // position + shift, MetalEngine.swift:432-435; nonzero only after a
    // bookmark of a state with image spans is restored).
    int32_t *dpos = nullptr;
    int32_t *picks = nullptr;    // picks[p]: the greedy pick made at position p
    int64_t pos = 0;
    int64_t rope_shift = 0;
    bool random = true;          // weights drawn from the seed (else loaded)
    bool have_pick = false;      // dtok holds the last greedy pick
    bool eager = false;          // generate: direct launches, not the graph
    std::atomic<bool> stop{false};
    std::vector<void *> allocs;
    hipGraphExec_t decode_exec = nullptr;
    hipGraph_t decode_graph = nullptr;
};

namespace {

int salloc(gd_stack *st, size_t bytes, void **p) {
    int rc = gd_alloc(st->ctx, bytes, p);
    if (rc == GD_OK) st->allocs.push_back(*p);
    return rc;
}

template <typename T>
int salloc_t(gd_stack *st, size_t count, T **p) {
    void *v = nullptr;
    int rc = salloc(st, count * sizeof(T), &v);
    *p = (T *)v;
    return rc;
}

// Weight allocation; with st->random set the weights are also filled from the
// seeded device streams, otherwise a loader fills them afterwards.
int q2w_make(gd_stack *st, int64_t K, int64_t R, uint64_t seed, gd_q2w *w) {
    int rc = gd_q2w_alloc(st->ctx, K, R, w);
    if (rc) return rc;
    st->allocs.push_back(w->codes);
    st->allocs.push_back(w->scales);
    return st->random ? gd_rand_q2w(st->ctx, w, seed, 0.01f, 0.05f) : GD_OK;
}

int f32_make(gd_stack *st, int64_t n, uint64_t seed, float lo, float hi, float **p) {
    int rc = salloc_t(st, (size_t)n, p);
    if (rc) return rc;
    return st->random ? gd_rand_uniform(st->ctx, *p, (size_t)n, seed, lo, hi) : GD_OK;
}

// One chunk of N tokens whose embeddings are already in st->x (f32 [N][E]):
// the layer stack, the final norm and the last token's logits + greedy pick.
// Positions come from st->dpos.  `decode` selects the single-token kernels.
int forward(gd_stack *st, int N, bool decode) {
    gd_ctx *ctx = st->ctx;
    const gd_stack_config &c = st->c;
    const int E = c.n_embd, FF = c.n_ff, H = c.n_head, HKV = c.n_head_kv;
    const int nV = c.n_v_head, nK = c.n_k_head;
    const float eps = c.eps, qScale = 1.0f / sqrtf((float)c.d_state);
    hipStream_t s = ctx->stream;
    int rc;
#define R_(call) do { if ((rc = (call)) != GD_OK) return rc; } while (0)
#define K_(name, ...) do { hipLaunchKernelGGL(name, __VA_ARGS__); GD_LAUNCHED(ctx, #name); } while (0)
    // Prefill: attn_norm of layer 0 here; every later norm is fused with the
    // residual add that precedes it (k_add_rmsnorm).  Decode: the projections
    // into the residual (out_proj, down) may split K into nd partials, the
    // first of which carries the residual x as its bias; the next fused-norm
    // GEMV sums the partials, normalizes in its x staging and writes the sum
    // back to x (which no kernel reads by then).
    int nd = 0;
    // Decode GDN layers whose value heads each have their own q/k head and a
    // 128-dim state: the state update split over workgroups by columns.
    const bool gdn_cols = decode && nK == nV && c.d_state == HD && st->valDim == nV * HD;
    auto consume = [&](const gd_q2w *w, const float *normw, float *hout, float *y,
                       uint16_t *glu) {
        return gd_gemv_mfma_norm(ctx, w, st->contrib, nd > 1 ? st->contrib + E : nullptr, nd - 1,
                                 E, normw, eps, hout, y, glu);
    };
    if (!decode)
        K_(k_add_rmsnorm, dim3(N), dim3(1024), 0, s, st->x, (const float *)nullptr,
           st->L[0].attn_norm, st->xn16, E, eps, 0, (int64_t)0);
    for (int il = 0; il < c.n_layer; il++) {
        StackLayer &ly = st->L[il];
        const int RP = ly.rec ? st->rp_rec : st->rp_att;
        // in_proj output: proj, or np split-K partials of it at pin.
        const float *pin = st->proj;
        int np = 1;
        // Gate columns left as tail partials by the in_proj GEMM (prefill).
        const float *tailp = nullptr;
        int tail_np = 0, tail_r0 = 0;
        if (decode) {
            if (il == 0)
                R_(gd_gemv_mfma_norm(ctx, &ly.in_proj, st->x, nullptr, 0, 0, ly.attn_norm, eps,
                                     nullptr, st->proj));
            else
                R_(consume(&ly.in_proj, ly.attn_norm, st->x, st->proj, nullptr));
        } else if (ly.rec) {
            // A split-K plan leaves its partials in contrib (free between the
            // residual add and out_proj); the conv front end and the gated
            // norm sum them as they read (up to 4, as contrib allows).
            const gd_gemm_plan pi = gd_gemm_choose(ctx, N, ly.in_proj.K, ly.in_proj.R, GD_F16);
            // An unsplit plan whose row tiles stop short of R by no more
            // than the gate columns (b, a: the last 2 nV rows) leaves those
            // as K-split tail partials in contrib (free until out_proj).
            const int tile_rows = pi.nw * pi.nt * 32;
            const int off_b = st->convDim + st->valDim;
            const int64_t r0 = (int64_t)ly.in_proj.R / tile_rows * tile_rows;
            if (pi.split > 1 && pi.split <= 4 &&
                (size_t)pi.split * N * RP <= (size_t)8 * st->c.max_batch * E) {
                R_(gd_gemm_launch(ctx, &ly.in_proj, N, st->xn16, GD_F16, st->contrib, GD_F32, pi));
                pin = st->contrib;
                np = pi.split;
            } else if (pi.split == 1 && !pi.ex && r0 < ly.in_proj.R && r0 >= off_b && TAIL_SPLITS <= TAIL_MAX &&
                       (size_t)TAIL_SPLITS * N * (ly.in_proj.R - r0) <= (size_t)8 * st->c.max_batch * E) {
                tail_np = TAIL_SPLITS;
                R_(gd_gemm_launch_tail(ctx, &ly.in_proj, N, st->xn16, st->proj, pi, st->contrib,
                                       &tail_np, &tail_r0));
                tailp = st->contrib;
            } else {
                R_(gd_q2_0_gemm(ctx, &ly.in_proj, N, st->xn16, GD_F16, st->proj, GD_F32));
            }
        } else {
            R_(gd_q2_0_gemm(ctx, &ly.in_proj, N, st->xn16, GD_F16, st->proj, GD_F32));
        }
        if (ly.rec) {
            const int off_z = st->convDim, off_b = off_z + st->valDim, off_a = off_b + nV;
            if (decode && nK == nV && c.d_state == HD) {
                if (gdn_cols) {
                    // The state over GS_COLS workgroups per head; the gated norm
                    // and the conv ring advance go with the out_proj below.
                    K_(k_gdn_step_cols<GS_COLS>, dim3(nV, GS_COLS), dim3(16 * (HD / GS_COLS)), 0, s,
                       st->proj, ly.conv_state, ly.conv_w, ly.dt, ly.a_neg, ly.rec_state,
                       ly.ssm_norm, st->o32, st->o32 + st->valDim, st->convDim, st->keyDim, off_z,
                       off_b, off_a, qScale, eps);
                } else {
                    K_(k_gdn_step, dim3(nV), dim3(64 * GS_W), 0, s, st->proj, ly.conv_state,
                       ly.conv_w, ly.dt, ly.a_neg, ly.rec_state, ly.ssm_norm, st->a16, st->convDim,
                       st->keyDim, off_z, off_b, off_a, qScale, eps);
                }
            } else if (decode) {
                K_(k_conv4, dim3(gd_blocks(st->convDim, 256)), dim3(256), 0, s, st->proj,
                   (int64_t)RP, ly.conv_state, ly.conv_w, st->conv_out, st->convDim, 1);
                // Fused gate + L2 norm + delta-rule step, state in place.
                R_(gd_gdn_decode(ctx, 1, nV, nK, c.d_state, st->conv_out,
                                 st->conv_out + st->keyDim, st->conv_out + 2 * st->keyDim,
                                 GD_F32, st->proj + off_a, st->proj + off_b, ly.dt, ly.a_neg,
                                 ly.rec_state, st->o32, qScale, eps));
            } else {
                const int64_t tasks = (int64_t)(st->convDim / HD) * ((N + CT - 1) / CT);
                const int64_t pstr = (int64_t)N * RP;
#define GD_CONV(NP_) K_(k_gdn_conv_prefill<NP_>, dim3(gd_blocks(tasks, 4)), dim3(256), 0, s, pin, \
                        (int64_t)RP, pstr, ly.conv_state, ly.conv_w, st->conv_out, st->convDim, \
                        2 * nK, N, eps, off_b, off_a, ly.dt, ly.a_neg, st->beta, st->g, nV, tailp, \
                        tail_r0, RP - tail_r0, tail_np, (int64_t)N * (RP - tail_r0))
                if (np == 1) GD_CONV(1); else if (np == 2) GD_CONV(2); else if (np == 3) GD_CONV(3); else GD_CONV(4);
#undef GD_CONV
                // Chunks of 32 tokens: the 32 x 32 UT transform is cheaper per token
                // than 64 x 64 and twice the (head, chunk) units fill the CUs; measured
                // faster for T 128..2048 and 16 or 48 heads (16 heads, T = 512:
                // 38.3 against 48.4 us, pp512 -1.8%).
                R_(gd_gdn_prefill(ctx, N, nV, nK, c.d_state, c.d_state, st->conv_out,
                                  st->convDim, st->conv_out + st->keyDim, st->convDim,
                                  st->conv_out + 2 * st->keyDim, st->convDim, GD_F32, st->g,
                                  st->beta, ly.rec_state, st->o32, st->valDim, GD_F32, qScale,
                                  32));
            }
            if (!(decode && nK == nV && c.d_state == HD))
            {
                const int64_t pstr = (int64_t)N * RP;
#define GD_ONORM(NP_) K_(k_onorm_silu<NP_>, dim3(gd_blocks((int64_t)N * nV, 4)), dim3(256), 0, s, \
                         st->o32, pin, (int64_t)RP, pstr, off_z, ly.ssm_norm, st->a16, nV, N, eps)
                if (np == 1) GD_ONORM(1); else if (np == 2) GD_ONORM(2); else if (np == 3) GD_ONORM(3); else GD_ONORM(4);
#undef GD_ONORM
            }
        } else {
            const int hd = c.head_dim;
            const float scale = 1.0f / sqrtf((float)hd);
            // Per-head q stride of the projection rows: the hybrid's fused
            // [q | gate] pairs, or the dense model's plain q (ungated).
            const int qs = c.dense ? hd : 2 * hd;
            uint16_t *kc = st->kv->k[ly.att], *vc = st->kv->v[ly.att];
            if (decode) {
                // One token: q/k preparation and the cache append happen
                // inside the attention launch.
                R_(gd_attn_decode_launch(ctx, hd, st->proj, qs, ly.q_norm, ly.k_norm, kc, vc,
                                         st->page_table, st->dpos, st->attn_part, st->a16, H, HKV,
                                         c.kv_block, scale, c.n_rot, c.rope_base, eps, st->rope_tab,
                                         c.max_ctx));
            } else {
                // The prefill normalizes and rotates q from the projection
                // rows itself where each rotation pair lies in one of its
                // lanes (n_rot a multiple of 64); prep then appends k, v only.
                const bool rawq = c.n_rot % 64 == 0;
                R_(gd_attn_prep_launch(ctx, hd, st->proj, (int64_t)RP, qs, ly.q_norm, ly.k_norm, st->q32,
                                       st->gate32, kc, vc, st->page_table, st->dpos, N, H,
                                       HKV, c.n_rot, c.rope_base, c.kv_block, eps, st->rope_tab, c.max_ctx,
                                       rawq ? H : 0));
                if (rawq)
                    R_(gd_attn_prefill_launch(ctx, hd, st->proj, st->proj + hd, (int64_t)RP, qs,
                                              ly.q_norm, c.n_rot, c.rope_base, eps, st->rope_tab,
                                              c.max_ctx, kc, vc, st->page_table, st->dpos, 0,
                                              st->a16, GD_F16, H, HKV, N, c.kv_block, scale,
                                              c.dense ? 0 : 1));
                else
                    R_(gd_attn_prefill_launch(ctx, hd, st->q32, st->gate32, (int64_t)H * hd, hd,
                                              nullptr, 0, 0.f, 0.f, nullptr, 0, kc, vc,
                                              st->page_table, st->dpos, 0, st->a16, GD_F16, H, HKV,
                                              N, c.kv_block, scale, c.dense ? 0 : 1));
            }
        }
        // Output projections feed only the residual add: a split-K plan
        // leaves its partials in contrib and k_add_rmsnorm sums them.
        int nsplit = 1;
        if (decode && ly.rec && gdn_cols) {
            // x = f16(rmsnorm_128(o) * ssm_norm * silu(z)) staged by the GEMV;
            // its side task advances the conv ring the step read.
            nd = 1;
            R_(gd_gemv_mfma_gated(ctx, &ly.out_proj, st->o32, st->o32 + st->valDim, eps, st->contrib,
                                  st->x, ly.conv_state, st->proj, st->convDim, st->convDim));
        } else if (decode) {
            nd = gd_gemv_ksplit(ctx, ly.out_proj.K, ly.out_proj.R);
            R_(gd_gemv_mfma(ctx, &ly.out_proj, st->a16, GD_F16, st->contrib, nd, st->x));
        } else {
            const gd_gemm_plan p = gd_gemm_choose(ctx, N, ly.out_proj.K, ly.out_proj.R, GD_F16);
            GD_REQUIRE(ctx, p.split <= 8, "stack: %d split-K partials (contrib holds 8)", p.split);
            nsplit = p.split;
            R_(gd_gemm_launch(ctx, &ly.out_proj, N, st->a16, GD_F16, st->contrib, GD_F32, p));
        }
        // gate_up with SwiGLU in its epilogue: a16 = silu(gate x) * (up x).
        if (decode) {
            R_(consume(&ly.gate_up, ly.post_norm, st->x, st->proj, st->a16));
        } else {
            K_(k_add_rmsnorm, dim3(N), dim3(1024), 0, s, st->x, st->contrib, ly.post_norm,
               st->xn16, E, eps, nsplit, (int64_t)N * E);
            R_(gd_gemm_glu(ctx, &ly.gate_up, N, st->xn16, st->a16));
        }
        nsplit = 1;
        if (decode) {
            nd = gd_gemv_ksplit(ctx, ly.down.K, ly.down.R);
            R_(gd_gemv_mfma(ctx, &ly.down, st->a16, GD_F16, st->contrib, nd, st->x));
        } else {
            const gd_gemm_plan p = gd_gemm_choose(ctx, N, ly.down.K, ly.down.R, GD_F16);
            GD_REQUIRE(ctx, p.split <= 8, "stack: %d split-K partials (contrib holds 8)", p.split);
            nsplit = p.split;
            R_(gd_gemm_launch(ctx, &ly.down, N, st->a16, GD_F16, st->contrib, GD_F32, p));
        }
        if (decode) {
            // The next in_proj (or the lm_head) adds and normalizes.
        } else if (il + 1 < c.n_layer) {
            K_(k_add_rmsnorm, dim3(N), dim3(1024), 0, s, st->x, st->contrib,
               st->L[il + 1].attn_norm, st->xn16, E, eps, nsplit, (int64_t)N * E);
        } else {
            // Only the last token's hidden feeds the logits: residual add and
            // final norm on that row alone.
            const int64_t last = (int64_t)(N - 1) * E;
            K_(k_add_rmsnorm, dim3(1), dim3(1024), 0, s, st->x + last, st->contrib + last,
               st->out_norm, st->xn16, E, eps, nsplit, (int64_t)N * E);
        }
    }
    // lm_head on the last token, greedy pick, position bump.
    if (decode)
        R_(consume(&st->head, st->out_norm, nullptr, st->logits, nullptr));
    else
        R_(gd_q2_0_gemv(ctx, &st->head, st->xn16, GD_F16, st->logits));
    K_(k_argmax_part, dim3(AMAX_BLOCKS), dim3(256), 0, s, st->logits, c.n_vocab, st->amax_v,
       st->amax_i);
    K_(k_argmax_final, dim3(1), dim3(AMAX_BLOCKS), 0, s, st->amax_v, st->amax_i, st->dtok,
       st->picks, st->dpos, N);
#undef K_
#undef R_
    return GD_OK;
}

int finish(gd_stack *st, int32_t *next, float *logits) {
    gd_ctx *ctx = st->ctx;
    int rc;
    if (logits && (rc = gd_download(ctx, logits, st->logits, (size_t)st->c.n_vocab * 4))) return rc;
    if (next && (rc = gd_download(ctx, next, st->dtok, 4))) return rc;
    return GD_OK;
}

// The captured decode step holds the KV pools' addresses: dropped when the
// pools move, captured again by the next gd_stack_generate.
void drop_graph(gd_stack *st) {
    if (st->decode_exec) (void)hipGraphExecDestroy(st->decode_exec);
    if (st->decode_graph) (void)hipGraphDestroy(st->decode_graph);
    st->decode_exec = nullptr;
    st->decode_graph = nullptr;
}

// A page of the stack's own pool for the stack to write (its graph dropped
// if the pools grew).
int take_page(gd_stack *st, int32_t *page) {
    const uint64_t gen = st->kv->generation;
    const int rc = st->kv->take(page);
    if (st->kv->generation != gen) drop_graph(st);
    return rc;
}

// Every logical page of positions [0, upto) mapped to a page of the live
// table: fresh pages for the ones past its end, their table entries uploaded.
int map_pages(gd_stack *st, int64_t upto) {
    const int B = st->c.kv_block;
    const size_t need = (size_t)((upto + B - 1) / B), first = st->live.size();
    if (need <= first) return GD_OK;
    GD_REQUIRE(st->ctx, need <= (size_t)st->max_pages, "stack: %lld positions pass max_ctx %d",
               (long long)upto, st->c.max_ctx);
    while (st->live.size() < need) {
        int32_t p;
        const int rc = take_page(st, &p);
        if (rc) return rc;
        st->live.push_back(p);
    }
    return gd_upload(st->ctx, st->page_table + first, st->live.data() + first,
                     (need - first) * sizeof(int32_t));
}

// The live table emptied (its pages back to the pool unless a bookmark holds them).
void release_live(gd_stack *st) {
    for (int32_t p : st->live) st->kv->drop(p);
    st->live.clear();
}

}  // namespace

extern "C" void gd_stack_destroy(gd_stack *st) {
    if (!st) return;
    drop_graph(st);
    if (st->kv) release_live(st);
    for (void *p : st->allocs) gd_free(st->ctx, p);
    delete st;
}


namespace {

// Allocate a stack of geometry *cfg.  random: draw every weight from `seed`
// (gd_stack_create); otherwise leave the weights for a loader.  untied: give
// the lm_head its own matrix instead of sharing the token embedding.
int create(gd_ctx *ctx, const gd_stack_config *cfg, uint64_t seed, bool random, bool untied,
           gd_stack **out) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, cfg && out, "gd_stack_create: null argument");
    const gd_stack_config &c = *cfg;
    GD_REQUIRE(ctx, c.n_layer > 0 && c.attn_interval > 0, "gd_stack_create: bad layer count");
    GD_REQUIRE(ctx, c.dense == 0 || c.dense == 1, "gd_stack_create: dense must be 0 or 1");
    GD_REQUIRE(ctx, c.head_dim == 128 || c.head_dim == 256,
               "gd_stack_create: head_dim must be 128 or 256");
    if (c.dense) {
        // Every layer attention (Model.swift:55-59): no GDN geometry.
        GD_REQUIRE(ctx, c.attn_interval == 1 && c.d_state == 0 && c.n_k_head == 0 &&
                        c.n_v_head == 0 && c.d_conv == 0,
                   "gd_stack_create: a dense stack has attn_interval 1 and d_state, n_k_head, "
                   "n_v_head, d_conv 0");
    } else {
        GD_REQUIRE(ctx, c.d_state == HD, "gd_stack_create: d_state must be 128");
        GD_REQUIRE(ctx, c.d_conv == 4, "gd_stack_create: d_conv must be 4");
        GD_REQUIRE(ctx, c.n_k_head > 0 && c.n_v_head % c.n_k_head == 0,
                   "gd_stack_create: n_v_head must be a multiple of n_k_head");
    }
    GD_REQUIRE(ctx, c.n_head > 0 && c.n_head_kv > 0 && c.n_head % c.n_head_kv == 0,
               "gd_stack_create: n_head must be a multiple of n_head_kv");
    GD_REQUIRE(ctx, c.n_rot > 0 && c.n_rot <= c.head_dim && c.n_rot % 2 == 0,
               "gd_stack_create: n_rot");
    GD_REQUIRE(ctx, c.n_embd % 128 == 0 && c.n_ff % 128 == 0 && c.n_vocab > 0,
               "gd_stack_create: n_embd and n_ff must be multiples of 128");
    GD_REQUIRE(ctx, c.n_embd <= 15744,
               "gd_stack_create: n_embd %d above 15744 (decode stages x one entry per thread)",
               c.n_embd);
    GD_REQUIRE(ctx, c.kv_block > 0 && c.max_ctx > 0 && c.max_batch > 0,
               "gd_stack_create: kv_block, max_ctx, max_batch must be positive");
    *out = nullptr;
    gd_stack *st = new gd_stack();
    st->ctx = ctx;
    st->c = c;
    st->random = random;
    st->keyDim = c.d_state * c.n_k_head;
    st->valDim = c.d_state * c.n_v_head;
    st->convDim = 2 * st->keyDim + st->valDim;
    st->rp_rec = st->convDim + st->valDim + 2 * c.n_v_head;
    const int hd = c.head_dim;
    st->rp_att = (c.dense ? 1 : 2) * c.n_head * hd + 2 * c.n_head_kv * hd;
    st->max_pages = (c.max_ctx + c.kv_block - 1) / c.kv_block;
    const int E = c.n_embd, FF = c.n_ff, B = c.max_batch;
    int rc = GD_OK;
#define C_(call) do { if ((rc = (call)) != GD_OK) { gd_stack_destroy(st); return rc; } } while (0)
    uint64_t sd = seed * 1000003ULL;
    auto next_seed = [&]() { sd += 2; return sd; };   // streams use seed and seed+1
    st->L.resize(c.n_layer);
    int natt = 0;
    for (int il = 0; il < c.n_layer; il++) {
        StackLayer &ly = st->L[il];
        ly.rec = (il + 1) % c.attn_interval != 0;     // Model.swift:37
        C_(f32_make(st, E, next_seed(), 0.8f, 1.2f, &ly.attn_norm));
        C_(f32_make(st, E, next_seed(), 0.8f, 1.2f, &ly.post_norm));
        if (ly.rec) {
            C_(q2w_make(st, E, st->rp_rec, next_seed(), &ly.in_proj));
            C_(q2w_make(st, st->valDim, E, next_seed(), &ly.out_proj));
            C_(f32_make(st, (int64_t)st->convDim * 4, next_seed(), -0.5f, 0.5f, &ly.conv_w));
            C_(f32_make(st, c.n_v_head, next_seed(), -0.5f, 0.5f, &ly.dt));
            C_(f32_make(st, c.n_v_head, next_seed(), -2.0f, -0.3f, &ly.a_neg));
            C_(f32_make(st, HD, next_seed(), 0.8f, 1.2f, &ly.ssm_norm));
            C_(salloc_t(st, (size_t)3 * st->convDim, &ly.conv_state));
            C_(salloc_t(st, (size_t)c.n_v_head * HD * HD, &ly.rec_state));
        } else {
            C_(q2w_make(st, E, st->rp_att, next_seed(), &ly.in_proj));
            C_(q2w_make(st, (int64_t)c.n_head * hd, E, next_seed(), &ly.out_proj));
            C_(f32_make(st, hd, next_seed(), 0.8f, 1.2f, &ly.q_norm));
            C_(f32_make(st, hd, next_seed(), 0.8f, 1.2f, &ly.k_norm));
            ly.att = natt++;
        }
        C_(q2w_make(st, E, 2 * (int64_t)FF, next_seed(), &ly.gate_up));
        C_(q2w_make(st, FF, E, next_seed(), &ly.down));
    }
    C_(q2w_make(st, E, c.n_vocab, next_seed(), &st->embd));
    C_(f32_make(st, E, next_seed(), 0.8f, 1.2f, &st->out_norm));
    if (untied)
        C_(q2w_make(st, E, c.n_vocab, next_seed(), &st->head));
    else
        st->head = st->embd;
    C_(salloc_t(st, (size_t)st->max_pages, &st->page_table));
    // KV pages start at twice what one prefill chunk fills (capped at
    // max_ctx) and grow on demand.
    st->kv = std::make_shared<KvPool>();
    st->kv->ctx = ctx;
    st->kv->block = c.kv_block;
    st->kv->page_elems = (size_t)c.kv_block * c.n_head_kv * hd;
    st->kv->k.assign(natt, nullptr);
    st->kv->v.assign(natt, nullptr);
    C_(st->kv->grow(std::min(st->max_pages, 2 * ((B + c.kv_block - 1) / c.kv_block + 1))));
    const int maxproj = std::max(std::max(st->rp_rec, st->rp_att), 2 * FF);
    C_(salloc_t(st, (size_t)B * E, &st->x));
    C_(salloc_t(st, (size_t)B * maxproj, &st->proj));
    C_(salloc_t(st, (size_t)B * st->convDim, &st->conv_out));
    // o32: prefill's GDN output rows; decode's o and gate (two rows).
    C_(salloc_t(st, (size_t)std::max(B, 2) * st->valDim, &st->o32));
    // Room for the split-K partials of the output projections (at most 8).
    C_(salloc_t(st, (size_t)8 * B * E, &st->contrib));
    C_(salloc_t(st, (size_t)B * c.n_v_head, &st->beta));
    C_(salloc_t(st, (size_t)B * c.n_v_head, &st->g));
    C_(salloc_t(st, (size_t)B * c.n_head * hd, &st->q32));
    C_(salloc_t(st, (size_t)B * c.n_head * hd, &st->gate32));
    C_(salloc_t(st, (size_t)c.n_vocab, &st->logits));
    C_(salloc_t(st, gd_attn_part_floats(hd, c.n_head), &st->attn_part));
    // Rotations of positions 0 .. max_ctx-1, formed once for every attention
    // layer and token (a restored rope shift may rotate past them: computed).
    C_(salloc_t(st, (size_t)c.max_ctx * c.n_rot, &st->rope_tab));
    C_(gd_rope_table(ctx, st->rope_tab, c.max_ctx, c.n_rot, c.rope_base));
    C_(salloc_t(st, (size_t)AMAX_BLOCKS, &st->amax_v));
    C_(salloc_t(st, (size_t)AMAX_BLOCKS, &st->amax_i));
    C_(salloc_t(st, (size_t)B * E, &st->xn16));
    const int a16n = std::max(std::max(st->valDim, c.n_head * hd), FF);
    C_(salloc_t(st, (size_t)B * a16n, &st->a16));
    C_(salloc_t(st, (size_t)B, &st->ids));
    C_(salloc_t(st, 2, &st->dpos));
    C_(salloc_t(st, 1, &st->dtok));
    C_(salloc_t(st, (size_t)c.max_ctx, &st->picks));
    C_(gd_stack_reset(st));
#undef C_
    *out = st;
    return GD_OK;
}

}  // namespace

extern "C" int gd_stack_create(gd_ctx *ctx, const gd_stack_config *cfg, uint64_t seed,
                               gd_stack **out) {
    return create(ctx, cfg, seed, true, false, out);
}

extern "C" int gd_stack_reset(gd_stack *st) {
    if (!st) return GD_EINVAL;
    gd_ctx *ctx = st->ctx;
    int rc;
    for (StackLayer &ly : st->L) {
        if (ly.rec) {
            if ((rc = gd_fill_u32(ctx, ly.conv_state, 0, (size_t)3 * st->convDim)) ||
                (rc = gd_fill_u32(ctx, ly.rec_state, 0, (size_t)st->c.n_v_head * HD * HD)))
                return rc;
        }
    }
    if ((rc = gd_fill_u32(ctx, st->dpos, 0, 2)) || (rc = gd_fill_u32(ctx, st->dtok, 0, 1)))
        return rc;
    release_live(st);
    st->pos = 0;
    st->rope_shift = 0;
    st->have_pick = false;
    st->stop.store(false);
    return gd_sync(ctx);
}

extern "C" int gd_stack_request_stop(gd_stack *st) {
    if (!st) return GD_EINVAL;
    st->stop.store(true);
    return GD_OK;
}

extern "C" int gd_stack_should_stop(gd_stack *st, int *raised) {
    if (!st || !raised) return GD_EINVAL;
    *raised = st->stop.load() ? 1 : 0;
    return GD_OK;
}

extern "C" int gd_stack_set_eager(gd_stack *st, int eager) {
    if (!st) return GD_EINVAL;
    GD_REQUIRE(st->ctx, eager == 0 || eager == 1, "gd_stack_set_eager: eager=%d not 0 or 1", eager);
    st->eager = eager != 0;
    return GD_OK;
}

extern "C" int gd_stack_prefill(gd_stack *st, const int32_t *ids, int n, int32_t *next,
                                float *logits) {
    if (!st) return GD_EINVAL;
    gd_ctx *ctx = st->ctx;
    GD_REQUIRE(ctx, ids && n > 0, "gd_stack_prefill: no tokens");
    GD_REQUIRE(ctx, st->pos + n <= st->c.max_ctx, "gd_stack_prefill: context %lld + %d > max_ctx %d",
               (long long)st->pos, n, st->c.max_ctx);
    for (int i = 0; i < n; i++)
        GD_REQUIRE(ctx, ids[i] >= 0 && ids[i] < st->c.n_vocab, "gd_stack_prefill: id %d out of vocab",
                   ids[i]);
    int rc;
    // A previous turn's stop must not end this one (MetalEngine.extend clears
    // the signal first, MetalEngine.swift:183-186); a stop raised while this
    // prefill runs is seen at the next chunk boundary and stays raised.
    st->stop.store(false);
    for (int i = 0; i < n; i += st->c.max_batch) {
        if (st->stop.load()) return gd_fail(ctx, GD_ESTOPPED, "prefill stopped");
        const int N = std::min(st->c.max_batch, n - i);
        if ((rc = map_pages(st, st->pos + N)) || (rc = gd_upload(ctx, st->ids, ids + i, (size_t)N * 4)) ||
            (rc = gd_q2_0_dequant_rows(ctx, &st->embd, st->ids, N, st->x)) ||
            (rc = forward(st, N, false)))
            return rc;
        st->pos += N;
        st->have_pick = true;
    }
    return finish(st, next, logits);
}

extern "C" int gd_stack_decode(gd_stack *st, int32_t token, int32_t *next, float *logits) {
    if (!st) return GD_EINVAL;
    gd_ctx *ctx = st->ctx;
    GD_REQUIRE(ctx, token >= 0 && token < st->c.n_vocab, "gd_stack_decode: token %d out of vocab",
               token);
    GD_REQUIRE(ctx, st->pos + 1 <= st->c.max_ctx, "gd_stack_decode: context full");
    int rc;
    if ((rc = map_pages(st, st->pos + 1)) || (rc = gd_upload(ctx, st->dtok, &token, 4))) return rc;
    if ((rc = gd_q2_0_dequant_rows(ctx, &st->embd, st->dtok, 1, st->x)) ||
        (rc = forward(st, 1, true)))
        return rc;
    st->pos += 1;
    st->have_pick = true;
    return finish(st, next, logits);
}

extern "C" int gd_stack_generate(gd_stack *st, int n, int32_t *tokens) {
    if (!st) return GD_EINVAL;
    gd_ctx *ctx = st->ctx;
    GD_REQUIRE(ctx, n >= 0 && tokens, "gd_stack_generate: bad arguments");
    GD_REQUIRE(ctx, st->pos + n <= st->c.max_ctx, "gd_stack_generate: context full");
    if (n == 0) return GD_OK;
    GD_REQUIRE(ctx, st->have_pick,
               "gd_stack_generate: no previous pick to continue from (prefill or decode first)");
    int rc;
    // An eager stack launches every step's kernels directly instead of
    // replaying the captured graph (same kernels and results; for profilers
    // that do not follow graph launches).
    const bool eager = st->eager;
    if ((rc = map_pages(st, st->pos + n))) return rc;
    // One decode step reads the previous pick from st->dtok, so the whole step
    // (embed .. argmax, position bump) replays with no host involvement.
    if (!st->decode_exec && !eager) {
        GD_HIP(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
        rc = gd_q2_0_dequant_rows(ctx, &st->embd, st->dtok, 1, st->x);
        if (rc == GD_OK) rc = forward(st, 1, true);
        hipGraph_t graph = nullptr;
        hipError_t e = hipStreamEndCapture(ctx->stream, &graph);
        if (rc != GD_OK) {
            if (graph) (void)hipGraphDestroy(graph);
            return rc;
        }
        if (e != hipSuccess) return gd_hip_fail(ctx, e, "decode graph capture");
        st->decode_graph = graph;
        GD_HIP(ctx, hipGraphInstantiate(&st->decode_exec, graph, nullptr, nullptr, 0));
    }
    // Each step records its pick at picks[position], so nothing syncs per
    // token; the picks are read back once at the end.  A raised stop ends the
    // loop before its next step (the decode loop's shouldStop gate).
    int done = 0;
    for (int i = 0; i < n; i++, done++) {
        if (st->stop.load()) break;
        if (eager) {
            if ((rc = gd_q2_0_dequant_rows(ctx, &st->embd, st->dtok, 1, st->x)) ||
                (rc = forward(st, 1, true)))
                return rc;
        } else {
            hipError_t e = hipGraphLaunch(st->decode_exec, ctx->stream);
            if (e != hipSuccess) return gd_hip_fail(ctx, e, "decode graph launch");
        }
    }
    if (done && (rc = gd_download(ctx, tokens, st->picks + st->pos, (size_t)done * 4))) return rc;
    st->pos += done;
    if (done < n) return gd_fail(ctx, GD_ESTOPPED, "generate stopped after %d of %d steps", done, n);
    return GD_OK;
}

extern "C" int gd_stack_kv_pages(gd_stack *st, int64_t *live, int64_t *held, int64_t *capacity) {
    if (!st) return GD_EINVAL;
    if (live) *live = (int64_t)st->live.size();
    if (held) *held = st->kv->held();
    if (capacity) *capacity = st->kv->cap;
    return GD_OK;
}

extern "C" int gd_stack_position(gd_stack *st, int64_t *pos) {
    if (!st || !pos) return GD_EINVAL;
    *pos = st->pos;
    return GD_OK;
}

extern "C" int gd_stack_tensor(gd_stack *st, int layer, const char *name, gd_q2w *w,
                               int64_t *row0, float **f32, int64_t *count) {
    if (!st || !name) return GD_EINVAL;
    gd_ctx *ctx = st->ctx;
    const std::string n(name);
    const gd_stack_config &c = st->c;
    // Rows [r0, r1) of matrix m.
    auto q = [&](const gd_q2w &m, int64_t r0 = 0, int64_t r1 = -1) {
        if (w) *w = m;
        if (row0) *row0 = r0;
        if (count) *count = (r1 < 0 ? m.R : r1) - r0;
        return GD_OK;
    };
    auto f = [&](float *p, int64_t cnt) {
        if (f32) *f32 = p;
        if (count) *count = cnt;
        return GD_OK;
    };
    if (layer < 0) {
        if (n == "token_embd") return q(st->embd);
        if (n == "output") return q(st->head);
        if (n == "output_norm") return f(st->out_norm, c.n_embd);
        return gd_fail(ctx, GD_EINVAL, "gd_stack_tensor: no global tensor '%s'", name);
    }
    GD_REQUIRE(ctx, layer < c.n_layer, "gd_stack_tensor: layer %d out of range", layer);
    StackLayer &ly = st->L[layer];
    if (n == "attn_norm") return f(ly.attn_norm, c.n_embd);
    // The pre-FFN norm: the dense lineage's file calls it ffn_norm
    // (Model.swift:103-106).
    if (n == (c.dense ? "ffn_norm" : "post_attention_norm")) return f(ly.post_norm, c.n_embd);
    if (n == "ffn_gate") return q(ly.gate_up, 0, c.n_ff);
    if (n == "ffn_up") return q(ly.gate_up, c.n_ff, 2 * (int64_t)c.n_ff);
    if (n == "ffn_down") return q(ly.down);
    if (ly.rec) {
        const int cd = st->convDim, vd = st->valDim, nv = c.n_v_head;
        if (n == "attn_qkv") return q(ly.in_proj, 0, cd);
        if (n == "attn_gate") return q(ly.in_proj, cd, cd + vd);
        if (n == "ssm_beta") return q(ly.in_proj, cd + vd, cd + vd + nv);
        if (n == "ssm_alpha") return q(ly.in_proj, cd + vd + nv, cd + vd + 2 * nv);
        if (n == "ssm_out") return q(ly.out_proj);
        if (n == "ssm_conv1d") return f(ly.conv_w, (int64_t)cd * 4);
        if (n == "ssm_dt") return f(ly.dt, nv);
        if (n == "ssm_a") return f(ly.a_neg, nv);
        if (n == "ssm_norm") return f(ly.ssm_norm, HD);
        if (n == "ssm_conv_state") return f(ly.conv_state, (int64_t)3 * cd);
        if (n == "ssm_state") return f(ly.rec_state, (int64_t)nv * HD * HD);
    } else {
        const int hd = c.head_dim, qf = (c.dense ? 1 : 2) * c.n_head * hd,
                  kv = c.n_head_kv * hd;
        if (n == "attn_q") return q(ly.in_proj, 0, qf);
        if (n == "attn_k") return q(ly.in_proj, qf, qf + kv);
        if (n == "attn_v") return q(ly.in_proj, qf + kv, qf + 2 * kv);
        if (n == "attn_output") return q(ly.out_proj);
        if (n == "attn_q_norm") return f(ly.q_norm, hd);
        if (n == "attn_k_norm") return f(ly.k_norm, hd);
    }
    return gd_fail(ctx, GD_EINVAL, "gd_stack_tensor: layer %d has no tensor '%s'", layer, name);
}

// ------------------------------------------------------------ GGUF weights

namespace {

// Tensors the stack reads, by the short names of gd_stack_tensor, for one
// layer kind (Model.swift:100-130) and for the whole model (:139-145).
const char *const k_common[] = {"attn_norm", "ffn_gate", "ffn_up", "ffn_down"};
const char *const k_rec[] = {"attn_qkv", "attn_gate", "ssm_beta", "ssm_alpha", "ssm_out",
                             "ssm_conv1d", "ssm_dt", "ssm_a", "ssm_norm"};
const char *const k_att[] = {"attn_q", "attn_k", "attn_v", "attn_output", "attn_q_norm",
                             "attn_k_norm"};

// The file's name for short name `name` of layer il (-1: global), as the
// reference looks it up (Model.swift:100-145): "<name>.weight", except the
// bias ssm_dt.bias and the bare ssm_a.
std::string gguf_name(int il, const std::string &name) {
    std::string s = il < 0 ? name : "blk." + std::to_string(il) + "." + name;
    if (name == "ssm_dt") return s + ".bias";
    if (name == "ssm_a") return s;
    return s + ".weight";
}

struct Item { int il; const char *name; };

std::vector<Item> load_list(const gd_stack *st) {
    std::vector<Item> v = {{-1, "token_embd"}, {-1, "output_norm"}};
    if (st->head.codes != st->embd.codes) v.push_back({-1, "output"});
    for (int il = 0; il < st->c.n_layer; il++) {
        for (const char *n : k_common) v.push_back({il, n});
        v.push_back({il, st->c.dense ? "ffn_norm" : "post_attention_norm"});
        if (st->L[il].rec)
            for (const char *n : k_rec) v.push_back({il, n});
        else
            for (const char *n : k_att) v.push_back({il, n});
    }
    return v;
}

// Upload one tensor of the file into its place in the stack: a Q2_0 matrix
// through the device staging buffer into its rows of the fused matrix, an
// f32 vector straight to its buffer.  Shapes and types must match exactly.
int load_tensor(gd_stack *st, const gd_gguf *g, const Item &it, void *staging,
                size_t staging_bytes) {
    gd_ctx *ctx = st->ctx;
    gd_q2w w{};
    int64_t row0 = 0, count = 0;
    float *f32 = nullptr;
    int rc = gd_stack_tensor(st, it.il, it.name, &w, &row0, &f32, &count);
    if (rc) return rc;
    const std::string gn = gguf_name(it.il, it.name);
    int ndim = 0, type = -1;
    int64_t dims[4];
    const void *data = nullptr;
    size_t bytes = 0;
    if (gd_gguf_tensor(g, gn.c_str(), &ndim, dims, &type, &data, &bytes) != GD_OK)
        return gd_fail(ctx, GD_EINVAL, "gd_stack_create_from_gguf: missing tensor %s", gn.c_str());
    if (f32) {
        const int64_t n = dims[0] * dims[1] * dims[2] * dims[3];
        GD_REQUIRE(ctx, type == 0 && n == count,
                   "gd_stack_create_from_gguf: %s must be f32 with %lld elements (type %d, %lld)",
                   gn.c_str(), (long long)count, type, (long long)n);
        GD_REQUIRE(ctx, std::string(it.name) != "ssm_conv1d" || dims[0] == st->c.d_conv,
                   "gd_stack_create_from_gguf: %s must be [d_conv, conv_dim]", gn.c_str());
        return gd_upload(ctx, f32, data, bytes);
    }
    GD_REQUIRE(ctx, type == 42 && ndim == 2 && dims[0] == w.K && dims[1] == count,
               "gd_stack_create_from_gguf: %s must be Q2_0 [%lld, %lld] (type %d, [%lld, %lld])",
               gn.c_str(), (long long)w.K, (long long)count, type, (long long)dims[0],
               (long long)(ndim > 1 ? dims[1] : 1));
    GD_REQUIRE(ctx, bytes <= staging_bytes, "gd_stack_create_from_gguf: staging too small");
    // The copy waits for the previous repack on the same stream, then the
    // host waits for the copy, so one staging buffer serves every tensor.
    if ((rc = gd_upload(ctx, staging, data, bytes))) return rc;
    return gd_q2_0_repack_rows(ctx, staging, 0, row0, count, &w);
}

}  // namespace

extern "C" int gd_stack_create_from_gguf(gd_ctx *ctx, const gd_gguf *g, int kv_block,
                                         int max_ctx, int max_batch, gd_stack **out) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, g && out, "gd_stack_create_from_gguf: null argument");
    *out = nullptr;
    gd_stack_config c{};
    if (gd_gguf_stack_config(g, &c) != GD_OK)
        return gd_fail(ctx, GD_EINVAL, "%s", gd_last_error(nullptr));
    c.kv_block = kv_block;
    c.max_ctx = max_ctx;
    c.max_batch = max_batch;
    // An absent output.weight means the lm_head is the token embedding
    // (Model.swift:145).
    const bool untied = gd_gguf_tensor(g, "output.weight", nullptr, nullptr, nullptr, nullptr,
                                       nullptr) == GD_OK;
    gd_stack *st = nullptr;
    int rc = create(ctx, &c, 0, false, untied, &st);
    if (rc) return rc;
    const std::vector<Item> items = load_list(st);
    size_t staging_bytes = 0;
    for (const Item &it : items) {
        int type = -1;
        size_t bytes = 0;
        if (gd_gguf_tensor(g, gguf_name(it.il, it.name).c_str(), nullptr, nullptr, &type, nullptr,
                           &bytes) == GD_OK && type == 42)
            staging_bytes = std::max(staging_bytes, bytes);
    }
    void *staging = nullptr;
    if ((rc = gd_alloc(ctx, staging_bytes, &staging))) { gd_stack_destroy(st); return rc; }
    for (const Item &it : items)
        if ((rc = load_tensor(st, g, it, staging, staging_bytes))) break;
    if (rc == GD_OK) rc = gd_sync(ctx);
    const int rc2 = gd_free(ctx, staging);
    if (rc == GD_OK) rc = rc2;
    if (rc) {
        gd_stack_destroy(st);
        return rc;
    }
    *out = st;
    return GD_OK;
}

// ------------------------------------------------------------ bookmarks

// A snapshot of the generation state (MetalEngine.Bookmark,
// MetalEngine.swift:455-483): position, rope shift, the last pick and every
// GDN layer's conv ring and recurrent state, copied whole into one device
// buffer (the recurrence cannot be paged), and the attention layers' K/V as
// pages of the stack's pool: completed pages shared with the live table, a
// partially filled tail page copied (MetalKVPool.snapshot, :102-110), so a
// bookmark costs O(tail) of KV, not O(context).
struct gd_bookmark {
    gd_ctx *ctx = nullptr;
    gd_stack_config c{};
    int64_t pos = 0;
    int64_t rope_shift = 0;      // rope position = position + shift
    bool have_pick = false;
    void *buf = nullptr;         // [pick | conv, rec per GDN layer]
    std::shared_ptr<KvPool> kv;  // the pool its pages live in
    std::vector<int32_t> pages;  // positions [0, pos), kv_block per page
};

namespace {

// A bookmark's state as one image: the pick, then per layer either its conv
// ring and recurrent state (f32) or its K and V over [0, pos) (f16), each
// array 256-byte aligned.  With kv = false (the device buffer of a
// bookmark) the attention layers take no room; the host image (kv = true)
// is what the byte formats are written from and read into.
struct BmLayout {
    size_t conv = 0, rec = 0, kv = 0, total = 0;   // element counts per layer; bytes
    std::vector<size_t> off;                       // per layer: byte offset of its first array
};

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

BmLayout bm_layout(const gd_stack *st, int64_t pos, bool kv = true) {
    BmLayout l;
    l.conv = (size_t)(st->c.d_conv - 1) * st->convDim;
    l.rec = (size_t)st->c.n_v_head * HD * HD;
    l.kv = (size_t)pos * st->c.n_head_kv * st->c.head_dim;
    size_t o = 256;                                  // the pick
    for (const StackLayer &ly : st->L) {
        l.off.push_back(o);
        o += ly.rec ? align256(l.conv * 4) + align256(l.rec * 4) : kv ? 2 * align256(l.kv * 2) : 0;
    }
    l.total = o;
    return l;
}

// K and V of positions [0, pos) of every attention layer, gathered from the
// pages into one device array [attention layer][K, V][pos][kv_dim] (f16),
// or scattered back from it.
int kv_gather(gd_ctx *ctx, const KvPool &pool, const std::vector<int32_t> &pages, int64_t pos,
              uint16_t *dev, bool scatter) {
    const int B = pool.block;
    const size_t pe = pool.page_elems, kvd = pe / B, span = (size_t)pos * kvd;
    int rc = GD_OK;
    for (size_t a = 0; a < pool.k.size(); a++)
        for (int kv = 0; kv < 2; kv++) {
            uint16_t *base = (kv ? pool.v : pool.k)[a];
            uint16_t *arr = dev + (2 * a + kv) * span;
            for (size_t i = 0; rc == GD_OK && i < pages.size(); i++) {
                const size_t n = std::min((size_t)B, (size_t)pos - i * B) * kvd;
                uint16_t *pg = base + (size_t)pages[i] * pe;
                rc = scatter ? gd_copy(ctx, pg, arr + i * B * kvd, n * 2)
                             : gd_copy(ctx, arr + i * B * kvd, pg, n * 2);
            }
        }
    return rc;
}

// dst <- the pages of positions [0, pos) given as `src` in pool `from`,
// held for a new owner in the stack's pool: a complete page of the same
// pool is shared; a partial tail page, or any page of another pool, is
// copied into a fresh page (on the context stream); pages of another page
// size go through a contiguous copy of the positions.
int adopt_pages(gd_stack *st, const std::shared_ptr<KvPool> &from, const std::vector<int32_t> &src,
                int64_t pos, std::vector<int32_t> &dst) {
    const int64_t B = st->c.kv_block;
    dst.clear();
    int rc = GD_OK;
    if (from->block != st->kv->block) {
        const size_t np = (size_t)((pos + B - 1) / B);
        for (size_t i = 0; rc == GD_OK && i < np; i++) {
            int32_t q;
            if ((rc = take_page(st, &q)) == GD_OK) dst.push_back(q);
        }
        void *tmp = nullptr;
        const size_t bytes = from->k.size() * 2 * (size_t)pos * (from->page_elems / from->block) * 2;
        if (rc == GD_OK && bytes && (rc = gd_alloc(st->ctx, bytes, &tmp)) == GD_OK) {
            rc = kv_gather(st->ctx, *from, src, pos, (uint16_t *)tmp, false);
            if (rc == GD_OK) rc = kv_gather(st->ctx, *st->kv, dst, pos, (uint16_t *)tmp, true);
            if (rc == GD_OK) rc = gd_sync(st->ctx);
            gd_free(st->ctx, tmp);
        }
        if (rc) {
            for (int32_t p : dst) st->kv->drop(p);
            dst.clear();
        }
        return rc;
    }
    for (size_t i = 0; rc == GD_OK && i < src.size(); i++) {
        const bool tail = (int64_t)(i + 1) * B > pos;
        if (from == st->kv && !tail) {
            st->kv->hold(src[i]);
            dst.push_back(src[i]);
            continue;
        }
        int32_t q;
        if ((rc = take_page(st, &q)) == GD_OK) {
            dst.push_back(q);
            rc = st->kv->copy_page(q, *from, src[i]);
        }
    }
    if (rc) {
        for (int32_t p : dst) st->kv->drop(p);
        dst.clear();
    }
    return rc;
}

// The host image (bm_layout with K/V) of bookmark b.
int bookmark_to_host(gd_stack *st, const gd_bookmark *b, std::vector<uint8_t> &host) {
    gd_ctx *ctx = st->ctx;
    const BmLayout lh = bm_layout(st, b->pos), ld = bm_layout(st, b->pos, false);
    host.assign(lh.total, 0);
    std::vector<uint8_t> dev(ld.total);
    int rc = gd_download(ctx, dev.data(), b->buf, ld.total);
    if (rc) return rc;
    memcpy(host.data(), dev.data(), 4);
    int natt = 0;
    for (int il = 0; il < st->c.n_layer; il++) {
        if (st->L[il].rec)
            memcpy(host.data() + lh.off[il], dev.data() + ld.off[il],
                   align256(lh.conv * 4) + lh.rec * 4);
        else
            natt++;
    }
    if (!natt || !b->pos) return GD_OK;
    const size_t span = lh.kv;
    void *tmp = nullptr;
    if ((rc = gd_alloc(ctx, (size_t)natt * 2 * span * 2, &tmp))) return rc;
    rc = kv_gather(ctx, *b->kv, b->pages, b->pos, (uint16_t *)tmp, false);
    std::vector<uint16_t> kvh(rc == GD_OK ? (size_t)natt * 2 * span : 0);
    if (rc == GD_OK) rc = gd_download(ctx, kvh.data(), tmp, kvh.size() * 2);
    gd_free(ctx, tmp);
    if (rc) return rc;
    for (int il = 0; il < st->c.n_layer; il++) {
        const StackLayer &ly = st->L[il];
        if (ly.rec) continue;
        for (int kv = 0; kv < 2; kv++)
            memcpy(host.data() + lh.off[il] + kv * align256(span * 2),
                   kvh.data() + (2 * (size_t)ly.att + kv) * span, span * 2);
    }
    return GD_OK;
}

bool same_geometry(const gd_stack_config &a, const gd_stack_config &b) {
    return a.n_layer == b.n_layer && a.attn_interval == b.attn_interval && a.dense == b.dense &&
           a.n_embd == b.n_embd && a.d_conv == b.d_conv && a.n_k_head == b.n_k_head &&
           a.n_v_head == b.n_v_head && a.d_state == b.d_state && a.n_head_kv == b.n_head_kv &&
           a.head_dim == b.head_dim;
}

int d2d(gd_ctx *ctx, void *dst, const void *src, size_t bytes) {
    return bytes ? gd_copy(ctx, dst, src, bytes) : GD_OK;
}

// Little-endian i64 and f32-run writer / bounds-checked reader of
// MetalEngine.serialize's byte format (MetalEngine.swift:490-584).
struct Out {
    uint8_t *p;
    size_t cap, n = 0;
    void put(const void *src, size_t b) {
        if (p && n + b <= cap) memcpy(p + n, src, b);
        n += b;
    }
    void i64(int64_t v) { put(&v, 8); }
};

struct In {
    const uint8_t *p;
    size_t len, n = 0;
    bool bad = false;
    int64_t i64() {
        int64_t v = 0;
        if (bad || len - n < 8) { bad = true; return 0; }
        memcpy(&v, p + n, 8);
        n += 8;
        return v;
    }
    // A run of `want` floats: its count must be `want`; returns its bytes.
    const uint8_t *floats(size_t want) {
        const int64_t c = i64();
        if (bad || c < 0 || (size_t)c != want || (len - n) / 4 < want) { bad = true; return nullptr; }
        const uint8_t *r = p + n;
        n += want * 4;
        return r;
    }
};

}  // namespace

extern "C" int gd_stack_bookmark(gd_stack *st, gd_bookmark **out) {
    if (!st) return GD_EINVAL;
    gd_ctx *ctx = st->ctx;
    GD_REQUIRE(ctx, out, "gd_stack_bookmark: null out pointer");
    *out = nullptr;
    const BmLayout l = bm_layout(st, st->pos, false);
    gd_bookmark *b = new gd_bookmark();
    b->ctx = ctx;
    b->c = st->c;
    b->pos = st->pos;
    b->rope_shift = st->rope_shift;
    b->have_pick = st->have_pick;
    b->kv = st->kv;
    int rc = gd_alloc(ctx, l.total, &b->buf);
    uint8_t *base = (uint8_t *)b->buf;
    if (rc == GD_OK) rc = d2d(ctx, base, st->dtok, 4);
    for (int il = 0; rc == GD_OK && il < st->c.n_layer; il++) {
        const StackLayer &ly = st->L[il];
        uint8_t *d = base + l.off[il];
        if (ly.rec && (rc = d2d(ctx, d, ly.conv_state, l.conv * 4)) == GD_OK)
            rc = d2d(ctx, d + align256(l.conv * 4), ly.rec_state, l.rec * 4);
    }
    const size_t np = (size_t)((st->pos + st->c.kv_block - 1) / st->c.kv_block);
    if (rc == GD_OK)
        rc = adopt_pages(st, st->kv, std::vector<int32_t>(st->live.begin(), st->live.begin() + np),
                         st->pos, b->pages);
    if (rc == GD_OK) rc = gd_sync(ctx);
    if (rc) {
        gd_bookmark_free(b);
        return rc;
    }
    *out = b;
    return GD_OK;
}

extern "C" void gd_bookmark_free(gd_bookmark *b) {
    if (!b) return;
    if (b->kv)
        for (int32_t p : b->pages) b->kv->drop(p);
    if (b->buf) gd_free(b->ctx, b->buf);
    delete b;
}

extern "C" int gd_stack_restore(gd_stack *st, const gd_bookmark *b) {
    if (!st) return GD_EINVAL;
    gd_ctx *ctx = st->ctx;
    GD_REQUIRE(ctx, b && b->buf, "gd_stack_restore: null bookmark");
    GD_REQUIRE(ctx, b->ctx == ctx, "gd_stack_restore: bookmark of another context");
    GD_REQUIRE(ctx, same_geometry(b->c, st->c) && b->pos <= st->c.max_ctx,
               "gd_stack_restore: bookmark of another geometry (or beyond max_ctx)");
    // The live table takes the bookmark's pages (its own copy of a partial
    // tail, so that a bookmark restored more than once is never written:
    // MetalKVPool.restore, :111-120), then lets its old pages go.
    std::vector<int32_t> pages;
    int rc = adopt_pages(st, b->kv, b->pages, b->pos, pages);
    if (rc) return rc;
    release_live(st);
    st->live = std::move(pages);
    if (!st->live.empty() &&
        (rc = gd_upload(ctx, st->page_table, st->live.data(), st->live.size() * sizeof(int32_t))))
        return rc;
    const BmLayout l = bm_layout(st, b->pos, false);
    const uint8_t *base = (const uint8_t *)b->buf;
    rc = d2d(ctx, st->dtok, base, 4);
    for (int il = 0; rc == GD_OK && il < st->c.n_layer; il++) {
        StackLayer &ly = st->L[il];
        const uint8_t *s = base + l.off[il];
        if (ly.rec && (rc = d2d(ctx, ly.conv_state, s, l.conv * 4)) == GD_OK)
            rc = d2d(ctx, ly.rec_state, s + align256(l.conv * 4), l.rec * 4);
    }
    if (rc == GD_OK) rc = gd_fill_u32(ctx, st->dpos, (uint32_t)b->pos, 1);
    if (rc == GD_OK) rc = gd_fill_u32(ctx, st->dpos + 1, (uint32_t)(int32_t)b->rope_shift, 1);
    if (rc == GD_OK) rc = gd_sync(ctx);
    if (rc) return rc;
    st->pos = b->pos;
    st->rope_shift = b->rope_shift;
    st->have_pick = b->have_pick;
    st->stop.store(false);
    return GD_OK;
}

extern "C" int gd_stack_serialize(gd_stack *st, const gd_bookmark *b, void *buf, size_t cap,
                                  size_t *len) {
    if (!st) return GD_EINVAL;
    gd_ctx *ctx = st->ctx;
    GD_REQUIRE(ctx, b && b->buf && len, "gd_stack_serialize: null argument");
    GD_REQUIRE(ctx, b->ctx == ctx && same_geometry(b->c, st->c),
               "gd_stack_serialize: bookmark of another stack geometry or context");
    const BmLayout l = bm_layout(st, b->pos);
    // Size pass (no data), then, given room, the bytes.
    auto emit = [&](Out &o, const uint8_t *host) {
        o.i64(b->pos);
        o.i64(b->rope_shift);
        for (int part = 0; part < 2; part++) {                 // conv dict, then rec dict
            int64_t n = 0;
            for (const StackLayer &ly : st->L) n += ly.rec;
            o.i64(n);
            for (int il = 0; il < st->c.n_layer; il++) {
                if (!st->L[il].rec) continue;
                const size_t cnt = part ? l.rec : l.conv;
                o.i64(il);
                o.i64((int64_t)cnt);
                const size_t at = l.off[il] + (part ? align256(l.conv * 4) : 0);
                o.put(host ? host + at : nullptr, cnt * 4);
            }
        }
        int64_t na = 0;
        for (const StackLayer &ly : st->L) na += !ly.rec;
        o.i64(na);
        std::vector<float> wide(host ? l.kv : 0);
        for (int il = 0; il < st->c.n_layer; il++) {
            if (st->L[il].rec) continue;
            o.i64(il);
            o.i64(b->pos);
            for (int kv = 0; kv < 2; kv++) {                   // half pages widened to f32
                o.i64((int64_t)l.kv);
                if (host) {
                    const _Float16 *h = (const _Float16 *)(host + l.off[il] +
                                                           kv * align256(l.kv * 2));
                    for (size_t i = 0; i < l.kv; i++) wide[i] = (float)h[i];
                }
                o.put(host ? wide.data() : nullptr, l.kv * 4);
            }
        }
    };
    Out sizer{nullptr, 0};
    emit(sizer, nullptr);
    *len = sizer.n;
    if (!buf) return GD_OK;
    GD_REQUIRE(ctx, cap >= sizer.n, "gd_stack_serialize: buffer of %zu bytes, need %zu", cap,
               sizer.n);
    std::vector<uint8_t> host;
    int rc = bookmark_to_host(st, b, host);
    if (rc) return rc;
    Out o{(uint8_t *)buf, cap};
    emit(o, host.data());
    return GD_OK;
}

// ------------------------------------------------- parked-state bytes (GDNS)

namespace {

// BonsaiEngine's parked-state format (BonsaiEngine.swift:65-112, through
// StateBytes.swift): the magic "GDNS" and an i64 version 1, the position, per
// GDN layer its conv ring then its state, per attention layer its length and
// its K pages then its V pages, each page a run of KVCache.pageP = 512
// positions x kv_dim f32 (Attention.swift:15-40).
constexpr char GDNS_MAGIC[4] = {'G', 'D', 'N', 'S'};
constexpr int64_t GDNS_VERSION = 1, GDNS_PAGE = 512;

// A bookmark from its host image (bm_layout with K/V): the GDN state into
// its device buffer, the K/V into fresh pages of the stack's pool.
int bookmark_from_host(gd_stack *st, const std::vector<uint8_t> &host, int64_t pos,
                       gd_bookmark **out, int64_t rope_shift = 0) {
    gd_ctx *ctx = st->ctx;
    const BmLayout lh = bm_layout(st, pos), ld = bm_layout(st, pos, false);
    gd_bookmark *b = new gd_bookmark();
    b->ctx = ctx;
    b->c = st->c;
    b->pos = pos;
    b->rope_shift = rope_shift;
    b->have_pick = false;        // neither format carries a pick: decode a token first
    b->kv = st->kv;
    std::vector<uint8_t> dev(ld.total, 0);
    int natt = 0;
    for (int il = 0; il < st->c.n_layer; il++) {
        if (st->L[il].rec)
            memcpy(dev.data() + ld.off[il], host.data() + lh.off[il],
                   align256(lh.conv * 4) + lh.rec * 4);
        else
            natt++;
    }
    int rc = gd_alloc(ctx, ld.total, &b->buf);
    if (rc == GD_OK) rc = gd_upload(ctx, b->buf, dev.data(), ld.total);
    const size_t np = (size_t)((pos + st->c.kv_block - 1) / st->c.kv_block);
    for (size_t i = 0; rc == GD_OK && i < np; i++) {
        int32_t q;
        if ((rc = take_page(st, &q)) == GD_OK) b->pages.push_back(q);
    }
    if (rc == GD_OK && natt && pos) {
        const size_t span = lh.kv;
        std::vector<uint16_t> kvh((size_t)natt * 2 * span);
        for (int il = 0; il < st->c.n_layer; il++) {
            const StackLayer &ly = st->L[il];
            if (ly.rec) continue;
            for (int kv = 0; kv < 2; kv++)
                memcpy(kvh.data() + (2 * (size_t)ly.att + kv) * span,
                       host.data() + lh.off[il] + kv * align256(span * 2), span * 2);
        }
        void *tmp = nullptr;
        if ((rc = gd_alloc(ctx, kvh.size() * 2, &tmp)) == GD_OK) {
            rc = gd_upload(ctx, tmp, kvh.data(), kvh.size() * 2);
            if (rc == GD_OK)
                rc = kv_gather(ctx, *st->kv, b->pages, pos, (uint16_t *)tmp, true);
            if (rc == GD_OK) rc = gd_sync(ctx);
            gd_free(ctx, tmp);
        }
    }
    if (rc) {
        gd_bookmark_free(b);
        return rc;
    }
    *out = b;
    return GD_OK;
}

}  // namespace

extern "C" int gd_stack_serialize_gdns(gd_stack *st, const gd_bookmark *b, void *buf,
                                       size_t cap, size_t *len) {
    if (!st) return GD_EINVAL;
    gd_ctx *ctx = st->ctx;
    GD_REQUIRE(ctx, b && b->buf && len, "gd_stack_serialize_gdns: null argument");
    GD_REQUIRE(ctx, b->ctx == ctx && same_geometry(b->c, st->c),
               "gd_stack_serialize_gdns: bookmark of another stack geometry or context");
    // The CPU engine has no image spans, and its bytes no rope shift.
    GD_REQUIRE(ctx, b->rope_shift == 0,
               "gd_stack_serialize_gdns: ropeShift %lld has no place in GDNS bytes",
               (long long)b->rope_shift);
    const BmLayout l = bm_layout(st, b->pos);
    const size_t kvd = (size_t)st->c.n_head_kv * st->c.head_dim;
    const int64_t npages = (b->pos + GDNS_PAGE - 1) / GDNS_PAGE;
    const size_t page = (size_t)GDNS_PAGE * kvd;
    auto emit = [&](Out &o, const uint8_t *host) {
        o.put(GDNS_MAGIC, 4);
        o.i64(GDNS_VERSION);
        o.i64(b->pos);
        int64_t nrec = 0, natt = 0;
        for (const StackLayer &ly : st->L) (ly.rec ? nrec : natt)++;
        o.i64(nrec);
        for (int il = 0; il < st->c.n_layer; il++) {
            if (!st->L[il].rec) continue;
            o.i64(il);
            o.i64((int64_t)l.conv);
            o.put(host ? host + l.off[il] : nullptr, l.conv * 4);
            o.i64((int64_t)l.rec);
            o.put(host ? host + l.off[il] + align256(l.conv * 4) : nullptr, l.rec * 4);
        }
        o.i64(natt);
        std::vector<float> wide(host ? page : 0);
        for (int il = 0; il < st->c.n_layer; il++) {
            if (st->L[il].rec) continue;
            o.i64(il);
            o.i64(b->pos);
            o.i64(npages);
            for (int kv = 0; kv < 2; kv++)                      // K pages, then V pages
                for (int64_t pg = 0; pg < npages; pg++) {
                    o.i64((int64_t)page);
                    if (host) {
                        // Positions past pos are zero, as a fresh page holds.
                        const _Float16 *h = (const _Float16 *)(host + l.off[il] +
                                                               kv * align256(l.kv * 2));
                        const size_t lo = (size_t)pg * page;
                        const size_t hi = std::min(lo + page, l.kv);
                        for (size_t i = lo; i < lo + page; i++)
                            wide[i - lo] = i < hi ? (float)h[i] : 0.f;
                    }
                    o.put(host ? wide.data() : nullptr, page * 4);
                }
        }
    };
    Out sizer{nullptr, 0};
    emit(sizer, nullptr);
    *len = sizer.n;
    if (!buf) return GD_OK;
    GD_REQUIRE(ctx, cap >= sizer.n, "gd_stack_serialize_gdns: buffer of %zu bytes, need %zu",
               cap, sizer.n);
    std::vector<uint8_t> host;
    int rc = bookmark_to_host(st, b, host);
    if (rc) return rc;
    Out o{(uint8_t *)buf, cap};
    emit(o, host.data());
    return GD_OK;
}

extern "C" int gd_stack_deserialize_gdns(gd_stack *st, const void *data, size_t n,
                                         gd_bookmark **out) {
    if (!st) return GD_EINVAL;
    gd_ctx *ctx = st->ctx;
    GD_REQUIRE(ctx, data && out, "gd_stack_deserialize_gdns: null argument");
    *out = nullptr;
    // BonsaiEngine.deserialize refuses bytes without its header
    // (StateBytes.readHeader); so does this.
    GD_REQUIRE(ctx, n >= 12 && memcmp(data, GDNS_MAGIC, 4) == 0,
               "gd_stack_deserialize_gdns: no GDNS header (not a parked state)");
    In in{(const uint8_t *)data, n, 4};
    const int64_t version = in.i64();
    GD_REQUIRE(ctx, version == GDNS_VERSION,
               "gd_stack_deserialize_gdns: version %lld, this build reads %lld",
               (long long)version, (long long)GDNS_VERSION);
    const int64_t pos = in.i64();
    GD_REQUIRE(ctx, !in.bad && pos >= 0 && pos <= st->c.max_ctx,
               "gd_stack_deserialize_gdns: position %lld outside [0, max_ctx %d]",
               (long long)pos, st->c.max_ctx);
    const BmLayout l = bm_layout(st, pos);
    std::vector<uint8_t> host(l.total, 0);
    int64_t nrec = 0, natt = 0;
    for (const StackLayer &ly : st->L) (ly.rec ? nrec : natt)++;
    // The layers must be exactly this stack's, in ascending order.
    auto next_layer = [&](int after, bool rec) {
        for (int j = after + 1; j < st->c.n_layer; j++)
            if (st->L[j].rec == rec) return j;
        return -1;
    };
    const int64_t cnt = in.i64();
    GD_REQUIRE(ctx, !in.bad && cnt == nrec,
               "gd_stack_deserialize_gdns: %lld GDN layers in the data, the stack has %lld",
               (long long)cnt, (long long)nrec);
    int il = -1;
    for (int64_t k = 0; k < cnt; k++) {
        const int want = next_layer(il, true);
        const int64_t got = in.i64();
        GD_REQUIRE(ctx, !in.bad && got == want,
                   "gd_stack_deserialize_gdns: GDN layer %lld where %d was expected",
                   (long long)got, want);
        il = want;
        const uint8_t *conv = in.floats(l.conv);
        const uint8_t *rec = conv ? in.floats(l.rec) : nullptr;
        GD_REQUIRE(ctx, !in.bad, "gd_stack_deserialize_gdns: layer %d state: bad count or "
                   "truncated", il);
        memcpy(host.data() + l.off[il], conv, l.conv * 4);
        memcpy(host.data() + l.off[il] + align256(l.conv * 4), rec, l.rec * 4);
    }
    const int64_t na = in.i64();
    GD_REQUIRE(ctx, !in.bad && na == natt,
               "gd_stack_deserialize_gdns: %lld attention layers in the data, the stack has "
               "%lld", (long long)na, (long long)natt);
    const size_t kvd = (size_t)st->c.n_head_kv * st->c.head_dim;
    const size_t page = (size_t)GDNS_PAGE * kvd;
    const int64_t npages = (pos + GDNS_PAGE - 1) / GDNS_PAGE;
    il = -1;
    for (int64_t k = 0; k < na; k++) {
        const int want = next_layer(il, false);
        const int64_t got = in.i64(), len = in.i64(), np = in.i64();
        GD_REQUIRE(ctx, !in.bad && got == want && len == pos && np == npages,
                   "gd_stack_deserialize_gdns: attention layer %lld with %lld positions in %lld "
                   "pages where layer %d with %lld in %lld was expected", (long long)got,
                   (long long)len, (long long)np, want, (long long)pos, (long long)npages);
        il = want;
        for (int kv = 0; kv < 2; kv++) {
            _Float16 *h = (_Float16 *)(host.data() + l.off[il] + kv * align256(l.kv * 2));
            for (int64_t pg = 0; pg < npages; pg++) {
                const uint8_t *src = in.floats(page);
                GD_REQUIRE(ctx, !in.bad, "gd_stack_deserialize_gdns: layer %d %s page %lld: "
                           "not %zu floats, or truncated", il, kv ? "V" : "K", (long long)pg,
                           page);
                // Positions below pos, rounded to the cache's halves (nearest even).
                const size_t lo = (size_t)pg * page, m = std::min(page, l.kv - lo);
                for (size_t i = 0; i < m; i++) {
                    float f;
                    memcpy(&f, src + 4 * i, 4);
                    h[lo + i] = (_Float16)f;
                }
            }
        }
    }
    GD_REQUIRE(ctx, in.n == n, "gd_stack_deserialize_gdns: %zu trailing bytes", n - in.n);
    return bookmark_from_host(st, host, pos, out);
}

extern "C" int gd_stack_deserialize(gd_stack *st, const void *data, size_t n,
                                    gd_bookmark **out) {
    if (!st) return GD_EINVAL;
    gd_ctx *ctx = st->ctx;
    GD_REQUIRE(ctx, data && out, "gd_stack_deserialize: null argument");
    *out = nullptr;
    In in{(const uint8_t *)data, n};
    const int64_t pos = in.i64(), rope_shift = in.i64();
    GD_REQUIRE(ctx, !in.bad && pos >= 0 && pos <= st->c.max_ctx,
               "gd_stack_deserialize: position %lld outside [0, max_ctx %d]", (long long)pos,
               st->c.max_ctx);
    // Rope positions (position + shift) must stay in int32 over the context.
    GD_REQUIRE(ctx, rope_shift >= -(1LL << 30) && rope_shift <= (1LL << 30),
               "gd_stack_deserialize: ropeShift %lld out of range", (long long)rope_shift);
    const BmLayout l = bm_layout(st, pos);
    std::vector<uint8_t> host(l.total, 0);
    // Each dict must list exactly this stack's GDN (or attention) layers, in
    // ascending order, as serialize writes them.
    for (int part = 0; part < 2; part++) {
        const int64_t cnt = in.i64();
        int il = -1;
        for (int64_t k = 0; k < cnt && !in.bad; k++) {
            const int64_t want = [&] {
                for (int j = il + 1; j < st->c.n_layer; j++) if (st->L[j].rec) return j;
                return -1;
            }();
            const int64_t got = in.i64();
            GD_REQUIRE(ctx, !in.bad && want >= 0 && got == want,
                       "gd_stack_deserialize: GDN layer %lld where %lld was expected",
                       (long long)got, (long long)want);
            il = (int)got;
            const size_t c = part ? l.rec : l.conv;
            const uint8_t *src = in.floats(c);
            GD_REQUIRE(ctx, !in.bad, "gd_stack_deserialize: layer %d state: bad count or "
                       "truncated", il);
            memcpy(host.data() + l.off[il] + (part ? align256(l.conv * 4) : 0), src, c * 4);
        }
        int64_t nrec = 0;
        for (const StackLayer &ly : st->L) nrec += ly.rec;
        GD_REQUIRE(ctx, !in.bad && cnt == nrec,
                   "gd_stack_deserialize: %lld GDN layers in the data, the stack has %lld",
                   (long long)cnt, (long long)nrec);
    }
    const int64_t na = in.i64();
    int64_t natt = 0;
    for (const StackLayer &ly : st->L) natt += !ly.rec;
    GD_REQUIRE(ctx, !in.bad && na == natt,
               "gd_stack_deserialize: %lld attention layers in the data, the stack has %lld",
               (long long)na, (long long)natt);
    int il = -1;
    for (int64_t k = 0; k < na; k++) {
        int want = -1;
        for (int j = il + 1; j < st->c.n_layer; j++) if (!st->L[j].rec) { want = j; break; }
        const int64_t got = in.i64(), len = in.i64();
        GD_REQUIRE(ctx, !in.bad && got == want && len == pos,
                   "gd_stack_deserialize: attention layer %lld with %lld positions where "
                   "layer %d with %lld was expected", (long long)got, (long long)len, want,
                   (long long)pos);
        il = want;
        for (int kv = 0; kv < 2; kv++) {
            const uint8_t *src = in.floats(l.kv);
            GD_REQUIRE(ctx, !in.bad, "gd_stack_deserialize: layer %d K/V: bad count or "
                       "truncated", il);
            // f32 back to the cache's halves, round to nearest even.
            _Float16 *h = (_Float16 *)(host.data() + l.off[il] + kv * align256(l.kv * 2));
            for (size_t i = 0; i < l.kv; i++) {
                float f;
                memcpy(&f, src + 4 * i, 4);
                h[i] = (_Float16)f;
            }
        }
    }
    GD_REQUIRE(ctx, in.n == n, "gd_stack_deserialize: %zu trailing bytes", n - in.n);
    return bookmark_from_host(st, host, pos, out, rope_shift);
}
