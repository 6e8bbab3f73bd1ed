// Internal declarations shared by the HIP translation units of libgadeon_hip.
// Host side: the context object, error plumbing and launch checks.
// Device side: f16 helpers, wave reductions and the LCG jump-ahead.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stdio.h>
#include <string>
#include <atomic>

#include "../../include/gadeon_hip.h"

struct gd_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t ev_start = nullptr;
    hipEvent_t ev_stop = nullptr;
    int num_cus = 0;
    void *ws = nullptr;          // grow-only workspace (chunked GDN prefill)
    size_t ws_bytes = 0;
    // This device's copy of the allocation-free prefill's scratch array
    // (hipGetSymbolAddress at context creation; null if that failed).
    void *prefill_scratch = nullptr;
    std::string err;
};

// Look up this device's address of the prefill scratch array (device current).
int gd_prefill_scratch_attach(gd_ctx *ctx);

// Record `msg` as the context's last error and return `code`.
int gd_fail(gd_ctx *ctx, int code, const char *fmt, ...);
// Grow-only context workspace of at least `bytes`; valid until the next call.
int gd_ctx_workspace(gd_ctx *ctx, size_t bytes, void **out);
// Map a HIP error to a GD code with a message naming `what`.
int gd_hip_fail(gd_ctx *ctx, hipError_t e, const char *what);
// Matrix-core GEMV (checked by the caller); ksplit > 1 writes K-split partial
// rows to y + z * R.  bias (if not null, f32 [R]) is added to the rows of
// split 0.
int gd_gemv_mfma(gd_ctx *ctx, const gd_q2w *w, const void *x, int x_dtype, float *y, int ksplit,
                 const float *bias = nullptr);
// GEMV of x = f16(o * rs * g) (rs the 1/rms of each 128-element block of o,
// one head; g = norm weight * silu(z), the gate) plus bias; ring (if not
// null): advance the conv ring of ring_n channels (rows ring_stride apart,
// new row ring_src) in the same launch.
int gd_gemv_mfma_gated(gd_ctx *ctx, const gd_q2w *w, const float *o, const float *g, float eps,
                       float *y, const float *bias, float *ring, const float *ring_src, int ring_n,
                       int ring_stride);
// GEMV of x = f16(rmsnorm(h + sum of nd delta partials) * normw); hout <- the
// sum if not null.
// glu_out (if not null): w = [gate; up] and glu_out = f16(silu(gate x) * up x)
// replaces y.
int gd_gemv_mfma_norm(gd_ctx *ctx, const gd_q2w *w, const float *h, const float *delta, int nd,
                      int dstride, const float *normw, float eps, float *hout, float *y,
                      uint16_t *glu_out = nullptr);
// Token-serial gdnScanBatch (gdn_scan_batch, Kernels.metal:1525-1565) for
// state sizes other than the chunked prefill's 128 (dS <= 1024).
int gd_gdn_scan_batch_serial(gd_ctx *ctx, const float *convOutN, int keyDim, int valueDim,
                             int convDim, const float *gN, const float *betaN, float *S,
                             float *oN, int nV, int nK, int dS, float qScale, int64_t N);
// K splits an f16-x GEMV of this shape should use (partials summed by the consumer).
int gd_gemv_ksplit(gd_ctx *ctx, int64_t K, int64_t R);
// Prefill GEMM plan: MT x 32 tokens by 4 x NT x 32 weight rows per
// workgroup, K split `split` ways into f32 partials.
// nw: waves per workgroup; ex = 1: the 4 x 2 x 8 tile with a seventeenth
// 32-row fragment (544 rows a workgroup; f32 out or split partials only).
struct gd_gemm_plan { int mt, nt, split; int nw = 4; int ex = 0; };
gd_gemm_plan gd_gemm_choose(gd_ctx *ctx, int64_t T, int64_t K, int64_t R, int x_dtype);
// split > 1: y_dtype f32 and Y holds split * T * R partials, summed by the caller.
int gd_gemm_launch(gd_ctx *ctx, const gd_q2w *w, int64_t T, const void *X, int x_dtype, void *Y,
                   int y_dtype, const gd_gemm_plan &p);
// An unsplit plain plan over whole row tiles (rows below *tail_r0) plus the
// rows past them as K-split f32 partials tailY[z][t][r - *tail_r0] in the
// same launch (*tail_nz: at most, then the count made; summed by the caller).
int gd_gemm_launch_tail(gd_ctx *ctx, const gd_q2w *w, int64_t T, const void *X, float *Y,
                        const gd_gemm_plan &p, float *tailY, int *tail_nz, int *tail_r0);
// SwiGLU GEMM: w = [gate; up] (2 * ff rows), f16 X [T][K] -> f16 out [T][ff].
// tile17: -1 the planner's choice, 1 one launch of the 17-fragment (4, 2, 8)
// tile, 0 the planner's choice among the others.
int gd_gemm_glu(gd_ctx *ctx, const gd_q2w *w, int64_t T, const void *X, uint16_t *out,
                int tile17 = -1);

// Attention kernels (attention.hip) for head dims 128 and 256, as the stack
// launches them: prefill prep (q/k norm + rope + cache append), flash
// prefill (out f16 or f32), fused decode (prep + split + combine, f16 out),
// and the size of the decode split partials.  qs is the per-head q stride of
// the projection rows: 2 hd for fused [q | gate] pairs (gated output), hd
// for plain q (ungated).  For prep and fused decode, pos_ptr holds two ints:
// the (first) token's position and the rope shift (rotation at position +
// shift, KV slot at position).  Prep does heads hbeg .. H + HKV - 1 (hbeg 0
// or H: kv only).  The prefill reads q (and the gate) of (token n, head h) at
// q + n q_tstride + h q_hstride; with q_norm set these are raw projection
// rows that it normalizes and rotates itself (n_rot a multiple of 64,
// pos_ptr as for prep), else k_attn_prep's output.
int gd_attn_prep_launch(gd_ctx *ctx, int hd, const float *proj, int64_t stride, int qs,
                        const float *q_norm, const float *k_norm, float *q_out, float *gate_out,
                        uint16_t *kc, uint16_t *vc, const int32_t *page_table,
                        const int32_t *pos_ptr, int N, int H, int HKV, int n_rot, float base,
                        int block, float eps, const float *rope_tab, int rope_n, int hbeg);
int gd_attn_prefill_launch(gd_ctx *ctx, int hd, const float *q, const float *gate,
                           int64_t q_tstride, int q_hstride, const float *q_norm, int n_rot,
                           float base, float eps, const float *rope_tab, int rope_n,
                           const uint16_t *kc, const uint16_t *vc, const int32_t *page_table,
                           const int32_t *pos_ptr, int pos_add, void *out, int out_dtype, int H,
                           int HKV, int N, int block, float scale, int gated);
int gd_attn_decode_launch(gd_ctx *ctx, int hd, const float *proj, int qs, const float *q_norm,
                          const float *k_norm, uint16_t *kc, uint16_t *vc,
                          const int32_t *page_table, const int32_t *pos_ptr, float *part,
                          uint16_t *out, int H, int HKV, int block, float scale, int n_rot,
                          float base, float eps, const float *rope_tab, int rope_n);
size_t gd_attn_part_floats(int hd, int H);
// The rotation table of prep and fused decode: for positions 0 .. n-1, the
// n_rot/2 (cos, sin) f32 pairs of the partial NEOX rope (rope positions
// outside it are computed in the kernels, to the same bits).
int gd_rope_table(gd_ctx *ctx, float *tab, int n, int n_rot, float base);

#define GD_CHECK_CTX(ctx) \
    do { if (!(ctx)) return GD_EINVAL; } while (0)

#define GD_REQUIRE(ctx, cond, ...) \
    do { if (!(cond)) return gd_fail((ctx), GD_EINVAL, __VA_ARGS__); } while (0)

#define GD_HIP(ctx, call) \
    do { hipError_t e_ = (call); \
         if (e_ != hipSuccess) return gd_hip_fail((ctx), e_, #call); } while (0)

// After a hipLaunchKernelGGL: report a launch failure with the kernel name.
#define GD_LAUNCHED(ctx, name) \
    do { hipError_t e_ = hipGetLastError(); \
         if (e_ != hipSuccess) return gd_fail((ctx), GD_ELAUNCH, \
             "%s launch: %s", (name), hipGetErrorString(e_)); } while (0)

static inline unsigned gd_blocks(int64_t n, int per) {
    return (unsigned)((n + per - 1) / per);
}

// ------------------------------------------------- device Q2_0 weight layout
// Rows come in groups of 16 and K in steps of 512 (4 blocks of 128).
//   codes:  one 2 KiB tile per (row group, step): [half h][block-in-step kb]
//           [row-in-group r][16 bytes] holds code bytes 16h..16h+15 of block
//           4*step+kb of row 16*group+r.  The 64 lanes of a wave reading
//           lane*16 + h*1024 get exactly the matrix-core A operand layout
//           (lane = 16*kb + r), one contiguous 1 KiB per load instruction.
//   scales: [row group][block/16][block%16][r] f16, so the 16 rows of a block
//           are 32 contiguous bytes.
//   Inside each code dword (16 codes of a block) the codes are interleaved by
//   nibble: code i < 8 at bits 4i, code 8 + i at bits 4i + 2.  A mask (w &
//   0x33333333, or (w >> 2) & 0x33333333) then leaves 8 consecutive codes c
//   as the e2m1 nibbles c/2, the fp4 operand order of the matrix cores and
//   of the fp4 -> f16 conversion.
// Rows past R and blocks past K/128 are padding and hold zeros.
__host__ __device__ constexpr int gd_q2_bitpos(int i) { return i < 8 ? 4 * i : 4 * (i - 8) + 2; }
// 2-bit fields of a 16-bit value spread to the low bits of 8 nibbles, and back.
__host__ __device__ inline uint32_t gd_q2_spread(uint32_t x) {
    x &= 0xffffu;
    x = (x | (x << 8)) & 0x00ff00ffu;
    x = (x | (x << 4)) & 0x0f0f0f0fu;
    return (x | (x << 2)) & 0x33333333u;
}
__host__ __device__ inline uint32_t gd_q2_gather(uint32_t x) {
    x &= 0x33333333u;
    x = (x | (x >> 2)) & 0x0f0f0f0fu;
    x = (x | (x >> 4)) & 0x00ff00ffu;
    return (x | (x >> 8)) & 0xffffu;
}
// A code dword as the GGUF block stores it (code i at bits 2i) <-> device.
__host__ __device__ inline uint32_t gd_q2_to_dev(uint32_t w) {
    return gd_q2_spread(w) | (gd_q2_spread(w >> 16) << 2);
}
__host__ __device__ inline uint32_t gd_q2_from_dev(uint32_t w) {
    return gd_q2_gather(w) | (gd_q2_gather(w >> 2) << 16);
}
__host__ __device__ inline int64_t gd_q2_steps(int64_t K) { return (K / 128 + 3) / 4; }
__host__ __device__ inline int64_t gd_q2_bgroups(int64_t K) { return (K / 128 + 15) / 16; }
__host__ __device__ inline int64_t gd_q2_rgroups(int64_t R) { return (R + 15) / 16; }
__host__ __device__ inline size_t gd_q2_codes_bytes(int64_t K, int64_t R) {
    return (size_t)gd_q2_rgroups(R) * gd_q2_steps(K) * 2048;
}
__host__ __device__ inline size_t gd_q2_scales_count(int64_t K, int64_t R) {
    return (size_t)gd_q2_rgroups(R) * gd_q2_bgroups(K) * 256;
}
// Byte offset of code bytes 16h..16h+15 of block `blk` of row `row`.
__host__ __device__ inline size_t gd_q2_code_off(int64_t row, int64_t blk, int h,
                                                 int64_t steps) {
    return (((size_t)(row >> 4) * steps + (size_t)(blk >> 2)) << 11) + ((size_t)h << 10) +
           ((size_t)(((blk & 3) << 4) | (row & 15)) << 4);
}
// Index (in f16 units) of the scale of block `blk` of row `row`.
// Raw buffer resource over `bytes` bytes at p.  A load whose VGPR offset lies
// past the end returns zeros without touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t gd_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes,
                                             0x00020000);
}

__host__ __device__ inline size_t gd_q2_scale_idx(int64_t row, int64_t blk, int64_t bgroups) {
    return (((((size_t)(row >> 4) * bgroups + (size_t)(blk >> 4)) << 4) | (size_t)(blk & 15))
            << 4) | (size_t)(row & 15);
}

// ---------------------------------------------------------------- device side

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float gd_h2f(uint16_t h) {
    return (float)__builtin_bit_cast(f16, h);
}
__device__ __forceinline__ uint16_t gd_f2h(float x) {
    return __builtin_bit_cast(uint16_t, (f16)x);   // RNE
}

__device__ __forceinline__ float gd_silu(float x) { return x / (1.0f + expf(-x)); }
__device__ __forceinline__ float gd_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
// Stable softplus, relu(x) + log1p(exp(-|x|)) (Kernels.swift:7-10).
__device__ __forceinline__ float gd_softplus(float x) {
    return fmaxf(x, 0.0f) + log1pf(expf(-fabsf(x)));
}

// DPP lane moves within a row of 16 lanes (no LDS round trip, unlike a
// general shuffle): quad_perm (1,0,3,2) and (2,3,0,1) exchange with lane
// i ^ 1 and i ^ 2; the half-row mirror takes lane 7 - i of each 8, the row
// mirror lane 15 - i of each 16.
template <int CTRL> __device__ __forceinline__ float gd_dpp(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int GD_DPP_XOR1 = 0xB1, GD_DPP_XOR2 = 0x4E, GD_DPP_HALF_MIRROR = 0x141,
              GD_DPP_MIRROR = 0x140;

// Sum over each row of 16 lanes, every lane of the row getting it: after the
// quad exchanges each quad's lanes hold the same value, so the half-row
// mirror pairs each lane with one holding the other quad's sum, and the row
// mirror likewise for the other half-row.  The whole wave must be active.
__device__ __forceinline__ float gd_row_sum(float v) {
    v += gd_dpp<GD_DPP_XOR1>(v);
    v += gd_dpp<GD_DPP_XOR2>(v);
    v += gd_dpp<GD_DPP_HALF_MIRROR>(v);
    return v + gd_dpp<GD_DPP_MIRROR>(v);
}

// Sum over the 64 lanes of a wave, every lane getting the total: the row
// sums, then the four rows (r0 + r1) + (r2 + r3).  The whole wave must be
// active.
__device__ __forceinline__ float gd_wave_sum(float v) {
    v = gd_row_sum(v);
    auto row = [&](int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)); };
    return (row(0) + row(16)) + (row(32) + row(48));
}

// Sum over a block of `nthreads` (multiple of 64, <= 1024); `red` is LDS of
// at least nthreads/64 floats.  Every thread gets the total.
__device__ __forceinline__ float gd_block_sum(float v, float *red) {
    v = gd_wave_sum(v);
    const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = 0.0f;
    for (int i = 0; i < nw; i++) t += red[i];
    return t;
}

// The reference test LCG (MetalSelfTest.swift:12-21) with O(log n) jump-ahead:
// state after n steps from s is A^n s + C (A^n - 1)/(A - 1), composed by
// squaring the affine map.
#define GD_LCG_A 6364136223846793005ULL
#define GD_LCG_C 1442695040888963407ULL
#define GD_LCG_SEED_MIX 0x9E3779B97F4A7C15ULL

__host__ __device__ __forceinline__ uint64_t gd_lcg_skip(uint64_t s, uint64_t n) {
    uint64_t a = GD_LCG_A, c = GD_LCG_C;      // current map x -> a x + c
    uint64_t ra = 1, rc = 0;                  // accumulated map
    while (n) {
        if (n & 1) { ra = ra * a; rc = rc * a + c; }
        c = c * (a + 1);
        a = a * a;
        n >>= 1;
    }
    return ra * s + rc;
}
