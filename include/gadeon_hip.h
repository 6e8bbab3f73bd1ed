/*
 * gadeon_hip.h -- C ABI of the MI355X (gfx950) implementation of Gadeon's
 * quantized hot path: Q2_0 ternary GEMV/GEMM and the Gated DeltaNet (GDN)
 * recurrence, plus the glue a Bonsai-shaped hybrid stack needs around them.
 *
 * The surface mirrors the reference's typed dispatch layer `MetalEnc`
 * (LLM/src/Metal/MetalEnc.swift): one entry per kernel, asynchronous on the
 * context's single in-order HIP stream, with the same argument meaning.  The
 * runtime half (`MetalContext`, LLM/src/Metal/MetalContext.swift) becomes
 * gd_ctx_* / gd_alloc / gd_upload.
 *
 * Conventions
 *   - Every entry returns int: GD_OK (0) or a negative GD_E* code.  Entries
 *     never abort; gd_last_error(ctx) returns the message of the last failure
 *     on that context.  (Reference: MetalErr, MetalContext.swift:331-349, and
 *     the non-throwing dispatch methods of MetalEnc.swift:9-13.)
 *   - Device pointers are plain `void*` from gd_alloc.  The caller owns every
 *     device buffer; the context owns only its stream and events.
 *   - Compute entries enqueue on the context stream and return immediately;
 *     gd_sync / gd_download block.  One context must not be used from two
 *     threads at once (MetalBackend.swift:3-4: the session serializes calls).
 *   - Dimension names follow the reference's GEMV/GEMM convention, spelled
 *     out: K = reduction length (GGUF ne0), R = output rows (reference "M",
 *     GGUF ne1), T = tokens (reference "N").  out[T][R] = X[T][K] . W[R][K]^T.
 *   - Activation dtype codes: GD_F32 (IEEE binary32) and GD_F16 (binary16,
 *     passed as uint16_t bit patterns).
 */
#ifndef GADEON_HIP_H
#define GADEON_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- error codes --------------------------------------------------------- */
#define GD_OK        0
#define GD_EINVAL   -1   /* bad argument: shape, alignment, null pointer   */
#define GD_ENODEV   -2   /* no HIP device / device index out of range      */
#define GD_ENOMEM   -3   /* device allocation failed                       */
#define GD_ELAUNCH  -4   /* kernel launch failed                           */
#define GD_EHIP     -5   /* any other HIP runtime error                    */
#define GD_ESTOPPED -6   /* cooperative stop observed between chunks       */

#define GD_F32 0
#define GD_F16 1

/* Q2_0 block geometry: 128 weights in 34 bytes {f16 d; u8 qs[32]}.
 * Reference: Quant.swift:2-12, GGUF.swift:13 (type 42), Kernels.metal:2484-2490. */
#define GD_Q2_0_QK          128
#define GD_Q2_0_BLOCK_BYTES 34

typedef struct gd_ctx gd_ctx;

/* ---- runtime: MetalContext (MetalContext.swift:103-305) ------------------ */

/* Number of visible HIP devices (0 when none).  Does not create a context. */
int gd_device_count(int *n);

/* Create a context on `device`: sets the device, creates one default-priority
 * stream and the timing events.  Replaces MetalContext.init (MetalContext.swift:103-129). */
int gd_ctx_create(int device, gd_ctx **out);
void gd_ctx_destroy(gd_ctx *ctx);

/* Message of the last failing call on ctx ("" if none).  ctx may be NULL:
 * then the message of the last failing gd_ctx_create in this process. */
const char *gd_last_error(const gd_ctx *ctx);

/* Device memory, owned by the caller (MetalContext.makeF32, :291-305). */
int gd_alloc(gd_ctx *ctx, size_t bytes, void **dptr);
int gd_free(gd_ctx *ctx, void *dptr);
/* Host->device / device->host copies.  Both are synchronous with respect to
 * the context stream (download waits for all enqueued work first). */
int gd_upload(gd_ctx *ctx, void *dst, const void *src, size_t bytes);
int gd_download(gd_ctx *ctx, void *dst, const void *src, size_t bytes);
/* Device->device copy and fill, enqueued on the stream (fill via a kernel, so
 * the call is safe inside stream capture). */
int gd_copy(gd_ctx *ctx, void *dst, const void *src, size_t bytes);
int gd_fill_u32(gd_ctx *ctx, void *dst, uint32_t value, size_t count);
/* dst[i] = src[i] converted between GD_F32 and GD_F16 (RNE), i < n. */
int gd_cast(gd_ctx *ctx, const void *src, int src_dtype, void *dst, int dst_dtype,
            size_t n);
/* Block until every call enqueued on ctx has finished. */
int gd_sync(gd_ctx *ctx);

/* Stream-ordered timing with HIP events recorded on the context stream, the
 * same stream every compute entry launches on.  gd_timer_stop waits for the
 * stop event and returns the elapsed milliseconds. */
int gd_timer_start(gd_ctx *ctx);
int gd_timer_stop(gd_ctx *ctx, float *ms);

/* ---- recorded command sequences ---------------------------------------------
 * The reference encodes all dispatches of a token or chunk into one Metal
 * command buffer and commits it once (MetalEngine.swift:657-728).  Here the
 * compute entries called between gd_graph_begin and gd_graph_end are recorded
 * into a HIP graph instead of running; gd_graph_launch replays the recording
 * on the context stream with the same arguments (pointers, shapes), so one
 * host call issues the whole sequence.  Only enqueue-only entries may be
 * recorded: no gd_sync, gd_download, gd_upload, gd_alloc/free or timer calls,
 * and no entry that has to grow the context workspace (run it once before
 * recording).  A failing entry inside a recording leaves the capture open;
 * gd_graph_end then fails and discards it. */
typedef struct gd_graph gd_graph;
int gd_graph_begin(gd_ctx *ctx);
int gd_graph_end(gd_ctx *ctx, gd_graph **out);
int gd_graph_launch(gd_ctx *ctx, gd_graph *g);
void gd_graph_destroy(gd_graph *g);

/* ---- Q2_0 codec (host; no GPU needed) -------------------------------------
 * The reference only decodes Q2_0 (Quant.swift:15-30); these are its exact
 * inverse.  Code c in {0,1,2,3} means weight (c-1)*d; code of weight j of a
 * block sits in qs[j>>2] at bits 2*(j&3), LSB-first (Quant.swift:4-7). */

/* Pack n weights (n % 128 == 0): codes[n] (each 0..3) and one f16 scale bit
 * pattern per 128 weights -> n/128 blocks of 34 bytes. */
int gd_q2_0_pack(const uint8_t *codes, const uint16_t *scales, size_t n,
                 uint8_t *blocks);
/* Unpack n/128 blocks -> codes[n], scales[n/128] (bit patterns as stored). */
int gd_q2_0_unpack(const uint8_t *blocks, size_t n, uint8_t *codes,
                   uint16_t *scales);

/* ---- Q2_0 device weights ---------------------------------------------------
 * On the device a Q2_0 matrix [R][K] is held as two planes in the layout the
 * MI355X kernels stream, with the same 2.125 bits per weight as the GGUF
 * blocks (plus zero padding of R to a multiple of 16 and K/128 blocks to a
 * multiple of 4):
 *   codes:  2 KiB tiles of 16 rows x 512 K, each the exact matrix-core
 *           operand order of one wave (one contiguous 1 KiB per load);
 *   scales: f16, the 16 rows of a block contiguous.
 * The layout is internal: weights enter through gd_q2_0_repack/upload and
 * leave through gd_q2_0_export(_rows).  Reference weights arrive as GGUF
 * bytes (GGUF.swift:107-117) and are repacked once at upload, where
 * MetalContext wraps the mmap without a copy (MetalContext.swift:193-212). */
typedef struct gd_q2w {
    void *codes;    /* device, ceil(R/16)*ceil(K/512)*2048 bytes, 256-aligned */
    void *scales;   /* device, ceil(R/16)*ceil(K/2048)*256 f16, 8-aligned     */
    int64_t K;      /* reduction length, multiple of 128                   */
    int64_t R;      /* output rows                                          */
} gd_q2w;

/* Allocate the two zeroed planes of a K x R matrix (free with gd_q2w_free). */
int gd_q2w_alloc(gd_ctx *ctx, int64_t K, int64_t R, gd_q2w *w);
int gd_q2w_free(gd_ctx *ctx, gd_q2w *w);
/* Repack R rows of GGUF Q2_0 blocks already in device memory (at byte offset
 * woff of `gguf`, the MetalEnc WeightRef.local) into the planes of w. */
int gd_q2_0_repack(gd_ctx *ctx, const void *gguf, uint64_t woff, gd_q2w *w);
/* Repack nrows rows of GGUF blocks (device memory, byte offset woff) into rows
 * [row0, row0+nrows) of w: one GGUF tensor into its slice of a fused
 * projection (MetalContext.swift:146-191 maps each tensor as its own window;
 * here tensors that read the same input share one matrix). */
int gd_q2_0_repack_rows(gd_ctx *ctx, const void *gguf, uint64_t woff, int64_t row0,
                        int64_t nrows, gd_q2w *w);
/* Host GGUF blocks -> freshly allocated device planes (upload + repack). */
int gd_q2_0_upload(gd_ctx *ctx, const void *host_blocks, int64_t K, int64_t R,
                   gd_q2w *w);
/* Device planes -> GGUF blocks in device memory (inverse of repack). */
int gd_q2_0_export(gd_ctx *ctx, const gd_q2w *w, void *gguf_out);
/* Rows [row0, row0+nrows) of w -> nrows*K/128 GGUF blocks in device memory
 * (one tensor of a fused projection, as GGUF stores it). */
int gd_q2_0_export_rows(gd_ctx *ctx, const gd_q2w *w, int64_t row0, int64_t nrows,
                        void *gguf_out);

/* ---- Q2_0 GEMV (decode): MetalEnc.gemv, MetalEnc.swift:78-99 -----------------
 * y[r] = sum_k W[r,k] * x[k] for r < R, f32 accumulate, f32 out.
 * x dtype GD_F32 (the reference's buffer type; split exactly into two f16
 * halves in-kernel) or GD_F16 (the BASELINE decode activations).
 * Replaces the Metal kernel q2_0_gemv (Kernels.metal:30-119) and the CPU
 * Q2_0.matvec (Quant.swift:36-77). */
int gd_q2_0_gemv(gd_ctx *ctx, const gd_q2w *w, const void *x, int x_dtype,
                 float *y);

/* y = W x (+ bias if not null) with x = f16(rmsnorm(o_h) * w_norm * silu(z))
 * over each 128-element block h of o (one value head): the gated norm of a
 * GDN layer's output (GDN.swift:113-115; rmsnorm_rows + mul_silu,
 * Kernels.metal:751-768, 1126-1131) done in the GEMV's x staging, as the
 * stack's decode feeds its GDN out_proj.  o, z f32 [K], w_norm f32 [128],
 * bias and y f32 [R]; K a multiple of 128, at most 30720.  No counterpart in
 * the reference (it runs the norm and the GEMV as separate dispatches). */
int gd_q2_0_gemv_gated(gd_ctx *ctx, const gd_q2w *w, const float *o, const float *z,
                       const float *w_norm, float eps, const float *bias, float *y);

/* gd_q2_0_gemv with K cut into `ksplit` (1..4) ranges whose partial rows go
 * to y + z * R (y holds ksplit * R floats); *nsplit receives the number of
 * partials written (it can be lower than ksplit for short K).  Summing them
 * gives gd_q2_0_gemv's y.  A short R leaves CUs idle unless K is split; the
 * partials are meant for a consumer that adds them anyway (the residual
 * delta of gd_q2_0_gemv_norm).  No counterpart in the reference. */
int gd_q2_0_gemv_split(gd_ctx *ctx, const gd_q2w *w, const void *x, int x_dtype,
                       float *y, int ksplit, int *nsplit);

/* Decode GEMV with the residual add and RMSNorm that precede it fused into
 * the x staging: h' = h + sum of nd partials delta + z * delta_stride (nd = 0
 * or delta null: none), x = h' * w_norm / sqrt(mean(h'^2) + eps), y = W x,
 * with x taken at f32 precision (about 20 bits: W (h' * w_norm) formed from
 * it, then scaled by the 1/rms), as the reference's decode GEMV reads f32 x.
 * hout (may be null, must not alias h) receives h'.  The result of
 * gd_add + gd_rmsnorm(.., GD_F32, ..) + gd_q2_0_gemv (MetalEnc.addInplace +
 * rmsnorm + gemv, MetalEnc.swift:213-236, 572-597, 78-99) in one launch
 * instead of three.  h, delta, w_norm and hout are f32 [K], 16-byte aligned
 * (delta_stride a multiple of 4); K <= 15744.  With glu_out not null, W is
 * [gate; up] (R = 2 ff rows, ff a multiple of 16) and glu_out[r] =
 * f16(silu(gate_r . x) * (up_r . x)), r < ff, replaces y (y unused): the
 * feed-forward's SwiGLU (Kernels.metal:1118-1139 silu_mul) fused in. */
int gd_q2_0_gemv_norm(gd_ctx *ctx, const gd_q2w *w, const float *h, const float *delta,
                      int nd, int64_t delta_stride, const float *w_norm, float eps,
                      float *hout, float *y, uint16_t *glu_out);

/* ---- Q2_0 GEMM (prefill): MetalEnc.gemm, MetalEnc.swift:145-189 --------------
 * Y[t][r] = sum_k X[t][k] * W[r][k], token-major X[T][K] and Y[T][R].
 * Weights are dequantized exactly to f16 in registers and multiplied on fp16
 * MFMA with f32 accumulation (reference: q2_0_gemm_mm_h,
 * Kernels.metal:372-466, which stages both operands as half).  X dtype GD_F32
 * is rounded to f16 while staging, as the reference does (Kernels.metal:428);
 * Y dtype GD_F32 or GD_F16 (round-to-nearest-even of the f32 accumulator).
 * The tile shape and K split are chosen by a cost model of the MI355X. */
int gd_q2_0_gemm(gd_ctx *ctx, const gd_q2w *w, int64_t T, const void *X,
                 int x_dtype, void *Y, int y_dtype);

/* gd_q2_0_gemm with an explicit plan: workgroups of nw waves (4 or 8), each
 * wave mt*32 tokens by nt*32 weight rows, (mt, nt) in {(1,1), (2,1), (4,1),
 * (2,2), (4,2), (8,1)} ((1,1) and (8,1) with 4 waves only), and K split
 * `split` ways (1..16; partials summed in the context workspace).  For
 * tuning and for tests that cover every kernel variant; no counterpart in
 * the reference. */
int gd_q2_0_gemm_plan(gd_ctx *ctx, const gd_q2w *w, int64_t T, const void *X,
                      int x_dtype, void *Y, int y_dtype, int mt, int nt, int split, int nw);
/* gd_q2_0_gemm on the 4 x 2 x 8 tile that also holds a seventeenth 32-row
 * fragment (544 rows a workgroup), K split `split` ways; it writes f32, so
 * f16 Y needs split > 1 (partials summed in the workspace).  For tuning and
 * for tests that cover the planner's choices; no counterpart in the
 * reference. */
int gd_q2_0_gemm_plan17(gd_ctx *ctx, const gd_q2w *w, int64_t T, const void *X,
                        int x_dtype, void *Y, int y_dtype, int split);

/* gd_q2_0_gemm (f16 X, f32 Y) on an unsplit tile (mt, nt, nw as for
 * gd_q2_0_gemm_plan) over the rows below *tail_r0 = R rounded down to the
 * tile's rows, with the remaining rows (R must not be a whole number of tiles)
 * run in the same launch as K-split units: at most tail_split splits,
 * *tail_nz made, f32 partials tailY[z][t][r - *tail_r0] (summed by the
 * caller in split order); Y's rows from *tail_r0 on are not written.  The
 * stack runs its GDN in_proj so (its last 32 rows are the gate columns).
 * For tests; no counterpart in the reference. */
int gd_q2_0_gemm_plan_tail(gd_ctx *ctx, const gd_q2w *w, int64_t T, const void *X, float *Y,
                           int mt, int nt, int nw, int tail_split, float *tailY, int *tail_nz,
                           int *tail_r0);

/* Feed-forward GEMM with SwiGLU fused into the epilogue: W is [gate; up]
 * (R = 2 ff rows, ff a multiple of 16), X f16 [T][K], out f16 [T][ff] =
 * silu(X gate^T) * (X up^T), as gd_q2_0_gemm (f32 Y) followed by the
 * reference's silu_mul (Kernels.metal:1118-1139) and an f16 rounding, without
 * the f32 intermediate (the columns of a second launch may go through f32
 * K-split partials in the context workspace, which the call may grow).  No
 * counterpart in the reference as one call. */
int gd_q2_0_gemm_swiglu(gd_ctx *ctx, const gd_q2w *w, int64_t T, const void *X,
                        uint16_t *out);
/* gd_q2_0_gemm_swiglu with the tile choice made by the caller: tile17 = 1
 * runs every column in one launch of the 4 x 2 x 8 tile that also holds a
 * seventeenth 16-column fragment (272 columns a workgroup, what the planner
 * picks for ff = 17408 at T = 512); tile17 = 0 keeps the planner's choice
 * among the other tiles.  For tuning and for tests that cover both; no
 * counterpart in the reference. */
int gd_q2_0_gemm_swiglu_plan(gd_ctx *ctx, const gd_q2w *w, int64_t T, const void *X,
                             uint16_t *out, int tile17);

/* ---- Q2_0 row dequant: MetalEnc.dequantRow / embedBatch ----------------------
 * out[n][k] = (code-1)*d of row ids[n], exactly (f16 * small integer is exact
 * in f32).  Reference: q2_0_dequant_row (Kernels.metal:472-485), embed_batch
 * (Kernels.metal:1468-1485), Q2_0.dequant (Quant.swift:15-30). */
int gd_q2_0_dequant_rows(gd_ctx *ctx, const gd_q2w *w, const int32_t *ids,
                         int64_t n, float *out);

/* ---- GDN glue (MetalEnc.swift:603-653, 720-733; Kernels.metal:1146-1243) ----- */

/* beta = sigmoid(bPre); g = softplus(aPre + dt[h]) * aNeg[h], h = i % nV,
 * for i < count.  MetalEnc.gdnGate (MetalEnc.swift:603-618), gdn_gate
 * (Kernels.metal:1146-1168), GDN.swift:39-42. */
int gd_gdn_gate(gd_ctx *ctx, const float *bPre, const float *aPre,
                const float *dt, const float *aNeg, float *beta, float *g,
                int nV, int64_t count);

/* Causal depthwise conv + silu over N tokens with the (dConv-1)-deep ring
 * state[(dConv-1)][convDim] (time-minor), weights cw[convDim][dConv].
 * N == 1 is MetalEnc.gdnConv, N > 1 MetalEnc.gdnConvBatch.  Reference:
 * gdn_conv / gdn_conv_batch (Kernels.metal:1174-1199, 1490-1520), GDN.swift:44-62. */
int gd_gdn_conv(gd_ctx *ctx, const float *qkvMix, float *convState,
                const float *cw, float *out, int convDim, int dConv,
                int64_t N);

/* x / sqrt(sum(x^2) + eps) over `rowsPerTok` rows of length d per token,
 * token n based at n*tokStride (floats), for `tokens` tokens.
 * MetalEnc.l2normRows(Batch) (MetalEnc.swift:249-272), Kernels.swift:41-52. */
int gd_l2norm_rows(gd_ctx *ctx, float *x, int d, int rowsPerTok,
                   int64_t tokStride, int64_t tokens, float eps);

/* In-place x * w / sqrt(mean(x^2) + eps) per row of length d (w[d]).
 * MetalEnc.rmsnormRows (MetalEnc.swift:238-247), Kernels.swift:26-37. */
int gd_rmsnorm_rows(gd_ctx *ctx, float *x, int d, int64_t rows,
                    const float *w, float eps);

/* y[row] = x[row] * w / sqrt(mean(x^2) + eps), rows of length n, into f32
 * or f16 y.  MetalEnc.rmsnorm / rmsnormBatch (MetalEnc.swift:213-236). */
int gd_rmsnorm(gd_ctx *ctx, const float *x, const float *w, void *y,
               int y_dtype, int64_t n, int64_t rows, float eps);

/* Elementwise glue: a = silu(a)*b (silu_mul), a = a*silu(b) (mul_silu),
 * x += y (add_inplace).  MetalEnc.swift:572-597, Kernels.metal:1118-1139. */
int gd_silu_mul(gd_ctx *ctx, float *a, const float *b, int64_t n);
int gd_mul_silu(gd_ctx *ctx, float *a, const float *b, int64_t n);
int gd_add(gd_ctx *ctx, float *x, const float *y, int64_t n);

/* ---- gated GQA attention over an f16 paged KV cache ---------------------------
 * Head dims 128 and 256.  The cache of one attention layer is a pool of
 * pages of `page_size` positions, each position kv_dim = head_dim * n_head_kv
 * f16 values (k_cache and v_cache); position p lives in page page_table[p /
 * page_size] at slot p % page_size.  The reference's table holds page
 * addresses (MetalKVPool.swift: bindless kAddr / vAddr); this one holds page
 * indices into one allocation.  q, k, v rows are f32 [tokens][heads][head_dim]
 * as in MetalEnc. */

/* q_full [N][n_head][2 head_dim] (per head q | gate, the hybrid's fused
 * projection) -> q and gate [N][n_head][head_dim].  MetalEnc.splitQGate(Batch)
 * (MetalEnc.swift:656-665, 780-791), Attention.swift:84-93. */
int gd_split_q_gate(gd_ctx *ctx, const float *q_full, float *q, float *gate,
                    int head_dim, int n_head, int64_t N);

/* Partial NEOX rope in place on x [N][n_head][head_dim]: dims i < n_rot/2 and
 * i + n_rot/2 of each head turn by (base_pos + n) * base^(-2i/n_rot).
 * MetalEnc.rope / ropeBatch (MetalEnc.swift:560-569, 817-828), Kern.ropeNeox
 * (Kernels.swift:66-84). */
int gd_rope(gd_ctx *ctx, float *x, int head_dim, int n_head, int n_rot, float base,
            int base_pos, int64_t N);

/* k, v [N][kv_dim] f32 -> the cache at positions base_pos .. base_pos+N-1,
 * rounded to f16.  MetalEnc.kvAppend / kvAppendBatch (MetalEnc.swift:667-677,
 * 830-847), kv_append / kv_append_batch (Kernels.metal:1446-1466, 1726-1766). */
int gd_kv_append(gd_ctx *ctx, const float *k, const float *v, uint16_t *k_cache,
                 uint16_t *v_cache, const int32_t *page_table, int kv_dim, int base_pos,
                 int page_size, int64_t N);

/* One query per head over cached positions lo .. T-1 (the token's own k, v
 * appended first): out[h] = softmax((q_h . k_t) * scale) . v_t, times
 * sigmoid(gate[h]) when gated (1; 0: plain).  q, gate, out [n_head][head_dim]
 * f32.  part: scratch of n_head * 16 * (head_dim + 2) floats (the key-split
 * partials).  MetalEnc.attnPaged (MetalEnc.swift:679-706), attn_head
 * (Kernels.metal:1423-1445). */
int gd_attn_paged(gd_ctx *ctx, const float *q, const uint16_t *k_cache,
                  const uint16_t *v_cache, const int32_t *page_table, const float *gate,
                  float *out, float *part, int head_dim, int n_head, int n_head_kv, int T,
                  int kv_dim, int page_size, float scale, int gated, int lo);

/* N causal queries at positions base_pos + n over the cached positions
 * 0 .. base_pos + n (their own keys appended first): qN, gateN, outN
 * [N][n_head][head_dim] f32, 16-byte aligned.  window must be 0 (the whole
 * history; the reference's sliding window serves another model family).
 * MetalEnc.attnBatch (MetalEnc.swift:966-1025), attn_batch / attn_batch_mm
 * (Kernels.metal:1767-2022). */
int gd_attn_batch(gd_ctx *ctx, const float *q, const uint16_t *k_cache,
                  const uint16_t *v_cache, const int32_t *page_table, const float *gate,
                  float *out, int head_dim, int n_head, int n_head_kv, int kv_dim,
                  int page_size, float scale, int base_pos, int64_t N, int gated, int window);

/* ---- GDN recurrence -----------------------------------------------------------
 * State S[nV][dS][dS] f32, key-major: S[h][i*dS + j], i = key, j = value
 * (GDN.swift:9-16, Kernels.metal:1225).  Head map hk = hv % nK
 * (GDN.swift:79).  Per token and value head:
 *   gamma = exp(g); S *= gamma; sk = S^T k; delta = beta*(v - sk);
 *   S += k (x) delta; o = qScale * S^T q            (GDN.swift:84-108) */

/* One token, q/k already L2-normalized: MetalEnc.gdnScan (MetalEnc.swift:636-653),
 * gdn_scan (Kernels.metal:1206-1243).  q,k [nK*dS], v [nV*dS], g,beta [nV]. */
int gd_gdn_scan(gd_ctx *ctx, const float *q, const float *k, const float *v,
                const float *g, const float *beta, float *S, float *o,
                int nV, int nK, int dS, float qScale);

/* N tokens out of the conv output rows convOutN[N][convDim] = [q|k|v]:
 * MetalEnc.gdnScanBatch (MetalEnc.swift:741-778), which serves any dS with
 * gdn_scan_batch2 (dS % 32 == 0, dS <= 256) or gdn_scan_batch
 * (Kernels.metal:1525-1625).  dS = 128 runs the chunked kernel below; any
 * other dS up to 1024 a token-serial scan in the reference's order. */
int gd_gdn_scan_batch(gd_ctx *ctx, const float *convOutN, int keyDim,
                      int valueDim, int convDim, const float *gN,
                      const float *betaN, float *S, float *oN, int nV, int nK,
                      int dS, float qScale, int64_t N);

/* Fused state-carry decode step for B independent sequences (no reference
 * counterpart as one kernel: it fuses gdn_gate, l2norm_rows x2 and gdn_scan,
 * MetalEngine.swift:730-754).  Per sequence b:
 *   q,k raw [B][nK][dS], v [B][nV][dS] (dtype io_dtype), o [B][nV][dS]
 *   (io_dtype), S [B][nV][dS][dS] f32 in place.
 *   If dt != NULL: beta = sigmoid(beta_in), g = softplus(g_in + dt)*aNeg
 *   (pre-activations [B][nV]); else beta_in/g_in are beta and g.
 *   q and k are L2-normalized with eps before use. */
int gd_gdn_decode(gd_ctx *ctx, int B, int nV, int nK, int dS,
                  const void *q, const void *k, const void *v, int io_dtype,
                  const float *g_in, const float *beta_in, const float *dt,
                  const float *aNeg, float *S, void *o, float qScale,
                  float eps);

/* Chunked prefill of T tokens for one sequence (new: the reference scans
 * token by token; the chunk identity is the closed form of
 * LLM/src/CoreML/MtpRollback.swift:3-12, 20-42).
 *   q,k [T][nK][dk], v [T][nV][dv] (io_dtype, row stride given in elements:
 *   q_stride, k_stride, v_stride between tokens), g, beta [T][nV] f32,
 *   S [nV][dk][dv] f32 in/out, o [T][nV][dv] (o_dtype, stride o_stride).
 *   q/k are used as given (normalize first with gd_l2norm_rows).  C is the
 *   chunk length (16, 32 or 64; 32 is the fastest on MI355X at T 128..2048);
 *   T need not be a multiple of C.
 *   Currently dk == dv == 128. */
int gd_gdn_prefill(gd_ctx *ctx, int64_t T, int nV, int nK, int dk, int dv,
                   const void *q, int64_t q_stride, const void *k,
                   int64_t k_stride, const void *v, int64_t v_stride,
                   int io_dtype, const float *g, const float *beta, float *S,
                   void *o, int64_t o_stride, int o_dtype, float qScale,
                   int C);

/* gd_gdn_prefill for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference.  Same arguments and results as
 * gd_gdn_prefill, whose per-chunk operands go through a context workspace
 * that may grow with hipMalloc; here they live in a fixed device array of
 * GD_GDN_PREFILL_SCRATCH_BYTES per GPU, held until the process ends, and the
 * call allocates nothing.  Shapes needing more are rejected with GD_EINVAL:
 * the scratch takes nV * ceil(T/C) * b bytes, b = 98,560 (f16 io) or 147,712
 * (f32 io) at C = 64, so e.g. 16 heads fit T <= 896 (f32) / 1344 (f16).
 * Every call on a GPU shares the array (nothing in it needs to start at
 * zero: each call writes all it reads), so calls that overlap on one GPU --
 * from two streams or threads -- race. */
#define GD_GDN_PREFILL_SCRATCH_BYTES (32u << 20)
int gd_gdn_prefill_noalloc(gd_ctx *ctx, int64_t T, int nV, int nK, int dk, int dv,
                           const void *q, int64_t q_stride, const void *k,
                           int64_t k_stride, const void *v, int64_t v_stride,
                           int io_dtype, const float *g, const float *beta, float *S,
                           void *o, int64_t o_stride, int o_dtype, float qScale,
                           int C);

/* ---- synthetic data on the device -----------------------------------------
 * Counter-addressable copy of the reference's test LCG
 * (MetalSelfTest.swift:12-21): element i of stream `seed` is the (i+1)-th
 * state s = s*6364136223846793005 + 1442695040888963407 from
 * s0 = seed + 0x9E3779B97F4A7C15, bits = s >> 33.  Each thread jumps ahead
 * to its run, so the stream is identical to the sequential one. */

/* out[i] = bits/2^32 * (hi-lo) + lo  (f32), i < n. */
int gd_rand_uniform(gd_ctx *ctx, float *out, size_t n, uint64_t seed,
                    float lo, float hi);
/* Normal(mean, std) by Box-Muller on the pairs (2i, 2i+1) of the stream,
 * into f32 or f16. */
int gd_rand_normal(gd_ctx *ctx, void *out, int dtype, size_t n, uint64_t seed,
                   float mean, float std);
/* A random Q2_0 matrix straight into device planes: codes iid uniform over
 * {0,1,2} (ternary -1,0,+1, p = 1/3 each: code = (bits*3)>>32 of stream
 * `seed`), scales RNE-f16 of lo + (hi-lo)*u over stream seed+1. */
int gd_rand_q2w(gd_ctx *ctx, gd_q2w *w, uint64_t seed, float lo, float hi);

/* ---- Bonsai-shape stack (config 4) -----------------------------------------------
 * A GDN/attention hybrid (qwen35, e.g. the random-init 64-layer config 4) or
 * a dense all-attention qwen3 stack, driven exactly like MetalEngine.extend /
 * decode (MetalEngine.swift:183-257, 405-451, 657-796) and the CPU oracle
 * BonsaiEngine.forward (BonsaiEngine.swift:155-178). */
typedef struct gd_stack_config {
    int n_layer;        /* 64 */
    int n_embd;         /* 5120 */
    int n_ff;           /* 17408 */
    int n_head;         /* 40 (attention q heads) */
    int n_head_kv;      /* 8 */
    int head_dim;       /* 128 (attention head dim: 128 or 256) */
    int n_rot;          /* 64 (partial NEOX rope) */
    float rope_base;    /* 1e7 */
    float eps;          /* 1e-6 */
    int n_vocab;        /* 151936 */
    int attn_interval;  /* 4: attention where (il+1) % 4 == 0 */
    int d_state;        /* 128 */
    int n_k_head;       /* 16 */
    int n_v_head;       /* 16 */
    int d_conv;         /* 4 */
    int kv_block;       /* 16 positions per KV page */
    int max_ctx;        /* KV capacity in positions */
    int max_batch;      /* largest prefill chunk (tokens) */
    int dense;          /* 0: qwen35 hybrid; 1: dense qwen3 lineage (BonsaiConfig.dense,
                           Model.swift:23-25): attention in every layer
                           (attn_interval 1), q projected without a gate, output
                           ungated; d_state, n_k_head, n_v_head, d_conv 0 */
} gd_stack_config;

typedef struct gd_stack gd_stack;

int gd_stack_create(gd_ctx *ctx, const gd_stack_config *cfg, uint64_t seed,
                    gd_stack **out);
void gd_stack_destroy(gd_stack *st);
/* Clear GDN conv/recurrent state, KV pages and position (BonsaiEngine.reset). */
int gd_stack_reset(gd_stack *st);
/* Prefill n ids onto the current state (chunks of cfg.max_batch) and return
 * the greedy next token (MetalEngine.extend).  logits may be NULL, else it
 * receives the last token's n_vocab f32 logits (host memory). */
int gd_stack_prefill(gd_stack *st, const int32_t *ids, int n, int32_t *next,
                     float *logits);
/* One token (MetalEngine.decode). */
int gd_stack_decode(gd_stack *st, int32_t token, int32_t *next,
                    float *logits);
/* n greedy decode steps continuing from the token the last prefill/decode
 * picked, with no host round trip between steps (the step is captured once
 * as a HIP graph; the picked id stays on the device).  tokens[n] receives the
 * n ids generated.  Equivalent to n chained gd_stack_decode calls.  A raised
 * stop ends it before its next step with GD_ESTOPPED; the steps already made
 * stay made (tokens[0 .. k) and the position, gd_stack_position, advance by
 * those k). */
int gd_stack_generate(gd_stack *st, int n, int32_t *tokens);
/* Cooperative stop (MetalEngine.requestStop / shouldStop, MetalEngine.swift:
 * 15-25, 79-81), safe from another thread.  gd_stack_prefill clears the
 * signal when it starts (a previous turn's stop does not end the next,
 * MetalEngine.swift:183-186) and returns GD_ESTOPPED at the next chunk
 * boundary once it is raised; gd_stack_generate checks it before each step.
 * The signal stays raised until the next prefill or gd_stack_reset;
 * gd_stack_should_stop reads it (*raised = 1 or 0). */
int gd_stack_request_stop(gd_stack *st);
int gd_stack_should_stop(gd_stack *st, int *raised);
/* eager = 1: gd_stack_generate launches every step's kernels directly
 * instead of replaying the captured decode graph (the same kernels in the
 * same order, the same results; for kernel-trace profilers that do not
 * follow graph launches).  0 (the default) replays the graph.  No
 * counterpart in the reference (MetalEngine reuses its command buffers). */
int gd_stack_set_eager(gd_stack *st, int eager);

/* Weight and state introspection for parity tests: tensor `name` of layer
 * `layer` (-1 for global tensors).  A Q2_0 tensor fills *w with the matrix
 * that holds it (projections that read the same input are fused into one
 * matrix), *row0 with its first row there and *count with its row count
 * (read it with gd_q2_0_export_rows); f32 tensors fill *f32 and *count.  Names follow the GGUF ones used in Model.swift:100-145
 * ("attn_norm", "attn_qkv", "attn_gate", "ssm_beta", "ssm_alpha", "ssm_dt",
 * "ssm_a", "ssm_conv1d", "ssm_norm", "ssm_out", "attn_q", "attn_k", "attn_v",
 * "attn_output", "attn_q_norm", "attn_k_norm", "post_attention_norm",
 * "ffn_gate", "ffn_up", "ffn_down", "token_embd", "output" (the lm_head,
 * token_embd's matrix when tied), "output_norm",
 * "ssm_conv_state", "ssm_state"). */
int gd_stack_tensor(gd_stack *st, int layer, const char *name, gd_q2w *w,
                    int64_t *row0, float **f32, int64_t *count);
int gd_stack_position(gd_stack *st, int64_t *pos);
/* KV page accounting (any pointer may be NULL): *live = pages mapped by the
 * live state, *held = pages of the stack's pool held by the live state or a
 * bookmark, *capacity = pages each attention layer's K (and V) pool holds.
 * Pages are kv_block positions; the pool starts at twice a prefill chunk and
 * doubles on demand (MetalKVPool allocates pages lazily, MetalKVPool.swift:
 * 53-66); a bookmark shares the completed pages and holds a copy of a partial
 * tail page (MetalKVPool.snapshot, :102-110).  No counterpart in the
 * reference as a call: memory accounting and tests. */
int gd_stack_kv_pages(gd_stack *st, int64_t *live, int64_t *held, int64_t *capacity);

/* ---- Bookmarks: MetalEngine.bookmark / restore / serialize / deserialize -------
 * (MetalEngine.swift:455-584).  A bookmark is a device-memory snapshot of the
 * generation state: position, rope shift, the last greedy pick, each GDN layer's conv ring
 * and recurrent state, each attention layer's K/V over positions [0, pos).
 * It stays valid across later decode, reset and prefill calls and can be
 * restored any number of times, into the stack it came from or another of
 * the same geometry on the same context.  gd_stack_serialize writes the bytes
 * of MetalEngine.serialize: i64 pos, i64 ropeShift, the conv and the rec
 * dicts (i64 count, then per GDN layer in ascending order i64 layer, i64 n,
 * n f32), and the KV dict (i64 count, then per attention layer i64 layer,
 * i64 len, i64 n, n f32 of K, i64 n, n f32 of V, each [len][n_head_kv *
 * head_dim]); all little-endian, KV widened from the cache's halves.  Call it
 * with buf NULL to get the size in *len.  gd_stack_deserialize checks every
 * count and layer index against the stack and returns a bookmark to restore;
 * that format carries no pick, so after restoring it the next call must be
 * gd_stack_decode (gd_stack_generate fails until then).  ropeShift is what
 * MetalEngine keeps after an image span compressed the M-RoPE positions:
 * from then on a token at position p is rotated at p + ropeShift while its
 * KV slot and causality stay at p (MetalEngine.swift:432-435); restoring a
 * bookmark restores it, gd_stack_reset clears it (this build has no vision
 * prefill of its own, so only restored states carry one). */
typedef struct gd_bookmark gd_bookmark;

int gd_stack_bookmark(gd_stack *st, gd_bookmark **out);
int gd_stack_restore(gd_stack *st, const gd_bookmark *b);
void gd_bookmark_free(gd_bookmark *b);
int gd_stack_serialize(gd_stack *st, const gd_bookmark *b, void *buf, size_t cap, size_t *len);
int gd_stack_deserialize(gd_stack *st, const void *data, size_t n, gd_bookmark **out);
/* The same bookmark in the CPU engine's parked-state bytes, BonsaiEngine.serialize /
 * deserialize (BonsaiEngine.swift:65-112, StateBytes.swift:11-72): the magic "GDNS",
 * i64 version 1, i64 pos, i64 count of GDN layers, then per GDN layer in ascending
 * order i64 layer, i64 n, n f32 of its conv ring, i64 n, n f32 of its state; i64
 * count of attention layers, then per attention layer i64 layer, i64 len, i64
 * pages, that many K pages then as many V pages, each i64 n, n f32 of 512 positions
 * (KVCache.pageP) x n_head_kv * head_dim, positions past len zero.  The reader
 * refuses bytes without that header or version (BonsaiEngine.deserialize returns
 * nil), and checks every count, layer index and page size against the stack; K/V
 * are rounded to the cache's halves.  A state parked by the CPU engine thus
 * resumes on this stack, and the other way round.  The CPU engine has no
 * image spans: a bookmark with a nonzero ropeShift is refused. */
int gd_stack_serialize_gdns(gd_stack *st, const gd_bookmark *b, void *buf, size_t cap,
                            size_t *len);
int gd_stack_deserialize_gdns(gd_stack *st, const void *data, size_t n, gd_bookmark **out);

/* ---- GGUF v3 reader (host only): GGUF.swift:45-117 ---------------------------
 * gd_gguf_open maps the file read-only and parses the header, the metadata and
 * the tensor directory; tensor data starts at the first multiple of
 * general.alignment (default 32) after the directory (GGUF.swift:83-99).  All
 * reads are bounds-checked: a truncated or corrupt file fails with GD_EINVAL.
 * These entries need no device and no context; their failures are reported
 * by gd_last_error(NULL).  Pointers handed out stay valid until
 * gd_gguf_close. */
typedef struct gd_gguf gd_gguf;

int gd_gguf_open(const char *path, gd_gguf **out);          /* GGUF(path:) */
void gd_gguf_close(gd_gguf *g);
int gd_gguf_info(const gd_gguf *g, int64_t *n_tensors, int64_t *n_kv, int *version);
/* GGUF.tensor(name) / maybe(name): dims (ne0 fastest; unused dims 1), ggml
 * type (0 f32, 1 f16, 42 Q2_0, ...), a pointer to its bytes in the mapping
 * and their count.  Any out pointer may be NULL; an absent name fails.
 * gd_gguf_open rejects a file with a tensor type outside GGUFType
 * (GGUF.swift:7-14), as the reference does, or whose bytes pass the end. */
int gd_gguf_tensor(const gd_gguf *g, const char *name, int *ndim, int64_t dims[4],
                   int *type, const void **data, size_t *bytes);
/* Metadata, GGUF.int / double / bool / string / ints / doubles
 * (GGUF.swift:121-172): get_int reads integer types of any width (not bool,
 * as GGUF.int); get_float reads f32/f64 and integers; get_bool reads bool and
 * integers; arrays of integers or bools read as int64, of f32/f64 as double.
 * An absent key or one of another type fails. */
int gd_gguf_get_int(const gd_gguf *g, const char *key, int64_t *v);
int gd_gguf_get_float(const gd_gguf *g, const char *key, double *v);
int gd_gguf_get_bool(const gd_gguf *g, const char *key, int *v);
int gd_gguf_get_string(const gd_gguf *g, const char *key, const char **v);
int gd_gguf_get_ints(const gd_gguf *g, const char *key, const int64_t **v, int64_t *n);
int gd_gguf_get_floats(const gd_gguf *g, const char *key, const double **v, int64_t *n);
/* BonsaiConfig(gguf) (Model.swift:39-69): general.architecture "qwen35" (the
 * default when absent) gives the hybrid, "qwen3" the dense lineage (dense 1,
 * attn_interval 1, no ssm keys read); rope.dimension_count defaults to
 * key_length.  kv_block, max_ctx and max_batch are left 0 (they are runtime
 * choices). */
int gd_gguf_stack_config(const gd_gguf *g, gd_stack_config *cfg);
/* BonsaiModel(path:) + upload (Model.swift:133-148, MetalContext.swift:
 * 146-191): a stack whose weights are the file's tensors, repacked into the
 * fused matrices.  The lm_head is output.weight when present, else the token
 * embedding (Model.swift:145).  Every tensor the stack reads must be present
 * with its exact shape: Q2_0 matrices, f32 norms/conv/dt/a.  The file may be
 * closed once this returns. */
int gd_stack_create_from_gguf(gd_ctx *ctx, const gd_gguf *g, int kv_block, int max_ctx,
                              int max_batch, gd_stack **out);

#ifdef __cplusplus
}
#endif

#endif /* GADEON_HIP_H */
