// Q2_0 GEMV on the matrix cores: y[r] = sum_k W[r,k] x[k], as one kernel
// launch.  The kernel body, with its design notes, is gemv::run
// (gemv_core.h); this file holds the kernel and the host side: the work
// split, the K-split choice and the entry points the C ABI and the stack call.
#include "gemv_core.h"

namespace {

using gemv::GluOut;
using gemv::LDS_BYTES;
using gemv::NW;
using gemv::NormIn;
using gemv::xlds_bytes;

// ND: residual partials of the fused input (XT = 2) loaded with h and w;
// SE: x elements each staging thread converts (8 or 16).
template <int XT, bool KBP, bool F4, int ND, int SE = 16>
__global__ __launch_bounds__(64 * NW) void q2_0_gemv_mfma_kernel(gemv::Task t) {
    extern __shared__ __align__(16) uint32_t lds[];
    gemv::run<XT, KBP, F4, ND, SE>(t, (int)blockIdx.x, (int)blockIdx.y, lds);
}

// x staging bytes of a GEMV over nblk Q2 blocks: the fp4 kernel's where its
// staging and one set's per-block partials fit, else the f16 kernel's.
struct XStage { size_t bytes; bool f4; };
XStage x_stage(int nblk, bool f32x) {
    const size_t f4 = gemv::xlds_bytes_f4(nblk);
    if (f4 + (size_t)256 * ((nblk + 3) / 4) <= LDS_BYTES) return {f4, true};
    return {xlds_bytes(nblk, f32x), false};
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

// The task of one GEMV launch on `cus` workgroups, its LDS bytes and whether
// it keeps per-block partials.
int make_task(gd_ctx *ctx, const gd_q2w *w, const void *x, float *y, size_t xlds,
              const NormIn &nin, int ksplit, const GluOut &glu, int cus, const float *bias,
              gemv::Task *t, size_t *lds_out, bool *kbp,
              const gemv::RingAdv &ring = gemv::RingAdv{nullptr, nullptr, 0, 0}) {
    const int64_t K = w->K, R = w->R;
    const int nblk = (int)(K >> 7), steps = (nblk + 3) / 4;
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
    *t = gemv::Task{(const uint8_t *)w->codes, (const uint16_t *)w->scales, x, y, bias, (int)K, (int)R,
                    (int)nsets, (int)sp.per, sp.ksteps, sp.nz, (int)sp.grid,
                    {gemv::item_magic(sp.ksteps), gemv::item_magic(steps - (sp.nz - 1) * sp.ksteps)},
                    nin, glu, ring};
    *lds_out = lds;
    *kbp = sp.kbp;
    return GD_OK;
}

template <int XT>
int launch(gd_ctx *ctx, const gd_q2w *w, const void *x, float *y, XStage xs,
           const NormIn &nin = NormIn{nullptr, nullptr, nullptr, 0.f, 0, 0}, int ksplit = 1,
           const GluOut &glu = GluOut{nullptr, 0}, const float *bias = nullptr,
           const gemv::RingAdv &ring = gemv::RingAdv{nullptr, nullptr, 0, 0}) {
    const int cus = ctx->num_cus > 0 ? ctx->num_cus : 256;
    gemv::Task t;
    size_t lds;
    bool kbp;
    int rc = make_task(ctx, w, x, y, xs.bytes, nin, ksplit, glu, cus, bias, &t, &lds, &kbp, ring);
    if (rc) return rc;
    if constexpr (XT == 3) {
        // The gated head norm has the fp4 body with per-block partials only.
        GD_REQUIRE(ctx, xs.f4 && kbp, "gd_gemv_gated: K=%lld R=%lld does not fit the fp4 body",
                   (long long)w->K, (long long)w->R);
        hipLaunchKernelGGL((q2_0_gemv_mfma_kernel<3, true, true, 0>), dim3((unsigned)t.gx, t.nz),
                           dim3(64 * NW), lds, ctx->stream, t);
        GD_LAUNCHED(ctx, "q2_0_gemv_mfma");
        return GD_OK;
    } else {
        constexpr int NDM = XT == 2 ? gemv::ND_UNROLL : 0;
        const int nd = std::min(nin.nd, NDM);
        // The fp4 kernel with per-block partials and f32 x (four pieces) stages 8
        // elements a thread where all of x then fits one pass of the workgroup's
        // threads: the staging VALU work is spread over twice the waves.  (With
        // f16 x, three pieces, 16 a thread measured faster.)
        const int nblk = (int)(w->K >> 7);
        const bool se8 = XT != 0 && xs.f4 && kbp && (nblk + 5) * 16 <= 64 * NW;
        auto pick = [&](auto ndc) {
            constexpr int ND = decltype(ndc)::value;
            if constexpr (XT != 0)
                if (se8) return q2_0_gemv_mfma_kernel<XT, true, true, ND, 8>;
            return xs.f4 ? (kbp ? q2_0_gemv_mfma_kernel<XT, true, true, ND> : q2_0_gemv_mfma_kernel<XT, false, true, ND>)
                         : (kbp ? q2_0_gemv_mfma_kernel<XT, true, false, ND> : q2_0_gemv_mfma_kernel<XT, false, false, ND>);
        };
        auto kern = nd == 0 ? pick(std::integral_constant<int, 0>{})
                  : nd == 1 ? pick(std::integral_constant<int, NDM >= 1 ? 1 : 0>{})
                            : pick(std::integral_constant<int, NDM >= 2 ? 2 : 0>{});
        hipLaunchKernelGGL(kern, dim3((unsigned)t.gx, t.nz), dim3(64 * NW), lds, ctx->stream, t);
        GD_LAUNCHED(ctx, "q2_0_gemv_mfma");
        return GD_OK;
    }
}

}  // namespace


// GEMV on the matrix cores for f16 or f32 x (the caller has checked w, x, y).
// ksplit > 1 cuts K into that many splits whose partial rows go to y + z * R
// (the caller sums them; gd_gemv_ksplit says how many there are).  bias (if
// not null) is added to the rows of split 0.
int gd_gemv_mfma(gd_ctx *ctx, const gd_q2w *w, const void *x, int x_dtype, float *y,
                 int ksplit, const float *bias) {
    const int64_t K = w->K;
    const int XT = x_dtype == GD_F32 ? 1 : 0;
    const int nblk = (int)(K >> 7);
    const XStage xs = x_stage(nblk, XT);
    GD_REQUIRE(ctx, xs.bytes + (size_t)64 * ((nblk + 3) / 4) <= LDS_BYTES,
               "gd_q2_0_gemv: K=%lld too long for LDS staging of %s x", (long long)K,
               XT ? "f32" : "f16");
    const NormIn none{nullptr, nullptr, nullptr, 0.f, 0, 0};
    const GluOut noglu{nullptr, 0};
    return XT ? launch<1>(ctx, w, x, y, xs, none, ksplit, noglu, bias)
              : launch<0>(ctx, w, x, y, xs, none, ksplit, noglu, bias);
}

// GEMV of x = f16(o * rs * g), rs the 1/rms of o over each 128-element block
// (one value head) and g the gate (norm weight times silu(z)) (the caller
// has checked w, K % 128 == 0 and the pointers).  bias (if not null) is
// added to y.  ring (if not null): the conv ring advance of ring_n channels
// (rows ring_stride floats apart, the new row from ring_src), a side task of
// the same launch.
int gd_gemv_mfma_gated(gd_ctx *ctx, const gd_q2w *w, const float *o, const float *g, float eps,
                       float *y, const float *bias, float *ring, const float *ring_src, int ring_n,
                       int ring_stride) {
    const int nblk = (int)(w->K >> 7);
    const XStage xs = x_stage(nblk, true);
    return launch<3>(ctx, w, o, y, xs, NormIn{g, nullptr, nullptr, eps, 0, 0}, 1, GluOut{nullptr, 0},
                     bias, gemv::RingAdv{ring, ring_src, ring_n, ring_stride});
}

// K splits (1..4) for an f16-x GEMV whose partial rows the consumer can sum:
// the count that minimizes the tiles streamed by the busiest CU (the
// workgroups hold whole sets, so a short R leaves CUs idle unless K is
// split), plus a small charge per extra partial.  Returns the number of
// splits the launch will actually make.
int gd_gemv_ksplit(gd_ctx *ctx, int64_t K, int64_t R) {
    const int nblk = (int)(K >> 7), steps = (nblk + 3) / 4;
    const size_t xlds = x_stage(nblk, false).bytes;
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
    const XStage xs = x_stage(nblk, false);
    GD_REQUIRE(ctx, (nblk + 5) * 8 <= 1024, "gd_gemv_norm: K=%lld too long (at most 15744)",
               (long long)w->K);
    GD_REQUIRE(ctx, !glu_out || w->R % 32 == 0, "gd_gemv_norm: SwiGLU needs R = 2 x 16k rows");
    const GluOut glu{glu_out, glu_out ? (int)(w->R / 32) : 0};
    return launch<2>(ctx, w, h, y, xs, NormIn{delta, normw, hout, eps, delta ? nd : 0, dstride}, 1,
                     glu);
}
