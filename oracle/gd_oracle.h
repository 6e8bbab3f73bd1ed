/*
 * gd_oracle.h -- CPU restatement of the reference's Q2_0 and Gated DeltaNet
 * math, used ONLY as the checker in tests/ and as the CPU baseline leg of
 * bench.py.  It is test infrastructure, never part of the product path: the
 * library (gadeon_amd/libgadeon_hip.so) neither links nor calls it.
 *
 * Every function names the reference file:line it restates.  f32 functions
 * keep the reference's operation order; *_f64 functions are independent
 * double-precision formulations used to pin the f32 ones.
 */
#ifndef GD_ORACLE_H
#define GD_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- deterministic inputs (MetalSelfTest.swift:12-21) ---------------------- */
void or_lcg_uniform(float *out, size_t n, uint64_t seed, float lo, float hi);
void or_lcg_normal(float *out, size_t n, uint64_t seed, float mean, float sd);
void or_lcg_normal_f16(uint16_t *out, size_t n, uint64_t seed, float mean, float sd);
/* GGUF Q2_0 blocks [R][K/128]: codes uniform over {0,1,2} from stream seed,
 * scales f16(lo + (hi-lo) u) from stream seed+1. */
void or_lcg_q2_0(uint8_t *blocks, int64_t K, int64_t R, uint64_t seed, float lo, float hi);

/* ---- f16 helpers (IEEE binary16, round to nearest even) -------------------- */
float or_h2f(uint16_t h);
uint16_t or_f2h(float f);

/* ---- Q2_0 (Quant.swift) ------------------------------------------------------ */
/* Quant.swift:15-30 */
void or_q2_0_dequant(const uint8_t *blocks, size_t n, float *out);
/* Quant.swift:36-77; rows split over `threads` pthreads (concurrentPerform, :52). */
void or_q2_0_matvec(const uint8_t *w, int64_t K, int64_t M, const float *x, float *out,
                    int threads);
/* The same T times over X[T][K] -> out[T][M] (token t's result is bit-identical
 * to or_q2_0_matvec of X[t]; prefill is T mat-vecs, BonsaiEngine.swift:33-37). */
void or_q2_0_matmat(const uint8_t *w, int64_t K, int64_t M, int64_t T, const float *X,
                    float *out, int threads);
/* Independent f64 brute force: out[m] = sum_k (code-1)*d*x[k] in double. */
void or_q2_0_matvec_f64(const uint8_t *w, int64_t K, int64_t M, const double *x, double *out);

/* ---- primitives (Kernels.swift:5-84) ---------------------------------------- */
float or_silu(float x);
float or_sigmoid(float x);
float or_softplus(float x);
/* Kern.rmsnorm (Kernels.swift:15-23) */
void or_rmsnorm(const float *x, const float *w, float *y, int64_t n, float eps);
/* Kern.rmsnormRows (Kernels.swift:26-37) */
void or_rmsnorm_rows(float *x, int d, int64_t rows, const float *w, float eps);
/* Kern.l2normRows (Kernels.swift:41-52) */
void or_l2norm_rows(float *x, int d, int64_t rows, float eps);
/* Kern.softmaxInPlace (Kernels.swift:54-61) */
void or_softmax(float *x, int n);
/* Kern.ropeNeox (Kernels.swift:66-84) */
void or_rope_neox(float *x, int headDim, int nHead, int nRot, float base, int pos);

/* ---- GDN (GDN.swift) ---------------------------------------------------------- */
/* Gates, GDN.swift:39-42: beta = sigmoid(bPre), g = softplus(aPre + dt[h]) * aNeg[h]. */
void or_gdn_gate(const float *bPre, const float *aPre, const float *dt, const float *aNeg,
                 float *beta, float *g, int nV, int64_t count);
/* Causal conv + silu + ring shift for one token, GDN.swift:44-62. */
void or_gdn_conv(const float *qkvMix, float *ring, const float *cw, float *out, int convDim,
                 int dConv);
/* The delta-rule scan for one token, GDN.swift:71-109, q/k already normalized. */
void or_gdn_scan(const float *q, const float *k, const float *v, const float *g,
                 const float *beta, float *S, float *o, int nV, int nK, int dS, float qScale);
/* Same recurrence in double (independent check of the f32 order). */
void or_gdn_scan_f64(const double *q, const double *k, const double *v, const double *g,
                     const double *beta, double *S, double *o, int nV, int nK, int dS,
                     double qScale);
/* Chunked (WY/UT) form in double for one sequence of T tokens:
 * q,k [T][nK][dk], v [T][nV][dv], g,beta [T][nV], S [nV][dk][dv], o [T][nV][dv]. */
void or_gdn_chunked_f64(int64_t T, int nV, int nK, int dk, int dv, const double *q,
                        const double *k, const double *v, const double *g, const double *beta,
                        double *S, double *o, double qScale, int C);

/* ---- closed form (MtpRollback.swift:20-60) ------------------------------------ */
void or_mtp_state_after(int m, int H, int DK, int DV, int C, const float *s0, const float *delta,
                        const float *k, const float *gcum, float *out);

/* ---- threaded batch of independent decode scans (CPU baseline) ---------------- */
/* B sequences, one token each: per sequence l2norm q,k (eps) then or_gdn_scan.
 * q,k [B][nK*dS], v/o [B][nV*dS], g/beta [B][nV], S [B][nV*dS*dS]. */
void or_gdn_decode_batch(int B, int nV, int nK, int dS, float *q, float *k, const float *v,
                         const float *g, const float *beta, float *S, float *o, float qScale,
                         float eps, int threads);

/* ---- Bonsai stack: the qwen35 hybrid or the dense qwen3 lineage
 *      (BonsaiEngine.swift:134-191, GDN.swift:20-120, Attention.swift:72-139) -- */
typedef struct or_stack_layer {
    int rec;                                    /* 1 = GDN layer, 0 = attention */
    const float *attn_norm, *post_norm;
    const uint8_t *wqkv, *wgate, *wbeta, *walpha, *ssm_out;   /* GGUF Q2_0 blocks */
    const float *conv_w, *dt, *a_neg, *ssm_norm;
    const uint8_t *wq, *wk, *wv, *wo;
    const float *q_norm, *k_norm;
    const uint8_t *ffn_gate, *ffn_up, *ffn_down;
    float *conv_state, *rec_state;              /* GDN state (caller-owned, zeroed) */
    float *kcache, *vcache;                     /* [max_ctx][n_head_kv*head_dim] */
} or_stack_layer;

typedef struct or_stack {
    int n_layer, n_embd, n_ff, n_head, n_head_kv, head_dim, n_rot;
    float rope_base, eps;
    int n_vocab, d_state, n_k_head, n_v_head, d_conv, max_ctx;
    int stage_f16;     /* OR_STAGE_* bits: f16 rounding as the reference GPU path does */
    int threads;
    int dense;         /* 1: the dense qwen3 lineage (plain q, ungated attention) */
    or_stack_layer *layers;
    const uint8_t *embd;                        /* token_embd */
    const float *out_norm;
    const uint8_t *head;                        /* output.weight; NULL: tied to embd
                                                   (Model.swift:145) */
    int rope_shift;    /* rope position = position + rope_shift (MetalEngine.swift:432-435) */
} or_stack;

#define OR_STAGE_MV 1   /* mat-vec inputs (the prefill GEMM's half tiles, Kernels.metal:428) */
#define OR_STAGE_KV 2   /* cached K/V (half KV pages, Kernels.metal:1446-1457) */
#define OR_STAGE_MVO 4  /* the inputs of the output projections only (ssm_out, attn_output,
                           ffn_down): this build's decode, whose norm-fed mat-vecs read
                           their inputs at f32 precision and the others f16 */

/* BonsaiEngine.forward for one token at position pos: hidden_out[n_embd] is
 * the post-final-norm hidden; logits_out[n_vocab] may be NULL. */
void or_stack_token(or_stack *st, int token, int pos, float *hidden_out, float *logits_out);
/* T tokens at positions pos0.. with the same per-token arithmetic as T calls
 * of or_stack_token, run layer by layer; hidden/logits of the last token. */
void or_stack_prefill(or_stack *st, const int *tokens, int T, int pos0, float *hidden_out,
                      float *logits_out);

#ifdef __cplusplus
}
#endif

#endif
