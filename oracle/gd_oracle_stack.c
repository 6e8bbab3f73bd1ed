/*
 * gd_oracle_stack.c -- token-by-token restatement of the reference's CPU
 * engine for the hybrid stack.  TEST INFRASTRUCTURE ONLY (see gd_oracle.h).
 *
 * Follows BonsaiEngine.forward (LLM/src/SIMD/BonsaiEngine.swift:155-178),
 * GDN.step (LLM/src/SIMD/GDN.swift:20-120) and Attn.step
 * (LLM/src/SIMD/Attention.swift:72-139) in their operation order, all f32.
 * stage_f16 is a bit set: OR_STAGE_MV rounds the input of every Q2_0 mat-vec
 * to f16 first, as the reference GPU's prefill GEMM stages its operands
 * (Kernels.metal:428; its decode GEMV reads f32 x, Kernels.metal:32-40, so a
 * caller leaves the bit clear for decode); OR_STAGE_KV rounds every cached
 * K/V value, as the reference's half KV pages hold them (MetalKVPool.swift,
 * kv_append Kernels.metal:1446-1457).
 *
 * or_stack_prefill runs T tokens layer by layer with the same per-token
 * arithmetic as T calls of or_stack_token: a layer's mat-vecs go through
 * or_q2_0_matmat (bit-identical per token), and the recurrent and attention
 * steps walk the tokens in order, so token t sees exactly the states tokens
 * < t left.  Only the hidden of the last token reaches the final norm and the
 * logits, which is all a prefill returns.
 */
#include "gd_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static void stage(int on, const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = on ? or_h2f(or_f2h(x[i])) : x[i];
}

/* Whether a mat-vec input is rounded to f16: every one with OR_STAGE_MV, an
 * output projection's (outp) with OR_STAGE_MVO as well. */
static int stage_mv(const or_stack *st, int outp) {
    return (st->stage_f16 & OR_STAGE_MV) || (outp && (st->stage_f16 & OR_STAGE_MVO));
}

static void matvec(const or_stack *st, const uint8_t *w, int64_t K, int64_t M, const float *x,
                   float *out, int outp) {
    float *xs = (float *)malloc(sizeof(float) * K);
    stage(stage_mv(st, outp), x, xs, K);
    or_q2_0_matvec(w, K, M, xs, out, st->threads);
    free(xs);
}

/* T mat-vecs: X [T][K] -> out [T][M]. */
static void matmat(const or_stack *st, const uint8_t *w, int64_t K, int64_t M, int64_t T,
                   const float *X, float *out, int outp) {
    float *xs = (float *)malloc(sizeof(float) * K * T);
    stage(stage_mv(st, outp), X, xs, K * T);
    or_q2_0_matmat(w, K, M, T, xs, out, st->threads);
    free(xs);
}

/* The recurrent part of GDN.step (GDN.swift:39-115) for one token, from its
 * projections qkv [convDim], z [valDim], bp, ap [nV] to the gated output o
 * [valDim] (the input of ssm_out); qkv is used as scratch. */
static void gdn_token(or_stack *st, or_stack_layer *L, float *qkv, const float *z,
                      const float *bp, const float *ap, float *o) {
    const int dS = st->d_state, nK = st->n_k_head, nV = st->n_v_head;
    const int keyDim = dS * nK, valDim = dS * nV, convDim = 2 * keyDim + valDim;
    float *beta = malloc(sizeof(float) * nV), *g = malloc(sizeof(float) * nV);
    float *conv = malloc(sizeof(float) * convDim);
    or_gdn_gate(bp, ap, L->dt, L->a_neg, beta, g, nV, nV);
    or_gdn_conv(qkv, L->conv_state, L->conv_w, conv, convDim, st->d_conv);
    or_l2norm_rows(conv, dS, nK, st->eps);               /* q */
    or_l2norm_rows(conv + keyDim, dS, nK, st->eps);      /* k */
    const float qScale = 1 / sqrtf((float)dS);
    or_gdn_scan(conv, conv + keyDim, conv + 2 * keyDim, g, beta, L->rec_state, o, nV, nK, dS,
                qScale);
    or_rmsnorm_rows(o, dS, nV, L->ssm_norm, st->eps);
    for (int i = 0; i < valDim; i++) o[i] *= or_silu(z[i]);
    free(beta); free(g); free(conv);
}

/* GDN.step (GDN.swift:20-120) over T tokens: nrm [T][E] -> out [T][E]. */
static void gdn_layer(or_stack *st, or_stack_layer *L, int T, const float *nrm, float *out) {
    const int dS = st->d_state, nK = st->n_k_head, nV = st->n_v_head;
    const int keyDim = dS * nK, valDim = dS * nV, convDim = 2 * keyDim + valDim;
    const int E = st->n_embd;
    float *qkv = malloc(sizeof(float) * convDim * T), *z = malloc(sizeof(float) * valDim * T);
    float *bp = malloc(sizeof(float) * nV * T), *ap = malloc(sizeof(float) * nV * T);
    float *o = malloc(sizeof(float) * valDim * T);
    if (T == 1) {
        matvec(st, L->wqkv, E, convDim, nrm, qkv, 0);
        matvec(st, L->wgate, E, valDim, nrm, z, 0);
        matvec(st, L->wbeta, E, nV, nrm, bp, 0);
        matvec(st, L->walpha, E, nV, nrm, ap, 0);
    } else {
        matmat(st, L->wqkv, E, convDim, T, nrm, qkv, 0);
        matmat(st, L->wgate, E, valDim, T, nrm, z, 0);
        matmat(st, L->wbeta, E, nV, T, nrm, bp, 0);
        matmat(st, L->walpha, E, nV, T, nrm, ap, 0);
    }
    for (int t = 0; t < T; t++)
        gdn_token(st, L, qkv + (int64_t)t * convDim, z + (int64_t)t * valDim, bp + (int64_t)t * nV,
                  ap + (int64_t)t * nV, o + (int64_t)t * valDim);
    if (T == 1) matvec(st, L->ssm_out, valDim, E, o, out, 1);
    else matmat(st, L->ssm_out, valDim, E, T, o, out, 1);
    free(qkv); free(z); free(bp); free(ap); free(o);
}

/* The attention part of Attn.step (Attention.swift:79-134) for one token at
 * position pos, from its projections qFull (hybrid: [2 nH hd], per head
 * q | gate; dense: [nH hd], plain q), k, v [nKV hd] to the output ao [nH hd]
 * (the input of wo), gated by sigmoid(gate) on the hybrid only
 * (Attention.swift:81-93, 132-134).  The KV cache is held contiguously by
 * position. */
static void attn_token(or_stack *st, or_stack_layer *L, const float *qFull, float *k, float *v,
                       int pos, float *ao) {
    const int hd = st->head_dim, nH = st->n_head, nKV = st->n_head_kv;
    const int group = nH / nKV, kvDim = hd * nKV, qs = st->dense ? hd : 2 * hd;
    float *q = malloc(sizeof(float) * hd * nH), *gate = malloc(sizeof(float) * hd * nH);
    for (int h = 0; h < nH; h++)
        for (int i = 0; i < hd; i++) {
            q[h * hd + i] = qFull[h * qs + i];
            gate[h * hd + i] = st->dense ? 0 : qFull[h * qs + hd + i];
        }
    or_rmsnorm_rows(q, hd, nH, L->q_norm, st->eps);
    or_rmsnorm_rows(k, hd, nKV, L->k_norm, st->eps);
    /* Rotated at position + ropeShift, cached at position (MetalEngine.swift:432-435). */
    or_rope_neox(q, hd, nH, st->n_rot, st->rope_base, pos + st->rope_shift);
    or_rope_neox(k, hd, nKV, st->n_rot, st->rope_base, pos + st->rope_shift);
    stage(st->stage_f16 & OR_STAGE_KV, k, L->kcache + (int64_t)pos * kvDim, kvDim);  /* kv.append */
    stage(st->stage_f16 & OR_STAGE_KV, v, L->vcache + (int64_t)pos * kvDim, kvDim);
    const int T = pos + 1;
    const float scale = 1 / sqrtf((float)hd);
    float *scores = malloc(sizeof(float) * T);
    for (int i = 0; i < hd * nH; i++) ao[i] = 0;
    for (int h = 0; h < nH; h++) {
        const int kvh = h / group;
        for (int t = 0; t < T; t++) {
            const float *kt = L->kcache + (int64_t)t * kvDim + kvh * hd;
            float s = 0;
            for (int i = 0; i < hd; i++) s += q[h * hd + i] * kt[i];
            scores[t] = s * scale;
        }
        or_softmax(scores, T);
        for (int t = 0; t < T; t++) {
            const float w = scores[t];
            const float *vt = L->vcache + (int64_t)t * kvDim + kvh * hd;
            for (int i = 0; i < hd; i++) ao[h * hd + i] += w * vt[i];
        }
    }
    if (!st->dense)
        for (int i = 0; i < hd * nH; i++) ao[i] *= or_sigmoid(gate[i]);
    free(q); free(gate); free(scores);
}

/* Attn.step (Attention.swift:72-139) over T tokens at positions pos0 ..:
 * nrm [T][E] -> out [T][E]. */
static void attn_layer(or_stack *st, or_stack_layer *L, int T, const float *nrm, int pos0,
                       float *out) {
    const int hd = st->head_dim, nH = st->n_head, nKV = st->n_head_kv, E = st->n_embd;
    const int kvDim = hd * nKV, qf = hd * (st->dense ? 1 : 2) * nH;
    float *qFull = malloc(sizeof(float) * qf * T), *k = malloc(sizeof(float) * kvDim * T);
    float *v = malloc(sizeof(float) * kvDim * T), *ao = malloc(sizeof(float) * hd * nH * T);
    if (T == 1) {
        matvec(st, L->wq, E, qf, nrm, qFull, 0);
        matvec(st, L->wk, E, kvDim, nrm, k, 0);
        matvec(st, L->wv, E, kvDim, nrm, v, 0);
    } else {
        matmat(st, L->wq, E, qf, T, nrm, qFull, 0);
        matmat(st, L->wk, E, kvDim, T, nrm, k, 0);
        matmat(st, L->wv, E, kvDim, T, nrm, v, 0);
    }
    for (int t = 0; t < T; t++)
        attn_token(st, L, qFull + (int64_t)t * qf, k + (int64_t)t * kvDim, v + (int64_t)t * kvDim,
                   pos0 + t, ao + (int64_t)t * hd * nH);
    if (T == 1) matvec(st, L->wo, hd * nH, E, ao, out, 1);
    else matmat(st, L->wo, hd * nH, E, T, ao, out, 1);
    free(qFull); free(k); free(v); free(ao);
}

/* BonsaiEngine.forward (BonsaiEngine.swift:155-178) for T tokens at positions
 * pos0 .. pos0+T-1, layer by layer; the last token's final hidden and logits. */
static void forward(or_stack *st, const int *tokens, int T, int pos0, float *hidden_out,
                    float *logits_out) {
    const int E = st->n_embd, FF = st->n_ff;
    const int64_t rowBytes = E / 128 * 34;
    float *x = malloc(sizeof(float) * E * T), *nrm = malloc(sizeof(float) * E * T);
    float *a = malloc(sizeof(float) * E * T), *gt = malloc(sizeof(float) * FF * T);
    float *up = malloc(sizeof(float) * FF * T);
    for (int t = 0; t < T; t++)                                             /* embed */
        or_q2_0_dequant(st->embd + (int64_t)tokens[t] * rowBytes, E, x + (int64_t)t * E);
    for (int il = 0; il < st->n_layer; il++) {
        or_stack_layer *L = &st->layers[il];
        for (int t = 0; t < T; t++)
            or_rmsnorm(x + (int64_t)t * E, L->attn_norm, nrm + (int64_t)t * E, E, st->eps);
        if (L->rec) gdn_layer(st, L, T, nrm, a);
        else attn_layer(st, L, T, nrm, pos0, a);
        for (int64_t i = 0; i < (int64_t)E * T; i++) x[i] += a[i];
        for (int t = 0; t < T; t++)
            or_rmsnorm(x + (int64_t)t * E, L->post_norm, nrm + (int64_t)t * E, E, st->eps);
        if (T == 1) {                                                       /* ffn */
            matvec(st, L->ffn_gate, E, FF, nrm, gt, 0);
            matvec(st, L->ffn_up, E, FF, nrm, up, 0);
        } else {
            matmat(st, L->ffn_gate, E, FF, T, nrm, gt, 0);
            matmat(st, L->ffn_up, E, FF, T, nrm, up, 0);
        }
        for (int64_t i = 0; i < (int64_t)FF * T; i++) gt[i] = or_silu(gt[i]) * up[i];
        if (T == 1) matvec(st, L->ffn_down, FF, E, gt, a, 1);
        else matmat(st, L->ffn_down, FF, E, T, gt, a, 1);
        for (int64_t i = 0; i < (int64_t)E * T; i++) x[i] += a[i];
    }
    or_rmsnorm(x + (int64_t)(T - 1) * E, st->out_norm, hidden_out, E, st->eps);
    if (logits_out)
        matvec(st, st->head ? st->head : st->embd, E, st->n_vocab, hidden_out, logits_out, 0);
    free(x); free(nrm); free(a); free(gt); free(up);
}

void or_stack_token(or_stack *st, int token, int pos, float *hidden_out, float *logits_out) {
    forward(st, &token, 1, pos, hidden_out, logits_out);
}

void or_stack_prefill(or_stack *st, const int *tokens, int T, int pos0, float *hidden_out,
                      float *logits_out) {
    if (T > 0) forward(st, tokens, T, pos0, hidden_out, logits_out);
}
