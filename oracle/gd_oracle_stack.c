/*
 * gd_oracle_stack.c -- token-by-token restatement of the reference's CPU
 * engine for the hybrid stack.  TEST INFRASTRUCTURE ONLY (see gd_oracle.h).
 *
 * Follows BonsaiEngine.forward (LLM/src/SIMD/BonsaiEngine.swift:155-178),
 * GDN.step (LLM/src/SIMD/GDN.swift:20-120) and Attn.step
 * (LLM/src/SIMD/Attention.swift:72-139) in their operation order, all f32.
 * With stage_f16 set, the input of every Q2_0 mat-vec and every cached K/V
 * value is rounded to f16 first: the reference GPU path stages GEMM operands
 * as half (Kernels.metal:428) and keeps its KV pages half (MetalKVPool.swift,
 * kv_append Kernels.metal:1446-1457).
 */
#include "gd_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static void stage(const or_stack *st, const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = st->stage_f16 ? or_h2f(or_f2h(x[i])) : x[i];
}

static void matvec(const or_stack *st, const uint8_t *w, int64_t K, int64_t M, const float *x,
                   float *out) {
    float *xs = (float *)malloc(sizeof(float) * K);
    stage(st, x, xs, K);
    or_q2_0_matvec(w, K, M, xs, out, st->threads);
    free(xs);
}

/* GDN.step (GDN.swift:20-120) */
static void gdn_step(or_stack *st, or_stack_layer *L, const float *n, float *out) {
    const int dS = st->d_state, nK = st->n_k_head, nV = st->n_v_head;
    const int keyDim = dS * nK, valDim = dS * nV, convDim = 2 * keyDim + valDim;
    const int E = st->n_embd;
    float *qkv = malloc(sizeof(float) * convDim), *z = malloc(sizeof(float) * valDim);
    float *bp = malloc(sizeof(float) * nV), *ap = malloc(sizeof(float) * nV);
    float *beta = malloc(sizeof(float) * nV), *g = malloc(sizeof(float) * nV);
    float *conv = malloc(sizeof(float) * convDim), *o = malloc(sizeof(float) * valDim);
    matvec(st, L->wqkv, E, convDim, n, qkv);
    matvec(st, L->wgate, E, valDim, n, z);
    matvec(st, L->wbeta, E, nV, n, bp);
    matvec(st, L->walpha, E, nV, n, ap);
    or_gdn_gate(bp, ap, L->dt, L->a_neg, beta, g, nV, nV);
    or_gdn_conv(qkv, L->conv_state, L->conv_w, conv, convDim, st->d_conv);
    or_l2norm_rows(conv, dS, nK, st->eps);               /* q */
    or_l2norm_rows(conv + keyDim, dS, nK, st->eps);      /* k */
    const float qScale = 1 / sqrtf((float)dS);
    or_gdn_scan(conv, conv + keyDim, conv + 2 * keyDim, g, beta, L->rec_state, o, nV, nK, dS,
                qScale);
    or_rmsnorm_rows(o, dS, nV, L->ssm_norm, st->eps);
    for (int i = 0; i < valDim; i++) o[i] *= or_silu(z[i]);
    matvec(st, L->ssm_out, valDim, E, o, out);
    free(qkv); free(z); free(bp); free(ap); free(beta); free(g); free(conv); free(o);
}

/* Attn.step (Attention.swift:72-139), KV cache held contiguously by position. */
static void attn_step(or_stack *st, or_stack_layer *L, const float *n, int pos, float *out) {
    const int hd = st->head_dim, nH = st->n_head, nKV = st->n_head_kv, E = st->n_embd;
    const int group = nH / nKV, kvDim = hd * nKV;
    float *qFull = malloc(sizeof(float) * hd * 2 * nH), *q = malloc(sizeof(float) * hd * nH);
    float *gate = malloc(sizeof(float) * hd * nH);
    float *k = malloc(sizeof(float) * kvDim), *v = malloc(sizeof(float) * kvDim);
    matvec(st, L->wq, E, hd * 2 * nH, n, qFull);
    for (int h = 0; h < nH; h++)
        for (int i = 0; i < hd; i++) {
            q[h * hd + i] = qFull[h * hd * 2 + i];
            gate[h * hd + i] = qFull[h * hd * 2 + hd + i];
        }
    matvec(st, L->wk, E, kvDim, n, k);
    matvec(st, L->wv, E, kvDim, n, v);
    or_rmsnorm_rows(q, hd, nH, L->q_norm, st->eps);
    or_rmsnorm_rows(k, hd, nKV, L->k_norm, st->eps);
    or_rope_neox(q, hd, nH, st->n_rot, st->rope_base, pos);
    or_rope_neox(k, hd, nKV, st->n_rot, st->rope_base, pos);
    stage(st, k, L->kcache + (int64_t)pos * kvDim, kvDim);      /* kv.append */
    stage(st, v, L->vcache + (int64_t)pos * kvDim, kvDim);
    const int T = pos + 1;
    const float scale = 1 / sqrtf((float)hd);
    float *scores = malloc(sizeof(float) * T), *ao = calloc((size_t)hd * nH, sizeof(float));
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
    for (int i = 0; i < hd * nH; i++) ao[i] *= or_sigmoid(gate[i]);
    matvec(st, L->wo, hd * nH, E, ao, out);
    free(qFull); free(q); free(gate); free(k); free(v); free(scores); free(ao);
}

void or_stack_token(or_stack *st, int token, int pos, float *hidden_out, float *logits_out) {
    const int E = st->n_embd, FF = st->n_ff;
    const int64_t rowBytes = E / 128 * 34;
    float *x = malloc(sizeof(float) * E), *nrm = malloc(sizeof(float) * E);
    float *a = malloc(sizeof(float) * E), *gt = malloc(sizeof(float) * FF);
    float *up = malloc(sizeof(float) * FF);
    or_q2_0_dequant(st->embd + (int64_t)token * rowBytes, E, x);          /* embed */
    for (int il = 0; il < st->n_layer; il++) {
        or_stack_layer *L = &st->layers[il];
        or_rmsnorm(x, L->attn_norm, nrm, E, st->eps);
        if (L->rec) gdn_step(st, L, nrm, a);
        else attn_step(st, L, nrm, pos, a);
        for (int i = 0; i < E; i++) x[i] += a[i];
        or_rmsnorm(x, L->post_norm, nrm, E, st->eps);
        matvec(st, L->ffn_gate, E, FF, nrm, gt);                          /* ffn */
        matvec(st, L->ffn_up, E, FF, nrm, up);
        for (int i = 0; i < FF; i++) gt[i] = or_silu(gt[i]) * up[i];
        matvec(st, L->ffn_down, FF, E, gt, a);
        for (int i = 0; i < E; i++) x[i] += a[i];
    }
    or_rmsnorm(x, st->out_norm, hidden_out, E, st->eps);
    if (logits_out) matvec(st, st->embd, E, st->n_vocab, hidden_out, logits_out);
    free(x); free(nrm); free(a); free(gt); free(up);
}
