// Gated GQA attention over an f16 paged KV cache, for head dims 128 and 256.
//
// Reference: Attn.step (LLM/src/SIMD/Attention.swift:72-139) and the Metal
// dispatches MetalEnc.splitQGate / kvAppend / attnPaged (MetalEnc.swift:
// 656-706), splitQGateBatch / ropeBatch / kvAppendBatch (:780-847) and
// attnBatch (:966-1025), driven by MetalEngine.attnLayer / attnBatchLayer
// (MetalEngine.swift:405-451, 756-796).  Per head h with kv head h / (nH/nKV):
// softmax over positions t <= pos of (q . k_t) * scale, times v_t, then times
// sigmoid(gate) when gated.  K and V are cached as f16 (half pages,
// MetalKVPool.swift), addressed through a page table: position p lives in
// page table[p / P] at slot p % P.  The reference's page table holds page
// addresses (bindless); here it holds page indices into one pool allocation,
// which is how a HIP caller would lay pages out.
//
// MI355X design:
//   * Decode (one query): flash decoding, DSPLIT key splits per head; each
//     wave takes whole keys, a lane holding HD/64 consecutive dims, with an
//     online softmax; a block merges its waves and writes (max, sum,
//     acc[HD]); a combine kernel merges the splits with the output gate.  The
//     stack's variant folds in the per-token preparation (split of q|gate,
//     RMS norm, partial NEOX rope, the cache append), so the new key never
//     round-trips through the cache within the step.
//   * Prefill (N queries): flash attention on the matrix cores, block (head,
//     64 queries); keys in blocks of 64 (32 for head dim 256) through LDS,
//     K and V as stored, V^T taken by the transposing LDS read; S^T = K Q^T
//     and O^T += V^T P^T on v_mfma_f32_16x16x32_f16 with the key order
//     inside the MFMA K dimension permuted so that P stays in registers; q
//     and P as f16 hi + lo pairs (about 22 bits), K and V the f16 cache, f32
//     accumulation.  In the stack the prefill normalizes and rotates q from
//     the projection rows itself and prep handles the kv heads only.
#include "gd_internal.h"

#include <type_traits>

namespace {

constexpr int DSPLIT = 16;      // key splits per head (decode)
constexpr int AQ = 64;          // queries per prefill block
// Keys per LDS block of the prefill: 64 for head dim 128 (each block's loads
// then have twice the arithmetic to land behind), 32 for 256 (its K and V
// tiles fill the static LDS at 32).
template <int HD> constexpr int prefill_keys() { return HD <= 128 ? 64 : 32; }

__device__ __forceinline__ int64_t kv_slot(const int32_t *pt, int pos, int block) {
    return (int64_t)pt[pos / block] * block + pos % block;
}

// cos and sin of the rotation of pair jj (< n_rot/2) at position pos
// (Kern.ropeNeox, Kernels.swift:66-84): from the table rtab[pos][jj] when it
// holds pos (rows 0 .. rtab_n - 1, formed by k_rope_table with this same
// arithmetic, so both give the same bits), else computed.
__device__ __forceinline__ float2 rope_cs(int jj, int n_rot, float base, int pos,
                                          const float2 *rtab, int rtab_n) {
    if (rtab && pos >= 0 && pos < rtab_n) return rtab[(int64_t)pos * (n_rot / 2) + jj];
    const float freq = powf(base, -2.0f * (float)jj / (float)n_rot);
    const float ang = (float)pos * freq;
    return make_float2(cosf(ang), sinf(ang));
}

// The table rope_cs reads: rows of n_rot/2 (cos, sin) pairs for positions
// 0 .. n-1.
__global__ void k_rope_table(float2 *tab, int n, int n_rot, float base) {
    const int half = n_rot / 2;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)n * half) return;
    const int jj = (int)(i % half), pos = (int)(i / half);
    const float freq = powf(base, -2.0f * (float)jj / (float)n_rot);
    const float ang = (float)pos * freq;
    tab[i] = make_float2(cosf(ang), sinf(ang));
}

// ---------------------------------------------------------------- prefill prep

// Attention prep (prefill), one wave per (token, head): q heads take their q
// (the first half of the hybrid's fused [q | gate] pair, qs = 2 HD, or the
// dense model's plain q, qs = HD), RMS-normalize it with q_norm and rotate
// it; kv heads normalize + rotate k and append k, v to the f16 cache at the
// token's position (Attention.swift:79-107).  Lane l holds dims l + 64 s.
// A block is one token and PREP_HEADS of its heads (PREP_WAVES waves, heads
// wave, wave + PREP_WAVES, ..): the rotation's cos and sin depend only on the
// token, so the block forms them once into LDS (the same powf / cosf / sinf
// per pair index as rope_cs) instead of once per head.  pos_ptr[0] is the
// first token's position (the KV slot), pos_ptr[1] the rope shift: tokens
// rotate at position + shift (MetalEngine.swift:432-435).  Heads hbeg ..
// H + HKV - 1 are done (hbeg = H: the kv heads only, for a prefill that
// prepares its q itself).
constexpr int PREP_WAVES = 4, PREP_HEADS = 12;
template <int HD>
__global__ __launch_bounds__(64 * PREP_WAVES) void k_attn_prep(
        const float *proj, int64_t stride, int qs, const float *q_norm, const float *k_norm,
        float *q_out, float *gate_out, uint16_t *kc, uint16_t *vc, const int32_t *page_table,
        const int32_t *pos_ptr, int N, int H, int HKV, int n_rot, float base, int block, float eps,
        const float2 *rtab, int rtab_n, int hbeg) {
    constexpr int S = HD / 64;
    __shared__ float rc[HD / 2], rs[HD / 2];
    const int groups = (H + HKV - hbeg + PREP_HEADS - 1) / PREP_HEADS;
    const int n = (int)(blockIdx.x / groups), g = (int)(blockIdx.x % groups);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int pos = pos_ptr[0] + n, rpos = pos + pos_ptr[1];
    const int half = n_rot / 2;
    for (int j = threadIdx.x; j < half; j += 64 * PREP_WAVES) {
        const float2 cs = rope_cs(j, n_rot, base, rpos, rtab, rtab_n);
        rc[j] = cs.x;
        rs[j] = cs.y;
    }
    __syncthreads();
    const float *row = proj + (int64_t)n * stride;
#pragma unroll
    for (int t = 0; t < PREP_HEADS / PREP_WAVES; t++) {
        const int h = hbeg + g * PREP_HEADS + wave + PREP_WAVES * t;
        if (h >= H + HKV) break;
        const bool is_q = h < H;
        const int kh = h - H;
        const float *src = is_q ? row + h * qs : row + H * qs + kh * HD;
        const float *nw = is_q ? q_norm : k_norm;
        float x[S], y[S];
        float ss = 0.f;
#pragma unroll
        for (int s = 0; s < S; s++) {
            x[s] = src[lane + 64 * s];
            ss += x[s] * x[s];
        }
        // RMS norm over the head (Kern.rmsnormRows, Kernels.swift:26-37).
        ss = gd_wave_sum(ss);
        const float sc = 1.0f / sqrtf(ss / (float)HD + eps);
#pragma unroll
        for (int s = 0; s < S; s++) y[s] = x[s] * sc * nw[lane + 64 * s];
        // Dim i pairs with i +- n_rot/2, held by another lane (or slot).
        float r[S];
#pragma unroll
        for (int k = 0; k < S; k++) {
            const int i = lane + 64 * k;
            const int ip = i < half ? i + half : i - half;          // partner dim
            float p[S];
#pragma unroll
            for (int s = 0; s < S; s++) p[s] = __shfl(y[s], ip & 63, 64);
            float pv = p[0];
#pragma unroll
            for (int s = 1; s < S; s++) pv = (ip >> 6) == s ? p[s] : pv;
            if (i < n_rot) {
                const int jj = i < half ? i : i - half;
                const float c = rc[jj], sn = rs[jj];
                r[k] = i < half ? y[k] * c - pv * sn : pv * sn + y[k] * c;
            } else {
                r[k] = y[k];
            }
        }
        if (is_q) {
            float *qo = q_out + ((int64_t)n * H + h) * HD;
            float *go = gate_out + ((int64_t)n * H + h) * HD;
#pragma unroll
            for (int s = 0; s < S; s++) {
                qo[lane + 64 * s] = r[s];
                if (qs == 2 * HD) go[lane + 64 * s] = row[h * qs + HD + lane + 64 * s];
            }
        } else {
            const int kvDim = HKV * HD;
            const int64_t slot = kv_slot(page_table, pos, block);
            const float *vs = row + H * qs + HKV * HD + kh * HD;
#pragma unroll
            for (int s = 0; s < S; s++) {
                kc[slot * kvDim + kh * HD + lane + 64 * s] = gd_f2h(r[s]);
                vc[slot * kvDim + kh * HD + lane + 64 * s] = gd_f2h(vs[lane + 64 * s]);
            }
        }
    }
}

// ---------------------------------------------------------------- prefill

// Where the prefill's queries and output gates come from: (token n, head h)
// at q + n tstride + h hstride, the gate likewise from gate.  norm null: q
// already normalized and rotated (k_attn_prep's q_out); else raw projection
// rows, normalized with norm and rotated (n_rot, base, the table rtab of
// rtab_n positions) by the prefill itself.
struct AttnQ {
    const float *q, *gate;
    int64_t tstride;
    int hstride;
    const float *norm;
    const float2 *rtab;
    int rtab_n, n_rot;
    float base, eps;
};

// Causal prefill attention with the sigmoid output gate (Attention.swift:
// 108-134), flash style on the matrix cores.  Block (head h, 64 queries):
// wave w owns queries 16w .. 16w+15; keys stream through LDS in blocks of
// AK (K and V as [key][d], V^T read by the transposing LDS read).  Per block a wave forms
// S^T = K Q^T (v_mfma_f32_16x16x32_f16, lane = one query column and four
// keys of each 16-key tile), updates its online softmax per query, and adds
// V^T P^T into O^T, 32 keys per MFMA.  The C layout of S^T is already the B
// operand of V^T P^T once the MFMA's K index 8g + e (g = lane / 16) stands
// for key 4g + e (e < 4) or 16 + 4g + e - 4 of its 32: the A operand (V^T)
// reads the same keys, so P never goes through LDS.  q and P enter as f16 hi + lo pairs (about 22
// bits), K and V are the f16 cache itself, accumulation is f32.  Queries sit
// at positions pos0 + n with pos0 = *pos_ptr (if not null) + pos_add.  With
// raw projection rows (qsrc.norm set) each lane group of a query holds all
// of its dims (lane g: 32 ks + 8 g + e), so the q RMS norm is a sum over
// the four groups and the rotation pairs (i, i + n_rot/2) lie in one lane
// when n_rot/2 is a multiple of 32 (the host checks).
template <int HD, typename OT>
__global__ __launch_bounds__(256) void k_attn_prefill(
        AttnQ qsrc, const uint16_t *kc, const uint16_t *vc,
        const int32_t *page_table, const int32_t *pos_ptr, int pos_add, OT *out, int H, int HKV,
        int N, int block, float scale, int gated) {
    constexpr int AK = prefill_keys<HD>();
    constexpr int TPK = 256 / AK;                         // staging threads per key
    constexpr int DPT = HD / TPK;                         // dims a thread stages per key
    constexpr int CH = DPT / 8;                           // 8-dim chunks a thread stages per operand
    __shared__ __attribute__((aligned(16))) f16 Ks[AK][HD + 8];
    // V rows padded by 32 bytes, so the 16 rows of a transposing read (below)
    // spread over the LDS banks (measured 1.5% faster than 16 bytes).
    __shared__ __attribute__((aligned(16))) f16 Vs[AK][HD + 16];
    // The last query blocks attend the most keys: they are dispatched first,
    // so the short ones fill the CUs behind them.
    const int h = blockIdx.x, q0 = (int)(gridDim.y - 1 - blockIdx.y) * AQ;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int lq = lane & 15, g = lane >> 4;
    const int kvh = h / (H / HKV);
    const int kvDim = HKV * HD;
    const int pos0 = (pos_ptr ? *pos_ptr : 0) + pos_add;
    const int n = q0 + 16 * w + lq;                       // this lane's query
    const bool valid = n < N;
    const int my_pos = pos0 + (valid ? n : N - 1);
    const int last = pos0 + min(q0 + AQ, N) - 1;          // last key any query here needs
    // Staging: thread t loads dims d0 .. d0 + DPT - 1 of key t / TPK of the
    // block.  The loads run ahead of the arithmetic: block k0 + AK's K and V
    // rows are requested before block k0's MFMAs, and the page-table entry
    // they need one block earlier still, so no block waits for a memory
    // round trip (blocks past `last` clamp to it: loaded, never used).
    const int sk = t / TPK, d0 = (t % TPK) * DPT;
    auto page_of = [&](int k0) { return page_table[min(k0 + sk, last) / block]; };
    u32x4 kv[2 * CH];                                     // K chunks, then V chunks
    auto fetch = [&](int k0, int page) {
        const int p = min(k0 + sk, last);
        const int64_t base = ((int64_t)page * block + p % block) * kvDim + kvh * HD + d0;
#pragma unroll
        for (int c = 0; c < CH; c++) {
            kv[c] = *(const u32x4 *)(kc + base + 8 * c);
            kv[CH + c] = *(const u32x4 *)(vc + base + 8 * c);
        }
    };
    fetch(0, page_of(0));
    int page_next = page_of(AK);
    // q after the first key block's loads, so their latencies overlap.
    // B operand of S^T: q[n][32 ks + 8 g + e] * scale, split hi + lo.
    const int64_t qoff = (int64_t)(valid ? n : N - 1) * qsrc.tstride + (int64_t)h * qsrc.hstride;
    f16x8 qh[HD / 32], ql[HD / 32];
    {
        const float *qrow = qsrc.q + qoff;
        float x[HD / 32][8];
#pragma unroll
        for (int ks = 0; ks < HD / 32; ks++) {
            const f32x4 a = *(const f32x4 *)(qrow + 32 * ks + 8 * g);
            const f32x4 b = *(const f32x4 *)(qrow + 32 * ks + 8 * g + 4);
#pragma unroll
            for (int e = 0; e < 8; e++) x[ks][e] = e < 4 ? a[e] : b[e - 4];
        }
        if (qsrc.norm) {
            // RMS norm over the head (Kern.rmsnormRows, Kernels.swift:26-37),
            // then the rotation of k_attn_prep at position + shift.
            float ss = 0.f;
#pragma unroll
            for (int ks = 0; ks < HD / 32; ks++)
#pragma unroll
                for (int e = 0; e < 8; e++) ss += x[ks][e] * x[ks][e];
            ss += __shfl_xor(ss, 16, 64);
            ss += __shfl_xor(ss, 32, 64);
            const float sc = 1.0f / sqrtf(ss / (float)HD + qsrc.eps);
#pragma unroll
            for (int ks = 0; ks < HD / 32; ks++) {
                const f32x4 na = *(const f32x4 *)(qsrc.norm + 32 * ks + 8 * g);
                const f32x4 nb = *(const f32x4 *)(qsrc.norm + 32 * ks + 8 * g + 4);
#pragma unroll
                for (int e = 0; e < 8; e++) x[ks][e] = x[ks][e] * sc * (e < 4 ? na[e] : nb[e - 4]);
            }
            const int rpos = my_pos + (pos_ptr ? pos_ptr[1] : 0);
            const int hk = qsrc.n_rot / 64;               // chunk offset of a dim's partner
#pragma unroll
            for (int ks = 0; ks < HD / 64; ks++) {
                if (ks >= hk) break;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const float2 cs = rope_cs(32 * ks + 8 * g + e, qsrc.n_rot, qsrc.base, rpos,
                                              qsrc.rtab, qsrc.rtab_n);
                    const float a = x[ks][e], b = x[ks + hk][e];
                    x[ks][e] = a * cs.x - b * cs.y;
                    x[ks + hk][e] = a * cs.y + b * cs.x;
                }
            }
        }
#pragma unroll
        for (int ks = 0; ks < HD / 32; ks++)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float v = x[ks][e] * scale;
                qh[ks][e] = (f16)v;
                ql[ks][e] = (f16)(v - (float)qh[ks][e]);
            }
    }
    f32x4 acc[HD / 16];                                   // O^T rows 16 dt + 4 g + v
#pragma unroll
    for (int dt = 0; dt < HD / 16; dt++) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.f;                         // this lane's keys only
    for (int k0 = 0; k0 <= last; k0 += AK) {
        __syncthreads();
#pragma unroll
        for (int c = 0; c < CH; c++) {
            *(u32x4 *)&Ks[sk][d0 + 8 * c] = kv[c];
            *(u32x4 *)&Vs[sk][d0 + 8 * c] = kv[CH + c];
        }
        __syncthreads();
        fetch(k0 + AK, page_next);
        page_next = page_of(k0 + 2 * AK);
        // Keep the loads here: the compiler would sink them below the MFMAs,
        // next to the LDS writes that wait for them.
        __builtin_amdgcn_sched_barrier(0);
        // S^T tiles kt: keys 16 kt + 4 g + v for query lq.
        constexpr int NKT = AK / 16;
        f32x4 sc[NKT];
#pragma unroll
        for (int kt = 0; kt < NKT; kt++) {
            sc[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < HD / 32; ks++) {
                const f16x8 ka = *(const f16x8 *)&Ks[16 * kt + lq][32 * ks + 8 * g];
                sc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qh[ks], sc[kt], 0, 0, 0);
                sc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, ql[ks], sc[kt], 0, 0, 0);
            }
        }
        // Causal mask (and the clamped duplicates past `last`), then the
        // online softmax of query lq over its lane group's keys.
        float bmax = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < NKT; kt++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int kp = k0 + 16 * kt + 4 * g + v;
                if (kp > my_pos) sc[kt][v] = -INFINITY;
                bmax = fmaxf(bmax, sc[kt][v]);
            }
        bmax = fmaxf(bmax, __shfl_xor(bmax, 16, 64));
        bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
        const float mn = fmaxf(m, bmax);                  // finite: key k0 <= my_pos
        // The softmax exponents are <= 0 (or -inf for masked keys: 0), where
        // the hardware exp2 behind __expf is accurate to a few ulp.
        const float alpha = __expf(m - mn);
        m = mn;
        l *= alpha;
#pragma unroll
        for (int dt = 0; dt < HD / 16; dt++) acc[dt] *= alpha;
        // P of key group kg (keys 32 kg ..): tiles 2 kg and 2 kg + 1.
        f16x8 ph[AK / 32], pl[AK / 32];
#pragma unroll
        for (int kt = 0; kt < NKT; kt++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const float pv = __expf(sc[kt][v] - mn);
                l += pv;
                const f16 hi = (f16)pv;
                ph[kt >> 1][4 * (kt & 1) + v] = hi;
                pl[kt >> 1][4 * (kt & 1) + v] = (f16)(pv - (float)hi);
            }
        // O^T += V^T P^T: A lane row d = 16 dt + lq, the same 8 keys of each
        // group, read from V as stored ([key][d]) by the transposing LDS
        // read: within each 16 lanes, lane l receives element l % 4 of the
        // 8 bytes that lanes l / 4 + 4k (k = 0..3) address, so lane j
        // addressing dims 16 dt + 4 (j % 4) .. of key 4 g + j / 4 (+ 16)
        // gives lane l keys 4 g + k (16 + 4 g + k) of dim 16 dt + l.
        typedef short s16x4 __attribute__((ext_vector_type(4)));
        typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
#pragma unroll
        for (int kg = 0; kg < AK / 32; kg++)
#pragma unroll
            for (int dt = 0; dt < HD / 16; dt++) {
                const f16 *vr = &Vs[32 * kg + 4 * g + (lq >> 2)][16 * dt + 4 * (lq & 3)];
                const f16x4 v0 = __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)vr));
                const f16x4 v1 = __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (lds_s16x4 *)(vr + 16 * (HD + 16))));
                const f16x8 va = f16x8{v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
                acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, ph[kg], acc[dt], 0, 0, 0);
                acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pl[kg], acc[dt], 0, 0, 0);
            }
    }
    // Total weight of query lq: the four lane groups' partial sums.
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    if (valid) {
        const float inv = 1.0f / l;
        const float *grow = qsrc.gate + (int64_t)n * qsrc.tstride + (int64_t)h * qsrc.hstride;
        OT *orow = out + ((int64_t)n * H + h) * HD;
#pragma unroll
        for (int dt = 0; dt < HD / 16; dt++) {
            const int d = 16 * dt + 4 * g;
            float o[4];
            if (gated) {
                const f32x4 gv = *(const f32x4 *)(grow + d);
#pragma unroll
                for (int v = 0; v < 4; v++) o[v] = acc[dt][v] * inv * gd_sigmoid(gv[v]);
            } else {
#pragma unroll
                for (int v = 0; v < 4; v++) o[v] = acc[dt][v] * inv;
            }
            if constexpr (sizeof(OT) == 2) {
                *(uint64_t *)(orow + d) = (uint64_t)gd_f2h(o[0]) | ((uint64_t)gd_f2h(o[1]) << 16) |
                                          ((uint64_t)gd_f2h(o[2]) << 32) | ((uint64_t)gd_f2h(o[3]) << 48);
            } else {
                *(f32x4 *)(orow + d) = f32x4{o[0], o[1], o[2], o[3]};
            }
        }
    }
}

// ---------------------------------------------------------------- decode

// Decode attention for one query token, split over keys (flash decoding):
// block (head h, split sp) of 2 HD threads (NWD = HD / 32 waves).
//   FUSED (the stack): the block prepares its own q from the projection row
//   (q of head h at h qs: the q half of a [q | gate] pair when qs = 2 HD,
//   plain q when qs = HD; RMS norm, rope; threads 0..HD-1) and the
//   new k and v (threads HD..2HD-1), rounded to f16 as the cache stores them;
//   the split that holds key pos uses them for that key instead of reading
//   the cache, and the first q head of each kv group appends them.  No block
//   reads the cache at pos.
//   Otherwise (gd_attn_paged): q arrives prepared, the T keys lo .. T-1 are
//   all cached.
// Each wave takes whole keys j = lo + NWD sp + w + STEP i with a lane holding
// HD/64 consecutive dims, keeping an online-softmax partial; the block
// merges its waves and writes (max, sum, acc[HD]) for the split; the combine
// kernel merges the splits (Attention.swift:108-134).  A wave keeps the K
// and V of its next KB keys in flight (a register ring), their page-table
// entries one round ahead of them, so a key waits for neither.
template <int HD, bool FUSED>
__global__ __launch_bounds__(2 * HD) void k_attn_decode(
        const float *src, int qs, const float *q_norm, const float *k_norm, uint16_t *kc,
        uint16_t *vc, const int32_t *page_table, const int32_t *pos_ptr, int T, int lo, float *part,
        int H, int HKV, int block, float scale, int n_rot, float base, float eps,
        const float2 *rtab, int rtab_n) {
    constexpr int NT = 2 * HD, NWD = NT / 64, DPL = HD / 64, WPH = HD / 64;
    constexpr int STEP = DSPLIT * NWD, KB = 8;
    __shared__ float wm[NWD], wl[NWD];
    __shared__ float wacc[NWD][HD];
    __shared__ float nrm[2][HD], rot[2][HD], vnew[HD], red[NWD];
    const int h = blockIdx.x, sp = blockIdx.y, t = threadIdx.x;
    const int lane = t & 63, w = __builtin_amdgcn_readfirstlane(t >> 6);
    const int kvh = h / (H / HKV), kvDim = HKV * HD;
    // Keys read from the cache: [lo, pos) for the stack (pos = the new
    // token's position, taken from its registers), [lo, T) otherwise.
    const int pos = FUSED ? *pos_ptr : T;
    const bool has_pos = FUSED && sp == (pos / NWD) % DSPLIT;   // wave pos % NWD takes key pos
    // A lane's DPL f16 dims of one key: one dword (HD 128) or two (HD 256).
    using U = typename std::conditional<DPL == 2, uint32_t, u32x2>::type;
    auto ld = [&](const uint16_t *p) { return *(const U *)p; };
    auto word = [](const U &u, int i) -> uint32_t {
        if constexpr (DPL == 2) return u;
        else return u[i];
    };
    // Cached keys of this wave: j0 + STEP i, i < nk.  Every load below is
    // unconditional (the compiler waits exactly only for straight-line
    // loads): a key past the last reads position jlast instead, whose page
    // exists (the new token's, or the last cached key's), and is not used.
    const int j0 = lo + sp * NWD + w;
    const int nk = j0 < pos ? (pos - 1 - j0) / STEP + 1 : 0;
    const int jlast = FUSED ? pos : T - 1;
    auto kpos = [&](int i) {
        const int jj = j0 + i * STEP;
        return jj < pos ? jj : jlast;
    };
    // Cache slots of keys i0 .. i0 + KB - 1, lane l holding key i0 + l % KB:
    // its page-table entry (a load) and its position in the page.
    struct Slots { int pe, off; };
    auto entries = [&](int i0) {
        const int kp = kpos(i0 + (lane & (KB - 1)));
        return Slots{page_table[kp / block], kp % block};
    };
    // K and V of key i, whose slot is in lane i % KB of sl.
    auto fetch = [&](int i, const Slots &sl, U &kk, U &vv) {
        const int l = i & (KB - 1);
        const int64_t slot = (int64_t)__builtin_amdgcn_readlane(sl.pe, l) * block +
                             __builtin_amdgcn_readlane(sl.off, l);
        const int64_t b = slot * kvDim + kvh * HD + DPL * lane;
        kk = ld(kc + b);
        vv = ld(vc + b);
    };
    // The first KB keys' slots go out first; after the q/k inputs, their K
    // and V, then the next KB keys' slots (the order of the loop below, so
    // that no loaded register is copied at its end).  Nothing the q/k work
    // waits for is requested after them: completion is in order, so it would
    // wait for the keys too.
    const Slots pg0 = entries(0);
    __builtin_amdgcn_sched_barrier(0);
    Slots pg;
    U kr[KB], vr[KB];
    auto prime = [&]() {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < KB; s++) fetch(s, pg0, kr[s], vr[s]);
        pg = entries(KB);
        __builtin_amdgcn_sched_barrier(0);
    };
    if constexpr (FUSED) {
        // q of head h (hf = 0) and k of kv head kvh (hf = 1): RMS norm over
        // the head, then the partial NEOX rope, as k_attn_prep.
        const int H2 = H * qs;
        const int hf = t / HD, i = t % HD;
        const float x = hf == 0 ? src[h * qs + i] : src[H2 + kvh * HD + i];
        const float nw = hf == 0 ? q_norm[i] : k_norm[i];
        const float vx = src[H2 + HKV * HD + kvh * HD + i];
        // The rotation at position + shift (pos_ptr[1]) from its table row
        // when the table holds it (a dummy read of src otherwise), and the
        // page entry of the new token's position, which is cached at pos.
        const int half = n_rot / 2, rpos = pos + pos_ptr[1];
        const int jj = i < half ? i : (i < n_rot ? i - half : 0);
        const bool in_tab = rtab && rpos >= 0 && rpos < rtab_n;
        const float2 tcs = in_tab ? rtab[(int64_t)rpos * half + jj] : *(const float2 *)src;
        const int pe_new = page_table[pos / block];
        prime();
        const float sq = gd_wave_sum(x * x);
        if (lane == 0) red[w] = sq;
        __syncthreads();
        float ss = 0.f;
#pragma unroll
        for (int k = 0; k < WPH; k++) ss += red[hf * WPH + k];
        const float sc = 1.0f / sqrtf(ss / (float)HD + eps);
        float y = x * sc * nw;
        nrm[hf][i] = y;
        __syncthreads();
        if (i < n_rot) {
            const float2 cs = in_tab ? tcs : rope_cs(jj, n_rot, base, rpos, nullptr, 0);
            const float mine = nrm[hf][i], pv = i < half ? nrm[hf][i + half] : nrm[hf][i - half];
            y = i < half ? mine * cs.x - pv * cs.y : pv * cs.y + mine * cs.x;
        }
        rot[hf][i] = y;
        if (hf == 1) vnew[i] = vx;
        __syncthreads();
        if (hf == 1 && has_pos && h % (H / HKV) == 0) {
            const int64_t slot = (int64_t)pe_new * block + pos % block;
            kc[slot * kvDim + kvh * HD + i] = gd_f2h(y);
            vc[slot * kvDim + kvh * HD + i] = gd_f2h(vnew[i]);
        }
    } else {
        const float qx = t < HD ? src[(int64_t)h * HD + t] : 0.f;
        prime();
        if (t < HD) rot[0][t] = qx;
        __syncthreads();
    }
    float qv[DPL], a[DPL];
#pragma unroll
    for (int e = 0; e < DPL; e++) {
        qv[e] = rot[0][DPL * lane + e] * scale;
        a[e] = 0.f;
    }
    float m = -INFINITY, l = 0.f;
    auto consume = [&](U kk, U vv) {
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < DPL; e++)
            s += qv[e] * gd_h2f((uint16_t)((word(kk, e >> 1) >> (16 * (e & 1))) & 0xffff));
        s = gd_wave_sum(s);
        const float mn = fmaxf(m, s);
        const float al = expf(m - mn), p = expf(s - mn);
        l = l * al + p;
#pragma unroll
        for (int e = 0; e < DPL; e++)
            a[e] = fmaf(p, gd_h2f((uint16_t)((word(vv, e >> 1) >> (16 * (e & 1))) & 0xffff)), a[e] * al);
        m = mn;
    };
    // Cached keys, KB a round: each slot's key, then the key a round later
    // into the slot, then the slots of the round after next.  The last round
    // requests nothing.
    int i = 0;
    for (; i + KB < nk; i += KB) {
#pragma unroll
        for (int s = 0; s < KB; s++) {
            consume(kr[s], vr[s]);
            fetch(i + KB + s, pg, kr[s], vr[s]);
        }
        pg = entries(i + 2 * KB);
    }
#pragma unroll
    for (int s = 0; s < KB; s++)
        if (i + s < nk) consume(kr[s], vr[s]);
    if constexpr (FUSED) {
        // Key pos, from this block's own copy (f16, as cached).
        if (has_pos && w == pos % NWD) {
            uint32_t kw[DPL / 2], vw[DPL / 2];
#pragma unroll
            for (int e = 0; e < DPL / 2; e++) {
                kw[e] = (uint32_t)gd_f2h(rot[1][DPL * lane + 2 * e]) |
                        ((uint32_t)gd_f2h(rot[1][DPL * lane + 2 * e + 1]) << 16);
                vw[e] = (uint32_t)gd_f2h(vnew[DPL * lane + 2 * e]) |
                        ((uint32_t)gd_f2h(vnew[DPL * lane + 2 * e + 1]) << 16);
            }
            U kk, vv;
            if constexpr (DPL == 2) { kk = kw[0]; vv = vw[0]; }
            else { kk = u32x2{kw[0], kw[1]}; vv = u32x2{vw[0], vw[1]}; }
            consume(kk, vv);
        }
    }
    if (lane == 0) { wm[w] = m; wl[w] = l; }
#pragma unroll
    for (int e = 0; e < DPL; e++) wacc[w][DPL * lane + e] = a[e];
    __syncthreads();
    if (t < HD) {
        float M = -INFINITY;
#pragma unroll
        for (int i = 0; i < NWD; i++) M = fmaxf(M, wm[i]);
        float L = 0.f, A = 0.f;
#pragma unroll
        for (int i = 0; i < NWD; i++) {
            const float f = wm[i] == -INFINITY ? 0.f : expf(wm[i] - M);
            L += wl[i] * f;
            A += wacc[i][t] * f;
        }
        float *p = part + ((int64_t)h * DSPLIT + sp) * (HD + 2);
        p[t] = A;
        if (t == 0) { p[HD] = M; p[HD + 1] = L; }
    }
}

// Merges the DSPLIT partials of head h (HD threads): out[h][d] = A / L,
// times sigmoid of the raw gate gate[h * gstride + d] when gated.
template <int HD, typename OT>
__global__ void k_attn_combine(const float *part, const float *gate, int gstride, int gated,
                               OT *out) {
    const int h = blockIdx.x, t = threadIdx.x;
    const float *p = part + (int64_t)h * DSPLIT * (HD + 2);
    float M = -INFINITY;
    for (int s = 0; s < DSPLIT; s++) M = fmaxf(M, p[s * (HD + 2) + HD]);
    float L = 0.f, A = 0.f;
    for (int s = 0; s < DSPLIT; s++) {
        const float ms = p[s * (HD + 2) + HD];
        const float f = ms == -INFINITY ? 0.f : expf(ms - M);
        L += p[s * (HD + 2) + HD + 1] * f;
        A += p[s * (HD + 2) + t] * f;
    }
    float o = A / L;
    if (gated) o *= gd_sigmoid(gate[(int64_t)h * gstride + t]);
    if constexpr (sizeof(OT) == 2) out[(int64_t)h * HD + t] = gd_f2h(o);
    else out[(int64_t)h * HD + t] = o;
}

// ---------------------------------------------------------------- glue

// qFull [N][nH][2 hd] (per head q | gate, Attention.swift:84-93) -> q, gate.
__global__ void k_split_q_gate(const float *qf, float *q, float *gate, int hd, int64_t total) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;   // over N * nH * hd
    if (i >= total) return;
    const int64_t head = i / hd, d = i % hd;
    q[i] = qf[head * 2 * hd + d];
    gate[i] = qf[head * 2 * hd + hd + d];
}

// x [N][nH][hd] f32, in place: the first n_rot dims of each head rotated
// NEOX-style at position base_pos + n (Kern.ropeNeox, Kernels.swift:66-84).
__global__ void k_rope(float *x, int hd, int nH, int n_rot, float base, int base_pos,
                       int64_t total) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;   // over N * nH * n_rot/2
    if (i >= total) return;
    const int half = n_rot / 2;
    const int j = (int)(i % half);
    const int64_t head = i / half;
    const int n = (int)(head / nH);
    float *p = x + head * hd;
    const float freq = powf(base, -2.0f * (float)j / (float)n_rot);
    const float ang = (float)(base_pos + n) * freq;
    const float c = cosf(ang), s = sinf(ang);
    const float a = p[j], b = p[j + half];
    p[j] = a * c - b * s;
    p[j + half] = a * s + b * c;
}

// k, v [N][kvDim] f32 -> the f16 cache at positions base_pos + n.
__global__ void k_kv_append(const float *k, const float *v, uint16_t *kc, uint16_t *vc,
                            const int32_t *page_table, int kv_dim, int base_pos, int block,
                            int64_t total) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;   // over N * kvDim
    if (i >= total) return;
    const int n = (int)(i / kv_dim), d = (int)(i % kv_dim);
    const int64_t slot = kv_slot(page_table, base_pos + n, block);
    kc[slot * kv_dim + d] = gd_f2h(k[i]);
    vc[slot * kv_dim + d] = gd_f2h(v[i]);
}

}  // namespace

// ---------------------------------------------------------------- launchers

int gd_attn_prep_launch(gd_ctx *ctx, int hd, const float *proj, int64_t stride, int qs,
                        const float *q_norm, const float *k_norm, float *q_out, float *gate_out,
                        uint16_t *kc, uint16_t *vc, const int32_t *page_table,
                        const int32_t *pos_ptr, int N, int H, int HKV, int n_rot, float base,
                        int block, float eps, const float *rope_tab, int rope_n, int hbeg) {
    GD_REQUIRE(ctx, n_rot >= 0 && n_rot <= hd && n_rot % 2 == 0, "attention prep: n_rot=%d", n_rot);
    GD_REQUIRE(ctx, hbeg == 0 || hbeg == H, "attention prep: first head %d", hbeg);
    const float2 *rtab = (const float2 *)rope_tab;
    const dim3 grid((unsigned)((int64_t)N * ((H + HKV - hbeg + PREP_HEADS - 1) / PREP_HEADS)));
    const dim3 blk(64 * PREP_WAVES);
    if (hd == 128)
        hipLaunchKernelGGL(k_attn_prep<128>, grid, blk, 0, ctx->stream, proj, stride, qs,
                           q_norm, k_norm, q_out, gate_out, kc, vc, page_table, pos_ptr, N, H,
                           HKV, n_rot, base, block, eps, rtab, rope_n, hbeg);
    else
        hipLaunchKernelGGL(k_attn_prep<256>, grid, blk, 0, ctx->stream, proj, stride, qs,
                           q_norm, k_norm, q_out, gate_out, kc, vc, page_table, pos_ptr, N, H,
                           HKV, n_rot, base, block, eps, rtab, rope_n, hbeg);
    GD_LAUNCHED(ctx, "k_attn_prep");
    return GD_OK;
}

int gd_attn_prefill_launch(gd_ctx *ctx, int hd, const float *q, const float *gate,
                           int64_t q_tstride, int q_hstride, const float *q_norm, int n_rot,
                           float base, float eps, const float *rope_tab, int rope_n,
                           const uint16_t *kc, const uint16_t *vc, const int32_t *page_table,
                           const int32_t *pos_ptr, int pos_add, void *out, int out_dtype, int H,
                           int HKV, int N, int block, float scale, int gated) {
    GD_REQUIRE(ctx, !q_norm || (n_rot >= 0 && n_rot <= hd && n_rot % 64 == 0 && pos_ptr),
               "attention prefill: raw q needs n_rot a multiple of 64 (n_rot=%d) and positions",
               n_rot);
    GD_REQUIRE(ctx, q_tstride % 4 == 0 && q_hstride % 4 == 0,
               "attention prefill: q strides must keep rows 16-byte aligned");
    const AttnQ qsrc{q, gate, q_tstride, q_hstride, q_norm, (const float2 *)rope_tab, rope_n, n_rot,
                     base, eps};
    const dim3 grid((unsigned)H, gd_blocks(N, AQ));
#define GD_AP(HD_, OT_) hipLaunchKernelGGL((k_attn_prefill<HD_, OT_>), grid, dim3(256), 0, \
        ctx->stream, qsrc, kc, vc, page_table, pos_ptr, pos_add, (OT_ *)out, H, HKV, N, block, \
        scale, gated)
    if (hd == 128) { if (out_dtype == GD_F16) GD_AP(128, uint16_t); else GD_AP(128, float); }
    else { if (out_dtype == GD_F16) GD_AP(256, uint16_t); else GD_AP(256, float); }
#undef GD_AP
    GD_LAUNCHED(ctx, "k_attn_prefill");
    return GD_OK;
}

// Fused decode (the stack): split + combine into f16 out.  qs = 2 hd: the
// hybrid's fused [q | gate] rows, output gated; qs = hd: plain q, ungated.
// pos_ptr[0] is the token's position, pos_ptr[1] the rope shift.
int gd_attn_decode_launch(gd_ctx *ctx, int hd, const float *proj, int qs, const float *q_norm,
                          const float *k_norm, uint16_t *kc, uint16_t *vc,
                          const int32_t *page_table, const int32_t *pos_ptr, float *part,
                          uint16_t *out, int H, int HKV, int block, float scale, int n_rot,
                          float base, float eps, const float *rope_tab, int rope_n) {
    const dim3 grid((unsigned)H, DSPLIT);
    const float2 *rtab = (const float2 *)rope_tab;
    const int gated = qs == 2 * hd;
    if (hd == 128) {
        hipLaunchKernelGGL((k_attn_decode<128, true>), grid, dim3(256), 0, ctx->stream, proj, qs,
                           q_norm, k_norm, kc, vc, page_table, pos_ptr, 0, 0, part, H, HKV, block,
                           scale, n_rot, base, eps, rtab, rope_n);
        GD_LAUNCHED(ctx, "k_attn_decode");
        hipLaunchKernelGGL((k_attn_combine<128, uint16_t>), dim3(H), dim3(128), 0, ctx->stream,
                           part, proj + 128, 2 * 128, gated, out);
    } else {
        hipLaunchKernelGGL((k_attn_decode<256, true>), grid, dim3(512), 0, ctx->stream, proj, qs,
                           q_norm, k_norm, kc, vc, page_table, pos_ptr, 0, 0, part, H, HKV, block,
                           scale, n_rot, base, eps, rtab, rope_n);
        GD_LAUNCHED(ctx, "k_attn_decode");
        hipLaunchKernelGGL((k_attn_combine<256, uint16_t>), dim3(H), dim3(256), 0, ctx->stream,
                           part, proj + 256, 2 * 256, gated, out);
    }
    GD_LAUNCHED(ctx, "k_attn_combine");
    return GD_OK;
}

size_t gd_attn_part_floats(int hd, int H) { return (size_t)H * DSPLIT * (hd + 2); }

int gd_rope_table(gd_ctx *ctx, float *tab, int n, int n_rot, float base) {
    GD_REQUIRE(ctx, tab && n > 0 && n_rot > 0 && n_rot % 2 == 0, "rope table: bad arguments");
    const int64_t total = (int64_t)n * (n_rot / 2);
    hipLaunchKernelGGL(k_rope_table, dim3(gd_blocks(total, 256)), dim3(256), 0, ctx->stream,
                       (float2 *)tab, n, n_rot, base);
    GD_LAUNCHED(ctx, "k_rope_table");
    return GD_OK;
}

// ---------------------------------------------------------------- C ABI

extern "C" int gd_split_q_gate(gd_ctx *ctx, const float *q_full, float *q, float *gate, int hd,
                               int n_head, int64_t N) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, q_full && q && gate && hd > 0 && n_head > 0 && N >= 0,
               "gd_split_q_gate: bad arguments");
    const int64_t total = N * n_head * hd;
    if (!total) return GD_OK;
    hipLaunchKernelGGL(k_split_q_gate, dim3(gd_blocks(total, 256)), dim3(256), 0, ctx->stream,
                       q_full, q, gate, hd, total);
    GD_LAUNCHED(ctx, "gd_split_q_gate");
    return GD_OK;
}

extern "C" int gd_rope(gd_ctx *ctx, float *x, int head_dim, int n_head, int n_rot, float base,
                       int base_pos, int64_t N) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, x && head_dim > 0 && n_head > 0 && N >= 0 && base_pos >= 0,
               "gd_rope: bad arguments");
    GD_REQUIRE(ctx, n_rot > 0 && n_rot % 2 == 0 && n_rot <= head_dim,
               "gd_rope: n_rot %d must be even and at most head_dim %d", n_rot, head_dim);
    const int64_t total = N * n_head * (n_rot / 2);
    if (!total) return GD_OK;
    hipLaunchKernelGGL(k_rope, dim3(gd_blocks(total, 256)), dim3(256), 0, ctx->stream, x,
                       head_dim, n_head, n_rot, base, base_pos, total);
    GD_LAUNCHED(ctx, "gd_rope");
    return GD_OK;
}

extern "C" int gd_kv_append(gd_ctx *ctx, const float *k, const float *v, uint16_t *k_cache,
                            uint16_t *v_cache, const int32_t *page_table, int kv_dim,
                            int base_pos, int page_size, int64_t N) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, k && v && k_cache && v_cache && page_table && kv_dim > 0 && page_size > 0 &&
                        base_pos >= 0 && N >= 0,
               "gd_kv_append: bad arguments");
    const int64_t total = N * kv_dim;
    if (!total) return GD_OK;
    hipLaunchKernelGGL(k_kv_append, dim3(gd_blocks(total, 256)), dim3(256), 0, ctx->stream, k, v,
                       k_cache, v_cache, page_table, kv_dim, base_pos, page_size, total);
    GD_LAUNCHED(ctx, "gd_kv_append");
    return GD_OK;
}

namespace {

int check_attn(gd_ctx *ctx, const char *fn, int hd, int n_head, int n_head_kv, int kv_dim,
               int page_size, int gated, const void *gate) {
    GD_REQUIRE(ctx, hd == 128 || hd == 256, "%s: head_dim %d (takes 128 or 256)", fn, hd);
    GD_REQUIRE(ctx, n_head > 0 && n_head_kv > 0 && n_head % n_head_kv == 0,
               "%s: n_head %d not a multiple of n_head_kv %d", fn, n_head, n_head_kv);
    GD_REQUIRE(ctx, kv_dim == hd * n_head_kv, "%s: kv_dim %d != head_dim * n_head_kv", fn, kv_dim);
    GD_REQUIRE(ctx, page_size > 0, "%s: page size %d", fn, page_size);
    GD_REQUIRE(ctx, gated == 0 || (gated == 1 && gate), "%s: gated must be 0 or 1 (with gate)", fn);
    return GD_OK;
}

}  // namespace

extern "C" int gd_attn_paged(gd_ctx *ctx, const float *q, const uint16_t *k_cache,
                             const uint16_t *v_cache, const int32_t *page_table,
                             const float *gate, float *out, float *part, int hd, int n_head,
                             int n_head_kv, int T, int kv_dim, int page_size, float scale,
                             int gated, int lo) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, q && k_cache && v_cache && page_table && out && part,
               "gd_attn_paged: null pointer");
    int rc = check_attn(ctx, "gd_attn_paged", hd, n_head, n_head_kv, kv_dim, page_size, gated, gate);
    if (rc) return rc;
    GD_REQUIRE(ctx, T > 0 && lo >= 0 && lo < T, "gd_attn_paged: keys [lo=%d, T=%d) empty", lo, T);
    const dim3 grid((unsigned)n_head, DSPLIT);
    uint16_t *kc = const_cast<uint16_t *>(k_cache), *vc = const_cast<uint16_t *>(v_cache);
    if (hd == 128) {
        hipLaunchKernelGGL((k_attn_decode<128, false>), grid, dim3(256), 0, ctx->stream, q,
                           128, nullptr, nullptr, kc, vc, page_table, nullptr, T, lo, part, n_head,
                           n_head_kv, page_size, scale, 0, 0.f, 0.f, nullptr, 0);
        GD_LAUNCHED(ctx, "gd_attn_paged");
        hipLaunchKernelGGL((k_attn_combine<128, float>), dim3(n_head), dim3(128), 0, ctx->stream,
                           part, gate, 128, gated, out);
    } else {
        hipLaunchKernelGGL((k_attn_decode<256, false>), grid, dim3(512), 0, ctx->stream, q,
                           256, nullptr, nullptr, kc, vc, page_table, nullptr, T, lo, part, n_head,
                           n_head_kv, page_size, scale, 0, 0.f, 0.f, nullptr, 0);
        GD_LAUNCHED(ctx, "gd_attn_paged");
        hipLaunchKernelGGL((k_attn_combine<256, float>), dim3(n_head), dim3(256), 0, ctx->stream,
                           part, gate, 256, gated, out);
    }
    GD_LAUNCHED(ctx, "gd_attn_paged combine");
    return GD_OK;
}

extern "C" int gd_attn_batch(gd_ctx *ctx, const float *q, const uint16_t *k_cache,
                             const uint16_t *v_cache, const int32_t *page_table,
                             const float *gate, float *out, int hd, int n_head, int n_head_kv,
                             int kv_dim, int page_size, float scale, int base_pos, int64_t N,
                             int gated, int window) {
    GD_CHECK_CTX(ctx);
    GD_REQUIRE(ctx, q && k_cache && v_cache && page_table && out, "gd_attn_batch: null pointer");
    int rc = check_attn(ctx, "gd_attn_batch", hd, n_head, n_head_kv, kv_dim, page_size, gated, gate);
    if (rc) return rc;
    GD_REQUIRE(ctx, base_pos >= 0 && N >= 0 && N < (1LL << 31), "gd_attn_batch: base_pos/N");
    GD_REQUIRE(ctx, window == 0, "gd_attn_batch: window %d (only 0, the whole history)", window);
    GD_REQUIRE(ctx, ((uintptr_t)q | (uintptr_t)out | (uintptr_t)(gated ? gate : q)) % 16 == 0,
               "gd_attn_batch: q, gate and out must be 16-byte aligned");
    if (!N) return GD_OK;
    return gd_attn_prefill_launch(ctx, hd, q, gated ? gate : q, (int64_t)n_head * hd, hd, nullptr, 0,
                                  0.f, 0.f, nullptr, 0, k_cache, v_cache, page_table, nullptr,
                                  base_pos, out, GD_F32, n_head, n_head_kv, (int)N, page_size,
                                  scale, gated);
}
