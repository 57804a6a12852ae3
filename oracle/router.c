/*
 * TEST INFRASTRUCTURE ONLY -- CPU oracle for the MoE routing path.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library, and only as the
 * checker; the product path (trenowanie_generatora_obrazkow_amd) never calls it.
 *
 * Plain-C restatement of:
 *   - the softmax top-k router.  The reference has no softmax top-k router (its production gate is remote HF code);
 *     the conventions follow the in-repo router restatement aurora/hf_pipeline.py:352-361 (fp32 logits from
 *     F.linear(x.float(), W.float()) at :352, top-k at :359 via topk, renormalisation w / (sum + 1e-20) * scaling
 *     at :359).  This file fixes what the reference leaves open, and the HIP kernel replicates it operation by
 *     operation so that ids, weights and logits are bit-exact:
 *       * dot product order (both routers): the row in 64-element blocks, block b feeding partial chain b % 4;
 *         each chain is a sequence of fmas from +0.0f, acc_c = fmaf(x[i], w[e][i], acc_c), its blocks in increasing
 *         order, inside block b step s (0..15) taking the elements 64b + 16q + s for q = 0..3 in that order (what
 *         chained v_mfma_f32_16x16x4_f32 steps compute when k-lane q holds the 16 consecutive elements
 *         64b + 16q .. 64b + 16q + 15); elements past d are skipped; dot = (acc_0 + acc_1) + (acc_2 + acc_3);
 *         logit = dot (+ bias[e] when a bias is given, one rounded addition);
 *       * softmax: m = max logit; ex_e = hexp(logit_e - m); denominator S uses the same lane/butterfly structure
 *         (lane l sums experts l, l+64, ...); p_e = ex_e / S (IEEE division);
 *       * selection on the logits, descending, ties to the lower expert index (softmax is monotone, so this is
 *         torch.topk's order wherever two probabilities are not rounded to the same float);
 *       * weights: w_j = p_{e_j}; renorm: s = w_0 + w_1 + ... (in j order), w_j = w_j / (s + 1e-20f) * scaling;
 *         otherwise w_j = w_j * scaling.
 *   - the sigmoid, group-limited router of BailingMoeV2 (aurora/hf_pipeline.py:352-359): its logits are those of
 *     orc_router_logits without a bias (the same order); orc_sigmoid_group_from_logits below states the
 *     orders of the selection;
 *   - hexp: exp by Cody-Waite range reduction (Cephes split ln2 = 0.693359375 - 2.12194440e-4), a degree-7 Taylor
 *     polynomial in Horner form with fmaf, and exponent scaling by ldexpf; arguments below -87 give 0, above 88
 *     infinity.  The softmax uses it for x <= 0; the sigmoid 1 / (1 + hexp(-x)) for any x.
 *   - the stable counting sort of aurora/hf_compat.py:69-72 (flat = topk_ids.reshape(-1); order =
 *     flat.argsort(stable=True); counts = bincount(flat)) and the index derivation of :78 (a_idx = order // k,
 *     y_idx = order) -- as a second, loop-based restatement next to numpy's stable argsort.
 *   - make_schedule, aurora/moe_triton.py:93-107 (BLOCK_M rows per block; grid upper bound ceil(M/BLOCK_M) + E).
 *
 * Build: gcc -O2 -ffp-contract=off -fPIC -shared router.c -lm (see oracle/build.py).  -ffp-contract=off keeps every
 * a*b+c as two rounded operations unless written as fmaf, which is what the kernel does.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static float bf16_to_f32(uint16_t v) {
    uint32_t u = (uint32_t)v << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* float -> bf16 round to nearest even, NaN -> 0x7fc0 (c10::BFloat16's rule). */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float orc_hexp(float x) {
    if (x < -87.0f) return 0.0f;
    if (x > 88.0f) return INFINITY;
    float n = rintf(x * 0x1.715476p+0f);
    float r = fmaf(-n, 0x1.63p-1f, x);
    r = fmaf(-n, -0x1.bd0106p-13f, r);
    float p = 0x1.a01a02p-13f;
    p = fmaf(p, r, 0x1.6c16c2p-10f);
    p = fmaf(p, r, 0x1.111112p-7f);
    p = fmaf(p, r, 0x1.555556p-5f);
    p = fmaf(p, r, 0x1.555556p-3f);
    p = fmaf(p, r, 0x1.0p-1f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)n);
}

/* xor butterfly over 64 lane values (offsets 32, 16, ..., 1): the softmax denominator's reduction */
static float butterfly64(float* v) {
    for (int s = 32; s >= 1; s >>= 1) {
        float nv[64];
        for (int l = 0; l < 64; ++l) nv[l] = v[l] + v[l ^ s];
        memcpy(v, nv, sizeof(nv));
    }
    return v[0];
}

/* logits (T, E) fp32 in the order described above; x rows have stride ldx (elements). */
void orc_router_logits(const uint16_t* x, int64_t ldx, const uint16_t* wr, const float* bias, int64_t T, int64_t d,
                       int E, float* logits) {
    const int64_t nb = (d + 63) / 64;
    for (int64_t t = 0; t < T; ++t) {
        const uint16_t* xr = x + t * ldx;
        for (int e = 0; e < E; ++e) {
            const uint16_t* wrow = wr + (int64_t)e * d;
            float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            for (int64_t b = 0; b < nb; ++b)
                for (int s = 0; s < 16; ++s)
                    for (int q = 0; q < 4; ++q) {
                        const int64_t i = 64 * b + 16 * q + s;
                        if (i < d) acc[b % 4] = fmaf(bf16_to_f32(xr[i]), bf16_to_f32(wrow[i]), acc[b % 4]);
                    }
            const float dot = (acc[0] + acc[1]) + (acc[2] + acc[3]);
            logits[t * E + e] = bias ? dot + bias[e] : dot;
        }
    }
}

/* softmax + top-k + (re)normalisation from given fp32 logits.  probs (T, E) optional. */
void orc_topk_from_logits(const float* logits, int64_t T, int E, int k, int renorm, float scaling, int32_t* ids,
                          float* w, float* probs) {
    float* ex = (float*)malloc(sizeof(float) * E);
    unsigned char* taken = (unsigned char*)malloc(E);
    for (int64_t t = 0; t < T; ++t) {
        const float* lg = logits + t * E;
        float m = -INFINITY;
        for (int e = 0; e < E; ++e) m = fmaxf(m, lg[e]);
        float v[64];
        for (int l = 0; l < 64; ++l) v[l] = 0.0f;
        for (int e = 0; e < E; ++e) {
            ex[e] = orc_hexp(lg[e] - m);
            v[e & 63] = v[e & 63] + ex[e];
        }
        float S = butterfly64(v);
        if (probs)
            for (int e = 0; e < E; ++e) probs[t * E + e] = ex[e] / S;
        memset(taken, 0, E);
        float sel[64];
        for (int j = 0; j < k; ++j) {
            int best = -1;
            for (int e = 0; e < E; ++e) {
                if (taken[e]) continue;
                if (best < 0 || lg[e] > lg[best]) best = e;
            }
            taken[best] = 1;
            ids[t * k + j] = best;
            sel[j] = ex[best] / S;
        }
        if (renorm) {
            float s = sel[0];
            for (int j = 1; j < k; ++j) s = s + sel[j];
            float den = s + 1e-20f;
            for (int j = 0; j < k; ++j) w[t * k + j] = sel[j] / den * scaling;
        } else {
            for (int j = 0; j < k; ++j) w[t * k + j] = sel[j] * scaling;
        }
    }
    free(ex);
    free(taken);
}

void orc_route(const uint16_t* x, int64_t ldx, const uint16_t* wr, const float* bias, int64_t T, int64_t d, int E,
               int k, int renorm, float scaling, float* logits, int32_t* ids, float* w) {
    orc_router_logits(x, ldx, wr, bias, T, d, E, logits);
    orc_topk_from_logits(logits, T, E, k, renorm, scaling, ids, w, NULL);
}

/* The sigmoid, group-limited router of BailingMoeV2 (aurora/hf_pipeline.py:352-359) from given fp32 logits (no
 * bias in them).  Follows the reference's steps, with the orders the kernel fixes:
 *   score_e = 1 / (1 + hexp(-logit_e)) (IEEE division); routing_e = score_e + bias_e (selection only, :353);
 *   groups of eg = E / n_group consecutive experts; a group's value = the sum of its two largest routing values
 *   (the largest plus the second largest with multiplicity, :354); the topk_group groups with the largest values
 *   are kept (ties to the lower group, :355); experts of the other groups are masked to -inf (:356-357);
 *   the k largest masked routing values are selected in descending order (ties to the lower expert, :357);
 *   weights: w_j = score_{e_j}; s = w_0 + w_1 + ... in j order; w_j = w_j / (s + 1e-20f) * scaling (:358-359).
 * scores (T, E) optional.  topk_group >= n_group keeps every group. */
void orc_sigmoid_group_from_logits(const float* logits, int64_t T, int E, int k, int n_group, int topk_group,
                                   const float* bias, float scaling, int32_t* ids, float* w, float* scores) {
    float* sc = (float*)malloc(sizeof(float) * E);
    float* key = (float*)malloc(sizeof(float) * E);
    unsigned char* taken = (unsigned char*)malloc(E);
    float gval[256];
    unsigned char gkeep[256];
    int eg = E / n_group;
    for (int64_t t = 0; t < T; ++t) {
        const float* lg = logits + t * E;
        for (int e = 0; e < E; ++e) {
            sc[e] = 1.0f / (1.0f + orc_hexp(-lg[e]));
            key[e] = bias ? sc[e] + bias[e] : sc[e];
            if (scores) scores[t * E + e] = sc[e];
        }
        if (topk_group < n_group) {
            for (int g = 0; g < n_group; ++g) {
                /* largest, then the largest of the rest with one instance of it removed */
                int i1 = g * eg;
                for (int e = g * eg + 1; e < (g + 1) * eg; ++e)
                    if (key[e] > key[i1]) i1 = e;
                float m2 = -INFINITY;
                for (int e = g * eg; e < (g + 1) * eg; ++e)
                    if (e != i1 && key[e] > m2) m2 = key[e];
                gval[g] = key[i1] + m2;
                gkeep[g] = 0;
            }
            for (int j = 0; j < topk_group; ++j) {
                int best = -1;
                for (int g = 0; g < n_group; ++g)
                    if (!gkeep[g] && (best < 0 || gval[g] > gval[best])) best = g;
                gkeep[best] = 1;
            }
            for (int e = 0; e < E; ++e)
                if (!gkeep[e / eg]) key[e] = -INFINITY;
        }
        memset(taken, 0, E);
        float sel[64];
        for (int j = 0; j < k; ++j) {
            int best = -1;
            for (int e = 0; e < E; ++e) {
                if (taken[e]) continue;
                if (best < 0 || key[e] > key[best]) best = e;
            }
            taken[best] = 1;
            ids[t * k + j] = best;
            sel[j] = sc[best];
        }
        float s = sel[0];
        for (int j = 1; j < k; ++j) s = s + sel[j];
        float den = s + 1e-20f;
        for (int j = 0; j < k; ++j) w[t * k + j] = sel[j] / den * scaling;
    }
    free(sc);
    free(key);
    free(taken);
}

/* Stable counting sort of the flat (token-major, slot-minor) expert ids: counts, order, a_idx, inv_pos.
 * Returns -1 if an id is out of [0, E). */
int orc_dispatch(const int64_t* ids, int64_t M, int k, int E, int64_t* counts, int64_t* order, int32_t* a_idx,
                 int32_t* inv_pos) {
    int64_t* next = (int64_t*)calloc((size_t)E, sizeof(int64_t));
    for (int e = 0; e < E; ++e) counts[e] = 0;
    for (int64_t f = 0; f < M; ++f) {
        if (ids[f] < 0 || ids[f] >= E) { free(next); return -1; }
        counts[ids[f]]++;
    }
    int64_t run = 0;
    for (int e = 0; e < E; ++e) { next[e] = run; run += counts[e]; }
    for (int64_t f = 0; f < M; ++f) {
        int64_t p = next[ids[f]]++;
        order[p] = f;
        a_idx[p] = (int32_t)(f / k);
        inv_pos[f] = (int32_t)p;
    }
    free(next);
    return 0;
}

/* make_schedule (aurora/moe_triton.py:93-107), block by block, from its definition: experts in order, each split
 * into ceil(count / block_m) blocks of block_m rows; blocks past the last get expert -1 and the clamped values of
 * the last expert (the reference's torch.where / clamp). */
void orc_make_schedule(const int64_t* counts, int E, int64_t M, int block_m, int32_t* block_e, int32_t* block_row,
                       int32_t* row_end) {
    int64_t nb = (M + block_m - 1) / block_m + E;
    int64_t b = 0, start = 0;
    int64_t last_start = 0, last_nblk_cum = 0;
    for (int e = 0; e < E; ++e) {
        int64_t nblk = (counts[e] + block_m - 1) / block_m;
        for (int64_t i = 0; i < nblk && b < nb; ++i, ++b) {
            block_e[b] = e;
            block_row[b] = (int32_t)(start + i * block_m);
            row_end[b] = (int32_t)(start + counts[e]);
        }
        last_nblk_cum += nblk;
        if (e == E - 1) last_start = start;
        start += counts[e];
    }
    int64_t last_first_block = last_nblk_cum - (E > 0 ? (counts[E - 1] + block_m - 1) / block_m : 0);
    for (; b < nb; ++b) {
        block_e[b] = -1;
        block_row[b] = (int32_t)(last_start + (b - last_first_block) * block_m);
        row_end[b] = (int32_t)(last_start + counts[E - 1]);
    }
}
