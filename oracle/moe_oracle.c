/*
 * CPU oracle for the MoE-layer hot path: router logits and router tail.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (the HIP library or the Python package) links,
 * loads or calls this file; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
 * it, as the checker.
 *
 * Router logits (the gate GEMV, reference e2e.py:57-59 calls it as self.gate(x)):
 *   logit[t,e] = sum_i x[t,i] * Wr[e,i]  (+ b[e])
 * computed in fp32 in one fixed order, the order the gfx950 router kernel uses, so that logits and
 * therefore top-k ids are bit-identical between CPU and GPU:
 *   - the d inputs are cut into chunks of 8 consecutive elements; lane l (0..63) takes chunks
 *     l, l+64, l+128, ... in increasing order and within a chunk accumulates the 8 products in
 *     element order with a fused multiply-add, starting from +0.0f;
 *   - the 64 lane partials a[0..63] are combined by a fixed tree (the DPP reduction the kernel uses):
 *     quads Q[q] = (a[4q] + a[4q+1]) + (a[4q+2] + a[4q+3]), half-rows H[h] = Q[2h] + Q[2h+1],
 *     rows R[r] = H[2r] + H[2r+1], total = (R[3] + R[2]) + (R[1] + R[0]);
 *   - the bias is added last (one fp32 addition).
 *
 * Router tail (reference moelab/router.py:15-66, semantics router.py:1-12):
 *   - NaN logits count as -inf (router.py:23);
 *   - k rounds of arg-max over the not-yet-selected ids; among equal values the LOWEST expert id
 *     wins (router.py:36-42);
 *   - with fewer than k finite logits the remaining slots take the lowest unused ids and weight 0
 *     (router.py:43-51);
 *   - norm != 0: w_r = exp(v_r - v_0) / sum_r' exp(v_r' - v_0)  (softmax over the top-k, equal to the
 *     renormalised full softmax; router.py:56-64);
 *   - norm == 0: w_r = exp(v_r - m) / sum_{finite e} exp(v_e - m), m = max logit (the full-softmax
 *     probability; router.py:29-33, 58-59);
 *   - all weights are then multiplied by `scale` (DeepSeek-V2's routed_scaling_factor,
 *     reference e2e.py:138-140; 1.0 elsewhere).
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, so no multiply-add is fused behind our back).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* logits [T, E] = x [T, d] (bf16) . Wr [E, d]^T (bf16) (+ bias [E] fp32 or NULL), order as above. */
int oracle_router_logits(const uint16_t *x, const uint16_t *wr, const float *bias, int T, int d, int E,
                         float *logits) {
    if (d % 8 != 0) return -1;
    const int nchunk = d / 8;
    for (int t = 0; t < T; ++t) {
        const uint16_t *xr = x + (size_t)t * d;
        for (int e = 0; e < E; ++e) {
            const uint16_t *wrow = wr + (size_t)e * d;
            float part[64];
            for (int l = 0; l < 64; ++l) {
                float acc = 0.0f;
                for (int c = l; c < nchunk; c += 64)
                    for (int i = 0; i < 8; ++i)
                        acc = fmaf(bf16_to_f32(xr[8 * c + i]), bf16_to_f32(wrow[8 * c + i]), acc);
                part[l] = acc;
            }
            float q[16], h[8], r[4];
            for (int i = 0; i < 16; ++i) q[i] = (part[4 * i] + part[4 * i + 1]) + (part[4 * i + 2] + part[4 * i + 3]);
            for (int i = 0; i < 8; ++i) h[i] = q[2 * i] + q[2 * i + 1];
            for (int i = 0; i < 4; ++i) r[i] = h[2 * i] + h[2 * i + 1];
            float v = (r[3] + r[2]) + (r[1] + r[0]);
            if (bias) v = v + bias[e];
            logits[(size_t)t * E + e] = v;
        }
    }
    return 0;
}

/* idx [T, k] int32, wts [T, k] fp32 from logits [T, E] fp32. */
int oracle_topk(const float *logits, int T, int E, int k, int norm, float scale, int32_t *idx, float *wts) {
    if (k < 1 || k > E) return -1;
    for (int t = 0; t < T; ++t) {
        const float *lg = logits + (size_t)t * E;
        float m0 = -INFINITY;
        for (int e = 0; e < E; ++e) {
            float v = isnan(lg[e]) ? -INFINITY : lg[e];
            if (v > m0) m0 = v;
        }
        float den = 0.0f;
        if (!norm) {
            for (int e = 0; e < E; ++e) {
                float v = isnan(lg[e]) ? -INFINITY : lg[e];
                if (v != -INFINITY) den += expf(v - m0);
            }
        }
        float topv[1024];
        int32_t topi[1024];
        for (int r = 0; r < k; ++r) {
            float best = -INFINITY;
            int bi = -1;
            for (int e = 0; e < E; ++e) {
                int used = 0;
                for (int q = 0; q < r; ++q) used |= (topi[q] == e);
                if (used) continue;
                float v = isnan(lg[e]) ? -INFINITY : lg[e];
                if (v > best) { best = v; bi = e; }    /* strict: the first (lowest) id keeps a tie */
            }
            if (bi < 0) {                               /* no finite candidate left */
                int sel = 0;
                for (int used = 1; used;) {
                    used = 0;
                    for (int q = 0; q < r; ++q) used |= (topi[q] == sel);
                    if (used) ++sel;
                }
                bi = sel;
                best = -INFINITY;
            }
            topv[r] = best;
            topi[r] = bi;
        }
        float s = 0.0f;
        for (int r = 0; r < k; ++r) s += expf(topv[r] - topv[0]);
        const float off = norm ? topv[0] : m0;
        if (!norm) s = den;
        for (int r = 0; r < k; ++r) {
            idx[(size_t)t * k + r] = topi[r];
            wts[(size_t)t * k + r] = expf(topv[r] - off) / s * scale;
        }
    }
    return 0;
}
