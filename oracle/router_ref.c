/*
 * TEST INFRASTRUCTURE ONLY -- the CPU checker for the routing half of the MoE forward.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this.
 * The product path never calls it.
 *
 * Restates, in plain C, the routing semantics of the reference:
 *   - gating logits in fp32: NativeRouter.gating -> F.linear(x.float(), W.float())
 *     (nexttransformer/scaling/megatron_moe.py:95-99; reference_blocks.py:37)
 *   - top-k on the logits, softmax over the k selected (pre_softmax=False,
 *     megatron_moe.py:43; reference_blocks.py:37-38)
 *   - expert-major, token-ascending permutation and per-expert counts:
 *     ids = mapping.T.nonzero()[:, 1]; counts = mapping.sum(0) (megatron_moe.py:142-143)
 *
 * The reference leaves the fp32 summation order to the BLAS library and the order of equal
 * logits to torch.topk. This checker fixes both, identically to the HIP router:
 *   logit(t,e) = c_0 + c_1 + ... (left to right), c_j = fmaf-chain over features
 *   [128 j, min(128 j + 128, d)) ascending from 0.0f; then + bias[e] if a bias is given.
 *   Equal logits: the lower expert index ranks first.
 * Build: gcc -O2 -ffp-contract=off -fPIC -shared (explicit fmaf keeps the FMAs fused while
 * nothing else is contracted).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define CHUNK 128

static float bf16_to_f32(uint16_t v) {
    uint32_t u = ((uint32_t)v) << 16;
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

/* logits[t*E + e]; w is the router weight in its module layout [E, d]. */
void oracle_router_logits(const uint16_t* x, int64_t ld_x, const float* w, const float* bias,
                          int64_t T, int32_t d, int32_t E, float* logits) {
    float* row = (float*)malloc(sizeof(float) * (size_t)d);
    for (int64_t t = 0; t < T; ++t) {
        for (int32_t i = 0; i < d; ++i) row[i] = bf16_to_f32(x[t * ld_x + i]);
        for (int32_t e = 0; e < E; ++e) {
            const float* we = w + (int64_t)e * d;
            float total = 0.0f;
            for (int32_t c0 = 0; c0 < d; c0 += CHUNK) {
                int32_t c1 = c0 + CHUNK < d ? c0 + CHUNK : d;
                float acc = 0.0f;
                for (int32_t i = c0; i < c1; ++i) acc = fmaf(row[i], we[i], acc);
                total = (c0 == 0) ? acc : total + acc;
            }
            if (bias) total = total + bias[e];
            logits[t * E + e] = total;
        }
    }
    free(row);
}

/* a ranks before b: larger logit, or equal logit and lower index. */
static int better(float va, int32_t ia, float vb, int32_t ib) {
    return va > vb || (va == vb && ia < ib);
}

/*
 * Top-k by logit with the tie rule, in descending order (torch.topk(sorted=True) order).
 * score_fn 0: weights = softmax over the k selected logits (reference_blocks.py:38).
 * score_fn 1: weights = sigmoid(l) / sum of the selected sigmoids.
 * Weights are computed in double and rounded to float.
 */
void oracle_topk(const float* logits, int64_t T, int32_t E, int32_t k, int32_t score_fn,
                 int32_t* ids, float* weights) {
    for (int64_t t = 0; t < T; ++t) {
        const float* l = logits + t * E;
        int32_t sel[64];
        float val[64];
        int32_t n = 0;
        for (int32_t e = 0; e < E; ++e) {
            float v = l[e];
            if (n < k) {
                int32_t p = n++;
                while (p > 0 && better(v, e, val[p - 1], sel[p - 1])) {
                    val[p] = val[p - 1];
                    sel[p] = sel[p - 1];
                    --p;
                }
                val[p] = v;
                sel[p] = e;
            } else if (better(v, e, val[k - 1], sel[k - 1])) {
                int32_t p = k - 1;
                while (p > 0 && better(v, e, val[p - 1], sel[p - 1])) {
                    val[p] = val[p - 1];
                    sel[p] = sel[p - 1];
                    --p;
                }
                val[p] = v;
                sel[p] = e;
            }
        }
        double w[64], sum = 0.0;
        for (int32_t j = 0; j < k; ++j) {
            w[j] = score_fn == 0 ? exp((double)val[j] - (double)val[0])
                                 : 1.0 / (1.0 + exp(-(double)val[j]));
            sum += w[j];
        }
        for (int32_t j = 0; j < k; ++j) {
            ids[t * k + j] = sel[j];
            weights[t * k + j] = (float)(w[j] / sum);
        }
    }
}

/*
 * Counting sort of the T*k assignments by expert, stable in token order: the order of
 * mapping.T.nonzero() (megatron_moe.py:142).
 *   counts[E], offsets[E+1], src_row[T*k] (token of each permuted row),
 *   dest[T*k] (permuted row of assignment (t, j), in the caller's slot order).
 */
void oracle_route_plan(const int32_t* ids, int64_t T, int32_t k, int32_t E, int32_t* counts,
                       int32_t* offsets, int32_t* src_row, int32_t* dest) {
    memset(counts, 0, sizeof(int32_t) * (size_t)E);
    for (int64_t a = 0; a < T * k; ++a) counts[ids[a]]++;
    offsets[0] = 0;
    for (int32_t e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + counts[e];
    int32_t* cursor = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
    memcpy(cursor, offsets, sizeof(int32_t) * (size_t)E);
    for (int64_t t = 0; t < T; ++t) {
        for (int32_t j = 0; j < k; ++j) {
            int32_t e = ids[t * k + j];
            int32_t r = cursor[e]++;
            src_row[r] = (int32_t)t;
            dest[t * k + j] = r;
        }
    }
    free(cursor);
}
