// softmax_row.h — softmax cross-entropy of one row by one wave64 (device code, shared by the
// softmax-CE kernel and the fused conv-net step).
//
// The backward follows the reference's op-by-op rules, so the gradient through the row max
// (tensor/gradient_ruleset.go:307-320, no stop-gradient in the reference) is reproduced.
#pragma once
#include <float.h>

#include "ah_common.h"

#define AH_INV_LN2 ((float)(1.0 / 0.693147180559945309417232121458176568))
#define AH_LN2 ((float)0.693147180559945309417232121458176568)

namespace ah {

// zr: the row's C logits; a: the loss scale (-1/B); dz: the row's logit gradient (written).
// Returns the row's log-probability of its label (0 for a label outside [0, C)). Every lane of the
// wave must call it.
__device__ __forceinline__ float softmax_ce_row(const float *zr, int lab, int C, float a, float *dz, int lane) {
#pragma clang fp contract(off)   // each reference op rounds on its own (no fused multiply-add)
    float m = -FLT_MAX;
    for (int c = lane; c < C; c += 64) m = fmaxf(m, zr[c]);
    m = wave_max(m);
    float tie = 0.0f, s = 0.0f;
    for (int c = lane; c < C; c += 64) {
        float v = zr[c];
        tie += (v == m) ? 1.0f : 0.0f;
        s += exp2f((v - m) * AH_INV_LN2);
    }
    tie = wave_sum(tie);
    s = wave_sum(s);
    float ls = log2f(s) * AH_LN2;
    const float rl = (lab >= 0 && lab < C) ? ((zr[lab] - m) - ls) : 0.0f;
    float gls = (lab >= 0 && lab < C) ? -a : 0.0f;       // Sum_c -(a*onehot)
    float glog2 = gls * AH_LN2;
    float gs = glog2 * (1.0f / (s * AH_LN2));
    float gm = 0.0f;
    for (int c = lane; c < C; c += 64) {
        float v = zr[c];
        float e = exp2f((v - m) * AH_INV_LN2);
        float glogp = (c == lab) ? a : 0.0f;
        float gzs = glogp + ((gs * e) * AH_LN2) * AH_INV_LN2;
        gm += -gzs;
        dz[c] = gzs;
    }
    gm = wave_sum(gm);
    float share = gm * (1.0f / tie);
    for (int c = lane; c < C; c += 64)
        if (zr[c] == m) dz[c] += share;
    return rl;
}

// softmax_ce_row with the row held in registers: VPR values per lane (C <= 64 * VPR, loaded by
// softmax_ce_row_load; columns past C hold -FLT_MAX), lane l holding columns l, l + 64, ... in order, so every per-lane sum adds the same terms in the same order as
// softmax_ce_row and each result has the same bits. Writes the row's dz and adds it to col[j] (the
// running column sums of the rows this wave handles); returns the row's log-probability of its label.
// v: the row's values as softmax_ce_row_load leaves them.
template <int VPR>
__device__ __forceinline__ void softmax_ce_row_load(const float *zr, int C, int lane, float (&v)[VPR]) {
#pragma unroll
    for (int j = 0; j < VPR; j++) {
        const int c = lane + 64 * j;
        v[j] = c < C ? zr[c] : -FLT_MAX;
    }
}
template <int VPR>
__device__ __forceinline__ float softmax_ce_row_regs(const float (&v)[VPR], const float *zr, int lab, int C, float a,
                                                     float *dz, int lane, float (&col)[VPR]) {
#pragma clang fp contract(off)
    float e[VPR];
    float m = -FLT_MAX;
#pragma unroll
    for (int j = 0; j < VPR; j++) m = fmaxf(m, v[j]);
    m = wave_max(m);
    float tie = 0.0f, s = 0.0f;
#pragma unroll
    for (int j = 0; j < VPR; j++) {
        e[j] = exp2f((v[j] - m) * AH_INV_LN2);
        if (lane + 64 * j < C) {
            tie += (v[j] == m) ? 1.0f : 0.0f;
            s += e[j];
        }
    }
    tie = wave_sum(tie);
    s = wave_sum(s);
    float ls = log2f(s) * AH_LN2;
    const float rl = (lab >= 0 && lab < C) ? ((zr[lab] - m) - ls) : 0.0f;
    float gls = (lab >= 0 && lab < C) ? -a : 0.0f;
    float glog2 = gls * AH_LN2;
    float gs = glog2 * (1.0f / (s * AH_LN2));
    float gm = 0.0f;
#pragma unroll
    for (int j = 0; j < VPR; j++) {
        const int c = lane + 64 * j;
        float glogp = (c == lab) ? a : 0.0f;
        e[j] = glogp + ((gs * e[j]) * AH_LN2) * AH_INV_LN2;   // the row's gzs
        if (c < C) gm += -e[j];
    }
    gm = wave_sum(gm);
    float share = gm * (1.0f / tie);
#pragma unroll
    for (int j = 0; j < VPR; j++) {
        const int c = lane + 64 * j;
        if (c < C) {
            float d = e[j];
            if (v[j] == m) d += share;
            dz[c] = d;
            col[j] += d;
        }
    }
    return rl;
}

}  // namespace ah
