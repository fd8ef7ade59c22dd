/*
 * anneal_oracle.c — CPU restatement of georgebuilds/anneal training-step semantics.
 *
 * TEST INFRASTRUCTURE ONLY (see anneal_oracle.h). Built with -O2 -ffp-contract=off so
 * every f32 operation is rounded individually, in the order written here.
 *
 * Reference anchors used throughout (paths inside the reference tree):
 *   tensor/ops.go:56-65      Exp = exp2(x * (1/ln2)), Log = log2(x) * ln2
 *   tensor/ops.go:92-98      Div(a,b) = a * Recip(b)
 *   tensor/reduce.go:71-92   Mean = Sum * Recip(n)
 *   tensor/reduce.go:105-166 Matmul = Sum(Mul(Expand A, Expand B), axis -2)
 *   tensor/gradient.go:45-121 reverse traversal; adjoint accumulation prev.Add(g)
 *   tensor/gradient_ruleset.go:68-326 per-op rules
 *   tensor/nn/nn.go:111,154,217,328 ReLU / Linear / Conv2d / MaxPool2D graphs
 *   codegen/lower.go:654-719 serial reduce, f16 reduce widened to an f32 accumulator
 *   codegen/wgsl.go:376-386  max identity = -FLT_MAX
 */
#include "anneal_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define INV_LN2 ((float)(1.0 / 0.693147180559945309417232121458176568))
#define LN2F ((float)0.693147180559945309417232121458176568)
#define NEG_FLT_MAX (-FLT_MAX)

int ora_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

static float *falloc(size_t n) {
    float *p = (float *)calloc(n ? n : 1, sizeof(float));
    if (!p) abort();
    return p;
}

/* ── f16 codec: uop/dtype.go:392-487 ─────────────────────────────────────── */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t ora_f32_to_f16(float f) {
    uint32_t bits = f2u(f);
    uint16_t sign = (uint16_t)(bits >> 31);
    int32_t exp = (int32_t)((bits >> 23) & 0xFF) - 127;
    uint32_t frac = bits & 0x7FFFFF;
    if (exp == 128) {                      /* NaN / Inf: dtype.go:399-409 */
        if (frac != 0) {
            uint16_t m16 = (uint16_t)(frac >> 13);
            if (m16 == 0) m16 = 1;
            return (uint16_t)((sign << 15) | 0x7C00 | m16);
        }
        return (uint16_t)((sign << 15) | 0x7C00);
    }
    if (exp > 15) return (uint16_t)((sign << 15) | 0x7C00);       /* overflow */
    if (exp < -25) return (uint16_t)(sign << 15);                  /* underflow */
    if (exp < -14) {                                               /* subnormal, RTNE */
        uint32_t m = frac | 0x800000;
        uint32_t shift = (uint32_t)(-1 - exp);
        uint32_t mr = m >> (shift - 1);
        if ((mr & 1) && ((mr & 2) || (m & ((1u << (shift - 1)) - 1)))) mr += 2;
        return (uint16_t)((sign << 15) | (uint16_t)(mr >> 1));
    }
    uint32_t mr = frac >> 12;                                      /* normal, RTNE */
    if ((mr & 1) && ((mr & 2) || (frac & 0xFFF))) mr += 2;
    uint16_t m16 = (uint16_t)(mr >> 1);
    int32_t e16 = exp + 15;
    if (m16 & 0x400) { m16 &= 0x3FF; e16++; }
    if (e16 > 30) return (uint16_t)((sign << 15) | 0x7C00);
    return (uint16_t)((sign << 15) | ((uint16_t)e16 << 10) | m16);
}

float ora_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1F;
    uint32_t frac = h & 0x3FF;
    uint32_t bits;
    if (exp == 0) {
        if (frac == 0) {
            bits = sign;
        } else {
            uint32_t e32 = 127 - 14;
            while (!(frac & 0x400)) { frac <<= 1; e32--; }
            frac &= 0x3FF;
            bits = sign | (e32 << 23) | (frac << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000 | (frac << 13);
    } else {
        bits = sign | ((exp + 112) << 23) | (frac << 13);
    }
    return u2f(bits);
}

float ora_quantize_f16(float f) { return ora_f16_to_f32(ora_f32_to_f16(f)); }

void ora_f32_to_f16_array(const float *src, uint16_t *dst, int64_t n) {
    for (int64_t i = 0; i < n; i++) dst[i] = ora_f32_to_f16(src[i]);
}
void ora_f16_to_f32_array(const uint16_t *src, float *dst, int64_t n) {
    for (int64_t i = 0; i < n; i++) dst[i] = ora_f16_to_f32(src[i]);
}

/* f16 ALU op evaluated as in WGSL f16 arithmetic: exact f32 op, rounded to f16. */
static float q16(float v) { return ora_quantize_f16(v); }

/* ── Primitive compositions ──────────────────────────────────────────────── */

void ora_matmul(const float *A, const float *B, int M, int K, int N, float *C) {
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            float acc = 0.0f;
            for (int k = 0; k < K; k++) acc = acc + A[(size_t)m * K + k] * B[(size_t)k * N + n];
            C[(size_t)m * N + n] = acc;
        }
}

/* Graph of webgpu_test.go:278-458: y = Sum(x⊗W), diff = y - t, loss = Mean(diff*diff). */
void ora_linear_mse(const float *x, const float *W, const float *t, int M, int K, int N,
                    float *loss, float *gx, float *gW) {
    float *y = falloc((size_t)M * N), *gy = falloc((size_t)M * N);
    ora_matmul(x, W, M, K, N, y);
    float rn = 1.0f / (float)(M * N);          /* Recip(divisor), reduce.go:90-91 */
    float s = 0.0f;
    for (int i = 0; i < M * N; i++) { float d = y[i] - t[i]; s = s + d * d; }
    if (loss) *loss = s * rn;
    for (int i = 0; i < M * N; i++) {          /* Mul rule twice into one src, gradient_ruleset.go:137-140 */
        float d = y[i] - t[i];
        gy[i] = rn * d + rn * d;
    }
    if (gx)
        for (int m = 0; m < M; m++)
            for (int k = 0; k < K; k++) {
                float acc = 0.0f;
                for (int n = 0; n < N; n++) acc = acc + gy[m * N + n] * W[k * N + n];
                gx[m * K + k] = acc;
            }
    if (gW)
        for (int k = 0; k < K; k++)
            for (int n = 0; n < N; n++) {
                float acc = 0.0f;
                for (int m = 0; m < M; m++) acc = acc + gy[m * N + n] * x[m * K + k];
                gW[k * N + n] = acc;
            }
    free(y); free(gy);
}

void ora_exp2_sum_grad(const float *x, int n, float *loss, float *gx) {
    float s = 0.0f;
    for (int i = 0; i < n; i++) s = s + exp2f(x[i]);
    if (loss) *loss = s;
    if (gx)
        for (int i = 0; i < n; i++) gx[i] = (1.0f * exp2f(x[i])) * LN2F;   /* gradient_ruleset.go:79-82 */
}

void ora_maxpool2d(const float *x, int N, int C, int H, int W, int kH, int kW, int sH, int sW,
                   float *out, const float *adjw, float *gx) {
    int oH = (H - kH) / sH + 1, oW = (W - kW) / sW + 1;
    int overlap = !(kH <= sH && kW <= sW);
    if (gx) memset(gx, 0, sizeof(float) * (size_t)N * C * H * W);
    for (int nc = 0; nc < N * C; nc++) {
        const float *xp = x + (size_t)nc * H * W;
        for (int oh = 0; oh < oH; oh++)
            for (int ow = 0; ow < oW; ow++) {
                float m;
                if (!overlap) {
                    m = NEG_FLT_MAX;                  /* reduce identity, wgsl.go:376-386 */
                    for (int i = 0; i < kH; i++)
                        for (int j = 0; j < kW; j++) m = fmaxf(m, xp[(oh * sH + i) * W + ow * sW + j]);
                } else {                              /* binary Maximum chain, nn.go:374-386 */
                    m = xp[(oh * sH) * W + ow * sW];
                    for (int i = 0; i < kH; i++)
                        for (int j = 0; j < kW; j++)
                            if (i || j) m = fmaxf(m, xp[(oh * sH + i) * W + ow * sW + j]);
                }
                size_t oi = (size_t)nc * oH * oW + oh * oW + ow;
                if (out) out[oi] = m;
                if (!gx) continue;
                float adj = adjw ? adjw[oi] : 1.0f;
                float *gp = gx + (size_t)nc * H * W;
                if (!overlap) {                       /* tie split, gradient_ruleset.go:307-320 */
                    float tie = 0.0f;
                    for (int i = 0; i < kH; i++)
                        for (int j = 0; j < kW; j++)
                            tie = tie + (xp[(oh * sH + i) * W + ow * sW + j] == m ? 1.0f : 0.0f);
                    float share = adj * (1.0f / tie);
                    for (int i = 0; i < kH; i++)
                        for (int j = 0; j < kW; j++)
                            if (xp[(oh * sH + i) * W + ow * sW + j] == m)
                                gp[(oh * sH + i) * W + ow * sW + j] += share;
                } else {                              /* first tied position wins, gradient_ruleset.go:153-161 */
                    int done = 0;
                    for (int i = 0; i < kH && !done; i++)
                        for (int j = 0; j < kW && !done; j++)
                            if (xp[(oh * sH + i) * W + ow * sW + j] == m) {
                                gp[(oh * sH + i) * W + ow * sW + j] += adj;
                                done = 1;
                            }
                }
            }
    }
}

/*
 * Softmax cross-entropy composed from reference ops (the harness graph used by configs 1, 2, 4):
 *   m  = z.Max([1], keepdim)                 zs = z.Sub(m)
 *   e  = zs.Exp()  = Exp2(zs * f32(1/ln2))   s  = e.Sum([1], keepdim)
 *   ls = s.Log()   = Log2(s) * f32(ln2)      logp = zs.Sub(ls)
 *   loss = logp.Mul(onehot).Sum(all) * ConstScalar(f32(-1/B))
 * The backward below follows gradient_ruleset.go rule by rule, including the gradient through
 * the row max (no stop-gradient exists in the reference) with its tie split.
 */
void ora_softmax_ce(const float *z, const int32_t *labels, int B, int C, float *loss, float *dz) {
    float a = (float)(-1.0 / (double)B);
    float total = 0.0f;
    float *e = falloc((size_t)C), *gzs = falloc((size_t)C);
    for (int b = 0; b < B; b++) {
        const float *zr = z + (size_t)b * C;
        float m = NEG_FLT_MAX;
        for (int c = 0; c < C; c++) m = fmaxf(m, zr[c]);
        float tie = 0.0f, s = 0.0f;
        for (int c = 0; c < C; c++) tie = tie + (zr[c] == m ? 1.0f : 0.0f);
        for (int c = 0; c < C; c++) { e[c] = exp2f((zr[c] - m) * INV_LN2); s = s + e[c]; }
        float ls = log2f(s) * LN2F;
        for (int c = 0; c < C; c++) {
            float logp = (zr[c] - m) - ls;
            float oh = (labels[b] == c) ? 1.0f : 0.0f;
            total = total + logp * oh;
        }
        if (!dz) continue;
        /* backward */
        float gls = 0.0f;
        for (int c = 0; c < C; c++) {
            float oh = (labels[b] == c) ? 1.0f : 0.0f;
            gls = gls + (-(a * oh));                       /* Sub src1 -> Neg -> Expand-sum */
        }
        float glog2 = gls * LN2F;                          /* Mul by ln2 constant */
        float gs = glog2 * (1.0f / (s * LN2F));            /* Log2 rule: adj.Div(x*ln2) */
        float gm = 0.0f;
        for (int c = 0; c < C; c++) {
            float oh = (labels[b] == c) ? 1.0f : 0.0f;
            float glogp = a * oh;
            float gv = (gs * e[c]) * LN2F;                 /* Exp2 rule */
            float gzs2 = gv * INV_LN2;                     /* Mul by 1/ln2 constant */
            gzs[c] = glogp + gzs2;                         /* adjoint accumulation */
            gm = gm + (-gzs[c]);                           /* Sub src1 -> Neg -> Expand-sum */
        }
        float share = gm * (1.0f / tie);                   /* Max-reduce rule, tie split */
        for (int c = 0; c < C; c++)
            dz[(size_t)b * C + c] = gzs[c] + (zr[c] == m ? share : 0.0f);
    }
    if (loss) *loss = total * a;
    free(e); free(gzs);
}

/* ── Linear-layer helpers (f32) ──────────────────────────────────────────── */

/* Z[M,N] = Sum_k X[M,K] W[N,K] + b[N]  (Linear.Forward nn.go:154-162: x.Matmul(W.Permute) + bias) */
static void lin_fwd(const float *X, const float *W, const float *b, int M, int N, int K, float *Z) {
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            float acc = 0.0f;
            const float *xr = X + (size_t)m * K, *wr = W + (size_t)n * K;
            for (int k = 0; k < K; k++) acc = acc + xr[k] * wr[k];
            Z[(size_t)m * N + n] = b ? acc + b[n] : acc;
        }
}
/* dW[N,K] = Sum_m G[m,n] X[m,k]   (Expand rule over the batch axis, gradient_ruleset.go:207-233) */
static void lin_dw(const float *G, const float *X, int M, int N, int K, float *dW) {
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++)
        for (int k = 0; k < K; k++) {
            float acc = 0.0f;
            for (int m = 0; m < M; m++) acc = acc + G[(size_t)m * N + n] * X[(size_t)m * K + k];
            dW[(size_t)n * K + k] = acc;
        }
}
/* dX[M,K] = Sum_n G[m,n] W[n,k] */
static void lin_dx(const float *G, const float *W, int M, int N, int K, float *dX) {
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; m++)
        for (int k = 0; k < K; k++) {
            float acc = 0.0f;
            for (int n = 0; n < N; n++) acc = acc + G[(size_t)m * N + n] * W[(size_t)n * K + k];
            dX[(size_t)m * K + k] = acc;
        }
}
static void colsum(const float *G, int M, int N, float *db) {
    for (int n = 0; n < N; n++) {
        float acc = 0.0f;
        for (int m = 0; m < M; m++) acc = acc + G[(size_t)m * N + n];
        db[n] = acc;
    }
}
/* SGD on the f32 master value, nn.go:69-76 */
static void sgd(float *p, const float *g, size_t n, float lr) {
    for (size_t i = 0; i < n; i++) p[i] = p[i] - lr * g[i];
}

/* ── Config 1 / 4: two-layer MLP with softmax-CE ─────────────────────────── */

void ora_mlp_ce_step(const float *x, const int32_t *labels, int B, int D, int Hd, int C,
                     float *W1, float *b1, float *W2, float *b2, float lr,
                     float *loss, float *dW1o, float *db1o, float *dW2o, float *db2o) {
    float *Z1 = falloc((size_t)B * Hd), *H1 = falloc((size_t)B * Hd), *Z2 = falloc((size_t)B * C);
    float *dZ2 = falloc((size_t)B * C), *dH1 = falloc((size_t)B * Hd);
    float *dW1 = falloc((size_t)Hd * D), *db1 = falloc(Hd), *dW2 = falloc((size_t)C * Hd), *db2 = falloc(C);
    lin_fwd(x, W1, b1, B, Hd, D, Z1);
    for (size_t i = 0; i < (size_t)B * Hd; i++) H1[i] = fmaxf(Z1[i], 0.0f);
    lin_fwd(H1, W2, b2, B, C, Hd, Z2);
    ora_softmax_ce(Z2, labels, B, C, loss, dZ2);
    colsum(dZ2, B, C, db2);
    lin_dw(dZ2, H1, B, C, Hd, dW2);
    lin_dx(dZ2, W2, B, C, Hd, dH1);
    for (size_t i = 0; i < (size_t)B * Hd; i++) dH1[i] = (Z1[i] == H1[i]) ? dH1[i] : 0.0f;  /* Max rule */
    colsum(dH1, B, Hd, db1);
    lin_dw(dH1, x, B, Hd, D, dW1);
    if (dW1o) memcpy(dW1o, dW1, sizeof(float) * (size_t)Hd * D);
    if (db1o) memcpy(db1o, db1, sizeof(float) * Hd);
    if (dW2o) memcpy(dW2o, dW2, sizeof(float) * (size_t)C * Hd);
    if (db2o) memcpy(db2o, db2, sizeof(float) * C);
    sgd(W1, dW1, (size_t)Hd * D, lr); sgd(b1, db1, Hd, lr);
    sgd(W2, dW2, (size_t)C * Hd, lr); sgd(b2, db2, C, lr);
    free(Z1); free(H1); free(Z2); free(dZ2); free(dH1); free(dW1); free(db1); free(dW2); free(db2);
}

/* ── Config 2: conv net ──────────────────────────────────────────────────── */

/* Conv2d 3x3, stride 1, pad 1 (nn.go:217-303): out[n,co,h,w] = Sum_k im2col[n,hw,k] Wflat[co,k] + b[co],
 * k = ci*9 + kh*3 + kw accumulated in order. */
static void conv_fwd(const float *x, int N, int Ci, int H, const float *w, const float *b, int Co, float *out) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int n = 0; n < N; n++)
        for (int co = 0; co < Co; co++)
            for (int h = 0; h < H; h++)
                for (int wv = 0; wv < H; wv++) {
                    float acc = 0.0f;
                    for (int ci = 0; ci < Ci; ci++)
                        for (int kh = 0; kh < 3; kh++)
                            for (int kw = 0; kw < 3; kw++) {
                                int y = h + kh - 1, xx = wv + kw - 1;
                                float v = (y >= 0 && y < H && xx >= 0 && xx < H)
                                              ? x[(((size_t)n * Ci + ci) * H + y) * H + xx] : 0.0f;
                                acc = acc + v * w[((size_t)co * Ci + ci) * 9 + kh * 3 + kw];
                            }
                    out[(((size_t)n * Co + co) * H + h) * H + wv] = acc + b[co];
                }
}
/* dW[co,k] = Sum_{n,hw} g[n,co,hw] * im2col[n,hw,k]; db[co] = Sum_{n,h,w} g */
static void conv_bwd_w(const float *x, const float *g, int N, int Ci, int H, int Co, float *dw, float *db) {
#pragma omp parallel for schedule(static)
    for (int co = 0; co < Co; co++) {
        for (int ci = 0; ci < Ci; ci++)
            for (int kh = 0; kh < 3; kh++)
                for (int kw = 0; kw < 3; kw++) {
                    float acc = 0.0f;
                    for (int n = 0; n < N; n++)
                        for (int h = 0; h < H; h++)
                            for (int wv = 0; wv < H; wv++) {
                                int y = h + kh - 1, xx = wv + kw - 1;
                                float v = (y >= 0 && y < H && xx >= 0 && xx < H)
                                              ? x[(((size_t)n * Ci + ci) * H + y) * H + xx] : 0.0f;
                                acc = acc + g[(((size_t)n * Co + co) * H + h) * H + wv] * v;
                            }
                    dw[((size_t)co * Ci + ci) * 9 + kh * 3 + kw] = acc;
                }
        float acc = 0.0f;
        for (int n = 0; n < N; n++)
            for (int i = 0; i < H * H; i++) acc = acc + g[((size_t)n * Co + co) * H * H + i];
        db[co] = acc;
    }
}
/* dx via col2im: gim[n,hw,k] = Sum_co g[n,co,hw] Wflat[co,k]; dx accumulates the K shifted columns in k order. */
static void conv_bwd_x(const float *g, const float *w, int N, int Ci, int H, int Co, float *dx) {
    memset(dx, 0, sizeof(float) * (size_t)N * Ci * H * H);
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++)
        for (int ci = 0; ci < Ci; ci++)
            for (int kh = 0; kh < 3; kh++)
                for (int kw = 0; kw < 3; kw++)
                    for (int h = 0; h < H; h++)
                        for (int wv = 0; wv < H; wv++) {
                            int y = h + kh - 1, xx = wv + kw - 1;
                            if (y < 0 || y >= H || xx < 0 || xx >= H) continue;
                            float acc = 0.0f;
                            for (int co = 0; co < Co; co++)
                                acc = acc + g[(((size_t)n * Co + co) * H + h) * H + wv] *
                                                w[((size_t)co * Ci + ci) * 9 + kh * 3 + kw];
                            dx[(((size_t)n * Ci + ci) * H + y) * H + xx] += acc;
                        }
}

void ora_convnet_step(const float *x, const int32_t *labels, int N, int Hin, int C1, int C2, int NC,
                      float *cw1, float *cb1, float *cw2, float *cb2, float *fw, float *fb, float lr,
                      float *loss, float *dcw1o, float *dcb1o, float *dcw2o, float *dcb2o,
                      float *dfwo, float *dfbo) {
    int H1 = Hin, P1 = Hin / 2, P2 = Hin / 4, F = C2 * P2 * P2;
    size_t nz1 = (size_t)N * C1 * H1 * H1, np1 = (size_t)N * C1 * P1 * P1;
    size_t nz2 = (size_t)N * C2 * P1 * P1, np2 = (size_t)N * C2 * P2 * P2;
    float *z1 = falloc(nz1), *h1 = falloc(nz1), *p1 = falloc(np1);
    float *z2 = falloc(nz2), *h2 = falloc(nz2), *p2 = falloc(np2), *lg = falloc((size_t)N * NC);
    float *dlg = falloc((size_t)N * NC), *dp2 = falloc(np2), *dh2 = falloc(nz2), *dp1 = falloc(np1),
          *dh1 = falloc(nz1);
    float *dcw1 = falloc((size_t)C1 * 9), *dcb1 = falloc(C1), *dcw2 = falloc((size_t)C2 * C1 * 9),
          *dcb2 = falloc(C2), *dfw = falloc((size_t)NC * F), *dfb = falloc(NC);

    conv_fwd(x, N, 1, H1, cw1, cb1, C1, z1);
    for (size_t i = 0; i < nz1; i++) h1[i] = fmaxf(z1[i], 0.0f);
    ora_maxpool2d(h1, N, C1, H1, H1, 2, 2, 2, 2, p1, NULL, NULL);
    conv_fwd(p1, N, C1, P1, cw2, cb2, C2, z2);
    for (size_t i = 0; i < nz2; i++) h2[i] = fmaxf(z2[i], 0.0f);
    ora_maxpool2d(h2, N, C2, P1, P1, 2, 2, 2, 2, p2, NULL, NULL);
    lin_fwd(p2, fw, fb, N, NC, F, lg);                 /* p2 reshaped [N, C2*P2*P2] */
    ora_softmax_ce(lg, labels, N, NC, loss, dlg);

    colsum(dlg, N, NC, dfb);
    lin_dw(dlg, p2, N, NC, F, dfw);
    lin_dx(dlg, fw, N, NC, F, dp2);
    ora_maxpool2d(h2, N, C2, P1, P1, 2, 2, 2, 2, NULL, dp2, dh2);
    for (size_t i = 0; i < nz2; i++) dh2[i] = (z2[i] == h2[i]) ? dh2[i] : 0.0f;
    conv_bwd_w(p1, dh2, N, C1, P1, C2, dcw2, dcb2);
    conv_bwd_x(dh2, cw2, N, C1, P1, C2, dp1);
    ora_maxpool2d(h1, N, C1, H1, H1, 2, 2, 2, 2, NULL, dp1, dh1);
    for (size_t i = 0; i < nz1; i++) dh1[i] = (z1[i] == h1[i]) ? dh1[i] : 0.0f;
    conv_bwd_w(x, dh1, N, 1, H1, C1, dcw1, dcb1);

    if (dcw1o) memcpy(dcw1o, dcw1, sizeof(float) * C1 * 9);
    if (dcb1o) memcpy(dcb1o, dcb1, sizeof(float) * C1);
    if (dcw2o) memcpy(dcw2o, dcw2, sizeof(float) * C2 * C1 * 9);
    if (dcb2o) memcpy(dcb2o, dcb2, sizeof(float) * C2);
    if (dfwo) memcpy(dfwo, dfw, sizeof(float) * (size_t)NC * F);
    if (dfbo) memcpy(dfbo, dfb, sizeof(float) * NC);
    sgd(cw1, dcw1, (size_t)C1 * 9, lr); sgd(cb1, dcb1, C1, lr);
    sgd(cw2, dcw2, (size_t)C2 * C1 * 9, lr); sgd(cb2, dcb2, C2, lr);
    sgd(fw, dfw, (size_t)NC * F, lr); sgd(fb, dfb, NC, lr);
    free(z1); free(h1); free(p1); free(z2); free(h2); free(p2); free(lg); free(dlg); free(dp2);
    free(dh2); free(dp1); free(dh1); free(dcw1); free(dcb1); free(dcw2); free(dcb2); free(dfw); free(dfb);
}

/* ── Config 3: f16 three-layer MLP ───────────────────────────────────────── */

/* Z = f16(f16(acc) + b): the matmul is an f16 ReduceAxis whose loads are widened to f32
 * (lower.go:640-645, exact products), narrowed with f16(acc) (lower.go:712), then the f16
 * bias Add rounds again. */
static void lin_fwd_f16(const float *X, const float *W, const float *b, int M, int N, int K, float *Z) {
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            float acc = 0.0f;
            const float *xr = X + (size_t)m * K, *wr = W + (size_t)n * K;
            for (int k = 0; k < K; k++) acc = acc + xr[k] * wr[k];
            Z[(size_t)m * N + n] = q16(q16(acc) + b[n]);
        }
}

void ora_mlp3_f16_step(const float *x, const float *t, int B, int D0, int D1, int D2, int D3,
                       float *W1, float *b1, float *W2, float *b2, float *W3, float *b3, float lr,
                       float *loss, float *dW1o, float *db1o, float *dW2o, float *db2o, float *dW3o,
                       float *db3o) {
    size_t n1 = (size_t)D1 * D0, n2 = (size_t)D2 * D1, n3 = (size_t)D3 * D2;
    /* Parameter.Load quantizes the f32 master to the f16 leaf (nn.go:56-61, tensor.go:58-68) */
    float *w1 = falloc(n1), *w2 = falloc(n2), *w3 = falloc(n3), *c1 = falloc(D1), *c2 = falloc(D2), *c3 = falloc(D3);
    for (size_t i = 0; i < n1; i++) w1[i] = q16(W1[i]);
    for (size_t i = 0; i < n2; i++) w2[i] = q16(W2[i]);
    for (size_t i = 0; i < n3; i++) w3[i] = q16(W3[i]);
    for (int i = 0; i < D1; i++) c1[i] = q16(b1[i]);
    for (int i = 0; i < D2; i++) c2[i] = q16(b2[i]);
    for (int i = 0; i < D3; i++) c3[i] = q16(b3[i]);
    float *Z1 = falloc((size_t)B * D1), *H1 = falloc((size_t)B * D1);
    float *Z2 = falloc((size_t)B * D2), *H2 = falloc((size_t)B * D2), *P = falloc((size_t)B * D3);
    lin_fwd_f16(x, w1, c1, B, D1, D0, Z1);
    for (size_t i = 0; i < (size_t)B * D1; i++) H1[i] = fmaxf(Z1[i], 0.0f);
    lin_fwd_f16(H1, w2, c2, B, D2, D1, Z2);
    for (size_t i = 0; i < (size_t)B * D2; i++) H2[i] = fmaxf(Z2[i], 0.0f);
    lin_fwd_f16(H2, w3, c3, B, D3, D2, P);

    /* loss = Sum(d*d) * f32(1/(B*D3)): f16 reduce, body widened to f32 (lower.go:640-716),
     * narrowed f16(acc) — overflows to +Inf for large sums, as the reference does. */
    float scale = (float)(1.0 / ((double)B * (double)D3));
    float acc = 0.0f;
    for (size_t i = 0; i < (size_t)B * D3; i++) { float d = P[i] - t[i]; acc = acc + d * d; }
    if (loss) *loss = q16(acc) * scale;

    /* dP = (scale*d) + (scale*d), d = f16 Sub (outside any f16 reduce) */
    float *gP = falloc((size_t)B * D3);
    for (size_t i = 0; i < (size_t)B * D3; i++) {
        float d = q16(P[i] - t[i]);
        gP[i] = scale * d + scale * d;
    }
    float *dW3 = falloc(n3), *db3 = falloc(D3), *dH2 = falloc((size_t)B * D2);
    float *dW2 = falloc(n2), *db2 = falloc(D2), *dH1 = falloc((size_t)B * D1);
    float *dW1 = falloc(n1), *db1 = falloc(D1);
    colsum(gP, B, D3, db3);
    lin_dw(gP, H2, B, D3, D2, dW3);
    lin_dx(gP, w3, B, D3, D2, dH2);
    for (size_t i = 0; i < (size_t)B * D2; i++) dH2[i] = (Z2[i] == H2[i]) ? dH2[i] : 0.0f;
    colsum(dH2, B, D2, db2);
    lin_dw(dH2, H1, B, D2, D1, dW2);
    lin_dx(dH2, w2, B, D2, D1, dH1);
    for (size_t i = 0; i < (size_t)B * D1; i++) dH1[i] = (Z1[i] == H1[i]) ? dH1[i] : 0.0f;
    colsum(dH1, B, D1, db1);
    lin_dw(dH1, x, B, D1, D0, dW1);
    if (dW1o) memcpy(dW1o, dW1, sizeof(float) * n1);
    if (db1o) memcpy(db1o, db1, sizeof(float) * D1);
    if (dW2o) memcpy(dW2o, dW2, sizeof(float) * n2);
    if (db2o) memcpy(db2o, db2, sizeof(float) * D2);
    if (dW3o) memcpy(dW3o, dW3, sizeof(float) * n3);
    if (db3o) memcpy(db3o, db3, sizeof(float) * D3);
    sgd(W1, dW1, n1, lr); sgd(b1, db1, D1, lr);
    sgd(W2, dW2, n2, lr); sgd(b2, db2, D2, lr);
    sgd(W3, dW3, n3, lr); sgd(b3, db3, D3, lr);
    free(w1); free(w2); free(w3); free(c1); free(c2); free(c3); free(Z1); free(H1); free(Z2); free(H2);
    free(P); free(gP); free(dW3); free(db3); free(dH2); free(dW2); free(db2); free(dH1); free(dW1); free(db1);
}

/* ── Config 5: movement + row-reduce chain ───────────────────────────────── */

void ora_chain_step(const float *X, const float *g, int R, int Cc, float *loss, float *dX, float *dg) {
    const float eps = 1e-6f;
    const float rR = 1.0f / (float)R;            /* Mean: Sum * Recip(R) */
    double dummy = 0; (void)dummy;
    float *rowloss = falloc(Cc);
#pragma omp parallel
    {
        float *y = falloc(R), *e = falloc(R), *S = falloc(R), *gS = falloc(R), *gzs = falloc(R);
#pragma omp for schedule(static)
        for (int i = 0; i < Cc; i++) {
            for (int j = 0; j < R; j++) y[j] = X[(size_t)j * Cc + i];   /* Permute(1,0); Pad/Shrink are identity */
            float m = NEG_FLT_MAX, tie = 0.0f, s = 0.0f;
            for (int j = 0; j < R; j++) m = fmaxf(m, y[j]);
            for (int j = 0; j < R; j++) tie = tie + (y[j] == m ? 1.0f : 0.0f);
            for (int j = 0; j < R; j++) { e[j] = exp2f((y[j] - m) * INV_LN2); s = s + e[j]; }
            float rs = 1.0f / s;
            float sq = 0.0f;
            for (int j = 0; j < R; j++) { S[j] = e[j] * rs; sq = sq + S[j] * S[j]; }
            float q = sq * rR;
            float T = sqrtf(q + eps);
            float r = 1.0f / T;
            float gi = g[i];
            float lsum = 0.0f, dgi = 0.0f, gR = 0.0f;
            for (int j = 0; j < R; j++) {
                float A = S[j] * r;
                lsum = lsum + A * gi;
                dgi = dgi + A;                          /* Expand rule over the row of out = A*g */
                gR = gR + gi * S[j];                    /* Mul rule then Expand-sum into r */
            }
            rowloss[i] = lsum;
            if (dg) dg[i] = dgi;
            if (!dX) continue;
            float gT = ((-gR) * r) * r;                 /* Recip rule */
            float gu = gT * (1.0f / (2.0f * T));        /* Sqrt rule: adj.Div(2*node) */
            float gsq = gu * rR;                        /* Mul by Recip(R) */
            float gRs = 0.0f;
            for (int j = 0; j < R; j++) {
                float t2 = gsq * S[j];
                gS[j] = ((gi * r) + t2) + t2;           /* A-branch first, then both Mul(S,S) srcs */
                gRs = gRs + gS[j] * e[j];
            }
            float gs = ((-gRs) * rs) * rs;              /* Recip rule on s */
            float gm = 0.0f;
            for (int j = 0; j < R; j++) {
                float ge = gS[j] * rs + gs;             /* Mul(e, Recip s) rule, then Sum-expand */
                float gv = (ge * e[j]) * LN2F;          /* Exp2 rule */
                gzs[j] = gv * INV_LN2;
                gm = gm + (-gzs[j]);
            }
            float share = gm * (1.0f / tie);
            for (int j = 0; j < R; j++)
                dX[(size_t)j * Cc + i] = gzs[j] + (y[j] == m ? share : 0.0f);
        }
        free(y); free(e); free(S); free(gS); free(gzs);
    }
    if (loss) {
        /* Sum over the [Cc, R] output in row-major order */
        float tot = 0.0f;
        for (int i = 0; i < Cc; i++) tot = tot + rowloss[i];
        *loss = tot;
    }
    free(rowloss);
}

/* ── f64 forward losses (finite-difference checks) ───────────────────────── */

static double ce_loss_f64(const double *z, const int32_t *labels, int B, int C) {
    double tot = 0.0;
    for (int b = 0; b < B; b++) {
        const double *zr = z + (size_t)b * C;
        double m = -DBL_MAX, s = 0.0;
        for (int c = 0; c < C; c++) m = fmax(m, zr[c]);
        for (int c = 0; c < C; c++) s += exp(zr[c] - m);
        tot += (zr[labels[b]] - m) - log(s);
    }
    return -tot / B;
}
static void lin_f64(const double *X, const double *W, const double *b, int M, int N, int K, double *Z) {
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            double acc = 0.0;
            for (int k = 0; k < K; k++) acc += X[(size_t)m * K + k] * W[(size_t)n * K + k];
            Z[(size_t)m * N + n] = acc + (b ? b[n] : 0.0);
        }
}

double ora_mlp_ce_loss_f64(const double *x, const int32_t *labels, int B, int D, int Hd, int C,
                           const double *W1, const double *b1, const double *W2, const double *b2) {
    double *h = (double *)calloc((size_t)B * Hd, 8), *z = (double *)calloc((size_t)B * C, 8);
    lin_f64(x, W1, b1, B, Hd, D, h);
    for (size_t i = 0; i < (size_t)B * Hd; i++) h[i] = fmax(h[i], 0.0);
    lin_f64(h, W2, b2, B, C, Hd, z);
    double l = ce_loss_f64(z, labels, B, C);
    free(h); free(z);
    return l;
}

static void conv_f64(const double *x, int N, int Ci, int H, const double *w, const double *b, int Co, double *out) {
    for (int n = 0; n < N; n++)
        for (int co = 0; co < Co; co++)
            for (int h = 0; h < H; h++)
                for (int wv = 0; wv < H; wv++) {
                    double acc = b[co];
                    for (int ci = 0; ci < Ci; ci++)
                        for (int kh = 0; kh < 3; kh++)
                            for (int kw = 0; kw < 3; kw++) {
                                int y = h + kh - 1, xx = wv + kw - 1;
                                if (y < 0 || y >= H || xx < 0 || xx >= H) continue;
                                acc += x[(((size_t)n * Ci + ci) * H + y) * H + xx] *
                                       w[((size_t)co * Ci + ci) * 9 + kh * 3 + kw];
                            }
                    out[(((size_t)n * Co + co) * H + h) * H + wv] = acc;
                }
}
static void relu_pool_f64(const double *z, int NC, int H, double *p) {
    int P = H / 2;
    for (int c = 0; c < NC; c++)
        for (int i = 0; i < P; i++)
            for (int j = 0; j < P; j++) {
                double m = -DBL_MAX;
                for (int a = 0; a < 2; a++)
                    for (int bb = 0; bb < 2; bb++)
                        m = fmax(m, fmax(z[((size_t)c * H + 2 * i + a) * H + 2 * j + bb], 0.0));
                p[((size_t)c * P + i) * P + j] = m;
            }
}

double ora_convnet_loss_f64(const double *x, const int32_t *labels, int N, int Hin, int C1, int C2,
                            int NC, const double *cw1, const double *cb1, const double *cw2,
                            const double *cb2, const double *fw, const double *fb) {
    int P1 = Hin / 2, P2 = Hin / 4, F = C2 * P2 * P2;
    double *z1 = (double *)calloc((size_t)N * C1 * Hin * Hin, 8), *p1 = (double *)calloc((size_t)N * C1 * P1 * P1, 8);
    double *z2 = (double *)calloc((size_t)N * C2 * P1 * P1, 8), *p2 = (double *)calloc((size_t)N * F, 8);
    double *lg = (double *)calloc((size_t)N * NC, 8);
    conv_f64(x, N, 1, Hin, cw1, cb1, C1, z1);
    relu_pool_f64(z1, N * C1, Hin, p1);
    conv_f64(p1, N, C1, P1, cw2, cb2, C2, z2);
    relu_pool_f64(z2, N * C2, P1, p2);
    lin_f64(p2, fw, fb, N, NC, F, lg);
    double l = ce_loss_f64(lg, labels, N, NC);
    free(z1); free(p1); free(z2); free(p2); free(lg);
    return l;
}

double ora_mlp3_loss_f64(const double *x, const double *t, int B, int D0, int D1, int D2, int D3,
                         const double *W1, const double *b1, const double *W2, const double *b2,
                         const double *W3, const double *b3) {
    double *h1 = (double *)calloc((size_t)B * D1, 8), *h2 = (double *)calloc((size_t)B * D2, 8);
    double *p = (double *)calloc((size_t)B * D3, 8);
    lin_f64(x, W1, b1, B, D1, D0, h1);
    for (size_t i = 0; i < (size_t)B * D1; i++) h1[i] = fmax(h1[i], 0.0);
    lin_f64(h1, W2, b2, B, D2, D1, h2);
    for (size_t i = 0; i < (size_t)B * D2; i++) h2[i] = fmax(h2[i], 0.0);
    lin_f64(h2, W3, b3, B, D3, D2, p);
    double s = 0.0;
    for (size_t i = 0; i < (size_t)B * D3; i++) s += (p[i] - t[i]) * (p[i] - t[i]);
    free(h1); free(h2); free(p);
    return s / ((double)B * D3);
}

double ora_chain_loss_f64(const double *X, const double *g, int R, int Cc) {
    double tot = 0.0;
    for (int i = 0; i < Cc; i++) {
        double m = -DBL_MAX, s = 0.0, sq = 0.0, row = 0.0;
        for (int j = 0; j < R; j++) m = fmax(m, X[(size_t)j * Cc + i]);
        for (int j = 0; j < R; j++) s += exp(X[(size_t)j * Cc + i] - m);
        for (int j = 0; j < R; j++) { double S = exp(X[(size_t)j * Cc + i] - m) / s; sq += S * S; }
        double r = 1.0 / sqrt(sq / R + 1e-6);
        for (int j = 0; j < R; j++) row += exp(X[(size_t)j * Cc + i] - m) / s * r * g[i];
        tot += row;
    }
    return tot;
}
