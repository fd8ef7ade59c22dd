/*
 * anneal_oracle.h — CPU restatement of georgebuilds/anneal's training-step semantics.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product library (anneal_amd/) links,
 * loads or calls this code; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only as the checker / the CPU baseline.
 *
 * Every function restates the value the reference's lazy graph produces for the
 * op composition named in its comment. The reference is Go + generated WGSL; its
 * scheduler cannot be run here (no Go toolchain), so the oracle follows the op
 * decompositions in tensor/ops.go, tensor/reduce.go, tensor/gradient_ruleset.go,
 * tensor/nn/nn.go and the accumulator/narrowing rules in codegen/lower.go.
 *
 * Conventions:
 *   - all floating point is IEEE f32 evaluated in program order (built with
 *     -ffp-contract=off), reductions accumulate sequentially in index order like
 *     the reference's serial reduce loop (codegen/lower.go:654-719);
 *   - ±Inf constants and the max-reduce identity are ±FLT_MAX
 *     (codegen/wgsl.go:318-329,376-386);
 *   - Exp(x) = exp2(x * f32(1/ln2)), Log(x) = log2(x) * f32(ln2) (tensor/ops.go:56-65);
 *   - Div(a,b) = a * (1/b) (tensor/ops.go:92-98, codegen/wgsl.go:263);
 *   - ReLU = Max(x, 0), tie gradient to src0 (tensor/nn/nn.go:111; gradient_ruleset.go:153-161);
 *   - max-reduce backward splits ties: adj * (1/tieCount) (gradient_ruleset.go:307-320).
 *
 * Parity pinning (which test pins which function) is listed in tests/test_oracle_golden.py.
 */
#ifndef ANNEAL_ORACLE_H
#define ANNEAL_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* f16 codec — uop/dtype.go:392 (Float32ToFloat16), :447 (Float16ToFloat32), :478 (Quantize). */
uint16_t ora_f32_to_f16(float f);
float ora_f16_to_f32(uint16_t h);
float ora_quantize_f16(float f);
void ora_f32_to_f16_array(const float *src, uint16_t *dst, int64_t n);
void ora_f16_to_f32_array(const uint16_t *src, float *dst, int64_t n);

/* C[M,N] = A[M,K] @ B[K,N] as Sum(Mul(Expand A, Expand B), axis=-2) — tensor/reduce.go:105-166. */
void ora_matmul(const float *A, const float *B, int M, int K, int N, float *C);

/* y = x@W (x[M,K], W[K,N]); loss = Mean((y-t)^2) = Sum(...)*recip(M*N) (reduce.go:71-92);
 * gradients of loss w.r.t. x and W (webgpu_test.go:278-458 graph). Any out pointer may be NULL. */
void ora_linear_mse(const float *x, const float *W, const float *t, int M, int K, int N,
                    float *loss, float *gx, float *gW);

/* loss = Sum(exp2(x)); gx = d loss / dx (gradient_ruleset.go:78-82). */
void ora_exp2_sum_grad(const float *x, int n, float *loss, float *gx);

/* MaxPool2D (tensor/nn/nn.go:328-387), both the non-overlapping reduce path and the
 * overlapping binary-Maximum chain; gx = gradient of Sum(out * adjw) w.r.t. x where
 * adjw is the per-output adjoint (NULL = ones). */
void ora_maxpool2d(const float *x, int N, int C, int H, int W, int kH, int kW, int sH, int sW,
                   float *out, const float *adjw, float *gx);

/* Softmax cross-entropy composed from reference tensor ops (see anneal_oracle.c):
 * loss = Sum(onehot * (z - m - Log(Sum(Exp(z - m))))) * f32(-1/B); dz = d loss / d z. */
void ora_softmax_ce(const float *z, const int32_t *labels, int B, int C, float *loss, float *dz);

/* ── Config steps ─────────────────────────────────────── */

/* Two-layer MLP, f32: Linear(D->H)+ReLU, Linear(H->C), softmax-CE, Backward, SGD (configs 1 and 4).
 * W1[H,D], b1[H], W2[C,H], b2[C] are updated in place; grads written when non-NULL. */
void ora_mlp_ce_step(const float *x, const int32_t *labels, int B, int D, int Hd, int C,
                     float *W1, float *b1, float *W2, float *b2, float lr,
                     float *loss, float *dW1, float *db1, float *dW2, float *db2);

/* Small conv net, f32 (config 2). x[N,1,28,28]; conv1 W[8,1,3,3] b[8]; conv2 W[16,8,3,3] b[16];
 * fc W[10,784] b[10]. Generic in N, Hin (multiple of 4), C1, C2, classes. Params updated in place. */
void ora_convnet_step(const float *x, const int32_t *labels, int N, int Hin, int C1, int C2, int NC,
                      float *cw1, float *cb1, float *cw2, float *cb2, float *fw, float *fb, float lr,
                      float *loss, float *dcw1, float *dcb1, float *dcw2, float *dcb2,
                      float *dfw, float *dfb);

/* Three-layer MLP with f16 storage (config 3): Linear(D0->D1) ReLU, Linear(D1->D2) ReLU,
 * Linear(D2->D3), loss = Sum((p-t)*(p-t)) * f32(1/(B*D3)); f32 master weights (nn.go:56-76).
 * x, t are f32 arrays already holding f16-representable values. Weights updated in place. */
void ora_mlp3_f16_step(const float *x, const float *t, int B, int D0, int D1, int D2, int D3,
                       float *W1, float *b1, float *W2, float *b2, float *W3, float *b3, float lr,
                       float *loss, float *dW1, float *db1, float *dW2, float *db2, float *dW3,
                       float *db3);

/* Movement/reduce chain (config 5). X[R,Cc]; Y = Shrink(Pad(Permute(X,(1,0)))) [Cc,R];
 * S = softmax(Y, axis=1); out = S * recip(sqrt(mean(S*S, axis=1) + 1e-6)) * g[Cc,1];
 * loss = Sum(out); dX, dg = gradients. */
void ora_chain_step(const float *X, const float *g, int R, int Cc, float *loss, float *dX, float *dg);

/* f64 forward-only losses with the same graph and no f16 rounding, for finite-difference
 * checks of the gradients above. */
double ora_mlp_ce_loss_f64(const double *x, const int32_t *labels, int B, int D, int Hd, int C,
                           const double *W1, const double *b1, const double *W2, const double *b2);
double ora_convnet_loss_f64(const double *x, const int32_t *labels, int N, int Hin, int C1, int C2,
                            int NC, const double *cw1, const double *cb1, const double *cw2,
                            const double *cb2, const double *fw, const double *fb);
double ora_mlp3_loss_f64(const double *x, const double *t, int B, int D0, int D1, int D2, int D3,
                         const double *W1, const double *b1, const double *W2, const double *b2,
                         const double *W3, const double *b3);
double ora_chain_loss_f64(const double *X, const double *g, int R, int Cc);

int ora_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
