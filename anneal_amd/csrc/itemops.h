// itemops.h — host launchers for the stand-alone kernels behind the executor's "tmpl:" keys.
#pragma once
#include "ah_common.h"

namespace ah {

enum RedOp : int { RED_SUM = 0, RED_MAX = 1, RED_SUMSQ = 2 };
constexpr int kRedRows = 64;   // rows per column-reduce chunk

// Zeroes `bytes` (rounded up to whole 4-byte words) with a kernel, so graph capture records no memset node.
hipError_t zero_fill(void *p, long bytes, hipStream_t s);
// Contraction operand prologues: dst = z ? Where(z == max(z, 0), src, 0) : max(src, 0), n elements of f32
// (or f16 when f16 is set).
hipError_t operand_prologue(const void *src, const void *z, bool f16, long n, void *dst, hipStream_t s);
// The same prologues into an f32 operand from sources of mixed types (an f16 activation or weight
// widened into an f32 contraction): kind 1 ReLU, 2 ReLU-backward mask (z >= 0 keeps src), 3 widening
// only; src_f16 / z_f16 give the stored types. Widening is exact.
hipError_t operand_prologue_f32(const void *src, bool src_f16, const void *z, bool z_f16, int kind, long n, float *dst,
                                hipStream_t s);
// *differs (zeroed first) becomes 1 when any of the `words` 32-bit words of a and b differ.
hipError_t words_differ(const void *a, const void *b, long words, int *differs, hipStream_t s);
// out[m] = scale * reduce_n G[m, n] (scale not applied to max); G is f32, or f16 when f16 is set, and the
// reduction runs in f32.
hipError_t reduce_rows(const void *G, bool f16, int M, int N, int op, float scale, float *out, hipStream_t s);
// out[n] = scale * reduce_m G[m, n]; work holds reduce_cols_workspace(M, N) floats. Deterministic. With Z
// (same shape as G, f16 or f32) each element is masked first: Where(Z >= 0, G, 0), the ReLU backward mask.
long reduce_cols_workspace(int M, int N);
hipError_t reduce_cols(const void *G, bool f16, int M, int N, int op, float scale, float *work, float *out, hipStream_t s,
                       const void *Z = nullptr, bool z_f16 = false);
// MaxPool2D over [NC, H, W] with window kH x kW and stride sH x sW (no padding), and its backward.
hipError_t maxpool_fwd(const float *X, long NC, int H, int W, int kH, int kW, int sH, int sW, float *out, hipStream_t s);
hipError_t maxpool_bwd(const float *X, const float *adj, long NC, int H, int W, int kH, int kW, int sH, int sW,
                       float *dX, hipStream_t s);
// 3x3, padding 1, stride 1 convolution of [N, Ci, H, H] with w [Co, Ci, 3, 3], optional bias and tagged ReLU.
hipError_t conv3x3_fwd(const float *X, int N, int Ci, int H, const float *w, const float *b, int Co, int relu, float *Y,
                       hipStream_t s);
// db[co] = sum of G[n, co, :, :] over n and the HW positions.
hipError_t conv_bias_grad(const float *G, int N, int Co, int HW, float *db, hipStream_t s);
// out = p - lr * (scale * g)
hipError_t sgd_out(const float *p, const float *g, long n, float lr, float scale, float *out, hipStream_t s);
// out[0] = f16(sum of parts[0..n)) * scale
hipError_t mse_loss(const float *parts, long n, float scale, float *out, hipStream_t s);

}  // namespace ah
