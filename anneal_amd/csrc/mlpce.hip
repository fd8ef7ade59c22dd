// mlpce.hip — the MLP softmax-CE train step (Linear-ReLU-Linear, config 1's shape class) as two
// three kernels (gfx950).
//
// The per-op step is eight dependent launches of a few microseconds each (GEMMs, softmax-CE, column
// sums, the tail); at B = 64, D = 784, H = 128, C = 10 none of them has enough work to fill the GPU.
// Here:
//  1. mlpce_hidden_kernel: tiles of 8 samples x 8 hidden units, each output's 784-term dot split
//     over 16 lanes (16-byte loads straight from memory) and summed by DPP, bias + ReLU (sign-tagged,
//     as the GEMM epilogue).
//  2. mlpce_head_kernel: one wave per sample: logits, softmax-CE, the logit gradient and dH.
//  3. mlpce_grad_kernel: workgroup d owns the input columns [8d, 8d+8) of W1 (dW1 over the batch and
//     the SGD update); one more workgroup takes dW2, db2, db1, the loss and their updates.
// The reference evaluates the same graph op by op (tensor/nn/nn.go Linear/ReLU/CrossEntropy; the
// gradient rules of tensor/gradient_ruleset.go); the softmax-CE row is the shared softmax_row.h code.
#include <float.h>

#include "ah_common.h"
#include "mlpce.h"
#include "softmax_row.h"

namespace ah {

constexpr int kMlpThreads = 1024;
constexpr int kMlpMaxB = 64, kMlpMaxH = 128, kMlpMaxC = 16, kMlpMaxD = 896;
constexpr int kW2Ld = kMlpMaxH + 16;
constexpr int kHidTile = 8;    // samples and hidden units per hidden-layer workgroup
constexpr int kGradCols = 8;   // input columns of W1 per gradient workgroup

template <int CTRL>
__device__ __forceinline__ float mlp_dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// Sum over each row of 16 lanes in a fixed order; every lane of the row holds it.
__device__ __forceinline__ float mlp_row16(float v) {
    v += mlp_dpp<0xB1>(v);    // quad_perm [1,0,3,2]
    v += mlp_dpp<0x4E>(v);    // quad_perm [2,3,0,1]
    v += mlp_dpp<0x141>(v);   // row_half_mirror
    v += mlp_dpp<0x140>(v);   // row_mirror
    return v;
}

__global__ __launch_bounds__(kMlpThreads) void mlpce_hidden_kernel(const float *__restrict__ x,
                                                                   const float *__restrict__ W1,
                                                                   const float *__restrict__ b1, int B, int D, int H,
                                                                   float *__restrict__ Hout) {
    // 64 outputs x 16 lanes: output o = (sample o / 8, unit o % 8) of the tile; lane ks reads the 16-byte
    // chunks ks, ks+16, ... of both rows straight from memory (the tile's 8 + 8 rows stay in L1/L2)
    constexpr int kChunks = (kMlpMaxD / 4 + 15) / 16;
    const int tid = threadIdx.x, o = tid / 16, ks = tid % 16;
    const int n = blockIdx.x * kHidTile + o / kHidTile, j = blockIdx.y * kHidTile + o % kHidTile;
    const bool live = n < B && j < H;
    const float *xr = x + (long)(live ? n : 0) * D, *wr = W1 + (long)(live ? j : 0) * D;
    float acc = 0.0f;
    if (D % 4 == 0) {
        floatx4 xv[kChunks], wv[kChunks];
#pragma unroll
        for (int m = 0; m < kChunks; m++) {
            const int k = 4 * (ks + 16 * m);
            const bool in = live && k < D;
            xv[m] = in ? *(const floatx4 *)(xr + k) : (floatx4){};
            wv[m] = in ? *(const floatx4 *)(wr + k) : (floatx4){};
        }
#pragma unroll
        for (int m = 0; m < kChunks; m++)
#pragma unroll
            for (int u = 0; u < 4; u++) acc += xv[m][u] * wv[m][u];
    } else if (live) {
        for (int k = ks; k < D; k += 16) acc += xr[k] * wr[k];
    }
    acc = mlp_row16(acc);
    if (ks == 0 && live) Hout[(long)n * H + j] = relu_tag(acc + b1[j]);
}

// Softmax-CE and the hidden-layer gradient: one wave per sample. Writes dz[n] (the logit gradient, scaled
// by a), dH[n] (zero where the ReLU was off) and rowloss[n].
__global__ __launch_bounds__(256) void mlpce_head_kernel(const int32_t *__restrict__ lab, const float *__restrict__ Hg,
                                                         const float *__restrict__ W2, const float *__restrict__ b2,
                                                         int B, int H, int C, float a, float *__restrict__ dz,
                                                         float *__restrict__ dH, float *__restrict__ rowloss) {
    constexpr int Q = kMlpMaxH / 64;
    __shared__ float lgs[4][kMlpMaxC], dzs[4][kMlpMaxC];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, n = blockIdx.x * 4 + w;
    if (n >= B) return;   // whole waves leave; nothing below synchronizes the workgroup
    // every load first: the sample's hidden row, W2's columns of this lane, the label and the biases
    float hv[Q], w2v[kMlpMaxC][Q];
#pragma unroll
    for (int q = 0; q < Q; q++) hv[q] = lane + 64 * q < H ? Hg[(long)n * H + lane + 64 * q] : 0.0f;
#pragma unroll
    for (int c = 0; c < kMlpMaxC; c++)
#pragma unroll
        for (int q = 0; q < Q; q++) w2v[c][q] = (c < C && lane + 64 * q < H) ? W2[(long)c * H + lane + 64 * q] : 0.0f;
    const int label = lab[n];
    const float bv = lane < C ? b2[lane] : 0.0f;
    // the C logits' shuffle trees in flight together
    float v[kMlpMaxC];
#pragma unroll
    for (int c = 0; c < kMlpMaxC; c++) {
        v[c] = 0.0f;
#pragma unroll
        for (int q = 0; q < Q; q++) v[c] += hv[q] * w2v[c][q];
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1)
#pragma unroll
        for (int c = 0; c < kMlpMaxC; c++) v[c] += __shfl_xor(v[c], o, 64);
    if (lane < C) {
        float mine = v[0];
#pragma unroll
        for (int c = 1; c < kMlpMaxC; c++) mine = lane == c ? v[c] : mine;
        lgs[w][lane] = mine + bv;
    }
    const float r = softmax_ce_row(lgs[w], label, C, a, dzs[w], lane);
    if (lane == 0) rowloss[n] = r;
    if (lane < C) dz[(long)n * C + lane] = dzs[w][lane];
#pragma unroll
    for (int q = 0; q < Q; q++) {
        const int j = lane + 64 * q;
        float g = 0.0f;
#pragma unroll
        for (int c = 0; c < kMlpMaxC; c++)
            if (c < C) g += dzs[w][c] * w2v[c][q];
        if (j < H) dH[(long)n * H + j] = relu_dead(hv[q]) ? 0.0f : g;
    }
}

// Copies n floats (n <= 8192, both pointers 16-byte aligned when n % 4 == 0) global -> LDS with every
// load issued before the first store.
__device__ __forceinline__ void mlp_stage(float *dst, const float *src, int n) {
    constexpr int kPer = kMlpMaxB * kMlpMaxH / 4 / kMlpThreads;   // 16-byte chunks per thread
    if (n % 4 == 0) {
        floatx4 v[kPer];
#pragma unroll
        for (int u = 0; u < kPer; u++) {
            const int c = threadIdx.x + u * kMlpThreads;
            v[u] = 4 * c < n ? *(const floatx4 *)(src + 4 * c) : (floatx4){};
        }
#pragma unroll
        for (int u = 0; u < kPer; u++) {
            const int c = threadIdx.x + u * kMlpThreads;
            if (4 * c < n) *(floatx4 *)(dst + 4 * c) = v[u];
        }
    } else {
        for (int i = threadIdx.x; i < n; i += kMlpThreads) dst[i] = src[i];
    }
}

// Weight gradients and SGD. Workgroup d < ceil(D/8) owns the input columns [8d, 8d+8) of W1 (and
// workgroup 0 also b1); the one after them takes W2, b2 and the loss.
__global__ __launch_bounds__(kMlpThreads) void mlpce_grad_kernel(const float *__restrict__ x,
                                                                 const float *__restrict__ Hg,
                                                                 const float *__restrict__ dz,
                                                                 const float *__restrict__ dH,
                                                                 const float *__restrict__ rowloss, int B, int D,
                                                                 int H, int C, MlpSgd S) {
    __shared__ __align__(16) float hs[kMlpMaxB * kMlpMaxH];
    __shared__ float xt[kMlpMaxB * kGradCols];
    __shared__ float dzs[kMlpMaxB * kMlpMaxC];
    const int tid = threadIdx.x, i0 = blockIdx.x * kGradCols;
    if (i0 >= D) {   // the extra workgroup: dW2, db2, loss
        mlp_stage(hs, Hg, B * H);
        for (int i = tid; i < B * C; i += kMlpThreads) dzs[i] = dz[i];
        __syncthreads();
        for (int o = tid; o < C * H; o += kMlpThreads) {
            const int c = o / H, j = o % H;
            float g = 0.0f;
            for (int n = 0; n < B; n++) g += dzs[n * C + c] * hs[n * H + j];
            if (S.gW2) S.gW2[o] = g;
            S.W2[o] = S.W2[o] - S.lr * g;
        }
        if (tid < C) {
            float g = 0.0f;
            for (int n = 0; n < B; n++) g += dzs[n * C + tid];
            if (S.gb2) S.gb2[tid] = g;
            S.b2[tid] = S.b2[tid] - S.lr * g;
        }
        if (tid < 64) {
            float l = 0.0f;
            for (int n = tid; n < B; n += 64) l += rowloss[n];
            l = wave_sum(l);
            if (tid == 0) S.loss[0] = l * S.loss_scale;
        }
        return;
    }
    const int ni = min(kGradCols, D - i0);
    mlp_stage(hs, dH, B * H);
    for (int i = tid; i < B * kGradCols; i += kMlpThreads) {
        const int n = i / kGradCols, q = i % kGradCols;
        xt[i] = q < ni ? x[(long)n * D + i0 + q] : 0.0f;
    }
    __syncthreads();
    if (blockIdx.x == 0)
        for (int j = tid; j < H; j += kMlpThreads) {   // db1
            float g = 0.0f;
            for (int n = 0; n < B; n++) g += hs[n * H + j];
            if (S.gb1) S.gb1[j] = g;
            S.b1[j] = S.b1[j] - S.lr * g;
        }
    for (int o = tid; o < H * kGradCols; o += kMlpThreads) {   // W1[j][i0 + q]
        const int j = o / kGradCols, q = o % kGradCols;
        if (q >= ni) continue;
        float g = 0.0f;
        for (int n = 0; n < B; n++) g += hs[n * H + j] * xt[n * kGradCols + q];
        const long wi = (long)j * D + i0 + q;
        if (S.gW1) S.gW1[wi] = g;
        S.W1[wi] = S.W1[wi] - S.lr * g;
    }
}

bool mlpce_fused_ok(int B, int D, int H, int C) {
    return B > 0 && B <= kMlpMaxB && D > 0 && D <= kMlpMaxD && H > 0 && H <= kMlpMaxH && C > 0 && C <= kMlpMaxC;
}

hipError_t mlpce_hidden(const float *x, const float *W1, const float *b1, int B, int D, int H, float *Hout,
                        hipStream_t s) {
    if (!mlpce_fused_ok(B, D, H, 1)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(mlpce_hidden_kernel, dim3((B + kHidTile - 1) / kHidTile, (H + kHidTile - 1) / kHidTile),
                       dim3(kMlpThreads), 0, s, x, W1, b1, B, D, H, Hout);
    return hipGetLastError();
}

hipError_t mlpce_head(const int32_t *lab, const float *Hin, const float *W2, const float *b2, int B, int H, int C,
                      float a, float *dz, float *dH, float *rowloss, hipStream_t s) {
    if (!mlpce_fused_ok(B, 1, H, C)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(mlpce_head_kernel, dim3((B + 3) / 4), dim3(256), 0, s, lab, Hin, W2, b2, B, H, C, a, dz, dH,
                       rowloss);
    return hipGetLastError();
}

hipError_t mlpce_grad(const float *x, const float *Hin, const float *dz, const float *dH, const float *rowloss, int B,
                      int D, int H, int C, const MlpSgd &sgd, hipStream_t s) {
    if (!mlpce_fused_ok(B, D, H, C)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(mlpce_grad_kernel, dim3((D + kGradCols - 1) / kGradCols + 1), dim3(kMlpThreads), 0, s, x, Hin,
                       dz, dH, rowloss, B, D, H, C, sgd);
    return hipGetLastError();
}

}  // namespace ah
