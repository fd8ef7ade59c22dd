// conv.hip — direct 3x3 convolution, fused ReLU + 2x2 max-pool, and their backward (config 2).
//
// The reference lowers Conv2d to im2col built from K padded one-column tensors plus one batched matmul
// (tensor/nn/nn.go:217-303): every im2col element is a K-term sum with one non-zero term, so the value
// equals the direct convolution computed here with the same k = ci*9 + kh*3 + kw accumulation order.
// MaxPool2D(2,2,2,2) is the non-overlapping reduce path (nn.go:350-372): max with -FLT_MAX identity,
// backward split equally over tied maxima (tensor/gradient_ruleset.go:307-320).
#include <float.h>

#include "ah_common.h"
#include "conv.h"

namespace ah {

// One thread per pooled output: 4 conv outputs (+bias, ReLU-tagged) and their max.
__global__ __launch_bounds__(256) void conv_fwd_relu_pool_kernel(const float *X, int N, int Ci, int H, const float *w,
                                                                  const float *b, int Co, float *Hout, float *Pout) {
    const int P = H / 2;
    long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    long total = (long)N * Co * P * P;
    if (idx >= total) return;
    int pw = idx % P, ph = (idx / P) % P, co = (idx / ((long)P * P)) % Co, n = idx / ((long)P * P * Co);
    float m = -FLT_MAX;
    for (int dy = 0; dy < 2; dy++)
        for (int dx = 0; dx < 2; dx++) {
            int h = 2 * ph + dy, wv = 2 * pw + dx;
            float acc = 0.0f;
            for (int ci = 0; ci < Ci; ci++) {
                const float *xp = X + ((long)n * Ci + ci) * H * H;
                const float *wp = w + ((long)co * Ci + ci) * 9;
#pragma unroll
                for (int kh = 0; kh < 3; kh++)
#pragma unroll
                    for (int kw = 0; kw < 3; kw++) {
                        int y = h + kh - 1, xx = wv + kw - 1;
                        float v = (y >= 0 && y < H && xx >= 0 && xx < H) ? xp[y * H + xx] : 0.0f;
                        acc = acc + v * wp[kh * 3 + kw];
                    }
            }
            float hv = relu_tag(acc + b[co]);
            Hout[(((long)n * Co + co) * H + h) * H + wv] = hv;
            m = fmaxf(m, hv);
        }
    Pout[idx] = m;
}

// Pool backward (tie split) fused with the ReLU mask: one thread per pooling window.
__global__ __launch_bounds__(256) void pool_relu_bwd_kernel(const float *dP, const float *Hact, const float *Pv, int NC,
                                                             int H, float *dZ) {
    const int P = H / 2;
    long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long)NC * P * P) return;
    int pw = idx % P, ph = (idx / P) % P;
    long nc = idx / ((long)P * P);
    const float *hp = Hact + nc * H * H;
    float m = Pv[idx];
    float v[4];
    float tie = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        v[q] = hp[(2 * ph + (q >> 1)) * H + 2 * pw + (q & 1)];
        tie = tie + (v[q] == m ? 1.0f : 0.0f);
    }
    float share = dP[idx] * (1.0f / tie);
#pragma unroll
    for (int q = 0; q < 4; q++) {
        float g = (v[q] == m) ? share : 0.0f;
        dZ[nc * H * H + (2 * ph + (q >> 1)) * H + 2 * pw + (q & 1)] = relu_dead(v[q]) ? 0.0f : g;
    }
}

// dX[n,ci,y,x] = sum_{co,kh,kw} G[n,co,y-kh+1,x-kw+1] * w[co,ci,kh,kw]   (col2im of the im2col adjoint)
__global__ __launch_bounds__(256) void conv_bwd_x_kernel(const float *G, const float *w, int N, int Ci, int H, int Co,
                                                          float *dX) {
    long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long)N * Ci * H * H) return;
    int xx = idx % H, y = (idx / H) % H, ci = (idx / ((long)H * H)) % Ci, n = idx / ((long)H * H * Ci);
    float acc = 0.0f;
#pragma unroll
    for (int kh = 0; kh < 3; kh++)
#pragma unroll
        for (int kw = 0; kw < 3; kw++) {
            int h = y - kh + 1, wv = xx - kw + 1;
            if (h < 0 || h >= H || wv < 0 || wv >= H) continue;
            float part = 0.0f;
            for (int co = 0; co < Co; co++)
                part = part + G[(((long)n * Co + co) * H + h) * H + wv] * w[((long)co * Ci + ci) * 9 + kh * 3 + kw];
            acc += part;
        }
    dX[idx] = acc;
}

// Weight/bias gradient, stage 1: block (co, ci, split) owns the 9 weights of (co, ci) (and the bias
// when ci == 0) over one contiguous share of the N*H*H positions, reduced with an LDS tree; the share's
// 10 partial sums go to part[split][co][ci][10]. Splitting the positions keeps enough blocks in flight
// when Co*Ci is small (conv1: 8 weight groups over 25088 positions each).
__global__ __launch_bounds__(256) void conv_bwd_w_partial_kernel(const float *X, const float *G, int N, int Ci, int H,
                                                                  int Co, int S, float *part) {
    __shared__ float red[10][256];
    const int co = blockIdx.x, ci = blockIdx.y, sp = blockIdx.z, tid = threadIdx.x;
    float acc[10];
#pragma unroll
    for (int q = 0; q < 10; q++) acc[q] = 0.0f;
    const long HH = (long)H * H, total = (long)N * HH;
    const long chunk = (total + S - 1) / S, i0 = (long)sp * chunk, i1 = min(total, i0 + chunk);
    for (long i = i0 + tid; i < i1; i += 256) {
        int n = i / HH, p = i % HH, h = p / H, wv = p % H;
        float g = G[((long)n * Co + co) * HH + p];
        const float *xp = X + ((long)n * Ci + ci) * HH;
#pragma unroll
        for (int kh = 0; kh < 3; kh++)
#pragma unroll
            for (int kw = 0; kw < 3; kw++) {
                int y = h + kh - 1, xx = wv + kw - 1;
                float v = (y >= 0 && y < H && xx >= 0 && xx < H) ? xp[y * H + xx] : 0.0f;
                acc[kh * 3 + kw] += g * v;
            }
        acc[9] += g;
    }
#pragma unroll
    for (int q = 0; q < 10; q++) red[q][tid] = acc[q];
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (tid < o)
#pragma unroll
            for (int q = 0; q < 10; q++) red[q][tid] += red[q][tid + o];
        __syncthreads();
    }
    if (tid < 10) part[(((long)sp * Co + co) * Ci + ci) * 10 + tid] = red[tid][0];
}

// Stage 2: one thread per (co, ci, q) adds the S partials in split order (deterministic) and applies
// SGD to the weight (q < 9) or the bias (q == 9, ci == 0).
__global__ __launch_bounds__(256) void conv_bwd_w_finalize_kernel(const float *part, int S, int Co, int Ci, float *w,
                                                                   float *b, float lr, float *gw, float *gb) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= Co * Ci * 10) return;
    const int q = idx % 10, ci = (idx / 10) % Ci, co = idx / (10 * Ci);
    float g = 0.0f;
    for (int sp = 0; sp < S; sp++) g += part[(((long)sp * Co + co) * Ci + ci) * 10 + q];
    if (q < 9) {
        long wi = ((long)co * Ci + ci) * 9 + q;
        if (gw) gw[wi] = g;
        if (w) w[wi] = w[wi] - lr * g;   // w == nullptr: gradients only
    } else if (ci == 0) {
        if (gb) gb[co] = g;
        if (b) b[co] = b[co] - lr * g;
    }
}

int conv_bwd_w_splits(int N, int Ci, int H, int Co) {
    long groups = (long)Co * Ci, total = (long)N * H * H;
    long s = 512 / groups;                 // about 512 blocks in flight
    if (s > total / 1024) s = total / 1024;   // and at least ~4 positions per thread
    return (int)(s < 1 ? 1 : s > 64 ? 64 : s);
}

hipError_t conv_fwd_relu_pool(const float *X, int N, int Ci, int H, const float *w, const float *b, int Co, float *Hout,
                              float *Pout, hipStream_t s) {
    // 64-thread blocks: config 2's conv2 has 25088 pooled outputs, so 256-thread blocks would leave
    // most of the 256 CUs idle
    long total = (long)N * Co * (H / 2) * (H / 2);
    hipLaunchKernelGGL(conv_fwd_relu_pool_kernel, dim3((total + 63) / 64), dim3(64), 0, s, X, N, Ci, H, w, b, Co,
                       Hout, Pout);
    return hipGetLastError();
}
hipError_t pool_relu_bwd(const float *dP, const float *Hact, const float *Pv, int NC, int H, float *dZ, hipStream_t s) {
    long total = (long)NC * (H / 2) * (H / 2);
    hipLaunchKernelGGL(pool_relu_bwd_kernel, dim3((total + 255) / 256), dim3(256), 0, s, dP, Hact, Pv, NC, H, dZ);
    return hipGetLastError();
}
hipError_t conv_bwd_x(const float *G, const float *w, int N, int Ci, int H, int Co, float *dX, hipStream_t s) {
    long total = (long)N * Ci * H * H;
    hipLaunchKernelGGL(conv_bwd_x_kernel, dim3((total + 63) / 64), dim3(64), 0, s, G, w, N, Ci, H, Co, dX);
    return hipGetLastError();
}
hipError_t conv_bwd_w_partial(const float *X, const float *G, int N, int Ci, int H, int Co, float *part, hipStream_t s) {
    const int S = conv_bwd_w_splits(N, Ci, H, Co);
    hipLaunchKernelGGL(conv_bwd_w_partial_kernel, dim3(Co, Ci, S), dim3(256), 0, s, X, G, N, Ci, H, Co, S, part);
    return hipGetLastError();
}
hipError_t conv_bwd_w_finalize(const float *part, int N, int Ci, int H, int Co, float *w, float *b, float lr, float *gw,
                               float *gb, hipStream_t s) {
    const int S = conv_bwd_w_splits(N, Ci, H, Co);
    const int n = Co * Ci * 10;
    hipLaunchKernelGGL(conv_bwd_w_finalize_kernel, dim3((n + 255) / 256), dim3(256), 0, s, part, S, Co, Ci, w, b, lr, gw, gb);
    return hipGetLastError();
}

}  // namespace ah
