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

// Weight/bias gradient with the SGD update fused: block (co, ci) owns 9 weights (and the bias when
// ci == 0), reduces over the N*H*H positions with an LDS tree, then updates them in place.
__global__ __launch_bounds__(256) void conv_bwd_w_sgd_kernel(const float *X, const float *G, int N, int Ci, int H,
                                                              int Co, float *w, float *b, float lr, float *gw,
                                                              float *gb) {
    __shared__ float red[10][256];
    const int co = blockIdx.x, ci = blockIdx.y, tid = threadIdx.x;
    float acc[10];
#pragma unroll
    for (int q = 0; q < 10; q++) acc[q] = 0.0f;
    const long HH = (long)H * H;
    for (long i = tid; i < (long)N * HH; i += 256) {
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
    if (tid < 9) {
        long wi = ((long)co * Ci + ci) * 9 + tid;
        float g = red[tid][0];
        if (gw) gw[wi] = g;
        w[wi] = w[wi] - lr * g;
    } else if (tid == 9 && ci == 0) {
        float g = red[9][0];
        if (gb) gb[co] = g;
        b[co] = b[co] - lr * g;
    }
}

hipError_t conv_fwd_relu_pool(const float *X, int N, int Ci, int H, const float *w, const float *b, int Co, float *Hout,
                              float *Pout, hipStream_t s) {
    long total = (long)N * Co * (H / 2) * (H / 2);
    hipLaunchKernelGGL(conv_fwd_relu_pool_kernel, dim3((total + 255) / 256), dim3(256), 0, s, X, N, Ci, H, w, b, Co,
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
    hipLaunchKernelGGL(conv_bwd_x_kernel, dim3((total + 255) / 256), dim3(256), 0, s, G, w, N, Ci, H, Co, dX);
    return hipGetLastError();
}
hipError_t conv_bwd_w_sgd(const float *X, const float *G, int N, int Ci, int H, int Co, float *w, float *b, float lr,
                          float *gw, float *gb, hipStream_t s) {
    hipLaunchKernelGGL(conv_bwd_w_sgd_kernel, dim3(Co, Ci), dim3(256), 0, s, X, G, N, Ci, H, Co, w, b, lr, gw, gb);
    return hipGetLastError();
}

}  // namespace ah
