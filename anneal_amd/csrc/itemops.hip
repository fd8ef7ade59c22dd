// itemops.hip — stand-alone kernels behind the "tmpl:" keys of the executor that the device-resident
// steps do not need in this form: deterministic row/column reductions, MaxPool2D forward and backward
// for any window and stride, 3x3 convolution without pooling and its bias gradient, elementwise SGD,
// and the MSE loss finalize over per-wave partials.
//
// Reduction identities and tie rules follow the reference: Max starts from -FLT_MAX (codegen/wgsl.go:376-386),
// max backward splits the adjoint equally over tied maxima for reduce-path pooling and gives it to the
// first tied position for the overlapping Maximum chain (tensor/gradient_ruleset.go:153-161,307-320,
// tensor/nn/nn.go:328-386).
#include <float.h>

#include "ah_common.h"
#include "itemops.h"

namespace ah {

// ── zero fill (a kernel, not hipMemsetAsync, so it may be captured in a graph) ─────────────────────
__global__ void zero_u32_kernel(uint32_t *p, long n) {
    long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long stride = (long)gridDim.x * blockDim.x;
    for (; i < n; i += stride) p[i] = 0u;
}

// ── word comparison: *differs = 1 when any 32-bit word of a and b differs ──
__global__ void words_differ_kernel(const uint32_t *a, const uint32_t *b, long n, int *differs) {
    long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long stride = (long)gridDim.x * blockDim.x;
    bool d = false;
    for (; i < n; i += stride) d |= a[i] != b[i];
    if (__any(d) && (threadIdx.x & 63) == 0) *differs = 1;   // a plain vector store of the same value
}

// ── contraction operand prologues ──
// ReLU is Maximum(x, 0) in the reference; its backward keeps adj where z == max(z, 0), i.e. z >= 0
// (-0 included, NaN excluded, as the comparison there decides).
template <typename T>
__global__ void operand_prologue_kernel(const T *src, const T *z, long n, T *dst) {
    long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long stride = (long)gridDim.x * blockDim.x;
    for (; i < n; i += stride) {
        const T v = src[i];
        if (z) dst[i] = z[i] >= (T)0.0f ? v : (T)0.0f;
        else dst[i] = v > (T)0.0f ? v : (T)0.0f;
    }
}

template <typename TS, typename TZ>
__global__ void operand_prologue_f32_kernel(const TS *src, const TZ *z, int kind, long n, float *dst) {
    long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long stride = (long)gridDim.x * blockDim.x;
    for (; i < n; i += stride) {
        const float v = (float)src[i];
        if (kind == 2) dst[i] = (float)z[i] >= 0.0f ? v : 0.0f;
        else if (kind == 1) dst[i] = v > 0.0f ? v : 0.0f;
        else dst[i] = v;
    }
}

// ── reductions over a row-major [M, N] f32 matrix ──────────────────────────────────────────────────
__device__ __forceinline__ float red_init(int op) { return op == RED_MAX ? -FLT_MAX : 0.0f; }
__device__ __forceinline__ float red_step(int op, float acc, float v) {
    return op == RED_MAX ? fmaxf(acc, v) : op == RED_SUMSQ ? acc + v * v : acc + v;
}
__device__ __forceinline__ float red_join(int op, float a, float b) { return op == RED_MAX ? fmaxf(a, b) : a + b; }

// out[m] = scale * reduce_n G[m, n]: one wave per row, lanes stride the row, fixed shuffle tree.
template <typename T>
__global__ __launch_bounds__(256) void reduce_rows_kernel(const T *G, int M, int N, int op, float scale, float *out) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= M) return;
    const T *g = G + (long)row * N;
    float acc = red_init(op);
    for (int c = lane; c < N; c += 64) acc = red_step(op, acc, (float)g[c]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) acc = red_join(op, acc, __shfl_xor(acc, o, 64));
    if (lane == 0) out[row] = op == RED_MAX ? acc : acc * scale;
}

// Column reduce, pass 1: block (column group of 64, row chunk) folds kRedRows rows with 4 row lanes per
// column, then the 4 lanes in a fixed order; the chunk's value goes to part[chunk][n]. With Z, an element
// enters as Where(Z == max(Z, 0), G, 0) (the ReLU backward mask, gradient_ruleset.go:153-161), else 0.
template <typename T, typename TZ>
__global__ __launch_bounds__(256) void reduce_cols_partial_kernel(const T *G, const TZ *Z, int M, int N, int op, float *part) {
    __shared__ float red[4][64];
    const int col = blockIdx.x * 64 + (threadIdx.x & 63), sub = threadIdx.x >> 6;
    const int r0 = blockIdx.y * kRedRows, r1 = min(M, r0 + kRedRows);
    float acc = red_init(op);
    if (col < N)
        for (int r = r0 + sub; r < r1; r += 4) {
            const long i = (long)r * N + col;
            float v = (float)G[i];
            if (Z) v = (float)Z[i] >= 0.0f ? v : 0.0f;
            acc = red_step(op, acc, v);
        }
    red[sub][threadIdx.x & 63] = acc;
    __syncthreads();
    if (sub == 0 && col < N) {
        const int t = threadIdx.x;
        part[(long)blockIdx.y * N + col] = red_join(op, red_join(op, red[0][t], red[1][t]), red_join(op, red[2][t], red[3][t]));
    }
}

// Pass 2: out[n] = scale * fold of the chunk values in chunk order.
__global__ __launch_bounds__(256) void reduce_cols_final_kernel(const float *part, int chunks, int N, int op,
                                                                 float scale, float *out) {
    const int col = blockIdx.x * 256 + threadIdx.x;
    if (col >= N) return;
    float acc = chunks > 0 ? part[col] : red_init(op);   // an empty reduce yields the identity
    for (int c = 1; c < chunks; c++) acc = red_join(op, acc, part[(long)c * N + col]);
    out[col] = op == RED_MAX ? acc : acc * scale;
}

// ── MaxPool2D ──────────────────────────────────────────────────────────────────────────────────────
// Window max: the reduce path (kH <= sH and kW <= sW) starts from the -FLT_MAX identity; the overlapping
// path is a chain of binary Maximum ops starting from the window's first element (nn.go:374-386).
__device__ __forceinline__ float window_max(const float *xp, int W, int h0, int w0, int kH, int kW, bool overlap) {
    float m = overlap ? xp[h0 * W + w0] : -FLT_MAX;
    for (int i = 0; i < kH; i++)
        for (int j = 0; j < kW; j++)
            if (!overlap || i || j) m = fmaxf(m, xp[(h0 + i) * W + w0 + j]);
    return m;
}

__global__ __launch_bounds__(256) void maxpool_fwd_kernel(const float *X, long NC, int H, int W, int kH, int kW,
                                                           int sH, int sW, int oH, int oW, float *out) {
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= NC * oH * oW) return;
    const int ow = idx % oW, oh = (idx / oW) % oH;
    const long nc = idx / ((long)oH * oW);
    const bool overlap = !(kH <= sH && kW <= sW);
    out[idx] = window_max(X + nc * H * W, W, oh * sH, ow * sW, kH, kW, overlap);
}

// Backward as a gather: one thread per input element visits the windows that contain it in (oh, ow)
// order and adds its share of each window's adjoint, so every element receives the same additions, in
// the same order, as the window-by-window scatter (0 + share1 + share2 ...). Reduce path: share =
// adj * (1/tie) for every element equal to the window max (tie = number of such elements, counted as a
// float sum). Overlapping path: the whole adjoint goes to the first element (row-major) equal to the max.
__global__ __launch_bounds__(256) void maxpool_bwd_kernel(const float *X, const float *adj, long NC, int H, int W,
                                                           int kH, int kW, int sH, int sW, int oH, int oW, float *dX) {
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= NC * H * W) return;
    const int w = idx % W, h = (idx / W) % H;
    const long nc = idx / ((long)H * W);
    const float *xp = X + nc * H * W;
    const float *ap = adj + nc * oH * oW;
    const bool overlap = !(kH <= sH && kW <= sW);
    const float xv = xp[h * W + w];
    const int oh0 = h - kH + 1 > 0 ? (h - kH + 1 + sH - 1) / sH : 0, oh1 = min(h / sH, oH - 1);
    const int ow0 = w - kW + 1 > 0 ? (w - kW + 1 + sW - 1) / sW : 0, ow1 = min(w / sW, oW - 1);
    float acc = 0.0f;
    for (int oh = oh0; oh <= oh1; oh++)
        for (int ow = ow0; ow <= ow1; ow++) {
            const int h0 = oh * sH, w0 = ow * sW;
            const float m = window_max(xp, W, h0, w0, kH, kW, overlap);
            if (xv != m) continue;
            const float a = ap[(long)oh * oW + ow];
            if (!overlap) {
                float tie = 0.0f;
                for (int i = 0; i < kH; i++)
                    for (int j = 0; j < kW; j++) tie = tie + (xp[(h0 + i) * W + w0 + j] == m ? 1.0f : 0.0f);
                acc += a * (1.0f / tie);
            } else {
                int first = -1;
                for (int i = 0; i < kH && first < 0; i++)
                    for (int j = 0; j < kW && first < 0; j++)
                        if (xp[(h0 + i) * W + w0 + j] == m) first = (h0 + i) * W + w0 + j;
                if (first == h * W + w) acc += a;
            }
        }
    dX[idx] = acc;
}

// ── 3x3 convolution, padding 1, stride 1 (Conv2d as the reference lowers it, nn.go:217-303) ───────
// Accumulates k = ci*9 + kh*3 + kw in order, then adds the bias; optional tagged ReLU.
__global__ __launch_bounds__(64) void conv3x3_fwd_kernel(const float *X, int N, int Ci, int H, const float *w,
                                                          const float *b, int Co, int relu, float *Y) {
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long)N * Co * H * H) return;
    const int x = idx % H, y = (idx / H) % H, co = (idx / ((long)H * H)) % Co;
    const long n = idx / ((long)H * H * Co);
    float acc = 0.0f;
    for (int ci = 0; ci < Ci; ci++) {
        const float *xp = X + (n * Ci + ci) * H * H;
        const float *wp = w + ((long)co * Ci + ci) * 9;
#pragma unroll
        for (int kh = 0; kh < 3; kh++)
#pragma unroll
            for (int kw = 0; kw < 3; kw++) {
                const int yy = y + kh - 1, xx = x + kw - 1;
                const float v = (yy >= 0 && yy < H && xx >= 0 && xx < H) ? xp[yy * H + xx] : 0.0f;
                acc = acc + v * wp[kh * 3 + kw];
            }
    }
    const float z = acc + (b ? b[co] : 0.0f);
    Y[idx] = relu ? relu_tag(z) : z;
}

// db[co] = sum over (n, y, x) of G[n, co, y, x]: one block per channel, fixed-order tree.
__global__ __launch_bounds__(256) void conv_bias_grad_kernel(const float *G, int N, int Co, int HW, float *db) {
    __shared__ float red[256];
    const int co = blockIdx.x;
    float acc = 0.0f;
    for (long i = threadIdx.x; i < (long)N * HW; i += 256) {
        const long n = i / HW, p = i % HW;
        acc += G[(n * Co + co) * HW + p];
    }
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
        __syncthreads();
    }
    if (threadIdx.x == 0) db[co] = red[0];
}

// ── SGD into a new buffer: out = p - lr * (scale * g)  (Parameter.SGDStep, nn.go:69-76) ────────────
__global__ void sgd_out_kernel(const float *p, const float *g, long n, float lr, float scale, float *out) {
    long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long stride = (long)gridDim.x * blockDim.x;
    for (; i < n; i += stride) out[i] = p[i] - lr * (scale * g[i]);
}

// ── MSE loss finalize: fixed-order sum of per-wave partials, f16 narrowing (lower.go:712), scale ───
__global__ __launch_bounds__(256) void mse_loss_kernel(const float *parts, long n, float scale, float *out) {
    __shared__ float red[256];
    float acc = 0.0f;
    for (long i = threadIdx.x; i < n; i += 256) acc += parts[i];
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
        __syncthreads();
    }
    if (threadIdx.x == 0) out[0] = q16(red[0]) * scale;
}

// ── host launchers ─────────────────────────────────────────────────────────────────────────────────

static unsigned grid_of(long n, int block, long cap = 1L << 20) {
    long g = (n + block - 1) / block;
    return (unsigned)(g < 1 ? 1 : g > cap ? cap : g);
}

hipError_t zero_fill(void *p, long bytes, hipStream_t s) {
    const long words = (bytes + 3) / 4;
    if (words <= 0) return hipSuccess;
    hipLaunchKernelGGL(zero_u32_kernel, dim3(grid_of(words, 256, 4096)), dim3(256), 0, s, (uint32_t *)p, words);
    return hipGetLastError();
}

hipError_t operand_prologue(const void *src, const void *z, bool f16, long n, void *dst, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (f16)
        hipLaunchKernelGGL(operand_prologue_kernel<half_t>, dim3(grid_of(n, 256, 8192)), dim3(256), 0, s, (const half_t *)src,
                           (const half_t *)z, n, (half_t *)dst);
    else
        hipLaunchKernelGGL(operand_prologue_kernel<float>, dim3(grid_of(n, 256, 8192)), dim3(256), 0, s, (const float *)src,
                           (const float *)z, n, (float *)dst);
    return hipGetLastError();
}

hipError_t operand_prologue_f32(const void *src, bool src_f16, const void *z, bool z_f16, int kind, long n, float *dst,
                                hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (kind < 1 || kind > 3 || (kind == 2 && !z)) return hipErrorInvalidValue;
    const dim3 grid(grid_of(n, 256, 8192)), block(256);
    if (src_f16 && z_f16)
        hipLaunchKernelGGL((operand_prologue_f32_kernel<half_t, half_t>), grid, block, 0, s, (const half_t *)src, (const half_t *)z, kind, n, dst);
    else if (src_f16)
        hipLaunchKernelGGL((operand_prologue_f32_kernel<half_t, float>), grid, block, 0, s, (const half_t *)src, (const float *)z, kind, n, dst);
    else if (z_f16)
        hipLaunchKernelGGL((operand_prologue_f32_kernel<float, half_t>), grid, block, 0, s, (const float *)src, (const half_t *)z, kind, n, dst);
    else
        hipLaunchKernelGGL((operand_prologue_f32_kernel<float, float>), grid, block, 0, s, (const float *)src, (const float *)z, kind, n, dst);
    return hipGetLastError();
}

hipError_t words_differ(const void *a, const void *b, long words, int *differs, hipStream_t s) {
    hipError_t e = zero_fill(differs, 4, s);
    if (e != hipSuccess || words <= 0) return e;
    hipLaunchKernelGGL(words_differ_kernel, dim3(grid_of(words, 256, 4096)), dim3(256), 0, s, (const uint32_t *)a,
                       (const uint32_t *)b, words, differs);
    return hipGetLastError();
}

long reduce_cols_workspace(int M, int N) { return (long)((M + kRedRows - 1) / kRedRows) * N; }

hipError_t reduce_rows(const void *G, bool f16, int M, int N, int op, float scale, float *out, hipStream_t s) {
    if (M <= 0) return hipSuccess;
    if (f16) hipLaunchKernelGGL(reduce_rows_kernel<half_t>, dim3((M + 3) / 4), dim3(256), 0, s, (const half_t *)G, M, N, op, scale, out);
    else hipLaunchKernelGGL(reduce_rows_kernel<float>, dim3((M + 3) / 4), dim3(256), 0, s, (const float *)G, M, N, op, scale, out);
    return hipGetLastError();
}

hipError_t reduce_cols(const void *G, bool f16, int M, int N, int op, float scale, float *work, float *out, hipStream_t s,
                       const void *Z, bool z_f16) {
    if (N <= 0) return hipSuccess;
    const int chunks = M > 0 ? (M + kRedRows - 1) / kRedRows : 0;
    const dim3 grid((N + 63) / 64, chunks), block(256);
    if (chunks > 0) {
        if (f16 && z_f16)
            hipLaunchKernelGGL((reduce_cols_partial_kernel<half_t, half_t>), grid, block, 0, s, (const half_t *)G, (const half_t *)Z, M, N, op, work);
        else if (f16)
            hipLaunchKernelGGL((reduce_cols_partial_kernel<half_t, float>), grid, block, 0, s, (const half_t *)G, (const float *)Z, M, N, op, work);
        else if (z_f16)
            hipLaunchKernelGGL((reduce_cols_partial_kernel<float, half_t>), grid, block, 0, s, (const float *)G, (const half_t *)Z, M, N, op, work);
        else
            hipLaunchKernelGGL((reduce_cols_partial_kernel<float, float>), grid, block, 0, s, (const float *)G, (const float *)Z, M, N, op, work);
    }
    hipLaunchKernelGGL(reduce_cols_final_kernel, dim3((N + 255) / 256), dim3(256), 0, s, work, chunks, N, op, scale, out);
    return hipGetLastError();
}

hipError_t maxpool_fwd(const float *X, long NC, int H, int W, int kH, int kW, int sH, int sW, float *out, hipStream_t s) {
    const int oH = (H - kH) / sH + 1, oW = (W - kW) / sW + 1;
    const long n = NC * oH * oW;
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(maxpool_fwd_kernel, dim3(grid_of(n, 256)), dim3(256), 0, s, X, NC, H, W, kH, kW, sH, sW, oH, oW, out);
    return hipGetLastError();
}

hipError_t maxpool_bwd(const float *X, const float *adj, long NC, int H, int W, int kH, int kW, int sH, int sW,
                       float *dX, hipStream_t s) {
    const int oH = (H - kH) / sH + 1, oW = (W - kW) / sW + 1;
    const long n = NC * H * W;
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(maxpool_bwd_kernel, dim3(grid_of(n, 256)), dim3(256), 0, s, X, adj, NC, H, W, kH, kW, sH, sW,
                       oH, oW, dX);
    return hipGetLastError();
}

hipError_t conv3x3_fwd(const float *X, int N, int Ci, int H, const float *w, const float *b, int Co, int relu, float *Y,
                       hipStream_t s) {
    const long n = (long)N * Co * H * H;
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(conv3x3_fwd_kernel, dim3(grid_of(n, 64)), dim3(64), 0, s, X, N, Ci, H, w, b, Co, relu, Y);
    return hipGetLastError();
}

hipError_t conv_bias_grad(const float *G, int N, int Co, int HW, float *db, hipStream_t s) {
    if (Co <= 0) return hipSuccess;
    hipLaunchKernelGGL(conv_bias_grad_kernel, dim3(Co), dim3(256), 0, s, G, N, Co, HW, db);
    return hipGetLastError();
}

hipError_t sgd_out(const float *p, const float *g, long n, float lr, float scale, float *out, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(sgd_out_kernel, dim3(grid_of(n, 256, 2048)), dim3(256), 0, s, p, g, n, lr, scale, out);
    return hipGetLastError();
}

hipError_t mse_loss(const float *parts, long n, float scale, float *out, hipStream_t s) {
    hipLaunchKernelGGL(mse_loss_kernel, dim3(1), dim3(256), 0, s, parts, n, scale, out);
    return hipGetLastError();
}

}  // namespace ah
