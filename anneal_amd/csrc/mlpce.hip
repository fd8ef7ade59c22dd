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
        // the parameters it updates and the row losses are loaded with the staged operands, so the
        // updates need no second round trip to memory
        constexpr int kW2Per = kMlpMaxC * kMlpMaxH / kMlpThreads;
        static_assert(kMlpMaxB <= 64 && kMlpMaxC <= kMlpThreads, "one row loss per lane of wave 0");
        float w2old[kW2Per];
#pragma unroll
        for (int u = 0; u < kW2Per; u++) w2old[u] = tid + u * kMlpThreads < C * H ? S.W2[tid + u * kMlpThreads] : 0.0f;
        const float b2old = tid < C ? S.b2[tid] : 0.0f;
        const float rl = tid < B ? rowloss[tid] : 0.0f;
        mlp_stage(hs, Hg, B * H);
        for (int i = tid; i < B * C; i += kMlpThreads) dzs[i] = dz[i];
        __syncthreads();
#pragma unroll
        for (int u = 0; u < kW2Per; u++) {
            const int o = tid + u * kMlpThreads;
            if (o >= C * H) break;
            const int c = o / H, j = o % H;
            float g = 0.0f;
            for (int n = 0; n < B; n++) g += dzs[n * C + c] * hs[n * H + j];
            if (S.gW2) S.gW2[o] = g;
            S.W2[o] = w2old[u] - S.lr * g;
        }
        if (tid < C) {
            float g = 0.0f;
            for (int n = 0; n < B; n++) g += dzs[n * C + tid];
            if (S.gb2) S.gb2[tid] = g;
            S.b2[tid] = b2old - S.lr * g;
        }
        if (tid < 64) {
            const float l = wave_sum(rl);
            if (tid == 0) S.loss[0] = l * S.loss_scale;
        }
        return;
    }
    const int ni = min(kGradCols, D - i0);
    // this thread's W1 entries (and workgroup 0's biases) loaded with the staged operands
    constexpr int kW1Per = kMlpMaxH * kGradCols / kMlpThreads;
    static_assert(kMlpMaxH <= kMlpThreads, "one hidden bias per thread");
    float w1old[kW1Per];
#pragma unroll
    for (int u = 0; u < kW1Per; u++) {
        const int o = tid + u * kMlpThreads, j = o / kGradCols, q = o % kGradCols;
        w1old[u] = j < H && q < ni ? S.W1[(long)j * D + i0 + q] : 0.0f;
    }
    const float b1old = blockIdx.x == 0 && tid < H ? S.b1[tid] : 0.0f;
    mlp_stage(hs, dH, B * H);
    for (int i = tid; i < B * kGradCols; i += kMlpThreads) {
        const int n = i / kGradCols, q = i % kGradCols;
        xt[i] = q < ni ? x[(long)n * D + i0 + q] : 0.0f;
    }
    __syncthreads();
    if (blockIdx.x == 0 && tid < H) {   // db1
        float g = 0.0f;
        for (int n = 0; n < B; n++) g += hs[n * H + tid];
        if (S.gb1) S.gb1[tid] = g;
        S.b1[tid] = b1old - S.lr * g;
    }
#pragma unroll
    for (int u = 0; u < kW1Per; u++) {   // W1[j][i0 + q]
        const int o = tid + u * kMlpThreads, j = o / kGradCols, q = o % kGradCols;
        if (j >= H || q >= ni) continue;
        float g = 0.0f;
        for (int n = 0; n < B; n++) g += hs[n * H + j] * xt[n * kGradCols + q];
        const long wi = (long)j * D + i0 + q;
        if (S.gW1) S.gW1[wi] = g;
        S.W1[wi] = w1old[u] - S.lr * g;
    }
}

// ── small batches at wide layers (config 4 at N <= 8) ──────────────────────
// Four kernels instead of the GEMM step's eight: the two linear layers as dots over 16 lanes, the
// hidden-layer gradient over column blocks of W2, and every weight gradient with its SGD update as
// one streaming pass over W1 and W2.

constexpr int kSmallB = 8, kSmallMaxC = 512;
constexpr int kSmallUnits = 8;    // hidden units per workgroup of the dH kernel
constexpr int kGradRows = 4;      // weight rows per thread of the small-batch gradient kernel

// out[n][j] = in[n] . W[j] + b[j] (ReLU, sign-tagged, when RELU): 8 samples x JT rows per workgroup,
// 16 lanes per output with 16-byte loads, 8 in flight per operand and lane. K % 4 == 0. A long K takes
// fewer rows per workgroup (JT = 2), so more CUs read W: a CU keeps only so many misses in flight.
template <bool RELU, int JT>
__global__ __launch_bounds__(128 * JT) void mlp_lin_kernel(const float *__restrict__ in, const float *__restrict__ W,
                                                           const float *__restrict__ b, int B, int K, int J,
                                                           float *__restrict__ out) {
    const int tid = threadIdx.x, o = tid / 16, ks = tid % 16;
    const int n = blockIdx.x * 8 + o / JT, j = blockIdx.y * JT + o % JT;
    const bool live = n < B && j < J;
    const float *ar = in + (long)(live ? n : 0) * K, *wr = W + (long)(live ? j : 0) * K;
    float acc = 0.0f;
    for (int k0 = 4 * ks; k0 < K; k0 += 4 * 16 * 8) {
        floatx4 av[8], wv[8];
#pragma unroll
        for (int m = 0; m < 8; m++) {
            const int k = k0 + 64 * m;
            const bool ok = live && k < K;
            av[m] = ok ? *(const floatx4 *)(ar + k) : (floatx4){};
            wv[m] = ok ? *(const floatx4 *)(wr + k) : (floatx4){};
        }
#pragma unroll
        for (int m = 0; m < 8; m++)
#pragma unroll
            for (int u = 0; u < 4; u++) acc += av[m][u] * wv[m][u];
    }
    acc = mlp_row16(acc);
    if (ks == 0 && live) {
        const float z = acc + b[j];
        out[(long)n * J + j] = RELU ? relu_tag(z) : z;
    }
}

// Softmax-CE of every sample (each workgroup; workgroup 0 writes dz and rowloss), then dH for the
// kSmallUnits (U) hidden units [U * blockIdx.x, +U): wave w takes a share of the classes, its lane
// (j, s) the classes c0 + s, c0 + s + 64 / U, ... of that share for hidden unit j (64 / U rows of 4U
// bytes per load; all of a lane's W2 loads in flight at once), the lanes of a unit are added by
// shuffles, the waves' sums in wave order, and the ReLU mask applied. Few units per workgroup spread
// W2's reads over H / U workgroups: a CU keeps only so many misses in flight, so the read rate grows
// with the CUs reading.
__global__ __launch_bounds__(kMlpThreads) void mlp_small_dh_kernel(const int32_t *__restrict__ lab,
                                                                   const float *__restrict__ Z,
                                                                   const float *__restrict__ Hg,
                                                                   const float *__restrict__ W2, int B, int H, int C,
                                                                   float a, float *__restrict__ dz,
                                                                   float *__restrict__ dH,
                                                                   float *__restrict__ rowloss) {
    constexpr int NW = kMlpThreads / 64, SUBS = 64 / kSmallUnits;   // waves; lanes per hidden unit
    constexpr int CW = kSmallMaxC / NW / SUBS;                       // classes per lane, at most
    __shared__ float dzs[kSmallB * kSmallMaxC];
    __shared__ float zr[NW * kSmallB * 64];   // the logits, then the per-wave sums
    float *zs = zr;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, jl = lane % kSmallUnits, sub = lane / kSmallUnits;
    const int j = blockIdx.x * kSmallUnits + jl;
    const int cw = (C + NW - 1) / NW, c0 = w * cw, c1 = min(C, c0 + cw);
    float wv[CW];   // W2[c][j] for this lane's classes c = c0 + sub + SUBS * q
#pragma unroll
    for (int q = 0; q < CW; q++) {
        const int c = c0 + sub + SUBS * q;
        wv[q] = (c < c1 && j < H) ? W2[(long)c * H + j] : 0.0f;
    }
    // this thread's activation for the ReLU mask at the end (thread n * U + u: sample n, unit u)
    const int mn = tid / kSmallUnits, mj = blockIdx.x * kSmallUnits + tid % kSmallUnits;
    const bool mlive = tid < B * kSmallUnits && mj < H;
    const float hact = mlive ? Hg[(long)mn * H + mj] : 0.0f;
    static_assert(kMlpThreads / 64 >= kSmallB, "one wave per sample's softmax-CE");
    const int mylab = w < B ? lab[w] : 0;   // wave w's sample's label, loaded with everything else
    // the logits into LDS, every thread's loads in flight together
    static_assert(kSmallB * kSmallMaxC <= 4 * kMlpThreads, "logit staging is 4 values per thread");
    float zl[4];
#pragma unroll
    for (int u = 0; u < 4; u++) zl[u] = tid + u * kMlpThreads < B * C ? Z[tid + u * kMlpThreads] : 0.0f;
#pragma unroll
    for (int u = 0; u < 4; u++)
        if (tid + u * kMlpThreads < B * C) zs[tid + u * kMlpThreads] = zl[u];
    __syncthreads();
    if (w < B) {   // the row from LDS into registers once (the same sums, in the same order, as softmax_ce_row)
        constexpr int VPR = kSmallMaxC / 64;
        float v[VPR], unused[VPR] = {};
        softmax_ce_row_load<VPR>(zs + w * C, C, lane, v);
        const float r = softmax_ce_row_regs<VPR>(v, zs + w * C, mylab, C, a, dzs + w * C, lane, unused);
        if (blockIdx.x == 0 && lane == 0) rowloss[w] = r;
    }
    __syncthreads();
    if (blockIdx.x == 0)
        for (int i = tid; i < B * C; i += kMlpThreads) dz[i] = dzs[i];
    float acc[kSmallB];
#pragma unroll
    for (int n = 0; n < kSmallB; n++) {
        acc[n] = 0.0f;
        if (n < B)
#pragma unroll
            for (int q = 0; q < CW; q++) {
                const int c = c0 + sub + SUBS * q;
                if (c < c1) acc[n] += dzs[n * C + c] * wv[q];
            }
#pragma unroll
        for (int o = kSmallUnits; o < 64; o <<= 1) acc[n] += __shfl_xor(acc[n], o);
    }
    if (sub == 0)
#pragma unroll
        for (int n = 0; n < kSmallB; n++) zr[(w * kSmallB + n) * kSmallUnits + jl] = acc[n];
    __syncthreads();
    if (mlive) {
        const int u = tid % kSmallUnits;
        float g = 0.0f;
        for (int q = 0; q < NW; q++) g += zr[(q * kSmallB + mn) * kSmallUnits + u];
        dH[(long)mn * H + mj] = relu_dead(hact) ? 0.0f : g;
    }
}

// dW1 = dH^T x and dW2 = dz^T H over the batch, with SGD, one float4 column chunk of kGradRows rows of W1
// or W2 per thread; the workgroups after those take the biases (one per thread) and the loss.
__global__ __launch_bounds__(256) void mlp_small_grad_kernel(const float *__restrict__ x, const float *__restrict__ Hg,
                                                             const float *__restrict__ dz, const float *__restrict__ dH,
                                                             const float *__restrict__ rowloss, int B, int D, int H,
                                                             int C, MlpSgd S) {
    // Weight units: kGradRows rows x one float4 column chunk (W1: rows j of H, chunks of D; W2: rows c of
    // C, chunks of H), so each activation chunk loaded serves kGradRows rows. H % 4 == 0 (mlp_small_ok),
    // so W1's rows divide; W2's last unit may hold fewer than kGradRows rows.
    const long n1 = (long)(H / kGradRows) * (D / 4), n2 = (long)((C + kGradRows - 1) / kGradRows) * (H / 4);
    const long nwb = (n1 + n2 + 255) / 256;   // workgroups for the weights; then (H + C) / 256 for the biases
    const long u = (long)blockIdx.x * 256 + threadIdx.x;
    if (blockIdx.x >= nwb) {   // one bias per thread (b1 then b2), its batch's terms loaded together; the loss
        const int t = (int)(blockIdx.x - nwb) * 256 + threadIdx.x;
        if (t < H + C) {
            const bool hid = t < H;
            const float *src = hid ? dH + t : dz + (t - H);
            const long ld = hid ? H : C;
            float d[kSmallB];
#pragma unroll
            for (int n = 0; n < kSmallB; n++) d[n] = n < B ? src[n * ld] : 0.0f;
            float g = 0.0f;
#pragma unroll
            for (int n = 0; n < kSmallB; n++)
                if (n < B) g += d[n];
            float *bp = hid ? S.b1 + t : S.b2 + (t - H);
            float *gb = hid ? S.gb1 : S.gb2;
            if (gb) gb[hid ? t : t - H] = g;
            *bp = *bp - S.lr * g;
        }
        if (blockIdx.x == nwb && threadIdx.x < 64) {
            float l = 0.0f;
            for (int n = threadIdx.x; n < B; n += 64) l += rowloss[n];
            l = wave_sum(l);
            if (threadIdx.x == 0) S.loss[0] = l * S.loss_scale;
        }
        return;
    }
    const float *act, *adj;
    float *Wp, *gp;
    int row0, nrows, i, len, ald, jld;
    if (u < n1) {   // W1[j][i .. i+3] += over n: dH[n][j] * x[n][i .. i+3]
        const int per = D / 4, v = (int)u;
        row0 = kGradRows * (v / per); i = 4 * (v % per);
        nrows = H; len = D; act = x; ald = D; adj = dH; jld = H; Wp = S.W1; gp = S.gW1;
    } else if (u < n1 + n2) {   // W2[c][j .. j+3] += over n: dz[n][c] * H[n][j .. j+3]
        const int per = H / 4, v = (int)(u - n1);
        row0 = kGradRows * (v / per); i = 4 * (v % per);
        nrows = C; len = H; act = Hg; ald = H; adj = dz; jld = C; Wp = S.W2; gp = S.gW2;
    } else {
        return;
    }
    floatx4 v[kSmallB], wold[kGradRows];
    float sc[kGradRows][kSmallB];
#pragma unroll
    for (int n = 0; n < kSmallB; n++) v[n] = n < B ? *(const floatx4 *)(act + (long)n * ald + i) : (floatx4){};
#pragma unroll
    for (int r = 0; r < kGradRows; r++) {
        const bool ok = row0 + r < nrows;
        wold[r] = ok ? *(const floatx4 *)(Wp + (long)(row0 + r) * len + i) : (floatx4){};
#pragma unroll
        for (int n = 0; n < kSmallB; n++) sc[r][n] = ok && n < B ? adj[(long)n * jld + row0 + r] : 0.0f;
    }
#pragma unroll
    for (int r = 0; r < kGradRows; r++) {
        if (row0 + r >= nrows) break;
        floatx4 g = {};
#pragma unroll
        for (int n = 0; n < kSmallB; n++) g += sc[r][n] * v[n];
        const long e = (long)(row0 + r) * len + i;
        if (gp) *(floatx4 *)(gp + e) = g;
        *(floatx4 *)(Wp + e) = wold[r] - S.lr * g;
    }
}

bool mlp_small_ok(int B, int D, int H, int C) {
    return B > 0 && B <= kSmallB && D % 4 == 0 && H % 4 == 0 && C > 0 && C <= kSmallMaxC;
}

hipError_t mlp_small_step(const float *x, const int32_t *lab, int B, int D, int H, int C, float a, float *Hbuf,
                          float *Z, float *dz, float *dH, float *rowloss, const MlpSgd &S, hipStream_t s, int part) {
    if (!mlp_small_ok(B, D, H, C)) return hipErrorInvalidValue;
    switch (part) {
        case 0:
            if (D >= 1024)
                hipLaunchKernelGGL((mlp_lin_kernel<true, 2>), dim3((B + 7) / 8, (H + 1) / 2), dim3(256), 0, s, x, S.W1,
                                   S.b1, B, D, H, Hbuf);
            else
                hipLaunchKernelGGL((mlp_lin_kernel<true, 8>), dim3((B + 7) / 8, (H + 7) / 8), dim3(1024), 0, s, x, S.W1,
                                   S.b1, B, D, H, Hbuf);
            break;
        case 1:
            if (H >= 1024)
                hipLaunchKernelGGL((mlp_lin_kernel<false, 2>), dim3((B + 7) / 8, (C + 1) / 2), dim3(256), 0, s, Hbuf,
                                   S.W2, S.b2, B, H, C, Z);
            else
                hipLaunchKernelGGL((mlp_lin_kernel<false, 8>), dim3((B + 7) / 8, (C + 7) / 8), dim3(1024), 0, s, Hbuf,
                                   S.W2, S.b2, B, H, C, Z);
            break;
        case 2:
            hipLaunchKernelGGL(mlp_small_dh_kernel, dim3((H + kSmallUnits - 1) / kSmallUnits), dim3(kMlpThreads), 0, s, lab, Z, Hbuf, S.W2, B,
                               H, C, a, dz, dH, rowloss);
            break;
        default: {
            const long units = (long)(H / kGradRows) * (D / 4) + (long)((C + kGradRows - 1) / kGradRows) * (H / 4);
            const unsigned nb = (unsigned)((H + C + 255) / 256);
            hipLaunchKernelGGL(mlp_small_grad_kernel, dim3((unsigned)((units + 255) / 256) + nb), dim3(256), 0, s, x, Hbuf,
                               dz, dH, rowloss, B, D, H, C, S);
        }
    }
    return hipGetLastError();
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
