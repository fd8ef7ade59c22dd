// convnet.hip — the config-2 train step as two sample-parallel kernels (gfx950).
//
// conv1(1->C1) ReLU pool2 -> conv2(C1->C2) ReLU pool2 -> flatten -> Linear -> softmax-CE.
// Forward: workgroup (n, g) stages sample n's padded input in LDS, computes all of conv1 (cheap: one
// input channel) and conv2's output-channel group g, and the group's share of the logits. It stores
// the pooled planes, the per-window ReLU/argmax bytes (4 tie bits, 4 dead-ReLU bits; the conv outputs
// themselves never leave registers) and the partial logits.
// Backward: workgroup (n, c) owns conv1 channel c (conv2's input channel c). It sums the partial logits,
// evaluates softmax-CE, rebuilds dP2 and the padded conv2 output gradient of the whole sample in LDS
// (cheap), then computes conv2's input gradient for channel c, conv2's weight gradient for the pairs
// (all co, c), the pool/ReLU backward of channel c, and conv1's weight gradient for channel c. The
// sample's parameter gradients go to one row of `part`; the step's tail kernel sums the rows in sample
// order and applies SGD.
//
// The reference evaluates the same graph op by op (tensor/nn/nn.go:217-303 conv as im2col + matmul,
// nn.go:350-372 max-pool, gradient_ruleset.go:153-161 ReLU mask and :307-320 the tie split). The
// conv forward and input gradient keep the k = ci*9 + kh*3 + kw accumulation order of the per-op
// kernels in conv.hip, so they give the same bits; the weight gradients are summed per sample, then
// over samples.
#include <float.h>

#include "ah_common.h"
#include "convnet.h"
#include "softmax_row.h"

namespace ah {

constexpr int kFwdThreads = 512;
constexpr int kBwdThreads = 1024;
constexpr int kNetMaxNC = 16;   // the fc weights of a thread's feature stay in registers
constexpr int kFwdGroupCh = 4;  // conv2 output channels per forward workgroup

// A plane of `rows` rows in LDS: row stride ld, plane stride ps. ld = 2 (mod 8) and ps = 1 (mod 32)
// spread the lanes of a wave over the banks when they differ by channel and by a run of four rows
// (the weight-gradient sweep) or by 2x2 output block (the conv and input-gradient patches).
struct Plane {
    int ld, ps;
};
__host__ __device__ inline Plane net_plane(int rows, int width) {
    Plane p;
    p.ld = width + ((2 - width) % 8 + 8) % 8;
    p.ps = rows * p.ld + ((1 - rows * p.ld) % 32 + 32) % 32;
    return p;
}

__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// A filter's 9 taps, stored at a 16-byte aligned LDS address with a stride of 12 floats, read as three
// 16-byte loads (issued together, rather than one load and wait per tap).
#define WEIGHTS9(p)                                                                                      \
    {((const float4 *)(p))[0].x, ((const float4 *)(p))[0].y, ((const float4 *)(p))[0].z,                  \
     ((const float4 *)(p))[0].w, ((const float4 *)(p))[1].x, ((const float4 *)(p))[1].y,                  \
     ((const float4 *)(p))[1].z, ((const float4 *)(p))[1].w, ((const float4 *)(p))[2].x}

// conv3x3 (pad 1) + bias + ReLU (tagged) + 2x2 max-pool over zero-padded input planes. A wave owns an
// output channel (so the weights are wave-uniform) and a lane a pooling window: the window's four conv
// outputs share one 4x4 input patch per input channel. Weights w[c][ci][12] (taps 0-8), biases b[c].
// Pooled value -> out[c*out.ps + (ph+off)*out.ld +
// pw+off]; the window's tie and dead-ReLU bits -> mask[c*P*P + win].
__device__ void net_conv_pool(const float *in, Plane pin, int Ci, int H, const float *w, const float *b, int Co,
                              float *out, Plane pout, int off, uint8_t *mask, int nw) {
    const int P = H / 2, lane = threadIdx.x & 63;
    for (int c = wave_id(); c < Co; c += nw) {
        const float *wc = w + c * Ci * 12;
        const float bc = b[c];
        for (int win = lane; win < P * P; win += 64) {
            const int ph = win / P, pw = win % P;
            float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll 2
            for (int ci = 0; ci < Ci; ci++) {
                const float *xp = in + ci * pin.ps + 2 * ph * pin.ld + 2 * pw;
                float t[4][4];
#pragma unroll
                for (int r = 0; r < 4; r++)
#pragma unroll
                    for (int q = 0; q < 4; q++) t[r][q] = xp[r * pin.ld + q];
                const float wr[9] = WEIGHTS9(wc + ci * 12);
#pragma unroll
                for (int kh = 0; kh < 3; kh++)
#pragma unroll
                    for (int kw = 0; kw < 3; kw++) {
                        const float wt = wr[kh * 3 + kw];
                        a0 = a0 + t[kh][kw] * wt;
                        a1 = a1 + t[kh][kw + 1] * wt;
                        a2 = a2 + t[kh + 1][kw] * wt;
                        a3 = a3 + t[kh + 1][kw + 1] * wt;
                    }
            }
            const float hv[4] = {relu_tag(a0 + bc), relu_tag(a1 + bc), relu_tag(a2 + bc), relu_tag(a3 + bc)};
            float m = -FLT_MAX;
#pragma unroll
            for (int q = 0; q < 4; q++) m = fmaxf(m, hv[q]);
            unsigned bits = 0;
#pragma unroll
            for (int q = 0; q < 4; q++) bits |= ((hv[q] == m) ? 1u : 0u) << q | (relu_dead(hv[q]) ? 1u : 0u) << (4 + q);
            mask[c * P * P + win] = (uint8_t)bits;
            out[c * pout.ps + (ph + off) * pout.ld + pw + off] = m;
        }
    }
}

// Pool backward (equal split over tied maxima) fused with the ReLU mask, from the window bytes.
__device__ void net_pool_bwd(const float *dP, int C, int P, const uint8_t *mask, float *out, Plane pout, int off) {
    for (int i = threadIdx.x; i < C * P * P; i += blockDim.x) {
        const int c = i / (P * P), win = i % (P * P), ph = win / P, pw = win % P;
        const unsigned bits = mask[i];
        const float tie = (float)__builtin_popcount(bits & 15u);
        const float share = dP[i] * (1.0f / tie);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float g = ((bits >> q) & 1u) ? share : 0.0f;
            out[c * pout.ps + (2 * ph + (q >> 1) + off) * pout.ld + 2 * pw + (q & 1) + off] =
                ((bits >> (4 + q)) & 1u) ? 0.0f : g;
        }
    }
}

// The sum of a wave's 64 values, in every lane, in a fixed order: DPP within each row of 16 lanes
// (quad xor 1, quad xor 2, half-row mirror, row mirror), then the four row sums in order.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_total(float v) {
    v += dpp_mov<0xB1>(v);    // quad_perm [1,0,3,2]
    v += dpp_mov<0x4E>(v);    // quad_perm [2,3,0,1]
    v += dpp_mov<0x141>(v);   // row_half_mirror
    v += dpp_mov<0x140>(v);   // row_mirror
    const int b = __builtin_bit_cast(int, v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
    return (r0 + r1) + (r2 + r3);
}

// dX[y][x] = sum over (kh, kw) of (sum over co of G[co][y-kh+1][x-kw+1] * w[co][kh][kw]) for one input
// channel, G in zero-padded planes: the order of the per-op kernel. A lane owns one output; waves
// w0 .. w0+nw-1 take part. Weights w[co][12] (taps 0-8).
__device__ void net_conv_dx1(const float *G, Plane pg, int Co, int H, const float *w, float *dX, int w0, int nw) {
    const int wv = wave_id() - w0;
    if (wv < 0 || wv >= nw) return;
    for (int o = wv * 64 + (threadIdx.x & 63); o < H * H; o += nw * 64) {
        const int y = o / H, x = o % H;
        float p[9];
#pragma unroll
        for (int k = 0; k < 9; k++) p[k] = 0.0f;
        const float *gp = G + y * pg.ld + x;   // padded rows y..y+2 = G rows y-1..y+1
#pragma unroll 2
        for (int co = 0; co < Co; co++) {
            float t[3][3];
#pragma unroll
            for (int r = 0; r < 3; r++)
#pragma unroll
                for (int q = 0; q < 3; q++) t[r][q] = gp[co * pg.ps + r * pg.ld + q];
            const float wr[9] = WEIGHTS9(w + co * 12);
#pragma unroll
            for (int kh = 0; kh < 3; kh++)
#pragma unroll
                for (int kw = 0; kw < 3; kw++) p[kh * 3 + kw] = p[kh * 3 + kw] + t[2 - kh][2 - kw] * wr[kh * 3 + kw];
        }
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < 9; k++) acc += p[k];
        dX[o] = acc;
    }
}

// DPP sum over each row of 16 lanes (quad xor 1, quad xor 2, half-row mirror, row mirror); every lane
// of the row holds the row's sum.
__device__ __forceinline__ float row16_total(float v) {
    v += dpp_mov<0xB1>(v);
    v += dpp_mov<0x4E>(v);
    v += dpp_mov<0x141>(v);
    v += dpp_mov<0x140>(v);
    return v;
}

// Weight and bias gradients of one sample for Co output channels and one input channel:
// dW[co][tap] = sum_p G[co][p] * X[p + tap], db[co] = sum_p G[co][p], G[co][y][x] = G[co*pg.ps + y*pg.ld
// + x], X zero-padded. A block of Lb lanes (16 when H <= 16, else 64) owns a channel: lane b sweeps
// row b % Ry (Ry = 16 or 32) over column segment b / Ry with a sliding 3x3 window; the block's partial
// sums are combined in a fixed DPP order. Waves w0 .. w0+nw-1 take part. Results: dw[co * dw_stride +
// tap], and db[co] when db is not null.
__device__ void net_conv_dw_rows(const float *G, Plane pg, const float *X, Plane px, int H, int Co,
                                 float *__restrict__ dw, int dw_stride, float *__restrict__ db, int w0, int nw) {
    const int wv = wave_id() - w0, lane = threadIdx.x & 63;
    if (wv < 0 || wv >= nw) return;
    const int Lb = H <= 16 ? 16 : 64, Ry = H <= 16 ? 16 : 32, S = Lb / Ry, cols = (H + S - 1) / S;
    const int per_wave = 64 / Lb;
    for (int cb = wv * per_wave; cb < Co; cb += nw * per_wave) {   // wave-uniform loop
        const int b = lane % Lb, co = cb + lane / Lb, y = b % Ry, x0 = (b / Ry) * cols, x1 = min(H, x0 + cols);
        float acc[10];
#pragma unroll
        for (int k = 0; k < 10; k++) acc[k] = 0.0f;
        if (co < Co && y < H) {
            const float *xr = X + y * px.ld;   // padded rows y..y+2 are input rows y-1..y+1
            const float *gr = G + co * pg.ps + y * pg.ld;
            float c0[3], c1[3], c2[3];
#pragma unroll
            for (int k = 0; k < 3; k++) { c0[k] = xr[k * px.ld + x0]; c1[k] = xr[k * px.ld + x0 + 1]; }
            for (int x = x0; x < x1; x++) {
#pragma unroll
                for (int k = 0; k < 3; k++) c2[k] = xr[k * px.ld + x + 2];
                const float g = gr[x];
#pragma unroll
                for (int k = 0; k < 3; k++) {
                    acc[k * 3 + 0] += g * c0[k];
                    acc[k * 3 + 1] += g * c1[k];
                    acc[k * 3 + 2] += g * c2[k];
                }
                acc[9] += g;
#pragma unroll
                for (int k = 0; k < 3; k++) { c0[k] = c1[k]; c1[k] = c2[k]; }
            }
        }
#pragma unroll
        for (int k = 0; k < 10; k++) acc[k] = row16_total(acc[k]);
        if (Lb == 64) {
#pragma unroll
            for (int k = 0; k < 10; k++) {
                const int bits = __builtin_bit_cast(int, acc[k]);
                acc[k] = (__builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 0)) +
                          __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 16))) +
                         (__builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 32)) +
                          __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 48)));
            }
        }
        if (b < 10 && co < Co) {
            float mine = acc[0];
#pragma unroll
            for (int k = 1; k < 10; k++) mine = b == k ? acc[k] : mine;
            if (b < 9) dw[co * dw_stride + b] = mine;
            else if (db) db[co] = mine;
        }
    }
}

// ── the two kernels ─────────────────────────────────────────────────────────

// Global workspace between the kernels, offsets in floats (mask bytes packed four to a float).
struct NetWs {
    long p1, p2, lgp, m1, m2, total;
};
__host__ __device__ inline int net_groups(int C2) { return (C2 + kFwdGroupCh - 1) / kFwdGroupCh; }
__host__ __device__ inline NetWs net_ws(int N, int Hin, int C1, int C2, int NC) {
    const long P1 = Hin / 2, P2 = Hin / 4, F = (long)C2 * P2 * P2;
    NetWs w;
    long o = 0;
    w.p1 = o;  o += (long)N * C1 * P1 * P1;              // pooled conv1, [n][c][P1][P1]
    w.p2 = o;  o += (long)N * F;                         // pooled conv2 (the fc input), [n][F]
    w.lgp = o; o += (long)N * net_groups(C2) * NC;       // partial logits, [n][group][NC]
    w.m1 = o;  o += ((long)N * C1 * P1 * P1 + 3) / 4;    // conv1 window bytes, [n][c][P1*P1]
    w.m2 = o;  o += ((long)N * F + 3) / 4;               // conv2 window bytes, [n][F]
    w.total = o;
    return w;
}

// Forward LDS layout (floats; the mask bytes at the end).
struct FwdLayout {
    Plane px, p1;
    int xs, p1s, w1, w2, b1, b2, p2g, red, m1, total;
};
__host__ __device__ inline FwdLayout fwd_layout(int Hin, int C1) {
    const int P1 = Hin / 2, P2 = Hin / 4;
    FwdLayout L;
    L.px = net_plane(Hin + 2, Hin + 2);   // the input, zero-padded by one
    L.p1 = net_plane(P1 + 2, P1 + 2);     // pooled conv1, zero-padded by one (conv2's input)
    int o = 0;
    L.xs = o;  o += L.px.ps;
    L.p1s = o; o += C1 * L.p1.ps;
    o = (o + 3) & ~3;
    L.w1 = o;  o += C1 * 12;                          // conv1 weights [c][12]
    L.w2 = o;  o += kFwdGroupCh * C1 * 12;            // the group's conv2 weights [c][ci][12]
    L.b1 = o;  o += C1;
    L.b2 = o;  o += kFwdGroupCh;
    L.p2g = o; o += kFwdGroupCh * P2 * P2;            // the group's pooled conv2 planes
    L.red = o; o += kNetMaxNC * (kFwdThreads / 64);   // per-wave logit partials
    L.m1 = o;  o += (C1 * P1 * P1 + 3) / 4;
    L.total = o;
    return L;
}

__global__ __launch_bounds__(kFwdThreads) void convnet_fwd_kernel(
    const float *__restrict__ x, const float *__restrict__ cw1, const float *__restrict__ cb1,
    const float *__restrict__ cw2, const float *__restrict__ cb2, const float *__restrict__ fw, int Hin, int C1,
    int C2, int NC, float *__restrict__ ws) {
    extern __shared__ float lds[];
    constexpr int NW = kFwdThreads / 64;
    const int n = blockIdx.x, g = blockIdx.y, tid = threadIdx.x, lane = tid & 63, G = gridDim.y;
    const int P1 = Hin / 2, P2 = Hin / 4, F = C2 * P2 * P2;
    const int c0 = g * kFwdGroupCh, nc = min(C2, c0 + kFwdGroupCh) - c0, Fg = nc * P2 * P2, fbase = c0 * P2 * P2;
    const FwdLayout L = fwd_layout(Hin, C1);
    const NetWs W = net_ws(gridDim.x, Hin, C1, C2, NC);
    float *xs = lds + L.xs, *p1s = lds + L.p1s, *w1s = lds + L.w1, *w2s = lds + L.w2, *p2g = lds + L.p2g;
    uint8_t *m1s = (uint8_t *)(lds + L.m1);

    // the fc weights of this thread's feature, loaded now and used after the convolutions
    float fwv[kNetMaxNC];
#pragma unroll
    for (int k = 0; k < kNetMaxNC; k++) fwv[k] = (k < NC && tid < Fg) ? fw[(long)k * F + fbase + tid] : 0.0f;

    // every global load of the staging is issued before the first LDS store
    const float *xn = x + (long)n * Hin * Hin;
    float xv[3];
#pragma unroll
    for (int j = 0; j < 3; j++) {
        const int i = tid + j * kFwdThreads, yy = i / L.px.ld, xx = i % L.px.ld;
        const bool in = i < L.px.ps && yy >= 1 && yy <= Hin && xx >= 1 && xx <= Hin;
        xv[j] = in ? xn[(yy - 1) * Hin + xx - 1] : 0.0f;
    }
    const float w1v = tid < C1 * 9 ? cw1[tid] : 0.0f;
    const float w2v = tid < nc * C1 * 9 ? cw2[(long)c0 * C1 * 9 + tid] : 0.0f;
    const float b1v = tid < C1 ? cb1[tid] : 0.0f;
    const float b2v = tid < nc ? cb2[c0 + tid] : 0.0f;
#pragma unroll
    for (int j = 0; j < 3; j++)
        if (tid + j * kFwdThreads < L.px.ps) xs[tid + j * kFwdThreads] = xv[j];
    if (tid < C1 * 9) w1s[(tid / 9) * 12 + tid % 9] = w1v;
    if (tid < nc * C1 * 9) w2s[(tid / 9) * 12 + tid % 9] = w2v;
    if (tid < C1) lds[L.b1 + tid] = b1v;
    if (tid < nc) lds[L.b2 + tid] = b2v;
    for (int i = tid; i < C1 * L.p1.ps; i += kFwdThreads) p1s[i] = 0.0f;
    __syncthreads();

    net_conv_pool(xs, L.px, 1, Hin, w1s, lds + L.b1, C1, p1s, L.p1, 1, m1s, NW);
    __syncthreads();
    net_conv_pool(p1s, L.p1, C1, P1, w2s, lds + L.b2, nc, p2g, Plane{P2, P2 * P2}, 0,
                  (uint8_t *)(ws + W.m2) + (long)n * F + fbase, NW);
    if (g == 0) {   // conv1's pooled planes and window bytes, for the backward
        float *p1g = ws + W.p1 + (long)n * C1 * P1 * P1;
        for (int i = tid; i < C1 * P1 * P1; i += kFwdThreads) {
            const int c = i / (P1 * P1), y = (i / P1) % P1, xx = i % P1;
            p1g[i] = p1s[c * L.p1.ps + (y + 1) * L.p1.ld + xx + 1];
        }
        uint8_t *m1g = (uint8_t *)(ws + W.m1) + (long)n * C1 * P1 * P1;
        for (int i = tid; i < C1 * P1 * P1; i += kFwdThreads) m1g[i] = m1s[i];
    }
    __syncthreads();

    // the group's share of the logits: per-wave sums, then the waves in order
    const float pv = tid < Fg ? p2g[tid] : 0.0f;
    if (tid < Fg) ws[W.p2 + (long)n * F + fbase + tid] = pv;
    float v[kNetMaxNC];
#pragma unroll
    for (int k = 0; k < kNetMaxNC; k++) v[k] = k < NC ? wave_total(pv * fwv[k]) : 0.0f;
    float *red = lds + L.red;
    if (lane < NC) {
        float mine = v[0];
#pragma unroll
        for (int k = 1; k < kNetMaxNC; k++) mine = lane == k ? v[k] : mine;
        red[lane * NW + wave_id()] = mine;
    }
    __syncthreads();
    if (tid < NC) {
        float s = 0.0f;
        for (int q = 0; q < NW; q++) s += red[tid * NW + q];
        ws[W.lgp + ((long)n * G + g) * NC + tid] = s;
    }
}

// Backward LDS layout (floats; the mask bytes at the end).
struct BwdLayout {
    Plane px, p1, pz1;
    int xs, p1c, gs, p2, lg, dlg, dp1, z1, w2c, lgp, m2, m1, total;
};
__host__ __device__ inline BwdLayout bwd_layout(int Hin, int C1, int C2, int NC) {
    const int P1 = Hin / 2, P2 = Hin / 4;
    BwdLayout L;
    L.px = net_plane(Hin + 2, Hin + 2);
    L.p1 = net_plane(P1 + 2, P1 + 2);
    L.pz1 = net_plane(Hin, Hin);
    int o = 0;
    L.xs = o;  o += L.px.ps;                 // the input, zero-padded (conv1's weight gradient)
    L.p1c = o; o += L.p1.ps;                 // pooled conv1 channel c, zero-padded
    L.gs = o;  o += C2 * L.p1.ps;            // conv2's output gradient, zero-padded
    L.p2 = o;  o += C2 * P2 * P2;            // pooled conv2, then its gradient
    L.lg = o;  o += NC;
    L.dlg = o; o += NC;
    L.dp1 = o; o += P1 * P1;                 // gradient of pooled conv1 channel c
    L.z1 = o;  o += L.pz1.ps;                // conv1's output gradient, channel c
    o = (o + 3) & ~3;
    L.w2c = o; o += C2 * 12;                 // conv2 weights of input channel c, [co][12]
    L.lgp = o; o += net_groups(C2) * NC + NC + 1;   // partial logits, fc bias, label
    L.m2 = o;  o += (C2 * P2 * P2 + 3) / 4;
    L.m1 = o;  o += (P1 * P1 + 3) / 4;
    L.total = o;
    return L;
}

__global__ __launch_bounds__(kBwdThreads) void convnet_bwd_kernel(
    const float *__restrict__ x, const int32_t *__restrict__ lab, const float *__restrict__ cw2,
    const float *__restrict__ fw, const float *__restrict__ fb, int Hin, int C1, int C2, int NC, int G, float a,
    const float *__restrict__ ws, float *__restrict__ rowloss, float *__restrict__ part, long part_ld) {
    extern __shared__ float lds[];
    constexpr int NW = kBwdThreads / 64;
    const int n = blockIdx.x, c = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
    const int P1 = Hin / 2, P2 = Hin / 4, F = C2 * P2 * P2;
    const BwdLayout L = bwd_layout(Hin, C1, C2, NC);
    const NetWs W = net_ws(gridDim.x, Hin, C1, C2, NC);
    const NetPart O = net_part(Hin, C1, C2, NC);
    float *xs = lds + L.xs, *p1c = lds + L.p1c, *gs = lds + L.gs, *p2 = lds + L.p2, *lg = lds + L.lg;
    float *dlg = lds + L.dlg, *dp1 = lds + L.dp1, *z1 = lds + L.z1, *w2c = lds + L.w2c;
    uint8_t *m2 = (uint8_t *)(lds + L.m2), *m1 = (uint8_t *)(lds + L.m1);
    float *row = part + (long)n * part_ld;

    float fwv[kNetMaxNC];
#pragma unroll
    for (int k = 0; k < kNetMaxNC; k++) fwv[k] = (k < NC && tid < F) ? fw[(long)k * F + tid] : 0.0f;
    // every global load of the staging is issued before the first LDS store
    const float *xn = x + (long)n * Hin * Hin;
    const float *p1n = ws + W.p1 + ((long)n * C1 + c) * P1 * P1;
    const uint8_t *m2n = (const uint8_t *)(ws + W.m2) + (long)n * F;
    const uint8_t *m1n = (const uint8_t *)(ws + W.m1) + ((long)n * C1 + c) * P1 * P1;
    float xv[2], p1v, p2v, w2v, lgv = 0.0f;
    uint8_t m2v, m1v;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int i = tid + j * kBwdThreads, yy = i / L.px.ld, xx = i % L.px.ld;
        const bool in = i < L.px.ps && yy >= 1 && yy <= Hin && xx >= 1 && xx <= Hin;
        xv[j] = in ? xn[(yy - 1) * Hin + xx - 1] : 0.0f;
    }
    {
        const int yy = tid / L.p1.ld, xx = tid % L.p1.ld;
        const bool in = tid < L.p1.ps && yy >= 1 && yy <= P1 && xx >= 1 && xx <= P1;
        p1v = in ? p1n[(yy - 1) * P1 + xx - 1] : 0.0f;
    }
    p2v = tid < F ? ws[W.p2 + (long)n * F + tid] : 0.0f;
    m2v = tid < F ? m2n[tid] : 0;
    m1v = tid < P1 * P1 ? m1n[tid] : 0;
    w2v = tid < C2 * 9 ? cw2[((long)(tid / 9) * C1 + c) * 9 + tid % 9] : 0.0f;
    if (tid < G * NC) lgv = ws[W.lgp + (long)n * G * NC + tid];
    else if (tid < G * NC + NC) lgv = fb[tid - G * NC];
    else if (tid == G * NC + NC) lgv = __int_as_float(lab[n]);
#pragma unroll
    for (int j = 0; j < 2; j++)
        if (tid + j * kBwdThreads < L.px.ps) xs[tid + j * kBwdThreads] = xv[j];
    if (tid < L.p1.ps) p1c[tid] = p1v;
    if (tid < F) { p2[tid] = p2v; m2[tid] = m2v; }
    if (tid < P1 * P1) m1[tid] = m1v;
    if (tid < C2 * 9) w2c[(tid / 9) * 12 + tid % 9] = w2v;
    if (tid <= G * NC + NC) lds[L.lgp + tid] = lgv;
    for (int i = tid; i < C2 * L.p1.ps; i += kBwdThreads) gs[i] = 0.0f;
    __syncthreads();
    if (wave_id() == 0) {   // the logits: the groups' partial sums in order, then the bias
        const float *lgs = lds + L.lgp;
        for (int k = lane; k < NC; k += 64) {
            float v = 0.0f;
            for (int q = 0; q < G; q++) v += lgs[q * NC + k];
            lg[k] = v + lgs[G * NC + k];
        }
        const float rl = softmax_ce_row(lg, __float_as_int(lgs[G * NC + NC]), NC, a, dlg, lane);
        if (lane == 0 && c == 0) rowloss[n] = rl;
    }
    __syncthreads();

    // fc backward: dP2 in place of P2; this workgroup's slice of the sample's dfw row (rank one), dfb
    if (tid < F) {
        const float pv = p2[tid];
        const int Fs = (F + gridDim.y - 1) / gridDim.y;
        const bool mine = tid >= c * Fs && tid < (c + 1) * Fs;
        float d = 0.0f;
#pragma unroll
        for (int k = 0; k < kNetMaxNC; k++) {
            if (k >= NC) break;
            const float gk = dlg[k];
            if (mine) row[O.fw + (long)k * F + tid] = gk * pv;
            d += gk * fwv[k];
        }
        p2[tid] = d;
    }
    if (c == 0 && tid < NC) row[O.fb + tid] = dlg[tid];
    __syncthreads();

    net_pool_bwd(p2, C2, P2, m2, gs, L.p1, 1);   // dZ2 of the whole sample, padded
    __syncthreads();
    // conv2's input gradient for channel c (waves 0-3) beside its weight gradient for the pairs (co, c)
    net_conv_dx1(gs, L.p1, C2, P1, w2c, dp1, 0, 4);
    net_conv_dw_rows(gs + L.p1.ld + 1, L.p1, p1c, L.p1, P1, C2, row + O.cw2 + c * 9, C1 * 9, c == 0 ? row + O.cb2 : nullptr,
                     4, NW - 4);
    __syncthreads();
    net_pool_bwd(dp1, 1, P1, m1, z1, L.pz1, 0);   // dZ1 of channel c
    __syncthreads();
    net_conv_dw_rows(z1, L.pz1, xs, L.px, Hin, 1, row + O.cw1 + c * 9, 9, row + O.cb1 + c, 0, NW);
}

static size_t fwd_lds_bytes(int Hin, int C1) { return (size_t)fwd_layout(Hin, C1).total * sizeof(float); }
static size_t bwd_lds_bytes(int Hin, int C1, int C2, int NC) {
    return (size_t)bwd_layout(Hin, C1, C2, NC).total * sizeof(float);
}

bool convnet_fused_ok(int Hin, int C1, int C2, int NC) {
    if (Hin % 4 || Hin <= 0 || C1 <= 0 || C2 <= 0 || NC <= 0 || NC > kNetMaxNC) return false;
    const long P2 = Hin / 4, F = (long)C2 * P2 * P2;
    const BwdLayout B = bwd_layout(Hin, C1, C2, NC);
    const FwdLayout A = fwd_layout(Hin, C1);
    return F <= kBwdThreads && kFwdGroupCh * P2 * P2 <= kFwdThreads && B.px.ps <= 2 * kBwdThreads &&
           A.px.ps <= 3 * kFwdThreads && kFwdGroupCh * C1 * 9 <= kFwdThreads &&
           net_groups(C2) * NC + NC + 1 <= kBwdThreads &&
           B.p1.ps <= kBwdThreads && C2 * 9 <= kBwdThreads && fwd_lds_bytes(Hin, C1) <= 64 * 1024 &&
           bwd_lds_bytes(Hin, C1, C2, NC) <= 64 * 1024;
}
long convnet_fused_ws_floats(int N, int Hin, int C1, int C2, int NC) { return net_ws(N, Hin, C1, C2, NC).total; }

hipError_t convnet_fwd_fused(const float *x, const float *cw1, const float *cb1, const float *cw2, const float *cb2,
                             const float *fw, int B, int Hin, int C1, int C2, int NC, float *ws, hipStream_t s) {
    if (!convnet_fused_ok(Hin, C1, C2, NC) || B <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(convnet_fwd_kernel, dim3(B, net_groups(C2)), dim3(kFwdThreads), fwd_lds_bytes(Hin, C1), s, x,
                       cw1, cb1, cw2, cb2, fw, Hin, C1, C2, NC, ws);
    return hipGetLastError();
}

hipError_t convnet_bwd_fused(const float *x, const int32_t *lab, const float *cw2, const float *fw, const float *fb, int B,
                             int Hin, int C1, int C2, int NC, float a, const float *ws, float *rowloss, float *part,
                             hipStream_t s) {
    if (!convnet_fused_ok(Hin, C1, C2, NC) || B <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(convnet_bwd_kernel, dim3(B, C1), dim3(kBwdThreads), bwd_lds_bytes(Hin, C1, C2, NC), s, x, lab,
                       cw2, fw, fb, Hin, C1, C2, NC, net_groups(C2), a, ws, rowloss, part, net_part(Hin, C1, C2, NC).total);
    return hipGetLastError();
}

}  // namespace ah
