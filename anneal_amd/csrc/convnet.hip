// convnet.hip — the config-2 train step of one sample in one workgroup (gfx950).
//
// conv1(1->C1) ReLU pool2 -> conv2(C1->C2) ReLU pool2 -> flatten -> Linear -> softmax-CE, forward and
// backward, with every intermediate of the sample resident in LDS: the padded input, the padded
// pooled conv1 planes, the pooled conv2 vector (reused for its gradient), the logits, the padded conv2
// output gradient (reused for the conv1 output gradient) and conv1's pooled gradient. A pooling
// window's ReLU/argmax facts are kept as one byte (4 tie bits, 4 dead-ReLU bits), so the conv outputs
// themselves never leave registers. The sample's parameter gradients go to one row of `part`; the
// step's tail kernel sums the rows in sample order and applies SGD.
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

constexpr int kNetThreads = 1024;
constexpr int kNetMaxNC = 16;   // the fc weights of a thread's feature stay in registers
constexpr int kNetWaves = kNetThreads / 64;

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

// LDS layout, in floats (the mask bytes at the end). Host and device evaluate the same function.
struct NetLayout {
    Plane px, p1, pz1;
    int xs, p1s, p2s, lg, dlg, red, gs, dp1s, w1, w2, masks, total;
};
__host__ __device__ inline NetLayout net_layout(int Hin, int C1, int C2, int NC) {
    const int P1 = Hin / 2, P2 = Hin / 4;
    NetLayout L;
    L.px = net_plane(Hin + 2, Hin + 2);   // the input, zero-padded by one
    L.p1 = net_plane(P1 + 2, P1 + 2);     // pooled conv1 (conv2's input) and dZ2, zero-padded by one
    L.pz1 = net_plane(Hin, Hin);          // dZ1
    int o = 0;
    L.xs = o;    o += L.px.ps;
    L.p1s = o;   o += C1 * L.p1.ps;
    L.p2s = o;   o += C2 * P2 * P2;            // pooled conv2 (= the fc input), then its gradient
    L.lg = o;    o += NC;
    L.dlg = o;   o += NC;
    L.red = o;   o += kNetMaxNC * kNetWaves;   // per-wave logit partials
    L.gs = o;    o += (C2 * L.p1.ps > C1 * L.pz1.ps) ? C2 * L.p1.ps : C1 * L.pz1.ps;   // dZ2, then dZ1
    L.dp1s = o;  o += C1 * P1 * P1;            // gradient of pooled conv1
    L.w1 = o;    o += C1 * 9 + C1;             // conv weights and biases (read wave-uniform: LDS broadcasts)
    L.w2 = o;    o += C2 * C1 * 9 + C2;
    L.masks = o; o += (C1 * P1 * P1 + C2 * P2 * P2 + 3) / 4;
    L.total = o;
    return L;
}

__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// conv3x3 (pad 1) + bias + ReLU (tagged) + 2x2 max-pool over zero-padded input planes. A wave owns an
// output channel (so the weights are wave-uniform) and a lane a pooling window: the window's four conv
// outputs share one 4x4 input patch per input channel. Pooled value -> out[c*out.ps + (ph+off)*out.ld +
// pw+off]; the window's tie and dead-ReLU bits -> mask[c*P*P + win].
__device__ void net_conv_pool(const float *in, Plane pin, int Ci, int H, const float *w, const float *b, int Co,
                              float *out, Plane pout, int off, uint8_t *mask) {
    const int P = H / 2, lane = threadIdx.x & 63;
    for (int c = wave_id(); c < Co; c += kNetWaves) {
        const float *wc = w + c * Ci * 9;
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
#pragma unroll
                for (int kh = 0; kh < 3; kh++)
#pragma unroll
                    for (int kw = 0; kw < 3; kw++) {
                        const float wt = wc[ci * 9 + kh * 3 + kw];
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
    for (int i = threadIdx.x; i < C * P * P; i += kNetThreads) {
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

// dX[ci][y][x] = sum over (kh, kw) of (sum over co of G[co][y-kh+1][x-kw+1] * w[co][ci][kh][kw]), G in
// zero-padded planes. A wave (of the first nw) owns an input channel, a lane a 2x2 output block (one 4x4
// G patch per co).
__device__ void net_conv_dx(const float *G, Plane pg, int Co, int H, const float *w, int Ci, float *dX, int nw) {
    const int Q = H / 2, lane = threadIdx.x & 63;
    if (wave_id() >= nw) return;
    for (int ci = wave_id(); ci < Ci; ci += nw)
        for (int blk = lane; blk < Q * Q; blk += 64) {
            const int by = blk / Q, bx = blk % Q;
            float p[4][9];
#pragma unroll
            for (int q = 0; q < 4; q++)
#pragma unroll
                for (int k = 0; k < 9; k++) p[q][k] = 0.0f;
#pragma unroll 2
            for (int co = 0; co < Co; co++) {
                const float *gp = G + co * pg.ps + 2 * by * pg.ld + 2 * bx;
                float t[4][4];
#pragma unroll
                for (int r = 0; r < 4; r++)
#pragma unroll
                    for (int q = 0; q < 4; q++) t[r][q] = gp[r * pg.ld + q];
                const float *wc = w + (co * Ci + ci) * 9;
#pragma unroll
                for (int kh = 0; kh < 3; kh++)
#pragma unroll
                    for (int kw = 0; kw < 3; kw++) {
                        const float wt = wc[kh * 3 + kw];
#pragma unroll
                        for (int q = 0; q < 4; q++)
                            p[q][kh * 3 + kw] = p[q][kh * 3 + kw] + t[(q >> 1) - kh + 2][(q & 1) - kw + 2] * wt;
                    }
            }
#pragma unroll
            for (int q = 0; q < 4; q++) {
                float acc = 0.0f;
#pragma unroll
                for (int k = 0; k < 9; k++) acc += p[q][k];
                dX[ci * H * H + (2 * by + (q >> 1)) * H + 2 * bx + (q & 1)] = acc;
            }
        }
}

// One sample's weight and bias gradients: dW[co][ci][tap] = sum_p G[co][p] * X[ci][p + tap] and
// db[co] = sum_p G[co][p]. G[co][y][x] = G[co*pg.ps + y*pg.ld + x]; X in zero-padded planes. Each
// (co, ci) pair is split over RS = R*S consecutive lanes (R row ranges times S column ranges), each
// lane sweeping a 3x3 window along its part of the rows; the RS partial sums are combined with a fixed
// shuffle tree. Waves w0 .. w0+nw-1 take part.
__device__ void net_conv_dw(const float *G, Plane pg, const float *X, Plane px, int Ci, int H, int Co,
                            float *__restrict__ dw, float *__restrict__ db, int w0, int nw) {
    const int lane = threadIdx.x & 63, pairs = Co * Ci, wv = wave_id() - w0;
    if (wv < 0 || wv >= nw) return;
    int R = 1, S = 1;
    while (R * S < 64 && pairs * R * S * 2 <= nw * 64) {   // rows first, then columns
        if (R * 2 <= H) R *= 2;
        else if (S * 2 <= H / 4) S *= 2;
        else break;
    }
    const int RS = R * S, rows = (H + R - 1) / R, cols = (H + S - 1) / S;
    for (int base = wv * 64; base < pairs * RS; base += nw * 64) {
        const int item = base + lane, pair = item / RS, r = (item % RS) / S, sc = item % S;
        const bool live = item < pairs * RS;
        const int co = live ? pair / Ci : 0, ci = live ? pair % Ci : 0;
        float acc[10];
#pragma unroll
        for (int k = 0; k < 10; k++) acc[k] = 0.0f;
        const int y0 = live ? r * rows : H, y1 = min(H, y0 + rows);
        const int x0 = sc * cols, x1 = min(H, x0 + cols);
        for (int y = y0; y < y1; y++) {
            const float *xr = X + ci * px.ps + y * px.ld;   // padded rows y..y+2 are input rows y-1..y+1
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
        for (int o = RS / 2; o >= 1; o >>= 1)
#pragma unroll
            for (int k = 0; k < 10; k++) acc[k] += __shfl_xor(acc[k], o, 64);
        if (live && item % RS == 0) {
#pragma unroll
            for (int k = 0; k < 9; k++) dw[pair * 9 + k] = acc[k];
            if (ci == 0) db[co] = acc[9];
        }
    }
}

__global__ __launch_bounds__(kNetThreads) void convnet_step_kernel(
    const float *__restrict__ x, const int32_t *__restrict__ lab, const float *__restrict__ cw1,
    const float *__restrict__ cb1, const float *__restrict__ cw2, const float *__restrict__ cb2,
    const float *__restrict__ fw, const float *__restrict__ fb, int Hin, int C1, int C2, int NC, float a,
    float *__restrict__ rowloss, float *__restrict__ part, long part_ld) {
    extern __shared__ float lds[];
    const int n = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    const int P1 = Hin / 2, P2 = Hin / 4, F = C2 * P2 * P2;
    const NetLayout L = net_layout(Hin, C1, C2, NC);
    float *xs = lds + L.xs, *p1s = lds + L.p1s, *p2s = lds + L.p2s, *lg = lds + L.lg, *dlg = lds + L.dlg;
    float *gs = lds + L.gs, *dp1s = lds + L.dp1s, *w1s = lds + L.w1, *w2s = lds + L.w2;
    uint8_t *m1 = (uint8_t *)(lds + L.masks), *m2 = m1 + C1 * P1 * P1;
    const NetPart O = net_part(Hin, C1, C2, NC);
    float *row = part + (long)n * part_ld;

    // the fc weights of this thread's feature f = tid, and the label, are loaded now and used after the
    // convolutions
    float fwv[kNetMaxNC];
#pragma unroll
    for (int k = 0; k < kNetMaxNC; k++) fwv[k] = (k < NC && tid < F) ? fw[(long)k * F + tid] : 0.0f;
    const int label = lab[n];

    // stage the padded input and the conv parameters; clear the planes whose borders must read as zero
    const float *xn = x + (long)n * Hin * Hin;
    const int W1 = Hin + 2;
    for (int i = tid; i < W1 * W1; i += kNetThreads) {
        const int yy = i / W1, xx = i % W1;
        const bool in = yy >= 1 && yy <= Hin && xx >= 1 && xx <= Hin;
        xs[yy * L.px.ld + xx] = in ? xn[(yy - 1) * Hin + xx - 1] : 0.0f;
    }
    for (int i = tid; i < C1 * L.p1.ps; i += kNetThreads) p1s[i] = 0.0f;
    for (int i = tid; i < C2 * L.p1.ps; i += kNetThreads) gs[i] = 0.0f;
    for (int i = tid; i < C1 * 9; i += kNetThreads) w1s[i] = cw1[i];
    for (int i = tid; i < C1; i += kNetThreads) w1s[C1 * 9 + i] = cb1[i];
    for (int i = tid; i < C2 * C1 * 9; i += kNetThreads) w2s[i] = cw2[i];
    for (int i = tid; i < C2; i += kNetThreads) w2s[C2 * C1 * 9 + i] = cb2[i];
    __syncthreads();

    net_conv_pool(xs, L.px, 1, Hin, w1s, w1s + C1 * 9, C1, p1s, L.p1, 1, m1);
    __syncthreads();
    net_conv_pool(p1s, L.p1, C1, P1, w2s, w2s + C2 * C1 * 9, C2, p2s, Plane{P2, P2 * P2}, 0, m2);
    __syncthreads();

    // fc: thread f multiplies its feature into every logit; per-wave sums, then the waves in order
    {
        const float pv = tid < F ? p2s[tid] : 0.0f;
        float *red = lds + L.red;
        float v[kNetMaxNC];   // all logits' shuffle trees in flight together (fwv[k] = 0 for k >= NC)
#pragma unroll
        for (int k = 0; k < kNetMaxNC; k++) v[k] = pv * fwv[k];
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1)
#pragma unroll
            for (int k = 0; k < kNetMaxNC; k++) v[k] += __shfl_xor(v[k], o, 64);
        if (lane < NC) {
            float mine = v[0];
#pragma unroll
            for (int k = 1; k < kNetMaxNC; k++) mine = lane == k ? v[k] : mine;
            red[lane * kNetWaves + wave_id()] = mine;
        }
        __syncthreads();
        if (tid < NC) {
            float v = 0.0f;
            for (int q = 0; q < kNetWaves; q++) v += red[tid * kNetWaves + q];
            lg[tid] = v + fb[tid];
        }
        __syncthreads();
        if (wave_id() == 0) {
            const float rl = softmax_ce_row(lg, label, NC, a, dlg, lane);
            if (lane == 0) rowloss[n] = rl;
        }
        __syncthreads();
        // fc backward: this sample's dfw row (rank one) and dfb, and dP2 in place of P2
        if (tid < F) {
            float d = 0.0f;
#pragma unroll
            for (int k = 0; k < kNetMaxNC; k++) {
                if (k >= NC) break;
                const float g = dlg[k];
                row[O.fw + (long)k * F + tid] = g * pv;
                d += g * fwv[k];
            }
            p2s[tid] = d;
        }
        if (tid < NC) row[O.fb + tid] = dlg[tid];
    }
    __syncthreads();

    net_pool_bwd(p2s, C2, P2, m2, gs, L.p1, 1);   // dZ2, padded
    __syncthreads();
    {   // the input gradient and the weight gradient of conv2 side by side, on disjoint waves
        const int nx = C1 < kNetWaves / 2 ? C1 : kNetWaves / 2;
        net_conv_dx(gs, L.p1, C2, P1, w2s, C1, dp1s, nx);
        net_conv_dw(gs + L.p1.ld + 1, L.p1, p1s, L.p1, C1, P1, C2, row + O.cw2, row + O.cb2, nx, kNetWaves - nx);
    }
    __syncthreads();
    net_pool_bwd(dp1s, C1, P1, m1, gs, L.pz1, 0);   // dZ1 over dZ2's space
    __syncthreads();
    net_conv_dw(gs, L.pz1, xs, L.px, 1, Hin, C1, row + O.cw1, row + O.cb1, 0, kNetWaves);
}

size_t convnet_fused_lds_bytes(int Hin, int C1, int C2, int NC) {
    return (size_t)net_layout(Hin, C1, C2, NC).total * sizeof(float);
}
bool convnet_fused_ok(int Hin, int C1, int C2, int NC) {
    const long F = (long)C2 * (Hin / 4) * (Hin / 4);
    return Hin % 4 == 0 && Hin > 0 && C1 > 0 && C2 > 0 && NC > 0 && NC <= kNetMaxNC && F <= kNetThreads &&
           convnet_fused_lds_bytes(Hin, C1, C2, NC) <= 64 * 1024;
}

hipError_t convnet_step_fused(const float *x, const int32_t *lab, const float *cw1, const float *cb1, const float *cw2,
                              const float *cb2, const float *fw, const float *fb, int B, int Hin, int C1, int C2, int NC,
                              float a, float *rowloss, float *part, hipStream_t s) {
    if (!convnet_fused_ok(Hin, C1, C2, NC) || B <= 0) return hipErrorInvalidValue;
    const NetPart O = net_part(Hin, C1, C2, NC);
    hipLaunchKernelGGL(convnet_step_kernel, dim3(B), dim3(kNetThreads), convnet_fused_lds_bytes(Hin, C1, C2, NC), s, x,
                       lab, cw1, cb1, cw2, cb2, fw, fb, Hin, C1, C2, NC, a, rowloss, part, O.total);
    return hipGetLastError();
}

}  // namespace ah
