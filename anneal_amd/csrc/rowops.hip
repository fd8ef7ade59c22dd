// rowops.hip — row reductions, loss-gradient epilogues and small elementwise kernels (gfx950).
//
// Softmax cross-entropy: one wave64 per row, shuffle reductions for the row max, the tie count and
// the exp-sum; the backward follows the reference's op-by-op rules so the gradient through the row
// max (tensor/gradient_ruleset.go:307-320, no stop-gradient in the reference) is reproduced.
//
// Movement chain (config 5): two streaming passes over X in its stored [R, Cc] layout. A Y-row is an
// X-column, so lanes own columns and walk rows: every wave load is a contiguous 1 KiB row segment
// (float4 per lane) and no transpose is ever materialized. Pass 1 keeps online (max, tie count,
// sum e, sum e^2) per column; a per-column finalize folds the row chunks and evaluates the
// backward's per-row scalars; pass 2 re-reads X and writes dX in the same layout.
#include <float.h>

#include <algorithm>
#include <mutex>

#include "ah_common.h"
#include "rowops.h"
#include "softmax_row.h"

namespace ah {

// ── small elementwise kernels ───────────────────────────────────────────────

__global__ void fill_f32_kernel(float *p, long n, float v) {
    long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    long stride = (long)gridDim.x * blockDim.x;
    for (; i < n; i += stride) p[i] = v;
}

// amp * u, u uniform in [-1, 1) from a 32-bit integer hash of (seed, i); optional f16 copy.
__global__ void fill_hash_kernel(float *p, half_t *p16, long n, uint32_t seed, float amp) {
    long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    long stride = (long)gridDim.x * blockDim.x;
    for (; i < n; i += stride) {
        uint32_t h = (uint32_t)i * 0x9E3779B1u ^ (uint32_t)(i >> 32) ^ seed;
        h ^= h >> 16; h *= 0x7FEB352Du; h ^= h >> 15; h *= 0x846CA68Bu; h ^= h >> 16;
        const float v = amp * ((float)(h >> 8) * (1.0f / 8388608.0f) - 1.0f);
        if (p) p[i] = v;
        if (p16) p16[i] = (half_t)v;
    }
}

__global__ void cast_f32_f16_kernel(const float *src, half_t *dst, long n) {
    long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    long stride = (long)gridDim.x * blockDim.x;
    for (; i < n; i += stride) dst[i] = (half_t)src[i];
}

// p -= lr * (scale * g); optional f16 copy and gradient output. Parameter.SGDStep (nn.go:69-76).
__global__ void sgd_kernel(float *p, const float *g, long n, float lr, float scale, half_t *p16, float *gout) {
    long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    long stride = (long)gridDim.x * blockDim.x;
    for (; i < n; i += stride) {
        float gv = scale * g[i];
        if (gout) gout[i] = gv;
        float w = p[i] - lr * gv;
        asm volatile("" : "+v"(w));   // the f16 copy is f16 of the stored f32 value
        p[i] = w;
        if (p16) p16[i] = (half_t)w;
    }
}

// colsum[n] += sum_m G[m, n]   (bias gradient: Expand rule, tensor/gradient_ruleset.go:207-233)
__global__ __launch_bounds__(256) void colsum_kernel(const float *G, int M, int N, long ld, int rows_per_block,
                                                      float *out) {
    __shared__ float red[4][64];
    int col = blockIdx.x * 64 + (threadIdx.x & 63);
    int sub = threadIdx.x >> 6;
    int r0 = blockIdx.y * rows_per_block;
    int r1 = min(M, r0 + rows_per_block);
    float acc = 0.0f;
    if (col < N)
        for (int r = r0 + sub; r < r1; r += 4) acc += G[(long)r * ld + col];
    red[sub][threadIdx.x & 63] = acc;
    __syncthreads();
    if (sub == 0 && col < N) {
        float v = ((red[0][threadIdx.x] + red[1][threadIdx.x]) + red[2][threadIdx.x]) + red[3][threadIdx.x];
        atomicAdd(out + col, v);
    }
}

// ── softmax cross-entropy ───────────────────────────────────────────────────
// loss = Sum(onehot * logp) * a,  a = f32(-1/B); see the oracle's ora_softmax_ce for the op list.
__global__ __launch_bounds__(256) void softmax_ce_kernel(const float *z, const int32_t *labels, int B, int C,
                                                          float a, float *dz, float *rowloss) {
    int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    int lane = threadIdx.x & 63;
    if (row >= B) return;
    const float rl = softmax_ce_row(z + (long)row * C, labels[row], C, a, dz + (long)row * C, lane);
    if (lane == 0) rowloss[row] = rl;
}

// Softmax-CE with the logit gradient's column sums (the output bias gradient) fused in: each wave
// takes rows blockIdx.x * kSmWaves + wave, then every kSmWaves * gridDim.x rows further, holding each
// row in registers, and keeps the column sums of its rows' dz in registers; the block's waves add theirs
// in wave order into partial row blockIdx.x of part[gridDim.x][C] (summed in row order by the step's
// tail), so the result does not depend on timing. With 16 waves per block and up to 256 blocks, a batch
// of up to 4096 rows gives every wave one row: the row's three dependent wave reductions then overlap
// across waves instead of running back to back in one.
constexpr int kSmWaves = 16;
template <int VPR>
__global__ __launch_bounds__(64 * kSmWaves) void softmax_ce_cols_kernel(const float *z, const int32_t *labels, int B, int C,
                                                                        float a, float *dz, float *rowloss, float *part) {
    __shared__ float red[kSmWaves][64 * VPR];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float col[VPR];
#pragma unroll
    for (int j = 0; j < VPR; j++) col[j] = 0.0f;
    // the next row's loads are issued before this row's arithmetic, so a wave with several rows keeps
    // one row's loads in flight
    const int step = gridDim.x * kSmWaves;
    int row = blockIdx.x * kSmWaves + wave;
    float nv[VPR];
    if (row < B) softmax_ce_row_load<VPR>(z + (long)row * C, C, lane, nv);
    for (; row < B; row += step) {
        float v[VPR];
#pragma unroll
        for (int j = 0; j < VPR; j++) v[j] = nv[j];
        if (row + step < B) softmax_ce_row_load<VPR>(z + (long)(row + step) * C, C, lane, nv);
        const float rl = softmax_ce_row_regs<VPR>(v, z + (long)row * C, labels[row], C, a, dz + (long)row * C, lane, col);
        if (lane == 0) rowloss[row] = rl;
    }
#pragma unroll
    for (int j = 0; j < VPR; j++) red[wave][lane + 64 * j] = col[j];
    __syncthreads();
    for (int c = threadIdx.x; c < C; c += 64 * kSmWaves) {
        float acc = red[0][c];
        for (int w = 1; w < kSmWaves; w++) acc += red[w][c];
        part[(long)blockIdx.x * C + c] = acc;
    }
}

// out[0] = (Sum_i v[i]) * a   (single block, fixed-order tree)
__global__ __launch_bounds__(256) void sum_scale_kernel(const float *v, int n, float a, float *out) {
    __shared__ float red[256];
    float acc = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) acc += v[i];
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
        __syncthreads();
    }
    if (threadIdx.x == 0) out[0] = red[0] * a;
}

// MSE loss finalize: f16 reduce narrowing f16(acc) (codegen/lower.go:712) then * scale in f32.
__global__ void mse_finalize_kernel(const float *acc, float scale, float *out) {
    if (threadIdx.x == 0 && blockIdx.x == 0) out[0] = q16(acc[0]) * scale;
}

// ── config 5: movement + row-reduce chain ───────────────────────────────────

// exp2 of a non-positive argument as the bare v_exp_f32: results below 2^-126 flush to zero (they are
// below f32's normal range and change no sum they enter; exp2f's denormal fix-up costs ~5 VALU ops
// per element, which is most of these streaming kernels' per-element work).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

struct ColStat {
    float m, t, s, q;
};

__device__ __forceinline__ void stat_push(ColStat &st, float y) {
    if (y > st.m) {
        float f = exp2f((st.m - y) * AH_INV_LN2);
        st.s = st.s * f + 1.0f;
        st.q = st.q * (f * f) + 1.0f;
        st.m = y;
        st.t = 1.0f;
    } else {
        float e = exp2f((y - st.m) * AH_INV_LN2);
        st.s += e;
        st.q += e * e;
        st.t += (y == st.m) ? 1.0f : 0.0f;
    }
}

__device__ __forceinline__ ColStat stat_merge(const ColStat &a, const ColStat &b) {
    ColStat r;
    r.m = fmaxf(a.m, b.m);
    float fa = exp2f((a.m - r.m) * AH_INV_LN2), fb = exp2f((b.m - r.m) * AH_INV_LN2);
    if (a.s == 0.0f) fa = 0.0f;
    if (b.s == 0.0f) fb = 0.0f;
    r.s = a.s * fa + b.s * fb;
    r.q = a.q * (fa * fa) + b.q * (fb * fb);
    r.t = (a.m == r.m ? a.t : 0.0f) + (b.m == r.m ? b.t : 0.0f);
    return r;
}

// Pass 1. Block = 4 waves over the same 256 columns (lane owns 4 consecutive columns);
// blockIdx.y selects a chunk of `rch` rows, waves interleave rows within it. Each wave issues 8 row
// loads (8 KiB) before consuming any, so enough bytes are in flight to cover HBM latency.
__global__ __launch_bounds__(256) void chain_stats_kernel(const float *X, int R, int Cc, int rch, ColStat *part) {
    __shared__ ColStat sh[4][256];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c0 = blockIdx.x * 256 + lane * 4;
    const int r0 = blockIdx.y * rch, r1 = min(R, r0 + rch);
    ColStat st[4];
#pragma unroll
    for (int u = 0; u < 4; u++) st[u] = ColStat{-FLT_MAX, 0.0f, 0.0f, 0.0f};
    if (c0 < Cc) {
        int r = r0 + wave;
        for (; r + 28 < r1; r += 32) {
            floatx4 v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = *(const floatx4 *)(X + (long)(r + 4 * j) * Cc + c0);
#pragma unroll
            for (int u = 0; u < 4; u++) {
                // Rescale once per 8 rows to the batch max, then accumulate without branches
                // (the element equal to the new max contributes exp2(0) = 1 exactly, as in stat_push).
                float mb = v[0][u];
#pragma unroll
                for (int j = 1; j < 8; j++) mb = fmaxf(mb, v[j][u]);
                if (mb > st[u].m) {
                    const float f = exp2f((st[u].m - mb) * AH_INV_LN2);
                    st[u].s *= f;
                    st[u].q *= f * f;
                    st[u].t = 0.0f;
                    st[u].m = mb;
                }
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float e = fast_exp2((v[j][u] - st[u].m) * AH_INV_LN2);
                    st[u].s += e;
                    st[u].q += e * e;
                    st[u].t += (v[j][u] == st[u].m) ? 1.0f : 0.0f;
                }
            }
        }
        for (; r < r1; r += 4) {
            floatx4 v = *(const floatx4 *)(X + (long)r * Cc + c0);
#pragma unroll
            for (int u = 0; u < 4; u++) stat_push(st[u], v[u]);
        }
    }
#pragma unroll
    for (int u = 0; u < 4; u++) sh[wave][lane * 4 + u] = st[u];
    __syncthreads();
    int col = blockIdx.x * 256 + threadIdx.x;
    if (col < Cc) {
        ColStat a = stat_merge(stat_merge(sh[0][threadIdx.x], sh[1][threadIdx.x]),
                               stat_merge(sh[2][threadIdx.x], sh[3][threadIdx.x]));
        part[(long)blockIdx.y * Cc + col] = a;
    }
}

// Per-column finalize: fold the chunk partials, then the reference backward's per-row scalars.
// Block = 16 columns x 16 partial groups: group p folds partials p, p+16, ... (coalesced 256-byte rows),
// the 16 group results are merged in a fixed order (deterministic), then one thread per column
// evaluates the scalars. coef[col] = {m, rs, g*r, gsq, gs, share, dg, loss_row}; lossp[block] is the
// block's sum of loss_row (summed by the gradient pass).
constexpr int kFinCols = 16;
constexpr int kFinGroups = 256 / kFinCols;
__global__ __launch_bounds__(256) void chain_finalize_kernel(const ColStat *part, int nchunks, int R, int Cc,
                                                              const float *g, float *coef, float *dg, float *lossp) {
    __shared__ ColStat sh[kFinGroups][kFinCols];
    __shared__ float lsum[kFinCols];
    const int cl = threadIdx.x % kFinCols, grp = threadIdx.x / kFinCols;
    const int col = blockIdx.x * kFinCols + cl;
    ColStat a{-FLT_MAX, 0.0f, 0.0f, 0.0f};
    if (col < Cc)
        for (int k0 = grp; k0 < nchunks; k0 += 8 * kFinGroups) {   // 8 loads in flight, then the merges
            ColStat v[8];
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (k0 + u * kFinGroups < nchunks) v[u] = part[(long)(k0 + u * kFinGroups) * Cc + col];
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (k0 + u * kFinGroups < nchunks) a = stat_merge(a, v[u]);
        }
    sh[grp][cl] = a;
    __syncthreads();
    if (grp == 0) {
        float lrow = 0.0f;
        if (col < Cc) {
#pragma unroll
            for (int k = 1; k < kFinGroups; k++) a = stat_merge(a, sh[k][cl]);
            const float eps = 1e-6f;
            const float rR = 1.0f / (float)R;
            float rs = 1.0f / a.s;
            float sumS = a.s * rs;             // Sum_j e_j * rs
            float sq = a.q * (rs * rs);        // Sum_j (e_j * rs)^2
            float q = sq * rR;
            float T = sqrtf(q + eps);
            float r = 1.0f / T;
            float gi = g[col];
            float gR = gi * sumS;
            float gT = ((-gR) * r) * r;
            float gu = gT * (1.0f / (2.0f * T));
            float gsq = gu * rR;
            float gRs = (gi * r) * a.s + 2.0f * gsq * (rs * a.q);
            float gs = ((-gRs) * rs) * rs;
            float gm = -(AH_LN2 * AH_INV_LN2) * (rs * gRs + gs * a.s);
            float share = gm * (1.0f / a.t);
            float *cf = coef + (long)col * 8;
            lrow = gi * (r * sumS);
            *(floatx4 *)cf = floatx4{a.m, rs, gi * r, gsq};
            *(floatx4 *)(cf + 4) = floatx4{gs, share, r * sumS, lrow};
            dg[col] = r * sumS;
        }
        lsum[cl] = lrow;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float acc = 0.0f;
        for (int k = 0; k < kFinCols; k++) acc += lsum[k];
        lossp[blockIdx.x] = acc;
    }
}

// Pass 2: dX[j, i] from X[j, i] and the per-column scalars; each wave loads its 8 rows before
// computing. Block (0, 0) also sums the finalize blocks' loss partials in a fixed order.
__global__ __launch_bounds__(256) void chain_grad_kernel(const float *X, int R, int Cc, int rch, const float *coef,
                                                          float *dX, const float *lossp, int nlossp, float *loss) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (blockIdx.x == 0 && blockIdx.y == 0 && wave == 0) {
        float acc = 0.0f;
        for (int i = lane; i < nlossp; i += 64) acc += lossp[i];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
        if (lane == 0) loss[0] = acc;
    }
    const int c0 = blockIdx.x * 256 + lane * 4;
    if (c0 >= Cc) return;
    float m[4], rs[4], gr[4], gsq[4], gs[4], sh[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const floatx4 a = *(const floatx4 *)(coef + (long)(c0 + u) * 8);
        const floatx4 b = *(const floatx4 *)(coef + (long)(c0 + u) * 8 + 4);
        m[u] = a[0]; rs[u] = a[1]; gr[u] = a[2]; gsq[u] = a[3]; gs[u] = b[0]; sh[u] = b[1];
    }
    const int r0 = blockIdx.y * rch, r1 = min(R, r0 + rch);
    // 8 rows in flight per wave. X is read with ordinary loads: the stats pass has just streamed it, so
    // much of it is still in the Infinity Cache (a non-temporal load measured 20-30% slower here).
    for (int rb = r0 + wave; rb < r1; rb += 32) {
        floatx4 v[8];
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (rb + 4 * j < r1) v[j] = *(const floatx4 *)(X + (long)(rb + 4 * j) * Cc + c0);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            if (rb + 4 * j >= r1) break;
            floatx4 o;
#pragma unroll
            for (int u = 0; u < 4; u++) {
                float y = v[j][u];
                float e = fast_exp2((y - m[u]) * AH_INV_LN2);
                float S = e * rs[u];
                float t2 = gsq[u] * S;
                float gS = (gr[u] + t2) + t2;
                float ge = gS * rs[u] + gs[u];
                float gzs = ((ge * e) * AH_LN2) * AH_INV_LN2;
                o[u] = gzs + ((y == m[u]) ? sh[u] : 0.0f);
            }
            __builtin_nontemporal_store(o, (floatx4 *)(dX + (long)(rb + 4 * j) * Cc + c0));
        }
    }
}

// ── config 5 in one pass over HBM: strips of X held on chip ─────────────────────
// Every softmax / RMS row of the chain is one column of X, and dg, the loss terms and dX of a column
// need only that column. So one workgroup per CU takes a strip of 16 columns x R rows (R = 4096 or
// 8192: up to 512 KiB), keeps all of it on chip (kResRegs float4 per thread in VGPRs, kResLds in LDS through
// LDS-DMA), and runs the whole chain on it: the column max, sum e, sum e^2 and the tie count
// (accumulated while the strip lands, see below), the per-column scalars of chain_finalize, dg, and dX
// written once from the on-chip copy. HBM sees X read once and dX written once; the three-kernel chain reads X
// twice and moves its column partials through memory. Thread t owns columns c0 + 4 (t & 3) .. + 3 of
// rows (t >> 2) + 128 i. Every sum is a fixed tree (slots in order, then lanes by xor, then waves in
// order), so results are deterministic. Each workgroup stores its 16 columns' loss terms summed in
// column order; the last to arrive (arrival counter, zero before and after the launch) adds the strips'
// sums in strip order.
constexpr int kResThreads = 512, kResRowLanes = kResThreads / 4, kResCols = 16;
constexpr int kResMaxRegs = 45, kResMaxLds = 19;   // float4 slots per thread in VGPRs / in LDS (152 KiB)

__device__ __forceinline__ float res_tree_max(float v) {   // over the 16 lanes of a wave with equal lane & 3
    v = fmaxf(v, __shfl_xor(v, 4, 64));
    v = fmaxf(v, __shfl_xor(v, 8, 64));
    v = fmaxf(v, __shfl_xor(v, 16, 64));
    return fmaxf(v, __shfl_xor(v, 32, 64));
}
__device__ __forceinline__ float res_tree_sum(float v) {
    v += __shfl_xor(v, 4, 64);
    v += __shfl_xor(v, 8, 64);
    v += __shfl_xor(v, 16, 64);
    return v + __shfl_xor(v, 32, 64);
}

// NS: float4 slots per thread, R = 128 * NS rows.
template <int NS>
__global__ __launch_bounds__(kResThreads) void chain_resident_kernel(const float *X, int R, int Cc, const float *g,
                                                                      float *dX, float *dg, float *lossp, int *counter,
                                                                      float *loss) {
    constexpr int kResRegs = NS < kResMaxRegs ? NS : kResMaxRegs, kResLds = NS - kResRegs;
    static_assert(kResLds <= kResMaxLds, "the strip does not fit on chip");
    __shared__ __attribute__((aligned(1024))) floatx4 held[kResLds > 0 ? kResLds : 1][kResThreads];
    __shared__ float red[4][kResThreads / 64][kResCols];               // per wave: max, sum e, sum e^2, ties
    __shared__ __attribute__((aligned(16))) float coef[6][kResCols];   // dX factors A, B, column max, -, tie share, loss term
    __shared__ int ticket;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nstrips = Cc / kResCols;
    int strip = blockIdx.x;
    if ((nstrips & 7) == 0) strip = (strip & 7) * (nstrips >> 3) + (strip >> 3);   // neighbouring strips share an XCD
    const int q = tid & 3, rl = tid >> 2;
    // Buffer accesses from the strip's first column: the lane's offset in one VGPR, the slot's row
    // offset (wave-uniform) in the scalar offset, so the 64 slots cost no address registers. The
    // caller guarantees R * Cc * 4 < 2^31.
    typedef unsigned u4 __attribute__((ext_vector_type(4)));
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void *)(X + strip * kResCols), (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t dr = __builtin_amdgcn_make_buffer_rsrc((void *)(dX + strip * kResCols), (short)0, 0x7fffffff, 0x00020000);
    const int voff = (rl * Cc + 4 * q) * 4;
    const int rstepB = kResRowLanes * Cc * 4;
    // 1. the strip: register slots first (they are consumed first), then the LDS slots
    floatx4 v[kResRegs];
#pragma unroll
    for (int i = 0; i < kResRegs; i++)
        v[i] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(xr, voff, i * rstepB, 0));
#pragma unroll
    for (int j = 0; j < kResLds; j++)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (__attribute__((address_space(3))) void *)&held[j][wave * 64], 16,
                                                     voff, (kResRegs + j) * rstepB, 0, 0);
    // 2-3. Statistics while the strip lands. Each thread takes a provisional max mt of its own first
    // kProv slots, then, slot by slot as the loads arrive, adds e = 2^(x/ln2 - mt/ln2) and e^2 to its
    // column sums and keeps the exact running max with the count of elements equal to it. Once every
    // slot has landed, the column max m is the max of the running maxima, the tie count the sum of the
    // counts of the threads whose running max is m, and each thread's sums are rescaled by
    // 2^((mt - m_w)/ln2) to its wave's max m_w, each wave's by 2^((m_w - m)/ln2) to the column max.
    // x stays in place; the dX pass recomputes e against m. An element more than 2^60 above the
    // thread's reference (where e^2 could overflow) first moves the reference to itself, rescaling the
    // thread's sums (no such element occurs unless the strip's values grow by a factor e^41 along the
    // column).
    constexpr int kProv = 8;
    static_assert(kResRegs >= kProv, "the provisional max takes register slots");
    float mt[4] = {-FLT_MAX, -FLT_MAX, -FLT_MAX, -FLT_MAX};
#pragma unroll
    for (int i = 0; i < kProv; i++)
#pragma unroll
        for (int u = 0; u < 4; u++) mt[u] = fmaxf(mt[u], v[i][u]);
    float mct[4], mr[4], cnt[4], se[4] = {}, sq[4] = {};
#pragma unroll
    for (int u = 0; u < 4; u++) {
        mct[u] = mt[u] * AH_INV_LN2;
        mr[u] = -FLT_MAX;
        cnt[u] = 0.0f;
    }
    auto stat = [&](const floatx4 &x) {
        float d[4];
#pragma unroll
        for (int u = 0; u < 4; u++) d[u] = __builtin_fmaf(x[u], AH_INV_LN2, -mct[u]);
        // one wave-uniform test per slot for the (never taken on ordinary data) re-base
        const float dm = fmaxf(fmaxf(d[0], d[1]), fmaxf(d[2], d[3]));
        if (__builtin_amdgcn_ballot_w64(dm > 60.0f)) {
#pragma unroll
            for (int u = 0; u < 4; u++) {
                if (d[u] > 60.0f) {
                    const float f = fast_exp2(-d[u]);
                    se[u] *= f;
                    sq[u] *= f * f;
                    mct[u] = x[u] * AH_INV_LN2;
                    d[u] = __builtin_fmaf(x[u], AH_INV_LN2, -mct[u]);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const float e = fast_exp2(d[u]);
            se[u] += e;
            sq[u] += e * e;
            const float mn = fmaxf(mr[u], x[u]);
            cnt[u] = (mn == mr[u] ? cnt[u] : 0.0f) + (x[u] == mn ? 1.0f : 0.0f);   // count of the running max
            mr[u] = mn;
        }
        // materialise the running values after every slot (left free, the compiler runs one sum over
        // all slots before the next, keeping every slot's e live in between)
        asm volatile("" : "+v"(se[0]), "+v"(se[1]), "+v"(se[2]), "+v"(se[3]), "+v"(sq[0]), "+v"(sq[1]), "+v"(sq[2]),
                     "+v"(sq[3]), "+v"(cnt[0]), "+v"(cnt[1]), "+v"(cnt[2]), "+v"(cnt[3]), "+v"(mr[0]), "+v"(mr[1]),
                     "+v"(mr[2]), "+v"(mr[3]));
    };
#pragma unroll
    for (int i = 0; i < kResRegs; i++) stat(v[i]);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wave's LDS-DMA has landed (each lane reads its own)
#pragma unroll 2
    for (int j = 0; j < kResLds; j++) {
        const floatx4 x = *(volatile floatx4 *)&held[j][tid];
        stat(x);
    }
    // 4. Column statistics in one cross-wave round: each wave folds its 16 lanes of a column (max,
    // then the sums rescaled to the wave's max, the tie count at that max) and lanes 0-3 post the
    // wave's (max, sum e, sum e^2, ties) per column; thread c < 16 folds the 8 waves of column c in
    // order, rescaling each wave's sums to the column max, and evaluates the column's scalars
    // (chain_finalize's rules); every thread then reads its 4 columns' scalars back.
    float m[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        m[u] = res_tree_max(mr[u]);                    // the wave's max of the column
        const float f = fast_exp2(mct[u] - m[u] * AH_INV_LN2);   // 2^((mt - m_w)/ln2) <= 1
        se[u] = res_tree_sum(se[u] * f);
        sq[u] = res_tree_sum(sq[u] * (f * f));
        cnt[u] = res_tree_sum(mr[u] == m[u] ? cnt[u] : 0.0f);
    }
    if (lane < 4)
#pragma unroll
        for (int u = 0; u < 4; u++) {
            red[0][wave][4 * lane + u] = m[u];
            red[1][wave][4 * lane + u] = se[u];
            red[2][wave][4 * lane + u] = sq[u];
            red[3][wave][4 * lane + u] = cnt[u];
        }
    __syncthreads();
    if (tid < kResCols) {
        float mm = red[0][0][tid];
        for (int w = 1; w < kResThreads / 64; w++) mm = fmaxf(mm, red[0][w][tid]);
        const float mmc = mm * AH_INV_LN2;
        float s_ = 0.0f, q_ = 0.0f, t_ = 0.0f;
        for (int w = 0; w < kResThreads / 64; w++) {
            const float mw = red[0][w][tid];
            const float f = fast_exp2(__builtin_fmaf(mw, AH_INV_LN2, -mmc));
            s_ += red[1][w][tid] * f;
            q_ += red[2][w][tid] * (f * f);
            t_ += mw == mm ? red[3][w][tid] : 0.0f;
        }
        const int c = strip * kResCols + tid;
        const float eps = 1e-6f, rR = 1.0f / (float)R;
        const float r_s = 1.0f / s_;
        const float sumS = s_ * r_s;
        const float sqq = q_ * (r_s * r_s);
        const float qm = sqq * rR;
        const float T = sqrtf(qm + eps);
        const float r = 1.0f / T;
        const float gi = g[c];
        const float gR = gi * sumS;
        const float gT = ((-gR) * r) * r;
        const float gu = gT * (1.0f / (2.0f * T));
        const float gsq_ = gu * rR;
        const float gRs = (gi * r) * s_ + 2.0f * gsq_ * (r_s * q_);
        const float gs_ = ((-gRs) * r_s) * r_s;
        const float gm = -(AH_LN2 * AH_INV_LN2) * (r_s * gRs + gs_ * s_);
        // dX = e * (gr * r_s + gs) + e^2 * (2 gsq r_s^2), plus the tie share where x is the max: the
        // per-element backward of S = e * r_s through sum e and sum S^2, with its per-column factors
        // gathered (the reference's op order rounds them per element; the difference is at f32 rounding)
        coef[0][tid] = (gi * r) * r_s + gs_;
        coef[1][tid] = 2.0f * gsq_ * (r_s * r_s);
        coef[4][tid] = gm * (1.0f / t_);
        coef[5][tid] = gi * (r * sumS);
        coef[2][tid] = mm;
        dg[c] = r * sumS;
    }
    __syncthreads();
    float ca[4], cb[4], sh[4], mc[4];
    {
        const floatx4 a = *(const floatx4 *)&coef[0][4 * q], b = *(const floatx4 *)&coef[1][4 * q],
                      mx = *(const floatx4 *)&coef[2][4 * q], e = *(const floatx4 *)&coef[4][4 * q];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            ca[u] = a[u];
            cb[u] = b[u];
            m[u] = mx[u];
            mc[u] = mx[u] * AH_INV_LN2;
            sh[u] = e[u];
        }
    }
    // 5. dX from the held strip: the register slots, then the LDS slots two at a time. The LDS slots are
    // read through volatile loads in every pass: otherwise the compiler may keep one pass's reads live in
    // registers for the next, which the held strip leaves no room for.
    auto each = [&](auto &&f) {
#pragma unroll
        for (int i = 0; i < kResRegs; i++) f(i, v[i]);
#pragma unroll 2
        for (int j = 0; j < kResLds; j++) {
            const floatx4 x = *(volatile floatx4 *)&held[j][tid];
            f(kResRegs + j, x);
        }
    };
    // The stores' row offset is a running value advanced through an empty asm after each slot, so only
    // the current one is live (all 64 kept from the loads overflow the SGPRs into VGPR lanes).
    int soff = 0;
    each([&](int i, const floatx4 &x) {
        floatx4 o;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const float e = fast_exp2(__builtin_fmaf(x[u], AH_INV_LN2, -mc[u]));
            const float gzs = (ca[u] + cb[u] * e) * e;
            o[u] = gzs + (x[u] == m[u] ? sh[u] : 0.0f);
        }
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, o), dr, voff, soff, 0);
        soff += rstepB;
        asm volatile("" : "+s"(soff));
        // Wait states after the 16-byte store before anything may rewrite its data registers. Without
        // them the compiler placed a VALU write to the store's first data VGPR two instructions later,
        // behind a v_readlane of a spilled SGPR, and that dword of some lanes was stored already
        // overwritten (observed: element 0 of the float4 in lanes 12-15 of a wave).
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_nop 4" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
    });
    // 6. loss: this strip's 16 terms in column order, then the strips in order by the last to arrive
    __syncthreads();
    if (tid == 0) {
        float a = 0.0f;
        for (int c = 0; c < kResCols; c++) a += coef[5][c];
        __hip_atomic_store(lossp + strip, a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ticket = ticket_take_atomic_partials(counter);   // lossp[] is written and read as atomics
    }
    __syncthreads();
    if (ticket != (int)gridDim.x - 1 || wave != 0) return;
    // lane k adds strips k*P .. k*P+P-1 in order, then the lanes in a fixed tree
    const int per = (nstrips + 63) / 64;
    float a = 0.0f;
    for (int k = 0; k < per; k++) {
        const int s2 = lane * per + k;
        if (s2 < nstrips) a += __hip_atomic_load(lossp + s2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    a = wave_sum(a);
    if (lane == 0) {
        loss[0] = a;
        __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Row counts with an instantiated strip program: R = 8192 (64 float4 slots per thread: 45 in VGPRs, 19 in
// LDS) and R = 4096 (32, all in VGPRs); other shapes take the three-kernel chain.
bool chain_resident_fits(int R, int Cc) {
    return (R == 128 * 64 || R == 128 * 32) && Cc >= kResCols && Cc % kResCols == 0 && (long)R * Cc * 4 < (1L << 31);
}

hipError_t chain_resident(const float *X, const float *g, int R, int Cc, float *lossp, int *counter, float *dX, float *dg,
                          float *loss, hipStream_t s) {
    if (!chain_resident_fits(R, Cc)) return hipErrorInvalidValue;
    if (R == 128 * 64)
        hipLaunchKernelGGL(chain_resident_kernel<64>, dim3(Cc / kResCols), dim3(kResThreads), 0, s, X, R, Cc, g, dX, dg,
                           lossp, counter, loss);
    else
        hipLaunchKernelGGL(chain_resident_kernel<32>, dim3(Cc / kResCols), dim3(kResThreads), 0, s, X, R, Cc, g, dX, dg,
                           lossp, counter, loss);
    return hipGetLastError();
}

// ── step tail: bias SGD for several parameters + loss finalize, in one launch ─────
// Each accumulator element (or partial-row entry) is read and re-zeroed by the thread that sums it,
// leaving the accumulators ready for the next step's atomics or partial stores (no zero-fill launch).
__device__ __forceinline__ float block_sum_512(float v, float *red) {   // fixed order: waves, then 8 slots
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return ((red[0] + red[1]) + (red[2] + red[3])) + ((red[4] + red[5]) + (red[6] + red[7]));
}

__global__ __launch_bounds__(512) void tail_kernel(TailArgs t) {
    static_assert(kTailCols * kTailChunks == 512, "tail block is 512 threads");
    // The loss has a block of its own (the last), so its reduction runs beside the parameters' instead
    // of ahead of one block's share of them.
    const int ncol = gridDim.x - (t.loss_mode != 0 ? 1 : 0);
    if ((int)blockIdx.x == ncol) {
        __shared__ float red[8];
        if (t.loss_mode == 1 && t.loss_parts > 0) {
            // per-wave partials, summed in a fixed order, then the f16(acc) narrowing (lower.go:712)
            float acc = 0.0f;
            int i = threadIdx.x;
            for (; i + 7 * 512 < t.loss_parts; i += 8 * 512) {   // 8 loads in flight, then the zeroing
                float v[8];
#pragma unroll
                for (int j = 0; j < 8; j++) v[j] = t.lossacc[i + j * 512];
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    acc += v[j];
                    t.lossacc[i + j * 512] = 0.0f;
                }
            }
            for (; i < t.loss_parts; i += 512) {
                acc += t.lossacc[i];
                t.lossacc[i] = 0.0f;
            }
            acc = block_sum_512(acc, red);
            if (threadIdx.x == 0) {
                t.loss_out[0] = q16(acc) * t.loss_scale;
                if (t.loss_sum) t.loss_sum[0] = acc;
            }
        } else if (t.loss_mode == 1) {
            if (threadIdx.x == 0) {
                if (t.loss_sum) t.loss_sum[0] = t.lossacc[0];
                t.loss_out[0] = q16(t.lossacc[0]) * t.loss_scale;   // f16(acc) narrowing, lower.go:712
                t.lossacc[0] = 0.0f;
            }
        } else if (t.loss_mode == 2) {
            float acc = 0.0f;
            for (int i = threadIdx.x; i < t.nrow; i += 512) acc += t.rowloss[i];
            acc = block_sum_512(acc, red);
            if (threadIdx.x == 0) t.loss_out[0] = acc * t.loss_scale;
        }
        return;
    }
    // kTailCols consecutive elements per block pass, so a half-wave reads 128 contiguous bytes of a
    // partial row; the rows of a partial-row accumulator are split into kTailChunks chunks (up to 16
    // loads in flight per thread), and the chunk sums are combined in a fixed order, so the result is
    // deterministic.
    long total = 0;
    for (int s = 0; s < t.nseg; s++) total += t.seg[s].n;
    __shared__ float part[kTailChunks][kTailCols];
    const int e = threadIdx.x % kTailCols, q = threadIdx.x / kTailCols;
    for (long base = (long)blockIdx.x * kTailCols; base < total; base += (long)ncol * kTailCols) {
        const long i = base + e;
        long k = i;
        int s = 0;
        if (i < total)
            while (k >= t.seg[s].n) { k -= t.seg[s].n; s++; }
        const TailSeg &g = t.seg[s];
        // the parameter's old value is loaded with the gradient partials, not after their sum
        const float pold = (q == 0 && i < total) ? g.p[k] : 0.0f;
        float a = 0.0f;
        if (i < total) {
            if (g.acc_rows > 0) {
                const int rq = (g.acc_rows + kTailChunks - 1) / kTailChunks, r0 = q * rq;
                const int r1 = min(r0 + rq, g.acc_rows);
                float *const col = g.acc + k;
                float p[16] = {};
                for (int r = r0; r < r1; r += 16) {   // rows past r1 are predicated off, so p[] stays in registers
                    float v[16];
#pragma unroll
                    for (int j = 0; j < 16; j++) v[j] = r + j < r1 ? col[(long)(r + j) * g.acc_ld] : 0.0f;
#pragma unroll
                    for (int j = 0; j < 16; j++) {
                        p[j] += v[j];
                        if (r + j < r1 && !g.keep) col[(long)(r + j) * g.acc_ld] = 0.0f;
                    }
                }
#pragma unroll
                for (int w = 8; w > 0; w >>= 1)
#pragma unroll
                    for (int j = 0; j < w; j++) p[j] += p[j + w];
                a = p[0];
            } else if (q == 0) {
                a = g.acc[k];
                if (!g.keep) g.acc[k] = 0.0f;
            }
        }
        part[q][e] = a;
        __syncthreads();
        if (q == 0 && i < total) {
            float sum = 0.0f;
#pragma unroll
            for (int c = 0; c < kTailChunks; c++) sum += part[c][e];
            const float gv = g.scale * sum;
            if (g.gout) g.gout[k] = gv;
            float w = pold - t.lr * gv;
            asm volatile("" : "+v"(w));   // the f16 copy is f16 of the stored f32 value
            g.p[k] = w;
            if (g.p16) g.p16[k] = (half_t)w;
        }
        __syncthreads();
    }
}

hipError_t step_tail(const TailArgs &t, hipStream_t s) {
    long total = 0;
    for (int i = 0; i < t.nseg; i++) total += t.seg[i].n;
    int blocks = (int)std::min<long>(std::max<long>((total + kTailCols - 1) / kTailCols, 1), 2048);
    if (t.loss_mode != 0) blocks++;   // the loss block
    hipLaunchKernelGGL(tail_kernel, dim3(blocks), dim3(kTailCols * kTailChunks), 0, s, t);
    return hipGetLastError();
}

// ── host launchers ──────────────────────────────────────────────────────────

static int grid_for(long n) {
    long g = (n + 255) / 256;
    return (int)(g < 2048 ? (g < 1 ? 1 : g) : 2048);
}

hipError_t fill_f32(float *p, long n, float v, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(fill_f32_kernel, dim3(grid_for(n)), dim3(256), 0, s, p, n, v);
    return hipGetLastError();
}
hipError_t fill_hash(float *p, half_t *p16, long n, uint32_t seed, float amp, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(fill_hash_kernel, dim3(grid_for(n)), dim3(256), 0, s, p, p16, n, seed, amp);
    return hipGetLastError();
}
hipError_t cast_f32_f16(const float *src, half_t *dst, long n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(cast_f32_f16_kernel, dim3(grid_for(n)), dim3(256), 0, s, src, dst, n);
    return hipGetLastError();
}
hipError_t sgd_update(float *p, const float *g, long n, float lr, float scale, half_t *p16, float *gout,
                      hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(sgd_kernel, dim3(grid_for(n)), dim3(256), 0, s, p, g, n, lr, scale, p16, gout);
    return hipGetLastError();
}
hipError_t colsum_add(const float *G, int M, int N, long ld, float *out, hipStream_t s) {
    if (M <= 0 || N <= 0) return hipSuccess;
    int rpb = 64;
    dim3 grid((N + 63) / 64, (M + rpb - 1) / rpb);
    hipLaunchKernelGGL(colsum_kernel, grid, dim3(256), 0, s, G, M, N, ld, rpb, out);
    return hipGetLastError();
}
hipError_t softmax_ce(const float *z, const int32_t *labels, int B, int C, float a, float *dz, float *rowloss,
                      hipStream_t s) {
    if (B <= 0) return hipSuccess;
    hipLaunchKernelGGL(softmax_ce_kernel, dim3((B + 3) / 4), dim3(256), 0, s, z, labels, B, C, a, dz, rowloss);
    return hipGetLastError();
}
int softmax_ce_cols_blocks(int B) {
    const int b = (B + kSmWaves - 1) / kSmWaves;
    return b < kSoftmaxColsMaxBlocks ? (b < 1 ? 1 : b) : kSoftmaxColsMaxBlocks;
}
hipError_t softmax_ce_cols(const float *z, const int32_t *labels, int B, int C, float a, float *dz, float *rowloss,
                           float *part, hipStream_t s) {
    if (B <= 0) return hipSuccess;
    const dim3 grid(softmax_ce_cols_blocks(B)), block(64 * kSmWaves);
    if (C <= 64) hipLaunchKernelGGL(softmax_ce_cols_kernel<1>, grid, block, 0, s, z, labels, B, C, a, dz, rowloss, part);
    else if (C <= 128) hipLaunchKernelGGL(softmax_ce_cols_kernel<2>, grid, block, 0, s, z, labels, B, C, a, dz, rowloss, part);
    else if (C <= 256) hipLaunchKernelGGL(softmax_ce_cols_kernel<4>, grid, block, 0, s, z, labels, B, C, a, dz, rowloss, part);
    else if (C <= 512) hipLaunchKernelGGL(softmax_ce_cols_kernel<8>, grid, block, 0, s, z, labels, B, C, a, dz, rowloss, part);
    else if (C <= kSoftmaxColsMaxC) hipLaunchKernelGGL(softmax_ce_cols_kernel<16>, grid, block, 0, s, z, labels, B, C, a, dz, rowloss, part);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}
hipError_t sum_scale(const float *v, int n, float a, float *out, hipStream_t s) {
    hipLaunchKernelGGL(sum_scale_kernel, dim3(1), dim3(256), 0, s, v, n, a, out);
    return hipGetLastError();
}
hipError_t mse_finalize(const float *acc, float scale, float *out, hipStream_t s) {
    hipLaunchKernelGGL(mse_finalize_kernel, dim3(1), dim3(64), 0, s, acc, scale, out);
    return hipGetLastError();
}

// Workspace: word 0 is the resident path's arrival counter (zero before the first call, left zero by
// every call; the three-kernel path never touches it), then from float 64 either path's arrays.
constexpr long kChainHead = 64;
long chain_workspace_floats(int R, int Cc) {
    int nch = (R + kChainStatsRows - 1) / kChainStatsRows;
    const long three = (long)nch * Cc * 4 + (long)Cc * 8 + (Cc + kFinCols - 1) / kFinCols;
    return kChainHead + std::max(three, (long)(Cc / kResCols));
}

hipError_t chain_step(const float *X, const float *g, int R, int Cc, float *work, float *dX, float *dg, float *loss,
                      hipStream_t s, int phase) {
    if (Cc % 4 != 0 || R <= 0) return hipErrorInvalidValue;
    if (phase < 0 && chain_resident_fits(R, Cc))
        return chain_resident(X, g, R, Cc, work + kChainHead, (int *)work, dX, dg, loss, s);
    work += kChainHead;
    const int nch = (R + kChainStatsRows - 1) / kChainStatsRows;
    const int nfin = (Cc + kFinCols - 1) / kFinCols;
    ColStat *part = (ColStat *)work;
    float *coef = work + (long)nch * Cc * 4;
    float *lossp = coef + (long)Cc * 8;
    if (phase < 0 || phase == 0)
        hipLaunchKernelGGL(chain_stats_kernel, dim3((Cc + 255) / 256, nch), dim3(256), 0, s, X, R, Cc, kChainStatsRows, part);
    if (phase < 0 || phase == 1)
        hipLaunchKernelGGL(chain_finalize_kernel, dim3(nfin), dim3(256), 0, s, part, nch, R, Cc, g, coef, dg, lossp);
    if (phase < 0 || phase == 2) {
        int nch2 = (R + kChainGradRows - 1) / kChainGradRows;
        hipLaunchKernelGGL(chain_grad_kernel, dim3((Cc + 255) / 256, nch2), dim3(256), 0, s, X, R, Cc, kChainGradRows,
                           coef, dX, lossp, nfin, loss);
    }
    return hipGetLastError();
}

}  // namespace ah

// ── config-5 chain without allocation ───────────────────────────────────────
// The chain's workspace (per-chunk column partials, per-column coefficients, loss partials) lives in a
// file-scope device array instead of a hipMalloc'd buffer, for callers that cannot allocate (graph
// capture, serving loops). Every GPU the library runs on holds its own copy of `scratch` at its own
// address until the process ends; host code must use the address hipGetSymbolAddress returned for the
// current device, never the array's name (which is only a host-side stand-in).
// The chain writes every workspace entry before reading it (chain_stats fills every chunk partial,
// chain_finalize every coefficient and loss partial; the resident path every strip's loss sum), except
// the resident path's arrival counter in word 0: static storage starts at zero and every call leaves
// it zero, so nothing needs clearing between calls.
namespace ah {
namespace {
constexpr long kChainScratchFloats = 1L << 22;   // 16 MiB: R x Cc up to 16320 x 4096 (config 5, 8192 x 4096, needs 2.13M floats)
constexpr int kMaxDevices = 64;
static __device__ __align__(256) float scratch[kChainScratchFloats];
float *g_scratch_ptr[kMaxDevices];
}  // namespace

long chain_scratch_floats() { return kChainScratchFloats; }

// Looks up this device's copy of `scratch`, with `ordinal` the current device. Called once per device,
// from ah_open; later calls return the stored address.
hipError_t chain_scratch_init(int ordinal, float **out) {
    if (ordinal < 0 || ordinal >= kMaxDevices) return hipErrorInvalidDevice;
    // handles opened from several threads look the address up under one lock (the table is per process)
    static std::mutex mu;
    std::lock_guard<std::mutex> lock(mu);
    if (!g_scratch_ptr[ordinal]) {
        void *p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch_ptr[ordinal] = (float *)p;
    }
    *out = g_scratch_ptr[ordinal];
    return hipSuccess;
}

}  // namespace ah
