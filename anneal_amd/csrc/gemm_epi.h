// gemm_epi.h — fused GEMM epilogues shared by the contraction kernels.
//
// The epilogue walks a wave's FM x FN grid of 32x32 accumulator blocks column-block by column-block.
// The inputs a column block needs (ReLU activations for the mask, targets for MSE, master weights for
// SGD) are all loaded before any of its results is stored, so FM*16 loads per lane are in flight at
// once instead of each waiting behind a store to a possibly aliasing address.
#pragma once
#include "ah_common.h"
#include "gemm.h"

namespace ah {

// Accumulator layout of a 32x32 MFMA block: element r of lane l is row 8*(r/4) + 4*(l/32) + r%4,
// column l%32.
__device__ __forceinline__ int acc_row(int r, int lane) { return (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3); }

// Applies the epilogue to one accumulator value; returns its contribution to the column sum.
template <int EPI, typename T>
__device__ __forceinline__ float epi_apply(const GemmDesc &d, int m, int n, float acc, float in, float bias,
                                           float &lossp) {
    T *C = (T *)d.C;
    const long ci = (long)m * d.ldc + n;
    if constexpr (EPI == EPI_STORE) {
        const float v = d.scale * acc;
        C[ci] = (T)v;
        return v;
    } else if constexpr (EPI == EPI_BIAS || EPI == EPI_BIAS_RELU) {
        float z;
        if constexpr (sizeof(T) == 2) z = q16(q16(acc) + bias);      // f16(f16(acc) + b)
        else z = acc + bias;
        if constexpr (EPI == EPI_BIAS_RELU) C[ci] = relu_tag((T)z);
        else C[ci] = (T)z;
        return 0.0f;
    } else if constexpr (EPI == EPI_MSE) {
        const float p = q16(q16(acc) + bias);
        const float diff = p - in;
        lossp += diff * diff;
        const float dd = q16(diff);
        C[ci] = (T)dd;
        return dd;
    } else if constexpr (EPI == EPI_MASK) {
        const float v = relu_dead(in) ? 0.0f : d.scale * acc;
        C[ci] = (T)v;
        if (sizeof(T) == 2 && d.C2) ((T *)d.C2)[ci] = (T)(v - (float)(T)v);
        return v;
    } else {  // EPI_SGD
        const float g = d.scale * acc;
        if (d.gout) d.gout[ci] = g;
        float w = in - d.lr * g;
        asm volatile("" : "+v"(w));   // W16 is f16 of the stored W32 (no differently rounded fused op)
        d.W32[ci] = w;
        if (d.W16) ((half_t *)d.W16)[ci] = (half_t)w;
        return 0.0f;
    }
}

// Wave-tile epilogue. mb, nb: global row/column of the wave's first accumulator block.
// FULL: the whole FM*32 x FN*32 wave tile is in bounds, so no per-element predicate is needed
// (per-element branches would each hold an exec mask and exhaust the scalar registers).
template <int EPI, typename T, int FM, int FN, bool FULL>
__device__ __forceinline__ void epilogue_impl(const GemmDesc &d, const floatx16 (&acc)[FM][FN], int mb, int nb,
                                              int lane) {
    constexpr bool IN = EPI == EPI_MASK || EPI == EPI_MSE || EPI == EPI_SGD;
    float lossp = 0.0f;
    const long ldc = d.ldc, lda = d.ldaux;
#pragma unroll
    for (int j = 0; j < FN; j++) {
        const int n = nb + j * 32 + (lane & 31);
        const bool nv = FULL || n < d.N;
        // 1. inputs of this column block: FM*16 independent loads in flight
        float in[FM][16];
        if constexpr (IN) {
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int m = mb + i * 32 + acc_row(r, lane);
                    const bool v = FULL || (nv && m < d.M);
                    if constexpr (EPI == EPI_SGD) in[i][r] = v ? d.W32[m * ldc + n] : 0.0f;
                    else in[i][r] = v ? (float)((const T *)d.aux)[m * lda + n] : 0.0f;
                }
        }
        float bias = 0.0f;
        if constexpr (EPI == EPI_BIAS || EPI == EPI_BIAS_RELU || EPI == EPI_MSE) {
            if (nv) bias = sizeof(T) == 2 ? (float)((const T *)d.bias)[n] : ((const float *)d.bias)[n];
        }
        // 2. results
        float cs = 0.0f;
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = mb + i * 32 + acc_row(r, lane);
                if (FULL || (nv && m < d.M)) cs += epi_apply<EPI, T>(d, m, n, acc[i][j][r], in[i][r], bias, lossp);
            }
        if (d.colsum) {
            cs += __shfl_xor(cs, 32, 64);
            if (lane < 32 && nv) {
                if (d.colsum_ld) d.colsum[(long)(mb / 32) * d.colsum_ld + n] = cs;
                else atomicAdd(d.colsum + n, cs);
            }
        }
    }
    if constexpr (EPI == EPI_MSE) {
        lossp = wave_sum(lossp);
        if (lane == 0) {
            if (d.loss_ld) d.lossacc[(long)(mb / 32) * d.loss_ld + nb / 32] = lossp;
            else atomicAdd(d.lossacc, lossp);
        }
    }
}

template <int EPI, typename T, int FM, int FN>
__device__ __forceinline__ void epilogue_tile(const GemmDesc &d, const floatx16 (&acc)[FM][FN], int mb, int nb, int lane) {
    if (mb + FM * 32 <= d.M && nb + FN * 32 <= d.N) epilogue_impl<EPI, T, FM, FN, true>(d, acc, mb, nb, lane);
    else epilogue_impl<EPI, T, FM, FN, false>(d, acc, mb, nb, lane);
}

// ── LDS-staged epilogue ─────────────────────────────────────────────────────
// The wave's accumulators are written to a wave-private LDS region (FM*32 rows x 64 columns of f32,
// 256 bytes per row, the two 128-byte halves of a row swapped on rows with bit 2 set so that the two
// row groups one ds_write_b32 touches land in different banks), then read back as 4 consecutive
// columns per lane: every global access becomes one 16-byte (f32) or 8-byte (f16) vector and only a
// handful of registers are live per row group. Requires the whole wave tile in bounds, ldc/ldaux
// multiples of 4 and 16-byte aligned arrays (checked by the caller).

template <typename T>
struct Vec4 { typedef T type __attribute__((ext_vector_type(4))); };

// MI 32: the 32x32 accumulator layout's two row groups of one write are rows 4 apart, so bit 2 of the
// row swaps the halves. MI 16: the four row groups of a 16x16 layout's write are rows 4 apart, so bits
// 2-3 of the row rotate 16-column quarters.
template <int MI = 32>
__device__ __forceinline__ int epi_lds_off(int row, int col) {
    if constexpr (MI == 32) return row * 256 + ((col ^ ((row & 4) << 3)) << 2);
    else return row * 256 + ((col ^ (((row >> 2) & 3) << 4)) << 2);
}
// Row / column in its 32x32 block of element r of lane l of a wave's accumulators: MI 32 is the
// MFMA's own layout; MI 16 holds the block as four 16x16 MFMA blocks, quarter r/4 (row half, column
// half), element r%4 of lane l at row 4*(l/16) + r%4, column l%16 of the quarter.
template <int MI>
__device__ __forceinline__ int acc_row_mi(int r, int lane) {
    if constexpr (MI == 32) return acc_row(r, lane);
    else return 16 * (r >> 3) + 4 * (lane >> 4) + (r & 3);
}
template <int MI>
__device__ __forceinline__ int acc_col_mi(int r, int lane) {
    if constexpr (MI == 32) return lane & 31;
    else return 16 * ((r >> 2) & 1) + (lane & 15);
}

template <int EPI, typename T>
__device__ __forceinline__ floatx4 epi_in4(const GemmDesc &d, long m, int n) {
    if constexpr (EPI == EPI_SGD) return *(const floatx4 *)(d.W32 + m * d.ldc + n);
    else if constexpr (EPI == EPI_MASK || EPI == EPI_MSE) {
        typename Vec4<T>::type h = *(const typename Vec4<T>::type *)((const T *)d.aux + m * d.ldaux + n);
        return (floatx4){(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
    } else return (floatx4){};
}

// A wave's accumulators as FM x FN 32x32 blocks, element r of lane l of block (i, j): AccView32 over
// 32x32 MFMA blocks, AccView16 over 16x16 ones (block (i, j) is 16x16 blocks 2i..2i+1 x 2j..2j+1,
// quarter r/8 by row, (r/4)%2 by column, element r%4 of each; acc_row_mi<16> / acc_col_mi<16>).
template <int FM, int FN>
struct AccView32 {
    const floatx16 (&a)[FM][FN];
    __device__ __forceinline__ float operator()(int i, int j, int r) const { return a[i][j][r]; }
};
template <int FM, int FN>
struct AccView16 {
    const floatx4 (&a)[2 * FM][2 * FN];
    __device__ __forceinline__ float operator()(int i, int j, int r) const { return a[2 * i + (r >> 3)][2 * j + ((r >> 2) & 1)][r & 3]; }
};

template <int EPI, typename T, int FM, int FN, int MI, class View>
__device__ __forceinline__ void epilogue_lds_view(const GemmDesc &d, const View &acc, int mb, int nb, int lane, char *wlds);

template <int EPI, typename T, int FM, int FN, int MI = 32>
__device__ __forceinline__ void epilogue_lds(const GemmDesc &d, const floatx16 (&acc)[FM][FN], int mb, int nb, int lane,
                                             char *wlds) {
    epilogue_lds_view<EPI, T, FM, FN, MI>(d, AccView32<FM, FN>{acc}, mb, nb, lane, wlds);
}

template <int EPI, typename T, int FM, int FN, int MI, class View>
__device__ __forceinline__ void epilogue_lds_view(const GemmDesc &d, const View &acc, int mb, int nb, int lane, char *wlds) {
    constexpr int ROWS = FM * 32;
    constexpr int G = EPI == EPI_MSE ? 4 : 8;   // row groups whose inputs are loaded together
    typedef typename Vec4<T>::type T4;
    float lossp = 0.0f;
    // Scalars are read into locals: a struct field multiplied into a vector is lowered as a 16-byte
    // vector load at the field's address, which pins that part of the argument struct in memory.
    const float sc = d.scale, lr = d.lr;
    float *const colsum = d.colsum;
    const int colsum_ld = d.colsum_ld;
    void *const c2 = EPI == EPI_MASK ? d.C2 : nullptr;
    const int c4 = (lane & 15) * 4;
    // every slab's bias columns, loaded before the first slab (one load latency, not one per slab)
    floatx4 biasv[FN / 2];
#pragma unroll
    for (int jp = 0; jp < FN / 2; jp++) {
        biasv[jp] = (floatx4){};
        if constexpr (EPI == EPI_BIAS || EPI == EPI_BIAS_RELU || EPI == EPI_MSE) {
            const int n = nb + jp * 64 + c4;
            if constexpr (sizeof(T) == 2) {
                T4 b = *(const T4 *)((const T *)d.bias + n);
                biasv[jp] = (floatx4){(float)b[0], (float)b[1], (float)b[2], (float)b[3]};
            } else {
                biasv[jp] = *(const floatx4 *)((const float *)d.bias + n);
            }
        }
    }
#pragma unroll
    for (int jp = 0; jp < FN / 2; jp++) {
        // 1. accumulators -> LDS
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int jj = 0; jj < 2; jj++)
#pragma unroll
                for (int r = 0; r < 16; r++)
                    *(float *)(wlds + epi_lds_off<MI>(i * 32 + acc_row_mi<MI>(r, lane), jj * 32 + acc_col_mi<MI>(r, lane))) =
                        acc(i, 2 * jp + jj, r);
        __builtin_amdgcn_s_waitcnt(0xc07f);     // lgkmcnt(0): this wave's LDS writes have landed
        __builtin_amdgcn_wave_barrier();
        const int n = nb + jp * 64 + c4;
        const floatx4 bias = biasv[jp];
        floatx4 cs = {};
        // 2. LDS -> global, 4 rows per instruction (row = 4t + lane/16), G row groups at a time
#pragma unroll
        for (int t0 = 0; t0 < ROWS / 4; t0 += G) {
            floatx4 in[G];
#pragma unroll
            for (int u = 0; u < G; u++) in[u] = epi_in4<EPI, T>(d, (long)(mb + 4 * (t0 + u) + (lane >> 4)), n);
#pragma unroll
            for (int u = 0; u < G; u++) {
                const int row = 4 * (t0 + u) + (lane >> 4);
                const long m = mb + row;
                const floatx4 a = *(const floatx4 *)(wlds + epi_lds_off<MI>(row, c4));
                floatx4 v;
                if constexpr (EPI == EPI_STORE) {
                    v = sc * a;
                    T4 o = {(T)v[0], (T)v[1], (T)v[2], (T)v[3]};
                    *(T4 *)((T *)d.C + m * d.ldc + n) = o;
                } else if constexpr (EPI == EPI_BIAS || EPI == EPI_BIAS_RELU) {
                    T4 o;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        float z = sizeof(T) == 2 ? q16(q16(a[e]) + bias[e]) : a[e] + bias[e];
                        o[e] = EPI == EPI_BIAS_RELU ? relu_tag((T)z) : (T)z;
                    }
                    *(T4 *)((T *)d.C + m * d.ldc + n) = o;
                    v = (floatx4){};
                } else if constexpr (EPI == EPI_MSE) {
                    T4 o;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float p = q16(q16(a[e]) + bias[e]);
                        const float diff = p - in[u][e];
                        lossp += diff * diff;
                        v[e] = q16(diff);
                        o[e] = (T)v[e];
                    }
                    *(T4 *)((T *)d.C + m * d.ldc + n) = o;
                } else if constexpr (EPI == EPI_MASK) {
                    T4 o;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        v[e] = relu_dead(in[u][e]) ? 0.0f : sc * a[e];
                        o[e] = (T)v[e];
                    }
                    *(T4 *)((T *)d.C + m * d.ldc + n) = o;
                    if (sizeof(T) == 2 && c2) {   // the rounding residue as a second f16 plane
                        T4 lo;
#pragma unroll
                        for (int e = 0; e < 4; e++) lo[e] = (T)(v[e] - (float)o[e]);
                        *(T4 *)((T *)c2 + m * d.ldc + n) = lo;
                    }
                } else {  // EPI_SGD
                    const floatx4 g = sc * a;
                    if (d.gout) *(floatx4 *)(d.gout + m * d.ldc + n) = g;
                    floatx4 w = in[u] - lr * g;
                    // W16 must be f16 of the stored W32: the empty asm pins w as one f32 value, so the
                    // compiler cannot fold the f16 conversion into a differently rounded fused op
                    asm volatile("" : "+v"(w));
                    *(floatx4 *)(d.W32 + m * d.ldc + n) = w;
                    if (d.W16) {
                        typedef half_t h4 __attribute__((ext_vector_type(4)));
                        h4 w16 = {(half_t)w[0], (half_t)w[1], (half_t)w[2], (half_t)w[3]};
                        *(h4 *)((half_t *)d.W16 + m * d.ldc + n) = w16;
                    }
                    v = (floatx4){};
                }
                cs += v;
            }
        }
        if (colsum) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float x = cs[e];
                x += __shfl_xor(x, 16, 64);
                x += __shfl_xor(x, 32, 64);
                cs[e] = x;
            }
            if (lane < 16) {
                float *const row = colsum + (long)(mb / 32) * colsum_ld;   // colsum itself when atomic
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    if (colsum_ld) row[n + e] = cs[e];
                    else atomicAdd(colsum + n + e, cs[e]);
                }
            }
        }
        __builtin_amdgcn_wave_barrier();
    }
    if constexpr (EPI == EPI_MSE) {
        lossp = wave_sum(lossp);
        if (lane == 0) {
            if (d.loss_ld) d.lossacc[(long)(mb / 32) * d.loss_ld + nb / 32] = lossp;
            else atomicAdd(d.lossacc, lossp);
        }
    }
}

}  // namespace ah
