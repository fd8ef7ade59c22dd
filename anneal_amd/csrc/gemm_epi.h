// gemm_epi.h — fused GEMM epilogues shared by the contraction kernels.
#pragma once
#include "ah_common.h"
#include "gemm.h"

namespace ah {

// ── Epilogues ────────────────────────────────────────────────────────────────
// Each returns the value that enters the per-column sum (bias gradient), or 0.

template <int EPI, typename T>
__device__ __forceinline__ float epilogue(const GemmDesc &d, int m, int n, float acc, float &lossp) {
    T *C = (T *)d.C;
    long ci = (long)m * d.ldc + n;
    if constexpr (EPI == EPI_STORE) {
        float v = d.scale * acc;
        C[ci] = (T)v;
        return v;
    } else if constexpr (EPI == EPI_BIAS || EPI == EPI_BIAS_RELU) {
        float z;
        if constexpr (sizeof(T) == 2) z = q16(q16(acc) + (float)((const T *)d.bias)[n]);
        else z = acc + ((const float *)d.bias)[n];
        if constexpr (EPI == EPI_BIAS_RELU) C[ci] = relu_tag((T)z);
        else C[ci] = (T)z;
        return 0.0f;
    } else if constexpr (EPI == EPI_MSE) {
        float p = q16(q16(acc) + (float)((const T *)d.bias)[n]);
        float t = (float)((const T *)d.aux)[(long)m * d.ldaux + n];
        float diff = p - t;
        lossp += diff * diff;
        float dd = q16(diff);
        C[ci] = (T)dd;
        return dd;
    } else if constexpr (EPI == EPI_MASK) {
        T h = ((const T *)d.aux)[(long)m * d.ldaux + n];
        float v = relu_dead(h) ? 0.0f : d.scale * acc;
        C[ci] = (T)v;
        return v;
    } else {  // EPI_SGD
        float g = d.scale * acc;
        if (d.gout) d.gout[ci] = g;
        float w = d.W32[ci];
        w = w - d.lr * g;
        d.W32[ci] = w;
        if (d.W16) ((half_t *)d.W16)[ci] = (half_t)w;
        return 0.0f;
    }
}

}  // namespace ah
