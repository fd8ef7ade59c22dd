// gemm.h — descriptor for the MFMA contraction templates (host + device).
//
// One descriptor covers every GEMM-shaped REDUCE(ADD, MUL(..)) the reference scheduler emits for a
// Linear layer (tensor/reduce.go:105-166 via tensor/nn/nn.go:154-162) and its backward
// (tensor/gradient_ruleset.go:137-140, 207-233, 285-306):
//   C[m,n] = epilogue( sum_k A(m,k) * B(n,k) )
// A(m,k) is read from a row-major [M,K] array (ta=0, "K-contiguous") or a [K,M] array (ta=1);
// B(n,k) from [N,K] (tb=0) or [K,N] (tb=1). Forward Linear is (0,0); dX = dY·W is (0,1);
// dW = dYᵀ·X is (1,1).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ah {

// Number of f16 kernel variants (table Var<V> in gemm16_kernel.h); variant 0 means the tuned choice.
constexpr int kGemm16Variants = 39;
// Split-K workspace of a device: counters for up to kSplitKMaxTiles tiles, then kSplitKPartFloats floats.
constexpr int kSplitKMaxTiles = 4096;
constexpr long kSplitKPartFloats = 4L << 20;

enum GemmDtype : int { GEMM_F32 = 0, GEMM_F16 = 1 };

enum GemmEpi : int {
    EPI_STORE = 0,      // C = scale*acc
    EPI_BIAS = 1,       // C = acc + bias[n]            (f16: f16(f16(acc) + bias))
    EPI_BIAS_RELU = 2,  // C = relu_tag(acc + bias[n])
    EPI_MSE = 3,        // f16: P = f16(f16(acc)+bias); C = f16(P - aux); loss += (P-aux)^2; colsum += C
    EPI_MASK = 4,       // C = relu_dead(aux) ? 0 : scale*acc; colsum += C (unrounded)
    EPI_SGD = 5,        // g = scale*acc; gout = g (opt); W32 -= lr*g; W16 = f16(W32) (opt)
};

struct GemmDesc {
    int dtype;        // GemmDtype of A and B
    int epi;          // GemmEpi
    int ta, tb;       // operand layouts (see above)
    int M, N, K;
    const void *A;
    const void *B;
    long lda, ldb;    // row strides of the stored arrays, in elements
    void *C;          // output (type = dtype, except EPI_SGD which writes W32/W16)
    long ldc;
    const void *bias; // [N], type = dtype
    const void *aux;  // [M,N] with ldaux, type = dtype (MSE targets / ReLU activations)
    long ldaux;
    float *colsum;    // [N] f32 accumulator (atomic), optional
    float *W32;       // EPI_SGD master weights [M,N] (row stride ldc)
    void *W16;        // EPI_SGD f16 copy, optional
    float *gout;      // EPI_SGD gradient output [M,N] (row stride ldc), optional
    float *lossacc;   // EPI_MSE scalar accumulator
    // Two-plane adjoint (f16 kernels): with A2 set the contraction runs over K twice, the second pass
    // reading A2 (same layout and lda as A) against the same B: C = epi(sum_k (A + A2)(m,k) B(n,k)). An f32
    // operand carried as hi = f16(a), lo = f16(a - hi) keeps ~22 bits of it through f16 MFMAs.
    const void *A2;
    // EPI_MASK of an f16 contraction: with C2 set, the f32 value v is stored as C = f16(v) and
    // C2 = f16(v - f16(v)) (the two planes a following two-plane contraction reads)
    void *C2;
    int tile;         // 0 = auto, else 64 / 128 / 256 (square tiles)
    int variant;      // f16 kernel variant (0 = auto; table Var<V> in gemm16_kernel.h), the tuning hook
    int kgroups;      // f32 tiled kernel: wave sets splitting K (0 = auto, else 1 / 2 / 4 as the tile admits;
                      // a fixed value also turns off the automatic split of K across workgroups)
    int splits;       // f32 tiled kernel: workgroups splitting K per tile (0 = auto, 1 = none, else 2..16;
                      // needs the split-K workspace below, without which there is no split)
    // Deterministic partial sums instead of atomics (0 = atomic accumulation into colsum[N] / lossacc[0]):
    // with colsum_ld > 0 each wave stores the column sums of its rows, which start at a multiple of 32,
    // to colsum[(row / 32) * colsum_ld + n]; with loss_ld > 0 each wave stores its MSE partial to
    // lossacc[(row / 32) * loss_ld + col / 32] (row, col: the wave tile's first element). Entries no
    // wave writes are left as they are, so the reader sums every entry and re-zeroes it.
    int colsum_ld;
    int loss_ld;
    // Split-K workspace of the f32 tiled kernel (shapes with too few tiles for the CUs and a long K): two
    // ints per tile, the first its arrival counter, zero between launches (the finishing workgroup
    // resets it), then f32 partial tiles, sk_cap floats. Null: no split. Filled in by the dispatcher.
    int *sk_sync;
    float *sk_part;
    long sk_cap;
    // The float scalars sit beside the ints, away from the pointers: the compiler may merge loads of
    // neighbouring fields into one vector, and a vector mixing pointers and floats is kept in memory.
    float scale;
    float lr;
};

// Two independent f16 contractions in one launch (gemm16_pair.hip): d0's tiles split over K into
// nsplit workgroups each, then d1's tiles (items1 of them; none for a split d0 alone).
struct G16PairArgs {
    GemmDesc d0, d1;
    int nsplit;     // K splits of each d0 tile
    int items0;     // d0 workgroups: tiles x nsplit
    int *count;     // one arrival counter per d0 tile, zero before and after a launch
    float *part;    // tiles x nsplit partial tiles of BM*BM floats
};
// Variants a paired launch can use (256x256 tiles, one k-group).
constexpr int kG16PairVariants[] = {27, 30};
// Launches the pair with `variant` when the shapes, layouts and epilogues admit it (every tile whole,
// vector epilogues, K/nsplit whole stages); returns false, launching nothing, otherwise.
bool gemm16_pair_try_launch(const GemmDesc &d0, int nsplit, const GemmDesc *d1, int variant, int *count,
                            float *part, long part_floats, hipStream_t s, hipError_t *err);

hipError_t gemm_launch(const GemmDesc &d, hipStream_t s);
bool gemm16_try_launch(const GemmDesc &d, hipStream_t s, hipError_t *err);

// Template parameters of an f16 variant (table Var<V> in gemm16_kernel.h): tile BM x BN, wave layout
// WVM x WVN, k per LDS stage BK, stages in flight NS, fetch mode, cross-barrier prefetch XB, k-groups KG.
struct G16Params {
    int bm, bn, wvm, wvn, bk, ns, fetch, xb, kg, mi;   // mi: MFMA shape, 32 (32x32x16) or 16 (16x16x32)
};
bool gemm16_variant_params(int variant, G16Params *out);
// The variant an f16 contraction with variant 0 and no tuned choice runs (chosen by shape).
int gemm16_default_variant(const GemmDesc &d);
// f32 contractions with direct global->LDS stages (gemm32d.hip): GemmDesc::tile = kGemm32dBase + i selects
// configuration i (tile, k per stage, stages in flight) of gemm32d_config; kgroups does not apply, and
// splits > 1 splits K across workgroups as the register-staged kernel does (gemm32d_splits). A shape a
// configuration does not take (gemm32d_ok) runs the automatic choice instead (gemm_launch).
constexpr int kGemm32dBase = 1000, kGemm32dConfigs = 5;
bool gemm32d_config(int tile, int *bm, int *bk, int *ns);
bool gemm32d_ok(const GemmDesc &d, int bm, int bk);
int gemm32d_splits(const GemmDesc &d, int bm, int bk);
hipError_t gemm32d_launch(const GemmDesc &d, hipStream_t s);
// k-groups an f32 tile size admits (LDS budget): 64 -> 1, 2, 4; 128 -> 1, 2; 256 -> 1.
inline bool gemm32_kgroups_ok(int tile, int kg) {
    return kg == 1 || (kg == 2 && tile <= 128) || (kg == 4 && tile == 64);
}

}  // namespace ah
