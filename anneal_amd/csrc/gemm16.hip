// gemm16.hip — host dispatch of the f16 MFMA contraction (kernel template: gemm16_kernel.h; each
// variant is compiled in its own translation unit from gemm16_var.hip).
#include "gemm16_kernel.h"

namespace ah {

#define AH_G16_DECL(n) hipError_t gemm16_variant_##n(const GemmDesc &d, hipStream_t s);
AH_G16_DECL(1) AH_G16_DECL(2) AH_G16_DECL(3) AH_G16_DECL(4) AH_G16_DECL(5) AH_G16_DECL(6) AH_G16_DECL(7)
AH_G16_DECL(8) AH_G16_DECL(9) AH_G16_DECL(10) AH_G16_DECL(11) AH_G16_DECL(12) AH_G16_DECL(13)
AH_G16_DECL(14) AH_G16_DECL(15) AH_G16_DECL(16) AH_G16_DECL(17) AH_G16_DECL(18) AH_G16_DECL(19)
AH_G16_DECL(20) AH_G16_DECL(21) AH_G16_DECL(22) AH_G16_DECL(23) AH_G16_DECL(24) AH_G16_DECL(25)
AH_G16_DECL(26) AH_G16_DECL(27) AH_G16_DECL(28)
AH_G16_DECL(29) AH_G16_DECL(30) AH_G16_DECL(31)
AH_G16_DECL(32) AH_G16_DECL(33) AH_G16_DECL(34) AH_G16_DECL(35) AH_G16_DECL(36) AH_G16_DECL(37)
AH_G16_DECL(38) AH_G16_DECL(39)
#undef AH_G16_DECL

namespace {
typedef hipError_t (*VariantFn)(const GemmDesc &, hipStream_t);
const VariantFn kVariants[g16::kMaxVariant + 1] = {
    nullptr, gemm16_variant_1, gemm16_variant_2, gemm16_variant_3, gemm16_variant_4, gemm16_variant_5,
    gemm16_variant_6, gemm16_variant_7, gemm16_variant_8, gemm16_variant_9, gemm16_variant_10,
    gemm16_variant_11, gemm16_variant_12, gemm16_variant_13, gemm16_variant_14, gemm16_variant_15,
    gemm16_variant_16, gemm16_variant_17, gemm16_variant_18, gemm16_variant_19, gemm16_variant_20,
    gemm16_variant_21, gemm16_variant_22, gemm16_variant_23, gemm16_variant_24, gemm16_variant_25,
    gemm16_variant_26, gemm16_variant_27, gemm16_variant_28,
    gemm16_variant_29, gemm16_variant_30, gemm16_variant_31, gemm16_variant_32, gemm16_variant_33,
    gemm16_variant_34, gemm16_variant_35, gemm16_variant_36, gemm16_variant_37, gemm16_variant_38,
    gemm16_variant_39};

// k-groups of the variant (the K split must give each group whole 64-wide stages)
int variant_kgroups(int v) {
    switch (v) {
#define AH_G16_KG(n) case n: return g16::Var<n>::KG;
        AH_G16_KG(1) AH_G16_KG(2) AH_G16_KG(3) AH_G16_KG(4) AH_G16_KG(5) AH_G16_KG(6) AH_G16_KG(7)
        AH_G16_KG(8) AH_G16_KG(9) AH_G16_KG(10) AH_G16_KG(11) AH_G16_KG(12) AH_G16_KG(13)
        AH_G16_KG(14) AH_G16_KG(15) AH_G16_KG(16) AH_G16_KG(17) AH_G16_KG(18) AH_G16_KG(19)
        AH_G16_KG(20) AH_G16_KG(21) AH_G16_KG(22) AH_G16_KG(23) AH_G16_KG(24) AH_G16_KG(25)
        AH_G16_KG(26) AH_G16_KG(27) AH_G16_KG(28)
        AH_G16_KG(29) AH_G16_KG(30) AH_G16_KG(31)
        AH_G16_KG(32) AH_G16_KG(33) AH_G16_KG(34) AH_G16_KG(35) AH_G16_KG(36) AH_G16_KG(37)
        AH_G16_KG(38) AH_G16_KG(39)
#undef AH_G16_KG
        default: return 1;
    }
}
}  // namespace

bool gemm16_variant_params(int v, G16Params *out) {
    switch (v) {
#define AH_G16_P(n)                                                                                          \
    case n:                                                                                                  \
        *out = {g16::Var<n>::BM, g16::Var<n>::BM, g16::Var<n>::WVM, g16::Var<n>::WVN, g16::Var<n>::BK,     \
                g16::Var<n>::NS, g16::Var<n>::FETCH, g16::Var<n>::XB ? 1 : 0, g16::Var<n>::KG, g16::Var<n>::MI};            \
        return true;
        AH_G16_P(1) AH_G16_P(2) AH_G16_P(3) AH_G16_P(4) AH_G16_P(5) AH_G16_P(6) AH_G16_P(7)
        AH_G16_P(8) AH_G16_P(9) AH_G16_P(10) AH_G16_P(11) AH_G16_P(12) AH_G16_P(13)
        AH_G16_P(14) AH_G16_P(15) AH_G16_P(16) AH_G16_P(17) AH_G16_P(18) AH_G16_P(19)
        AH_G16_P(20) AH_G16_P(21) AH_G16_P(22) AH_G16_P(23) AH_G16_P(24) AH_G16_P(25)
        AH_G16_P(26) AH_G16_P(27) AH_G16_P(28) AH_G16_P(29) AH_G16_P(30) AH_G16_P(31)
        AH_G16_P(32) AH_G16_P(33) AH_G16_P(34) AH_G16_P(35) AH_G16_P(36) AH_G16_P(37) AH_G16_P(38) AH_G16_P(39)
#undef AH_G16_P
        default: return false;
    }
}

int gemm16_default_variant(const GemmDesc &d) {
    int tile = d.tile;
    if (tile == 0) {
        long t256 = (long)((d.M + 255) / 256) * ((d.N + 255) / 256);
        tile = t256 >= 224 ? 256 : 128;
    }
    return tile == 256 ? 3 : 1;
}

// Returns true (and launches) when the shape/alignment admits the direct-to-LDS f16 kernel.
bool gemm16_try_launch(const GemmDesc &d, hipStream_t s, hipError_t *err) {
    using namespace g16;
    if (d.dtype != GEMM_F16 || d.K <= 0 || d.K % 64) return false;   // every variant's stage divides 64
    if (d.tile != 0 && d.tile != 128 && d.tile != 256) return false;
    if (d.variant < 0 || d.variant > kMaxVariant) return false;
    int v = d.variant;
    if (v == 0) v = gemm16_default_variant(d);   // by shape: 256x256 tiles when they fill the chip, else 128x128
    if (d.K % (64 * variant_kgroups(v))) return false;   // k-groups contract whole stages
    bool ok = (d.ta ? operand_ok<1>(d.A, d.lda, d.M) : operand_ok<0>(d.A, d.lda, d.M)) &&
              (d.tb ? operand_ok<1>(d.B, d.ldb, d.N) : operand_ok<0>(d.B, d.ldb, d.N));
    if (ok && d.A2) ok = d.ta ? operand_ok<1>(d.A2, d.lda, d.M) : operand_ok<0>(d.A2, d.lda, d.M);
    if (!ok) return false;
    *err = kVariants[v](d, s);
    return true;
}

hipError_t gemm16_pair_variant_27(const G16PairArgs &p, int items1, bool *supported, hipStream_t s);
hipError_t gemm16_pair_variant_30(const G16PairArgs &p, int items1, bool *supported, hipStream_t s);

namespace {
// The vector (LDS-staged) epilogue's conditions with every tile whole.
bool pair_operand_ok(const GemmDesc &d, int bm) {
    using namespace g16;
    if (d.dtype != GEMM_F16 || d.M % bm || d.N % bm || d.K % 64 || d.ldc % 4 || d.ldaux % 4 || d.A2 || d.C2) return false;
    const uintptr_t a = (uintptr_t)d.C | (uintptr_t)d.aux | (uintptr_t)d.bias | (uintptr_t)d.W32 |
                        (uintptr_t)d.W16 | (uintptr_t)d.gout;
    if (a & 15) return false;
    return (d.ta ? operand_ok<1>(d.A, d.lda, d.M) : operand_ok<0>(d.A, d.lda, d.M)) &&
           (d.tb ? operand_ok<1>(d.B, d.ldb, d.N) : operand_ok<0>(d.B, d.ldb, d.N));
}
}  // namespace

bool gemm16_pair_try_launch(const GemmDesc &d0, int nsplit, const GemmDesc *d1, int variant, int *count,
                            float *part, long part_floats, hipStream_t s, hipError_t *err) {
    using namespace g16;
    constexpr int BM = 256;
    if (variant != 27 && variant != 30) return false;
    static_assert(Var<27>::BM == BM && Var<30>::BM == BM && Var<27>::KG == 1 && Var<30>::KG == 1, "pair variants");
    if (nsplit < 1 || nsplit > 8 || d0.K % (64 * nsplit)) return false;
    if (!pair_operand_ok(d0, BM) || (d1 && !pair_operand_ok(*d1, BM))) return false;
    const long tiles0 = (long)(d0.M / BM) * (d0.N / BM);
    if (nsplit > 1 && (!count || !part || tiles0 * nsplit * BM * BM > part_floats)) return false;
    G16PairArgs p;
    p.d0 = d0;
    if (d1) p.d1 = *d1;
    else p.d1 = d0;
    p.nsplit = nsplit;
    p.items0 = (int)(tiles0 * nsplit);
    p.count = count;
    p.part = part;
    const int items1 = d1 ? (d1->M / BM) * (d1->N / BM) : 0;
    bool supported = false;
    hipError_t e = variant == 27 ? gemm16_pair_variant_27(p, items1, &supported, s)
                                 : gemm16_pair_variant_30(p, items1, &supported, s);
    if (!supported) return false;
    *err = e;
    return true;
}

}  // namespace ah
