// gemm16_var.hip — one f16 contraction variant per translation unit. The Makefile compiles this file
// once per variant with -DAH_G16_V=<n>, so the variants build in parallel.
#include "gemm16_kernel.h"

#ifndef AH_G16_V
#error "compile with -DAH_G16_V=<variant>"
#endif
#define AH_G16_NAME2(n) gemm16_variant_##n
#define AH_G16_NAME(n) AH_G16_NAME2(n)

namespace ah {
hipError_t AH_G16_NAME(AH_G16_V)(const GemmDesc &d, hipStream_t s) { return g16::run_variant<AH_G16_V>(d, s); }
}  // namespace ah
