// rowops.h — host launchers for row reductions, elementwise and chain kernels.
#pragma once
#include "ah_common.h"

namespace ah {

constexpr int kChainStatsRows = 64;   // rows per pass-1 block (chunk partials folded per column)
constexpr int kChainGradRows = 32;    // rows per pass-2 block
constexpr int kTailCols = 32;         // step tail: elements per block pass (one per thread of a chunk)
constexpr int kTailChunks = 16;       // step tail: row chunks of a partial-row accumulator

hipError_t fill_f32(float *p, long n, float v, hipStream_t s);
// p[i] and/or p16[i] = amp * (a hash of (seed, i) mapped to [-1, 1)); either pointer may be null.
hipError_t fill_hash(float *p, half_t *p16, long n, uint32_t seed, float amp, hipStream_t s);
hipError_t cast_f32_f16(const float *src, half_t *dst, long n, hipStream_t s);
hipError_t sgd_update(float *p, const float *g, long n, float lr, float scale, half_t *p16, float *gout,
                      hipStream_t s);
hipError_t colsum_add(const float *G, int M, int N, long ld, float *out, hipStream_t s);
// softmax_ce plus the column sums of dz as partial rows part[softmax_ce_cols_blocks(B)][C] (each row
// rewritten by every call; their row-order sum is the output bias gradient). C <= kSoftmaxColsMaxC.
constexpr int kSoftmaxColsMaxC = 1024;
constexpr int kSoftmaxColsMaxBlocks = 256;
int softmax_ce_cols_blocks(int B);
hipError_t softmax_ce_cols(const float *z, const int32_t *labels, int B, int C, float a, float *dz, float *rowloss,
                           float *part, hipStream_t s);
hipError_t softmax_ce(const float *z, const int32_t *labels, int B, int C, float a, float *dz, float *rowloss,
                      hipStream_t s);
hipError_t sum_scale(const float *v, int n, float a, float *out, hipStream_t s);
hipError_t mse_finalize(const float *acc, float scale, float *out, hipStream_t s);

struct TailSeg {
    float *p;        // f32 master parameter
    half_t *p16;     // optional f16 copy
    float *acc;      // gradient accumulator (re-zeroed)
    float *gout;     // optional gradient output
    long n;
    float scale;     // gradient = scale * acc
    int acc_rows;    // > 0: acc holds acc_rows partial rows (row stride acc_ld), summed in row order
    long acc_ld;
    int keep;        // nonzero: leave acc as it is (its producer rewrites it every step)
};
struct TailArgs {
    TailSeg seg[6];
    int nseg;
    float lr;
    int loss_mode;   // 0 none, 1 f16-narrowed accumulator * loss_scale, 2 sum(rowloss) * loss_scale
    float *lossacc;
    int loss_parts;  // loss_mode 1: > 0 sums lossacc[0 .. loss_parts) in a fixed order (and re-zeroes)
    float loss_scale;
    const float *rowloss;
    int nrow;
    float *loss_out;
    float *loss_sum;  // loss_mode 1, optional: the f32 sum before the f16 narrowing
};
hipError_t step_tail(const TailArgs &t, hipStream_t s);

long chain_workspace_floats(int R, int Cc);
// Capacity (floats) of the file-scope chain workspace used by ah_chain_step_noalloc, and its address on
// the device `ordinal` (the current device at the call).
long chain_scratch_floats();
hipError_t chain_scratch_init(int ordinal, float **out);
// Config 5 with each 16-column strip of X held on chip (one pass over HBM): for R = 4096 or 8192 and
// Cc a multiple of 16. lossp: Cc/16 floats; counter: one int, zero before the call and left zero.
bool chain_resident_fits(int R, int Cc);
hipError_t chain_resident(const float *X, const float *g, int R, int Cc, float *lossp, int *counter, float *dX, float *dg,
                          float *loss, hipStream_t s);
// The whole config-5 chain (phase -1: the resident kernel where it fits, else the three kernels below)
// or one of its three kernels (phase 0 stats, 1 finalize, 2 gradient). work: chain_workspace_floats
// floats whose first word is zero before the first call (every call leaves it zero).
hipError_t chain_step(const float *X, const float *g, int R, int Cc, float *work, float *dX, float *dg, float *loss,
                      hipStream_t s, int phase = -1);

}  // namespace ah
