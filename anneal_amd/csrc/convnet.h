// convnet.h — host launcher of the fused one-sample-per-workgroup conv-net train step (config 2).
#pragma once
#include "ah_common.h"

namespace ah {

// Offsets (floats) of each parameter's gradient inside one sample's row of the partial buffer; the row
// stride is `total`.
struct NetPart {
    long cw1, cb1, cw2, cb2, fw, fb, total;
};
__host__ __device__ inline NetPart net_part(int Hin, int C1, int C2, int NC) {
    const long F = (long)C2 * (Hin / 4) * (Hin / 4);
    NetPart o;
    o.cw1 = 0;
    o.cb1 = o.cw1 + (long)C1 * 9;
    o.cw2 = o.cb1 + C1;
    o.cb2 = o.cw2 + (long)C2 * C1 * 9;
    o.fw = o.cb2 + C2;
    o.fb = o.fw + (long)NC * F;
    o.total = o.fb + NC;
    return o;
}

// True when a sample's working set fits one workgroup's LDS (64 KiB); otherwise the per-op kernels of
// conv.h serve the step.
bool convnet_fused_ok(int Hin, int C1, int C2, int NC);
size_t convnet_fused_lds_bytes(int Hin, int C1, int C2, int NC);
// One workgroup per sample: forward, softmax-CE (rowloss[n] = the label's log-probability, the logit
// gradient scaled by a) and backward; writes sample n's parameter gradients to part[n * total ..].
hipError_t convnet_step_fused(const float *x, const int32_t *lab, const float *cw1, const float *cb1, const float *cw2,
                              const float *cb2, const float *fw, const float *fb, int B, int Hin, int C1, int C2, int NC,
                              float a, float *rowloss, float *part, hipStream_t s);

}  // namespace ah
