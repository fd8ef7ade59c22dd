// convnet.h — host launcher of the sample-parallel conv-net train step (config 2).
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

// True when the two kernels' LDS working sets fit 64 KiB per workgroup (and the fc sizes fit their
// register/thread mapping); otherwise the per-op kernels of conv.h serve the step.
bool convnet_fused_ok(int Hin, int C1, int C2, int NC);
// Floats of the workspace the two kernels exchange through, for batches up to N.
long convnet_fused_ws_floats(int N, int Hin, int C1, int C2, int NC);
// Forward: workgroups over samples x conv2 channel groups; writes the pooled planes, window bytes and
// partial logits to ws.
hipError_t convnet_fwd_fused(const float *x, const float *cw1, const float *cb1, const float *cw2, const float *cb2,
                             const float *fw, int B, int Hin, int C1, int C2, int NC, float *ws, hipStream_t s);
// Backward: workgroups over samples x conv1 channels; softmax-CE (rowloss[n] = the label's
// log-probability, the logit gradient scaled by a), then sample n's parameter gradients to
// part[n * total ..].
hipError_t convnet_bwd_fused(const float *x, const int32_t *lab, const float *cw2, const float *fw, const float *fb, int B,
                             int Hin, int C1, int C2, int NC, float a, const float *ws, float *rowloss, float *part,
                             hipStream_t s);

}  // namespace ah
