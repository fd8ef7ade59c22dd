// conv.h — host launchers for the config-2 convolution / pooling kernels.
#pragma once
#include "ah_common.h"

namespace ah {

hipError_t conv_fwd_relu_pool(const float *X, int N, int Ci, int H, const float *w, const float *b, int Co, float *Hout,
                              float *Pout, hipStream_t s);
hipError_t pool_relu_bwd(const float *dP, const float *Hact, const float *Pv, int NC, int H, float *dZ, hipStream_t s);
hipError_t conv_bwd_x(const float *G, const float *w, int N, int Ci, int H, int Co, float *dX, hipStream_t s);
// Weight/bias gradient with SGD in two launches: partial sums over position splits, then a
// deterministic fold + update. `part` holds conv_bwd_w_splits(..) * Co * Ci * 10 floats.
int conv_bwd_w_splits(int N, int Ci, int H, int Co);
hipError_t conv_bwd_w_partial(const float *X, const float *G, int N, int Ci, int H, int Co, float *part, hipStream_t s);
hipError_t conv_bwd_w_finalize(const float *part, int N, int Ci, int H, int Co, float *w, float *b, float lr, float *gw,
                               float *gb, hipStream_t s);

}  // namespace ah
