// conv.h — host launchers for the config-2 convolution / pooling kernels.
#pragma once
#include "ah_common.h"

namespace ah {

hipError_t conv_fwd_relu_pool(const float *X, int N, int Ci, int H, const float *w, const float *b, int Co, float *Hout,
                              float *Pout, hipStream_t s);
hipError_t pool_relu_bwd(const float *dP, const float *Hact, const float *Pv, int NC, int H, float *dZ, hipStream_t s);
hipError_t conv_bwd_x(const float *G, const float *w, int N, int Ci, int H, int Co, float *dX, hipStream_t s);
hipError_t conv_bwd_w_sgd(const float *X, const float *G, int N, int Ci, int H, int Co, float *w, float *b, float lr,
                          float *gw, float *gb, hipStream_t s);

}  // namespace ah
