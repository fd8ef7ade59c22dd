// mlpce.h — host launchers of the three-kernel MLP softmax-CE train step (config 1's shape class).
#pragma once
#include "ah_common.h"

namespace ah {

// True when the three kernels serve the shape: batch B up to 64, hidden width H up to 128, at most 16
// classes, input width D up to 896 (otherwise the GEMM-based step serves it).
bool mlpce_fused_ok(int B, int D, int H, int C);

// Hidden layer: Hout[n][j] = ReLU(x[n] . W1[j] + b1[j]) (ReLU outputs sign-tagged as the GEMM epilogue
// writes them), W1 stored [H][D].
hipError_t mlpce_hidden(const float *x, const float *W1, const float *b1, int B, int D, int H, float *Hout,
                        hipStream_t s);

// Parameters updated by the gradient kernel, their gradient outputs (null: not stored), the SGD step and
// the loss (sum of the rows' label log-probabilities times loss_scale).
struct MlpSgd {
    float *W1, *b1, *W2, *b2;
    float *gW1, *gb1, *gW2, *gb2;
    float lr, loss_scale;
    float *loss;
};
// Softmax-CE and the hidden-layer gradient, one wave per sample: dz (the logit gradient, scaled by a),
// dH (zero where the ReLU was off) and rowloss (the label's log-probability).
hipError_t mlpce_head(const int32_t *lab, const float *Hin, const float *W2, const float *b2, int B, int H, int C,
                      float a, float *dz, float *dH, float *rowloss, hipStream_t s);
// Weight gradients over the batch and SGD for every parameter, and the loss.
hipError_t mlpce_grad(const float *x, const float *Hin, const float *dz, const float *dH, const float *rowloss, int B,
                      int D, int H, int C, const MlpSgd &sgd, hipStream_t s);

// Small batches (B <= 8) at wide layers (D % 4 == 0, H % 4 == 0, C <= 512; config 4 at N = 1 and 7):
// part 0 the hidden layer into Hbuf, 1 the logits into Z, 2 softmax-CE (dz, rowloss) and dH, 3 every
// weight gradient with SGD, the biases and the loss. Launched in that order on one stream.
bool mlp_small_ok(int B, int D, int H, int C);
hipError_t mlp_small_step(const float *x, const int32_t *lab, int B, int D, int H, int C, float a, float *Hbuf,
                          float *Z, float *dz, float *dH, float *rowloss, const MlpSgd &S, hipStream_t s, int part);

}  // namespace ah
