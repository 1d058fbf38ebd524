// Host interface of the narrow output-layer kernels (skinny.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>

#include "device_common.h"

namespace volta {

struct OutLayerArgs {
  const float* act;   // act_{n-1} [B x K]
  const float* W;     // W_{n-1} [K x N]
  const float* bias;  // b_{n-1} [N]
  int B, K, N;
  int loss;           // enum volta_loss
  const float* y;     // MSE targets [B x N]
  const int32_t* labels;  // CE labels [B]
  float* out;         // act_n = z [B x N]
  float* delta;       // delta_{n-1} [B x N]
  float* partials;    // per-block loss (when more than one block)
  DevScalars* scalars;
  const float2* bc_table;
  int bc_len;
  // launch_out_layer_dx only: delta_{n-2} = (delta_{n-1} W^T) * f'(layer n-2)
  int dx_act;               // activation of layer n-2 (enum volta_activation)
  const float* dx_pre;      // its pre-activation [B x K] (null when not kept)
  float* dx_out;            // delta_{n-2} [B x K]
  unsigned* loss_counter;   // arrival ticket of the blocks (zero between launches)
  // launch_out_layer_dx only: 1 = leave the loss sum to a later launch (the
  // dW group of the step): the blocks only store their partials, block 0
  // advances the step counter, and no arrival ticket is taken
  int defer_loss;
};

struct NarrowDwArgs {
  const float* act;    // act_i [B x R]
  const float* delta;  // delta_i [B x N]
  int B, R, N;
  int opt;             // enum volta_optimizer (AdamW as Adam with wd)
  float* w;            // W_i [R x N], updated in place
  float* m;            // Adam m / Adagrad G for W_i
  float* v;            // Adam v for W_i
  float* b;            // b_i [N]
  float* bm;
  float* bv;
  float* grad;         // optional dW copy
  float* bgrad;        // optional db copy
  float wd, b1, b2, eps;
  DevScalars* scalars;
};

// Largest batch the narrow dW serves (one round of four 64-row chunks of
// the batch); larger batches take the TN GEMM.
constexpr int kNarrowMaxB = 256;

int out_layer_blocks(int B);
hipError_t launch_out_layer(const OutLayerArgs& p, hipStream_t st);
// The output layer, its loss head and the output layer's dX in one launch
// (one batch row per wave, 4 rows per block; the last block to finish adds
// the blocks' losses in block order).  For B <= kNarrowMaxB with a
// K x N W of at most kOutWlFloats floats when N > 1.
int out_layer_dx_blocks(int B);
bool out_layer_dx_supported(int B, int K, int N);
hipError_t launch_out_layer_dx(const OutLayerArgs& p, hipStream_t st);
// The step's loss from the per-strip partials an earlier output launch
// stored (launch_smallm_out_head), added by block (0, 0) of a later launch
// in a fixed order (a tree over each 256 strips, the chunks in order); its
// non-finite flag likewise.  partials == null: none.
struct LossDefer {
  const float* partials = nullptr;
  int blocks = 0;
  float denom = 1.0f;
  DevScalars* scalars = nullptr;
};

// The step's loss from the output launch's strip partials, by a 256-thread
// block: 256 partials at a time (one per thread; `p0`, the first chunk's,
// loaded by the caller before its own work), each chunk added as a fixed
// tree (wave butterflies, then the four waves in order), the chunks in
// order; thread 0 stores loss = sum / denom and flags a non-finite one.
// Every thread of the block calls it (it synchronizes the block).
__device__ __forceinline__ void deferred_loss_tree(const LossDefer& ld, float p0, int t) {
  __shared__ float wsum[4];
  float sum = 0.0f;
  for (int c = 0; c < ld.blocks; c += 256) {
    float v = c == 0 ? p0 : ld.partials[min(c + t, ld.blocks - 1)];
    v = c + t < ld.blocks ? v : 0.0f;
    v = wave_sum(v);
    __syncthreads();
    if ((t & 63) == 0) wsum[t >> 6] = v;
    __syncthreads();
    const float cs = (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
    sum = c == 0 ? cs : sum + cs;
  }
  if (t == 0) {
    const float loss = sum / ld.denom;
    ld.scalars->loss = loss;
    if (!(fabsf(loss) <= 3.402823466e38f)) atomicOr(&ld.scalars->flags, (uint32_t)VOLTA_STATUS_NONFINITE_LOSS);
  }
}
hipError_t launch_outer_dx(const float* delta, const float* W, int B, int R, int K, int act, const float* aux_act,
                           const float* aux_pre, float* out, hipStream_t st, const LossDefer& ld = LossDefer{});
hipError_t launch_narrow_dw(const NarrowDwArgs& p, hipStream_t st);

}  // namespace volta
