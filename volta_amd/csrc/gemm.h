// Host/device interface of the fp32 MFMA GEMM family (gemm.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>

#include "device_common.h"
#include "recorder.h"

namespace volta {

enum GemmLayout {
  GEMM_NN = 0,  // A [M x K] row-major, B [K x N] row-major   (forward)
  GEMM_NT = 1,  // A [M x K] row-major, B [N x K] row-major   (dX = delta W^T)
  GEMM_TN = 2,  // A [K x M] row-major, B [K x N] row-major   (dW = act^T delta)
};

enum EpiKind {
  EPI_STORE = 0,     // out = acc
  EPI_BIAS_ACT = 1,  // pre = acc + bias; out = f(pre)     (f = identity for the output layer)
  EPI_DX_ACT = 2,    // out = acc * f'(aux_pre, aux_act)
  EPI_SGD = 3,       // out = out + (-lr) * acc            (W updated in place)
};

struct EpiArgs {
  int kind;
  int act;                  // enum volta_activation, or kIdentity
  int ldc;
  float* out;
  float* pre;               // EPI_BIAS_ACT: where to keep the pre-activation (may be null)
  const float* bias;        // EPI_BIAS_ACT
  const float* aux_act;     // EPI_DX_ACT: activation output of the layer below
  const float* aux_pre;     // EPI_DX_ACT: its pre-activation (null when not kept)
  const DevScalars* scalars;  // EPI_SGD: learning rate
};

struct GemmArgs {
  const float* A;
  const float* B;
  int lda, ldb;
  int M, N, K;
  int k_per_split;
  float* partial;  // split-K workspace: splits planes of M*N floats
  EpiArgs epi;
};

enum GemmTile { TILE_64x64 = 0, TILE_128x128 = 1 };

struct GemmPlan {
  int layout = GEMM_NN;
  int tile = TILE_64x64;
  int splits = 1;
  int k_per_split = 0;
  bool vec = false;
  size_t workspace_floats(int M, int N) const { return splits > 1 ? (size_t)splits * M * N : 0; }
};

GemmPlan gemm_plan(int layout, int M, int N, int K, bool vec, int num_cus);
// `bytes` is the caller's algorithmic HBM traffic of the product (for the
// profiler); `rec`/`label` are optional.
hipError_t gemm_launch(const GemmPlan& p, const GemmArgs& a, hipStream_t st, Recorder* rec = nullptr,
                       const char* label = "gemm", double bytes = 0.0);

}  // namespace volta
