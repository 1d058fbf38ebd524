// Host interface of the non-GEMM step kernels (step_kernels.hip).
#pragma once

#include <hip/hip_runtime.h>

#include "device_common.h"
#include "recorder.h"

namespace volta {

// Parameter, gradient and optimizer-state buffers are flat, one segment per
// W_i and per b_i, each padded to kSegAlign floats so every optimizer
// workgroup stays inside one segment.
constexpr int kSegAlign = 1024;
constexpr int kMaxSegments = 2 * (VOLTA_MAX_LAYER_SIZES - 1);

struct SegTable {
  int n;
  int64_t off[kMaxSegments];    // first float of the segment in the flat buffer
  int64_t count[kMaxSegments];  // real (unpadded) element count
  float wd[kMaxSegments];       // weight decay applied to this segment
};

hipError_t launch_loss_mse(const float* yhat, const float* y, float* delta, int nt, DevScalars* sc,
                           const float2* bc_table, int bc_len, hipStream_t st);
hipError_t launch_loss_ce(const float* z, const int32_t* labels, float* delta, int B, int C,
                          DevScalars* sc, const float2* bc_table, int bc_len, hipStream_t st);
hipError_t launch_adam(float* w, float* m, float* v, const float* g, const SegTable& segs,
                       int64_t total, const DevScalars* sc, float b1, float b2, float eps,
                       hipStream_t st);
hipError_t launch_adagrad(float* w, float* G, const float* g, const SegTable& segs, int64_t total,
                          const DevScalars* sc, float eps, hipStream_t st);

}  // namespace volta
