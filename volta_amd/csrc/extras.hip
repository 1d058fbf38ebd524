// Codegen extras of the generated step, in the reference's arithmetic order:
//   softmax as the hidden activation (:727-740, :898-906);
//   LayerNorm after each hidden activation (:745-772) and its backward with
//   the SGD update of gamma/beta (:829-887);
//   inverted dropout with masks from the reference's LCG (:774-788,
//   :888-892) -- every element's draw is found by jumping the LCG ahead, so
//   the mask does not depend on the launch shape;
//   gradient clipping by the global norm of the deltas (:936-955).
// Row statistics (LayerNorm mean/variance, the backward's row means) are
// sequential f32 sums by one thread per row, as in the reference; column
// sums are sequential over the batch, one thread per column.  The global
// norm of the clip is a fixed-order tree (it differs from the reference's
// sequential sum only in rounding).
#include <algorithm>

#include "extras.h"

namespace volta {

namespace {

constexpr uint64_t kLcgA = 6364136223846793005ULL;
constexpr uint64_t kLcgC = 1442695040888963407ULL;

// State after m draws from s: the affine map s -> A*s + C applied m times,
// composed by squaring (maps of one LCG commute).
__device__ __forceinline__ uint64_t lcg_jump(uint64_t s, uint64_t m) {
  uint64_t a = kLcgA, c = kLcgC, ra = 1, rc = 0;
  while (m) {
    if (m & 1) {
      ra = a * ra;
      rc = a * rc + c;
    }
    c = a * c + c;
    a = a * a;
    m >>= 1;
  }
  return ra * s + rc;
}

__global__ void __launch_bounds__(256) hidden_fwd_kernel(HiddenFwdArgs a) {
  __shared__ float stat[4];
  const int b = blockIdx.x, c = a.c;
  float* row = a.act + (size_t)b * c;
  if (a.softmax) {
    // :727-740: first maximum (strict >), exp(pre - max), sum in column
    // order, times 1/sum
    if (threadIdx.x == 0) {
      float mx = row[0];
      for (int j = 1; j < c; ++j)
        if (row[j] > mx) mx = row[j];
      stat[2] = mx;
    }
    __syncthreads();
    const float mx = stat[2];
    for (int j = threadIdx.x; j < c; j += blockDim.x) row[j] = expf(row[j] - mx);
    __syncthreads();
    if (threadIdx.x == 0) {
      float sum = 0.0f;
      for (int j = 0; j < c; ++j) sum = sum + row[j];
      stat[3] = 1.0f / sum;
    }
    __syncthreads();
    const float inv = stat[3];
    for (int j = threadIdx.x; j < c; j += blockDim.x) row[j] = row[j] * inv;
    __syncthreads();
  }
  float mu = 0.0f, is = 0.0f;
  if (a.gamma) {
    if (threadIdx.x == 0) {
      float m = 0.0f;
      for (int j = 0; j < c; ++j) m = m + row[j];
      m = m / (float)c;
      float var = 0.0f;
      for (int j = 0; j < c; ++j) {
        const float d = row[j] - m;
        var = var + d * d;
      }
      var = var / (float)c;
      const float s = 1.0f / sqrtf(var + 1e-5f);
      if (a.mu) {
        a.mu[b] = m;
        a.inv_std[b] = s;
      }
      stat[0] = m;
      stat[1] = s;
    }
    __syncthreads();
    mu = stat[0];
    is = stat[1];
  }
  const uint64_t base = a.mask ? a.scalars->rng : 0;
  for (int j = threadIdx.x; j < c; j += blockDim.x) {
    float x = row[j];
    if (a.gamma) {
      const float xhat = (x - mu) * is;
      x = xhat * a.gamma[j] + a.beta[j];
    }
    if (a.mask) {
      const uint64_t k = (uint64_t)b * c + j;
      const uint64_t s = lcg_jump(base, a.rng_offset + k + 1);
      const float r = (float)(s >> 33) / 2147483648.0f;
      const uint8_t keep = r >= a.p ? 1 : 0;
      a.mask[k] = keep;
      x = x * ((float)keep * a.keep_scale);
    }
    row[j] = x;
  }
}

// LayerNorm gradient columns: dgamma[j] = sum_b dout*xhat, dbeta[j] =
// sum_b dout, xhat recomputed from the output as (y - beta)/(gamma + 1e-12).
__global__ void __launch_bounds__(256) ln_bwd_cols_kernel(HiddenBwdArgs a) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= a.c) return;
  const float g = a.gamma[j], be = a.beta[j];
  float dg = 0.0f, db = 0.0f;
  for (int b = 0; b < a.B; ++b) {
    const size_t k = (size_t)b * a.c + j;
    const float xh = (a.act[k] - be) / (g + 1e-12f);
    const float dout = a.delta[k];
    dg = dg + dout * xh;
    db = db + dout;
  }
  a.dgamma[j] = dg;
  a.dbeta[j] = db;
}

// Row pass: LayerNorm backward (row means of d_xhat and d_xhat*xhat by
// thread 0 in column order), dropout mask, activation derivative.  ReLU's
// derivative takes the pre-activation (the output is no longer relu(pre));
// sigmoid/tanh take the layer output as the reference does.
__global__ void __launch_bounds__(256) hidden_bwd_rows_kernel(HiddenBwdArgs a) {
  __shared__ float stat[3];
  const int b = blockIdx.x, c = a.c;
  float* d = a.delta + (size_t)b * c;
  const float* y = a.act + (size_t)b * c;
  float sum_d = 0.0f, sum_dxh = 0.0f, is = 0.0f;
  if (a.gamma) {
    if (threadIdx.x == 0) {
      float s1 = 0.0f, s2 = 0.0f;
      for (int j = 0; j < c; ++j) {
        const float g = a.gamma[j];
        const float xh = (y[j] - a.beta[j]) / (g + 1e-12f);
        const float dout = d[j];
        s1 = s1 + dout * g;
        s2 = s2 + dout * g * xh;
      }
      stat[0] = s1 / (float)c;
      stat[1] = s2 / (float)c;
    }
    __syncthreads();
    sum_d = stat[0];
    sum_dxh = stat[1];
    is = a.inv_std[b];
  }
  const float* pre = a.pre + (size_t)b * c;
  for (int j = threadIdx.x; j < c; j += blockDim.x) {
    float x = d[j];
    if (a.gamma) {
      const float g = a.gamma[j];
      const float xh = (y[j] - a.beta[j]) / (g + 1e-12f);
      const float d_xhat = x * g;
      x = is * (d_xhat - sum_d - xh * sum_dxh);
    }
    if (a.mask) x = x * ((float)a.mask[(size_t)b * c + j] * a.keep_scale);
    if (a.act_kind != VOLTA_ACT_SOFTMAX) {
      const float p = pre[j];
      x = x * act_derivative(a.act_kind, p, a.act_kind == VOLTA_ACT_RELU ? p : y[j]);
    }
    d[j] = x;
  }
  if (a.act_kind == VOLTA_ACT_SOFTMAX) {
    // :898-906: dot(d, y) in column order, then d = y * (d - dot)
    __syncthreads();
    if (threadIdx.x == 0) {
      float dot = 0.0f;
      for (int j = 0; j < c; ++j) dot = dot + d[j] * y[j];
      stat[2] = dot;
    }
    __syncthreads();
    const float dot = stat[2];
    for (int j = threadIdx.x; j < c; j += blockDim.x) d[j] = y[j] * (d[j] - dot);
  }
}

__global__ void __launch_bounds__(256) ln_update_kernel(float* gamma, float* beta, const float* dg, const float* db,
                                                        int c, const DevScalars* s) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= c) return;
  const float lr = s->lr;
  gamma[j] = gamma[j] - lr * dg[j];
  beta[j] = beta[j] - lr * db[j];
}

__global__ void rng_advance_kernel(DevScalars* s, uint64_t draws) {
  if (threadIdx.x == 0 && blockIdx.x == 0) s->rng = lcg_jump(s->rng, draws);
}

// Sum of squares of every delta element: block k covers a fixed contiguous
// range of the layers' deltas taken in layer order; lanes add their strided
// elements, then a fixed butterfly and wave order.
__global__ void __launch_bounds__(256) clip_partials_kernel(ClipArgs a) {
  __shared__ float wave_part[4];
  int64_t total = 0;
  for (int i = 0; i < a.n; ++i) total += a.count[i];
  const int64_t chunk = (total + gridDim.x - 1) / gridDim.x;
  const int64_t lo = (int64_t)blockIdx.x * chunk, hi = lo + chunk < total ? lo + chunk : total;
  float s = 0.0f;
  int layer = 0;
  int64_t layer_lo = 0;
  for (int64_t g = lo + threadIdx.x; g < hi; g += blockDim.x) {
    while (g >= layer_lo + a.count[layer]) {
      layer_lo += a.count[layer];
      ++layer;
    }
    const float v = a.delta[layer][g - layer_lo];
    s = s + v * v;
  }
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) wave_part[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) a.partials[blockIdx.x] = wave_part[0] + wave_part[1] + wave_part[2] + wave_part[3];
}

__global__ void clip_finish_kernel(ClipArgs a) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  float gsq = 0.0f;
  for (int k = 0; k < kClipBlocks; ++k) gsq = gsq + a.partials[k];
  const float gnorm = sqrtf(gsq);
  a.scalars->clip_scale = gnorm > a.clip ? a.clip / gnorm : 1.0f;
}

// delta *= scale for every layer (x * 1.0f is x, so no test of scale < 1).
__global__ void __launch_bounds__(256) clip_apply_kernel(ClipArgs a) {
  const float scale = a.scalars->clip_scale;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int i = 0; i < a.n; ++i) {
    float* d = a.delta[i];
    for (int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; k < a.count[i]; k += stride)
      d[k] = d[k] * scale;
  }
}

}  // namespace

hipError_t launch_hidden_fwd(const HiddenFwdArgs& a, hipStream_t st) {
  if (!a.gamma && !a.mask && !a.softmax) return hipSuccess;
  hipLaunchKernelGGL(hidden_fwd_kernel, dim3(a.B), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_hidden_bwd(const HiddenBwdArgs& a, float* gamma, float* beta, const DevScalars* scalars,
                             hipStream_t st) {
  const int cb = (a.c + 255) / 256;
  if (a.gamma) {
    hipLaunchKernelGGL(ln_bwd_cols_kernel, dim3(cb), dim3(256), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(hidden_bwd_rows_kernel, dim3(a.B), dim3(256), 0, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !a.gamma) return e;
  hipLaunchKernelGGL(ln_update_kernel, dim3(cb), dim3(256), 0, st, gamma, beta, a.dgamma, a.dbeta, a.c, scalars);
  return hipGetLastError();
}

hipError_t launch_rng_advance(DevScalars* scalars, uint64_t draws, hipStream_t st) {
  hipLaunchKernelGGL(rng_advance_kernel, dim3(1), dim3(64), 0, st, scalars, draws);
  return hipGetLastError();
}

hipError_t launch_clip(const ClipArgs& a, hipStream_t st) {
  if (a.n < 1 || a.n > 16 || !a.partials || !a.scalars) return hipErrorInvalidValue;
  int64_t total = 0;
  for (int i = 0; i < a.n; ++i) {
    if (!a.delta[i] || a.count[i] < 1) return hipErrorInvalidValue;
    total += a.count[i];
  }
  hipLaunchKernelGGL(clip_partials_kernel, dim3(kClipBlocks), dim3(256), 0, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(clip_finish_kernel, dim3(1), dim3(64), 0, st, a);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int blocks = (int)std::min<int64_t>((total + 255) / 256, 2048);
  hipLaunchKernelGGL(clip_apply_kernel, dim3(blocks), dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace volta
