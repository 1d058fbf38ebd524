// Codegen extras of the generated step, in the reference's arithmetic order:
//   softmax as the hidden activation (:727-740, :898-906);
//   LayerNorm after each hidden activation (:745-772) and its backward with
//   the SGD update of gamma/beta (:829-887);
//   inverted dropout with masks from the reference's LCG (:774-788,
//   :888-892) -- every element's draw is found by jumping the LCG ahead, so
//   the mask does not depend on the launch shape;
//   gradient clipping by the global norm of the deltas (:936-955): partial
//   sums of squares, then one pass that forms the factor and scales.
// Row statistics (the softmax maximum and sum, LayerNorm mean/variance, the
// backward's row means and the softmax dot product) are block reductions
// over one row per 256-thread block: each thread folds its column-strided
// elements in column order, then a fixed butterfly per wave and the four
// waves in order -- deterministic, and different from the reference's
// sequential f32 sums only in rounding (the maximum is exact: the fold keeps
// the reference's first-maximum rule, so NaN handling matches too).  Column
// sums over the batch (dgamma, dbeta) are four interleaved batch-order sums
// added in a fixed order.  The global norm of the clip is a fixed-order tree
// as well.
#include <algorithm>

#include "extras.h"

namespace volta {

namespace {

constexpr uint64_t kLcgA = 6364136223846793005ULL;
constexpr uint64_t kLcgC = 1442695040888963407ULL;

// The affine map s -> A*s + C of m draws, composed by squaring (maps of one
// LCG commute).
struct LcgMap {
  uint64_t a, c;
};
__device__ __forceinline__ LcgMap lcg_map(uint64_t m) {
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
  return {ra, rc};
}

// State after m draws from s.
__device__ __forceinline__ uint64_t lcg_jump(uint64_t s, uint64_t m) {
  const LcgMap f = lcg_map(m);
  return f.a * s + f.c;
}

// Sum of v over the 256 threads of the block, the same value in every
// thread: a fixed butterfly per wave, then the four waves in order.  `part`
// is 4 floats of LDS; the block must be converged.
__device__ __forceinline__ float block_sum(float v, float* part) {
  v = wave_sum(v);
  __syncthreads();  // earlier readers of part are done
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
  __syncthreads();
  return ((part[0] + part[1]) + part[2]) + part[3];
}

// The reference's first maximum of a row (mx = row[0]; mx = row[j] if
// row[j] > mx, :727-733) over the block: threads fold their strided columns
// (thread 0 starting from row[0], the others from -inf), then partial maxima
// are combined lowest columns first with the same strict comparison, so the
// result -- including a NaN in row[0] -- is the sequential one.
__device__ __forceinline__ float block_first_max(const float* row, int c, float* part) {
  float mx = threadIdx.x == 0 ? row[0] : -INFINITY;
  for (int j = threadIdx.x == 0 ? 256 : threadIdx.x; j < c; j += 256)
    if (row[j] > mx) mx = row[j];
  // lane l combines with lane l + off, keeping the lower lane's value unless
  // the higher one is strictly greater
  for (int off = 1; off < 64; off <<= 1) {
    const float o = __shfl_down(mx, off, kWave);
    if ((threadIdx.x & (2 * off - 1)) == 0 && o > mx) mx = o;
  }
  __syncthreads();
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = mx;
  __syncthreads();
  float m = part[0];
  for (int w = 1; w < 4; ++w)
    if (part[w] > m) m = part[w];
  return m;
}

__global__ void __launch_bounds__(256) hidden_fwd_kernel(HiddenFwdArgs a) {
  __shared__ float part[4];
  const int b = blockIdx.x, c = a.c;
  float* row = a.act + (size_t)b * c;
  if (a.softmax) {
    // :727-740: first maximum (strict >), exp(pre - max), their sum, times
    // 1/sum
    const float mx = block_first_max(row, c, part);
    float s = 0.0f;
    for (int j = threadIdx.x; j < c; j += blockDim.x) {
      const float e = expf(row[j] - mx);
      row[j] = e;
      s = s + e;
    }
    const float inv = 1.0f / block_sum(s, part);
    for (int j = threadIdx.x; j < c; j += blockDim.x) row[j] = row[j] * inv;
    __syncthreads();
  }
  float mu = 0.0f, is = 0.0f;
  if (a.gamma) {
    // :745-760: mean, then the mean of squared deviations
    float s = 0.0f;
    for (int j = threadIdx.x; j < c; j += blockDim.x) s = s + row[j];
    mu = block_sum(s, part) / (float)c;
    float v = 0.0f;
    for (int j = threadIdx.x; j < c; j += blockDim.x) {
      const float d = row[j] - mu;
      v = v + d * d;
    }
    const float var = block_sum(v, part) / (float)c;
    is = 1.0f / sqrtf(var + 1e-5f);
    if (a.mu && threadIdx.x == 0) {
      a.mu[b] = mu;
      a.inv_std[b] = is;
    }
  }
  // Element k = b*c + j of the layer draws state jump(base, offset + k + 1):
  // the thread's first element by one jump from the stream, its next ones
  // (blockDim.x apart) by the map of blockDim.x draws -- the same states as
  // a jump per element.
  uint64_t st = 0;
  LcgMap stride{1, 0};
  if (a.mask) {
    st = lcg_jump(a.scalars->rng, a.rng_offset + (uint64_t)b * c + threadIdx.x + 1);
    stride = lcg_map(blockDim.x);
  }
  for (int j = threadIdx.x; j < c; j += blockDim.x) {
    float x = row[j];
    if (a.gamma) {
      const float xhat = (x - mu) * is;
      x = xhat * a.gamma[j] + a.beta[j];
    }
    if (a.mask) {
      const uint64_t k = (uint64_t)b * c + j;
      const float r = (float)(st >> 33) / 2147483648.0f;
      const uint8_t keep = r >= a.p ? 1 : 0;
      a.mask[k] = keep;
      x = x * ((float)keep * a.keep_scale);
      st = stride.a * st + stride.c;
    }
    row[j] = x;
  }
}

// LayerNorm gradient columns: dgamma[j] = sum_b dout*xhat, dbeta[j] =
// sum_b dout, xhat recomputed from the output as (y - beta)/(gamma + 1e-12)
// (:829-838).  A block covers 64 columns; wave w sums rows b = w, w + 4, ...
// in batch order (its loads unrolled eight rows deep), and the four wave
// partials are added in wave order.
__global__ void __launch_bounds__(256) ln_bwd_cols_kernel(HiddenBwdArgs a) {
  __shared__ float pg[4][64], pb[4][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = blockIdx.x * 64 + lane;
  const int jj = j < a.c ? j : a.c - 1;  // loads stay in bounds; the store is guarded
  const float g = a.gamma[jj], be = a.beta[jj];
  float dg = 0.0f, db = 0.0f;
#pragma unroll 8
  for (int b = w; b < a.B; b += 4) {
    const size_t k = (size_t)b * a.c + jj;
    const float xh = (a.act[k] - be) / (g + 1e-12f);
    const float dout = a.delta[k];
    dg = dg + dout * xh;
    db = db + dout;
  }
  pg[w][lane] = dg;
  pb[w][lane] = db;
  __syncthreads();
  if (w == 0 && j < a.c) {
    a.dgamma[j] = ((pg[0][lane] + pg[1][lane]) + pg[2][lane]) + pg[3][lane];
    a.dbeta[j] = ((pb[0][lane] + pb[1][lane]) + pb[2][lane]) + pb[3][lane];
  }
}

// Row pass: LayerNorm backward (row means of d_xhat and d_xhat*xhat by
// thread 0 in column order), dropout mask, activation derivative.  ReLU's
// derivative takes the pre-activation (the output is no longer relu(pre));
// sigmoid/tanh take the layer output as the reference does.
__global__ void __launch_bounds__(256) hidden_bwd_rows_kernel(HiddenBwdArgs a) {
  __shared__ float part[4];
  const int b = blockIdx.x, c = a.c;
  float* d = a.delta + (size_t)b * c;
  const float* y = a.act + (size_t)b * c;
  float sum_d = 0.0f, sum_dxh = 0.0f, is = 0.0f;
  if (a.gamma) {
    // :840-860: row means of d_xhat and d_xhat * xhat
    float s1 = 0.0f, s2 = 0.0f;
    for (int j = threadIdx.x; j < c; j += blockDim.x) {
      const float g = a.gamma[j];
      const float xh = (y[j] - a.beta[j]) / (g + 1e-12f);
      const float dout = d[j];
      s1 = s1 + dout * g;
      s2 = s2 + dout * g * xh;
    }
    sum_d = block_sum(s1, part) / (float)c;
    sum_dxh = block_sum(s2, part) / (float)c;
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
    // :898-906: dot(d, y), then d = y * (d - dot); every thread reads back
    // only the columns it wrote above
    float s = 0.0f;
    for (int j = threadIdx.x; j < c; j += blockDim.x) s = s + d[j] * y[j];
    const float dot = block_sum(s, part);
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

// The clip factor from the partial sums of squares (every block forms the
// same sum: one partial per thread, a fixed butterfly per wave, the four
// waves in order; block 0 records it), then delta *= scale for every layer
// (x * 1.0f is x, so no test of scale < 1).
static_assert(kClipBlocks == 256, "one partial per thread of the apply block");
__global__ void __launch_bounds__(256) clip_apply_kernel(ClipArgs a) {
  __shared__ float wave_part[4];
  float v = wave_sum(a.partials[threadIdx.x]);
  if ((threadIdx.x & 63) == 0) wave_part[threadIdx.x >> 6] = v;
  __syncthreads();
  const float gsq = ((wave_part[0] + wave_part[1]) + wave_part[2]) + wave_part[3];
  const float gnorm = sqrtf(gsq);
  const float scale = gnorm > a.clip ? a.clip / gnorm : 1.0f;
  if (blockIdx.x == 0 && threadIdx.x == 0) a.scalars->clip_scale = scale;
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
    hipLaunchKernelGGL(ln_bwd_cols_kernel, dim3((a.c + 63) / 64), dim3(256), 0, st, a);
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
  const int blocks = (int)std::min<int64_t>((total + 255) / 256, 2048);
  hipLaunchKernelGGL(clip_apply_kernel, dim3(blocks), dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace volta
