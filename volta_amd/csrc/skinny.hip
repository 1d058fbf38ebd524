// Kernels for the narrow output layer (L[n] <= 16 columns: the regression
// head of width 1 or a classifier head of width ~10).  Its three products
// are too thin for MFMA tiles (a 64-wide tile would be >90% padding), so
// they are done with wavefront-wide dot products instead:
//
//   out_layer_kernel   z = act_{n-1} W + b, the loss head and delta_{n-1}
//   outer_dx_kernel    delta_{n-2} = (delta_{n-1} W^T) * f'   (K = L[n])
//   narrow_dw_kernel   dW = act^T delta, db, optimizer update (N = L[n])
//
// Every sum has a fixed order: per-lane k-strided partials then a fixed
// butterfly (out_layer), or a sequential loop in the reference's order
// (outer_dx over k, narrow_dw over the batch).
#include "skinny.h"

namespace volta {

// One output row z[0..N) of the output layer, computed by a whole wave:
// lane l sums k = l, l+64, ..., then a fixed butterfly adds the lanes.
template <int NMAX>
__device__ __forceinline__ void wave_row(const float* __restrict__ a, const float* __restrict__ W, int K, int N,
                                         float* z) {
  const int lane = threadIdx.x & 63;
  float acc[NMAX];
#pragma unroll
  for (int j = 0; j < NMAX; ++j) acc[j] = 0.0f;
  for (int k = lane; k < K; k += 64) {
    const float x = a[k];
    const float* w = W + (size_t)k * N;
#pragma unroll
    for (int j = 0; j < NMAX; ++j)
      if (j < N) acc[j] = acc[j] + x * w[j];
  }
#pragma unroll
  for (int j = 0; j < NMAX; ++j) z[j] = wave_sum(acc[j]);
}

// Loss head of one row (same definitions as the MFMA path's loss epilogue):
// MSE (:792-798) d = z - y, loss += d^2, delta = 2d/nt; softmax-CE
// (interpreter.rs:762-812, autograd.rs:467-534).  Returns the row's loss.
// (Loops run to NMAX with a j < N guard so z stays in registers.)
template <int NMAX>
__device__ __forceinline__ float head_row(const OutLayerArgs& p, const float* z, int m) {
  const int N = p.N;
  float* out = p.out + (size_t)m * N;
  float* d = p.delta + (size_t)m * N;
#pragma unroll
  for (int j = 0; j < NMAX; ++j)
    if (j < N) out[j] = z[j];
  if (p.loss == VOLTA_LOSS_MSE) {
    const float nt = (float)(p.B * N);
    const float* y = p.y + (size_t)m * N;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < NMAX; ++j) {
      if (j < N) {
        const float dj = z[j] - y[j];
        acc = acc + dj * dj;
        d[j] = 2.0f * dj / nt;
      }
    }
    return acc;
  }
  const float bf = (float)p.B;
  const int lab = p.labels[m];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < NMAX; ++j)
    if (j < N) mx = fmaxf(mx, z[j]);
  float sum = 0.0f;
#pragma unroll
  for (int j = 0; j < NMAX; ++j)
    if (j < N) sum = sum + expf(z[j] - mx);
  const float lse = mx + logf(sum);
  float sample = __builtin_nanf("");
#pragma unroll
  for (int j = 0; j < NMAX; ++j) {
    if (j < N) {
      const bool on = j == lab;
      if (on) sample = -(z[j] - lse);
      d[j] = (expf(z[j] - mx) / sum - (on ? 1.0f : 0.0f)) / bf;
    }
  }
  if (lab < 0 || lab >= N) atomicOr(&p.scalars->flags, (uint32_t)VOLTA_STATUS_BAD_ARGUMENT);
  return sample;
}

// Block b handles rows [b*rows_per_block, ...): wave w takes every
// (waves)-th row.  The block's loss is the sum of its waves' row sums in
// wave order; with one block it finishes the step's loss directly,
// otherwise it lands in partials[b] for loss_finish_kernel.
template <int NMAX>
__global__ void __launch_bounds__(1024) out_layer_kernel(OutLayerArgs p, int rows_per_block) {
  __shared__ float wave_loss[16];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int waves = blockDim.x >> 6;
  const int r0 = blockIdx.x * rows_per_block;
  const int r1 = min(p.B, r0 + rows_per_block);
  float wl = 0.0f;
  for (int m = r0 + wave; m < r1; m += waves) {
    float z[NMAX];
    wave_row<NMAX>(p.act + (size_t)m * p.K, p.W, p.K, p.N, z);
    if (lane == 0) {
#pragma unroll
      for (int j = 0; j < NMAX; ++j)
        if (j < p.N) z[j] = z[j] + p.bias[j];
      wl = wl + head_row<NMAX>(p, z, m);
    }
  }
  if (lane == 0) wave_loss[wave] = wl;
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = wave_loss[0];
    for (int w = 1; w < waves; ++w) s = s + wave_loss[w];
    if (gridDim.x == 1) {
      const float denom = p.loss == VOLTA_LOSS_MSE ? (float)(p.B * p.N) : (float)p.B;
      step_epilogue(p.scalars, p.bc_table, p.bc_len, s / denom);
    } else {
      p.partials[blockIdx.x] = s;
    }
  }
}

// Sum the per-block losses in block order and finish the step's loss.
__global__ void __launch_bounds__(64) loss_finish_kernel(OutLayerArgs p, int blocks) {
  if (threadIdx.x != 0) return;
  float s = p.partials[0];
  for (int b = 1; b < blocks; ++b) s = s + p.partials[b];
  const float denom = p.loss == VOLTA_LOSS_MSE ? (float)(p.B * p.N) : (float)p.B;
  step_epilogue(p.scalars, p.bc_table, p.bc_len, s / denom);
}

// delta_out[b][j] = (sum_{k<K} delta[b][k] * W[j][k]) * f'(layer below)[b][j]
// for K <= 16 (reference order: k ascending, :919-929).
__global__ void __launch_bounds__(256)
outer_dx_kernel(const float* __restrict__ delta, const float* __restrict__ W, int B, int R, int K, int act,
                const float* __restrict__ aux_act, const float* __restrict__ aux_pre, float* __restrict__ out) {
  const size_t total = (size_t)B * R;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
    const int b = (int)(idx / R), j = (int)(idx % R);
    const float* d = delta + (size_t)b * K;
    const float* w = W + (size_t)j * K;
    float s = 0.0f;
    for (int k = 0; k < K; ++k) s = s + d[k] * w[k];
    const float y = aux_act[idx];
    const float pre = aux_pre ? aux_pre[idx] : y;
    out[idx] = s * act_derivative(act, pre, y);
  }
}

// dW[j][k] = sum_b act[b][j] * delta[b][k] (b ascending, as sgemm_tn sums),
// one thread per row j of W; delta is staged in LDS.  Block 0 also forms
// db[k] = sum_b delta[b][k] (:931-933).  Then the optimizer update of W and
// b (same element functions as the MFMA path).
template <int NMAX>
__global__ void __launch_bounds__(256) narrow_dw_kernel(NarrowDwArgs p) {
  extern __shared__ float sdelta[];  // [B x N]
  const int B = p.B, N = p.N, R = p.R;
  for (int i = threadIdx.x; i < B * N; i += blockDim.x) sdelta[i] = p.delta[i];
  __syncthreads();
  const float lr = p.scalars->lr;
  const float bc1 = p.scalars->bc1, bc2 = p.scalars->bc2;
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j < R) {
    float acc[NMAX];
#pragma unroll
    for (int k = 0; k < NMAX; ++k) acc[k] = 0.0f;
    for (int b = 0; b < B; ++b) {
      const float a = p.act[(size_t)b * R + j];
#pragma unroll
      for (int k = 0; k < NMAX; ++k)
        if (k < N) acc[k] = acc[k] + a * sdelta[b * N + k];
    }
    const int64_t count = (int64_t)R * N;
    const int64_t vec_end = count - count % 8;
#pragma unroll
    for (int k = 0; k < NMAX; ++k) {
      if (k >= N) break;
      const int64_t idx = (int64_t)j * N + k;
      if (p.grad) p.grad[idx] = acc[k];
      if (p.opt == VOLTA_OPT_SGD) {
        const float nlr = -lr;
        p.w[idx] = p.w[idx] + nlr * acc[k];
      } else if (p.opt == VOLTA_OPT_ADAGRAD) {
        adagrad_elem(p.w + idx, p.m + idx, acc[k], lr, p.eps);
      } else {
        adam_elem(p.w + idx, p.m + idx, p.v + idx, acc[k], idx >= vec_end, lr, bc1, bc2, p.b1, p.b2, p.eps,
                  p.wd);
      }
    }
  }
  if (blockIdx.x == 0 && threadIdx.x < N) {
    const int k = threadIdx.x;
    float db = 0.0f;
    for (int b = 0; b < B; ++b) db = db + sdelta[b * N + k];
    if (p.bgrad) p.bgrad[k] = db;
    if (p.opt == VOLTA_OPT_SGD) {
      p.b[k] = p.b[k] - lr * db;
    } else if (p.opt == VOLTA_OPT_ADAGRAD) {
      adagrad_elem(p.b + k, p.bm + k, db, lr, p.eps);
    } else {
      adam_elem(p.b + k, p.bm + k, p.bv + k, db, k >= N - N % 8, lr, bc1, bc2, p.b1, p.b2, p.eps, 0.0f);
    }
  }
}

// ---------------------------------------------------------------------------
int out_layer_blocks(int B) { return B <= 256 ? 1 : (B + 15) / 16; }

hipError_t launch_out_layer(const OutLayerArgs& p, hipStream_t st) {
  if (p.N > 16 || p.N < 1) return hipErrorInvalidValue;
  const int blocks = out_layer_blocks(p.B);
  const int rows = blocks == 1 ? p.B : 16;
  if (blocks > 1 && !p.partials) return hipErrorInvalidValue;
  if (p.N <= 1)
    hipLaunchKernelGGL(out_layer_kernel<1>, dim3(blocks), dim3(1024), 0, st, p, rows);
  else if (p.N <= 4)
    hipLaunchKernelGGL(out_layer_kernel<4>, dim3(blocks), dim3(1024), 0, st, p, rows);
  else
    hipLaunchKernelGGL(out_layer_kernel<16>, dim3(blocks), dim3(1024), 0, st, p, rows);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || blocks == 1) return e;
  hipLaunchKernelGGL(loss_finish_kernel, dim3(1), dim3(64), 0, st, p, blocks);
  return hipGetLastError();
}

hipError_t launch_outer_dx(const float* delta, const float* W, int B, int R, int K, int act, const float* aux_act,
                           const float* aux_pre, float* out, hipStream_t st) {
  if (K > 16 || K < 1) return hipErrorInvalidValue;
  const size_t total = (size_t)B * R;
  const int blocks = (int)std::min<size_t>((total + 255) / 256, 8192);
  hipLaunchKernelGGL(outer_dx_kernel, dim3(blocks), dim3(256), 0, st, delta, W, B, R, K, act, aux_act, aux_pre,
                     out);
  return hipGetLastError();
}

hipError_t launch_narrow_dw(const NarrowDwArgs& p, hipStream_t st) {
  if (p.N > 16 || p.N < 1 || (size_t)p.B * p.N * sizeof(float) > kNarrowDwLdsBytes) return hipErrorInvalidValue;
  const int blocks = (p.R + 255) / 256;
  const size_t lds = (size_t)p.B * p.N * sizeof(float);
  if (p.N <= 1)
    hipLaunchKernelGGL(narrow_dw_kernel<1>, dim3(blocks), dim3(256), lds, st, p);
  else if (p.N <= 4)
    hipLaunchKernelGGL(narrow_dw_kernel<4>, dim3(blocks), dim3(256), lds, st, p);
  else
    hipLaunchKernelGGL(narrow_dw_kernel<16>, dim3(blocks), dim3(256), lds, st, p);
  return hipGetLastError();
}

}  // namespace volta
