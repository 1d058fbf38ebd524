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

#include "narrow_dw.h"

namespace volta {

// Output rows z[g][0..N) of RG rows (rows[g], valid where rows[g] >= 0),
// computed by a whole wave: lane l sums k = l, l+64, ... in ascending order,
// then a fixed butterfly adds the lanes.  The k loop runs in chunks of C
// values per lane whose loads (activations of all RG rows and the matching
// rows of W) are all issued before the chunk's first multiply, so a chunk
// costs one memory latency.
template <int NMAX, int RG, int C>
__device__ __forceinline__ void wave_rows(const OutLayerArgs& p, const int* rows, float (*z)[NMAX]) {
  const int lane = threadIdx.x & 63;
  const int K = p.K, N = p.N;
  float acc[RG][NMAX];
#pragma unroll
  for (int g = 0; g < RG; ++g)
#pragma unroll
    for (int j = 0; j < NMAX; ++j) acc[g][j] = 0.0f;
  for (int k0 = lane; k0 < K; k0 += 64 * C) {
    float x[RG][C], wv[C][NMAX];
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int k = k0 + 64 * c;
#pragma unroll
      for (int j = 0; j < NMAX; ++j) wv[c][j] = k < K && j < N ? p.W[(size_t)k * N + j] : 0.0f;
#pragma unroll
      for (int g = 0; g < RG; ++g) x[g][c] = k < K && rows[g] >= 0 ? p.act[(size_t)rows[g] * K + k] : 0.0f;
    }
#pragma unroll
    for (int g = 0; g < RG; ++g)
#pragma unroll
      for (int c = 0; c < C; ++c) {
        if (k0 + 64 * c < K) {
#pragma unroll
          for (int j = 0; j < NMAX; ++j)
            if (j < N) acc[g][j] = acc[g][j] + x[g][c] * wv[c][j];
        }
      }
  }
#pragma unroll
  for (int g = 0; g < RG; ++g)
#pragma unroll
    for (int j = 0; j < NMAX; ++j) z[g][j] = wave_sum(acc[g][j]);
}

// Loss head of one row (same definitions as the MFMA path's loss epilogue):
// MSE (:792-798) d = z - y, loss += d^2, delta = 2d/nt; softmax-CE
// (interpreter.rs:762-812, autograd.rs:467-534).  Returns the row's loss.
// `y` holds the row's targets (MSE), `lab` its label (CE), both loaded
// before z was computed.  (Loops run to NMAX with a j < N guard so z stays
// in registers.)
template <int NMAX>
__device__ __forceinline__ float head_row(const OutLayerArgs& p, const float* z, const float* y, int lab, int m) {
  const int N = p.N;
  float* out = p.out + (size_t)m * N;
  float* d = p.delta + (size_t)m * N;
#pragma unroll
  for (int j = 0; j < NMAX; ++j)
    if (j < N) out[j] = z[j];
  if (p.loss == VOLTA_LOSS_MSE) {
    const float nt = (float)(p.B * N);
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
// (waves)-th row, RG rows at a time (in increasing row order).  The block's
// loss is the sum of its waves' row sums in wave order; with one block it
// finishes the step's loss directly, otherwise it lands in partials[b] for
// loss_finish_kernel.  Lane 0 loads the bias, the targets/labels of its
// rows and the next step counter before the dot products.
template <int NMAX>
__global__ void __launch_bounds__(1024) out_layer_kernel(OutLayerArgs p, int rows_per_block) {
  // rows per group and k per lane per chunk, sized to stay within the 128
  // registers a 1024-thread block allows
  constexpr int RG = NMAX >= 16 ? 1 : 4;
  constexpr int C = NMAX >= 16 ? 2 : 4;
  __shared__ float wave_loss[16];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int waves = blockDim.x >> 6;
  const int r0 = blockIdx.x * rows_per_block;
  const int r1 = min(p.B, r0 + rows_per_block);
  const int N = p.N;
  const bool single = gridDim.x == 1;
  StepNext next{};
  if (single && threadIdx.x == 0) next = step_prefetch(p.scalars, p.bc_table, p.bc_len);
  float bias[NMAX];
#pragma unroll
  for (int j = 0; j < NMAX; ++j) bias[j] = lane == 0 && j < N ? p.bias[j] : 0.0f;
  float wl = 0.0f;
  for (int m0 = r0 + wave; m0 < r1; m0 += waves * RG) {
    int rows[RG];
    float y[RG][NMAX];
    int lab[RG];
#pragma unroll
    for (int g = 0; g < RG; ++g) {
      const int m = m0 + g * waves;
      rows[g] = m < r1 ? m : -1;
      lab[g] = 0;
      if (lane == 0 && rows[g] >= 0) {
        if (p.loss == VOLTA_LOSS_MSE) {
#pragma unroll
          for (int j = 0; j < NMAX; ++j) y[g][j] = j < N ? p.y[(size_t)m * N + j] : 0.0f;
        } else {
          lab[g] = p.labels[m];
        }
      }
    }
    float z[RG][NMAX];
    wave_rows<NMAX, RG, C>(p, rows, z);
    if (lane == 0) {
#pragma unroll
      for (int g = 0; g < RG; ++g) {
        if (rows[g] < 0) continue;
#pragma unroll
        for (int j = 0; j < NMAX; ++j)
          if (j < N) z[g][j] = z[g][j] + bias[j];
        wl = wl + head_row<NMAX>(p, z[g], y[g], lab[g], rows[g]);
      }
    }
  }
  if (lane == 0) wave_loss[wave] = wl;
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = wave_loss[0];
    for (int w = 1; w < waves; ++w) s = s + wave_loss[w];
    if (single) {
      const float denom = p.loss == VOLTA_LOSS_MSE ? (float)(p.B * p.N) : (float)p.B;
      step_finish(p.scalars, next, p.bc_table != nullptr, s / denom);
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
    const float y = aux_act[idx];
    const float pre = (aux_pre ? aux_pre : aux_act)[idx];
    float s = 0.0f;
    for (int k = 0; k < K; ++k) s = s + d[k] * w[k];
    out[idx] = s * act_derivative(act, pre, y);
  }
}

// Stand-alone launch: one wave per block, so R/64 CUs share the loads.
template <int NMAX>
__global__ void __launch_bounds__(64) narrow_dw_kernel(NarrowDwArgs p) {
  extern __shared__ float sdelta[];
  narrow_dw_block<NMAX>(p, blockIdx.x, sdelta);
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
  if (p.opt != VOLTA_OPT_SGD && p.opt != VOLTA_OPT_ADAM && p.opt != VOLTA_OPT_ADAGRAD) return hipErrorInvalidValue;
  const int blocks = (p.R + 63) / 64;
  const size_t lds = (size_t)p.B * p.N * sizeof(float);
  if (p.N <= 1)
    hipLaunchKernelGGL(narrow_dw_kernel<1>, dim3(blocks), dim3(64), lds, st, p);
  else if (p.N <= 4)
    hipLaunchKernelGGL(narrow_dw_kernel<4>, dim3(blocks), dim3(64), lds, st, p);
  else
    hipLaunchKernelGGL(narrow_dw_kernel<16>, dim3(blocks), dim3(64), lds, st, p);
  return hipGetLastError();
}

}  // namespace volta
