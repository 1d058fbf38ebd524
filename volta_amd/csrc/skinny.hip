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
// butterfly (out_layer), a sequential loop in the reference's order
// (outer_dx over k), or interleaved accumulators over the batch added
// pairwise (narrow_dw).
#include "skinny.h"

#include "narrow_dw.h"
#include "out_head.h"

namespace volta {

// Block b handles rows [b*rows_per_block, ...): wave w takes every
// (waves)-th row, RG rows at a time (in increasing row order).  The block's
// loss is the sum of its waves' row sums in wave order; with one block it
// finishes the step's loss directly, otherwise it lands in partials[b] for
// loss_finish_kernel.  Lane 0 loads the bias, the targets/labels of its
// rows and the next step counter before the dot products.
// W of at most kOutWlFloats floats (60 KiB) is staged in LDS, at most
// kOutStage per thread of the 1024-thread block.
constexpr int kOutStage = 15;
constexpr int kOutWlFloats = kOutStage * 1024;

template <int NMAX, bool WL>
__global__ void __launch_bounds__(1024) out_layer_kernel(OutLayerArgs p, int rows_per_block) {
  // rows per group and k per lane per chunk, sized to stay within the 128
  // registers a 1024-thread block allows
  constexpr int RG = NMAX >= 16 ? 1 : 4;
  constexpr int C = NMAX >= 16 ? (WL ? 16 : 2) : 4;
  __shared__ float wave_loss[16];
  extern __shared__ float w_lds[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int waves = blockDim.x >> 6;
  const int r0 = blockIdx.x * rows_per_block;
  const int r1 = min(p.B, r0 + rows_per_block);
  const int N = p.N;
  const bool single = gridDim.x == 1;
  StepNext next{};
  if (single && threadIdx.x == 0) next = step_prefetch(p.scalars, p.bc_table, p.bc_len);
  if constexpr (WL) {
    // W to LDS: coalesced, every load issued before the first store
    const int KN = p.K * N;
    float t[kOutStage];
#pragma unroll
    for (int it = 0; it < kOutStage; ++it) t[it] = p.W[min((int)threadIdx.x + 1024 * it, KN - 1)];
#pragma unroll
    for (int it = 0; it < kOutStage; ++it)
      if ((int)threadIdx.x + 1024 * it < KN) w_lds[threadIdx.x + 1024 * it] = t[it];
    __syncthreads();
  }
  float bias[NMAX];
#pragma unroll
  for (int j = 0; j < NMAX; ++j) bias[j] = p.bias[min(j, N - 1)];
  const bool mse = p.loss == VOLTA_LOSS_MSE;
  float wl = 0.0f;
  for (int m0 = r0 + wave; m0 < r1; m0 += waves * RG) {
    int rows[RG];
    float y[RG][NMAX];
    int lab[RG];
#pragma unroll
    for (int g = 0; g < RG; ++g) {
      const int m = m0 + g * waves;
      rows[g] = m < r1 ? m : -1;
      const int mc = m < r1 ? m : r0;  // clamped: a row this block owns
      // targets (MSE) or label (CE) of the row, loaded by every lane
#pragma unroll
      for (int j = 0; j < NMAX; ++j) y[g][j] = mse ? p.y[(size_t)mc * N + min(j, N - 1)] : 0.0f;
      lab[g] = mse ? 0 : p.labels[mc];
    }
    float z[RG][NMAX];
    wave_rows<NMAX, RG, C, WL>(p, w_lds, rows, z);
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

// Sum the per-block losses in block order and finish the step's loss.  The
// wave loads every partial at once (lane l: blocks l, l + 64, ...) into LDS,
// then lane 0 adds them in block order.
constexpr int kLossFinishMax = 4096;
__global__ void __launch_bounds__(64) loss_finish_kernel(OutLayerArgs p, int blocks) {
  __shared__ float part[kLossFinishMax];
  const bool staged = blocks <= kLossFinishMax;
  if (staged)
    for (int b = threadIdx.x; b < blocks; b += 64) part[b] = p.partials[b];
  __syncthreads();
  if (threadIdx.x != 0) return;
  float s = staged ? part[0] : p.partials[0];
  for (int b = 1; b < blocks; ++b) s = s + (staged ? part[b] : p.partials[b]);
  const float denom = p.loss == VOLTA_LOSS_MSE ? (float)(p.B * p.N) : (float)p.B;
  step_epilogue(p.scalars, p.bc_table, p.bc_len, s / denom);
}

// The narrow output layer, its loss head and its dX in one launch (B <=
// kNarrowMaxB).  Wave w of block b owns batch row m = 4b + w:
//   z = act_{n-1}[m] W + bias     (wave_rows: lane k-strided, fixed butterfly)
//   delta_{n-1}[m] and the row loss (head_delta, identical in every lane;
//                                     lane 0 stores z and the deltas)
//   delta_{n-2}[m][k] = (sum_j delta_{n-1}[m][j] W[k][j]) * f'(pre, act)
//                                    for the lane's k = lane + 64c (j ascending,
//                                    outer_dx_kernel's order)
// Everything but the loss is row-local.  The block's row losses are added in
// row order into partials[b].  With defer_loss (the small-batch step, whose
// grouped dW launch adds the partials later) block 0 only advances the Adam
// step counter; otherwise the last block to finish (integer ticket, an
// agent-scope release and acquire) adds the partials in block order and
// records the step's loss, the non-finite flag and the step counter.  A
// separate one-block output launch plus the outer-product dX launch cost
// more: one CU for 64 rows, and a dependent launch between them.

template <int NMAX, bool WL>
__global__ void __launch_bounds__(kOutDxRows * 64) out_layer_dx_kernel(OutLayerArgs p) {
  __shared__ float wave_loss[kOutDxRows];
  __shared__ unsigned last_block;
  extern __shared__ float w_lds[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int N = p.N, K = p.K;
  if constexpr (WL) {
    const int KN = K * N;
    for (int i0 = 0; i0 < KN; i0 += kOutDxRows * 64 * kOutStage) {
      float t[kOutStage];
#pragma unroll
      for (int it = 0; it < kOutStage; ++it) t[it] = p.W[min(i0 + (int)threadIdx.x + kOutDxRows * 64 * it, KN - 1)];
#pragma unroll
      for (int it = 0; it < kOutStage; ++it) {
        const int i = i0 + (int)threadIdx.x + kOutDxRows * 64 * it;
        if (i < KN) w_lds[i] = t[it];
      }
    }
    __syncthreads();
  }
  // the next step counter and its bias corrections, in case this block
  // finishes last (nothing else in the launch writes them); with the loss
  // deferred, block 0 alone reads and advances the counter
  StepNext next{};
  if (threadIdx.x == 0 && (!p.defer_loss || blockIdx.x == 0)) next = step_prefetch(p.scalars, p.bc_table, p.bc_len);
  const float row_loss = out_dx_row<NMAX, WL>(p, w_lds, blockIdx.x * kOutDxRows + wave);
  if (lane == 0) wave_loss[wave] = row_loss;
  __syncthreads();
  if (threadIdx.x == 0) {
    float sb = wave_loss[0];
    for (int w = 1; w < kOutDxRows; ++w) sb = sb + wave_loss[w];
    p.partials[blockIdx.x] = sb;
    if (p.defer_loss) {
      // a later launch of the step adds the partials (deferred_loss_finish):
      // no agent-scope fence or ticket here
      if (blockIdx.x == 0 && p.bc_table) {
        p.scalars->t = next.t;
        p.scalars->bc1 = next.bc.x;
        p.scalars->bc2 = next.bc.y;
      }
      return;
    }
    __threadfence();
    last_block = atomicAdd(p.loss_counter, 1u) == gridDim.x - 1 ? 1u : 0u;
    if (last_block) {
      __threadfence();
      out_dx_finish(p, (int)gridDim.x, next);
    }
  }
}

int out_layer_dx_blocks(int B) { return (B + kOutDxRows - 1) / kOutDxRows; }

bool out_layer_dx_supported(int B, int K, int N) {
  return B >= 1 && B <= kNarrowMaxB && K >= 1 && N >= 1 && N <= 16 &&
         (N == 1 || (size_t)K * N <= (size_t)kOutWlFloats);
}

hipError_t launch_out_layer_dx(const OutLayerArgs& p, hipStream_t st) {
  if (!out_layer_dx_supported(p.B, p.K, p.N) || !p.partials || (!p.loss_counter && !p.defer_loss) || !p.dx_out)
    return hipErrorInvalidValue;
  const dim3 grid(out_layer_dx_blocks(p.B)), block(kOutDxRows * 64);
  const bool wl = p.N > 1;
  const size_t lds = wl ? (size_t)p.K * p.N * sizeof(float) : 0;
  if (p.N <= 1)
    hipLaunchKernelGGL((out_layer_dx_kernel<1, false>), grid, block, 0, st, p);
  else if (p.N <= 4)
    hipLaunchKernelGGL((out_layer_dx_kernel<4, true>), grid, block, lds, st, p);
  else
    hipLaunchKernelGGL((out_layer_dx_kernel<16, true>), grid, block, lds, st, p);
  return hipGetLastError();
}

// delta_out[b][j] = (sum_{k<K} delta[b][k] * W[j][k]) * f'(layer below)[b][j]
// for K <= KMAX <= 16 (reference order: k ascending, :919-929).  Thread j of
// a block keeps row j of W in registers for the block's RB batch rows, whose
// deltas are staged in LDS; its loads (W row, then the activation operands
// of all RB rows) are unconditional (clamped indices) and issued together.
// RB = 16 on large layers (the W row is loaded once per 16 outputs), 1 on
// small ones (more blocks).
template <int KMAX, int RB>
__global__ void __launch_bounds__(256)
outer_dx_kernel(const float* __restrict__ delta, const float* __restrict__ W, int B, int R, int K, int act,
                const float* __restrict__ aux_act, const float* __restrict__ aux_pre, float* __restrict__ out,
                LossDefer ld) {
  static_assert(RB * KMAX <= 256, "one staged delta per thread");
  __shared__ float sd[RB * KMAX];
  const int t = threadIdx.x;
  const int j = blockIdx.x * 256 + t, jc = min(j, R - 1);
  const int b0 = blockIdx.y * RB;
  const float dv = delta[(size_t)min(b0 + t / KMAX, B - 1) * K + min(t % KMAX, K - 1)];
  float wv[KMAX];
#pragma unroll
  for (int k = 0; k < KMAX; ++k) wv[k] = W[(size_t)jc * K + min(k, K - 1)];
  const float* pp = aux_pre ? aux_pre : aux_act;
  // block (0, 0) also forms the step's loss (below): its first 256 partials
  // are loaded now, so their latency runs under the block's products
  const bool loss_block = ld.partials && blockIdx.x == 0 && blockIdx.y == 0;  // block-uniform
  const float p0 = loss_block ? ld.partials[min(t, ld.blocks - 1)] : 0.0f;
  float y[RB], pr[RB];
  if (aux_pre) {  // uniform: f' from the kept pre-activation
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const size_t o = (size_t)min(b0 + r, B - 1) * R + jc;
      y[r] = aux_act[o];
      pr[r] = pp[o];
    }
  } else {  // f' from the output: one load per element
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      y[r] = aux_act[(size_t)min(b0 + r, B - 1) * R + jc];
      pr[r] = y[r];
    }
  }
  if (t < RB * KMAX) sd[t] = dv;
  __syncthreads();
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
      const float u = s + sd[r * KMAX + k] * wv[k];
      s = k < K ? u : s;
    }
    if (j < R && b0 + r < B) out[(size_t)(b0 + r) * R + j] = s * act_derivative(act, pr[r], y[r]);
  }
  if (loss_block) deferred_loss_tree(ld, p0, t);  // the step's loss
}

// Stand-alone launch: 64 rows of W per block.
template <int NMAX>
__global__ void __launch_bounds__(kNarrowThreads) narrow_dw_kernel(NarrowDwArgs p) {
  extern __shared__ float lds[];
  narrow_dw_block<NMAX>(p, blockIdx.x, lds);
}

// ---------------------------------------------------------------------------
int out_layer_blocks(int B) { return B <= 256 ? 1 : (B + 15) / 16; }

hipError_t launch_out_layer(const OutLayerArgs& p, hipStream_t st) {
  if (p.N > 16 || p.N < 1) return hipErrorInvalidValue;
  const int blocks = out_layer_blocks(p.B);
  const int rows = blocks == 1 ? p.B : 16;
  if (blocks > 1 && !p.partials) return hipErrorInvalidValue;
  // with one column, lanes read consecutive floats of W: no staging needed
  const bool wl = p.N > 1 && (size_t)p.K * p.N <= (size_t)kOutWlFloats;
  const size_t lds = wl ? (size_t)p.K * p.N * sizeof(float) : 0;
  if (p.N <= 1) {
    if (wl) hipLaunchKernelGGL((out_layer_kernel<1, true>), dim3(blocks), dim3(1024), lds, st, p, rows);
    else hipLaunchKernelGGL((out_layer_kernel<1, false>), dim3(blocks), dim3(1024), 0, st, p, rows);
  } else if (p.N <= 4) {
    if (wl) hipLaunchKernelGGL((out_layer_kernel<4, true>), dim3(blocks), dim3(1024), lds, st, p, rows);
    else hipLaunchKernelGGL((out_layer_kernel<4, false>), dim3(blocks), dim3(1024), 0, st, p, rows);
  } else {
    if (wl) hipLaunchKernelGGL((out_layer_kernel<16, true>), dim3(blocks), dim3(1024), lds, st, p, rows);
    else hipLaunchKernelGGL((out_layer_kernel<16, false>), dim3(blocks), dim3(1024), 0, st, p, rows);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || blocks == 1) return e;
  hipLaunchKernelGGL(loss_finish_kernel, dim3(1), dim3(64), 0, st, p, blocks);
  return hipGetLastError();
}

template <int KMAX>
static void launch_outer_k(bool big, dim3 blocks, hipStream_t st, const float* delta, const float* W, int B, int R,
                           int K, int act, const float* aux_act, const float* aux_pre, float* out,
                           const LossDefer& ld) {
  if (big)
    hipLaunchKernelGGL((outer_dx_kernel<KMAX, 16>), blocks, dim3(256), 0, st, delta, W, B, R, K, act, aux_act,
                       aux_pre, out, ld);
  else
    hipLaunchKernelGGL((outer_dx_kernel<KMAX, 1>), blocks, dim3(256), 0, st, delta, W, B, R, K, act, aux_act,
                       aux_pre, out, ld);
}

hipError_t launch_outer_dx(const float* delta, const float* W, int B, int R, int K, int act, const float* aux_act,
                           const float* aux_pre, float* out, hipStream_t st, const LossDefer& ld) {
  if (K > 16 || K < 1) return hipErrorInvalidValue;
  if (ld.partials && (ld.blocks < 1 || !ld.scalars)) return hipErrorInvalidValue;
  // 16 batch rows per block once the layer has a million outputs
  const bool big = (size_t)B * R >= ((size_t)1 << 20);
  const dim3 blocks((R + 255) / 256, (B + (big ? 16 : 1) - 1) / (big ? 16 : 1));
  if (K <= 1) launch_outer_k<1>(big, blocks, st, delta, W, B, R, K, act, aux_act, aux_pre, out, ld);
  else if (K <= 4) launch_outer_k<4>(big, blocks, st, delta, W, B, R, K, act, aux_act, aux_pre, out, ld);
  else launch_outer_k<16>(big, blocks, st, delta, W, B, R, K, act, aux_act, aux_pre, out, ld);
  return hipGetLastError();
}

hipError_t launch_narrow_dw(const NarrowDwArgs& p, hipStream_t st) {
  if (p.N > 16 || p.N < 1 || p.B < 1 || p.B > kNarrowMaxB) return hipErrorInvalidValue;
  if (p.opt != VOLTA_OPT_SGD && p.opt != VOLTA_OPT_ADAM && p.opt != VOLTA_OPT_ADAGRAD) return hipErrorInvalidValue;
  const int blocks = (p.R + kNarrowRows - 1) / kNarrowRows;
  const dim3 block(kNarrowThreads);
  if (p.N <= 1)
    hipLaunchKernelGGL(narrow_dw_kernel<1>, dim3(blocks), block, narrow_lds_floats<1>(p.B, p.N) * 4, st, p);
  else if (p.N <= 4)
    hipLaunchKernelGGL(narrow_dw_kernel<4>, dim3(blocks), block, narrow_lds_floats<4>(p.B, p.N) * 4, st, p);
  else
    hipLaunchKernelGGL(narrow_dw_kernel<16>, dim3(blocks), block, narrow_lds_floats<16>(p.B, p.N) * 4, st, p);
  return hipGetLastError();
}

}  // namespace volta
