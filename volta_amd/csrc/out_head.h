// Row-level device code of the narrow output layer (L[n] <= 16 columns),
// shared by skinny.hip's output launches and the last hidden layer's
// forward launch that also runs the output layer (gemm.hip).
#pragma once

#include <hip/hip_runtime.h>

#include "device_common.h"
#include "skinny.h"

namespace volta {

// Output rows z[g][0..N) of RG rows (rows[g], valid where rows[g] >= 0),
// computed by a whole wave: lane l sums k = l, l+64, ... in ascending order,
// then a fixed butterfly adds the lanes.  The k loop runs in chunks of C
// values per lane whose activation loads (all RG rows) are issued before
// the chunk's first multiply, so a chunk costs one memory latency.  W comes
// from the block's LDS copy `wl` (WL) -- lane l reads row k of W, so for
// N > 1 global loads of W would touch a cache line per lane for each of its
// N columns -- or, for one column or a W too large to stage, from global
// memory with the chunk's other loads.  Every global load is unconditional (clamped row and k;
// terms outside the matrix are not added), so no branch or wait separates
// them.
template <int NMAX, int RG, int C, bool WL>
__device__ __forceinline__ void wave_rows(const OutLayerArgs& p, const float* wl, const int* rows,
                                          float (*z)[NMAX]) {
  const int lane = threadIdx.x & 63;
  const int K = p.K, N = p.N;
  float acc[RG][NMAX];
#pragma unroll
  for (int g = 0; g < RG; ++g)
#pragma unroll
    for (int j = 0; j < NMAX; ++j) acc[g][j] = 0.0f;
  for (int kb = 0; kb < K; kb += 64 * C) {
    float x[RG][C], wg[WL ? 1 : C][NMAX];
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int kc = min(kb + 64 * c + lane, K - 1);
      if constexpr (!WL) {
#pragma unroll
        for (int j = 0; j < NMAX; ++j) wg[c][j] = p.W[(size_t)kc * N + min(j, N - 1)];
      }
#pragma unroll
      for (int g = 0; g < RG; ++g) x[g][c] = p.act[(size_t)(rows[g] >= 0 ? rows[g] : 0) * K + kc];
    }
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int kc = min(kb + 64 * c + lane, K - 1);
      float wv[NMAX];
#pragma unroll
      for (int j = 0; j < NMAX; ++j) wv[j] = WL ? wl[kc * N + min(j, N - 1)] : wg[WL ? 0 : c][j];
#pragma unroll
      for (int g = 0; g < RG; ++g) {
        const bool in = kb + 64 * c + lane < K && rows[g] >= 0;
#pragma unroll
        for (int j = 0; j < NMAX; ++j) {
          const float t = acc[g][j] + x[g][c] * wv[j];
          acc[g][j] = in && j < N ? t : acc[g][j];
        }
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
// (interpreter.rs:762-812, autograd.rs:467-534).  head_delta forms the
// row's deltas and returns its loss without storing anything, so every lane
// of a wave can hold the deltas; head_row also stores z and the deltas.
// `y` holds the row's targets (MSE), `lab` its label (CE), both loaded
// before z was computed.  (Loops run to NMAX with a j < N guard so z stays
// in registers.)
template <int NMAX>
__device__ __forceinline__ float head_delta(const OutLayerArgs& p, const float* z, const float* y, int lab,
                                            float* d) {
  const int N = p.N;
  if (p.loss == VOLTA_LOSS_MSE) {
    const float nt = (float)(p.B * N);
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < NMAX; ++j) {
      if (j < N) {
        const float dj = z[j] - y[j];
        acc = acc + dj * dj;
        d[j] = 2.0f * dj / nt;
      } else {
        d[j] = 0.0f;
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
    } else {
      d[j] = 0.0f;
    }
  }
  return sample;
}

template <int NMAX>
__device__ __forceinline__ float head_row(const OutLayerArgs& p, const float* z, const float* y, int lab, int m) {
  const int N = p.N;
  float d[NMAX];
  const float l = head_delta<NMAX>(p, z, y, lab, d);
  float* out = p.out + (size_t)m * N;
  float* dd = p.delta + (size_t)m * N;
#pragma unroll
  for (int j = 0; j < NMAX; ++j) {
    if (j < N) {
      out[j] = z[j];
      dd[j] = d[j];
    }
  }
  if (p.loss != VOLTA_LOSS_MSE && (lab < 0 || lab >= N)) atomicOr(&p.scalars->flags, (uint32_t)VOLTA_STATUS_BAD_ARGUMENT);
  return l;
}

// Rows (waves) per block of the output launch that also forms dX_{n-1}.
constexpr int kOutDxRows = 4;
constexpr int kOutDxMaxBlocks = (kNarrowMaxB + kOutDxRows - 1) / kOutDxRows;

// Batch row m of the output layer, computed by one wave: z = act_{n-1}[m] W
// + b, the loss head (z and delta_{n-1} stored by lane 0), and the row of
// delta_{n-2} = (delta_{n-1} W^T) * f'(layer n-2).  Returns the row's loss
// (0 for m >= B, whose loads are clamped and whose results are not stored).
template <int NMAX, bool WL>
__device__ __forceinline__ float out_dx_row(const OutLayerArgs& p, const float* w_lds, int m) {
  constexpr int C = 4;
  const int lane = threadIdx.x & 63;
  const int N = p.N, K = p.K;
  const bool has = m < p.B;
  const int mc = has ? m : p.B - 1;
  const bool mse = p.loss == VOLTA_LOSS_MSE;
  float bias[NMAX], y[NMAX];
#pragma unroll
  for (int j = 0; j < NMAX; ++j) {
    bias[j] = p.bias[min(j, N - 1)];
    y[j] = mse ? p.y[(size_t)mc * N + min(j, N - 1)] : 0.0f;
  }
  const int lab = mse ? 0 : p.labels[mc];
  const int rows[1] = {has ? m : -1};
  float z[1][NMAX];
  wave_rows<NMAX, 1, C, WL>(p, w_lds, rows, z);
#pragma unroll
  for (int j = 0; j < NMAX; ++j) z[0][j] = z[0][j] + bias[j];
  float d[NMAX];
  const float row_loss = head_delta<NMAX>(p, z[0], y, lab, d);
  if (has && lane == 0) (void)head_row<NMAX>(p, z[0], y, lab, m);

  // delta_{n-2} of this row
  if (has) {
    const float* act = p.act + (size_t)m * K;
    const float* pre = p.dx_pre ? p.dx_pre + (size_t)m * K : act;
    float* out = p.dx_out + (size_t)m * K;
    for (int kb = 0; kb < K; kb += 64 * C) {
      float av[C], pv[C], wv[C][NMAX];
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const int kc = min(kb + 64 * c + lane, K - 1);
        av[c] = act[kc];
        pv[c] = pre[kc];
#pragma unroll
        for (int j = 0; j < NMAX; ++j) wv[c][j] = WL ? w_lds[kc * N + min(j, N - 1)] : p.W[(size_t)kc * N + min(j, N - 1)];
      }
#pragma unroll
      for (int c = 0; c < C; ++c) {
        float sacc = 0.0f;
#pragma unroll
        for (int j = 0; j < NMAX; ++j) {
          const float u = sacc + d[j] * wv[c][j];
          sacc = j < N ? u : sacc;
        }
        const int k = kb + 64 * c + lane;
        if (k < K) out[k] = sacc * act_derivative(p.dx_act, pv[c], av[c]);
      }
    }
  }
  return has ? row_loss : 0.0f;
}

// Rows rows[g] (g < RG) of a one-column output layer computed together by
// one wave, as out_dx_row computes each (wave_rows adds every row in the
// same k order whatever RG, then the same loss head), MSE only: lane 0
// writes each row's z to z_rows[g] and its delta_{n-1} to d_rows[g] (also
// for rows >= B), and every lane gets the row losses in losses[g] (0 for
// rows >= B).  Nothing is stored to global memory.
template <int RG>
__device__ __forceinline__ void out_head_rows(const OutLayerArgs& p, const int* rows, float* z_rows, float* d_rows,
                                              float* losses) {
  const int lane = threadIdx.x & 63;
  const float bias = p.bias[0];
  int wr[RG];
  float y[RG][1];
#pragma unroll
  for (int g = 0; g < RG; ++g) {
    const bool has = rows[g] < p.B;
    wr[g] = has ? rows[g] : -1;
    y[g][0] = p.y[has ? rows[g] : p.B - 1];
  }
  float z[RG][1];
  wave_rows<1, RG, 4, false>(p, nullptr, wr, z);
#pragma unroll
  for (int g = 0; g < RG; ++g) {
    z[g][0] = z[g][0] + bias;
    float d[1];
    const float l = head_delta<1>(p, z[g], y[g], 0, d);
    if (lane == 0) {
      z_rows[g] = z[g][0];
      d_rows[g] = d[0];
    }
    losses[g] = wr[g] >= 0 ? l : 0.0f;
  }
}

// The step's loss from the per-block partials (blocks of kOutDxRows rows,
// all loads issued together, added in block order), then the step counter
// and the arrival ticket reset; run by the one thread that arrived last.
__device__ __forceinline__ float out_dx_loss_sum(const float* partials, int nblocks) {
  float part[kOutDxMaxBlocks];
#pragma unroll
  for (int b = 0; b < kOutDxMaxBlocks; ++b) part[b] = partials[min(b, nblocks - 1)];
  float total = part[0];
#pragma unroll
  for (int b = 1; b < kOutDxMaxBlocks; ++b) {
    const float t = total + part[b];
    total = b < nblocks ? t : total;
  }
  return total;
}

__device__ __forceinline__ float out_dx_loss_denom(const OutLayerArgs& p) {
  return p.loss == VOLTA_LOSS_MSE ? (float)(p.B * p.N) : (float)p.B;
}

__device__ __forceinline__ void out_dx_finish(const OutLayerArgs& p, int nblocks, const StepNext& next) {
  step_finish(p.scalars, next, p.bc_table != nullptr, out_dx_loss_sum(p.partials, nblocks) / out_dx_loss_denom(p));
  *p.loss_counter = 0u;
}

// The deferred form: the loss of the partials an earlier output launch
// stored (launch_out_layer_dx with defer_loss), the same sum in block order,
// and its non-finite flag; the step counter was advanced by that launch.
__device__ __forceinline__ void deferred_loss_finish(DevScalars* sc, const float* partials, int nblocks,
                                                     float denom) {
  const float loss = out_dx_loss_sum(partials, nblocks) / denom;
  sc->loss = loss;
  if (!(fabsf(loss) <= 3.402823466e38f)) atomicOr(&sc->flags, (uint32_t)VOLTA_STATUS_NONFINITE_LOSS);
}

}  // namespace volta
