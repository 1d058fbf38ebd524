// Non-GEMM kernels of the MLP step: the stand-alone loss heads (used when the
// output layer is wider than one GEMM tile) and flat optimizer passes (the
// step fuses the optimizer into the dW epilogue; these run the same element
// functions over whole buffers for checks).  All reductions use a fixed
// association order and no floating-point atomics.
#include "step_kernels.h"

namespace volta {

// Block-wide sum with a fixed order: butterfly inside each wave, then wave
// partials added in wave order by thread 0.  Result valid in thread 0.
template <int THREADS>
__device__ __forceinline__ float block_sum_fixed(float v, float* lds) {
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) lds[wave] = v;
  __syncthreads();
  float s = 0.0f;
  if (threadIdx.x == 0) {
    s = lds[0];
    for (int w = 1; w < THREADS / kWave; ++w) s = s + lds[w];
  }
  return s;
}

// MSE head (mlp_train_rust_codegen.rs:792-798): d = yhat - y,
// loss = sum(d^2)/nt, delta = 2*d/nt with nt = B*Ln.
__global__ void __launch_bounds__(1024)
loss_mse_kernel(const float* __restrict__ yhat, const float* __restrict__ y, float* __restrict__ delta,
                int nt, DevScalars* sc, const float2* bc_table, int bc_len) {
  __shared__ float lds[1024 / kWave];
  const float ntf = (float)nt;
  float acc = 0.0f;
  for (int k = threadIdx.x; k < nt; k += 1024) {
    const float d = yhat[k] - y[k];
    acc = acc + d * d;
    delta[k] = 2.0f * d / ntf;
  }
  const float s = block_sum_fixed<1024>(acc, lds);
  if (threadIdx.x == 0) step_epilogue(sc, bc_table, bc_len, s / ntf);
}

// Softmax cross-entropy head with integer labels.
// Loss (interpreter.rs:762-812): per row max, sum of exp(z - max),
// lse = max + ln(sum), sample loss -(z_label - lse); mean over B.
// Gradient (autograd.rs:467-534): (softmax(z) - onehot) / B with
// softmax = exp(z - max) / sum (kernels/reduce.rs:203-213).
// One thread per row; an out-of-range label raises BAD_ARGUMENT and makes
// that row's loss NaN (it is never used as an index).
__global__ void __launch_bounds__(1024)
loss_ce_kernel(const float* __restrict__ z, const int32_t* __restrict__ labels,
               float* __restrict__ delta, int B, int C, DevScalars* sc, const float2* bc_table,
               int bc_len) {
  __shared__ float lds[1024 / kWave];
  const float bf = (float)B;
  float acc = 0.0f;
  bool bad = false;
  for (int b = threadIdx.x; b < B; b += 1024) {
    const float* zr = z + (size_t)b * C;
    float* dr = delta + (size_t)b * C;
    const int lab = labels[b];
    float mx = -INFINITY;
    for (int j = 0; j < C; ++j) mx = fmaxf(mx, zr[j]);
    float sum = 0.0f;
    for (int j = 0; j < C; ++j) sum = sum + expf(zr[j] - mx);
    const float lse = mx + logf(sum);
    float sample = __builtin_nanf("");
    for (int j = 0; j < C; ++j) {
      const bool on = j == lab;
      if (on) sample = -(zr[j] - lse);
      dr[j] = (expf(zr[j] - mx) / sum - (on ? 1.0f : 0.0f)) / bf;
    }
    bad |= lab < 0 || lab >= C;
    acc = acc + sample;
  }
  const int any_bad = __syncthreads_or(bad ? 1 : 0);
  const float s = block_sum_fixed<1024>(acc, lds);
  if (threadIdx.x == 0) {
    if (any_bad) atomicOr(&sc->flags, (uint32_t)VOLTA_STATUS_BAD_ARGUMENT);
    step_epilogue(sc, bc_table, bc_len, s / bf);
  }
}

// Find the segment holding flat element `base` (segments are padded to
// kSegAlign floats, so a whole block lies in one segment).
__device__ __forceinline__ int find_segment(const SegTable& t, int64_t base) {
  int s = 0;
  for (int i = 1; i < t.n; ++i)
    if (base >= t.off[i]) s = i;
  return s;
}

// Adam / AdamW over a flat segmented buffer (adam_update,
// mlp_train_rust_codegen.rs:326-388; the tail rule is per segment).
__global__ void __launch_bounds__(256)
adam_kernel(float* __restrict__ w, float* __restrict__ m, float* __restrict__ v,
            const float* __restrict__ g, SegTable segs, const DevScalars* __restrict__ sc,
            float b1, float b2, float eps) {
  const int64_t base = (int64_t)blockIdx.x * kSegAlign;
  const int s = find_segment(segs, base);
  const float lr = sc->lr;
  const AdamRcp rc = adam_rcp(sc->bc1, sc->bc2);
  const float wd = segs.wd[s];
  const int64_t count = segs.count[s];
  const int64_t vec_end = count - count % 8;
  for (int e = threadIdx.x; e < kSegAlign; e += 256) {
    const int64_t local = base - segs.off[s] + e;
    if (local >= count) continue;
    const int64_t k = base + e;
    adam_elem(w + k, m + k, v + k, g[k], local >= vec_end, lr, rc, b1, b2, eps, wd);
  }
}

// Adagrad over a flat segmented buffer (mlp_train_rust_codegen.rs:967-985).
__global__ void __launch_bounds__(256)
adagrad_kernel(float* __restrict__ w, float* __restrict__ G, const float* __restrict__ g,
               SegTable segs, const DevScalars* __restrict__ sc, float eps) {
  const int64_t base = (int64_t)blockIdx.x * kSegAlign;
  const int s = find_segment(segs, base);
  const float lr = sc->lr;
  const int64_t count = segs.count[s];
  for (int e = threadIdx.x; e < kSegAlign; e += 256) {
    const int64_t local = base - segs.off[s] + e;
    if (local >= count) continue;
    const int64_t k = base + e;
    adagrad_elem(w + k, G + k, g[k], lr, eps);
  }
}

// ---------------------------------------------------------------------------
hipError_t launch_loss_mse(const float* yhat, const float* y, float* delta, int nt, DevScalars* sc,
                           const float2* bc_table, int bc_len, hipStream_t st) {
  hipLaunchKernelGGL(loss_mse_kernel, dim3(1), dim3(1024), 0, st, yhat, y, delta, nt, sc, bc_table,
                     bc_len);
  return hipGetLastError();
}

hipError_t launch_loss_ce(const float* z, const int32_t* labels, float* delta, int B, int C,
                          DevScalars* sc, const float2* bc_table, int bc_len, hipStream_t st) {
  hipLaunchKernelGGL(loss_ce_kernel, dim3(1), dim3(1024), 0, st, z, labels, delta, B, C, sc, bc_table,
                     bc_len);
  return hipGetLastError();
}

hipError_t launch_adam(float* w, float* m, float* v, const float* g, const SegTable& segs,
                       int64_t total, const DevScalars* sc, float b1, float b2, float eps,
                       hipStream_t st) {
  const int blocks = (int)(total / kSegAlign);
  hipLaunchKernelGGL(adam_kernel, dim3(blocks), dim3(256), 0, st, w, m, v, g, segs, sc, b1, b2, eps);
  return hipGetLastError();
}

hipError_t launch_adagrad(float* w, float* G, const float* g, const SegTable& segs, int64_t total,
                          const DevScalars* sc, float eps, hipStream_t st) {
  const int blocks = (int)(total / kSegAlign);
  hipLaunchKernelGGL(adagrad_kernel, dim3(blocks), dim3(256), 0, st, w, G, g, segs, sc, eps);
  return hipGetLastError();
}

}  // namespace volta
