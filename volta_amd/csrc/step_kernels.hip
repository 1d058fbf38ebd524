// Non-GEMM kernels of the MLP step: loss heads, bias-gradient column sums,
// flat optimizer passes.  All reductions use a fixed association order and
// no atomics, so two runs on the same inputs are bit-identical.
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

// Once per step, after the loss: advance the Adam step counter and publish
// the bias corrections 1 - beta^t, looked up in a table the host filled with
// the same f32 powf the reference calls (mlp_train_rust_codegen.rs:803-811).
__device__ __forceinline__ void step_epilogue(DevScalars* sc, const float2* bc_table, int bc_len,
                                              float loss) {
  sc->loss = loss;
  if (!(fabsf(loss) <= 3.402823466e38f)) sc->flags |= VOLTA_STATUS_NONFINITE_LOSS;
  if (bc_table) {
    const uint32_t t = sc->t + 1u;
    sc->t = t;
    const float2 bc = bc_table[t < (uint32_t)bc_len ? t : (uint32_t)(bc_len - 1)];
    sc->bc1 = bc.x;
    sc->bc2 = bc.y;
  }
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
    float sample = 0.0f;
    bool hit = false;
    for (int j = 0; j < C; ++j) {
      const bool on = j == lab;
      hit |= on;
      if (on) sample = -(zr[j] - lse);
      dr[j] = (expf(zr[j] - mx) / sum - (on ? 1.0f : 0.0f)) / bf;
    }
    if (!hit) {
      bad = true;
      sample = __builtin_nanf("");
    }
    acc = acc + sample;
  }
  const int any_bad = __syncthreads_or(bad ? 1 : 0);
  const float s = block_sum_fixed<1024>(acc, lds);
  if (threadIdx.x == 0) {
    if (any_bad) sc->flags |= VOLTA_STATUS_BAD_ARGUMENT;
    step_epilogue(sc, bc_table, bc_len, s / bf);
  }
}

// Bias gradient db[j] = sum_b delta[b, j] (mlp_train_rust_codegen.rs:931-933).
// Stage 1: block (x, y) sums rows [y*rows_per_part, ...) of 256 columns in
// row order.  With one part it writes db directly (and, for SGD, applies
// b -= lr*db, :986-991); otherwise it writes partial[y][j].
__global__ void __launch_bounds__(256)
colsum_kernel(const float* __restrict__ delta, int B, int c, int rows_per_part,
              float* __restrict__ out, float* __restrict__ bias, const DevScalars* sc) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= c) return;
  const int r0 = blockIdx.y * rows_per_part;
  const int r1 = min(B, r0 + rows_per_part);
  float s = 0.0f;
  for (int r = r0; r < r1; ++r) s = s + delta[(size_t)r * c + j];
  if (gridDim.y == 1) {
    out[j] = s;
    if (bias) bias[j] = bias[j] - sc->lr * s;
  } else {
    out[(size_t)blockIdx.y * c + j] = s;
  }
}

// Stage 2: db[j] = sum over parts in part order (+ SGD bias update).
__global__ void __launch_bounds__(256)
colsum_final_kernel(const float* __restrict__ partial, int parts, int c, float* __restrict__ db,
                    float* __restrict__ bias, const DevScalars* sc) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= c) return;
  float s = partial[j];
  for (int p = 1; p < parts; ++p) s = s + partial[(size_t)p * c + j];
  db[j] = s;
  if (bias) bias[j] = bias[j] - sc->lr * s;
}

// Find the segment holding flat element `base` (segments are padded to
// kSegAlign floats, so a whole block lies in one segment).
__device__ __forceinline__ int find_segment(const SegTable& t, int64_t base) {
  int s = 0;
  for (int i = 1; i < t.n; ++i)
    if (base >= t.off[i]) s = i;
  return s;
}

// Adam / AdamW over the flat parameter buffer, one element per thread
// (adam_update_slice, mlp_train_rust_codegen.rs:341-388; AdamW decays
// weights only, :960-966).  The reference computes v with (1-b2)*(g*g) in
// its 8-wide loop and ((1-b2)*g)*g in the scalar tail (last n%8 elements of
// each buffer); the same split is kept per segment.
__global__ void __launch_bounds__(256)
adam_kernel(float* __restrict__ w, float* __restrict__ m, float* __restrict__ v,
            const float* __restrict__ g, SegTable segs, const DevScalars* __restrict__ sc,
            float b1, float b2, float eps) {
  const int64_t base = (int64_t)blockIdx.x * kSegAlign;
  const int s = find_segment(segs, base);
  const float lr = sc->lr, bc1 = sc->bc1, bc2 = sc->bc2;
  const float wd = segs.wd[s];
  const int64_t count = segs.count[s];
  const int64_t vec_end = count - count % 8;
  const float omb1 = 1.0f - b1, omb2 = 1.0f - b2;
  for (int e = threadIdx.x; e < kSegAlign; e += 256) {
    const int64_t local = base - segs.off[s] + e;
    if (local >= count) continue;
    const int64_t k = base + e;
    const float gk = g[k];
    const float m1 = b1 * m[k] + omb1 * gk;
    const float v1 = local >= vec_end ? b2 * v[k] + omb2 * gk * gk : b2 * v[k] + omb2 * (gk * gk);
    m[k] = m1;
    v[k] = v1;
    const float w0 = w[k];
    const float mhat = m1 / bc1;
    const float vhat = v1 / bc2;
    const float denom = sqrtf(vhat) + eps;
    w[k] = w0 - lr * (mhat / denom + wd * w0);
  }
}

// Adagrad (mlp_train_rust_codegen.rs:967-985): G += g^2; w -= lr*g/(sqrt(G)+eps).
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
    const float gk = g[k];
    const float Gk = G[k] + gk * gk;
    G[k] = Gk;
    w[k] = w[k] - lr * gk / (sqrtf(Gk) + eps);
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

int colsum_parts(int B) {
  if (B <= 256) return 1;
  int parts = B / 128;
  return parts > 32 ? 32 : parts;
}

hipError_t launch_colsum(const float* delta, int B, int c, float* db, float* bias, const DevScalars* sc,
                         float* workspace, hipStream_t st, Recorder* rec, const char* label) {
  const int parts = colsum_parts(B);
  const int rpp = (B + parts - 1) / parts;
  dim3 grid((c + 255) / 256, parts);
  // algorithmic traffic of db = colsum(delta): 4(B*c + c) bytes
  const double bytes = 4.0 * ((double)B * c + c);
  if (parts == 1) {
    hipLaunchKernelGGL(colsum_kernel, grid, dim3(256), 0, st, delta, B, c, rpp, db, bias, sc);
    hipError_t e = hipGetLastError();
    return e != hipSuccess ? e : mark(rec, label, (double)B * c, bytes);
  }
  hipLaunchKernelGGL(colsum_kernel, grid, dim3(256), 0, st, delta, B, c, rpp, workspace,
                     (float*)nullptr, sc);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) e = mark(rec, label, (double)B * c, bytes);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(colsum_final_kernel, dim3((c + 255) / 256), dim3(256), 0, st, workspace, parts, c,
                     db, bias, sc);
  e = hipGetLastError();
  return e != hipSuccess ? e : mark(rec, std::string(label) + ".final", (double)parts * c, 4.0 * ((double)parts * c + c));
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
