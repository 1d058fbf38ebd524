// Device-side helpers shared by the gfx950 kernels of the MLP step.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/volta_train.h"

namespace volta {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;

// Per-handle scalars the captured step reads and writes on the device, so a
// graph replay needs no host-side argument patching.
struct DevScalars {
  float lr;        // learning rate of the current step (host uploads on change)
  float bc1;       // Adam bias corrections for the current step
  float bc2;
  uint32_t t;      // Adam step counter (incremented once per step on device)
  float loss;      // loss of the most recent step
  uint32_t flags;  // sticky VOLTA_STATUS_* bits raised on the device
  float clip_scale;  // gradient clipping: factor applied to the deltas of this step
  uint64_t rng;      // dropout LCG state at the start of the step's forward
};

// Hidden activations, mlp_train_rust_codegen.rs:563-596 (forward) and
// :893-916 (derivative).  Same expression order as the reference; the
// library is built with -ffp-contract=off so nothing is fused into FMAs.
// kIdentity marks the linear output layer.  kRtSigmoid is the runtime
// interpreter's sigmoid (kernels/activations.rs:82-90), used by graph
// execution: the same 1/(1+e^-x) for x >= 0, e^x/(1+e^x) below.
constexpr int kIdentity = -1;
constexpr int kRtSigmoid = 16;

__device__ __forceinline__ float d_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

__device__ __forceinline__ float act_forward(int act, float x) {
  switch (act) {
    case VOLTA_ACT_RELU: return x > 0.0f ? x : 0.0f;
    case VOLTA_ACT_SIGMOID: return d_sigmoid(x);
    case kRtSigmoid: {
      if (x >= 0.0f) return 1.0f / (1.0f + expf(-x));
      const float e = expf(x);
      return e / (1.0f + e);
    }
    case VOLTA_ACT_TANH: return tanhf(x);
    case VOLTA_ACT_LEAKY_RELU: return x > 0.0f ? x : 0.01f * x;
    case VOLTA_ACT_SILU: return x * d_sigmoid(x);
    case VOLTA_ACT_GELU: {
      const float c = 0.7978845608f, k = 0.044715f;
      const float v = c * (x + k * x * x * x);
      return 0.5f * x * (1.0f + tanhf(v));
    }
    default: return x;
  }
}

// f'(.) given the pre-activation `pre` and the activation output `y`.
// ReLU's mask uses y > 0, which equals pre > 0 because y = max(pre, 0)
// (so ReLU layers need not keep `pre`).
__device__ __forceinline__ float act_derivative(int act, float pre, float y) {
  switch (act) {
    case VOLTA_ACT_RELU: return y > 0.0f ? 1.0f : 0.0f;
    case VOLTA_ACT_SIGMOID: return y * (1.0f - y);
    case VOLTA_ACT_TANH: return 1.0f - y * y;
    case VOLTA_ACT_LEAKY_RELU: return pre > 0.0f ? 1.0f : 0.01f;
    case VOLTA_ACT_SILU: {
      const float s = d_sigmoid(pre);
      return s * (1.0f + pre * (1.0f - s));
    }
    case VOLTA_ACT_GELU: {
      const float c = 0.7978845608f, k = 0.044715f;
      const float v = c * (pre + k * pre * pre * pre);
      const float t = tanhf(v);
      const float t2 = 1.0f - t * t;
      return 0.5f * (1.0f + t) + 0.5f * pre * t2 * c * (1.0f + 3.0f * k * pre * pre);
    }
    default: return 1.0f;
  }
}

// Activations whose derivative needs the pre-activation stored.
__host__ __device__ inline bool act_needs_pre(int act) {
  return act == VOLTA_ACT_LEAKY_RELU || act == VOLTA_ACT_SILU || act == VOLTA_ACT_GELU;
}

// x / c for a per-step constant c, as (float)((double)x * rc) with
// rc = 1.0 / (double)c: the correctly rounded fp32 quotient for every x.  For
// fp32 x and c the exact quotient is never a midpoint between two fp32
// numbers and lies at least 2^-49 (relative) from every midpoint, while the
// double product is within about 2^-52 of it, so both round to the same
// float (likewise for subnormal, zero, infinite and NaN x).  A third of the
// cost of the fp32 division sequence.
__device__ __forceinline__ float div_by_const(float x, double rc) { return (float)((double)x * rc); }

// A double every lane of the wave holds alike, moved to scalar registers so
// it costs no vector registers where it is kept (readfirstlane of each half).
__device__ __forceinline__ double wave_uniform(double x) {
  const uint64_t b = (uint64_t)__double_as_longlong(x);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)b);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// Reciprocals of Adam's two bias corrections for div_by_const (once per
// thread).  bc1 and bc2 are per-step scalars, the same in every lane.
struct AdamRcp {
  double r1, r2;
};
__device__ __forceinline__ AdamRcp adam_rcp(float bc1, float bc2) {
  return {wave_uniform(1.0 / (double)bc1), wave_uniform(1.0 / (double)bc2)};
}

// One Adam/AdamW element update (adam_update_slice,
// mlp_train_rust_codegen.rs:341-388).  `tail` marks the last (n mod 8)
// elements of a buffer, which the reference updates in its scalar loop with
// v = b2*v + ((1-b2)*g)*g instead of (1-b2)*(g*g).  mhat = m/bc1 and
// vhat = v/bc2 are the reference's fp32 quotients (div_by_const).
__device__ __forceinline__ void adam_elem(float* w, float* m, float* v, float g, bool tail, float lr,
                                          AdamRcp rc, float b1, float b2, float eps, float wd) {
  const float m1 = b1 * *m + (1.0f - b1) * g;
  const float v1 = tail ? b2 * *v + (1.0f - b2) * g * g : b2 * *v + (1.0f - b2) * (g * g);
  *m = m1;
  *v = v1;
  const float w0 = *w;
  const float mhat = div_by_const(m1, rc.r1);
  const float vhat = div_by_const(v1, rc.r2);
  const float denom = sqrtf(vhat) + eps;
  *w = w0 - lr * (mhat / denom + wd * w0);
}

// One Adagrad element update (mlp_train_rust_codegen.rs:967-985).
__device__ __forceinline__ void adagrad_elem(float* w, float* G, float g, float lr, float eps) {
  const float Gk = *G + g * g;
  *G = Gk;
  *w = *w - lr * g / (sqrtf(Gk) + eps);
}

// Once per step, after the loss: record it, raise the non-finite flag, and
// advance the Adam step counter and its bias corrections 1 - beta^t, read
// from a table the host filled with the same f32 powf the reference calls
// (mlp_train_rust_codegen.rs:803-811).  Single thread.
__device__ __forceinline__ void step_epilogue(DevScalars* sc, const float2* bc_table, int bc_len, float loss) {
  sc->loss = loss;
  if (!(fabsf(loss) <= 3.402823466e38f)) atomicOr(&sc->flags, (uint32_t)VOLTA_STATUS_NONFINITE_LOSS);
  if (bc_table) {
    const uint32_t t = sc->t + 1u;
    sc->t = t;
    const float2 bc = bc_table[t < (uint32_t)bc_len ? t : (uint32_t)(bc_len - 1)];
    sc->bc1 = bc.x;
    sc->bc2 = bc.y;
  }
}

// step_epilogue split in two so its loads (step counter, then the table
// entry) overlap the kernel's main work: step_prefetch at kernel start,
// step_finish at the end (same stores as step_epilogue).  Single thread;
// nothing else may change the counter in between.
struct StepNext {
  uint32_t t;
  float2 bc;
};

__device__ __forceinline__ StepNext step_prefetch(const DevScalars* sc, const float2* bc_table, int bc_len) {
  StepNext s{};
  if (bc_table) {
    s.t = sc->t + 1u;
    s.bc = bc_table[s.t < (uint32_t)bc_len ? s.t : (uint32_t)(bc_len - 1)];
  }
  return s;
}

__device__ __forceinline__ void step_finish(DevScalars* sc, const StepNext& s, bool has_table, float loss) {
  sc->loss = loss;
  if (!(fabsf(loss) <= 3.402823466e38f)) atomicOr(&sc->flags, (uint32_t)VOLTA_STATUS_NONFINITE_LOSS);
  if (has_table) {
    sc->t = s.t;
    sc->bc1 = s.bc.x;
    sc->bc2 = s.bc.y;
  }
}

// Fixed-order wavefront sum (butterfly over 64 lanes).  Every lane ends with
// the same value and the association order depends only on lane indices,
// so results are bit-identical run to run.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

}  // namespace volta
