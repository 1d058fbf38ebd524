// Runtime optimizer of the Volta IR on the GPU (include/volta_backend.h):
// optimizer::apply_gradients (src/engine/ir/optimizer.rs:108-658) over a
// fixed list of device-resident parameter tensors, all tensors in one
// multi-tensor launch.
//
// Layout: the tensors are cut into chunks of kRtChunk elements, one
// workgroup per chunk (a host-built table maps workgroup -> tensor, chunk);
// thread t of a chunk updates elements t, t+256, t+512, t+768, so every load
// and store of a wave is one contiguous 256-byte run.  Every load is
// unconditional (index clamped to the tensor), stores are guarded.  The
// optimizer state of each kind (Adam m/v, RMSprop v/buf, Adagrad acc, LARS
// velocity) is one device arena over all tensors, allocated zero-filled the
// first time a configuration needs it.
//
// Arithmetic: the reference's f32 expressions in its order (built with
// -ffp-contract=off, IEEE division and square root), so every update equals
// the CPU oracle's bit for bit; the step counter and the Adam/AdamW bias
// corrections 1 - powi(beta, step) are host values, passed as arguments.
// LARS norms are a fixed-order tree (per-thread partials, a block tree, then
// one workgroup per tensor over the block partials): deterministic, and equal
// to the reference's sequential sums up to rounding.
//
// HBM-bound: bytes per element and step (reads + writes): SGD 12, Adagrad 20,
// RMSprop 20 (28 with momentum), Adam/AdamW 28, LARS 20 (+8 for the norms).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/volta_backend.h"

namespace volta {
namespace {

constexpr int kRtThreads = 256;
constexpr int kRtPer = 4;
constexpr int kRtChunk = kRtThreads * kRtPer;

thread_local std::string g_rt_err;

struct RtTensor {
  float* p;
  const float* g;  // null: no gradient this step (skipped)
  float* s0;       // first state buffer of the kind (or null)
  float* s1;       // second state buffer (Adam v, RMSprop momentum buffer)
  int64_t count;
};

struct RtArgs {
  const RtTensor* tensors;
  const int2* blocks;  // workgroup -> (tensor, chunk)
  float lr, b1, b2, om1, om2, bias1, bias2, eps, wd, alpha, om_alpha, mo, tc;
  const float2* norms;  // LARS: (|p|, |g|) per tensor
};

// The update of one element, in the reference's expression order.
template <int KIND, bool MOM>
__device__ __forceinline__ void rt_elem(const RtArgs& a, float local_lr, float& p, float g, float& s0, float& s1) {
  if constexpr (KIND == VOLTA_RT_SGD) {
    p = p - a.lr * g;  // :224
  } else if constexpr (KIND == VOLTA_RT_ADAM || KIND == VOLTA_RT_ADAMW) {
    s0 = a.b1 * s0 + a.om1 * g;        // :333
    s1 = a.b2 * s1 + a.om2 * (g * g);  // :334
    const float mh = s0 / a.bias1;
    const float vh = s1 / a.bias2;
    if constexpr (KIND == VOLTA_RT_ADAMW)
      p = p - a.lr * (mh / (sqrtf(vh) + a.eps) + a.wd * p);  // :438
    else
      p = p - a.lr * (mh / (sqrtf(vh) + a.eps));  // :338
  } else if constexpr (KIND == VOLTA_RT_RMSPROP) {
    const float gwd = g + a.wd * p;
    s0 = a.alpha * s0 + a.om_alpha * gwd * gwd;  // :524, :535
    if constexpr (MOM) {
      s1 = a.mo * s1 + a.lr * gwd / (sqrtf(s0) + a.eps);  // :525
      p = p - s1;
    } else {
      p = p - a.lr * gwd / (sqrtf(s0) + a.eps);  // :536
    }
  } else if constexpr (KIND == VOLTA_RT_ADAGRAD) {
    const float gwd = g + a.wd * p;  // :597-599
    s0 = s0 + gwd * gwd;
    p = p - a.lr * gwd / (sqrtf(s0) + a.eps);
  } else {  // LARS :649-652
    const float upd = local_lr * (g + a.wd * p);
    s0 = a.mo * s0 + upd;
    p = p - s0;
  }
}

template <int KIND, bool MOM>
__global__ void __launch_bounds__(kRtThreads) rt_apply_kernel(RtArgs a) {
  const int2 bt = a.blocks[blockIdx.x];
  const RtTensor t = a.tensors[bt.x];
  if (!t.g) return;  // whole workgroup
  constexpr bool kS0 = KIND != VOLTA_RT_SGD;
  constexpr bool kS1 = KIND == VOLTA_RT_ADAM || KIND == VOLTA_RT_ADAMW || (KIND == VOLTA_RT_RMSPROP && MOM);
  float local_lr = a.lr;
  if constexpr (KIND == VOLTA_RT_LARS) {
    const float2 nm = a.norms[bt.x];
    // :631-635: lr * trust * |p| / (|g| + wd * |p| + eps) when both norms are positive
    if (nm.x > 0.0f && nm.y > 0.0f) local_lr = a.lr * a.tc * nm.x / (nm.y + a.wd * nm.x + a.eps);
  }
  const int64_t base = (int64_t)bt.y * kRtChunk + threadIdx.x;
  const int64_t last = t.count - 1;
  float p[kRtPer], g[kRtPer], s0[kRtPer], s1[kRtPer];
#pragma unroll
  for (int j = 0; j < kRtPer; ++j) {
    const int64_t i = min(base + (int64_t)j * kRtThreads, last);
    p[j] = t.p[i];
    g[j] = t.g[i];
    s0[j] = kS0 ? t.s0[i] : 0.0f;
    s1[j] = kS1 ? t.s1[i] : 0.0f;
  }
#pragma unroll
  for (int j = 0; j < kRtPer; ++j) rt_elem<KIND, MOM>(a, local_lr, p[j], g[j], s0[j], s1[j]);
#pragma unroll
  for (int j = 0; j < kRtPer; ++j) {
    const int64_t i = base + (int64_t)j * kRtThreads;
    if (i <= last) {
      t.p[i] = p[j];
      if (kS0) t.s0[i] = s0[j];
      if (kS1) t.s1[i] = s1[j];
    }
  }
}

// Fixed-order sum of the workgroup's values (pairwise tree in LDS).
__device__ __forceinline__ float2 block_sum2(float2 v, float2* sh) {
  sh[threadIdx.x] = v;
  __syncthreads();
#pragma unroll
  for (int s = kRtThreads / 2; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) {
      sh[threadIdx.x].x = sh[threadIdx.x].x + sh[threadIdx.x + s].x;
      sh[threadIdx.x].y = sh[threadIdx.x].y + sh[threadIdx.x + s].y;
    }
    __syncthreads();
  }
  return sh[0];
}

// LARS, stage 1: (sum p^2, sum g^2) of each chunk of a tensor with a gradient.
__global__ void __launch_bounds__(kRtThreads) rt_norm_partials(RtArgs a, float2* partials) {
  __shared__ float2 sh[kRtThreads];
  const int2 bt = a.blocks[blockIdx.x];
  const RtTensor t = a.tensors[bt.x];
  if (!t.g) return;
  const int64_t base = (int64_t)bt.y * kRtChunk + threadIdx.x;
  const int64_t last = t.count - 1;
  float p[kRtPer], g[kRtPer];
#pragma unroll
  for (int j = 0; j < kRtPer; ++j) {
    const int64_t i = min(base + (int64_t)j * kRtThreads, last);
    p[j] = t.p[i];
    g[j] = t.g[i];
  }
  float2 s = make_float2(0.0f, 0.0f);
#pragma unroll
  for (int j = 0; j < kRtPer; ++j) {
    const bool in = base + (int64_t)j * kRtThreads <= last;
    s.x = in ? s.x + p[j] * p[j] : s.x;
    s.y = in ? s.y + g[j] * g[j] : s.y;
  }
  s = block_sum2(s, sh);
  if (threadIdx.x == 0) partials[blockIdx.x] = s;
}

// LARS, stage 2: one workgroup per tensor adds its chunks' partials (thread
// t takes chunks t, t+256, ... in order, then the tree) and takes the roots.
__global__ void __launch_bounds__(kRtThreads) rt_norm_finish(RtArgs a, const int* first_block, const float2* partials,
                                                              float2* norms) {
  __shared__ float2 sh[kRtThreads];
  const int ti = blockIdx.x;
  if (!a.tensors[ti].g) return;
  const int b0 = first_block[ti], b1 = first_block[ti + 1];
  float2 s = make_float2(0.0f, 0.0f);
  for (int b = b0 + (int)threadIdx.x; b < b1; b += kRtThreads) {
    const float2 v = partials[b];
    s.x = s.x + v.x;
    s.y = s.y + v.y;
  }
  s = block_sum2(s, sh);
  if (threadIdx.x == 0) norms[ti] = make_float2(sqrtf(s.x), sqrtf(s.y));
}

// Rust's f32::powi: compiler-builtins' __powisf2, square-and-multiply in f32.
float powi_f32(float a, int32_t b) {
  const bool recip = b < 0;
  uint32_t e = b < 0 ? (uint32_t)(-(int64_t)b) : (uint32_t)b;
  float r = 1.0f;
  for (;;) {
    if (e & 1u) r = r * a;
    e >>= 1;
    if (e == 0) break;
    a = a * a;
  }
  return recip ? 1.0f / r : r;
}

// Rust Display of an f32 (shortest round-trip decimal; NaN, inf).
std::string show(float x) {
  if (std::isnan(x)) return "NaN";
  if (std::isinf(x)) return x > 0 ? "inf" : "-inf";
  char buf[64];
  for (int prec = 1; prec <= 9; ++prec) {
    std::snprintf(buf, sizeof buf, "%.*g", prec, (double)x);
    if (std::strtof(buf, nullptr) == x) break;
  }
  return buf;
}

bool pos(float x) { return std::isfinite(x) && x > 0.0f; }
bool nonneg(float x) { return std::isfinite(x) && x >= 0.0f; }
bool unit(float x) { return x >= 0.0f && x < 1.0f; }

}  // namespace
}  // namespace volta

using namespace volta;

struct VoltaRtOptimizer {
  int32_t n = 0;
  std::vector<int64_t> counts;
  std::vector<int64_t> off;  // element offset of each tensor in a state arena (64-float aligned)
  int64_t total = 0;
  int64_t step = 0;
  hipStream_t stream = nullptr;
  int nblocks = 0;
  int2* blocks = nullptr;       // device: workgroup -> (tensor, chunk)
  int* first_block = nullptr;   // device: n + 1 workgroup offsets
  RtTensor* tensors = nullptr;  // device descriptor table
  RtTensor* staging = nullptr;  // pinned host copy of the table
  float2* partials = nullptr;   // LARS
  float2* norms = nullptr;
  float* state[6] = {};
  std::vector<char> created[6];
};

namespace {

int fail(const std::string& m) {
  g_rt_err = m;
  return -1;
}

bool ok(hipError_t e, const char* what) {
  if (e == hipSuccess) return true;
  g_rt_err = std::string(what) + ": " + hipGetErrorString(e);
  return false;
}

void release(VoltaRtOptimizer* h) {
  if (!h) return;
  for (float* s : h->state)
    if (s) (void)hipFree(s);
  if (h->blocks) (void)hipFree(h->blocks);
  if (h->first_block) (void)hipFree(h->first_block);
  if (h->tensors) (void)hipFree(h->tensors);
  if (h->partials) (void)hipFree(h->partials);
  if (h->norms) (void)hipFree(h->norms);
  if (h->staging) (void)hipHostFree(h->staging);
  if (h->stream) (void)hipStreamDestroy(h->stream);
  delete h;
}

// State arena `which`, zero-filled on first use.
bool ensure_state(VoltaRtOptimizer* h, int which) {
  if (h->state[which]) return true;
  const size_t bytes = (size_t)h->total * sizeof(float);
  if (!ok(hipMalloc((void**)&h->state[which], bytes), "volta_rt: state allocation")) return false;
  return ok(hipMemsetAsync(h->state[which], 0, bytes, h->stream), "volta_rt: state clear");
}

// Configuration checks in the reference's order (optimizer.rs:198-620); on
// success fills the kernel arguments.
int validate(VoltaRtOptimizer* h, const volta_rt_config& c, RtArgs& a) {
  const float lr = c.lr;
  a.lr = lr;
  switch (c.kind) {
    case VOLTA_RT_SGD:
      if (!pos(lr)) return fail("SGD learning rate must be a finite positive number, got " + show(lr));
      return 0;
    case VOLTA_RT_ADAM:
    case VOLTA_RT_ADAMW: {
      const std::string nm = c.kind == VOLTA_RT_ADAMW ? "AdamW" : "Adam";
      if (!pos(lr)) return fail(nm + " learning rate must be a finite positive number, got " + show(lr));
      if (!unit(c.beta1)) return fail(nm + " beta1 must be in [0, 1), got " + show(c.beta1));
      if (!unit(c.beta2)) return fail(nm + " beta2 must be in [0, 1), got " + show(c.beta2));
      if (!pos(c.epsilon)) return fail(nm + " epsilon must be a finite positive number, got " + show(c.epsilon));
      if (c.kind == VOLTA_RT_ADAMW && !nonneg(c.weight_decay))
        return fail("AdamW weight_decay must be a finite non-negative number, got " + show(c.weight_decay));
      if (h->step > INT32_MAX) return fail("Optimizer step overflow for " + nm + " bias correction");
      a.bias1 = 1.0f - powi_f32(c.beta1, (int32_t)h->step);
      a.bias2 = 1.0f - powi_f32(c.beta2, (int32_t)h->step);
      if (a.bias1 <= 0.0f || a.bias2 <= 0.0f)
        return fail(nm + " bias correction underflowed (bias1=" + show(a.bias1) + ", bias2=" + show(a.bias2) +
                    "); step=" + std::to_string(h->step));
      a.b1 = c.beta1;
      a.b2 = c.beta2;
      a.om1 = 1.0f - c.beta1;
      a.om2 = 1.0f - c.beta2;
      a.eps = c.epsilon;
      a.wd = c.weight_decay;
      return 0;
    }
    case VOLTA_RT_RMSPROP:
      if (!pos(lr)) return fail("RMSprop learning rate must be a finite positive number, got " + show(lr));
      if (!unit(c.alpha)) return fail("RMSprop alpha must be in [0, 1), got " + show(c.alpha));
      if (!pos(c.epsilon)) return fail("RMSprop epsilon must be a finite positive number, got " + show(c.epsilon));
      if (!nonneg(c.weight_decay))
        return fail("RMSprop weight_decay must be a finite non-negative number, got " + show(c.weight_decay));
      if (!nonneg(c.momentum))
        return fail("RMSprop momentum must be a finite non-negative number, got " + show(c.momentum));
      a.alpha = c.alpha;
      a.om_alpha = 1.0f - c.alpha;
      a.eps = c.epsilon;
      a.wd = c.weight_decay;
      a.mo = c.momentum;
      return 0;
    case VOLTA_RT_ADAGRAD:
      if (!pos(lr)) return fail("Adagrad learning rate must be a finite positive number, got " + show(lr));
      if (!pos(c.epsilon)) return fail("Adagrad epsilon must be a finite positive number, got " + show(c.epsilon));
      if (!nonneg(c.weight_decay))
        return fail("Adagrad weight_decay must be a finite non-negative number, got " + show(c.weight_decay));
      a.eps = c.epsilon;
      a.wd = c.weight_decay;
      return 0;
    case VOLTA_RT_LARS:
      if (!pos(lr)) return fail("LARS learning rate must be a finite positive number, got " + show(lr));
      a.mo = c.momentum;
      a.wd = c.weight_decay;
      a.tc = c.trust_coeff;
      a.eps = c.epsilon;
      return 0;
    default:
      return fail("volta_rt_apply_gradients: unknown optimizer kind");
  }
}

template <int KIND, bool MOM>
void launch_apply(VoltaRtOptimizer* h, const RtArgs& a) {
  hipLaunchKernelGGL((rt_apply_kernel<KIND, MOM>), dim3(h->nblocks), dim3(kRtThreads), 0, h->stream, a);
}

}  // namespace

namespace volta {
// volta_rt_last_error's text for the graph-execution calls (rt_graph.hip).
void rt_set_error(const std::string& m) { g_rt_err = m; }
}  // namespace volta

extern "C" {

VoltaRtOptimizer* volta_rt_optimizer_new(int32_t n, const int64_t* counts) {
  if (n < 1 || !counts) {
    g_rt_err = "volta_rt_optimizer_new: need n >= 1 and counts";
    return nullptr;
  }
  auto* h = new VoltaRtOptimizer;
  h->n = n;
  std::vector<int2> blocks;
  std::vector<int> first(n + 1, 0);
  for (int i = 0; i < n; ++i) {
    if (counts[i] < 1) {
      release(h);
      g_rt_err = "volta_rt_optimizer_new: every tensor needs at least one element";
      return nullptr;
    }
    h->counts.push_back(counts[i]);
    h->off.push_back(h->total);
    h->total += (counts[i] + 63) / 64 * 64;
    first[i] = (int)blocks.size();
    const int64_t chunks = (counts[i] + kRtChunk - 1) / kRtChunk;
    if ((int64_t)blocks.size() + chunks > INT32_MAX / 2) {
      release(h);
      g_rt_err = "volta_rt_optimizer_new: too many elements";
      return nullptr;
    }
    for (int64_t c = 0; c < chunks; ++c) blocks.push_back(make_int2(i, (int)c));
  }
  first[n] = (int)blocks.size();
  h->nblocks = (int)blocks.size();
  for (auto& c : h->created) c.assign(n, 0);
  if (!ok(hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking), "volta_rt: stream") ||
      !ok(hipMalloc((void**)&h->blocks, blocks.size() * sizeof(int2)), "volta_rt: allocation") ||
      !ok(hipMalloc((void**)&h->first_block, first.size() * sizeof(int)), "volta_rt: allocation") ||
      !ok(hipMalloc((void**)&h->tensors, (size_t)n * sizeof(RtTensor)), "volta_rt: allocation") ||
      !ok(hipHostMalloc((void**)&h->staging, (size_t)n * sizeof(RtTensor)), "volta_rt: pinned allocation") ||
      !ok(hipMemcpy(h->blocks, blocks.data(), blocks.size() * sizeof(int2), hipMemcpyHostToDevice),
          "volta_rt: upload") ||
      !ok(hipMemcpy(h->first_block, first.data(), first.size() * sizeof(int), hipMemcpyHostToDevice),
          "volta_rt: upload")) {
    release(h);
    return nullptr;
  }
  return h;
}

void volta_rt_optimizer_free(VoltaRtOptimizer* h) {
  if (h && h->stream) (void)hipStreamSynchronize(h->stream);
  release(h);
}

int64_t volta_rt_step(const VoltaRtOptimizer* h) { return h ? h->step : -1; }

const char* volta_rt_last_error(void) { return g_rt_err.c_str(); }

int32_t volta_rt_apply_gradients(VoltaRtOptimizer* h, const volta_rt_config* cfg, float* const* params,
                                 const float* const* grads) {
  if (!h || !cfg || !params || !grads) return fail("volta_rt_apply_gradients: bad arguments");
  h->step = h->step + 1;  // before validation, as optimizer.rs:114
  RtArgs a{};
  if (validate(h, *cfg, a) != 0) return -1;
  for (int i = 0; i < h->n; ++i)
    if (grads[i] && !params[i]) return fail("volta_rt_apply_gradients: a tensor with a gradient has no parameter");
  const int kind = cfg->kind;
  const bool mom = kind == VOLTA_RT_RMSPROP && cfg->momentum > 0.0f;
  int b0 = -1, b1 = -1;  // state arenas this configuration uses
  switch (kind) {
    case VOLTA_RT_ADAM:
    case VOLTA_RT_ADAMW: b0 = VOLTA_RT_ADAM_M; b1 = VOLTA_RT_ADAM_V; break;
    case VOLTA_RT_RMSPROP: b0 = VOLTA_RT_RMS_V; b1 = mom ? VOLTA_RT_RMS_BUF : -1; break;
    case VOLTA_RT_ADAGRAD: b0 = VOLTA_RT_ADAGRAD_ACC; break;
    case VOLTA_RT_LARS: b0 = VOLTA_RT_LARS_VEL; break;
    default: break;
  }
  if ((b0 >= 0 && !ensure_state(h, b0)) || (b1 >= 0 && !ensure_state(h, b1))) return -1;
  for (int i = 0; i < h->n; ++i) {
    RtTensor& t = h->staging[i];
    t.p = params[i];
    t.g = grads[i];
    t.s0 = b0 >= 0 ? h->state[b0] + h->off[i] : nullptr;
    t.s1 = b1 >= 0 ? h->state[b1] + h->off[i] : nullptr;
    t.count = h->counts[i];
  }
  if (!ok(hipMemcpyAsync(h->tensors, h->staging, (size_t)h->n * sizeof(RtTensor), hipMemcpyHostToDevice, h->stream),
          "volta_rt: descriptor upload"))
    return -1;
  a.tensors = h->tensors;
  a.blocks = h->blocks;
  if (kind == VOLTA_RT_LARS) {
    if (!h->partials && (!ok(hipMalloc((void**)&h->partials, (size_t)h->nblocks * sizeof(float2)), "volta_rt: LARS") ||
                         !ok(hipMalloc((void**)&h->norms, (size_t)h->n * sizeof(float2)), "volta_rt: LARS")))
      return -1;
    hipLaunchKernelGGL(rt_norm_partials, dim3(h->nblocks), dim3(kRtThreads), 0, h->stream, a, h->partials);
    hipLaunchKernelGGL(rt_norm_finish, dim3(h->n), dim3(kRtThreads), 0, h->stream, a, h->first_block, h->partials,
                       h->norms);
    a.norms = h->norms;
  }
  switch (kind) {
    case VOLTA_RT_SGD: launch_apply<VOLTA_RT_SGD, false>(h, a); break;
    case VOLTA_RT_ADAM: launch_apply<VOLTA_RT_ADAM, false>(h, a); break;
    case VOLTA_RT_ADAMW: launch_apply<VOLTA_RT_ADAMW, false>(h, a); break;
    case VOLTA_RT_RMSPROP:
      if (mom) launch_apply<VOLTA_RT_RMSPROP, true>(h, a);
      else launch_apply<VOLTA_RT_RMSPROP, false>(h, a);
      break;
    case VOLTA_RT_ADAGRAD: launch_apply<VOLTA_RT_ADAGRAD, false>(h, a); break;
    default: launch_apply<VOLTA_RT_LARS, false>(h, a); break;
  }
  if (!ok(hipGetLastError(), "volta_rt: launch") || !ok(hipStreamSynchronize(h->stream), "volta_rt: apply"))
    return -1;
  for (int i = 0; i < h->n; ++i) {
    if (!grads[i]) continue;
    if (b0 >= 0) h->created[b0][i] = 1;
    if (b1 >= 0) h->created[b1][i] = 1;
  }
  return 0;
}

int32_t volta_rt_get_state(const VoltaRtOptimizer* h, int32_t which, int32_t i, float* out) {
  if (!h || which < 0 || which > 5 || i < 0 || i >= h->n || !out) return fail("volta_rt_get_state: bad arguments");
  if (!h->created[which][i] || !h->state[which]) return fail("volta_rt_get_state: no such state entry");
  if (!ok(hipMemcpy(out, h->state[which] + h->off[i], (size_t)h->counts[i] * sizeof(float), hipMemcpyDeviceToHost),
          "volta_rt_get_state"))
    return -1;
  return 0;
}

void volta_rt_capabilities_get(volta_rt_capabilities* out) {
  // What a HIP backend declares (backend_capabilities.rs:44-58), beside the
  // reference's CudaBackend (backend.rs:117-131): a GPU backend for training,
  // with Adam (which the CUDA backend lacks); every reduction of this library
  // has a fixed order, so Strict is the default and Balanced/Fast requests
  // are served by the same strict kernels.
  if (!out) return;
  std::memset(out, 0, sizeof *out);
  out->backend = 2;        // Hip
  out->device_class = 1;   // Gpu
  out->vendor = 2;         // Amd
  out->maturity = 0;       // Experimental, as the reference marks its GPU backend
  out->supports_inference = 1;
  out->supports_training = 1;
  out->supports_runtime_execution = 1;
  out->supports_gradient_updates = 1;
  out->supports_adam = 1;
  out->supports_strict_determinism = 1;
  out->supports_balanced_determinism = 1;
  out->supports_fast_determinism = 1;
  out->default_determinism = 0;  // Strict
}

}  // extern "C"
