/*
 * Runtime optimizer of the Volta IR on one GPU: the update that a HIP
 * backend's Backend::apply_gradients runs over the trained parameter
 * tensors.  The reference's trait method (src/engine/ir/backend.rs:28-40)
 * calls optimizer::apply_gradients (src/engine/ir/optimizer.rs:108-178) on
 * host tensors keyed by ValueId; this interface keeps the tensors and the
 * OptimizerState (optimizer.rs:80-94) on the device, keyed by index, and runs
 * every tensor's update in one multi-tensor launch.
 *
 * Implemented by libvolta_hip.so (device pointers) and by the CPU oracle
 * liboracle_volta.so (host pointers; test infrastructure), so one harness can
 * drive either.  The Rust binding a maintainer would add is in
 * INTEGRATION.md.
 */
#ifndef VOLTA_BACKEND_H
#define VOLTA_BACKEND_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* OptimizerConfig variants (optimizer.rs:37-79). */
enum volta_rt_kind {
  VOLTA_RT_SGD = 0,
  VOLTA_RT_ADAM = 1,
  VOLTA_RT_ADAMW = 2,
  VOLTA_RT_RMSPROP = 3,
  VOLTA_RT_ADAGRAD = 4,
  VOLTA_RT_LARS = 5
};

/* One OptimizerConfig; fields its variant does not have are ignored.
 * Sgd{lr}; Adam{lr,beta1,beta2,epsilon}; AdamW{..,weight_decay};
 * RmsProp{lr,alpha,epsilon,weight_decay,momentum}; Adagrad{lr,epsilon,
 * weight_decay}; Lars{lr,momentum,weight_decay,trust_coeff,epsilon}. */
typedef struct volta_rt_config {
  int32_t kind; /* enum volta_rt_kind */
  float lr;
  float beta1;
  float beta2;
  float epsilon;
  float weight_decay;
  float alpha;
  float momentum;
  float trust_coeff;
} volta_rt_config;

/* OptimizerState buffers (optimizer.rs:83-93). */
enum volta_rt_buffer {
  VOLTA_RT_ADAM_M = 0,
  VOLTA_RT_ADAM_V = 1,
  VOLTA_RT_RMS_V = 2,
  VOLTA_RT_RMS_BUF = 3,
  VOLTA_RT_ADAGRAD_ACC = 4,
  VOLTA_RT_LARS_VEL = 5
};

typedef struct VoltaRtOptimizer VoltaRtOptimizer;

/* OptimizerState::default() for n parameter tensors of counts[i] elements
 * (counts[i] >= 1).  State buffers are created zero-filled the first time an
 * update needs them for a tensor, as the reference's entry().or_insert does.
 * Returns NULL on bad arguments or allocation failure (message in
 * volta_rt_last_error). */
VoltaRtOptimizer* volta_rt_optimizer_new(int32_t n, const int64_t* counts);

/* Releases the state.  NULL is ignored. */
void volta_rt_optimizer_free(VoltaRtOptimizer* h);

/* apply_gradients (optimizer.rs:108-178): the step counter advances first,
 * then the configuration is validated as the reference validates it, then
 * params[i] (counts[i] floats) is updated in place from grads[i] for every i
 * whose grads[i] is not NULL -- the reference skips parameters without a
 * gradient.  libvolta_hip: device pointers, one launch for all tensors (two
 * for LARS, whose per-tensor norms come first), synchronous.  Returns 0, or
 * -1 with the reference's message in volta_rt_last_error (the step counter
 * has still advanced, as in the reference). */
int32_t volta_rt_apply_gradients(VoltaRtOptimizer* h, const volta_rt_config* cfg, float* const* params,
                                 const float* const* grads);

/* OptimizerState::step. */
int64_t volta_rt_step(const VoltaRtOptimizer* h);

/* Copies state buffer `which` (enum volta_rt_buffer) of tensor i to host
 * memory (counts[i] floats).  Returns -1 when the reference would have no
 * such entry (the buffer was never created for that tensor). */
int32_t volta_rt_get_state(const VoltaRtOptimizer* h, int32_t which, int32_t i, float* out);

/* Message of the last failing call on this thread ("" if none). */
const char* volta_rt_last_error(void);

/* BackendCapabilities (backend_capabilities.rs:44-58) of this backend.
 * Enumerations as integers: backend (0 Cpu, 1 Cuda, 2 Hip -- a value the
 * reference's BackendKind would gain), device_class (0 Cpu, 1 Gpu), vendor
 * (0 GenericCpu, 1 Nvidia, 2 Amd), maturity (0 Experimental, 1 Validated),
 * default_determinism (0 Strict, 1 Balanced, 2 Fast). */
typedef struct volta_rt_capabilities {
  int32_t backend;
  int32_t device_class;
  int32_t vendor;
  int32_t maturity;
  uint8_t supports_inference;
  uint8_t supports_training;
  uint8_t supports_runtime_execution;
  uint8_t supports_gradient_updates;
  uint8_t supports_adam;
  uint8_t supports_strict_determinism;
  uint8_t supports_balanced_determinism;
  uint8_t supports_fast_determinism;
  int32_t default_determinism;
} volta_rt_capabilities;

void volta_rt_capabilities_get(volta_rt_capabilities* out);

#ifdef __cplusplus
}
#endif

#endif /* VOLTA_BACKEND_H */
