/*
 * The runtime Backend of the Volta IR on one GPU: the optimizer update of
 * Backend::apply_gradients (below) and graph execution of
 * Backend::compile / execute_value / execute_terminal for MLP graphs (at the
 * end of this file).
 *
 * Runtime optimizer: the update that a HIP backend's
 * Backend::apply_gradients runs over the trained parameter tensors.  The
 * reference's trait method (src/engine/ir/backend.rs:28-40) calls
 * optimizer::apply_gradients (src/engine/ir/optimizer.rs:108-178) on host
 * tensors keyed by ValueId; this interface keeps the tensors and the
 * OptimizerState (optimizer.rs:80-94) on the device, keyed by index, and runs
 * every tensor's update in one multi-tensor launch.
 *
 * Implemented by libvolta_hip.so (device pointers) and by the CPU oracle
 * liboracle_volta.so (host pointers; test infrastructure), so one harness can
 * drive either.
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

/* ------------------------------------------------------------------------
 * Graph execution: Backend::compile / execute_value / execute_terminal
 * (backend.rs:24-69) for the runtime's MLP graphs, reached as
 * compile_plan_for_backend (runtime.rs:148-181) reaches them: compile through
 * a process-wide plan cache (compile_or_get_cached, plan_cache.rs:8-51), then
 * execute.
 *
 * The graph crosses the boundary as flat tables: the nodes of Graph in graph
 * order (each the ValueId it defines and its operand ValueIds), the
 * ExecutionPlan's schedule as node indices, and one binding per distinct
 * Input/Parameter name with the shape bound to it (Graph::bind_input_shape /
 * bind_parameter_shape).  What the HIP backend lowers is the graph
 * lower_model_to_graph builds (lowering.rs:87-140) and its Gemm form
 * (train_api.rs:316-345): one chain from a bound [rows x r] tensor through
 * layers of MatMul by a bound [r x c] weight, Add of a bound [1 x c] bias
 * (either operand order) or Gemm{alpha = 1, beta 0 or 1}, an optional Relu,
 * Sigmoid or Gelu, and at the end an optional row Softmax, with Output nodes
 * anywhere.  Each layer runs as one MFMA GEMM launch whose epilogue adds the
 * bias and applies the activation (the compile-train forward kernels), the
 * Softmax as one more launch.  Any other op, a value consumed off the chain,
 * or a shape mismatch is a compile error (the message names the node): the
 * caller keeps such graphs on the reference's CPU backend.
 *
 * libvolta_hip: binding pointers and the output are device pointers and
 * execution is synchronous on a stream of the compiled program.  The CPU
 * oracle (test infrastructure) implements the same calls on host pointers by
 * interpreting every scheduled node as the reference's interpreter does.
 * ------------------------------------------------------------------------ */

/* Op kinds of Op (op.rs:51-...) that an MLP graph is made of; every other op
 * is passed as VOLTA_RT_OP_OTHER.  ElementwiseChain{ops: [Relu]} and the
 * like (one op) are passed as that op. */
enum volta_rt_op {
  VOLTA_RT_OP_OTHER = 0,
  VOLTA_RT_OP_INPUT = 1,     /* Input(name): binding */
  VOLTA_RT_OP_PARAMETER = 2, /* Parameter(name): binding */
  VOLTA_RT_OP_OUTPUT = 3,    /* Output(in0) */
  VOLTA_RT_OP_MATMUL = 4,    /* MatMul(in0, in1) */
  VOLTA_RT_OP_ADD = 5,       /* Add(in0, in1) */
  VOLTA_RT_OP_GEMM = 6,      /* Gemm{lhs: in0, rhs: in1, bias: in2 (-1 = None), alpha, beta} */
  VOLTA_RT_OP_RELU = 7,      /* Relu(in0) */
  VOLTA_RT_OP_SIGMOID = 8,   /* Sigmoid(in0) */
  VOLTA_RT_OP_GELU = 9,      /* Gelu(in0): tanh approximation */
  VOLTA_RT_OP_SOFTMAX = 10   /* Softmax(in0): over each row of a 2-D tensor */
};

typedef struct volta_rt_node {
  int32_t op;      /* enum volta_rt_op */
  int32_t output;  /* ValueId the node defines (node.output) */
  int32_t in0, in1, in2; /* operand ValueIds, -1 where absent */
  int32_t binding; /* Input / Parameter: index into the binding table */
  float alpha, beta; /* Gemm */
} volta_rt_node;

typedef struct volta_rt_binding {
  int64_t rows, cols; /* bound shape; a 1-D [c] shape is passed as rows = 1 */
} volta_rt_binding;

typedef struct volta_rt_graph {
  int32_t n_nodes;
  const volta_rt_node* nodes;   /* Graph::nodes, graph order */
  int32_t n_ordered;
  const int32_t* ordered_nodes; /* ExecutionPlan::schedule.ordered_nodes (node indices) */
  int32_t n_bindings;
  const volta_rt_binding* bindings;
  uint64_t graph_fingerprint;    /* ExecutionPlan::graph_fingerprint */
  uint64_t shape_signature_hash; /* ExecutionPlan::shape_signature_hash */
  int64_t peak_bytes;            /* ExecutionPlan::allocation.peak_bytes */
} volta_rt_graph;

/* CompiledProgram (backend.rs:12-17). */
typedef struct volta_rt_compiled {
  int64_t schedule_len;
  int64_t peak_bytes;
  uint64_t fingerprint;
} volta_rt_compiled;

/* compile_or_get_cached (plan_cache.rs:21-51) with this backend: the cache
 * key is (backend Hip, determinism 0 Strict / 1 Balanced / 2 Fast,
 * graph_fingerprint, shape_signature_hash).  A hit whose graph differs from
 * the cached one (the same fingerprints for other contents) is compiled
 * again and replaces the entry.  Returns 0 and fills *out, or -1 with the
 * message in volta_rt_last_error.  Host work only: device state is created by
 * the first execution on each device. */
int32_t volta_rt_compile(const volta_rt_graph* g, int32_t determinism, volta_rt_compiled* out);

/* Backend::execute_value (backend.rs:55-69): the value `target` (a ValueId)
 * of graph g with its bindings bound to bindings[i] (one pointer per binding,
 * rows x cols floats, row-major), written to out ([rows x cols], capacity
 * out_capacity floats) and its shape to out_shape[0..1].  Compiles through the
 * cache first.  Returns 0, or -1 with the message in volta_rt_last_error.
 * Calls on one compiled program are serialised. */
int32_t volta_rt_execute_value(const volta_rt_graph* g, int32_t determinism, int32_t target,
                               const float* const* bindings, float* out, int64_t out_capacity, int64_t* out_shape);

/* Backend::execute_terminal (backend.rs:42-53): execute_value of the terminal
 * value -- the operand of the last Output node in graph order, else the
 * value the last node defines (interpreter.rs:281-288). */
int32_t volta_rt_execute_terminal(const volta_rt_graph* g, int32_t determinism, const float* const* bindings,
                                  float* out, int64_t out_capacity, int64_t* out_shape);

/* clear_plan_cache (plan_cache.rs:53-59). */
void volta_rt_clear_plan_cache(void);

/* Backend::compile calls made through the cache since the process started
 * (what the reference's CountingCompileBackend counts, train.rs:1296-1316). */
int64_t volta_rt_compile_count(void);

#ifdef __cplusplus
}
#endif

#endif /* VOLTA_BACKEND_H */
