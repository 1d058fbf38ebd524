/*
 * volta_train.h -- C ABI of the MI355X (gfx950) compile-train MLP step.
 *
 * The first six entry points are the exported symbols of the training
 * library that Volta's `compile-train` generates; argument order, types and
 * meaning are kept so a caller of that library can link this one instead:
 *
 *   Rust generator: /root/reference/src/engine/ir/codegen/mlp_train_rust_codegen.rs
 *     volta_train_init        :640-667
 *     volta_train_set_params  :669-675
 *     volta_train_get_params  :677-684
 *     volta_train_loss        :686
 *     volta_train_free        :688-696
 *     volta_train_step        :698-994
 *   C generator export list:  /root/reference/src/engine/ir/codegen/mlp_train_codegen.rs:112-124
 *
 * Everything after those six is an extension under a new name.  The
 * reference bakes the topology and the optimizer constants into the
 * generated library; here they live in a `volta_mlp_spec`, set once per
 * process with volta_train_configure() (or the VOLTA_MLP_SPEC environment
 * variable) or passed per handle to volta_train_init_spec().
 *
 * Two libraries implement this header:
 *   volta_amd/libvolta_hip.so      -- the product: HIP kernels for gfx950
 *   oracle/liboracle_volta.so      -- the CPU restatement used as the checker
 *
 * The library leaves the process environment alone.  HIP replays the step
 * graph from the kernel packets it recorded at instantiation unless the
 * host sets DEBUG_CLR_GRAPH_PACKET_CAPTURE=0 before its first HIP call
 * (then the nodes are dispatched in order as stream launches, which is
 * faster for this chain of short dependent kernels); that choice is the
 * host's.
 *
 * Layout conventions (all row-major fp32, as in the reference):
 *   W_i  [L[i] x L[i+1]],  b_i [L[i+1]],  X [B x L[0]],  Y [B x L[n]]
 *
 * Threading: a handle is not thread-safe (same as the reference).  Calls on
 * different handles may run concurrently.
 */
#ifndef VOLTA_TRAIN_H
#define VOLTA_TRAIN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct VoltaTrainHandle VoltaTrainHandle;

/* ---------------------------------------------------------------------- */
/* Reference ABI (six symbols)                                             */
/* ---------------------------------------------------------------------- */

/* Allocate a handle for a fixed batch size using the process-wide spec
 * (volta_train_configure / VOLTA_MLP_SPEC).  Weights are drawn with the
 * reference's LCG Xavier-uniform stream, seed 42, in layer order; biases and
 * optimizer state start at zero (mlp_train_rust_codegen.rs:629-667).
 * Returns NULL on failure (see volta_train_last_error). */
VoltaTrainHandle* volta_train_init(int32_t batch);

/* One training step on host arrays X [B x L0] and Y [B x Ln] with learning
 * rate lr (mlp_train_rust_codegen.rs:698-994): forward, MSE loss, backward,
 * optimizer update.  The GPU library may return before the step has
 * finished on the device; volta_train_loss / volta_train_get_params /
 * volta_train_sync wait for it.  X and Y may be reused by the caller as soon
 * as the call returns. */
void volta_train_step(VoltaTrainHandle* h, const float* X, const float* Y, float lr);

/* Loss of the most recent step (mean over B*Ln for MSE, mean over B for
 * softmax-CE).  mlp_train_rust_codegen.rs:686 */
float volta_train_loss(VoltaTrainHandle* h);

/* Fill wo[i] / bo[i] (i < n_weight_layers) with pointers to host arrays
 * holding the current W_i and b_i.  The pointers stay valid until
 * volta_train_free; the GPU library refreshes the host mirror on each call.
 * mlp_train_rust_codegen.rs:677-684 */
void volta_train_get_params(VoltaTrainHandle* h, float** wo, float** bo);

/* Copy W_i [L[li] x L[li+1]] and b_i [L[li+1]] into layer li.  An
 * out-of-range li is ignored, as in the reference (:669-675); the
 * extension volta_train_status reports it. */
void volta_train_set_params(VoltaTrainHandle* h, int32_t li, const float* w, const float* b);

/* Release the handle and everything it owns.  NULL is allowed (:688-696). */
void volta_train_free(VoltaTrainHandle* h);

/* ---------------------------------------------------------------------- */
/* Extensions (no counterpart among the reference's exports)               */
/* ---------------------------------------------------------------------- */

#define VOLTA_MAX_LAYER_SIZES 17 /* up to 16 weight layers */

/* Hidden activation; names follow mlp_train_rust_codegen.rs:272-278. */
enum volta_activation {
  VOLTA_ACT_RELU = 0,
  VOLTA_ACT_SIGMOID = 1,
  VOLTA_ACT_TANH = 2,
  VOLTA_ACT_LEAKY_RELU = 3,
  VOLTA_ACT_SILU = 4,
  VOLTA_ACT_GELU = 5, /* tanh approximation, :580-596 */
  VOLTA_ACT_SOFTMAX = 6 /* row softmax over each hidden layer's units, :727-740, :898-906 */
};

/* Optimizer; mlp_train_rust_codegen.rs:264-268. */
enum volta_optimizer {
  VOLTA_OPT_SGD = 0,
  VOLTA_OPT_ADAM = 1,
  VOLTA_OPT_ADAMW = 2,
  VOLTA_OPT_ADAGRAD = 3
};

/* Loss head.  MSE is the generated step's loss (:792-798).  Softmax
 * cross-entropy follows the IR runtime (interpreter.rs:762-812,
 * autograd.rs:467-534) and takes int32 class labels. */
enum volta_loss {
  VOLTA_LOSS_MSE = 0,
  VOLTA_LOSS_SOFTMAX_CE = 1
};

typedef struct volta_mlp_spec {
  int32_t n_sizes;                       /* layer sizes incl. input and output, 2..17 */
  int32_t sizes[VOLTA_MAX_LAYER_SIZES];  /* L[0..n_sizes-1] */
  int32_t activation;                    /* enum volta_activation (hidden layers) */
  int32_t optimizer;                     /* enum volta_optimizer */
  int32_t loss;                          /* enum volta_loss */
  /* Optimizer constants.  The reference hard-codes beta1=0.9, beta2=0.999,
   * eps=1e-8 (Adam/AdamW/Adagrad) and weight_decay=0.01 (AdamW, weights
   * only) at mlp_train_rust_codegen.rs:807-813; volta_mlp_spec_default
   * fills exactly those. */
  float beta1;
  float beta2;
  float eps;
  float weight_decay;
  /* Codegen extras of the generated step (0 = off, the default):
   *   clip_grad  > 0: after the backward deltas, scale every delta by
   *              clip/||deltas|| when the norm over all layers' deltas
   *              exceeds clip (:936-955; db_i keeps the unscaled deltas).
   *   dropout_p  in [0, 1): inverted dropout after each hidden activation,
   *              mask from the LCG stream seeded 12345678 (:774-788).
   *   layernorm  1: LayerNorm (eps 1e-5) after each hidden activation,
   *              gamma=1/beta=0 at init, updated by plain SGD (:745-772,
   *              :829-887). */
  float clip_grad;
  float dropout_p;
  int32_t layernorm;
} volta_mlp_spec;

/* Fill *spec with the reference's constants for the given topology. */
void volta_mlp_spec_default(volta_mlp_spec* spec, int32_t n_sizes, const int32_t* sizes,
                            int32_t activation, int32_t optimizer, int32_t loss);

/* Parse "512-1024-1024-512-256-1:relu:adam[:mse|:ce][:eps=1e-10][:wd=0.01]
 * [:beta1=..][:beta2=..]" into *spec.  Returns 0 on success. */
int32_t volta_mlp_spec_parse(const char* text, volta_mlp_spec* spec);

/* Set the process-wide spec used by volta_train_init(batch).  Without it,
 * volta_train_init parses the VOLTA_MLP_SPEC environment variable.
 * Returns 0 on success. */
int32_t volta_train_configure(const volta_mlp_spec* spec);

/* Allocate a handle for an explicit spec.  Returns NULL on failure. */
VoltaTrainHandle* volta_train_init_spec(const volta_mlp_spec* spec, int32_t batch);

/* Softmax cross-entropy step: labels are B int32 class indices in
 * [0, L[n]).  Only valid when spec.loss == VOLTA_LOSS_SOFTMAX_CE. */
void volta_train_step_labels(VoltaTrainHandle* h, const float* X, const int32_t* labels,
                             float lr);

/* Step on inputs that are already in device memory (GPU library only; the
 * CPU oracle treats the pointers as host pointers).  Y is float [B x Ln]
 * for MSE or int32 [B] for softmax-CE.  When X/Y are the handle's own
 * resident batch buffers (volta_train_batch_buffers) no copy is made.
 * Returns 0 on success. */
int32_t volta_train_step_device(VoltaTrainHandle* h, const float* X, const void* Y, float lr);

/* Device pointers of the handle's resident batch: X [B x L0] and the
 * target buffer (float [B x Ln] or int32 [B]).  Returns 0 on success. */
int32_t volta_train_batch_buffers(VoltaTrainHandle* h, float** X, void** Y);

/* Wait until every enqueued step has finished.  Returns 0 or an error code. */
int32_t volta_train_sync(VoltaTrainHandle* h);

/* Status bits, sticky until volta_train_clear_status. */
#define VOLTA_STATUS_NONFINITE_LOSS 1 /* a step produced a NaN/Inf loss */
#define VOLTA_STATUS_BAD_ARGUMENT   2 /* an entry point rejected its arguments */
#define VOLTA_STATUS_DEVICE_ERROR   4 /* a HIP call failed */
int32_t volta_train_status(VoltaTrainHandle* h);
void volta_train_clear_status(VoltaTrainHandle* h);

/* Last error message of the calling thread ("" when none). */
const char* volta_train_last_error(void);

/* Number of weight layers (n_sizes - 1) and the batch size of a handle. */
int32_t volta_train_num_layers(VoltaTrainHandle* h);
int32_t volta_train_batch(VoltaTrainHandle* h);

/* Training state export/import for resumable training (the generated
 * library has no way to save it).  The state is laid out per layer as
 * [m_W | m_b | v_W | v_b] (Adam/AdamW) or [G_W | G_b] (Adagrad), layers in
 * order (SGD has no optimizer state), followed, when the spec has
 * LayerNorm, by [gamma_i | beta_i] for each hidden layer i = 0..n-2.
 * `step` is the Adam step counter t.  volta_train_state_size returns the
 * float count.  The dropout stream has its own pair of calls below. */
int64_t volta_train_state_size(VoltaTrainHandle* h);

/* Copy one intermediate buffer of the most recent step to host memory
 * `out` (for tests and debugging; the reference keeps the same buffers in
 * its Handle, mlp_train_rust_codegen.rs:442-560):
 *   VOLTA_BUF_ACT    act_i   [B x L[i]],   i = 0..n
 *   VOLTA_BUF_DELTA  delta_i [B x L[i+1]], i = 0..n-1 (after the activation
 *                    derivative has been applied)
 *   VOLTA_BUF_GRAD_W dW_i    [L[i] x L[i+1]] (GPU library: only when the
 *                    handle was created with VOLTA_KEEP_GRADS=1, since the
 *                    optimizer update is fused into the dW product)
 *   VOLTA_BUF_GRAD_B db_i    [L[i+1]] (same condition)
 * Returns the number of floats written, or -1. */
#define VOLTA_BUF_ACT 0
#define VOLTA_BUF_DELTA 1
#define VOLTA_BUF_GRAD_W 2
#define VOLTA_BUF_GRAD_B 3
/*   VOLTA_BUF_LN_GAMMA   gamma_i [L[i+1]], i = 0..n-2 (spec.layernorm)
 *   VOLTA_BUF_LN_BETA    beta_i  [L[i+1]]
 *   VOLTA_BUF_DROPOUT_MASK keep mask of hidden layer i as 0.0/1.0
 *                        [B x L[i+1]] (spec.dropout_p > 0) */
#define VOLTA_BUF_LN_GAMMA 4
#define VOLTA_BUF_LN_BETA 5
#define VOLTA_BUF_DROPOUT_MASK 6
/*   VOLTA_BUF_PRE        pre_i [B x L[i+1]], i = 0..n-2: the hidden layer's
 *                        pre-activation act_i W_i + b_i (GPU library: kept
 *                        only where the backward needs it -- leaky ReLU,
 *                        SiLU, GELU, softmax, LayerNorm or dropout) */
#define VOLTA_BUF_PRE 7
/*   VOLTA_BUF_LN_DGAMMA  dgamma_i [L[i+1]], i = 0..n-2 (spec.layernorm): the
 *                        LayerNorm scale gradient the step applied (:843-887)
 *   VOLTA_BUF_LN_DBETA   dbeta_i  [L[i+1]]
 *   VOLTA_BUF_CLIP_SCALE one float (layer ignored): the factor the step
 *                        multiplied every delta by (spec.clip_grad > 0; 1
 *                        when the norm was within the limit, :936-955) */
#define VOLTA_BUF_LN_DGAMMA 8
#define VOLTA_BUF_LN_DBETA 9
#define VOLTA_BUF_CLIP_SCALE 10
int64_t volta_train_debug_buffer(VoltaTrainHandle* h, int32_t kind, int32_t layer, float* out);
int32_t volta_train_get_state(VoltaTrainHandle* h, float* state, int64_t* step);
int32_t volta_train_set_state(VoltaTrainHandle* h, const float* state, int64_t step);

/* The dropout LCG state (the reference Handle's dropout_rng, seeded
 * 12345678 at alloc, :553, and advanced once per hidden element per
 * step, :777), for resuming a run with dropout.  Return 0, or -1. */
int32_t volta_train_get_dropout_rng(VoltaTrainHandle* h, uint64_t* rng);
int32_t volta_train_set_dropout_rng(VoltaTrainHandle* h, uint64_t rng);

/* Change the optimizer hyperparameters of a live handle (the generated
 * library bakes them in, mlp_train_rust_codegen.rs:803-811, :957-993):
 * Adam/AdamW beta1 and beta2, eps (Adam/AdamW/Adagrad), AdamW weight decay
 * (weights only).  The step counter and optimizer state are kept; the next
 * step uses the new values.  Waits for enqueued steps.  Returns 0, or -1
 * (volta_train_last_error) for values outside the ranges the spec accepts. */
int32_t volta_train_set_hparams(VoltaTrainHandle* h, float beta1, float beta2, float eps, float weight_decay);

/* Forward pass only, with the handle's current parameters: out [rows x Ln]
 * = the output layer's pre-activation (no loss, no softmax) for host input
 * X [rows x L0]; any rows > 0 (run B rows at a time).  Synchronous.  Uses
 * the handle's activation buffers, which the next step recomputes.
 * Returns 0 on success. */
int32_t volta_train_infer(VoltaTrainHandle* h, const float* X, int64_t rows, float* out);

/* Allocation-free variant of volta_train_infer.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (serving
 * loops, harnesses that forbid hipMalloc).
 * X [rows x L0] and out [rows x Ln] are 16-byte aligned device buffers; the
 * forward runs on the handle's weights and activation buffers with its
 * split-K partial planes in a static 64 MiB device array per GPU (held from
 * library load to process end); rows whose plan needs more are rejected
 * with an error.  Nothing is allocated, freed or synchronized: the launches
 * are enqueued on the handle's own stream, not on a stream of the caller,
 * so a caller's stream capture does not record them and nothing orders
 * them after the caller's work: finish the work that writes X first (e.g.
 * synchronize the stream that produced it), and call volta_train_sync
 * before reading out.  Calls that overlap on one GPU share that GPU's
 * scratch and race.  Returns 0, or -1 with volta_train_last_error() set. */
int32_t volta_train_infer_device_noalloc(VoltaTrainHandle* h, const float* X, int64_t rows, float* out);

/* The inference library's entry point (codegen/inner.rs:198; contract
 * docs/ARCHITECTURE.md:125-141): output = forward(input) for in_n = rows*L0
 * input floats, writing rows*Ln floats (out_n must be at least that).  The
 * reference embeds trained weights in the inference library; here the model
 * is the handle given to volta_infer_bind (null unbinds; the binding is
 * process-wide).  On an error `output` is left untouched and
 * volta_train_last_error() says why. */
int32_t volta_infer_bind(VoltaTrainHandle* h);
void volta_infer(const float* input, int64_t in_n, float* output, int64_t out_n);

/* The model of an inference library made by `volta-hip compile` (the
 * reference's `volta compile`, main.rs:158-215 -> executor.rs:1684-1744,
 * whose library embeds the trained weights, codegen/inner.rs:190-262): the
 * forward graph lower_model_to_graph builds (lowering.rs:87-140) -- each
 * layer MatMul by W_i then Add of b_i; hidden layers followed by ReLU when
 * hidden_act is VOLTA_ACT_RELU, by nothing when it is -1 -- with the
 * parameters `params` ([W_0 | b_0 | W_1 | b_1 | ...], host float32, W_i
 * row-major [L_i x L_i+1]) copied to the device.  Run it with
 * volta_train_infer (any row count, host buffers); release it with
 * volta_train_free.  Returns NULL, with volta_train_last_error() set, on bad
 * arguments, no device, or a device failure. */
VoltaTrainHandle* volta_infer_model_create(int32_t n_sizes, const int32_t* sizes, int32_t hidden_act,
                                           const float* params);

#ifdef __cplusplus
}
#endif

#endif /* VOLTA_TRAIN_H */
