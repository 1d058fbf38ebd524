// Host runtime of the gfx950 compile-train MLP step: the C ABI of
// include/volta_train.h on top of one device arena and a fixed launch
// sequence, planned once at init and enqueued as it stands every step (or,
// with VOLTA_GRAPH=1, captured once as a hipGraph and replayed).
//
// Mapping onto the reference:
//   Handle + alloc (mlp_train_rust_codegen.rs:442-560)  -> Handle, one arena
//   LCG Xavier init, seed 42 (:629-667)                 -> lcg_xavier_init
//   volta_train_step body (:698-994)                    -> enqueue_step()
//   get/set_params, loss, free (:669-696)               -> host mirror + copies
//
// The step's launch order (a topological order of the step's dataflow):
//   fwd_0 .. fwd_{n-2}          GEMM NN + bias + activation (in the split-K
//                               reduction when K is split); opt-in, a
//                               small-batch product on few CUs over two halves
//                               of K into two planes, which the next forward
//                               launch adds with the bias and activation
//   fwd_{n-1} + loss            narrow output kernel (L_n <= 16), GEMM with the
//                               loss head in its epilogue (<= 64), or GEMM +
//                               loss kernel: delta_{n-1}, loss, Adam t
//   dX_{n-1}                    outer product (L_n <= 16) or GEMM NT; merged
//                               into the output launch where that is narrow
// then, when every dW runs on the small-K tile (batch <= 256: C1-C4 up to
// B=256):
//   dX_i, i = n-2 .. 1          one launch each, on their own wave count (the
//                               output launch also forms dX_{n-2} where that
//                               product runs on 16-wave small-M workgroups)
//   dW_{n-1} .. dW_0            one grouped launch (dw_group_kernel)
// and otherwise (larger batches):
//   dX_i | dW_{i+1}             one paired launch, i = n-2 .. 1 (where both
//                               fit the paired kernels, else two launches)
//   dW_1 | dW_0                 one paired launch
// With LayerNorm, dropout, softmax hidden activations or gradient clipping
// the backward runs unpaired (enqueue_step's extras branch).
// dX_i: GEMM NT with epilogue * f'(layer i-1) -> delta_{i-1}.  dW_i: GEMM TN
// whose epilogue applies SGD/Adam/AdamW/Adagrad to W_i, and to b_i from the
// column sums of delta_i (db_i) the same kernel forms.  dX_i reads W_i before
// dW_i rewrites it (a later launch), so every delta comes from the pre-update
// weights, as in the reference's two-phase backward.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "extras.h"
#include "narrow_dw.h"
#include "gemm.h"
#include "skinny.h"
#include "spec.h"
#include "step_kernels.h"

namespace volta {

// How the output layer and the loss head run.
enum OutMode {
  OUT_NARROW = 0,     // L[n] <= 16: out_layer_kernel (dot products + loss head)
  OUT_GEMM_LOSS = 1,  // L[n] <= 64: MFMA GEMM with the loss head in its epilogue
  OUT_GEMM = 2,       // wider: MFMA GEMM, then a stand-alone loss kernel
};

static std::string hip_msg(const char* what, hipError_t e) {
  return std::string(what) + ": " + hipGetErrorString(e);
}

// Reference lcg_xavier_init (mlp_train_rust_codegen.rs:629-638).
static void lcg_xavier_init(float* w, size_t n, int r, int c, uint64_t* rng) {
  const float lim = std::sqrt(6.0f / ((float)r + (float)c));
  for (size_t i = 0; i < n; ++i) {
    *rng = *rng * 6364136223846793005ULL + 1442695040888963407ULL;
    const float f = (float)((*rng >> 11) & ((1ULL << 53) - 1)) / (float)(1ULL << 53);
    w[i] = (f * 2.0f - 1.0f) * lim;
  }
}

static size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

struct LayerPlan {
  int r = 0, c = 0;
  int64_t w_off = 0, b_off = 0;  // float offsets into the flat parameter buffer
  GemmPlan fwd, dx, dw;
};

struct Handle {
  volta_mlp_spec spec{};
  int B = 0, n = 0;
  std::vector<int> L;
  int device = 0;
  int num_cus = 256;
  hipStream_t stream = nullptr;

  // --- device arena ---------------------------------------------------------
  char* arena = nullptr;
  size_t arena_bytes = 0;
  int64_t flat = 0;  // padded float count of the flat parameter buffer
  float* params = nullptr;
  float* grads = nullptr;
  float* opt_a = nullptr;  // Adam m / Adagrad G
  float* opt_b = nullptr;  // Adam v
  std::vector<float*> act;    // act[0..n]; act[0] is the resident X
  std::vector<float*> pre;    // pre[0..n-2]; null where the activation needs no pre
  std::vector<float*> delta;  // delta[0..n-1]
  void* target = nullptr;     // resident Y (float [B x Ln]) or labels (int32 [B])
  float* gemm_ws = nullptr;   // split-K partial planes: [0, ws_half) and [ws_half, 2*ws_half), one
                              // region per operation of a paired launch
  size_t ws_half = 0;         // floats
  bool pair_backward = true;  // dX_i and dW_{i+1} in one launch (VOLTA_NO_PAIR=1: separate)
  unsigned* counters = nullptr;   // split-K arrival counters (+1: loss counter)
  int n_counters = 0;
  float* loss_partials = nullptr;  // one float per output-layer M-tile
  int out_mode = 0;           // OUT_NARROW / OUT_GEMM_LOSS / OUT_GEMM (output layer + loss head)
  bool narrow_dx = false;     // dX of the output layer as an outer product (L[n] <= 16)
  bool out_dx_merged = false; // ... formed by the output layer's own launch (out_layer_dx_kernel)
  bool fwd_head = false;      // ... and that launch folded into the last hidden forward launch (opt-in)
  bool tail_merge = false;    // ... or that launch and dX_{n-2} in one (gemm_smallm_tail; VOLTA_NO_TAIL=1: off)
  bool narrow_dw = false;     // dW of the output layer by narrow_dw_kernel
  bool out_mfma = false;      // large batch: the narrow output layer on small-M tiles, its loss summed by dX_{n-1}
  std::vector<int> fwd_khalf; // per layer: > 0 runs its forward over two halves of K (this one first),
                              // its output formed by the next forward launch (0: one launch)
  bool keep_grads = false;    // also store dW/db in `grads` (VOLTA_KEEP_GRADS=1)
  DevScalars* scalars = nullptr;
  float2* bc_table = nullptr;  // own allocation (its length depends on beta1/beta2)
  int bc_len = 0;
  float* infer_x = nullptr;    // inference input rows (allocated on first use)
  float* infer_ws = nullptr;   // split-K workspace of inference plans (grown on demand)
  float* scratch = nullptr;    // this device's static scratch (allocation-free inference)
  bool dx_alone = false;       // small-batch backward: dX launches alone, dW products grouped
  bool dw_group = false;       // ... in one launch (off with VOLTA_NO_PAIR)
  bool ext_dw_group = false;   // codegen extras: phase 2's dW products in one launch likewise
  int dw_group_tn = 0;         // columns of the group's small-K tiles: 0 picks per group; VOLTA_DW_GROUP_TN 32 or 64
  int dw_tn_pick[2] = {0, 0};  // the width each group uses (main, extras), fixed at its first build
  size_t infer_ws_floats = 0;
  SegTable segs{};
  std::vector<LayerPlan> layers;

  // --- codegen extras (spec.layernorm / dropout_p / clip_grad) --------------
  bool ext_ln = false, ext_drop = false, ext_clip = false;
  bool ext_softmax = false;          // softmax hidden activation (a row operation)
  std::vector<float*> ln_g, ln_b;    // gamma, beta [L[i+1]] per hidden layer i < n-1
  std::vector<float*> ln_mu, ln_is;  // row statistics [B]
  std::vector<float*> ln_dg, ln_db;  // gradients [L[i+1]]
  std::vector<uint8_t*> mask;        // dropout keep mask [B x L[i+1]]
  float* clip_partials = nullptr;    // [kClipBlocks]
  bool hidden_ext() const { return ext_ln || ext_drop || ext_softmax; }
  bool extras() const { return hidden_ext() || ext_clip; }
  // activation of the hidden layers' GEMM epilogue (softmax runs after it)
  int gemm_act() const { return ext_softmax ? kIdentity : spec.activation; }
  // inference model of a `volta-hip compile` library whose hidden layers
  // carry no activation (volta_infer_model_create)
  bool infer_linear = false;

  // --- launch sequence -------------------------------------------------------
  bool use_graph = false;  // replay the sequence from a captured hipGraph (VOLTA_GRAPH=1)
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;

  // --- host side -------------------------------------------------------------
  float* h_params = nullptr;  // pinned mirror returned by get_params
  float* h_stage_x = nullptr;   // pinned [X | gap | Y] (one allocation)
  void* h_stage_y = nullptr;    // its Y part, stage_y_off bytes in
  size_t stage_y_off = 0;
  hipEvent_t stage_free = nullptr;  // staging buffers may be overwritten
  static constexpr int kLrSlots = 64;
  float* h_lr = nullptr;
  hipEvent_t lr_ev[kLrSlots] = {};
  bool lr_pending[kLrSlots] = {};
  int lr_slot = 0;
  bool lr_known = false;
  float cur_lr = 0.0f;
  int32_t status = 0;

  ~Handle();
};

Handle::~Handle() {
  // Teardown is best effort: errors here have no caller to report to.
  if (stream) (void)hipStreamSynchronize(stream);
  if (exec) (void)hipGraphExecDestroy(exec);
  if (graph) (void)hipGraphDestroy(graph);
  for (auto& e : lr_ev)
    if (e) (void)hipEventDestroy(e);
  if (stage_free) (void)hipEventDestroy(stage_free);
  if (h_params) (void)hipHostFree(h_params);
  if (h_stage_x) (void)hipHostFree(h_stage_x);
  if (h_lr) (void)hipHostFree(h_lr);
  if (bc_table) (void)hipFree(bc_table);
  if (infer_x) (void)hipFree(infer_x);
  if (infer_ws) (void)hipFree(infer_ws);
  if (arena) (void)hipFree(arena);
  if (stream) (void)hipStreamDestroy(stream);
}

#define VOLTA_CHECK(call)                                   \
  do {                                                      \
    hipError_t e_ = (call);                                 \
    if (e_ != hipSuccess) {                                 \
      set_last_error(hip_msg(#call, e_));                   \
      return false;                                         \
    }                                                       \
  } while (0)

// LayerNorm / dropout of hidden layer i over `rows` rows of act_{i+1}
// (training: statistics kept and dropout drawn; inference: LayerNorm only).
static HiddenFwdArgs hidden_fwd_args(const Handle* h, int i, int rows, bool train) {
  HiddenFwdArgs f{};
  f.act = h->act[i + 1];
  f.B = rows;
  f.c = h->L[i + 1];
  f.softmax = h->ext_softmax ? 1 : 0;
  if (h->ext_ln) {
    f.gamma = h->ln_g[i];
    f.beta = h->ln_b[i];
    f.mu = train ? h->ln_mu[i] : nullptr;
    f.inv_std = train ? h->ln_is[i] : nullptr;
  }
  if (train && h->ext_drop) {
    f.mask = h->mask[i];
    f.p = h->spec.dropout_p;
    f.keep_scale = 1.0f / (1.0f - h->spec.dropout_p);
    uint64_t off = 0;
    for (int k = 0; k < i; ++k) off += (uint64_t)h->B * h->L[k + 1];
    f.rng_offset = off;
  }
  f.scalars = h->scalars;
  return f;
}

// Tile width of a dW group (VOLTA_DW_GROUP_TN, else picked once from the
// group's tile counts and the device's residency) and its products' first
// workgroups.  `which`: 0 the step's group, 1 the extras step's.
static void set_group_width(Handle* h, DwGroup& d, int which) {
  int& tn = h->dw_tn_pick[which];
  if (!tn) tn = h->dw_group_tn ? h->dw_group_tn : dw_group_pick_tile_n(d, h->num_cus);
  d.tile_n = tn;
  d.start[0] = 0;
  for (int i = 0; i < d.n; ++i) d.start[i + 1] = d.start[i] + dw_group_tiles(d.g[i], tn);
}

// Enqueue one whole step on `st` (captured into the graph once, with
// VOLTA_GRAPH=1).  With a recorder attached, an event follows every kernel
// (profiling only).
static bool enqueue_step(Handle* h, hipStream_t st, Recorder* rec = nullptr) {
  const volta_mlp_spec& s = h->spec;
  const int n = h->n, B = h->B;
  const int Ln = h->L[n];
  char label[64];
  auto base_args = [&](GemmArgs& a) {
    a.partial = h->gemm_ws;
    a.counters = h->counters;
    a.epi.scalars = h->scalars;
  };
  // Operations of the backward pass (:819-993): the grouped dW launch of a
  // small-batch step is built from them before the forward, every other
  // backward launch after it.
  const int sopt = s.optimizer == VOLTA_OPT_SGD ? 2 : s.optimizer == VOLTA_OPT_ADAGRAD ? 4 : 6;
  // dX_i as a GEMM (i > 0 and not the narrow output layer)
  auto make_dx = [&](int i, float* ws) {
    const LayerPlan& lp = h->layers[i];
    PairOp o;
    o.kind = PAIR_GEMM;
    o.plan = lp.dx;
    GemmArgs& a = o.args;
    base_args(a);
    a.partial = ws;
    a.A = h->delta[i];
    a.lda = lp.c;
    a.B = h->params + lp.w_off;
    a.ldb = lp.c;
    a.M = B;
    a.N = lp.r;
    a.K = lp.c;
    a.epi.kind = EPI_DX_ACT;
    a.epi.act = s.activation;
    a.epi.ldc = lp.r;
    a.epi.out = h->delta[i - 1];
    a.epi.aux_act = h->act[i];
    a.epi.aux_pre = h->pre[i - 1];
    return o;
  };
  // dW_i = act_i^T delta_i with db_i = column sums of delta_i and the
  // optimizer update of W_i and b_i (GEMM epilogue, or the narrow kernel for
  // the output layer).
  auto make_dw = [&](int i, float* ws) {
    const LayerPlan& lp = h->layers[i];
    PairOp o;
    const int opt = s.optimizer == VOLTA_OPT_ADAMW ? VOLTA_OPT_ADAM : s.optimizer;
    const float wd = s.optimizer == VOLTA_OPT_ADAMW ? s.weight_decay : 0.0f;
    if (i == n - 1 && h->narrow_dw) {
      o.kind = PAIR_NARROW_DW;
      NarrowDwArgs& d = o.nd;
      d.act = h->act[i];
      d.delta = h->delta[i];
      d.B = B;
      d.R = lp.r;
      d.N = lp.c;
      d.opt = opt;
      d.w = h->params + lp.w_off;
      d.b = h->params + lp.b_off;
      d.m = h->opt_a ? h->opt_a + lp.w_off : nullptr;
      d.v = h->opt_b ? h->opt_b + lp.w_off : nullptr;
      d.bm = h->opt_a ? h->opt_a + lp.b_off : nullptr;
      d.bv = h->opt_b ? h->opt_b + lp.b_off : nullptr;
      d.grad = h->keep_grads ? h->grads + lp.w_off : nullptr;
      d.bgrad = h->keep_grads ? h->grads + lp.b_off : nullptr;
      d.wd = wd;
      d.b1 = s.beta1;
      d.b2 = s.beta2;
      d.eps = s.eps;
      d.scalars = h->scalars;
      return o;
    }
    o.kind = PAIR_GEMM;
    o.plan = lp.dw;
    GemmArgs& a = o.args;
    base_args(a);
    a.partial = ws;
    a.A = h->act[i];
    a.lda = lp.r;
    a.B = h->delta[i];
    a.ldb = lp.c;
    a.M = lp.r;
    a.N = lp.c;
    a.K = B;
    a.colsum_b = 1;
    EpiArgs& e = a.epi;
    e.kind = EPI_DW_OPT;
    e.ldc = lp.c;
    e.opt = opt;
    e.out = h->params + lp.w_off;
    e.b = h->params + lp.b_off;
    e.m = h->opt_a ? h->opt_a + lp.w_off : nullptr;
    e.v = h->opt_b ? h->opt_b + lp.w_off : nullptr;
    e.bm = h->opt_a ? h->opt_a + lp.b_off : nullptr;
    e.bv = h->opt_b ? h->opt_b + lp.b_off : nullptr;
    e.grad = h->keep_grads ? h->grads + lp.w_off : nullptr;
    e.bgrad = h->keep_grads ? h->grads + lp.b_off : nullptr;
    e.count = (int64_t)lp.r * lp.c;
    e.wd = wd;
    e.b1 = s.beta1;
    e.b2 = s.beta2;
    e.eps = s.eps;
    return o;
  };
  // algorithmic figures (flops, bytes) of dX_i and dW_i:
  //   dX: 4(B*c + r*c + 2*B*r); dW + db + optimizer: 4(B*r + B*c) + 4*s*(r*c + c)
  //   with s = 2 (SGD), 4 (Adagrad), 6 (Adam/AdamW) beyond the gradient.
  auto dx_cost = [&](int i) {
    const LayerPlan& lp = h->layers[i];
    return std::make_pair(2.0 * B * lp.r * lp.c, 4.0 * ((double)B * lp.c + (double)lp.r * lp.c + 2.0 * B * lp.r));
  };
  auto dw_cost = [&](int i) {
    const LayerPlan& lp = h->layers[i];
    return std::make_pair(2.0 * B * lp.r * lp.c,
                          4.0 * ((double)B * lp.r + (double)B * lp.c) + 4.0 * sopt * ((double)lp.r * lp.c + lp.c));
  };
  // Small-batch steps run every dW in one grouped launch after the dX
  // chain.  It is built before the forward so the output launch knows
  // whether it may leave the step's loss sum to that launch (no arrival
  // ticket and agent-scope fences in the output launch).
  DwGroup group;
  std::string group_label;
  double group_fl = 0.0, group_by = 0.0;
  bool group_ok = false, defer_loss = false;
  if (h->dx_alone) {
    for (int i = n - 1; i >= 0; --i) {
      const PairOp o = make_dw(i, h->gemm_ws);
      if (o.kind == PAIR_NARROW_DW) {
        group.nd = o.nd;
        group.narrow_blocks = (o.nd.R + kNarrowRows - 1) / kNarrowRows;
      } else {
        group.g[group.n] = o.args;
        group.g[group.n].k_per_split = o.plan.k_per_split;
        ++group.n;
      }
      char lx[32];
      std::snprintf(lx, sizeof lx, "dw%d+db+opt", i);
      group_label += (group_label.empty() ? "" : "|") + std::string(lx);
      group_fl += dw_cost(i).first;
      group_by += dw_cost(i).second;
    }
    set_group_width(h, group, 0);
    defer_loss = h->dw_group && h->out_mode == OUT_NARROW && h->out_dx_merged && !h->fwd_head;
    if (defer_loss) {
      group.loss_partials = h->loss_partials;
      group.loss_blocks = out_layer_dx_blocks(B);
      group.loss_denom = s.loss == VOLTA_LOSS_MSE ? (float)(B * Ln) : (float)B;
      group.loss_scalars = h->scalars;
    }
    group_ok = h->dw_group && dw_group_supported(group);
    if (!group_ok && defer_loss) {
      defer_loss = false;
      group.loss_partials = nullptr;
      group_ok = h->dw_group && dw_group_supported(group);
    }
  }
  // The narrow output layer's arguments (layer n-1), with its dX_{n-1}
  // fields when that is formed in the same launch.
  auto out_args = [&]() {
    const LayerPlan& lp = h->layers[n - 1];
    OutLayerArgs o{};
    o.act = h->act[n - 1];
    o.W = h->params + lp.w_off;
    o.bias = h->params + lp.b_off;
    o.B = B;
    o.K = lp.r;
    o.N = lp.c;
    o.loss = s.loss;
    o.y = static_cast<const float*>(h->target);
    o.labels = static_cast<const int32_t*>(h->target);
    o.out = h->act[n];
    o.delta = h->delta[n - 1];
    o.partials = h->loss_partials;
    o.scalars = h->scalars;
    o.bc_table = h->bc_table;
    o.bc_len = h->bc_len;
    if (h->out_dx_merged) {
      o.dx_act = s.activation;
      o.dx_pre = h->pre[n - 2];
      o.dx_out = h->delta[n - 2];
      o.loss_counter = h->counters + h->n_counters - 1;
      o.defer_loss = defer_loss ? 1 : 0;
    }
    return o;
  };
  // algorithmic bytes of the narrow output layer: 4(B*r + r*c + B*c) + loss
  // head 8*B*c; with its dX: + 4*B*r (act re-read from cache not counted)
  auto out_bytes = [&]() {
    const LayerPlan& lp = h->layers[n - 1];
    return 4.0 * ((double)B * lp.r + (double)lp.r * lp.c + (double)B * lp.c) + 8.0 * B * lp.c +
           (h->out_dx_merged ? 4.0 * (double)B * lp.r : 0.0);
  };
  bool head_done = false;  // the output layer ran in the last hidden forward launch
  // The output launch and dX_{n-2} in one launch when the product runs on
  // the 16-wave small-M tile and the loss sum is left to the dW group.
  bool tail = false;
  if (h->tail_merge && defer_loss && h->out_mode == OUT_NARROW) {
    const PairOp t = make_dx(n - 2, h->gemm_ws);
    tail = tail_supported(t.plan, t.args, out_args());
  }
  // Forward (:702-789); the output layer also runs the loss head (:792-798).
  for (int i = 0; i < n; ++i) {
    const LayerPlan& lp = h->layers[i];
    const bool last = i == n - 1;
    if (last && head_done) continue;
    if (last && h->out_mfma) {
      GemmArgs a{};
      base_args(a);
      a.A = h->act[i];
      a.lda = lp.r;
      a.B = h->params + lp.w_off;
      a.ldb = lp.c;
      a.M = B;
      a.N = lp.c;
      a.K = lp.r;
      a.epi.kind = EPI_ROWS;
      a.epi.bias = h->params + lp.b_off;
      VOLTA_CHECK(launch_smallm_out_head(a, out_args(), st));
      std::snprintf(label, sizeof label, "fwd%d+loss", i);
      VOLTA_CHECK(mark(rec, label, 2.0 * B * lp.r * lp.c, out_bytes()));
      continue;
    }
    if (last && h->out_mode == OUT_NARROW) {
      const OutLayerArgs o = out_args();
      const double fb = out_bytes();
      if (tail) {
        // ... and dX_{n-2}, whose A operand each workgroup forms from its rows
        const PairOp t = make_dx(n - 2, h->gemm_ws);
        VOLTA_CHECK(launch_smallm_tail(t.plan, t.args, o, st));
        std::snprintf(label, sizeof label, "fwd%d+loss+dx%d+dx%d", i, i, i - 1);
        VOLTA_CHECK(mark(rec, label, 4.0 * B * lp.r * lp.c + dx_cost(n - 2).first, fb + dx_cost(n - 2).second));
        continue;
      }
      if (h->out_dx_merged) {
        // the output layer's dX_{n-1} in the same launch (row-local)
        VOLTA_CHECK(launch_out_layer_dx(o, st));
        std::snprintf(label, sizeof label, "fwd%d+loss+dx%d", i, i);
        VOLTA_CHECK(mark(rec, label, 4.0 * B * lp.r * lp.c, fb));
        continue;
      }
      VOLTA_CHECK(launch_out_layer(o, st));
      std::snprintf(label, sizeof label, "fwd%d+loss", i);
      VOLTA_CHECK(mark(rec, label, 2.0 * B * lp.r * lp.c, fb));
      continue;
    }
    GemmArgs a{};
    base_args(a);
    a.A = h->act[i];
    a.lda = lp.r;
    a.B = h->params + lp.w_off;
    a.ldb = lp.c;
    a.M = B;
    a.N = lp.c;
    a.K = lp.r;
    a.epi.kind = last && h->out_mode == OUT_GEMM_LOSS ? EPI_LOSS : EPI_BIAS_ACT;
    a.epi.act = last ? kIdentity : h->gemm_act();
    a.epi.ldc = lp.c;
    a.epi.out = h->act[i + 1];
    a.epi.pre = last ? nullptr : h->pre[i];
    a.epi.bias = h->params + lp.b_off;
    if (last) {
      a.epi.loss = s.loss;
      a.epi.y = static_cast<const float*>(h->target);
      a.epi.labels = static_cast<const int32_t*>(h->target);
      a.epi.delta = h->delta[n - 1];
      a.epi.loss_partials = h->loss_partials;
      a.epi.loss_counter = h->counters + h->n_counters - 1;
      a.epi.loss_tiles = (B + 63) / 64;
      a.epi.bc_table = h->bc_table;
      a.epi.bc_len = h->bc_len;
    }
    std::snprintf(label, sizeof label, last && h->out_mode == OUT_GEMM_LOSS ? "fwd%d+loss" : "fwd%d", i);
    // algorithmic bytes: 4(B*r + r*c + B*c*(2 if hidden else 1)) (+ loss head)
    const double bytes = 4.0 * ((double)B * lp.r + (double)lp.r * lp.c + (double)B * lp.c * (last ? 1 : 2)) +
                         (last && h->out_mode == OUT_GEMM_LOSS ? 8.0 * B * Ln : 0.0);
    if (!last && h->fwd_khalf[i]) {
      // two halves of K into the workspace's planes (4(B*r + r*c + 2*B*c))
      VOLTA_CHECK(launch_smallm_khalves(lp.fwd, a, h->gemm_ws, h->fwd_khalf[i], st));
      std::snprintf(label, sizeof label, "fwd%d.khalves", i);
      VOLTA_CHECK(mark(rec, label, 2.0 * a.M * a.N * a.K,
                       4.0 * ((double)B * lp.r + (double)lp.r * lp.c + 2.0 * B * lp.c)));
      continue;
    }
    if (!last && i > 0 && h->fwd_khalf[i - 1]) {
      // layer i-1's planes + bias + activation as this product's A operand
      // (+ 4(B*r + r + B*r [+ B*r pre]) beyond this layer's own bytes)
      const LayerPlan& pl = h->layers[i - 1];
      PlaneArgs pa;
      pa.p1 = h->gemm_ws + (size_t)B * pl.c;
      pa.bias = h->params + pl.b_off;
      pa.act_out = h->act[i];
      pa.pre_out = h->pre[i - 1];
      pa.act = h->gemm_act();
      a.A = h->gemm_ws;
      VOLTA_CHECK(launch_smallm_planes(lp.fwd, a, pa, st));
      std::snprintf(label, sizeof label, "fwd%d.sum+fwd%d", i - 1, i);
      VOLTA_CHECK(mark(rec, label, 2.0 * a.M * a.N * a.K,
                       bytes + 4.0 * ((double)B * lp.r * (pa.pre_out ? 3.0 : 2.0) + lp.r)));
      continue;
    }
    if (i == n - 2 && h->fwd_head) {
      const OutLayerArgs o = out_args();
      GemmArgs af = a;
      af.k_per_split = lp.fwd.k_per_split;
      if (fwd_head_supported(lp.fwd, af, o, h->n_counters - 1)) {
        VOLTA_CHECK(launch_fwd_head(lp.fwd, a, o, h->counters, h->n_counters - 1, st));
        const LayerPlan& lo = h->layers[n - 1];
        std::snprintf(label, sizeof label, "fwd%d+fwd%d+loss+dx%d", i, i + 1, i + 1);
        VOLTA_CHECK(mark(rec, label, 2.0 * a.M * a.N * a.K + 4.0 * B * lo.r * lo.c, bytes + out_bytes()));
        head_done = true;
        continue;
      }
    }
    VOLTA_CHECK(gemm_launch(lp.fwd, a, st, rec, label, bytes));
    if (!last && h->hidden_ext()) {
      VOLTA_CHECK(launch_hidden_fwd(hidden_fwd_args(h, i, B, true), st));
      std::snprintf(label, sizeof label, "fwd%d.ln_dropout", i);
      VOLTA_CHECK(mark(rec, label, 0.0, 4.0 * 3.0 * B * lp.c));
      if (h->ext_drop && i == n - 2) {
        uint64_t draws = 0;
        for (int k = 0; k < n - 1; ++k) draws += (uint64_t)B * h->L[k + 1];
        VOLTA_CHECK(launch_rng_advance(h->scalars, draws, st));
        VOLTA_CHECK(mark(rec, "rng_advance", 0.0, 0.0));
      }
    }
  }
  if (h->out_mode == OUT_GEMM) {  // output layer wider than one tile: stand-alone loss head
    if (s.loss == VOLTA_LOSS_MSE)
      VOLTA_CHECK(launch_loss_mse(h->act[n], static_cast<const float*>(h->target), h->delta[n - 1], B * Ln,
                                  h->scalars, h->bc_table, h->bc_len, st));
    else
      VOLTA_CHECK(launch_loss_ce(h->act[n], static_cast<const int32_t*>(h->target), h->delta[n - 1], B, Ln,
                                 h->scalars, h->bc_table, h->bc_len, st));
    VOLTA_CHECK(mark(rec, "loss", 0.0, 12.0 * B * Ln));
  }
  // Backward (:819-993).  dX_i reads W_i before dW_i updates it in place,
  // so every delta comes from the pre-update weights.
  //
  // Launch order: dX_{n-1}; then (dX_i with dW_{i+1}) for i = n-2 .. 1; then
  // (dW_1 with dW_0).  The two operations of a pair touch disjoint buffers
  // (dX_i reads W_i, delta_i; dW_{i+1} rewrites W_{i+1}, b_{i+1} and their
  // optimizer state), and each pair runs after the launch that produced its
  // inputs (delta_i from dX_{i+1}, delta_{i+1} from dX_{i+2}).  A pair the
  // paired kernel does not cover runs as two launches in the same order.
  auto run_single = [&](const PairOp& o, const char* lbl, std::pair<double, double> cost) -> bool {
    if (o.kind == PAIR_NARROW_DW) {
      VOLTA_CHECK(launch_narrow_dw(o.nd, st));
      VOLTA_CHECK(mark(rec, lbl, cost.first, cost.second));
      return true;
    }
    VOLTA_CHECK(gemm_launch(o.plan, o.args, st, rec, lbl, cost.second));
    return true;
  };
  auto run_pair = [&](const PairOp& x, const char* lx, std::pair<double, double> cx, const PairOp& y,
                      const char* ly, std::pair<double, double> cy) -> bool {
    if (h->pair_backward && pair_supported(x, y)) {
      std::snprintf(label, sizeof label, "%s|%s", lx, ly);
      VOLTA_CHECK(pair_launch(x, y, st, rec, label, cx.first + cy.first, cx.second + cy.second));
      return true;
    }
    return run_single(x, lx, cx) && run_single(y, ly, cy);
  };
  char lx[32], ly[32];
  float* ws0 = h->gemm_ws;
  float* ws1 = h->gemm_ws ? h->gemm_ws + h->ws_half : nullptr;
  if (h->extras()) {
    // Codegen extras (:824-892, :936-955).  Phase 1, i = n-1 .. 0: the
    // hidden layer's LayerNorm backward, dropout mask and f' (its dX ran
    // with the identity derivative), b_i from db_i when clipping (db comes
    // from the unscaled deltas), dX_i.  Then the clip scales every delta,
    // and phase 2 runs dW_i (W_i only when clipping).  No paired launches:
    // the clip needs every delta before the first dW.
    const int dx_act = h->hidden_ext() ? kIdentity : s.activation;
    for (int i = n - 1; i >= 0; --i) {
      const LayerPlan& lp = h->layers[i];
      if (i != n - 1 && h->hidden_ext()) {
        HiddenBwdArgs a{};
        a.delta = h->delta[i];
        a.act = h->act[i + 1];
        a.pre = h->pre[i];
        a.B = B;
        a.c = lp.c;
        a.act_kind = s.activation;
        if (h->ext_ln) {
          a.gamma = h->ln_g[i];
          a.beta = h->ln_b[i];
          a.inv_std = h->ln_is[i];
          a.dgamma = h->ln_dg[i];
          a.dbeta = h->ln_db[i];
        }
        if (h->ext_drop) {
          a.mask = h->mask[i];
          a.keep_scale = 1.0f / (1.0f - s.dropout_p);
        }
        VOLTA_CHECK(launch_hidden_bwd(a, h->ext_ln ? h->ln_g[i] : nullptr, h->ext_ln ? h->ln_b[i] : nullptr,
                                      h->scalars, st));
        std::snprintf(lx, sizeof lx, "bwd%d.ln_dropout", i);
        VOLTA_CHECK(mark(rec, lx, 0.0, 4.0 * 5.0 * B * lp.c));
      }
      if (h->ext_clip) {
        EpiArgs e{};
        e.opt = s.optimizer == VOLTA_OPT_ADAMW ? VOLTA_OPT_ADAM : s.optimizer;
        e.b = h->params + lp.b_off;
        e.bm = h->opt_a ? h->opt_a + lp.b_off : nullptr;
        e.bv = h->opt_b ? h->opt_b + lp.b_off : nullptr;
        e.bgrad = h->keep_grads ? h->grads + lp.b_off : nullptr;
        e.b1 = s.beta1;
        e.b2 = s.beta2;
        e.eps = s.eps;
        e.scalars = h->scalars;
        VOLTA_CHECK(launch_bias_update(e, h->delta[i], B, lp.c, st));
        std::snprintf(lx, sizeof lx, "db%d+opt", i);
        VOLTA_CHECK(mark(rec, lx, (double)B * lp.c, 4.0 * B * lp.c));
      }
      if (i == 0) break;
      std::snprintf(lx, sizeof lx, "dx%d", i);
      if (i == n - 1 && h->narrow_dx) {
        VOLTA_CHECK(launch_outer_dx(h->delta[i], h->params + lp.w_off, B, lp.r, lp.c, dx_act, h->act[i],
                                    h->pre[i - 1], h->delta[i - 1], st));
        VOLTA_CHECK(mark(rec, lx, dx_cost(i).first, dx_cost(i).second));
      } else {
        PairOp o = make_dx(i, ws0);
        o.args.epi.act = dx_act;
        if (!run_single(o, lx, dx_cost(i))) return false;
      }
    }
    if (h->ext_clip) {
      ClipArgs c{};
      c.n = n;
      for (int i = 0; i < n; ++i) {
        c.delta[i] = h->delta[i];
        c.count[i] = (int64_t)B * h->L[i + 1];
      }
      c.clip = s.clip_grad;
      c.partials = h->clip_partials;
      c.scalars = h->scalars;
      VOLTA_CHECK(launch_clip(c, st));
      double cnt = 0.0;
      for (int i = 0; i < n; ++i) cnt += (double)B * h->L[i + 1];
      VOLTA_CHECK(mark(rec, "clip", 3.0 * cnt, 12.0 * cnt));
    }
    // phase 2: every dW (W only when clipping: b_i took its update above)
    auto ext_dw = [&](int i) {
      PairOp o = make_dw(i, ws0);
      if (h->ext_clip) {
        o.args.colsum_b = 0;
        o.args.epi.b = nullptr;
        o.nd.b = nullptr;
      }
      return o;
    };
    if (h->ext_dw_group) {
      DwGroup d;
      std::string lab;
      double fl = 0.0, by = 0.0;
      for (int i = n - 1; i >= 0; --i) {
        const PairOp o = ext_dw(i);
        if (o.kind == PAIR_NARROW_DW) {
          d.nd = o.nd;
          d.narrow_blocks = (o.nd.R + kNarrowRows - 1) / kNarrowRows;
        } else {
          d.g[d.n] = o.args;
          d.g[d.n].k_per_split = o.plan.k_per_split;
          ++d.n;
        }
        std::snprintf(lx, sizeof lx, h->ext_clip ? "dw%d+opt" : "dw%d+db+opt", i);
        lab += (lab.empty() ? "" : "|") + std::string(lx);
        fl += dw_cost(i).first;
        by += dw_cost(i).second;
      }
      set_group_width(h, d, 1);
      if (dw_group_supported(d)) {
        VOLTA_CHECK(dw_group_launch(d, st, rec, lab.c_str(), fl, by));
        return true;
      }
    }
    for (int i = n - 1; i >= 0; --i) {
      std::snprintf(lx, sizeof lx, h->ext_clip ? "dw%d+opt" : "dw%d+db+opt", i);
      if (!run_single(ext_dw(i), lx, dw_cost(i))) return false;
    }
    return true;
  }
  // dX_{n-1} (already formed by the output launch when merged)
  if (n > 1 && !h->out_dx_merged) {
    const int i = n - 1;
    const LayerPlan& lp = h->layers[i];
    std::snprintf(lx, sizeof lx, "dx%d", i);
    if (h->narrow_dx) {
      LossDefer ld;
      if (h->out_mfma) {  // the step's loss from the output launch's strip partials
        ld.partials = h->loss_partials;
        ld.blocks = (B + 15) / 16;
        ld.denom = s.loss == VOLTA_LOSS_MSE ? (float)(B * Ln) : (float)B;
        ld.scalars = h->scalars;
      }
      VOLTA_CHECK(launch_outer_dx(h->delta[i], h->params + lp.w_off, B, lp.r, lp.c, s.activation, h->act[i],
                                  h->pre[i - 1], h->delta[i - 1], st, ld));
      VOLTA_CHECK(mark(rec, lx, dx_cost(i).first, dx_cost(i).second));
    } else if (!run_single(make_dx(i, ws0), lx, dx_cost(i))) {
      return false;
    }
  }
  if (h->dx_alone) {
    // Small-batch step: the dX chain alone (each on its grid's wave count),
    // then every dW product in one launch -- dW_i only needs act_i and
    // delta_i, and dX_i has read W_i before that launch updates it.
    for (int i = n - 2; i >= 1; --i) {
      if (i == n - 2 && tail) continue;  // ran with the output launch
      std::snprintf(lx, sizeof lx, "dx%d", i);
      if (!run_single(make_dx(i, ws0), lx, dx_cost(i))) return false;
    }
    if (group_ok) {
      VOLTA_CHECK(dw_group_launch(group, st, rec, group_label.c_str(), group_fl, group_by));
      return true;
    }
    // one launch each (VOLTA_NO_PAIR, or a narrow dW whose staged deltas
    // exceed the small-K tile's LDS)
    for (int i = n - 1; i >= 0; --i) {
      std::snprintf(lx, sizeof lx, "dw%d+db+opt", i);
      if (!run_single(make_dw(i, ws0), lx, dw_cost(i))) return false;
    }
    return true;
  }
  for (int i = n - 2; i >= 1; --i) {
    std::snprintf(lx, sizeof lx, "dx%d", i);
    std::snprintf(ly, sizeof ly, "dw%d+db+opt", i + 1);
    if (!run_pair(make_dx(i, ws0), lx, dx_cost(i), make_dw(i + 1, ws1), ly, dw_cost(i + 1))) return false;
  }
  if (n > 1) {
    std::snprintf(lx, sizeof lx, "dw%d+db+opt", 1);
    std::snprintf(ly, sizeof ly, "dw%d+db+opt", 0);
    if (!run_pair(make_dw(1, ws0), lx, dw_cost(1), make_dw(0, ws1), ly, dw_cost(0))) return false;
  } else {
    if (!run_single(make_dw(0, ws0), "dw0+db+opt", dw_cost(0))) return false;
  }
  return true;
}

// Adam bias-correction table: entry t = (1 - b1^t, 1 - b2^t) in f32 powf,
// up to the first t where both round to exactly 1.0f (later steps use the
// last entry, which is then exact).  (Re)allocated whenever beta1/beta2 are
// set; the caller has synchronized the stream.
static bool make_bc_table(Handle* h) {
  const volta_mlp_spec& s = h->spec;
  if (h->bc_table) {
    VOLTA_CHECK(hipFree(h->bc_table));
    h->bc_table = nullptr;
    h->bc_len = 0;
  }
  if (s.optimizer != VOLTA_OPT_ADAM && s.optimizer != VOLTA_OPT_ADAMW) return true;
  std::vector<float2> bc;
  bc.push_back(make_float2(1.0f, 1.0f));  // t = 0 is never used
  const int kMaxTable = 1 << 24;
  for (int t = 1; t < kMaxTable; ++t) {
    const float b1 = 1.0f - powf(s.beta1, (float)t);
    const float b2 = 1.0f - powf(s.beta2, (float)t);
    bc.push_back(make_float2(b1, b2));
    if (b1 == 1.0f && b2 == 1.0f) break;
  }
  VOLTA_CHECK(hipMalloc((void**)&h->bc_table, bc.size() * sizeof(float2)));
  VOLTA_CHECK(hipMemcpy(h->bc_table, bc.data(), bc.size() * sizeof(float2), hipMemcpyHostToDevice));
  h->bc_len = (int)bc.size();
  return true;
}

// Capture the step into a fresh graph (hyperparameters are kernel
// arguments, so a change of them is a new capture).
static bool capture(Handle* h) {
  if (h->exec) {
    VOLTA_CHECK(hipGraphExecDestroy(h->exec));
    h->exec = nullptr;
  }
  if (h->graph) {
    VOLTA_CHECK(hipGraphDestroy(h->graph));
    h->graph = nullptr;
  }
  if (!h->use_graph) return true;
  VOLTA_CHECK(hipStreamBeginCapture(h->stream, hipStreamCaptureModeThreadLocal));
  const bool ok = enqueue_step(h, h->stream);
  hipGraph_t g = nullptr;
  const hipError_t e = hipStreamEndCapture(h->stream, &g);
  if (!ok) {
    if (g) (void)hipGraphDestroy(g);
    return false;
  }
  VOLTA_CHECK(e);
  h->graph = g;
  VOLTA_CHECK(hipGraphInstantiate(&h->exec, h->graph, nullptr, nullptr, 0));
  return true;
}

// ---------------------------------------------------------------------------
// Static scratch for the allocation-free inference entry point
// (volta_train_infer_device_noalloc): the split-K partial planes of its
// forward products.  Every GPU the library runs on holds its own copy of
// the array from module load until the process ends.  In host code
// `scratch` names a host-side stand-in, not a device address: the device
// address of each GPU's copy comes from hipGetSymbolAddress, taken once per
// device (at volta_train_init on that device, with it current) and kept in
// g_scratch_dev.
// ---------------------------------------------------------------------------
constexpr size_t kScratchFloats = size_t(16) << 20;  // 64 MiB
static __device__ __align__(256) float scratch[kScratchFloats];

static std::mutex g_scratch_mu;
static std::vector<float*> g_scratch_dev;  // device address per device ordinal (null until taken)

// Device address of `dev`'s scratch copy; `dev` must be the current device.
static float* scratch_address(int dev) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (dev < 0) return nullptr;
  if ((int)g_scratch_dev.size() <= dev) g_scratch_dev.resize(dev + 1, nullptr);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_last_error(hip_msg("hipGetSymbolAddress(scratch)", e));
      return nullptr;
    }
    g_scratch_dev[dev] = static_cast<float*>(p);
  }
  return g_scratch_dev[dev];
}

static bool build(Handle* h) {
  const volta_mlp_spec& s = h->spec;
  const int n = h->n, B = h->B;
  VOLTA_CHECK(hipGetDevice(&h->device));
  VOLTA_CHECK(hipDeviceGetAttribute(&h->num_cus, hipDeviceAttributeMultiprocessorCount, h->device));
  h->scratch = scratch_address(h->device);  // null: the allocation-free entry point reports it
  VOLTA_CHECK(hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking));
  const char* kg = std::getenv("VOLTA_KEEP_GRADS");
  h->keep_grads = kg && *kg && *kg != '0';
  h->ext_ln = s.layernorm != 0 && n > 1;
  h->ext_drop = s.dropout_p > 0.0f && n > 1;
  h->ext_clip = s.clip_grad > 0.0f;
  h->ext_softmax = s.activation == VOLTA_ACT_SOFTMAX && n > 1;

  // Flat parameter layout [W0 | b0 | W1 | b1 | ...], segments padded.
  h->layers.resize(n);
  int64_t off = 0;
  h->segs.n = 2 * n;
  for (int i = 0; i < n; ++i) {
    LayerPlan& lp = h->layers[i];
    lp.r = h->L[i];
    lp.c = h->L[i + 1];
    lp.w_off = off;
    off += align_up((size_t)lp.r * lp.c, kSegAlign);
    lp.b_off = off;
    off += align_up((size_t)lp.c, kSegAlign);
    h->segs.off[2 * i] = lp.w_off;
    h->segs.count[2 * i] = (int64_t)lp.r * lp.c;
    h->segs.wd[2 * i] = s.optimizer == VOLTA_OPT_ADAMW ? s.weight_decay : 0.0f;
    h->segs.off[2 * i + 1] = lp.b_off;
    h->segs.count[2 * i + 1] = lp.c;
    h->segs.wd[2 * i + 1] = 0.0f;  // the generated step never decays biases (:966)
  }
  h->flat = off;

  // GEMM plans.  Vector (16-byte) operand loads need the contiguous extent
  // and leading dimension to be multiples of 4 floats.  The output layer's
  // loss head runs in its GEMM when the layer fits one 64-wide tile.
  const int Ln = h->L[n];
  h->out_mode = Ln <= 16 ? OUT_NARROW : Ln <= 64 ? OUT_GEMM_LOSS : OUT_GEMM;
  h->narrow_dx = Ln <= 16 && n > 1;
  const char* nod = std::getenv("VOLTA_NO_OUT_DX");
  h->out_dx_merged = h->narrow_dx && !h->extras() && !(nod && *nod && *nod != '0') &&
                     out_layer_dx_supported(B, h->L[n - 1], Ln);
  // Opt-in: its per-workgroup release fence costs more than the launch it
  // saves on C2/C3 (0.0613 -> 0.0643, 0.1035 -> 0.1096 ms), less on C1
  // (0.0402 -> 0.0384 ms).
  const char* fh = std::getenv("VOLTA_FWD_HEAD");
  h->fwd_head = h->out_dx_merged && Ln == 1 && fh && *fh && *fh != '0';
  const char* nt = std::getenv("VOLTA_NO_TAIL");
  h->tail_merge = h->out_dx_merged && !h->fwd_head && Ln == 1 && n >= 3 && !(nt && *nt && *nt != '0');
  h->narrow_dw = Ln <= 16 && B <= kNarrowMaxB;
  // A narrow output layer of more rows than the one-launch output kernels
  // take (C5: 4096 rows of 10 classes) runs on MFMA, one 16-row strip per
  // 16-wave small-M workgroup, with each row's loss head after the product;
  // the strips' loss partials are added by the outer-product dX_{n-1}
  // launch that follows (no loss launch of its own).  The wave dot
  // products of out_layer_kernel plus the loss launch took 28.7 us at C5.
  // VOLTA_OUT_MFMA=0 keeps them.
  const char* om = std::getenv("VOLTA_OUT_MFMA");
  h->out_mfma = h->out_mode == OUT_NARROW && !h->extras() && h->narrow_dx && !h->out_dx_merged &&
                out_layer_blocks(B) > 1 && !(om && *om == '0');
  size_t ws_floats = 0;
  int max_tiles = 1;
  for (int i = 0; i < n; ++i) {
    LayerPlan& lp = h->layers[i];
    const bool vr = lp.r % 4 == 0, vc = lp.c % 4 == 0;
    const bool loss_gemm = i == n - 1 && h->out_mode == OUT_GEMM_LOSS;
    lp.fwd = gemm_plan(GEMM_NN, B, lp.c, lp.r, vr && vc, h->num_cus, !loss_gemm);
    if (loss_gemm) lp.fwd.tile = TILE_64x64;
    lp.dx = gemm_plan(GEMM_NT, B, lp.r, lp.c, vc, h->num_cus);
    lp.dw = gemm_plan(GEMM_TN, lp.r, lp.c, B, vr && vc, h->num_cus);
    ws_floats = std::max(ws_floats, lp.fwd.workspace_floats(B, lp.c));
    if (i > 0) ws_floats = std::max(ws_floats, lp.dx.workspace_floats(B, lp.r));
    ws_floats = std::max(ws_floats, lp.dw.workspace_floats(lp.r, lp.c));
    max_tiles = std::max(max_tiles, lp.fwd.tiles(B, lp.c));
    max_tiles = std::max(max_tiles, lp.dx.tiles(B, lp.r));
    max_tiles = std::max(max_tiles, lp.dw.tiles(lp.r, lp.c));
  }
  h->n_counters = max_tiles + 1;  // last one: the loss head's tile counter
  const char* np = std::getenv("VOLTA_NO_PAIR");
  h->pair_backward = !(np && *np && *np != '0') && !h->extras();
  // Small-batch backward (every dW on the small-K tile, the output layer's
  // possibly narrow): the dX products run alone with their grid's wave
  // count, and the dW products share one launch after them (VOLTA_NO_PAIR:
  // one launch each, same plans, same bits).
  int n_small = 0;
  bool all_small = n >= 2;
  for (int i = 0; i < n; ++i) {
    if (i == n - 1 && h->narrow_dw) continue;
    all_small = all_small && h->layers[i].dw.tile == TILE_DW_SMALLK;
    ++n_small;
  }
  h->dx_alone = !h->extras() && all_small && n_small <= kMaxDwGroup;
  h->dw_group = h->dx_alone && h->pair_backward;
  // The extras step runs its dX products alone anyway and its dW products
  // after every delta: those share one launch under the same conditions.
  h->ext_dw_group = h->extras() && all_small && n_small <= kMaxDwGroup && !(np && *np && *np != '0');
  const char* gtn = std::getenv("VOLTA_DW_GROUP_TN");
  if (gtn && *gtn) h->dw_group_tn = std::atoi(gtn) == 64 ? 64 : 32;
  else h->dw_group_tn = 0;
  if (h->dx_alone || h->ext_dw_group)
    for (int i = 1; i < n; ++i) {
      LayerPlan& lp = h->layers[i];
      if (lp.dx.tile == TILE_SMALLM) lp.dx.waves = gemm_smallm_waves(false, B, lp.r, h->num_cus);
    }
  // Opt-in (VOLTA_FWD_SPLIT=1): a hidden forward product on the 16-wave
  // small-M tile whose grid has at most half a workgroup per CU and a K of
  // at least 512, followed by another hidden forward product on the 16-wave
  // small-M tile, runs its two halves of K as two workgroups each (twice the
  // CUs, half the K each) into two partial planes of the workspace, and the
  // next launch adds them, the bias and the activation as it loads its A
  // operand and stores the layer's output (C2's fwd2 into fwd3, C1's fwd1
  // into fwd2).  Where the halves are whole wave ranges of the one-launch
  // product (K a power-of-two multiple of 512: C1, C2) the sums are the same
  // tree, so the bits are too.  Slower: the halves save 1.6 us of C2's fwd2,
  // and forming the A operand from the planes costs fwd3 2.1 us (C2 50.3 ->
  // 51.2 us, C1 28.6 -> 30.1).  Not with the codegen extras (their row
  // kernels run between the forward launches) or into the opt-in head
  // launch.
  h->fwd_khalf.assign(n, 0);
  const char* fsp = std::getenv("VOLTA_FWD_SPLIT");
  if (!h->extras() && fsp && *fsp && *fsp != '0')
    for (int i = 0; i + 2 < n; ++i) {
      if ((i > 0 && h->fwd_khalf[i - 1]) || (i + 1 == n - 2 && h->fwd_head)) continue;
      const LayerPlan& pl = h->layers[i];
      const LayerPlan& cl = h->layers[i + 1];
      const int tiles = pl.fwd.tiles(B, pl.c);
      if (pl.fwd.tile == TILE_SMALLM && pl.fwd.vec && pl.fwd.waves == 16 && pl.r >= 512 &&
          2 * tiles <= h->num_cus && cl.fwd.tile == TILE_SMALLM && cl.fwd.vec && cl.fwd.waves == 16) {
        h->fwd_khalf[i] = (pl.r / 2 + 15) / 16 * 16;
        ws_floats = std::max(ws_floats, (size_t)2 * B * pl.c);
      }
    }
  ws_floats = align_up(ws_floats, 64);
  h->ws_half = ws_floats;
  ws_floats *= 2;

  const bool adam = s.optimizer == VOLTA_OPT_ADAM || s.optimizer == VOLTA_OPT_ADAMW;

  // One arena, 256-byte aligned sub-buffers.
  struct Req {
    void** dst;
    size_t bytes;
  };
  std::vector<Req> reqs;
  auto req = [&](void** dst, size_t bytes) { reqs.push_back({dst, align_up(std::max<size_t>(bytes, 4), 256)}); };
  req((void**)&h->scalars, sizeof(DevScalars));
  req((void**)&h->params, (size_t)h->flat * 4);
  if (h->keep_grads) req((void**)&h->grads, (size_t)h->flat * 4);
  if (adam || s.optimizer == VOLTA_OPT_ADAGRAD) req((void**)&h->opt_a, (size_t)h->flat * 4);
  if (adam) req((void**)&h->opt_b, (size_t)h->flat * 4);
  h->act.assign(n + 1, nullptr);
  h->pre.assign(n, nullptr);
  h->delta.assign(n, nullptr);
  // the targets right after act_0, 256-byte aligned, with the same gap as in
  // the pinned staging buffer: a host-staged step copies both in one transfer
  req((void**)&h->act[0], (size_t)B * h->L[0] * 4);
  req(&h->target, s.loss == VOLTA_LOSS_MSE ? (size_t)B * h->L[n] * 4 : (size_t)B * 4);
  for (int i = 1; i <= n; ++i) req((void**)&h->act[i], (size_t)B * h->L[i] * 4);
  for (int i = 0; i < n - 1; ++i)
    if (act_needs_pre(s.activation) || h->hidden_ext()) req((void**)&h->pre[i], (size_t)B * h->L[i + 1] * 4);
  h->ln_g.assign(n, nullptr);
  h->ln_b.assign(n, nullptr);
  h->ln_mu.assign(n, nullptr);
  h->ln_is.assign(n, nullptr);
  h->ln_dg.assign(n, nullptr);
  h->ln_db.assign(n, nullptr);
  h->mask.assign(n, nullptr);
  for (int i = 0; i < n - 1; ++i) {
    const size_t c = h->L[i + 1];
    if (h->ext_ln) {
      req((void**)&h->ln_g[i], c * 4);
      req((void**)&h->ln_b[i], c * 4);
      req((void**)&h->ln_mu[i], (size_t)B * 4);
      req((void**)&h->ln_is[i], (size_t)B * 4);
      req((void**)&h->ln_dg[i], c * 4);
      req((void**)&h->ln_db[i], c * 4);
    }
    if (h->ext_drop) req((void**)&h->mask[i], (size_t)B * c);
  }
  if (h->ext_clip) req((void**)&h->clip_partials, kClipBlocks * 4);
  for (int i = 0; i < n; ++i) req((void**)&h->delta[i], (size_t)B * h->L[i + 1] * 4);
  if (ws_floats) req((void**)&h->gemm_ws, ws_floats * 4);
  req((void**)&h->counters, (size_t)h->n_counters * sizeof(unsigned));
  req((void**)&h->loss_partials,
      (size_t)std::max({(B + 63) / 64, out_layer_blocks(B), out_layer_dx_blocks(B)}) * 4);
  size_t total = 0;
  for (auto& r : reqs) total += r.bytes;
  h->arena_bytes = total;
  VOLTA_CHECK(hipMalloc((void**)&h->arena, total));
  VOLTA_CHECK(hipMemsetAsync(h->arena, 0, total, h->stream));
  size_t pos = 0;
  for (auto& r : reqs) {
    *r.dst = h->arena + pos;
    pos += r.bytes;
  }
  if (!make_bc_table(h)) return false;

  // Host side: pinned parameter mirror, input staging, lr slots.
  VOLTA_CHECK(hipHostMalloc((void**)&h->h_params, (size_t)h->flat * 4, hipHostMallocDefault));
  // [X | gap | Y], laid out as act_0 and the targets are in the arena
  h->stage_y_off = align_up((size_t)B * h->L[0] * 4, 256);
  VOLTA_CHECK(hipHostMalloc((void**)&h->h_stage_x, h->stage_y_off + (size_t)B * std::max(h->L[n], 1) * 4,
                            hipHostMallocDefault));
  h->h_stage_y = reinterpret_cast<char*>(h->h_stage_x) + h->stage_y_off;
  VOLTA_CHECK(hipHostMalloc((void**)&h->h_lr, Handle::kLrSlots * sizeof(float), hipHostMallocDefault));
  VOLTA_CHECK(hipEventCreateWithFlags(&h->stage_free, hipEventDisableTiming));
  for (auto& e : h->lr_ev) VOLTA_CHECK(hipEventCreateWithFlags(&e, hipEventDisableTiming));

  // Reference init: LCG Xavier-uniform W from one stream seeded 42, b = 0.
  std::memset(h->h_params, 0, (size_t)h->flat * 4);
  uint64_t rng = 42;
  for (int i = 0; i < n; ++i) {
    const LayerPlan& lp = h->layers[i];
    lcg_xavier_init(h->h_params + lp.w_off, (size_t)lp.r * lp.c, lp.r, lp.c, &rng);
  }
  VOLTA_CHECK(hipMemcpyAsync(h->params, h->h_params, (size_t)h->flat * 4, hipMemcpyHostToDevice, h->stream));
  // Extras state: gamma = 1, beta = 0 (:660-668); dropout LCG seed (:553).
  std::vector<float> ones(h->ext_ln ? (size_t)*std::max_element(h->L.begin(), h->L.end()) : 0, 1.0f);
  const uint64_t seed = 12345678ULL;
  for (int i = 0; i < n - 1 && h->ext_ln; ++i)
    VOLTA_CHECK(hipMemcpyAsync(h->ln_g[i], ones.data(), (size_t)h->L[i + 1] * 4, hipMemcpyHostToDevice, h->stream));
  VOLTA_CHECK(hipMemcpyAsync(&h->scalars->rng, &seed, sizeof seed, hipMemcpyHostToDevice, h->stream));
  VOLTA_CHECK(hipStreamSynchronize(h->stream));

  // The step's launches are enqueued directly by default: the same fixed
  // sequence, and on this GPU faster than replaying it from a captured
  // hipGraph in either of HIP's graph dispatch modes (C2 51.0 us per step
  // against 52.4 with in-order node dispatch and 56.7 with HIP's default
  // recorded packets; C1 28.7 against 30.7 / 33.5; C5 alike).
  // VOLTA_GRAPH=1 captures the sequence once and replays it.
  const char* eg = std::getenv("VOLTA_GRAPH");
  const char* ng = std::getenv("VOLTA_NO_GRAPH");
  h->use_graph = eg && *eg && *eg != '0' && !(ng && *ng && *ng != '0');
  return capture(h);
}

// Plans of the forward products for `rows` <= B rows (a smaller M may split
// K where the step's plan did not); returns the split-K workspace they need
// in floats.
static size_t forward_plans(const Handle* h, int rows, std::vector<GemmPlan>* plans) {
  plans->assign(h->n, GemmPlan{});
  size_t ws = 0;
  for (int i = 0; i < h->n; ++i) {
    const LayerPlan& lp = h->layers[i];
    (*plans)[i] = gemm_plan(GEMM_NN, rows, lp.c, lp.r, lp.fwd.vec, h->num_cus);
    (*plans)[i].inkernel_reduce = false;
    ws = std::max(ws, (*plans)[i].workspace_floats(rows, lp.c));
  }
  return ws;
}

// Forward pass only for `rows` <= B rows of `x` (device, [rows x L0]):
// hidden layers as in the step (bias + activation epilogue, or the split-K
// reduction through `ws`, then LayerNorm when the spec has it; dropout is a
// training-only transform) into the handle's activations, the output layer
// with the identity into `out` (device, [rows x Ln]).
static bool enqueue_forward_into(Handle* h, const std::vector<GemmPlan>& plans, int rows, const float* x, float* out,
                                 float* ws, hipStream_t st) {
  const int n = h->n;
  for (int i = 0; i < n; ++i) {
    const LayerPlan& lp = h->layers[i];
    const bool last = i == n - 1;
    GemmArgs a{};
    a.partial = ws;
    a.counters = h->counters;
    a.epi.scalars = h->scalars;
    a.A = i == 0 ? x : h->act[i];
    a.lda = lp.r;
    a.B = h->params + lp.w_off;
    a.ldb = lp.c;
    a.M = rows;
    a.N = lp.c;
    a.K = lp.r;
    a.epi.kind = EPI_BIAS_ACT;
    a.epi.act = last || h->infer_linear ? kIdentity : h->gemm_act();
    a.epi.ldc = lp.c;
    a.epi.out = last ? out : h->act[i + 1];
    a.epi.bias = h->params + lp.b_off;
    VOLTA_CHECK(gemm_launch(plans[i], a, st));
    if (!last && (h->ext_ln || h->ext_softmax))
      VOLTA_CHECK(launch_hidden_fwd(hidden_fwd_args(h, i, rows, false), st));
  }
  return true;
}

// The same for rows already in h->infer_x, result in act[n]; the handle's
// inference workspace grows (hipMalloc) when a plan needs more.
static bool enqueue_forward(Handle* h, int rows, hipStream_t st) {
  std::vector<GemmPlan> plans;
  const size_t ws = forward_plans(h, rows, &plans);
  if (ws > h->infer_ws_floats) {
    VOLTA_CHECK(hipStreamSynchronize(st));
    if (h->infer_ws) VOLTA_CHECK(hipFree(h->infer_ws));
    h->infer_ws = nullptr;
    h->infer_ws_floats = 0;
    VOLTA_CHECK(hipMalloc((void**)&h->infer_ws, ws * sizeof(float)));
    h->infer_ws_floats = ws;
  }
  return enqueue_forward_into(h, plans, rows, h->infer_x, h->act[h->n], h->infer_ws, st);
}

static void fail(Handle* h, int bits, const std::string& msg) {
  if (h) h->status |= bits;
  set_last_error(msg);
}

// Make the device learning rate equal `lr` for the next step.  A change is
// uploaded from a pinned slot; a slot is reused only after its copy ran.
static bool set_lr(Handle* h, float lr) {
  if (h->lr_known && std::memcmp(&lr, &h->cur_lr, 4) == 0) return true;
  const int slot = h->lr_slot;
  h->lr_slot = (slot + 1) % Handle::kLrSlots;
  if (h->lr_pending[slot]) VOLTA_CHECK(hipEventSynchronize(h->lr_ev[slot]));
  h->h_lr[slot] = lr;
  VOLTA_CHECK(hipMemcpyAsync(&h->scalars->lr, &h->h_lr[slot], sizeof(float), hipMemcpyHostToDevice, h->stream));
  VOLTA_CHECK(hipEventRecord(h->lr_ev[slot], h->stream));
  h->lr_pending[slot] = true;
  h->cur_lr = lr;
  h->lr_known = true;
  return true;
}

static bool launch_step(Handle* h) {
  if (h->use_graph) {
    VOLTA_CHECK(hipGraphLaunch(h->exec, h->stream));
    return true;
  }
  return enqueue_step(h, h->stream);
}

// Stage host inputs through pinned memory so the caller may reuse X/Y at once.
static bool stage_inputs(Handle* h, const float* X, const void* Y, size_t ybytes) {
  const size_t xbytes = (size_t)h->B * h->L[0] * 4;
  VOLTA_CHECK(hipEventSynchronize(h->stage_free));
  std::memcpy(h->h_stage_x, X, xbytes);
  std::memcpy(h->h_stage_y, Y, ybytes);
  // act_0 and the targets are adjacent in the arena as in the staging buffer
  // (the gap is copied too): one host-to-device transfer per step
  if (static_cast<char*>(h->target) != reinterpret_cast<char*>(h->act[0]) + h->stage_y_off) return false;
  VOLTA_CHECK(hipMemcpyAsync(h->act[0], h->h_stage_x, h->stage_y_off + ybytes, hipMemcpyHostToDevice, h->stream));
  VOLTA_CHECK(hipEventRecord(h->stage_free, h->stream));
  return true;
}

static bool sync(Handle* h) {
  VOLTA_CHECK(hipStreamSynchronize(h->stream));
  return true;
}

}  // namespace volta

using volta::Handle;
using volta::set_last_error;

static Handle* H(VoltaTrainHandle* h) { return reinterpret_cast<Handle*>(h); }

extern "C" {

VoltaTrainHandle* volta_train_init_spec(const volta_mlp_spec* spec, int32_t batch) {
  std::string why;
  if (!spec || !volta::validate_spec(*spec, &why)) {
    set_last_error("volta_train_init_spec: invalid spec: " + why);
    return nullptr;
  }
  if (batch <= 0 || batch > (1 << 24)) {
    set_last_error("volta_train_init_spec: batch must be in [1, 16777216]");
    return nullptr;
  }
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0) {
    set_last_error("volta_train_init_spec: no HIP device");
    return nullptr;
  }
  std::unique_ptr<Handle> h(new (std::nothrow) Handle());
  if (!h) {
    set_last_error("volta_train_init_spec: out of host memory");
    return nullptr;
  }
  h->spec = *spec;
  h->B = batch;
  h->n = spec->n_sizes - 1;
  h->L.assign(spec->sizes, spec->sizes + spec->n_sizes);
  if (!volta::build(h.get())) return nullptr;
  return reinterpret_cast<VoltaTrainHandle*>(h.release());
}

VoltaTrainHandle* volta_train_init(int32_t batch) {
  volta_mlp_spec s;
  if (!volta::resolve_default_spec(&s)) return nullptr;
  return volta_train_init_spec(&s, batch);
}

void volta_train_step(VoltaTrainHandle* vh, const float* X, const float* Y, float lr) {
  Handle* h = H(vh);
  if (!h) return;
  if (!X || !Y || h->spec.loss != VOLTA_LOSS_MSE) {
    volta::fail(h, VOLTA_STATUS_BAD_ARGUMENT, "volta_train_step: null input or spec loss is not MSE");
    return;
  }
  if (!volta::stage_inputs(h, X, Y, (size_t)h->B * h->L[h->n] * 4) || !volta::set_lr(h, lr) ||
      !volta::launch_step(h))
    h->status |= VOLTA_STATUS_DEVICE_ERROR;
}

void volta_train_step_labels(VoltaTrainHandle* vh, const float* X, const int32_t* labels, float lr) {
  Handle* h = H(vh);
  if (!h) return;
  if (!X || !labels || h->spec.loss != VOLTA_LOSS_SOFTMAX_CE) {
    volta::fail(h, VOLTA_STATUS_BAD_ARGUMENT,
                "volta_train_step_labels: null input or spec loss is not softmax-CE");
    return;
  }
  const int C = h->L[h->n];
  for (int i = 0; i < h->B; ++i)
    if (labels[i] < 0 || labels[i] >= C) {
      volta::fail(h, VOLTA_STATUS_BAD_ARGUMENT, "volta_train_step_labels: label out of range");
      return;
    }
  if (!volta::stage_inputs(h, X, labels, (size_t)h->B * 4) || !volta::set_lr(h, lr) || !volta::launch_step(h))
    h->status |= VOLTA_STATUS_DEVICE_ERROR;
}

int32_t volta_train_step_device(VoltaTrainHandle* vh, const float* X, const void* Y, float lr) {
  Handle* h = H(vh);
  if (!h) return -1;
  if (!X || !Y) {
    volta::fail(h, VOLTA_STATUS_BAD_ARGUMENT, "volta_train_step_device: null input");
    return -1;
  }
  const size_t ybytes = h->spec.loss == VOLTA_LOSS_MSE ? (size_t)h->B * h->L[h->n] * 4 : (size_t)h->B * 4;
  bool ok = true;
  if (X != h->act[0])
    ok = ok && hipMemcpyAsync(h->act[0], X, (size_t)h->B * h->L[0] * 4, hipMemcpyDeviceToDevice, h->stream) ==
                   hipSuccess;
  if (Y != h->target)
    ok = ok && hipMemcpyAsync(h->target, Y, ybytes, hipMemcpyDeviceToDevice, h->stream) == hipSuccess;
  ok = ok && volta::set_lr(h, lr) && volta::launch_step(h);
  if (!ok) {
    h->status |= VOLTA_STATUS_DEVICE_ERROR;
    return -1;
  }
  return 0;
}

int32_t volta_train_batch_buffers(VoltaTrainHandle* vh, float** X, void** Y) {
  Handle* h = H(vh);
  if (!h || !X || !Y) return -1;
  *X = h->act[0];
  *Y = h->target;
  return 0;
}

float volta_train_loss(VoltaTrainHandle* vh) {
  Handle* h = H(vh);
  if (!h) return NAN;
  float loss = NAN;
  if (!volta::sync(h) ||
      hipMemcpy(&loss, &h->scalars->loss, sizeof(float), hipMemcpyDeviceToHost) != hipSuccess) {
    h->status |= VOLTA_STATUS_DEVICE_ERROR;
    return NAN;
  }
  return loss;
}

void volta_train_get_params(VoltaTrainHandle* vh, float** wo, float** bo) {
  Handle* h = H(vh);
  if (!h || !wo || !bo) return;
  if (!volta::sync(h) ||
      hipMemcpy(h->h_params, h->params, (size_t)h->flat * 4, hipMemcpyDeviceToHost) != hipSuccess)
    h->status |= VOLTA_STATUS_DEVICE_ERROR;
  for (int i = 0; i < h->n; ++i) {
    wo[i] = h->h_params + h->layers[i].w_off;
    bo[i] = h->h_params + h->layers[i].b_off;
  }
}

void volta_train_set_params(VoltaTrainHandle* vh, int32_t li, const float* w, const float* b) {
  Handle* h = H(vh);
  if (!h) return;
  if (li < 0 || li >= h->n || !w || !b) {
    volta::fail(h, VOLTA_STATUS_BAD_ARGUMENT, "volta_train_set_params: layer index out of range");
    return;
  }
  const volta::LayerPlan& lp = h->layers[li];
  if (!volta::sync(h) ||
      hipMemcpy(h->params + lp.w_off, w, (size_t)lp.r * lp.c * 4, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(h->params + lp.b_off, b, (size_t)lp.c * 4, hipMemcpyHostToDevice) != hipSuccess)
    h->status |= VOLTA_STATUS_DEVICE_ERROR;
}

// The handle bound for volta_infer (volta_infer_bind); cleared when freed.
static std::mutex g_infer_mu;
static VoltaTrainHandle* g_infer_model = nullptr;

void volta_train_free(VoltaTrainHandle* vh) {
  if (!vh) return;
  {
    std::lock_guard<std::mutex> lock(g_infer_mu);
    if (g_infer_model == vh) g_infer_model = nullptr;
  }
  delete H(vh);
}

int32_t volta_train_sync(VoltaTrainHandle* vh) {
  Handle* h = H(vh);
  if (!h) return -1;
  if (!volta::sync(h)) {
    h->status |= VOLTA_STATUS_DEVICE_ERROR;
    return -1;
  }
  return 0;
}

int32_t volta_train_status(VoltaTrainHandle* vh) {
  Handle* h = H(vh);
  if (!h) return VOLTA_STATUS_BAD_ARGUMENT;
  uint32_t dev_flags = 0;
  if (!volta::sync(h) ||
      hipMemcpy(&dev_flags, &h->scalars->flags, sizeof(uint32_t), hipMemcpyDeviceToHost) != hipSuccess)
    h->status |= VOLTA_STATUS_DEVICE_ERROR;
  return h->status | (int32_t)dev_flags;
}

void volta_train_clear_status(VoltaTrainHandle* vh) {
  Handle* h = H(vh);
  if (!h) return;
  h->status = 0;
  const uint32_t zero = 0;
  if (!volta::sync(h) ||
      hipMemcpy(&h->scalars->flags, &zero, sizeof(uint32_t), hipMemcpyHostToDevice) != hipSuccess)
    h->status |= VOLTA_STATUS_DEVICE_ERROR;
}

// Per-kernel profile of the step: runs `reps` steps kernel by kernel on the
// resident batch (they train the model like any other step) with an event
// after every kernel, and writes one line per kernel to `out`:
//   "<label>\t<avg ms>\t<algorithmic flops>\t<algorithmic bytes>\n"
// Returns the number of kernels per step, or -1.
int32_t volta_hip_profile_step(VoltaTrainHandle* vh, int32_t reps, char* out, int32_t out_len) {
  Handle* h = H(vh);
  if (!h || reps <= 0 || !out || out_len <= 0) return -1;
  std::vector<std::string> labels;
  std::vector<double> total_ms, flops, bytes;
  for (int r = 0; r < reps; ++r) {
    volta::Recorder rec;
    rec.st = h->stream;
    if (hipEventCreate(&rec.start) != hipSuccess || hipEventRecord(rec.start, h->stream) != hipSuccess ||
        !volta::enqueue_step(h, h->stream, &rec) || hipStreamSynchronize(h->stream) != hipSuccess) {
      h->status |= VOLTA_STATUS_DEVICE_ERROR;
      return -1;
    }
    if (r == 0) {
      for (auto& m : rec.marks) {
        labels.push_back(m.label);
        flops.push_back(m.flops);
        bytes.push_back(m.bytes);
      }
      total_ms.assign(labels.size(), 0.0);
    }
    hipEvent_t prev = rec.start;
    for (size_t k = 0; k < rec.marks.size() && k < labels.size(); ++k) {
      float ms = 0.0f;
      if (hipEventElapsedTime(&ms, prev, rec.marks[k].ev) != hipSuccess) ms = 0.0f;
      total_ms[k] += ms;
      prev = rec.marks[k].ev;
    }
  }
  std::string text;
  char line[256];
  for (size_t k = 0; k < labels.size(); ++k) {
    std::snprintf(line, sizeof line, "%s\t%.6f\t%.6g\t%.6g\n", labels[k].c_str(), total_ms[k] / reps, flops[k],
                  bytes[k]);
    text += line;
  }
  std::snprintf(out, (size_t)out_len, "%s", text.c_str());
  return (int32_t)labels.size();
}

// Duration of launch `index` of the step: the step's launch sequence is
// enqueued on the handle's stream with an event before and after that
// launch only (the other launches run back to back as in a step), `reps`
// times; the same is done with the two events recorded back to back at that
// position.  Writes the mean bracketed time to avg_ms[0], the mean
// back-to-back (marker) time to avg_ms[1], and the launch's label to
// `label`.  Test and benchmark use.
int32_t volta_hip_time_kernel(VoltaTrainHandle* vh, int32_t index, int32_t reps, float* avg_ms, char* label,
                              int32_t label_len) {
  Handle* h = H(vh);
  if (!h || index < 0 || reps <= 0 || !avg_ms) return -1;
  double total[2] = {0.0, 0.0};
  std::string lab;
  // Every timed step is preceded by about 0.2 ms of ordinary steps (as
  // volta_train_step_device runs them), so the host has enqueued the timed
  // step's launches (a few microseconds of host work each) before the GPU
  // reaches them: the launch then starts when its predecessor ends, as in a
  // run of steps, and its interval holds no host enqueue time, which the
  // back-to-back marker pair would not see.
  int prelude = 1;
  {
    hipEvent_t e0 = nullptr, e1 = nullptr;
    float step_ms = 0.0f;
    const bool ok = hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess &&
                    hipEventRecord(e0, h->stream) == hipSuccess && volta::launch_step(h) &&
                    hipEventRecord(e1, h->stream) == hipSuccess && hipStreamSynchronize(h->stream) == hipSuccess &&
                    hipEventElapsedTime(&step_ms, e0, e1) == hipSuccess;
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (!ok) {
      volta::set_last_error("volta_hip_time_kernel: step timing failed");
      return -1;
    }
    prelude = std::min(8, std::max(1, (int)std::ceil(0.2 / std::max(step_ms, 1e-3f))));
  }
  for (int r = 0; r < 2 * reps; ++r) {
    const bool empty = r % 2 == 1;
    volta::Recorder rec;
    rec.st = h->stream;
    rec.target = index;
    rec.empty = empty;
    float ms = 0.0f;
    for (int k = 0; k < prelude; ++k)
      if (!volta::launch_step(h)) return -1;
    if (hipEventCreate(&rec.before) != hipSuccess || hipEventCreate(&rec.after) != hipSuccess ||
        (index == 0 && hipEventRecord(rec.before, h->stream) != hipSuccess) ||
        (index == 0 && empty && hipEventRecord(rec.after, h->stream) != hipSuccess)) {
      volta::set_last_error("volta_hip_time_kernel: event setup failed");
      return -1;
    }
    if (!volta::enqueue_step(h, h->stream, &rec)) return -1;
    if (rec.count <= index) {
      volta::set_last_error("volta_hip_time_kernel: index beyond the step's launches");
      return -1;
    }
    const hipError_t e0 = hipStreamSynchronize(h->stream);
    const hipError_t e2 = e0 == hipSuccess ? hipEventElapsedTime(&ms, rec.before, rec.after) : e0;
    if (e2 != hipSuccess) {
      volta::set_last_error(std::string("volta_hip_time_kernel: ") + hipGetErrorString(e2));
      return -1;
    }
    total[empty ? 1 : 0] += ms;
    if (!empty) lab = rec.target_label;
  }
  avg_ms[0] = (float)(total[0] / reps);
  avg_ms[1] = (float)(total[1] / reps);
  if (label && label_len > 0) std::snprintf(label, (size_t)label_len, "%s", lab.c_str());
  return 0;
}

int64_t volta_train_debug_buffer(VoltaTrainHandle* vh, int32_t kind, int32_t layer, float* out) {
  Handle* h = H(vh);
  if (!h || !out) return -1;
  const float* src = nullptr;
  size_t count = 0;
  const int n = h->n, B = h->B;
  switch (kind) {
    case VOLTA_BUF_ACT:
      if (layer < 0 || layer > n) return -1;
      src = h->act[layer];
      count = (size_t)B * h->L[layer];
      break;
    case VOLTA_BUF_DELTA:
      if (layer < 0 || layer >= n) return -1;
      src = h->delta[layer];
      count = (size_t)B * h->L[layer + 1];
      break;
    case VOLTA_BUF_GRAD_W:
      if (layer < 0 || layer >= n || !h->keep_grads) return -1;
      src = h->grads + h->layers[layer].w_off;
      count = (size_t)h->layers[layer].r * h->layers[layer].c;
      break;
    case VOLTA_BUF_GRAD_B:
      if (layer < 0 || layer >= n || !h->keep_grads) return -1;
      src = h->grads + h->layers[layer].b_off;
      count = (size_t)h->layers[layer].c;
      break;
    case VOLTA_BUF_PRE:
      if (layer < 0 || layer >= n - 1 || !h->pre[layer]) return -1;
      src = h->pre[layer];
      count = (size_t)B * h->L[layer + 1];
      break;
    case VOLTA_BUF_LN_GAMMA:
    case VOLTA_BUF_LN_BETA:
      if (layer < 0 || layer >= n - 1 || !h->ext_ln) return -1;
      src = kind == VOLTA_BUF_LN_GAMMA ? h->ln_g[layer] : h->ln_b[layer];
      count = (size_t)h->L[layer + 1];
      break;
    case VOLTA_BUF_LN_DGAMMA:
    case VOLTA_BUF_LN_DBETA:
      if (layer < 0 || layer >= n - 1 || !h->ext_ln) return -1;
      src = kind == VOLTA_BUF_LN_DGAMMA ? h->ln_dg[layer] : h->ln_db[layer];
      count = (size_t)h->L[layer + 1];
      break;
    case VOLTA_BUF_CLIP_SCALE:
      if (!h->ext_clip) return -1;
      src = &h->scalars->clip_scale;
      count = 1;
      break;
    case VOLTA_BUF_DROPOUT_MASK: {
      if (layer < 0 || layer >= n - 1 || !h->ext_drop) return -1;
      count = (size_t)B * h->L[layer + 1];
      std::vector<uint8_t> m(count);
      if (!volta::sync(h) || hipMemcpy(m.data(), h->mask[layer], count, hipMemcpyDeviceToHost) != hipSuccess) {
        h->status |= VOLTA_STATUS_DEVICE_ERROR;
        return -1;
      }
      for (size_t k = 0; k < count; ++k) out[k] = (float)m[k];
      return (int64_t)count;
    }
    default:
      return -1;
  }
  if (!volta::sync(h) || hipMemcpy(out, src, count * sizeof(float), hipMemcpyDeviceToHost) != hipSuccess) {
    h->status |= VOLTA_STATUS_DEVICE_ERROR;
    return -1;
  }
  return (int64_t)count;
}

// Bytes of the handle's device arena (reported by the benchmark).
int64_t volta_hip_arena_bytes(VoltaTrainHandle* vh) {
  Handle* h = H(vh);
  return h ? (int64_t)h->arena_bytes : -1;
}

int32_t volta_train_num_layers(VoltaTrainHandle* vh) {
  Handle* h = H(vh);
  return h ? h->n : -1;
}

int32_t volta_train_batch(VoltaTrainHandle* vh) {
  Handle* h = H(vh);
  return h ? h->B : -1;
}

int64_t volta_train_state_size(VoltaTrainHandle* vh) {
  Handle* h = H(vh);
  if (!h) return -1;
  int64_t per = 0;
  for (auto& lp : h->layers) per += (int64_t)lp.r * lp.c + lp.c;
  int64_t ln = 0;
  for (int i = 0; i < h->n - 1 && h->ext_ln; ++i) ln += 2 * (int64_t)h->L[i + 1];
  switch (h->spec.optimizer) {
    case VOLTA_OPT_ADAM:
    case VOLTA_OPT_ADAMW: return 2 * per + ln;
    case VOLTA_OPT_ADAGRAD: return per + ln;
    default: return ln;
  }
}

// State order per layer: [m_W | m_b | v_W | v_b] (Adam/AdamW) or [G_W | G_b],
// then [gamma_i | beta_i] per hidden layer with LayerNorm.
static bool state_copy(Handle* h, float* host, bool to_host) {
  const bool adam = h->spec.optimizer == VOLTA_OPT_ADAM || h->spec.optimizer == VOLTA_OPT_ADAMW;
  std::vector<float*> bufs;
  if (adam) bufs = {h->opt_a, h->opt_b};
  else if (h->spec.optimizer == VOLTA_OPT_ADAGRAD) bufs = {h->opt_a};
  float* p = host;
  for (auto& lp : h->layers) {
    for (float* dev : bufs) {
      const size_t nw = (size_t)lp.r * lp.c, nb = lp.c;
      hipError_t e1, e2;
      if (to_host) {
        e1 = hipMemcpy(p, dev + lp.w_off, nw * 4, hipMemcpyDeviceToHost);
        e2 = hipMemcpy(p + nw, dev + lp.b_off, nb * 4, hipMemcpyDeviceToHost);
      } else {
        e1 = hipMemcpy(dev + lp.w_off, p, nw * 4, hipMemcpyHostToDevice);
        e2 = hipMemcpy(dev + lp.b_off, p + nw, nb * 4, hipMemcpyHostToDevice);
      }
      if (e1 != hipSuccess || e2 != hipSuccess) return false;
      p += nw + nb;
    }
  }
  // LayerNorm [gamma_i | beta_i] per hidden layer
  for (int i = 0; i < h->n - 1 && h->ext_ln; ++i) {
    const size_t c = h->L[i + 1];
    for (float* dev : {h->ln_g[i], h->ln_b[i]}) {
      const hipError_t e = to_host ? hipMemcpy(p, dev, c * 4, hipMemcpyDeviceToHost)
                                   : hipMemcpy(dev, p, c * 4, hipMemcpyHostToDevice);
      if (e != hipSuccess) return false;
      p += c;
    }
  }
  return true;
}

int32_t volta_train_get_state(VoltaTrainHandle* vh, float* state, int64_t* step) {
  Handle* h = H(vh);
  if (!h || (!state && volta_train_state_size(vh) > 0)) return -1;
  uint32_t t = 0;
  if (!volta::sync(h) || !state_copy(h, state, true) ||
      hipMemcpy(&t, &h->scalars->t, sizeof(uint32_t), hipMemcpyDeviceToHost) != hipSuccess) {
    h->status |= VOLTA_STATUS_DEVICE_ERROR;
    return -1;
  }
  if (step) *step = t;
  return 0;
}

int32_t volta_train_get_dropout_rng(VoltaTrainHandle* vh, uint64_t* rng) {
  Handle* h = H(vh);
  if (!h || !rng) return -1;
  if (!volta::sync(h) || hipMemcpy(rng, &h->scalars->rng, sizeof(uint64_t), hipMemcpyDeviceToHost) != hipSuccess) {
    h->status |= VOLTA_STATUS_DEVICE_ERROR;
    return -1;
  }
  return 0;
}

int32_t volta_train_set_dropout_rng(VoltaTrainHandle* vh, uint64_t rng) {
  Handle* h = H(vh);
  if (!h) return -1;
  if (!volta::sync(h) || hipMemcpy(&h->scalars->rng, &rng, sizeof(uint64_t), hipMemcpyHostToDevice) != hipSuccess) {
    h->status |= VOLTA_STATUS_DEVICE_ERROR;
    return -1;
  }
  return 0;
}

int32_t volta_train_set_hparams(VoltaTrainHandle* vh, float beta1, float beta2, float eps, float weight_decay) {
  Handle* h = H(vh);
  if (!h) return -1;
  volta_mlp_spec s = h->spec;
  s.beta1 = beta1;
  s.beta2 = beta2;
  s.eps = eps;
  s.weight_decay = weight_decay;
  std::string why;
  if (!volta::validate_spec(s, &why)) {
    volta::fail(h, VOLTA_STATUS_BAD_ARGUMENT, "volta_train_set_hparams: " + why);
    return -1;
  }
  if (!volta::sync(h)) {
    h->status |= VOLTA_STATUS_DEVICE_ERROR;
    return -1;
  }
  h->spec = s;
  for (int i = 0; i < h->n; ++i) h->segs.wd[2 * i] = s.optimizer == VOLTA_OPT_ADAMW ? s.weight_decay : 0.0f;
  if (!volta::make_bc_table(h) || !volta::capture(h)) {
    h->status |= VOLTA_STATUS_DEVICE_ERROR;
    return -1;
  }
  return 0;
}

int32_t volta_train_infer(VoltaTrainHandle* vh, const float* X, int64_t rows, float* out) {
  Handle* h = H(vh);
  if (!h) return -1;
  if (!X || !out || rows <= 0) {
    volta::fail(h, VOLTA_STATUS_BAD_ARGUMENT, "volta_train_infer: bad arguments");
    return -1;
  }
  const int B = h->B, L0 = h->L[0], Ln = h->L[h->n];
  if (!h->infer_x && hipMalloc((void**)&h->infer_x, (size_t)B * L0 * sizeof(float)) != hipSuccess) {
    volta::fail(h, VOLTA_STATUS_DEVICE_ERROR, "volta_train_infer: device allocation failed");
    return -1;
  }
  for (int64_t r0 = 0; r0 < rows; r0 += B) {
    const int m = (int)std::min<int64_t>(B, rows - r0);
    if (hipMemcpyAsync(h->infer_x, X + r0 * L0, (size_t)m * L0 * sizeof(float), hipMemcpyHostToDevice,
                       h->stream) != hipSuccess ||
        !volta::enqueue_forward(h, m, h->stream) ||
        hipMemcpyAsync(out + r0 * Ln, h->act[h->n], (size_t)m * Ln * sizeof(float), hipMemcpyDeviceToHost,
                       h->stream) != hipSuccess ||
        hipStreamSynchronize(h->stream) != hipSuccess) {
      volta::fail(h, VOLTA_STATUS_DEVICE_ERROR, "volta_train_infer: device error");
      return -1;
    }
  }
  return 0;
}

// Allocation-free variant of volta_train_infer for callers that cannot
// allocate device memory (code under stream capture, serving loops): X and
// out are device buffers, the forward's split-K partial planes go to this
// device's static scratch, and nothing is allocated, freed or synchronized.
// The launches are enqueued on the handle's stream (volta_train_sync before
// reading `out`).  Calls that overlap on one GPU share its scratch and race.
int32_t volta_train_infer_device_noalloc(VoltaTrainHandle* vh, const float* X, int64_t rows, float* out) {
  Handle* h = H(vh);
  if (!h) return -1;
  const char* fn = "volta_train_infer_device_noalloc";
  if (!X || !out || rows <= 0) {
    volta::fail(h, VOLTA_STATUS_BAD_ARGUMENT, std::string(fn) + ": bad arguments");
    return -1;
  }
  if (((uintptr_t)X | (uintptr_t)out) & 15) {
    volta::fail(h, VOLTA_STATUS_BAD_ARGUMENT, std::string(fn) + ": X and out must be 16-byte aligned device pointers");
    return -1;
  }
  if (!h->scratch) {
    volta::fail(h, VOLTA_STATUS_DEVICE_ERROR, std::string(fn) + ": the static scratch address is unavailable");
    return -1;
  }
  const int B = h->B, L0 = h->L[0], Ln = h->L[h->n];
  // every chunk is B rows but the last; check both plans before launching
  std::vector<volta::GemmPlan> full, tail;
  const int tail_rows = (int)(rows % B);
  const size_t need = std::max(rows >= B ? volta::forward_plans(h, B, &full) : 0,
                               tail_rows ? volta::forward_plans(h, tail_rows, &tail) : 0);
  if (need > volta::kScratchFloats) {
    volta::fail(h, VOLTA_STATUS_BAD_ARGUMENT,
                std::string(fn) + ": the forward at this row count needs " + std::to_string(need * 4) +
                    " bytes of split-K workspace; the static scratch holds " +
                    std::to_string(volta::kScratchFloats * 4));
    return -1;
  }
  for (int64_t r0 = 0; r0 < rows; r0 += B) {
    const int m = (int)std::min<int64_t>(B, rows - r0);
    if (!volta::enqueue_forward_into(h, m == B ? full : tail, m, X + r0 * L0, out + r0 * Ln, h->scratch,
                                     h->stream)) {
      h->status |= VOLTA_STATUS_DEVICE_ERROR;
      return -1;
    }
  }
  return 0;
}

int32_t volta_infer_bind(VoltaTrainHandle* vh) {
  std::lock_guard<std::mutex> lock(g_infer_mu);
  g_infer_model = vh;
  return 0;
}

void volta_infer(const float* input, int64_t in_n, float* output, int64_t out_n) {
  std::lock_guard<std::mutex> lock(g_infer_mu);
  Handle* h = H(g_infer_model);
  if (!h) {
    set_last_error("volta_infer: no model bound (volta_infer_bind)");
    return;
  }
  const int L0 = h->L[0], Ln = h->L[h->n];
  if (!input || !output || in_n <= 0 || in_n % L0 != 0 || out_n < in_n / L0 * Ln) {
    volta::fail(h, VOLTA_STATUS_BAD_ARGUMENT, "volta_infer: in_n must be rows*L0 and out_n >= rows*Ln");
    return;
  }
  (void)volta_train_infer(g_infer_model, input, in_n / L0, output);
}

// Rows per forward chunk of an inference model (its handle's batch): every
// call of volta_train_infer runs its rows this many at a time.
constexpr int32_t kInferModelChunk = 1024;

VoltaTrainHandle* volta_infer_model_create(int32_t n_sizes, const int32_t* sizes, int32_t hidden_act,
                                           const float* params) {
  if (n_sizes < 2 || n_sizes > VOLTA_MAX_LAYER_SIZES || !sizes || !params ||
      (hidden_act != VOLTA_ACT_RELU && hidden_act != -1)) {
    set_last_error("volta_infer_model_create: bad arguments");
    return nullptr;
  }
  volta_mlp_spec s;
  volta_mlp_spec_default(&s, n_sizes, sizes, VOLTA_ACT_RELU, VOLTA_OPT_SGD, VOLTA_LOSS_MSE);
  VoltaTrainHandle* vh = volta_train_init_spec(&s, kInferModelChunk);
  if (!vh) return nullptr;
  Handle* h = H(vh);
  h->infer_linear = hidden_act == -1;
  const float* p = params;
  for (int i = 0; i < h->n; ++i) {
    const int64_t r = h->L[i], c = h->L[i + 1];
    volta_train_set_params(vh, i, p, p + r * c);
    p += r * c + c;
  }
  if (!volta::sync(h) || h->status != 0) {
    set_last_error("volta_infer_model_create: device error while copying the parameters");
    volta_train_free(vh);
    return nullptr;
  }
  return vh;
}

int32_t volta_train_set_state(VoltaTrainHandle* vh, const float* state, int64_t step) {
  Handle* h = H(vh);
  if (!h || step < 0 || step > 0xffffffffLL || (!state && volta_train_state_size(vh) > 0)) {
    if (h) volta::fail(h, VOLTA_STATUS_BAD_ARGUMENT, "volta_train_set_state: bad arguments");
    return -1;
  }
  const uint32_t t = (uint32_t)step;
  if (!volta::sync(h) || !state_copy(h, const_cast<float*>(state), false) ||
      hipMemcpy(&h->scalars->t, &t, sizeof(uint32_t), hipMemcpyHostToDevice) != hipSuccess) {
    h->status |= VOLTA_STATUS_DEVICE_ERROR;
    return -1;
  }
  return 0;
}

}  // extern "C"
