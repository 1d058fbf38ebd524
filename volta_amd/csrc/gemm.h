// Host/device interface of the fp32 MFMA GEMM family (gemm.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>

#include "device_common.h"
#include "recorder.h"
#include "skinny.h"

namespace volta {

enum GemmLayout {
  GEMM_NN = 0,  // A [M x K] row-major, B [K x N] row-major   (forward)
  GEMM_NT = 1,  // A [M x K] row-major, B [N x K] row-major   (dX = delta W^T)
  GEMM_TN = 2,  // A [K x M] row-major, B [K x N] row-major   (dW = act^T delta)
};

enum EpiKind {
  EPI_STORE = 0,     // out = acc
  EPI_BIAS_ACT = 1,  // pre = acc + bias; out = f(pre)     (f = identity for the output layer)
  EPI_DX_ACT = 2,    // out = acc * f'(aux_pre, aux_act)
  EPI_DW_OPT = 3,    // acc is dW: optimizer update of W (and of b from the fused column sums)
  EPI_LOSS = 4,      // output layer + loss head: out = acc + bias, delta, loss
  EPI_ROWS = 5,      // small-M tile only: acc + bias into the workgroup's LDS rows (the output head)
};

struct EpiArgs {
  int kind;
  int act;                  // enum volta_activation, or kIdentity
  int ldc;
  float* out;               // result; for EPI_DW_OPT the weights W_i (updated in place)
  float* pre;               // EPI_BIAS_ACT: where to keep the pre-activation (may be null)
  const float* bias;        // EPI_BIAS_ACT / EPI_LOSS
  const float* aux_act;     // EPI_DX_ACT: activation output of the layer below
  const float* aux_pre;     // EPI_DX_ACT: its pre-activation (null when not kept)
  DevScalars* scalars;      // lr, bias corrections, loss, flags

  // EPI_DW_OPT: optimizer over W_i (index m*ldc + n) and, when `b` is set,
  // over b_i from the column sums of delta_i that the same kernel computes.
  int opt;                  // enum volta_optimizer
  float* m;                 // Adam m / Adagrad G for W_i
  float* v;                 // Adam v for W_i
  float* grad;              // optional copy of dW_i (debugging), may be null
  int64_t count;            // elements of W_i (the reference's n for the tail rule)
  float wd, b1, b2, eps;
  float* b;                 // b_i (null: column sums not fused)
  float* bm;                // state for b_i
  float* bv;
  float* bgrad;             // optional copy of db_i, may be null

  // EPI_LOSS
  int loss;                 // enum volta_loss
  const float* y;           // MSE targets [M x N]
  const int32_t* labels;    // CE labels [M]
  float* delta;             // seed gradient [M x N]
  float* loss_partials;     // one float per M-tile
  unsigned* loss_counter;   // arrival counter (zero between launches)
  int loss_tiles;           // number of M-tiles
  const float2* bc_table;   // Adam bias-correction table (null without Adam)
  int bc_len;
};

struct GemmArgs {
  const float* A;
  const float* B;
  int lda, ldb;
  int M, N, K;
  int k_per_split;
  float* partial;       // split-K workspace: splits planes of (M+1)*N floats
  unsigned* counters;   // split-K arrival counters, one per output tile, zero between launches
  int colsum_b;         // 1: also sum the B operand over k (dW: db = sum_b delta)
  EpiArgs epi;
};

// TILE_SMALLM: 16x16 output tiles, the whole K range in one workgroup
// (split over its 4 or 8 waves), for NN/NT products with few rows (B <= 256).
// TILE_DW_SMALLK: 32x32 tiles of the TN (dW) product with a short K
// (K = B <= 256), the optimizer applied on 16-byte rows.
// TILE_BIG: 256x256 tiles, direct-to-LDS operand loads, one workgroup per
// CU, for exact 256-multiples with at least one tile per CU (C5's 4096 x 4096
// products).  TILE_BIG128: the same pipeline on 128x128 tiles, for exact
// 128-multiples whose 128x128 grid has a tile per CU and whose 256x256 grid
// does not (C5's 4096 x 1024 and 1024 x 4096 products).  TILE_NARROW_TN: a
// TN product of at most 16 columns with a long K (the output layer's dW at
// a large batch), 64 rows per workgroup, K split, then the reduce launch.
enum GemmTile { TILE_64x64 = 0, TILE_128x128 = 1, TILE_64x64_K64 = 2, TILE_SMALLM = 3, TILE_DW_SMALLK = 4,
                TILE_BIG = 5, TILE_BIG128 = 6, TILE_NARROW_TN = 7 };

struct GemmPlan {
  int layout = GEMM_NN;
  int tile = TILE_64x64;
  int splits = 1;
  int k_per_split = 0;
  bool vec = false;
  bool inkernel_reduce = false;  // split-K reduced by the last slice (else a second kernel)
  int waves = 0;                 // TILE_SMALLM: waves per workgroup (4 or 8)
  int kgroups = 1;               // 64x64 / 128x128: K slices inside one workgroup (splits = 1)
  bool stage = true;             // TILE_SMALLM at 16 waves: operands staged in LDS (VOLTA_SMALLM_STAGE=0: off)
  int tiles(int M, int N) const {
    const int t = tile == TILE_BIG ? 256 : tile == TILE_128x128 || tile == TILE_BIG128 ? 128 : tile == TILE_SMALLM ? 16
                  : tile == TILE_DW_SMALLK ? 32 : 64;
    return ((M + t - 1) / t) * ((N + t - 1) / t);
  }
  size_t workspace_floats(int M, int N) const { return splits > 1 ? (size_t)splits * (M + 1) * N : 0; }
};

// Tile and split-K plan of one product.  `small_m`: the small-M tile may be
// chosen (NN/NT products whose epilogue is per element: not the loss head).
GemmPlan gemm_plan(int layout, int M, int N, int K, bool vec, int num_cus, bool small_m = true);
// TILE_NARROW_TN's K slice (a multiple of 4, at most 128) and split count
// for an M x N x K product on num_cus CUs.
void narrow_tn_split_plan(int M, int K, int num_cus, int* k_per_split, int* splits);

// Waves per workgroup of a small-M product of M x N outputs: 4 when it runs
// in a 256-thread paired launch, else by the grid's size (16, 8 or 4).
int gemm_smallm_waves(bool paired, int M, int N, int num_cus);

// `bytes` is the caller's algorithmic HBM traffic of the product (for the
// profiler); `rec`/`label` are optional.
hipError_t gemm_launch(const GemmPlan& p, const GemmArgs& a, hipStream_t st, Recorder* rec = nullptr,
                       const char* label = "gemm", double bytes = 0.0);

// The last hidden layer's forward product (plan p: small-M tile, bias +
// activation, 8 waves) and the output layer of width 1 (o, with its dX
// fields and loss ticket) in one launch; strip_counters: one zeroed
// counter per 16 rows of the batch (at least (M + 15) / 16 of the
// n_counters), left zero.
// The one-column output layer (loss head, dX_{n-1}) and the dX_{n-2}
// product planned as `p` in one launch (gemm_smallm_tail; loss deferred).
// A hidden forward product over two halves of its K (plan p: 16-wave small-M
// tile, 16-byte rows), each half's raw partial tile into its plane of
// `planes` (2*M*N floats, 16-byte aligned); k_half a multiple of 16 inside
// (0, K).  The next forward product adds them as it loads its A operand:
struct PlaneArgs {
  const float* p1 = nullptr;    // the second plane (args.A is the first; row stride args.lda)
  const float* bias = nullptr;  // the previous layer's bias
  float* act_out = nullptr;     // the previous layer's output [M x lda]
  float* pre_out = nullptr;     // the previous layer's pre-activation, or null
  int act = 0;                  // the previous layer's activation (device code)
};
bool khalves_supported(const GemmPlan& p, const GemmArgs& a, int k_half);
hipError_t launch_smallm_khalves(const GemmPlan& p, const GemmArgs& a, float* planes, int k_half, hipStream_t st);
bool planes_supported(const GemmPlan& p, const GemmArgs& a, const PlaneArgs& pa);
hipError_t launch_smallm_planes(const GemmPlan& p, const GemmArgs& a, const PlaneArgs& pa, hipStream_t st);
// The narrow output layer of a large batch (L_n <= 16, more rows than the
// one-launch output kernels take) on 16-wave small-M tiles, one per 16-row
// strip: z = act_{n-1} W + b on MFMA, then the loss head per row
// (head_row: z, delta_{n-1}, the row loss); each workgroup stores its rows'
// loss sum in row order to o.partials[strip], block 0 advances the step
// counter, and a later launch adds the partials (the outer-product dX_{n-1}
// launch, LossDefer).  `a` carries A = act_{n-1}, B = W, M = B, N = L_n,
// K = L_{n-1} and the bias (a.epi.bias).
bool out_head_gemm_supported(const GemmArgs& a, const OutLayerArgs& o);
hipError_t launch_smallm_out_head(const GemmArgs& a, const OutLayerArgs& o, hipStream_t st);
bool tail_supported(const GemmPlan& p, const GemmArgs& a, const OutLayerArgs& o);
hipError_t launch_smallm_tail(const GemmPlan& p, const GemmArgs& a, const OutLayerArgs& o, hipStream_t st);
bool fwd_head_supported(const GemmPlan& p, const GemmArgs& a, const OutLayerArgs& o, int n_counters);
hipError_t launch_fwd_head(const GemmPlan& p, const GemmArgs& a, const OutLayerArgs& o, unsigned* strip_counters,
                           int n_counters, hipStream_t st);

// b_i update (optimizer of EpiArgs: opt, b, bm, bv, bgrad, b1, b2, eps,
// scalars) from db_i = the column sums of delta_i [B x N], b ascending.
hipError_t launch_bias_update(const EpiArgs& e, const float* delta, int B, int N, hipStream_t st);

// One operation of a paired launch (two independent operations of the
// backward pass in one kernel launch: no buffer one writes is touched by the
// other).
enum PairKind { PAIR_NONE = 0, PAIR_GEMM = 1, PAIR_NARROW_DW = 2 };

struct PairOp {
  int kind = PAIR_NONE;
  GemmPlan plan;        // PAIR_GEMM
  GemmArgs args{};      // PAIR_GEMM (args.partial: this operation's own workspace)
  NarrowDwArgs nd{};    // PAIR_NARROW_DW
};

// Whether a and b can share one launch: dX (NT, activation-derivative
// epilogue; 64x64 or small-M tiles) or dW (TN, optimizer epilogue; 64x64 or
// small-K tiles) products with 16-byte rows, or the narrow output-layer dW
// whose staged delta fits the launch's LDS.
bool pair_supported(const PairOp& a, const PairOp& b);

// Both operations in one launch, then the split-K reductions either needs.
hipError_t pair_launch(const PairOp& a, const PairOp& b, hipStream_t st, Recorder* rec, const char* label,
                       double flops, double bytes);

// Every dW product of a small-batch step in one launch: the small-K dW
// tiles of up to kMaxDwGroup products and the narrow output-layer dW.  The
// products are independent of each other (each reads its own act_i and
// delta_i and rewrites only W_i, b_i and their state), so once the last dX
// has run they share one launch.
constexpr int kMaxDwGroup = 8;
struct DwGroup {
  int n = 0;                        // small-K dW products (plan TILE_DW_SMALLK)
  GemmArgs g[kMaxDwGroup];
  int start[kMaxDwGroup + 1] = {};  // first workgroup of product i after the narrow ones; start[n] = total
  int tile_n = 32;                  // columns of the small-K tiles: 32, or 64 (the wide form, same results)
  int narrow_blocks = 0;            // 0: no narrow dW
  NarrowDwArgs nd{};
  // the step's loss, when the output launch deferred it (launch_out_layer_dx
  // with defer_loss): workgroup 0 adds the partials in block order
  const float* loss_partials = nullptr;
  int loss_blocks = 0;
  float loss_denom = 1.0f;
  DevScalars* loss_scalars = nullptr;
};
bool dw_group_supported(const DwGroup& d);
// Workgroups of product `a` in a group whose small-K tiles are 32 x tile_n.
int dw_group_tiles(const GemmArgs& a, int tile_n);
// Tile width for group `d` (its products, narrow part and narrow width set;
// start[] and tile_n not read): 64 when the 32-wide tiles need more than one
// round of the workgroups the device keeps resident and the 64-wide ones fit
// in one (residency from the occupancy query of the kernel the launch would
// run), else 32.  Both widths give bit-identical results.
int dw_group_pick_tile_n(const DwGroup& d, int num_cus);
hipError_t dw_group_launch(const DwGroup& d, hipStream_t st, Recorder* rec, const char* label, double flops,
                           double bytes);

}  // namespace volta
