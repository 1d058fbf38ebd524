// Lowering of a runtime MLP graph onto the forward GEMM kernels (rt_lower.h).
//
// The graph is walked in schedule order, as the reference's executors walk
// it (interpreter.rs / cuda/executor.rs:65-91), keeping the head of one
// chain: a bound [rows x r] tensor, then per layer MatMul (or Gemm) by a
// bound weight, the bias Add, an activation, and at the end a Softmax.
// Every chain value is recorded with its (layer, stage), so execute_value
// can return any of them by running the chain up to that layer and ending
// the last launch at that stage.
#include "rt_lower.h"

#include <cfloat>
#include <cmath>
#include <cstring>

namespace volta {

namespace {

const char* op_name(int op) {
  switch (op) {
    case VOLTA_RT_OP_INPUT: return "Input";
    case VOLTA_RT_OP_PARAMETER: return "Parameter";
    case VOLTA_RT_OP_OUTPUT: return "Output";
    case VOLTA_RT_OP_MATMUL: return "MatMul";
    case VOLTA_RT_OP_ADD: return "Add";
    case VOLTA_RT_OP_GEMM: return "Gemm";
    case VOLTA_RT_OP_RELU: return "Relu";
    case VOLTA_RT_OP_SIGMOID: return "Sigmoid";
    case VOLTA_RT_OP_GELU: return "Gelu";
    case VOLTA_RT_OP_SOFTMAX: return "Softmax";
    default: return "an op outside the MLP subset";
  }
}

uint64_t fnv(uint64_t h, int64_t v) {
  for (int i = 0; i < 8; ++i) {
    h ^= (uint64_t)(v >> (8 * i)) & 0xff;
    h *= 1099511628211ull;
  }
  return h;
}

int64_t bits(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return (int64_t)u;
}

std::string shape_str(int64_t r, int64_t c) { return "[" + std::to_string(r) + ", " + std::to_string(c) + "]"; }

}  // namespace

std::vector<int64_t> rt_canonical(const volta_rt_graph& g) {
  std::vector<int64_t> v;
  v.reserve(4 + (size_t)g.n_nodes * 8 + g.n_ordered + 2 * (size_t)g.n_bindings);
  v.push_back(g.n_nodes);
  for (int i = 0; i < g.n_nodes; ++i) {
    const volta_rt_node& n = g.nodes[i];
    v.insert(v.end(), {n.op, n.output, n.in0, n.in1, n.in2, n.binding, bits(n.alpha), bits(n.beta)});
  }
  v.push_back(g.n_ordered);
  for (int i = 0; i < g.n_ordered; ++i) v.push_back(g.ordered_nodes[i]);
  v.push_back(g.n_bindings);
  for (int i = 0; i < g.n_bindings; ++i) v.insert(v.end(), {g.bindings[i].rows, g.bindings[i].cols});
  v.push_back(g.peak_bytes);
  return v;
}

bool rt_lower(const volta_rt_graph& g, RtLowered* out, std::string* err) {
  auto fail = [&](const std::string& m) {
    *err = "HIP backend: " + m;
    return false;
  };
  if (g.n_nodes < 1 || !g.nodes) return fail("the graph has no nodes");
  if (g.n_ordered < 1 || !g.ordered_nodes) return fail("the schedule is empty");
  if (g.n_bindings < 0 || (g.n_bindings > 0 && !g.bindings)) return fail("binding table missing");
  constexpr int64_t kMaxDim = int64_t(1) << 30;
  for (int i = 0; i < g.n_bindings; ++i) {
    const volta_rt_binding& b = g.bindings[i];
    if (b.rows < 1 || b.cols < 1 || b.rows > kMaxDim || b.cols > kMaxDim || b.rows * b.cols > INT32_MAX)
      return fail("binding " + std::to_string(i) + " has shape " + shape_str(b.rows, b.cols) +
                  " (each bound tensor needs 1 to 2^31-1 elements)");
  }

  RtLowered L;
  // terminal value: the last Output in graph order, else the last node's value
  for (int i = g.n_nodes - 1; i >= 0 && L.terminal < 0; --i)
    if (g.nodes[i].op == VOLTA_RT_OP_OUTPUT) L.terminal = g.nodes[i].in0;
  if (L.terminal < 0) L.terminal = g.nodes[g.n_nodes - 1].output;

  std::vector<char> seen(g.n_nodes, 0);
  int32_t head = -1;  // ValueId at the head of the chain
  auto where = [&](int k, const volta_rt_node& n) {
    return std::string("node ") + std::to_string(k) + " (" + op_name(n.op) + ")";
  };
  auto bound = [&](int32_t v, const volta_rt_binding** b) {
    auto it = L.values.find(v);
    if (it == L.values.end() || it->second.stage != RT_BOUND) return false;
    *b = &g.bindings[it->second.binding];
    return true;
  };
  // Starts a layer: y = lhs x W (MatMul or Gemm).
  auto start_layer = [&](int k, const volta_rt_node& n) -> bool {
    const volta_rt_binding* w = nullptr;
    if (!bound(n.in1, &w)) return fail(where(k, n) + ": the right operand must be a bound weight tensor");
    const volta_rt_binding* xb = nullptr;
    int64_t lhs_rows = 0, lhs_cols = 0;
    RtLayer layer;
    if (bound(n.in0, &xb)) {
      if (!L.layers.empty())
        return fail(where(k, n) + ": a second chain (the backend lowers one MLP chain per graph)");
      lhs_rows = xb->rows;
      lhs_cols = xb->cols;
      layer.x_binding = L.values[n.in0].binding;
      L.rows = xb->rows;
    } else {
      if (n.in0 != head || head < 0)
        return fail(where(k, n) + ": its left operand (value " + std::to_string(n.in0) +
                    ") is not the head of the chain");
      const RtValue& hv = L.values[head];
      if (hv.stage == RT_SOFTMAX) return fail(where(k, n) + ": a product of a Softmax output is not lowered");
      lhs_rows = L.rows;
      lhs_cols = L.layers.back().c;
    }
    if (lhs_cols != w->rows)
      return fail("Shape mismatch in MatMul: lhs " + shape_str(lhs_rows, lhs_cols) + " rhs " +
                  shape_str(w->rows, w->cols));
    if (L.rows * w->cols > INT32_MAX) return fail(where(k, n) + ": the output has more than 2^31-1 elements");
    layer.w_binding = L.values[n.in1].binding;
    layer.r = (int)w->rows;
    layer.c = (int)w->cols;
    L.layers.push_back(layer);
    return true;
  };
  auto bias_of = [&](int32_t v, int c, int* binding) {
    const volta_rt_binding* b = nullptr;
    if (!bound(v, &b) || b->rows != 1 || b->cols != c) return false;
    *binding = L.values[v].binding;
    return true;
  };

  for (int s = 0; s < g.n_ordered; ++s) {
    const int k = g.ordered_nodes[s];
    if (k < 0 || k >= g.n_nodes) return fail("schedule entry " + std::to_string(s) + " is out of range");
    if (seen[k]) return fail("node " + std::to_string(k) + " is scheduled twice");
    seen[k] = 1;
    const volta_rt_node& n = g.nodes[k];
    if (L.values.count(n.output))
      return fail("SSA violation: ValueId " + std::to_string(n.output) + " assigned more than once");
    const int li = (int)L.layers.size() - 1;
    switch (n.op) {
      case VOLTA_RT_OP_INPUT:
      case VOLTA_RT_OP_PARAMETER:
        if (n.binding < 0 || n.binding >= g.n_bindings) return fail(where(k, n) + ": binding out of range");
        L.values[n.output] = RtValue{RT_BOUND, -1, n.binding};
        break;
      case VOLTA_RT_OP_OUTPUT: {
        auto it = L.values.find(n.in0);
        if (it == L.values.end()) return fail(where(k, n) + ": its value is not computed before it");
        L.values[n.output] = it->second;
        break;
      }
      case VOLTA_RT_OP_MATMUL:
        if (!start_layer(k, n)) return false;
        L.values[n.output] = RtValue{RT_MM, (int)L.layers.size() - 1, -1};
        head = n.output;
        break;
      case VOLTA_RT_OP_GEMM: {
        // Tensor::gemm (tensor.rs:481-503): alpha scales when |alpha-1| > EPSILON,
        // the bias is added when beta != 0 and scaled when |beta-1| > EPSILON.
        if (std::fabs(n.alpha - 1.0f) > FLT_EPSILON)
          return fail(where(k, n) + ": alpha other than 1 is not lowered");
        const bool with_bias = n.in2 >= 0 && n.beta != 0.0f;
        if (with_bias && std::fabs(n.beta - 1.0f) > FLT_EPSILON)
          return fail(where(k, n) + ": beta other than 0 or 1 is not lowered");
        if (!start_layer(k, n)) return false;
        RtLayer& ly = L.layers.back();
        if (with_bias && !bias_of(n.in2, ly.c, &ly.b_binding))
          return fail(where(k, n) + ": the bias must be a bound [1, " + std::to_string(ly.c) + "] tensor");
        L.values[n.output] = RtValue{with_bias ? RT_PRE : RT_MM, (int)L.layers.size() - 1, -1};
        head = n.output;
        break;
      }
      case VOLTA_RT_OP_ADD: {
        int32_t chain = -1, other = -1;
        if (head >= 0 && n.in0 == head) chain = n.in0, other = n.in1;
        else if (head >= 0 && n.in1 == head) chain = n.in1, other = n.in0;
        if (chain < 0 || L.values[head].stage != RT_MM)
          return fail(where(k, n) + ": Add is lowered only as the bias of the chain's MatMul");
        if (!bias_of(other, L.layers[li].c, &L.layers[li].b_binding))
          return fail(where(k, n) + ": the bias must be a bound [1, " + std::to_string(L.layers[li].c) + "] tensor");
        L.values[n.output] = RtValue{RT_PRE, li, -1};
        head = n.output;
        break;
      }
      case VOLTA_RT_OP_RELU:
      case VOLTA_RT_OP_SIGMOID:
      case VOLTA_RT_OP_GELU: {
        if (head < 0 || n.in0 != head || (L.values[head].stage != RT_MM && L.values[head].stage != RT_PRE))
          return fail(where(k, n) + ": an activation is lowered only on a layer's product or bias sum");
        L.layers[li].act = n.op == VOLTA_RT_OP_RELU ? RT_ACT_RELU : n.op == VOLTA_RT_OP_SIGMOID ? RT_ACT_SIGMOID
                                                                                               : RT_ACT_GELU;
        L.values[n.output] = RtValue{RT_ACT, li, -1};
        head = n.output;
        break;
      }
      case VOLTA_RT_OP_SOFTMAX: {
        if (head < 0 || n.in0 != head || L.values[head].stage == RT_SOFTMAX || L.values[head].stage == RT_BOUND)
          return fail(where(k, n) + ": Softmax is lowered only on the chain's last layer");
        L.layers[li].softmax = true;
        L.values[n.output] = RtValue{RT_SOFTMAX, li, -1};
        head = n.output;
        break;
      }
      default:
        return fail(where(k, n) + " is not lowered; keep this graph on the CPU backend");
    }
  }
  if (L.layers.empty()) return fail("the graph has no MatMul or Gemm layer");

  uint64_t h = 1469598103934665603ull;
  h = fnv(h, L.rows);
  for (const RtLayer& ly : L.layers)
    for (int64_t v : {(int64_t)ly.x_binding, (int64_t)ly.w_binding, (int64_t)ly.b_binding, (int64_t)ly.r,
                      (int64_t)ly.c, (int64_t)ly.act, (int64_t)ly.softmax})
      h = fnv(h, v);
  for (int64_t v : rt_canonical(g)) h = fnv(h, v);
  L.fingerprint = h;
  *out = std::move(L);
  return true;
}

}  // namespace volta
