// ===========================================================================
// TEST INFRASTRUCTURE -- CPU oracle of graph execution.  Not part of the
// product.
//
// A CPU restatement of the reference's interpreter for the ops an MLP graph
// is made of, behind the graph-execution C ABI of include/volta_backend.h
// (host pointers), so the tests drive it and the HIP backend alike.  Unlike
// the HIP backend, which pattern-matches the graph into fused layers, this
// walks every scheduled node and evaluates it alone, as the reference's
// execute_value_with_schedule_context does (interpreter.rs:265-330): a
// mistake in the backend's lowering (a dropped bias, a wrong stage, an
// activation on the wrong layer) shows as a difference.
//
// Ops and the reference functions they follow:
//   MatMul    kernels/math.rs:109-180 (gemm crate; here fp32, k ascending,
//             no FMA -- the crate's order is its own, so parity with it is
//             within fp32 rounding)
//   Add       Tensor::add_broadcast, tensor.rs:338-340 (numpy broadcasting)
//   Gemm      Tensor::gemm, tensor.rs:481-503
//   Relu      kernels/activations.rs:7-32      max as `v > 0 ? v : 0`
//   Sigmoid   kernels/activations.rs:67-90     piecewise in the sign of x
//   Gelu      kernels/activations.rs:121-143   tanh approximation
//   Softmax   kernels/reduce.rs:189-220        per row, sequential sum
//   Output    the value it names
// Shapes are 2-D (a 1-D [c] tensor is carried as [1, c], which broadcasts
// the same way against 2-D operands).
//
// Pinned by tests/test_rt_graph_oracle.py: the reference's own expected
// values (interpreter.rs:1880-1955 MatMul 19/22/43/50, ReLU clamping, softmax
// summing to one; tensor.rs:518-620 add_broadcast extending rank, two-sided
// and scalar, gemm with a vector bias 22..64), closed forms of each
// activation in fp64, and a float64 torch forward of random MLP graphs.
// ===========================================================================
#include <cfloat>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "../include/volta_backend.h"

void oracle_rt_set_error(const std::string& m);

namespace {

struct T {
  int64_t r = 0, c = 0;
  std::vector<float> d;
};

int64_t g_compiles = 0;

bool err(const std::string& m) {
  oracle_rt_set_error(m);
  return false;
}

std::string shp(const T& t) { return "[" + std::to_string(t.r) + ", " + std::to_string(t.c) + "]"; }

bool matmul(const T& a, const T& b, T* o) {
  if (a.c != b.r) return err("Shape mismatch in matmul: [" + std::to_string(a.r) + "x" + std::to_string(a.c) +
                             "] @ [" + std::to_string(b.r) + "x" + std::to_string(b.c) + "]");
  o->r = a.r;
  o->c = b.c;
  o->d.assign((size_t)a.r * b.c, 0.0f);
  // each output element accumulates its k terms in ascending order from 0
  // (the loop nest runs j innermost so B's rows stream)
  for (int64_t i = 0; i < a.r; ++i) {
    float* out = o->d.data() + i * b.c;
    for (int64_t k = 0; k < a.c; ++k) {
      const float x = a.d[i * a.c + k];
      const float* brow = b.d.data() + k * b.c;
      for (int64_t j = 0; j < b.c; ++j) out[j] = out[j] + x * brow[j];
    }
  }
  return true;
}

bool add_broadcast(const T& a, const T& b, T* o) {
  auto dim = [](int64_t x, int64_t y, int64_t* z) {
    if (x == y || y == 1) return *z = x, true;
    if (x == 1) return *z = y, true;
    return false;
  };
  int64_t r, c;
  if (!dim(a.r, b.r, &r) || !dim(a.c, b.c, &c))
    return err("Shape mismatch in add_broadcast: " + shp(a) + " vs " + shp(b));
  o->r = r;
  o->c = c;
  o->d.resize((size_t)r * c);
  for (int64_t i = 0; i < r; ++i)
    for (int64_t j = 0; j < c; ++j) {
      const float x = a.d[(a.r == 1 ? 0 : i) * a.c + (a.c == 1 ? 0 : j)];
      const float y = b.d[(b.r == 1 ? 0 : i) * b.c + (b.c == 1 ? 0 : j)];
      o->d[i * c + j] = x + y;
    }
  return true;
}

float relu(float v) { return v > 0.0f ? v : 0.0f; }

float sigmoid(float x) {
  if (x >= 0.0f) return 1.0f / (1.0f + std::exp(-x));
  const float ex = std::exp(x);
  return ex / (1.0f + ex);
}

float gelu(float x) {
  const float k_sqrt_2_over_pi = 0.7978846f, k_coeff = 0.044715f;
  const float inner = k_sqrt_2_over_pi * (x + k_coeff * x * x * x);
  const float t = std::tanh(inner);
  return x * 0.5f * (1.0f + t);
}

void softmax_rows(T* t) {
  for (int64_t i = 0; i < t->r; ++i) {
    float* row = t->d.data() + i * t->c;
    float m = -INFINITY;
    for (int64_t j = 0; j < t->c; ++j) m = std::fmax(m, row[j]);
    std::vector<float> e(t->c);
    float s = 0.0f;
    for (int64_t j = 0; j < t->c; ++j) e[j] = std::exp(row[j] - m);
    for (int64_t j = 0; j < t->c; ++j) s = s + e[j];
    for (int64_t j = 0; j < t->c; ++j) row[j] = e[j] / s;
  }
}

// Interprets the schedule; the value `target` into *out.
bool run(const volta_rt_graph* g, int32_t target, bool terminal, const float* const* bindings, T* out) {
  if (!g || !g->nodes || g->n_nodes < 1 || !g->ordered_nodes || g->n_ordered < 1)
    return err("oracle: empty graph or schedule");
  if (g->n_bindings > 0 && (!g->bindings || !bindings)) return err("oracle: binding table missing");
  if (terminal) {
    target = -1;
    for (int i = g->n_nodes - 1; i >= 0 && target < 0; --i)
      if (g->nodes[i].op == VOLTA_RT_OP_OUTPUT) target = g->nodes[i].in0;
    if (target < 0) target = g->nodes[g->n_nodes - 1].output;
  }
  std::map<int32_t, T> v;
  auto get = [&](int32_t id, const T** t) {
    auto it = v.find(id);
    if (it == v.end()) return err("ValueId " + std::to_string(id) + " not computed");
    *t = &it->second;
    return true;
  };
  for (int s = 0; s < g->n_ordered; ++s) {
    const int k = g->ordered_nodes[s];
    if (k < 0 || k >= g->n_nodes) return err("Schedule node out of range: " + std::to_string(k));
    const volta_rt_node& n = g->nodes[k];
    if (v.count(n.output))
      return err("SSA violation: ValueId " + std::to_string(n.output) + " assigned more than once");
    T o;
    const T *a = nullptr, *b = nullptr, *c = nullptr;
    switch (n.op) {
      case VOLTA_RT_OP_INPUT:
      case VOLTA_RT_OP_PARAMETER: {
        if (n.binding < 0 || n.binding >= g->n_bindings || !bindings[n.binding])
          return err("oracle: binding of node " + std::to_string(k) + " missing");
        const volta_rt_binding& bd = g->bindings[n.binding];
        o.r = bd.rows;
        o.c = bd.cols;
        o.d.assign(bindings[n.binding], bindings[n.binding] + bd.rows * bd.cols);
        break;
      }
      case VOLTA_RT_OP_OUTPUT:
        if (!get(n.in0, &a)) return false;
        o = *a;
        break;
      case VOLTA_RT_OP_MATMUL:
        if (!get(n.in0, &a) || !get(n.in1, &b) || !matmul(*a, *b, &o)) return false;
        break;
      case VOLTA_RT_OP_ADD:
        if (!get(n.in0, &a) || !get(n.in1, &b) || !add_broadcast(*a, *b, &o)) return false;
        break;
      case VOLTA_RT_OP_GEMM: {
        if (!get(n.in0, &a) || !get(n.in1, &b) || !matmul(*a, *b, &o)) return false;
        if (std::fabs(n.alpha - 1.0f) > FLT_EPSILON)
          for (float& x : o.d) x = x * n.alpha;
        if (n.in2 >= 0 && n.beta != 0.0f) {
          if (!get(n.in2, &c)) return false;
          T bias = *c;
          if (std::fabs(n.beta - 1.0f) > FLT_EPSILON)
            for (float& x : bias.d) x = x * n.beta;
          T sum;
          if (!add_broadcast(o, bias, &sum)) return false;
          o = std::move(sum);
        }
        break;
      }
      case VOLTA_RT_OP_RELU:
      case VOLTA_RT_OP_SIGMOID:
      case VOLTA_RT_OP_GELU:
        if (!get(n.in0, &a)) return false;
        o = *a;
        for (float& x : o.d) x = n.op == VOLTA_RT_OP_RELU ? relu(x) : n.op == VOLTA_RT_OP_SIGMOID ? sigmoid(x) : gelu(x);
        break;
      case VOLTA_RT_OP_SOFTMAX:
        if (!get(n.in0, &a)) return false;
        o = *a;
        softmax_rows(&o);
        break;
      default:
        return err("oracle: unsupported op at node " + std::to_string(k));
    }
    v[n.output] = std::move(o);
  }
  const T* t = nullptr;
  if (!get(target, &t)) return false;
  *out = *t;
  return true;
}

int execute(const volta_rt_graph* g, int32_t target, bool terminal, const float* const* bindings, float* out,
            int64_t cap, int64_t* shape) {
  T t;
  if (!run(g, target, terminal, bindings, &t)) return -1;
  if (shape) {
    shape[0] = t.r;
    shape[1] = t.c;
  }
  if (!out || cap < (int64_t)t.d.size()) return err("oracle: output too small"), -1;
  std::memcpy(out, t.d.data(), t.d.size() * sizeof(float));
  return 0;
}

}  // namespace

extern "C" {

int32_t volta_rt_compile(const volta_rt_graph* g, int32_t determinism, volta_rt_compiled* out) {
  if (!g || determinism < 0 || determinism > 2) return err("oracle: bad arguments"), -1;
  ++g_compiles;
  if (out) {
    out->schedule_len = g->n_ordered;
    out->peak_bytes = g->peak_bytes;
    out->fingerprint = 0;
  }
  return 0;
}

int32_t volta_rt_execute_value(const volta_rt_graph* g, int32_t determinism, int32_t target,
                               const float* const* bindings, float* out, int64_t out_capacity, int64_t* out_shape) {
  (void)determinism;
  return execute(g, target, false, bindings, out, out_capacity, out_shape);
}

int32_t volta_rt_execute_terminal(const volta_rt_graph* g, int32_t determinism, const float* const* bindings,
                                  float* out, int64_t out_capacity, int64_t* out_shape) {
  (void)determinism;
  return execute(g, -1, true, bindings, out, out_capacity, out_shape);
}

void volta_rt_clear_plan_cache(void) {}

int64_t volta_rt_compile_count(void) { return g_compiles; }

}  // extern "C"
