// Graph execution of the HIP backend (include/volta_backend.h): compile,
// execute_value and execute_terminal of the runtime's Backend trait
// (src/engine/ir/backend.rs:24-69) for MLP graphs, through a process-wide
// plan cache keyed as compile_or_get_cached keys it (plan_cache.rs:8-51).
//
// compile lowers the graph (rt_lower.cpp) into layers; execute runs layers
// 0..L of the chain for a value of layer L, each as one forward GEMM launch
// of the compile-train kernels (gemm.hip) whose epilogue adds the bias and
// applies the activation, so a layer costs one pass over its output instead
// of the reference executor's three ops with a host round trip each
// (cuda/executor.rs:137-246).  The last launch ends at the requested stage:
// the plain product (EPI_STORE), the bias sum (identity epilogue), the
// activation, or the activation followed by a row Softmax (one wave per row).
// Intermediate layers ping-pong between two device buffers of the program.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <cmath>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "gemm.h"
#include "rt_lower.h"

namespace volta {
namespace {

// Row softmax in place over a [rows x cols] matrix, one wave per row
// (kernels/reduce.rs:203-214): m = max of the row, e_j = exp(x_j - m),
// y_j = e_j / sum e.  The max is exact in any order; the sum is a fixed
// lane-strided order and a fixed butterfly, so results are run-to-run
// identical and within rounding of the reference's sequential sum.
__global__ void __launch_bounds__(256) rt_softmax_rows(float* __restrict__ x, int rows, int cols) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  float* p = x + (size_t)row * cols;
  float m = -INFINITY;
  for (int j = lane; j < cols; j += 64) m = fmaxf(m, p[j]);
  for (int off = 32; off; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  float s = 0.0f;
  for (int j = lane; j < cols; j += 64) s = s + expf(p[j] - m);
  for (int off = 32; off; off >>= 1) s = s + __shfl_xor(s, off);
  for (int j = lane; j < cols; j += 64) p[j] = expf(p[j] - m) / s;
}

int device_act(int a) {
  switch (a) {
    case RT_ACT_RELU: return VOLTA_ACT_RELU;
    case RT_ACT_SIGMOID: return kRtSigmoid;
    case RT_ACT_GELU: return VOLTA_ACT_GELU;
    default: return kIdentity;
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// One launch sequence of a program captured as a hipGraph: the layers up to
// `last` ending at `stage`, on the binding and output pointers of `key`.
struct Captured {
  int last = -1, stage = 0;
  std::vector<const void*> key;
  hipGraphExec_t exec = nullptr;
  uint64_t used = 0;  // recency, for eviction
};
constexpr size_t kMaxCaptured = 8;
constexpr size_t kRecent = 4;

// Device state of a program on one device: two activation buffers, the
// split-K workspace and arrival counters (zero between launches), a zero
// bias for layers without one, the epilogue's scalar block, a stream, and
// the launch sequences captured so far.
struct DevState {
  int num_cus = 0;
  hipStream_t stream = nullptr;
  void* arena = nullptr;
  float* buf[2] = {};
  float* ws = nullptr;
  size_t ws_floats = 0;
  unsigned* counters = nullptr;
  float* zeros = nullptr;
  DevScalars* scalars = nullptr;
  std::vector<GemmPlan> plans[2];  // per layer: [0] element-wise operands, [1] 16-byte operands
  std::vector<Captured> captured;
  std::vector<Captured> recent;  // the last kRecent sequences that ran without a graph (no exec)
  uint64_t tick = 0;
};

struct Program {
  RtLowered low;
  std::vector<int64_t> canon;
  volta_rt_compiled info{};
  std::mutex mu;
  std::map<int, DevState> dev;
  ~Program() {
    for (auto& kv : dev) {
      for (Captured& c : kv.second.captured) (void)hipGraphExecDestroy(c.exec);
      if (kv.second.stream) (void)hipStreamDestroy(kv.second.stream);
      if (kv.second.arena) (void)hipFree(kv.second.arena);
    }
  }
};

struct Key {
  int determinism;
  uint64_t graph_fp;
  uint64_t shape_hash;
  bool operator<(const Key& o) const {
    if (determinism != o.determinism) return determinism < o.determinism;
    if (graph_fp != o.graph_fp) return graph_fp < o.graph_fp;
    return shape_hash < o.shape_hash;
  }
};

// Never destroyed: programs hold device memory that must not be released
// after the HIP runtime has shut down at process exit.
std::mutex g_cache_mu;
auto* g_cache = new std::map<Key, std::shared_ptr<Program>>();
std::atomic<int64_t> g_compiles{0};
std::atomic<int64_t> g_replays{0};  // executions run as a captured graph (test hook)

int fail(const std::string& m) {
  rt_set_error(m);
  return -1;
}

bool hip_ok(hipError_t e, const char* what) {
  if (e == hipSuccess) return true;
  rt_set_error(std::string("HIP backend: ") + what + ": " + hipGetErrorString(e));
  return false;
}

// compile_or_get_cached (plan_cache.rs:21-51).
std::shared_ptr<Program> compile_cached(const volta_rt_graph* g, int determinism) {
  if (!g) {
    rt_set_error("HIP backend: graph is NULL");
    return nullptr;
  }
  if (determinism < 0 || determinism > 2) {
    rt_set_error("HIP backend: determinism must be 0 (Strict), 1 (Balanced) or 2 (Fast)");
    return nullptr;
  }
  const Key key{determinism, g->graph_fingerprint, g->shape_signature_hash};
  std::vector<int64_t> canon;
  {
    std::lock_guard<std::mutex> lk(g_cache_mu);
    auto it = g_cache->find(key);
    if (it != g_cache->end()) {
      canon = rt_canonical(*g);
      if (it->second->canon == canon) return it->second;
    }
  }
  if (canon.empty()) canon = rt_canonical(*g);
  auto p = std::make_shared<Program>();
  std::string err;
  if (!rt_lower(*g, &p->low, &err)) {
    rt_set_error(err);
    return nullptr;
  }
  p->canon = std::move(canon);
  p->info.schedule_len = g->n_ordered;
  p->info.peak_bytes = g->peak_bytes;
  p->info.fingerprint = p->low.fingerprint;
  std::lock_guard<std::mutex> lk(g_cache_mu);
  (*g_cache)[key] = p;
  g_compiles.fetch_add(1);
  return p;
}

// Plan of layer ly's product for `rows` rows; vec when every operand and the
// output allow 16-byte accesses.
GemmPlan layer_plan(const RtLayer& ly, int64_t rows, bool vec, int num_cus) {
  return gemm_plan(GEMM_NN, (int)rows, ly.c, ly.r, vec && ly.r % 4 == 0 && ly.c % 4 == 0, num_cus);
}

DevState* device_state(Program* p, std::string* err) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    *err = std::string("HIP backend: no device: ") + hipGetErrorString(e);
    return nullptr;
  }
  auto it = p->dev.find(dev);
  if (it != p->dev.end()) return &it->second;
  DevState s;
  if ((e = hipDeviceGetAttribute(&s.num_cus, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) {
    *err = std::string("HIP backend: device query: ") + hipGetErrorString(e);
    return nullptr;
  }
  const RtLowered& L = p->low;
  int max_c = 1, max_tiles = 1;
  // the plans are fixed here, with the workspace and counters they need
  for (const RtLayer& ly : L.layers) {
    max_c = std::max(max_c, ly.c);
    for (int vec = 0; vec < 2; ++vec) {
      const GemmPlan gp = layer_plan(ly, L.rows, vec == 1, s.num_cus);
      s.plans[vec].push_back(gp);
      s.ws_floats = std::max(s.ws_floats, gp.workspace_floats((int)L.rows, ly.c));
      max_tiles = std::max(max_tiles, gp.tiles((int)L.rows, ly.c));
    }
  }
  const size_t buf_bytes = ((size_t)L.rows * max_c * sizeof(float) + 255) / 256 * 256;
  const size_t ws_bytes = (s.ws_floats * sizeof(float) + 255) / 256 * 256;
  const size_t ctr_bytes = ((size_t)(max_tiles + 1) * sizeof(unsigned) + 255) / 256 * 256;
  const size_t zero_bytes = ((size_t)max_c * sizeof(float) + 255) / 256 * 256;
  const size_t sc_bytes = (sizeof(DevScalars) + 255) / 256 * 256;
  const size_t total = 2 * buf_bytes + ws_bytes + ctr_bytes + zero_bytes + sc_bytes;
  if ((e = hipMalloc(&s.arena, total)) != hipSuccess) {
    *err = std::string("HIP backend: hipMalloc of ") + std::to_string(total) + " bytes: " + hipGetErrorString(e);
    return nullptr;
  }
  char* a = static_cast<char*>(s.arena);
  s.buf[0] = reinterpret_cast<float*>(a);
  s.buf[1] = reinterpret_cast<float*>(a + buf_bytes);
  s.ws = ws_bytes ? reinterpret_cast<float*>(a + 2 * buf_bytes) : nullptr;
  s.counters = reinterpret_cast<unsigned*>(a + 2 * buf_bytes + ws_bytes);
  s.zeros = reinterpret_cast<float*>(a + 2 * buf_bytes + ws_bytes + ctr_bytes);
  s.scalars = reinterpret_cast<DevScalars*>(a + 2 * buf_bytes + ws_bytes + ctr_bytes + zero_bytes);
  if ((e = hipStreamCreate(&s.stream)) != hipSuccess ||
      (e = hipMemsetAsync(a + 2 * buf_bytes + ws_bytes, 0, ctr_bytes + zero_bytes + sc_bytes, s.stream)) !=
          hipSuccess ||
      (e = hipStreamSynchronize(s.stream)) != hipSuccess) {
    *err = std::string("HIP backend: device state: ") + hipGetErrorString(e);
    if (s.stream) (void)hipStreamDestroy(s.stream);
    (void)hipFree(s.arena);
    return nullptr;
  }
  return &(p->dev[dev] = s);
}

// The launches of layers 0..last on s's stream, the last one ending at
// `target_stage`: one forward GEMM per layer (bias and activation in the
// epilogue), then the row softmax where the value asks for it.
bool enqueue_layers(const RtLowered& L, DevState& s, int last, int target_stage, const float* const* bindings,
                    float* out) {
  for (int i = 0; i <= last; ++i) {
    const RtLayer& ly = L.layers[i];
    const int full = ly.softmax ? RT_SOFTMAX : ly.act != RT_ACT_NONE ? RT_ACT : ly.b_binding >= 0 ? RT_PRE : RT_MM;
    const int stage = i == last ? target_stage : full;
    GemmArgs a{};
    a.A = i == 0 ? bindings[ly.x_binding] : s.buf[(i - 1) & 1];
    a.lda = ly.r;
    a.B = bindings[ly.w_binding];
    a.ldb = ly.c;
    a.M = (int)L.rows;
    a.N = ly.c;
    a.K = ly.r;
    a.partial = s.ws;
    a.counters = s.counters;
    a.epi.scalars = s.scalars;
    a.epi.ldc = ly.c;
    a.epi.out = i == last ? out : s.buf[i & 1];
    const float* bias = ly.b_binding >= 0 ? bindings[ly.b_binding] : nullptr;
    if (stage == RT_MM || (stage != RT_PRE && !bias && ly.act == RT_ACT_NONE)) {
      a.epi.kind = EPI_STORE;
    } else {
      a.epi.kind = EPI_BIAS_ACT;
      a.epi.bias = bias ? bias : s.zeros;
      a.epi.act = stage == RT_PRE ? kIdentity : device_act(ly.act);
    }
    const bool vec = aligned16(a.A) && aligned16(a.B) && aligned16(a.epi.out) &&
                     (a.epi.kind != EPI_BIAS_ACT || aligned16(a.epi.bias));
    if (!hip_ok(gemm_launch(s.plans[vec ? 1 : 0][i], a, s.stream), "layer launch")) return false;
    if (stage == RT_SOFTMAX) {
      hipLaunchKernelGGL(rt_softmax_rows, dim3((unsigned)((L.rows + 3) / 4)), dim3(256), 0, s.stream, out,
                         (int)L.rows, ly.c);
      if (!hip_ok(hipGetLastError(), "softmax launch")) return false;
    }
  }
  return true;
}

int execute(const volta_rt_graph* g, int determinism, int32_t target, bool terminal, const float* const* bindings,
            float* out, int64_t out_capacity, int64_t* out_shape) {
  std::shared_ptr<Program> prog = compile_cached(g, determinism);
  if (!prog) return -1;
  const RtLowered& L = prog->low;
  if (terminal) target = L.terminal;
  auto vit = L.values.find(target);
  if (vit == L.values.end())
    return fail("HIP backend: ValueId " + std::to_string(target) + " is not computed by this graph");
  const RtValue tv = vit->second;
  int64_t rows, cols;
  if (tv.stage == RT_BOUND) {
    rows = g->bindings[tv.binding].rows;
    cols = g->bindings[tv.binding].cols;
  } else {
    rows = L.rows;
    cols = L.layers[tv.layer].c;
  }
  if (out_shape) {
    out_shape[0] = rows;
    out_shape[1] = cols;
  }
  if (!out || !bindings) return fail("HIP backend: output or binding table is NULL");
  if (out_capacity < rows * cols)
    return fail("HIP backend: the output holds " + std::to_string(out_capacity) + " floats; value " +
                std::to_string(target) + " has " + std::to_string(rows * cols));
  const int last = tv.stage == RT_BOUND ? -1 : tv.layer;
  for (int i = 0; i <= last; ++i) {
    const RtLayer& ly = L.layers[i];
    if ((ly.x_binding >= 0 && !bindings[ly.x_binding]) || !bindings[ly.w_binding] ||
        (ly.b_binding >= 0 && !bindings[ly.b_binding]))
      return fail("HIP backend: a binding layer " + std::to_string(i) + " reads is NULL");
  }
  if (tv.stage == RT_BOUND && !bindings[tv.binding]) return fail("HIP backend: the requested binding is NULL");

  std::lock_guard<std::mutex> lk(prog->mu);
  std::string err;
  DevState* s = device_state(prog.get(), &err);
  if (!s) return fail(err);
  if (tv.stage == RT_BOUND) {
    if (!hip_ok(hipMemcpyAsync(out, bindings[tv.binding], (size_t)rows * cols * sizeof(float),
                               hipMemcpyDeviceToDevice, s->stream), "copy") ||
        !hip_ok(hipStreamSynchronize(s->stream), "synchronize"))
      return -1;
    return 0;
  }
  // By default the launches are enqueued directly: the layers depend on each
  // other, the host enqueues them faster than the GPU runs them, and a
  // replay of the same sequence captured as a hipGraph measured slower in
  // every dispatch mode (C2 topology, 64 rows: 35 us per call direct, 40-47
  // us replayed; C5, 4096 rows: 1.60 vs 1.64 ms).  With VOLTA_RT_GRAPH=1 the
  // sequence is keyed by the pointers it reads and writes: a graph of its
  // launches is captured when a key comes again among the last kRecent
  // sequences run directly, and replayed whenever it comes after that (an
  // LRU of kMaxCaptured per program and device); callers that pass new
  // pointers every call still run the launches directly.
  std::vector<const void*> key;
  key.reserve(3 * (last + 1) + 1);
  for (int i = 0; i <= last; ++i) {
    const RtLayer& ly = L.layers[i];
    key.push_back(ly.x_binding >= 0 ? bindings[ly.x_binding] : nullptr);
    key.push_back(bindings[ly.w_binding]);
    key.push_back(ly.b_binding >= 0 ? bindings[ly.b_binding] : nullptr);
  }
  key.push_back(out);
  const char* eg = std::getenv("VOLTA_RT_GRAPH");
  const bool use_graph = eg && *eg && *eg != '0';
  ++s->tick;
  Captured* hit = nullptr;
  if (use_graph)
    for (Captured& c : s->captured)
      if (c.last == last && c.stage == tv.stage && c.key == key) hit = &c;
  auto seen = std::find_if(s->recent.begin(), s->recent.end(), [&](const Captured& c) {
    return c.last == last && c.stage == tv.stage && c.key == key;
  });
  if (!hit && use_graph && seen != s->recent.end()) {
    s->recent.erase(seen);
    if (s->captured.size() >= kMaxCaptured) {
      auto lru = std::min_element(s->captured.begin(), s->captured.end(),
                                  [](const Captured& x, const Captured& y) { return x.used < y.used; });
      (void)hipGraphExecDestroy(lru->exec);
      s->captured.erase(lru);
    }
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    if (!hip_ok(hipStreamBeginCapture(s->stream, hipStreamCaptureModeThreadLocal), "begin capture")) return -1;
    const bool queued = enqueue_layers(L, *s, last, tv.stage, bindings, out);
    const hipError_t ec = hipStreamEndCapture(s->stream, &graph);
    if (!queued || !hip_ok(ec, "end capture")) {
      if (graph) (void)hipGraphDestroy(graph);
      return -1;
    }
    const hipError_t ei = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (!hip_ok(ei, "instantiate")) return -1;
    Captured c;
    c.last = last;
    c.stage = tv.stage;
    c.key = key;
    c.exec = exec;
    s->captured.push_back(std::move(c));
    hit = &s->captured.back();
  }
  if (hit) {
    hit->used = s->tick;
    if (!hip_ok(hipGraphLaunch(hit->exec, s->stream), "graph launch")) return -1;
    g_replays.fetch_add(1);
  } else {
    if (!enqueue_layers(L, *s, last, tv.stage, bindings, out)) return -1;
    if (seen == s->recent.end()) {
      if (s->recent.size() >= kRecent) s->recent.erase(s->recent.begin());
      Captured c;
      c.last = last;
      c.stage = tv.stage;
      c.key = std::move(key);
      s->recent.push_back(std::move(c));
    }
  }
  return hip_ok(hipStreamSynchronize(s->stream), "synchronize") ? 0 : -1;
}

}  // namespace
}  // namespace volta

using namespace volta;

extern "C" {

int32_t volta_rt_compile(const volta_rt_graph* g, int32_t determinism, volta_rt_compiled* out) {
  std::shared_ptr<Program> p = compile_cached(g, determinism);
  if (!p) return -1;
  if (out) *out = p->info;
  return 0;
}

int32_t volta_rt_execute_value(const volta_rt_graph* g, int32_t determinism, int32_t target,
                               const float* const* bindings, float* out, int64_t out_capacity, int64_t* out_shape) {
  return execute(g, determinism, target, false, bindings, out, out_capacity, out_shape);
}

int32_t volta_rt_execute_terminal(const volta_rt_graph* g, int32_t determinism, const float* const* bindings,
                                  float* out, int64_t out_capacity, int64_t* out_shape) {
  return execute(g, determinism, -1, true, bindings, out, out_capacity, out_shape);
}

void volta_rt_clear_plan_cache(void) {
  std::lock_guard<std::mutex> lk(g_cache_mu);
  g_cache->clear();
}

int64_t volta_rt_compile_count(void) { return g_compiles.load(); }

// Test hook: how many executions ran as a replay of a captured graph.
int64_t volta_hip_rt_graph_replays(void) { return g_replays.load(); }

}  // extern "C"
