// Lowering of a runtime MLP graph (include/volta_backend.h, volta_rt_graph)
// onto the forward GEMM kernels: host code, shared by the HIP backend's
// compile and execute calls.
#pragma once

#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/volta_backend.h"

namespace volta {

// Where a ValueId of the chain sits: a bound tensor, or a stage of layer i.
enum RtStage { RT_BOUND = 0, RT_MM = 1, RT_PRE = 2, RT_ACT = 3, RT_SOFTMAX = 4 };

// Activations of the runtime graph (interpreter semantics,
// kernels/activations.rs:7-166).
enum RtAct { RT_ACT_NONE = 0, RT_ACT_RELU = 1, RT_ACT_SIGMOID = 2, RT_ACT_GELU = 3 };

struct RtLayer {
  int x_binding = -1;  // first layer: its bound input; later layers: -1 (previous output)
  int w_binding = -1;
  int b_binding = -1;  // -1: no bias
  int r = 0, c = 0;
  int act = RT_ACT_NONE;
  bool softmax = false;
};

struct RtValue {
  int stage = RT_BOUND;
  int layer = -1;    // chain stages
  int binding = -1;  // RT_BOUND
};

struct RtLowered {
  int64_t rows = 0;                           // rows of the chain (the batch)
  std::vector<RtLayer> layers;
  std::unordered_map<int32_t, RtValue> values;  // every ValueId the backend can return
  int32_t terminal = -1;                      // execute_terminal's value
  uint64_t fingerprint = 0;                   // CompiledProgram::fingerprint
};

// Lowers g; false with a message naming the node on anything outside the
// subset the header describes.
bool rt_lower(const volta_rt_graph& g, RtLowered* out, std::string* err);

// g as a flat list (nodes, schedule, bindings, peak bytes): two graphs with
// equal lists lower to the same program.
std::vector<int64_t> rt_canonical(const volta_rt_graph& g);

// Sets the text volta_rt_last_error returns on this thread.
void rt_set_error(const std::string& m);

}  // namespace volta
