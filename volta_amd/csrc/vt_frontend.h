// Front end for `compile-train`: the MLP subset of the Volta language (.vt),
// reduced to the spec of the training library.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "../../include/volta_train.h"

namespace volta {

struct VtTrainPlan {
  volta_mlp_spec spec{};
  std::string model;          // first model declared (the one compile-train builds)
  bool rust = true;           // compile-train --rust (else the default C path)
  bool trained = false;       // a `train <model> on <dataset>` statement names it
  double lr = 0.0;            // resolved learning rate of the last such statement (0: none)
  int64_t epochs = 0;         // its resolved epochs
  int64_t batch = 0;          // its resolved batch
  std::vector<std::string> notes;  // what the reference would do that this build does not
};

// Parse `source` and resolve the first model as `volta compile-train --rust`
// (rust) or plain `volta compile-train` (the C path) does (executor.rs:
// 1759-1863, guards :3147-3189).  Returns false with a message (line:column:
// text) on a parse error or an unsupported model.
bool vt_compile_train_plan(const std::string& source, VtTrainPlan* plan, std::string* error, bool rust = true);

// The model `volta compile` builds an inference library for (main.rs:
// 158-215 -> executor.rs:1684-1744): the first model's layers, and the
// hidden activation of the forward graph lower_model_to_graph builds for it
// (lowering.rs:87-140): ReLU for activation 'relu', none for every other
// activation the lowering drops.  'sigmoid' (a Sigmoid node) and 'softmax' (a
// final Softmax node) fail as the reference's inference codegen fails on
// those ops (codegen/inner.rs:395-399).  No compile-train guard applies: the
// reference trains the model in its interpreter first.
struct VtInferPlan {
  std::string model;
  std::vector<int> sizes;
  std::string activation;   // model.activation as written
  bool relu_hidden = true;  // false: hidden layers without activation
  bool trained = false;     // a `train` statement names the model
  std::vector<std::string> notes;
};
bool vt_compile_infer_plan(const std::string& source, VtInferPlan* plan, std::string* error);

// One-line description of a plan ("model=... layers=a-b-c activation=...").
std::string vt_plan_summary(const VtTrainPlan& plan);

}  // namespace volta
