// MLP spec helpers shared by the HIP library and the CPU oracle: defaults,
// validation and the text form "512-1024-1-...:relu:adam[:mse|:ce][:k=v]".
//
// The defaults are the constants the reference's generator bakes into the
// step (mlp_train_rust_codegen.rs:807-813): beta1 0.9, beta2 0.999,
// eps 1e-8, AdamW weight decay 0.01.  Activation and optimizer names follow
// mlp_train_rust_codegen.rs:264-278.
#include "spec.h"

#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <cmath>
#include <cstring>
#include <mutex>
#include <string>

namespace volta {

static thread_local std::string g_last_error;

void set_last_error(const std::string& msg) { g_last_error = msg; }
const char* last_error() { return g_last_error.c_str(); }

const char* activation_name(int a) {
  switch (a) {
    case VOLTA_ACT_RELU: return "relu";
    case VOLTA_ACT_SIGMOID: return "sigmoid";
    case VOLTA_ACT_TANH: return "tanh";
    case VOLTA_ACT_LEAKY_RELU: return "leaky_relu";
    case VOLTA_ACT_SILU: return "silu";
    case VOLTA_ACT_GELU: return "gelu";
    case VOLTA_ACT_SOFTMAX: return "softmax";
    default: return "?";
  }
}

const char* optimizer_name(int o) {
  switch (o) {
    case VOLTA_OPT_SGD: return "sgd";
    case VOLTA_OPT_ADAM: return "adam";
    case VOLTA_OPT_ADAMW: return "adamw";
    case VOLTA_OPT_ADAGRAD: return "adagrad";
    default: return "?";
  }
}

bool validate_spec(const volta_mlp_spec& s, std::string* why) {
  auto fail = [&](const std::string& m) {
    if (why) *why = m;
    return false;
  };
  if (s.n_sizes < 2 || s.n_sizes > VOLTA_MAX_LAYER_SIZES)
    return fail("n_sizes must be in [2, " + std::to_string(VOLTA_MAX_LAYER_SIZES) + "]");
  for (int i = 0; i < s.n_sizes; ++i)
    if (s.sizes[i] <= 0 || s.sizes[i] > (1 << 20))
      return fail("layer size " + std::to_string(i) + " out of range (1..1048576)");
  for (int i = 0; i + 1 < s.n_sizes; ++i)
    if ((int64_t)s.sizes[i] * s.sizes[i + 1] >= ((int64_t)1 << 30))
      return fail("layer " + std::to_string(i) + " has 2^30 or more weights");
  if (s.activation < VOLTA_ACT_RELU || s.activation > VOLTA_ACT_SOFTMAX)
    return fail("unknown activation");
  if (s.optimizer < VOLTA_OPT_SGD || s.optimizer > VOLTA_OPT_ADAGRAD)
    return fail("unknown optimizer");
  if (s.loss != VOLTA_LOSS_MSE && s.loss != VOLTA_LOSS_SOFTMAX_CE) return fail("unknown loss");
  if (s.loss == VOLTA_LOSS_SOFTMAX_CE && s.sizes[s.n_sizes - 1] < 2)
    return fail("softmax cross-entropy needs at least 2 output classes");
  if (!(s.eps > 0.0f)) return fail("eps must be > 0");
  if (!(s.beta1 >= 0.0f && s.beta1 < 1.0f)) return fail("beta1 must be in [0, 1)");
  if (!(s.beta2 >= 0.0f && s.beta2 < 1.0f)) return fail("beta2 must be in [0, 1)");
  if (!(s.weight_decay >= 0.0f)) return fail("weight_decay must be >= 0");
  if (!(s.clip_grad >= 0.0f) || std::isinf(s.clip_grad)) return fail("clip_grad must be finite and >= 0");
  if (!(s.dropout_p >= 0.0f && s.dropout_p < 1.0f)) return fail("dropout_p must be in [0, 1)");
  if (s.layernorm != 0 && s.layernorm != 1) return fail("layernorm must be 0 or 1");
  return true;
}

}  // namespace volta

using volta::set_last_error;

extern "C" void volta_mlp_spec_default(volta_mlp_spec* spec, int32_t n_sizes,
                                       const int32_t* sizes, int32_t activation,
                                       int32_t optimizer, int32_t loss) {
  if (!spec) return;
  std::memset(spec, 0, sizeof(*spec));
  spec->n_sizes = n_sizes;
  for (int i = 0; i < n_sizes && i < VOLTA_MAX_LAYER_SIZES && sizes; ++i)
    spec->sizes[i] = sizes[i];
  spec->activation = activation;
  spec->optimizer = optimizer;
  spec->loss = loss;
  spec->beta1 = 0.9f;
  spec->beta2 = 0.999f;
  spec->eps = 1e-8f;
  spec->weight_decay = optimizer == VOLTA_OPT_ADAMW ? 0.01f : 0.0f;
}

static bool parse_float(const std::string& s, float* out) {
  errno = 0;
  char* end = nullptr;
  float v = std::strtof(s.c_str(), &end);
  if (errno != 0 || end == s.c_str() || *end != '\0') return false;
  *out = v;
  return true;
}

extern "C" int32_t volta_mlp_spec_parse(const char* text, volta_mlp_spec* spec) {
  if (!text || !spec) {
    set_last_error("volta_mlp_spec_parse: null argument");
    return -1;
  }
  std::string t(text);
  std::vector<std::string> fields;
  size_t pos = 0;
  while (true) {
    size_t q = t.find(':', pos);
    fields.push_back(t.substr(pos, q == std::string::npos ? std::string::npos : q - pos));
    if (q == std::string::npos) break;
    pos = q + 1;
  }
  if (fields.size() < 3) {
    set_last_error("spec must be 'sizes:activation:optimizer[:loss][:key=value...]'");
    return -1;
  }
  int32_t sizes[VOLTA_MAX_LAYER_SIZES];
  int n = 0;
  {
    const std::string& f = fields[0];
    size_t p = 0;
    while (p <= f.size()) {
      size_t q = f.find_first_of("-,x", p);
      std::string tok = f.substr(p, q == std::string::npos ? std::string::npos : q - p);
      char* end = nullptr;
      long v = std::strtol(tok.c_str(), &end, 10);
      if (tok.empty() || *end != '\0' || v <= 0 || n >= VOLTA_MAX_LAYER_SIZES) {
        set_last_error("bad layer size list '" + f + "'");
        return -1;
      }
      sizes[n++] = (int32_t)v;
      if (q == std::string::npos) break;
      p = q + 1;
    }
  }
  int act = -1;
  {
    const std::string& a = fields[1];
    if (a == "relu" || a.empty()) act = VOLTA_ACT_RELU;
    else if (a == "sigmoid") act = VOLTA_ACT_SIGMOID;
    else if (a == "tanh") act = VOLTA_ACT_TANH;
    else if (a == "leaky_relu" || a == "leakyrelu") act = VOLTA_ACT_LEAKY_RELU;
    else if (a == "silu") act = VOLTA_ACT_SILU;
    else if (a == "gelu") act = VOLTA_ACT_GELU;
    else if (a == "softmax") act = VOLTA_ACT_SOFTMAX;
    else {
      set_last_error("unknown activation '" + a + "'");
      return -1;
    }
  }
  int opt = -1;
  {
    const std::string& o = fields[2];
    if (o == "sgd" || o.empty()) opt = VOLTA_OPT_SGD;
    else if (o == "adam") opt = VOLTA_OPT_ADAM;
    else if (o == "adamw") opt = VOLTA_OPT_ADAMW;
    else if (o == "adagrad") opt = VOLTA_OPT_ADAGRAD;
    else {
      set_last_error("unknown optimizer '" + o + "'");
      return -1;
    }
  }
  volta_mlp_spec s;
  volta_mlp_spec_default(&s, n, sizes, act, opt, VOLTA_LOSS_MSE);
  for (size_t i = 3; i < fields.size(); ++i) {
    const std::string& f = fields[i];
    if (f == "mse") {
      s.loss = VOLTA_LOSS_MSE;
      continue;
    }
    if (f == "ce" || f == "softmax_ce" || f == "cross_entropy") {
      s.loss = VOLTA_LOSS_SOFTMAX_CE;
      continue;
    }
    if (f == "ln" || f == "layernorm") {
      s.layernorm = 1;
      continue;
    }
    size_t eq = f.find('=');
    if (eq == std::string::npos) {
      set_last_error("unknown spec field '" + f + "'");
      return -1;
    }
    std::string key = f.substr(0, eq), val = f.substr(eq + 1);
    float v;
    if (!parse_float(val, &v)) {
      set_last_error("bad number in spec field '" + f + "'");
      return -1;
    }
    if (key == "eps") s.eps = v;
    else if (key == "wd" || key == "weight_decay") s.weight_decay = v;
    else if (key == "beta1" || key == "b1") s.beta1 = v;
    else if (key == "beta2" || key == "b2") s.beta2 = v;
    else if (key == "clip" || key == "clip_grad") s.clip_grad = v;
    else if (key == "dropout") s.dropout_p = v;
    else {
      set_last_error("unknown spec key '" + key + "'");
      return -1;
    }
  }
  std::string why;
  if (!volta::validate_spec(s, &why)) {
    set_last_error("invalid spec: " + why);
    return -1;
  }
  *spec = s;
  return 0;
}

extern "C" const char* volta_train_last_error(void) { return volta::last_error(); }

namespace {
std::mutex g_spec_mu;
bool g_spec_set = false;
volta_mlp_spec g_spec;
}  // namespace

extern "C" int32_t volta_train_configure(const volta_mlp_spec* spec) {
  if (!spec) {
    set_last_error("volta_train_configure: null spec");
    return -1;
  }
  std::string why;
  if (!volta::validate_spec(*spec, &why)) {
    set_last_error("volta_train_configure: invalid spec: " + why);
    return -1;
  }
  std::lock_guard<std::mutex> lk(g_spec_mu);
  g_spec = *spec;
  g_spec_set = true;
  return 0;
}

bool volta::resolve_default_spec(volta_mlp_spec* out) {
  {
    std::lock_guard<std::mutex> lk(g_spec_mu);
    if (g_spec_set) {
      *out = g_spec;
      return true;
    }
  }
  const char* env = std::getenv("VOLTA_MLP_SPEC");
  if (!env || !*env) {
    set_last_error(
        "volta_train_init: no topology; call volta_train_configure or set VOLTA_MLP_SPEC");
    return false;
  }
  return volta_mlp_spec_parse(env, out) == 0;
}
