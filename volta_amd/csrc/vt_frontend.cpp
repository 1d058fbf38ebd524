// .vt front end for compile-train: lexes the indentation-structured Volta
// source (frontend/lexer.rs: 4-space indents, '#' comments, no tabs), parses
// the model / dataset / train statements (frontend/parser.rs:136-181) and
// resolves the first model the way `volta compile-train --rust` does
// (executor.rs:1806-1863): layers and activation from the model block, the
// optimizer from the last `train` statement naming the model (autopilot
// precedence train > model > rule, autopilot.rs:143-160) or, with no train
// statement, the model's own optimizer or SGD; then the compile-train guards
// (executor.rs:3147-3189) and this library's own limits.
#include "vt_frontend.h"

#include "../../include/volta_vt.h"

#include <algorithm>
#include <cctype>
#include <cmath>
#include <cstdio>
#include <map>
#include <sstream>

#include "spec.h"

namespace volta {
namespace {

enum TokKind { T_IDENT, T_INT, T_FLOAT, T_STR, T_SYM };

struct Tok {
  TokKind kind;
  std::string text;
  double num = 0.0;
  int line = 0, col = 0;
};

struct Line {
  int indent = 0;  // columns of leading spaces
  int number = 0;
  std::vector<Tok> toks;
};

struct Fail {
  std::string msg;
};

[[noreturn]] void fail_at(int line, int col, const std::string& m) {
  throw Fail{std::to_string(line) + ":" + std::to_string(col) + ": " + m};
}

// Split the source into non-blank logical lines of tokens.
std::vector<Line> lex(const std::string& src) {
  std::vector<Line> out;
  std::istringstream in(src);
  std::string raw;
  int number = 0;
  while (std::getline(in, raw)) {
    ++number;
    if (!raw.empty() && raw.back() == '\r') raw.pop_back();
    size_t i = 0;
    while (i < raw.size() && (raw[i] == ' ' || raw[i] == '\t')) {
      if (raw[i] == '\t') fail_at(number, (int)i + 1, "tabs are not allowed for indentation; use 4 spaces");
      ++i;
    }
    Line ln;
    ln.indent = (int)i;
    ln.number = number;
    while (i < raw.size()) {
      const char c = raw[i];
      const int col = (int)i + 1;
      if (c == ' ' || c == '\t') {
        ++i;
      } else if (c == '#') {
        break;
      } else if (std::isdigit((unsigned char)c)) {
        size_t j = i;
        while (j < raw.size() && std::isdigit((unsigned char)raw[j])) ++j;
        bool flt = false;
        if (j + 1 < raw.size() && raw[j] == '.' && std::isdigit((unsigned char)raw[j + 1])) {
          flt = true;
          ++j;
          while (j < raw.size() && std::isdigit((unsigned char)raw[j])) ++j;
        }
        Tok t{flt ? T_FLOAT : T_INT, raw.substr(i, j - i), 0.0, number, col};
        t.num = std::strtod(t.text.c_str(), nullptr);
        ln.toks.push_back(t);
        i = j;
      } else if (std::isalpha((unsigned char)c) || c == '_') {
        size_t j = i;
        while (j < raw.size() && (std::isalnum((unsigned char)raw[j]) || raw[j] == '_')) ++j;
        ln.toks.push_back({T_IDENT, raw.substr(i, j - i), 0.0, number, col});
        i = j;
      } else if (c == '"') {
        std::string s;
        size_t j = i + 1;
        bool closed = false;
        while (j < raw.size()) {
          if (raw[j] == '"') {
            closed = true;
            ++j;
            break;
          }
          if (raw[j] == '\\' && j + 1 < raw.size()) {
            const char e = raw[j + 1];
            s += e == 'n' ? '\n' : e == 't' ? '\t' : e == 'r' ? '\r' : e;
            j += 2;
            continue;
          }
          s += raw[j++];
        }
        if (!closed) fail_at(number, col, "unclosed string literal");
        ln.toks.push_back({T_STR, s, 0.0, number, col});
        i = j;
      } else {
        static const char* two[] = {"==", "!=", ">=", "<=", "->", ".."};
        std::string sym(1, c);
        for (const char* t : two)
          if (raw.compare(i, 2, t) == 0) sym = t;
        ln.toks.push_back({T_SYM, sym, 0.0, number, col});
        i += sym.size();
      }
    }
    if (!ln.toks.empty()) out.push_back(ln);
  }
  return out;
}

// A property value after '-' folding: number, symbol (identifier or
// keyword), string or bool.
struct Value {
  enum Kind { NUM, INT, SYM, STR } kind;
  double num = 0.0;
  std::string text;
  int line = 0, col = 0;
};

struct Property {
  std::string key;
  std::vector<Value> values;
  int line = 0, col = 0;
};

struct Block {
  std::vector<Property> props;
};

Property parse_property(const Line& ln, const std::map<std::string, double>& vars) {
  Property p;
  const auto& t = ln.toks;
  if (t[0].kind != T_IDENT) fail_at(ln.number, t[0].col, "invalid property: missing property key");
  p.key = t[0].text;
  p.line = ln.number;
  p.col = t[0].col;
  for (size_t k = 1; k < t.size(); ++k) {
    Value v;
    v.line = ln.number;
    v.col = t[k].col;
    if (t[k].kind == T_SYM && t[k].text == "-") {
      if (k + 1 >= t.size() || (t[k + 1].kind != T_INT && t[k + 1].kind != T_FLOAT))
        fail_at(ln.number, t[k].col, "invalid property value; '-' must be followed by a number");
      ++k;
      v.kind = t[k].kind == T_INT ? Value::INT : Value::NUM;
      v.num = -t[k].num;
    } else if (t[k].kind == T_INT || t[k].kind == T_FLOAT) {
      v.kind = t[k].kind == T_INT ? Value::INT : Value::NUM;
      v.num = t[k].num;
    } else if (t[k].kind == T_STR) {
      v.kind = Value::STR;
      v.text = t[k].text;
    } else if (t[k].kind == T_IDENT) {
      auto it = vars.find(t[k].text);
      if (it != vars.end()) {  // a top-level numeric variable
        v.kind = std::floor(it->second) == it->second ? Value::INT : Value::NUM;
        v.num = it->second;
      } else {
        v.kind = Value::SYM;
        v.text = t[k].text;
      }
    } else {
      fail_at(ln.number, t[k].col, "invalid property value '" + t[k].text + "'");
    }
    p.values.push_back(v);
  }
  if (p.values.empty()) fail_at(ln.number, t[0].col, "invalid property structure: missing property value");
  return p;
}

const Property* find(const Block& b, const char* key) {
  for (const auto& p : b.props)
    if (p.key == key) return &p;
  return nullptr;
}

void check_unique(const Block& b, const char* ctx) {
  for (size_t i = 0; i < b.props.size(); ++i)
    for (size_t j = 0; j < i; ++j)
      if (b.props[i].key == b.props[j].key)
        fail_at(b.props[i].line, b.props[i].col, "duplicate '" + b.props[i].key + "' in " + ctx + " block");
}

void warn_unknown(const Block& b, const char* ctx, std::initializer_list<const char*> known,
                  std::vector<std::string>* notes) {
  for (const auto& p : b.props) {
    bool ok = false;
    for (const char* k : known) ok = ok || p.key == k;
    if (!ok) notes->push_back("unknown property '" + p.key + "' in " + ctx + " block (ignored)");
  }
}

const Value& single(const Property& p, const std::string& label) {
  if (p.values.size() != 1) fail_at(p.line, p.col, label + " expects exactly one value");
  return p.values[0];
}

int64_t int_of(const Value& v, const std::string& label) {
  if (v.kind != Value::INT) fail_at(v.line, v.col, label + " expects an integer");
  return (int64_t)v.num;
}

double num_of(const Value& v, const std::string& label) {
  if (v.kind != Value::INT && v.kind != Value::NUM) fail_at(v.line, v.col, label + " expects a number");
  return v.num;
}

std::string sym_of(const Value& v, const std::string& label) {
  if (v.kind != Value::SYM && v.kind != Value::STR) fail_at(v.line, v.col, label + " expects a name");
  std::string s = v.text;
  std::transform(s.begin(), s.end(), s.begin(), [](unsigned char c) { return (char)std::tolower(c); });
  return s;
}

void allowed(const Value& v, const std::string& label, const std::string& s,
             std::initializer_list<const char*> names) {
  for (const char* n : names)
    if (s == n) return;
  std::string all;
  for (const char* n : names) all += std::string(all.empty() ? "" : ", ") + n;
  fail_at(v.line, v.col, "invalid property: " + label + " has invalid value '" + s + "'; allowed: " + all);
}

// language-level names (rules.rs:39-49)
const std::initializer_list<const char*> kActivations = {"relu", "sigmoid", "tanh", "softmax", "leaky_relu",
                                                         "leakyrelu", "silu", "gelu"};
const std::initializer_list<const char*> kOptimizers = {"adam", "adamw", "sgd", "rmsprop", "rms_prop", "adagrad"};
const std::initializer_list<const char*> kDevices = {"cpu", "gpu", "cuda", "auto"};

struct Statement {
  std::string kind;  // model / dataset / train
  std::string name, data;
  Block block;
  int line = 0;
};

// The three commands that resolve the first model: compile-train on the C
// path, compile-train --rust, and compile (the inference library).
enum PlanMode { PLAN_C, PLAN_RUST, PLAN_INFER };

bool plan_first_model(const std::string& source, PlanMode mode, VtTrainPlan* plan, std::string* act_name,
                      std::string* error) {
  const bool rust = mode == PLAN_RUST;
  try {
    const std::vector<Line> lines = lex(source);
    std::vector<Statement> stmts;
    std::map<std::string, double> vars;
    std::vector<std::string> notes;
    bool after_if = false;  // the previous top-level statement was an if / elif block
    for (size_t li = 0; li < lines.size();) {
      const Line& ln = lines[li];
      if (ln.indent != 0) fail_at(ln.number, 1, "unexpected indentation");
      const Tok& head = ln.toks[0];
      Statement st;
      st.line = ln.number;
      const std::string kw = head.kind == T_IDENT ? head.text : "";
      // Statements of the language outside compile-train's input: the
      // reference's executor runs them before compiling the first model
      // (main.rs:224-246); none of them changes the generated library, so
      // they are parsed structurally (header line and indented block) and
      // noted, not run.  elif / else only follow an if block
      // (parser.rs:78-81).
      if (kw == "save" || kw == "load" || kw == "infer" || kw == "fn" || kw == "struct" || kw == "loop" ||
          kw == "for" || kw == "if" || kw == "elif" || kw == "else" || kw == "return" || kw == "precision" ||
          kw == "memory") {
        if ((kw == "elif" || kw == "else") && !after_if)
          fail_at(ln.number, head.col, "Unexpected keyword in this position");
        after_if = kw == "if" || kw == "elif";
        notes.push_back("line " + std::to_string(ln.number) + ": '" + kw +
                        "' statement not run (the reference's interpreter runs it before compiling the first "
                        "model; it does not change the generated library)");
        ++li;
        while (li < lines.size() && lines[li].indent > 0) ++li;
        continue;
      }
      after_if = false;
      if (head.kind != T_IDENT)
        fail_at(ln.number, head.col,
                "Unexpected token at start of statement (start a statement with an identifier, or a keyword "
                "such as model, dataset, train, if, loop, fn, print, save, load)");
      if (kw == "model" || kw == "dataset") {
        if (ln.toks.size() != 2 || ln.toks[1].kind != T_IDENT)
          fail_at(ln.number, head.col, "use: " + kw + " <name>");
        st.kind = kw;
        st.name = ln.toks[1].text;
      } else if (kw == "train") {
        if (ln.toks.size() != 4 || ln.toks[1].kind != T_IDENT || ln.toks[2].text != "on" ||
            ln.toks[3].kind != T_IDENT)
          fail_at(ln.number, head.col, "invalid train syntax; use: train <model_name> on <dataset_name>");
        st.kind = kw;
        st.name = ln.toks[1].text;
        st.data = ln.toks[3].text;
      } else if (kw == "print") {
        notes.push_back("line " + std::to_string(ln.number) + ": print skipped");
        ++li;
        continue;
      } else if (ln.toks.size() >= 2) {
        // top-level variable: `name <number>` or `name = <number>`
        size_t k = 1;
        if (ln.toks[k].kind == T_SYM && ln.toks[k].text == "=") ++k;
        double sign = 1.0;
        if (k < ln.toks.size() && ln.toks[k].kind == T_SYM && ln.toks[k].text == "-") {
          sign = -1.0;
          ++k;
        }
        if (k + 1 == ln.toks.size() && (ln.toks[k].kind == T_INT || ln.toks[k].kind == T_FLOAT)) {
          vars[head.text] = sign * ln.toks[k].num;
        } else {
          notes.push_back("line " + std::to_string(ln.number) + ": non-numeric variable '" + head.text +
                          "' skipped");
        }
        ++li;
        continue;
      } else {
        fail_at(ln.number, head.col,
                "Unknown keyword '" + head.text + "' (a variable needs a value: '" + head.text + " <expression>')");
      }
      ++li;
      // property block: the following lines indented by exactly 4
      if (li < lines.size() && lines[li].indent > 0) {
        if (lines[li].indent != 4) fail_at(lines[li].number, 1, "inconsistent indentation (use 4 spaces)");
        while (li < lines.size() && lines[li].indent > 0) {
          if (lines[li].indent != 4) fail_at(lines[li].number, 1, "inconsistent indentation (use 4 spaces)");
          st.block.props.push_back(parse_property(lines[li], vars));
          ++li;
        }
      } else if (st.kind == "model") {
        fail_at(st.line, 1, "missing indent for property block");
      }
      stmts.push_back(st);
    }

    // the first model declared
    const Statement* model = nullptr;
    for (const auto& s : stmts)
      if (s.kind == "model") {
        model = &s;
        break;
      }
    if (!model) throw Fail{"No models found — declare a model first"};
    const Block& mb = model->block;
    check_unique(mb, "model");
    warn_unknown(mb, "model", {"layers", "activation", "optimizer", "precision", "memory", "seed", "use",
                               "dropout", "layernorm"}, &notes);
    const Property* layers = find(mb, "layers");
    if (!layers) fail_at(model->line, 1, "invalid property: missing required property 'layers' in model");
    if (layers->values.size() < 2) fail_at(layers->line, layers->col, "model.layers must have at least 2 values");
    if ((int)layers->values.size() > VOLTA_MAX_LAYER_SIZES)
      fail_at(layers->line, layers->col, "model.layers has more than " + std::to_string(VOLTA_MAX_LAYER_SIZES) +
                                             " values (this library's limit)");
    std::vector<int> sizes;
    for (const auto& v : layers->values) {
      const int64_t x = int_of(v, "model.layers");
      if (x <= 0) fail_at(v.line, v.col, "model.layers values must be > 0, found " + std::to_string(x));
      if (x > (1 << 20)) fail_at(v.line, v.col, "model.layers value above this library's limit 1048576");
      sizes.push_back((int)x);
    }
    std::string activation = "relu";  // AUTOPILOT_DEFAULT_ACTIVATION
    if (const Property* p = find(mb, "activation")) {
      const Value& v = single(*p, "model.activation");
      activation = sym_of(v, "model.activation");
      allowed(v, "model.activation", activation, kActivations);
    }
    std::string model_opt;
    double model_lr = 0.0;
    if (const Property* p = find(mb, "optimizer")) {
      if (p->values.empty() || p->values.size() > 2) fail_at(p->line, p->col, "model.optimizer expects 1 or 2 values");
      model_opt = sym_of(p->values[0], "model.optimizer");
      allowed(p->values[0], "model.optimizer", model_opt, kOptimizers);
      if (p->values.size() == 2) {
        model_lr = num_of(p->values[1], "model.optimizer learning rate");
        if (!(model_lr > 0.0)) fail_at(p->values[1].line, p->values[1].col, "model.optimizer learning rate must be > 0");
      }
    }
    if (const Property* p = find(mb, "use"))
      fail_at(p->line, p->col,
              "Model '" + model->name + "' uses template '" + sym_of(single(*p, "model.use"), "model.use") +
                  "'. `compile-train` is MLP-only and does not support function-backed/custom training graphs.");
    // codegen extras of the model (executor.rs:1930-1971 -> :1839-1841)
    double dropout = 0.0;
    if (const Property* p = find(mb, "dropout")) {
      dropout = num_of(single(*p, "model.dropout"), "model.dropout");
      if (!(dropout >= 0.0 && dropout < 1.0)) fail_at(p->line, p->col, "model.dropout must be in [0, 1)");
    }
    bool layernorm = false;
    if (const Property* p = find(mb, "layernorm")) {
      const std::string s = sym_of(single(*p, "model.layernorm"), "model.layernorm");
      layernorm = s == "yes" || s == "true" || s == "on";
    }

    // every train statement needs a declared model and an earlier dataset
    // (executor.rs:930-957)
    for (const auto& s : stmts) {
      if (s.kind != "train") continue;
      bool have_model = false, have_data = false;
      for (const auto& d : stmts) {
        have_model = have_model || (d.kind == "model" && d.name == s.name && d.line < s.line);
        have_data = have_data || (d.kind == "dataset" && d.name == s.data && d.line < s.line);
      }
      if (!have_data) fail_at(s.line, 1, "Undefined dataset: '" + s.data + "'");
      if (!have_model) fail_at(s.line, 1, "Undefined model: '" + s.name + "'");
    }
    // train statements naming the model; the last one decides (each run
    // overwrites the model's optimizer, executor.rs:1294-1301)
    const int nlayers = (int)sizes.size();
    const Statement* train = nullptr;
    for (const auto& s : stmts) {
      if (s.kind == "train" && s.name == model->name) train = &s;
    }
    std::string optimizer;
    VtTrainPlan out;
    if (train) {
      const Block& tb = train->block;
      check_unique(tb, "train");
      warn_unknown(tb, "train", {"epochs", "device", "optimizer", "lr", "batch", "precision", "clip_grad",
                                 "weight_decay", "warmup_steps", "lr_schedule", "early_stopping",
                                 "gradient_accumulation"}, &notes);
      // autopilot precedence (autopilot.rs:130-196)
      out.epochs = 10;  // AUTOPILOT_DEFAULT_EPOCHS
      if (const Property* p = find(tb, "epochs")) {
        out.epochs = int_of(single(*p, "train.epochs"), "train.epochs");
        if (out.epochs < 0) fail_at(p->line, p->col, "train.epochs must be non-negative");
      }
      if (const Property* p = find(tb, "device")) {
        const Value& v = single(*p, "train.device");
        allowed(v, "train.device", sym_of(v, "train.device"), kDevices);
      }
      if (const Property* p = find(tb, "optimizer")) {
        const Value& v = single(*p, "train.optimizer");
        optimizer = sym_of(v, "train.optimizer");
        allowed(v, "train.optimizer", optimizer, kOptimizers);
      } else if (!model_opt.empty()) {
        optimizer = model_opt;
      } else {
        optimizer = nlayers <= 6 ? "adam" : "adamw";  // small/medium vs large model rule
      }
      out.lr = nlayers <= 3 ? 0.001 : nlayers <= 6 ? 0.0007 : 0.0003;
      if (model_lr > 0.0) out.lr = model_lr;
      if (const Property* p = find(tb, "lr")) {
        out.lr = num_of(single(*p, "train.lr"), "train.lr");
        if (!(out.lr > 0.0)) fail_at(p->line, p->col, "train.lr must be > 0");
      }
      out.batch = 32;  // AUTOPILOT_DEFAULT_BATCH
      for (const auto& d : stmts)
        if (d.kind == "dataset" && d.name == train->data)
          if (const Property* p = find(d.block, "batch")) out.batch = int_of(single(*p, "dataset.batch"), "dataset.batch");
      if (const Property* p = find(tb, "batch")) {
        out.batch = int_of(single(*p, "train.batch"), "train.batch");
        if (out.batch <= 0) fail_at(p->line, p->col, "train.batch must be > 0");
      }
      if (find(tb, "weight_decay"))
        notes.push_back("train.weight_decay shapes the interpreter's training only; the generated step "
                        "uses the compile-train constant (AdamW 0.01 on weights)");
      if (out.epochs > 0 && rust)
        notes.push_back("the reference trains the model in its interpreter for " + std::to_string(out.epochs) +
                        " epoch(s) first; its --rust library does not take those weights (the generator "
                        "ignores them, mlp_train_rust_codegen.rs:249-251) and starts from the LCG Xavier init "
                        "(seed 42), as this library does");
      if (out.epochs > 0 && mode == PLAN_INFER)
        notes.push_back("the reference trains the model in its interpreter for " + std::to_string(out.epochs) +
                        " epoch(s) and embeds those weights; this build has no interpreter: compile --weights "
                        "FILE supplies them");
      if (out.epochs > 0 && mode == PLAN_C)
        notes.push_back("the reference's C-path library exports volta_train_load_pretrained with the weights "
                        "its interpreter trained for " + std::to_string(out.epochs) +
                        " epoch(s) (mlp_train_codegen.rs:386-413); this build has no interpreter: the library "
                        "starts from the LCG Xavier init (seed 42), and compile-train --weights FILE embeds "
                        "trained weights and exports volta_train_load_pretrained");
      out.trained = true;
    } else {
      optimizer = model_opt.empty() ? "sgd" : model_opt;
    }
    // gradient clipping: the last training run of the model that sets
    // clip_grad (must be positive) leaves it in the model state
    // (executor.rs:1299, :2370-2387)
    double clip = 0.0;
    for (const auto& s : stmts) {
      if (s.kind != "train" || s.name != model->name) continue;
      if (const Property* p = find(s.block, "clip_grad")) {
        const double c = num_of(single(*p, "train.clip_grad"), "train.clip_grad");
        if (!(c > 0.0)) fail_at(p->line, p->col, "train.clip_grad must be positive");
        clip = c;
      }
    }
    if (mode == PLAN_INFER) {
      // compile: the forward graph of lower_model_to_graph has no dropout
      // or LayerNorm (lowering.rs:87-140); the optimizer only trained it
      if (dropout > 0.0 || layernorm)
        notes.push_back("the reference's inference graph (lowering.rs:87-140) has no dropout or LayerNorm; "
                        "the inference library follows it");
      dropout = 0.0;
      layernorm = false;
      clip = 0.0;
      optimizer = "sgd";
    } else if (rust) {
      // compile-train --rust guard (executor.rs:3174-3189)
      if (!(optimizer == "sgd" || optimizer == "adam" || optimizer == "adamw" || optimizer == "adagrad"))
        throw Fail{"Model '" + model->name + "' requests optimizer '" + optimizer +
                   "', but `compile-train --rust` supports only SGD, Adam, AdamW, and Adagrad today. "
                   "Use runtime `train` for RMSProp or other optimizers."};
    } else {
      // default (C) compile-train guard (executor.rs:3160-3172); the C
      // step has ReLU hidden layers, MSE and SGD whatever the model says
      // and none of the codegen extras (mlp_train_codegen.rs:291-384)
      if (optimizer != "sgd")
        throw Fail{"Model '" + model->name + "' requests optimizer '" + optimizer +
                   "', but the default C compile-train path supports only SGD today. Use `compile-train --rust` "
                   "for Adam/AdamW/Adagrad, or use runtime `train`."};
      if (activation != "relu") {
        notes.push_back("the C compile-train path generates ReLU hidden layers whatever model.activation says "
                        "(mlp_train_codegen.rs:316-321); activation '" + activation +
                        "' applies with --rust only, and this library follows the path chosen");
        activation = "relu";
      }
      if (dropout > 0.0 || layernorm || clip > 0.0) {
        notes.push_back("the C compile-train path generates no dropout, LayerNorm or gradient clipping; they "
                        "apply with --rust only, and this library follows the path chosen");
        dropout = 0.0;
        layernorm = false;
        clip = 0.0;
      }
    }

    const int act = activation == "relu" ? VOLTA_ACT_RELU
                    : activation == "sigmoid" ? VOLTA_ACT_SIGMOID
                    : activation == "tanh" ? VOLTA_ACT_TANH
                    : (activation == "leaky_relu" || activation == "leakyrelu") ? VOLTA_ACT_LEAKY_RELU
                    : activation == "silu" ? VOLTA_ACT_SILU
                    : activation == "softmax" ? VOLTA_ACT_SOFTMAX
                                           : VOLTA_ACT_GELU;
    const int opt = optimizer == "sgd" ? VOLTA_OPT_SGD
                    : optimizer == "adam" ? VOLTA_OPT_ADAM
                    : optimizer == "adamw" ? VOLTA_OPT_ADAMW
                                           : VOLTA_OPT_ADAGRAD;
    volta_mlp_spec_default(&out.spec, (int32_t)sizes.size(), sizes.data(), act, opt, VOLTA_LOSS_MSE);
    out.spec.clip_grad = (float)clip;
    out.spec.dropout_p = (float)dropout;
    out.spec.layernorm = layernorm ? 1 : 0;
    std::string why;
    if (!validate_spec(out.spec, &why)) throw Fail{"model '" + model->name + "': " + why};
    out.model = model->name;
    out.rust = rust;
    out.notes = notes;
    *plan = out;
    if (act_name) *act_name = activation;
    return true;
  } catch (const Fail& f) {
    if (error) *error = f.msg;
    return false;
  }
}

}  // namespace

bool vt_compile_train_plan(const std::string& source, VtTrainPlan* plan, std::string* error, bool rust) {
  return plan_first_model(source, rust ? PLAN_RUST : PLAN_C, plan, nullptr, error);
}

bool vt_compile_infer_plan(const std::string& source, VtInferPlan* plan, std::string* error) {
  VtTrainPlan p;
  std::string act;
  if (!plan_first_model(source, PLAN_INFER, &p, &act, error)) return false;
  // lower_model_to_graph's hidden layers: Relu for "relu", Sigmoid for
  // "sigmoid", nothing otherwise; the last layer: Softmax for "softmax"
  // (lowering.rs:121-134).  The inference codegen lowers MatMul, Add and
  // Relu and refuses Sigmoid and Softmax (codegen/inner.rs:395-399).
  if (act == "sigmoid" || act == "softmax") {
    if (error) *error = std::string("Unsupported op in codegen: ") + (act == "sigmoid" ? "Sigmoid" : "Softmax");
    return false;
  }
  plan->model = p.model;
  plan->sizes.assign(p.spec.sizes, p.spec.sizes + p.spec.n_sizes);
  plan->activation = act;
  plan->relu_hidden = act == "relu";
  plan->trained = p.trained;
  plan->notes = p.notes;
  if (!plan->relu_hidden && plan->sizes.size() > 2)
    plan->notes.push_back("the reference's inference graph applies no activation for '" + act +
                          "' (lower_model_to_graph emits Relu or Sigmoid only, lowering.rs:121-129): the hidden "
                          "layers are linear, in the reference's library and in this one");
  return true;
}

std::string vt_plan_summary(const VtTrainPlan& p) {
  static const char* acts[] = {"relu", "sigmoid", "tanh", "leaky_relu", "silu", "gelu", "softmax"};
  static const char* opts[] = {"sgd", "adam", "adamw", "adagrad"};
  std::string layers;
  for (int i = 0; i < p.spec.n_sizes; ++i) layers += (i ? "-" : "") + std::to_string(p.spec.sizes[i]);
  char buf[512];
  std::snprintf(buf, sizeof buf, "model=%s path=%s layers=%s activation=%s optimizer=%s loss=mse", p.model.c_str(),
                p.rust ? "rust" : "c", layers.c_str(), acts[p.spec.activation], opts[p.spec.optimizer]);
  std::string s = buf;
  if (p.spec.clip_grad > 0.0f) {
    std::snprintf(buf, sizeof buf, " clip_grad=%g", p.spec.clip_grad);
    s += buf;
  }
  if (p.spec.dropout_p > 0.0f) {
    std::snprintf(buf, sizeof buf, " dropout=%g", p.spec.dropout_p);
    s += buf;
  }
  if (p.spec.layernorm) s += " layernorm=yes";
  if (p.trained) {
    std::snprintf(buf, sizeof buf, " lr=%g epochs=%lld batch=%lld", p.lr, (long long)p.epochs, (long long)p.batch);
    s += buf;
  }
  return s;
}

}  // namespace volta

// ---------------------------------------------------------------------------
// C entry point (include/volta_vt.h)
// ---------------------------------------------------------------------------
extern "C" int32_t volta_vt_compile_train_spec(const char* source, volta_mlp_spec* spec, char* summary,
                                                int32_t summary_len) {
  return volta_vt_compile_train_spec_path(source, 1, spec, summary, summary_len);
}

extern "C" int32_t volta_vt_compile_train_spec_path(const char* source, int32_t rust, volta_mlp_spec* spec,
                                                     char* summary, int32_t summary_len) {
  if (!source || !spec) {
    volta::set_last_error("volta_vt_compile_train_spec: null argument");
    return -1;
  }
  volta::VtTrainPlan plan;
  std::string err;
  if (!volta::vt_compile_train_plan(source, &plan, &err, rust != 0)) {
    volta::set_last_error(err);
    return -1;
  }
  *spec = plan.spec;
  if (summary && summary_len > 0) {
    std::string s = volta::vt_plan_summary(plan);
    for (const auto& n : plan.notes) s += "\nnote: " + n;
    std::snprintf(summary, (size_t)summary_len, "%s", s.c_str());
  }
  return 0;
}
