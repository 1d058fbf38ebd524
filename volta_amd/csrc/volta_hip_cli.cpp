// volta-hip: the command line of the MI355X training library, for the two
// subcommands of the reference CLI that make libraries of a model: `volta
// compile-train` (main.rs:219-274, argument rules main.rs:587-650) and `volta
// compile` (the inference library, main.rs:158-215, rules main.rs:541-586).
//
//   volta-hip check FILE.vt [--rust]
//       print the training spec compile-train takes from FILE (and notes on
//       what the reference would do that this library does not)
//   volta-hip compile-train FILE.vt [-o OUT] [--rust] [--cpu-target portable|native]
//                           [--weights FILE.f32] [--keep-source]
//       write a shared library for that model: it exports the six
//       volta_train_* symbols of the reference's generated library (plus
//       volta_train_step_labels, volta_train_status, volta_train_last_error)
//       with the topology and optimizer baked in, and forwards them to
//       libvolta_hip.so (found beside this executable, opened with dlopen so
//       each generated library keeps its own spec).  --rust selects the
//       reference's Rust code path (any of SGD/Adam/AdamW/Adagrad, the
//       model's activation and codegen extras); without it the spec follows
//       the default C path (SGD, ReLU hidden layers, no extras).  OUT
//       defaults to FILE with the extension .train_rust.so (--rust) or
//       .train.so, as the reference names them.  --cpu-target is accepted
//       and checked as the reference checks it; it selects the reference's
//       CPU code generation and has no counterpart on the GPU.
//       Extensions: --weights embeds trained parameters (raw little-endian
//       float32, [W_0 | b_0 | W_1 | b_1 | ...], each W_i row-major [L_i x
//       L_i+1]) rounded to 8 decimal places as the reference's literals are,
//       and exports volta_train_load_pretrained, the C path's loader of
//       trained weights (mlp_train_codegen.rs:386-413); --keep-source keeps
//       the generated C source beside OUT.
//   volta-hip compile FILE.vt --weights FILE.f32 [-o OUT] [--cpu-target portable|native]
//                     [--keep-source]
//       write the model's inference library: it exports volta_infer(input,
//       in_n, output, out_n) (codegen/inner.rs:198) with the weights
//       embedded bit for bit, as the reference embeds its trained weights,
//       and runs the forward graph lower_model_to_graph builds for the first
//       model (lowering.rs:87-140) on the GPU.  The reference trains the
//       model in its interpreter first; this build has no interpreter, so
//       --weights is required.  OUT defaults to FILE with the extension .so.
//
// Exit status: 0 success, 1 compile error (message on stderr), 2 usage.
#include <unistd.h>

#include <climits>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <sstream>
#include <string>
#include <vector>

#include "../../include/volta_train.h"
#include "vt_frontend.h"

namespace {

int usage() {
  std::fprintf(stderr,
               "usage: volta-hip check FILE.vt [--rust]\n"
               "       volta-hip compile-train FILE.vt [-o OUT] [--rust] [--cpu-target portable|native]\n"
               "                               [--weights FILE.f32] [--keep-source]\n"
               "       volta-hip compile FILE.vt --weights FILE.f32 [-o OUT] [--cpu-target portable|native]\n"
               "                         [--keep-source]\n");
  return 2;
}

int arg_error(const std::string& msg) {
  std::fprintf(stderr, "%s\n", msg.c_str());
  return 2;
}

bool read_file(const std::string& path, std::string* out) {
  std::ifstream f(path, std::ios::binary);
  if (!f) return false;
  std::ostringstream ss;
  ss << f.rdbuf();
  *out = ss.str();
  return true;
}

std::string self_dir() {
  char buf[PATH_MAX];
  const ssize_t n = readlink("/proc/self/exe", buf, sizeof buf - 1);
  if (n <= 0) return ".";
  buf[n] = 0;
  std::string p(buf);
  const size_t s = p.rfind('/');
  return s == std::string::npos ? "." : p.substr(0, s);
}

std::string c_string(const std::string& s) {
  std::string o = "\"";
  for (char c : s) {
    if (c == '"' || c == '\\') o += '\\';
    if (c == '\n') {
      o += "\\n";
      continue;
    }
    o += c;
  }
  return o + "\"";
}

// A file path as the quoted operand of an assembler directive written inside
// a C string literal: escaped first for the assembler's string syntax (\"
// and \\, octal escapes for control characters), then that text escaped for
// C.
std::string asm_path_in_c(const std::string& path) {
  std::string a;
  for (unsigned char c : path) {
    if (c == '"' || c == '\\') {
      a += '\\';
      a += (char)c;
    } else if (c < 0x20 || c == 0x7f) {
      char b[8];
      std::snprintf(b, sizeof b, "\\%03o", c);
      a += b;
    } else {
      a += (char)c;
    }
  }
  std::string o;
  for (char c : a) {
    if (c == '"' || c == '\\') o += '\\';
    o += c;
  }
  return o;
}

// The assembler block that places a file's bytes in the library's read-only
// data under `symbol` (16-byte aligned).
std::string incbin_block(const std::string& symbol, const std::string& path) {
  return "__asm__(\".section .rodata\\n.balign 16\\n.type " + symbol + ", @object\\n" + symbol + ":\\n.incbin \\\"" +
         asm_path_in_c(path) + "\\\"\\n.previous\\n\");\nextern const float " + symbol + "[];\n";
}

// C source of the per-model library.

std::string generate(const volta::VtTrainPlan& plan, const std::string& vt_path, const std::string& lib_path,
                     const std::string& weights_path) {
  const volta_mlp_spec& s = plan.spec;
  std::ostringstream o;
  o << "/* Training library for model '" << plan.model << "' from " << vt_path << ",\n"
    << " * generated by volta-hip compile-train: " << volta::vt_plan_summary(plan) << ".\n"
    << " * Exports the six volta_train_* symbols of the reference's generated\n"
    << " * library; the work is done by " << lib_path << ". */\n"
    << "#include <dlfcn.h>\n#include <stddef.h>\n#include <stdint.h>\n\n"
    << "typedef struct {\n  int32_t n_sizes;\n  int32_t sizes[" << VOLTA_MAX_LAYER_SIZES << "];\n"
    << "  int32_t activation, optimizer, loss;\n  float beta1, beta2, eps, weight_decay;\n"
    << "  float clip_grad, dropout_p;\n  int32_t layernorm;\n} spec_t;\n"
    << "_Static_assert(sizeof(spec_t) == " << sizeof(volta_mlp_spec) << ", \"volta_mlp_spec layout\");\n\n"
    << "static const spec_t kSpec = {" << s.n_sizes << ", {";
  for (int i = 0; i < VOLTA_MAX_LAYER_SIZES; ++i) o << (i ? ", " : "") << (i < s.n_sizes ? s.sizes[i] : 0);
  char hp[256];
  std::snprintf(hp, sizeof hp,
                "}, %d, %d, %d, (float)%.9g, (float)%.9g, (float)%.9g, (float)%.9g, (float)%.9g, (float)%.9g, "
                "%d};\n\n",
                s.activation, s.optimizer, s.loss, s.beta1, s.beta2, s.eps, s.weight_decay, s.clip_grad,
                s.dropout_p, s.layernorm);
  o << hp
    << "static void* (*p_init_spec)(const spec_t*, int32_t);\n"
    << "static void (*p_step)(void*, const float*, const float*, float);\n"
    << "static void (*p_step_labels)(void*, const float*, const int32_t*, float);\n"
    << "static float (*p_loss)(void*);\n"
    << "static void (*p_get_params)(void*, float**, float**);\n"
    << "static void (*p_set_params)(void*, int32_t, const float*, const float*);\n"
    << "static void (*p_free)(void*);\n"
    << "static int32_t (*p_status)(void*);\n"
    << "static const char* (*p_last_error)(void);\n"
    << "static const char* g_error = \"\";\n\n"
    << "__attribute__((constructor)) static void volta_model_load(void) {\n"
    << "  void* h = dlopen(" << c_string(lib_path) << ", RTLD_NOW | RTLD_LOCAL);\n"
    << "  if (!h) { g_error = dlerror(); return; }\n"
    << "  *(void**)&p_init_spec = dlsym(h, \"volta_train_init_spec\");\n"
    << "  *(void**)&p_step = dlsym(h, \"volta_train_step\");\n"
    << "  *(void**)&p_step_labels = dlsym(h, \"volta_train_step_labels\");\n"
    << "  *(void**)&p_loss = dlsym(h, \"volta_train_loss\");\n"
    << "  *(void**)&p_get_params = dlsym(h, \"volta_train_get_params\");\n"
    << "  *(void**)&p_set_params = dlsym(h, \"volta_train_set_params\");\n"
    << "  *(void**)&p_free = dlsym(h, \"volta_train_free\");\n"
    << "  *(void**)&p_status = dlsym(h, \"volta_train_status\");\n"
    << "  *(void**)&p_last_error = dlsym(h, \"volta_train_last_error\");\n"
    << "}\n\n"
    << "void* volta_train_init(int32_t batch) { return p_init_spec ? p_init_spec(&kSpec, batch) : NULL; }\n"
    << "void volta_train_step(void* h, const float* x, const float* y, float lr) { if (p_step) p_step(h, x, y, lr); }\n"
    << "void volta_train_step_labels(void* h, const float* x, const int32_t* l, float lr) {\n"
    << "  if (p_step_labels) p_step_labels(h, x, l, lr);\n}\n"
    << "float volta_train_loss(void* h) { return p_loss ? p_loss(h) : 0.0f / 0.0f; }\n"
    << "void volta_train_get_params(void* h, float** wo, float** bo) { if (p_get_params) p_get_params(h, wo, bo); }\n"
    << "void volta_train_set_params(void* h, int32_t li, const float* w, const float* b) {\n"
    << "  if (p_set_params) p_set_params(h, li, w, b);\n}\n"
    << "void volta_train_free(void* h) { if (p_free) p_free(h); }\n"
    << "int32_t volta_train_status(void* h) { return p_status ? p_status(h) : 4; }\n"
    << "const char* volta_train_last_error(void) { return p_last_error ? p_last_error() : g_error; }\n";
  if (!weights_path.empty()) {
    // trained parameters embedded in the library's read-only data
    o << "\n" << incbin_block("volta_pretrained_blob", weights_path)
      << "void volta_train_load_pretrained(void* h) {\n"
      << "  const float* p = volta_pretrained_blob;\n";
    for (int i = 0; i + 1 < s.n_sizes; ++i) {
      const long long r = s.sizes[i], c = s.sizes[i + 1];
      o << "  if (p_set_params) p_set_params(h, " << i << ", p, p + " << r * c << ");\n"
        << "  p += " << r * c + c << ";\n";
    }
    o << "}\n";
  }
  return o.str();
}

// C source of a `compile` library: the reference's inference library
// (codegen/inner.rs:190-262: weights embedded as constant globals, one
// exported symbol volta_infer(input, in_n, output, out_n)).  The model is
// created on the GPU at the first call (volta_infer_model_create in
// libvolta_hip.so, opened with dlopen) and lives until the process ends.
std::string generate_infer(const volta::VtInferPlan& plan, const std::string& vt_path, const std::string& lib_path,
                           const std::string& weights_path) {
  const int n = (int)plan.sizes.size();
  std::string layers;
  for (int i = 0; i < n; ++i) layers += (i ? "-" : "") + std::to_string(plan.sizes[i]);
  std::ostringstream o;
  o << "/* Inference library for model '" << plan.model << "' from " << vt_path << ",\n"
    << " * generated by volta-hip compile: layers " << layers << ", hidden layers MatMul + Add"
    << (plan.relu_hidden ? " + Relu" : "") << ".\n"
    << " * Exports volta_infer(input, in_n, output, out_n) with the trained weights\n"
    << " * embedded; the forward runs on the GPU through " << lib_path << ". */\n"
    << "#include <dlfcn.h>\n#include <pthread.h>\n#include <stdint.h>\n#include <stdio.h>\n\n"
    << incbin_block("volta_model_blob", weights_path) << "\n"
    << "static const int32_t kSizes[" << n << "] = {";
  for (int i = 0; i < n; ++i) o << (i ? ", " : "") << plan.sizes[i];
  o << "};\n"
    << "static void* (*p_create)(int32_t, const int32_t*, int32_t, const float*);\n"
    << "static int32_t (*p_infer)(void*, const float*, int64_t, float*);\n"
    << "static const char* (*p_last_error)(void);\n"
    << "static void* g_model;\n"
    << "static char g_error[512];\n"
    << "static pthread_once_t g_once = PTHREAD_ONCE_INIT;\n"
    << "static pthread_mutex_t g_mu = PTHREAD_MUTEX_INITIALIZER;\n\n"
    << "static void set_error(const char* what, const char* why) {\n"
    << "  snprintf(g_error, sizeof g_error, \"%s%s\", what, why ? why : \"\");\n}\n\n"
    << "static void volta_model_open(void) {\n"
    << "  void* h = dlopen(" << c_string(lib_path) << ", RTLD_NOW | RTLD_LOCAL);\n"
    << "  if (!h) { set_error(\"volta_infer: \", dlerror()); return; }\n"
    << "  *(void**)&p_create = dlsym(h, \"volta_infer_model_create\");\n"
    << "  *(void**)&p_infer = dlsym(h, \"volta_train_infer\");\n"
    << "  *(void**)&p_last_error = dlsym(h, \"volta_train_last_error\");\n"
    << "  if (!p_create || !p_infer || !p_last_error) {\n"
    << "    set_error(\"volta_infer: the GPU library lacks volta_infer_model_create\", 0);\n    return;\n  }\n"
    << "  g_model = p_create(" << n << ", kSizes, " << (plan.relu_hidden ? VOLTA_ACT_RELU : -1)
    << ", volta_model_blob);\n"
    << "  if (!g_model) set_error(\"volta_infer: \", p_last_error());\n"
    << "}\n\n"
    << "/* rows = in_n / " << plan.sizes[0] << " input rows, as many as output holds (out_n / "
    << plan.sizes[n - 1] << "); one row per call is\n"
    << " * the reference's graph (input bound to [1, " << plan.sizes[0] << "], executor.rs:1718). */\n"
    << "void volta_infer(const float* input, int64_t in_n, float* output, int64_t out_n) {\n"
    << "  pthread_once(&g_once, volta_model_open);\n"
    << "  if (!g_model) return;\n"
    << "  if (!input || !output || in_n < " << plan.sizes[0] << " || out_n < " << plan.sizes[n - 1] << ") {\n"
    << "    set_error(\"volta_infer: input must hold a row of " << plan.sizes[0] << " floats and output one of "
    << plan.sizes[n - 1] << "\", 0);\n    return;\n  }\n"
    << "  int64_t rows = in_n / " << plan.sizes[0] << ";\n"
    << "  if (rows > out_n / " << plan.sizes[n - 1] << ") rows = out_n / " << plan.sizes[n - 1] << ";\n"
    << "  pthread_mutex_lock(&g_mu);\n"
    << "  if (p_infer(g_model, input, rows, output) != 0) set_error(\"volta_infer: \", p_last_error());\n"
    << "  else g_error[0] = 0;\n"
    << "  pthread_mutex_unlock(&g_mu);\n"
    << "}\n\n"
    << "/* Why the last volta_infer call wrote nothing (\"\" after a call that wrote its output). */\n"
    << "const char* volta_infer_last_error(void) { return g_error; }\n";
  return o.str();
}

int check(const std::string& path, bool rust) {
  std::string src, err;
  if (!read_file(path, &src)) {
    std::fprintf(stderr, "cannot read %s\n", path.c_str());
    return 2;
  }
  volta::VtTrainPlan plan;
  if (!volta::vt_compile_train_plan(src, &plan, &err, rust)) {
    std::fprintf(stderr, "compile-train error: %s: %s\n", path.c_str(), err.c_str());
    return 1;
  }
  std::printf("%s\n", volta::vt_plan_summary(plan).c_str());
  for (const auto& n : plan.notes) std::printf("note: %s\n", n.c_str());
  return 0;
}

struct TrainArgs {
  std::string path, out, cpu_target = "portable", weights;
  bool rust = false, keep = false;
};

int compile_train(const TrainArgs& a) {
  std::string src, err;
  if (!read_file(a.path, &src)) {
    std::fprintf(stderr, "cannot read %s\n", a.path.c_str());
    return 2;
  }
  volta::VtTrainPlan plan;
  if (!volta::vt_compile_train_plan(src, &plan, &err, a.rust)) {
    std::fprintf(stderr, "compile-train error: %s: %s\n", a.path.c_str(), err.c_str());
    return 1;
  }
  std::string out = a.out;
  if (out.empty()) {  // Path::with_extension("train_rust.so" / "train.so") (executor.rs:1790-1797, 1849-1856)
    const size_t dot = a.path.rfind('.'), slash = a.path.rfind('/');
    out = (dot != std::string::npos && (slash == std::string::npos || dot > slash) ? a.path.substr(0, dot) : a.path) +
          (a.rust ? ".train_rust.so" : ".train.so");
  }
  char lib_real[PATH_MAX];
  const std::string lib = self_dir() + "/libvolta_hip.so";
  if (!realpath(lib.c_str(), lib_real)) {
    std::fprintf(stderr, "compile-train error: %s not found (build it with python -m volta_amd.build)\n",
                 lib.c_str());
    return 1;
  }
  std::string weights_real;
  if (!a.weights.empty()) {
    char w[PATH_MAX];
    long long want = 0;
    for (int i = 0; i + 1 < plan.spec.n_sizes; ++i)
      want += ((long long)plan.spec.sizes[i] * plan.spec.sizes[i + 1] + plan.spec.sizes[i + 1]) * 4;
    std::ifstream f(a.weights, std::ios::binary | std::ios::ate);
    if (!f || !realpath(a.weights.c_str(), w)) {
      std::fprintf(stderr, "compile-train error: cannot read weights file %s\n", a.weights.c_str());
      return 1;
    }
    if ((long long)f.tellg() != want) {
      std::fprintf(stderr, "compile-train error: weights file %s holds %lld bytes; model '%s' needs %lld "
                   "(float32 [W_0 | b_0 | W_1 | b_1 | ...])\n", a.weights.c_str(), (long long)f.tellg(),
                   plan.model.c_str(), want);
      return 1;
    }
    weights_real = w;
  }
  // The reference's C-path loader embeds each trained value as a decimal
  // literal with 8 places ("{v:.8}f", mlp_train_codegen.rs:393-405), which
  // the C compiler rounds back to the nearest float: the library embeds the
  // same values (%.8f of the float, then strtof), written beside OUT.
  std::string rounded;
  if (!weights_real.empty()) {
    std::ifstream f(weights_real, std::ios::binary);
    std::vector<float> v((size_t)(std::ifstream(weights_real, std::ios::binary | std::ios::ate).tellg() / 4));
    f.read(reinterpret_cast<char*>(v.data()), (std::streamsize)(v.size() * 4));
    for (float& x : v) {
      char buf[96];
      std::snprintf(buf, sizeof buf, "%.8f", (double)x);
      x = std::strtof(buf, nullptr);
    }
    rounded = out + ".weights";
    std::ofstream g(rounded, std::ios::binary);
    g.write(reinterpret_cast<const char*>(v.data()), (std::streamsize)(v.size() * 4));
    char rr[PATH_MAX];
    if (!f || !g || !g.flush() || !realpath(rounded.c_str(), rr)) {
      std::fprintf(stderr, "compile-train error: cannot write %s\n", rounded.c_str());
      return 1;
    }
    rounded = rr;
  }
  const std::string csrc = out + ".c";
  {
    std::ofstream f(csrc);
    f << generate(plan, a.path, lib_real, rounded);
    if (!f) {
      std::fprintf(stderr, "cannot write %s\n", csrc.c_str());
      return 1;
    }
  }
  const char* cc = std::getenv("CC");
  const std::string cmd = std::string(cc && *cc ? cc : "cc") + " -O2 -shared -fPIC -o '" + out + "' '" + csrc +
                          "' -ldl";
  const int rc = std::system(cmd.c_str());
  if (!a.keep) {
    std::remove(csrc.c_str());
    if (!rounded.empty()) std::remove(rounded.c_str());
  }
  if (rc != 0) {
    std::fprintf(stderr, "compile-train error: C compiler failed: %s\n", cmd.c_str());
    return 1;
  }
  std::printf("Training DLL compiled: %s (cpu-target=%s)\n", out.c_str(), a.cpu_target.c_str());
  std::printf("%s\n", volta::vt_plan_summary(plan).c_str());
  if (!weights_real.empty()) std::printf("note: trained weights from %s: volta_train_load_pretrained\n",
                                         weights_real.c_str());
  for (const auto& n : plan.notes) std::printf("note: %s\n", n.c_str());
  return 0;
}

// OUT of `compile`: Path::with_extension("so") of FILE (executor.rs:1734-1737).
std::string default_output(const std::string& path, const std::string& ext) {
  const size_t dot = path.rfind('.'), slash = path.rfind('/');
  return (dot != std::string::npos && (slash == std::string::npos || dot > slash) ? path.substr(0, dot) : path) + ext;
}

struct InferArgs {
  std::string path, out, cpu_target = "portable", weights;
  bool keep = false;
};

int compile_infer(const InferArgs& a) {
  std::string src, err;
  if (!read_file(a.path, &src)) {
    std::fprintf(stderr, "cannot read %s\n", a.path.c_str());
    return 2;
  }
  volta::VtInferPlan plan;
  if (!volta::vt_compile_infer_plan(src, &plan, &err)) {
    std::fprintf(stderr, "Compile error: %s: %s\n", a.path.c_str(), err.c_str());
    return 1;
  }
  if (a.weights.empty()) {  // executor.rs:1702-1705: the model must carry weights
    std::fprintf(stderr, "Compile error: Model '%s' has no weights — train it first (this build has no "
                 "interpreter to train it: pass --weights FILE)\n", plan.model.c_str());
    return 1;
  }
  const std::string out = a.out.empty() ? default_output(a.path, ".so") : a.out;
  char lib_real[PATH_MAX];
  const std::string lib = self_dir() + "/libvolta_hip.so";
  if (!realpath(lib.c_str(), lib_real)) {
    std::fprintf(stderr, "Compile error: %s not found (build it with python -m volta_amd.build)\n", lib.c_str());
    return 1;
  }
  long long want = 0;
  for (size_t i = 0; i + 1 < plan.sizes.size(); ++i)
    want += ((long long)plan.sizes[i] * plan.sizes[i + 1] + plan.sizes[i + 1]) * 4;
  char w[PATH_MAX];
  std::ifstream f(a.weights, std::ios::binary | std::ios::ate);
  if (!f || !realpath(a.weights.c_str(), w)) {
    std::fprintf(stderr, "Compile error: cannot read weights file %s\n", a.weights.c_str());
    return 1;
  }
  if ((long long)f.tellg() != want) {
    std::fprintf(stderr, "Compile error: weights file %s holds %lld bytes; model '%s' needs %lld "
                 "(float32 [W_0 | b_0 | W_1 | b_1 | ...])\n", a.weights.c_str(), (long long)f.tellg(),
                 plan.model.c_str(), want);
    return 1;
  }
  const std::string csrc = out + ".c";
  {
    std::ofstream g(csrc);
    g << generate_infer(plan, a.path, lib_real, w);
    if (!g) {
      std::fprintf(stderr, "cannot write %s\n", csrc.c_str());
      return 1;
    }
  }
  const char* cc = std::getenv("CC");
  const std::string cmd = std::string(cc && *cc ? cc : "cc") + " -O2 -shared -fPIC -o '" + out + "' '" + csrc +
                          "' -ldl -lpthread";
  const int rc = std::system(cmd.c_str());
  if (!a.keep) std::remove(csrc.c_str());
  if (rc != 0) {
    std::fprintf(stderr, "Compile error: C compiler failed: %s\n", cmd.c_str());
    return 1;
  }
  std::printf("Compiled: %s (cpu-target=%s)\n", out.c_str(), a.cpu_target.c_str());
  for (const auto& n : plan.notes) std::printf("note: %s\n", n.c_str());
  return 0;
}

// compile's arguments, checked as the reference checks them (main.rs:
// 541-586) plus this tool's --weights and --keep-source.
int parse_compile(int argc, char** argv, InferArgs* a) {
  const std::string cmd = "compile";
  bool have_out = false;
  for (int i = 2; i < argc; ++i) {
    const std::string x = argv[i];
    if (x == "-o") {
      if (i + 1 >= argc || argv[i + 1][0] == '-') return arg_error("'" + cmd + " -o' requires an output path");
      if (have_out) return arg_error("'" + cmd + "' accepts '-o' at most once");
      a->out = argv[++i];
      have_out = true;
    } else if (x == "--cpu-target" || x.rfind("--cpu-target=", 0) == 0) {
      std::string v;
      if (x == "--cpu-target") {
        if (i + 1 >= argc) return arg_error("'" + cmd + " --cpu-target' requires 'portable' or 'native'");
        v = argv[++i];
      } else {
        v = x.substr(std::strlen("--cpu-target="));
      }
      if (v != "portable" && v != "native")
        return arg_error("'" + cmd + " --cpu-target' accepts only 'portable' or 'native', got '" + v + "'");
      a->cpu_target = v;
    } else if (x == "--keep-source") {
      a->keep = true;
    } else if (x == "--weights") {
      if (i + 1 >= argc) return arg_error("'" + cmd + " --weights' requires a file");
      a->weights = argv[++i];
    } else if (!x.empty() && x[0] == '-') {
      return arg_error("'" + cmd + "' does not accept flag '" + x + "'");
    } else {
      if (!a->path.empty()) return arg_error("'" + cmd + "' expects exactly one .vt file");
      a->path = x;
    }
  }
  if (a->path.empty()) return arg_error("'" + cmd + "' expects a .vt file path");
  return 0;
}

// compile-train's arguments, checked as the reference checks them
// (main.rs:587-650) plus this tool's --weights and --keep-source.
int parse_compile_train(int argc, char** argv, TrainArgs* a) {
  const std::string cmd = "compile-train";
  bool have_out = false;
  for (int i = 2; i < argc; ++i) {
    const std::string x = argv[i];
    if (x == "-o") {
      if (i + 1 >= argc || argv[i + 1][0] == '-') return arg_error("'" + cmd + " -o' requires an output path");
      if (have_out) return arg_error("'" + cmd + "' accepts '-o' at most once");
      a->out = argv[++i];
      have_out = true;
    } else if (x == "--cpu-target" || x.rfind("--cpu-target=", 0) == 0) {
      std::string v;
      if (x == "--cpu-target") {
        if (i + 1 >= argc) return arg_error("'" + cmd + " --cpu-target' requires 'portable' or 'native'");
        v = argv[++i];
      } else {
        v = x.substr(std::strlen("--cpu-target="));
      }
      if (v != "portable" && v != "native")
        return arg_error("'" + cmd + " --cpu-target' accepts only 'portable' or 'native', got '" + v + "'");
      a->cpu_target = v;
    } else if (x == "--rust") {
      if (a->rust) return arg_error("'" + cmd + "' accepts '--rust' at most once");
      a->rust = true;
    } else if (x == "--keep-source") {
      a->keep = true;
    } else if (x == "--weights") {
      if (i + 1 >= argc) return arg_error("'" + cmd + " --weights' requires a file");
      a->weights = argv[++i];
    } else if (!x.empty() && x[0] == '-') {
      return arg_error("'" + cmd + "' does not accept flag '" + x + "'");
    } else {
      if (!a->path.empty()) return arg_error("'" + cmd + "' expects exactly one .vt file");
      a->path = x;
    }
  }
  if (a->path.empty()) return arg_error("'" + cmd + "' expects a .vt file path");
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) return usage();
  const std::string cmd = argv[1];
  if (cmd == "check") {
    if (argc == 3) return check(argv[2], false);
    if (argc == 4 && std::string(argv[3]) == "--rust") return check(argv[2], true);
    if (argc == 4 && std::string(argv[2]) == "--rust") return check(argv[3], true);
    return usage();
  }
  if (cmd == "compile-train") {
    TrainArgs a;
    const int rc = parse_compile_train(argc, argv, &a);
    return rc ? rc : compile_train(a);
  }
  if (cmd == "compile") {
    InferArgs a;
    const int rc = parse_compile(argc, argv, &a);
    return rc ? rc : compile_infer(a);
  }
  return usage();
}
