// ===========================================================================
// TEST INFRASTRUCTURE -- CPU oracle of the runtime optimizer.  Not part of
// the product.
//
// A CPU restatement of Volta's runtime optimizer, optimizer::apply_gradients
// (/root/reference/src/engine/ir/optimizer.rs:108-658), behind the same C ABI
// as the HIP implementation (include/volta_backend.h) so one harness drives
// both.  Tensors are host buffers here, keyed by index instead of ValueId.
//
// Fidelity rules:
//  * fp32 in the reference's expression order, no FMA contraction (built
//    with -ffp-contract=off); sqrtf and '/' are IEEE (correctly rounded).
//  * The step counter advances before validation (:114); validation order
//    and messages follow each apply_* function.  Numbers are printed with the
//    shortest round-trip form, Rust-style NaN/inf.
//  * Adam/AdamW bias corrections use f32::powi (:277-278, :388-389), which
//    Rust lowers to the compiler-builtins/compiler-rt routine __powisf2:
//    square-and-multiply in f32 (restated in powi_f32 below).
//  * State buffers are created zero-filled the first time a tensor with a
//    gradient needs them (entry().or_insert, :303-318 etc.).
//  * LARS norms are sequential f32 sums of x*x (:628-629).
//
// Pinned by (tests/test_rt_optimizer_oracle.py): the reference's own tests
// of optimizer.rs (:676-1045: SGD 1.0 - 0.1*0.5 = 0.95, three SGD steps to
// 0.85 with step = 3, the Adam step-1 KAT 0.5 -> 0.499000, Adagrad monotone
// decrease, every rejection case and the word its message must contain),
// closed forms (Adam/AdamW step 1, RMSprop and Adagrad with a constant
// gradient, LARS local rate), powi against exact products, skipped
// tensors, and state creation.
// ===========================================================================
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../include/volta_backend.h"

namespace {

thread_local std::string g_rt_err;

// Shortest decimal that reads back as x (Rust's Display for f32 is the
// shortest round-trip form; NaN and infinities as Rust prints them).
std::string fmt_f32(float x) {
  if (std::isnan(x)) return "NaN";
  if (std::isinf(x)) return x > 0 ? "inf" : "-inf";
  char buf[64];
  for (int prec = 1; prec <= 9; ++prec) {
    std::snprintf(buf, sizeof buf, "%.*g", prec, (double)x);
    if (std::strtof(buf, nullptr) == x) break;
  }
  return buf;
}

// compiler-rt / compiler-builtins __powisf2: square-and-multiply in f32.
float powi_f32(float a, int32_t b) {
  const bool recip = b < 0;
  uint32_t e = b < 0 ? (uint32_t)(-(int64_t)b) : (uint32_t)b;
  float r = 1.0f;
  for (;;) {
    if (e & 1u) r = r * a;
    e >>= 1;
    if (e == 0) break;
    a = a * a;
  }
  return recip ? 1.0f / r : r;
}

bool finite_pos(float x) { return std::isfinite(x) && x > 0.0f; }
bool finite_nonneg(float x) { return std::isfinite(x) && x >= 0.0f; }
bool unit_interval(float x) { return x >= 0.0f && x < 1.0f; }  // (0.0..1.0).contains(&x); false for NaN

int fail(const std::string& msg) {
  g_rt_err = msg;
  return -1;
}

}  // namespace

struct VoltaRtOptimizer {
  int32_t n = 0;
  std::vector<int64_t> counts;
  uint64_t step = 0;
  std::vector<std::vector<float>> buf[6];  // per volta_rt_buffer, per tensor (empty: not created)
};

namespace {

float* state(VoltaRtOptimizer* h, int which, int i) {
  std::vector<float>& b = h->buf[which][i];
  if (b.empty()) b.assign((size_t)h->counts[i], 0.0f);
  return b.data();
}

}  // namespace

// volta_rt_last_error's text for the graph interpreter (rt_graph.cpp).
void oracle_rt_set_error(const std::string& m) { g_rt_err = m; }

extern "C" {

VoltaRtOptimizer* volta_rt_optimizer_new(int32_t n, const int64_t* counts) {
  if (n < 1 || !counts) {
    g_rt_err = "volta_rt_optimizer_new: need n >= 1 and counts";
    return nullptr;
  }
  auto* h = new VoltaRtOptimizer;
  h->n = n;
  for (int i = 0; i < n; ++i) {
    if (counts[i] < 1) {
      delete h;
      g_rt_err = "volta_rt_optimizer_new: every tensor needs at least one element";
      return nullptr;
    }
    h->counts.push_back(counts[i]);
  }
  for (auto& b : h->buf) b.resize(n);
  return h;
}

void volta_rt_optimizer_free(VoltaRtOptimizer* h) { delete h; }

int64_t volta_rt_step(const VoltaRtOptimizer* h) { return h ? (int64_t)h->step : -1; }

const char* volta_rt_last_error(void) { return g_rt_err.c_str(); }

int32_t volta_rt_get_state(const VoltaRtOptimizer* h, int32_t which, int32_t i, float* out) {
  if (!h || which < 0 || which > 5 || i < 0 || i >= h->n || !out) return fail("volta_rt_get_state: bad arguments");
  const std::vector<float>& b = h->buf[which][i];
  if (b.empty()) return fail("volta_rt_get_state: no such state entry");
  std::memcpy(out, b.data(), b.size() * sizeof(float));
  return 0;
}

void volta_rt_capabilities_get(volta_rt_capabilities* out) {
  // the reference's CpuBackend (backend.rs: capabilities)
  if (!out) return;
  std::memset(out, 0, sizeof *out);
  out->backend = 0;
  out->device_class = 0;
  out->vendor = 0;
  out->maturity = 1;
  out->supports_inference = out->supports_training = out->supports_runtime_execution = 1;
  out->supports_gradient_updates = out->supports_adam = 1;
  out->supports_strict_determinism = out->supports_balanced_determinism = out->supports_fast_determinism = 1;
  out->default_determinism = 0;  // Strict (backend.rs:74-90)
}

int32_t volta_rt_apply_gradients(VoltaRtOptimizer* h, const volta_rt_config* cfg, float* const* params,
                                 const float* const* grads) {
  if (!h || !cfg || !params || !grads) return fail("volta_rt_apply_gradients: bad arguments");
  h->step = h->step + 1;  // saturating in the reference; 2^64 steps are not reachable
  const float lr = cfg->lr;
  switch (cfg->kind) {
    case VOLTA_RT_SGD: {  // apply_sgd (:198-228)
      if (!finite_pos(lr)) return fail("SGD learning rate must be a finite positive number, got " + fmt_f32(lr));
      for (int i = 0; i < h->n; ++i) {
        if (!grads[i]) continue;
        float* p = params[i];
        const float* g = grads[i];
        for (int64_t k = 0; k < h->counts[i]; ++k) p[k] = p[k] - lr * g[k];
      }
      return 0;
    }
    case VOLTA_RT_ADAM:
    case VOLTA_RT_ADAMW: {  // apply_adam (:230-343), apply_adamw (:345-444)
      const bool w = cfg->kind == VOLTA_RT_ADAMW;
      const std::string nm = w ? "AdamW" : "Adam";
      const float b1 = cfg->beta1, b2 = cfg->beta2, eps = cfg->epsilon, wd = cfg->weight_decay;
      if (!finite_pos(lr)) return fail(nm + " learning rate must be a finite positive number, got " + fmt_f32(lr));
      if (!unit_interval(b1)) return fail(nm + " beta1 must be in [0, 1), got " + fmt_f32(b1));
      if (!unit_interval(b2)) return fail(nm + " beta2 must be in [0, 1), got " + fmt_f32(b2));
      if (!finite_pos(eps)) return fail(nm + " epsilon must be a finite positive number, got " + fmt_f32(eps));
      if (w && !finite_nonneg(wd))
        return fail("AdamW weight_decay must be a finite non-negative number, got " + fmt_f32(wd));
      if (h->step > (uint64_t)INT32_MAX) return fail("Optimizer step overflow for " + nm + " bias correction");
      const float bias1 = 1.0f - powi_f32(b1, (int32_t)h->step);
      const float bias2 = 1.0f - powi_f32(b2, (int32_t)h->step);
      if (bias1 <= 0.0f || bias2 <= 0.0f)
        return fail(nm + " bias correction underflowed (bias1=" + fmt_f32(bias1) + ", bias2=" + fmt_f32(bias2) +
                    "); step=" + std::to_string(h->step));
      const float om1 = 1.0f - b1, om2 = 1.0f - b2;
      for (int i = 0; i < h->n; ++i) {
        if (!grads[i]) continue;
        float* m = state(h, VOLTA_RT_ADAM_M, i);
        float* v = state(h, VOLTA_RT_ADAM_V, i);
        float* p = params[i];
        const float* g = grads[i];
        for (int64_t k = 0; k < h->counts[i]; ++k) {
          m[k] = b1 * m[k] + om1 * g[k];
          v[k] = b2 * v[k] + om2 * (g[k] * g[k]);
          const float mh = m[k] / bias1;
          const float vh = v[k] / bias2;
          if (w) p[k] = p[k] - lr * (mh / (std::sqrt(vh) + eps) + wd * p[k]);
          else p[k] = p[k] - lr * (mh / (std::sqrt(vh) + eps));
        }
      }
      return 0;
    }
    case VOLTA_RT_RMSPROP: {  // apply_rmsprop (:446-541)
      const float al = cfg->alpha, eps = cfg->epsilon, wd = cfg->weight_decay, mo = cfg->momentum;
      if (!finite_pos(lr)) return fail("RMSprop learning rate must be a finite positive number, got " + fmt_f32(lr));
      if (!unit_interval(al)) return fail("RMSprop alpha must be in [0, 1), got " + fmt_f32(al));
      if (!finite_pos(eps)) return fail("RMSprop epsilon must be a finite positive number, got " + fmt_f32(eps));
      if (!finite_nonneg(wd))
        return fail("RMSprop weight_decay must be a finite non-negative number, got " + fmt_f32(wd));
      if (!finite_nonneg(mo)) return fail("RMSprop momentum must be a finite non-negative number, got " + fmt_f32(mo));
      for (int i = 0; i < h->n; ++i) {
        if (!grads[i]) continue;
        float* v = state(h, VOLTA_RT_RMS_V, i);
        float* p = params[i];
        const float* g = grads[i];
        if (mo > 0.0f) {
          float* b = state(h, VOLTA_RT_RMS_BUF, i);
          for (int64_t k = 0; k < h->counts[i]; ++k) {
            const float gwd = g[k] + wd * p[k];
            v[k] = al * v[k] + (1.0f - al) * gwd * gwd;
            b[k] = mo * b[k] + lr * gwd / (std::sqrt(v[k]) + eps);
            p[k] = p[k] - b[k];
          }
        } else {
          for (int64_t k = 0; k < h->counts[i]; ++k) {
            const float gwd = g[k] + wd * p[k];
            v[k] = al * v[k] + (1.0f - al) * gwd * gwd;
            p[k] = p[k] - lr * gwd / (std::sqrt(v[k]) + eps);
          }
        }
      }
      return 0;
    }
    case VOLTA_RT_ADAGRAD: {  // apply_adagrad (:543-603)
      const float eps = cfg->epsilon, wd = cfg->weight_decay;
      if (!finite_pos(lr)) return fail("Adagrad learning rate must be a finite positive number, got " + fmt_f32(lr));
      if (!finite_pos(eps)) return fail("Adagrad epsilon must be a finite positive number, got " + fmt_f32(eps));
      if (!finite_nonneg(wd))
        return fail("Adagrad weight_decay must be a finite non-negative number, got " + fmt_f32(wd));
      for (int i = 0; i < h->n; ++i) {
        if (!grads[i]) continue;
        float* a = state(h, VOLTA_RT_ADAGRAD_ACC, i);
        float* p = params[i];
        const float* g = grads[i];
        for (int64_t k = 0; k < h->counts[i]; ++k) {
          const float gwd = g[k] + wd * p[k];
          a[k] = a[k] + gwd * gwd;
          p[k] = p[k] - lr * gwd / (std::sqrt(a[k]) + eps);
        }
      }
      return 0;
    }
    case VOLTA_RT_LARS: {  // apply_lars (:605-658)
      const float mo = cfg->momentum, wd = cfg->weight_decay, tc = cfg->trust_coeff, eps = cfg->epsilon;
      if (!finite_pos(lr)) return fail("LARS learning rate must be a finite positive number, got " + fmt_f32(lr));
      for (int i = 0; i < h->n; ++i) {
        if (!grads[i]) continue;
        float* p = params[i];
        const float* g = grads[i];
        float ps = 0.0f, gs = 0.0f;
        for (int64_t k = 0; k < h->counts[i]; ++k) ps = ps + p[k] * p[k];
        for (int64_t k = 0; k < h->counts[i]; ++k) gs = gs + g[k] * g[k];
        const float pn = std::sqrt(ps), gn = std::sqrt(gs);
        const float local = pn > 0.0f && gn > 0.0f ? lr * tc * pn / (gn + wd * pn + eps) : lr;
        float* vel = state(h, VOLTA_RT_LARS_VEL, i);
        for (int64_t k = 0; k < h->counts[i]; ++k) {
          const float upd = local * (g[k] + wd * p[k]);
          vel[k] = mo * vel[k] + upd;
          p[k] = p[k] - vel[k];
        }
      }
      return 0;
    }
    default:
      return fail("volta_rt_apply_gradients: unknown optimizer kind");
  }
}

// powi as the oracle computes it (for the tests of the restatement).
float volta_oracle_powi(float a, int32_t b) { return powi_f32(a, b); }

}  // extern "C"
