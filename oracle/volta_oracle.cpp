// ===========================================================================
// TEST INFRASTRUCTURE -- the CPU oracle.  Not part of the product.
//
// A CPU restatement of the training step that Volta's `compile-train`
// generator emits (/root/reference/src/engine/ir/codegen/
// mlp_train_rust_codegen.rs:249-997).  It exists to check the HIP library:
// only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
// it.  It exports the same C ABI (include/volta_train.h) so one harness can
// drive either library, plus a few oracle-only entry points (volta_oracle_*)
// for an fp64 twin and for kernel-level checks.
//
// Fidelity rules followed here (and why):
//  * fp32 arithmetic in the reference's expression order, no FMA contraction
//    (Rust never contracts; the build uses -ffp-contract=off).
//  * GEMMs sum over k in ascending order per output element.  The reference
//    calls the `gemm` 0.19 crate, whose blocking order is not pinned by any
//    reference test, so bit-equality with the reference DLL is not claimed.
//  * Loss and bias-gradient reductions are sequential, as at :792-798 and
//    :931-933.
//  * Adam uses host powf bias correction (:803-811) and reproduces the
//    vector/scalar-tail split of adam_update_slice (:341-388): elements in
//    the last (n mod 8) positions of each buffer use ((1-b2)*g)*g, the rest
//    (1-b2)*(g*g).
//  * The fp64 twin ("truth") runs the same algorithm in double.
//
// Parity status of each function is recorded next to it ("pinned by ...").
// ===========================================================================
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

#include "../include/volta_train.h"
#include "../volta_amd/csrc/spec.h"

using volta::set_last_error;

namespace {

// --------------------------------------------------------------------------
// Init: reference lcg_xavier_init, mlp_train_rust_codegen.rs:629-638, called
// with one continuing stream seeded 42 over layers 0..n-1 (:653-658).
// Pinned by tests/test_oracle.py (range, moments, stream continuity).
// --------------------------------------------------------------------------
void lcg_xavier_init(float* w, size_t n, int r, int c, uint64_t* rng) {
  const float lim = std::sqrt(6.0f / ((float)r + (float)c));
  for (size_t i = 0; i < n; ++i) {
    *rng = *rng * 6364136223846793005ULL + 1442695040888963407ULL;
    const float f = (float)((*rng >> 11) & ((1ULL << 53) - 1)) / (float)(1ULL << 53);
    w[i] = (f * 2.0f - 1.0f) * lim;
  }
}

// --------------------------------------------------------------------------
// Activations, mlp_train_rust_codegen.rs:563-596 (forward) and :893-916
// (backward).  ReLU is inline at :731 / :894.  Pinned by finite differences
// of the fp64 twin and by the torch-made goldens (tests/golden/).
// --------------------------------------------------------------------------
template <typename T>
inline T sigmoid(T x) { return T(1) / (T(1) + std::exp(-x)); }

template <typename T>
inline T act_fwd(int act, T x) {
  switch (act) {
    case VOLTA_ACT_RELU: return x > T(0) ? x : T(0);
    case VOLTA_ACT_SIGMOID: return sigmoid(x);
    case VOLTA_ACT_TANH: return std::tanh(x);
    case VOLTA_ACT_LEAKY_RELU: return x > T(0) ? x : T(0.01) * x;
    case VOLTA_ACT_SILU: return x * sigmoid(x);
    case VOLTA_ACT_GELU: {
      const T c = T(0.7978845608), k = T(0.044715);
      const T v = c * (x + k * x * x * x);
      return T(0.5) * x * (T(1) + std::tanh(v));
    }
  }
  return x;
}

// Derivative factor.  relu/leaky/silu/gelu take the pre-activation, sigmoid
// and tanh the post-activation value y (:893-916).
template <typename T>
inline T act_bwd(int act, T pre, T y) {
  switch (act) {
    case VOLTA_ACT_RELU: return pre > T(0) ? T(1) : T(0);
    case VOLTA_ACT_SIGMOID: return y * (T(1) - y);
    case VOLTA_ACT_TANH: return T(1) - y * y;
    case VOLTA_ACT_LEAKY_RELU: return pre > T(0) ? T(1) : T(0.01);
    case VOLTA_ACT_SILU: {
      const T s = sigmoid(pre);
      return s * (T(1) + pre * (T(1) - s));
    }
    case VOLTA_ACT_GELU: {
      const T c = T(0.7978845608), k = T(0.044715);
      const T v = c * (pre + k * pre * pre * pre);
      const T t = std::tanh(v);
      const T t2 = T(1) - t * t;
      return T(0.5) * (T(1) + t) + T(0.5) * pre * t2 * c * (T(1) + T(3) * k * pre * pre);
    }
  }
  return T(1);
}

inline bool needs_pre(int act) {
  return act == VOLTA_ACT_RELU || act == VOLTA_ACT_LEAKY_RELU || act == VOLTA_ACT_SILU ||
         act == VOLTA_ACT_GELU;
}

// --------------------------------------------------------------------------
// GEMMs.  C = A·B with every C element summed over k in ascending order,
// starting from 0 (the generator calls gemm with alpha=0, beta=1 so the
// destination is not read: :310-317).  Pinned against the reference's own C
// GEMM (gemm_shim.c, built by oracle/Makefile into oracle/_ref/) and exactly
// on integer-valued inputs.
// --------------------------------------------------------------------------

// C[m x n] = A[m x k] · B[k x n]
template <typename T>
void gemm_nn(T* C, const T* A, const T* B, int m, int k, int n) {
  const int JB = 512;
#pragma omp parallel for schedule(static)
  for (int i0 = 0; i0 < m; i0 += 4) {
    const int i1 = i0 + 4 < m ? i0 + 4 : m;
    for (int j0 = 0; j0 < n; j0 += JB) {
      const int j1 = j0 + JB < n ? j0 + JB : n;
      for (int i = i0; i < i1; ++i)
        for (int j = j0; j < j1; ++j) C[(size_t)i * n + j] = T(0);
      for (int p = 0; p < k; ++p) {
        const T* Bp = B + (size_t)p * n;
        for (int i = i0; i < i1; ++i) {
          const T a = A[(size_t)i * k + p];
          T* Ci = C + (size_t)i * n;
          for (int j = j0; j < j1; ++j) Ci[j] = Ci[j] + a * Bp[j];
        }
      }
    }
  }
}

// C[m x n] = A^T · B with A stored [k x m] (sgemm_tn, :315-317).  The sum
// over k is ascending for every element.
template <typename T>
void gemm_tn(T* C, const T* A, const T* B, int m, int k, int n) {
  const int JB = 512;
#pragma omp parallel for schedule(static)
  for (int i0 = 0; i0 < m; i0 += 4) {
    const int i1 = i0 + 4 < m ? i0 + 4 : m;
    for (int j0 = 0; j0 < n; j0 += JB) {
      const int j1 = j0 + JB < n ? j0 + JB : n;
      for (int i = i0; i < i1; ++i)
        for (int j = j0; j < j1; ++j) C[(size_t)i * n + j] = T(0);
      for (int p = 0; p < k; ++p) {
        const T* Bp = B + (size_t)p * n;
        for (int i = i0; i < i1; ++i) {
          const T a = A[(size_t)p * m + i];
          T* Ci = C + (size_t)i * n;
          for (int j = j0; j < j1; ++j) Ci[j] = Ci[j] + a * Bp[j];
        }
      }
    }
  }
}

#ifdef VOLTA_CPU_REF_GEMM
// CPU-baseline build only (oracle/_ref/libvolta_cpu_ref.so, never a
// checker): the fp32 step's GEMMs are the reference's own C GEMM
// (gemm_shim.c:152-210, compiled from its source by oracle/Makefile), as
// the reference's C compile-train path calls them (mlp_train_codegen.rs:
// 291-384).  The fp64 twin keeps the loops above.
extern "C" {
void volta_gemm_f32(float* C, const float* A, const float* B, int64_t m, int64_t k, int64_t n);
void volta_gemm_tn_f32(float* C, const float* A, const float* B, int64_t m, int64_t k, int64_t n);
}
template <>
void gemm_nn<float>(float* C, const float* A, const float* B, int m, int k, int n) {
  volta_gemm_f32(C, A, B, m, k, n);
}
template <>
void gemm_tn<float>(float* C, const float* A, const float* B, int m, int k, int n) {
  volta_gemm_tn_f32(C, A, B, m, k, n);
}
#endif

// dst[cols x rows] = src[rows x cols]^T (fast_transpose, :389-440).
template <typename T>
void transpose(T* dst, const T* src, int rows, int cols) {
#pragma omp parallel for schedule(static)
  for (int j = 0; j < cols; ++j)
    for (int i = 0; i < rows; ++i) dst[(size_t)j * rows + i] = src[(size_t)i * cols + j];
}

// --------------------------------------------------------------------------
// The network state (Handle, :442-560) and the step (:698-994).
// --------------------------------------------------------------------------
template <typename T>
struct Net {
  volta_mlp_spec spec;
  int B = 0, n = 0;
  std::vector<int> L;
  std::vector<std::vector<T>> w, b, dw, db, mw, vw, mb, vb, gw, gb;
  std::vector<std::vector<T>> act, pre, delta;
  std::vector<T> wt;  // transpose scratch for dX
  // codegen extras (:745-788, :829-892, :936-955)
  std::vector<std::vector<T>> ln_g, ln_b, ln_mu, ln_is, ln_dg, ln_db;
  std::vector<std::vector<uint8_t>> mask;
  uint64_t dropout_rng = 12345678ULL;  // alloc: dropout_rng: 12345678u64 (:553)
  uint64_t adam_step = 0;
  T last_loss = T(0);
  T clip_scale = T(1);  // factor the last step applied to the deltas (clipping)
  // inference model of a `volta compile` library whose graph has no hidden
  // activation (lower_model_to_graph drops all but Relu/Sigmoid,
  // lowering.rs:121-129)
  bool linear_hidden = false;

  void alloc(const volta_mlp_spec& s, int batch) {
    spec = s;
    B = batch;
    n = s.n_sizes - 1;
    L.assign(s.sizes, s.sizes + s.n_sizes);
    auto sz = [](std::vector<std::vector<T>>& v, int cnt) { v.assign(cnt, {}); };
    sz(w, n); sz(b, n); sz(dw, n); sz(db, n); sz(mw, n); sz(vw, n); sz(mb, n); sz(vb, n);
    sz(gw, n); sz(gb, n); sz(delta, n); sz(act, n + 1); sz(pre, n);
    sz(ln_g, n); sz(ln_b, n); sz(ln_mu, n); sz(ln_is, n); sz(ln_dg, n); sz(ln_db, n);
    mask.assign(n, {});
    size_t maxw = 0;
    for (int i = 0; i < n; ++i) {
      const size_t r = L[i], c = L[i + 1];
      w[i].assign(r * c, T(0)); b[i].assign(c, T(0));
      dw[i].assign(r * c, T(0)); db[i].assign(c, T(0));
      if (s.optimizer == VOLTA_OPT_ADAM || s.optimizer == VOLTA_OPT_ADAMW) {
        mw[i].assign(r * c, T(0)); vw[i].assign(r * c, T(0));
        mb[i].assign(c, T(0)); vb[i].assign(c, T(0));
      }
      if (s.optimizer == VOLTA_OPT_ADAGRAD) {
        gw[i].assign(r * c, T(0)); gb[i].assign(c, T(0));
      }
      delta[i].assign((size_t)B * c, T(0));
      if (i < n - 1) pre[i].assign((size_t)B * c, T(0));
      if (i < n - 1 && s.layernorm) {
        ln_g[i].assign(c, T(1)); ln_b[i].assign(c, T(0));  // gamma = 1, beta = 0 (:660-668)
        ln_mu[i].assign(B, T(0)); ln_is[i].assign(B, T(0));
        ln_dg[i].assign(c, T(0)); ln_db[i].assign(c, T(0));
      }
      if (i < n - 1 && s.dropout_p > 0.0f) mask[i].assign((size_t)B * c, 0);
      maxw = r * c > maxw ? r * c : maxw;
    }
    for (int i = 0; i <= n; ++i) act[i].assign((size_t)B * L[i], T(0));
    wt.assign(maxw, T(0));
  }

  // Forward through the hidden layers and the output layer (:702-789).
  void forward(const T* X, bool train = true) {
    std::memcpy(act[0].data(), X, sizeof(T) * (size_t)B * L[0]);
    for (int i = 0; i < n; ++i) {
      const int r = L[i], c = L[i + 1];
      const bool last = i == n - 1;
      T* dst = last ? act[n].data() : pre[i].data();
      gemm_nn(dst, act[i].data(), w[i].data(), B, r, c);
      for (int bi = 0; bi < B; ++bi)
        for (int j = 0; j < c; ++j) dst[(size_t)bi * c + j] = dst[(size_t)bi * c + j] + b[i][j];
      if (!last) {
        T* a = act[i + 1].data();
        const size_t cnt = (size_t)B * c;
        if (linear_hidden) std::copy(dst, dst + cnt, a);
        else if (spec.activation == VOLTA_ACT_SOFTMAX) softmax_fwd(dst, a, c);
        else
          for (size_t k = 0; k < cnt; ++k) a[k] = act_fwd<T>(spec.activation, dst[k]);
        if (spec.layernorm) layernorm_fwd(i);
        if (train && spec.dropout_p > 0.0f) dropout_fwd(i);
      }
    }
  }

  // Softmax as the hidden activation (:727-740): per row, the first maximum
  // (strict >, j ascending), e = exp(pre - max) summed in column order, then
  // act = e * (1 / sum).
  void softmax_fwd(const T* pre_i, T* a, int c) {
    for (int bi = 0; bi < B; ++bi) {
      const T* p = pre_i + (size_t)bi * c;
      T* r = a + (size_t)bi * c;
      T mx = p[0];
      for (int j = 1; j < c; ++j)
        if (p[j] > mx) mx = p[j];
      T sum = T(0);
      for (int j = 0; j < c; ++j) {
        const T e = std::exp(p[j] - mx);
        r[j] = e;
        sum = sum + e;
      }
      const T inv = T(1) / sum;
      for (int j = 0; j < c; ++j) r[j] = r[j] * inv;
    }
  }

  // LayerNorm after the activation (:745-772): per row, sequential f32
  // mean and biased variance, eps 1e-5, then xhat * gamma + beta.
  void layernorm_fwd(int i) {
    const int c = L[i + 1];
    T* a = act[i + 1].data();
    for (int bi = 0; bi < B; ++bi) {
      T* r = a + (size_t)bi * c;
      T mu = T(0);
      for (int j = 0; j < c; ++j) mu = mu + r[j];
      mu = mu / T(c);
      ln_mu[i][bi] = mu;
      T var = T(0);
      for (int j = 0; j < c; ++j) {
        const T d = r[j] - mu;
        var = var + d * d;
      }
      var = var / T(c);
      const T is = T(1) / std::sqrt(var + T(1e-5f));
      ln_is[i][bi] = is;
      for (int j = 0; j < c; ++j) {
        const T xhat = (r[j] - mu) * is;
        r[j] = xhat * ln_g[i][j] + ln_b[i][j];
      }
    }
  }

  // Inverted dropout (:774-788): one LCG draw per element in row-major
  // order, r = (rng >> 33) / 2^31 in f32, keep when r >= p.
  void dropout_fwd(int i) {
    const size_t cnt = (size_t)B * L[i + 1];
    const float p = spec.dropout_p;
    const float keep_scale = 1.0f / (1.0f - p);
    T* a = act[i + 1].data();
    for (size_t k = 0; k < cnt; ++k) {
      dropout_rng = dropout_rng * 6364136223846793005ULL + 1442695040888963407ULL;
      const float r = (float)(dropout_rng >> 33) / 2147483648.0f;
      const uint8_t keep = r >= p ? 1 : 0;
      mask[i][k] = keep;
      a[k] = a[k] * (T((float)keep) * T(keep_scale));
    }
  }

  // LayerNorm backward and its SGD update of gamma/beta (:829-887), in the
  // reference's order: xhat recomputed from the stored output as
  // (y - beta) / (gamma + 1e-12), per-row means of d_xhat and d_xhat*xhat.
  void layernorm_bwd(int i, T lr) {
    const int c = L[i + 1];
    T* d = delta[i].data();
    const T* y = act[i + 1].data();
    std::vector<T>& g = ln_g[i];
    std::vector<T>& be = ln_b[i];
    std::vector<T>& dg = ln_dg[i];
    std::vector<T>& dbe = ln_db[i];
    std::fill(dg.begin(), dg.end(), T(0));
    std::fill(dbe.begin(), dbe.end(), T(0));
    for (int bi = 0; bi < B; ++bi) {
      const size_t base = (size_t)bi * c;
      const T is = ln_is[i][bi];
      T sum_d = T(0), sum_dxh = T(0);
      for (int j = 0; j < c; ++j) {
        const T xh = (y[base + j] - be[j]) / (g[j] + T(1e-12f));
        const T dout = d[base + j];
        dg[j] = dg[j] + dout * xh;
        dbe[j] = dbe[j] + dout;
        sum_d = sum_d + dout * g[j];
        sum_dxh = sum_dxh + dout * g[j] * xh;
      }
      sum_d = sum_d / T(c);
      sum_dxh = sum_dxh / T(c);
      for (int j = 0; j < c; ++j) {
        const T xh = (y[base + j] - be[j]) / (g[j] + T(1e-12f));
        const T d_xhat = d[base + j] * g[j];
        d[base + j] = is * (d_xhat - sum_d - xh * sum_dxh);
      }
    }
    for (int j = 0; j < c; ++j) g[j] = g[j] - lr * dg[j];
    for (int j = 0; j < c; ++j) be[j] = be[j] - lr * dbe[j];
  }

  // MSE loss and seed gradient, :792-798.  Pinned by torch goldens.
  void loss_mse(const T* Y) {
    const size_t nt = (size_t)B * L[n];
    const T ntf = T(nt);
    T lacc = T(0);
    T* d_out = delta[n - 1].data();
    const T* yhat = act[n].data();
    for (size_t k = 0; k < nt; ++k) {
      const T d = yhat[k] - Y[k];
      lacc = lacc + d * d;
      d_out[k] = T(2) * d / ntf;
    }
    last_loss = lacc / ntf;
  }

  // Softmax cross-entropy from logits with one-hot targets given as labels:
  // loss per interpreter.rs:762-812 (row max, sequential exp-sum, log-sum-exp,
  // mean over B), gradient per autograd.rs:467-534 ((softmax - t) / B with
  // softmax per kernels/reduce.rs:203-213).  Pinned by torch goldens and the
  // uniform-logits closed form (loss = ln C).
  void loss_ce(const int32_t* labels) {
    const int C = L[n];
    const T* z = act[n].data();
    T* d_out = delta[n - 1].data();
    T loss_sum = T(0);
    const T bf = T(B);
    std::vector<T> e(C);
    for (int bi = 0; bi < B; ++bi) {
      const T* zr = z + (size_t)bi * C;
      T mx = -INFINITY;
      for (int j = 0; j < C; ++j) mx = std::fmax(mx, zr[j]);
      T sum_exp = T(0);
      for (int j = 0; j < C; ++j) sum_exp = sum_exp + std::exp(zr[j] - mx);
      const T lse = mx + std::log(sum_exp);
      const int lab = labels[bi];
      T sample = T(0);
      for (int j = 0; j < C; ++j) {
        const T t = j == lab ? T(1) : T(0);
        sample = sample - t * (zr[j] - lse);
      }
      loss_sum = loss_sum + sample;
      // gradient: softmax recomputed the way reduce::softmax does it
      T s2 = T(0);
      for (int j = 0; j < C; ++j) {
        e[j] = std::exp(zr[j] - mx);
        s2 = s2 + e[j];
      }
      for (int j = 0; j < C; ++j) {
        const T t = j == lab ? T(1) : T(0);
        d_out[(size_t)bi * C + j] = (e[j] / s2 - t) / bf;
      }
    }
    last_loss = loss_sum / bf;
  }

  // Adam/AdamW element update, adam_update_slice :341-388.  `tail` selects
  // the scalar-tail expression for v.
  static inline void adam_elem(T* w, T* m, T* v, T g, T b1, T b2, T bc1, T bc2, T lr, T eps,
                               T wd, bool tail) {
    const T m1 = b1 * *m + (T(1) - b1) * g;
    const T v1 = tail ? b2 * *v + (T(1) - b2) * g * g : b2 * *v + (T(1) - b2) * (g * g);
    *m = m1;
    *v = v1;
    const T w0 = *w;
    const T mhat = m1 / bc1;
    const T vhat = v1 / bc2;
    const T denom = std::sqrt(vhat) + eps;
    *w = w0 - lr * (mhat / denom + wd * w0);
  }

  // adam_update (:326-340): buffers of at least 2^17 elements are cut into
  // 8192-element chunks updated in parallel (Rayon there, OpenMP here).
  // Every chunk but the last is a multiple of 8 long, so the scalar-tail
  // elements are the last (cnt mod 8) of the buffer either way and the
  // result does not depend on the thread count.
  static void adam_update(T* w, T* m, T* v, const T* g, size_t cnt, T b1, T b2, T bc1, T bc2,
                          T lr, T eps, T wd) {
    const size_t vec_end = cnt - cnt % 8;
    const size_t kChunk = 8192;
    const long long chunks = (long long)((cnt + kChunk - 1) / kChunk);
#pragma omp parallel for schedule(static) if (cnt >= (size_t(1) << 17))
    for (long long q = 0; q < chunks; ++q) {
      const size_t k0 = (size_t)q * kChunk, k1 = std::min(cnt, k0 + kChunk);
      for (size_t k = k0; k < k1; ++k)
        adam_elem(w + k, m + k, v + k, g[k], b1, b2, bc1, bc2, lr, eps, wd, k >= vec_end);
    }
  }

  // Adagrad, :967-985.
  static void adagrad_update(T* w, T* G, const T* g, size_t cnt, T lr, T eps) {
    for (size_t k = 0; k < cnt; ++k) {
      const T gk = g[k];
      G[k] = G[k] + gk * gk;
      w[k] = w[k] - lr * gk / (std::sqrt(G[k]) + eps);
    }
  }

  void backward_and_update(T lr) {
    const int act_kind = spec.activation;
    // Adam bias correction with f32 powf on the host step counter (:803-811).
    T bc1 = T(1), bc2 = T(1);
    const bool adam = spec.optimizer == VOLTA_OPT_ADAM || spec.optimizer == VOLTA_OPT_ADAMW;
    if (adam) {
      adam_step += 1;
      const float t = (float)adam_step;
      bc1 = T(1.0f - powf(spec.beta1, t));
      bc2 = T(1.0f - powf(spec.beta2, t));
      if (sizeof(T) == sizeof(double)) {
        bc1 = T(1) - std::pow(T(spec.beta1), T(adam_step));
        bc2 = T(1) - std::pow(T(spec.beta2), T(adam_step));
      }
    }
    // Phase 1: deltas for every layer, then db (:819-934).
    for (int i = n - 1; i >= 0; --i) {
      const int r = L[i], c = L[i + 1];
      const size_t cnt = (size_t)B * c;
      T* d = delta[i].data();
      if (i != n - 1) {
        // LayerNorm backward, then the dropout mask, then the activation
        // derivative (:824-916); sigmoid/tanh take act_{i+1}, which holds
        // the LayerNorm/dropout output when those are on (:908-914).
        if (spec.layernorm) layernorm_bwd(i, lr);
        if (spec.dropout_p > 0.0f) {
          const float keep_scale = 1.0f / (1.0f - spec.dropout_p);
          for (size_t k = 0; k < cnt; ++k) d[k] = d[k] * (T((float)mask[i][k]) * T(keep_scale));
        }
        const T* p = pre[i].data();
        const T* y = act[i + 1].data();
        if (act_kind == VOLTA_ACT_SOFTMAX) {
          // dx = y * (upstream - dot(upstream, y)) per row, y = act_{i+1}
          // (the LayerNorm/dropout output when those are on) (:898-906)
          for (int bi = 0; bi < B; ++bi) {
            const size_t base = (size_t)bi * c;
            T dot = T(0);
            for (int j = 0; j < c; ++j) dot = dot + d[base + j] * y[base + j];
            for (int j = 0; j < c; ++j) d[base + j] = y[base + j] * (d[base + j] - dot);
          }
        } else {
          for (size_t k = 0; k < cnt; ++k) d[k] = d[k] * act_bwd<T>(act_kind, p[k], y[k]);
        }
      }
      if (i > 0) {
        // delta_{i-1} = delta_i · W_i^T, computed as (W_i · delta_i^T)^T in the
        // reference (:919-929); summing over k ascending either way.
        transpose(wt.data(), w[i].data(), r, c);  // wt [c x r]
        gemm_nn(delta[i - 1].data(), d, wt.data(), B, c, r);
      }
      T* dbi = db[i].data();
      for (int j = 0; j < c; ++j) dbi[j] = T(0);
      for (int bi = 0; bi < B; ++bi)
        for (int j = 0; j < c; ++j) dbi[j] = dbi[j] + d[(size_t)bi * c + j];
    }
    // Gradient clipping by the global norm of the deltas (:936-955), after
    // db was formed from the unscaled deltas.
    if (spec.clip_grad > 0.0f) {
      T gsq = T(0);
      for (int i = 0; i < n; ++i)
        for (const T v : delta[i]) gsq = gsq + v * v;
      const T gnorm = std::sqrt(gsq);
      const T cv = T(spec.clip_grad);
      const T scale = gnorm > cv ? cv / gnorm : T(1);
      clip_scale = scale;
      if (scale < T(1))
        for (int i = 0; i < n; ++i)
          for (T& v : delta[i]) v = v * scale;
    }
    // Phase 2: parameter updates, last layer first (:957-993).
    const T tlr = lr;
    for (int i = n - 1; i >= 0; --i) {
      const int r = L[i], c = L[i + 1];
      const size_t rc = (size_t)r * c;
      gemm_tn(dw[i].data(), act[i].data(), delta[i].data(), r, B, c);
      if (adam) {
        const T wd = spec.optimizer == VOLTA_OPT_ADAMW ? T(spec.weight_decay) : T(0);
        adam_update(w[i].data(), mw[i].data(), vw[i].data(), dw[i].data(), rc, T(spec.beta1),
                    T(spec.beta2), bc1, bc2, tlr, T(spec.eps), wd);
        adam_update(b[i].data(), mb[i].data(), vb[i].data(), db[i].data(), (size_t)c,
                    T(spec.beta1), T(spec.beta2), bc1, bc2, tlr, T(spec.eps), T(0));
      } else if (spec.optimizer == VOLTA_OPT_ADAGRAD) {
        adagrad_update(w[i].data(), gw[i].data(), dw[i].data(), rc, tlr, T(spec.eps));
        adagrad_update(b[i].data(), gb[i].data(), db[i].data(), (size_t)c, tlr, T(spec.eps));
      } else {
        // sgd_fused_tn: W = 1*W + (-lr)*(act^T delta)  (:321-324, :986-991)
        T* wi = w[i].data();
        const T* g = dw[i].data();
        const T nlr = -tlr;
#pragma omp parallel for schedule(static) if (rc >= (size_t(1) << 17))
        for (long long k = 0; k < (long long)rc; ++k) wi[k] = wi[k] + nlr * g[k];
        for (int k = 0; k < c; ++k) b[i][k] = b[i][k] - tlr * db[i][k];
      }
    }
  }
};

// The handle bound for volta_infer (volta_infer_bind); cleared when freed.
static std::mutex g_infer_mu;
static VoltaTrainHandle* g_infer_model = nullptr;

static void unbind_infer(VoltaTrainHandle* vh) {
  std::lock_guard<std::mutex> lock(g_infer_mu);
  if (g_infer_model == vh) g_infer_model = nullptr;
}

struct Handle {
  int precision = 32;  // 32: reference-faithful fp32; 64: fp64 twin
  Net<float> f;
  Net<double> d;
  std::vector<std::vector<float>> w_mirror, b_mirror;  // fp64 twin -> fp32 view
  int32_t status = 0;
  std::vector<double> xbuf, ybuf;
};

Handle* make_handle(const volta_mlp_spec* spec, int32_t batch, int precision) {
  std::string why;
  if (!spec || !volta::validate_spec(*spec, &why)) {
    set_last_error("oracle init: invalid spec: " + why);
    return nullptr;
  }
  if (batch <= 0) {
    set_last_error("oracle init: batch must be > 0");
    return nullptr;
  }
  auto h = std::make_unique<Handle>();
  h->precision = precision;
  const int n = spec->n_sizes - 1;
  // Weights from the reference LCG stream (f32) for both precisions.
  std::vector<std::vector<float>> w0(n);
  uint64_t rng = 42;
  for (int i = 0; i < n; ++i) {
    const int r = spec->sizes[i], c = spec->sizes[i + 1];
    w0[i].assign((size_t)r * c, 0.0f);
    lcg_xavier_init(w0[i].data(), w0[i].size(), r, c, &rng);
  }
  if (precision == 64) {
    h->d.alloc(*spec, batch);
    for (int i = 0; i < n; ++i)
      for (size_t k = 0; k < w0[i].size(); ++k) h->d.w[i][k] = w0[i][k];
    h->w_mirror.resize(n);
    h->b_mirror.resize(n);
    for (int i = 0; i < n; ++i) {
      h->w_mirror[i].assign(w0[i].size(), 0.0f);
      h->b_mirror[i].assign((size_t)spec->sizes[i + 1], 0.0f);
    }
  } else {
    h->f.alloc(*spec, batch);
    for (int i = 0; i < n; ++i) h->f.w[i] = w0[i];
  }
  return h.release();
}

}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" {

VoltaTrainHandle* volta_train_init_spec(const volta_mlp_spec* spec, int32_t batch) {
  return reinterpret_cast<VoltaTrainHandle*>(make_handle(spec, batch, 32));
}

VoltaTrainHandle* volta_train_init(int32_t batch) {
  volta_mlp_spec s;
  if (!volta::resolve_default_spec(&s)) return nullptr;
  return volta_train_init_spec(&s, batch);
}

// fp64 twin of the same algorithm ("truth" for error budgets).
VoltaTrainHandle* volta_oracle_init_f64(const volta_mlp_spec* spec, int32_t batch) {
  return reinterpret_cast<VoltaTrainHandle*>(make_handle(spec, batch, 64));
}

static Handle* H(VoltaTrainHandle* h) { return reinterpret_cast<Handle*>(h); }

static void step_impl(Handle* h, const float* X, const float* Y, const int32_t* labels, float lr) {
  if (h->precision == 64) {
    Net<double>& net = h->d;
    const size_t nx = (size_t)net.B * net.L[0];
    h->xbuf.assign(X, X + nx);
    net.forward(h->xbuf.data());
    if (labels) {
      net.loss_ce(labels);
    } else {
      const size_t ny = (size_t)net.B * net.L[net.n];
      h->ybuf.assign(Y, Y + ny);
      net.loss_mse(h->ybuf.data());
    }
    net.backward_and_update((double)lr);
    if (!std::isfinite(net.last_loss)) h->status |= VOLTA_STATUS_NONFINITE_LOSS;
  } else {
    Net<float>& net = h->f;
    net.forward(X);
    if (labels) net.loss_ce(labels);
    else net.loss_mse(Y);
    net.backward_and_update(lr);
    if (!std::isfinite(net.last_loss)) h->status |= VOLTA_STATUS_NONFINITE_LOSS;
  }
}

void volta_train_step(VoltaTrainHandle* vh, const float* X, const float* Y, float lr) {
  Handle* h = H(vh);
  if (!h) return;
  const volta_mlp_spec& s = h->precision == 64 ? h->d.spec : h->f.spec;
  if (!X || !Y || s.loss != VOLTA_LOSS_MSE) {
    h->status |= VOLTA_STATUS_BAD_ARGUMENT;
    set_last_error("volta_train_step: null input or spec loss is not MSE");
    return;
  }
  step_impl(h, X, Y, nullptr, lr);
}

void volta_train_step_labels(VoltaTrainHandle* vh, const float* X, const int32_t* labels,
                             float lr) {
  Handle* h = H(vh);
  if (!h) return;
  const volta_mlp_spec& s = h->precision == 64 ? h->d.spec : h->f.spec;
  const int B = h->precision == 64 ? h->d.B : h->f.B;
  if (!X || !labels || s.loss != VOLTA_LOSS_SOFTMAX_CE) {
    h->status |= VOLTA_STATUS_BAD_ARGUMENT;
    set_last_error("volta_train_step_labels: null input or spec loss is not softmax-CE");
    return;
  }
  const int C = s.sizes[s.n_sizes - 1];
  for (int i = 0; i < B; ++i)
    if (labels[i] < 0 || labels[i] >= C) {
      h->status |= VOLTA_STATUS_BAD_ARGUMENT;
      set_last_error("volta_train_step_labels: label out of range");
      return;
    }
  step_impl(h, X, nullptr, labels, lr);
}

int32_t volta_train_step_device(VoltaTrainHandle* vh, const float* X, const void* Y, float lr) {
  Handle* h = H(vh);
  if (!h) return -1;
  const volta_mlp_spec& s = h->precision == 64 ? h->d.spec : h->f.spec;
  if (s.loss == VOLTA_LOSS_SOFTMAX_CE)
    volta_train_step_labels(vh, X, static_cast<const int32_t*>(Y), lr);
  else
    volta_train_step(vh, X, static_cast<const float*>(Y), lr);
  return (h->status & VOLTA_STATUS_BAD_ARGUMENT) ? -1 : 0;
}

int32_t volta_train_batch_buffers(VoltaTrainHandle*, float**, void**) {
  set_last_error("the CPU oracle has no resident device batch");
  return -1;
}

float volta_train_loss(VoltaTrainHandle* vh) {
  Handle* h = H(vh);
  if (!h) return NAN;
  return h->precision == 64 ? (float)h->d.last_loss : h->f.last_loss;
}

double volta_oracle_loss_f64(VoltaTrainHandle* vh) {
  Handle* h = H(vh);
  if (!h) return NAN;
  return h->precision == 64 ? h->d.last_loss : (double)h->f.last_loss;
}

void volta_train_get_params(VoltaTrainHandle* vh, float** wo, float** bo) {
  Handle* h = H(vh);
  if (!h || !wo || !bo) return;
  if (h->precision == 64) {
    for (int i = 0; i < h->d.n; ++i) {
      for (size_t k = 0; k < h->w_mirror[i].size(); ++k) h->w_mirror[i][k] = (float)h->d.w[i][k];
      for (size_t k = 0; k < h->b_mirror[i].size(); ++k) h->b_mirror[i][k] = (float)h->d.b[i][k];
      wo[i] = h->w_mirror[i].data();
      bo[i] = h->b_mirror[i].data();
    }
  } else {
    for (int i = 0; i < h->f.n; ++i) {
      wo[i] = h->f.w[i].data();
      bo[i] = h->f.b[i].data();
    }
  }
}

// fp64 parameters of layer li (either precision).
int32_t volta_oracle_get_params_f64(VoltaTrainHandle* vh, int32_t li, double* w, double* b) {
  Handle* h = H(vh);
  if (!h) return -1;
  const int n = h->precision == 64 ? h->d.n : h->f.n;
  if (li < 0 || li >= n) return -1;
  if (h->precision == 64) {
    std::copy(h->d.w[li].begin(), h->d.w[li].end(), w);
    std::copy(h->d.b[li].begin(), h->d.b[li].end(), b);
  } else {
    std::copy(h->f.w[li].begin(), h->f.w[li].end(), w);
    std::copy(h->f.b[li].begin(), h->f.b[li].end(), b);
  }
  return 0;
}

void volta_train_set_params(VoltaTrainHandle* vh, int32_t li, const float* w, const float* b) {
  Handle* h = H(vh);
  if (!h) return;
  const int n = h->precision == 64 ? h->d.n : h->f.n;
  if (li < 0 || li >= n || !w || !b) {
    h->status |= VOLTA_STATUS_BAD_ARGUMENT;
    return;
  }
  if (h->precision == 64) {
    for (size_t k = 0; k < h->d.w[li].size(); ++k) h->d.w[li][k] = w[k];
    for (size_t k = 0; k < h->d.b[li].size(); ++k) h->d.b[li][k] = b[k];
  } else {
    std::copy(w, w + h->f.w[li].size(), h->f.w[li].begin());
    std::copy(b, b + h->f.b[li].size(), h->f.b[li].begin());
  }
}

void volta_train_free(VoltaTrainHandle* vh) {
  if (!vh) return;
  unbind_infer(vh);
  delete H(vh);
}

int32_t volta_train_sync(VoltaTrainHandle*) { return 0; }

int32_t volta_train_status(VoltaTrainHandle* vh) {
  Handle* h = H(vh);
  return h ? h->status : VOLTA_STATUS_BAD_ARGUMENT;
}

void volta_train_clear_status(VoltaTrainHandle* vh) {
  if (Handle* h = H(vh)) h->status = 0;
}

int32_t volta_train_num_layers(VoltaTrainHandle* vh) {
  Handle* h = H(vh);
  if (!h) return -1;
  return h->precision == 64 ? h->d.n : h->f.n;
}

int32_t volta_train_batch(VoltaTrainHandle* vh) {
  Handle* h = H(vh);
  if (!h) return -1;
  return h->precision == 64 ? h->d.B : h->f.B;
}

}  // extern "C"

// Training state in the ABI's order: per layer [m_W | m_b | v_W | v_b]
// (Adam/AdamW) or [G_W | G_b] (Adagrad), then, with LayerNorm, [gamma_i |
// beta_i] per hidden layer.  Either precision; the fp64 twin converts
// from/to float so it can be started from a float state.
template <typename T>
static std::vector<std::vector<T>*> state_buffers(Net<T>& f) {
  std::vector<std::vector<T>*> v;
  for (int i = 0; i < f.n; ++i) {
    if (f.spec.optimizer == VOLTA_OPT_ADAM || f.spec.optimizer == VOLTA_OPT_ADAMW) {
      v.insert(v.end(), {&f.mw[i], &f.mb[i], &f.vw[i], &f.vb[i]});
    } else if (f.spec.optimizer == VOLTA_OPT_ADAGRAD) {
      v.insert(v.end(), {&f.gw[i], &f.gb[i]});
    }
  }
  if (f.spec.layernorm)
    for (int i = 0; i < f.n - 1; ++i) v.insert(v.end(), {&f.ln_g[i], &f.ln_b[i]});
  return v;
}

template <typename T>
static int64_t state_size(Net<T>& f) {
  int64_t total = 0;
  for (auto* v : state_buffers(f)) total += (int64_t)v->size();
  return total;
}

template <typename T>
static void state_get(Net<T>& f, float* p, int64_t* step) {
  for (auto* v : state_buffers(f))
    for (size_t k = 0; k < v->size(); ++k) *p++ = (float)(*v)[k];
  if (step) *step = (int64_t)f.adam_step;
}

template <typename T>
static void state_set(Net<T>& f, const float* p, int64_t step) {
  for (auto* v : state_buffers(f))
    for (size_t k = 0; k < v->size(); ++k) (*v)[k] = T(*p++);
  f.adam_step = (uint64_t)step;
}

extern "C" {

int64_t volta_train_state_size(VoltaTrainHandle* vh) {
  Handle* h = H(vh);
  if (!h) return -1;
  return h->precision == 64 ? state_size(h->d) : state_size(h->f);
}

int32_t volta_train_get_state(VoltaTrainHandle* vh, float* state, int64_t* step) {
  Handle* h = H(vh);
  if (!h || (!state && volta_train_state_size(vh) > 0)) return -1;
  if (h->precision == 64) state_get(h->d, state, step);
  else state_get(h->f, state, step);
  return 0;
}

int32_t volta_train_set_state(VoltaTrainHandle* vh, const float* state, int64_t step) {
  Handle* h = H(vh);
  if (!h || step < 0 || (!state && volta_train_state_size(vh) > 0)) return -1;
  if (h->precision == 64) state_set(h->d, state, step);
  else state_set(h->f, state, step);
  return 0;
}

int32_t volta_train_get_dropout_rng(VoltaTrainHandle* vh, uint64_t* rng) {
  Handle* h = H(vh);
  if (!h || !rng) return -1;
  *rng = h->precision == 64 ? h->d.dropout_rng : h->f.dropout_rng;
  return 0;
}

int32_t volta_train_set_dropout_rng(VoltaTrainHandle* vh, uint64_t rng) {
  Handle* h = H(vh);
  if (!h) return -1;
  h->d.dropout_rng = rng;
  h->f.dropout_rng = rng;
  return 0;
}

}  // extern "C"

template <typename T>
static int64_t copy_out(const std::vector<T>& v, float* out) {
  for (size_t k = 0; k < v.size(); ++k) out[k] = (float)v[k];
  return (int64_t)v.size();
}

template <typename T>
static int64_t copy_out(const std::vector<T>& v, double* out) {
  for (size_t k = 0; k < v.size(); ++k) out[k] = (double)v[k];
  return (int64_t)v.size();
}

template <typename T, typename O>
static int64_t debug_buffer(Net<T>& f, int kind, int layer, O* out) {
  switch (kind) {
    case VOLTA_BUF_ACT: return layer >= 0 && layer <= f.n ? copy_out(f.act[layer], out) : -1;
    case VOLTA_BUF_DELTA: return layer >= 0 && layer < f.n ? copy_out(f.delta[layer], out) : -1;
    case VOLTA_BUF_GRAD_W: return layer >= 0 && layer < f.n ? copy_out(f.dw[layer], out) : -1;
    case VOLTA_BUF_GRAD_B: return layer >= 0 && layer < f.n ? copy_out(f.db[layer], out) : -1;
    case VOLTA_BUF_PRE:
      return layer >= 0 && layer < f.n - 1 && f.pre[layer].size() ? copy_out(f.pre[layer], out) : -1;
    case VOLTA_BUF_LN_GAMMA:
      return f.spec.layernorm && layer >= 0 && layer < f.n - 1 ? copy_out(f.ln_g[layer], out) : -1;
    case VOLTA_BUF_LN_BETA:
      return f.spec.layernorm && layer >= 0 && layer < f.n - 1 ? copy_out(f.ln_b[layer], out) : -1;
    case VOLTA_BUF_LN_DGAMMA:
      return f.spec.layernorm && layer >= 0 && layer < f.n - 1 ? copy_out(f.ln_dg[layer], out) : -1;
    case VOLTA_BUF_LN_DBETA:
      return f.spec.layernorm && layer >= 0 && layer < f.n - 1 ? copy_out(f.ln_db[layer], out) : -1;
    case VOLTA_BUF_CLIP_SCALE:
      if (!(f.spec.clip_grad > 0.0f)) return -1;
      out[0] = (O)f.clip_scale;
      return 1;
    case VOLTA_BUF_DROPOUT_MASK:
      if (!(f.spec.dropout_p > 0.0f) || layer < 0 || layer >= f.n - 1) return -1;
      for (size_t k = 0; k < f.mask[layer].size(); ++k) out[k] = (O)f.mask[layer][k];
      return (int64_t)f.mask[layer].size();
  }
  return -1;
}

extern "C" {

int64_t volta_train_debug_buffer(VoltaTrainHandle* vh, int32_t kind, int32_t layer, float* out) {
  Handle* h = H(vh);
  if (!h || !out) return -1;
  return h->precision == 64 ? debug_buffer(h->d, kind, layer, out) : debug_buffer(h->f, kind, layer, out);
}

// The same buffers in double: the fp64 twin's values without rounding to
// fp32 (the fp32 oracle's values widened).
int64_t volta_oracle_debug_buffer_f64(VoltaTrainHandle* vh, int32_t kind, int32_t layer, double* out) {
  Handle* h = H(vh);
  if (!h || !out) return -1;
  return h->precision == 64 ? debug_buffer(h->d, kind, layer, out) : debug_buffer(h->f, kind, layer, out);
}

// ---------------------------------------------------------------------------
// Kernel-level oracle entry points (fp32), used to check single HIP kernels.
// ---------------------------------------------------------------------------

// C[m x n] = op(A) · op(B); ta: A stored [k x m]; tb: B stored [n x k].
void volta_oracle_gemm(float* C, const float* A, const float* B, int32_t m, int32_t k, int32_t n,
                       int32_t ta, int32_t tb) {
  std::vector<float> bt;
  const float* Bn = B;
  if (tb) {
    bt.resize((size_t)k * n);
    transpose(bt.data(), B, n, k);
    Bn = bt.data();
  }
  if (ta) gemm_tn(C, A, Bn, m, k, n);
  else gemm_nn(C, A, Bn, m, k, n);
}

// Adam/AdamW update of one buffer (adam_update, :326-388).
void volta_oracle_adam(float* w, float* m, float* v, const float* g, int64_t cnt, float b1, float b2,
                       float bc1, float bc2, float lr, float eps, float wd) {
  Net<float>::adam_update(w, m, v, g, (size_t)cnt, b1, b2, bc1, bc2, lr, eps, wd);
}

void volta_oracle_adagrad(float* w, float* G, const float* g, int64_t cnt, float lr, float eps) {
  Net<float>::adagrad_update(w, G, g, (size_t)cnt, lr, eps);
}

void volta_oracle_lcg_xavier(float* w, int64_t cnt, int32_t r, int32_t c, uint64_t* rng) {
  lcg_xavier_init(w, (size_t)cnt, r, c, rng);
}

// Adam's bias correction 1 - beta^t as the step computes it: f32 powf of
// the step counter (:803-811).
float volta_oracle_bias_correction(float beta, int64_t t) { return 1.0f - powf(beta, (float)t); }

// Activation derivative over n elements in double (checks of whole buffers).
void volta_oracle_act_bwd_f64_n(int32_t act, const double* pre, const double* y, double* out, int64_t n) {
  for (int64_t k = 0; k < n; ++k) out[k] = act_bwd<double>(act, pre[k], y[k]);
}

float volta_oracle_act_fwd(int32_t act, float x) { return act_fwd<float>(act, x); }
float volta_oracle_act_bwd(int32_t act, float pre, float y) { return act_bwd<float>(act, pre, y); }
double volta_oracle_act_fwd_f64(int32_t act, double x) { return act_fwd<double>(act, x); }
double volta_oracle_act_bwd_f64(int32_t act, double pre, double y) {
  return act_bwd<double>(act, pre, y);
}

int32_t volta_oracle_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

// Thread count of the OpenMP loops (CPU-baseline timing at a stated count).
void volta_oracle_set_threads(int32_t n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Hyperparameters of a live handle, and the forward-only entry points
// (same contract as include/volta_train.h).
// ---------------------------------------------------------------------------
template <typename T>
static void infer_rows(Net<T>& net, const float* X, int64_t rows, float* out) {
  const int B = net.B, L0 = net.L[0], Ln = net.L[net.n];
  std::vector<T> xb((size_t)B * L0, T(0));
  for (int64_t r0 = 0; r0 < rows; r0 += B) {
    const int64_t m = std::min<int64_t>(B, rows - r0);
    std::fill(xb.begin(), xb.end(), T(0));
    for (int64_t k = 0; k < m * L0; ++k) xb[(size_t)k] = (T)X[r0 * L0 + k];
    net.forward(xb.data(), false);  // inference: LayerNorm, no dropout
    for (int64_t k = 0; k < m * Ln; ++k) out[r0 * Ln + k] = (float)net.act[net.n][(size_t)k];
  }
}

extern "C" {

int32_t volta_train_set_hparams(VoltaTrainHandle* vh, float beta1, float beta2, float eps, float weight_decay) {
  Handle* h = H(vh);
  if (!h) return -1;
  volta_mlp_spec s = h->precision == 64 ? h->d.spec : h->f.spec;
  s.beta1 = beta1;
  s.beta2 = beta2;
  s.eps = eps;
  s.weight_decay = weight_decay;
  std::string why;
  if (!volta::validate_spec(s, &why)) {
    h->status |= VOLTA_STATUS_BAD_ARGUMENT;
    set_last_error("volta_train_set_hparams: " + why);
    return -1;
  }
  if (h->precision == 64) h->d.spec = s;
  else h->f.spec = s;
  return 0;
}

int32_t volta_train_infer(VoltaTrainHandle* vh, const float* X, int64_t rows, float* out) {
  Handle* h = H(vh);
  if (!h) return -1;
  if (!X || !out || rows <= 0) {
    h->status |= VOLTA_STATUS_BAD_ARGUMENT;
    set_last_error("volta_train_infer: bad arguments");
    return -1;
  }
  if (h->precision == 64) infer_rows(h->d, X, rows, out);
  else infer_rows(h->f, X, rows, out);
  return 0;
}

// The inference model of a `volta compile` library: the forward graph of
// lower_model_to_graph (lowering.rs:87-140) with ReLU hidden layers
// (hidden_act VOLTA_ACT_RELU) or none (-1), parameters [W_0|b_0|W_1|...].
VoltaTrainHandle* volta_infer_model_create(int32_t n_sizes, const int32_t* sizes, int32_t hidden_act,
                                           const float* params) {
  if (n_sizes < 2 || n_sizes > VOLTA_MAX_LAYER_SIZES || !sizes || !params ||
      (hidden_act != VOLTA_ACT_RELU && hidden_act != -1)) {
    set_last_error("volta_infer_model_create: bad arguments");
    return nullptr;
  }
  volta_mlp_spec s;
  volta_mlp_spec_default(&s, n_sizes, sizes, VOLTA_ACT_RELU, VOLTA_OPT_SGD, VOLTA_LOSS_MSE);
  VoltaTrainHandle* vh = volta_train_init_spec(&s, 64);
  if (!vh) return nullptr;
  H(vh)->f.linear_hidden = hidden_act == -1;
  const float* p = params;
  for (int i = 0; i + 1 < n_sizes; ++i) {
    const int64_t r = sizes[i], c = sizes[i + 1];
    volta_train_set_params(vh, i, p, p + r * c);
    p += r * c + c;
  }
  return vh;
}

// The CPU library's memory is host memory: the allocation-free variant is
// volta_train_infer on the same buffers.
int32_t volta_train_infer_device_noalloc(VoltaTrainHandle* vh, const float* X, int64_t rows, float* out) {
  return volta_train_infer(vh, X, rows, out);
}

int32_t volta_infer_bind(VoltaTrainHandle* vh) {
  std::lock_guard<std::mutex> lock(g_infer_mu);
  g_infer_model = vh;
  return 0;
}

void volta_infer(const float* input, int64_t in_n, float* output, int64_t out_n) {
  std::lock_guard<std::mutex> lock(g_infer_mu);
  Handle* h = H(g_infer_model);
  if (!h) {
    set_last_error("volta_infer: no model bound (volta_infer_bind)");
    return;
  }
  const std::vector<int>& L = h->precision == 64 ? h->d.L : h->f.L;
  const int L0 = L.front(), Ln = L.back();
  if (!input || !output || in_n <= 0 || in_n % L0 != 0 || out_n < in_n / L0 * Ln) {
    h->status |= VOLTA_STATUS_BAD_ARGUMENT;
    set_last_error("volta_infer: in_n must be rows*L0 and out_n >= rows*Ln");
    return;
  }
  (void)volta_train_infer(g_infer_model, input, in_n / L0, output);
}

}  // extern "C"
