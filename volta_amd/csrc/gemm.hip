// fp32 GEMM family on CDNA4 fp32 MFMA (v_mfma_f32_32x32x2_f32), with the
// step's other work fused into the epilogue: bias + activation (forward),
// activation derivative (dX), bias-gradient column sums + optimizer update
// (dW), and the loss head (output layer).
//
//   C[M x N] = sum_k A(m,k) * B(k,n)
//
// Operand storage (row-major in memory, as the reference keeps them):
//   A_KC:  A(m,k) = A[m*lda + k]   (forward act_i, dX delta_i)
//   A_MC:  A(m,k) = A[k*lda + m]   (dW: act_i^T)
//   B_KC:  B(k,n) = B[n*ldb + k]   (dX: W_i^T)
//   B_NC:  B(k,n) = B[k*ldb + n]   (forward W_i, dW delta_i)
// None of the three products of the step (NN forward, NT dX, TN dW) needs an
// explicit transpose: each operand tile goes to LDS in its memory order and
// the MFMA operands are read out of LDS in either order (see load_frag).
//
// k-order inside one MFMA: a 64-lane wave holds two k values per MFMA (lane
// half h = lane/32).  Within each group of 8 k values, MFMA s (0..3) takes
// k = 8g + 4h + s, so a lane's four operands of a group are four consecutive
// k of one row -- a single 16-byte LDS read for K-contiguous tiles.  The
// order is fixed, so results are bit-identical from run to run.
//
// Split-K: blockIdx.y selects a K slice.  Each slice writes its partial tile
// to its own workspace plane, then bumps the tile's arrival counter; the
// last slice to arrive adds the planes in slice order (0, 1, ...) and runs
// the epilogue.  The sum order is fixed whatever the arrival order, and the
// counter is an integer, so results stay bit-identical; the last slice
// resets the counter to zero for the next launch.
#include "gemm.h"
#include "narrow_dw.h"
#include "out_head.h"

#include <cstdlib>
#include <type_traits>

namespace volta {

template <int BM, int BN, int BK, int WM, int WN>
struct Tile {
  static constexpr int kWavesM = BM / WM;
  static constexpr int kWavesN = BN / WN;
  static constexpr int kThreads = kWavesM * kWavesN * kWave;
  static constexpr int TM = WM / 32;  // 32x32 MFMA blocks per wave (rows)
  static constexpr int TN = WN / 32;
  static_assert(BK % 8 == 0, "BK must be a multiple of 8");
  static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile must be 32-aligned");
};

// LDS row strides (floats).  K-contiguous tiles are stored [rows][BK+4]:
// the +4 shifts consecutive rows by 4 banks so the 16-byte fragment reads of
// 8 consecutive rows hit distinct banks.  MN-contiguous tiles are stored
// [BK][rows+4].
template <int ROWS, int BK, bool KC>
struct LdsTile {
  static constexpr int kStride = KC ? (BK + 4) : (ROWS + 4);
  static constexpr int kFloats = KC ? ROWS * (BK + 4) : BK * (ROWS + 4);
};

// Load the ROWS x BK tile of an operand (rows = M or N index) starting at
// (row0, k0) into registers, 4 consecutive floats per slot along the
// contiguous dimension.  Out-of-range elements read as 0.
template <int ROWS, int BK, bool KC, bool VEC, int THREADS>
struct TileLoader {
  static constexpr int kSlots = ROWS * BK / 4;
  static constexpr int kPerThread = (kSlots + THREADS - 1) / THREADS;
  floatx4 v[kPerThread];

  __device__ __forceinline__ void load(const float* __restrict__ p, int ld, int rows, int K,
                                       int row0, int k0, int tid) {
#pragma unroll
    for (int it = 0; it < kPerThread; ++it) {
      const int slot = tid + it * THREADS;
      floatx4 x = {0.f, 0.f, 0.f, 0.f};
      if (slot < kSlots) {
        int r, kk;
        if (KC) {  // slot -> (row, 4 consecutive k)
          r = slot / (BK / 4);
          kk = (slot % (BK / 4)) * 4;
        } else {   // slot -> (k, 4 consecutive rows)
          kk = slot / (ROWS / 4);
          r = (slot % (ROWS / 4)) * 4;
        }
        const int gr = row0 + r, gk = k0 + kk;
        if (KC) {
          if (gr < rows) {
            const float* src = p + (size_t)gr * ld + gk;
            if (VEC) {
              if (gk < K) x = *reinterpret_cast<const floatx4*>(src);
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (gk + e < K) x[e] = src[e];
            }
          }
        } else {
          if (gk < K) {
            const float* src = p + (size_t)gk * ld + gr;
            if (VEC) {
              if (gr < rows) x = *reinterpret_cast<const floatx4*>(src);
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (gr + e < rows) x[e] = src[e];
            }
          }
        }
      }
      v[it] = x;
    }
  }

  __device__ __forceinline__ void store(float* lds, int tid) const {
#pragma unroll
    for (int it = 0; it < kPerThread; ++it) {
      const int slot = tid + it * THREADS;
      if (slot < kSlots) {
        int r, kk;
        if (KC) {
          r = slot / (BK / 4);
          kk = (slot % (BK / 4)) * 4;
          *reinterpret_cast<floatx4*>(lds + r * LdsTile<ROWS, BK, KC>::kStride + kk) = v[it];
        } else {
          kk = slot / (ROWS / 4);
          r = (slot % (ROWS / 4)) * 4;
          *reinterpret_cast<floatx4*>(lds + kk * LdsTile<ROWS, BK, KC>::kStride + r) = v[it];
        }
      }
    }
  }
};

// f(I, J) for the blocks (I, J) of a TM x TN grid in row order, with I and
// J as std::integral_constant (compile-time indices).
template <int B, int TM, int TN, class F>
__device__ __forceinline__ void static_for_blocks(F&& f) {
  if constexpr (B < TM * TN) {
    f(std::integral_constant<int, B / TN>{}, std::integral_constant<int, B % TN>{});
    static_for_blocks<B + 1, TM, TN>(f);
  }
}

// The 4 operands (k = 8g + 4h + s, s = 0..3) of lane (row, h) for k-group g.
template <int ROWS, int BK, bool KC>
__device__ __forceinline__ floatx4 load_frag(const float* lds, int row, int h, int g) {
  constexpr int S = LdsTile<ROWS, BK, KC>::kStride;
  if (KC) {
    return *reinterpret_cast<const floatx4*>(lds + row * S + 8 * g + 4 * h);
  } else {
    floatx4 f;
#pragma unroll
    for (int s = 0; s < 4; ++s) f[s] = lds[(8 * g + 4 * h + s) * S + row];
    return f;
  }
}

// ---------------------------------------------------------------------------
// Element epilogues (called once per output element m < M, n < N).
// ---------------------------------------------------------------------------
template <int EPI>
__device__ __forceinline__ void apply_epilogue(const EpiArgs& e, int m, int n, float acc, AdamRcp rc = {}) {
  const size_t idx = (size_t)m * e.ldc + n;
  switch (EPI) {
    case EPI_STORE:
      e.out[idx] = acc;
      break;
    case EPI_BIAS_ACT: {
      // pre = act_i W_i + b_i (:716-724), act_{i+1} = f(pre) (:725-743)
      const float v = acc + e.bias[n];
      if (e.pre) e.pre[idx] = v;
      e.out[idx] = act_forward(e.act, v);
      break;
    }
    case EPI_DX_ACT: {
      // delta_{i-1} = (delta_i W_i^T) * f'(layer i-1)  (:893-929)
      const float y = e.aux_act[idx];
      const float p = e.aux_pre ? e.aux_pre[idx] : y;
      e.out[idx] = acc * act_derivative(e.act, p, y);
      break;
    }
    case EPI_DW_OPT: {
      if (e.grad) e.grad[idx] = acc;
      const float lr = e.scalars->lr;
      if (e.opt == VOLTA_OPT_SGD) {
        // sgd_fused_tn: W = 1*W + (-lr) * (act_i^T delta_i)  (:321-324)
        const float nlr = -lr;
        e.out[idx] = e.out[idx] + nlr * acc;
      } else if (e.opt == VOLTA_OPT_ADAGRAD) {
        adagrad_elem(e.out + idx, e.m + idx, acc, lr, e.eps);
      } else {
        const bool tail = (int64_t)idx >= e.count - e.count % 8;
        adam_elem(e.out + idx, e.m + idx, e.v + idx, acc, tail, lr, rc, e.b1,
                  e.b2, e.eps, e.wd);
      }
      break;
    }
    default:
      break;
  }
}

// Optimizer state of the 16 elements of W_i a lane updates in the dW
// epilogue (column n, rows m_base + 8*(v/4) + (v%4)), split into its loads
// and the update + stores, so a kernel can issue the loads early and let
// their latency run under the product.  32-bit element offsets (W_i has
// fewer than 2^30 elements, checked at launch): one offset register per
// element serves W, m and v alike.
struct DwState {
  float w[16], s1[16], s2[16];

  // Registers v_lo <= v < v_hi only (the others are neither loaded nor stored).
  __device__ __forceinline__ void load(const EpiArgs& e, int m_base, int n, int M, int N, int v_lo, int v_hi) {
    const uint32_t n32 = (uint32_t)n, ldc = (uint32_t)e.ldc;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int m = m_base + 8 * (v >> 2) + (v & 3);
      const uint32_t o = (uint32_t)m * ldc + n32;
      const bool ok = m < M && n < N && v >= v_lo && v < v_hi;
      w[v] = ok ? e.out[o] : 0.0f;
      s1[v] = ok && e.opt != VOLTA_OPT_SGD ? e.m[o] : 0.0f;
      s2[v] = ok && (e.opt == VOLTA_OPT_ADAM || e.opt == VOLTA_OPT_ADAMW) ? e.v[o] : 0.0f;
    }
  }

  // Caller guarantees n < N.
  __device__ __forceinline__ void update_store(const EpiArgs& e, const floatx16& acc, int m_base, int n, int M,
                                               int v_lo, int v_hi) {
    const float lr = e.scalars->lr;
    const uint32_t n32 = (uint32_t)n, ldc = (uint32_t)e.ldc;
    auto row = [&](int v) { return m_base + 8 * (v >> 2) + (v & 3); };
    auto off = [&](int v) { return (uint32_t)row(v) * ldc + n32; };
    if (e.opt == VOLTA_OPT_SGD) {
      // sgd_fused_tn: W = 1*W + (-lr) * (act_i^T delta_i)  (:321-324)
      const float nlr = -lr;
#pragma unroll
      for (int v = 0; v < 16; ++v) w[v] = w[v] + nlr * acc[v];
    } else if (e.opt == VOLTA_OPT_ADAGRAD) {
#pragma unroll
      for (int v = 0; v < 16; ++v) adagrad_elem(&w[v], &s1[v], acc[v], lr, e.eps);
    } else {
      const AdamRcp rc = adam_rcp(e.scalars->bc1, e.scalars->bc2);
      const uint32_t vec_end = (uint32_t)(e.count - e.count % 8);
#pragma unroll
      for (int v = 0; v < 16; ++v)
        adam_elem(&w[v], &s1[v], &s2[v], acc[v], off(v) >= vec_end, lr, rc, e.b1, e.b2, e.eps, e.wd);
    }
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      if (row(v) < M && v >= v_lo && v < v_hi) {
        e.out[off(v)] = w[v];
        if (e.opt != VOLTA_OPT_SGD) e.m[off(v)] = s1[v];
        if (e.opt == VOLTA_OPT_ADAM || e.opt == VOLTA_OPT_ADAMW) e.v[off(v)] = s2[v];
        if (e.grad) e.grad[off(v)] = acc[v];
      }
    }
  }
};

// Epilogue for the 16 accumulators a lane holds of one 32x32 block: column n,
// rows m_base + 8*(v/4) + (v%4), registers v_lo <= v < v_hi of them.  All
// loads are issued before any store so the memory accesses of the elements
// overlap (the element-by-element form serialises them, since the compiler
// cannot prove the buffers disjoint).
template <int EPI>
__device__ __forceinline__ void block_epilogue(const EpiArgs& e, const floatx16& acc, int m_base, int n, int M,
                                               int N, int v_lo = 0, int v_hi = 16) {
  if (n >= N) return;
  auto row = [&](int v) { return m_base + 8 * (v >> 2) + (v & 3); };
  auto mine = [&](int v) { return v >= v_lo && v < v_hi; };
  if constexpr (EPI == EPI_BIAS_ACT) {
    const float b = e.bias[n];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int m = row(v);
      if (m < M && mine(v)) {
        const size_t idx = (size_t)m * e.ldc + n;
        const float x = acc[v] + b;  // pre = act_i W_i + b_i (:716-724)
        if (e.pre) e.pre[idx] = x;
        e.out[idx] = act_forward(e.act, x);  // act_{i+1} = f(pre) (:725-743)
      }
    }
  } else if constexpr (EPI == EPI_DX_ACT) {
    // delta_{i-1} = (delta_i W_i^T) * f'(layer i-1)  (:893-929)
    const float* pp = e.aux_pre ? e.aux_pre : e.aux_act;
    float y[16], p[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int m = row(v);
      const size_t idx = (size_t)m * e.ldc + n;
      y[v] = m < M && mine(v) ? e.aux_act[idx] : 0.0f;
      p[v] = m < M && mine(v) ? pp[idx] : 0.0f;
    }
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int m = row(v);
      if (m < M && mine(v)) e.out[(size_t)m * e.ldc + n] = acc[v] * act_derivative(e.act, p[v], y[v]);
    }
  } else if constexpr (EPI == EPI_DW_OPT) {
    DwState st;
    st.load(e, m_base, n, M, N, v_lo, v_hi);
    st.update_store(e, acc, m_base, n, M, v_lo, v_hi);
  } else {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int m = row(v);
      if (m < M && mine(v)) e.out[(size_t)m * e.ldc + n] = acc[v];
    }
  }
}

// Four consecutive floats: one 16-byte access when V4 (the caller checked
// the alignment), else four 4-byte ones.
template <bool V4>
__device__ __forceinline__ floatx4 load4(const float* p) {
  if constexpr (V4) return *reinterpret_cast<const floatx4*>(p);
  else return floatx4{p[0], p[1], p[2], p[3]};
}
template <bool V4>
__device__ __forceinline__ void store4(float* p, const floatx4& x) {
  if constexpr (V4) {
    *reinterpret_cast<floatx4*>(p) = x;
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) p[q] = x[q];
  }
}

// Epilogue of four 32x32 blocks j = 0..3 whose columns interleave: block j's
// column of the lane is n4 + j, so the lane holds four consecutive columns of
// each of its 16 rows m_base + RS*(8*(v/4) + (v%4)) (the 256x256 tile with an
// MN-contiguous B operand, RS = 2 where the A operand's rows interleave too;
// exact tiles, every row and column in range).  Rows go four at a time,
// every load of a group issued before its stores, with 16-byte accesses
// when V4 -- the same per-element arithmetic as block_epilogue.
template <int EPI, bool V4, int RS>
__device__ __forceinline__ void quad_epilogue(const EpiArgs& e, const floatx16& a0, const floatx16& a1,
                                              const floatx16& a2, const floatx16& a3, int m_base, int n4) {
  static_assert(EPI == EPI_STORE || EPI == EPI_BIAS_ACT || EPI == EPI_DW_OPT, "no interleaved form");
  const uint32_t ldc = (uint32_t)e.ldc;
  auto off = [&](int v) { return (uint32_t)(m_base + RS * (8 * (v >> 2) + (v & 3))) * ldc + (uint32_t)n4; };
  auto val = [&](int v) { return floatx4{a0[v], a1[v], a2[v], a3[v]}; };
  if constexpr (EPI == EPI_STORE) {
#pragma unroll
    for (int v = 0; v < 16; ++v) store4<V4>(e.out + off(v), val(v));
  } else if constexpr (EPI == EPI_BIAS_ACT) {
    const floatx4 b = load4<V4>(e.bias + n4);
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      floatx4 x = val(v), y;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        x[q] = x[q] + b[q];  // pre = act_i W_i + b_i (:716-724)
        y[q] = act_forward(e.act, x[q]);  // act_{i+1} = f(pre) (:725-743)
      }
      if (e.pre) store4<V4>(e.pre + off(v), x);
      store4<V4>(e.out + off(v), y);
    }
  } else {
    const float lr = e.scalars->lr;
    const bool has1 = e.opt != VOLTA_OPT_SGD, has2 = e.opt == VOLTA_OPT_ADAM || e.opt == VOLTA_OPT_ADAMW;
    const AdamRcp rc = has2 ? adam_rcp(e.scalars->bc1, e.scalars->bc2) : AdamRcp{};
    const uint32_t vec_end = (uint32_t)(e.count - e.count % 8);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      floatx4 w[4], s1[4], s2[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint32_t o = off(4 * r + t);
        w[t] = load4<V4>(e.out + o);
        s1[t] = has1 ? load4<V4>(e.m + o) : floatx4{};
        s2[t] = has2 ? load4<V4>(e.v + o) : floatx4{};
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int v = 4 * r + t;
        const uint32_t o = off(v);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float g = val(v)[q];
          if (e.opt == VOLTA_OPT_SGD) {
            w[t][q] = w[t][q] + (-lr) * g;  // sgd_fused_tn: W = 1*W + (-lr) * (act_i^T delta_i)  (:321-324)
          } else if (e.opt == VOLTA_OPT_ADAGRAD) {
            float a = w[t][q], b = s1[t][q];
            adagrad_elem(&a, &b, g, lr, e.eps);
            w[t][q] = a, s1[t][q] = b;
          } else {
            float a = w[t][q], b = s1[t][q], c = s2[t][q];
            adam_elem(&a, &b, &c, g, o + q >= vec_end, lr, rc, e.b1, e.b2, e.eps, e.wd);
            w[t][q] = a, s1[t][q] = b, s2[t][q] = c;
          }
        }
        store4<V4>(e.out + o, w[t]);
        if (has1) store4<V4>(e.m + o, s1[t]);
        if (has2) store4<V4>(e.v + o, s2[t]);
        if (e.grad) store4<V4>(e.grad + o, val(v));
      }
    }
  }
}

// Whether every buffer the interleaved epilogue (or the four-wide reduce)
// touches takes 16-byte accesses at column multiples of 4.
__host__ __device__ __forceinline__ bool quad_aligned(const EpiArgs& e, int epi) {
  auto a16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  bool ok = e.ldc % 4 == 0 && a16(e.out);
  if (epi == EPI_BIAS_ACT) ok = ok && a16(e.bias) && a16(e.pre);
  if (epi == EPI_DX_ACT) ok = ok && a16(e.aux_act) && a16(e.aux_pre);
  if (epi == EPI_DW_OPT) ok = ok && a16(e.m) && a16(e.v) && a16(e.grad);
  return ok;
}

// Adam's bias-correction reciprocals when the epilogue runs Adam/AdamW.
__device__ __forceinline__ AdamRcp adam_rcp_of(const EpiArgs& e) {
  return e.opt == VOLTA_OPT_ADAM || e.opt == VOLTA_OPT_ADAMW ? adam_rcp(e.scalars->bc1, e.scalars->bc2) : AdamRcp{};
}

// b_i[n] and its optimizer state, loaded ahead of the update (same
// arithmetic as apply_bias_update below).
struct BiasState {
  float b = 0.0f, m = 0.0f, v = 0.0f;

  __device__ __forceinline__ void load(const EpiArgs& e, int n) {
    b = e.b[n];
    if (e.opt != VOLTA_OPT_SGD) m = e.bm[n];
    if (e.opt == VOLTA_OPT_ADAM || e.opt == VOLTA_OPT_ADAMW) v = e.bv[n];
  }

  __device__ __forceinline__ void update_store(const EpiArgs& e, int n, int N, float db, AdamRcp rc) {
    if (e.bgrad) e.bgrad[n] = db;
    const float lr = e.scalars->lr;
    if (e.opt == VOLTA_OPT_SGD) {
      e.b[n] = b - lr * db;  // b -= lr*db (:986-991)
    } else if (e.opt == VOLTA_OPT_ADAGRAD) {
      adagrad_elem(&b, &m, db, lr, e.eps);
      e.b[n] = b;
      e.bm[n] = m;
    } else {
      adam_elem(&b, &m, &v, db, n >= N - N % 8, lr, rc, e.b1, e.b2, e.eps, 0.0f);
      e.b[n] = b;
      e.bm[n] = m;
      e.bv[n] = v;
    }
  }
};

// Bias update from the fused column sum db_i[n] (:931-933, :957-993).  The
// generated step never decays biases (:966).
__device__ __forceinline__ void apply_bias_update(const EpiArgs& e, int n, int N, float db, AdamRcp rc) {
  if (e.bgrad) e.bgrad[n] = db;
  const float lr = e.scalars->lr;
  if (e.opt == VOLTA_OPT_SGD) {
    e.b[n] = e.b[n] - lr * db;  // b -= lr*db (:986-991)
  } else if (e.opt == VOLTA_OPT_ADAGRAD) {
    adagrad_elem(e.b + n, e.bm + n, db, lr, e.eps);
  } else {
    const bool tail = n >= N - N % 8;
    adam_elem(e.b + n, e.bm + n, e.bv + n, db, tail, lr, rc, e.b1, e.b2, e.eps,
              0.0f);
  }
}

// Output layer + loss head on a staged tile (z[mm][nn] = acc + bias, one
// thread per row).  MSE (:792-798): d = z - y, loss += d^2, delta = 2d/nt.
// Softmax-CE (interpreter.rs:762-812, autograd.rs:467-534): row max,
// sum exp(z - max), lse, sample loss -(z_label - lse), delta = (p - onehot)/B.
// Returns the row's loss contribution; raises BAD_ARGUMENT for a label
// outside [0, N) (it is never used as an index).
__device__ __forceinline__ float loss_row(const EpiArgs& e, const float* z, int m, int N, int M) {
  float* out = e.out + (size_t)m * N;
  float* d = e.delta + (size_t)m * N;
  for (int j = 0; j < N; ++j) out[j] = z[j];
  if (e.loss == VOLTA_LOSS_MSE) {
    const float nt = (float)(M * N);
    const float* y = e.y + (size_t)m * N;
    float acc = 0.0f;
    for (int j = 0; j < N; ++j) {
      const float dj = z[j] - y[j];
      acc = acc + dj * dj;
      d[j] = 2.0f * dj / nt;
    }
    return acc;
  }
  const float bf = (float)M;
  const int lab = e.labels[m];
  float mx = -INFINITY;
  for (int j = 0; j < N; ++j) mx = fmaxf(mx, z[j]);
  float sum = 0.0f;
  for (int j = 0; j < N; ++j) sum = sum + expf(z[j] - mx);
  const float lse = mx + logf(sum);
  float sample = __builtin_nanf("");
  for (int j = 0; j < N; ++j) {
    const bool on = j == lab;
    if (on) sample = -(z[j] - lse);
    d[j] = (expf(z[j] - mx) / sum - (on ? 1.0f : 0.0f)) / bf;
  }
  if (lab < 0 || lab >= N) atomicOr(&e.scalars->flags, (uint32_t)VOLTA_STATUS_BAD_ARGUMENT);
  return sample;
}

// Loss head for one output-layer tile staged in LDS (z[mm*ZS + nn] =
// acc + bias, rows m0.. of the batch).  One thread per row; the tile's sum
// goes to loss_partials[tm]; with one tile it is the total, otherwise the
// last tile to finish adds the partials in tile order.
template <int BM>
__device__ __forceinline__ void loss_tile(const EpiArgs& e, const float* z, int ZS, int m0, int tm, int M, int N,
                                          float* lds_rows) {
  const int tid = threadIdx.x;
  if (tid < BM) lds_rows[tid] = m0 + tid < M ? loss_row(e, z + tid * ZS, m0 + tid, N, M) : 0.0f;
  __syncthreads();
  if (tid == 0) {
    float s = 0.0f;
    for (int r = 0; r < BM && m0 + r < M; ++r) s = s + lds_rows[r];
    const float denom = e.loss == VOLTA_LOSS_MSE ? (float)(M * N) : (float)M;
    if (e.loss_tiles == 1) {
      step_epilogue(e.scalars, e.bc_table, e.bc_len, s / denom);
    } else {
      e.loss_partials[tm] = s;
      __threadfence();
      const unsigned ticket = atomicAdd(e.loss_counter, 1u);
      if (ticket == (unsigned)e.loss_tiles - 1u) {
        __threadfence();
        float total = 0.0f;
        for (int t = 0; t < e.loss_tiles; ++t) total = total + e.loss_partials[t];
        step_epilogue(e.scalars, e.bc_table, e.bc_len, total / denom);
        *e.loss_counter = 0u;
      }
    }
  }
}

// Split-K planes whose loads the last slice of a tile issues together.
constexpr int kInkPlanes = 4;

// EPI is the epilogue kind (compile time, so each launch carries only its
// own epilogue).  INK selects how a split-K launch is reduced: false -- each
// slice stores its partial plane and splitk_reduce finishes in a second
// kernel; true -- the last slice to arrive (integer ticket) reduces.
//
// The tile body is a device function of the block coordinates (bx = output
// tile, by = K slice of gy) and of its LDS (two A buffers, two B buffers,
// BM + 2 floats), so a launch may also run it beside another operation.
//
// KG > 1 splits K inside the workgroup instead (gy = 1): KG groups of the
// tile's waves, group z taking K slice z (k_per_split each) with its own two
// A and two B buffers (lds_a0: KG x 2 A buffers, lds_b0 right after it: KG x
// 2 B buffers).  Every group runs as many stages as group 0, computing only
// inside its slice, so the workgroup barriers match.  The partial tiles are
// then added through the (free) operand LDS in slice order -- the sum
// splitk_reduce forms over KG planes -- each group finishing 16/KG of every
// block's 16 accumulator rows, and the epilogue runs on those rows.
template <int BM, int BN, int BK, int WM, int WN, bool A_KC, bool B_KC, bool VEC, int EPI, bool INK, int KG = 1>
__device__ __forceinline__ void gemm_tile(const GemmArgs& args, int bx, int by, int gy, float* lds_a0,
                                          float* lds_b0, float* lds_small) {
  using T = Tile<BM, BN, BK, WM, WN>;
  constexpr int THREADS = T::kThreads;
  using LA = LdsTile<BM, BK, A_KC>;
  using LB = LdsTile<BN, BK, B_KC>;
  static_assert(KG == 1 || (EPI != EPI_LOSS && !INK), "K groups finish whole tiles in their own epilogue");
  const int grp = KG > 1 ? (int)threadIdx.x / THREADS : 0;  // workgroup-uniform per wave
  float* const lds_x = lds_a0;  // the K groups' exchange area (all operand buffers)
  auto lds_a = [&](int i) { return lds_a0 + (grp * 2 + i) * LA::kFloats; };
  auto lds_b = [&](int i) { return lds_b0 + (grp * 2 + i) * LB::kFloats; };

  const int tid = KG > 1 ? (int)threadIdx.x % THREADS : (int)threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / T::kWavesN;
  const int wn = wave % T::kWavesN;
  const int h = lane >> 5;
  const int l32 = lane & 31;
  const int M = args.M, N = args.N;

  // Tile coordinates.  bx walks N fastest so neighbouring
  // workgroups share the same A rows.
  const int tiles_n = (N + BN - 1) / BN;
  const int tm = bx / tiles_n;
  const int tn = bx % tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;

  const int kbeg = (KG > 1 ? grp : by) * args.k_per_split;
  const int kend = min(args.K, kbeg + args.k_per_split);
  // Stages: a K group runs as many as group 0 (whose slice is the longest).
  const int n_stages = KG > 1 ? (min(args.K, args.k_per_split) + BK - 1) / BK : (kend - kbeg + BK - 1) / BK;
  // Column sums of B over k (dW's db = sum_b delta), taken from the MFMA B
  // fragments the waves already hold: the first row of waves (wm == 0) of
  // the first row of tiles adds its fragments in k order per lane half,
  // then the two halves are added.  Fixed order, no extra LDS traffic.
  constexpr bool kColsum = EPI == EPI_DW_OPT && !B_KC;
  const bool colsum = kColsum && args.colsum_b && tm == 0 && wm == 0;
  float cs[T::TN];
#pragma unroll
  for (int j = 0; j < T::TN; ++j) cs[j] = 0.0f;

  TileLoader<BM, BK, A_KC, VEC, THREADS> la;
  TileLoader<BN, BK, B_KC, VEC, THREADS> lb;

  floatx16 acc[T::TM][T::TN];
#pragma unroll
  for (int i = 0; i < T::TM; ++i)
#pragma unroll
    for (int j = 0; j < T::TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // MFMAs of one BK-deep stage held in LDS.  Fragments are double-buffered
  // in registers: those of group g + 1 are read from LDS before the MFMAs of
  // group g are issued, so the LDS latency hides behind the matrix work.
  auto compute_stage = [&](const float* a_s, const float* b_s, auto&& mid) {
    floatx4 fa_n[T::TM], fb_n[T::TN];
#pragma unroll
    for (int i = 0; i < T::TM; ++i) fa_n[i] = load_frag<BM, BK, A_KC>(a_s, wm * WM + i * 32 + l32, h, 0);
#pragma unroll
    for (int j = 0; j < T::TN; ++j) fb_n[j] = load_frag<BN, BK, B_KC>(b_s, wn * WN + j * 32 + l32, h, 0);
#pragma unroll
    for (int g = 0; g < BK / 8; ++g) {
      floatx4 fa[T::TM], fb[T::TN];
#pragma unroll
      for (int i = 0; i < T::TM; ++i) fa[i] = fa_n[i];
#pragma unroll
      for (int j = 0; j < T::TN; ++j) fb[j] = fb_n[j];
      if (g + 1 < BK / 8) {
#pragma unroll
        for (int i = 0; i < T::TM; ++i)
          fa_n[i] = load_frag<BM, BK, A_KC>(a_s, wm * WM + i * 32 + l32, h, g + 1);
#pragma unroll
        for (int j = 0; j < T::TN; ++j)
          fb_n[j] = load_frag<BN, BK, B_KC>(b_s, wn * WN + j * 32 + l32, h, g + 1);
      }
      // keep the scheduler from sinking those reads below the MFMAs
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < T::TM; ++i)
#pragma unroll
          for (int j = 0; j < T::TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i][s], fb[j][s], acc[i][j], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      if (g == BK / 16 - 1) {
        mid();
        __builtin_amdgcn_sched_barrier(0);
      }
      if (kColsum && colsum) {
        // rows beyond kend were loaded as zeros; adding them changes nothing
#pragma unroll
        for (int j = 0; j < T::TN; ++j)
#pragma unroll
          for (int s = 0; s < 4; ++s) cs[j] = cs[j] + fb[j][s];
      }
    }
  };

  if (n_stages > 0) {
    if (kbeg < kend) {
      la.load(args.A, args.lda, M, kend, m0, kbeg, tid);
      lb.load(args.B, args.ldb, N, kend, n0, kbeg, tid);
      la.store(lds_a(0), tid);
      lb.store(lds_b(0), tid);
    }
    __syncthreads();

    int buf = 0;
    for (int st = 0; st < n_stages; ++st) {
      const int k0 = kbeg + st * BK;
      const bool active = KG == 1 || k0 < kend;  // a K group past its slice only meets the barriers
      const bool more = k0 + BK < kend;
      if (more) {
        la.load(args.A, args.lda, M, kend, m0, k0 + BK, tid);
        lb.load(args.B, args.ldb, N, kend, n0, k0 + BK, tid);
      }
      if (active) {
        __builtin_amdgcn_s_setprio(1);
        compute_stage(lds_a(buf), lds_b(buf), [] {});
        __builtin_amdgcn_s_setprio(0);
      }
      if (more) {
        la.store(lds_a(buf ^ 1), tid);
        lb.store(lds_b(buf ^ 1), tid);
      }
      __syncthreads();
      buf ^= 1;
    }
  }

  // Column sums: add the two lane halves (same value in both lanes); lanes
  // of half 0 own column n0 + wn*WN + j*32 + l32.
  if (kColsum && colsum) {
#pragma unroll
    for (int j = 0; j < T::TN; ++j) cs[j] = cs[j] + __shfl_xor(cs[j], 32, kWave);
  }
  const bool cs_owner = kColsum && colsum && h == 0 && grp == 0;

  // Accumulator rows (registers v) this group finishes.
  const int v_lo = grp * 16 / KG, v_hi = (grp + 1) * 16 / KG;
  if constexpr (KG > 1) {
    // Slot of (group z, this wave, block (i, j), register v): lane-minor, so
    // a wave's 64 lanes write and read 256 consecutive bytes.
    constexpr int kBlocks = T::TM * T::TN;
    constexpr int kWavesG = THREADS / kWave;
    static_assert(KG * (BM * BN + BN) <= 2 * KG * (LA::kFloats + LB::kFloats), "exchange does not fit");
    auto slot = [&](int z, int b, int v) { return lds_x + (((z * kWavesG + wave) * kBlocks + b) * 16 + v) * kWave + lane; };
    float* const cs_x = lds_x + KG * BM * BN;  // column sums of group z: cs_x[z * BN + column]
#pragma unroll
    for (int b = 0; b < kBlocks; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v)
        if (v < v_lo || v >= v_hi) *slot(grp, b, v) = acc[b / T::TN][b % T::TN][v];
    if (kColsum && colsum && h == 0 && grp > 0) {
#pragma unroll
      for (int j = 0; j < T::TN; ++j) cs_x[grp * BN + wn * WN + j * 32 + l32] = cs[j];
    }
    __syncthreads();
#pragma unroll
    for (int b = 0; b < kBlocks; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v)
        if (v >= v_lo && v < v_hi) {
          const float own = acc[b / T::TN][b % T::TN][v];
          float sum = grp == 0 ? own : *slot(0, b, v);
#pragma unroll
          for (int z = 1; z < KG; ++z) sum = sum + (z == grp ? own : *slot(z, b, v));
          acc[b / T::TN][b % T::TN][v] = sum;
        }
    if (cs_owner) {
#pragma unroll
      for (int j = 0; j < T::TN; ++j)
#pragma unroll
        for (int z = 1; z < KG; ++z) cs[j] = cs[j] + cs_x[z * BN + wn * WN + j * 32 + l32];
    }
  }

  // Accumulator register v of lane (h, l32) in block (i, j) holds row
  // 8*(v/4) + 4*h + (v%4), column l32 of that 32x32 block.
  if (gy > 1) {
    // Split-K: publish this slice's partial tile (row M of each plane holds
    // the column sums).
    const size_t plane = (size_t)(M + 1) * N;
    float* mine = args.partial + (size_t)by * plane;
#pragma unroll
    for (int i = 0; i < T::TM; ++i)
#pragma unroll
      for (int j = 0; j < T::TN; ++j) {
        const int n = n0 + wn * WN + j * 32 + l32;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int m = m0 + wm * WM + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
          if (m < M && n < N) mine[(size_t)m * N + n] = acc[i][j][v];
        }
      }
    if (cs_owner) {
#pragma unroll
      for (int j = 0; j < T::TN; ++j) {
        const int n = n0 + wn * WN + j * 32 + l32;
        if (n < N) mine[(size_t)M * N + n] = cs[j];
      }
    }
    if constexpr (!INK) {
      return;  // splitk_reduce finishes
    } else {
      // Release this slice's plane and take the tile's ticket; the slice
      // that arrives last adds the planes in slice order -- its own from
      // its registers -- exactly as splitk_reduce adds them, then runs the
      // epilogue.  Per 32x32 block every plane's loads are issued before
      // the first add (kInkPlanes at a time), so the reduction waits one
      // memory latency per block and chunk rather than one per register.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
      __syncthreads();
      if (tid == 0) {
        const unsigned ticket = __hip_atomic_fetch_add(&args.counters[bx], 1u, __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT);
        lds_small[BM] = ticket == (unsigned)gy - 1u ? 1.0f : 0.0f;
      }
      __syncthreads();
      if (lds_small[BM] == 0.0f) return;
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      const float* planes = args.partial;
      static_for_blocks<0, T::TM, T::TN>([&](auto I, auto J) {
        constexpr int i = decltype(I)::value, j = decltype(J)::value;
        const int n = n0 + wn * WN + j * 32 + l32;
        const int nc = n < N ? n : N - 1;  // clamped: every load in bounds, unused values discarded
        float s[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) s[v] = 0.0f;
        for (int z0 = 0; z0 < gy; z0 += kInkPlanes) {
          float p[kInkPlanes][16];
#pragma unroll
          for (int q = 0; q < kInkPlanes; ++q) {
            const int z = z0 + q < gy ? z0 + q : gy - 1;
            const float* src = planes + (size_t)z * plane + nc;
            if (z != by) {
#pragma unroll
              for (int v = 0; v < 16; ++v) {
                const int m = m0 + wm * WM + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                p[q][v] = src[(size_t)(m < M ? m : M - 1) * N];
              }
            } else {
#pragma unroll
              for (int v = 0; v < 16; ++v) p[q][v] = acc[i][j][v];
            }
          }
#pragma unroll
          for (int q = 0; q < kInkPlanes; ++q) {
            const int z = z0 + q;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
              const float t = z == 0 ? p[q][v] : s[v] + p[q][v];
              s[v] = z < gy ? t : s[v];
            }
          }
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = s[v];
        __builtin_amdgcn_sched_barrier(0);
      });
      if (cs_owner) {
#pragma unroll
        for (int j = 0; j < T::TN; ++j) {
          const int n = n0 + wn * WN + j * 32 + l32;
          const float* src = planes + (size_t)M * N + (n < N ? n : N - 1);
          float s = by == 0 ? cs[j] : src[0];
          for (int z = 1; z < gy; ++z) s = s + (z == by ? cs[j] : src[(size_t)z * plane]);
          cs[j] = s;
        }
      }
      if (tid == 0) args.counters[bx] = 0u;
    }
  }

  const EpiArgs& e = args.epi;
  if constexpr (EPI == EPI_LOSS) {
    // Output layer (N <= BN): stage z = acc + bias for the whole tile in the
    // (now free) A buffers, then the per-row loss head.
    static_assert(BM * (BN + 1) <= 2 * LA::kFloats, "loss staging does not fit");
    float* z = lds_a(0);
    constexpr int ZS = BN + 1;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < T::TM; ++i)
#pragma unroll
      for (int j = 0; j < T::TN; ++j) {
        const int nn = wn * WN + j * 32 + l32;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int mm = wm * WM + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
          if (nn < N) z[mm * ZS + nn] = acc[i][j][v] + e.bias[nn];
        }
      }
    __syncthreads();
    loss_tile<BM>(e, z, ZS, m0, tm, M, N, lds_small);
  } else {
    // Blocks in (i, j) order, unrolled at compile time: a loop the unroller
    // gives up on (it did for 4x4 blocks of 32x32) would index the
    // accumulators at run time and put them in scratch memory.
    static_for_blocks<0, T::TM, T::TN>([&](auto I, auto J) {
      constexpr int i = decltype(I)::value, j = decltype(J)::value;
      block_epilogue<EPI>(e, acc[i][j], m0 + wm * WM + i * 32 + 4 * h, n0 + wn * WN + j * 32 + l32, M, N, v_lo,
                          v_hi);
      // one block's loads at a time: hoisting the next block's loads
      // above these stores would raise the register count (occupancy)
      // of the whole kernel
      __builtin_amdgcn_sched_barrier(0);
    });
    if constexpr (kColsum) {
      if (cs_owner && e.b) {
        const AdamRcp rc = adam_rcp_of(e);
#pragma unroll
        for (int j = 0; j < T::TN; ++j) {
          const int n = n0 + wn * WN + j * 32 + l32;
          if (n < N) apply_bias_update(e, n, N, cs[j], rc);
        }
      }
    }
  }
}

// Output tile of workgroup `bx`.  Workgroups are dispatched round-robin
// over the 8 XCDs (workgroup bx runs on XCD bx % 8), and each XCD has its
// own L2.  When the tile grid splits into 8 equal rectangles, XCD x takes
// rectangle x in row order, so an XCD's workgroups share the A row panels
// and B column panels of one sub-grid instead of every XCD streaming all of
// A (the identity order puts tiles tn, tn + 8, ... of every row on one XCD).
// The rectangle shape is the one closest to square in tiles.
__device__ __forceinline__ int xcd_tile(int bx, int tiles_m, int tiles_n) {
  const int tiles = tiles_m * tiles_n;
  if (tiles < 64 || (tiles & 7)) return bx;
  int rm = 0, best = 1 << 30;
  for (int c = 1; c <= 8; c *= 2) {  // rm x (8 / rm) rectangles
    const int cn = 8 / c;
    if (tiles_m % c || tiles_n % cn) continue;
    const int hm = tiles_m / c, hn = tiles_n / cn;
    const int d = hm > hn ? hm - hn : hn - hm;
    if (d < best) best = d, rm = c;
  }
  if (!rm) return bx;
  const int rn = 8 / rm, hm = tiles_m / rm, hn = tiles_n / rn;
  const int x = bx & 7, j = bx >> 3;
  const int tm = (x / rn) * hm + j / hn, tn = (x % rn) * hn + j % hn;
  return tm * tiles_n + tn;
}

// Two waves per SIMD at least (at most 256 vector + accumulation registers
// a lane): the 128x128 dW tile with an Adam epilogue otherwise settles a
// few registers above that and runs at half occupancy.
template <int BM, int BN, int BK, int WM, int WN, bool A_KC, bool B_KC, bool VEC, int EPI, bool INK>
__global__ void __launch_bounds__((BM / WM) * (BN / WN) * 64) __attribute__((amdgpu_waves_per_eu(2)))
gemm_f32_mfma(GemmArgs args) {
  __shared__ __attribute__((aligned(16))) float lds_a[2 * LdsTile<BM, BK, A_KC>::kFloats];
  __shared__ __attribute__((aligned(16))) float lds_b[2 * LdsTile<BN, BK, B_KC>::kFloats];
  __shared__ float lds_small[BM + 2];
  const int bx = xcd_tile(blockIdx.x, (args.M + BM - 1) / BM, (args.N + BN - 1) / BN);
  gemm_tile<BM, BN, BK, WM, WN, A_KC, B_KC, VEC, EPI, INK>(args, bx, blockIdx.y, gridDim.y, lds_a, lds_b, lds_small);
}

// The tile with K split over KG groups of its waves inside the workgroup
// (gemm_tile with KG): one launch, no partial planes, the same sums as KG
// slices reduced by splitk_reduce.  One workgroup per CU (the operand LDS
// of KG groups), KG waves per SIMD.
template <int BM, int BN, int BK, int WM, int WN, bool A_KC, bool B_KC, bool VEC, int EPI, int KG>
__global__ void __launch_bounds__(KG * (BM / WM) * (BN / WN) * 64) __attribute__((amdgpu_waves_per_eu(2)))
gemm_f32_mfma_kg(GemmArgs args) {
  constexpr int kLa = LdsTile<BM, BK, A_KC>::kFloats, kLb = LdsTile<BN, BK, B_KC>::kFloats;
  __shared__ __attribute__((aligned(16))) float lds[2 * KG * (kLa + kLb)];
  const int bx = xcd_tile(blockIdx.x, (args.M + BM - 1) / BM, (args.N + BN - 1) / BN);
  gemm_tile<BM, BN, BK, WM, WN, A_KC, B_KC, VEC, EPI, false, KG>(args, bx, 0, 1, lds, lds + 2 * KG * kLa, nullptr);
}

// ---------------------------------------------------------------------------
// Large tile for the C5-scale products: 256x256 outputs per workgroup, eight
// waves of 64x128 (a 2x4 grid of 32x32 accumulator blocks each: 128
// accumulation registers), one workgroup -- two waves per SIMD -- per CU.
// Operand tiles (BK = 32 k) go from global memory straight into LDS
// (global_load_lds_dwordx4: no register staging and no LDS stores),
// double-buffered in two distinct LDS arrays: the loads of stage s+1 are
// issued before the MFMAs of stage s, and a wave issues 128 MFMAs per stage
// between its two synchronisations (wait for its own loads, then the
// workgroup barrier).
//
// LDS layouts.  K-contiguous tile [256 rows][32 k] in 16-byte chunks: (row
// r, k-quad q) at chunk r*8 + (q ^ ((r >> 1) & 7)), so the fragment reads of
// 16 consecutive rows at one k-quad hit all 16 four-bank groups of the 64
// banks (rows 2m and 2m+1 lie in opposite halves, m = 0..7 permutes the
// quads); each load instruction fills 64 consecutive chunks: 8 rows, their
// k-quads permuted, from 8 whole 128-byte row segments.  MN-contiguous tile
// [32 k][256]: one k row of 256 floats per load instruction.  An
// MN-contiguous A operand is read as four 4-byte reads per fragment (a
// lane's four k of one row), conflict-free across consecutive rows; an
// MN-contiguous B operand as one 16-byte read per MFMA step (big_bq: four
// consecutive columns of one k, one per accumulator block), 16 lanes
// covering 256 consecutive bytes.
//
// Exact tiles only (M, N multiples of 256, K of 64, 16-byte aligned rows and
// bases): every load is in bounds without a guard; gemm_plan checks.
// ---------------------------------------------------------------------------
constexpr int kBigBM = 256, kBigBK = 32;
constexpr int kBigTileFloats = kBigBM * kBigBK;  // one operand tile of one stage (32 KB)

typedef __attribute__((address_space(3))) void* LdsVoidPtr;

// Issue this wave's 4 of the 32 one-kilobyte load instructions of an operand
// tile (rows row0.., k k0..k0+31) into `tile`; `wave` (0..7) is wave-uniform.
// Instruction j = wave + 8t fills chunks 64j..64j+63: K-contiguous, rows
// 8j..8j+7 (lane: row 8j + lane/8, k-quad (lane & 7) ^ ((row >> 1) & 7));
// MN-contiguous, k row j.  32-bit element offsets (big_tile_fits bounds the
// operands).
template <bool KC>
__device__ __forceinline__ void big_load(const float* __restrict__ p, int ld, int row0, int k0, float* tile,
                                         int wave, int lane) {
  uint32_t off, step;
  if constexpr (KC) {
    const int r = wave * 8 + (lane >> 3);
    const int q = (lane & 7) ^ ((r >> 1) & 7);  // rows 64t apart share the swizzle
    off = (uint32_t)(row0 + r) * (uint32_t)ld + (uint32_t)(k0 + 4 * q);
    step = 64u * (uint32_t)ld;
  } else {
    off = (uint32_t)(k0 + wave) * (uint32_t)ld + (uint32_t)(row0 + 4 * lane);
    step = 8u * (uint32_t)ld;
  }
#pragma unroll
  for (int t = 0; t < 4; ++t)
    __builtin_amdgcn_global_load_lds((const void*)(p + off + t * step), (LdsVoidPtr)(tile + (wave + 8 * t) * 256), 16,
                                     0, 0);
}

// The 4 operands (k = 8g + 4h + s) of lane (row, h) for k-group g.  (For an
// MN-contiguous B operand the tile reads big_bq instead.)
template <bool KC>
__device__ __forceinline__ floatx4 big_frag(const float* tile, int row, int h, int g) {
  if constexpr (KC) {
    const int q = 2 * g + h;
    return *reinterpret_cast<const floatx4*>(tile + 4 * (row * 8 + (q ^ ((row >> 1) & 7))));
  } else {
    floatx4 f;
#pragma unroll
    for (int s = 0; s < 4; ++s) f[s] = tile[(8 * g + 4 * h + s) * kBigBM + row];
    return f;
  }
}

// MN-contiguous B operand, one 16-byte read per MFMA step: lane (c, h) takes
// columns 4c..4c+3 of k row 8g + 4h + s, the B operands of its four 32x32
// blocks j = 0..3 at step s -- block j's column of lane c is 4c + j.  The k
// of every product is unchanged (8g + 4h + s), so each output sums the same
// products in the same order as the one-block-per-32-columns mapping.
__device__ __forceinline__ floatx4 big_bq(const float* tile, int col4, int h, int g, int s) {
  return *reinterpret_cast<const floatx4*>(tile + (8 * g + 4 * h + s) * kBigBM + col4);
}

// MN-contiguous A operand likewise, one 8-byte read per MFMA step: lane
// (r, h) takes rows 2r and 2r+1 of k row 8g + 4h + s, the A operands of its
// two 32x32 row blocks i = 0, 1 -- block i's row of lane r is 2r + i.
typedef float floatx2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ floatx2 big_aq(const float* tile, int row2, int h, int g, int s) {
  return *reinterpret_cast<const floatx2*>(tile + (8 * g + 4 * h + s) * kBigBM + row2);
}

template <bool A_KC, bool B_KC, int EPI>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) gemm_big(GemmArgs args) {
  __shared__ __attribute__((aligned(16))) float lds_a0[kBigTileFloats];
  __shared__ __attribute__((aligned(16))) float lds_b0[kBigTileFloats];
  __shared__ __attribute__((aligned(16))) float lds_a1[kBigTileFloats];
  __shared__ __attribute__((aligned(16))) float lds_b1[kBigTileFloats];
  constexpr int TM = 2, TN = 4, WM = 64, WN = 128;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1, h = lane >> 5, l32 = lane & 31;
  const int M = args.M, N = args.N, K = args.K;
  const int tiles_n = N / kBigBM;
  const int bx = xcd_tile(blockIdx.x, M / kBigBM, tiles_n);
  const int tm = bx / tiles_n, tn = bx % tiles_n;
  const int m0 = tm * kBigBM, n0 = tn * kBigBM;

  constexpr bool kColsum = EPI == EPI_DW_OPT && !B_KC;
  const bool colsum = kColsum && args.colsum_b && tm == 0 && wm == 0;
  float cs[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) cs[j] = 0.0f;

  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // Column of block j held by lane l32 (B MN-contiguous: 4 l32 + j, big_bq);
  // first row of block i held by lane half h (A MN-contiguous: rows
  // interleave, block i's MFMA row r is 2r + i, big_aq).
  auto col = [&](int j) { return B_KC ? j * 32 + l32 : 4 * l32 + j; };
  auto row_base = [&](int i) { return m0 + wm * WM + (A_KC ? i * 32 + 4 * h : i + 8 * h); };
  constexpr int kRowStride = A_KC ? 1 : 2;
  static_assert(TM == 2, "the MN-contiguous A reads cover two blocks per step");
  // A fragment t of k-group g: K-contiguous, block t's four steps; MN-
  // contiguous, steps 2t and 2t+1 of both blocks ({s0 i0, s0 i1, s1 i0, s1 i1}).
  auto a_frag = [&](const float* a_s, int t, int g) {
    if constexpr (A_KC) {
      return big_frag<true>(a_s, wm * WM + t * 32 + l32, h, g);
    } else {
      const floatx2 x = big_aq(a_s, wm * WM + 2 * l32, h, g, 2 * t);
      const floatx2 y = big_aq(a_s, wm * WM + 2 * l32, h, g, 2 * t + 1);
      return floatx4{x[0], x[1], y[0], y[1]};
    }
  };
  auto a_op = [&](const floatx4* fa, int i, int s) { return A_KC ? fa[i][s] : fa[s >> 1][2 * (s & 1) + i]; };
  // B fragment t of k-group g: K-contiguous, block t's four steps; MN-
  // contiguous, step t's four blocks.
  auto b_frag = [&](const float* b_s, int t, int g) {
    if constexpr (B_KC) return big_frag<true>(b_s, wn * WN + t * 32 + l32, h, g);
    else return big_bq(b_s, wn * WN + 4 * l32, h, g, t);
  };
  static_assert(TN == 4, "the MN-contiguous B reads cover four blocks per step");

  // One stage: the fragments of k-group g + 1 are read from LDS before the
  // 32 MFMAs of group g are issued, so their latency hides behind the
  // matrix work; the wave's priority is raised while it issues MFMAs.
  auto compute = [&](const float* a_s, const float* b_s) {
    floatx4 fa_n[TM], fb_n[TN];
#pragma unroll
    for (int t = 0; t < TM; ++t) fa_n[t] = a_frag(a_s, t, 0);
#pragma unroll
    for (int t = 0; t < TN; ++t) fb_n[t] = b_frag(b_s, t, 0);
#pragma unroll
    for (int g = 0; g < kBigBK / 8; ++g) {
      floatx4 fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[i] = fa_n[i];
#pragma unroll
      for (int j = 0; j < TN; ++j) fb[j] = fb_n[j];
      if (g + 1 < kBigBK / 8) {
#pragma unroll
        for (int t = 0; t < TM; ++t) fa_n[t] = a_frag(a_s, t, g + 1);
#pragma unroll
        for (int t = 0; t < TN; ++t) fb_n[t] = b_frag(b_s, t, g + 1);
      }
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a_op(fa, i, s), B_KC ? fb[j][s] : fb[s][j], acc[i][j], 0,
                                                             0, 0);
      __builtin_amdgcn_s_setprio(0);
      __builtin_amdgcn_sched_barrier(0);
      if (kColsum && colsum) {
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int s = 0; s < 4; ++s) cs[j] = cs[j] + (B_KC ? fb[j][s] : fb[s][j]);
      }
    }
  };

  // Stage s reads buffer s & 1; the loads of stage s + 1 go to the other
  // buffer, which every wave finished reading before the barrier of stage s.
  // S is even (big_tile_fits: K a multiple of 64), so every pass of the
  // loop runs both stages.
  const int S = K / kBigBK;
  big_load<A_KC>(args.A, args.lda, m0, 0, lds_a0, wave, lane);
  big_load<B_KC>(args.B, args.ldb, n0, 0, lds_b0, wave, lane);
  for (int s = 0; s < S; s += 2) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    big_load<A_KC>(args.A, args.lda, m0, (s + 1) * kBigBK, lds_a1, wave, lane);
    big_load<B_KC>(args.B, args.ldb, n0, (s + 1) * kBigBK, lds_b1, wave, lane);
    __builtin_amdgcn_sched_barrier(0);  // the loads stay ahead of this stage's MFMAs
    compute(lds_a0, lds_b0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (s + 2 < S) {
      big_load<A_KC>(args.A, args.lda, m0, (s + 2) * kBigBK, lds_a0, wave, lane);
      big_load<B_KC>(args.B, args.ldb, n0, (s + 2) * kBigBK, lds_b0, wave, lane);
    }
    __builtin_amdgcn_sched_barrier(0);
    compute(lds_a1, lds_b1);
  }

  if (kColsum && colsum) {
#pragma unroll
    for (int j = 0; j < TN; ++j) cs[j] = cs[j] + __shfl_xor(cs[j], 32, kWave);
  }
  const bool cs_owner = kColsum && colsum && h == 0;
  const EpiArgs& e = args.epi;
  if constexpr (B_KC) {
    static_assert(A_KC, "every layout with a K-contiguous B has a K-contiguous A");
    static_for_blocks<0, TM, TN>([&](auto I, auto J) {
      constexpr int i = decltype(I)::value, j = decltype(J)::value;
      block_epilogue<EPI>(e, acc[i][j], row_base(i), n0 + wn * WN + col(j), M, N);
      __builtin_amdgcn_sched_barrier(0);
    });
  } else {
    // the lane's four blocks of a row hold four consecutive columns
    const bool v4 = quad_aligned(e, EPI);
    const int n4 = n0 + wn * WN + 4 * l32;
    static_for_blocks<0, TM, 1>([&](auto I, auto) {
      constexpr int i = decltype(I)::value;
      if (v4) quad_epilogue<EPI, true, kRowStride>(e, acc[i][0], acc[i][1], acc[i][2], acc[i][3], row_base(i), n4);
      else quad_epilogue<EPI, false, kRowStride>(e, acc[i][0], acc[i][1], acc[i][2], acc[i][3], row_base(i), n4);
      __builtin_amdgcn_sched_barrier(0);
    });
  }
  if constexpr (kColsum) {
    if (cs_owner && e.b) {
      const AdamRcp rc = adam_rcp_of(e);
#pragma unroll
      for (int j = 0; j < TN; ++j) apply_bias_update(e, n0 + wn * WN + col(j), N, cs[j], rc);
    }
  }
}

// ---------------------------------------------------------------------------
// 128x128 direct-to-LDS tile (TILE_BIG128): the 256x256 tile's pipeline for
// products whose 256x256 grid would leave CUs idle while their 128x128 grid
// has a tile per CU (C5's 4096 x 1024 and 1024 x 4096 products: 256 tiles,
// the whole K in each workgroup, no split and no reduce launch).  Eight
// waves (two per SIMD) in a 2 x 4 grid, each a 64x32 sub-tile: two 32x32
// blocks of v_mfma_f32_32x32x2f32.  BK = 64: a stage is 64 KB of operands
// (the 256x256 tile's bytes and load instructions per stage) and 8192 MFMA
// cycles per SIMD between two barriers.  Every sum runs in the 256x256
// tile's k order (k-group g, lane half h, step s: k = 8g + 4h + s), the bias
// column sums too, and the epilogue arithmetic is the same, so both tiles
// give the same bits on the products they both serve.
//
// LDS layouts.  K-contiguous [128 rows][64 k] in 16-byte chunks: (row r,
// k-quad q) at chunk 16r + (q ^ (r & 15)): a row spans the 64 banks once,
// and the fragment reads of 16 consecutive rows at one k-quad hit all 16
// four-bank groups; each load instruction fills 64 consecutive chunks (4
// whole rows, 16 lanes per 256-byte row segment).  MN-contiguous
// [64 k][128]: a load instruction fills two k rows; fragments are read one
// float per MFMA step, 32 lanes on 32 consecutive floats.
//
// Exact tiles only (M, N multiples of 128, K of 128, 16-byte aligned rows
// and bases): every load is in bounds without a guard; gemm_launch checks.
// ---------------------------------------------------------------------------
constexpr int kB2 = 128, kB2K = 64;
constexpr int kB2TileFloats = kB2 * kB2K;  // one operand tile of one stage (32 KB)

// Issue this wave's 4 of the 32 one-kilobyte load instructions of an operand
// tile (rows row0.., k k0..k0+63) into `tile`.  Instruction j = wave + 8t:
// K-contiguous, rows 4j..4j+3 (lane: row 4j + lane/16, k-quad
// (lane & 15) ^ (row & 15)); MN-contiguous, k rows 2j and 2j + 1 (lane: k row
// 2j + lane/32, columns 4(lane & 31)..+3).  32-bit element offsets
// (big128_tile_fits bounds the operands).
template <bool KC>
__device__ __forceinline__ void b128_load(const float* __restrict__ p, int ld, int row0, int k0, float* tile,
                                          int wave, int lane) {
  uint32_t off, step;
  if constexpr (KC) {
    const int r = 4 * wave + (lane >> 4);  // rows 32t apart share the swizzle
    const int q = (lane & 15) ^ (r & 15);
    off = (uint32_t)(row0 + r) * (uint32_t)ld + (uint32_t)(k0 + 4 * q);
    step = 32u * (uint32_t)ld;
  } else {
    off = (uint32_t)(k0 + 2 * wave + (lane >> 5)) * (uint32_t)ld + (uint32_t)(row0 + 4 * (lane & 31));
    step = 16u * (uint32_t)ld;
  }
#pragma unroll
  for (int t = 0; t < 4; ++t)
    __builtin_amdgcn_global_load_lds((const void*)(p + off + t * step), (LdsVoidPtr)(tile + (wave + 8 * t) * 256), 16,
                                     0, 0);
}

// The 4 operands (k = 8g + 4h + s, s = 0..3) of lane (row, h) for k-group g.
template <bool KC>
__device__ __forceinline__ floatx4 b128_frag(const float* tile, int row, int h, int g) {
  if constexpr (KC) {
    const int q = 2 * g + h;
    return *reinterpret_cast<const floatx4*>(tile + 4 * (16 * row + (q ^ (row & 15))));
  } else {
    floatx4 f;
#pragma unroll
    for (int s = 0; s < 4; ++s) f[s] = tile[(8 * g + 4 * h + s) * kB2 + row];
    return f;
  }
}

template <bool A_KC, bool B_KC, int EPI>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) gemm_big128(GemmArgs args) {
  __shared__ __attribute__((aligned(16))) float lds_a0[kB2TileFloats];
  __shared__ __attribute__((aligned(16))) float lds_b0[kB2TileFloats];
  __shared__ __attribute__((aligned(16))) float lds_a1[kB2TileFloats];
  __shared__ __attribute__((aligned(16))) float lds_b1[kB2TileFloats];
  constexpr int TM = 2, WM = 64, WN = 32;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3, h = lane >> 5, l32 = lane & 31;
  const int M = args.M, N = args.N, K = args.K;
  const int tiles_n = N / kB2;
  const int bx = xcd_tile(blockIdx.x, M / kB2, tiles_n);
  const int tm = bx / tiles_n, tn = bx % tiles_n;
  const int m0 = tm * kB2, n0 = tn * kB2;

  constexpr bool kColsum = EPI == EPI_DW_OPT && !B_KC;
  const bool colsum = kColsum && args.colsum_b && tm == 0 && wm == 0;
  float cs = 0.0f;

  floatx16 acc[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[i][v] = 0.0f;

  const int arow = wm * WM + l32, bcol = wn * WN + l32;
  // One stage: the fragments of k-group g + 1 are read from LDS before the
  // 8 MFMAs of group g are issued; the wave's priority is raised while it
  // issues MFMAs.
  auto compute = [&](const float* a_s, const float* b_s) {
    floatx4 fa_n[TM], fb_n;
#pragma unroll
    for (int i = 0; i < TM; ++i) fa_n[i] = b128_frag<A_KC>(a_s, arow + 32 * i, h, 0);
    fb_n = b128_frag<B_KC>(b_s, bcol, h, 0);
#pragma unroll
    for (int g = 0; g < kB2K / 8; ++g) {
      floatx4 fa[TM], fb;
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[i] = fa_n[i];
      fb = fb_n;
      if (g + 1 < kB2K / 8) {
#pragma unroll
        for (int i = 0; i < TM; ++i) fa_n[i] = b128_frag<A_KC>(a_s, arow + 32 * i, h, g + 1);
        fb_n = b128_frag<B_KC>(b_s, bcol, h, g + 1);
      }
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < TM; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i][s], fb[s], acc[i], 0, 0, 0);
      __builtin_amdgcn_s_setprio(0);
      __builtin_amdgcn_sched_barrier(0);
      if (kColsum && colsum) {
#pragma unroll
        for (int s = 0; s < 4; ++s) cs = cs + fb[s];
      }
    }
  };

  // Stage s reads buffer s & 1; the loads of stage s + 1 go to the other
  // buffer, which every wave finished reading before the barrier of stage s.
  // S is even (K a multiple of 128), so every pass of the loop runs both.
  const int S = K / kB2K;
  b128_load<A_KC>(args.A, args.lda, m0, 0, lds_a0, wave, lane);
  b128_load<B_KC>(args.B, args.ldb, n0, 0, lds_b0, wave, lane);
  for (int s = 0; s < S; s += 2) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    b128_load<A_KC>(args.A, args.lda, m0, (s + 1) * kB2K, lds_a1, wave, lane);
    b128_load<B_KC>(args.B, args.ldb, n0, (s + 1) * kB2K, lds_b1, wave, lane);
    __builtin_amdgcn_sched_barrier(0);  // the loads stay ahead of this stage's MFMAs
    compute(lds_a0, lds_b0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (s + 2 < S) {
      b128_load<A_KC>(args.A, args.lda, m0, (s + 2) * kB2K, lds_a0, wave, lane);
      b128_load<B_KC>(args.B, args.ldb, n0, (s + 2) * kB2K, lds_b0, wave, lane);
    }
    __builtin_amdgcn_sched_barrier(0);
    compute(lds_a1, lds_b1);
  }

  if (kColsum && colsum) cs = cs + __shfl_xor(cs, 32, kWave);
  const EpiArgs& e = args.epi;
  static_for_blocks<0, TM, 1>([&](auto I, auto) {
    constexpr int i = decltype(I)::value;
    block_epilogue<EPI>(e, acc[i], m0 + wm * WM + i * 32 + 4 * h, n0 + bcol, M, N);
    __builtin_amdgcn_sched_barrier(0);
  });
  if constexpr (kColsum) {
    if (colsum && h == 0 && e.b) apply_bias_update(e, n0 + bcol, N, cs, adam_rcp_of(e));
  }
}

// Whether the 128x128 direct-to-LDS tile serves a product: exact
// 128-multiples, K a multiple of 128 and at least 1024 (a shorter K keeps
// the 64x64 grid's several workgroups per CU), 16-byte aligned operand rows,
// a 128x128 grid of at least one workgroup per CU whose 256x256 grid has
// fewer.
static bool big128_tile_fits(int layout, int M, int N, int K, bool vec, int num_cus) {
  const char* bt = std::getenv("VOLTA_BIG128");
  if (bt && *bt == '0') return false;
  const size_t a_elems = (size_t)M * K, b_elems = (size_t)N * K;
  return vec && layout >= GEMM_NN && layout <= GEMM_TN && M % kB2 == 0 && N % kB2 == 0 && K % (2 * kB2K) == 0 &&
         K >= 1024 && (M / kB2) * (N / kB2) >= num_cus && (M / kBigBM) * (N / kBigBM) < num_cus &&
         a_elems < ((size_t)1 << 31) && b_elems < ((size_t)1 << 31);
}

// Whether the large tile serves a product: exact 256-multiples, K of 32,
// 16-byte aligned operand rows, a grid of at least one workgroup per CU.
static bool big_tile_fits(int layout, int M, int N, int K, bool vec, int num_cus) {
  const char* bt = std::getenv("VOLTA_BIG_TILE");
  if (bt && *bt == '0') return false;
  // every operand element offset must fit 32 bits (big_load)
  const size_t a_elems = (size_t)M * K, b_elems = (size_t)N * K;
  return vec && layout >= GEMM_NN && layout <= GEMM_TN && M % kBigBM == 0 && N % kBigBM == 0 &&
         K % (2 * kBigBK) == 0 && K >= 4 * kBigBK && (M / kBigBM) * (N / kBigBM) >= num_cus &&
         a_elems < ((size_t)1 << 31) && b_elems < ((size_t)1 << 31);
}

// ---------------------------------------------------------------------------
// Small-M tile (M up to a few 16-row tiles: the B=64 forward and dX
// products).  One workgroup of 4 (or 8) waves owns a 16x16 output tile over
// the whole K range.  Wave w takes the w-th quarter (eighth) of K, rounded
// up to whole 16-k groups, loads its operands straight into registers
// (nothing is shared between the waves, so no LDS staging and no barrier in
// the K loop) and accumulates them on v_mfma_f32_16x16x4f32; the partial
// tiles are then added in wave order through LDS and the epilogue runs one
// element per thread.  K never
// leaves the workgroup -- no split-K workspace and no second launch -- while
// the grid (M/16 x N/16 tiles) still spreads over the CUs.
//
// v_mfma_f32_16x16x4f32 (one block): lane l supplies A(l%16, k) and
// B(k, l%16) for its k, and register v of lane l receives D(4*(l/16) + v, l%16).
// Within a group of 16 k values starting at kb, MFMA s (0..3) takes
// k = kb + 4q + s in lane quarter q = l/16, so a lane's four A operands of a
// group are four consecutive k of one row (one 16-byte load); likewise the
// B operands of the NT product (dX: rows of W_i).  Group g accumulates into
// accumulator g % 4 (chains of a quarter of the wave's terms), and the four
// accumulators, then the waves' tiles, are added as pairwise trees: a fixed
// order, with shorter rounding chains than one running sum.
// ---------------------------------------------------------------------------
constexpr int kSmallChunk = 16;    // 16-k groups per register chunk (256 k)
constexpr int kSmallStage = 16 * 64;  // floats of one staged operand strip (16 rows x 64 k)
constexpr int kSmallRedStride = 80;  // LDS floats per (wave, register) row of partials
template <int NW>
struct SmallLds {
  static constexpr int kFloats = NW * 4 * kSmallRedStride;
};

// Tile order: workgroups are handed to the 8 XCDs round-robin by index, and
// every XCD has its own L2.  The tiles that read the same columns of B (one
// strip of W_i; for the NN product two strips share each 128-byte line) are
// given indices of one residue mod 8, so that strip is fetched into one L2.
template <int SW>
__device__ __forceinline__ void smallm_coords(int blk, int tiles_m, int tiles_n, int& tm, int& tn) {
  if (tiles_n % (8 * SW) == 0) {
    const int xcd = blk & 7, j = blk >> 3;
    const int per = tiles_m * SW;
    const int grp = j / per, loc = j % per;
    tm = loc / SW;
    tn = (grp * 8 + xcd) * SW + loc % SW;
  } else {
    tm = blk % tiles_m;
    tn = blk / tiles_m;
  }
}

// The A operand of the dX product below a one-column output layer, formed
// in registers (smallm_tile with AH > 0): A(m, k) = (0 + d[m - m0] * W[k]) *
// f'(pre[m][k], act[m][k]) -- the row of delta_{n-2} that out_dx_row stores,
// from the same operands in the same order.  args.A then holds act_{n-1}
// (lda its row stride); `pre` is read only for AH == 2 (else f' takes act
// for both).  With `dx_out` set (workgroup-uniform) the tile also stores
// the A values it forms, its rows of delta_{n-2}, every element once: the
// last chunk's after the tile's last barrier (from the operand registers
// they replace), earlier chunks' as they are formed.
//
// AH == 3 (a forward product whose A operand is the previous layer's output,
// left by that layer's launch as two partial planes over halves of its K):
// A(m, k) = f((P0[m][k] + P1[m][k]) + b[k]) with args.A = P0, `pre` = P1
// (both of row stride lda), `w` = b and `act` = f; with `dx_out` set the
// tile also stores the A values (the previous layer's output) and, with
// `pre_out` set, the pre-activations, every element once.
struct SmallHead {
  const float* pre = nullptr;  // pre-activation of layer n-2 [M x lda] (AH == 3: the second plane)
  const float* w = nullptr;    // W_{n-1} [K x 1] (AH == 3: the previous layer's bias)
  const float* d = nullptr;    // the tile's 16 row deltas delta_{n-1} (LDS)
  float* dx_out = nullptr;     // delta_{n-2} [M x lda] (AH == 3: the previous layer's output), or null
  float* pre_out = nullptr;    // AH == 3: the previous layer's pre-activation [M x lda], or null
  int act = 0;                 // activation of layer n-2 (AH == 3: of the previous layer)
  float* zrows = nullptr;      // EPI_ROWS: the tile's 16 rows of acc + bias (LDS, row stride 17)
};
struct SmallNoop {
  __device__ void operator()() const {}
};

// NW waves per workgroup (4, or 8 for a stand-alone launch), each taking
// one NW-th of the K range.  With AH > 0 every thread calls `pre` once,
// after its first chunk's loads are issued and before any product term (the
// row deltas hd.d are read after it), and `post` once, after the tile's last
// barrier.
//
// STG = SW > 0 (16 waves, 16-byte rows, AH == 0): the A strip of each
// wave's chunk, SW k wide (and the B strip of an NT product), goes to a
// wave-private LDS area `stg` (kSmallStage floats per operand and wave) by
// direct-to-LDS loads whose lanes cover 256/SW rows x 4*SW contiguous bytes
// per instruction, and the MFMA fragments are read from there (16-byte
// chunk (r, c) of a strip at r*SW/4 + (c ^ (r % (SW/4))): conflict-free
// reads of 8 rows at one k-quad).  A load instruction of the register path
// covers 16 rows x 64 bytes, which the memory pipeline serves measurably
// slower.  SW = 32 only for a wave range of at most 32 k (one chunk, two
// groups).  Same operands, same order: bit-identical to the register path.
template <bool B_KC, bool VEC, int EPI, int NW, int AH = 0, class Pre = SmallNoop, class Post = SmallNoop,
          int SW = 0>
__device__ __forceinline__ void smallm_tile(const GemmArgs& args, int blk, float* lds,
                                            const SmallHead& hd = SmallHead{}, Pre pre = Pre{}, Post post = Post{},
                                            float* stg = nullptr) {
  constexpr bool STG = SW > 0;
  static_assert(SW == 0 || SW == 32 || SW == 64, "staged strips 32 or 64 k wide");
  static_assert(!STG || (VEC && NW == 16 && AH == 0), "staged operands: 16 waves, 16-byte rows, no head operand");
  static_assert(NW == 4 || NW == 8 || NW == 16, "wave trees for 4, 8 or 16 partial tiles");
  static_assert(AH == 0 || AH == 3 || (B_KC && VEC && EPI == EPI_DX_ACT && NW == 16),
                "head operand: NT dX product, 16-byte rows, 16 waves");
  static_assert(AH != 3 || (!B_KC && VEC && EPI == EPI_BIAS_ACT && NW == 16),
                "plane operand: NN forward product, 16-byte rows, 16 waves");
  // 16-wave workgroups (four waves per SIMD) hold a quarter chunk per wave
  constexpr int CH = NW == 16 ? kSmallChunk / 4 : kSmallChunk;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int M = args.M, N = args.N, K = args.K;
  const int tiles_m = (M + 15) / 16, tiles_n = (N + 15) / 16;
  int tm, tn;
  smallm_coords<B_KC ? 1 : 2>(blk, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * 16, n0 = tn * 16;
  // this wave's K range: NW-ths rounded up to whole 16-k groups
  const int kq = (K + NW * 16 - 1) / (NW * 16) * 16;
  const int kbeg = wave * kq, kend = min(K, kbeg + kq);
  const bool row_ok = m0 + r < M, col_ok = n0 + r < N;
  const int lda = args.lda, ldb = args.ldb;
  // lane's base pointers: A row m0+r; B row n0+r (NT) or column n0+r (NN)
  // (row 0 / column 0 stand in for rows and columns outside the matrix)
  const float* pa = args.A + (size_t)(row_ok ? m0 + r : 0) * lda;
  const float* pb = B_KC ? args.B + (size_t)(col_ok ? n0 + r : 0) * ldb : args.B + (col_ok ? n0 + r : 0);
  const float* pp = AH >= 2 ? hd.pre + (size_t)(row_ok ? m0 + r : 0) * lda : pa;
  // head operand: pre-activation (AH == 3: the second plane, then the
  // pre-activation formed), W_{n-1} (AH == 3: the bias)
  floatx4 fp[AH >= 2 ? CH : 1], fw[AH > 0 ? CH : 1];

  // A chunk's loads: per group unconditional within the lane (k clamped
  // into the wave's range), keeping the raw values; compute() replaces those
  // outside the matrix by zero.  (Guarded loads, or selects placed between
  // the loads, make the compiler wait for earlier loads in the middle of
  // the chunk.)  Groups past the wave's range are skipped as a whole
  // (wave-uniform).  Only called with kc < kend.
  auto load = [&](floatx4(&fa)[CH], floatx4(&fb)[CH], int kc) {
#pragma unroll
    for (int g = 0; g < CH; ++g) {
      if (kc + 16 * g >= kend) break;
      const int k = kc + 16 * g + 4 * q;  // this lane's first k of the group
      if (VEC) {  // K % 4 == 0 and every range bound is a multiple of 4
        const int kl = min(k, kend - 4);
        fa[g] = *reinterpret_cast<const floatx4*>(pa + kl);
        if constexpr (AH >= 2) fp[g] = *reinterpret_cast<const floatx4*>(pp + kl);
        if constexpr (AH > 0) fw[g] = *reinterpret_cast<const floatx4*>(hd.w + kl);
        if (B_KC) {
          fb[g] = *reinterpret_cast<const floatx4*>(pb + kl);
        } else {
#pragma unroll
          for (int s = 0; s < 4; ++s) fb[g][s] = pb[(size_t)(kl + s) * ldb];
        }
      } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int kl = min(k + s, kend - 1);
          fa[g][s] = pa[kl];
          fb[g][s] = B_KC ? pb[kl] : pb[(size_t)kl * ldb];
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  // The epilogue's operands (bias; the layer's output and pre-activation for
  // the activation derivative) of the element thread t < 256 finishes,
  // (t / 16, t % 16), loaded before the operands: loads complete in issue
  // order, so they cost no wait of their own, and the epilogue then runs
  // without a dependent memory latency.  Unconditional (index clamped).
  const EpiArgs& ep = args.epi;
  const int em = m0 + (tid >> 4), en = n0 + (tid & 15);
  const bool eok = tid < 256 && em < M && en < N;
  const size_t eidx = eok ? (size_t)em * ep.ldc + en : 0;
  float e_y = 0.0f, e_p = 0.0f;
  if constexpr (EPI == EPI_BIAS_ACT || EPI == EPI_ROWS) e_y = ep.bias[eok ? en : 0];
  if constexpr (EPI == EPI_DX_ACT) {
    e_y = ep.aux_act[eidx];
    e_p = ep.aux_pre ? ep.aux_pre[eidx] : e_y;
  }

  floatx4 acc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) acc[c] = floatx4{0.f, 0.f, 0.f, 0.f};
  static_assert(kSmallChunk % 4 == 0, "a chunk must hold whole rounds of the four accumulators");
  float dr = 0.0f;  // head operand: delta_{n-1} of the lane's row
  // (the head operand's A values replace the chunk's act values in fa)
  auto compute = [&](floatx4(&fa)[CH], const floatx4(&fb)[CH], int kc) {
#pragma unroll
    for (int g = 0; g < CH; ++g) {
      if (kc + 16 * g < kend) {  // wave-uniform
        const int k = kc + 16 * g + 4 * q;
        floatx4 xa;  // head operand: the lane's four A values of the group
        if constexpr (AH == 3) {
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const float pv = (fa[g][s] + fp[g][s]) + fw[g][s];  // pre = act W + b (:716-724), two halves of K
            fp[g][s] = pv;
            xa[s] = act_forward(hd.act, pv);  // (:725-743)
          }
          fa[g] = xa;
        } else if constexpr (AH > 0) {
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const float av = fa[g][s];
            float pv = av;
            if constexpr (AH == 2) pv = fp[g][s];
            xa[s] = (0.0f + dr * fw[g][s]) * act_derivative(hd.act, pv, av);
          }
          fa[g] = xa;
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const bool in = VEC ? k < kend : k + s < kend;
          float x;
          if constexpr (AH > 0) x = in && row_ok ? xa[s] : 0.0f;
          else x = in && row_ok ? fa[g][s] : 0.0f;
          const float y = in && col_ok ? fb[g][s] : 0.0f;
          acc[g & 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(x, y, acc[g & 3], 0, 0, 0);
        }
      }
    }
  };
  // One register chunk covers the wave's range for K <= 256 * waves (every
  // small-batch product of the step): all its loads are in flight together,
  // then its MFMAs run.  Longer ranges take one memory latency per chunk.
  floatx4 fa[CH], fb[CH];
  // head operand: store chunk kc's A values (rows of delta_{n-2})
  auto store_a = [&](int kc) {
    if constexpr (AH > 0) {
      if (!hd.dx_out || !row_ok) return;
#pragma unroll
      for (int g = 0; g < CH; ++g) {
        const int k = kc + 16 * g + 4 * q;
        if (kc + 16 * g < kend && k < kend) *reinterpret_cast<floatx4*>(hd.dx_out + (size_t)(m0 + r) * lda + k) = fa[g];
        if constexpr (AH == 3) {
          if (hd.pre_out && kc + 16 * g < kend && k < kend)
            *reinterpret_cast<floatx4*>(hd.pre_out + (size_t)(m0 + r) * lda + k) = fp[g];
        }
      }
    }
  };
  int last_kc = -1;
  if constexpr (AH > 0) {
    if (kbeg < kend) load(fa, fb, kbeg);
    if constexpr (AH != 3) {
      pre();  // every wave, once
      dr = hd.d[r];
    }
    for (int kc = kbeg; kc < kend; kc += 16 * CH) {
      if (kc != kbeg) load(fa, fb, kc);
      compute(fa, fb, kc);
      if (kc + 16 * CH < kend) store_a(kc);
      else last_kc = kc;
    }
  } else if constexpr (STG) {
    // this wave's strips: 16 rows x SW k each (SW / 16 groups of 16 k; with
    // SW = 32 the wave's range is one chunk of at most 32 k, so compute()
    // stops after group 1)
    static_assert(CH == 4, "a chunk is 64 k");
    constexpr int LPR = SW / 4;    // lanes (16-byte chunks) per strip row
    constexpr int RPI = 64 / LPR;  // strip rows per load instruction
    float* sa = stg + wave * kSmallStage;
    float* sb = stg + (NW + wave) * kSmallStage;
    const float* ra = args.A;
    const float* rb = args.B;
    for (int kc = kbeg; kc < kend; kc += 16 * CH) {
      // instruction i fills rows RPI*i..RPI*i+RPI-1: lane l takes row
      // RPI*i + l/LPR and the k-quad whose swizzled slot is l % LPR; k
      // clamped into the wave's range, rows outside the matrix read row 0
      // (both masked at the MFMAs)
#pragma unroll
      for (int i = 0; i < 16 / RPI; ++i) {
        const int rr = RPI * i + lane / LPR;
        const int c = (lane % LPR) ^ (rr % LPR);
        const int kl = min(kc + 4 * c, kend - 4);
        const int ar = m0 + rr < M ? m0 + rr : 0;
        __builtin_amdgcn_global_load_lds((const void*)(ra + (size_t)ar * lda + kl), (LdsVoidPtr)(sa + 256 * i), 16,
                                         0, 0);
        if constexpr (B_KC) {
          const int br = n0 + rr < N ? n0 + rr : 0;
          __builtin_amdgcn_global_load_lds((const void*)(rb + (size_t)br * ldb + kl), (LdsVoidPtr)(sb + 256 * i),
                                           16, 0, 0);
        }
      }
      if constexpr (!B_KC) {  // NN: the B operand's columns straight into registers
#pragma unroll
        for (int g = 0; g < CH; ++g) {
          if (kc + 16 * g >= kend) break;
          const int kl = min(kc + 16 * g + 4 * q, kend - 4);
#pragma unroll
          for (int s2 = 0; s2 < 4; ++s2) fb[g][s2] = pb[(size_t)(kl + s2) * ldb];
        }
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
      for (int g = 0; g < SW / 16; ++g) {
        if (kc + 16 * g >= kend) break;
        const int slot = 4 * (r * LPR + ((4 * g + q) ^ (r % LPR)));
        fa[g] = *reinterpret_cast<const floatx4*>(sa + slot);
        if constexpr (B_KC) fb[g] = *reinterpret_cast<const floatx4*>(sb + slot);
      }
      compute(fa, fb, kc);
    }
  } else {
    for (int kc = kbeg; kc < kend; kc += 16 * CH) {
      load(fa, fb, kc);
      compute(fa, fb, kc);
    }
  }

  // Partial tiles to LDS: row (wave, v) holds register v of every lane.
#pragma unroll
  for (int v = 0; v < 4; ++v)
    lds[(wave * 4 + v) * kSmallRedStride + lane] = (acc[0][v] + acc[1][v]) + (acc[2][v] + acc[3][v]);
  __syncthreads();
  if constexpr (AH > 0) {
    if (last_kc >= 0) store_a(last_kc);
    post();
  }
  // Element (i, j) of the tile: lane 16*(i/4) + j, register i%4 of each
  // wave; the waves' values added as (w0 + w1) + (w2 + w3) (then the same
  // for w4..w7, and the two halves).  Threads 0..255 hold one element each.
  if (tid >= 256) return;
  const int i = tid >> 4, j = tid & 15;
  const int src = (i & 3) * kSmallRedStride + 16 * (i >> 2) + j;
  constexpr int kW = 4 * kSmallRedStride;
  auto quad = [&](int w) {
    return (lds[w * kW + src] + lds[(w + 1) * kW + src]) + (lds[(w + 2) * kW + src] + lds[(w + 3) * kW + src]);
  };
  float sum = quad(0);
  if constexpr (NW == 8) sum = sum + quad(4);
  if constexpr (NW == 16) sum = (sum + quad(4)) + (quad(8) + quad(12));
  const int m = m0 + i, n = n0 + j;
  if (m < M && n < N) {
    // apply_epilogue's arithmetic on the prefetched operands
    if constexpr (EPI == EPI_BIAS_ACT) {
      const float v = sum + e_y;  // pre = act_i W_i + b_i (:716-724)
      if (ep.pre) ep.pre[eidx] = v;
      ep.out[eidx] = act_forward(ep.act, v);  // (:725-743)
    } else if constexpr (EPI == EPI_DX_ACT) {
      ep.out[eidx] = sum * act_derivative(ep.act, e_p, e_y);  // (:893-929)
    } else if constexpr (EPI == EPI_ROWS) {
      hd.zrows[i * 17 + j] = sum + e_y;  // z = act_{n-1} W + b (:792-798)
    } else {
      apply_epilogue<EPI>(ep, m, n, sum);
    }
  }
}

template <bool B_KC, bool VEC, int EPI, int NW>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(NW == 16 ? 4 : 2)))
gemm_smallm(GemmArgs args) {
  __shared__ float lds[SmallLds<NW>::kFloats];
  smallm_tile<B_KC, VEC, EPI, NW>(args, blockIdx.x, lds);
}

// 16 waves with staged operands (smallm_tile's STG), strips SW k wide:
// 64 KB of LDS per operand staged (A; B too for the NT product).
template <bool B_KC, int EPI, int SW>
__global__ void __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(4)))
gemm_smallm_stg(GemmArgs args) {
  __shared__ float lds[SmallLds<16>::kFloats];
  __shared__ __attribute__((aligned(16))) float stg[(B_KC ? 32 : 16) * kSmallStage];
  smallm_tile<B_KC, true, EPI, 16, 0, SmallNoop, SmallNoop, SW>(args, blockIdx.x, lds, SmallHead{}, SmallNoop{},
                                                               SmallNoop{}, stg);
}

// Staged strip width of a 16-wave small-M launch: 64 k for wave ranges of
// 48 k or more, 32 k for 32-k ranges, none (registers) for 16-k ranges, whose
// register loads already cover a whole range per instruction.  (smallm_tile's
// wave range: K / 16 rounded up to whole 16-k groups.)
static int smallm_stage_width(int K) {
  const int kq = (K + 255) / 256 * 16;
  return kq >= 48 ? 64 : kq == 32 ? 32 : 0;
}

// The narrow output layer of a large batch on the small-M tile (one 16-row
// strip per workgroup, the strip's z rows in LDS), then the loss head of
// each row by one thread (head_row: the same per-row code as the
// wave-dot-product output kernels), the strip's loss sum in row order into
// partials[strip], and the step counter advanced by block 0.  The loss
// itself is formed by a later launch of the step from the partials.
template <bool VEC>
__global__ void __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(4)))
gemm_smallm_out_head(GemmArgs args, OutLayerArgs p) {
  __shared__ float lds[SmallLds<16>::kFloats];
  __shared__ float zrows[16 * 17];
  __shared__ float row_loss[16];
  StepNext next{};
  if (threadIdx.x == 0 && blockIdx.x == 0) next = step_prefetch(p.scalars, p.bc_table, p.bc_len);
  const int tid = threadIdx.x, m0 = blockIdx.x * 16;  // tiles_n == 1: workgroup b owns strip b
  // the row's targets or label, loaded before the product
  const int rm = min(m0 + tid, p.B - 1);
  float y[16];
  int lab = 0;
  if (tid < 16) {
#pragma unroll
    for (int j = 0; j < 16; ++j) y[j] = p.loss == VOLTA_LOSS_MSE ? p.y[(size_t)rm * p.N + min(j, p.N - 1)] : 0.0f;
    if (p.loss != VOLTA_LOSS_MSE) lab = p.labels[rm];
  }
  SmallHead hd;
  hd.zrows = zrows;
  smallm_tile<false, VEC, EPI_ROWS, 16>(args, blockIdx.x, lds, hd);
  __syncthreads();
  if (tid < 16) {
    float z[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) z[j] = zrows[tid * 17 + min(j, p.N - 1)];
    row_loss[tid] = m0 + tid < p.B ? head_row<16>(p, z, y, lab, m0 + tid) : 0.0f;
  }
  __syncthreads();
  if (tid == 0) {
    const int rows = min(16, p.B - m0);
    float s = row_loss[0];
    for (int r = 1; r < rows; ++r) s = s + row_loss[r];
    p.partials[blockIdx.x] = s;
    if (blockIdx.x == 0 && p.bc_table) {
      p.scalars->t = next.t;
      p.scalars->bc1 = next.bc.x;
      p.scalars->bc2 = next.bc.y;
    }
  }
}

// A forward product over two halves of its K (a grid of at most half a
// workgroup per CU: C2's fwd2, 128 tiles): workgroup (z, t) runs tile t over
// half z of K on the 16-wave small-M tile and stores its raw partial tile to
// plane z, planes + z*M*N (row stride N).  The next forward launch adds the
// two planes, the bias and the activation as it loads its A operand
// (gemm_smallm_planes).
template <bool VEC>
__global__ void __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(4)))
gemm_smallm_khalves(GemmArgs args, float* planes, int k_half) {
  __shared__ float lds[SmallLds<16>::kFloats];
  const int tiles = ((args.M + 15) / 16) * ((args.N + 15) / 16);
  const int z = blockIdx.x >= tiles ? 1 : 0;
  GemmArgs a = args;
  a.A = args.A + (size_t)z * k_half;
  a.B = args.B + (size_t)z * k_half * args.ldb;
  a.K = z ? args.K - k_half : k_half;
  a.epi.kind = EPI_STORE;
  a.epi.ldc = args.N;
  a.epi.out = planes + (size_t)z * args.M * args.N;
  smallm_tile<false, VEC, EPI_STORE, 16>(a, blockIdx.x - z * tiles, lds);
}

// The forward product after gemm_smallm_khalves: A(m, k) = f((P0 + P1)[m][k]
// + b[k]) formed as it is loaded (smallm_tile, AH == 3), then the product,
// bias and activation of this layer as usual.  The first column tile of
// every 16-row strip also stores the strip's A values (the previous layer's
// output) and pre-activations, so later launches read them as if the
// previous layer had run on its own.
template <bool VEC>
__global__ void __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(4)))
gemm_smallm_planes(GemmArgs args, PlaneArgs p) {
  __shared__ float lds[SmallLds<16>::kFloats];
  const int tiles_m = (args.M + 15) / 16, tiles_n = (args.N + 15) / 16;
  int tm, tn;
  smallm_coords<2>(blockIdx.x, tiles_m, tiles_n, tm, tn);
  SmallHead hd;
  hd.pre = p.p1;
  hd.w = p.bias;
  hd.act = p.act;
  hd.dx_out = tn == 0 ? p.act_out : nullptr;
  hd.pre_out = tn == 0 ? p.pre_out : nullptr;
  smallm_tile<false, VEC, EPI_BIAS_ACT, 16, 3>(args, blockIdx.x, lds, hd);
}

// The last hidden layer's forward product (small-M tile, bias + activation)
// and, in the same launch, the output layer of width 1 with its loss head
// and dX_{n-1} -- one dependent launch fewer than running the output layer
// on its own (out_layer_dx_kernel).  The output layer needs whole rows of
// the hidden layer's output, so each 16-row strip is finished by the
// workgroup that stores the strip's last tile: every thread releases its
// stores (agent-scope fence), one thread takes the strip's ticket, and the
// workgroup that arrives last acquires the strip and runs the stand-alone
// output launch's per-row code (out_dx_row) for its 16 rows, two per wave.
// It adds its rows' losses into the stand-alone launch's per-4-row
// partials, in row order, and the last strip to finish forms the step's
// loss from them in the same block order; so parameters, activations,
// deltas and loss equal the two-launch path's bit for bit.
template <bool VEC>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2)))
gemm_smallm_head(GemmArgs args, OutLayerArgs p, unsigned* strip_counters) {
  __shared__ float lds[SmallLds<8>::kFloats];
  __shared__ float row_loss[16];
  __shared__ unsigned last_tile;
  smallm_tile<false, VEC, EPI_BIAS_ACT, 8>(args, blockIdx.x, lds);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int tiles_m = (args.M + 15) / 16, tiles_n = (args.N + 15) / 16;
  int tm, tn;
  smallm_coords<2>(blockIdx.x, tiles_m, tiles_n, tm, tn);
  // The barrier completes every wave's tile stores into this XCD's L2; one
  // agent-scope release by thread 0 then writes them back for the other
  // XCDs (a fence per wave costs a write-back per wave), and one acquire by
  // the last workgroup's thread 0 invalidates this CU's caches before the
  // strip is read.
  __syncthreads();
  if (tid == 0) {
    __threadfence();
    last_tile = atomicAdd(strip_counters + tm, 1u) == (unsigned)(tiles_n - 1) ? 1u : 0u;
    if (last_tile) __threadfence();
  }
  __syncthreads();
  if (!last_tile) return;  // workgroup-uniform
  StepNext next{};
  if (tid == 0) {
    strip_counters[tm] = 0u;
    next = step_prefetch(p.scalars, p.bc_table, p.bc_len);
  }
  const float l0 = out_dx_row<1, false>(p, nullptr, 16 * tm + wave);
  const float l1 = out_dx_row<1, false>(p, nullptr, 16 * tm + 8 + wave);
  if (lane == 0) {
    row_loss[wave] = l0;
    row_loss[8 + wave] = l1;
  }
  __syncthreads();
  if (tid == 0) {
    const int nblocks = (p.B + kOutDxRows - 1) / kOutDxRows;
#pragma unroll
    for (int g = 0; g < 16 / kOutDxRows; ++g) {
      const int b = (16 / kOutDxRows) * tm + g;
      float sb = row_loss[kOutDxRows * g];
      for (int w = 1; w < kOutDxRows; ++w) sb = sb + row_loss[kOutDxRows * g + w];
      if (b < nblocks) p.partials[b] = sb;
    }
    __threadfence();
    if (atomicAdd(p.loss_counter, 1u) == (unsigned)(tiles_m - 1)) {
      __threadfence();
      out_dx_finish(p, nblocks, next);
    }
  }
}

// The one-column output layer with its loss head and dX_{n-1}, and the dX
// product below it (dX_{n-2} on the 16-wave small-M tile), in one launch:
// one dependent launch fewer than out_layer_dx_kernel followed by that
// product.  The product's A operand, delta_{n-2}, is row-local: every
// workgroup forms the deltas delta_{n-1} of its 16-row strip (one row per
// wave with the output launch's own per-row arithmetic, out_head_rows) and
// then A from act_{n-1}, W_{n-1} and the pre-activation in registers
// (SmallHead), so no workgroup waits for another.  The strip's first
// column tile (tn == 0) also stores what the output launch stores -- z and
// delta_{n-1}, the rows of delta_{n-2} that the dW launch reads (the A
// values as it forms them), the loss partials of the strip's four 4-row
// blocks (the output launch's blocks, added in the same order) -- and
// strip 0's advances the step counter, all after the tile's last barrier
// (off the path from the row heads to the product); the loss sum is left
// to the step's dW launch (defer_loss).  MSE only (z and delta_{n-1} are stored without
// the CE label check).  Parameters, activations, deltas and the loss equal
// the two-launch path's bit for bit.  (Where dX_{n-2} takes 4-wave
// workgroups -- a grid above one workgroup per CU -- the same launch with
// four rows per wave is slower than the two launches: C3 0.088 -> 0.095 ms,
// C4 B=256 0.101 -> 0.104 ms.)
template <bool HP>
__global__ void __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(4)))
gemm_smallm_tail(GemmArgs args, OutLayerArgs p) {
  constexpr int NW = 16;
  static_assert(16 % kOutDxRows == 0, "a strip holds whole loss blocks of the output launch");
  __shared__ float lds[SmallLds<NW>::kFloats];
  __shared__ float z_rows[16], d_rows[16], row_loss[16];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int tiles_m = (args.M + 15) / 16, tiles_n = (args.N + 15) / 16;
  int tm, tn;
  smallm_coords<1>(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const bool writer = tn == 0;  // workgroup-uniform
  // row 16*tm + wave of the strip: z, delta_{n-1} and the loss to LDS
  auto head = [&]() {
    const int rows[1] = {16 * tm + wave};
    float ls[1];
    out_head_rows<1>(p, rows, z_rows + wave, d_rows + wave, ls);
    if (lane == 0) row_loss[wave] = ls[0];
    __syncthreads();
  };
  // the output launch's stores of this strip (first column tile only)
  auto tail_stores = [&]() {
    if (!writer) return;
    if (tid < 16) {
      const int m = 16 * tm + tid;
      if (m < p.B) {
        p.out[m] = z_rows[tid];
        p.delta[m] = d_rows[tid];
      }
    } else if (tid == 64) {
      const int nblocks = (p.B + kOutDxRows - 1) / kOutDxRows;
#pragma unroll
      for (int g = 0; g < 16 / kOutDxRows; ++g) {
        const int b = (16 / kOutDxRows) * tm + g;
        float sb = row_loss[kOutDxRows * g];
        for (int w = 1; w < kOutDxRows; ++w) sb = sb + row_loss[kOutDxRows * g + w];
        if (b < nblocks) p.partials[b] = sb;
      }
      if (tm == 0 && p.bc_table) {
        const StepNext next = step_prefetch(p.scalars, p.bc_table, p.bc_len);
        p.scalars->t = next.t;
        p.scalars->bc1 = next.bc.x;
        p.scalars->bc2 = next.bc.y;
      }
    }
  };
  SmallHead hd;
  hd.pre = HP ? p.dx_pre : nullptr;
  hd.w = p.W;
  hd.d = d_rows;
  hd.dx_out = writer ? p.dx_out : nullptr;
  hd.act = p.dx_act;
  smallm_tile<true, true, EPI_DX_ACT, NW, HP ? 2 : 1>(args, blockIdx.x, lds, hd, head, tail_stores);
}

// ---------------------------------------------------------------------------
// dW tile for a short reduction (K = B <= 256: the small-batch step).  A
// workgroup owns a 32x32 tile of W_i -- 4 elements per thread -- so a launch
// keeps several workgroups on each CU and the optimizer arithmetic of one
// overlaps the memory traffic of another.  (A 64x64 tile leaves about 1.5
// waves per SIMD at B=64, and its phases -- operands, product, optimizer
// state loads, arithmetic, stores -- then run in lockstep over the chip.)
//   1. 64-k slices of act_i^T (A(m,k) = act[k*lda + m]) and delta_i
//      (B(k,n) = delta[k*ldb + n]) go to LDS with 16-byte loads.  The
//      thread's float4 of W_i, m and v, and the state of one b_i element,
//      are loaded right after the first slice: vector loads complete in
//      issue order, so the wait for the operands does not wait for them, and
//      their latency runs under the product.  Every load is unconditional
//      (clamped address, value selected afterwards), which keeps the
//      compiler's wait counts exact.
//   2. wave w computes the 16x16 block (w/2, w%2) on v_mfma_f32_16x16x4f32
//      in the small-M tile's k order, the even and odd 16-k groups of each
//      slice in two accumulators, added at the end.
//   3. the dW tile goes through LDS; thread t updates row t/8, columns
//      4(t%8)..+3 of the tile: one float4 of W, m and v.
//   4. in the first row of tiles, thread j < 32 forms db_i[n0 + j] as
//      delta[0][n] + delta[1][n] + ... (batch ascending, the reference's
//      order, :931-933) and updates b_i[n0 + j].
// Needs M, N and the leading dimensions to be multiples of 4 and the
// operands 16-byte aligned (checked at launch).
// ---------------------------------------------------------------------------
constexpr int kDwT = 32;
constexpr int kDwK = 64;
constexpr int kDwS = kDwT + 4;   // LDS row stride of the [k][32] operand slices
constexpr int kDwDS = kDwT + 1;  // LDS row stride of the dW tile
constexpr int kDwLds = 2 * kDwK * kDwS + kDwT * kDwDS;
// The wide form (32x64 tiles of W): a [k][64] B slice, and the dW tile over
// the A slice once the product has consumed it.
constexpr int kDwTW = 64;
constexpr int kDwLdsW = kDwK * kDwS + kDwK * (kDwTW + 4);
static_assert(kDwT * (kDwTW + 1) <= kDwK * kDwS, "the wide dW tile fits over the A slice");

// `tid` (0..255): the thread's index among the tile's 256.  TN: the tile's
// columns, 32 (four float4 loads of W/m/v state per thread's element group)
// or 64 (the wide form: half the workgroups, each thread owning two float4
// of W, in rows r and r + 16).  Both forms add the 16-k groups of every
// slice into two accumulators per block (even groups, odd groups) and then
// the two: every element of dW sums the same products in the same order,
// so the two forms give bit-identical results.
template <int EPI, int TN = kDwT>
__device__ __forceinline__ void dw_smallk_tile(const GemmArgs& args, int blk, float* lds, int tid) {
  static_assert(EPI == EPI_DW_OPT || EPI == EPI_STORE, "epilogues of the dW tile");
  static_assert(TN == kDwT || TN == kDwTW, "tile widths of the dW tile");
  constexpr int SB = TN + 4;          // LDS row stride of the B slice
  constexpr int DS = TN + 1;          // LDS row stride of the dW tile
  constexpr int NB = TN / 32;         // 16-column blocks per wave
  constexpr int BIT = TN / 16;        // float4 of the B slice per thread
  constexpr int CPR = TN / 4;         // float4 per row of the tile
  constexpr int EIT = kDwT * CPR / 256;  // float4 of W per thread
  constexpr int RSTEP = 256 / CPR;    // rows between a thread's float4 of W
  const int lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, q = lane >> 4;
  const int wm = wave >> 1, wn = wave & 1;
  const int M = args.M, N = args.N, K = args.K;
  const int tiles_n = (N + TN - 1) / TN;
  const int tm = blk / tiles_n, tn = blk % tiles_n;
  const int m0 = tm * kDwT, n0 = tn * TN;
  float* la = lds;                // la[kk*kDwS + mm] = A(m0 + mm, k0 + kk)
  float* lb = lds + kDwK * kDwS;  // lb[kk*SB + nn] = B(k0 + kk, n0 + nn)
  // ld[mm*DS + nn] = dW(m0 + mm, n0 + nn): after both slices (32 wide), over
  // the A slice (64 wide)
  float* ld = TN == kDwT ? lds + 2 * kDwK * kDwS : lds;
  const EpiArgs& e = args.epi;
  const floatx4 zero4 = {0.f, 0.f, 0.f, 0.f};

  // One 64-k slice of both operands: 64 rows of 8 float4 of A (two per
  // thread) and 64 rows of TN/4 float4 of B (TN/16 per thread).
  floatx4 xa[2], xb[BIT];
  auto load_slice = [&](int k0) {
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int slot = tid + 256 * it;
      const int kk = slot >> 3, c4 = (slot & 7) * 4;
      const int k = k0 + kk;
      const bool kok = k < K;
      const bool aok = kok && m0 + c4 < M;
      const size_t ka = kok ? (size_t)k : 0;
      const floatx4 va = *reinterpret_cast<const floatx4*>(args.A + ka * args.lda + (aok ? m0 + c4 : 0));
      xa[it] = aok ? va : zero4;
    }
#pragma unroll
    for (int it = 0; it < BIT; ++it) {
      const int slot = tid + 256 * it;
      const int kk = slot / CPR, c4 = (slot % CPR) * 4;
      const int k = k0 + kk;
      const bool kok = k < K;
      const bool bok = kok && n0 + c4 < N;
      const size_t kb = kok ? (size_t)k : 0;
      const floatx4 vb = *reinterpret_cast<const floatx4*>(args.B + kb * args.ldb + (bok ? n0 + c4 : 0));
      xb[it] = bok ? vb : zero4;
    }
  };
  auto store_slice = [&]() {
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int slot = tid + 256 * it;
      const int kk = slot >> 3, c4 = (slot & 7) * 4;
      *reinterpret_cast<floatx4*>(la + kk * kDwS + c4) = xa[it];
    }
#pragma unroll
    for (int it = 0; it < BIT; ++it) {
      const int slot = tid + 256 * it;
      const int kk = slot / CPR, c4 = (slot % CPR) * 4;
      *reinterpret_cast<floatx4*>(lb + kk * SB + c4) = xb[it];
    }
  };

  // This thread's elements of the tile (float4 j in row row0 + j*RSTEP)
  // and, for the first row of tiles, its column of b_i.
  const int row0 = tid / CPR, c4 = (tid % CPR) * 4;
  const int gn = n0 + c4;
  bool own[EIT];
  uint32_t o[EIT];
#pragma unroll
  for (int j = 0; j < EIT; ++j) {
    const int gm = m0 + row0 + j * RSTEP;
    own[j] = gm < M && gn < N;  // N % 4 == 0: the whole float4 is in range
    o[j] = own[j] ? (uint32_t)gm * (uint32_t)e.ldc + (uint32_t)gn : 0u;
  }
  const int bn = n0 + (tid & (TN - 1));
  const bool do_db = EPI == EPI_DW_OPT && args.colsum_b && e.b && tm == 0;

  load_slice(0);
  __builtin_amdgcn_sched_barrier(0);
  floatx4 w4[EIT], m4[EIT], v4[EIT];
  BiasState bst;
  // SGD/Adagrad read their absent state buffers from W's own address (same lines)
  const float* pm = e.m ? e.m : e.out;
  const float* pv = e.v ? e.v : e.out;
  // the state loaded before the product (all of it in the 32-wide form; the
  // wide form's second float4 after it, which keeps the kernel within five
  // waves per SIMD without spills)
  constexpr int EARLY = TN == kDwT ? EIT : 1;
  auto load_state = [&](int j) {
    w4[j] = *reinterpret_cast<const floatx4*>(e.out + o[j]);
    m4[j] = *reinterpret_cast<const floatx4*>(pm + o[j]);
    v4[j] = *reinterpret_cast<const floatx4*>(pv + o[j]);
  };
  auto load_bias_state = [&]() {
    const float* pb = e.b ? e.b : e.out;
    const uint32_t ob = e.b && bn < N ? (uint32_t)bn : 0u;
    bst.b = pb[ob];
    bst.m = (e.bm ? e.bm : pb)[ob];
    bst.v = (e.bv ? e.bv : pb)[ob];
  };
  if constexpr (EPI == EPI_DW_OPT) {
#pragma unroll
    for (int j = 0; j < EARLY; ++j) load_state(j);
    if constexpr (TN == kDwT) load_bias_state();
  }
  __builtin_amdgcn_sched_barrier(0);

  // accumulators per block: 16-k group g of a slice adds into acc[nb][g % 2]
  // (two per block in both widths: the same order, and the wide form stays
  // within five waves per SIMD)
  constexpr int NACC = 2;
  floatx4 acc[NB][NACC];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int c = 0; c < NACC; ++c) acc[nb][c] = zero4;
  float db = 0.0f;
  for (int k0 = 0; k0 < K; k0 += kDwK) {
    if (k0 > 0) {
      __syncthreads();  // the previous slice is consumed
      load_slice(k0);
    }
    store_slice();
    __syncthreads();
    if (do_db && tid < TN) {
      // batch order; each batch of 8 reads is issued before its first add
      // (8 registers, not the slice's 64: the kernel's occupancy)
      const int kn = min(kDwK, K - k0);
#pragma unroll
      for (int k1 = 0; k1 < kDwK; k1 += 8) {
        float col[8];
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) col[kk] = lb[(k1 + kk) * SB + tid];
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          const float t = db + col[kk];
          db = k1 + kk < kn ? t : db;
        }
      }
    }
#pragma unroll
    for (int g = 0; g < kDwK / 16; ++g)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int kk = 16 * g + 4 * q + s;
        const float a = la[kk * kDwS + wm * 16 + r16];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const float b = lb[kk * SB + (wn * NB + nb) * 16 + r16];
          acc[nb][g % NACC] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[nb][g % NACC], 0, 0, 0);
        }
      }
  }
  if constexpr (EPI == EPI_DW_OPT) {
#pragma unroll
    for (int j = EARLY; j < EIT; ++j) load_state(j);
    if constexpr (TN != kDwT) load_bias_state();
  }
  if constexpr (TN != kDwT) __syncthreads();  // the dW tile goes over the A slice
  // register v of lane (r16, q) of block nb: dW(wm*16 + 4q + v, (wn*NB + nb)*16 + r16)
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float sum = acc[nb][0][v] + acc[nb][1][v];
      ld[(wm * 16 + 4 * q + v) * DS + (wn * NB + nb) * 16 + r16] = sum;
    }
  __syncthreads();
  floatx4 g4[EIT];
#pragma unroll
  for (int j = 0; j < EIT; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) g4[j][i] = ld[(row0 + j * RSTEP) * DS + c4 + i];

  if constexpr (EPI == EPI_STORE) {
#pragma unroll
    for (int j = 0; j < EIT; ++j)
      if (own[j]) *reinterpret_cast<floatx4*>(e.out + o[j]) = g4[j];
  } else {
#pragma unroll
    for (int j = 0; j < EIT; ++j)
      if (own[j] && e.grad) *reinterpret_cast<floatx4*>(e.grad + o[j]) = g4[j];
    const float lr = e.scalars->lr;
    const AdamRcp rc = adam_rcp_of(e);
    const uint32_t vec_end = (uint32_t)(e.count - e.count % 8);
#pragma unroll
    for (int j = 0; j < EIT; ++j) {
      float w[4], sm[4], sv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        w[i] = w4[j][i];
        sm[i] = m4[j][i];
        sv[i] = v4[j][i];
      }
      if (e.opt == VOLTA_OPT_SGD) {
        // sgd_fused_tn: W = 1*W + (-lr) * (act_i^T delta_i)  (:321-324)
        const float nlr = -lr;
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = w[i] + nlr * g4[j][i];
      } else if (e.opt == VOLTA_OPT_ADAGRAD) {
#pragma unroll
        for (int i = 0; i < 4; ++i) adagrad_elem(&w[i], &sm[i], g4[j][i], lr, e.eps);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          adam_elem(&w[i], &sm[i], &sv[i], g4[j][i], o[j] + i >= vec_end, lr, rc, e.b1, e.b2, e.eps, e.wd);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        w4[j][i] = w[i];
        m4[j][i] = sm[i];
        v4[j][i] = sv[i];
      }
      if (own[j]) {
        *reinterpret_cast<floatx4*>(e.out + o[j]) = w4[j];
        if (e.opt != VOLTA_OPT_SGD) *reinterpret_cast<floatx4*>(e.m + o[j]) = m4[j];
        if (e.opt == VOLTA_OPT_ADAM || e.opt == VOLTA_OPT_ADAMW) *reinterpret_cast<floatx4*>(e.v + o[j]) = v4[j];
      }
    }
    if (do_db && tid < TN && bn < N) bst.update_store(e, bn, N, db, rc);
  }
}

template <int EPI>
__global__ void __launch_bounds__(256) gemm_dw_smallk(GemmArgs args) {
  __shared__ __attribute__((aligned(16))) float lds[kDwLds];
  dw_smallk_tile<EPI>(args, blockIdx.x, lds, threadIdx.x);
}

// ---------------------------------------------------------------------------
// Narrow TN product with a long reduction (TILE_NARROW_TN: the output
// layer's dW at a large batch, N = L_n <= 16 columns, K = B rows of the
// batch), where a 64x64 MFMA tile would be mostly padding on a grid of a few
// dozen workgroups.  Workgroup (mb, z) owns rows m0..m0+63 of the product
// (lane m of every wave) over K slice z: the slice's B rows (delta) are
// staged in LDS, wave w adds the products of slice rows w, w + 4, w + 8, ...
// in order (every A load of them issued first: one per row, 64 lanes on 256
// consecutive bytes of act), and the four waves' sums are added
// (w0 + w1) + (w2 + w3) into plane z of the split-K workspace; with a bias,
// the slice's column sums of B (rows in order) go to the plane's row M.
// splitk_reduce then adds the planes in order and runs the epilogue.
constexpr int kNarrowTnK = 128;  // largest slice

// sd[kk*NMAX + n] = B[(k0 + kk)*ldb + min(n, N-1)] for the slice's nk rows,
// by the workgroup's 256 threads: load() issues every load, store() writes
// them to LDS (split so that other loads can be issued in between; a loop
// with a run-time trip count would wait for each load in turn).
template <int NMAX>
struct SliceStage {
  static constexpr int IT = (kNarrowTnK * NMAX + 255) / 256;
  float v[IT];
  __device__ __forceinline__ void load(const float* B, int ldb, int k0, int nk, int N, int t) {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int i = min(t + 256 * it, nk * NMAX - 1);
      const int kk = i / NMAX, n = i % NMAX;
      v[it] = B[(size_t)(k0 + kk) * ldb + min(n, N - 1)];
    }
  }
  __device__ __forceinline__ void store(float* sd, int nk, int t) const {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int i = t + 256 * it;
      if (i < nk * NMAX) sd[i] = v[it];
    }
  }
};

// Column n of the staged slice summed in row order, sd[n] + sd[NMAX + n] +
// ... (rows < nk), its LDS reads issued eight at a time.
template <int NMAX>
__device__ __forceinline__ float slice_colsum(const float* sd, int nk, int n) {
  float cs = sd[n];
#pragma unroll
  for (int k1 = 1; k1 < kNarrowTnK; k1 += 8) {
    float col[8];
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) col[kk] = sd[min(k1 + kk, kNarrowTnK - 1) * NMAX + n];
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      const float u = cs + col[kk];
      cs = k1 + kk < nk ? u : cs;
    }
  }
  return cs;
}

template <int NMAX>
__global__ void __launch_bounds__(256) narrow_tn_split(GemmArgs a) {
  __shared__ __attribute__((aligned(16))) float sd[kNarrowTnK * NMAX];
  __shared__ float red[3][64 * NMAX];
  constexpr int PER = kNarrowTnK / 4;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int M = a.M, N = a.N;
  const int m0 = blockIdx.x * 64, z = blockIdx.y;
  const int k0 = z * a.k_per_split, nk = min(a.k_per_split, a.K - k0);
  const int mc = min(m0 + lane, M - 1);
  // the slice's B rows first, then every A load: the products of row i
  // wait only for the loads up to row i's
  SliceStage<NMAX> stage;
  stage.load(a.B, a.ldb, k0, nk, N, t);
  float av[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int kk = min(w + 4 * i, nk - 1);
    av[i] = a.A[(size_t)(k0 + kk) * a.lda + mc];
  }
  stage.store(sd, nk, t);
  __syncthreads();
  float acc[NMAX];
#pragma unroll
  for (int j = 0; j < NMAX; ++j) acc[j] = 0.0f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int kk = w + 4 * i;
    if (kk < nk) {  // wave-uniform
      // the row's B values: one broadcast read per four columns
      float bv[NMAX];
      if constexpr (NMAX % 4 == 0) {
#pragma unroll
        for (int q = 0; q < NMAX / 4; ++q) {
          const floatx4 v = *reinterpret_cast<const floatx4*>(sd + kk * NMAX + 4 * q);
#pragma unroll
          for (int e = 0; e < 4; ++e) bv[4 * q + e] = v[e];
        }
      } else {
#pragma unroll
        for (int j = 0; j < NMAX; ++j) bv[j] = sd[kk * NMAX + j];
      }
#pragma unroll
      for (int j = 0; j < NMAX; ++j) acc[j] = acc[j] + av[i] * bv[j];
    }
  }
  if (w > 0) {
#pragma unroll
    for (int j = 0; j < NMAX; ++j) red[w - 1][lane * NMAX + j] = acc[j];
  }
  __syncthreads();
  float* plane = a.partial + (size_t)z * (M + 1) * N;
  if (w == 0 && m0 + lane < M) {
#pragma unroll
    for (int j = 0; j < NMAX; ++j)
      if (j < N)
        plane[(size_t)(m0 + lane) * N + j] =
            (acc[j] + red[0][lane * NMAX + j]) + (red[1][lane * NMAX + j] + red[2][lane * NMAX + j]);
  }
  if (a.colsum_b && blockIdx.x == 0 && w == 1 && lane < N) {
    plane[(size_t)M * N + lane] = slice_colsum<NMAX>(sd, nk, lane);
  }
}

void narrow_tn_split_plan(int M, int K, int num_cus, int* k_per_split, int* splits) {
  const int mb = (M + 63) / 64;
  int kps = kNarrowTnK;
  while (kps > 32 && (size_t)mb * ((K + kps - 1) / kps) < (size_t)2 * num_cus) kps /= 2;
  *k_per_split = kps;
  *splits = (K + kps - 1) / kps;
}

// Planes whose loads splitk_reduce issues together (more planes: a loop).
constexpr int kReduceUnroll = 16;

// Second kernel of a split-K launch: add the planes in slice order, then the
// epilogue (and, for dW, the bias update from the summed column sums kept in
// row M of each plane).  One thread per W consecutive elements of a row;
// every load a thread needs (all planes, bias or activation operands) is
// issued before the first use, so the kernel waits one memory latency.
template <int EPI, int W>
__global__ void __launch_bounds__(256) splitk_reduce(GemmArgs a, int splits) {
  const int M = a.M, N = a.N;
  const size_t plane = (size_t)(M + 1) * N;
  const size_t total = (size_t)M * N;
  const size_t extra = EPI == EPI_DW_OPT && a.colsum_b ? (size_t)N : 0;
  const size_t items = (total + extra) / W;  // W divides N
  const EpiArgs& e = a.epi;
  AdamRcp rc{};
  if constexpr (EPI == EPI_DW_OPT) rc = adam_rcp_of(e);
  for (size_t it = (size_t)blockIdx.x * blockDim.x + threadIdx.x; it < items;
       it += (size_t)gridDim.x * blockDim.x) {
    const size_t idx = it * W;
    float s[W];
    if (splits <= kReduceUnroll) {
      float p[kReduceUnroll][W];
#pragma unroll
      for (int z = 0; z < kReduceUnroll; ++z)
        if (z < splits) {
          const float* src = a.partial + (size_t)z * plane + idx;
          if constexpr (W == 4) {
            const floatx4 v = *reinterpret_cast<const floatx4*>(src);
#pragma unroll
            for (int q = 0; q < W; ++q) p[z][q] = v[q];
          } else {
            p[z][0] = src[0];
          }
        }
#pragma unroll
      for (int q = 0; q < W; ++q) s[q] = p[0][q];
#pragma unroll
      for (int z = 1; z < kReduceUnroll; ++z)
        if (z < splits) {
#pragma unroll
          for (int q = 0; q < W; ++q) s[q] = s[q] + p[z][q];
        }
    } else if constexpr (W == 1) {
      // kReduceUnroll planes' loads at a time, added in plane order (the
      // narrow products split K the most)
      s[0] = a.partial[idx];
      for (int z0 = 1; z0 < splits; z0 += kReduceUnroll) {
        float p[kReduceUnroll];
#pragma unroll
        for (int z = 0; z < kReduceUnroll; ++z) p[z] = a.partial[(size_t)min(z0 + z, splits - 1) * plane + idx];
#pragma unroll
        for (int z = 0; z < kReduceUnroll; ++z) s[0] = z0 + z < splits ? s[0] + p[z] : s[0];
      }
    } else {
#pragma unroll
      for (int q = 0; q < W; ++q) s[q] = a.partial[idx + q];
      for (int z = 1; z < splits; ++z)
#pragma unroll
        for (int q = 0; q < W; ++q) s[q] = s[q] + a.partial[(size_t)z * plane + idx + q];
    }
    if (idx < total) {
      const int m = (int)(idx / N), n = (int)(idx % N);
      const size_t o = (size_t)m * e.ldc + n;
      if constexpr (EPI == EPI_BIAS_ACT) {
        float b[W];
#pragma unroll
        for (int q = 0; q < W; ++q) b[q] = e.bias[n + q];
        float x[W], y[W];
#pragma unroll
        for (int q = 0; q < W; ++q) {
          x[q] = s[q] + b[q];  // pre = act_i W_i + b_i (:716-724)
          y[q] = act_forward(e.act, x[q]);
        }
        if constexpr (W == 4) {  // 16-byte stores (launch_reduce checked the alignment)
          if (e.pre) *reinterpret_cast<floatx4*>(e.pre + o) = floatx4{x[0], x[1], x[2], x[3]};
          *reinterpret_cast<floatx4*>(e.out + o) = floatx4{y[0], y[1], y[2], y[3]};
        } else {
          if (e.pre) e.pre[o] = x[0];
          e.out[o] = y[0];
        }
      } else if constexpr (EPI == EPI_DX_ACT) {
        const float* pp = e.aux_pre ? e.aux_pre : e.aux_act;
        float y[W], pr[W], d[W];
        if constexpr (W == 4) {
          const floatx4 y4 = *reinterpret_cast<const floatx4*>(e.aux_act + o);
          const floatx4 p4 = *reinterpret_cast<const floatx4*>(pp + o);
#pragma unroll
          for (int q = 0; q < W; ++q) y[q] = y4[q], pr[q] = p4[q];
        } else {
          y[0] = e.aux_act[o];
          pr[0] = pp[o];
        }
#pragma unroll
        for (int q = 0; q < W; ++q) d[q] = s[q] * act_derivative(e.act, pr[q], y[q]);
        if constexpr (W == 4) *reinterpret_cast<floatx4*>(e.out + o) = floatx4{d[0], d[1], d[2], d[3]};
        else e.out[o] = d[0];
      } else if constexpr (EPI == EPI_DW_OPT && W == 4) {
        // the four elements' W and optimizer state loaded together (16-byte
        // accesses: launch_reduce checked the alignment), then the same
        // per-element update as apply_epilogue, then the stores -- instead
        // of one dependent load-update-store per element
        const float lr = e.scalars->lr;
        const bool has1 = e.opt != VOLTA_OPT_SGD, has2 = e.opt == VOLTA_OPT_ADAM || e.opt == VOLTA_OPT_ADAMW;
        floatx4 w = *reinterpret_cast<const floatx4*>(e.out + o);
        floatx4 s1 = has1 ? *reinterpret_cast<const floatx4*>(e.m + o) : floatx4{};
        floatx4 s2 = has2 ? *reinterpret_cast<const floatx4*>(e.v + o) : floatx4{};
        const int64_t vec_end = e.count - e.count % 8;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (e.opt == VOLTA_OPT_SGD) {
            w[q] = w[q] + (-lr) * s[q];  // sgd_fused_tn: W = 1*W + (-lr) * (act_i^T delta_i)  (:321-324)
          } else if (e.opt == VOLTA_OPT_ADAGRAD) {
            float a = w[q], b = s1[q];
            adagrad_elem(&a, &b, s[q], lr, e.eps);
            w[q] = a, s1[q] = b;
          } else {
            float a = w[q], b = s1[q], c = s2[q];
            adam_elem(&a, &b, &c, s[q], (int64_t)(o + q) >= vec_end, lr, rc, e.b1, e.b2, e.eps, e.wd);
            w[q] = a, s1[q] = b, s2[q] = c;
          }
        }
        if (e.grad) *reinterpret_cast<floatx4*>(e.grad + o) = floatx4{s[0], s[1], s[2], s[3]};
        *reinterpret_cast<floatx4*>(e.out + o) = w;
        if (has1) *reinterpret_cast<floatx4*>(e.m + o) = s1;
        if (has2) *reinterpret_cast<floatx4*>(e.v + o) = s2;
      } else {
#pragma unroll
        for (int q = 0; q < W; ++q) apply_epilogue<EPI>(e, m, n + q, s[q], rc);
      }
    } else if constexpr (EPI == EPI_DW_OPT) {
#pragma unroll
      for (int q = 0; q < W; ++q) apply_bias_update(e, (int)(idx + q - total), N, s[q], rc);
    }
  }
}

// ---------------------------------------------------------------------------
// Host-side dispatch.
// ---------------------------------------------------------------------------
template <int BM, int BN, int BK, int WM, int WN, bool A_KC, bool B_KC, int EPI, int KG>
static hipError_t launch_kg(const GemmArgs& a, bool vec, hipStream_t st) {
  using T = Tile<BM, BN, BK, WM, WN>;
  const int tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  if (vec) hipLaunchKernelGGL((gemm_f32_mfma_kg<BM, BN, BK, WM, WN, A_KC, B_KC, true, EPI, KG>), dim3(tiles),
                              dim3(KG * T::kThreads), 0, st, a);
  else hipLaunchKernelGGL((gemm_f32_mfma_kg<BM, BN, BK, WM, WN, A_KC, B_KC, false, EPI, KG>), dim3(tiles),
                          dim3(KG * T::kThreads), 0, st, a);
  return hipGetLastError();
}

template <int BM, int BN, int BK, int WM, int WN, bool A_KC, bool B_KC, int EPI>
static hipError_t launch_epi(const GemmArgs& a, bool vec, int splits, bool ink, hipStream_t st, int kg = 1) {
  using T = Tile<BM, BN, BK, WM, WN>;
  // K groups where their operand LDS fits the CU's 160 KB
  constexpr int kStageFloats = LdsTile<BM, BK, A_KC>::kFloats + LdsTile<BN, BK, B_KC>::kFloats;
  if constexpr (EPI != EPI_LOSS && BK == 32) {
    if constexpr (2 * 2 * kStageFloats * 4 <= 160 * 1024) {
      if (kg == 2) return launch_kg<BM, BN, BK, WM, WN, A_KC, B_KC, EPI, 2>(a, vec, st);
    }
    // (four groups: 16 waves, 128 registers a lane -- too few for the
    // optimizer epilogue's state, which would spill)
    if constexpr (2 * 4 * kStageFloats * 4 <= 160 * 1024 && 4 * T::kThreads <= 1024 && EPI != EPI_DW_OPT) {
      if (kg == 4) return launch_kg<BM, BN, BK, WM, WN, A_KC, B_KC, EPI, 4>(a, vec, st);
    }
  }
  if (kg != 1) return hipErrorInvalidValue;
  const int tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  dim3 grid(tiles, splits), block(T::kThreads);
  if (ink) {
    if (vec) hipLaunchKernelGGL((gemm_f32_mfma<BM, BN, BK, WM, WN, A_KC, B_KC, true, EPI, true>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((gemm_f32_mfma<BM, BN, BK, WM, WN, A_KC, B_KC, false, EPI, true>), grid, block, 0, st, a);
  } else {
    if (vec) hipLaunchKernelGGL((gemm_f32_mfma<BM, BN, BK, WM, WN, A_KC, B_KC, true, EPI, false>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((gemm_f32_mfma<BM, BN, BK, WM, WN, A_KC, B_KC, false, EPI, false>), grid, block, 0, st, a);
  }
  return hipGetLastError();
}

// Valid (layout, epilogue) pairs of the step: NN with BIAS_ACT / LOSS /
// STORE, NT with DX_ACT / STORE, TN with DW_OPT / STORE.
template <int BM, int BN, int BK, int WM, int WN>
static hipError_t launch_cfg(const GemmArgs& a, int layout, bool vec, int splits, bool ink, hipStream_t st,
                             int kg = 1) {
  const int k = a.epi.kind;
  switch (layout) {
    case GEMM_NN:
      if (k == EPI_BIAS_ACT)
        return launch_epi<BM, BN, BK, WM, WN, true, false, EPI_BIAS_ACT>(a, vec, splits, ink, st, kg);
      if (k == EPI_STORE) return launch_epi<BM, BN, BK, WM, WN, true, false, EPI_STORE>(a, vec, splits, ink, st, kg);
      if constexpr (BM * (BN + 1) <= 2 * LdsTile<BM, BK, true>::kFloats) {
        if (k == EPI_LOSS && kg == 1)
          return launch_epi<BM, BN, BK, WM, WN, true, false, EPI_LOSS>(a, vec, splits, true, st);
      }
      break;
    case GEMM_NT:
      if (k == EPI_DX_ACT) return launch_epi<BM, BN, BK, WM, WN, true, true, EPI_DX_ACT>(a, vec, splits, ink, st, kg);
      if (k == EPI_STORE) return launch_epi<BM, BN, BK, WM, WN, true, true, EPI_STORE>(a, vec, splits, ink, st, kg);
      break;
    case GEMM_TN:
      if (k == EPI_DW_OPT)
        return launch_epi<BM, BN, BK, WM, WN, false, false, EPI_DW_OPT>(a, vec, splits, ink, st, kg);
      if (k == EPI_STORE) return launch_epi<BM, BN, BK, WM, WN, false, false, EPI_STORE>(a, vec, splits, ink, st, kg);
      break;
  }
  return hipErrorInvalidValue;
}

template <int EPI>
static hipError_t launch_reduce(const GemmArgs& a, int splits, hipStream_t st) {
  const size_t total = (size_t)a.M * a.N + (EPI == EPI_DW_OPT && a.colsum_b ? a.N : 0);
  const bool v4 = a.N % 4 == 0 && a.epi.ldc % 4 == 0 && (EPI == EPI_STORE || quad_aligned(a.epi, EPI));
  const size_t items = v4 ? total / 4 : total;
  const int blocks = (int)std::min<size_t>((items + 255) / 256, 1 << 20);
  if (v4) hipLaunchKernelGGL((splitk_reduce<EPI, 4>), dim3(blocks), dim3(256), 0, st, a, splits);
  else hipLaunchKernelGGL((splitk_reduce<EPI, 1>), dim3(blocks), dim3(256), 0, st, a, splits);
  return hipGetLastError();
}

// Small-M products: NN with BIAS_ACT / STORE, NT with DX_ACT / STORE.
// Waves per workgroup of a small-M launch (forward NN or dX NT): 16 while the
// grid has at most one workgroup per CU, else 4.  More waves split K into
// shorter chains per wave; a 16-wave workgroup fills its CU, so a larger grid
// would take two rounds, while 4-wave workgroups fit three to a CU.
// Measured on C2 (every grid <= 256 workgroups): 57.8 us/step with 8 waves
// against 56.7 with 16 (three alternating runs each); C3's 512-workgroup
// fwd0/fwd1 4.16/14.36 us with 4 against 5.28/16.1 us with 8.  A dX in a
// 256-thread paired launch takes 4 (the large-batch pairs); the small-batch
// step runs its dX launches alone.  VOLTA_SMALLM_WAVES=4, 8 or 16 fixes the
// count.
static int smallm_waves(bool b_kc, int blocks, int num_cus);

int gemm_smallm_waves(bool paired, int M, int N, int num_cus) {
  return paired ? 4 : smallm_waves(false, ((M + 15) / 16) * ((N + 15) / 16), num_cus);
}

static int smallm_waves(bool b_kc, int blocks, int num_cus) {
  const char* w = std::getenv("VOLTA_SMALLM_WAVES");
  int waves = blocks <= num_cus ? 16 : 4;
  if (w && *w) waves = std::atoi(w) == 4 ? 4 : std::atoi(w) == 16 ? 16 : 8;
  return b_kc ? 4 : waves;
}

template <bool B_KC, int EPI>
static hipError_t launch_smallm_epi(const GemmArgs& a, bool vec, int waves, bool stage, hipStream_t st) {
  const int blocks = ((a.M + 15) / 16) * ((a.N + 15) / 16);
  if (waves == 16) {
    const int sw = vec && stage ? smallm_stage_width(a.K) : 0;
    if (sw == 64) hipLaunchKernelGGL((gemm_smallm_stg<B_KC, EPI, 64>), dim3(blocks), dim3(1024), 0, st, a);
    else if (sw == 32) hipLaunchKernelGGL((gemm_smallm_stg<B_KC, EPI, 32>), dim3(blocks), dim3(1024), 0, st, a);
    else if (vec) hipLaunchKernelGGL((gemm_smallm<B_KC, true, EPI, 16>), dim3(blocks), dim3(1024), 0, st, a);
    else hipLaunchKernelGGL((gemm_smallm<B_KC, false, EPI, 16>), dim3(blocks), dim3(1024), 0, st, a);
  } else if (waves == 8) {
    if (vec) hipLaunchKernelGGL((gemm_smallm<B_KC, true, EPI, 8>), dim3(blocks), dim3(512), 0, st, a);
    else hipLaunchKernelGGL((gemm_smallm<B_KC, false, EPI, 8>), dim3(blocks), dim3(512), 0, st, a);
  } else {
    if (vec) hipLaunchKernelGGL((gemm_smallm<B_KC, true, EPI, 4>), dim3(blocks), dim3(256), 0, st, a);
    else hipLaunchKernelGGL((gemm_smallm<B_KC, false, EPI, 4>), dim3(blocks), dim3(256), 0, st, a);
  }
  return hipGetLastError();
}

// 16-byte operand loads need K, the leading dimensions of the K-contiguous
// operands and their base addresses to be multiples of 4 floats.
static bool smallm_vec_ok(const GemmArgs& a, int layout) {
  const auto al = [](const float* p) { return ((uintptr_t)p & 15u) == 0; };
  return a.K % 4 == 0 && a.lda % 4 == 0 && al(a.A) && (layout != GEMM_NT || (a.ldb % 4 == 0 && al(a.B)));
}

// The small-K dW tile: 16-byte rows of both operands and of W_i and its state.
static bool dw_smallk_ok(const GemmArgs& a, int layout) {
  const auto al = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  const EpiArgs& e = a.epi;
  if (layout != GEMM_TN || (e.kind != EPI_DW_OPT && e.kind != EPI_STORE)) return false;
  if (a.M % 4 || a.N % 4 || a.lda % 4 || a.ldb % 4 || e.ldc % 4 || !al(a.A) || !al(a.B) || !al(e.out)) return false;
  if (e.kind == EPI_DW_OPT && (!al(e.m) || !al(e.v) || !al(e.grad))) return false;
  if (a.colsum_b && e.kind != EPI_DW_OPT) return false;
  return (size_t)a.M * e.ldc < ((size_t)1 << 30);
}

static hipError_t launch_smallm(const GemmArgs& a, int layout, bool vec, int waves, bool stage, hipStream_t st) {
  if (vec && !smallm_vec_ok(a, layout)) return hipErrorInvalidValue;
  if (waves != 4 && waves != 8 && waves != 16) return hipErrorInvalidValue;
  if (layout == GEMM_NT && waves == 16 && !vec) return hipErrorInvalidValue;
  const int k = a.epi.kind;
  if (layout == GEMM_NN) {
    if (k == EPI_BIAS_ACT) return launch_smallm_epi<false, EPI_BIAS_ACT>(a, vec, waves, stage, st);
    if (k == EPI_STORE) return launch_smallm_epi<false, EPI_STORE>(a, vec, waves, stage, st);
  } else if (layout == GEMM_NT) {
    if (k == EPI_DX_ACT) return launch_smallm_epi<true, EPI_DX_ACT>(a, vec, waves, stage, st);
    if (k == EPI_STORE) return launch_smallm_epi<true, EPI_STORE>(a, vec, waves, stage, st);
  }
  return hipErrorInvalidValue;
}

bool fwd_head_supported(const GemmPlan& p, const GemmArgs& a, const OutLayerArgs& o, int n_counters) {
  const int tiles_m = (a.M + 15) / 16;
  return p.tile == TILE_SMALLM && p.layout == GEMM_NN && p.splits == 1 && a.epi.kind == EPI_BIAS_ACT &&
         p.waves == 8 && (!p.vec || smallm_vec_ok(a, GEMM_NN)) && o.N == 1 && o.B == a.M &&
         o.K == a.N && o.act == a.epi.out && o.B <= kNarrowMaxB && tiles_m <= n_counters && o.partials &&
         o.loss_counter && o.dx_out;
}

hipError_t launch_fwd_head(const GemmPlan& p, const GemmArgs& args_in, const OutLayerArgs& o,
                           unsigned* strip_counters, int n_counters, hipStream_t st) {
  GemmArgs a = args_in;
  a.k_per_split = p.k_per_split;
  if (!strip_counters || !fwd_head_supported(p, a, o, n_counters)) return hipErrorInvalidValue;
  const dim3 grid(((a.M + 15) / 16) * ((a.N + 15) / 16));
  if (p.vec) hipLaunchKernelGGL(gemm_smallm_head<true>, grid, dim3(512), 0, st, a, o, strip_counters);
  else hipLaunchKernelGGL(gemm_smallm_head<false>, grid, dim3(512), 0, st, a, o, strip_counters);
  return hipGetLastError();
}

// `a` is the dX_{n-2} product as planned (its A, delta_{n-2}, is replaced
// by the head operand); `o` the output launch's arguments with its dX.
bool tail_supported(const GemmPlan& p, const GemmArgs& a, const OutLayerArgs& o) {
  const auto al = [](const void* q) { return ((uintptr_t)q & 15u) == 0; };
  GemmArgs h = a;
  h.A = o.act;
  h.lda = o.K;
  return p.tile == TILE_SMALLM && p.layout == GEMM_NT && p.splits == 1 && p.vec && p.waves == 16 &&
         a.epi.kind == EPI_DX_ACT && o.N == 1 && o.B == a.M && o.K == a.K && o.B >= 1 && o.B <= kNarrowMaxB &&
         o.loss == VOLTA_LOSS_MSE && o.defer_loss && o.partials && o.scalars && o.dx_out && al(o.dx_out) && o.act &&
         o.W && al(o.W) &&
         (!o.dx_pre || al(o.dx_pre)) && smallm_vec_ok(h, GEMM_NT);
}

hipError_t launch_smallm_tail(const GemmPlan& p, const GemmArgs& args_in, const OutLayerArgs& o, hipStream_t st) {
  if (!tail_supported(p, args_in, o)) return hipErrorInvalidValue;
  GemmArgs a = args_in;
  a.A = o.act;
  a.lda = o.K;
  a.k_per_split = p.k_per_split;
  const dim3 grid(((a.M + 15) / 16) * ((a.N + 15) / 16));
  if (o.dx_pre) hipLaunchKernelGGL(gemm_smallm_tail<true>, grid, dim3(1024), 0, st, a, o);
  else hipLaunchKernelGGL(gemm_smallm_tail<false>, grid, dim3(1024), 0, st, a, o);
  return hipGetLastError();
}

bool out_head_gemm_supported(const GemmArgs& a, const OutLayerArgs& o) {
  return o.N >= 1 && o.N <= 16 && o.B == a.M && o.N == a.N && o.K == a.K && a.M > 0 && o.partials && o.scalars &&
         o.out && o.delta && a.epi.bias && (o.loss == VOLTA_LOSS_MSE ? o.y != nullptr : o.labels != nullptr) &&
         a.ldb == o.N && a.lda == o.K;
}

hipError_t launch_smallm_out_head(const GemmArgs& a, const OutLayerArgs& o, hipStream_t st) {
  if (!out_head_gemm_supported(a, o)) return hipErrorInvalidValue;
  const dim3 grid((a.M + 15) / 16);
  if (smallm_vec_ok(a, GEMM_NN)) hipLaunchKernelGGL(gemm_smallm_out_head<true>, grid, dim3(1024), 0, st, a, o);
  else hipLaunchKernelGGL(gemm_smallm_out_head<false>, grid, dim3(1024), 0, st, a, o);
  return hipGetLastError();
}

bool khalves_supported(const GemmPlan& p, const GemmArgs& a, int k_half) {
  return p.tile == TILE_SMALLM && p.layout == GEMM_NN && p.splits == 1 && p.vec && a.M > 0 && a.N > 0 &&
         k_half > 0 && k_half < a.K && k_half % 16 == 0 && a.ldb % 4 == 0 && smallm_vec_ok(a, GEMM_NN);
}

hipError_t launch_smallm_khalves(const GemmPlan& p, const GemmArgs& args_in, float* planes, int k_half,
                                 hipStream_t st) {
  if (!khalves_supported(p, args_in, k_half) || !planes || ((uintptr_t)planes & 15u)) return hipErrorInvalidValue;
  const dim3 grid(2 * ((args_in.M + 15) / 16) * ((args_in.N + 15) / 16));
  hipLaunchKernelGGL(gemm_smallm_khalves<true>, grid, dim3(1024), 0, st, args_in, planes, k_half);
  return hipGetLastError();
}

bool planes_supported(const GemmPlan& p, const GemmArgs& a, const PlaneArgs& pa) {
  const auto al = [](const void* q) { return ((uintptr_t)q & 15u) == 0; };
  return p.tile == TILE_SMALLM && p.layout == GEMM_NN && p.splits == 1 && p.vec && p.waves == 16 &&
         a.epi.kind == EPI_BIAS_ACT && smallm_vec_ok(a, GEMM_NN) && pa.p1 && al(pa.p1) && pa.bias && al(pa.bias) &&
         pa.act_out && al(pa.act_out) && (!pa.pre_out || al(pa.pre_out));
}

hipError_t launch_smallm_planes(const GemmPlan& p, const GemmArgs& a, const PlaneArgs& pa, hipStream_t st) {
  if (!planes_supported(p, a, pa)) return hipErrorInvalidValue;
  const dim3 grid(((a.M + 15) / 16) * ((a.N + 15) / 16));
  hipLaunchKernelGGL(gemm_smallm_planes<true>, grid, dim3(1024), 0, st, a, pa);
  return hipGetLastError();
}

template <bool A_KC, bool B_KC, int EPI>
static hipError_t launch_big_epi(const GemmArgs& a, hipStream_t st) {
  const dim3 grid((a.M / kBigBM) * (a.N / kBigBM));
  hipLaunchKernelGGL((gemm_big<A_KC, B_KC, EPI>), grid, dim3(512), 0, st, a);
  return hipGetLastError();
}

template <bool A_KC, bool B_KC, int EPI>
static hipError_t launch_big128_epi(const GemmArgs& a, hipStream_t st) {
  const dim3 grid((a.M / kB2) * (a.N / kB2));
  hipLaunchKernelGGL((gemm_big128<A_KC, B_KC, EPI>), grid, dim3(512), 0, st, a);
  return hipGetLastError();
}

static hipError_t launch_big128(const GemmArgs& a, int layout, hipStream_t st) {
  const int k = a.epi.kind;
  switch (layout) {
    case GEMM_NN:
      if (k == EPI_BIAS_ACT) return launch_big128_epi<true, false, EPI_BIAS_ACT>(a, st);
      if (k == EPI_STORE) return launch_big128_epi<true, false, EPI_STORE>(a, st);
      break;
    case GEMM_NT:
      if (k == EPI_DX_ACT) return launch_big128_epi<true, true, EPI_DX_ACT>(a, st);
      if (k == EPI_STORE) return launch_big128_epi<true, true, EPI_STORE>(a, st);
      break;
    case GEMM_TN:
      if (k == EPI_DW_OPT) return launch_big128_epi<false, false, EPI_DW_OPT>(a, st);
      if (k == EPI_STORE) return launch_big128_epi<false, false, EPI_STORE>(a, st);
      break;
  }
  return hipErrorInvalidValue;
}

static hipError_t launch_big(const GemmArgs& a, int layout, hipStream_t st) {
  const int k = a.epi.kind;
  switch (layout) {
    case GEMM_NN:
      if (k == EPI_BIAS_ACT) return launch_big_epi<true, false, EPI_BIAS_ACT>(a, st);
      if (k == EPI_STORE) return launch_big_epi<true, false, EPI_STORE>(a, st);
      break;
    case GEMM_NT:
      if (k == EPI_DX_ACT) return launch_big_epi<true, true, EPI_DX_ACT>(a, st);
      if (k == EPI_STORE) return launch_big_epi<true, true, EPI_STORE>(a, st);
      break;
    case GEMM_TN:
      if (k == EPI_DW_OPT) return launch_big_epi<false, false, EPI_DW_OPT>(a, st);
      if (k == EPI_STORE) return launch_big_epi<false, false, EPI_STORE>(a, st);
      break;
  }
  return hipErrorInvalidValue;
}

hipError_t gemm_launch(const GemmPlan& p, const GemmArgs& args_in, hipStream_t st, Recorder* rec,
                       const char* label, double bytes) {
  GemmArgs a = args_in;
  a.k_per_split = p.k_per_split;
  if (p.splits > 1 && (!a.partial || !a.counters)) return hipErrorInvalidValue;
  if (a.epi.kind == EPI_LOSS && (p.tile == TILE_128x128 || a.N > 64)) return hipErrorInvalidValue;
  if (a.colsum_b && p.layout != GEMM_TN) return hipErrorInvalidValue;
  // the optimizer epilogue indexes W_i with 32-bit element offsets
  if (a.epi.kind == EPI_DW_OPT && (size_t)a.M * a.epi.ldc >= ((size_t)1 << 30)) return hipErrorInvalidValue;
  // The loss head always reduces in-kernel (it needs whole rows).
  const bool ink = p.inkernel_reduce || a.epi.kind == EPI_LOSS;
  hipError_t err;
  if (p.tile == TILE_SMALLM) {
    if (p.splits != 1) return hipErrorInvalidValue;
    if ((err = launch_smallm(a, p.layout, p.vec, p.waves, p.stage, st)) != hipSuccess) return err;
    return mark(rec, label, 2.0 * a.M * a.N * a.K, bytes);
  }
  if (p.tile == TILE_BIG) {
    // exact tiles and 16-byte aligned operands, or no launch
    const bool fits = p.splits == 1 && a.M % kBigBM == 0 && a.N % kBigBM == 0 && a.K % (2 * kBigBK) == 0 &&
                      a.lda % 4 == 0 && a.ldb % 4 == 0 && ((uintptr_t)a.A & 15) == 0 && ((uintptr_t)a.B & 15) == 0;
    if (!fits) return hipErrorInvalidValue;
    if ((err = launch_big(a, p.layout, st)) != hipSuccess) return err;
    return mark(rec, label, 2.0 * a.M * a.N * a.K, bytes);
  }
  if (p.tile == TILE_BIG128) {
    const bool fits = p.splits == 1 && a.M % kB2 == 0 && a.N % kB2 == 0 && a.K % (2 * kB2K) == 0 &&
                      a.lda % 4 == 0 && a.ldb % 4 == 0 && ((uintptr_t)a.A & 15) == 0 && ((uintptr_t)a.B & 15) == 0 &&
                      (size_t)a.M * a.K < ((size_t)1 << 31) && (size_t)a.N * a.K < ((size_t)1 << 31);
    if (!fits) return hipErrorInvalidValue;
    if ((err = launch_big128(a, p.layout, st)) != hipSuccess) return err;
    return mark(rec, label, 2.0 * a.M * a.N * a.K, bytes);
  }
  if (p.tile == TILE_NARROW_TN) {
    // K slices of at most kNarrowTnK rows into the planes, then the reduce
    const bool ok = p.layout == GEMM_TN && a.N >= 1 && a.N <= 16 && p.splits >= 2 && a.partial &&
                    p.k_per_split >= 1 && p.k_per_split <= kNarrowTnK && p.k_per_split % 4 == 0 &&
                    (size_t)(p.splits - 1) * p.k_per_split < (size_t)a.K &&
                    (size_t)p.splits * p.k_per_split >= (size_t)a.K &&
                    (a.epi.kind == EPI_DW_OPT || a.epi.kind == EPI_STORE);
    if (!ok) return hipErrorInvalidValue;
    const dim3 grid((a.M + 63) / 64, p.splits);
    if (a.N <= 1) hipLaunchKernelGGL(narrow_tn_split<1>, grid, dim3(256), 0, st, a);
    else if (a.N <= 4) hipLaunchKernelGGL(narrow_tn_split<4>, grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL(narrow_tn_split<16>, grid, dim3(256), 0, st, a);
    if ((err = hipGetLastError()) != hipSuccess) return err;
    if ((err = mark(rec, label, 2.0 * a.M * a.N * a.K, bytes)) != hipSuccess) return err;
    err = a.epi.kind == EPI_DW_OPT ? launch_reduce<EPI_DW_OPT>(a, p.splits, st) : launch_reduce<EPI_STORE>(a, p.splits, st);
    if (err != hipSuccess) return err;
    const double t = (double)a.M * a.N;
    return mark(rec, std::string(label) + ".splitk_reduce", (double)p.splits * t,
                4.0 * ((double)p.splits * t + 2.0 * t));
  }
  if (p.tile == TILE_DW_SMALLK) {
    if (p.splits != 1 || !dw_smallk_ok(a, p.layout)) return hipErrorInvalidValue;
    const dim3 grid(p.tiles(a.M, a.N));
    if (a.epi.kind == EPI_DW_OPT) hipLaunchKernelGGL(gemm_dw_smallk<EPI_DW_OPT>, grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL(gemm_dw_smallk<EPI_STORE>, grid, dim3(256), 0, st, a);
    if ((err = hipGetLastError()) != hipSuccess) return err;
    return mark(rec, label, 2.0 * a.M * a.N * a.K, bytes);
  }
  if (p.kgroups > 1) {
    // K groups inside the workgroup: every group's slice starts inside K
    const bool ok = p.splits == 1 && a.epi.kind != EPI_LOSS && (p.kgroups == 2 || p.kgroups == 4) &&
                    (p.kgroups == 2 || (p.tile == TILE_64x64 && a.epi.kind != EPI_DW_OPT)) && (size_t)(p.kgroups - 1) * p.k_per_split < (size_t)a.K &&
                    (size_t)p.kgroups * p.k_per_split >= (size_t)a.K && p.k_per_split % 32 == 0;
    if (!ok) return hipErrorInvalidValue;
  }
  switch (p.tile) {
    case TILE_64x64: err = launch_cfg<64, 64, 32, 32, 32>(a, p.layout, p.vec, p.splits, ink, st, p.kgroups); break;
    case TILE_128x128:
      err = launch_cfg<128, 128, 32, 64, 64>(a, p.layout, p.vec, p.splits, ink, st, p.kgroups);
      break;
    case TILE_64x64_K64:
      if (p.kgroups != 1) return hipErrorInvalidValue;
      err = launch_cfg<64, 64, 64, 32, 32>(a, p.layout, p.vec, p.splits, ink, st);
      break;
    default: return hipErrorInvalidValue;
  }
  if (err != hipSuccess) return err;
  err = mark(rec, label, 2.0 * a.M * a.N * a.K, bytes);
  if (err != hipSuccess || p.splits == 1 || ink) return err;
  switch (a.epi.kind) {
    case EPI_STORE: err = launch_reduce<EPI_STORE>(a, p.splits, st); break;
    case EPI_BIAS_ACT: err = launch_reduce<EPI_BIAS_ACT>(a, p.splits, st); break;
    case EPI_DX_ACT: err = launch_reduce<EPI_DX_ACT>(a, p.splits, st); break;
    case EPI_DW_OPT: err = launch_reduce<EPI_DW_OPT>(a, p.splits, st); break;
    default: return hipErrorInvalidValue;
  }
  if (err != hipSuccess) return err;
  const double t = (double)a.M * a.N;
  return mark(rec, std::string(label) + ".splitk_reduce", (double)p.splits * t, 4.0 * ((double)p.splits * t + 2.0 * t));
}

// ---------------------------------------------------------------------------
// Paired launches: blocks [0, na) run operation A, the rest operation B.
// ---------------------------------------------------------------------------
template <int EPI, bool A_KC, bool B_KC>
struct GemmOp64 {  // 64x64 tiles, BK 32, 16-byte rows, split-K by a separate reduction
  using Args = GemmArgs;
  static constexpr int kLa = LdsTile<64, 32, A_KC>::kFloats;
  static constexpr int kLb = LdsTile<64, 32, B_KC>::kFloats;
  static constexpr int kLds = 2 * kLa + 2 * kLb + 64 + 2;
  static __device__ __forceinline__ void run(const GemmArgs& a, int blk, float* lds) {
    const int tiles = ((a.M + 63) / 64) * ((a.N + 63) / 64);
    const int gy = (a.K + a.k_per_split - 1) / a.k_per_split;
    gemm_tile<64, 64, 32, 32, 32, A_KC, B_KC, true, EPI, false>(a, blk % tiles, blk / tiles, gy, lds,
                                                                lds + 2 * kLa, lds + 2 * kLa + 2 * kLb);
  }
};

struct SmallDxOp {  // dX on small-M tiles (16-byte rows), no split
  using Args = GemmArgs;
  static constexpr int kLds = SmallLds<4>::kFloats;
  static __device__ __forceinline__ void run(const GemmArgs& a, int blk, float* lds) {
    smallm_tile<true, true, EPI_DX_ACT, 4>(a, blk, lds);
  }
};

struct DwSmallOp {  // dW on small-K tiles, optimizer epilogue
  using Args = GemmArgs;
  static constexpr int kLds = kDwLds;
  static __device__ __forceinline__ void run(const GemmArgs& a, int blk, float* lds) {
    dw_smallk_tile<EPI_DW_OPT>(a, blk, lds, threadIdx.x);
  }
};

template <int NMAX>
struct NarrowDwOp {  // staged delta in the launch's LDS
  using Args = NarrowDwArgs;
  static constexpr int kLds = 0;
  static __device__ __forceinline__ void run(const NarrowDwArgs& p, int blk, float* lds) {
    narrow_dw_block<NMAX>(p, blk, lds);
  }
};

template <class OA, class OB>
struct PairLds {
  static constexpr int kFloats = OA::kLds > OB::kLds ? OA::kLds : (OB::kLds > 0 ? OB::kLds : 1);
};

// Waves per SIMD a paired launch is compiled for: two in general; five for
// two small-K dW operations (C2's last launch has 1536 workgroups; six
// would need 80 registers and spills).
template <class OA, class OB>
struct PairOccupancy {
  static constexpr int kWaves = 2;
};

template <class OA, class OB>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(PairOccupancy<OA, OB>::kWaves)))
pair_kernel(typename OA::Args a, typename OB::Args b, int na) {
  __shared__ __attribute__((aligned(16))) float lds[PairLds<OA, OB>::kFloats];
  if ((int)blockIdx.x < na) OA::run(a, blockIdx.x, lds);
  else OB::run(b, blockIdx.x - na, lds);
}

template <>
struct PairOccupancy<DwSmallOp, DwSmallOp> {
  static constexpr int kWaves = 5;
};

using DxOp = GemmOp64<EPI_DX_ACT, true, true>;
using DwOp = GemmOp64<EPI_DW_OPT, false, false>;

static int op_blocks(const PairOp& o) {
  if (o.kind == PAIR_GEMM) return o.plan.tiles(o.args.M, o.args.N) * o.plan.splits;
  return (o.nd.R + kNarrowRows - 1) / kNarrowRows;
}

static int op_lds_floats(const PairOp& o) {
  if (o.kind != PAIR_GEMM) return 0;
  if (o.plan.tile == TILE_SMALLM) return SmallDxOp::kLds;
  if (o.plan.tile == TILE_DW_SMALLK) return DwSmallOp::kLds;
  return o.plan.layout == GEMM_NT ? DxOp::kLds : DwOp::kLds;
}

bool pair_supported(const PairOp& a, const PairOp& b) {
  auto gemm_ok = [](const PairOp& o) {
    if (o.plan.tile == TILE_SMALLM)
      return o.plan.vec && o.plan.splits == 1 && o.plan.layout == GEMM_NT && o.args.epi.kind == EPI_DX_ACT &&
             o.plan.waves == 4 && smallm_vec_ok(o.args, GEMM_NT);
    if (o.plan.tile == TILE_DW_SMALLK)
      return o.plan.splits == 1 && o.args.epi.kind == EPI_DW_OPT && dw_smallk_ok(o.args, GEMM_TN);
    // GemmOp64 runs K slice blk / tiles of ceil(K / k_per_split) and the
    // pair launches tiles * splits blocks, so the two must agree: a plan
    // whose slices run as K groups inside one workgroup (kgroups > 1,
    // splits 1) launches on its own.
    const int kps = std::max(o.plan.k_per_split, 1);
    return o.plan.tile == TILE_64x64 && o.plan.vec && !o.plan.inkernel_reduce && o.plan.kgroups == 1 &&
           (o.args.K + kps - 1) / kps == o.plan.splits &&
           ((o.plan.layout == GEMM_NT && o.args.epi.kind == EPI_DX_ACT) ||
            (o.plan.layout == GEMM_TN && o.args.epi.kind == EPI_DW_OPT)) &&
           (o.plan.splits == 1 || o.args.partial) &&
           (o.args.epi.kind != EPI_DW_OPT || (size_t)o.args.M * o.args.epi.ldc < ((size_t)1 << 30));
  };
  auto narrow_ok = [](const PairOp& o) {
    return o.nd.N >= 1 && o.nd.N <= 16 && o.nd.B >= 1 && o.nd.B <= kNarrowMaxB &&
           (o.nd.opt == VOLTA_OPT_SGD || o.nd.opt == VOLTA_OPT_ADAM || o.nd.opt == VOLTA_OPT_ADAGRAD);
  };
  const PairOp* ops[2] = {&a, &b};
  int lds = 0;
  for (const PairOp* o : ops) {
    if (o->kind == PAIR_GEMM && !gemm_ok(*o)) return false;
    if (o->kind == PAIR_NARROW_DW && !narrow_ok(*o)) return false;
    if (o->kind == PAIR_NONE) return false;
    lds = std::max(lds, op_lds_floats(*o));
  }
  // the pairs of the backward order: (dX, dW), (dX, narrow dW), (dW, dW), (narrow dW, dW)
  const bool a_dx = a.kind == PAIR_GEMM && a.plan.layout == GEMM_NT;
  const bool b_dw = b.kind == PAIR_GEMM && b.plan.layout == GEMM_TN;
  if (!((a_dx && (b_dw || b.kind == PAIR_NARROW_DW)) || (!a_dx && b_dw))) return false;
  // tile combinations with a paired kernel (the 64x64 dX beside 64x64 dW
  // or narrow dW; a dW beside a dW of the same tile)
  const bool b_small = b.kind == PAIR_GEMM && b.plan.tile == TILE_DW_SMALLK;
  if (a_dx && a.plan.tile != TILE_SMALLM && b_small) return false;
  if (a.kind == PAIR_GEMM && !a_dx && (a.plan.tile == TILE_DW_SMALLK) != b_small) return false;
  for (const PairOp* o : ops)  // the narrow dW stages its deltas and partial sums in the GEMM's LDS
    if (o->kind == PAIR_NARROW_DW && narrow_lds_floats_n(o->nd.B, o->nd.N) > lds) return false;
  // no split product in the pair may share the other's workspace
  if (a.kind == PAIR_GEMM && b.kind == PAIR_GEMM && a.plan.splits > 1 && b.plan.splits > 1 &&
      a.args.partial == b.args.partial)
    return false;
  return true;
}

template <class OA, class OB>
static hipError_t launch_pair_t(const typename OA::Args& a, int na, const typename OB::Args& b, int nb,
                                hipStream_t st) {
  hipLaunchKernelGGL((pair_kernel<OA, OB>), dim3(na + nb), dim3(256), 0, st, a, b, na);
  return hipGetLastError();
}

template <class OA>
static hipError_t launch_with_narrow(const typename OA::Args& aa, int na, const PairOp& b, hipStream_t st) {
  const int nb = op_blocks(b);
  if (b.nd.N <= 1) return launch_pair_t<OA, NarrowDwOp<1>>(aa, na, b.nd, nb, st);
  if (b.nd.N <= 4) return launch_pair_t<OA, NarrowDwOp<4>>(aa, na, b.nd, nb, st);
  return launch_pair_t<OA, NarrowDwOp<16>>(aa, na, b.nd, nb, st);
}

static hipError_t reduce_after(const PairOp& o, hipStream_t st) {
  if (o.kind != PAIR_GEMM || o.plan.splits == 1) return hipSuccess;
  GemmArgs a = o.args;
  a.k_per_split = o.plan.k_per_split;
  if (o.args.epi.kind == EPI_DX_ACT) return launch_reduce<EPI_DX_ACT>(a, o.plan.splits, st);
  return launch_reduce<EPI_DW_OPT>(a, o.plan.splits, st);
}

// The step's dW products in one launch: workgroups [0, narrow_blocks) run
// the narrow output-layer dW (its staged deltas and partial sums in the
// small-K tile's LDS), the rest the small-K tiles of product i for
// workgroups [start[i], start[i+1]) after them.
static_assert(sizeof(DwGroup) <= 4000, "DwGroup is passed by value as a kernel argument (4 KiB limit)");

// Five waves per SIMD (at most 96 registers) where the narrow part's state
// fits them (NMAX <= 4); the 16-wide narrow dW needs more (at 96 it spilled
// 27 registers), so four.
template <int NMAX, int TN>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NMAX <= 4 ? 5 : 3))) dw_group_kernel(DwGroup d) {
  __shared__ __attribute__((aligned(16))) float lds[TN == kDwT ? kDwLds : (kDwLdsW > kDwLds ? kDwLdsW : kDwLds)];
  int b = blockIdx.x;
  if (b == 0 && threadIdx.x == 0 && d.loss_partials)
    deferred_loss_finish(d.loss_scalars, d.loss_partials, d.loss_blocks, d.loss_denom);
  if (b < d.narrow_blocks) {
    narrow_dw_block<NMAX, true>(d.nd, b, lds);
    return;
  }
  b -= d.narrow_blocks;
  int i = 0;
#pragma unroll
  for (int k = 1; k < kMaxDwGroup; ++k)
    if (k < d.n && b >= d.start[k]) i = k;
  dw_smallk_tile<EPI_DW_OPT, TN>(d.g[i], b - d.start[i], lds, threadIdx.x);
}

int dw_group_tiles(const GemmArgs& a, int tile_n) {
  return ((a.M + kDwT - 1) / kDwT) * ((a.N + tile_n - 1) / tile_n);
}

// The group kernel a launch of `narrow_n` narrow columns and tile width
// `tile_n` runs (as dw_group_launch selects it).
static const void* dw_group_fn(int narrow_n, int tile_n) {
  if (tile_n == kDwTW) {
    if (narrow_n <= 1) return reinterpret_cast<const void*>(&dw_group_kernel<1, kDwTW>);
    if (narrow_n <= 4) return reinterpret_cast<const void*>(&dw_group_kernel<4, kDwTW>);
    return reinterpret_cast<const void*>(&dw_group_kernel<16, kDwTW>);
  }
  if (narrow_n <= 1) return reinterpret_cast<const void*>(&dw_group_kernel<1, kDwT>);
  if (narrow_n <= 4) return reinterpret_cast<const void*>(&dw_group_kernel<4, kDwT>);
  return reinterpret_cast<const void*>(&dw_group_kernel<16, kDwT>);
}

int dw_group_pick_tile_n(const DwGroup& d, int num_cus) {
  const int nn = d.narrow_blocks ? d.nd.N : 1;
  int t32 = d.narrow_blocks, t64 = d.narrow_blocks;
  for (int i = 0; i < d.n; ++i) {
    t32 += dw_group_tiles(d.g[i], kDwT);
    t64 += dw_group_tiles(d.g[i], kDwTW);
  }
  int r32 = 0, r64 = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&r32, dw_group_fn(nn, kDwT), 256, 0) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&r64, dw_group_fn(nn, kDwTW), 256, 0) != hipSuccess ||
      r32 < 1 || r64 < 1) {
    (void)hipGetLastError();
    return kDwT;
  }
  return t32 > r32 * num_cus && t64 <= r64 * num_cus ? kDwTW : kDwT;
}

bool dw_group_supported(const DwGroup& d) {
  if (d.n < 1 || d.n > kMaxDwGroup || d.start[0] != 0) return false;
  if (d.tile_n != kDwT && d.tile_n != kDwTW) return false;
  if (d.loss_partials && (!d.loss_scalars || d.loss_blocks < 1 || d.loss_blocks > kOutDxMaxBlocks)) return false;
  for (int i = 0; i < d.n; ++i) {
    const GemmArgs& a = d.g[i];
    if (a.epi.kind != EPI_DW_OPT || !dw_smallk_ok(a, GEMM_TN)) return false;
    if (d.start[i + 1] - d.start[i] != dw_group_tiles(a, d.tile_n)) return false;
  }
  if (d.narrow_blocks) {
    const NarrowDwArgs& p = d.nd;
    if (p.N < 1 || p.N > 16 || p.B < 1 || p.B > kNarrowMaxB || narrow_lds_floats_n(p.B, p.N) > kDwLds) return false;
    if (p.opt != VOLTA_OPT_SGD && p.opt != VOLTA_OPT_ADAM && p.opt != VOLTA_OPT_ADAGRAD) return false;
    if (d.narrow_blocks != (p.R + kNarrowRows - 1) / kNarrowRows) return false;
  }
  return true;
}

hipError_t dw_group_launch(const DwGroup& d, hipStream_t st, Recorder* rec, const char* label, double flops,
                           double bytes) {
  if (!dw_group_supported(d)) return hipErrorInvalidValue;
  const dim3 grid(d.narrow_blocks + d.start[d.n]);
  const int nn = d.narrow_blocks ? d.nd.N : 1;
  // (the same selection as dw_group_fn)
  if (d.tile_n == kDwTW) {
    if (nn <= 1) hipLaunchKernelGGL((dw_group_kernel<1, kDwTW>), grid, dim3(256), 0, st, d);
    else if (nn <= 4) hipLaunchKernelGGL((dw_group_kernel<4, kDwTW>), grid, dim3(256), 0, st, d);
    else hipLaunchKernelGGL((dw_group_kernel<16, kDwTW>), grid, dim3(256), 0, st, d);
  } else {
    if (nn <= 1) hipLaunchKernelGGL((dw_group_kernel<1, kDwT>), grid, dim3(256), 0, st, d);
    else if (nn <= 4) hipLaunchKernelGGL((dw_group_kernel<4, kDwT>), grid, dim3(256), 0, st, d);
    else hipLaunchKernelGGL((dw_group_kernel<16, kDwT>), grid, dim3(256), 0, st, d);
  }
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  return mark(rec, label, flops, bytes);
}

hipError_t pair_launch(const PairOp& a, const PairOp& b, hipStream_t st, Recorder* rec, const char* label,
                       double flops, double bytes) {
  if (!pair_supported(a, b)) return hipErrorInvalidValue;
  const int na = op_blocks(a), nb = op_blocks(b);
  GemmArgs aa = a.args, bb = b.args;
  aa.k_per_split = a.plan.k_per_split;
  bb.k_per_split = b.plan.k_per_split;

  hipError_t err;
  const bool b_small = b.kind == PAIR_GEMM && b.plan.tile == TILE_DW_SMALLK;
  if (a.kind == PAIR_GEMM && a.plan.layout == GEMM_NT && a.plan.tile == TILE_SMALLM) {
    if (b.kind != PAIR_GEMM) err = launch_with_narrow<SmallDxOp>(aa, na, b, st);
    else if (b_small) err = launch_pair_t<SmallDxOp, DwSmallOp>(aa, na, bb, nb, st);
    else err = launch_pair_t<SmallDxOp, DwOp>(aa, na, bb, nb, st);
  } else if (a.kind == PAIR_GEMM && a.plan.layout == GEMM_NT) {
    err = b.kind == PAIR_GEMM ? launch_pair_t<DxOp, DwOp>(aa, na, bb, nb, st) : launch_with_narrow<DxOp>(aa, na, b, st);
  } else if (a.kind == PAIR_GEMM) {
    err = b_small ? launch_pair_t<DwSmallOp, DwSmallOp>(aa, na, bb, nb, st)
                  : launch_pair_t<DwOp, DwOp>(aa, na, bb, nb, st);
  } else if (b_small) {
    if (a.nd.N <= 1) err = launch_pair_t<NarrowDwOp<1>, DwSmallOp>(a.nd, na, bb, nb, st);
    else if (a.nd.N <= 4) err = launch_pair_t<NarrowDwOp<4>, DwSmallOp>(a.nd, na, bb, nb, st);
    else err = launch_pair_t<NarrowDwOp<16>, DwSmallOp>(a.nd, na, bb, nb, st);
  } else if (a.nd.N <= 1) {
    err = launch_pair_t<NarrowDwOp<1>, DwOp>(a.nd, na, bb, nb, st);
  } else if (a.nd.N <= 4) {
    err = launch_pair_t<NarrowDwOp<4>, DwOp>(a.nd, na, bb, nb, st);
  } else {
    err = launch_pair_t<NarrowDwOp<16>, DwOp>(a.nd, na, bb, nb, st);
  }
  if (err != hipSuccess) return err;
  if ((err = mark(rec, label, flops, bytes)) != hipSuccess) return err;
  for (const PairOp* o : {&a, &b}) {
    if (o->kind != PAIR_GEMM || o->plan.splits == 1) continue;
    if ((err = reduce_after(*o, st)) != hipSuccess) return err;
    const double t = (double)o->args.M * o->args.N;
    if ((err = mark(rec, std::string(label) + ".splitk_reduce", (double)o->plan.splits * t,
                    4.0 * ((double)o->plan.splits * t + 2.0 * t))) != hipSuccess)
      return err;
  }
  return hipSuccess;
}

GemmPlan gemm_plan(int layout, int M, int N, int K, bool vec, int num_cus, bool small_m) {
  GemmPlan p;
  p.layout = layout;
  p.vec = vec;
  // 16-wave small-M launches stage their operands in LDS (smallm_tile's
  // STG); VOLTA_SMALLM_STAGE=0 loads them straight into registers
  const char* sg = std::getenv("VOLTA_SMALLM_STAGE");
  p.stage = !(sg && *sg == '0');
  // 128x128 tiles only where there is enough K to amortise them (a short K,
  // dW at small batch, is epilogue bound and wants the 4x larger grid) and
  // where their grid has a tile per CU (M*N >= 256 * 128^2 = 4M outputs):
  // below that the 64x64 grid needs a quarter of the K split and its reduce
  // reads a quarter of the planes (C4 B=1024, 1024 x 1024 products: 0.280 ->
  // 0.256 ms/step; C5's 4096 x 1024 products keep 128x128, 4.61 against
  // 4.87 ms/step).  VOLTA_TILE128_MIN_MN changes the threshold.
  const char* t128 = std::getenv("VOLTA_TILE128_MIN_MN");
  const size_t mn128 = t128 && *t128 ? (size_t)std::atoll(t128) : (size_t)4096 * 1024;
  p.tile = ((size_t)M * N >= mn128 && M >= 128 && N >= 128 && K > 256) ? TILE_128x128 : TILE_64x64;
  const char* sb = std::getenv("VOLTA_SMALL_BK");
  if (p.tile == TILE_64x64 && sb && std::atoi(sb) == 64) p.tile = TILE_64x64_K64;
  if (big_tile_fits(layout, M, N, K, vec, num_cus)) {
    p.tile = TILE_BIG;
    p.splits = 1;
    p.k_per_split = K;
    return p;
  }
  // The 128x128 direct-to-LDS tile where the 256x256 grid would leave CUs
  // idle but the 128x128 grid has a tile per CU: no split, no reduce launch
  // (C5's 4096 x 1024 and 1024 x 4096 products, which the register-staged
  // 128x128 tile ran split in two plus a reduce).  VOLTA_BIG128=0 turns it
  // off.
  if (big128_tile_fits(layout, M, N, K, vec, num_cus)) {
    p.tile = TILE_BIG128;
    p.splits = 1;
    p.k_per_split = K;
    return p;
  }
  const int tiles = p.tiles(M, N);
  const int bk = p.tile == TILE_64x64_K64 ? 64 : 32;
  // Smallest K slice (VOLTA_SPLITK_MIN_K): 128, and 64 for a forward product
  // with few enough rows for the small-M tile below (a plan that splits K is
  // what sends it there, K >= 128; the loss-head GEMM of those batches too).
  // 64 for every forward product split C4 B=1024's fwd3 (1024 x 256, K =
  // 512, 64 tiles) eight ways instead of four: 0.2398 -> 0.2380 ms/step with
  // 128, the reduce reading half the planes.
  const char* sm = std::getenv("VOLTA_SMALLM_MAX_M");
  const int small_max = sm && *sm ? std::atoi(sm) : 256;
  const char* mk = std::getenv("VOLTA_SPLITK_MIN_K");
  const int min_k =
      mk && *mk ? std::max(32, std::atoi(mk)) : (layout == GEMM_NN && M <= small_max ? 64 : 128);
  const char* ik = std::getenv("VOLTA_SPLITK_INKERNEL");
  p.inkernel_reduce = ik && *ik && *ik != '0';
  const char* sw = std::getenv("VOLTA_SPLITK_WGS_PER_CU");
  const int wgs_per_cu = sw && *sw ? std::max(1, std::atoi(sw)) : 2;
  int splits = 1;
  // Split K while the grid is below ~wgs_per_cu workgroups per CU (two: a
  // second wave per SIMD hides the first one's memory latency) and each
  // slice keeps at least min_k values of k.
  while (tiles * splits * 2 <= wgs_per_cu * num_cus && K / (splits * 2) >= min_k && splits < 32) splits *= 2;
  int kps = (K + splits - 1) / splits;
  kps = ((kps + bk - 1) / bk) * bk;
  splits = (K + kps - 1) / kps;
  p.splits = splits < 1 ? 1 : splits;
  p.k_per_split = kps;
  // A product the 64x64 plan would split over K runs on the small-M tile
  // instead when it has few rows: the reduction over K stays inside each
  // workgroup, which saves the reduce launch (B <= 256 by default;
  // VOLTA_SMALLM_MAX_M changes the limit, 0 turns the tile off).  Measured
  // with the small-K dW tile below: C4 B=256 0.1624 -> 0.1415 ms/step; at
  // B=1024 both tiles are slower than the 64x64 family (0.45 vs 0.30 ms).
  // ... except a dX product (NT) with a long reduction: there the 16x16
  // tiles' operand re-reads from L2 cost more than the split's reduce launch
  // (C3's dX_1, 64 x 2048 x 2048: 18.4 us on the small-M tile against
  // 7.3 + 2.2 us split).  VOLTA_NT_SPLIT_MIN sets the M*K threshold (with
  // K >= 1024); 0 keeps every such product on the small-M tile.
  const char* ns = std::getenv("VOLTA_NT_SPLIT_MIN");
  const long nt_split_min = ns && *ns ? std::atol(ns) : 131072L;
  const bool nt_long = layout == GEMM_NT && nt_split_min > 0 && K >= 1024 && (long)M * K >= nt_split_min;
  if (small_m && (layout == GEMM_NN || layout == GEMM_NT) && p.splits > 1 && M <= small_max && !nt_long) {
    p.tile = TILE_SMALLM;
    p.splits = 1;
    p.k_per_split = K;
    p.waves = smallm_waves(layout == GEMM_NT, ((M + 15) / 16) * ((N + 15) / 16), num_cus);
  }
  // dW with a short reduction (K = B) on 32x32 tiles: more workgroups per
  // CU to overlap the optimizer's streaming and arithmetic (K <= 256 by
  // default; VOLTA_DW_SMALLK_MAX_K changes the limit, 0 turns the tile off).
  const char* dk = std::getenv("VOLTA_DW_SMALLK_MAX_K");
  const int dw_kmax = dk && *dk ? std::atoi(dk) : 256;
  if (layout == GEMM_TN && vec && M % 4 == 0 && N % 4 == 0 && K <= dw_kmax) {
    p.tile = TILE_DW_SMALLK;
    p.splits = 1;
    p.k_per_split = K;
  }
  // A narrow TN product (N <= 16) with a long K: 64 rows of the product per
  // workgroup over K slices (TILE_NARROW_TN) and the reduce launch, instead
  // of 64x64 MFMA tiles that are at least 3/4 padding (the output layer's
  // dW of C4 B=1024 and C5).  VOLTA_NARROW_TN=0 keeps the 64x64 tiles.
  const char* nt = std::getenv("VOLTA_NARROW_TN");
  if (layout == GEMM_TN && N <= 16 && K > 256 && p.tile != TILE_DW_SMALLK && !(nt && *nt == '0')) {
    p.tile = TILE_NARROW_TN;
    p.kgroups = 1;
    p.inkernel_reduce = false;
    narrow_tn_split_plan(M, K, num_cus, &p.k_per_split, &p.splits);  // K > 256: at least 3 slices
  }
  // K groups (gemm_tile's KG): a split of up to 2 slices (4 on the 64x64
  // tile but for dW) runs inside one workgroup instead, the slices on groups
  // of its waves: no partial planes, no reduce launch, the same sums.  By
  // default only for a product on 64x64 tiles split in two whose grid
  // already has a tile per CU, forward or a dX with K >= 1024 (C4 B=1024's
  // fwd0 and fwd1: 17.4 -> 17.3 and 28.5 -> 26.9 us against split + reduce,
  // one launch fewer each; dX_1 alone in 26.1 us where the paired dX_1 |
  // dW_2 launch and its reduces took 47.5 us, dW_2 alone 16.9).  Elsewhere
  // slower: a grid of fewer tiles than CUs then runs on fewer CUs (C4
  // B=1024 dX_3 7.7 -> 9.7 us), four groups meet at every stage's barrier
  // (fwd2 17.8 -> 25.8 us), the dW pairs and a short-K dX pair are faster
  // paired, and 128x128 tiles lose their second workgroup per CU (C5 4.63
  // -> 4.64 ms).  VOLTA_KGROUPS=1 takes them wherever they apply, 0
  // nowhere.  Only where the epilogue is per element (small_m is false for
  // the loss-head product); such a product launches on its own, never in a
  // paired launch.
  const char* kg = std::getenv("VOLTA_KGROUPS");
  const int kg_max = p.tile == TILE_64x64 && layout != GEMM_TN ? 4 : p.tile == TILE_64x64 || p.tile == TILE_128x128 ? 2 : 1;
  const bool kg_auto = !(kg && *kg) && (layout == GEMM_NN || (layout == GEMM_NT && K >= 1024)) &&
                       p.tile == TILE_64x64 && p.splits == 2 && tiles >= num_cus;
  if (((kg && *kg == '1') || kg_auto) && small_m && !p.inkernel_reduce && p.splits > 1 && p.splits <= kg_max) {
    p.kgroups = p.splits;
    p.splits = 1;
  }
  return p;
}

// Bias update from db[n] = sum_b delta[b][n] (:931-933), for steps whose
// dW launches run without the fused column sums (gradient clipping forms db
// from the deltas before they are scaled, :936-955).  A block covers 64
// columns; wave w sums rows b = w, w + 4, ... in batch order (loads unrolled
// eight rows deep), and the four partials are added in wave order.
__global__ void __launch_bounds__(256) bias_update_kernel(EpiArgs e, const float* __restrict__ delta, int B, int N) {
  __shared__ float part[4][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int n = blockIdx.x * 64 + lane;
  const int nn = n < N ? n : N - 1;  // loads stay in bounds; the update is guarded
  float db = 0.0f;
#pragma unroll 8
  for (int b = w; b < B; b += 4) db = db + delta[(size_t)b * N + nn];
  part[w][lane] = db;
  __syncthreads();
  if (w == 0 && n < N)
    apply_bias_update(e, n, N, ((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane], adam_rcp_of(e));
}

hipError_t launch_bias_update(const EpiArgs& e, const float* delta, int B, int N, hipStream_t st) {
  if (!e.b || !e.scalars || !delta || B < 1 || N < 1) return hipErrorInvalidValue;
  // the state apply_bias_update reads: m for Adagrad, m and v for Adam and AdamW
  const bool adam = e.opt == VOLTA_OPT_ADAM || e.opt == VOLTA_OPT_ADAMW;
  if (e.opt != VOLTA_OPT_SGD && (!e.bm || (adam && !e.bv))) return hipErrorInvalidValue;
  hipLaunchKernelGGL(bias_update_kernel, dim3((N + 63) / 64), dim3(256), 0, st, e, delta, B, N);
  return hipGetLastError();
}

}  // namespace volta
