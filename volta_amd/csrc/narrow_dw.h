// Device code of the narrow output layer's dW (also run beside a GEMM in
// one launch by gemm.hip).
#pragma once

#include <hip/hip_runtime.h>

#include "device_common.h"
#include "skinny.h"

namespace volta {

// Rows of W a block of kNarrowThreads threads updates, and the LDS floats
// it needs beyond the staged deltas (the waves' partial sums).
constexpr int kNarrowThreads = 256;
constexpr int kNarrowRows = 64;
// Deltas a thread stages at most (B <= kNarrowMaxB, N <= 16).
constexpr int kNarrowStage = kNarrowMaxB * 16 / kNarrowThreads;
template <int NMAX>
struct NarrowLds {
  static constexpr int kPartials = (kNarrowThreads / 64) * NMAX * 64;
};

// Floats of LDS a narrow dW block uses: the B x N deltas (padded to 4), then
// the partial sums.
template <int NMAX>
__host__ __device__ inline int narrow_lds_floats(int B, int N) {
  return (B * N + 3) / 4 * 4 + NarrowLds<NMAX>::kPartials;
}

// The same for the instantiation that serves N columns (NMAX = 1, 4 or 16).
__host__ __device__ inline int narrow_lds_floats_n(int B, int N) {
  return N <= 1 ? narrow_lds_floats<1>(B, N) : N <= 4 ? narrow_lds_floats<4>(B, N) : narrow_lds_floats<16>(B, N);
}

// dW[j][k] = sum_b act[b][j] * delta[b][k] for the kNarrowRows rows j of W
// of this block: lane l of wave q takes row j = block*64 + l and, of every
// 64 batch rows, the 16 rows 16q..16q+15 (ascending; all chunks into one
// partial), and the four waves' partials are added as (P0 + P1) + (P2 + P3)
// by wave 0, which runs the optimizer on W.  Block 0 also forms db[k] =
// sum_b delta[b][k] (:931-933) over four interleaved accumulators (b mod 4)
// added pairwise.  Latency: every global load is unconditional (clamped
// addresses; values outside the batch are never used); the delta staging
// loads go first, so staging waits for them alone, then the activations
// (16 a thread for each of up to four 64-row chunks a round) and wave 0's
// optimizer state; the staged deltas are read from LDS in batches before
// the multiplies, and guards are selects.
// KU (64-row chunks whose loads one round issues together), SB (deltas a
// thread holds while staging them), DBC (the bias column's reads issued
// before their adds) and the batch of staged deltas read before the
// multiplies trade registers for memory latency: the stand-alone launches
// keep the widest settings; the grouped dW launch, whose small-K tiles share
// its register budget, takes the narrow ones (LEAN).
template <int NMAX, bool LEAN = false>
__device__ __forceinline__ void narrow_dw_block(const NarrowDwArgs& p, int block, float* lds) {
  constexpr int kQ = 16;  // batch rows per wave per 64-row chunk
  constexpr int kU = LEAN ? 1 : 4;  // 64-row chunks whose loads one round issues together
  constexpr int kSB = LEAN ? 4 : kNarrowStage;  // deltas per staging batch
  constexpr int kDBatch = LEAN ? (NMAX == 1 ? 8 : NMAX <= 4 ? 4 : 2)
                               : (NMAX == 1 ? 16 : NMAX <= 4 ? 8 : 2);  // batch rows per LDS read batch
  const int B = p.B, N = p.N, R = p.R;
  const int tid = threadIdx.x, lane = tid & 63, q = tid >> 6;
  const int j = block * kNarrowRows + lane;
  const bool own = j < R;
  const int jc = own ? j : 0;
  const bool sgd = p.opt == VOLTA_OPT_SGD, adam = p.opt == VOLTA_OPT_ADAM;
  const int BN = B * N;
  float* sdelta = lds;
  float* part = lds + (BN + 3) / 4 * 4;  // part[(q*NMAX + k)*64 + lane]
  // staged deltas: at most kNarrowStage per thread (B <= kNarrowMaxB, N <=
  // 16), kSB at a time; the first batch's loads go before the activations'
  float dst[kSB];
  auto stage_load = [&](int i0) {
#pragma unroll
    for (int i = 0; i < kSB; ++i) {
      if ((i0 + i) * kNarrowThreads >= BN) break;  // block-uniform
      dst[i] = p.delta[min(tid + (i0 + i) * kNarrowThreads, BN - 1)];
    }
  };
  auto stage_store = [&](int i0) {
#pragma unroll
    for (int i = 0; i < kSB; ++i) {
      if ((i0 + i) * kNarrowThreads >= BN) break;
      if (tid + (i0 + i) * kNarrowThreads < BN) sdelta[tid + (i0 + i) * kNarrowThreads] = dst[i];
    }
  };
  stage_load(0);
  // activations of a round: chunk u holds batch rows b0 + 64u + 16q + c
  float a[kU][kQ];
  auto load_round = [&](int b0) {
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      if (b0 + 64 * u >= B) break;  // wave-uniform
#pragma unroll
      for (int c = 0; c < kQ; ++c) a[u][c] = p.act[(size_t)min(b0 + 64 * u + kQ * q + c, B - 1) * R + jc];
    }
  };
  load_round(0);
  float w[NMAX], s1[NMAX], s2[NMAX];
  const float* pm = sgd ? p.w : p.m;
  const float* pv = adam ? p.v : p.w;
#pragma unroll
  for (int k = 0; k < NMAX; ++k) {
    const size_t idx = (size_t)jc * N + min(k, N - 1);
    w[k] = p.w[idx];
    s1[k] = pm[idx];
    s2[k] = pv[idx];
  }
  // bias state (block 0, threads k < N; no bias work when p.b is null)
  const bool bown = block == 0 && tid < N && p.b;
  const int kb = min(tid, N - 1);
  const float* pb = p.b ? p.b : p.w;
  const float bw = pb[kb];
  const float bs1 = (sgd || !p.b ? pb : p.bm)[kb];
  const float bs2 = (adam && p.b ? p.bv : pb)[kb];
  const float lr = p.scalars->lr;
  const AdamRcp rc = adam_rcp(p.scalars->bc1, p.scalars->bc2);
  stage_store(0);
  for (int i0 = kSB; i0 < kNarrowStage && i0 * kNarrowThreads < BN; i0 += kSB) {
    stage_load(i0);
    stage_store(i0);
  }
  __syncthreads();

  float acc[NMAX];
#pragma unroll
  for (int k = 0; k < NMAX; ++k) acc[k] = 0.0f;
  for (int r0 = 0; r0 < B; r0 += 64 * kU) {
    if (r0 > 0) load_round(r0);
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int b0 = r0 + 64 * u;
      if (b0 >= B) break;  // wave-uniform
#pragma unroll
      for (int c0 = 0; c0 < kQ; c0 += kDBatch) {
        float d[kDBatch][NMAX];
#pragma unroll
        for (int c = 0; c < kDBatch; ++c)
#pragma unroll
          for (int k = 0; k < NMAX; ++k) d[c][k] = sdelta[min(b0 + kQ * q + c0 + c, B - 1) * N + min(k, N - 1)];
#pragma unroll
        for (int c = 0; c < kDBatch; ++c) {
          const bool in = b0 + kQ * q + c0 + c < B;
#pragma unroll
          for (int k = 0; k < NMAX; ++k) {
            const float t = acc[k] + a[u][c0 + c] * d[c][k];
            acc[k] = in && k < N ? t : acc[k];
          }
        }
      }
    }
  }
#pragma unroll
  for (int k = 0; k < NMAX; ++k) part[(q * NMAX + k) * 64 + lane] = acc[k];
  __syncthreads();
  if (q != 0) return;
#pragma unroll
  for (int k = 0; k < NMAX; ++k) {
    const float* pk = part + k * 64 + lane;
    acc[k] = (pk[0] + pk[NMAX * 64]) + (pk[2 * NMAX * 64] + pk[3 * NMAX * 64]);
  }
  if (own) {
    const int64_t count = (int64_t)R * N;
    const int64_t vec_end = count - count % 8;
    // columns k >= N are skipped by a guard, not a break: a loop with a
    // data-dependent exit around this body was left rolled (the registers
    // then indexed at run time, in scratch memory)
#pragma unroll
    for (int k = 0; k < NMAX; ++k) {
      if (k >= N) continue;
      const int64_t idx = (int64_t)j * N + k;
      if (sgd) {
        const float nlr = -lr;
        w[k] = w[k] + nlr * acc[k];
      } else if (p.opt == VOLTA_OPT_ADAGRAD) {
        adagrad_elem(&w[k], &s1[k], acc[k], lr, p.eps);
      } else {
        adam_elem(&w[k], &s1[k], &s2[k], acc[k], idx >= vec_end, lr, rc, p.b1, p.b2, p.eps, p.wd);
      }
    }
#pragma unroll
    for (int k = 0; k < NMAX; ++k) {
      if (k >= N) continue;
      const size_t idx = (size_t)j * N + k;
      if (p.grad) p.grad[idx] = acc[k];
      p.w[idx] = w[k];
      if (!sgd) p.m[idx] = s1[k];
      if (adam) p.v[idx] = s2[k];
    }
  }
  if (bown) {
    const int k = threadIdx.x;
    // four interleaved accumulators; each chunk's reads are issued before
    // its first add
    constexpr int kDbChunk = LEAN ? 16 : 64;
    float dba[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int b0 = 0; b0 < B; b0 += kDbChunk) {
      float d[kDbChunk];
#pragma unroll
      for (int c = 0; c < kDbChunk; ++c) d[c] = sdelta[min(b0 + c, B - 1) * N + k];
#pragma unroll
      for (int c = 0; c < kDbChunk; ++c) {
        const float t = dba[c & 3] + d[c];
        dba[c & 3] = b0 + c < B ? t : dba[c & 3];
      }
    }
    const float db = (dba[0] + dba[1]) + (dba[2] + dba[3]);
    if (p.bgrad) p.bgrad[k] = db;
    float x = bw, y1 = bs1, y2 = bs2;
    if (sgd) {
      x = x - lr * db;
    } else if (p.opt == VOLTA_OPT_ADAGRAD) {
      adagrad_elem(&x, &y1, db, lr, p.eps);
    } else {
      adam_elem(&x, &y1, &y2, db, k >= N - N % 8, lr, rc, p.b1, p.b2, p.eps, 0.0f);
    }
    p.b[k] = x;
    if (!sgd) p.bm[k] = y1;
    if (adam) p.bv[k] = y2;
  }
}

}  // namespace volta
