// Device code of the narrow output layer's dW (also run beside a GEMM in
// one launch by gemm.hip).
#pragma once

#include <hip/hip_runtime.h>

#include "device_common.h"
#include "skinny.h"

namespace volta {

// dW[j][k] = sum_b act[b][j] * delta[b][k] (b ascending, as sgemm_tn sums),
// one thread per row j of W (rows block*blockDim.x + threadIdx.x); delta is
// staged in LDS.  Block 0 also forms db[k] = sum_b
// delta[b][k] (:931-933).  Then the optimizer update of W and b (same
// element functions as the MFMA path).  Latency: the optimizer state, the
// scalars and the first chunk of act are loaded before the LDS staging
// barrier, and act is read in chunks of kChunk rows whose loads are all
// issued before the chunk's first multiply.
template <int NMAX>
__device__ __forceinline__ void narrow_dw_block(const NarrowDwArgs& p, int block, float* sdelta /* [B x N] */) {
  constexpr int kChunk = 64;
  const int B = p.B, N = p.N, R = p.R;
  const int j = block * blockDim.x + threadIdx.x;
  const bool own = j < R;
  const bool sgd = p.opt == VOLTA_OPT_SGD, adam = p.opt == VOLTA_OPT_ADAM;
  const float lr = p.scalars->lr;
  const AdamRcp rc = adam_rcp(p.scalars->bc1, p.scalars->bc2);
  float w[NMAX], s1[NMAX], s2[NMAX];
#pragma unroll
  for (int k = 0; k < NMAX; ++k) {
    const size_t idx = (size_t)j * N + k;
    const bool ok = own && k < N;
    w[k] = ok ? p.w[idx] : 0.0f;
    s1[k] = ok && !sgd ? p.m[idx] : 0.0f;
    s2[k] = ok && adam ? p.v[idx] : 0.0f;
  }
  // bias state (block 0, threads k < N; no bias work when p.b is null)
  const bool bown = block == 0 && (int)threadIdx.x < N && p.b;
  const float bw = bown ? p.b[threadIdx.x] : 0.0f;
  const float bs1 = bown && !sgd ? p.bm[threadIdx.x] : 0.0f;
  const float bs2 = bown && adam ? p.bv[threadIdx.x] : 0.0f;
  float a[kChunk];
#pragma unroll
  for (int c = 0; c < kChunk; ++c) a[c] = own && c < B ? p.act[(size_t)c * R + j] : 0.0f;
  for (int i = threadIdx.x; i < B * N; i += blockDim.x) sdelta[i] = p.delta[i];
  __syncthreads();

  float acc[NMAX];
#pragma unroll
  for (int k = 0; k < NMAX; ++k) acc[k] = 0.0f;
  for (int b0 = 0; b0 < B; b0 += kChunk) {
    if (b0 > 0) {
#pragma unroll
      for (int c = 0; c < kChunk; ++c) a[c] = own && b0 + c < B ? p.act[(size_t)(b0 + c) * R + j] : 0.0f;
    }
#pragma unroll
    for (int c = 0; c < kChunk; ++c) {
      if (b0 + c < B) {
#pragma unroll
        for (int k = 0; k < NMAX; ++k)
          if (k < N) acc[k] = acc[k] + a[c] * sdelta[(b0 + c) * N + k];
      }
    }
  }
  if (own) {
    const int64_t count = (int64_t)R * N;
    const int64_t vec_end = count - count % 8;
#pragma unroll
    for (int k = 0; k < NMAX; ++k) {
      if (k >= N) break;
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
      if (k >= N) break;
      const size_t idx = (size_t)j * N + k;
      if (p.grad) p.grad[idx] = acc[k];
      p.w[idx] = w[k];
      if (!sgd) p.m[idx] = s1[k];
      if (adam) p.v[idx] = s2[k];
    }
  }
  if (bown) {
    const int k = threadIdx.x;
    float db = 0.0f;
    for (int b = 0; b < B; ++b) db = db + sdelta[b * N + k];
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
