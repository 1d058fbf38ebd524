// Codegen extras of the generated step (LayerNorm, dropout, gradient
// clipping; mlp_train_rust_codegen.rs:745-788, :829-892, :936-955), as
// kernels around the GEMMs (extras.hip).
#pragma once

#include <hip/hip_runtime.h>

#include "device_common.h"

namespace volta {

// One hidden layer's forward extras on act [B x c] (after the activation;
// with `softmax` act holds the pre-activation and the row softmax comes
// first).
struct HiddenFwdArgs {
  float* act;            // [B x c], updated in place
  int B, c;
  int softmax;           // 1: act = softmax(act) per row first
  const float* gamma;    // LayerNorm (null: off)
  const float* beta;
  float* mu;             // [B] per-row statistics kept for the backward
  float* inv_std;        // [B] (both null: not kept, inference)
  uint8_t* mask;         // dropout (null: off) [B x c]
  float p, keep_scale;
  uint64_t rng_offset;   // draws before this layer's first element in the step
  const DevScalars* scalars;  // rng = the step's starting state
};

// One hidden layer's backward extras on delta [B x c] (gradient w.r.t. the
// layer's final output): LayerNorm backward, dropout mask, activation
// derivative (softmax: the row form y * (d - dot(d, y))), in that order.
struct HiddenBwdArgs {
  float* delta;          // [B x c], updated in place
  const float* act;      // layer output (after LayerNorm / dropout)
  const float* pre;      // pre-activation
  int B, c, act_kind;
  const float* gamma;    // LayerNorm (null: off), pre-update values
  const float* beta;
  const float* inv_std;
  float* dgamma;         // [c] column sums (written by ln_bwd_cols)
  float* dbeta;
  const uint8_t* mask;   // dropout (null: off)
  float keep_scale;
};

hipError_t launch_hidden_fwd(const HiddenFwdArgs& a, hipStream_t st);
// LayerNorm backward: gamma/beta gradients (columns), then the row pass
// (with dropout mask and activation derivative), then gamma/beta -= lr * grad.
hipError_t launch_hidden_bwd(const HiddenBwdArgs& a, float* gamma, float* beta, const DevScalars* scalars,
                             hipStream_t st);
// Advance the step's dropout state by `draws` (after the forward).
hipError_t launch_rng_advance(DevScalars* scalars, uint64_t draws, hipStream_t st);

// Gradient clipping over every layer's delta (up to 16 buffers): the global
// norm, scale = clip/norm when the norm exceeds clip (else 1, kept in
// scalars->clip_scale), then every delta multiplied by scale in place.
struct ClipArgs {
  int n;
  float* delta[16];
  int64_t count[16];
  float clip;
  float* partials;       // [kClipBlocks]
  DevScalars* scalars;   // receives clip_scale
};
constexpr int kClipBlocks = 256;
hipError_t launch_clip(const ClipArgs& a, hipStream_t st);

}  // namespace volta
