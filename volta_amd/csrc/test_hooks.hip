// Kernel-level entry points for the GPU tests: run one GEMM of the family on
// device pointers, synchronously, so its numerics can be checked in
// isolation.  Not part of the reference ABI.
#include <hip/hip_runtime.h>

#include "gemm.h"
#include "spec.h"

extern "C" {

// C[M x N] = op(A) op(B) for layout GEMM_NN / GEMM_NT / GEMM_TN (see gemm.h).
// force_tile < 0 and force_splits <= 0 select the runtime's own plan.
int32_t volta_hip_gemm(int32_t layout, const float* A, const float* B, float* Cm, int32_t M, int32_t N,
                       int32_t K, int32_t force_tile, int32_t force_splits) {
  using namespace volta;
  if (layout < GEMM_NN || layout > GEMM_TN || M <= 0 || N <= 0 || K <= 0 || !A || !B || !Cm) {
    set_last_error("volta_hip_gemm: bad arguments");
    return -1;
  }
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
    set_last_error("volta_hip_gemm: no device");
    return -1;
  }
  // Leading dimensions follow from the layout (dense row-major operands).
  const int lda = layout == GEMM_TN ? M : K;
  const int ldb = layout == GEMM_NT ? K : N;
  const int contig_a = layout == GEMM_TN ? M : K;
  const int contig_b = layout == GEMM_NT ? K : N;
  const bool vec = contig_a % 4 == 0 && contig_b % 4 == 0;
  GemmPlan p = gemm_plan(layout, M, N, K, vec, cus);
  if (force_tile > TILE_128x128) {
    set_last_error("volta_hip_gemm: unknown tile");
    return -1;
  }
  if (force_tile >= 0) p.tile = force_tile;
  if (force_splits > 0) {
    int kps = (K + force_splits - 1) / force_splits;
    kps = (kps + 31) / 32 * 32;
    p.k_per_split = kps;
    p.splits = (K + kps - 1) / kps;
  }
  float* ws = nullptr;
  if (p.splits > 1 && hipMalloc((void**)&ws, p.workspace_floats(M, N) * sizeof(float)) != hipSuccess) {
    set_last_error("volta_hip_gemm: workspace allocation failed");
    return -1;
  }
  GemmArgs a{};
  a.A = A;
  a.B = B;
  a.lda = lda;
  a.ldb = ldb;
  a.M = M;
  a.N = N;
  a.K = K;
  a.partial = ws;
  a.epi.kind = EPI_STORE;
  a.epi.ldc = N;
  a.epi.out = Cm;
  hipError_t e = gemm_launch(p, a, nullptr);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (ws) hipFree(ws);
  if (e != hipSuccess) {
    set_last_error(std::string("volta_hip_gemm: ") + hipGetErrorString(e));
    return -1;
  }
  return 0;
}

}  // extern "C"
