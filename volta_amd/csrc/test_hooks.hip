// Kernel-level entry points for the GPU tests: run one GEMM of the family on
// device pointers, synchronously, so its numerics can be checked in
// isolation.  Not part of the reference ABI.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "gemm.h"
#include "spec.h"
#include "step_kernels.h"

namespace {
// Plain 16-byte copy: the reference kernel for scaling HBM counters
// (FETCH_SIZE / WRITE_SIZE read for a known number of bytes).
__global__ void __launch_bounds__(256) calibration_copy_kernel(const float4* __restrict__ src,
                                                               float4* __restrict__ dst, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}
}  // namespace

extern "C" {

// Copy `bytes` (a multiple of 16) from src to dst with calibration_copy_kernel,
// `reps` times, synchronously.  Used to scale HBM counter readings.
int32_t volta_hip_calibration_copy(void* dst, const void* src, int64_t bytes, int32_t reps) {
  if (!dst || !src || bytes <= 0 || bytes % 16 != 0 || reps <= 0) return -1;
  const size_t n = (size_t)bytes / 16;
  const int blocks = (int)std::min<size_t>((n + 255) / 256, 8192);
  for (int r = 0; r < reps; ++r)
    hipLaunchKernelGGL(calibration_copy_kernel, dim3(blocks), dim3(256), 0, 0, static_cast<const float4*>(src),
                       static_cast<float4*>(dst), n);
  return hipGetLastError() == hipSuccess && hipDeviceSynchronize() == hipSuccess ? 0 : -1;
}

// C[M x N] = op(A) op(B) for layout GEMM_NN / GEMM_NT / GEMM_TN (see gemm.h).
// force_tile < 0 and force_splits == 0 select the runtime's own plan;
// force_splits > 0 splits K over that many launch slices (reduced by a
// second kernel), force_splits = -G over G groups of one workgroup's waves.
// The planner's choice for one product (gemm_plan; host code only, no
// device call): out[0..5] = tile (GemmTile), splits, k_per_split, kgroups,
// waves, vec.  `small_m` as the step passes it (0 for the loss-head
// product).  Test use.
int32_t volta_hip_gemm_plan(int32_t layout, int32_t M, int32_t N, int32_t K, int32_t vec, int32_t num_cus,
                            int32_t small_m, int32_t* out) {
  using namespace volta;
  if (layout < GEMM_NN || layout > GEMM_TN || M <= 0 || N <= 0 || K <= 0 || num_cus <= 0 || !out) {
    set_last_error("volta_hip_gemm_plan: bad arguments");
    return -1;
  }
  const GemmPlan p = gemm_plan(layout, M, N, K, vec != 0, num_cus, small_m != 0);
  out[0] = p.tile;
  out[1] = p.splits;
  out[2] = p.k_per_split;
  out[3] = p.kgroups;
  out[4] = p.waves;
  out[5] = p.vec ? 1 : 0;
  return 0;
}

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
  if (force_tile > TILE_NARROW_TN) {
    set_last_error("volta_hip_gemm: unknown tile");
    return -1;
  }
  if (force_tile >= 0 && force_tile != p.tile) {
    // the plan's K groups (if any) become split launches on another tile
    p.tile = force_tile;
    p.splits *= p.kgroups;
    p.kgroups = 1;
  }
  const char* sw = std::getenv("VOLTA_SMALLM_WAVES");
  if (p.tile == TILE_SMALLM && p.waves == 0) {  // forced onto a shape planned otherwise
    p.waves = layout == GEMM_NT || (sw && std::atoi(sw) == 4) ? 4 : (sw && std::atoi(sw) == 16) ? 16 : 8;
  }
  // a dX product as the small-batch step runs it (16 waves) on request
  if (p.tile == TILE_SMALLM && layout == GEMM_NT && sw && std::atoi(sw) == 16) p.waves = 16;
  if (force_tile == TILE_SMALLM || force_tile == TILE_DW_SMALLK || force_tile == TILE_BIG ||
      force_tile == TILE_BIG128) {  // whole K in each workgroup
    p.splits = 1;
    p.k_per_split = K;
  }
  if (force_tile == TILE_NARROW_TN) narrow_tn_split_plan(M, K, cus, &p.k_per_split, &p.splits);
  if (force_splits != 0) {
    const int g = force_splits > 0 ? force_splits : -force_splits;
    int kps = (K + g - 1) / g;
    kps = (kps + 31) / 32 * 32;
    p.k_per_split = kps;
    p.splits = force_splits > 0 ? (K + kps - 1) / kps : 1;
    p.kgroups = force_splits > 0 ? 1 : (K + kps - 1) / kps;
  }
  float* ws = nullptr;
  unsigned* counters = nullptr;
  if (p.splits > 1) {
    const size_t cbytes = (size_t)p.tiles(M, N) * sizeof(unsigned);
    if (hipMalloc((void**)&ws, p.workspace_floats(M, N) * sizeof(float)) != hipSuccess ||
        hipMalloc((void**)&counters, cbytes) != hipSuccess || hipMemset(counters, 0, cbytes) != hipSuccess) {
      if (ws) (void)hipFree(ws);
      if (counters) (void)hipFree(counters);
      set_last_error("volta_hip_gemm: workspace allocation failed");
      return -1;
    }
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
  a.counters = counters;
  a.epi.kind = EPI_STORE;
  a.epi.ldc = N;
  a.epi.out = Cm;
  hipError_t e = gemm_launch(p, a, nullptr);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (ws) (void)hipFree(ws);
  if (counters) (void)hipFree(counters);
  if (e != hipSuccess) {
    set_last_error(std::string("volta_hip_gemm: ") + hipGetErrorString(e));
    return -1;
  }
  return 0;
}

// Device memory for tests, so they need no second GPU runtime in-process.
void* volta_hip_device_alloc(int64_t bytes) {
  void* p = nullptr;
  if (bytes <= 0 || hipMalloc(&p, (size_t)bytes) != hipSuccess) return nullptr;
  return p;
}

int32_t volta_hip_device_free(void* p) { return hipFree(p) == hipSuccess ? 0 : -1; }

// kind: 1 host->device, 2 device->host, 3 device->device.  Synchronous.
int32_t volta_hip_copy(void* dst, const void* src, int64_t bytes, int32_t kind) {
  const hipMemcpyKind k = kind == 1 ? hipMemcpyHostToDevice
                          : kind == 2 ? hipMemcpyDeviceToHost
                                      : hipMemcpyDeviceToDevice;
  if (bytes < 0 || kind < 1 || kind > 3) return -1;
  return hipMemcpy(dst, src, (size_t)bytes, k) == hipSuccess ? 0 : -1;
}

// One optimizer pass over a single buffer of `count` floats, as the step
// runs it for one parameter segment.  kind: VOLTA_OPT_ADAM (AdamW when
// wd != 0) or VOLTA_OPT_ADAGRAD (then v is unused and m holds G).
int32_t volta_hip_optimizer(int32_t kind, float* w, float* m, float* v, const float* g, int64_t count,
                            float lr, float bc1, float bc2, float b1, float b2, float eps, float wd) {
  using namespace volta;
  if (count <= 0 || !w || !m || !g || (kind == VOLTA_OPT_ADAM && !v) ||
      (kind != VOLTA_OPT_ADAM && kind != VOLTA_OPT_ADAGRAD)) {
    set_last_error("volta_hip_optimizer: bad arguments");
    return -1;
  }
  // The kernels walk whole kSegAlign blocks; stage through padded buffers.
  const int64_t padded = (count + kSegAlign - 1) / kSegAlign * kSegAlign;
  float* buf = nullptr;
  DevScalars* sc = nullptr;
  const size_t bytes = (size_t)padded * 4;
  if (hipMalloc((void**)&buf, 4 * bytes) != hipSuccess) return -1;
  if (hipMalloc((void**)&sc, sizeof(DevScalars)) != hipSuccess) {
    (void)hipFree(buf);
    return -1;
  }
  float *dw = buf, *dm = buf + padded, *dv = buf + 2 * padded, *dg = buf + 3 * padded;
  DevScalars hs{};
  hs.lr = lr;
  hs.bc1 = bc1;
  hs.bc2 = bc2;
  SegTable segs{};
  segs.n = 1;
  segs.off[0] = 0;
  segs.count[0] = count;
  segs.wd[0] = wd;
  hipError_t e = hipMemset(buf, 0, 4 * bytes);
  if (e == hipSuccess) e = hipMemcpy(sc, &hs, sizeof hs, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(dw, w, count * 4, hipMemcpyDeviceToDevice);
  if (e == hipSuccess) e = hipMemcpy(dm, m, count * 4, hipMemcpyDeviceToDevice);
  if (e == hipSuccess && v) e = hipMemcpy(dv, v, count * 4, hipMemcpyDeviceToDevice);
  if (e == hipSuccess) e = hipMemcpy(dg, g, count * 4, hipMemcpyDeviceToDevice);
  if (e == hipSuccess)
    e = kind == VOLTA_OPT_ADAM ? launch_adam(dw, dm, dv, dg, segs, padded, sc, b1, b2, eps, nullptr)
                               : launch_adagrad(dw, dm, dg, segs, padded, sc, eps, nullptr);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e == hipSuccess) e = hipMemcpy(w, dw, count * 4, hipMemcpyDeviceToDevice);
  if (e == hipSuccess) e = hipMemcpy(m, dm, count * 4, hipMemcpyDeviceToDevice);
  if (e == hipSuccess && v) e = hipMemcpy(v, dv, count * 4, hipMemcpyDeviceToDevice);
  (void)hipFree(buf);
  (void)hipFree(sc);
  if (e != hipSuccess) {
    set_last_error(std::string("volta_hip_optimizer: ") + hipGetErrorString(e));
    return -1;
  }
  return 0;
}

}  // extern "C"
