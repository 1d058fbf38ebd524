// fp32 GEMM family on CDNA4 fp32 MFMA (v_mfma_f32_32x32x2_f32), with the
// step's elementwise work fused into the epilogue.
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
// Split-K: blockIdx.z selects a K slice; slices write partial sums to a
// workspace that splitk_reduce adds in slice order (no atomics).
#include "gemm.h"

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
// Epilogues: called once per output element (m < M, n < N) with the fp32
// accumulator.  They are also used by splitk_reduce.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void apply_epilogue(const EpiArgs& e, int m, int n, float acc) {
  const size_t idx = (size_t)m * e.ldc + n;
  switch (e.kind) {
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
    case EPI_SGD: {
      // sgd_fused_tn: W = 1*W + (-lr) * (act_i^T delta_i)  (:321-324)
      const float nlr = -e.scalars->lr;
      e.out[idx] = e.out[idx] + nlr * acc;
      break;
    }
  }
}

template <int BM, int BN, int BK, int WM, int WN, bool A_KC, bool B_KC, bool VEC>
__global__ void __launch_bounds__((BM / WM) * (BN / WN) * 64)
gemm_f32_mfma(GemmArgs args) {
  using T = Tile<BM, BN, BK, WM, WN>;
  constexpr int THREADS = T::kThreads;
  using LA = LdsTile<BM, BK, A_KC>;
  using LB = LdsTile<BN, BK, B_KC>;
  __shared__ __attribute__((aligned(16))) float lds_a[2][LA::kFloats];
  __shared__ __attribute__((aligned(16))) float lds_b[2][LB::kFloats];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / T::kWavesN;
  const int wn = wave % T::kWavesN;
  const int h = lane >> 5;
  const int l32 = lane & 31;

  // Tile coordinates.  blockIdx.x walks N fastest so neighbouring
  // workgroups share the same A rows.
  const int tiles_n = (args.N + BN - 1) / BN;
  const int tm = blockIdx.x / tiles_n;
  const int tn = blockIdx.x % tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;

  const int kbeg = blockIdx.y * args.k_per_split;
  const int kend = min(args.K, kbeg + args.k_per_split);

  TileLoader<BM, BK, A_KC, VEC, THREADS> la;
  TileLoader<BN, BK, B_KC, VEC, THREADS> lb;

  floatx16 acc[T::TM][T::TN];
#pragma unroll
  for (int i = 0; i < T::TM; ++i)
#pragma unroll
    for (int j = 0; j < T::TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  if (kbeg < kend) {
    la.load(args.A, args.lda, args.M, kend, m0, kbeg, tid);
    lb.load(args.B, args.ldb, args.N, kend, n0, kbeg, tid);
    la.store(lds_a[0], tid);
    lb.store(lds_b[0], tid);
    __syncthreads();

    int buf = 0;
    for (int k0 = kbeg; k0 < kend; k0 += BK) {
      const bool more = k0 + BK < kend;
      if (more) {
        la.load(args.A, args.lda, args.M, kend, m0, k0 + BK, tid);
        lb.load(args.B, args.ldb, args.N, kend, n0, k0 + BK, tid);
      }
      const float* a_s = lds_a[buf];
      const float* b_s = lds_b[buf];
#pragma unroll
      for (int g = 0; g < BK / 8; ++g) {
        floatx4 fa[T::TM], fb[T::TN];
#pragma unroll
        for (int i = 0; i < T::TM; ++i)
          fa[i] = load_frag<BM, BK, A_KC>(a_s, wm * WM + i * 32 + l32, h, g);
#pragma unroll
        for (int j = 0; j < T::TN; ++j)
          fb[j] = load_frag<BN, BK, B_KC>(b_s, wn * WN + j * 32 + l32, h, g);
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int i = 0; i < T::TM; ++i)
#pragma unroll
            for (int j = 0; j < T::TN; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i][s], fb[j][s], acc[i][j], 0, 0, 0);
      }
      if (more) {
        la.store(lds_a[buf ^ 1], tid);
        lb.store(lds_b[buf ^ 1], tid);
      }
      __syncthreads();
      buf ^= 1;
    }
  }

  // Epilogue.  Accumulator register v of lane (h, l32) in block (i, j) holds
  // row 8*(v/4) + 4*h + (v%4), column l32 of that 32x32 block.
  EpiArgs e = args.epi;
  if (gridDim.y > 1) {  // split-K partial: plain store into this slice's plane
    e.kind = EPI_STORE;
    e.out = args.partial + (size_t)blockIdx.y * args.M * args.N;
    e.ldc = args.N;
  }
#pragma unroll
  for (int i = 0; i < T::TM; ++i)
#pragma unroll
    for (int j = 0; j < T::TN; ++j) {
      const int n = n0 + wn * WN + j * 32 + l32;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = m0 + wm * WM + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
        if (m < args.M && n < args.N) apply_epilogue(e, m, n, acc[i][j][v]);
      }
    }
}

// Sum the split-K planes in slice order, then apply the real epilogue.
__global__ void __launch_bounds__(256) splitk_reduce(const float* __restrict__ partial, int splits,
                                                     int M, int N, EpiArgs e) {
  const size_t total = (size_t)M * N;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
    float s = partial[idx];
    for (int z = 1; z < splits; ++z) s = s + partial[(size_t)z * total + idx];
    apply_epilogue(e, (int)(idx / N), (int)(idx % N), s);
  }
}

// ---------------------------------------------------------------------------
// Host-side dispatch.
// ---------------------------------------------------------------------------
template <int BM, int BN, int BK, int WM, int WN>
static hipError_t launch_cfg(const GemmArgs& a, int layout, bool vec, int splits, hipStream_t st) {
  using T = Tile<BM, BN, BK, WM, WN>;
  const int tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  dim3 grid(tiles, splits), block(T::kThreads);
#define VOLTA_LAUNCH(AK, BKC, V) \
  hipLaunchKernelGGL((gemm_f32_mfma<BM, BN, BK, WM, WN, AK, BKC, V>), grid, block, 0, st, a)
  switch (layout) {
    case GEMM_NN: if (vec) VOLTA_LAUNCH(true, false, true); else VOLTA_LAUNCH(true, false, false); break;
    case GEMM_NT: if (vec) VOLTA_LAUNCH(true, true, true); else VOLTA_LAUNCH(true, true, false); break;
    case GEMM_TN: if (vec) VOLTA_LAUNCH(false, false, true); else VOLTA_LAUNCH(false, false, false); break;
    default: return hipErrorInvalidValue;
  }
#undef VOLTA_LAUNCH
  return hipGetLastError();
}

hipError_t gemm_launch(const GemmPlan& p, const GemmArgs& args_in, hipStream_t st, Recorder* rec,
                       const char* label, double bytes) {
  GemmArgs a = args_in;
  a.k_per_split = p.k_per_split;
  hipError_t err;
  switch (p.tile) {
    case TILE_64x64: err = launch_cfg<64, 64, 32, 32, 32>(a, p.layout, p.vec, p.splits, st); break;
    case TILE_128x128: err = launch_cfg<128, 128, 32, 64, 64>(a, p.layout, p.vec, p.splits, st); break;
    default: return hipErrorInvalidValue;
  }
  if (err != hipSuccess) return err;
  err = mark(rec, label, 2.0 * a.M * a.N * a.K, bytes);
  if (err != hipSuccess || p.splits == 1) return err;
  const size_t total = (size_t)a.M * a.N;
  int blocks = (int)std::min<size_t>((total + 255) / 256, 4096);
  hipLaunchKernelGGL(splitk_reduce, dim3(blocks), dim3(256), 0, st, a.partial, p.splits, a.M, a.N,
                     a.epi);
  err = hipGetLastError();
  if (err != hipSuccess) return err;
  return mark(rec, std::string(label) + ".splitk_reduce", (double)p.splits * total,
              4.0 * ((double)p.splits * total + 2.0 * total));
}

static int tile_bm(int t) { return t == TILE_64x64 ? 64 : 128; }
static int tile_bn(int t) { return t == TILE_64x64 ? 64 : 128; }

GemmPlan gemm_plan(int layout, int M, int N, int K, bool vec, int num_cus) {
  GemmPlan p;
  p.layout = layout;
  p.vec = vec;
  p.tile = ((size_t)M * N >= (size_t)1024 * 1024 && M >= 128 && N >= 128) ? TILE_128x128 : TILE_64x64;
  const int tiles = ((M + tile_bm(p.tile) - 1) / tile_bm(p.tile)) * ((N + tile_bn(p.tile) - 1) / tile_bn(p.tile));
  const int bk = 32;
  int splits = 1;
  // Split K while the grid is below ~2 workgroups per CU and each slice keeps
  // at least 256 k values.
  while (tiles * splits * 2 <= 2 * num_cus && K / (splits * 2) >= 256 && splits < 32) splits *= 2;
  int kps = (K + splits - 1) / splits;
  kps = ((kps + bk - 1) / bk) * bk;
  splits = (K + kps - 1) / kps;
  p.splits = splits < 1 ? 1 : splits;
  p.k_per_split = kps;
  return p;
}

}  // namespace volta
