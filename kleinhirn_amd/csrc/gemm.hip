// C = act(A W^T + bias) on CDNA4 matrix cores.
//
// Both operands are K-contiguous (activations [M, K] row-major, weights PyTorch [N, K] never
// transposed), which is the layout MFMA fragments want: lane l of a 32x32 tile reads 8 (f16) or 1
// (f32) consecutive k values of row l % 32. A 256-thread block (4 wavefronts, 2 x 2) computes a
// 128 x 128 tile; each wavefront holds a 64 x 64 sub-tile as 2 x 2 accumulators of
// v_mfma_f32_32x32x16_f16 (f16 storage) or v_mfma_f32_32x32x2f32 (f32 storage). The K loop stages
// 128-byte-wide slabs of A and W through LDS (rows padded by 16 bytes, so the 16-byte fragment
// reads of 8 consecutive rows hit distinct banks) with a register prefetch of the next slab.
// f32 accumulation; bias and activation are applied to the finished sum, as in the reference
// (src/wasm/plan.ts:126-154), then rounded once to the storage type.
//
// A second kernel computes small or unaligned products (head steps with a handful of output
// classes) with one wavefront per (row, 4 columns).
#include "kernels.h"
#include "device.h"

namespace kh {

namespace {

constexpr int BM = 128, BN = 128, NT = 256;

template <typename T>
struct Mfma;

template <>
struct Mfma<half_t> {
  static constexpr int BK = 64;      // k per LDS slab
  static constexpr int KSTEP = 16;   // k per MFMA
  static constexpr int KLANE = 8;    // k values per lane per MFMA
  static constexpr int LDK = BK + 8; // padded LDS row (halves)
  typedef half8v frag;
  __device__ static frag load(const half_t *p) { return *reinterpret_cast<const half8v *>(p); }
  __device__ static float16v mma(frag a, frag b, float16v c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mfma<float> {
  static constexpr int BK = 32;
  static constexpr int KSTEP = 2;
  static constexpr int KLANE = 1;
  static constexpr int LDK = BK + 4;
  typedef float frag;
  __device__ static frag load(const float *p) { return *p; }
  __device__ static float16v mma(frag a, frag b, float16v c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
};

// 16-byte chunk of a row
template <typename T>
struct Chunk {
  static constexpr int ELEMS = 16 / sizeof(T);
  typedef half8v vec_h;
  typedef float4v vec_f;
};

template <typename T>
__global__ void __launch_bounds__(NT, 2) gemm_mfma_kernel(GemmArgs g, int tiles_n) {
  typedef Mfma<T> MF;
  constexpr int BK = MF::BK, LDK = MF::LDK, CE = Chunk<T>::ELEMS;
  constexpr int CPR = BK / CE;             // 16-byte chunks per slab row (8)
  constexpr int LOADS = BM * CPR / NT;     // chunks per thread per operand (4)
  __shared__ __attribute__((aligned(16))) T sA[BM * LDK];
  __shared__ __attribute__((aligned(16))) T sB[BN * LDK];

  const int z = blockIdx.z;
  const T *A = (const T *)g.a + (int64_t)z * g.a_bs;
  const T *W = (const T *)g.w + (int64_t)z * g.w_bs;

  // tile order: consecutive blocks share the A row block (n fastest)
  const int tile = blockIdx.x;
  const int m0 = (tile / tiles_n) * BM;
  const int n0 = (tile % tiles_n) * BN;

  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int crow = t / CPR, ccol = (t % CPR) * CE;  // chunk row (+32 i) and column

  typedef uint4 raw;  // 16 bytes
  raw ra[LOADS], rb[LOADS];

  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < LOADS; i++) {
      int r = crow + i * (NT / CPR);
      int kk = k0 + ccol;
      int am = m0 + r < g.M ? m0 + r : g.M - 1;
      int bn = n0 + r < g.N ? n0 + r : g.N - 1;
      if (kk < g.K) {
        ra[i] = *reinterpret_cast<const raw *>(A + (int64_t)am * g.lda + kk);
        rb[i] = *reinterpret_cast<const raw *>(W + (int64_t)bn * g.ldw + kk);
      } else {
        ra[i] = make_uint4(0, 0, 0, 0);
        rb[i] = make_uint4(0, 0, 0, 0);
      }
    }
  };
  auto sstore = [&]() {
#pragma unroll
    for (int i = 0; i < LOADS; i++) {
      int r = crow + i * (NT / CPR);
      *reinterpret_cast<raw *>(&sA[r * LDK + ccol]) = ra[i];
      *reinterpret_cast<raw *>(&sB[r * LDK + ccol]) = rb[i];
    }
  };

  float16v acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

  const int arow = wm * 64 + (lane & 31);
  const int brow = wn * 64 + (lane & 31);
  const int kl = (lane >> 5) * MF::KLANE;

  gload(0);
  sstore();
  __syncthreads();
  for (int k0 = 0; k0 < g.K; k0 += BK) {
    const bool more = k0 + BK < g.K;
    if (more) gload(k0 + BK);
#pragma unroll
    for (int kk = 0; kk < BK; kk += MF::KSTEP) {
      typename MF::frag af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; i++) af[i] = MF::load(&sA[(arow + i * 32) * LDK + kk + kl]);
#pragma unroll
      for (int j = 0; j < 2; j++) bf[j] = MF::load(&sB[(brow + j * 32) * LDK + kk + kl]);
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = MF::mma(af[i], bf[j], acc[i][j]);
    }
    __syncthreads();
    if (more) {
      sstore();
      __syncthreads();
    }
  }

  // epilogue: lane l holds column l % 32 and rows 8 (r / 4) + 4 (l / 32) + r % 4 of each 32 x 32
  const T *bias = (const T *)g.bias;
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int col = n0 + wn * 64 + j * 32 + (lane & 31);
    if (col >= g.N) continue;
    const float bv = bias ? (float)bias[col] : 0.f;
#pragma unroll
    for (int i = 0; i < 2; i++) {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row >= g.M) continue;
        const float v = activate(acc[i][j][r] + bv, g.act);
        if (g.c_f32)
          ((float *)g.c)[(int64_t)z * g.c_bs + (int64_t)row * g.ldc + col] = v;
        else
          ((T *)g.c)[(int64_t)z * g.c_bs + (int64_t)row * g.ldc + col] = (T)v;
      }
    }
  }
}

// One wavefront per (row m, 4 columns): lanes stride over k, then a wavefront reduction.
template <typename T>
__global__ void __launch_bounds__(256) gemm_rowdot_kernel(GemmArgs g) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int ncol = (g.N + 3) / 4;
  const int z = blockIdx.z;
  const int64_t m = wid / ncol;
  const int n0 = (int)(wid % ncol) * 4;
  if (m >= g.M) return;
  const T *a = (const T *)g.a + (int64_t)z * g.a_bs + m * g.lda;
  const T *w = (const T *)g.w + (int64_t)z * g.w_bs;
  float s[4] = {0.f, 0.f, 0.f, 0.f};
  for (int k = lane; k < g.K; k += 64) {
    const float x = (float)a[k];
#pragma unroll
    for (int c = 0; c < 4; c++)
      if (n0 + c < g.N) s[c] += x * (float)w[(int64_t)(n0 + c) * g.ldw + k];
  }
#pragma unroll
  for (int c = 0; c < 4; c++) s[c] = wave_sum(s[c]);
  if (lane < 4 && n0 + lane < g.N) {
    float v = lane == 0 ? s[0] : lane == 1 ? s[1] : lane == 2 ? s[2] : s[3];
    const int col = n0 + lane;
    if (g.bias) v += (float)((const T *)g.bias)[col];
    v = activate(v, g.act);
    if (g.c_f32)
      ((float *)g.c)[(int64_t)z * g.c_bs + m * g.ldc + col] = v;
    else
      ((T *)g.c)[(int64_t)z * g.c_bs + m * g.ldc + col] = (T)v;
  }
}

template <typename T>
bool aligned16(const void *p) {
  return ((uintptr_t)p & 15) == 0;
}

}  // namespace

bool gemm_uses_mfma(bool f16, const GemmArgs &g) {
  const int ce = f16 ? 8 : 4;
  return !g.rowdot && g.N >= 32 && g.K % ce == 0 && g.lda % ce == 0 && g.ldw % ce == 0 &&
         g.a_bs % ce == 0 && g.w_bs % ce == 0 && aligned16<char>(g.a) && aligned16<char>(g.w);
}

void gemm(bool f16, const GemmArgs &g, hipStream_t s) {
  if (g.M <= 0 || g.N <= 0 || g.batch <= 0) return;
  if (gemm_uses_mfma(f16, g)) {
    const int tm = (g.M + BM - 1) / BM, tn = (g.N + BN - 1) / BN;
    dim3 grid((unsigned)(tm * tn), 1, (unsigned)g.batch);
    if (f16) hipLaunchKernelGGL((gemm_mfma_kernel<half_t>), grid, dim3(NT), 0, s, g, tn);
    else hipLaunchKernelGGL((gemm_mfma_kernel<float>), grid, dim3(NT), 0, s, g, tn);
  } else {
    const int64_t waves = (int64_t)g.M * ((g.N + 3) / 4);
    dim3 grid((unsigned)((waves + 3) / 4), 1, (unsigned)g.batch);
    if (f16) hipLaunchKernelGGL((gemm_rowdot_kernel<half_t>), grid, dim3(256), 0, s, g);
    else hipLaunchKernelGGL((gemm_rowdot_kernel<float>), grid, dim3(256), 0, s, g);
  }
}

}  // namespace kh
