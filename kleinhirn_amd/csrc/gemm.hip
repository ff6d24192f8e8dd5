// C = act(A W^T + bias) on CDNA4 matrix cores.
//
// Both operands are K-contiguous (activations [M, K] row-major, weights PyTorch [N, K] never
// transposed), the layout MFMA fragments want: lane l of a 32 x 32 tile reads 8 (f16) or 1 (f32)
// consecutive k values of row l % 32 with one LDS load. A block computes a BM x BN tile with
// WM x WN wavefronts; each wavefront holds a (BM/WM) x (BN/WN) sub-tile as 32 x 32 accumulators of
// v_mfma_f32_32x32x16_f16 (f16 storage) or v_mfma_f32_32x32x2f32 (f32 storage).
//
// Operands move global -> LDS with gfx950's direct loads (global_load_lds_dwordx4: each lane's
// 16 bytes land at LDS base + 16 * lane, no VGPR staging) into a ring of STAGES slabs of 128-byte
// rows (64 halves / 32 floats of k). The loads of slab i + STAGES - 1 are issued while slab i feeds
// the MFMAs, so STAGES - 1 slabs of every operand are in flight per CU; one barrier per slab.
// The 16-byte chunks of each row are XOR-swizzled by row (chunk c of row r sits at c ^ swz(r)):
// the lanes of one load instruction fetch the chunks in swizzled order, and the fragment reads of
// 16 consecutive rows hit 16 different bank groups.
//
// Larger wavefront tiles cut LDS traffic per MFMA (a 64 x 64 wavefront tile needs the full LDS
// bandwidth at the MFMA rate, 128 x 64 needs 3/4 of it); smaller block tiles keep more CUs busy on
// the short M of a ragged batch. The launcher picks per shape.
//
// f32 accumulation; bias and activation (a template parameter, so each kernel carries one
// activation) are applied to the finished sum, as in the reference (src/wasm/plan.ts:126-154), then
// rounded once to the storage type. Blocks are mapped XCD-aware: consecutive tiles of one row band
// land on the same XCD (blocks are dealt round-robin over the 8 XCDs), so the A band is read into
// one L2.
//
// Shapes whose K is not a multiple of the slab fall back to a register-staged variant, and narrow
// products (head steps with a handful of classes) to one wavefront per (row, 4 columns).
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "kernels.h"
#include "device.h"

namespace kh {

namespace {

typedef __attribute__((address_space(3))) void lds_void;
typedef const __attribute__((address_space(1))) void gbl_void;

// LDS swizzle of 128-byte slab rows: chunk c of row r sits at c ^ swz(r). The LDS serves 256 bytes
// (64 banks) per cycle, two 128-byte rows; with this key any 16 consecutive rows read at one
// chunk land in 16 distinct 16-byte bank groups.
__device__ __forceinline__ int swz(int row) { return (row >> 1) & 7; }

template <typename T>
struct Mfma;

template <>
struct Mfma<half_t> {
  static constexpr int BK = 64;      // k per LDS slab (128 bytes)
  static constexpr int KSTEP = 16;   // k per MFMA
  typedef half8v frag;
  __device__ static frag lds(const char *slab, int row, int kk, int g) {
    const int chunk = (kk * 2 + g) ^ swz(row);
    return *reinterpret_cast<const half8v *>(slab + row * 128 + chunk * 16);
  }
  __device__ static float16v mma(frag a, frag b, float16v c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mfma<float> {
  static constexpr int BK = 32;
  static constexpr int KSTEP = 2;
  typedef float frag;
  __device__ static frag lds(const char *slab, int row, int kk, int g) {
    const int k = kk * 2 + g;
    const int chunk = (k >> 2) ^ swz(row);
    return *reinterpret_cast<const float *>(slab + row * 128 + chunk * 16 + (k & 3) * 4);
  }
  __device__ static float16v mma(frag a, frag b, float16v c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
};

template <int ACT>
__device__ __forceinline__ float act_fn(float v) {
  if constexpr (ACT == 1) return fmaxf(v, 0.0f);
  else if constexpr (ACT == 2) return gelu_as(v);
  else if constexpr (ACT == 3) return tanhf(v);
  else if constexpr (ACT == 4) return v / (1.0f + __expf(-v));
  else return v;
}

template <typename T, int BM, int BN, int WM, int WN, int ACT, int FM, int FN>
__device__ __forceinline__ void epilogue(const GemmArgs &g, float16v (&acc)[FM][FN], int m0, int n0, int wm,
                                         int wn, int lane, int z) {
  constexpr int TM = BM / WM, TN = BN / WN;
  const int lg = lane >> 5;
  const T *bias = (const T *)g.bias;
#pragma unroll
  for (int j = 0; j < FN; j++) {
    const int col = n0 + wn * TN + j * 32 + (lane & 31);
    if (col >= g.N) continue;
    const float bv = bias ? (float)bias[col] : 0.f;
#pragma unroll
    for (int i = 0; i < FM; i++) {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int row = m0 + wm * TM + i * 32 + 8 * (r >> 2) + 4 * lg + (r & 3);
        if (row >= g.M) continue;
        const float v = act_fn<ACT>(acc[i][j][r] + bv);
        const int64_t o = (int64_t)z * g.c_bs + (int64_t)row * g.ldc + col;
        if (g.c_f32) ((float *)g.c)[o] = v;
        else ((T *)g.c)[o] = (T)v;
      }
    }
  }
}

// f16 epilogue through LDS: each wavefront writes its finished outputs into a row-major BM x BN
// tile (the operand ring is free after the K loop), then the block stores whole 16-byte chunks of
// rows, so a wavefront store instruction covers full 128-byte lines instead of 64-byte halves.
// Needs N % 8 == 0, ldc % 8 == 0 and BM * BN * 2 bytes of LDS.
template <int BM, int BN, int WM, int WN, int ACT, int FM, int FN>
__device__ __forceinline__ void epilogue_lds(const GemmArgs &g, float16v (&acc)[FM][FN], int m0, int n0, int wm,
                                             int wn, int lane, int z, char *smem) {
  constexpr int TM = BM / WM, TN = BN / WN, NT = 64 * WM * WN;
  constexpr int RB = BN * 2;  // bytes per LDS row
  const int lg = lane >> 5;
  const half_t *bias = (const half_t *)g.bias;
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");  // the ring is no longer read
#pragma unroll
  for (int j = 0; j < FN; j++) {
    const int c = wn * TN + j * 32 + (lane & 31);
    const int col = n0 + c;
    const float bv = bias && col < g.N ? (float)bias[col] : 0.f;
#pragma unroll
    for (int i = 0; i < FM; i++) {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int row = wm * TM + i * 32 + 8 * (r >> 2) + 4 * lg + (r & 3);
        // 16-byte chunks of a row rotated by row, so the 2-byte writes of 2 rows spread over banks
        const int chunk = ((c >> 3) + row) & (BN / 8 - 1);
        *reinterpret_cast<half_t *>(smem + row * RB + chunk * 16 + (c & 7) * 2) = (half_t)act_fn<ACT>(acc[i][j][r] + bv);
      }
    }
  }
  __syncthreads();
  constexpr int CPR = BN / 8;  // chunks per row
  half_t *C = (half_t *)g.c + (int64_t)z * g.c_bs;
#pragma unroll
  for (int q = threadIdx.x; q < BM * CPR; q += NT) {
    const int row = q / CPR, cc = q % CPR;
    const int grow = m0 + row, gcol = n0 + cc * 8;
    if (grow < g.M && gcol < g.N) {
      const int chunk = (cc + row) & (CPR - 1);
      *reinterpret_cast<uint4 *>(C + (int64_t)grow * g.ldc + gcol) =
          *reinterpret_cast<const uint4 *>(smem + row * RB + chunk * 16);
    }
  }
}

// LDS-DMA pipeline kernel; needs K % BK == 0.
// occupancy the kernel is built for: blocks per CU that fit the LDS ring (160 KB), wavefronts per SIMD;
// the register allocator may then keep a whole slab's fragments in flight
template <int BM, int BN, int WM, int WN, int STAGES>
constexpr int waves_per_simd() {
  const int blocks = (160 * 1024) / (STAGES * (BM + BN) * 128);
  const int w = blocks * WM * WN / 4;
  return w < 1 ? 1 : (w > 2 ? 2 : w);
}

template <typename T, int BM, int BN, int WM, int WN, int STAGES, int ACT>
__global__ void __launch_bounds__(64 * WM * WN)
__attribute__((amdgpu_waves_per_eu(waves_per_simd<BM, BN, WM, WN, STAGES>(), waves_per_simd<BM, BN, WM, WN, STAGES>())))
gemm_dma_kernel(GemmArgs g, int tiles_m, int tiles_n) {
  typedef Mfma<T> MF;
  constexpr int NW = WM * WN;
  constexpr int BK = MF::BK;
  constexpr int CE = 16 / sizeof(T);
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 32, FN = TN / 32;
  constexpr int GROUPS = (BM + BN) / 8;        // 8-row groups (1 KB each) per slab
  constexpr int P = GROUPS / NW;               // load instructions per wavefront per slab
  static_assert(P * NW == GROUPS, "row groups must split evenly over the wavefronts");
  static_assert((STAGES - 2) * P <= 63, "vmcnt range");
  constexpr int STAGE = (BM + BN) * 128;
  extern __shared__ __attribute__((aligned(1024))) char smem[];

  const int z = blockIdx.z;
  const T *A = (const T *)g.a + (int64_t)z * g.a_bs;
  const T *W = (const T *)g.w + (int64_t)z * g.w_bs;
  const int tile = xcd_tile(blockIdx.x, tiles_m * tiles_n);
  const int m0 = (tile / tiles_n) * BM;
  const int n0 = (tile % tiles_n) * BN;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int lg = lane >> 5;

  // this lane's source rows for its P load instructions (row clamped to the matrix)
  const int lrow = lane >> 3;
  const T *src[P];
#pragma unroll
  for (int p = 0; p < P; p++) {
    const int grp = wave * P + p;
    const int r = grp * 8 + lrow;  // row inside the A | W slab
    const int lchunk = (lane & 7) ^ swz(r);
    if (r < BM) {
      const int m = m0 + r < g.M ? m0 + r : g.M - 1;
      src[p] = A + (int64_t)m * g.lda + lchunk * CE;
    } else {
      const int n = n0 + (r - BM) < g.N ? n0 + (r - BM) : g.N - 1;
      src[p] = W + (int64_t)n * g.ldw + lchunk * CE;
    }
  }
  auto issue = [&](int stage, int k0) {
    char *base = smem + stage * STAGE;
#pragma unroll
    for (int p = 0; p < P; p++) {
      const int grp = wave * P + p;
      __builtin_amdgcn_global_load_lds((gbl_void *)(src[p] + k0), (lds_void *)(base + grp * 1024), 16, 0, 0);
    }
  };

  float16v acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

  const int arow = wm * TM + (lane & 31);
  const int brow = BM + wn * TN + (lane & 31);
  const int nk = g.K / BK;
#pragma unroll
  for (int s = 0; s < STAGES - 1; s++)
    if (s < nk) issue(s, s * BK);

  for (int it = 0; it < nk; it++) {
    // Slab `it` complete for this wavefront (later slabs may stay in flight), then a barrier: every
    // wavefront's part of slab `it` landed and slab it-1 is no longer read. Written as one asm
    // block: __syncthreads() would add a release fence, i.e. a wait for every outstanding load.
    // lgkmcnt(0): this wavefront's own LDS reads are complete before it signals the barrier. The
    // scheduler may sink the last MFMAs of a slab, and the waits for their operands, below the
    // asm; a read still in flight there could return the next issue's data (seen with two streams
    // loading a CU's LDS, where a read can be delayed by hundreds of cycles).
    if (it + STAGES - 2 < nk) {
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"((STAGES - 2) * P) : "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
    if (it + STAGES - 1 < nk) issue((it + STAGES - 1) % STAGES, (it + STAGES - 1) * BK);
    const char *slab = smem + (it % STAGES) * STAGE;
    constexpr int KK = BK / MF::KSTEP;
    typename MF::frag af[2][FM], bf[2][FN];
    auto rd = [&](int kk, int s) {
#pragma unroll
      for (int i = 0; i < FM; i++) af[s][i] = MF::lds(slab, arow + i * 32, kk, lg);
#pragma unroll
      for (int j = 0; j < FN; j++) bf[s][j] = MF::lds(slab, brow + j * 32, kk, lg);
    };
    // the MFMA phase outranks the other block's epilogue (VALU) on this CU
    __builtin_amdgcn_s_setprio(1);
    rd(0, 0);
#pragma unroll
    for (int kk = 0; kk < KK; kk++) {
      if (kk + 1 < KK) rd(kk + 1, (kk + 1) & 1);
#pragma unroll
      for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = MF::mma(af[kk & 1][i], bf[kk & 1][j], acc[i][j]);
    }
    // schedule: DMA issue, reads of step 0, then the reads of step kk + 1 spread between the MFMAs
    // of step kk
    __builtin_amdgcn_sched_group_barrier(0x020, P, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, FM + FN, 0);
#pragma unroll
    for (int kk = 0; kk < KK - 1; kk++) {
#pragma unroll
      for (int r = 0; r < FM + FN; r++) {
        __builtin_amdgcn_sched_group_barrier(0x008, (FM * FN + FM + FN - 1) / (FM + FN), 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
    }
    __builtin_amdgcn_sched_group_barrier(0x008, FM * FN, 0);
  }
  __builtin_amdgcn_s_setprio(0);
  if constexpr (sizeof(T) == 2) {
    if (!g.c_f32 && g.N % 8 == 0 && g.ldc % 8 == 0) {
      epilogue_lds<BM, BN, WM, WN, ACT>(g, acc, m0, n0, wm, wn, lane, z, smem);
      return;
    }
  }
  epilogue<T, BM, BN, WM, WN, ACT>(g, acc, m0, n0, wm, wn, lane, z);
}

// Persistent variant: a fixed grid of blocks walks the tiles (block b takes tiles b, b + G, ...),
// and the slab ring runs continuously over the block's (tile, k) sequence, so the first slabs of
// the next tile are in flight while the current tile's last MFMAs and its epilogue run. The
// epilogue stores straight from the accumulators (the ring stays busy). Needs K % BK == 0.
template <typename T, int BM, int BN, int WM, int WN, int STAGES, int ACT>
__global__ void __launch_bounds__(64 * WM * WN)
__attribute__((amdgpu_waves_per_eu(waves_per_simd<BM, BN, WM, WN, STAGES>(), waves_per_simd<BM, BN, WM, WN, STAGES>())))
gemm_persist_kernel(GemmArgs g, int tiles_m, int tiles_n) {
  typedef Mfma<T> MF;
  constexpr int NW = WM * WN;
  constexpr int BK = MF::BK;
  constexpr int CE = 16 / sizeof(T);
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 32, FN = TN / 32;
  constexpr int KK = BK / MF::KSTEP;
  constexpr int GROUPS = (BM + BN) / 8;
  constexpr int P = GROUPS / NW;
  static_assert(P * NW == GROUPS, "row groups must split evenly over the wavefronts");
  static_assert((STAGES - 2) * P <= 63, "vmcnt range");
  constexpr int STAGE = (BM + BN) * 128;
  extern __shared__ __attribute__((aligned(1024))) char smem[];

  const int ntiles = tiles_m * tiles_n;
  const int G = gridDim.x;
  const int b = blockIdx.x;
  const int my_tiles = b < ntiles ? (ntiles - 1 - b) / G + 1 : 0;
  const int nk = g.K / BK;
  const int total = my_tiles * nk;
  const T *A = (const T *)g.a;
  const T *W = (const T *)g.w;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int lg = lane >> 5;
  const int lrow = lane >> 3;

  auto tile_of = [&](int j, int &m0, int &n0) {
    const int t = xcd_tile(b + j * G, ntiles);
    m0 = (t / tiles_n) * BM;
    n0 = (t % tiles_n) * BN;
  };
  // global iteration q = (j, k): slab k of the block's j-th tile
  auto issue = [&](int q) {
    const int j = q / nk, k0 = (q - j * nk) * BK;
    int m0, n0;
    tile_of(j, m0, n0);
    char *base = smem + (q % STAGES) * STAGE;
#pragma unroll
    for (int p = 0; p < P; p++) {
      const int grp = wave * P + p;
      const int r = grp * 8 + lrow;
      const int lchunk = (lane & 7) ^ swz(r);
      const T *src;
      if (r < BM) {
        const int m = m0 + r < g.M ? m0 + r : g.M - 1;
        src = A + (int64_t)m * g.lda + lchunk * CE + k0;
      } else {
        const int n = n0 + (r - BM) < g.N ? n0 + (r - BM) : g.N - 1;
        src = W + (int64_t)n * g.ldw + lchunk * CE + k0;
      }
      __builtin_amdgcn_global_load_lds((gbl_void *)src, (lds_void *)(base + grp * 1024), 16, 0, 0);
    }
  };

  float16v acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int jj = 0; jj < FN; jj++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][jj][r] = 0.f;

  const int arow = wm * TM + (lane & 31);
  const int brow = BM + wn * TN + (lane & 31);
#pragma unroll
  for (int s = 0; s < STAGES - 1; s++)
    if (s < total) issue(s);

  for (int q = 0; q < total; q++) {
    if (q + STAGES - 2 < total) {
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"((STAGES - 2) * P) : "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
    if (q + STAGES - 1 < total) issue(q + STAGES - 1);
    const char *slab = smem + (q % STAGES) * STAGE;
    typename MF::frag af[2][FM], bf[2][FN];
    auto rd = [&](int kk, int s) {
#pragma unroll
      for (int i = 0; i < FM; i++) af[s][i] = MF::lds(slab, arow + i * 32, kk, lg);
#pragma unroll
      for (int jj = 0; jj < FN; jj++) bf[s][jj] = MF::lds(slab, brow + jj * 32, kk, lg);
    };
    rd(0, 0);
#pragma unroll
    for (int kk = 0; kk < KK; kk++) {
      if (kk + 1 < KK) rd(kk + 1, (kk + 1) & 1);
#pragma unroll
      for (int i = 0; i < FM; i++)
#pragma unroll
        for (int jj = 0; jj < FN; jj++) acc[i][jj] = MF::mma(af[kk & 1][i], bf[kk & 1][jj], acc[i][jj]);
    }
    // schedule: DMA issue, reads of step 0, then the reads of step kk + 1 spread between the MFMAs
    // of step kk
    __builtin_amdgcn_sched_group_barrier(0x020, P, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, FM + FN, 0);
#pragma unroll
    for (int kk = 0; kk < KK - 1; kk++) {
#pragma unroll
      for (int r = 0; r < FM + FN; r++) {
        __builtin_amdgcn_sched_group_barrier(0x008, (FM * FN + FM + FN - 1) / (FM + FN), 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
    }
    __builtin_amdgcn_sched_group_barrier(0x008, FM * FN, 0);
    if ((q + 1) % nk == 0) {
      int m0, n0;
      tile_of(q / nk, m0, n0);
      epilogue<T, BM, BN, WM, WN, ACT>(g, acc, m0, n0, wm, wn, lane, 0);
#pragma unroll
      for (int i = 0; i < FM; i++)
#pragma unroll
        for (int jj = 0; jj < FN; jj++)
#pragma unroll
          for (int r = 0; r < 16; r++) acc[i][jj][r] = 0.f;
    }
  }
}

// Register-staged variant for any K % 8 (f16) / K % 4 (f32): 128 x 128 tiles, two LDS stages.
template <typename T, int ACT>
__global__ void __launch_bounds__(256) gemm_reg_kernel(GemmArgs g, int tiles_m, int tiles_n) {
  typedef Mfma<T> MF;
  constexpr int BM = 128, BN = 128, WM = 2, WN = 2, NT = 256;
  constexpr int BK = MF::BK;
  constexpr int CE = 16 / sizeof(T);
  constexpr int TM = 64, TN = 64, FM = 2, FN = 2;
  constexpr int LA = BM * 8 / NT, LB = BN * 8 / NT;
  constexpr int STAGE = (BM + BN) * 128;
  extern __shared__ __attribute__((aligned(1024))) char smem[];

  const int z = blockIdx.z;
  const T *A = (const T *)g.a + (int64_t)z * g.a_bs;
  const T *W = (const T *)g.w + (int64_t)z * g.w_bs;
  const int tile = xcd_tile(blockIdx.x, tiles_m * tiles_n);
  const int m0 = (tile / tiles_n) * BM;
  const int n0 = (tile % tiles_n) * BN;
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int lg = lane >> 5;

  uint4 ra[LA], rb[LB];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < LA; i++) {
      const int q = t + i * NT, r = q >> 3, c = q & 7;
      const int kk = k0 + c * CE;
      const int am = m0 + r < g.M ? m0 + r : g.M - 1;
      const uint4 v = *reinterpret_cast<const uint4 *>(A + (int64_t)am * g.lda + (kk < g.K ? kk : 0));
      ra[i] = kk < g.K ? v : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < LB; i++) {
      const int q = t + i * NT, r = q >> 3, c = q & 7;
      const int kk = k0 + c * CE;
      const int bn = n0 + r < g.N ? n0 + r : g.N - 1;
      const uint4 v = *reinterpret_cast<const uint4 *>(W + (int64_t)bn * g.ldw + (kk < g.K ? kk : 0));
      rb[i] = kk < g.K ? v : make_uint4(0, 0, 0, 0);
    }
  };
  auto sstore = [&](int stage) {
    char *sa = smem + stage * STAGE;
    char *sb = sa + BM * 128;
#pragma unroll
    for (int i = 0; i < LA; i++) {
      const int q = t + i * NT, r = q >> 3, c = q & 7;
      *reinterpret_cast<uint4 *>(sa + r * 128 + ((c ^ swz(r)) << 4)) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < LB; i++) {
      const int q = t + i * NT, r = q >> 3, c = q & 7;
      *reinterpret_cast<uint4 *>(sb + r * 128 + ((c ^ swz(r)) << 4)) = rb[i];
    }
  };

  float16v acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;
  const int arow = wm * TM + (lane & 31);
  const int brow = BM + wn * TN + (lane & 31);
  gload(0);
  sstore(0);
  __syncthreads();
  int stage = 0;
  const int nk = (g.K + BK - 1) / BK;
  for (int it = 0; it < nk; it++) {
    const bool more = it + 1 < nk;
    if (more) gload((it + 1) * BK);
    const char *slab = smem + stage * STAGE;
#pragma unroll
    for (int kk = 0; kk < BK / MF::KSTEP; kk++) {
      typename MF::frag af[FM], bf[FN];
#pragma unroll
      for (int i = 0; i < FM; i++) af[i] = MF::lds(slab, arow + i * 32, kk, lg);
#pragma unroll
      for (int j = 0; j < FN; j++) bf[j] = MF::lds(slab, brow + j * 32, kk, lg);
#pragma unroll
      for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = MF::mma(af[i], bf[j], acc[i][j]);
    }
    if (more) sstore(stage ^ 1);
    __syncthreads();
    stage ^= 1;
  }
  epilogue<T, BM, BN, WM, WN, ACT>(g, acc, m0, n0, wm, wn, lane, z);
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
  constexpr int V = 16 / sizeof(T);  // elements per 16-byte load
  const bool vec = g.K % V == 0 && g.lda % V == 0 && g.ldw % V == 0 && ((uintptr_t)a & 15) == 0 &&
                   ((uintptr_t)w & 15) == 0;
  if (vec) {
    // 16-byte loads: a K = 768 f16 row is one and a half passes of the wavefront
    typedef T vec_t __attribute__((ext_vector_type(V)));
    for (int k = lane * V; k < g.K; k += 64 * V) {
      const vec_t x = *reinterpret_cast<const vec_t *>(a + k);
#pragma unroll
      for (int c = 0; c < 4; c++) {
        if (n0 + c >= g.N) continue;
        const vec_t y = *reinterpret_cast<const vec_t *>(w + (int64_t)(n0 + c) * g.ldw + k);
#pragma unroll
        for (int e = 0; e < V; e++) s[c] += (float)x[e] * (float)y[e];
      }
    }
  } else {
    for (int k = lane; k < g.K; k += 64) {
      const float x = (float)a[k];
#pragma unroll
      for (int c = 0; c < 4; c++)
        if (n0 + c < g.N) s[c] += x * (float)w[(int64_t)(n0 + c) * g.ldw + k];
    }
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


// f32 products of a few hundred rows (too few rows for 128 x 128 tiles: a short sequence, a CLS
// tail), on v_mfma_f32_32x32x2f32: one 32 x 32 output tile per block of four wavefronts. The K
// range is split in four contiguous quarters, one per wavefront, whose sums are added through LDS
// in a fixed order (((w0 + w1) + w2) + w3), so a tile's result does not depend on M or on the other
// tiles. Each lane loads 16-byte row pieces of A and W: the lane of row l % 32 and half h = l / 32
// takes elements h and h + 2 of each 4-element piece (k = 4q + h, then 4q + 2 + h: the k index the
// MFMA's lane h half holds). Rows past M load row M - 1 and are not stored. Needs K % 16 == 0,
// N % 32 == 0, 16-byte aligned rows (small_f32_ok).
template <int ACT>
__global__ void __launch_bounds__(256) gemm_small_f32_kernel(GemmArgs g, int tiles_n) {
  __shared__ float red[3][16][64];  // wavefronts 1..3's sums, [register][lane]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int z = blockIdx.z;
  const int m0 = (blockIdx.x / tiles_n) * 32, n0 = (blockIdx.x % tiles_n) * 32;
  const int r = lane & 31, h = lane >> 5;
  const int mrow = m0 + r < g.M ? m0 + r : g.M - 1;
  const float *a = (const float *)g.a + (int64_t)z * g.a_bs + (int64_t)mrow * g.lda;
  const float *w = (const float *)g.w + (int64_t)z * g.w_bs + (int64_t)(n0 + r) * g.ldw;
  const int kq = g.K / 4, k0 = wave * kq, k1 = k0 + kq;
  float16v acc = {};
#pragma unroll 4
  for (int k = k0; k < k1; k += 4) {
    const float4v x = *reinterpret_cast<const float4v *>(a + k);
    const float4v y = *reinterpret_cast<const float4v *>(w + k);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(h ? x[1] : x[0], h ? y[1] : y[0], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(h ? x[3] : x[2], h ? y[3] : y[2], acc, 0, 0, 0);
  }
  if (wave > 0) {
#pragma unroll
    for (int i = 0; i < 16; i++) red[wave - 1][i][lane] = acc[i];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int p = 0; p < 3; p++)
#pragma unroll
    for (int i = 0; i < 16; i++) acc[i] += red[p][i][lane];
  // register 4 q + e is row 8 q + 4 h + e of the tile, column r
  const int n = n0 + r;
  const float b = g.bias ? ((const float *)g.bias)[n] : 0.f;
  float *c = (float *)g.c + (int64_t)z * g.c_bs;
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const int m = m0 + 8 * (i >> 2) + 4 * h + (i & 3);
    if (m < g.M) c[(int64_t)m * g.ldc + n] = act_fn<ACT>(acc[i] + b);
  }
}

// Lean f16 kernel: the same slab ring as gemm_dma_kernel (two stages, direct-to-LDS loads,
// swizzled 128-byte rows) with the per-tile and per-slab vector-ALU work cut down, since with two
// blocks per CU every VALU slot competes with the other block's MFMAs:
//  * loads go through buffer resources over the tile's row panels (rows past M / N read as zero),
//    so a slab's k advance is one scalar offset and the LDS destination sits in M0;
//  * fragment read addresses are computed once per tile (rows arow + 32 i share the swizzle of
//    arow) and the loop is unrolled over the two stages, so every LDS read has a constant offset;
//  * the first MFMA of a tile takes a zero accumulator instead of zeroed registers;
//  * operands are swapped (D = W A^T per 32 x 32 tile), so a lane holds four consecutive output
//    columns of one row: bias, activation and the f16 conversion run on 4-wide groups that land in
//    LDS with one 8-byte write, and the block stores whole 16-byte row chunks.
// Needs f16 storage, K % 64 == 0, N % 8 == 0 and ldc % 8 == 0; one matrix (batch 1).
typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ __forceinline__ rsrc_t panel_rsrc(const void *base, uint32_t bytes) {
  // raw buffer, stride 0, num_records = bytes (word 3 of the gfx9 buffer descriptor)
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

// The bias values of this wavefront's accumulator columns, loaded once before the k loop so the
// epilogue waits for no load: bv[j][q] holds the 4 values of columns wn TN + 32 j + 8 q + 4 lg
// (+ 0..3), or for GeGLU those of the rows of W the tile's two halves take (columns n0 / 2 + c of
// each half of the product). Every lane loads, so the loads go out together; columns past N read
// column 0's values, which only reach outputs the store phase drops (nothing reads the loaded
// values here, so no wait for them comes before the k loop).
template <int BN, int WN, int EPI, int FN>
__device__ __forceinline__ void lean_bias(const GemmArgs &g, int n0, int wn, int lane, half4v (&bv)[FN][4]) {
  constexpr int TN = BN / WN;
  const int lg = lane >> 5;
  const half_t *bias = (const half_t *)g.bias;
#pragma unroll
  for (int j = 0; j < FN; j++)
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int nl = wn * TN + j * 32 + 8 * q;
      int n = n0 + nl + 4 * lg;
      if constexpr (EPI == EPI_GEGLU) n = (nl < BN / 2 ? (n0 >> 1) + nl : g.N / 2 + (n0 >> 1) + nl - BN / 2) + 4 * lg;
      bv[j][q] = bias ? *reinterpret_cast<const half4v *>(bias + (n < g.N ? n : 0)) : half4v{};
    }
}

// Lean epilogue, staging half: bias, activation and the f16 conversion of this wavefront's
// accumulators, written row-major into `lds` (rows of BN values, 16-byte chunks rotated by the row).
// acc[i][j][4 q + e] is row row0 + 32 i, column wn TN + 32 j + 8 q + 4 lg + e of the staged rows;
// bv[j][q] holds its bias values (lean_bias).
template <int BN, int WN, int ACT, int EPI, int FM, int FN>
__device__ __forceinline__ void lean_stage(const GemmArgs &g, float16v (&acc)[FM][FN], const half4v (&bv)[FN][4],
                                           char *lds, int wn, int lane, int row0) {
  constexpr int TN = BN / WN, RB = BN * 2, CPR = BN / 8;
  const int lg = lane >> 5;
#pragma unroll
  for (int j = 0; j < FN; j++)
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int nl = wn * TN + j * 32 + 8 * q;
      const float b[4] = {(float)bv[j][q][0], (float)bv[j][q][1], (float)bv[j][q][2], (float)bv[j][q][3]};
#pragma unroll
      for (int i = 0; i < FM; i++) {
        const int ml = row0 + i * 32;
        half4v o;
#pragma unroll
        for (int e = 0; e < 4; e++) o[e] = (half_t)act_fn<ACT>(acc[i][j][4 * q + e] + b[e]);
        const int chunk = ((nl >> 3) + ml) % CPR;
        *reinterpret_cast<half4v *>(lds + ml * RB + chunk * 16 + lg * 8) = o;
      }
    }
}

// EPI_LN rows (C = LayerNorm(residual + product) over whole rows: the tile spans the row, n0 = 0,
// N = BN). LPR lanes per row, PER 16-byte chunks per lane (lane l holds chunks k LPR + l): the
// lanes, the order of the sums and the shuffles of the separate MODE 2 LayerNorm over such rows,
// so both give the same bits. A row's lanes are LPR consecutive threads; the NT threads take RPP
// rows per pass, NP passes, so each shuffle has all its lanes.
template <int ROWS, int BN, int NW>
struct LnRows {
  static constexpr int PER = 3, LPR = BN / (8 * PER), NT = 64 * NW, RPP = NT / LPR, NP = ROWS / RPP;
  static_assert(LPR * PER * 8 == BN && (LPR & (LPR - 1)) == 0 && NT % LPR == 0 && ROWS % RPP == 0,
                "whole rows of 3 chunks per lane, a power-of-two lane group");
  half8v res[NP][PER];  // this thread's residual chunks, pass p, chunk k
  half8v gam[PER], bet[PER];  // its chunks of gamma and beta (the same in every pass)
};

// The residual chunks of every pass and the gamma and beta chunks, loaded before the tile is
// staged: their latency is paid once per tile, where loads in each pass waited once per pass.
template <int ROWS, int BN, int NW>
__device__ __forceinline__ void ln_preload(const GemmArgs &g, int grow0, LnRows<ROWS, BN, NW> &lr) {
  typedef LnRows<ROWS, BN, NW> R;
  const half_t *res = (const half_t *)g.ln_res;
  const int l = threadIdx.x % R::LPR;
#pragma unroll
  for (int k = 0; k < R::PER; k++) {
    const int e0 = (k * R::LPR + l) * 8;
    lr.gam[k] = *reinterpret_cast<const half8v *>((const half_t *)g.ln_g + e0);
    lr.bet[k] = g.ln_b ? *reinterpret_cast<const half8v *>((const half_t *)g.ln_b + e0) : half8v{};
  }
#pragma unroll
  for (int p = 0; p < R::NP; p++) {
    const int grow = grow0 + (int)threadIdx.x / R::LPR + p * R::RPP;
#pragma unroll
    for (int k = 0; k < R::PER; k++) {
      half8v ra = {};
      if (grow < g.M) ra = *reinterpret_cast<const half8v *>(res + (int64_t)grow * g.N + (k * R::LPR + l) * 8);
      lr.res[p][k] = ra;
    }
  }
}

template <int ROWS, int BN, int NW>
__device__ __forceinline__ void lean_store_ln(const GemmArgs &g, const char *lds, int grow0,
                                              const LnRows<ROWS, BN, NW> &lr) {
  typedef LnRows<ROWS, BN, NW> R;
  constexpr int PER = R::PER, LPR = R::LPR, RB = BN * 2, CPR = BN / 8;
  half_t *C = (half_t *)g.c;
  const bool beta = g.ln_b != nullptr;
  const int l = threadIdx.x % LPR;
  auto group_sum = [&](float x) {
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) x += __shfl_xor(x, o);
    return x;
  };
#pragma unroll
  for (int p = 0; p < R::NP; p++) {
    const int row = (int)threadIdx.x / LPR + p * R::RPP;
    const int grow = grow0 + row;
    const bool live = grow < g.M;  // the same for the row's lanes
    float v[PER][8];
#pragma unroll
    for (int k = 0; k < PER; k++) {
      const int cc = k * LPR + l;
      const half8v pr = *reinterpret_cast<const half8v *>(lds + row * RB + ((cc + row) % CPR) * 16);
      const half8v ra = lr.res[p][k];
#pragma unroll
      for (int i = 0; i < 8; i++) {
        v[k][i] = (float)ra[i];
        v[k][i] += (float)pr[i];
      }
    }
    float sm = 0.f;
#pragma unroll
    for (int k = 0; k < PER; k++)
#pragma unroll
      for (int i = 0; i < 8; i++) sm += v[k][i];
    const float mean = group_sum(sm) / (float)g.N;
    float sq = 0.f;
#pragma unroll
    for (int k = 0; k < PER; k++)
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const float d = v[k][i] - mean;
        sq += d * d;
      }
    const float var = group_sum(sq) / (float)g.N;
    const float inv = 1.0f / sqrtf(var + g.ln_eps);
    if (live) {
#pragma unroll
      for (int k = 0; k < PER; k++) {
        const int e0 = (k * LPR + l) * 8;
        float y[8];
#pragma unroll
        for (int i = 0; i < 8; i++)
          y[i] = (v[k][i] - mean) * inv * (float)lr.gam[k][i] + (beta ? (float)lr.bet[k][i] : 0.f);
        VecIO<half_t, 8>::store(C + (int64_t)grow * g.ldc + e0, y);
      }
    }
  }
}

// Lean epilogue, store half: ROWS staged rows (row r is C row grow0 + r) leave as whole 16-byte
// chunks, through the fused step of EPI; NT threads share the rows.
template <int ROWS, int BN, int NW, int EPI>
__device__ __forceinline__ void lean_store(const GemmArgs &g, const char *lds, int grow0, int n0) {
  constexpr int RB = BN * 2, CPR = BN / 8, NT = 64 * NW;
  half_t *C = (half_t *)g.c;
  auto chunk_at = [&](int row, int cc) {
    return *reinterpret_cast<const half8v *>(lds + row * RB + ((cc + row) % CPR) * 16);
  };
  if constexpr (EPI == EPI_GEGLU) {
    // output columns n0 / 2 .. n0 / 2 + BN / 2 of C [M, N / 2]: gelu(a) * b, a and b as stored
    constexpr int HC = CPR / 2;
    const int I = g.N / 2;
#pragma unroll
    for (int q = threadIdx.x; q < ROWS * HC; q += NT) {
      const int row = q / HC, cc = q % HC;
      const int grow = grow0 + row, gcol = (n0 >> 1) + cc * 8;
      if (grow < g.M && gcol < I) {
        const half8v x = chunk_at(row, cc), y = chunk_at(row, cc + HC);
        half8v o;
#pragma unroll
        for (int e = 0; e < 8; e++) o[e] = (half_t)(gelu_as((float)x[e]) * (float)y[e]);
        *reinterpret_cast<half8v *>(C + (int64_t)grow * g.ldc + gcol) = o;
      }
    }
  } else {
    // IT chunks per thread, chunk q = threadIdx.x + it NT. The global reads of a fused step (the
    // residual of RESADD; the positions and the cos/sin rows of RoPE) go out for BATCH chunks at a
    // time from clamped, always valid addresses, before any of them is used: one wait per batch
    // instead of one (or two) per chunk.
    constexpr int IT = ROWS * CPR / NT;
    static_assert(IT * NT == ROWS * CPR, "whole chunk rounds per thread");
    constexpr int BATCH = EPI == EPI_ROPE ? (IT % 4 == 0 ? 4 : 1) : IT;
#pragma unroll
    for (int b0 = 0; b0 < IT; b0 += BATCH) {
      [[maybe_unused]] half8v res[BATCH];
      [[maybe_unused]] float4v tc[BATCH][2], ts[BATCH][2];
      if constexpr (EPI == EPI_RESADD) {
#pragma unroll
        for (int u = 0; u < BATCH; u++) {
          const int q = threadIdx.x + (b0 + u) * NT;
          const int grow = grow0 + q / CPR, gcol = n0 + (q % CPR) * 8;
          const bool live = grow < g.M && gcol < g.N;
          res[u] = *reinterpret_cast<const half8v *>(live ? C + (int64_t)grow * g.ldc + gcol : C);
        }
      } else if constexpr (EPI == EPI_ROPE) {
        // rotate-half on q and k: d < D / 2 pairs with d + D / 2 of the same head (tiles start
        // at head boundaries); cos at table[pos][d], sin at table[pos][D + d]
        const int D = g.rope_d, half = D >> 1;
        int pos[BATCH];
#pragma unroll
        for (int u = 0; u < BATCH; u++) {
          const int grow = grow0 + (int)(threadIdx.x + (b0 + u) * NT) / CPR;
          pos[u] = g.row_pos[grow < g.M ? grow : 0];
        }
#pragma unroll
        for (int u = 0; u < BATCH; u++) {
          const int gcol = n0 + (int)((threadIdx.x + (b0 + u) * NT) % CPR) * 8;
          const int d0 = gcol % D;
          const float *t = g.rope_table + (int64_t)pos[u] * 2 * D + (d0 < half ? d0 : d0 - half);
          tc[u][0] = *reinterpret_cast<const float4v *>(t);
          tc[u][1] = *reinterpret_cast<const float4v *>(t + 4);
          ts[u][0] = *reinterpret_cast<const float4v *>(t + D);
          ts[u][1] = *reinterpret_cast<const float4v *>(t + D + 4);
        }
      }
#pragma unroll
      for (int u = 0; u < BATCH; u++) {
        const int q = threadIdx.x + (b0 + u) * NT;
        const int row = q / CPR, cc = q % CPR;
        const int grow = grow0 + row, gcol = n0 + cc * 8;
        if (grow < g.M && gcol < g.N) {
          half8v x = chunk_at(row, cc);
          half_t *dst = C + (int64_t)grow * g.ldc + gcol;
          if constexpr (EPI == EPI_ROPE) {
            if (gcol < g.rope_cols) {
              const int D = g.rope_d, half = D >> 1;
              const bool lo = gcol % D < half;
              const half8v y = chunk_at(row, lo ? cc + half / 8 : cc - half / 8);
              half8v o;
#pragma unroll
              for (int e = 0; e < 8; e++) {
                const float c = tc[u][e >> 2][e & 3], sn = ts[u][e >> 2][e & 3];
                o[e] = lo ? (half_t)((float)x[e] * c - (float)y[e] * sn) : (half_t)((float)x[e] * c + (float)y[e] * sn);
              }
              x = o;
            }
          } else if constexpr (EPI == EPI_RESADD) {
            // residual += product, in f32, rounded once (the add op on the stored product)
#pragma unroll
            for (int e = 0; e < 8; e++) x[e] = (half_t)((float)res[u][e] + (float)x[e]);
          }
          *reinterpret_cast<half8v *>(dst) = x;
        }
      }
    }
  }
}

template <int BM, int BN, int WM, int WN, int ACT, int EPI, int STAGES>
__device__ __forceinline__ void gemm_lean_body(const GemmArgs &g, int tiles_m, int tiles_n) {
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 32, FN = TN / 32;
  constexpr int GROUPS = (BM + BN) / 8;
  constexpr int P = GROUPS / NW;
  static_assert(P * NW == GROUPS, "row groups must split evenly over the wavefronts");
  static_assert(BN % 64 == 0, "whole 64-column MFMA pairs per tile");
  static_assert(BM * BN * 2 <= 2 * (BM + BN) * 128, "the output tile must fit the slab ring");
  constexpr int STAGE = (BM + BN) * 128;
  extern __shared__ __attribute__((aligned(1024))) char smem[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int lg = lane >> 5;

  // the tile's origin and the buffer resources and offsets of its row panels
  int m0, n0;
  rsrc_t ra, rw;
  uint32_t voff[P];
  auto setup = [&](int tile) {
    m0 = (tile / tiles_n) * BM;
    n0 = (tile % tiles_n) * BN;
    const int rows_a = min(BM, g.M - m0), rows_w = min(BN, g.N - n0);
    ra = panel_rsrc((const half_t *)g.a + (int64_t)m0 * g.lda, (uint32_t)(rows_a * g.lda * 2));
    // GeGLU: the tile's columns are BN / 2 rows of each half of W (all of W in one resource)
    rw = EPI == EPI_GEGLU ? panel_rsrc(g.w, (uint32_t)((int64_t)g.N * g.ldw * 2))
                          : panel_rsrc((const half_t *)g.w + (int64_t)n0 * g.ldw, (uint32_t)(rows_w * g.ldw * 2));
    // load p of this wavefront fills 8-row group wave * P + p: lane l writes row l / 8, position l % 8
#pragma unroll
    for (int p = 0; p < P; p++) {
      const int r = (wave * P + p) * 8 + (lane >> 3);
      const int c = (lane & 7) ^ swz(r);
      int wr = r - BM;
      if constexpr (EPI == EPI_GEGLU)
        wr = (n0 >> 1) + (wr < BN / 2 ? wr : g.N / 2 + wr - BN / 2);
      voff[p] = r < BM ? (uint32_t)((r * g.lda + c * 8) * 2) : (uint32_t)((wr * g.ldw + c * 8) * 2);
    }
  };
  setup(xcd_tile(blockIdx.x, tiles_m * tiles_n));
  auto issue = [&](int stage, int k0) {
#pragma unroll
    for (int p = 0; p < P; p++) {
      const int grp = wave * P + p;
      char *dst = smem + stage * STAGE + grp * 1024;
      if (grp * 8 < BM)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void *)dst, 16, voff[p], k0 * 2, 0, 0);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_void *)dst, 16, voff[p], k0 * 2, 0, 0);
    }
  };

  const int arow = wm * TM + (lane & 31);
  const int brow = BM + wn * TN + (lane & 31);
  int aaddr[4], baddr[4];
#pragma unroll
  for (int kk = 0; kk < 4; kk++) {
    aaddr[kk] = arow * 128 + (((kk * 2 + lg) ^ swz(arow)) << 4);
    baddr[kk] = brow * 128 + (((kk * 2 + lg) ^ swz(brow)) << 4);
  }

  float16v acc[FM][FN];
  const int nk = g.K / 64;
  issue(0, 0);
  half4v bv[FN][4];
  lean_bias<BN, WN, EPI, FN>(g, n0, wn, lane, bv);

  auto slab = [&](const char *base, auto first_t) {
    constexpr bool first = decltype(first_t)::value;
    half8v af[2][FM], bf[2][FN];
    auto rd = [&](int kk, int s) {
#pragma unroll
      for (int i = 0; i < FM; i++) af[s][i] = *reinterpret_cast<const half8v *>(base + aaddr[kk] + i * 4096);
#pragma unroll
      for (int j = 0; j < FN; j++) bf[s][j] = *reinterpret_cast<const half8v *>(base + baddr[kk] + j * 4096);
    };
    rd(0, 0);
#pragma unroll
    for (int kk = 0; kk < 4; kk++) {
      if (kk + 1 < 4) rd(kk + 1, (kk + 1) & 1);
#pragma unroll
      for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) {
          if (first && kk == 0) {
            const float16v zero = {};
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[0][j], af[0][i], zero, 0, 0, 0);
          } else {
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[kk & 1][j], af[kk & 1][i], acc[i][j], 0, 0, 0);
          }
        }
    }
    // instruction order of the slab: the first step's LDS reads, then each step's MFMAs with the
    // next step's reads between them (one read after each of the first MFMAs), so a read has a
    // step of MFMAs to land in before its value is used
    // (tiles whose steps have fewer MFMAs than reads keep the compiler's order)
    constexpr int NR = FM + FN, NM = FM * FN;
    if constexpr (NM >= NR) {
      __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
#pragma unroll
      for (int kk = 0; kk < 3; kk++) {
#pragma unroll
        for (int r = 0; r < NR; r++) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        if constexpr (NM > NR) __builtin_amdgcn_sched_group_barrier(0x008, NM - NR, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, NM, 0);
    }
  };

  if constexpr (STAGES == 2) {
    // slab s in stage s % 2: wait for this wavefront's loads of s and for its own LDS reads, then a
    // barrier (every part landed, and the stage the next issue overwrites is no longer read by a
    // read still in flight; the compiler may sink the last MFMAs and their operand waits below the
    // asm, so the reads must be waited here). The first slab is peeled
    // and the loop body holds two whole slabs, so the accumulators stay in place across iterations.
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (1 < nk) issue(1, 64);
    slab(smem, std::true_type{});
    int it = 1;
    for (; it + 1 < nk; it += 2) {
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      issue(0, (it + 1) * 64);
      slab(smem + STAGE, std::false_type{});
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      if (it + 2 < nk) issue(1, (it + 2) * 64);
      slab(smem, std::false_type{});
    }
    if (it < nk) {
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      slab(smem + STAGE, std::false_type{});
    }
  } else {
    // STAGES - 1 slabs in flight (short-M products, where the chain of slabs is the latency): at
    // slab s the loads of at most STAGES - 2 later slabs may be outstanding, P per slab per
    // wavefront; near the end fewer were issued, so the wait is for all of them
    static_assert((STAGES - 2) * P <= 63, "vmcnt counts up to 63 loads");
    for (int i = 1; i < STAGES - 1 && i < nk; i++) issue(i, i * 64);
    auto wait_for = [&](int sl) {
      if (sl + STAGES - 2 < nk) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"((STAGES - 2) * P) : "memory");
      else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };
    wait_for(0);
    if (STAGES - 1 < nk) issue(STAGES - 1, (STAGES - 1) * 64);
    slab(smem, std::true_type{});
    for (int it = 1; it < nk; it++) {
      wait_for(it);
      if (it + STAGES - 1 < nk) issue((it + STAGES - 1) % STAGES, (it + STAGES - 1) * 64);
      slab(smem + (it % STAGES) * STAGE, std::false_type{});
    }
  }

  // epilogue: acc[i][j][4 q + e] is C[m0 + arow + 32 i][n0 + wn TN + 32 j + 8 q + 4 lg + e]; the
  // tile goes row-major into LDS (16-byte chunks of a row rotated by the row) and leaves as
  // whole 16-byte chunks
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  if constexpr (EPI == EPI_LN) {
    LnRows<BM, BN, NW> lr;
    ln_preload<BM, BN, NW>(g, m0, lr);
    lean_stage<BN, WN, ACT, EPI>(g, acc, bv, smem, wn, lane, arow);
    // the staged rows are visible after this wavefront's LDS writes and the barrier; the residual
    // loads stay in flight across it
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    lean_store_ln<BM, BN, NW>(g, smem, m0, lr);
  } else {
    lean_stage<BN, WN, ACT, EPI>(g, acc, bv, smem, wn, lane, arow);
    __syncthreads();
    lean_store<BM, BN, NW, EPI>(g, smem, m0, n0);
  }
}

// (the body is a device function: the buffer-resource type exists only in device compilation)
template <int BM, int BN, int WM, int WN, int ACT, int EPI, int STAGES>
__global__ void __launch_bounds__(64 * WM * WN)
__attribute__((amdgpu_waves_per_eu(waves_per_simd<BM, BN, WM, WN, STAGES>(), waves_per_simd<BM, BN, WM, WN, STAGES>())))
gemm_lean_kernel(GemmArgs g, int tiles_m, int tiles_n) {
  gemm_lean_body<BM, BN, WM, WN, ACT, EPI, STAGES>(g, tiles_m, tiles_n);
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

template <typename K>
void set_smem(K kernel, int bytes) {
  (void)hipFuncSetAttribute((const void *)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}

template <typename T, int BM, int BN, int WM, int WN, int STAGES, int ACT>
void launch_dma(const GemmArgs &g, hipStream_t s) {
  const int tm = (g.M + BM - 1) / BM, tn = (g.N + BN - 1) / BN;
  constexpr int smem = STAGES * (BM + BN) * 128;
  static bool configured = false;
  if (!configured) {
    set_smem(gemm_dma_kernel<T, BM, BN, WM, WN, STAGES, ACT>, smem);
    configured = true;
  }
  dim3 grid((unsigned)(tm * tn), 1, (unsigned)g.batch);
  launch((gemm_dma_kernel<T, BM, BN, WM, WN, STAGES, ACT>), grid, dim3(64 * WM * WN), smem, s, g, tm,
                     tn);
}

template <typename T, int BM, int BN, int WM, int WN, int STAGES, int ACT>
void launch_persist(const GemmArgs &g, hipStream_t s, int blocks_per_cu) {
  const int tm = (g.M + BM - 1) / BM, tn = (g.N + BN - 1) / BN;
  constexpr int smem = STAGES * (BM + BN) * 128;
  static bool configured = false;
  if (!configured) {
    set_smem(gemm_persist_kernel<T, BM, BN, WM, WN, STAGES, ACT>, smem);
    configured = true;
  }
  const int grid = std::min(tm * tn, 256 * blocks_per_cu);
  launch((gemm_persist_kernel<T, BM, BN, WM, WN, STAGES, ACT>), dim3(grid), dim3(64 * WM * WN), smem, s,
                     g, tm, tn);
}


template <int BM, int BN, int WM, int WN, int ACT, int EPI, int STAGES>
void launch_lean_epi(const GemmArgs &g, hipStream_t s) {
  const int tm = (g.M + BM - 1) / BM, tn = (g.N + BN - 1) / BN;
  constexpr int smem = STAGES * (BM + BN) * 128;
  static bool configured = false;
  if (!configured) {
    set_smem(gemm_lean_kernel<BM, BN, WM, WN, ACT, EPI, STAGES>, smem);
    configured = true;
  }
  launch((gemm_lean_kernel<BM, BN, WM, WN, ACT, EPI, STAGES>), dim3(tm * tn), dim3(64 * WM * WN), smem, s, g, tm,
         tn);
}

template <int BM, int BN, int WM, int WN, int ACT, int STAGES = 2>
void launch_lean(const GemmArgs &g, hipStream_t s) {
  switch (g.epi) {
    case EPI_GEGLU: launch_lean_epi<BM, BN, WM, WN, ACT, EPI_GEGLU, STAGES>(g, s); break;
    case EPI_ROPE: launch_lean_epi<BM, BN, WM, WN, ACT, EPI_ROPE, STAGES>(g, s); break;
    case EPI_RESADD: launch_lean_epi<BM, BN, WM, WN, ACT, EPI_RESADD, STAGES>(g, s); break;
    default: launch_lean_epi<BM, BN, WM, WN, ACT, EPI_NONE, STAGES>(g, s); break;
  }
}

// shapes the lean kernel runs: f16, one matrix, whole 64-wide k slabs, 16-byte output chunks, and
// panel byte offsets within 32 bits
bool lean_ok(const GemmArgs &g) {
  return !g.c_f32 && g.batch == 1 && g.K % 64 == 0 && g.N % 8 == 0 && g.ldc % 8 == 0 &&
         (int64_t)256 * g.lda * 2 < ((int64_t)1 << 31) && (int64_t)256 * g.ldw * 2 < ((int64_t)1 << 31);
}

template <typename T, int ACT>
void launch_reg(const GemmArgs &g, hipStream_t s) {
  const int tm = (g.M + 127) / 128, tn = (g.N + 127) / 128;
  constexpr int smem = 2 * 256 * 128;
  static bool configured = false;
  if (!configured) {
    set_smem(gemm_reg_kernel<T, ACT>, smem);
    configured = true;
  }
  dim3 grid((unsigned)(tm * tn), 1, (unsigned)g.batch);
  launch((gemm_reg_kernel<T, ACT>), grid, dim3(256), smem, s, g, tm, tn);
}

constexpr int CUS = 256;

// Per-CU work of a lean configuration: the tiles the busiest CU runs times the tile's area (a
// launch of 258 tiles of 192 x 256 on 256 CUs takes two rounds, as long as 512 such tiles).
static int64_t lean_cost(const GemmArgs &g, int bm, int bn) {
  const int64_t tiles = (int64_t)((g.M + bm - 1) / bm) * ((g.N + bn - 1) / bn);
  return (tiles + CUS - 1) / CUS * bm * bn;
}

// Tile configurations. Lean f16 kernel: 8 = 192x128 (4 wavefronts of 96x64, two blocks per CU),
// 9 = 192x256 (8 wavefronts of 96x64), 10 = 128x128 (4 of 64x64), 11 = 64x64 (1), 12 = 128x384
// (8 of 64x96), 13 = 64x64 (4 of 32x32) with 8 slab stages, 7 slabs in flight (a few hundred rows:
// the slab chain is the latency), 14 = 256x256 (8 of 128x64). DMA kernel: 0 = 256x256 (8 of
// 128x64, 2 stages), 1 = 256x128 (4 of 128x64, 3 stages), 2 = 128x128 (4 of 64x64, 4 stages),
// 3 = 128x128 (4 of 64x64, 2 stages, two blocks per CU), 4 = 256x256 (4 of 128x128); persistent
// 5/6/7. KH_GEMM_TILE forces one (tuning runs).
int pick_tile(const GemmArgs &g, bool lean) {
  const char *e = getenv("KH_GEMM_TILE");
  const int forced = e ? atoi(e) : -1;
  // (a fused step runs in the lean kernel only)
  if (forced >= 0 && forced <= 14 && (forced < 8 ? g.epi == EPI_NONE : lean)) return forced;
  // measured on MI355X (f16, random data, encoder shapes M = 13k .. 1.2M): 192x128 leads in
  // general; 192x256 where N is a multiple of 256 and either narrow (N <= 768: one round of tiles
  // at M ~ 13k) or fed by a short K (<= 384, where the epilogue weighs most)
  // (a few hundred rows, e.g. a pooled head: 64 x 64 tiles, enough of them to spread over CUs)
  if (lean) {
    if (g.M <= 1024) return 13;
    // 256 x 256 (8 wavefronts of 128 x 64, one block per CU): 131 flop per loaded byte against
    // 78 for 192 x 128, so the k loop is no longer bound by the loads into LDS. It wins where the
    // product's K is short (<= 768) and the rows are many (c5's products +5-7 % each, c5 +2 % end
    // to end). At c2's size (and its two halves of ~6,400 rows on two streams) one block per CU
    // filled the chip worse than two of 192 x 128 in an earlier build: c2 lost 1.6 % with it on
    // the QKV product. With every product's weights prefetched and the halves launched
    // interleaved, the QKV product (no activation, N >= 2304) of c2's size and of its halves gains
    // with it: c2 +1.1 % (c3a, 16k rows, keeps 128 x 384, which divides its rows into whole rounds).
    if (g.K <= 768 && g.M >= 65536) return 14;
    if (g.K <= 768 && g.M >= 4096 && g.M <= 13312 && g.act == 0 && g.epi == EPI_NONE && g.N >= 2304 && g.N % 256 == 0)
      return 14;
    // very many rows (c5's 1.2M): per-tile efficiency decides, measured on the 384-wide models:
    // 128 x 384 for 384- and 768-wide outputs (one column tile: each A band is read once), 192 x 256
    // for wider ones fed by a short K
    if (g.M >= 524288) {
      if (g.N % 384 == 0 && g.N <= 768) return 12;
      if (g.N > 768 && g.N % 128 == 0 && g.K <= 384) return 9;
    }
    const int base = g.N % 256 == 0 && (g.N <= 768 || g.K <= 384) ? 9 : 8;
    // a row count just past a whole round of 192-row tiles (M = 16384: 86 row tiles) leaves the
    // last round nearly empty; 128 x 384 tiles divide such shapes into whole rounds
    const int64_t c_base = base == 9 ? lean_cost(g, 192, 256) : lean_cost(g, 192, 128);
    // (two blocks of 192 x 128 per CU run about 15 % faster per tile area than 128 x 384)
    if (g.N % 384 == 0 && lean_cost(g, 128, 384) * 5 < c_base * 4) return 12;
    return base;
  }
  if (g.batch == 1 && g.M >= 65536 && g.N >= 1024) return 6;
  return 3;
}

template <typename T, int ACT>
void launch_act(const GemmArgs &g, hipStream_t s) {
  if (g.K % Mfma<T>::BK != 0) {
    launch_reg<T, ACT>(g, s);
    return;
  }
  const bool lean = sizeof(T) == 2 && lean_ok(g);
  if constexpr (sizeof(T) == 2) {
    // residual + LayerNorm over whole rows: 128 x 384 tiles (384 = the row; gemm_epi_ok checks)
    if (g.epi == EPI_LN) {
      launch_lean_epi<128, 384, 2, 4, ACT, EPI_LN, 2>(g, s);
      return;
    }
  }
  int cfg = pick_tile(g, lean);
  if (cfg >= 5 && cfg <= 7 && g.batch > 1) cfg = 3;  // the persistent kernels walk one matrix
  if constexpr (sizeof(T) == 2) {
    switch (cfg) {
      case 8: launch_lean<192, 128, 2, 2, ACT>(g, s); return;
      case 9: launch_lean<192, 256, 2, 4, ACT>(g, s); return;
      case 10: launch_lean<128, 128, 2, 2, ACT>(g, s); return;
      case 11: launch_lean<64, 64, 1, 1, ACT>(g, s); return;
      case 12: launch_lean<128, 384, 2, 4, ACT>(g, s); return;
      case 13: launch_lean<64, 64, 2, 2, ACT, 8>(g, s); return;
      case 14: launch_lean<256, 256, 2, 4, ACT>(g, s); return;
      default: break;
    }
  }
  switch (cfg) {
    case 5: launch_persist<T, 128, 128, 2, 2, 2, ACT>(g, s, 2); break;
    case 6: launch_persist<T, 256, 256, 2, 4, 2, ACT>(g, s, 1); break;
    case 7: launch_persist<T, 128, 128, 2, 2, 3, ACT>(g, s, 1); break;
    case 0: launch_dma<T, 256, 256, 2, 4, 2, ACT>(g, s); break;
    case 1: launch_dma<T, 256, 128, 2, 2, 3, ACT>(g, s); break;
    case 2: launch_dma<T, 128, 128, 2, 2, 4, ACT>(g, s); break;
    case 4: launch_dma<T, 256, 256, 2, 2, 2, ACT>(g, s); break;
    default: launch_dma<T, 128, 128, 2, 2, 2, ACT>(g, s); break;
  }
}

template <typename T>
void launch_mfma(const GemmArgs &g, hipStream_t s) {
  switch (g.act) {
    case 1: launch_act<T, 1>(g, s); break;
    case 2: launch_act<T, 2>(g, s); break;
    case 3: launch_act<T, 3>(g, s); break;
    case 4: launch_act<T, 4>(g, s); break;
    default: launch_act<T, 0>(g, s); break;
  }
}

}  // namespace

bool gemm_epi_ok(bool f16, const GemmArgs &g) {
  if (g.epi == EPI_NONE) return true;
  if (!f16 || !gemm_uses_mfma(f16, g) || !lean_ok(g)) return false;
  switch (g.epi) {
    case EPI_GEGLU:  // both halves in one buffer resource; half tiles of whole 16-byte chunks
      return g.N % 16 == 0 && g.ldc >= g.N / 2 && (int64_t)g.N * g.ldw * 2 < ((int64_t)1 << 31);
    case EPI_ROPE:  // heads must not straddle tiles (the narrowest tile is 64 columns wide)
      return g.rope_table && g.row_pos && g.rope_d > 0 && g.rope_d % 16 == 0 && 64 % g.rope_d == 0 &&
             g.rope_cols <= g.N && g.rope_cols % g.rope_d == 0;
    case EPI_RESADD:
      return g.act == 0;
    case EPI_LN:  // rows of exactly one 384-wide tile
      return g.N == 384 && g.ldc == g.N;
    default:
      return false;
  }
}

bool gemm_uses_mfma(bool f16, const GemmArgs &g) {
  const int ce = f16 ? 8 : 4;
  // f32 products too small to fill the chip with 128 x 128 tiles (a short sequence) go to one
  // wavefront per row and 4 columns instead
  const int64_t tiles = (int64_t)((g.M + 127) / 128) * ((g.N + 127) / 128) * g.batch;
  if (!f16 && tiles < 64 && g.epi == EPI_NONE) return false;
  return !g.rowdot && g.N >= 32 && g.K % ce == 0 && g.lda % ce == 0 && g.ldw % ce == 0 && g.a_bs % ce == 0 &&
         g.w_bs % ce == 0 && aligned16(g.a) && aligned16(g.w);
}

// f32 products the small-tile MFMA kernel takes (those gemm_uses_mfma leaves to the wavefront-per-
// output kernel, with whole 32-column tiles and 4-element k pieces per wavefront quarter)
static bool small_f32_ok(bool f16, const GemmArgs &g) {
  return !f16 && !g.rowdot && g.epi == EPI_NONE && !gemm_uses_mfma(f16, g) && g.N % 32 == 0 && g.K % 16 == 0 &&
         g.lda % 4 == 0 && g.ldw % 4 == 0 && g.a_bs % 4 == 0 && g.w_bs % 4 == 0 && aligned16(g.a) &&
         aligned16(g.w);
}

bool gemm_on_mfma(bool f16, const GemmArgs &g) { return gemm_uses_mfma(f16, g) || small_f32_ok(f16, g); }

void gemm(bool f16, const GemmArgs &g, hipStream_t s) {
  if (g.M <= 0 || g.N <= 0 || g.batch <= 0) return;
  if (gemm_uses_mfma(f16, g)) {
    if (f16) launch_mfma<half_t>(g, s);
    else launch_mfma<float>(g, s);
  } else if (small_f32_ok(f16, g)) {
    const int tn = g.N / 32;
    dim3 grid((unsigned)(((g.M + 31) / 32) * tn), 1, (unsigned)g.batch);
    switch (g.act) {
      case 1: launch((gemm_small_f32_kernel<1>), grid, dim3(256), 0, s, g, tn); break;
      case 2: launch((gemm_small_f32_kernel<2>), grid, dim3(256), 0, s, g, tn); break;
      case 3: launch((gemm_small_f32_kernel<3>), grid, dim3(256), 0, s, g, tn); break;
      case 4: launch((gemm_small_f32_kernel<4>), grid, dim3(256), 0, s, g, tn); break;
      default: launch((gemm_small_f32_kernel<0>), grid, dim3(256), 0, s, g, tn); break;
    }
  } else {
    const int64_t waves = (int64_t)g.M * ((g.N + 3) / 4);
    dim3 grid((unsigned)((waves + 3) / 4), 1, (unsigned)g.batch);
    if (f16) launch((gemm_rowdot_kernel<half_t>), grid, dim3(256), 0, s, g);
    else launch((gemm_rowdot_kernel<float>), grid, dim3(256), 0, s, g);
  }
}

}  // namespace kh
