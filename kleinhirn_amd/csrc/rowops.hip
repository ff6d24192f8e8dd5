// Bandwidth-bound row kernels over packed rows: embedding gather + LayerNorm, LayerNorm with the
// residual fused, residual add, GeGLU, RoPE, pooling, row gather, f16 -> f32 readback.
// One 64-lane wavefront per row for the normalisations: the row stays in registers between the
// mean and the variance pass (variance = mean((v - mean)^2), the reference's two-pass form,
// src/wasm/plan.ts:386-411), loads are VEC-wide and coalesced across the wavefront.
#include <algorithm>

#include "kernels.h"
#include "device.h"

namespace kh {

namespace {

constexpr int ROWS_PER_BLOCK = 4;  // wavefronts (rows) per 256-thread block

// The weight prefetch a LayerNorm launch carries (PrefetchArgs): after its rows are stored, every
// thread of the grid reads its share of the ranges' 16-byte pieces (piece g, g + threads, ...), so
// the reads wait on nothing and the launch ends about one memory latency later. The XOR of the
// words is handed to an empty asm statement, so the compiler cannot drop the loads, and nothing is
// written.
__device__ __forceinline__ void prefetch_share(const PrefetchArgs &pf) {
  if (pf.total <= 0) return;
  const int64_t nth = (int64_t)gridDim.x * blockDim.x;
  uint32_t acc = 0;
  for (int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g < pf.total; g += nth) {
    int64_t off = g;
    int r = 0;
    while (r < PREFETCH_RANGES - 1 && off >= pf.n16[r]) {
      off -= pf.n16[r];
      r++;
    }
    const uint4 v = ((const uint4 *)pf.p[r])[off];
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  asm volatile("" ::"v"(acc));
}

// Per lane: PER groups of VEC contiguous elements; group g = k * 64 + lane.
template <typename T, int VEC, int PER>
__device__ __forceinline__ void ln_finish(float (&v)[PER][VEC], int N, const T *gamma, const T *beta,
                                          float eps, T *out, int lane, const float *scale) {
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < PER; k++) {
    int e0 = (k * WAVE + lane) * VEC;
#pragma unroll
    for (int i = 0; i < VEC; i++) s += (e0 + i < N) ? v[k][i] : 0.f;
  }
  float mean = wave_sum(s) / (float)N;
  float sq = 0.f;
#pragma unroll
  for (int k = 0; k < PER; k++) {
    int e0 = (k * WAVE + lane) * VEC;
#pragma unroll
    for (int i = 0; i < VEC; i++) {
      float d = v[k][i] - mean;
      sq += (e0 + i < N) ? d * d : 0.f;
    }
  }
  float var = wave_sum(sq) / (float)N;
  float inv = 1.0f / sqrtf(var + eps);
#pragma unroll
  for (int k = 0; k < PER; k++) {
    int e0 = (k * WAVE + lane) * VEC;
    if (e0 >= N) continue;
    float g[VEC], b[VEC], y[VEC];
    VecIO<T, VEC>::load(gamma + e0, g);
    if (beta) VecIO<T, VEC>::load(beta + e0, b);
#pragma unroll
    for (int i = 0; i < VEC; i++) y[i] = (v[k][i] - mean) * inv * g[i] + (beta ? b[i] : 0.f);
    if (scale) {
      const float sc = *scale;
#pragma unroll
      for (int i = 0; i < VEC; i++) y[i] *= sc;
    }
    VecIO<T, VEC>::store(out + e0, y);
  }
}

// ln_finish with gamma and beta already in registers (gm, bt; bt unused without beta): the same
// operations in the same order.
template <typename T, int VEC, int PER>
__device__ __forceinline__ void ln_finish_pre(float (&v)[PER][VEC], int N, const float (&gm)[PER][VEC],
                                              const float (&bt)[PER][VEC], bool beta, float eps, T *out, int lane,
                                              const float *scale) {
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < PER; k++) {
    int e0 = (k * WAVE + lane) * VEC;
#pragma unroll
    for (int i = 0; i < VEC; i++) s += (e0 + i < N) ? v[k][i] : 0.f;
  }
  float mean = wave_sum(s) / (float)N;
  float sq = 0.f;
#pragma unroll
  for (int k = 0; k < PER; k++) {
    int e0 = (k * WAVE + lane) * VEC;
#pragma unroll
    for (int i = 0; i < VEC; i++) {
      float d = v[k][i] - mean;
      sq += (e0 + i < N) ? d * d : 0.f;
    }
  }
  float var = wave_sum(sq) / (float)N;
  float inv = 1.0f / sqrtf(var + eps);
#pragma unroll
  for (int k = 0; k < PER; k++) {
    int e0 = (k * WAVE + lane) * VEC;
    if (e0 >= N) continue;
    float y[VEC];
#pragma unroll
    for (int i = 0; i < VEC; i++) y[i] = (v[k][i] - mean) * inv * gm[k][i] + (beta ? bt[k][i] : 0.f);
    if (scale) {
      const float sc = *scale;
#pragma unroll
      for (int i = 0; i < VEC; i++) y[i] *= sc;
    }
    VecIO<T, VEC>::store(out + e0, y);
  }
}

template <typename T, int VEC, int PER>
__global__ void __launch_bounds__(256) layernorm_kernel(const T *__restrict__ a, const T *__restrict__ b,
                                                        const T *__restrict__ gamma, const T *__restrict__ beta,
                                                        T *__restrict__ out, int64_t rows, int N, float eps,
                                                        const int32_t *__restrict__ ids, PrefetchArgs pf,
                                                        const float *__restrict__ row_scale) {
  int lane = threadIdx.x & 63;
  int64_t r = (int64_t)blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
  if (r >= rows) {
    prefetch_share(pf);
    return;
  }
  const T *ar = a + (ids ? (int64_t)ids[r] : r) * N;
  const T *br = b ? b + r * N : nullptr;
  float v[PER][VEC];
#pragma unroll
  for (int k = 0; k < PER; k++) {
    int e0 = (k * WAVE + lane) * VEC;
    if (e0 < N) {
      VecIO<T, VEC>::load(ar + e0, v[k]);
      if (br) {
        float y[VEC];
        VecIO<T, VEC>::load(br + e0, y);
#pragma unroll
        for (int i = 0; i < VEC; i++) v[k][i] += y[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < VEC; i++) v[k][i] = 0.f;
    }
  }
  ln_finish<T, VEC, PER>(v, N, gamma, beta, eps, out + r * N, lane, row_scale ? row_scale + r : nullptr);
  prefetch_share(pf);
}


// Several rows per wavefront: a group of LPR lanes (a power of two) holds one row as PER 16-byte
// chunks per lane, so every lane loads (a 768-wide f16 row: 32 lanes x 3 chunks, two rows per
// wavefront) and the reductions stay inside the group.
// The 16-byte chunk c of a row as VEC floats.
template <typename T, int VEC>
__device__ __forceinline__ void chunk_to_float(const uint4 &c, float *o) {
  T e[VEC];
  __builtin_memcpy(e, &c, 16);
#pragma unroll
  for (int i = 0; i < VEC; i++) o[i] = (float)e[i];
}

template <typename T, int LPR, int PER, bool RES>
__global__ void __launch_bounds__(256) layernorm_rows_kernel(const T *__restrict__ a, const T *__restrict__ b,
                                                             const T *__restrict__ gamma,
                                                             const T *__restrict__ beta, T *__restrict__ out,
                                                             int64_t rows, int N, float eps,
                                                             const int32_t *__restrict__ ids, PrefetchArgs pf,
                                                             const float *__restrict__ row_scale) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int RPW = WAVE / LPR;  // rows per wavefront
  const int lane = threadIdx.x & 63, l = lane % LPR;
  const int64_t r = ((int64_t)blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6)) * RPW + lane / LPR;
  if (r >= rows) {  // whole groups leave together: the shuffles below stay in a group
    prefetch_share(pf);
    return;
  }
  const T *ar = a + (ids ? (int64_t)ids[r] : r) * N;
  // every chunk the row needs (a, the residual b when RES, gamma, beta) is requested before the
  // first is used: one memory round trip per row instead of one per chunk
  uint4 ca[PER], cb[PER], cg[PER], ct[PER];
  const T *bt_src = beta ? beta : gamma;  // (gamma's chunks again without beta: never used)
#pragma unroll
  for (int k = 0; k < PER; k++) {
    const int e0 = (k * LPR + l) * VEC;
    ca[k] = *reinterpret_cast<const uint4 *>(ar + e0);
    if constexpr (RES) cb[k] = *reinterpret_cast<const uint4 *>(b + r * N + e0);
    cg[k] = *reinterpret_cast<const uint4 *>(gamma + e0);
    ct[k] = *reinterpret_cast<const uint4 *>(bt_src + e0);
  }
  float v[PER][VEC];
#pragma unroll
  for (int k = 0; k < PER; k++) {
    chunk_to_float<T, VEC>(ca[k], v[k]);
    if constexpr (RES) {
      float y[VEC];
      chunk_to_float<T, VEC>(cb[k], y);
#pragma unroll
      for (int i = 0; i < VEC; i++) v[k][i] += y[i];
    }
  }
  auto group_sum = [&](float x) {
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) x += __shfl_xor(x, o);
    return x;
  };
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < PER; k++)
#pragma unroll
    for (int i = 0; i < VEC; i++) s += v[k][i];
  const float mean = group_sum(s) / (float)N;
  float sq = 0.f;
#pragma unroll
  for (int k = 0; k < PER; k++)
#pragma unroll
    for (int i = 0; i < VEC; i++) {
      const float d = v[k][i] - mean;
      sq += d * d;
    }
  const float var = group_sum(sq) / (float)N;
  const float inv = 1.0f / sqrtf(var + eps);
#pragma unroll
  for (int k = 0; k < PER; k++) {
    const int e0 = (k * LPR + l) * VEC;
    float gm[VEC], bt[VEC], y[VEC];
    chunk_to_float<T, VEC>(cg[k], gm);
    chunk_to_float<T, VEC>(ct[k], bt);
#pragma unroll
    for (int i = 0; i < VEC; i++) y[i] = (v[k][i] - mean) * inv * gm[i] + (beta ? bt[i] : 0.f);
    if (row_scale) {
      const float sc = row_scale[r];
#pragma unroll
      for (int i = 0; i < VEC; i++) y[i] *= sc;
    }
    VecIO<T, VEC>::store(out + r * N + e0, y);
  }
  prefetch_share(pf);
}

// word + position + type in f32 ((word + pos) + type), then LayerNorm (src/wasm/plan.ts:433-447).
// Position row: tt >> 16 with POSIDS, else the row's position in its sequence + OFFSET, clamped to
// MAXPOS - 1. Type row: tt & 0xffff.
template <typename T, int VEC, int PER>
__global__ void __launch_bounds__(256) embln_kernel(EmbLnArgs a, Packing p, PrefetchArgs pf) {
  int lane = threadIdx.x & 63;
  int64_t r = (int64_t)blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
  if (r >= p.T) {
    prefetch_share(pf);
    return;
  }
  const int N = a.N;
  uint32_t t = a.tt ? a.tt[r] : 0u;
  int prow = a.posids ? (int)(t >> 16) : p.row_pos[r] + a.offset;
  prow = prow < a.maxpos - 1 ? prow : a.maxpos - 1;
  const T *word = a.word ? (const T *)a.word + r * N : (const T *)a.table + (int64_t)a.ids[r] * N;
  const T *pos = a.pos ? (const T *)a.pos + (int64_t)prow * N : nullptr;
  const T *typ = a.typ ? (const T *)a.typ + (int64_t)(t & 0xffffu) * N : nullptr;
  // all of the row's reads go out before the first is used: no branch between them (absent tables
  // and lanes past N read the word row's first chunk instead, unused), gamma and beta with them
  const T *ps = pos ? pos : word, *ys = typ ? typ : word;
  const T *gs = (const T *)a.gamma, *bs = a.beta ? (const T *)a.beta : gs;
  float w[PER][VEC], q[PER][VEC], y[PER][VEC], gm[PER][VEC], bt[PER][VEC];
#pragma unroll
  for (int k = 0; k < PER; k++) {
    const int e0 = (k * WAVE + lane) * VEC;
    const int ee = e0 < N ? e0 : 0;
    VecIO<T, VEC>::load(word + ee, w[k]);
    VecIO<T, VEC>::load(ps + ee, q[k]);
    VecIO<T, VEC>::load(ys + ee, y[k]);
    VecIO<T, VEC>::load(gs + ee, gm[k]);
    VecIO<T, VEC>::load(bs + ee, bt[k]);
  }
  float v[PER][VEC];
#pragma unroll
  for (int k = 0; k < PER; k++) {
    const bool in = (k * WAVE + lane) * VEC < N;
#pragma unroll
    for (int i = 0; i < VEC; i++) v[k][i] = in ? (w[k][i] + (pos ? q[k][i] : 0.f)) + (typ ? y[k][i] : 0.f) : 0.f;
  }
  ln_finish_pre<T, VEC, PER>(v, N, gm, bt, a.beta != nullptr, a.eps, (T *)a.out + r * N, lane,
                             a.row_scale ? a.row_scale + r : nullptr);
  prefetch_share(pf);
}

template <typename T, int VEC>
int pick_per(int N) {
  return (N + WAVE * VEC - 1) / (WAVE * VEC);
}

template <typename T, int VEC, typename F>
bool dispatch_per(int N, F &&f) {
  int per = pick_per<T, VEC>(N);
  switch (per) {
    case 1: f(std::integral_constant<int, 1>()); return true;
    case 2: f(std::integral_constant<int, 2>()); return true;
    case 3: f(std::integral_constant<int, 3>()); return true;
    case 4: f(std::integral_constant<int, 4>()); return true;
    case 5: f(std::integral_constant<int, 5>()); return true;
    case 6: f(std::integral_constant<int, 6>()); return true;
    case 8: f(std::integral_constant<int, 8>()); return true;
    default:
      if (per <= 8) { f(std::integral_constant<int, 8>()); return true; }
      if (per <= 12) { f(std::integral_constant<int, 12>()); return true; }
      if (per <= 16) { f(std::integral_constant<int, 16>()); return true; }
      return false;
  }
}

template <typename T>
void layernorm_t(const void *a, const void *b, const void *gamma, const void *beta, void *out, int64_t rows,
                 int N, float eps, const int32_t *ids, const PrefetchArgs &pf, const float *row_scale,
                 hipStream_t s) {
  // rows of 3 x 2^j 16-byte chunks (384- and 768-wide f16, 384-wide f32): groups of 2^j lanes
  constexpr int VEC16 = 16 / sizeof(T);
  if (N % (3 * VEC16) == 0) {
    const int lpr = N / (3 * VEC16);
    auto go_rows = [&](auto lpr_t) {
      constexpr int LPR = decltype(lpr_t)::value;
      const int64_t per_block = (int64_t)ROWS_PER_BLOCK * (WAVE / LPR);
      const dim3 grid((unsigned)((rows + per_block - 1) / per_block));
      if (b)
        launch((layernorm_rows_kernel<T, LPR, 3, true>), grid, dim3(256), 0, s, (const T *)a, (const T *)b,
               (const T *)gamma, (const T *)beta, (T *)out, rows, N, eps, ids, pf, row_scale);
      else
        launch((layernorm_rows_kernel<T, LPR, 3, false>), grid, dim3(256), 0, s, (const T *)a, (const T *)b,
               (const T *)gamma, (const T *)beta, (T *)out, rows, N, eps, ids, pf, row_scale);
    };
    switch (lpr) {
      case 8: go_rows(std::integral_constant<int, 8>()); return;
      case 16: go_rows(std::integral_constant<int, 16>()); return;
      case 32: go_rows(std::integral_constant<int, 32>()); return;
      case 64: go_rows(std::integral_constant<int, 64>()); return;
      default: break;
    }
  }
  dim3 grid((unsigned)((rows + ROWS_PER_BLOCK - 1) / ROWS_PER_BLOCK));
  auto go = [&](auto vec) {
    constexpr int VEC = decltype(vec)::value;
    dispatch_per<T, VEC>(N, [&](auto per) {
      constexpr int PER = decltype(per)::value;
      launch((layernorm_kernel<T, VEC, PER>), grid, dim3(256), 0, s, (const T *)a, (const T *)b,
                         (const T *)gamma, (const T *)beta, (T *)out, rows, N, eps, ids, pf, row_scale);
    });
  };
  // 16-byte loads where the width allows
  if (N % (16 / sizeof(T)) == 0) go(std::integral_constant<int, 16 / sizeof(T)>());
  else if (N % 4 == 0) go(std::integral_constant<int, 4>());
  else if (N % 2 == 0) go(std::integral_constant<int, 2>());
  else go(std::integral_constant<int, 1>());
}

template <typename T>
void embln_t(const EmbLnArgs &a, const Packing &p, const PrefetchArgs &pf, hipStream_t s) {
  dim3 grid((unsigned)((p.T + ROWS_PER_BLOCK - 1) / ROWS_PER_BLOCK));
  auto go = [&](auto vec) {
    constexpr int VEC = decltype(vec)::value;
    dispatch_per<T, VEC>(a.N, [&](auto per) {
      constexpr int PER = decltype(per)::value;
      launch((embln_kernel<T, VEC, PER>), grid, dim3(256), 0, s, a, p, pf);
    });
  };
  if (a.N % (16 / sizeof(T)) == 0) go(std::integral_constant<int, 16 / sizeof(T)>());
  else if (a.N % 4 == 0) go(std::integral_constant<int, 4>());
  else if (a.N % 2 == 0) go(std::integral_constant<int, 2>());
  else go(std::integral_constant<int, 1>());
}

// dst += src in f32, rounded to storage (src/plan/layers.ts:496-498); MODE 1 adds the row of the
// row's sequence.
template <typename T>
__global__ void __launch_bounds__(256) add_kernel(T *__restrict__ dst, const T *__restrict__ src, int64_t total,
                                                  int N, int mode, const int32_t *__restrict__ row_seq) {
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    float s = mode == 0 ? (float)src[i] : (float)src[(int64_t)row_seq[i / N] * N + i % N];
    dst[i] = (T)((float)dst[i] + s);
  }
}

template <typename VT, typename T, int VEC>
__global__ void __launch_bounds__(256) add_vec_kernel(T *__restrict__ dst, const T *__restrict__ src, int64_t nvec) {
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nvec; i += stride) {
    float x[VEC], y[VEC];
    VecIO<T, VEC>::load(dst + i * VEC, x);
    VecIO<T, VEC>::load(src + i * VEC, y);
#pragma unroll
    for (int k = 0; k < VEC; k++) x[k] += y[k];
    VecIO<T, VEC>::store(dst + i * VEC, x);
  }
}

// gate[r, j] = gelu(mid[r, j]) mid[r, I + j] (src/wasm/plan.ts:500-508)
template <typename T, int VEC>
__global__ void __launch_bounds__(256) geglu_kernel(const T *__restrict__ mid, T *__restrict__ gate, int64_t rows,
                                                    int I) {
  int64_t per_row = I / VEC;
  int64_t total = rows * per_row;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    int64_t r = i / per_row;
    int64_t j = (i - r * per_row) * VEC;
    float x[VEC], y[VEC], o[VEC];
    VecIO<T, VEC>::load(mid + r * 2 * I + j, x);
    VecIO<T, VEC>::load(mid + r * 2 * I + I + j, y);
#pragma unroll
    for (int k = 0; k < VEC; k++) o[k] = gelu_as(x[k]) * y[k];
    VecIO<T, VEC>::store(gate + r * I + j, o);
  }
}

// rotate-half RoPE on q and k of head h, table row = position of the row in its sequence
// (src/wasm/plan.ts:510-528)
template <typename T>
__global__ void __launch_bounds__(256) rope_kernel(T *__restrict__ qkv, const float *__restrict__ cossin,
                                                   int64_t rows, int H, int D, const int32_t *__restrict__ row_pos) {
  int half = D / 2;
  int64_t per_row = (int64_t)2 * H * half;
  int64_t total = rows * per_row;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    int64_t r = i / per_row;
    int rem = (int)(i - r * per_row);
    int sidx = rem / half, d = rem - sidx * half;
    T *base = qkv + r * 3 * H * D + (int64_t)sidx * D;
    const float *t = cossin + (int64_t)row_pos[r] * 2 * D;
    float x = (float)base[d], y = (float)base[d + half], c = t[d], sn = t[D + d];
    base[d] = (T)(x * c - y * sn);
    base[d + half] = (T)(y * c + x * sn);
  }
}

// masked mean (count floor 1e-9) or max per sequence and column (src/wasm/plan.ts:474-498); the
// valid rows of a packed sequence are all its rows.
template <typename T>
__global__ void __launch_bounds__(64) pool_kernel(const T *__restrict__ x, T *__restrict__ out, int N, int mode,
                                                  const int32_t *__restrict__ cu, const float *__restrict__ w) {
  int b = blockIdx.y;
  int d = blockIdx.x * 64 + threadIdx.x;
  if (d >= N) return;
  int r0 = cu[b], r1 = cu[b + 1];
  float acc = 0.f;
  if (w) {
    // masks that are not 0/1 prefixes: the mean weighs each row by its mask value (rows of value 0
    // skipped), the maximum takes the rows whose value exceeds 0.5 (src/wasm/plan.ts:474-495)
    float cnt = 0.f;
    bool found = false;
    for (int r = r0; r < r1; r++) {
      const float m = w[r];
      if (mode == 0) {
        if (m == 0.f) continue;
        acc += m * (float)x[(int64_t)r * N + d];
        cnt += m;
      } else if (m > 0.5f) {
        const float v = (float)x[(int64_t)r * N + d];
        acc = found ? fmaxf(acc, v) : v;
        found = true;
      }
    }
    out[(int64_t)b * N + d] = (T)(mode == 0 ? acc / fmaxf(cnt, 1e-9f) : acc);
    return;
  }
  if (mode == 0) {
    // rows added in order; 8 loads in flight ahead of the chain
    float cnt = 0.f;
    int r = r0;
    for (; r + 8 <= r1; r += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; u++) v[u] = (float)x[(int64_t)(r + u) * N + d];
#pragma unroll
      for (int u = 0; u < 8; u++) acc += v[u];
      cnt += 8.f;
    }
    for (; r < r1; r++) {
      acc += (float)x[(int64_t)r * N + d];
      cnt += 1.f;
    }
    out[(int64_t)b * N + d] = (T)(acc / fmaxf(cnt, 1e-9f));
  } else {
    bool found = false;
    for (int r = r0; r < r1; r++) {
      float v = (float)x[(int64_t)r * N + d];
      acc = found ? fmaxf(acc, v) : v;
      found = true;
    }
    out[(int64_t)b * N + d] = (T)acc;
  }
}

template <typename T>
__global__ void __launch_bounds__(256) gather_kernel(const T *__restrict__ x, const uint32_t *__restrict__ markers,
                                                     T *__restrict__ states, int K, int D, int B,
                                                     const int32_t *__restrict__ cu) {
  int64_t total = (int64_t)B * K * D;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    int64_t g = i / D;
    int d = (int)(i - g * D);
    int b = (int)(g / K);
    uint32_t m = markers ? markers[(int64_t)b * 3 * K + (g - (int64_t)b * K)] : 0u;
    int n = cu[b + 1] - cu[b];
    states[i] = (int64_t)m < n ? x[((int64_t)cu[b] + m) * D + d] : (T)0.f;
  }
}

// Row 0 of each sequence between the packed rows and one row per sequence (compact): packed ->
// compact copies row cu[b], compact -> compact copies row b; empty sequences give zeros (as the
// row gather of a pooled head reads them).
template <typename T>
__global__ void __launch_bounds__(256) first_rows_kernel(const T *__restrict__ src, T *__restrict__ dst, int D, int B,
                                                         const int32_t *__restrict__ cu, int from_packed) {
  const int64_t total = (int64_t)B * D;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int b = (int)(i / D), d = (int)(i - (int64_t)b * D);
    const int64_t row = from_packed ? cu[b] : b;
    dst[i] = cu[b + 1] > cu[b] ? src[row * D + d] : (T)0.f;
  }
}

template <typename T>
__global__ void __launch_bounds__(256) to_f32_kernel(const T *__restrict__ src, float *__restrict__ dst, int64_t n) {
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = (float)src[i];
}

unsigned grid_for(int64_t n, int per_thread = 1) {
  int64_t blocks = (n / per_thread + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 65536) blocks = 65536;
  return (unsigned)blocks;
}

}  // namespace

void first_rows(bool f16, const void *src, void *dst, int D, bool from_packed, const Packing &p, hipStream_t s) {
  const int64_t total = (int64_t)p.B * D;
  if (total <= 0) return;
  const dim3 grid((unsigned)std::min<int64_t>((total + 255) / 256, 4096));
  if (f16) launch((first_rows_kernel<half_t>), grid, dim3(256), 0, s, (const half_t *)src, (half_t *)dst, D, p.B, p.cu,
                  (int)from_packed);
  else launch((first_rows_kernel<float>), grid, dim3(256), 0, s, (const float *)src, (float *)dst, D, p.B, p.cu,
              (int)from_packed);
}

void layernorm(bool f16, const void *a, const void *b, const void *gamma, const void *beta, void *out,
               int64_t rows, int N, float eps, hipStream_t s, const int32_t *ids, const PrefetchArgs &pf,
               const float *row_scale) {
  if (rows <= 0) return;
  if (f16) layernorm_t<half_t>(a, b, gamma, beta, out, rows, N, eps, ids, pf, row_scale, s);
  else layernorm_t<float>(a, b, gamma, beta, out, rows, N, eps, ids, pf, row_scale, s);
}

void embln(bool f16, const EmbLnArgs &a, const Packing &p, hipStream_t s, const PrefetchArgs &pf) {
  if (p.T <= 0) return;
  if (f16) embln_t<half_t>(a, p, pf, s);
  else embln_t<float>(a, p, pf, s);
}

void add(bool f16, void *dst, const void *src, int64_t rows, int N, int mode, const Packing &p, hipStream_t s) {
  int64_t total = rows * N;
  if (total <= 0) return;
  if (mode == 0 && f16 && total % 8 == 0) {
    launch((add_vec_kernel<half8v, half_t, 8>), dim3(grid_for(total / 8)), dim3(256), 0, s,
                       (half_t *)dst, (const half_t *)src, total / 8);
  } else if (mode == 0 && !f16 && total % 4 == 0) {
    launch((add_vec_kernel<float4v, float, 4>), dim3(grid_for(total / 4)), dim3(256), 0, s,
                       (float *)dst, (const float *)src, total / 4);
  } else if (f16) {
    launch((add_kernel<half_t>), dim3(grid_for(total)), dim3(256), 0, s, (half_t *)dst,
                       (const half_t *)src, total, N, mode, p.row_seq);
  } else {
    launch((add_kernel<float>), dim3(grid_for(total)), dim3(256), 0, s, (float *)dst,
                       (const float *)src, total, N, mode, p.row_seq);
  }
}

void geglu(bool f16, const void *mid, void *gate, int64_t rows, int I, hipStream_t s) {
  if (rows <= 0) return;
  if (f16) {
    if (I % 8 == 0)
      launch((geglu_kernel<half_t, 8>), dim3(grid_for(rows * I / 8)), dim3(256), 0, s,
                         (const half_t *)mid, (half_t *)gate, rows, I);
    else
      launch((geglu_kernel<half_t, 1>), dim3(grid_for(rows * I)), dim3(256), 0, s,
                         (const half_t *)mid, (half_t *)gate, rows, I);
  } else {
    if (I % 4 == 0)
      launch((geglu_kernel<float, 4>), dim3(grid_for(rows * I / 4)), dim3(256), 0, s,
                         (const float *)mid, (float *)gate, rows, I);
    else
      launch((geglu_kernel<float, 1>), dim3(grid_for(rows * I)), dim3(256), 0, s,
                         (const float *)mid, (float *)gate, rows, I);
  }
}

void rope(bool f16, void *qkv, const float *cossin, int64_t rows, int H, int D, int L, const Packing &p,
          hipStream_t s) {
  (void)L;
  int64_t total = rows * 2 * H * (D / 2);
  if (total <= 0) return;
  if (f16)
    launch((rope_kernel<half_t>), dim3(grid_for(total)), dim3(256), 0, s, (half_t *)qkv, cossin,
                       rows, H, D, p.row_pos);
  else
    launch((rope_kernel<float>), dim3(grid_for(total)), dim3(256), 0, s, (float *)qkv, cossin, rows,
                       H, D, p.row_pos);
}

void pool(bool f16, const void *x, void *out, int N, int mode, const Packing &p, hipStream_t s) {
  if (p.B <= 0) return;
  dim3 grid((unsigned)((N + 63) / 64), (unsigned)p.B);
  if (f16)
    launch((pool_kernel<half_t>), grid, dim3(64), 0, s, (const half_t *)x, (half_t *)out, N, mode,
                       p.cu, p.row_w);
  else
    launch((pool_kernel<float>), grid, dim3(64), 0, s, (const float *)x, (float *)out, N, mode, p.cu, p.row_w);
}

void gather_rows(bool f16, const void *x, const uint32_t *markers, void *states, int K, int D, const Packing &p,
                 hipStream_t s) {
  int64_t total = (int64_t)p.B * K * D;
  if (total <= 0) return;
  if (f16)
    launch((gather_kernel<half_t>), dim3(grid_for(total)), dim3(256), 0, s, (const half_t *)x, markers,
                       (half_t *)states, K, D, p.B, p.cu);
  else
    launch((gather_kernel<float>), dim3(grid_for(total)), dim3(256), 0, s, (const float *)x, markers,
                       (float *)states, K, D, p.B, p.cu);
}

// one thread per marker (src/kernels/masklogits.wgsl; src/wasm/plan.ts:545-551)
template <typename T>
__global__ void __launch_bounds__(256) mask_logits_kernel(const T *__restrict__ raw, const uint32_t *__restrict__ packed,
                                                          float *__restrict__ logits, int K, float temp, int64_t total) {
  const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= total) return;
  const int64_t b = k / K;
  const float m = __uint_as_float(packed[b * 3 * K + K + (k - b * K)]);
  logits[k] = m > 0.5f ? (float)raw[k] / temp : -1e4f;
}

void mask_logits(bool f16, const void *raw, const uint32_t *packed, float *logits, int K, float temp, int64_t total,
                 hipStream_t s) {
  if (total <= 0) return;
  const dim3 grid((unsigned)((total + 255) / 256));
  if (f16)
    launch((mask_logits_kernel<half_t>), grid, dim3(256), 0, s, (const half_t *)raw, packed, logits, K, temp, total);
  else
    launch((mask_logits_kernel<float>), grid, dim3(256), 0, s, (const float *)raw, packed, logits, K, temp, total);
}

void to_f32(bool f16, const void *src, float *dst, int64_t n, hipStream_t s) {
  if (n <= 0) return;
  if (f16)
    launch((to_f32_kernel<half_t>), dim3(grid_for(n)), dim3(256), 0, s, (const half_t *)src, dst, n);
  else
    launch((to_f32_kernel<float>), dim3(grid_for(n)), dim3(256), 0, s, (const float *)src, dst, n);
}

}  // namespace kh
