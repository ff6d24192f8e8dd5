// Flash attention over packed (unpadded) rows on CDNA4 matrix cores.
//
// One 128-thread block per (64-query tile of one sequence, head): each of its two wavefronts owns
// 32 queries. Key/value tiles of 64 rows stream through LDS (K as [key][d], V transposed as
// [d][key]). Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16_f16 (f16) or
// v_mfma_f32_32x32x2f32 (f32): lane l then holds one query column (l % 32) and 16 keys per
// 32-key sub-tile, so the softmax row statistics need one cross-lane exchange (lane l ^ 32), the
// running max and sum stay per lane, and the probabilities feed the P V product as the B operand
// straight from the accumulator registers (O^T = V^T P^T). Only the keys of the query's own
// sequence are visited; with a sliding window only keys with |i - j| <= window.
//
// Masking follows the reference (src/wasm/plan.ts:573-634): excluded keys get exactly zero weight
// and never enter the maximum; packed rows are all valid queries and keys, so every query keeps at
// least itself and the normaliser is positive.
//
// DeBERTa relative attention adds (c2p[i][h][m] + p2c[j][h][m]) with m = bucket(i - j) to q.k
// before the scale (src/wasm/plan.ts:791-840); c2p and p2c come from the relative-position GEMMs.
#include "kernels.h"
#include "device.h"

namespace kh {

namespace {

constexpr int QT = ATTN_QTILE;  // queries per block (2 wavefronts x 32)
constexpr int KT = 64;          // keys per LDS tile

template <typename T>
struct AttnMfma;

template <>
struct AttnMfma<half_t> {
  static constexpr int KSTEP = 16, KLANE = 8;
  typedef half8v frag;
  __device__ static float16v mma(frag a, frag b, float16v c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};
template <>
struct AttnMfma<float> {
  static constexpr int KSTEP = 2, KLANE = 1;
  typedef float frag;
  __device__ static float16v mma(frag a, frag b, float16v c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
};

template <typename T, int D, bool REL>
__global__ void __launch_bounds__(128) attn_kernel(AttnArgs a, Packing p) {
  typedef AttnMfma<T> MF;
  constexpr int PADK = 16 / sizeof(T);   // 16 bytes of row padding
  constexpr int LDK = D + PADK;           // sK row
  // sVt row: 4 elements of padding (a 136-byte pitch for f16): the 4-key column writes of 8
  // threads 8 rows apart then spread over 4 bank groups, and 16 rows read at one key offset stay in
  // distinct banks
  constexpr int LDV = KT + 4;
  constexpr int DT = D / 32;              // 32-wide d sub-tiles of the output
  constexpr int QS = D / MF::KSTEP;       // MFMA k-steps over d
  constexpr int CE = 16 / sizeof(T);      // elements per 16-byte chunk
  constexpr int CPR = D / CE;             // chunks per key row
  __shared__ __attribute__((aligned(16))) T sK[KT * LDK];
  __shared__ __attribute__((aligned(16))) T sVt[D * LDV];

  const int2 tile = a.tiles[blockIdx.x];
  const int b = tile.x, q0 = tile.y;
  const int h = blockIdx.y;
  const int H = a.H;
  const int64_t base = p.cu[b];
  const int n = p.cu[b + 1] - p.cu[b];
  const int64_t rs = (int64_t)3 * H * D;  // qkv row stride
  const T *qkv = (const T *)a.qkv;

  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int g = lane >> 5;                       // lane group
  const int qi = q0 + w * 32 + (lane & 31);      // this lane's query (column)
  const bool qvalid = qi < n;
  const int qc = qvalid ? qi : n - 1;

  // Q fragments: B operand of S^T = K Q^T (column = query, k = d)
  typename MF::frag qf[QS];
#pragma unroll
  for (int s = 0; s < QS; s++) {
    const T *src = qkv + (base + qc) * rs + h * D + s * MF::KSTEP + g * MF::KLANE;
    if constexpr (sizeof(T) == 2) qf[s] = *reinterpret_cast<const half8v *>(src);
    else qf[s] = *src;
  }

  // key range of this tile: the window around [q0, q0 + QT) or the whole sequence
  int klo = 0, khi = n;
  if (a.window > 0) {
    klo = q0 - a.window > 0 ? q0 - a.window : 0;
    const int e = q0 + QT + a.window;
    khi = e < n ? e : n;
  }

  float16v o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; dt++)
#pragma unroll
    for (int r = 0; r < 16; r++) o[dt][r] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  for (int kb = klo; kb < khi; kb += KT) {
    // K tile [key][d] and V tile transposed [d][key]; rows past khi are zero. A thread moves one
    // 16-byte chunk of 4 consecutive keys: K rows as they are, V as 4-key vectors per d.
    for (int c = t; c < (KT / 4) * CPR; c += 128) {
      const int kr = (c / CPR) * 4, dc = (c % CPR) * CE;
      uint4 kv[4], vv[4];
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int j = kb + kr + u;
        kv[u] = make_uint4(0, 0, 0, 0);
        vv[u] = make_uint4(0, 0, 0, 0);
        if (j < khi) {
          const T *row = qkv + (base + j) * rs;
          kv[u] = *reinterpret_cast<const uint4 *>(row + (H + h) * D + dc);
          vv[u] = *reinterpret_cast<const uint4 *>(row + (2 * H + h) * D + dc);
        }
      }
#pragma unroll
      for (int u = 0; u < 4; u++) *reinterpret_cast<uint4 *>(&sK[(kr + u) * LDK + dc]) = kv[u];
      typedef T vec4_t __attribute__((ext_vector_type(4)));
#pragma unroll
      for (int e = 0; e < CE; e++) {
        vec4_t col;
#pragma unroll
        for (int u = 0; u < 4; u++) col[u] = reinterpret_cast<const T *>(&vv[u])[e];
        *reinterpret_cast<vec4_t *>(&sVt[(dc + e) * LDV + kr]) = col;
      }
    }
    __syncthreads();

    // S^T sub-tiles: 32 keys x 32 queries each
    float16v sc[2];
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
#pragma unroll
      for (int r = 0; r < 16; r++) sc[kt][r] = 0.f;
      const T *krow = &sK[(kt * 32 + (lane & 31)) * LDK + g * MF::KLANE];
#pragma unroll
      for (int s = 0; s < QS; s++) {
        typename MF::frag kf;
        if constexpr (sizeof(T) == 2) kf = *reinterpret_cast<const half8v *>(krow + s * MF::KSTEP);
        else kf = krow[s * MF::KSTEP];
        sc[kt] = MF::mma(kf, qf[s], sc[kt]);
      }
    }

    // scale (in base 2: scale * log2 e, so exp2 gives the same weights as exp), mask, maximum
    const float scale2 = a.scale * 1.4426950408889634f;
    float tmax = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int j = kb + kt * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        bool ok = qvalid && j < khi;
        if (a.window > 0) {
          const int dist = qi > j ? qi - j : j - qi;
          ok = ok && dist <= a.window;
        }
        float v = sc[kt][r];
        if constexpr (REL) {
          if (ok) {
            const int m = a.bucket[qi - j + a.lmax - 1];
            v += a.c2p[((base + qi) * H + h) * a.nb + m] + a.p2c[((base + j) * H + h) * a.nb + m];
          }
        }
        v = ok ? v * scale2 : -INFINITY;
        sc[kt][r] = v;
        tmax = fmaxf(tmax, v);
      }
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
    const float m_new = fmaxf(m_run, tmax);
    // a query with no key so far keeps its state (corr 1, weights exp2(-inf) = 0)
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float corr = __builtin_amdgcn_exp2f(m_run - m_use);
    float psum = 0.f;
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const float e = __builtin_amdgcn_exp2f(sc[kt][r] - m_use);
        sc[kt][r] = e;
        psum += e;
      }
    }
    l_run = l_run * corr + psum;
    m_run = m_new;
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
      for (int r = 0; r < 16; r++) o[dt][r] *= corr;

    // O^T += V^T P^T: k = keys; lane group g holds keys 4 g + {0..3} and 8 + 4 g + {0..3} of each
    // 16-key half, for both operands
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
      if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int hb = 0; hb < 2; hb++) {
          half8v pf;
#pragma unroll
          for (int v = 0; v < 8; v++) pf[v] = (half_t)sc[kt][8 * hb + v];
          const int k0 = kt * 32 + 16 * hb + 4 * g;
#pragma unroll
          for (int dt = 0; dt < DT; dt++) {
            const T *vr = &sVt[(dt * 32 + (lane & 31)) * LDV];
            const half4v lo = *reinterpret_cast<const half4v *>(vr + k0);
            const half4v hi = *reinterpret_cast<const half4v *>(vr + k0 + 8);
            half8v vf;
            vf[0] = lo[0]; vf[1] = lo[1]; vf[2] = lo[2]; vf[3] = lo[3];
            vf[4] = hi[0]; vf[5] = hi[1]; vf[6] = hi[2]; vf[7] = hi[3];
            o[dt] = MF::mma(vf, pf, o[dt]);
          }
        }
      } else {
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int key = kt * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
#pragma unroll
          for (int dt = 0; dt < DT; dt++) {
            const float vf = sVt[(dt * 32 + (lane & 31)) * LDV + key];
            o[dt] = MF::mma(vf, sc[kt][r], o[dt]);
          }
        }
      }
    }
    __syncthreads();
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  if (!qvalid) return;
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  T *out = (T *)a.ctx + (base + qi) * (int64_t)H * D + h * D;
  typedef T vec4_t __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int dt = 0; dt < DT; dt++) {
#pragma unroll
    for (int r4 = 0; r4 < 4; r4++) {
      // registers 4 r4 .. 4 r4 + 3 hold d .. d + 3 of this lane's query: one vector store
      const int d = dt * 32 + 8 * r4 + 4 * g;
      vec4_t v;
#pragma unroll
      for (int e = 0; e < 4; e++) v[e] = (T)(o[dt][4 * r4 + e] * inv);
      *reinterpret_cast<vec4_t *>(out + d) = v;
    }
  }
}

template <typename T, bool REL>
void launch_t(const AttnArgs &a, const Packing &p, hipStream_t s) {
  dim3 grid((unsigned)a.ntiles, (unsigned)a.H);
  if (a.D == 64) launch((attn_kernel<T, 64, REL>), grid, dim3(128), 0, s, a, p);
  else launch((attn_kernel<T, 32, REL>), grid, dim3(128), 0, s, a, p);
}

}  // namespace

void attention(bool f16, const AttnArgs &a, const Packing &p, hipStream_t s) {
  if (a.ntiles <= 0) return;
  const bool rel = a.c2p != nullptr;
  if (f16) {
    if (rel) launch_t<half_t, true>(a, p, s);
    else launch_t<half_t, false>(a, p, s);
  } else {
    if (rel) launch_t<float, true>(a, p, s);
    else launch_t<float, false>(a, p, s);
  }
}

}  // namespace kh
