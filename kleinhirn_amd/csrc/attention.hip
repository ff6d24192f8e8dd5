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
// DeBERTa relative attention adds q_i . pos_key[m] + k_j . pos_query[m] with m = bucket(i - j) to
// q_i . k_j before the scale (src/wasm/plan.ts:791-840). The 32 queries of a wavefront and a
// 32-key sub-tile span 63 distances i - j: per sub-tile the wavefront computes each term for the
// position rows of those distances (row r: bucket(dlo + r)) on MFMA (pos_key rows x its Q, then
// pos_query rows x the sub-tile's K), parks it in its own LDS scratch (row pitch 68 floats) and
// adds each score's entry from there, at offsets fixed by the score's register; the two terms
// take turns in one scratch. The position tables are read from L2; no [T, H, buckets] array
// exists. The bucket table (i - j -> position row) sits in LDS as 16-bit entries, sized by the
// plan's length.
#include <type_traits>

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

// Head dimensions other than 32 and 64 (PAD): the kernel runs at D (the next of 32, 64) with the
// columns a.D .. D - 1 read as zero (they add nothing to the products) and never stored; every
// access is then element-wise, as the rows' head offsets h a.D need not be 16-byte aligned.
template <typename T, bool PAD>
__device__ __forceinline__ typename AttnMfma<T>::frag load_frag(const T *row, int d, int Dr) {
  if constexpr (sizeof(T) == 2) {
    if constexpr (!PAD) {
      return *reinterpret_cast<const half8v *>(row + d);
    } else {
      half8v v;
#pragma unroll
      for (int e = 0; e < 8; e++) v[e] = d + e < Dr ? row[d + e] : (half_t)0;
      return v;
    }
  } else {
    if constexpr (!PAD) return row[d];
    else return d < Dr ? row[d] : 0.f;
  }
}
template <typename T, bool PAD>
__device__ __forceinline__ uint4 load_chunk(const T *row, int d, int Dr) {
  if constexpr (!PAD) {
    return *reinterpret_cast<const uint4 *>(row + d);
  } else {
    constexpr int CE = 16 / sizeof(T);
    T v[CE];
#pragma unroll
    for (int e = 0; e < CE; e++) v[e] = d + e < Dr ? row[d + e] : (T)0;
    uint4 r;
    __builtin_memcpy(&r, v, 16);
    return r;
  }
}

// Four wavefronts per SIMD on the standard path (short sequences are latency-bound), two on the
// relative path (half of each with PAD, whose element-wise loads hold more registers, or KM). WIN:
// a sliding window (a.window > 0) bounds the keys of each query. KM: masks other than 0/1 prefixes
// (p.row_w), a separate instantiation so the usual kernels keep their registers.
template <typename T, int D, bool REL, bool WIN, bool PAD, bool KM>
__global__ void __launch_bounds__(128)
__attribute__((amdgpu_waves_per_eu((PAD || KM) ? (REL ? 1 : 2) : (REL ? 2 : 4), 8)))
attn_kernel(AttnArgs a, Packing p) {
  typedef AttnMfma<T> MF;
  const int Dr = PAD ? a.D : D;           // the rows' head dimension
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
  constexpr int RP = 68;  // relative scratch pitch (floats)
  __shared__ __attribute__((aligned(16))) float sRel[REL ? 2 * 32 * RP : 1];  // [wave][32][RP]
  extern __shared__ short sBucket[];  // [2 lmax - 1] (dynamic: the relative path only)
  __shared__ float sKw[KM ? KT : 1];   // the key tile's mask values (masks other than 0/1 prefixes)

  // items (head, query tile), tiles fastest: the query tiles of one sequence and head run
  // together on one XCD and find its K and V rows in that XCD's L2
  const int H = a.H;
  int4 wk;  // {head, first query, first packed row, length}
  if (a.work) {
    wk = a.work[blockIdx.x];
  } else {
    const int item = xcd_tile(blockIdx.x, a.ntiles * H);
    const int4 tile = a.tiles[item % a.ntiles];
    wk = int4{item / a.ntiles, tile.y, tile.z, tile.w};
  }
  if (wk.x < 0) return;  // (the work list's padding: an XCD with fewer items)
  const int q0 = wk.y;
  const int h = wk.x;
  const int64_t base = wk.z;
  const int n = wk.w;
  const int64_t rs = (int64_t)3 * H * Dr;  // qkv row stride
  const int rs32 = 3 * H * Dr;
  const T *qkv = (const T *)a.qkv;

  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int g = lane >> 5;                       // lane group
  const int qi = q0 + w * 32 + (lane & 31);      // this lane's query (column)
  const bool qvalid = qi < n;
  const int qc = qvalid ? qi : n - 1;
  // masks other than 0/1 prefixes (p.row_w): keys count where their mask value exceeds 0.5, and a
  // query row whose value does not writes zeros (src/wasm/plan.ts:573-582)
  const float *kw = KM ? p.row_w : nullptr;
  const bool qkeep = !KM || kw[base + qc] > 0.5f;

  // Q fragments: B operand of S^T = K Q^T (column = query, k = d)
  typename MF::frag qf[QS];
#pragma unroll
  for (int s = 0; s < QS; s++) qf[s] = load_frag<T, PAD>(qkv + (base + qc) * rs + h * Dr, s * MF::KSTEP + g * MF::KLANE, Dr);

  // key range of this tile: the window around [q0, q0 + QT) or the whole sequence
  int klo = 0, khi = n;
  if (WIN) {
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
  // c2p rows of one 32-row distance block for this wavefront's queries: q . pos_key[bucket(d)]
  // for d = d0 + lane-row, as [row][query] accumulators (lane = query)
  const int64_t hd = (int64_t)H * Dr;
  // (the bucket table from LDS, or from global memory before the LDS copy is visible)
  [[maybe_unused]] auto c2p_block = [&](int d0, auto from_lds_t) {
    int di = d0 + (lane & 31) + a.lmax - 1;  // this lane's distance row
    di = di < 0 ? 0 : (di > 2 * a.lmax - 2 ? 2 * a.lmax - 2 : di);
    // < nb: the relidx table is checked against the tables
    const int pr = decltype(from_lds_t)::value ? (int)sBucket[di] : a.bucket[di];
    const T *pt = (const T *)a.pos_key + pr * hd + h * Dr;
    float16v c = {};
#pragma unroll
    for (int s = 0; s < QS; s++) c = MF::mma(load_frag<T, PAD>(pt, s * MF::KSTEP + g * MF::KLANE, Dr), qf[s], c);
    return c;
  };
  // The distance window of the sub-tile of keys kj0 .. kj0 + 31 starts at dlo = qw0 - kj0 - 31; the
  // next sub-tile's (32 keys on) starts 32 lower, so the first half of a window's c2p rows is the
  // second half of the next one's: each sub-tile computes one block and carries it to the next.
  // The carry into the first sub-tile is computed here.
  [[maybe_unused]] float16v c2p_carry;
  // p2c rows likewise: the A operands (pos_query rows of the distances) of a sub-tile's upper 32-row
  // block are those of the previous sub-tile's lower block, so each sub-tile loads one block of
  // position rows and carries it (f16; the f32 fragments of a block take 32 registers, and f32
  // loads both blocks)
  constexpr bool PQC = REL && sizeof(T) == 2;
  typedef typename MF::frag frag_t;
  // the position rows (of `table`) of the distance block starting at d0, as MFMA A fragments
  auto pos_frags = [&](const void *table, int d0, frag_t (&f)[QS], auto from_lds_t) {
    int di = d0 + (lane & 31) + a.lmax - 1;  // this lane's distance row
    di = di < 0 ? 0 : (di > 2 * a.lmax - 2 ? 2 * a.lmax - 2 : di);
    // < nb: the relidx table is checked against the tables
    const int pr = decltype(from_lds_t)::value ? (int)sBucket[di] : a.bucket[di];
    const T *pt = (const T *)table + pr * hd + h * Dr;
#pragma unroll
    for (int s = 0; s < QS; s++) f[s] = load_frag<T, PAD>(pt, s * MF::KSTEP + g * MF::KLANE, Dr);
  };
  [[maybe_unused]] frag_t pq_carry[QS];
  // f16: the pos_key rows of the next sub-tile's c2p block are loaded one sub-tile ahead (its
  // distances are the current ones minus 32), so their L2 latency passes under the current
  // sub-tile's work instead of stalling its c2p products
  [[maybe_unused]] frag_t pk_next[QS];
  if constexpr (REL) {
    // visible to every wavefront after the first K/V staging barrier; 8 entries per thread are
    // read before any is written (a loop of read, wait, write paid one round trip per entry)
    const int nbk = 2 * a.lmax - 1;
    for (int i0 = 0; i0 < nbk; i0 += 128 * 8) {
      int bv[8];
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int i = i0 + t + u * 128;
        bv[u] = a.bucket[i < nbk ? i : nbk - 1];
      }
#pragma unroll
      for (int u = 0; u < 8; u++)
        if (i0 + t + u * 128 < nbk) sBucket[i0 + t + u * 128] = (short)bv[u];
    }
    c2p_carry = c2p_block(q0 + w * 32 - (klo + 31) + 32, std::false_type{});
    if constexpr (PQC) {
      pos_frags(a.pos_query, q0 + w * 32 - (klo + 31) + 32, pq_carry, std::false_type{});
      pos_frags(a.pos_key, q0 + w * 32 - (klo + 31), pk_next, std::false_type{});
    }
  }

  // this head's K and V columns in the sequence's first row
  const T *k_seq = qkv + base * rs + (H + h) * Dr;
  const T *v_seq = k_seq + H * Dr;
  for (int kb = klo; kb < khi; kb += KT) {
    // K tile [key][d] and V tile transposed [d][key]. A thread moves one 16-byte chunk of 4
    // consecutive keys: K rows as they are, V as 4-key vectors per d, from one row offset per chunk
    // and no branch. Keys past khi load the sequence's last key instead: finite values whose
    // scores are masked and whose weights are exactly 0, so they add nothing to the output.
    for (int c = t; c < (KT / 4) * CPR; c += 128) {
      const int kr = (c / CPR) * 4, dc = (c % CPR) * CE;
      const int j0 = kb + kr;
      const int last = khi - 1 - j0;  // the chunk's last key that exists (u <= last)
      const int64_t off = (int64_t)j0 * rs + dc;
      uint4 kv[4], vv[4];
#pragma unroll
      for (int u = 0; u < 4; u++) {
        // (a row stride times at most 3 keys: 32-bit)
        const int du = (u < last ? u : last) * rs32;
        kv[u] = load_chunk<T, PAD>(k_seq + off + du, 0, Dr - dc);
        vv[u] = load_chunk<T, PAD>(v_seq + off + du, 0, Dr - dc);
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
    if constexpr (KM)
      for (int i = t; i < KT; i += 128) sKw[i] = kb + i < khi ? kw[base + kb + i] : 0.f;
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

    // Mask and maximum on the raw scores; the scale (in base 2: scale * log2 e, so exp2 gives the
    // same weights as exp) enters once, inside the exponent. Register r of sub-tile kt is key
    // kb + 32 kt + jl(r) with jl(r) a constant, so the key-range mask is one compare per score
    // against a limit; window bounds add two. A sub-tile wholly inside the sequence (and no
    // window) needs no mask. Lanes of queries past the sequence (the last query tile) compute on
    // a clamped query and are never stored; the maximum exchange pairs lanes of one query only.
    const float scale2 = a.scale * 1.4426950408889634f;
    float tmax = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
      if constexpr (REL) {
        // the sub-tile's distances i - j run over dlo .. dlo + 62: row r of the scratch holds the
        // term of distance dlo + r, computed from the position row of bucket(dlo + r), so a
        // score's term sits at a fixed offset from a per-lane base (no bucket lookup per score).
        // Score (query q, key jl) is at distance row q + 31 - jl: c2p[q][q + 31 - jl] and
        // p2c[jl][q + 31 - jl]. With jl = jc + 4 g (jc a constant per register) the lane's part
        // goes into the base and each read has a constant, non-negative offset. The c2p term is
        // added first, then the p2c term takes the same scratch (a wavefront's LDS operations
        // run in order: its reads of the first term precede the second term's writes).
        const int kj0 = kb + kt * 32, qw0 = q0 + w * 32;
        const int dlo = qw0 - (kj0 + 31);
        float *sw = sRel + w * 32 * RP;
        const T *krow = &sK[(kt * 32 + (lane & 31)) * LDK + g * MF::KLANE];
        auto term = [&](auto p2c_t) {
          constexpr bool P2C = decltype(p2c_t)::value;
          [[maybe_unused]] float16v c2p_lo;
          if constexpr (!P2C && PQC) {
            c2p_lo = float16v{};
#pragma unroll
            for (int s = 0; s < QS; s++) c2p_lo = MF::mma(pk_next[s], qf[s], c2p_lo);
            pos_frags(a.pos_key, dlo - 32, pk_next, std::true_type{});
          } else if constexpr (!P2C) {
            c2p_lo = c2p_block(dlo, std::true_type{});
          }
          [[maybe_unused]] frag_t pq_lo[QS];
          if constexpr (P2C && PQC) pos_frags(a.pos_query, dlo, pq_lo, std::true_type{});
#pragma unroll
          for (int mt = 0; mt < 2; mt++) {
            float16v c = {};
            if constexpr (P2C) {
              [[maybe_unused]] const T *pt = nullptr;
              if constexpr (!PQC) {
                int di = dlo + (lane & 31) + mt * 32 + a.lmax - 1;  // this lane's distance row
                di = di < 0 ? 0 : (di > 2 * a.lmax - 2 ? 2 * a.lmax - 2 : di);
                const int pr = sBucket[di];  // < nb: the relidx table is checked against the tables
                pt = (const T *)a.pos_query + pr * hd + h * Dr;
              }
#pragma unroll
              for (int s = 0; s < QS; s++) {
                typename MF::frag kf;
                if constexpr (sizeof(T) == 2) kf = *reinterpret_cast<const half8v *>(krow + s * MF::KSTEP);
                else kf = krow[s * MF::KSTEP];
                frag_t pf;
                if constexpr (PQC) pf = mt == 0 ? pq_lo[s] : pq_carry[s];
                else pf = load_frag<T, PAD>(pt, s * MF::KSTEP + g * MF::KLANE, Dr);
                // [m][key]: lane = key
                c = MF::mma(pf, kf, c);
              }
            } else {
              c = mt == 0 ? c2p_lo : c2p_carry;  // [m][query]: lane = query
            }
            // registers 4 r4 .. 4 r4 + 3 are distance rows 32 mt + 8 r4 + 4 g + {0..3}
#pragma unroll
            for (int r4 = 0; r4 < 4; r4++) {
              const int mm = mt * 32 + 8 * r4 + 4 * g;
              *reinterpret_cast<float4v *>(&sw[(lane & 31) * RP + mm]) =
                  float4v{c[4 * r4], c[4 * r4 + 1], c[4 * r4 + 2], c[4 * r4 + 3]};
            }
          }
          if constexpr (!P2C) c2p_carry = c2p_lo;
          if constexpr (P2C && PQC)
#pragma unroll
            for (int s = 0; s < QS; s++) pq_carry[s] = pq_lo[s];
          const float *base = P2C ? sw + (lane & 31) + 31 + 4 * g * (RP - 1) : sw + (lane & 31) * (RP + 1) - 4 * g;
#pragma unroll
          for (int r = 0; r < 16; r++) {
            const int jc = 8 * (r >> 2) + (r & 3);
            // read unconditionally (no branch per score); masked pairs are discarded below
            sc[kt][r] = sc[kt][r] + (P2C ? base[jc * (RP - 1)] : base[31 - jc]);
          }
        };
        term(std::false_type{});
        term(std::true_type{});
      }
      const int k0 = kb + kt * 32;
      // bit r: the key of register r has a mask value above 0.5 (all set for 0/1 prefix masks)
      [[maybe_unused]] uint32_t kbits = 0xffffu;
      if constexpr (KM) {
        kbits = 0;
#pragma unroll
        for (int r = 0; r < 16; r++) kbits |= (sKw[kt * 32 + 8 * (r >> 2) + 4 * g + (r & 3)] > 0.5f ? 1u : 0u) << r;
      }
      auto scores = [&](auto masked_t) {
        constexpr bool MASKED = decltype(masked_t)::value;
        [[maybe_unused]] const int lim = khi - k0;  // keys jl < lim exist
        [[maybe_unused]] const int wlo = qi - a.window - k0, whi = qi + a.window - k0;
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int jl = 8 * (r >> 2) + 4 * g + (r & 3);
          float v = sc[kt][r];
          if constexpr (MASKED) {
            bool ok = jl < lim;
            if constexpr (KM) ok = ok && ((kbits >> r) & 1u);
            if constexpr (WIN) ok = ok && jl >= wlo && jl <= whi;
            v = ok ? v : -INFINITY;
          }
          sc[kt][r] = v;
          tmax = fmaxf(tmax, v);
        }
      };
      if (WIN || KM || k0 + 32 > khi) scores(std::true_type{});
      else scores(std::false_type{});
    }
    tmax = fmaxf(tmax, xor32(tmax));
    const float m_new = fmaxf(m_run, tmax * scale2);
    // a query with no key so far keeps its state (corr 1, weights exp2(-inf) = 0)
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float corr = __builtin_amdgcn_exp2f(m_run - m_use);
    float psum = 0.f;
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[kt][r], scale2, -m_use));
        sc[kt][r] = e;
        psum += e;
      }
    }
    l_run = l_run * corr + psum;
    m_run = m_new;
    // (once the maxima settle, no lane rescales)
    if (__any(corr != 1.f)) {
#pragma unroll
      for (int dt = 0; dt < DT; dt++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[dt][r] *= corr;
    }

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

  const float l_tot = l_run + xor32(l_run);
  const float inv = l_tot > 0.f && qkeep ? 1.f / l_tot : 0.f;
  // The output tile leaves through LDS (the K tile's space, free after the key loop's last
  // barrier): a lane holds 4-value pieces of one query row, scattered over 32 rows per store;
  // staged, every row goes out as whole 16-byte chunks.
  constexpr int LDO = LDK;
  static_assert(QT * LDO <= KT * LDK, "the output tile must fit the K tile");
  T *sO = sK;
  typedef T vec4_t __attribute__((ext_vector_type(4)));
  const int ql = w * 32 + (lane & 31);
#pragma unroll
  for (int dt = 0; dt < DT; dt++) {
#pragma unroll
    for (int r4 = 0; r4 < 4; r4++) {
      // registers 4 r4 .. 4 r4 + 3 hold d .. d + 3 of this lane's query
      const int d = dt * 32 + 8 * r4 + 4 * g;
      vec4_t v;
#pragma unroll
      for (int e = 0; e < 4; e++) v[e] = (T)(o[dt][4 * r4 + e] * inv);
      *reinterpret_cast<vec4_t *>(sO + ql * LDO + d) = v;
    }
  }
  __syncthreads();
  // rows of queries past the sequence (clamped lanes) stay in LDS
  const int rows = n - q0 < QT ? n - q0 : QT;
  T *out = (T *)a.ctx + base * hd + h * Dr;
  for (int c = t; c < rows * CPR; c += 128) {
    const int r = c / CPR, dc = (c % CPR) * CE;
    if constexpr (!PAD) {
      *reinterpret_cast<uint4 *>(out + (int64_t)(q0 + r) * hd + dc) = *reinterpret_cast<const uint4 *>(sO + r * LDO + dc);
    } else {
#pragma unroll
      for (int e = 0; e < CE; e++)
        if (dc + e < Dr) out[(int64_t)(q0 + r) * hd + dc + e] = sO[r * LDO + dc + e];
    }
  }
}

template <typename T, bool REL, bool WIN>
void launch_w(const AttnArgs &a, const Packing &p, hipStream_t s) {
  dim3 grid((unsigned)(a.work ? a.nwork : a.ntiles * a.H));
  // the relative path's bucket table: 2 lmax - 1 16-bit entries of dynamic LDS
  const unsigned dyn = REL ? (unsigned)((2 * a.lmax - 1) * sizeof(short) + 3) / 4 * 4 : 0;
  // head dimensions 32 and 64 as they are; others padded to the next of the two (up to 64)
  auto go = [&](auto km_t) {
    constexpr bool KM = decltype(km_t)::value;
    if (a.D == 64) launch((attn_kernel<T, 64, REL, WIN, false, KM>), grid, dim3(128), dyn, s, a, p);
    else if (a.D == 32) launch((attn_kernel<T, 32, REL, WIN, false, KM>), grid, dim3(128), dyn, s, a, p);
    else if (a.D < 32) launch((attn_kernel<T, 32, REL, WIN, true, KM>), grid, dim3(128), dyn, s, a, p);
    else launch((attn_kernel<T, 64, REL, WIN, true, KM>), grid, dim3(128), dyn, s, a, p);
  };
  if (p.row_w) go(std::true_type{});
  else go(std::false_type{});
}

template <typename T, bool REL>
void launch_t(const AttnArgs &a, const Packing &p, hipStream_t s) {
  if (a.window > 0) launch_w<T, REL, true>(a, p, s);
  else launch_w<T, REL, false>(a, p, s);
}

}  // namespace

void attention(bool f16, const AttnArgs &a, const Packing &p, hipStream_t s) {
  if (a.ntiles <= 0) return;
  const bool rel = a.pos_key != nullptr;
  if (f16) {
    if (rel) launch_t<half_t, true>(a, p, s);
    else launch_t<half_t, false>(a, p, s);
  } else {
    if (rel) launch_t<float, true>(a, p, s);
    else launch_t<float, false>(a, p, s);
  }
}

}  // namespace kh
