/*
 * TEST INFRASTRUCTURE — the CPU parity oracle and CPU baseline of the HIP encoder runner.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this library; the
 * product path (libkh_hip.so) never does.
 *
 * f32 restatement of the reference's WASM-SIMD plan executor, src/wasm/plan.ts (AssemblyScript),
 * with the same computations per op kind, the same masking rules, the same summation structure
 * (4 x 16 register tiles over 16-column weight panels, k in order, bias and activation after the
 * sum, two-pass LayerNorm, softmax from the lowest finite f32) and the same work split across
 * threads (matmul items of rb x cb, LayerNorm items of 16 rows, GeGLU items of 8 rows, attention
 * items of qb query rows per (sequence, head), DeBERTa attention per (sequence, head)). Every
 * output element is computed by one thread with the serial code, so results do not depend on the
 * thread count (src/wasm/plan.ts:942-950). Threads are OpenMP threads instead of WASM workers.
 *
 * The multiply-add of the matmul tile is left to the compiler's contraction (-ffp-contract=fast),
 * which corresponds to the reference's relaxed-SIMD build (f32x4.relaxed_madd, src/wasm/plan.ts:
 * 232-238); the plain build keeps mul-then-add. Both builds are the reference's; their difference
 * is far below the 1e-3 logit tolerance.
 *
 * Third-party arithmetic: Mathf.exp / Mathf.tanh / Mathf.sqrt of AssemblyScript 0.28.20 become
 * libm expf / tanhf / sqrtf; this boundary is pinned only to the tolerance of the f64 checks in
 * tests/test_oracle.py.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define KHO_GEMM_P 1
#define KHO_GEMM_NT 2
#define KHO_LN 3
#define KHO_EMBLN 4
#define KHO_ADD 5
#define KHO_GATHER 6
#define KHO_POOL 7
#define KHO_GEGLU 8
#define KHO_ROPE 9
#define KHO_ATTSCORE 11
#define KHO_ATTSOFTMAX 12
#define KHO_ATTPV 13
#define KHO_ATTREL 14
#define KHO_ATTSOFTREL 15
#define KHO_ATTSTD 16
#define KHO_ATTRELF 17
#define KHO_MASKLOGITS 18

/* One op record: pointer arguments, integer arguments, float arguments in the order the
 * reference's host encodes them (src/plan/wasm.ts:330-407). */
typedef struct {
  int32_t code;
  int32_t rows_fixed; /* >= 0: fixed row count of the op; -1: the rows of the call */
  int32_t pad[2];
  void *p[8];
  int32_t v[14];
  float f[2];
} kho_op;

/* lowest finite f32: start of a softmax maximum (src/wasm/plan.ts:38-39) */
static const float LOWEST = -3.40282346638528859812e38f;

/* ---- exp and GELU ------------------------------------------------------------------------- */

/* e^x as the reference's vexp (src/wasm/plan.ts:57-75): x = n ln2 + r, e^r by the minimax
 * polynomial of Cephes expf (Moshier, Cephes Math Library), 2^n through the exponent bits,
 * inputs clamped to [-87.3, 88.3]. */
static inline float vexp1(float x) {
  x = fmaxf(fminf(x, 88.3762626647949f), -87.3365447504f);
  float n = floorf(x * 1.44269504088896341f + 0.5f);
  float r = x - n * 0.693359375f;
  r = r - n * -2.12194440e-4f;
  float y = 1.9875691500e-4f;
  y = y * r + 1.3981999507e-3f;
  y = y * r + 8.3334519073e-3f;
  y = y * r + 4.1665795894e-2f;
  y = y * r + 1.6666665459e-1f;
  y = y * r + 5.0000001201e-1f;
  y = y * r * r + r + 1.0f;
  union { int32_t i; float f; } p;
  p.i = ((int32_t)n + 127) << 23;
  return y * p.f;
}

/* GELU by erf, Abramowitz-Stegun 7.1.26, with the vexp above (vgelu, src/wasm/plan.ts:81-93) */
static inline float vgelu1(float v) {
  float u = v * 0.7071067811865476f;
  float t = 1.0f / (1.0f + 0.3275911f * fabsf(u));
  float p = 1.061405429f * t - 1.453152027f;
  p = p * t + 1.421413741f;
  p = p * t - 0.284496736f;
  p = p * t + 0.254829592f;
  p = p * t;
  float e = 1.0f - p * vexp1(-(u * u));
  float se = v >= 0 ? e : -e;
  return 0.5f * v * (1.0f + se);
}

/* the same GELU with libm exp (gelu, src/wasm/plan.ts:99-107) */
static inline float gelu_m(float v) {
  float u = v * 0.7071067811865476f;
  float t = 1.0f / (1.0f + 0.3275911f * fabsf(u));
  float p = (((((1.061405429f * t - 1.453152027f) * t) + 1.421413741f) * t - 0.284496736f) * t
             + 0.254829592f) * t;
  float e = 1.0f - p * expf(-u * u);
  return 0.5f * v * (1.0f + (v >= 0 ? e : -e));
}

/* ACT 0 none, 1 relu, 2 gelu, 3 tanh, 4 silu (src/wasm/plan.ts:109-116) */
static inline float activate(float v, int act) {
  if (act == 1) return fmaxf(v, 0.0f);
  if (act == 2) return gelu_m(v);
  if (act == 3) return tanhf(v);
  if (act == 4) return v / (1.0f + expf(-v));
  return v;
}

static inline float fin(float acc, float alpha, const float *bias, int n, int act) {
  float v = acc * alpha;
  if (bias) v += bias[n];
  return act ? activate(v, act) : v;
}

/* ---- matrix products ---------------------------------------------------------------------- */

/* bias and activation over an M x N block (src/wasm/plan.ts:130-154) */
static void bias_act(float *c, int ldc, const float *bias, int M, int N, int act) {
  for (int m = 0; m < M; m++) {
    float *r = c + (size_t)m * ldc;
    if (act == 2 || act == 0) {
      for (int n = 0; n < N; n++) {
        float v = r[n];
        if (bias) v += bias[n];
        r[n] = act ? vgelu1(v) : v;
      }
      continue;
    }
    for (int n = 0; n < N; n++) {
      float v = r[n];
      if (bias) v += bias[n];
      r[n] = act ? activate(v, act) : v;
    }
  }
}

/* C[m, n] = sum_k A[m, k] B[k, n], B row-major [K, N] with stride ldb; 4 rows x 16 columns per
 * tile, columns past N loaded and not stored (src/wasm/plan.ts:170-230). */
static void gemm_nn(const float *a, int lda, const float *b, int ldb, float *c, int ldc,
                    int M, int N, int K) {
  for (int mb = 0; mb < M; mb += 4) {
    int rows = M - mb < 4 ? M - mb : 4;
    for (int nb = 0; nb < N; nb += 16) {
      float acc[4][16];
      memset(acc, 0, sizeof(acc));
      int lanes = N - nb < 16 ? N - nb : 16;
      for (int k = 0; k < K; k++) {
        const float *w = b + (size_t)k * ldb + nb;
        float wv[16];
        for (int l = 0; l < 16; l++) wv[l] = l < lanes ? w[l] : 0.0f;
        for (int r = 0; r < rows; r++) {
          float x = a[(size_t)(mb + r) * lda + k];
          for (int l = 0; l < 16; l++) acc[r][l] += x * wv[l];
        }
      }
      for (int r = 0; r < rows; r++)
        for (int l = 0; l < lanes; l++) c[(size_t)(mb + r) * ldc + nb + l] = acc[r][l];
    }
  }
}

/* C[m, n] = sum_k A[m, k] B[k, n] for B packed in panels [ceil(N/16)][K][16]: full 4-row tiles,
 * then single rows (src/wasm/plan.ts:240-295). */
static void gemm_p(const float *a, int lda, const float *p, float *c, int ldc, int M, int N, int K) {
  size_t ps = (size_t)K * 16;
  int m = 0;
  for (; m + 4 <= M; m += 4) {
    const float *ar = a + (size_t)m * lda;
    for (int nb = 0; nb < N; nb += 16) {
      float acc[4][16];
      memset(acc, 0, sizeof(acc));
      const float *bp = p + (size_t)(nb >> 4) * ps;
      for (int k = 0; k < K; k++) {
        const float *w = bp + (size_t)k * 16;
        float x0 = ar[k], x1 = ar[lda + k], x2 = ar[2 * (size_t)lda + k], x3 = ar[3 * (size_t)lda + k];
        for (int l = 0; l < 16; l++) {
          acc[0][l] += x0 * w[l];
          acc[1][l] += x1 * w[l];
          acc[2][l] += x2 * w[l];
          acc[3][l] += x3 * w[l];
        }
      }
      int lanes = N - nb < 16 ? N - nb : 16;
      for (int r = 0; r < 4; r++)
        for (int l = 0; l < lanes; l++) c[(size_t)(m + r) * ldc + nb + l] = acc[r][l];
    }
  }
  for (; m < M; m++) {
    const float *ar = a + (size_t)m * lda;
    for (int nb = 0; nb < N; nb += 16) {
      float acc[16];
      memset(acc, 0, sizeof(acc));
      const float *bp = p + (size_t)(nb >> 4) * ps;
      for (int k = 0; k < K; k++) {
        float x = ar[k];
        for (int l = 0; l < 16; l++) acc[l] += x * bp[(size_t)k * 16 + l];
      }
      int lanes = N - nb < 16 ? N - nb : 16;
      for (int l = 0; l < lanes; l++) c[(size_t)m * ldc + nb + l] = acc[l];
    }
  }
}

/* sum_k a[k] w[k]: four lanes, then a scalar tail (src/wasm/plan.ts:297-307) */
static inline float dot4(const float *a, const float *w, int K) {
  float acc[4] = {0, 0, 0, 0};
  int k = 0;
  for (; k + 4 <= K; k += 4)
    for (int l = 0; l < 4; l++) acc[l] += a[k + l] * w[k + l];
  float s = acc[0] + acc[1] + acc[2] + acc[3];
  for (; k < K; k++) s += a[k] * w[k];
  return s;
}

/* C[m, n] = act(alpha sum_k A[m, k] B[n, k] + bias[n]) with B row-major [N, K]
 * (src/wasm/plan.ts:309-368); dot products along k. */
static void gemm_nt(const float *a, int lda, const float *b, int ldb, float *c, int ldc,
                    const float *bias, int M, int N, int K, float alpha, int act) {
  for (int m = 0; m < M; m++) {
    const float *r = a + (size_t)m * lda;
    for (int n = 0; n < N; n++)
      c[(size_t)m * ldc + n] = fin(dot4(r, b + (size_t)n * ldb, K), alpha, bias, n, act);
  }
}

/* ---- normalization ------------------------------------------------------------------------ */

/* ((v - mean) inv w + bias) scale, variance = mean((v - mean)^2) (src/wasm/plan.ts:386-411) */
static void norm_row(float *o, int N, const float *w, const float *bias, float eps, float scale) {
  float acc[4] = {0, 0, 0, 0};
  int d = 0;
  for (; d + 4 <= N; d += 4)
    for (int l = 0; l < 4; l++) acc[l] += o[d + l];
  float s = acc[0] + acc[1] + acc[2] + acc[3];
  for (; d < N; d++) s += o[d];
  float mean = s / (float)N;
  float sq4[4] = {0, 0, 0, 0};
  d = 0;
  for (; d + 4 <= N; d += 4)
    for (int l = 0; l < 4; l++) {
      float x = o[d + l] - mean;
      sq4[l] += x * x;
    }
  float sq = sq4[0] + sq4[1] + sq4[2] + sq4[3];
  for (; d < N; d++) {
    float x = o[d] - mean;
    sq += x * x;
  }
  float inv = 1.0f / sqrtf(sq / (float)N + eps);
  for (d = 0; d < N; d++) o[d] = ((o[d] - mean) * inv * w[d] + bias[d]) * scale;
}

/* MODE 0 LN(a), 1 LN(a) mask[row], 2 LN(a + b), rows r0 .. r1-1 (src/wasm/plan.ts:413-431) */
static void layernorm(const float *a, const float *b, const float *w, const float *bias,
                      const float *mask, float *out, int N, int mode, float eps, int r0, int r1) {
  for (int r = r0; r < r1; r++) {
    float *o = out + (size_t)r * N;
    const float *x = a + (size_t)r * N;
    if (mode == 2) {
      const float *y = b + (size_t)r * N;
      for (int d = 0; d < N; d++) o[d] = x[d] + y[d];
    } else if (o != x) {
      memcpy(o, x, (size_t)N * 4);
    }
    norm_row(o, N, w, bias, eps, mode == 1 ? mask[r] : 1.0f);
  }
}

/* LN(word + pos + type) (times the mask with MASKMUL); the position row is tt >> 16 with
 * POSIDS, else (r % L) + offset, clamped to maxpos - 1 (src/wasm/plan.ts:433-447). */
static void embln(const float *word, const float *pos, const float *typ, const uint32_t *tt,
                  const float *w, const float *bias, const float *mask, float *out, int N, int L,
                  int offset, int maxpos, float eps, int maskmul, int posids, int r0, int r1) {
  for (int r = r0; r < r1; r++) {
    uint32_t t = tt[r];
    int prow = posids ? (int)(t >> 16) : (r % L) + offset;
    if (prow > maxpos - 1) prow = maxpos - 1;
    const float *p = pos + (size_t)prow * N;
    const float *y = typ + (size_t)(t & 0xffff) * N;
    const float *x = word + (size_t)r * N;
    float *o = out + (size_t)r * N;
    for (int d = 0; d < N; d++) o[d] = x[d] + p[d] + y[d];
    norm_row(o, N, w, bias, eps, maskmul ? mask[r] : 1.0f);
  }
}

/* ---- small elementwise ops ---------------------------------------------------------------- */

/* MODE 0 dst += src; MODE 1 dst[i] += src[(i / (N L)) N + i % N] (src/wasm/plan.ts:451-464) */
static void add_op(float *dst, const float *src, long count, int N, int mode, int L) {
  if (mode == 0) {
    for (long i = 0; i < count; i++) dst[i] += src[i];
    return;
  }
  for (long i = 0; i < count; i++) dst[i] += src[(i / ((long)N * L)) * N + i % N];
}

/* states[g] = x[b L + markers[b 3 K + g - b K]] (src/wasm/plan.ts:466-472) */
static void gather(const uint32_t *markers, const float *x, float *states, int K, int D, int L,
                   int total) {
  for (int g = 0; g < total; g++) {
    int b = g / K;
    long row = (long)b * L + markers[b * 3 * K + (g - b * K)];
    memcpy(states + (size_t)g * D, x + (size_t)row * D, (size_t)D * 4);
  }
}

/* logits[k] = raw[k] / temp where the marker's mask word (f32 bits at b * 3K + K + k mod K, b = k / K)
 * exceeds 0.5, else -1e4 (src/wasm/plan.ts:545-551) */
static void masklogits(const float *raw, const uint32_t *packed, float *logits, int K, float temp, int total) {
  for (int k = 0; k < total; k++) {
    int b = k / K;
    float m;
    memcpy(&m, packed + (size_t)b * 3 * K + K + (k - b * K), 4);
    logits[k] = m > 0.5f ? raw[k] / temp : -1e4f;
  }
}

/* MODE 0 masked mean (count floor 1e-9), MODE 1 masked max (src/wasm/plan.ts:474-498) */
static void pool(const float *x, const float *mask, float *out, int L, int N, int mode, int batch) {
  for (int b = 0; b < batch; b++) {
    float *o = out + (size_t)b * N;
    for (int d = 0; d < N; d++) o[d] = 0;
    float cnt = 0;
    int found = 0;
    for (int i = 0; i < L; i++) {
      float m = mask[(size_t)b * L + i];
      const float *xr = x + ((size_t)b * L + i) * N;
      if (mode == 0) {
        if (m == 0) continue;
        for (int d = 0; d < N; d++) o[d] += m * xr[d];
        cnt += m;
      } else if (m > 0.5f) {
        for (int d = 0; d < N; d++) o[d] = found ? fmaxf(o[d], xr[d]) : xr[d];
        found = 1;
      }
    }
    if (mode == 0) {
      float den = fmaxf(cnt, 1e-9f);
      for (int d = 0; d < N; d++) o[d] /= den;
    }
  }
}

/* gate = gelu(mid[:, :I]) mid[:, I:] (src/wasm/plan.ts:500-508) */
static void geglu(const float *mid, float *gate, int I, int r0, int r1) {
  for (int r = r0; r < r1; r++) {
    const float *m = mid + (size_t)r * 2 * I;
    float *g = gate + (size_t)r * I;
    for (int j = 0; j < I; j++) g[j] = vgelu1(m[j]) * m[I + j];
  }
}

/* rotate-half RoPE on the q and k parts, table [L][cos D | sin D] (src/wasm/plan.ts:510-528) */
static void rope(float *qkv, const float *cossin, int L, int H, int D, int rows) {
  int hd = H * D, half = D / 2;
  for (int i = 0; i < rows; i++) {
    const float *t = cossin + (size_t)(i % L) * 2 * D;
    for (int s = 0; s < 2 * H; s++) {
      float *base = qkv + (size_t)i * 3 * hd + (size_t)s * D;
      for (int d = 0; d < half; d++) {
        float x = base[d], y = base[d + half], c = t[d], sn = t[D + d];
        base[d] = x * c - y * sn;
        base[d + half] = y * c + x * sn;
      }
    }
  }
}

/* ---- attention ---------------------------------------------------------------------------- */

/* first and last valid key per sequence; first = L when none (src/wasm/plan.ts:555-569) */
static void key_ranges(const float *mask, int32_t *kinfo, int L, int batch) {
  for (int b = 0; b < batch; b++) {
    int first = L, last = 0;
    for (int j = 0; j < L; j++) {
      if (mask[(size_t)b * L + j] > 0.5f) {
        if (first == L) first = j;
        last = j;
      }
    }
    kinfo[2 * b] = first;
    kinfo[2 * b + 1] = last;
  }
}

static inline int seq_rows(int rows, int b, int L) {
  int r = rows - b * L;
  return L < r ? L : r;
}

static inline int keep(const float *mask, int j, int il, int window) {
  if (mask[j] <= 0.5f) return 0;
  return window == 0 || abs(il - j) <= window;
}

/* Masked softmax over keys first .. first+n-1 of one score row (src/wasm/plan.ts:573-634):
 * masked keys and keys outside the window get exactly 0, a masked query row is all 0; `dense`
 * (every key valid, no window) uses vexp, the general path libm exp. */
static void softmax_row(float *p, int n, const float *mask, int first, int il, int window,
                        int qmask, int dense, float scale) {
  if (!qmask) {
    memset(p, 0, (size_t)n * 4);
    return;
  }
  if (dense) {
    float m = LOWEST;
    for (int j = 0; j < n; j++) {
      float x = p[j] * scale;
      p[j] = x;
      m = fmaxf(m, x);
    }
    float s = 0;
    for (int j = 0; j < n; j++) {
      float e = vexp1(p[j] - m);
      p[j] = e;
      s += e;
    }
    float vi = s > 0 ? 1.0f / s : 0.0f;
    for (int j = 0; j < n; j++) p[j] *= vi;
    return;
  }
  if (scale != 1.0f)
    for (int j = 0; j < n; j++) p[j] *= scale;
  float mx = LOWEST;
  for (int j = 0; j < n; j++)
    if (keep(mask, first + j, il, window)) mx = fmaxf(mx, p[j]);
  float sum = 0;
  for (int j = 0; j < n; j++) {
    float e = 0;
    if (keep(mask, first + j, il, window)) e = expf(p[j] - mx);
    p[j] = e;
    sum += e;
  }
  float inv = sum > 0 ? 1.0f / sum : 0.0f;
  for (int j = 0; j < n; j++) p[j] *= inv;
}

/* rows x[j ld + d] into panels [ceil(n/16)][D][16], lanes past n zero (src/wasm/plan.ts:636-650) */
static void pack_panels(const float *x, int ld, int n, int D, float *out) {
  int nb = (n + 15) >> 4;
  for (int pb = 0; pb < nb; pb++) {
    float *base = out + (size_t)pb * D * 16;
    int j0 = pb * 16;
    int lanes = n - j0 < 16 ? n - j0 : 16;
    if (lanes < 16) memset(base, 0, (size_t)D * 16 * 4);
    for (int l = 0; l < lanes; l++) {
      const float *src = x + (size_t)(j0 + l) * ld;
      for (int d = 0; d < D; d++) base[d * 16 + l] = src[d];
    }
  }
}

static int all_keys(const float *mask, int first, int last) {
  for (int j = first; j <= last; j++)
    if (mask[j] <= 0.5f) return 0;
  return 1;
}

/* scores[(row H + h) L + j] = SCALE q_row . k_j for keys first .. last (src/wasm/plan.ts:663-679) */
static void attscore(const float *qkv, float *scores, const int32_t *kinfo, int L, int H, int D,
                     float scale, int rows, int batch) {
  int hd = H * D;
  for (int b = 0; b < batch; b++) {
    int nq = seq_rows(rows, b, L), first = kinfo[2 * b], last = kinfo[2 * b + 1];
    if (nq <= 0 || first >= L) continue;
    for (int h = 0; h < H; h++)
      gemm_nt(qkv + (size_t)b * L * 3 * hd + h * D, 3 * hd,
              qkv + ((size_t)b * L + first) * 3 * hd + (H + h) * D, 3 * hd,
              scores + ((size_t)b * L * H + h) * L + first, H * L, NULL, nq, last - first + 1, D,
              scale, 0);
  }
}

static void attsoftmax(const float *mask, float *scores, const int32_t *kinfo, int L, int H,
                       int window, int rows) {
  for (int i = 0; i < rows; i++) {
    int b = i / L, first = kinfo[2 * b], last = kinfo[2 * b + 1];
    if (first >= L) continue;
    for (int h = 0; h < H; h++)
      softmax_row(scores + ((size_t)i * H + h) * L + first, last - first + 1, mask + (size_t)b * L,
                  first, i - b * L, window, mask[i] > 0.5f, 0, 1.0f);
  }
}

/* ctx[row][h D + d] = sum_j P[row][h][j] v_j (src/wasm/plan.ts:696-715) */
static void attpv(const float *scores, const float *qkv, float *ctx, const int32_t *kinfo, int L,
                  int H, int D, int rows, int batch) {
  int hd = H * D;
  for (int b = 0; b < batch; b++) {
    int nq = seq_rows(rows, b, L);
    if (nq <= 0) continue;
    int first = kinfo[2 * b], last = kinfo[2 * b + 1];
    if (first >= L) {
      memset(ctx + (size_t)b * L * hd, 0, (size_t)nq * hd * 4);
      continue;
    }
    for (int h = 0; h < H; h++)
      gemm_nn(scores + ((size_t)b * L * H + h) * L + first, H * L,
              qkv + ((size_t)b * L + first) * 3 * hd + (2 * H + h) * D, 3 * hd,
              ctx + (size_t)b * L * hd + h * D, hd, nq, D, last - first + 1);
  }
}

/* rel[row][h][m] = x_row . T[MOFF + m] over the positions the valid pairs reach
 * (src/wasm/plan.ts:717-735) */
static void attrel(const float *qkv, const float *table, const uint32_t *relidx, float *out,
                   const int32_t *kinfo, int H, int D, int NM, int moff, int part, int L, int rows,
                   int batch) {
  int hd = H * D;
  for (int b = 0; b < batch; b++) {
    int nq = seq_rows(rows, b, L), first = kinfo[2 * b], last = kinfo[2 * b + 1];
    if (nq <= 0 || first >= L) continue;
    int lo = (int)relidx[(size_t)first * L + last] - moff;
    int hi = (int)relidx[(size_t)last * L + first] - moff;
    for (int h = 0; h < H; h++)
      gemm_nt(qkv + (size_t)b * L * 3 * hd + (part * H + h) * D, 3 * hd,
              table + (size_t)(moff + lo) * hd + h * D, hd,
              out + ((size_t)b * L * H + h) * NM + lo, H * NM, NULL, nq, hi - lo + 1, D, 1.0f, 0);
  }
}

/* scores += (c2p[i][h][m] + p2c[j][h][m]) INVSCALE, m = relidx[i][j] - MOFF, then the masked
 * softmax (src/wasm/plan.ts:737-762) */
static void attsoftrel(const float *mask, const uint32_t *relidx, const float *c2p, const float *p2c,
                       float *scores, const int32_t *kinfo, int L, int H, int NM, int moff,
                       float invscale, int rows) {
  for (int i = 0; i < rows; i++) {
    int b = i / L, il = i - b * L, first = kinfo[2 * b], last = kinfo[2 * b + 1];
    if (first >= L) continue;
    int qm = mask[i] > 0.5f;
    for (int h = 0; h < H; h++) {
      float *p = scores + ((size_t)i * H + h) * L + first;
      if (qm) {
        const float *c = c2p + ((size_t)i * H + h) * NM;
        for (int j = first; j <= last; j++) {
          if (mask[(size_t)b * L + j] <= 0.5f) continue;
          int m = (int)relidx[(size_t)il * L + j] - moff;
          p[j - first] += (c[m] + p2c[(((size_t)b * L + j) * H + h) * NM + m]) * invscale;
        }
      }
      softmax_row(p, last - first + 1, mask + (size_t)b * L, first, il, 0, qm, 0, 1.0f);
    }
  }
}

/* fused standard attention of sequence b, head h, query rows i0 .. i1-1
 * (src/wasm/plan.ts:764-789) */
static void attstd_block(const float *qkv, const float *mask, float *ctx, const int32_t *kinfo,
                         float *scratch, int L, int H, int D, float scale, int window, int rows,
                         int b, int h, int i0, int i1) {
  int hd = H * D;
  int sr = seq_rows(rows, b, L);
  int e = i1 < sr ? i1 : sr;
  if (e <= i0) return;
  int first = kinfo[2 * b], last = kinfo[2 * b + 1];
  if (first >= L) {
    for (int i = i0; i < e; i++) memset(ctx + ((size_t)b * L + i) * hd + h * D, 0, (size_t)D * 4);
    return;
  }
  int nk = last - first + 1;
  int dense = window == 0 && all_keys(mask + (size_t)b * L, first, last);
  float *kp = scratch + (size_t)L * L;
  pack_panels(qkv + ((size_t)b * L + first) * 3 * hd + (H + h) * D, 3 * hd, nk, D, kp);
  gemm_p(qkv + ((size_t)b * L + i0) * 3 * hd + h * D, 3 * hd, kp, scratch, L, e - i0, nk, D);
  for (int i = i0; i < e; i++)
    softmax_row(scratch + (size_t)(i - i0) * L, nk, mask + (size_t)b * L, first, i, window,
                mask[(size_t)b * L + i] > 0.5f, dense, scale);
  gemm_nn(scratch, L, qkv + ((size_t)b * L + first) * 3 * hd + (2 * H + h) * D, 3 * hd,
          ctx + ((size_t)b * L + i0) * hd + h * D, hd, e - i0, D, nk);
}

/* fused DeBERTa attention of sequence b, head h: (q.k + q.posKey[p] + k.posQuery[p]) / SCALE
 * with p = relidx[i][j] (src/wasm/plan.ts:791-840) */
static void attrelf(const float *qkv, const float *pos_key, const float *pos_query,
                    const uint32_t *relidx, const float *mask, float *ctx, const int32_t *kinfo,
                    float *scratch, int L, int H, int D, float scale, int rows, int b, int h) {
  int hd = H * D, S = 2 * L;
  float *c2p = scratch + (size_t)L * L;
  float *p2c = c2p + (size_t)L * S;
  int nq = seq_rows(rows, b, L);
  if (nq <= 0) return;
  int first = kinfo[2 * b], last = kinfo[2 * b + 1];
  if (first >= L) {
    for (int i = 0; i < nq; i++) memset(ctx + ((size_t)b * L + i) * hd + h * D, 0, (size_t)D * 4);
    return;
  }
  int nk = last - first + 1;
  int lo = (int)relidx[(size_t)first * L + last];
  int np = (int)relidx[(size_t)last * L + first] - lo + 1;
  const float *q = qkv + (size_t)b * L * 3 * hd;
  float inv = 1.0f / scale;
  int dense = all_keys(mask + (size_t)b * L, first, last);
  float *kp = p2c + (size_t)L * S;
  pack_panels(q + (size_t)first * 3 * hd + (H + h) * D, 3 * hd, nk, D, kp);
  gemm_p(q + h * D, 3 * hd, kp, scratch, L, nq, nk, D);
  pack_panels(pos_key + (size_t)lo * hd + h * D, hd, np, D, kp);
  gemm_p(q + h * D, 3 * hd, kp, c2p, S, nq, np, D);
  pack_panels(pos_query + (size_t)lo * hd + h * D, hd, np, D, kp);
  gemm_p(q + (size_t)first * 3 * hd + (H + h) * D, 3 * hd, kp, p2c, S, nk, np, D);
  for (int i = 0; i < nq; i++) {
    float *p = scratch + (size_t)i * L;
    int qm = mask[(size_t)b * L + i] > 0.5f;
    if (qm) {
      for (int j = first; j <= last; j++) {
        int m = (int)relidx[(size_t)i * L + j] - lo;
        p[j - first] = (p[j - first] + c2p[(size_t)i * S + m] + p2c[(size_t)(j - first) * S + m]) * inv;
      }
    }
    softmax_row(p, nk, mask + (size_t)b * L, first, i, 0, qm, dense, 1.0f);
  }
  gemm_nn(scratch, L, q + (size_t)first * 3 * hd + (2 * H + h) * D, 3 * hd,
          ctx + (size_t)b * L * hd + h * D, hd, nq, D, nk);
}

/* ---- stream ------------------------------------------------------------------------------- */

typedef struct {
  int L, batch, rows;
  const float *mask;
  int32_t *kinfo;
  float *scratch;
  size_t scratch_per_thread; /* floats */
  int rb, cb, qb;
  long min_work;
} kho_ctx;

static inline int cdiv(int a, int b) { return (a + b - 1) / b; }
static inline int op_rows(const kho_op *op, int rows) { return op->rows_fixed >= 0 ? op->rows_fixed : rows; }

static void serial(const kho_ctx *cx, const kho_op *op, int n, float *scratch) {
  int L = cx->L, batch = cx->batch;
  const int32_t *kinfo = cx->kinfo;
  void *const *p = op->p;
  const int32_t *v = op->v;
  switch (op->code) {
  case KHO_GEMM_P:
  case KHO_GEMM_NT: {
    /* a, w, bias, c; N, K, act, M */
    int N = v[0], K = v[1], act = v[2], m = n < v[3] ? n : v[3];
    if (op->code == KHO_GEMM_P) {
      gemm_p((const float *)p[0], K, (const float *)p[1], (float *)p[3], N, m, N, K);
      if (p[2] || act) bias_act((float *)p[3], N, (const float *)p[2], m, N, act);
    } else {
      gemm_nt((const float *)p[0], K, (const float *)p[1], K, (float *)p[3], N, (const float *)p[2],
              m, N, K, 1.0f, act);
    }
    break;
  }
  case KHO_LN:
    layernorm((const float *)p[0], (const float *)p[1], (const float *)p[2], (const float *)p[3],
              (const float *)p[4], (float *)p[5], v[0], v[1], op->f[0], 0, n);
    break;
  case KHO_EMBLN:
    embln((const float *)p[0], (const float *)p[1], (const float *)p[2], (const uint32_t *)p[3],
          (const float *)p[4], (const float *)p[5], (const float *)p[6], (float *)p[7], v[0], v[1],
          v[2], v[3], op->f[0], v[4], v[5], 0, n);
    break;
  case KHO_ADD: {
    long total = (long)v[0], cnt = (long)n * v[1];
    add_op((float *)p[0], (const float *)p[1], total < cnt ? total : cnt, v[1], v[2], v[3]);
    break;
  }
  case KHO_GATHER:
    gather((const uint32_t *)p[0], (const float *)p[1], (float *)p[2], v[0], v[1], v[2], v[3]);
    break;
  case KHO_MASKLOGITS:
    masklogits((const float *)p[0], (const uint32_t *)p[1], (float *)p[2], v[0], op->f[0], v[1]);
    break;
  case KHO_POOL:
    pool((const float *)p[0], (const float *)p[1], (float *)p[2], v[0], v[1], v[2], v[3]);
    break;
  case KHO_GEGLU:
    geglu((const float *)p[0], (float *)p[1], v[0], 0, n);
    break;
  case KHO_ROPE:
    rope((float *)p[0], (const float *)p[1], v[0], v[1], v[2], n);
    break;
  case KHO_ATTSCORE:
    attscore((const float *)p[0], (float *)p[1], kinfo, v[0], v[1], v[2], op->f[0], n, batch);
    break;
  case KHO_ATTSOFTMAX:
    attsoftmax((const float *)p[0], (float *)p[1], kinfo, v[0], v[1], v[2], n);
    break;
  case KHO_ATTPV:
    attpv((const float *)p[0], (const float *)p[1], (float *)p[2], kinfo, v[0], v[1], v[2], n, batch);
    break;
  case KHO_ATTREL:
    attrel((const float *)p[0], (const float *)p[1], (const uint32_t *)p[2], (float *)p[3], kinfo,
           v[0], v[1], v[2], v[3], v[4], v[5], n, batch);
    break;
  case KHO_ATTSOFTREL:
    attsoftrel((const float *)p[0], (const uint32_t *)p[1], (const float *)p[2], (const float *)p[3],
               (float *)p[4], kinfo, v[0], v[1], v[2], v[3], op->f[0], n);
    break;
  case KHO_ATTSTD:
    for (int b = 0; b < batch; b++)
      for (int h = 0; h < v[1]; h++)
        attstd_block((const float *)p[0], (const float *)p[1], (float *)p[2], kinfo, scratch, v[0],
                     v[1], v[2], op->f[0], v[3], n, b, h, 0, v[0]);
    break;
  case KHO_ATTRELF:
    for (int b = 0; b < batch; b++)
      for (int h = 0; h < v[1]; h++)
        attrelf((const float *)p[0], (const float *)p[1], (const float *)p[2], (const uint32_t *)p[3],
                (const float *)p[4], (float *)p[5], kinfo, scratch, v[0], v[1], v[2], op->f[0], n, b, h);
    break;
  default:
    break;
  }
  (void)L;
}

/* work items of an op; 0 or 1: the op runs on one thread (src/wasm/plan.ts:961-980) */
static int items_of(const kho_ctx *cx, const kho_op *op, int n) {
  switch (op->code) {
  case KHO_GEMM_P: {
    int m = n < op->v[3] ? n : op->v[3];
    if ((long)m * op->v[0] * op->v[1] < cx->min_work) return 0;
    return cdiv(m, cx->rb) * cdiv(op->v[0], cx->cb);
  }
  case KHO_LN: return n >= 64 ? cdiv(n, 16) : 0;
  case KHO_GEGLU: return n >= 16 ? cdiv(n, 8) : 0;
  case KHO_ATTSTD: {
    int L = op->v[0];
    return cx->batch * op->v[1] * cdiv(cx->batch == 1 ? (n < L ? n : L) : L, cx->qb);
  }
  case KHO_ATTRELF: return cx->batch * op->v[1];
  default: return 0;
  }
}

/* item i of an op (src/wasm/plan.ts:982-1021) */
static void work(const kho_ctx *cx, const kho_op *op, int n, int i, float *scratch) {
  void *const *p = op->p;
  const int32_t *v = op->v;
  switch (op->code) {
  case KHO_GEMM_P: {
    int N = v[0], K = v[1], act = v[2], m = n < v[3] ? n : v[3];
    int nc = cdiv(N, cx->cb);
    int r0 = (i / nc) * cx->rb, c0 = (i % nc) * cx->cb;
    int rr = cx->rb < m - r0 ? cx->rb : m - r0;
    int cc = cx->cb < N - c0 ? cx->cb : N - c0;
    float *c = (float *)p[3] + (size_t)r0 * N + c0;
    gemm_p((const float *)p[0] + (size_t)r0 * K, K, (const float *)p[1] + (size_t)(c0 >> 4) * K * 16,
           c, N, rr, cc, K);
    const float *bias = (const float *)p[2];
    if (bias || act) bias_act(c, N, bias ? bias + c0 : NULL, rr, cc, act);
    break;
  }
  case KHO_LN: {
    int r1 = i * 16 + 16 < n ? i * 16 + 16 : n;
    layernorm((const float *)p[0], (const float *)p[1], (const float *)p[2], (const float *)p[3],
              (const float *)p[4], (float *)p[5], v[0], v[1], op->f[0], i * 16, r1);
    break;
  }
  case KHO_GEGLU: {
    int r1 = i * 8 + 8 < n ? i * 8 + 8 : n;
    geglu((const float *)p[0], (float *)p[1], v[0], i * 8, r1);
    break;
  }
  case KHO_ATTSTD: {
    int L = v[0], H = v[1];
    int nb = cdiv(cx->batch == 1 ? (n < L ? n : L) : L, cx->qb);
    int b = i / (H * nb), h = (i / nb) % H, q0 = (i % nb) * cx->qb;
    attstd_block((const float *)p[0], (const float *)p[1], (float *)p[2], cx->kinfo, scratch, L, H,
                 v[2], op->f[0], v[3], n, b, h, q0, q0 + cx->qb);
    break;
  }
  case KHO_ATTRELF: {
    int H = v[1];
    attrelf((const float *)p[0], (const float *)p[1], (const float *)p[2], (const uint32_t *)p[3],
            (const float *)p[4], (float *)p[5], cx->kinfo, scratch, v[0], H, v[2], op->f[0], n,
            i / H, i % H);
    break;
  }
  default:
    break;
  }
}

/* One forward over `rows` rows: key ranges from the mask, then every op in order, an op with
 * several items spread over `threads` OpenMP threads (src/wasm/plan.ts:854-873, 1023-1049).
 * Returns 0, or -1 for an unknown op code. */
int kho_run(const kho_op *ops, int nops, int L, int batch, const float *mask, int32_t *kinfo,
            float *scratch, size_t scratch_per_thread, int rows, int threads, int rb, int cb,
            int qb, long min_work) {
  kho_ctx cx = {L, batch, rows, mask, kinfo, scratch, scratch_per_thread,
                rb > 0 ? rb : 16, cb > 0 ? cb : 64, qb > 0 ? qb : 32, min_work > 0 ? min_work : 65536};
  for (int o = 0; o < nops; o++)
    if (ops[o].code < 1 || ops[o].code > KHO_MASKLOGITS || ops[o].code == 10) return -1;
  key_ranges(mask, kinfo, L, batch);
  for (int o = 0; o < nops; o++) {
    const kho_op *op = &ops[o];
    int n = op_rows(op, rows);
    int items = threads > 1 ? items_of(&cx, op, n) : 0;
    if (items > 1) {
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
#endif
      for (int i = 0; i < items; i++) {
        int tid = 0;
#ifdef _OPENMP
        tid = omp_get_thread_num();
#endif
        work(&cx, op, n, i, scratch + (size_t)tid * scratch_per_thread);
      }
    } else {
      serial(&cx, op, n, scratch);
    }
  }
  return 0;
}

/* exported single kernels for the closed-form tests */
void kho_softmax_row(float *p, int n, const float *mask, int first, int il, int window, int qmask, int dense,
                     float scale) {
  softmax_row(p, n, mask, first, il, window, qmask, dense, scale);
}
float kho_vexp(float x) { return vexp1(x); }
float kho_vgelu(float x) { return vgelu1(x); }
float kho_gelu(float x) { return gelu_m(x); }
int kho_op_size(void) { return (int)sizeof(kho_op); }
