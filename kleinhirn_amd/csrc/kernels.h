// Launch interface of the gfx950 kernels. Every launch is asynchronous on the given stream;
// operand shapes are checked by the caller (runner.hip) before a launch.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <cstdint>
#include <utility>

namespace kh {

// Events the next kernel launch of this thread records around itself (the per-launch profile sets
// them for one step at a time; null otherwise). hipExtLaunchKernelGGL timestamps the dispatch
// itself, so the measured time is the kernel's, without the gaps of separate event packets.
struct LaunchEvents {
  hipEvent_t start = nullptr, stop = nullptr;
};
extern thread_local LaunchEvents g_launch_events;

template <typename... KArgs, typename... Args>
inline void launch(void (*kernel)(KArgs...), dim3 grid, dim3 block, unsigned smem, hipStream_t s, Args &&...args) {
  if (g_launch_events.start)
    hipExtLaunchKernelGGL(kernel, grid, block, smem, s, g_launch_events.start, g_launch_events.stop, 0,
                          std::forward<Args>(args)...);
  else
    hipLaunchKernelGGL(kernel, grid, block, smem, s, std::forward<Args>(args)...);
}

// Activation codes of the plan's matmul ACT constant (src/plan/build.ts:91).
enum Act : int { ACT_NONE = 0, ACT_RELU = 1, ACT_GELU = 2, ACT_TANH = 3, ACT_SILU = 4 };

// C[M, N] = act(A[M, K] W[N, K]^T + bias[N]); row strides lda, ldw, ldc in elements.
struct GemmArgs {
  const void *a = nullptr;
  int64_t lda = 0;
  const void *w = nullptr;
  int64_t ldw = 0;
  const void *bias = nullptr;  // may be null
  void *c = nullptr;
  int64_t ldc = 0;
  int M = 0, N = 0, K = 0;
  int act = 0;
  // batched over z: pointer offsets (elements) per z index
  int batch = 1;
  int64_t a_bs = 0, w_bs = 0, c_bs = 0;
  bool c_f32 = false;  // write f32 output whatever the storage type (relative-position scores)
  // force the wavefront-per-output kernel (tests)
  bool rowdot = false;
  // fused step after the product (f16 lean kernel only; gemm_epi_ok tells when it runs):
  //  EPI_GEGLU: W holds [a | b] halves of N = 2 I rows; C [M, I] = gelu(a) * b
  //  EPI_ROPE: rotate-half RoPE on the first rope_cols columns (q and k), head dim rope_d, table
  //            [L][cos D | sin D] at the row's position row_pos[m]
  //  EPI_RESADD: C += product (C is the residual stream, updated in place)
  //  EPI_LN: C = LayerNorm(ln_res + product) over whole rows (gamma ln_g, beta ln_b, may be null;
  //          eps ln_eps), the MODE 2 LayerNorm of the separate step with its lanes and sums
  // each applied to the product rounded to the storage type, as the separate ops read it
  int epi = 0;
  const float *rope_table = nullptr;
  const int32_t *row_pos = nullptr;
  int rope_cols = 0, rope_d = 0;
  const void *ln_res = nullptr, *ln_g = nullptr, *ln_b = nullptr;
  float ln_eps = 0.f;
};
enum { EPI_NONE = 0, EPI_GEGLU = 1, EPI_ROPE = 2, EPI_RESADD = 3, EPI_LN = 4 };
void gemm(bool f16, const GemmArgs &g, hipStream_t s);
// true when the MFMA tile kernel runs this shape (else the wave-per-output kernel)
bool gemm_uses_mfma(bool f16, const GemmArgs &g);
// the product runs on MFMA (the tiled kernels, or for a few hundred f32 rows the 32 x 32 one)
bool gemm_on_mfma(bool f16, const GemmArgs &g);
// true when g's fused step (g.epi) can run inside the product for this shape and storage type
bool gemm_epi_ok(bool f16, const GemmArgs &g);

// Packed-row description of one run: cu[b] .. cu[b+1] are the rows of sequence b.
// With masks that are not 0/1 prefixes, a sequence's packed rows run to its last nonzero mask
// value and row_w [T] holds each row's mask value: keys and queries count where it exceeds 0.5,
// pooling and the mask-multiplied embeddings weigh by it. row_w is null for 0/1 prefix masks.
struct Packing {
  const int32_t *cu;       // [B + 1]
  const int32_t *row_pos;  // [T] position of the row inside its sequence
  const int32_t *row_seq;  // [T] sequence of the row
  int32_t B;
  int64_t T;
  const float *row_w = nullptr;  // [T] mask values, or null (every packed row 1)
};


// Ranges (16-byte pieces) a LayerNorm launch reads and discards after its rows: the weights of the
// products that follow it, brought into the memory-side cache just before they run. total is the
// sum of n16; nothing is written.
constexpr int PREFETCH_RANGES = 4;
struct PrefetchArgs {
  const void *p[PREFETCH_RANGES] = {};
  int64_t n16[PREFETCH_RANGES] = {};
  int64_t total = 0;
};

struct EmbLnArgs {
  const void *word = nullptr;    // packed word rows [T, N], or null with table + ids
  const void *table = nullptr;   // device word table [rows, N]
  const int32_t *ids = nullptr;  // packed ids [T]
  const void *pos = nullptr;     // [maxpos, N] or null (zero table)
  const void *typ = nullptr;     // [types, N] or null (zero table)
  const uint32_t *tt = nullptr;  // packed type ids [T] or null
  const void *gamma = nullptr, *beta = nullptr;
  void *out = nullptr;
  int N = 0, offset = 0, maxpos = 1, posids = 0;
  float eps = 0.f;
  const float *row_scale = nullptr;  // [T] multiplies each output row (MASKMUL), or null
};
void embln(bool f16, const EmbLnArgs &a, const Packing &p, hipStream_t s, const PrefetchArgs &pf = PrefetchArgs());

// GLiNER2 logits: logits[k] = raw[k] / temp where marker k's mask word (f32 bits at
// b * 3K + K + k mod K of the packed payloads, b = k / K) exceeds 0.5, else -1e4; total = B * K.
void mask_logits(bool f16, const void *raw, const uint32_t *packed, float *logits, int K, float temp, int64_t total,
                 hipStream_t s);

// LN over rows: MODE 2 adds b first. rows = T (packed) or B (sequence rows). With ids, row r is
// row ids[r] of a (the device word table), with the arithmetic of the same LN over gathered rows.
// row_scale [rows], when given, multiplies each output row (MODE 1, the mask-multiplied embedding).
void layernorm(bool f16, const void *a, const void *b, const void *gamma, const void *beta, void *out,
               int64_t rows, int N, float eps, hipStream_t s, const int32_t *ids = nullptr,
               const PrefetchArgs &pf = PrefetchArgs(), const float *row_scale = nullptr);

// dst += src (MODE 0) or dst[r] += src[seq(r)] (MODE 1), rounded to storage.
void add(bool f16, void *dst, const void *src, int64_t rows, int N, int mode, const Packing &p,
         hipStream_t s);

void geglu(bool f16, const void *mid, void *gate, int64_t rows, int I, hipStream_t s);

void rope(bool f16, void *qkv, const float *cossin, int64_t rows, int H, int D, int L,
          const Packing &p, hipStream_t s);

// mode 0 mean, 1 max over the packed rows of each sequence -> [B, N]
void pool(bool f16, const void *x, void *out, int N, int mode, const Packing &p, hipStream_t s);

// states[b K + k] = x[cu[b] + marker[b 3 K + k]] (zero row when the marker is past the sequence)
void gather_rows(bool f16, const void *x, const uint32_t *markers, void *states, int K, int D,
                 const Packing &p, hipStream_t s);

// Standard attention over packed rows: ctx = softmax(scale q k^T, window) v per (sequence, head).
// tiles: [ntiles] 64-query tiles as (sequence, first query, first packed row of the sequence,
// sequence length), so a block needs no second lookup of cu_seqlens.
struct AttnArgs {
  const void *qkv = nullptr;  // [T, 3 H D]
  void *ctx = nullptr;        // [T, H D]
  int H = 0, D = 0;
  float scale = 1.f;          // multiplies the score
  int window = 0;             // 0: global, else |i - j| <= window
  // DeBERTa relative terms: score = (q_i.k_j + q_i.pos_key[m] + k_j.pos_query[m]) * scale with
  // m = bucket[i - j + lmax - 1]; the position tables are [nb, H D] in the storage type
  const void *pos_key = nullptr;
  const void *pos_query = nullptr;
  const int32_t *bucket = nullptr;  // [2 lmax - 1]
  int nb = 0;
  int lmax = 0;
  const int4 *tiles;
  int ntiles;
  // the grid's blocks in dispatch order (null: item = xcd_tile(block)): block b runs work[b] =
  // {head, first query, first packed row, length} of its query tile ({-1, 0, 0, 0} for none), its
  // blocks' XCD b % 8 (see the runner's attention order); the tile itself is in the entry, so a
  // block reads one entry before its rows
  const int4 *work = nullptr;
  int nwork = 0;
};
void attention(bool f16, const AttnArgs &a, const Packing &p, hipStream_t s);
constexpr int ATTN_QTILE = 64;
constexpr int ATTN_DMAX = 64;  // largest head dimension (32 and 64 run as they are, others padded)
constexpr int ATTN_REL_LMAX = 2048;  // longest plan the relative attention kernel takes (its LDS bucket table)

// Row 0 of each sequence into one row per sequence (from_packed), or one row per sequence copied
// with empty sequences zeroed; rows of width D.
void first_rows(bool f16, const void *src, void *dst, int D, bool from_packed, const Packing &p, hipStream_t s);

// Convert storage rows to f32 (readback of f16 outputs).
void to_f32(bool f16, const void *src, float *dst, int64_t n, hipStream_t s);

}  // namespace kh
