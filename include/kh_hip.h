/*
 * kh_hip.h — C ABI of libkh_hip.so, the MI355X (gfx950) executor of kleinhirn encoder plans.
 *
 * The library is the device side of a `Backend` / `PlanRunner` pair (src/backend.ts:14-46 of the
 * reference). A host (hip-backend.ts over Node-API, or Python over ctypes) hands it the weights
 * of a manifest, then plans as JSON, then per call the RunInput arrays. Plain pointers and sizes
 * only; every entry point returns KH_OK (0) or an error code, and kh_last_error() gives the
 * message of the calling thread's last failure.
 *
 * Execution model: a plan's rows are stored packed (the rows of each sequence up to its last
 * nonzero mask value, back to back, cu_seqlens), derived from the mask at the first run after an
 * upload. Only those rows are computed; per-row outputs (token heads) are scattered back to the
 * plan's b * L + i layout on read. A mask that is not a 0/1 prefix is executed as the reference's
 * executor does (keys and queries count above 0.5, the mean pool and MASKMUL weigh by the value).
 * One HIP stream per plan; a context is single-threaded by contract (one call in flight per plan,
 * as src/encoder.ts:5-8 and 265-269 guarantee on the reference side).
 */
#ifndef KH_HIP_H
#define KH_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct kh_ctx kh_ctx;
typedef struct kh_plan kh_plan;

/* status codes */
#define KH_OK 0
#define KH_EINVAL 1        /* bad argument, malformed plan JSON, size mismatch */
#define KH_EUNSUPPORTED 2  /* a plan op or layout this executor does not run */
#define KH_EHIP 3          /* a HIP runtime call failed (message names it) */
#define KH_ENOMEM 4        /* device or host allocation failed */
#define KH_ELOST 5         /* an earlier device failure latched the context; every call fails */

/* tensor dtypes */
#define KH_F32 0
#define KH_F16 1
#define KH_U32 2

#define KH_ABI_VERSION 1

/* Message of the calling thread's last failure ("" when none). Valid until the next call on the
 * same thread. */
const char *kh_last_error(void);
int kh_abi_version(void);

/* Context on HIP device `device`; owns the device copies of the weights.
 * Replaces the weight upload of loadGpu (src/webgpu-backend.ts:53-101) / the WASM host's
 * addWeight (src/plan/wasm.ts:231-255). */
int kh_ctx_create(int device, kh_ctx **out);
int kh_ctx_destroy(kh_ctx *ctx);

/* One manifest tensor (name, dtype, row-major shape, bytes): copied to device memory before the
 * call returns. A name loaded twice is an error (src/plan/wasm.ts:233). */
int kh_weight_add(kh_ctx *ctx, const char *name, int dtype, const int64_t *shape, int ndim,
                  const void *data, size_t bytes);

/* Bytes of the loaded weights in device memory (Backend.weightBytes, src/backend.ts:32-33). */
int kh_ctx_weight_bytes(const kh_ctx *ctx, uint64_t *out);

/* Optional device-resident word table [rows, width] in `dtype` (the step before the plan: the
 * reference gathers word rows on the host, src/encoder.ts:271-282); enables kh_upload_ids. */
int kh_words_set(kh_ctx *ctx, int dtype, int64_t rows, int64_t width, const void *data, size_t bytes);

/* ---- manifest directories (format kleinhirn-weights-2) ------------------------------------ */

#define KH_LOAD_NO_SHA256 1  /* skip the sha256 checks (files verified before) */
#define KH_LOAD_CHECK_ROWS 2 /* also check every words.bin row against its checksum */
#define KH_LOAD_NO_WORDS 4   /* leave the word table alone (no device word table) */

typedef struct {
  int32_t version;       /* manifest version: 3 with words.bin, 2 with keepOnCpu word parts */
  int32_t tensors;       /* device tensors (keepOnCpu parts excluded) */
  int32_t shards;
  int32_t words_dtype;   /* KH_F16 / KH_F32, -1 when no word table was read */
  int64_t words_rows;
  int64_t words_width;
  uint64_t tensor_bytes; /* bytes of the device tensors */
  uint64_t file_bytes;   /* bytes read: shards and words.bin */
  double read_ms;        /* manifest parse, file mapping and layout checks */
  double sha256_ms;      /* hashing, summed over files (they hash in parallel) */
  double rows_ms;        /* words.bin row checksums (KH_LOAD_CHECK_ROWS) */
  double upload_ms;      /* host to device copies (kh_load_manifest) */
} kh_manifest_info;

/* Reads `manifest_path` (manifest.json) and every file it names and applies the checks of the
 * reference's loader, without a device: shard sizes and sha256 (fetchShardBytes,
 * src/weights.ts:150-173), words.bin size, row layout and sha256 (fetchWords, src/words.ts:98-114),
 * or the legacy keepOnCpu word table (loadWords, src/weights.ts:67-90). Errors carry the
 * reference's messages ("sha256 mismatch on shard-0.bin", ...). */
int kh_manifest_check(const char *manifest_path, int flags, kh_manifest_info *out);

/* The same checks, then every tensor straight to device memory (as kh_weight_add; replaces
 * loadWeights' upload loop, src/webgpu-backend.ts:53-101) and the word table as the context's
 * device word table (as kh_words_set; the row checksums of words.bin stay on the host). Nothing is
 * uploaded unless every check passes. */
int kh_load_manifest(kh_ctx *ctx, const char *manifest_path, int flags, kh_manifest_info *out);

/* SHA-256 of `bytes` bytes (the shard digest of src/weights.ts:161-165). */
int kh_sha256(const void *data, size_t bytes, uint8_t out[32]);

/* Checksum of one words.bin row without its checksum word (rowChecksum, src/words-format.ts:18-32);
 * `bytes` must be a multiple of 4. */
int kh_row_checksum(const void *row, size_t bytes, uint32_t row_id, uint32_t salt, uint32_t *out);

/* ---- batch scheduling over packed plans ----------------------------------------------------- */

typedef struct kh_sched kh_sched;

typedef struct {
  int32_t chunks;     /* plan runs */
  int32_t sequences;
  int64_t tokens;     /* valid rows computed */
  double wall_ms;     /* kh_sched_run from entry to return */
  double gpu_ms;      /* summed kh_last_run_ms of the runs */
  double host_ms;     /* packing, uploads and submits (overlapping the device) */
} kh_sched_stats;

/* A scheduler over `n` created plans of one context (their init tables set; the context's device
 * word table set), all pooled heads with the same output columns. The plans stay the caller's and
 * must outlive the scheduler. Replaces the chunking of runIdsBatch (src/encoder.ts:380-436: chunks
 * of at most 16 rows on plans of 1/4/8/16 sequences, src/cache.ts:9-18) for packed plans. */
int kh_sched_create(kh_plan *const *plans, int32_t n, kh_sched **out);

/* Runs `nseq` token id sequences (sequence i is ids[offsets[i] .. offsets[i + 1])) and writes one
 * output row per sequence, in input order. Sequences go in length order (sortByKey,
 * src/cache.ts:92-108) into chunks of at most B sequences of the plan with the smallest length
 * holding them, and at most `token_budget` tokens when it is positive; plans of one shape run in
 * turn, so the next chunk is packed while the previous one computes. `type_words` (nullable) holds
 * the u32 type word per token in the layout of `ids` (type in the low 16 bits, the position row of
 * POSIDS plans in the high 16, as kh_upload). */
int kh_sched_run(kh_sched *s, const int32_t *ids, const int64_t *offsets, int64_t nseq, const uint32_t *type_words,
                 int64_t token_budget, float *out, size_t out_count, kh_sched_stats *stats);

int kh_sched_destroy(kh_sched *s);

/* ---- scores from the outputs (the step after the plan) ------------------------------------ */

#define KH_SCORES_SOFTMAX 0 /* single-label classification: softmax per row, label = its argmax */
#define KH_SCORES_SIGMOID 1 /* multi-label: 1 / (1 + e^-logit), label = argmax of the logits */
#define KH_SCORES_RAW 2     /* regression: the logits, label = their argmax */
#define KH_SCORES_L2 3      /* embeddings: rows divided by max(|row|, 1e-12) */
#define KH_SCORES_OPTIONS 4 /* Julia's option probabilities: softmax with the exponentials summed and divided
                             * in double, one rounding per value (softmaxPrefix, src/julia.ts:57-65); pass the
                             * first min(markers, options) logits of a row as its columns; label = argmax */

/* Scores of a row-major [rows, cols] f32 array in the reference's arithmetic (f32 values,
 * double operations, one rounding to f32; softmax, l2normalize, argmaxRows with ties to the
 * lower index, src/tasks.ts:22-42, 72-84; the per-problem choice of classify,
 * src/encoder.ts:498-513). `index` (one per row) may be null. A non-finite input fails with
 * "output: k of n values are not finite" (assertFinite, src/tasks.ts:5-9). */
int kh_scores(const float *logits, int64_t rows, int32_t cols, int kind, float *scores, int32_t *index);

/* kh_read_output followed by kh_scores on the plan's output (pooled heads: one row per
 * sequence). */
int kh_read_scores(kh_plan *plan, int kind, float *scores, size_t count, int32_t *index, size_t index_count);

/* Indices of `n` scores by score, highest first, equal scores in index order (rerank,
 * src/encoder.ts:533-544). */
int kh_rank(const float *scores, int64_t n, int32_t *order);

/* Backend.check (src/backend.ts:34-35): KH_OK when the plan (JSON of the reference's Plan, typed
 * `init` tables left out) can run here, else an error naming every op that cannot. With a null
 * context only the plan's structure is checked (no weights, no device needed). */
int kh_plan_check(kh_ctx *ctx, const char *plan_json, size_t len);

/* Backend.runner (src/backend.ts:36, src/plan/executor.ts:85-99): builds every buffer and the
 * launch list up front. */
int kh_plan_create(kh_ctx *ctx, const char *plan_json, size_t len, kh_plan **out);

/* BufferDecl.init of buffer `id` (relidx, cossin, first, zero; src/plan/executor.ts:118-124). */
int kh_plan_init_buffer(kh_plan *plan, const char *id, const void *data, size_t bytes);

typedef struct {
  int32_t length;       /* PlanRunner.length */
  int32_t batch;        /* PlanRunner.batch */
  int32_t markers;      /* PlanRunner.markers */
  int32_t f16;          /* storage dtype of the plan */
  uint64_t bytes;       /* PlanRunner.bytes: device bytes held for this plan */
  int32_t out_rows;     /* Plan.output.rows */
  int32_t out_cols;     /* Plan.output.cols */
  int32_t launches;     /* kernel launches of one run (of one half when split) */
  int32_t streams;      /* 2 when the last run split the batch over two streams, else 1 */
} kh_plan_info;

int kh_plan_info_get(const kh_plan *plan, kh_plan_info *out);

/* PlanRunner.upload (src/plan/executor.ts:365-393): word rows [L * B, E] in the plan's storage
 * dtype, the f32 mask [L * B] and, for plans with a typeIds input, u32 type ids [L * B] (position
 * row in the high 16 bits for POSIDS). Copied before return. Any mask values: rows up to a
 * sequence's last nonzero value are computed (src/wasm/plan.ts:556-582, 474-495). */
int kh_upload(kh_plan *plan, const void *emb, size_t emb_bytes, const float *mask, size_t mask_count,
              const uint32_t *type_ids, size_t type_count);

/* Variant of kh_upload with token ids [L * B] instead of word rows: the rows are gathered from
 * the context's word table (kh_words_set) on the device. */
int kh_upload_ids(kh_plan *plan, const int32_t *ids, size_t id_count, const float *mask,
                  size_t mask_count, const uint32_t *type_ids, size_t type_count);

/* The packedMarkers part of PlanRunner.upload (RunInput.packedMarkers, src/plan/executor.ts:28,
 * 385-388) for plans with a markers input (GLiNER2 span heads): per sequence 3 * markers u32, the
 * marker row indices, the marker mask as f32 bits and the group ids; count up to
 * 3 * markers * batch (a shorter payload replaces only the first count values, as the reference's
 * upload does). Every row index must be below the plan length (KH_EINVAL at kh_run). Kept until
 * replaced; before the first call every slot is masked. A marker whose row lies past its
 * sequence's valid rows gathers a zero state (the reference reads the padding row's state). */
int kh_upload_markers(kh_plan *plan, const uint32_t *packed, size_t count);

/* The qtype part of PlanRunner.upload (RunInput.qtype, src/plan/executor.ts:30-31) for plans with
 * a rowSelect (the Julia head): type row qtype[b] of the rowSelect table is copied to row b of
 * its destination before the forward (src/plan/executor.ts:236-246, src/plan/wasm.ts:429-439);
 * count <= batch, sequences without an entry take row 0; a qtype past the table is KH_EINVAL at
 * kh_run. */
int kh_upload_qtypes(kh_plan *plan, const uint32_t *qtype, size_t count);

/* PlanRunner.run (src/plan/executor.ts:295-297): one forward over `rows` rows (the real rows of
 * a B = 1 call, L * B for a batch plan), enqueued on the plan's stream; returns without waiting.
 * A batch call with fewer than KH_SPLIT_T (environment, default 400000) valid rows runs as two
 * halves of about equal rows on two streams (KH_NO_SPLIT=1: one stream); outputs are the same. */
int kh_run(kh_plan *plan, int32_t rows);

/* PlanRunner.readOutput (src/plan/executor.ts:398-408): waits, then writes rows * cols f32
 * values (f16 storage converted; f32 output buffers, as a GLiNER2 plan's logits, as they are) in
 * the plan's output layout. */
int kh_read_output(kh_plan *plan, float *out, size_t count);

/* Waits for the plan's stream. */
int kh_sync(kh_plan *plan);

/* GPU milliseconds of the last kh_run (hipEvents on the plan's stream around its launches). */
int kh_last_run_ms(kh_plan *plan, float *ms);

/* Per-launch profile: runs one forward with an event pair around every launch and fills up to
 * `cap` records (name of the op, kernel, GPU ms, algorithmic FLOPs and bytes of that launch).
 * Returns the number of launches in *count. */
typedef struct {
  char name[48];
  char kernel[24];
  float ms;
  float reserved;
  double flops;
  double bytes;
} kh_launch_stat;

int kh_profile(kh_plan *plan, int32_t rows, kh_launch_stat *out, int32_t cap, int32_t *count);

/* Live per-launch timing: with tracing on, every kh_run records a HIP event pair around each of
 * its launches on the stream that launch runs on (both halves of a split batch); kh_trace_read
 * waits and returns the launches recorded since the last read (or kh_trace call) in launch order,
 * in the records of kh_profile, and clears them (a null `out` only sets *count). kh_trace(plan, 0)
 * stops recording. */
int kh_trace(kh_plan *plan, int32_t on);
int kh_trace_read(kh_plan *plan, kh_launch_stat *out, int32_t cap, int32_t *count);

/* Packed rows (sum of valid sequence lengths) of the last run. */
int kh_packed_rows(const kh_plan *plan, int64_t *out);

/* Raw bytes of a plan buffer as the last run left them (storage dtype, packed rows first): waits
 * for the plan's stream, copies min(bytes, buffer size) bytes. `half` 1 reads the buffer of the
 * second half of a split batch (the twin plan). Replaces the buffer reads of the reference's
 * capture tool (PlanRunner.readCapture, src/plan/executor.ts:177-195), for the layer-by-layer
 * comparisons of a debugging session; KH_EINVAL for a buffer without device memory. */
int kh_plan_read_buffer(kh_plan *plan, const char *id, int32_t half, void *out, size_t bytes);

int kh_plan_destroy(kh_plan *plan);

#ifdef __cplusplus
}
#endif

#endif /* KH_HIP_H */
