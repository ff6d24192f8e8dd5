// libkh_hip.so: the C ABI of include/kh_hip.h.
//
// A plan (the reference's Plan IR as JSON, src/plan/ir.ts:41-60) is lowered once at creation into
// a list of launch steps over packed rows: the attention op sequences of the reference's split
// kernels fuse into one flash-attention step (the same grouping the reference's WASM host makes,
// src/plan/wasm.ts:53-82), the per-op row dispatch of the reference ('rows', 'rows16', ...) becomes
// "all packed rows", and a fixed dispatch (pooled heads) becomes "one row per sequence". Buffers
// no step reads after the fusion (scores, c2p, p2c, kinfo, mask) get no device memory.
//
// Per call the host hands padded RunInput arrays (src/plan/executor.ts:25-32); the first run after
// an upload derives cu_seqlens from the mask, packs the valid rows into pinned memory and
// copies only those to the device.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <map>
#include <memory>
#include <set>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "../../include/kh_hip.h"
#include "json.h"
#include "kernels.h"
#include "manifest.h"
#include "postprocess.h"

namespace kh {

struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string &m) : std::runtime_error(m), code(c) {}
};

static thread_local std::string g_last_error;

thread_local LaunchEvents g_launch_events;

#define KH_CHECK(call)                                                                            \
  do {                                                                                            \
    hipError_t e_ = (call);                                                                       \
    if (e_ != hipSuccess)                                                                         \
      throw Error(KH_EHIP, std::string(#call) + ": " + hipGetErrorString(e_));                    \
  } while (0)

static void fail(int code, const std::string &m) { throw Error(code, m); }

static size_t elem_size(int dtype) { return dtype == KH_F16 ? 2 : 4; }

struct DevMem {
  void *p = nullptr;
  size_t bytes = 0;
  DevMem() = default;
  DevMem(const DevMem &) = delete;
  DevMem &operator=(const DevMem &) = delete;
  ~DevMem() { reset(); }
  void alloc(size_t n) {
    reset();
    if (n == 0) n = 16;
    hipError_t e = hipMalloc(&p, n);
    if (e != hipSuccess) {
      p = nullptr;
      fail(KH_ENOMEM, "hipMalloc of " + std::to_string(n) + " bytes: " + hipGetErrorString(e));
    }
    bytes = n;
  }
  void reset() {
    if (p) (void)hipFree(p);
    p = nullptr;
    bytes = 0;
  }
};

struct HostPinned {
  void *p = nullptr;
  size_t bytes = 0;
  ~HostPinned() { reset(); }
  void ensure(size_t n) {
    if (n <= bytes) return;
    reset();
    hipError_t e = hipHostMalloc(&p, n, hipHostMallocDefault);
    if (e != hipSuccess) {
      p = nullptr;
      fail(KH_ENOMEM, "hipHostMalloc of " + std::to_string(n) + " bytes: " + hipGetErrorString(e));
    }
    bytes = n;
  }
  void reset() {
    if (p) (void)hipHostFree(p);
    p = nullptr;
    bytes = 0;
  }
};

struct Weight {
  int dtype = KH_F32;
  std::vector<int64_t> shape;
  int64_t count = 0;
  std::unique_ptr<DevMem> mem;
};

}  // namespace kh

using namespace kh;

struct kh_ctx {
  int device = 0;
  std::map<std::string, Weight> weights;
  uint64_t weight_bytes = 0;
  bool lost = false;
  std::string lost_msg;
  // device word table
  int words_dtype = -1;
  int64_t words_rows = 0, words_width = 0;
  std::unique_ptr<DevMem> words;
};

namespace kh {

enum StepKind { S_EMBLN, S_LN, S_GEMM, S_ADD, S_GEGLU, S_ROPE, S_ATTN, S_POOL, S_GATHER, S_COMPACT, S_MASKL };

// A buffer reference of a step: device pointer resolved at plan creation.
struct Ref {
  std::string id;
  void *p = nullptr;
};

struct Step {
  StepKind kind;
  std::string name, kernel;
  bool seq_rows = false;  // fixed dispatch: one row per sequence (or rows_fixed rows)
  int64_t rows_fixed = 0;
  Ref in[7];
  int N = 0, K = 0, act = 0, mode = 0, I = 0, H = 0, D = 0, window = 0, offset = 0, maxpos = 1, posids = 0;
  int Kmk = 1;  // gather markers per sequence
  float eps = 0.f, scale = 1.f;
  bool rel = false;
  std::string markers_id;  // gather: the init buffer holding the markers
  int epi = 0;             // S_GEMM: fused step (EPI_*); in[4] holds a RoPE table, or with EPI_LN the
                           // residual (in[5], in[6]: the norm's gamma and beta; eps)
  int maskmul = 0;         // S_EMBLN: the output rows times the mask (MASKMUL)
  bool first_tiles = false;  // S_ATTN: only the first query tile of each sequence
};

// one traced launch: an event pair recorded around its dispatch on the stream it ran on
struct TraceRec {
  std::string name, kernel;
  double flops = 0, bytes = 0;
  hipEvent_t a = nullptr, b = nullptr;
};

struct Buffer {
  int64_t bytes = 0;
  std::string usage;
  bool used = false;
  bool seq_space = false;  // written by a fixed-dispatch op: rows are sequences
  bool packed_space = false;
  std::unique_ptr<DevMem> mem;
  std::vector<uint8_t> init;
  bool init_done = false;  // init holds what the device buffer (or the relidx bucket table) holds
};

static const std::set<std::string> kMatmul = {"matmul", "mmtile", "mmtile8", "mmtile16"};

static bool is_rows_dim(const Json &d) { return d.kind == Json::Str; }

}  // namespace kh

struct kh_plan {
  kh_ctx *ctx = nullptr;
  bool f16 = false;
  int L = 0, B = 0, markers = 0, E = 0;
  std::map<std::string, Buffer> bufs;
  std::vector<Step> steps;
  // the same forward with the tail after the last attention on one row per sequence (empty when the
  // plan has no such tail); it runs while every marker of the head's row gather is 0
  std::vector<Step> steps_pruned;
  std::string prune_markers;
  std::vector<uint8_t> markers_shadow;  // host copy of that markers buffer
  bool markers_first = true;
  std::string in_emb, in_mask, in_tt;
  std::string in_markers;             // packed marker payloads (GLiNER2 span heads), or empty
  std::vector<uint32_t> markers_host;  // the last kh_upload_markers payload
  bool markers_dirty = false;
  bool out_f32 = false;                // output buffer holds f32 whatever the storage dtype
  // rowSelect (Julia): row qtype[b] of the table weight copied to row b of dst before each run
  std::string rs_table, rs_dst;
  int64_t rs_row_bytes = 0;
  std::vector<uint32_t> qtype_host;
  std::string out_buf;
  int out_rows = 0, out_cols = 0;
  bool out_packed = false;
  hipStream_t stream = nullptr;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  bool ran = false;

  // A small batch runs as two halves on two streams: sequences [0, split) here, [split, B) on the
  // twin (the same plan, its own buffers and stream), so the kernels of one half fill the CUs the
  // other half's grids leave idle. split = 0: the whole batch here.
  std::string json;                                                    // the plan document
  std::vector<std::pair<std::string, std::vector<uint8_t>>> init_log;  // kh_plan_init_buffer calls
  kh_plan *twin = nullptr;
  bool is_twin = false;
  bool twin_failed = false;  // the twin could not be allocated: every batch runs whole
  int split = 0;
  hipEvent_t ev_twin = nullptr;
  // choose_split's answer for the current upload, row count and switches (-1: not computed)
  int split_memo = -1, split_memo_rows = -1;
  int64_t split_memo_env = -1;

  // live per-launch timing of kh_run (kh_trace / kh_trace_read)
  bool tracing = false;
  std::vector<TraceRec> trace;
  std::vector<hipEvent_t> ev_pool;

  // upload staging (host, padded layout as the caller gave it)
  // The uploaded word rows, packed once at upload into pinned memory: sequence b's first avail[b]
  // rows (up to its mask extent, and what the caller's array held) at row up_cu[b] of up_rows.
  // up_rows is this plan's pin_up, or for a twin the primary plan's, at its first moved sequence.
  HostPinned pin_up, pin_pack;
  const uint8_t *up_rows = nullptr;
  std::vector<int64_t> up_cu;
  std::vector<int32_t> avail;
  std::vector<float> mask_host;
  std::vector<uint32_t> tt_host;
  std::vector<int32_t> ids_host;
  bool by_ids = false;
  bool uploaded = false, dirty = true;
  int last_rows = -1;

  // packing of the current upload
  std::vector<int32_t> cu;
  int64_t T = 0;
  int ntiles = 0, ntiles_first = 0;
  int nwork = 0, nwork_first = 0;  // attention work lists (attn_order), 0: none
  int work_h = 0;                   // the head count they were built for
  double attn_pairs_global = 0;  // sum over sequences of n^2
  std::map<int, double> attn_pairs_window;  // window -> sum of visited (i, j) pairs
  double attn_pairs_first = 0;  // the same for the first query tile of each sequence
  std::map<int, double> attn_pairs_first_window;
  int64_t rows_first = 0;  // query rows of the first tiles
  HostPinned pin_meta;
  DevMem d_cu, d_row_pos, d_row_seq, d_tiles, d_tiles_first, d_tt, d_ids, d_work, d_work_first;
  // masks other than 0/1 prefixes: each packed row's mask value (Packing::row_w)
  bool masked = false;
  DevMem d_row_w;

  // relative attention
  std::vector<int32_t> bucket_host;
  DevMem d_bucket;
  int rel_nb = 0;
  double rel_rows_buckets = 0;  // sum over sequences of rows x buckets reached (c2p + p2c work)
  double rel_rows_buckets_first = 0;

  // cos/sin tables (f32)
  std::map<std::string, std::unique_ptr<DevMem>> tables;
};

namespace kh {

static Packing packing_of(kh_plan *pl) {
  Packing p;
  p.cu = (const int32_t *)pl->d_cu.p;
  p.row_pos = (const int32_t *)pl->d_row_pos.p;
  p.row_seq = (const int32_t *)pl->d_row_seq.p;
  p.B = pl->B;
  p.T = pl->T;
  p.row_w = pl->masked ? (const float *)pl->d_row_w.p : nullptr;
  return p;
}

// The rows of a sequence the forward computes: up to its last nonzero mask value. For a 0/1
// prefix mask these are its valid rows; any other mask keeps its holes and fractional values as
// rows whose mask value the kernels read (Packing::row_w), as the reference's executor does.
static int seq_extent(const float *m, int L) {
  int e = L;
  while (e > 0 && m[e - 1] == 0.f) e--;
  return e;
}

// ---- plan parsing and lowering -------------------------------------------------------------

struct Parsed {
  Json root;
  std::vector<Json> ops;  // flattened op list
};

static Parsed parse_plan(const char *json, size_t len) {
  Parsed p;
  if (!json || len == 0) fail(KH_EINVAL, "empty plan JSON");
  try {
    p.root = JsonReader(json, len).parse();
  } catch (const std::runtime_error &e) {
    fail(KH_EINVAL, e.what());
  }
  for (const Json &seg : p.root.at("segments").arr())
    for (const Json &op : seg.at("ops").arr()) p.ops.push_back(op);
  return p;
}

static int cint(const Json &op, const char *k) {
  const Json &c = op.at("constants");
  if (!c.has(k)) fail(KH_EINVAL, "op " + op.at("name").str() + ": constant " + k + " missing");
  return (int)c.at(k).integer();
}
static double cnum(const Json &op, const char *k) {
  const Json &c = op.at("constants");
  if (!c.has(k)) fail(KH_EINVAL, "op " + op.at("name").str() + ": constant " + k + " missing");
  return c.at(k).num();
}
static const std::string &bind(const Json &op, size_t i) {
  const auto &b = op.at("bind").arr();
  if (i >= b.size()) fail(KH_EINVAL, "op " + op.at("name").str() + ": binding " + std::to_string(i) + " missing");
  return b[i].str();
}
static const std::string &kern(const Json &op) { return op.at("kernel").str(); }

// Lowering: returns the steps; collects every unsupported op into `errors`.
static std::vector<Step> lower(const Parsed &pp, bool f16, int L, std::vector<std::string> &errors) {
  (void)f16;
  std::vector<Step> steps;
  const auto &ops = pp.ops;
  auto k = [&](size_t i) -> std::string { return i < ops.size() ? kern(ops[i]) : std::string(); };
  for (size_t i = 0; i < ops.size(); i++) {
    const Json &op = ops[i];
    const std::string &kn = kern(op);
    const std::string name = op.at("name").str();
    const auto &disp = op.at("dispatch").arr();
    try {
      Step s;
      s.name = name;
      s.kernel = kn;
      if (kn == "attscore" && k(i + 1) == "attsoftmax" && k(i + 2) == "attpv" &&
          bind(ops[i + 1], 1) == bind(op, 2) && bind(ops[i + 2], 0) == bind(op, 2)) {
        // standard attention, split form (src/plan/layers.ts:84-93)
        s.kind = S_ATTN;
        s.kernel = "attention";
        s.in[0].id = bind(op, 0);          // qkv
        s.in[1].id = bind(ops[i + 2], 4);  // ctx
        s.H = cint(op, "H");
        s.D = cint(op, "D");
        s.scale = (float)cnum(op, "SCALE");
        s.window = cint(ops[i + 1], "WINDOW");
        i += 2;
      } else if (kn == "mbflash" || kn == "mbattention") {
        s.kind = S_ATTN;
        s.kernel = "attention";
        s.in[0].id = bind(op, 0);
        s.in[1].id = bind(op, 2);
        s.H = cint(op, "H");
        s.D = cint(op, "D");
        s.scale = (float)cnum(op, "SCALE");
        s.window = cint(op, "WINDOW");
      } else if (kn == "attrel" && cint(op, "PART") == 0 && k(i + 1) == "attrel" && cint(ops[i + 1], "PART") == 1 &&
                 k(i + 2) == "attscore" && k(i + 3) == "attsoftrel" && k(i + 4) == "attpv") {
        // DeBERTa relative attention, split form (src/plan/layers.ts:61-80):
        // score = (q.k) SCALE + (c2p + p2c) INVSCALE with SCALE = INVSCALE = 1 / sqrt(3 D)
        s.kind = S_ATTN;
        s.kernel = "attention-rel";
        s.rel = true;
        s.in[0].id = bind(op, 0);           // qkv
        s.in[1].id = bind(ops[i + 4], 4);   // ctx
        s.in[2].id = bind(op, 1);           // posKey
        s.in[3].id = bind(ops[i + 1], 1);   // posQuery
        s.in[4].id = bind(op, 3);           // relidx
        s.H = cint(op, "H");
        s.D = cint(op, "D");
        s.scale = (float)cnum(ops[i + 3], "INVSCALE");
        i += 4;
      } else if (kn == "attention") {
        // fused DeBERTa attention: score = (q.k + c2p + p2c) / SCALE (src/kernels/attention.wgsl)
        s.kind = S_ATTN;
        s.rel = true;
        s.kernel = "attention-rel";
        s.in[0].id = bind(op, 0);
        s.in[1].id = bind(op, 5);
        s.in[2].id = bind(op, 1);
        s.in[3].id = bind(op, 2);
        s.in[4].id = bind(op, 3);
        s.H = cint(op, "H");
        s.D = cint(op, "D");
        s.scale = (float)(1.0 / cnum(op, "SCALE"));
      } else if (kMatmul.count(kn)) {
        s.kind = S_GEMM;
        for (int b = 0; b < 4; b++) s.in[b].id = bind(op, b);
        s.N = cint(op, "N");
        s.K = cint(op, "K");
        s.act = cint(op, "ACT");
        if (!is_rows_dim(disp.at(1))) {
          s.seq_rows = true;
          s.rows_fixed = cint(op, "M");
        }
        if (s.act < 0 || s.act > 4) fail(KH_EUNSUPPORTED, "activation " + std::to_string(s.act));
      } else if (kn == "layernorm") {
        s.kind = S_LN;
        for (int b = 0; b < 6; b++) s.in[b].id = bind(op, b);
        s.N = cint(op, "N");
        s.mode = cint(op, "MODE");
        s.eps = (float)cnum(op, "EPS");
        if (!is_rows_dim(disp.at(0))) {
          s.seq_rows = true;
          s.rows_fixed = disp.at(0).integer();
        }
        if (s.mode < 0 || s.mode > 2) fail(KH_EUNSUPPORTED, "layernorm MODE " + std::to_string(s.mode));
      } else if (kn == "embln") {
        s.kind = S_EMBLN;
        // word, pos, typ, typeIds, w, bias, mask, out
        static const int map[6] = {0, 1, 2, 4, 5, 7};
        for (int b = 0; b < 6; b++) s.in[b].id = bind(op, map[b]);
        s.markers_id = bind(op, 3);
        s.N = cint(op, "N");
        s.offset = cint(op, "OFFSET");
        s.maxpos = cint(op, "MAXPOS");
        s.posids = cint(op, "POSIDS");
        s.eps = (float)cnum(op, "EPS");
        s.maskmul = op.at("constants").has("MASKMUL") ? cint(op, "MASKMUL") : 0;
        if (cint(op, "L") != L) fail(KH_EINVAL, "embln L differs from the plan length");
      } else if (kn == "add") {
        s.kind = S_ADD;
        s.in[0].id = bind(op, 0);
        s.in[1].id = bind(op, 1);
        s.N = cint(op, "N");
        s.mode = cint(op, "MODE");
        if (s.mode != 0 && s.mode != 1) fail(KH_EUNSUPPORTED, "add MODE " + std::to_string(s.mode));
      } else if (kn == "geglu") {
        s.kind = S_GEGLU;
        s.in[0].id = bind(op, 0);
        s.in[1].id = bind(op, 1);
        s.I = cint(op, "I");
      } else if (kn == "rope") {
        s.kind = S_ROPE;
        s.in[0].id = bind(op, 0);
        s.in[1].id = bind(op, 1);
        s.H = cint(op, "H");
        s.D = cint(op, "D");
        if (s.D % 2) fail(KH_EUNSUPPORTED, "rope with odd head dimension");
      } else if (kn == "pool") {
        s.kind = S_POOL;
        s.in[0].id = bind(op, 0);
        s.in[1].id = bind(op, 2);
        s.N = cint(op, "N");
        s.mode = cint(op, "MODE");
        s.seq_rows = true;
      } else if (kn == "masklogits") {
        // raw, packed markers, f32 logits (src/plan/build.ts:371-375)
        s.kind = S_MASKL;
        for (int b = 0; b < 3; b++) s.in[b].id = bind(op, b);
        s.Kmk = cint(op, "K");
        s.scale = (float)cnum(op, "TEMP");
        s.seq_rows = true;
        if (s.Kmk < 1) fail(KH_EINVAL, "masklogits K must be positive");
      } else if (kn == "gather") {
        s.kind = S_GATHER;
        s.markers_id = bind(op, 0);
        s.in[0].id = bind(op, 1);
        s.in[1].id = bind(op, 2);
        s.Kmk = cint(op, "K");
        s.D = cint(op, "D");
        s.seq_rows = true;
      } else {
        fail(KH_EUNSUPPORTED, "kernel " + kn + " has no HIP computation (outside the encoder heads)");
      }
      if (s.kind == S_ATTN) {
        if (s.D < 1 || s.D > ATTN_DMAX)
          fail(KH_EUNSUPPORTED, "attention head dimension " + std::to_string(s.D) + " (1 .. " +
                                    std::to_string(ATTN_DMAX) + " supported)");
      }
      steps.push_back(std::move(s));
    } catch (const Error &e) {
      errors.push_back("op " + name + " (" + kn + "): " + e.what());
    } catch (const std::runtime_error &e) {
      errors.push_back("op " + name + " (" + kn + "): " + e.what());
    }
  }
  return steps;
}

static const Weight *weight_of(kh_ctx *ctx, const std::string &id) {
  if (id.rfind("w:", 0) != 0) return nullptr;
  auto it = ctx->weights.find(id.substr(2));
  return it == ctx->weights.end() ? nullptr : &it->second;
}

// Checks the weights and buffers every step binds; fills `errors`.
static void check_bindings(kh_ctx *ctx, const Parsed &pp, const std::vector<Step> &steps, bool f16,
                           std::vector<std::string> &errors) {
  std::map<std::string, int64_t> decl;
  for (const Json &b : pp.root.at("buffers").arr()) decl[b.at("id").str()] = b.at("bytes").integer();
  const int want = f16 ? KH_F16 : KH_F32;
  auto need_w = [&](const Step &s, const std::string &id, int64_t count, const char *what) {
    if (id == "zero" || id == "dummy") return;
    if (id.rfind("w:", 0) == 0) {
      const Weight *w = weight_of(ctx, id);
      if (!w) {
        errors.push_back("op " + s.name + ": weight " + id.substr(2) + " missing");
        return;
      }
      if (w->dtype != want)
        errors.push_back("op " + s.name + ": weight " + id.substr(2) + " is not in the plan's storage dtype");
      if (w->count < count)
        errors.push_back("op " + s.name + ": weight " + id.substr(2) + " has " + std::to_string(w->count) +
                         " elements, " + what + " needs " + std::to_string(count));
      return;
    }
    if (!decl.count(id)) errors.push_back("op " + s.name + ": unknown buffer " + id);
  };
  for (const Step &s : steps) {
    switch (s.kind) {
      case S_GEMM:
        need_w(s, s.in[1].id, (int64_t)s.N * s.K, "the matmul");
        need_w(s, s.in[2].id, s.N, "the bias");
        break;
      case S_LN:
        need_w(s, s.in[2].id, s.N, "the norm");
        need_w(s, s.in[3].id, s.N, "the norm bias");
        if (s.N > 4096) errors.push_back("op " + s.name + ": LayerNorm width above 4096");
        break;
      case S_EMBLN:
        need_w(s, s.in[1].id, (int64_t)s.maxpos * s.N, "the position table");
        need_w(s, s.in[3].id, s.N, "the norm");
        need_w(s, s.in[4].id, s.N, "the norm bias");
        if (s.N > 4096) errors.push_back("op " + s.name + ": embedding width above 4096");
        break;
      case S_ATTN:
        if (s.rel) {
          need_w(s, s.in[2].id, 0, "c2p");
          need_w(s, s.in[3].id, 0, "p2c");
        }
        break;
      default:
        break;
    }
    for (const Ref &r : s.in)
      if (!r.id.empty() && r.id.rfind("w:", 0) != 0 && r.id != "zero" && r.id != "dummy" && !decl.count(r.id))
        errors.push_back("op " + s.name + ": unknown buffer " + r.id);
  }
}


// ---- fusion of a product with its element-wise consumer ---------------------------------------

// slots a step only writes (its other referenced buffers are read)
static int write_only_slot(const Step &s) {
  switch (s.kind) {
    case S_GEMM: return 3;
    case S_LN: case S_EMBLN: return 5;
    case S_GEGLU: case S_ATTN: case S_POOL: case S_GATHER: case S_COMPACT: return 1;
    default: return -1;  // add and rope update in place: their slot 0 is read too
  }
}

// true when no step from `from` on reads buffer `id` before one overwrites it
static bool dead_after(const std::vector<Step> &steps, size_t from, const std::string &id) {
  for (size_t i = from; i < steps.size(); i++) {
    const Step &s = steps[i];
    const int wo = write_only_slot(s);
    for (int k = 0; k < (int)(sizeof(s.in) / sizeof(s.in[0])); k++)
      if (k != wo && s.in[k].id == id) return false;
    if (wo >= 0 && s.in[wo].id == id) return true;
  }
  return true;
}

// GEMM + GeGLU, GEMM + RoPE, GEMM + residual add and GEMM + residual LayerNorm (MODE 2 over
// 384-wide rows, one tile per row) run as one launch when the lean kernel takes the shape (the
// fused op is applied to the product rounded to the storage type, so results match the separate
// ops); the intermediate buffer then needs no memory.
static void fuse_steps(kh_plan *pl) {
  std::vector<Step> &st = pl->steps;
  std::vector<Step> out;
  for (size_t i = 0; i < st.size(); i++) {
    Step s = st[i];
    if (s.kind == S_GEMM && !s.seq_rows && i + 1 < st.size()) {
      const Step &n = st[i + 1];
      const std::string &c = s.in[3].id;
      GemmArgs g;
      g.lda = s.K;
      g.ldw = s.K;
      g.ldc = s.N;
      g.M = 1 << 20;
      g.N = s.N;
      g.K = s.K;
      g.act = s.act;
      g.a = g.w = (const void *)(uintptr_t)256;  // shape test only: aligned stand-ins
      Step fused = s;
      bool ok = false;
      if (n.kind == S_GEGLU && n.in[0].id == c && 2 * n.I == s.N && c != pl->out_buf && dead_after(st, i + 2, c)) {
        g.epi = EPI_GEGLU;
        g.ldc = n.I;
        if ((ok = gemm_epi_ok(pl->f16, g))) {
          fused.epi = EPI_GEGLU;
          fused.in[3] = n.in[1];
        }
      } else if (n.kind == S_ROPE && n.in[0].id == c && s.N == 3 * n.H * n.D) {
        g.epi = EPI_ROPE;
        g.rope_table = (const float *)(uintptr_t)256;
        g.row_pos = (const int32_t *)(uintptr_t)256;
        g.rope_cols = 2 * n.H * n.D;
        g.rope_d = n.D;
        if ((ok = gemm_epi_ok(pl->f16, g))) {
          fused.epi = EPI_ROPE;
          fused.in[4] = n.in[1];
          fused.H = n.H;
          fused.D = n.D;
        }
      } else if (n.kind == S_ADD && n.mode == 0 && n.in[1].id == c && n.N == s.N && c != pl->out_buf &&
                 dead_after(st, i + 2, c)) {
        g.epi = EPI_RESADD;
        if ((ok = gemm_epi_ok(pl->f16, g))) {
          fused.epi = EPI_RESADD;
          fused.in[3] = n.in[0];
          fused.name = s.name + "+" + n.name;
        }
      } else if (n.kind == S_LN && n.mode == 2 && n.in[1].id == c && n.in[0].id != c && n.N == s.N &&
                 n.in[0].id != pl->in_emb && c != pl->out_buf && dead_after(st, i + 2, c)) {
        g.epi = EPI_LN;
        if ((ok = gemm_epi_ok(pl->f16, g))) {
          fused.epi = EPI_LN;
          fused.in[3] = n.in[5];
          fused.in[4] = n.in[0];
          fused.in[5] = n.in[2];
          fused.in[6] = n.in[3];
          fused.eps = n.eps;
        }
      }
      if (ok) {
        if (fused.epi != EPI_RESADD) fused.name = s.name + "+" + n.name;
        out.push_back(fused);
        i++;
        continue;
      }
    }
    out.push_back(s);
  }
  st.swap(out);
}

// ---- one row per sequence after the last attention ----------------------------------------------

// Row buffers a row-local step reads and writes, with their row widths (elements). False for a
// step that is not row-local over the packed rows, or that takes a buffer as its weight.
struct RowUse {
  int slot, width;
  bool read, write;
};
static bool row_uses(const Step &s, std::vector<RowUse> &u) {
  u.clear();
  auto is_w = [](const std::string &id) { return id.rfind("w:", 0) == 0 || id == "zero" || id == "dummy"; };
  if (s.seq_rows) return false;
  switch (s.kind) {
    case S_GEMM:
      if (s.epi == EPI_ROPE || !is_w(s.in[1].id) || !is_w(s.in[2].id)) return false;
      u.push_back({0, s.K, true, false});
      u.push_back({3, s.epi == EPI_GEGLU ? s.N / 2 : s.N, s.epi == EPI_RESADD, true});
      if (s.epi == EPI_LN) u.push_back({4, s.N, true, false});
      return true;
    case S_LN:
      u.push_back({0, s.N, true, false});
      if (s.mode == 2) u.push_back({1, s.N, true, false});
      u.push_back({5, s.N, false, true});
      return true;
    case S_ADD:
      if (s.mode != 0) return false;
      u.push_back({1, s.N, true, false});
      u.push_back({0, s.N, true, true});
      return true;
    case S_GEGLU:
      u.push_back({0, 2 * s.I, true, false});
      u.push_back({1, s.I, false, true});
      return true;
    default:
      return false;
  }
}

// A pooled-CLS head gathers one row per sequence (pool 'cls' -> gather 'first' with K = 1,
// src/plan/build.ts:303-310): after the last attention only row 0 of each sequence reaches the
// output. The steps between that attention and the gather are row-local, so they run on B rows
// ("id@cls" buffers, one row per sequence) instead of T, the last attention computes only the first
// query tile of each sequence, and the gather becomes a copy of the B rows that zeroes empty
// sequences (as the gather does). Products and LayerNorms treat every row alike, so the B rows
// equal the full computation's row 0 of each sequence.
static void prune_tail(kh_plan *pl) {
  const std::vector<Step> &st = pl->steps;
  int g = -1, a = -1;
  for (int i = 0; i < (int)st.size(); i++) {
    if (st[i].kind == S_GATHER || st[i].kind == S_POOL) {
      if (g >= 0) return;
      g = i;
    }
  }
  // (marker heads gather rows their uploaded payload names: no tail on row 0)
  if (g < 0 || st[g].kind != S_GATHER || st[g].Kmk != 1 || !pl->in_markers.empty()) return;
  for (int i = 0; i < g; i++)
    if (st[i].kind == S_ATTN) a = i;
  if (a < 0) return;
  const int B = pl->B;
  const size_t es = pl->f16 ? 2 : 4;
  auto cls = [](const std::string &id) { return id + "@cls"; };
  std::map<std::string, int> width;      // tail buffer -> widest row it holds
  std::vector<std::pair<std::string, int>> live_in;  // read before the tail writes them
  std::set<std::string> written;
  std::vector<RowUse> u;
  std::vector<Step> tail;
  for (int i = a + 1; i < g; i++) {
    if (!row_uses(st[i], u)) return;
    Step t = st[i];
    for (const RowUse &r : u) {
      const std::string &id = st[i].in[r.slot].id;
      if (!pl->bufs.count(id) || id == pl->out_buf) return;
      if (r.read && !written.count(id)) {
        bool seen = false;
        for (auto &li : live_in) seen = seen || li.first == id;
        if (!seen) live_in.push_back({id, r.width});
      }
      width[id] = std::max(width[id], r.width);
      t.in[r.slot].id = cls(id);
    }
    for (const RowUse &r : u)
      if (r.write) written.insert(st[i].in[r.slot].id);
    t.seq_rows = true;
    t.rows_fixed = B;
    tail.push_back(std::move(t));
  }
  // the gather reads one row of width D per sequence
  const Step &gs = st[g];
  const std::string &src = gs.in[0].id;
  if (!pl->bufs.count(src) || !pl->bufs.count(gs.in[1].id)) return;
  if (!written.count(src)) {
    bool seen = false;
    for (auto &li : live_in) seen = seen || li.first == src;
    if (!seen) live_in.push_back({src, gs.D});
  }
  width[src] = std::max(width[src], gs.D);
  // head steps after the gather work on sequence rows and touch no buffer of the tail
  for (int i = g + 1; i < (int)st.size(); i++) {
    if (!st[i].seq_rows || st[i].kind == S_ATTN || st[i].kind == S_GATHER) return;
    for (const Ref &r : st[i].in)
      if (width.count(r.id)) return;
  }
  for (const auto &li : live_in) {
    const Buffer &b = pl->bufs.at(li.first);
    if (b.bytes < (int64_t)pl->L * B * li.second * (int64_t)es) return;  // not a [L * B, width] row buffer
  }

  std::vector<Step> out(st.begin(), st.begin() + a);
  Step at = st[a];
  at.first_tiles = true;
  out.push_back(at);
  for (const auto &li : live_in) {
    Step c;
    c.kind = S_COMPACT;
    c.name = "compact " + li.first;
    c.in[0].id = li.first;
    c.in[1].id = cls(li.first);
    c.D = width.at(li.first);
    c.mode = 1;
    c.seq_rows = true;
    out.push_back(c);
  }
  for (Step &t : tail) out.push_back(std::move(t));
  Step c;
  c.kind = S_COMPACT;
  c.name = gs.name;
  c.in[0].id = cls(src);
  c.in[1].id = gs.in[1].id;
  c.D = gs.D;
  c.mode = 0;
  c.seq_rows = true;
  out.push_back(c);
  for (int i = g + 1; i < (int)st.size(); i++) out.push_back(st[i]);
  for (const auto &w : width) {
    Buffer b;
    b.bytes = ((int64_t)B * w.second * (int64_t)es + 255) & ~(int64_t)255;
    b.usage = "rw";
    pl->bufs.emplace(cls(w.first), std::move(b));
  }
  pl->steps_pruned.swap(out);
  pl->prune_markers = gs.markers_id;
}

// The pruned list is valid while the gather takes row 0 of every sequence (marker b * 3 is 0).
static void check_markers(kh_plan *pl) {
  const std::vector<uint8_t> &m = pl->markers_shadow;
  bool first = (size_t)pl->B * 3 * 4 <= m.size();
  for (int b = 0; first && b < pl->B; b++) {
    uint32_t v;
    memcpy(&v, m.data() + (size_t)b * 12, 4);
    first = v == 0;
  }
  pl->markers_first = first;
}

static const std::vector<Step> &active_steps(const kh_plan *pl) {
  return !pl->steps_pruned.empty() && pl->markers_first ? pl->steps_pruned : pl->steps;
}

// ---- execution ---------------------------------------------------------------------------------

using LaunchHook = std::function<void(const Step &, const char *kernel, double flops, double bytes, bool begin)>;

static void *bufp(kh_plan *pl, const Ref &r) { return r.p; }

static void exec_step(kh_plan *pl, const Step &s, const LaunchHook &hook, const PrefetchArgs &pf) {
  hipStream_t st = pl->stream;
  const bool f16 = pl->f16;
  const size_t es = f16 ? 2 : 4;
  const Packing pk = packing_of(pl);
  const int64_t rows =
      s.seq_rows ? (s.kind == S_POOL || s.kind == S_GATHER || s.kind == S_COMPACT ? pl->B : s.rows_fixed) : pl->T;
  auto begin = [&](const char *k, double fl, double by) {
    if (hook) hook(s, k, fl, by, true);
  };
  auto end = [&]() {
    if (hook) hook(s, nullptr, 0, 0, false);
  };
  switch (s.kind) {
    case S_GEMM: {
      GemmArgs g;
      g.a = bufp(pl, s.in[0]);
      g.lda = s.K;
      g.w = bufp(pl, s.in[1]);
      g.ldw = s.K;
      g.bias = bufp(pl, s.in[2]);
      g.c = bufp(pl, s.in[3]);
      g.ldc = s.N;
      g.M = (int)rows;
      g.N = s.N;
      g.K = s.K;
      g.act = s.act;
      g.epi = s.epi;
      double out_elems = (double)rows * s.N;  // written (the residual add also reads them)
      if (s.epi == EPI_GEGLU) {
        g.ldc = s.N / 2;
        out_elems = (double)rows * s.N / 2;
      } else if (s.epi == EPI_ROPE) {
        g.rope_table = (const float *)bufp(pl, s.in[4]);
        g.row_pos = pk.row_pos;
        g.rope_cols = 2 * s.H * s.D;
        g.rope_d = s.D;
      } else if (s.epi == EPI_RESADD) {
        out_elems *= 2;
      } else if (s.epi == EPI_LN) {
        g.ln_res = bufp(pl, s.in[4]);
        g.ln_g = bufp(pl, s.in[5]);
        g.ln_b = bufp(pl, s.in[6]);
        g.ln_eps = s.eps;
        out_elems = 2.0 * rows * s.N + 2.0 * s.N;  // the residual read, the rows written, gamma and beta
      }
      begin(gemm_on_mfma(f16, g) ? "gemm_mfma" : "gemm_rowdot", 2.0 * rows * s.N * s.K,
            (double)es * ((double)rows * s.K + (double)s.N * s.K + out_elems + (g.bias ? s.N : 0)));
      gemm(f16, g, st);
      end();
      break;
    }
    case S_LN: {
      if (pl->by_ids && s.in[0].id == pl->in_emb) {
        // the embedding LN of plans without position or type tables (DeBERTa, ModernBERT) over
        // rows gathered from the device word table: the same LN kernel reading row ids[r] of the
        // table, so the result equals the LN of the uploaded rows bit for bit
        begin("layernorm", 8.0 * pl->T * s.N, 2.0 * es * pl->T * s.N + 4.0 * pl->T);
        layernorm(f16, pl->ctx->words->p, nullptr, bufp(pl, s.in[2]), bufp(pl, s.in[3]), bufp(pl, s.in[5]), pl->T,
                  s.N, s.eps, st, (const int32_t *)pl->d_ids.p, pf, s.mode == 1 ? pk.row_w : nullptr);
        end();
        break;
      }
      const void *b = s.mode == 2 ? bufp(pl, s.in[1]) : nullptr;
      begin("layernorm", 8.0 * rows * s.N, (double)es * ((s.mode == 2 ? 3.0 : 2.0) * rows * s.N + 2.0 * s.N));
      // MODE 1 multiplies by the mask: 1 on every packed row of a 0/1 prefix mask, else row_w
      layernorm(f16, bufp(pl, s.in[0]), b, bufp(pl, s.in[2]), bufp(pl, s.in[3]), bufp(pl, s.in[5]), rows, s.N, s.eps,
                st, nullptr, pf, s.mode == 1 && !s.seq_rows ? pk.row_w : nullptr);
      end();
      break;
    }
    case S_EMBLN: {
      EmbLnArgs a;
      a.word = pl->by_ids ? nullptr : bufp(pl, s.in[0]);
      a.table = pl->by_ids ? pl->ctx->words->p : nullptr;
      a.ids = pl->by_ids ? (const int32_t *)pl->d_ids.p : nullptr;
      a.pos = bufp(pl, s.in[1]);
      a.typ = bufp(pl, s.in[2]);
      a.tt = pl->in_tt.empty() ? nullptr : (const uint32_t *)pl->d_tt.p;
      a.gamma = bufp(pl, s.in[3]);
      a.beta = bufp(pl, s.in[4]);
      a.out = bufp(pl, s.in[5]);
      a.N = s.N;
      a.offset = s.offset;
      a.maxpos = s.maxpos;
      a.posids = s.posids;
      a.eps = s.eps;
      a.row_scale = s.maskmul ? pk.row_w : nullptr;
      const int tables = 1 + (a.pos ? 1 : 0) + (a.typ ? 1 : 0);
      begin("embln", 9.0 * pl->T * s.N, (double)es * (tables + 1.0) * pl->T * s.N + 4.0 * pl->T);
      embln(f16, a, pk, st, pf);
      end();
      break;
    }
    case S_ADD:
      begin("add", (double)rows * s.N, 3.0 * es * rows * s.N);
      add(f16, bufp(pl, s.in[0]), bufp(pl, s.in[1]), rows, s.N, s.mode, pk, st);
      end();
      break;
    case S_GEGLU:
      begin("geglu", 20.0 * rows * s.I, 3.0 * es * rows * s.I);
      geglu(f16, bufp(pl, s.in[0]), bufp(pl, s.in[1]), rows, s.I, st);
      end();
      break;
    case S_COMPACT:
      begin("compact", 0, 2.0 * es * pl->B * s.D);
      first_rows(f16, bufp(pl, s.in[0]), bufp(pl, s.in[1]), s.D, s.mode == 1, pk, st);
      end();
      break;
    case S_ROPE: {
      const float *table = (const float *)bufp(pl, s.in[1]);
      begin("rope", 6.0 * pl->T * 2 * s.H * (s.D / 2), 4.0 * es * pl->T * s.H * s.D);
      rope(f16, bufp(pl, s.in[0]), table, pl->T, s.H, s.D, pl->L, pk, st);
      end();
      break;
    }
    case S_POOL:
      begin("pool", (double)pl->T * s.N, (double)es * ((double)pl->T * s.N + (double)pl->B * s.N));
      pool(f16, bufp(pl, s.in[0]), bufp(pl, s.in[1]), s.N, s.mode, pk, st);
      end();
      break;
    case S_MASKL: {
      const int64_t total = (int64_t)pl->B * s.Kmk;
      begin("masklogits", (double)total, (double)total * (es + 4.0 + 4.0));
      mask_logits(f16, bufp(pl, s.in[0]), (const uint32_t *)bufp(pl, s.in[1]), (float *)bufp(pl, s.in[2]), s.Kmk,
                  s.scale, total, st);
      end();
      break;
    }
    case S_GATHER: {
      auto it = pl->bufs.find(s.markers_id);
      const uint32_t *mk = it != pl->bufs.end() && it->second.mem ? (const uint32_t *)it->second.mem->p : nullptr;
      begin("gather", 0, 2.0 * es * pl->B * s.Kmk * s.D);
      gather_rows(f16, bufp(pl, s.in[0]), mk, bufp(pl, s.in[1]), s.Kmk, s.D, pk, st);
      end();
      break;
    }
    case S_ATTN: {
      AttnArgs a;
      a.qkv = bufp(pl, s.in[0]);
      a.ctx = bufp(pl, s.in[1]);
      a.H = s.H;
      a.D = s.D;
      a.scale = s.scale;
      a.window = s.window;
      a.tiles = (const int4 *)(s.first_tiles ? pl->d_tiles_first.p : pl->d_tiles.p);
      a.ntiles = s.first_tiles ? pl->ntiles_first : pl->ntiles;
      a.nwork = s.first_tiles ? pl->nwork_first : pl->nwork;
      if (a.nwork > 0 && s.H == pl->work_h) a.work = (const int4 *)(s.first_tiles ? pl->d_work_first.p : pl->d_work.p);
      else a.nwork = 0;
      const double hd = (double)s.H * s.D;
      double pairs = s.first_tiles ? pl->attn_pairs_first : pl->attn_pairs_global;
      if (s.window > 0) pairs = (s.first_tiles ? pl->attn_pairs_first_window : pl->attn_pairs_window)[s.window];
      // q and ctx rows of the computed tiles, k and v of every row
      const double io_rows = s.first_tiles ? 2.0 * pl->T + 2.0 * pl->rows_first : 4.0 * pl->T;
      double rel_fl = 0;
      if (s.rel) {
        // q . pos_key[m] and k . pos_query[m] over the buckets each sequence reaches, inside the kernel
        a.pos_key = bufp(pl, s.in[2]);
        a.pos_query = bufp(pl, s.in[3]);
        a.bucket = (const int32_t *)pl->d_bucket.p;
        a.nb = pl->rel_nb;
        a.lmax = pl->L;
        rel_fl = 4.0 * hd * (s.first_tiles ? pl->rel_rows_buckets_first : pl->rel_rows_buckets);
      }
      begin(s.rel ? "attention_rel" : "attention", 4.0 * hd * pairs + rel_fl, (double)es * io_rows * hd);
      attention(f16, a, pk, st);
      end();
      break;
    }
  }
}

// ---- packing ----------------------------------------------------------------------------------

// Attention blocks in dispatch order. The dispatcher deals block b to XCD b % 8, and each XCD
// starts its blocks in order. A (sequence, head) group's query tiles stay on one XCD (they share the
// sequence's K and V rows in that XCD's L2). Groups go to the XCD with the least work so far,
// largest first (the longest-processing-time rule), and each XCD runs its longest groups first, so
// the blocks that visit the most key tiles do not start last. A block's work is taken as its key
// tiles plus a fixed cost: on a ragged batch the longest sequences' blocks visit several times the
// key tiles of the others (c2: 3 against 1.4 on average; c4: 128 against 80).
static std::vector<int4> attn_order(const std::vector<int4> &tiles, int H) {
  const int nt = (int)tiles.size();
  struct Group {
    double w;
    int t0, t1, h;
  };
  std::vector<Group> groups;
  for (int t0 = 0; t0 < nt;) {
    int t1 = t0;
    while (t1 < nt && tiles[t1].x == tiles[t0].x) t1++;  // a sequence's tiles are consecutive
    const double per = 0.3 + (tiles[t0].w + ATTN_QTILE - 1) / ATTN_QTILE;
    for (int h = 0; h < H; h++) groups.push_back({per * (t1 - t0), t0, t1, h});
    t0 = t1;
  }
  std::stable_sort(groups.begin(), groups.end(), [](const Group &a, const Group &b) { return a.w > b.w; });
  double load[8] = {};
  std::vector<int32_t> lists[8];
  for (const Group &g : groups) {
    int x = 0;
    for (int i = 1; i < 8; i++)
      if (load[i] < load[x]) x = i;
    load[x] += g.w;
    for (int t = g.t0; t < g.t1; t++) lists[x].push_back(g.h * nt + t);
  }
  size_t len = 0;
  for (const auto &l : lists) len = std::max(len, l.size());
  std::vector<int4> work(8 * len, int4{-1, 0, 0, 0});
  for (int x = 0; x < 8; x++)
    for (size_t i = 0; i < lists[x].size(); i++) {
      const int item = lists[x][i];
      const int4 &t = tiles[item % nt];
      work[x + 8 * i] = int4{item / nt, t.y, t.z, t.w};
    }
  return work;
}

static void pack(kh_plan *pl, int rows, int b_end) {
  const int L = pl->L, B = pl->B;
  std::vector<int32_t> n(B);
  bool masked = false;
  for (int b = 0; b < B; b++) {
    const float *m = pl->mask_host.data() + (size_t)b * L;
    const int len = seq_extent(m, L);
    int cap = b < b_end ? rows - b * L : 0;
    cap = cap < 0 ? 0 : (cap > L ? L : cap);
    n[b] = len < cap ? len : cap;
    for (int i = 0; i < n[b] && !masked; i++) masked = m[i] != 1.0f;
  }
  pl->cu.assign(B + 1, 0);
  for (int b = 0; b < B; b++) pl->cu[b + 1] = pl->cu[b] + n[b];
  const int64_t T = pl->cu[B];
  pl->T = T;
  std::vector<int32_t> row_pos(T > 0 ? T : 1), row_seq(T > 0 ? T : 1);
  std::vector<int4> tiles;
  pl->attn_pairs_global = 0;
  std::vector<int4> tiles_first;
  std::set<int> windows;
  for (const Step &s : pl->steps)
    if (s.kind == S_ATTN && s.window > 0) windows.insert(s.window);
  pl->attn_pairs_window.clear();
  pl->attn_pairs_first = 0;
  pl->attn_pairs_first_window.clear();
  pl->rows_first = 0;
  for (int b = 0; b < B; b++) {
    for (int i = 0; i < n[b]; i++) {
      row_pos[pl->cu[b] + i] = i;
      row_seq[pl->cu[b] + i] = b;
    }
    for (int q = 0; q < n[b]; q += ATTN_QTILE) tiles.push_back(make_int4(b, q, pl->cu[b], n[b]));
    const int nq = std::min(n[b], ATTN_QTILE);
    if (n[b] > 0) tiles_first.push_back(make_int4(b, 0, pl->cu[b], n[b]));
    pl->rows_first += nq;
    pl->attn_pairs_global += (double)n[b] * n[b];
    pl->attn_pairs_first += (double)nq * n[b];
    for (int w : windows) {
      double s = 0, s1 = 0;
      for (int i = 0; i < n[b]; i++) {
        const int lo = std::max(0, i - w), hi = std::min(n[b] - 1, i + w);
        s += hi - lo + 1;
        if (i < nq) s1 += hi - lo + 1;
      }
      pl->attn_pairs_window[w] += s;
      pl->attn_pairs_first_window[w] += s1;
    }
  }
  pl->ntiles = (int)tiles.size();
  pl->ntiles_first = (int)tiles_first.size();
  pl->rel_rows_buckets = 0;
  pl->rel_rows_buckets_first = 0;
  if (!pl->bucket_host.empty())
    for (int b = 0; b < B; b++)
      if (n[b] > 0) {
        // buckets reached by distances -(n - 1) .. n - 1, counted as the range between the two
        // extreme distances' buckets (exact for tables monotone in i - j, as DeBERTa's)
        const double range = pl->bucket_host[(L - 1) + (n[b] - 1)] - pl->bucket_host[(L - 1) - (n[b] - 1)] + 1;
        pl->rel_rows_buckets += (double)n[b] * range;
        // first tile: c2p over its query rows, p2c over every key row
        pl->rel_rows_buckets_first += 0.5 * (std::min(n[b], ATTN_QTILE) + n[b]) * range;
      }
  if (tiles.empty()) tiles.push_back(make_int4(0, 0, 0, 0));
  if (tiles_first.empty()) tiles_first.push_back(make_int4(0, 0, 0, 0));
  // attention dispatch order, for the plan's head count (steps with another take the plain order)
  int H = 0;
  for (const Step &s : pl->steps)
    if (s.kind == S_ATTN && H == 0) H = s.H;
  std::vector<int4> work, work_first;
  if (H > 0) {
    work = attn_order(tiles, H);
    work_first = attn_order(tiles_first, H);
  }
  pl->work_h = H;
  pl->nwork = (int)work.size();
  pl->nwork_first = (int)work_first.size();

  // metadata: cu | row_pos | row_seq | tiles | tt | ids, one pinned staging block
  const size_t es = pl->f16 ? 2 : 4;
  if (pl->d_cu.bytes < (size_t)(B + 1) * 4 || !pl->d_cu.p) pl->d_cu.alloc((size_t)(B + 1) * 4);
  if (pl->d_row_pos.bytes < (size_t)T * 4 || !pl->d_row_pos.p) pl->d_row_pos.alloc(std::max<int64_t>(T, 1) * 4);
  if (pl->d_row_seq.bytes < (size_t)T * 4 || !pl->d_row_seq.p) pl->d_row_seq.alloc(std::max<int64_t>(T, 1) * 4);
  if (pl->d_tiles.bytes < tiles.size() * sizeof(int4) || !pl->d_tiles.p) pl->d_tiles.alloc(tiles.size() * sizeof(int4));
  if (pl->d_tiles_first.bytes < tiles_first.size() * sizeof(int4) || !pl->d_tiles_first.p)
    pl->d_tiles_first.alloc(tiles_first.size() * sizeof(int4));
  if (!work.empty() && (pl->d_work.bytes < work.size() * sizeof(int4) || !pl->d_work.p))
    pl->d_work.alloc(work.size() * sizeof(int4));
  if (!work_first.empty() && (pl->d_work_first.bytes < work_first.size() * sizeof(int4) || !pl->d_work_first.p))
    pl->d_work_first.alloc(work_first.size() * sizeof(int4));
  KH_CHECK(hipStreamSynchronize(pl->stream));  // staging may still feed an earlier copy
  // ten blocks at most (cu, row_pos, row_seq, tiles, first tiles, the two work lists, type ids,
  // ids, markers), each 16-byte aligned
  const size_t T1 = (size_t)std::max<int64_t>(T, 1);
  const size_t meta = (size_t)(B + 1) * 4 + 5 * T1 * 4 + (tiles.size() + tiles_first.size()) * sizeof(int4) +
                      (work.size() + work_first.size()) * sizeof(int4) + pl->markers_host.size() * 4 + 11 * 16;
  pl->pin_meta.ensure(meta);
  char *mp = (char *)pl->pin_meta.p;
  char *const mend = mp + meta;
  auto put = [&](DevMem &dst, const void *src, size_t bytes) {
    if (mp + bytes > mend || bytes > dst.bytes) fail(KH_EINVAL, "internal: packing staging overflow");
    memcpy(mp, src, bytes);
    KH_CHECK(hipMemcpyAsync(dst.p, mp, bytes, hipMemcpyHostToDevice, pl->stream));
    mp += (bytes + 15) & ~(size_t)15;
  };
  put(pl->d_cu, pl->cu.data(), (size_t)(B + 1) * 4);
  put(pl->d_row_pos, row_pos.data(), (size_t)std::max<int64_t>(T, 1) * 4);
  put(pl->d_row_seq, row_seq.data(), (size_t)std::max<int64_t>(T, 1) * 4);
  put(pl->d_tiles, tiles.data(), tiles.size() * sizeof(int4));
  put(pl->d_tiles_first, tiles_first.data(), tiles_first.size() * sizeof(int4));
  if (!work.empty()) put(pl->d_work, work.data(), work.size() * sizeof(int4));
  if (!work_first.empty()) put(pl->d_work_first, work_first.data(), work_first.size() * sizeof(int4));
  pl->masked = masked;
  if (masked) {
    std::vector<float> w(T1, 0.f);
    for (int b = 0; b < B; b++)
      for (int i = 0; i < n[b]; i++) w[pl->cu[b] + i] = pl->mask_host[(size_t)b * L + i];
    if (pl->d_row_w.bytes < T1 * 4 || !pl->d_row_w.p) pl->d_row_w.alloc(T1 * 4);
    put(pl->d_row_w, w.data(), T1 * 4);
  }
  // packed type ids
  if (!pl->in_tt.empty()) {
    // type rows the embedding reads must exist (an out-of-range id would read past the table)
    int64_t type_rows = INT64_MAX;
    for (const Step &s : pl->steps)
      if (s.kind == S_EMBLN) {
        const Weight *w = weight_of(pl->ctx, s.in[2].id);
        type_rows = w ? w->count / std::max(1, s.N) : (s.in[2].id == "zero" ? 1 : 0);
      }
    std::vector<uint32_t> tt(std::max<int64_t>(T, 1), 0u);
    for (int b = 0; b < B; b++)
      for (int i = 0; i < n[b]; i++) {
        const uint32_t v = pl->tt_host.empty() ? 0u : pl->tt_host[(size_t)b * L + i];
        if ((int64_t)(v & 0xffffu) >= type_rows)
          fail(KH_EINVAL, "token type " + std::to_string(v & 0xffffu) + " outside the type table");
        tt[pl->cu[b] + i] = v;
      }
    if (pl->d_tt.bytes < tt.size() * 4 || !pl->d_tt.p) pl->d_tt.alloc(tt.size() * 4);
    put(pl->d_tt, tt.data(), tt.size() * 4);
  }
  // rowSelect: the type row of each sequence (device-to-device, ordered before the forward)
  if (!pl->rs_dst.empty()) {
    const Weight *w = weight_of(pl->ctx, pl->rs_table);
    const int64_t rows = w->count * (pl->f16 ? 2 : 4) / pl->rs_row_bytes;
    char *dst = (char *)pl->bufs.at(pl->rs_dst).mem->p;
    for (int b = 0; b < B; b++) {
      const uint32_t q = pl->qtype_host[b];
      if ((int64_t)q >= rows)
        fail(KH_EINVAL, "qtype " + std::to_string(q) + " of sequence " + std::to_string(b) + " outside the " +
                            std::to_string(rows) + " rows of " + pl->rs_table.substr(2));
      KH_CHECK(hipMemcpyAsync(dst + (size_t)b * pl->rs_row_bytes, (const char *)w->mem->p + (size_t)q * pl->rs_row_bytes,
                              pl->rs_row_bytes, hipMemcpyDeviceToDevice, pl->stream));
    }
  }
  // packed marker payloads: B blocks of 3 K u32 (row indices, mask bits, groups), rows within L
  if (!pl->in_markers.empty()) {
    const int K = pl->markers;
    for (int b = 0; b < B; b++)
      for (int k = 0; k < K; k++) {
        const uint32_t r = pl->markers_host[(size_t)b * 3 * K + k];
        if (r >= (uint32_t)L)
          fail(KH_EINVAL, "marker " + std::to_string(k) + " of sequence " + std::to_string(b) + " names row " +
                              std::to_string(r) + ", the plan length is " + std::to_string(L));
      }
    put(*pl->bufs.at(pl->in_markers).mem, pl->markers_host.data(), pl->markers_host.size() * 4);
  }
  // packed word rows or ids
  if (pl->by_ids) {
    std::vector<int32_t> ids(std::max<int64_t>(T, 1), 0);
    for (int b = 0; b < B; b++)
      for (int i = 0; i < n[b]; i++) {
        const int32_t id = pl->ids_host[(size_t)b * L + i];
        if (id < 0 || id >= pl->ctx->words_rows)
          fail(KH_EINVAL, "token id " + std::to_string(id) + " outside the word table");
        ids[pl->cu[b] + i] = id;
      }
    if (pl->d_ids.bytes < ids.size() * 4 || !pl->d_ids.p) pl->d_ids.alloc(ids.size() * 4);
    put(pl->d_ids, ids.data(), ids.size() * 4);
  } else {
    const size_t row = (size_t)pl->E * es;
    Buffer &eb = pl->bufs.at(pl->in_emb);
    if ((size_t)T * row > eb.mem->bytes) fail(KH_EINVAL, "packed rows exceed the emb buffer");
    // the upload packed each sequence's rows already: when this run takes all of them (the usual
    // case) they go to the device as they are; a run that takes fewer rows of some sequence (a
    // smaller row count) copies its rows once more, into pin_pack
    bool same = true;
    for (int b = 0; b < B; b++) {
      if (n[b] > pl->avail[b]) fail(KH_EINVAL, "word rows shorter than the mask's valid rows");
      same = same && pl->cu[b] == pl->up_cu[b] && n[b] == pl->avail[b];
    }
    const uint8_t *src = pl->up_rows;
    if (!same && T > 0) {
      pl->pin_pack.ensure((size_t)T * row);
      for (int b = 0; b < B; b++)
        if (n[b]) memcpy((char *)pl->pin_pack.p + (size_t)pl->cu[b] * row, pl->up_rows + (size_t)pl->up_cu[b] * row,
                         (size_t)n[b] * row);
      src = (const uint8_t *)pl->pin_pack.p;
    }
    if (T > 0) KH_CHECK(hipMemcpyAsync(eb.mem->p, src, (size_t)T * row, hipMemcpyHostToDevice, pl->stream));
  }
  pl->dirty = false;
  pl->last_rows = rows;
}

static void ensure_rel(kh_plan *pl) {
  bool rel = false;
  for (const Step &s : pl->steps) rel = rel || s.rel;
  if (!rel) return;
  if (!pl->d_bucket.p) fail(KH_EINVAL, "relative attention needs the relidx table (kh_plan_init_buffer)");
}

static int64_t env_int(const char *name, int64_t dflt);

// bytes of a product's weight matrix worth a prefetch (below this the product's own first reads
// are a small part of it)
constexpr size_t PREFETCH_MIN = 256 * 1024;
// rows below which a forward is bound by its launches' latency (c1: 128 rows): its products read
// their weights once anyway, and a prefetch would only move that read into the LayerNorm (a c1
// forward took 0.93 ms with it against 0.58 ms without)
constexpr int64_t PREFETCH_MIN_ROWS = 2048;

// A LayerNorm over the packed rows carries the weights of the products up to the next LayerNorm
// (PrefetchArgs: its threads read them after their rows), so those products find them in the
// memory-side cache: a layer's weights come cold from HBM otherwise, which costs a product up to
// a quarter of its time when the weights are a sizeable part of its operands (c2: 14 MB of
// weights per layer against 20 MB rows, FFN out's 4.7 MB against 79 MB). Products whose weights
// are under a 32nd of their row operand (c4, c5: under 1 MB against hundreds) gain nothing and
// are left out.
static PrefetchArgs prefetch_for(kh_plan *pl, const std::vector<Step> &steps, size_t i) {
  PrefetchArgs a;
  if (pl->T < PREFETCH_MIN_ROWS) return a;
  int r = 0;
  for (size_t j = i + 1; j < steps.size() && r < PREFETCH_RANGES; j++) {
    const Step &s = steps[j];
    if (s.kind == S_LN || s.kind == S_EMBLN) break;
    if (s.kind != S_GEMM || s.seq_rows) continue;
    const size_t es = pl->f16 ? 2 : 4;
    const size_t bytes = (size_t)s.N * s.K * es;
    if (bytes < PREFETCH_MIN || bytes * 32 < (size_t)pl->T * s.K * es) continue;
    a.p[r] = bufp(pl, s.in[1]);
    a.n16[r] = (int64_t)(bytes / 16);
    a.total += a.n16[r];
    r++;
  }
  return a;
}

static void run_steps(kh_plan *pl, const LaunchHook &hook) {
  const std::vector<Step> &steps = active_steps(pl);
  const bool pf = env_int("KH_NO_PREFETCH", 0) == 0;
  for (size_t i = 0; i < steps.size(); i++) {
    const bool ln = (steps[i].kind == S_LN || steps[i].kind == S_EMBLN) && !steps[i].seq_rows;
    exec_step(pl, steps[i], hook, pf && ln ? prefetch_for(pl, steps, i) : PrefetchArgs());
  }
  KH_CHECK(hipGetLastError());
}

// ---- the twin: the second half of a small batch on its own stream ------------------------------

static void init_buffer(kh_plan *plan, const char *id, const void *data, size_t bytes) {
  auto it = plan->bufs.find(id);
  if (it == plan->bufs.end()) fail(KH_EINVAL, std::string("plan buffer ") + id + " missing");
  Buffer &b = it->second;
  if ((int64_t)bytes > b.bytes) fail(KH_EINVAL, std::string("init of ") + id + " larger than the buffer");
  // an unchanged table needs no device write (the twin's shifted CLS markers on every upload)
  if (b.init.size() == bytes && (bytes == 0 || memcmp(b.init.data(), data, bytes) == 0) && b.init_done) return;
  // kernels already queued on the plan's stream may read the table being replaced: the copies
  // below are synchronous and unordered with that stream, so they wait for it first
  if (plan->stream) KH_CHECK(hipStreamSynchronize(plan->stream));
  b.init.assign((const uint8_t *)data, (const uint8_t *)data + bytes);
  b.init_done = true;
  const std::string sid = id;
  if (sid == "relidx") {
    // relidx[i][j] depends on i - j only: keep bucket(i - j) for i - j in [-(L-1), L-1]
    const int L = plan->L;
    if (bytes != (size_t)L * L * 4) fail(KH_EINVAL, "relidx must hold L * L u32");
    const uint32_t *t = (const uint32_t *)data;
    plan->bucket_host.assign(2 * L - 1, 0);
    for (int d = -(L - 1); d <= L - 1; d++) plan->bucket_host[d + L - 1] = (int32_t)(d >= 0 ? t[(size_t)d * L] : t[-d]);
    for (int i = 0; i < L; i++)
      for (int j = 0; j < L; j++)
        if ((int32_t)t[(size_t)i * L + j] != plan->bucket_host[i - j + L - 1])
          fail(KH_EUNSUPPORTED, "relidx is not a function of i - j");
    for (int32_t v : plan->bucket_host)
      if (v < 0 || v >= plan->rel_nb) fail(KH_EINVAL, "relidx entry outside the position table");
    plan->d_bucket.alloc(plan->bucket_host.size() * 4);
    KH_CHECK(hipMemcpy(plan->d_bucket.p, plan->bucket_host.data(), plan->bucket_host.size() * 4, hipMemcpyHostToDevice));
    return;
  }
  if (b.mem) KH_CHECK(hipMemcpy(b.mem->p, data, bytes, hipMemcpyHostToDevice));
  if (sid == plan->prune_markers) {
    memcpy(plan->markers_shadow.data(), data, bytes);
    check_markers(plan);
  }
}

static int64_t env_int(const char *name, int64_t dflt) {
  const char *e = getenv(name);
  return e && *e ? atoll(e) : dflt;
}

// Sequences [0, split) stay on this plan; 0 runs the batch whole. Only batch calls (rows = L * B)
// of plans whose output rows are per sequence or per token split, and only below KH_SPLIT_T valid
// rows (default 400000: a few hundred thousand rows of long sequences still leave the chip idle
// in attention phases the other half fills; at a million rows the halves gain nothing), with both
// halves holding
// about half the rows.
static int choose_split(const kh_plan *pl, int rows) {
  if (pl->is_twin || pl->twin_failed || pl->B < 2 || rows != pl->L * pl->B || env_int("KH_NO_SPLIT", 0)) return 0;
  if (!pl->in_markers.empty()) return 0;  // marker heads run whole
  const bool per_seq = !pl->out_packed && pl->out_rows == pl->B;
  const bool per_tok = pl->out_packed && pl->out_rows == pl->L * pl->B;
  if (!per_seq && !per_tok) return 0;
  std::vector<int64_t> pre(pl->B + 1, 0);
  for (int b = 0; b < pl->B; b++) {
    pre[b + 1] = pre[b] + seq_extent(pl->mask_host.data() + (size_t)b * pl->L, pl->L);
  }
  const int64_t T = pre[pl->B];
  if (T < env_int("KH_SPLIT_MIN", 2048) || T >= env_int("KH_SPLIT_T", 400000)) return 0;
  int split = 1;
  while (split < pl->B - 1 && 2 * pre[split] < T) split++;
  if (pre[split] == 0 || pre[split] == T) return 0;
  return split;
}

// device bytes of the plan's activation buffers (what a twin allocates again)
static int64_t plan_buffer_bytes(const kh_plan *pl) {
  int64_t n = 0;
  for (const auto &b : pl->bufs)
    if (b.second.mem) n += (int64_t)b.second.mem->bytes;
  return n;
}

// KH_ENOMEM when the twin cannot be allocated (KH_TWIN_MAX_BYTES caps its buffers, for tests of
// this path); the caller then runs the batch whole
static void ensure_twin(kh_plan *pl) {
  if (pl->twin) return;
  const int64_t cap = env_int("KH_TWIN_MAX_BYTES", -1);
  if (cap >= 0 && plan_buffer_bytes(pl) > cap)
    fail(KH_ENOMEM, "twin plan: " + std::to_string(plan_buffer_bytes(pl)) + " bytes of buffers over KH_TWIN_MAX_BYTES");
  kh_plan *t = nullptr;
  int rc = kh_plan_create(pl->ctx, pl->json.data(), pl->json.size(), &t);
  if (rc) fail(rc, std::string("twin plan: ") + kh_last_error());
  t->is_twin = true;
  for (const auto &in : pl->init_log) {
    rc = kh_plan_init_buffer(t, in.first.c_str(), in.second.data(), in.second.size());
    if (rc) {
      const std::string m = kh_last_error();
      kh_plan_destroy(t);
      fail(rc, "twin plan: " + m);
    }
  }
  KH_CHECK(hipEventCreateWithFlags(&pl->ev_twin, hipEventDisableTiming));
  pl->twin = t;
}

// bytes per sequence of a per-sequence init table (the gather markers: K triples of u32 per
// sequence, the row first); 0 for tables that do not index sequences
static size_t seq_stride(const kh_plan *pl, const std::string &id) {
  for (const Step &s : pl->steps)
    if (s.kind == S_GATHER && s.markers_id == id) return (size_t)s.Kmk * 3 * 4;
  return 0;
}

// a per-sequence init table as the twin holds it: sequence split + j at slot j, zeros after
static std::vector<uint8_t> shifted_table(const std::vector<uint8_t> &v, size_t per, int split) {
  std::vector<uint8_t> out(v.size(), 0);
  const size_t from = (size_t)split * per;
  if (from < v.size()) memcpy(out.data(), v.data() + from, v.size() - from);
  return out;
}

// the twin's host arrays: sequences [split, B) of this plan's upload at slots [0, B - split)
static void stage_twin(kh_plan *pl, int split) {
  kh_plan *t = pl->twin;
  for (const auto &in : pl->init_log)
    if (const size_t per = seq_stride(pl, in.first)) {
      const std::vector<uint8_t> v = shifted_table(in.second, per, split);
      init_buffer(t, in.first.c_str(), v.data(), v.size());
    }
  const size_t L = pl->L, M = L * pl->B, moved = (size_t)(pl->B - split) * L, from = (size_t)split * L;
  t->mask_host.assign(M, 0.f);
  memcpy(t->mask_host.data(), pl->mask_host.data() + from, moved * 4);
  t->tt_host.clear();
  if (!pl->tt_host.empty()) {
    t->tt_host.assign(M, 0u);
    memcpy(t->tt_host.data(), pl->tt_host.data() + from, moved * 4);
  }
  t->by_ids = pl->by_ids;
  if (pl->by_ids) {
    t->ids_host.assign(M, 0);
    memcpy(t->ids_host.data(), pl->ids_host.data() + from, moved * 4);
  } else {
    // the moved sequences' rows stay where this plan's upload packed them (contiguous from the
    // split's first row): the twin's copy to the device reads them there
    const size_t row = (size_t)pl->E * (pl->f16 ? 2 : 4);
    t->up_rows = pl->up_rows + (size_t)pl->up_cu[split] * row;
    t->up_cu.assign(pl->B + 1, pl->up_cu[pl->B] - pl->up_cu[split]);
    t->avail.assign(pl->B, 0);
    for (int b = split; b < pl->B; b++) {
      t->up_cu[b - split] = pl->up_cu[b] - pl->up_cu[split];
      t->avail[b - split] = pl->avail[b];
    }
  }
  t->uploaded = true;
  t->dirty = true;
}

// packs (when the upload or the split changed) and enqueues the forward of the whole batch
static void launch_forward(kh_plan *pl, int rows, const LaunchHook &hook, bool sequential) {
  // the split depends on the upload (dirty), the row count and the two switches
  const int64_t env =
      (env_int("KH_NO_SPLIT", 0) * 1000003 + env_int("KH_SPLIT_T", 400000)) * 1000003 + env_int("KH_SPLIT_MIN", 2048);
  if (pl->dirty || pl->split_memo < 0 || rows != pl->split_memo_rows || env != pl->split_memo_env) {
    pl->split_memo = choose_split(pl, rows);
    pl->split_memo_rows = rows;
    pl->split_memo_env = env;
  }
  int split = pl->split_memo;
  if (split > 0 && !pl->twin) {
    try {
      ensure_twin(pl);
    } catch (const Error &e) {
      if (e.code != KH_ENOMEM) throw;
      // out of device memory for the second half's buffers: this plan runs whole from now on
      (void)hipGetLastError();
      pl->twin_failed = true;
      pl->split_memo = split = 0;
    }
  }
  if (split > 0 && (pl->dirty || split != pl->split)) stage_twin(pl, split);
  if (pl->dirty || rows != pl->last_rows || split != pl->split) pack(pl, rows, split > 0 ? split : pl->B);
  pl->split = split;
  ensure_rel(pl);
  kh_plan *t = pl->twin;
  if (split > 0 && !hook) {
    // both halves packed (the second reads the rows this plan's upload packed, in place), then
    // their launches interleaved step by step, so that both streams have work from the start (a
    // call that uploads, runs and reads back pays the host's launch time once, not half after half)
    if (t->dirty) pack(t, t->L * t->B, t->B);
    ensure_rel(t);
    KH_CHECK(hipEventRecord(pl->ev0, pl->stream));
    // the twin's half starts with this call, not when the twin finished the previous call's half
    // (ev0 follows everything queued before on the plan's stream, the previous call's end included)
    KH_CHECK(hipStreamWaitEvent(t->stream, pl->ev0, 0));
    const std::vector<Step> &s1 = active_steps(pl), &s2 = active_steps(t);
    const bool pf = env_int("KH_NO_PREFETCH", 0) == 0;
    auto step = [&](kh_plan *p, const std::vector<Step> &st, size_t i) {
      const bool ln = (st[i].kind == S_LN || st[i].kind == S_EMBLN) && !st[i].seq_rows;
      // (the halves run in step, so the twin's products find the weights this plan's LayerNorms
      // brought in: only this plan's carry the prefetch; c2 +0.8 %)
      exec_step(p, st[i], hook, pf && ln && p == pl ? prefetch_for(p, st, i) : PrefetchArgs());
    };
    for (size_t i = 0; i < std::max(s1.size(), s2.size()); i++) {
      if (i < s1.size()) step(pl, s1, i);
      if (i < s2.size()) step(t, s2, i);
    }
    KH_CHECK(hipGetLastError());
    KH_CHECK(hipEventRecord(pl->ev_twin, t->stream));
    KH_CHECK(hipStreamWaitEvent(pl->stream, pl->ev_twin, 0));
    t->ran = true;
    KH_CHECK(hipEventRecord(pl->ev1, pl->stream));
    pl->ran = true;
    return;
  }
  KH_CHECK(hipEventRecord(pl->ev0, pl->stream));
  run_steps(pl, hook);
  if (split > 0) {
    if (t->dirty) pack(t, t->L * t->B, t->B);
    ensure_rel(t);
    if (sequential) KH_CHECK(hipStreamSynchronize(pl->stream));  // profiled halves one after the other
    KH_CHECK(hipStreamWaitEvent(t->stream, pl->ev0, 0));
    run_steps(t, hook);
    KH_CHECK(hipEventRecord(pl->ev_twin, t->stream));
    KH_CHECK(hipStreamWaitEvent(pl->stream, pl->ev_twin, 0));
    t->ran = true;
  }
  KH_CHECK(hipEventRecord(pl->ev1, pl->stream));
  pl->ran = true;
}

static hipEvent_t take_event(kh_plan *pl) {
  if (!pl->ev_pool.empty()) {
    hipEvent_t e = pl->ev_pool.back();
    pl->ev_pool.pop_back();
    return e;
  }
  hipEvent_t e;
  KH_CHECK(hipEventCreate(&e));
  return e;
}

// the traced launches of kh_run go to pl->trace (both halves of a split batch)
static LaunchHook trace_hook(kh_plan *pl) {
  return [pl](const Step &s, const char *k, double fl, double by, bool begin) {
    if (begin) {
      TraceRec r;
      r.name = s.name;
      r.kernel = k;
      r.flops = fl;
      r.bytes = by;
      r.a = take_event(pl);
      r.b = take_event(pl);
      pl->trace.push_back(r);
      g_launch_events.start = r.a;
      g_launch_events.stop = r.b;
    } else {
      g_launch_events = LaunchEvents();
    }
  };
}

static void release_trace(kh_plan *pl) {
  for (TraceRec &r : pl->trace) {
    pl->ev_pool.push_back(r.a);
    pl->ev_pool.push_back(r.b);
  }
  pl->trace.clear();
}

static void latch(kh_ctx *ctx, const Error &e) {
  if (e.code == KH_EHIP) {
    hipError_t q = hipGetLastError();
    (void)q;
    ctx->lost = true;
    ctx->lost_msg = e.what();
  }
}

}  // namespace kh

// ---- C ABI ------------------------------------------------------------------------------------

#define KH_API_BEGIN try {
#define KH_API_END                                                      \
  g_last_error.clear();                                                 \
  return KH_OK;                                                         \
  }                                                                     \
  catch (const kh::Error &e) {                                          \
    g_last_error = e.what();                                            \
    return e.code;                                                      \
  }                                                                     \
  catch (const std::bad_alloc &) {                                      \
    g_last_error = "host allocation failed";                            \
    return KH_ENOMEM;                                                   \
  }                                                                     \
  catch (const std::exception &e) {                                     \
    g_last_error = e.what();                                            \
    return KH_EINVAL;                                                   \
  }

static void require_live(kh_ctx *ctx) {
  if (!ctx) fail(KH_EINVAL, "null context");
  if (ctx->lost) fail(KH_ELOST, "context lost after an earlier device failure: " + ctx->lost_msg);
  KH_CHECK(hipSetDevice(ctx->device));
}

namespace kh {
// the message kh_last_error() returns, for the host-only parts of the library (sched.cpp)
void set_last_error(const std::string &m) { g_last_error = m; }
}  // namespace kh

extern "C" {

const char *kh_last_error(void) { return g_last_error.c_str(); }
int kh_abi_version(void) { return KH_ABI_VERSION; }

int kh_ctx_create(int device, kh_ctx **out) {
  KH_API_BEGIN
  if (!out) fail(KH_EINVAL, "null output pointer");
  int n = 0;
  KH_CHECK(hipGetDeviceCount(&n));
  if (device < 0 || device >= n) fail(KH_EINVAL, "device " + std::to_string(device) + " of " + std::to_string(n));
  KH_CHECK(hipSetDevice(device));
  auto *c = new kh_ctx();
  c->device = device;
  *out = c;
  KH_API_END
}

int kh_ctx_destroy(kh_ctx *ctx) {
  KH_API_BEGIN
  if (ctx) {
    (void)hipSetDevice(ctx->device);
    delete ctx;
  }
  KH_API_END
}

int kh_weight_add(kh_ctx *ctx, const char *name, int dtype, const int64_t *shape, int ndim, const void *data,
                  size_t bytes) {
  KH_API_BEGIN
  require_live(ctx);
  if (!name || !*name) fail(KH_EINVAL, "weight without a name");
  if (dtype != KH_F32 && dtype != KH_F16 && dtype != KH_U32) fail(KH_EINVAL, "weight dtype " + std::to_string(dtype));
  if (ndim < 0 || ndim > 8 || (ndim > 0 && !shape)) fail(KH_EINVAL, "weight shape");
  if (ctx->weights.count(name)) fail(KH_EINVAL, std::string("weight ") + name + " loaded twice");
  int64_t count = 1;
  std::vector<int64_t> sh;
  for (int i = 0; i < ndim; i++) {
    if (shape[i] < 0) fail(KH_EINVAL, "negative dimension");
    count *= shape[i];
    sh.push_back(shape[i]);
  }
  if ((size_t)count * elem_size(dtype) != bytes)
    fail(KH_EINVAL, std::string("weight ") + name + ": " + std::to_string(bytes) + " bytes for " +
                        std::to_string(count) + " elements");
  if (bytes && !data) fail(KH_EINVAL, "null weight data");
  Weight w;
  w.dtype = dtype;
  w.shape = sh;
  w.count = count;
  w.mem.reset(new DevMem());
  w.mem->alloc(bytes);
  if (bytes) KH_CHECK(hipMemcpy(w.mem->p, data, bytes, hipMemcpyHostToDevice));
  ctx->weight_bytes += bytes;
  ctx->weights.emplace(name, std::move(w));
  KH_API_END
}

int kh_ctx_weight_bytes(const kh_ctx *ctx, uint64_t *out) {
  KH_API_BEGIN
  if (!ctx || !out) fail(KH_EINVAL, "null argument");
  *out = ctx->weight_bytes;
  KH_API_END
}

int kh_words_set(kh_ctx *ctx, int dtype, int64_t rows, int64_t width, const void *data, size_t bytes) {
  KH_API_BEGIN
  require_live(ctx);
  if (dtype != KH_F32 && dtype != KH_F16) fail(KH_EINVAL, "word table dtype");
  if (rows <= 0 || width <= 0 || (size_t)(rows * width) * elem_size(dtype) != bytes || !data)
    fail(KH_EINVAL, "word table size");
  ctx->words.reset(new DevMem());
  ctx->words->alloc(bytes);
  KH_CHECK(hipMemcpy(ctx->words->p, data, bytes, hipMemcpyHostToDevice));
  ctx->words_dtype = dtype;
  ctx->words_rows = rows;
  ctx->words_width = width;
  KH_API_END
}

// ---- manifest directories ----------------------------------------------------------------------

// Host-to-device copies from pageable (mapped) memory through two pinned chunks: the CPU fills one
// chunk while the DMA engine drains the other.
struct Stager {
  static constexpr size_t CH = 32u << 20;
  hipStream_t s = nullptr;
  hipEvent_t ev[2] = {nullptr, nullptr};
  HostPinned buf[2];
  bool pending[2] = {false, false};
  int cur = 0;
  size_t used = 0;
  Stager() {
    KH_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    KH_CHECK(hipEventCreateWithFlags(&ev[0], hipEventDisableTiming));
    KH_CHECK(hipEventCreateWithFlags(&ev[1], hipEventDisableTiming));
    buf[0].ensure(CH);
    buf[1].ensure(CH);
  }
  ~Stager() {
    if (s) (void)hipStreamSynchronize(s);
    for (hipEvent_t e : ev)
      if (e) (void)hipEventDestroy(e);
    if (s) (void)hipStreamDestroy(s);
  }
  void flip() {
    KH_CHECK(hipEventRecord(ev[cur], s));
    pending[cur] = true;
    cur ^= 1;
    if (pending[cur]) KH_CHECK(hipEventSynchronize(ev[cur]));
    pending[cur] = false;
    used = 0;
  }
  // `rows` rows of `row` bytes, `stride` bytes apart in host memory, to dst back to back
  void put_rows(char *dst, const uint8_t *src, size_t rows, size_t row, size_t stride) {
    while (rows) {
      if (CH - used < row) flip();
      const size_t k = std::min(rows, (CH - used) / row);
      char *b = (char *)buf[cur].p + used;
      if (stride == row) memcpy(b, src, k * row);
      else
        for (size_t i = 0; i < k; i++) memcpy(b + i * row, src + i * stride, row);
      KH_CHECK(hipMemcpyAsync(dst, b, k * row, hipMemcpyHostToDevice, s));
      used += k * row;
      dst += k * row;
      src += k * stride;
      rows -= k;
    }
  }
  void put(void *dst, const uint8_t *src, size_t n) {
    // whole chunks, then the rest
    const size_t full = n / CH;
    if (full) put_rows((char *)dst, src, full, CH, CH);
    if (n % CH) put_rows((char *)dst + full * CH, src + full * CH, 1, n % CH, n % CH);
  }
  void finish() { KH_CHECK(hipStreamSynchronize(s)); }
};

static std::unique_ptr<mf::Loaded> read_manifest(const char *path, int flags) {
  if (!path || !*path) fail(KH_EINVAL, "null manifest path");
  try {
    return mf::load(path, flags);
  } catch (const std::runtime_error &e) {
    fail(KH_EINVAL, e.what());
  }
  return nullptr;
}

static void manifest_info(const mf::Loaded &L, kh_manifest_info *out) {
  memset(out, 0, sizeof(*out));
  out->version = L.version;
  out->shards = (int32_t)L.shards.size();
  out->words_dtype = L.words_dtype;
  out->words_rows = L.words_rows;
  out->words_width = L.words_width;
  for (const mf::Tensor &t : L.tensors)
    if (!t.keep_on_cpu) {
      out->tensors++;
      out->tensor_bytes += t.bytes;
    }
  out->file_bytes = L.file_bytes;
  out->read_ms = L.read_ms;
  out->sha256_ms = L.sha256_ms;
  out->rows_ms = L.rows_ms;
}

int kh_manifest_check(const char *manifest_path, int flags, kh_manifest_info *out) {
  KH_API_BEGIN
  auto L = read_manifest(manifest_path, flags);
  if (out) manifest_info(*L, out);
  KH_API_END
}

int kh_load_manifest(kh_ctx *ctx, const char *manifest_path, int flags, kh_manifest_info *out) {
  KH_API_BEGIN
  require_live(ctx);
  auto L = read_manifest(manifest_path, flags);
  for (const mf::Tensor &t : L->tensors)
    if (!t.keep_on_cpu && ctx->weights.count(t.name)) fail(KH_EINVAL, "weight " + t.name + " loaded twice");
  const auto t0 = std::chrono::steady_clock::now();
  std::vector<std::pair<std::string, uint64_t>> added;
  try {
    Stager st;
    for (const mf::Tensor &t : L->tensors) {
      if (t.keep_on_cpu) continue;
      Weight w;
      w.dtype = t.dtype;
      w.shape = t.shape;
      w.count = (int64_t)(t.bytes / elem_size(t.dtype));
      w.mem.reset(new DevMem());
      w.mem->alloc(t.bytes);
      if (t.bytes) st.put(w.mem->p, L->shards[t.shard]->p + t.offset, t.bytes);
      ctx->weight_bytes += t.bytes;
      ctx->weights.emplace(t.name, std::move(w));
      added.push_back({t.name, t.bytes});
    }
    std::unique_ptr<DevMem> words;
    if (L->words_data && !(flags & KH_LOAD_NO_WORDS)) {
      // rows of words.bin carry a checksum word after the values: the staging copy drops it
      const size_t row = (size_t)L->words_width * elem_size(L->words_dtype);
      words.reset(new DevMem());
      words->alloc(row * (size_t)L->words_rows);
      st.put_rows((char *)words->p, L->words_data, (size_t)L->words_rows, row, (size_t)L->words_stride);
    }
    st.finish();
    if (words) {
      ctx->words = std::move(words);
      ctx->words_dtype = L->words_dtype;
      ctx->words_rows = L->words_rows;
      ctx->words_width = L->words_width;
    }
  } catch (...) {
    for (const auto &n : added) {
      ctx->weight_bytes -= n.second;
      ctx->weights.erase(n.first);
    }
    throw;
  }
  if (out) {
    manifest_info(*L, out);
    out->upload_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
  }
  KH_API_END
}

int kh_sha256(const void *data, size_t bytes, uint8_t out[32]) {
  KH_API_BEGIN
  if (!out || (bytes && !data)) fail(KH_EINVAL, "null argument");
  mf::sha256(data, bytes, out);
  KH_API_END
}

int kh_row_checksum(const void *row, size_t bytes, uint32_t row_id, uint32_t salt, uint32_t *out) {
  KH_API_BEGIN
  if (!out || (bytes && !row)) fail(KH_EINVAL, "null argument");
  if (bytes % 4) fail(KH_EINVAL, "words: row of " + std::to_string(bytes) + " bytes is not whole u32 words");
  *out = mf::row_checksum((const uint8_t *)row, bytes, row_id, salt);
  KH_API_END
}

static std::string join_errors(const std::vector<std::string> &errs) {
  std::string m;
  for (const auto &e : errs) m += (m.empty() ? "" : "; ") + e;
  return m;
}

int kh_plan_check(kh_ctx *ctx, const char *plan_json, size_t len) {
  KH_API_BEGIN
  // a null context checks the plan's structure only (no weights, no device)
  Parsed pp = parse_plan(plan_json, len);
  const bool f16 = pp.root.at("f16").kind == Json::Bool && pp.root.at("f16").b;
  const int L = (int)pp.root.at("length").integer();
  std::vector<std::string> errors;
  auto steps = lower(pp, f16, L, errors);
  if (ctx) check_bindings(ctx, pp, steps, f16, errors);
  if (!errors.empty()) fail(KH_EUNSUPPORTED, join_errors(errors));
  KH_API_END
}

int kh_plan_create(kh_ctx *ctx, const char *plan_json, size_t len, kh_plan **out) {
  KH_API_BEGIN
  require_live(ctx);
  if (!out) fail(KH_EINVAL, "null output pointer");
  Parsed pp = parse_plan(plan_json, len);
  std::unique_ptr<kh_plan> pl(new kh_plan());
  pl->ctx = ctx;
  pl->json.assign(plan_json, len);
  pl->f16 = pp.root.at("f16").kind == Json::Bool && pp.root.at("f16").b;
  pl->L = (int)pp.root.at("length").integer();
  pl->B = (int)pp.root.at("batch").integer();
  pl->markers = (int)pp.root.at("markers").integer();
  pl->E = (int)pp.root.at("embeddingSize").integer();
  if (pl->L <= 0 || pl->B <= 0) fail(KH_EINVAL, "plan length and batch must be positive");
  std::vector<std::string> errors;
  pl->steps = lower(pp, pl->f16, pl->L, errors);
  check_bindings(ctx, pp, pl->steps, pl->f16, errors);
  const Json &inputs = pp.root.at("inputs");
  if (!errors.empty()) fail(KH_EUNSUPPORTED, join_errors(errors));
  if (inputs.has("markers")) {
    pl->in_markers = inputs.at("markers").str();
    if (pl->markers < 1) fail(KH_EINVAL, "a plan with a markers input needs markers >= 1");
  }
  if (pp.root.has("rowSelect") && pp.root.at("rowSelect").kind != Json::Null) {
    const Json &rs = pp.root.at("rowSelect");
    pl->rs_table = rs.at("table").str();
    pl->rs_dst = rs.at("dst").str();
    pl->rs_row_bytes = rs.at("rowBytes").integer();
    const Weight *w = weight_of(ctx, pl->rs_table);
    const int64_t es = pl->f16 ? 2 : 4;
    if (!w) fail(KH_EINVAL, "rowSelect table " + pl->rs_table + " missing");
    if (w->dtype != (pl->f16 ? KH_F16 : KH_F32) || pl->rs_row_bytes <= 0 || pl->rs_row_bytes % es ||
        w->count * es < pl->rs_row_bytes)
      fail(KH_EINVAL, "rowSelect table " + pl->rs_table + " does not hold rows of " + std::to_string(pl->rs_row_bytes) + " B");
    pl->qtype_host.assign(pl->B, 0u);
  }
  pl->in_emb = inputs.at("embeddings").str();
  pl->out_buf = pp.root.at("output").at("buffer").str();
  if (!getenv("KH_NO_FUSION")) fuse_steps(pl.get());
  pl->in_mask = inputs.at("mask").str();
  if (inputs.has("typeIds")) pl->in_tt = inputs.at("typeIds").str();
  const Json &o = pp.root.at("output");
  pl->out_buf = o.at("buffer").str();
  pl->out_rows = (int)o.at("rows").integer();
  pl->out_cols = (int)o.at("cols").integer();
  const std::string odt = o.at("dtype").str();
  if (odt != "storage" && odt != "f32") fail(KH_EUNSUPPORTED, "output dtype " + odt);
  pl->out_f32 = odt == "f32" || !pl->f16;

  for (const Json &b : pp.root.at("buffers").arr()) {
    Buffer buf;
    buf.bytes = b.at("bytes").integer();
    buf.usage = b.at("usage").str();
    pl->bufs.emplace(b.at("id").str(), std::move(buf));
  }
  if (!pl->in_markers.empty()) {
    // payloads start as masked slots at row 0 (logits -1e4) until kh_upload_markers
    pl->markers_host.assign((size_t)3 * pl->markers * pl->B, 0u);
    if (!pl->bufs.count(pl->in_markers) || pl->bufs.at(pl->in_markers).bytes < (int64_t)pl->markers_host.size() * 4)
      fail(KH_EINVAL, "markers buffer smaller than 3 * markers * batch u32");
  }
  if (!pl->rs_dst.empty() &&
      (!pl->bufs.count(pl->rs_dst) || pl->bufs.at(pl->rs_dst).bytes < pl->rs_row_bytes * pl->B))
    fail(KH_EINVAL, "rowSelect destination smaller than batch rows");
  if (!getenv("KH_NO_PRUNE")) prune_tail(pl.get());
  // row spaces and uses
  pl->bufs.at(pl->in_emb).packed_space = true;
  std::vector<Step *> all_steps;
  for (Step &s : pl->steps) all_steps.push_back(&s);
  for (Step &s : pl->steps_pruned) all_steps.push_back(&s);
  for (Step *sp : all_steps) {
    Step &s = *sp;
    for (Ref &r : s.in) {
      if (r.id.empty() || r.id.rfind("w:", 0) == 0 || r.id == "zero" || r.id == "dummy") continue;
      pl->bufs.at(r.id).used = true;
    }
    if (!s.markers_id.empty() && pl->bufs.count(s.markers_id)) pl->bufs.at(s.markers_id).used = true;
    const std::string *dst = nullptr;
    switch (s.kind) {
      case S_GEMM: dst = &s.in[3].id; break;
      case S_LN: dst = &s.in[5].id; break;
      case S_EMBLN: dst = &s.in[5].id; break;
      case S_GEGLU: dst = &s.in[1].id; break;
      case S_ATTN: dst = &s.in[1].id; break;
      case S_POOL: dst = &s.in[1].id; break;
      case S_GATHER: dst = &s.in[1].id; break;
      case S_COMPACT: dst = &s.in[1].id; break;
      case S_MASKL: dst = &s.in[2].id; break;
      default: break;
    }
    if (dst) {
      Buffer &b = pl->bufs.at(*dst);
      if (s.seq_rows) b.seq_space = true;
      else b.packed_space = true;
      if (b.seq_space && b.packed_space) fail(KH_EUNSUPPORTED, "buffer " + *dst + " holds both packed and sequence rows");
    }
  }
  pl->bufs.at(pl->out_buf).used = true;
  pl->bufs.at(pl->in_emb).used = true;
  pl->out_packed = pl->bufs.at(pl->out_buf).packed_space;
  // in-place kernels read what their destination held: the residual stream of a pre-norm layer
  for (Step *s : all_steps)
    if ((s->kind == S_ADD || s->kind == S_ROPE) && !s->seq_rows && pl->bufs.count(s->in[0].id))
      pl->bufs.at(s->in[0].id).packed_space = true;
  if (!pl->prune_markers.empty()) {
    const Buffer &mb = pl->bufs.at(pl->prune_markers);
    pl->markers_shadow.assign((size_t)mb.bytes, 0);  // device copy starts zeroed
    check_markers(pl.get());
  }

  KH_CHECK(hipSetDevice(ctx->device));
  KH_CHECK(hipStreamCreateWithFlags(&pl->stream, hipStreamNonBlocking));
  KH_CHECK(hipEventCreate(&pl->ev0));
  KH_CHECK(hipEventCreate(&pl->ev1));
  // relative attention: bucket table per (i - j) from the relidx init table (kh_plan_init_buffer)
  for (auto &kv : pl->bufs) {
    Buffer &b = kv.second;
    const std::string &id = kv.first;
    if (!b.used) continue;
    if (id == pl->in_mask || id == "kinfo" || id == "scores" || id == "c2p" || id == "p2c" || id == "dummy") continue;
    b.mem.reset(new DevMem());
    b.mem->alloc((size_t)b.bytes);
    KH_CHECK(hipMemset(b.mem->p, 0, (size_t)b.bytes));
  }
  // resolve step pointers
  for (Step *sp : all_steps) {
    Step &s = *sp;
    for (Ref &r : s.in) {
      if (r.id.empty()) continue;
      if (r.id == "zero" || r.id == "dummy") {
        r.p = nullptr;
      } else if (r.id.rfind("w:", 0) == 0) {
        const Weight *w = weight_of(ctx, r.id);
        r.p = w ? w->mem->p : nullptr;
      } else {
        Buffer &b = pl->bufs.at(r.id);
        r.p = b.mem ? b.mem->p : nullptr;
      }
    }
    if (s.kind == S_ATTN && s.rel) {
      if (pl->L > ATTN_REL_LMAX)
        fail(KH_EUNSUPPORTED, "op " + s.name + ": relative attention over more than " + std::to_string(ATTN_REL_LMAX) +
                                  " rows per sequence");
      const Weight *pk = weight_of(ctx, s.in[2].id);
      if (!pk || pk->shape.size() != 2 || pk->shape[1] != (int64_t)s.H * s.D)
        fail(KH_EINVAL, "op " + s.name + ": position table must be [2 * buckets, H * D]");
      pl->rel_nb = std::max(pl->rel_nb, (int)pk->shape[0]);
    }
  }
  *out = pl.release();
  KH_API_END
}



int kh_plan_init_buffer(kh_plan *plan, const char *id, const void *data, size_t bytes) {
  KH_API_BEGIN
  if (!plan || !id) fail(KH_EINVAL, "null argument");
  require_live(plan->ctx);
  init_buffer(plan, id, data, bytes);
  // kept for the twin (created at the first split run), and applied to it when it exists
  std::vector<uint8_t> copy((const uint8_t *)data, (const uint8_t *)data + bytes);
  bool logged = false;
  for (auto &in : plan->init_log)
    if (in.first == id) {
      in.second = copy;
      logged = true;
    }
  if (!logged) plan->init_log.push_back({id, copy});
  if (plan->twin) {
    // per-sequence tables move with the twin's sequences (stage_twin shifts them again when the
    // split changes)
    const size_t per = seq_stride(plan, id);
    if (per && plan->split > 0) {
      const std::vector<uint8_t> v = shifted_table(copy, per, plan->split);
      init_buffer(plan->twin, id, v.data(), v.size());
    } else {
      init_buffer(plan->twin, id, data, bytes);
    }
  }
  KH_API_END
}

int kh_plan_info_get(const kh_plan *plan, kh_plan_info *out) {
  KH_API_BEGIN
  if (!plan || !out) fail(KH_EINVAL, "null argument");
  memset(out, 0, sizeof(*out));
  out->length = plan->L;
  out->batch = plan->B;
  out->markers = plan->markers;
  out->f16 = plan->f16;
  uint64_t bytes = 0;
  for (const auto &kv : plan->bufs)
    if (kv.second.mem) bytes += kv.second.mem->bytes;
  if (plan->twin)
    for (const auto &kv : plan->twin->bufs)
      if (kv.second.mem) bytes += kv.second.mem->bytes;

  out->bytes = bytes;
  out->out_rows = plan->out_rows;
  out->out_cols = plan->out_cols;
  out->launches = (int32_t)active_steps(plan).size();
  out->streams = plan->split > 0 ? 2 : 1;
  KH_API_END
}

static void stage_common(kh_plan *plan, const float *mask, size_t mask_count, const uint32_t *tt, size_t tt_count) {
  const size_t M = (size_t)plan->L * plan->B;
  if (!mask || mask_count == 0 || mask_count > M) fail(KH_EINVAL, "mask must hold 1 .. L * B values");
  plan->mask_host.assign(M, 0.f);
  memcpy(plan->mask_host.data(), mask, mask_count * 4);
  plan->tt_host.clear();
  if (!plan->in_tt.empty()) {
    if (!tt) fail(KH_EINVAL, "plan needs typeIds");
    if (tt_count > M) fail(KH_EINVAL, "typeIds longer than the plan");
    plan->tt_host.assign(M, 0u);
    memcpy(plan->tt_host.data(), tt, tt_count * 4);
  }
  plan->uploaded = true;
  plan->dirty = true;
}

int kh_upload(kh_plan *plan, const void *emb, size_t emb_bytes, const float *mask, size_t mask_count,
              const uint32_t *type_ids, size_t type_count) {
  KH_API_BEGIN
  if (!plan) fail(KH_EINVAL, "null plan");
  require_live(plan->ctx);
  const auto &eb = plan->bufs.at(plan->in_emb);
  if (!emb && emb_bytes) fail(KH_EINVAL, "null word rows");
  if ((int64_t)emb_bytes > eb.bytes)
    fail(KH_EINVAL, "input emb has " + std::to_string(emb_bytes) + " B, the buffer " + std::to_string(eb.bytes));
  // copies still reading the pinned rows of the previous upload (this plan's, and its twin's,
  // which reads the same memory) must finish before they are overwritten
  if (plan->stream) KH_CHECK(hipStreamSynchronize(plan->stream));
  if (plan->twin && plan->twin->stream) KH_CHECK(hipStreamSynchronize(plan->twin->stream));
  stage_common(plan, mask, mask_count, type_ids, type_count);
  // only the rows a run can read (each sequence's rows up to its last nonzero mask value, a
  // ragged batch of 256 at L = 512 holds ~10 % of L * B) are copied, once, packed, into pinned
  // memory: a run that takes them all sends them to the device from there
  const size_t row = (size_t)plan->E * (plan->f16 ? 2 : 4);
  const size_t L = plan->L;
  plan->up_cu.assign(plan->B + 1, 0);
  plan->avail.assign(plan->B, 0);
  for (int b = 0; b < plan->B; b++) {
    const size_t len = (size_t)seq_extent(plan->mask_host.data() + (size_t)b * L, (int)L);
    const size_t from = (size_t)b * L * row;
    const size_t given = from >= emb_bytes ? 0 : (emb_bytes - from) / row;
    plan->avail[b] = (int32_t)std::min(len, given);
    plan->up_cu[b + 1] = plan->up_cu[b] + plan->avail[b];
  }
  plan->pin_up.ensure(std::max<size_t>((size_t)plan->up_cu[plan->B] * row, 16));
  // a few threads share the copy when it is large (c2: 20 MB; one thread copies ~10 GB/s)
  const size_t total = (size_t)plan->up_cu[plan->B] * row;
  const int nth = total < ((size_t)8 << 20) ? 1 : (int)std::min<unsigned>(8, std::max(1u, std::thread::hardware_concurrency()));
  auto copy_range = [&](int b0, int b1) {
    for (int b = b0; b < b1; b++)
      if (plan->avail[b])
        memcpy((char *)plan->pin_up.p + (size_t)plan->up_cu[b] * row, (const uint8_t *)emb + (size_t)b * L * row,
               (size_t)plan->avail[b] * row);
  };
  if (nth == 1) {
    copy_range(0, plan->B);
  } else {
    // sequence ranges of about equal rows per thread
    std::vector<std::thread> th;
    int b0 = 0;
    for (int k = 0; k < nth && b0 < plan->B; k++) {
      const int64_t goal = plan->up_cu[plan->B] * (k + 1) / nth;
      int b1 = b0;
      while (b1 < plan->B && (plan->up_cu[b1] < goal || b1 == b0)) b1++;
      if (k == nth - 1) b1 = plan->B;
      th.emplace_back(copy_range, b0, b1);
      b0 = b1;
    }
    for (auto &x : th) x.join();
  }
  plan->up_rows = (const uint8_t *)plan->pin_up.p;
  plan->by_ids = false;
  KH_API_END
}

int kh_upload_ids(kh_plan *plan, const int32_t *ids, size_t id_count, const float *mask, size_t mask_count,
                  const uint32_t *type_ids, size_t type_count) {
  KH_API_BEGIN
  if (!plan) fail(KH_EINVAL, "null plan");
  require_live(plan->ctx);
  kh_ctx *c = plan->ctx;
  if (!c->words) fail(KH_EINVAL, "no device word table (kh_words_set)");
  if (c->words_dtype != (plan->f16 ? KH_F16 : KH_F32) || c->words_width != plan->E)
    fail(KH_EINVAL, "word table dtype or width differs from the plan");
  const size_t M = (size_t)plan->L * plan->B;
  if (!ids || id_count > M) fail(KH_EINVAL, "ids must hold up to L * B values");
  // the word rows feed the embedding LN only (embln, or a layernorm without residual): the run
  // gathers them from the table inside that step
  for (const Step &s : plan->steps)
    for (int i = 0; i < 6; i++)
      if (s.in[i].id == plan->in_emb && !(i == 0 && (s.kind == S_EMBLN || (s.kind == S_LN && s.mode != 2))))
        fail(KH_EUNSUPPORTED, "op " + s.name + " reads the word rows: upload them (kh_upload)");
  stage_common(plan, mask, mask_count, type_ids, type_count);
  plan->ids_host.assign(M, 0);
  memcpy(plan->ids_host.data(), ids, id_count * 4);
  plan->by_ids = true;
  KH_API_END
}

int kh_upload_markers(kh_plan *plan, const uint32_t *packed, size_t count) {
  KH_API_BEGIN
  if (!plan) fail(KH_EINVAL, "null plan");
  require_live(plan->ctx);
  if (plan->in_markers.empty()) fail(KH_EINVAL, "the plan has no markers input");
  // as the reference's upload puts the array at the buffer's start (src/plan/wasm.ts:411-416): a
  // shorter payload leaves the later slots as they were, a longer one is an error
  const size_t want = (size_t)3 * plan->markers * plan->B;
  if ((count && !packed) || count > want)
    fail(KH_EINVAL, "packed markers hold " + std::to_string(count) + " u32, the plan takes up to 3 * " +
                        std::to_string(plan->markers) + " * " + std::to_string(plan->B) + " = " + std::to_string(want));
  if (count) memcpy(plan->markers_host.data(), packed, count * 4);
  plan->dirty = true;  // the payload travels with the next run's packed metadata
  KH_API_END
}

int kh_upload_qtypes(kh_plan *plan, const uint32_t *qtype, size_t count) {
  KH_API_BEGIN
  if (!plan) fail(KH_EINVAL, "null plan");
  require_live(plan->ctx);
  if (plan->rs_dst.empty()) fail(KH_EINVAL, "the plan has no rowSelect (type rows)");
  if (count > (size_t)plan->B || (count && !qtype))
    fail(KH_EINVAL, std::to_string(count) + " qtypes, the plan has " + std::to_string(plan->B) + " sequences");
  // sequences without an entry take row 0 (qtypes[b] ?? 0)
  std::fill(plan->qtype_host.begin(), plan->qtype_host.end(), 0u);
  if (count) memcpy(plan->qtype_host.data(), qtype, count * 4);
  plan->dirty = true;
  KH_API_END
}

int kh_run(kh_plan *plan, int32_t rows) {
  KH_API_BEGIN
  if (!plan) fail(KH_EINVAL, "null plan");
  require_live(plan->ctx);
  if (rows < 1 || rows > plan->L * plan->B)
    fail(KH_EINVAL, std::to_string(rows) + " rows, the plan has " + std::to_string(plan->L * plan->B));
  if (!plan->uploaded) fail(KH_EINVAL, "run before upload");
  try {
    if (plan->tracing) {
      launch_forward(plan, rows, trace_hook(plan), false);
      g_launch_events = LaunchEvents();
    } else {
      launch_forward(plan, rows, nullptr, false);
    }
  } catch (const Error &e) {
    g_launch_events = LaunchEvents();
    latch(plan->ctx, e);
    throw;
  }
  KH_API_END
}

int kh_sync(kh_plan *plan) {
  KH_API_BEGIN
  if (!plan) fail(KH_EINVAL, "null plan");
  require_live(plan->ctx);
  try {
    KH_CHECK(hipStreamSynchronize(plan->stream));
    if (plan->twin) KH_CHECK(hipStreamSynchronize(plan->twin->stream));
  } catch (const Error &e) {
    latch(plan->ctx, e);
    throw;
  }
  KH_API_END
}

int kh_last_run_ms(kh_plan *plan, float *ms) {
  KH_API_BEGIN
  if (!plan || !ms) fail(KH_EINVAL, "null argument");
  if (!plan->ran) fail(KH_EINVAL, "no run yet");
  KH_CHECK(hipEventSynchronize(plan->ev1));
  KH_CHECK(hipEventElapsedTime(ms, plan->ev0, plan->ev1));
  KH_API_END
}

int kh_plan_read_buffer(kh_plan *plan, const char *id, int32_t half, void *out, size_t bytes) {
  KH_API_BEGIN
  if (!plan || !id || (!out && bytes)) fail(KH_EINVAL, "null argument");
  require_live(plan->ctx);
  kh_plan *p = plan;
  if (half) {
    if (!plan->twin || plan->split <= 0) fail(KH_EINVAL, "the last run did not split the batch");
    p = plan->twin;
  }
  auto it = p->bufs.find(id);
  if (it == p->bufs.end() || !it->second.mem) fail(KH_EINVAL, std::string("plan buffer ") + id + " has no device memory");
  const size_t n = std::min(bytes, it->second.mem->bytes);
  try {
    KH_CHECK(hipStreamSynchronize(p->stream));
    if (n) KH_CHECK(hipMemcpy(out, it->second.mem->p, n, hipMemcpyDeviceToHost));
  } catch (const Error &e) {
    latch(plan->ctx, e);
    throw;
  }
  KH_API_END
}

int kh_packed_rows(const kh_plan *plan, int64_t *out) {
  KH_API_BEGIN
  if (!plan || !out) fail(KH_EINVAL, "null argument");
  *out = plan->T + (plan->split > 0 && plan->twin ? plan->twin->T : 0);
  KH_API_END
}

// the plan's own output (its sequences only) in the plan's output layout
static void read_into(kh_plan *plan, float *out, size_t n) {
  Buffer &b = plan->bufs.at(plan->out_buf);
  const size_t es = plan->f16 ? 2 : 4;
  const int cols = plan->out_cols;
  if (!plan->out_packed) {
    const size_t oes = plan->out_f32 ? 4 : es;
    std::vector<uint8_t> raw(n * oes);
    KH_CHECK(hipMemcpyAsync(raw.data(), b.mem->p, n * oes, hipMemcpyDeviceToHost, plan->stream));
    KH_CHECK(hipStreamSynchronize(plan->stream));
    // sequences without a valid row: zero output (the reference computes them from padding)
    for (size_t i = 0; i < n; i++) out[i] = plan->out_f32 ? ((const float *)raw.data())[i] : (float)((const _Float16 *)raw.data())[i];
    if (plan->out_rows == plan->B && plan->in_markers.empty())
      for (int bb = 0; bb < plan->B; bb++)
        if (plan->cu[bb + 1] == plan->cu[bb]) memset(out + (size_t)bb * cols, 0, (size_t)cols * 4);
  } else {
    // token rows: packed row cu[b] + i goes to b * L + i; rows past a sequence are zero
    const int64_t T = plan->T;
    std::vector<uint8_t> raw((size_t)std::max<int64_t>(T, 1) * cols * es);
    if (T > 0) KH_CHECK(hipMemcpyAsync(raw.data(), b.mem->p, (size_t)T * cols * es, hipMemcpyDeviceToHost, plan->stream));
    KH_CHECK(hipStreamSynchronize(plan->stream));
    memset(out, 0, n * 4);
    for (int bb = 0; bb < plan->B; bb++)
      for (int i = 0; i < plan->cu[bb + 1] - plan->cu[bb]; i++) {
        const size_t src = ((size_t)plan->cu[bb] + i) * cols, dst = ((size_t)bb * plan->L + i) * cols;
        if (dst + cols > n) break;
        for (int c = 0; c < cols; c++)
          out[dst + c] = plan->f16 ? (float)((const _Float16 *)raw.data())[src + c] : ((const float *)raw.data())[src + c];
      }
  }
}

int kh_read_output(kh_plan *plan, float *out, size_t count) {
  KH_API_BEGIN
  if (!plan || !out) fail(KH_EINVAL, "null argument");
  require_live(plan->ctx);
  if (!plan->ran) fail(KH_EINVAL, "read before run");
  const size_t n = (size_t)plan->out_rows * plan->out_cols;
  if (count < n) fail(KH_EINVAL, "output holds " + std::to_string(n) + " values, the array " + std::to_string(count));
  try {
    read_into(plan, out, n);
    if (plan->split > 0 && plan->twin) {
      // the twin's sequence j is sequence split + j of the batch
      std::vector<float> t(n);
      read_into(plan->twin, t.data(), n);
      const size_t per = plan->out_packed ? (size_t)plan->L * plan->out_cols : (size_t)plan->out_cols;
      const size_t moved = (size_t)(plan->B - plan->split) * per;
      memcpy(out + (size_t)plan->split * per, t.data(), moved * 4);
    }
  } catch (const Error &e) {
    latch(plan->ctx, e);
    throw;
  }
  KH_API_END
}

static void scores_of(const float *logits, int64_t rows, int32_t cols, int kind, float *scores, int32_t *index) {
  if (kind < KH_SCORES_SOFTMAX || kind > KH_SCORES_OPTIONS) fail(KH_EINVAL, "scores kind " + std::to_string(kind));
  if (rows < 0 || cols <= 0) fail(KH_EINVAL, "scores of " + std::to_string(rows) + " x " + std::to_string(cols));
  if (rows && (!logits || !scores)) fail(KH_EINVAL, "null argument");
  const int64_t bad = post::count_nonfinite(logits, rows * cols);
  if (bad)
    fail(KH_EINVAL, "output: " + std::to_string(bad) + " of " + std::to_string(rows * cols) + " values are not finite");
  for (int64_t r = 0; r < rows; r++)
    post::row_scores(logits + r * cols, cols, kind, scores + r * cols, index ? index + r : nullptr);
}

int kh_scores(const float *logits, int64_t rows, int32_t cols, int kind, float *scores, int32_t *index) {
  KH_API_BEGIN
  scores_of(logits, rows, cols, kind, scores, index);
  KH_API_END
}

int kh_read_scores(kh_plan *plan, int kind, float *scores, size_t count, int32_t *index, size_t index_count) {
  KH_API_BEGIN
  if (!plan || !scores) fail(KH_EINVAL, "null argument");
  if (plan->out_packed) fail(KH_EUNSUPPORTED, "scores of token rows: read the output and call kh_scores");
  const size_t n = (size_t)plan->out_rows * plan->out_cols;
  if (count < n) fail(KH_EINVAL, "output holds " + std::to_string(n) + " values, the array " + std::to_string(count));
  if (index && index_count < (size_t)plan->out_rows) fail(KH_EINVAL, "index array shorter than the output rows");
  std::vector<float> raw(n);
  const int rc = kh_read_output(plan, raw.data(), n);
  if (rc) fail(rc, kh_last_error());
  scores_of(raw.data(), plan->out_rows, plan->out_cols, kind, scores, index);
  KH_API_END
}

int kh_rank(const float *scores, int64_t n, int32_t *order) {
  KH_API_BEGIN
  if (n < 0 || (n && (!scores || !order))) fail(KH_EINVAL, "null argument");
  const int64_t bad = post::count_nonfinite(scores, n);
  if (bad) fail(KH_EINVAL, "output: " + std::to_string(bad) + " of " + std::to_string(n) + " values are not finite");
  post::rank(scores, n, order);
  KH_API_END
}

int kh_profile(kh_plan *plan, int32_t rows, kh_launch_stat *out, int32_t cap, int32_t *count) {
  KH_API_BEGIN
  if (!plan || !count) fail(KH_EINVAL, "null argument");
  require_live(plan->ctx);
  if (!plan->uploaded) fail(KH_EINVAL, "profile before upload");
  if (rows < 1 || rows > plan->L * plan->B) fail(KH_EINVAL, "rows outside the plan");
  struct Rec {
    std::string name, kernel;
    double flops, bytes;
    hipEvent_t a, b;
  };
  std::vector<Rec> recs;
  try {
    LaunchHook hook = [&](const Step &s, const char *k, double fl, double by, bool begin) {
      if (begin) {
        Rec r;
        r.name = s.name;
        r.kernel = k;
        r.flops = fl;
        r.bytes = by;
        KH_CHECK(hipEventCreate(&r.a));
        KH_CHECK(hipEventCreate(&r.b));
        recs.push_back(r);
        g_launch_events.start = r.a;  // the step's kernel records them around its own dispatch
        g_launch_events.stop = r.b;
      } else {
        g_launch_events = LaunchEvents();
      }
    };
    launch_forward(plan, rows, hook, true);
    KH_CHECK(hipStreamSynchronize(plan->stream));
  } catch (const Error &e) {
    g_launch_events = LaunchEvents();
    for (auto &r : recs) {
      (void)hipEventDestroy(r.a);
      (void)hipEventDestroy(r.b);
    }
    latch(plan->ctx, e);
    throw;
  }
  g_launch_events = LaunchEvents();
  *count = (int32_t)recs.size();
  for (size_t i = 0; i < recs.size(); i++) {
    float ms = 0;
    (void)hipEventElapsedTime(&ms, recs[i].a, recs[i].b);
    if ((int32_t)i < cap && out) {
      kh_launch_stat &o = out[i];
      memset(&o, 0, sizeof(o));
      snprintf(o.name, sizeof(o.name), "%s", recs[i].name.c_str());
      snprintf(o.kernel, sizeof(o.kernel), "%s", recs[i].kernel.c_str());
      o.ms = ms;
      o.flops = recs[i].flops;
      o.bytes = recs[i].bytes;
    }
    (void)hipEventDestroy(recs[i].a);
    (void)hipEventDestroy(recs[i].b);
  }
  KH_API_END
}

int kh_trace(kh_plan *plan, int32_t on) {
  KH_API_BEGIN
  if (!plan) fail(KH_EINVAL, "null plan");
  require_live(plan->ctx);
  KH_CHECK(hipStreamSynchronize(plan->stream));
  if (plan->twin) KH_CHECK(hipStreamSynchronize(plan->twin->stream));
  release_trace(plan);
  plan->tracing = on != 0;
  KH_API_END
}

int kh_trace_read(kh_plan *plan, kh_launch_stat *out, int32_t cap, int32_t *count) {
  KH_API_BEGIN
  if (!plan || !count) fail(KH_EINVAL, "null argument");
  require_live(plan->ctx);
  KH_CHECK(hipStreamSynchronize(plan->stream));
  if (plan->twin) KH_CHECK(hipStreamSynchronize(plan->twin->stream));
  *count = (int32_t)plan->trace.size();
  for (size_t i = 0; i < plan->trace.size() && (int32_t)i < cap && out; i++) {
    const TraceRec &r = plan->trace[i];
    float ms = 0;
    KH_CHECK(hipEventElapsedTime(&ms, r.a, r.b));
    kh_launch_stat &o = out[i];
    memset(&o, 0, sizeof(o));
    snprintf(o.name, sizeof(o.name), "%s", r.name.c_str());
    snprintf(o.kernel, sizeof(o.kernel), "%s", r.kernel.c_str());
    o.ms = ms;
    o.flops = r.flops;
    o.bytes = r.bytes;
  }
  if (out) release_trace(plan);  // a null array only counts
  KH_API_END
}

int kh_plan_destroy(kh_plan *plan) {
  KH_API_BEGIN
  if (plan) {
    (void)hipSetDevice(plan->ctx->device);
    if (plan->twin) kh_plan_destroy(plan->twin);
    if (plan->ev_twin) (void)hipEventDestroy(plan->ev_twin);
    if (plan->stream) (void)hipStreamSynchronize(plan->stream);
    if (plan->ev0) (void)hipEventDestroy(plan->ev0);
    if (plan->ev1) (void)hipEventDestroy(plan->ev1);
    release_trace(plan);
    for (hipEvent_t e : plan->ev_pool) (void)hipEventDestroy(e);
    hipStream_t s = plan->stream;
    delete plan;
    if (s) (void)hipStreamDestroy(s);
  }
  KH_API_END
}

}  // extern "C"
