// Batch scheduler over packed plans (kh_sched_* of include/kh_hip.h). Host code only: it drives
// plans through the public entry points (kh_upload_ids, kh_run, kh_read_output).
//
// The reference cuts a call into chunks of at most 16 rows, each padded to a plan of 1, 4, 8 or 16
// sequences at a row stride of the chunk's longest sequence rounded to 64, after sorting the inputs
// by length (src/encoder.ts:380-436, src/cache.ts:9-18, 81-108). Packed plans compute only the valid
// rows, so the plan length L bounds a sequence and the buffers, not the work: one chunk takes as
// many sequences as the plan holds (B) or as a token budget allows. Inputs are still taken in
// length order, so short sequences land on the plans with the smallest L that holds them. Plans of
// one shape are used in turn: while one runs on its stream, the next chunk is packed and submitted
// to another and the finished one is read back.
#include <algorithm>
#include <chrono>
#include <cstring>
#include <deque>
#include <numeric>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/kh_hip.h"

namespace kh {
void set_last_error(const std::string &m);  // the message kh_last_error() returns (runner.hip)
}

namespace {

struct Slot {
  kh_plan *plan;
  int L, B, cols;
  bool busy = false;
  std::vector<int64_t> seqs;  // input index of sequence b of the chunk
  std::vector<int32_t> ids;
  std::vector<float> mask;
  std::vector<uint32_t> tt;
  std::vector<float> out;
};

struct Fail : std::runtime_error {
  int code;
  Fail(int c, const std::string &m) : std::runtime_error(m), code(c) {}
};

}  // namespace

struct kh_sched {
  std::vector<Slot> slots;
  int cols = 0;
};

static void check(int rc) {
  if (rc != KH_OK) throw Fail(rc, kh_last_error());
}

int kh_sched_create(kh_plan *const *plans, int32_t n, kh_sched **out) {
  try {
    if (!plans || n <= 0 || !out) throw Fail(KH_EINVAL, "kh_sched_create needs one plan or more");
    auto *s = new kh_sched();
    for (int32_t i = 0; i < n; i++) {
      kh_plan_info info;
      int rc = kh_plan_info_get(plans[i], &info);
      if (rc) {
        delete s;
        throw Fail(rc, kh_last_error());
      }
      if (info.out_rows != info.batch || info.markers > 0) {
        delete s;
        throw Fail(KH_EUNSUPPORTED, "the scheduler runs pooled heads (one output row per sequence, no markers)");
      }
      if (i > 0 && info.out_cols != s->cols) {
        delete s;
        throw Fail(KH_EINVAL, "scheduler plans differ in output columns");
      }
      s->cols = info.out_cols;
      Slot sl;
      sl.plan = plans[i];
      sl.L = info.length;
      sl.B = info.batch;
      sl.cols = info.out_cols;
      sl.ids.assign((size_t)sl.L * sl.B, 0);
      sl.mask.assign((size_t)sl.L * sl.B, 0.f);
      sl.tt.assign((size_t)sl.L * sl.B, 0u);
      sl.out.assign((size_t)sl.B * sl.cols, 0.f);
      s->slots.push_back(std::move(sl));
    }
    *out = s;
    return KH_OK;
  } catch (const Fail &e) {
    kh::set_last_error(e.what());
    return e.code;
  } catch (const std::bad_alloc &) {
    kh::set_last_error("host allocation failed");
    return KH_ENOMEM;
  }
}

int kh_sched_destroy(kh_sched *s) {
  delete s;
  kh::set_last_error("");
  return KH_OK;
}

int kh_sched_run(kh_sched *s, const int32_t *ids, const int64_t *offsets, int64_t nseq, const uint32_t *type_words,
                 int64_t token_budget, float *out, size_t out_count, kh_sched_stats *stats) {
  const auto t0 = std::chrono::steady_clock::now();
  std::deque<int> inflight;
  kh_sched_stats st;
  memset(&st, 0, sizeof st);
  try {
    if (!s || !offsets || (nseq > 0 && (!ids || !out))) throw Fail(KH_EINVAL, "null argument");
    if (nseq < 0) throw Fail(KH_EINVAL, "negative sequence count");
    if (out_count < (size_t)nseq * s->cols)
      throw Fail(KH_EINVAL, "output holds " + std::to_string(out_count) + " values, " + std::to_string(nseq) +
                                " sequences need " + std::to_string((size_t)nseq * s->cols));
    int maxL = 0;
    for (const Slot &sl : s->slots) maxL = std::max(maxL, sl.L);
    std::vector<int64_t> len(nseq);
    for (int64_t i = 0; i < nseq; i++) {
      len[i] = offsets[i + 1] - offsets[i];
      if (len[i] < 0) throw Fail(KH_EINVAL, "offsets must not decrease");
      if (len[i] > maxL)
        throw Fail(KH_EINVAL, "sequence " + std::to_string(i) + " of " + std::to_string(len[i]) +
                                  " tokens exceeds the longest plan (" + std::to_string(maxL) + ")");
    }
    // length order (sortByKey, src/cache.ts:92-108): a stable sort, shortest first
    std::vector<int64_t> order(nseq);
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(), [&](int64_t a, int64_t b) { return len[a] < len[b]; });

    auto complete = [&](int k) {
      Slot &sl = s->slots[k];
      check(kh_read_output(sl.plan, sl.out.data(), sl.out.size()));
      float ms = 0;
      if (kh_last_run_ms(sl.plan, &ms) == KH_OK) st.gpu_ms += ms;
      for (size_t b = 0; b < sl.seqs.size(); b++)
        memcpy(out + (size_t)sl.seqs[b] * s->cols, sl.out.data() + b * s->cols, (size_t)s->cols * 4);
      sl.busy = false;
    };
    int64_t pos = 0;
    while (pos < nseq) {
      // the smallest plan length holding the chunk's first (shortest) sequence
      int L = 0;
      for (const Slot &sl : s->slots)
        if (sl.L >= len[order[pos]] && (L == 0 || sl.L < L)) L = sl.L;
      // a free plan of that length (the largest batch), else the oldest running one
      int k = -1;
      for (int i = 0; i < (int)s->slots.size(); i++)
        if (s->slots[i].L == L && !s->slots[i].busy && (k < 0 || s->slots[i].B > s->slots[k].B)) k = i;
      if (k < 0) {
        for (auto it = inflight.begin(); it != inflight.end(); ++it)
          if (s->slots[*it].L == L) {
            k = *it;
            inflight.erase(it);
            break;
          }
        if (k < 0) throw Fail(KH_EINVAL, "internal: no plan of length " + std::to_string(L));
        complete(k);
      }
      Slot &sl = s->slots[k];
      const auto th = std::chrono::steady_clock::now();
      sl.seqs.clear();
      std::fill(sl.mask.begin(), sl.mask.end(), 0.f);
      int64_t tokens = 0;
      while (pos < nseq && (int)sl.seqs.size() < sl.B && len[order[pos]] <= sl.L &&
             (token_budget <= 0 || sl.seqs.empty() || tokens + len[order[pos]] <= token_budget)) {
        const int64_t q = order[pos++];
        const size_t b = sl.seqs.size(), row = b * (size_t)sl.L;
        memcpy(sl.ids.data() + row, ids + offsets[q], (size_t)len[q] * 4);
        std::fill(sl.ids.begin() + row + len[q], sl.ids.begin() + row + sl.L, 0);
        std::fill(sl.mask.begin() + row, sl.mask.begin() + row + len[q], 1.f);
        if (type_words) {
          memcpy(sl.tt.data() + row, type_words + offsets[q], (size_t)len[q] * 4);
          std::fill(sl.tt.begin() + row + len[q], sl.tt.begin() + row + sl.L, 0u);
        }
        sl.seqs.push_back(q);
        tokens += len[q];
      }
      // rows of the unused sequences: zero ids, mask 0 (no valid row)
      std::fill(sl.ids.begin() + sl.seqs.size() * (size_t)sl.L, sl.ids.end(), 0);
      check(kh_upload_ids(sl.plan, sl.ids.data(), sl.ids.size(), sl.mask.data(), sl.mask.size(),
                          type_words ? sl.tt.data() : nullptr, type_words ? sl.tt.size() : 0));
      check(kh_run(sl.plan, sl.L * sl.B));
      st.host_ms += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - th).count();
      sl.busy = true;
      inflight.push_back(k);
      st.chunks++;
      st.tokens += tokens;
    }
    while (!inflight.empty()) {
      const int k = inflight.front();
      inflight.pop_front();
      complete(k);
    }
    st.sequences = (int32_t)nseq;
    st.wall_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    if (stats) *stats = st;
    kh::set_last_error("");
    return KH_OK;
  } catch (const Fail &e) {
    // leave no plan mid-flight: wait for what was submitted
    if (s) {
      for (int k : inflight) (void)kh_sync(s->slots[k].plan);
      for (Slot &sl : s->slots) sl.busy = false;
    }
    kh::set_last_error(e.what());
    return e.code;
  } catch (const std::bad_alloc &) {
    kh::set_last_error("host allocation failed");
    return KH_ENOMEM;
  }
}
