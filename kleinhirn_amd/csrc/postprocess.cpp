// Scores from encoder outputs on the host (the numeric part of src/tasks.ts and the classify /
// embed / rerank steps of src/encoder.ts:498-555), in the reference's arithmetic: values are f32,
// every operation runs in double (JavaScript numbers) and results round once to f32 where the
// reference stores them in a Float32Array.
#include "postprocess.h"

#include <algorithm>
#include <cmath>
#include <numeric>

#include "../../include/kh_hip.h"

namespace kh {
namespace post {

int64_t count_nonfinite(const float *v, int64_t n) {
  int64_t bad = 0;
  for (int64_t i = 0; i < n; i++) bad += std::isfinite(v[i]) ? 0 : 1;
  return bad;
}

// argmaxRows (src/tasks.ts:72-84): ties go to the lower index
static int32_t argmax(const float *r, int32_t cols) {
  int32_t best = 0;
  for (int32_t c = 1; c < cols; c++)
    if (r[c] > r[best]) best = c;
  return best;
}

void row_scores(const float *in, int32_t cols, int kind, float *out, int32_t *index) {
  switch (kind) {
    case KH_SCORES_SOFTMAX: {  // softmax (src/tasks.ts:22-33)
      double mx = -INFINITY;
      for (int32_t i = 0; i < cols; i++) mx = std::max(mx, (double)in[i]);
      double sum = 0;
      for (int32_t i = 0; i < cols; i++) {
        out[i] = (float)std::exp((double)in[i] - mx);
        sum += out[i];
      }
      for (int32_t i = 0; i < cols; i++) out[i] = (float)((double)out[i] / sum);
      if (index) *index = argmax(out, cols);
      break;
    }
    case KH_SCORES_OPTIONS: {  // softmaxPrefix (src/julia.ts:57-65): no f32 store before the sum
      double mx = -INFINITY;
      for (int32_t i = 0; i < cols; i++) mx = std::max(mx, (double)in[i]);
      double sum = 0;
      for (int32_t i = 0; i < cols; i++) sum += std::exp((double)in[i] - mx);
      for (int32_t i = 0; i < cols; i++) out[i] = (float)(std::exp((double)in[i] - mx) / sum);
      if (index) *index = argmax(out, cols);
      break;
    }
    case KH_SCORES_SIGMOID:  // multi-label: 1 / (1 + e^-v), the label of the largest logit
      for (int32_t i = 0; i < cols; i++) out[i] = (float)(1.0 / (1.0 + std::exp(-(double)in[i])));
      if (index) *index = argmax(in, cols);
      break;
    case KH_SCORES_L2: {  // l2normalize (src/tasks.ts:35-42)
      double sq = 0;
      for (int32_t i = 0; i < cols; i++) sq += (double)in[i] * (double)in[i];
      const double norm = std::max(std::sqrt(sq), 1e-12);
      for (int32_t i = 0; i < cols; i++) out[i] = (float)((double)in[i] / norm);
      if (index) *index = argmax(in, cols);
      break;
    }
    default:  // regression: the logits themselves
      for (int32_t i = 0; i < cols; i++) out[i] = in[i];
      if (index) *index = argmax(in, cols);
      break;
  }
}

void rank(const float *scores, int64_t n, int32_t *order) {
  // rerank (src/encoder.ts:533-544): by score, highest first; equal scores keep index order
  std::iota(order, order + n, 0);
  std::stable_sort(order, order + n, [&](int32_t a, int32_t b) { return scores[a] > scores[b]; });
}

}  // namespace post
}  // namespace kh
