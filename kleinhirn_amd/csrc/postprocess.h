// Scores from encoder outputs on the host (see postprocess.cpp). Host code only.
#pragma once

#include <cstdint>

namespace kh {
namespace post {

int64_t count_nonfinite(const float *v, int64_t n);
// one row of `cols` values: scores of `kind` (KH_SCORES_*) into out, the row's label into *index
void row_scores(const float *in, int32_t cols, int kind, float *out, int32_t *index);
// indices of `scores` by score, highest first, equal scores in index order
void rank(const float *scores, int64_t n, int32_t *order);

}  // namespace post
}  // namespace kh
