// Forward-pass instances writing the score matrix.
#include "fas_fwd.hpp"

namespace fas {

hipError_t launch_fwd_scores(const FwdParams& p, int dtype, int d, hipStream_t s) {
  if (p.bm == 64) return launch_fwd_mode<kFwdScores, 4, false, false, true>(p, dtype, d, s);
  if (p.bm == 128 && p.key_split2)
    return launch_fwd_mode<kFwdScores, 8, false, false, true>(p, dtype, d, s);
  if (p.bm == 128) return launch_fwd_mode<kFwdScores, 4>(p, dtype, d, s);
  if (p.bm != 256) return hipErrorInvalidValue;
  return launch_fwd_mode<kFwdScores, 8>(p, dtype, d, s);
}

}  // namespace fas
