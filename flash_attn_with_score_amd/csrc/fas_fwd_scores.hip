// Forward-pass instances writing the score matrix.
#include "fas_fwd.hpp"

namespace fas {

hipError_t launch_fwd_scores(const FwdParams& p, int dtype, int d, int waves, hipStream_t s) {
  if (d == 128 && waves == 4) return launch_fwd_mode<kFwdScores, 4>(p, dtype, d, s);
  return launch_fwd_mode<kFwdScores, 8>(p, dtype, d, s);
}

}  // namespace fas
