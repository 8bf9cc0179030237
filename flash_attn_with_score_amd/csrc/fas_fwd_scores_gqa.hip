// Score-writer instances with GQA packing (several query heads per
// workgroup).
#include "fas_fwd.hpp"

namespace fas {

hipError_t launch_fwd_scores_packed(const FwdParams& p, int dtype, int d, hipStream_t s) {
  return launch_fwd_mode<kFwdScores, 8, false, true>(p, dtype, d, s);
}

}  // namespace fas
