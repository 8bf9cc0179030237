// Forward-pass instances storing the cross-token region's raw scores.
#include "fas_fwd.hpp"

namespace fas {

hipError_t launch_fwd_region(const FwdParams& p, int dtype, int d, hipStream_t s) {
  return launch_fwd_mode<kFwdRegion, 8>(p, dtype, d, s);
}

}  // namespace fas
