// Forward-pass instances with GQA packing (several query heads per
// workgroup): plain output (+ base-2 LSE), per-row sums and the buffered
// cross-token region pass.
#include "fas_fwd.hpp"

namespace fas {

hipError_t launch_fwd_packed(const FwdParams& p, int mode, int dtype, int d, hipStream_t s) {
  switch (mode) {
    case kFwdPlain: return launch_fwd_mode<kFwdPlain, 8, false, true>(p, dtype, d, s);
    case kFwdRowSum: return launch_fwd_mode<kFwdRowSum, 8, false, true>(p, dtype, d, s);
    case kFwdRegion: return launch_fwd_mode<kFwdRegion, 8, false, true>(p, dtype, d, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace fas
