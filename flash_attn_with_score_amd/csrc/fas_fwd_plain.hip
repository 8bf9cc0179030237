// Forward-pass instances: plain output (+ base-2 LSE) and per-row sums.
#include "fas_fwd.hpp"

namespace fas {

hipError_t launch_fwd_plain(const FwdParams& p, int dtype, int d, int waves, hipStream_t s) {
  if (d == 128 && waves == 4) return launch_fwd_mode<kFwdPlain, 4>(p, dtype, d, s);
  return launch_fwd_mode<kFwdPlain, 8>(p, dtype, d, s);
}

hipError_t launch_fwd_rowsum(const FwdParams& p, int dtype, int d, int waves, hipStream_t s) {
  if (d == 128 && waves == 4) return launch_fwd_mode<kFwdRowSum, 4>(p, dtype, d, s);
  return launch_fwd_mode<kFwdRowSum, 8>(p, dtype, d, s);
}

}  // namespace fas
