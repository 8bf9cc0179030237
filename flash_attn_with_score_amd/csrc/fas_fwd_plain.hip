// Forward-pass instances: plain output (+ base-2 LSE) and per-row sums.
#include "fas_fwd.hpp"

namespace fas {

hipError_t launch_fwd_plain(const FwdParams& p, int dtype, int d, hipStream_t s) {
  return launch_fwd_mode<kFwdPlain, 8>(p, dtype, d, s);
}

hipError_t launch_fwd_rowsum(const FwdParams& p, int dtype, int d, hipStream_t s) {
  return launch_fwd_mode<kFwdRowSum, 8>(p, dtype, d, s);
}

}  // namespace fas
