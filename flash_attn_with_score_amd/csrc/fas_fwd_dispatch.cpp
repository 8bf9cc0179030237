// Dispatch of the forward pass to its per-mode translation units.
#include "fas_launch.hpp"

namespace fas {

hipError_t launch_fwd_plain(const FwdParams& p, int dtype, int d, int waves, hipStream_t s);
hipError_t launch_fwd_rowsum(const FwdParams& p, int dtype, int d, int waves, hipStream_t s);
hipError_t launch_fwd_scores(const FwdParams& p, int dtype, int d, int waves, hipStream_t s);
hipError_t launch_fwd_region(const FwdParams& p, int dtype, int d, int waves, hipStream_t s);

int fwd_rows_per_block(int d, int waves) { return (d == 128 && waves == 4) ? 128 : 256; }

hipError_t launch_fwd(const FwdParams& p, int mode, int dtype, int d, int waves, hipStream_t s) {
  switch (mode) {
    case kFwdPlain: return launch_fwd_plain(p, dtype, d, waves, s);
    case kFwdRowSum: return launch_fwd_rowsum(p, dtype, d, waves, s);
    case kFwdScores: return launch_fwd_scores(p, dtype, d, waves, s);
    case kFwdRegion: return launch_fwd_region(p, dtype, d, waves, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace fas
