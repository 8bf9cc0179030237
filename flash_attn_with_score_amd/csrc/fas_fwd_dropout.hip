// Forward-pass instances with dropout of the attention weights (plain, plain
// storing the keep bits, score-writer and row-sum modes; the buffered
// cross-token pass ignores dropout, as the reference does).
#include "fas_fwd.hpp"

namespace fas {

hipError_t launch_fwd_dropout(const FwdParams& p, int mode, int dtype, int d, hipStream_t s) {
  switch (mode) {
    case kFwdPlain: return launch_fwd_mode<kFwdPlain, 8, true>(p, dtype, d, s);
    case kFwdPlainKeepBits: return launch_fwd_mode<kFwdPlainKeepBits, 8, true>(p, dtype, d, s);
    case kFwdRowSum: return launch_fwd_mode<kFwdRowSum, 8, true>(p, dtype, d, s);
    case kFwdScores: return launch_fwd_mode<kFwdScores, 8, true>(p, dtype, d, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace fas
