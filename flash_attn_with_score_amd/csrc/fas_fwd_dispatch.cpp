// Dispatch of the forward pass to its per-mode translation units.
#include "fas_launch.hpp"

namespace fas {

hipError_t launch_fwd_plain(const FwdParams& p, int dtype, int d, hipStream_t s);
hipError_t launch_fwd_rowsum(const FwdParams& p, int dtype, int d, hipStream_t s);
hipError_t launch_fwd_scores(const FwdParams& p, int dtype, int d, hipStream_t s);
hipError_t launch_fwd_region(const FwdParams& p, int dtype, int d, hipStream_t s);
hipError_t launch_fwd_dropout(const FwdParams& p, int mode, int dtype, int d, hipStream_t s);
hipError_t launch_fwd_packed(const FwdParams& p, int mode, int dtype, int d, hipStream_t s);
hipError_t launch_fwd_scores_packed(const FwdParams& p, int dtype, int d, hipStream_t s);

// GQA-packed launches (p.pack > 1) take their own instances; the host never
// packs a launch with dropout.
hipError_t launch_fwd(const FwdParams& p, int mode, int dtype, int d, hipStream_t s) {
  // Only the unpacked score writer without dropout has 128-row and (key
  // split, 16-byte score rows) 64-row instances; every other launch is built
  // for 256-row blocks.
  const bool small_writer = mode == kFwdScores && p.pack == 1 && !p.dropout &&
                            ((p.bm == kFwdRows / 2 && (!p.key_split2 || p.vec_scores)) ||
                             (p.bm == kFwdRows / 4 && p.vec_scores));
  if (p.key_split2 && !(small_writer && p.bm == kFwdRows / 2)) return hipErrorInvalidValue;
  if (p.bm != kFwdRows && !small_writer) return hipErrorInvalidValue;
  if (p.pack > 1) {
    if (p.dropout && mode != kFwdRegion) return hipErrorInvalidValue;
    return mode == kFwdScores ? launch_fwd_scores_packed(p, dtype, d, s)
                              : launch_fwd_packed(p, mode, dtype, d, s);
  }
  if (p.dropout && mode != kFwdRegion) return launch_fwd_dropout(p, mode, dtype, d, s);
  switch (mode) {
    case kFwdPlain: return launch_fwd_plain(p, dtype, d, s);
    case kFwdRowSum: return launch_fwd_rowsum(p, dtype, d, s);
    case kFwdScores: return launch_fwd_scores(p, dtype, d, s);
    case kFwdRegion: return launch_fwd_region(p, dtype, d, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace fas
