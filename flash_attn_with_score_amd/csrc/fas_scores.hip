// Instances and launcher of the scores-only kernel (fas_scores.hpp).
#include "fas_launch.hpp"
#include "fas_scores.hpp"

static_assert(fas::kScoresKeysPerBlock == fas::kScoresKeys, "host and kernel key blocks");

namespace fas {

template <class E, int D>
static hipError_t scores_t(const ScoresParams& p, hipStream_t s) {
  const int64_t grid = (int64_t)p.B * p.H * p.nkb * p.nrs;
  if (grid > INT32_MAX) return hipErrorInvalidValue;
  if (grid > 0) {
    if (p.mask)
      hipLaunchKernelGGL((scores_kernel<E, D, true>), dim3((unsigned)grid), dim3(64 * kScoresWaves),
                         0, s, p);
    else
      hipLaunchKernelGGL((scores_kernel<E, D, false>), dim3((unsigned)grid), dim3(64 * kScoresWaves),
                         0, s, p);
  }
  return hipGetLastError();
}

hipError_t launch_scores(const ScoresParams& p, int dtype, int d, hipStream_t s) {
  if (dtype == 0) {
    switch (d) {
      case 16: return scores_t<F16, 16>(p, s);
      case 32: return scores_t<F16, 32>(p, s);
      case 64: return scores_t<F16, 64>(p, s);
      case 128: return scores_t<F16, 128>(p, s);
    }
  } else {
    switch (d) {
      case 16: return scores_t<BF16, 16>(p, s);
      case 32: return scores_t<BF16, 32>(p, s);
      case 64: return scores_t<BF16, 64>(p, s);
      case 128: return scores_t<BF16, 128>(p, s);
    }
  }
  return hipErrorInvalidValue;
}

}  // namespace fas
