// Instances and launcher of the scores-only kernel (fas_scores.hpp).
#include "fas_launch.hpp"
#include "fas_scores.hpp"

static_assert(fas::kScoresKeysPerBlock == fas::kScoresKeys, "host and kernel key blocks");
static_assert(fas::kScoresResidentRows == fas::kScoresResRows, "host and kernel resident rows");
static_assert(fas::kScoresResidentKeys == 64 * fas::kScoresWaves, "host and kernel resident blocks");
static_assert(fas::kScoresResidentBytes == fas::kScoresGroupBytes, "host and kernel group extents");

namespace fas {

template <class E, int D, bool MASK>
static void qres_launch(int rows, dim3 g, dim3 b, const ScoresParams& p, hipStream_t s) {
  if (rows == 32)
    hipLaunchKernelGGL((scores_qres_kernel<E, D, MASK, 32>), g, b, 0, s, p);
  else if (rows == 64)
    hipLaunchKernelGGL((scores_qres_kernel<E, D, MASK, 64>), g, b, 0, s, p);
  else if (rows == 128)
    hipLaunchKernelGGL((scores_qres_kernel<E, D, MASK, 128>), g, b, 0, s, p);
  else if (rows == 256)
    hipLaunchKernelGGL((scores_qres_kernel<E, D, MASK, 256>), g, b, 0, s, p);
  else
    hipLaunchKernelGGL((scores_qres_kernel<E, D, MASK, 512>), g, b, 0, s, p);
}

template <class E, int D>
static hipError_t scores_t(const ScoresParams& p, hipStream_t s) {
  if (p.ngrp > 0) {
    if (p.ngrp > p.nkb || !p.vec) return hipErrorInvalidValue;
    if (p.pshift < 0 || p.pshift > 3 || p.H % (1 << p.pshift) != 0 ||
        p.G % (1 << p.pshift) != 0 || (p.M << p.pshift) > kScoresResRows)
      return hipErrorInvalidValue;
    const int64_t grid = ((int64_t)p.B * p.H >> p.pshift) * p.ngrp;
    if (grid > INT32_MAX) return hipErrorInvalidValue;
    const dim3 g((unsigned)grid), b(64 * kScoresWaves);
    // Resident rows: the fewest of 32, 64, 128, 256 and 512 that cover the
    // group's 2^pshift * M rows (nkb counts 512-key blocks).
    const int vr = p.M << p.pshift;
    const int rows = vr <= 32 ? 32 : vr <= 64 ? 64 : vr <= 128 ? 128 : vr <= 256 ? 256 : 512;
    if (p.mask)
      qres_launch<E, D, true>(rows, g, b, p, s);
    else
      qres_launch<E, D, false>(rows, g, b, p, s);
    return hipGetLastError();
  }
  const int64_t grid = (int64_t)p.B * p.H * p.nkb * p.nrs;
  if (grid > INT32_MAX) return hipErrorInvalidValue;
  if (grid > 0) {
    const dim3 g((unsigned)grid), b(64 * kScoresWaves);
    if (p.mask && p.vec)
      hipLaunchKernelGGL((scores_kernel<E, D, true, true>), g, b, 0, s, p);
    else if (p.mask)
      hipLaunchKernelGGL((scores_kernel<E, D, true, false>), g, b, 0, s, p);
    else if (p.vec)
      hipLaunchKernelGGL((scores_kernel<E, D, false, true>), g, b, 0, s, p);
    else
      hipLaunchKernelGGL((scores_kernel<E, D, false, false>), g, b, 0, s, p);
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
