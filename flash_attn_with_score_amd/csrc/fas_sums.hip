// Instances and launchers of the column-sum kernels (fas_sums.hpp).
#include "fas_launch.hpp"
#include "fas_sums.hpp"

namespace fas {

template <class E, int D>
static hipError_t colsm_t(const ColsmParams& p, hipStream_t s) {
  // One workgroup per mirror pair of key blocks, head split and output group.
  const dim3 grid((unsigned)((int64_t)((p.nkb + 1) / 2) * p.nsplit * p.B * (p.H / p.fold)));
  if (p.lse_ln != nullptr)
    hipLaunchKernelGGL((colsm64_kernel<E, D, true, 0>), grid, dim3(512), 0, s, p);
  else if (p.dropout == 2)
    hipLaunchKernelGGL((colsm64_kernel<E, D, false, 2>), grid, dim3(512), 0, s, p);
  else if (p.dropout)
    hipLaunchKernelGGL((colsm64_kernel<E, D, false, 1>), grid, dim3(512), 0, s, p);
  else
    hipLaunchKernelGGL((colsm64_kernel<E, D, false, 0>), grid, dim3(512), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_colsm(const ColsmParams& p, int dtype, int d, bool buffered, hipStream_t s) {
  if (buffered) {
    // 256 keys per workgroup with 16-byte rows, else 64.
    const bool vec = p.split % 4 == 0;
    const int64_t nkb = (p.ncols + (vec ? 255 : 63)) / (vec ? 256 : 64);
    ColsmParams q = p;
    q.nkb = (int)nkb;
    const dim3 grid((unsigned)(nkb * p.nsplit * p.B * (p.H / p.fold)));
    if (vec)
      hipLaunchKernelGGL(colsm_buffered_kernel<true>, grid, dim3(256), 0, s, q);
    else
      hipLaunchKernelGGL(colsm_buffered_kernel<false>, grid, dim3(256), 0, s, q);
    return hipGetLastError();
  }
  if (dtype == 0) {
    switch (d) {
      case 16: return colsm_t<F16, 16>(p, s);
      case 32: return colsm_t<F16, 32>(p, s);
      case 64: return colsm_t<F16, 64>(p, s);
      case 128: return colsm_t<F16, 128>(p, s);
    }
  } else {
    switch (d) {
      case 16: return colsm_t<BF16, 16>(p, s);
      case 32: return colsm_t<BF16, 32>(p, s);
      case 64: return colsm_t<BF16, 64>(p, s);
      case 128: return colsm_t<BF16, 128>(p, s);
    }
  }
  return hipErrorInvalidValue;
}

template <class E, int D>
static hipError_t rawsum_t(const RawParams& p, bool suffix, hipStream_t s) {
  const unsigned bhk = (unsigned)(p.B * p.Hk);
  if (p.nblk > 0)
    hipLaunchKernelGGL((qsum_blocks_kernel<E, D>), dim3((unsigned)p.nblk, bhk), dim3(256), 0, s, p);
  if (suffix) {
    const unsigned nw = (unsigned)((p.M + 63) / 64 + p.nextra);
    if (nw > 0) hipLaunchKernelGGL((colraw_kernel<E, D, true>), dim3(nw, bhk), dim3(256), 0, s, p);
  } else {
    // Up to 8 groups of 64 keys per workgroup while at least 512
    // workgroups (two per CU) remain.
    const int64_t groups = (p.ncols + 63) / 64;
    RawParams q = p;
    q.kgroups = (int)std::max<int64_t>(1, std::min<int64_t>(8, groups * bhk / 512));
    const unsigned nw = (unsigned)((groups + q.kgroups - 1) / q.kgroups);
    if (nw > 0) hipLaunchKernelGGL((colraw_kernel<E, D, false>), dim3(nw, bhk), dim3(256), 0, s, q);
  }
  return hipGetLastError();
}

hipError_t launch_rawsum(const RawParams& p, int dtype, bool suffix, hipStream_t s) {
  if (dtype == 0) {
    switch (p.D) {
      case 16: return rawsum_t<F16, 16>(p, suffix, s);
      case 32: return rawsum_t<F16, 32>(p, suffix, s);
      case 64: return rawsum_t<F16, 64>(p, suffix, s);
      case 128: return rawsum_t<F16, 128>(p, suffix, s);
    }
  } else {
    switch (p.D) {
      case 16: return rawsum_t<BF16, 16>(p, suffix, s);
      case 32: return rawsum_t<BF16, 32>(p, suffix, s);
      case 64: return rawsum_t<BF16, 64>(p, suffix, s);
      case 128: return rawsum_t<BF16, 128>(p, suffix, s);
    }
  }
  return hipErrorInvalidValue;
}

}  // namespace fas
