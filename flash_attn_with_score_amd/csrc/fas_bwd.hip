// Instances and launcher of the backward kernels (fas_bwd.hpp).
#include "fas_bwd.hpp"
#include "fas_launch.hpp"

namespace fas {

// Instances: DROP 0 without dropout; with dropout, the dK/dV kernel reads
// the forward's keep words when given (2) or evaluates Philox (1).  dQ comes
// from the stored dS blocks when p.ds is set (bwd_dq_ds_kernel, no dropout
// instances: dS carries the mask); otherwise bwd_dq_kernel recomputes S and
// dP, reading keep bits when drop_bits holds them (2) or evaluating Philox (1).
template <class E, int D>
static hipError_t bwd_t(const BwdParams& p, hipStream_t s) {
  const int64_t bh = (int64_t)p.B * p.H;
  if (p.M > 0)
    hipLaunchKernelGGL((bwd_prep_kernel<E, D>), dim3((unsigned)(bh * p.nprep)), dim3(256), 0, s,
                       p);
  if (p.N > 0) {
    const int64_t rest = p.partial ? bh : (int64_t)p.B * p.Hk;
    const dim3 grid((unsigned)(rest * p.nkb));
    if (!p.dropout)
      hipLaunchKernelGGL((bwd_dkdv_kernel<E, D, 0>), grid, dim3(256), 0, s, p);
    else if (p.keep_keys)
      hipLaunchKernelGGL((bwd_dkdv_kernel<E, D, 2>), grid, dim3(256), 0, s, p);
    else
      hipLaunchKernelGGL((bwd_dkdv_kernel<E, D, 1>), grid, dim3(256), 0, s, p);
    if (p.partial) {
      const int64_t total = (int64_t)p.B * p.Hk * p.N * (D / 8);
      int64_t blocks = (total + 255) / 256;
      if (blocks > 16384) blocks = 16384;
      hipLaunchKernelGGL((bwd_dkdv_reduce_kernel<E, D>), dim3((unsigned)blocks), dim3(256), 0, s,
                         p);
    }
  }
  if (p.M > 0) {
    const dim3 grid((unsigned)(bh * p.nrb));
    if (p.ds) {
      const int bm = 32 * kBwdDqDsWaves;
      hipLaunchKernelGGL((bwd_dq_ds_kernel<E, D>), dim3((unsigned)(bh * ((p.Mpad + bm - 1) / bm))),
                         dim3(64 * kBwdDqDsWaves), 0, s, p);
    } else if (!p.dropout)
      hipLaunchKernelGGL((bwd_dq_kernel<E, D, 0>), grid, dim3(256), 0, s, p);
    else if (p.drop_bits)
      hipLaunchKernelGGL((bwd_dq_kernel<E, D, 2>), grid, dim3(256), 0, s, p);
    else
      hipLaunchKernelGGL((bwd_dq_kernel<E, D, 1>), grid, dim3(256), 0, s, p);
  }
  return hipGetLastError();
}

hipError_t launch_bwd(const BwdParams& p, int dtype, int d, hipStream_t s) {
  if (dtype == 0) {
    switch (d) {
      case 16: return bwd_t<F16, 16>(p, s);
      case 32: return bwd_t<F16, 32>(p, s);
      case 64: return bwd_t<F16, 64>(p, s);
      case 128: return bwd_t<F16, 128>(p, s);
    }
  } else {
    switch (d) {
      case 16: return bwd_t<BF16, 16>(p, s);
      case 32: return bwd_t<BF16, 32>(p, s);
      case 64: return bwd_t<BF16, 64>(p, s);
      case 128: return bwd_t<BF16, 128>(p, s);
    }
  }
  return hipErrorInvalidValue;
}

}  // namespace fas
