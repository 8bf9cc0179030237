// Host-side launchers of the gfx950 kernels, one per side-product mode.
// Each is defined in its own translation unit (fas_mode_*.hip) so the
// template instantiations compile in parallel.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fas_params.hpp"

namespace fas {

// One launcher per mode, each instantiated in its own translation unit.
hipError_t launch_scores(const KParams& p, int dtype, int d, hipStream_t s);
hipError_t launch_row_sum(const KParams& p, int dtype, int d, hipStream_t s);
hipError_t launch_col_sum(const KParams& p, int dtype, int d, hipStream_t s);
hipError_t launch_cross_qk(const KParams& p, int dtype, int d, hipStream_t s);
hipError_t launch_col_softmax(const KParams& p, int dtype, int d, hipStream_t s);
hipError_t launch_cross_softmax(const KParams& p, int dtype, int d, hipStream_t s);
hipError_t launch_cross_softmax_buf(const KParams& p, int dtype, int d, hipStream_t s);
hipError_t launch_fill_zero(float* p, int64_t s0, int64_t s1, int64_t s2, int64_t n0, int64_t n1,
                            int64_t n2, hipStream_t s);

}  // namespace fas
