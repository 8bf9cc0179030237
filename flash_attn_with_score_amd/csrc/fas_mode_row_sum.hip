// Instantiates the kModeRowSum kernels (fp16/bf16 x D in {16,32,64,128}).
#include "fas_kernel.hpp"

namespace fas {

hipError_t launch_row_sum(const KParams& p, int dtype, int d, hipStream_t s) {
  return launch_mode<kModeRowSum>(p, dtype, d, s);
}

}  // namespace fas
