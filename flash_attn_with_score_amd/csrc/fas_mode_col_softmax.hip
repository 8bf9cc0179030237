// Instantiates the kModeColSoftmax kernels (fp16/bf16 x D in {16,32,64,128}).
#include "fas_kernel.hpp"

namespace fas {

hipError_t launch_col_softmax(const KParams& p, int dtype, int d, hipStream_t s) {
  return launch_mode<kModeColSoftmax>(p, dtype, d, s);
}

}  // namespace fas
