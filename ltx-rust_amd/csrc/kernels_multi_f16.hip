// Instantiations of the several-LoRA fused kernel for f16 factors.
#include "kernels_multi_dev.h"

namespace ltxw {

hipError_t launch_fused_multi_f16(const JobTable& t, bool f32out, int ks, hipStream_t stream) {
  return launch_multi_fdt<2>(t, f32out, ks, stream);
}

}  // namespace ltxw
