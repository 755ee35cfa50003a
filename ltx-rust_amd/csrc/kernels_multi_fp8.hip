// Instantiations of the several-LoRA fused kernel for e4m3fn and e5m2 factors.
#include "kernels_multi_dev.h"

namespace ltxw {

hipError_t launch_fused_multi_e4m3fn(const JobTable& t, bool f32out, int ks, hipStream_t stream) {
  return launch_multi_fdt<3>(t, f32out, ks, stream);
}

hipError_t launch_fused_multi_e5m2(const JobTable& t, bool f32out, int ks, hipStream_t stream) {
  return launch_multi_fdt<4>(t, f32out, ks, stream);
}

}  // namespace ltxw
