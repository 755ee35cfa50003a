// Instantiations of the several-LoRA fused kernel for bf16 and f16 bases
// (no scale) with bf16 factors.
#include "kernels_multi_dev.h"

namespace ltxw {

hipError_t launch_fused_multi_base16(const JobTable& t, bool f32out, int ks, hipStream_t stream) {
  return launch_multi_fdt<0, true>(t, f32out, ks, stream);
}

}  // namespace ltxw
