// W4 prefill kernels with f32 group scales (the kernel is in prefill_kernel.h).
#include "prefill_kernel.h"

namespace qlin {

hipError_t launch_prefill_w4_f32(const TlArgs& a, bool hz, int shape, hipStream_t st) {
  if (hz) return launch_prefill_kind<WK_W4, true, DT_F32>(a, shape, st);
  return launch_prefill_kind<WK_W4, false, DT_F32>(a, shape, st);
}

}  // namespace qlin
