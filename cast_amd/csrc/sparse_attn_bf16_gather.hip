// The gathered bf16 attention kernel, instantiated and launched in a source of
// its own so that it keeps the default instruction scheduler (the other
// attention kernels are built for instruction-level parallelism).
#include "sparse_attn_kernel.h"

namespace rcsa {

int launch_bf16_gather(AttnArgs& a, dim3 grid, hipStream_t s) {
  sparse_attn_kernel<false, 128, 128, 128, 3, 64, 2, true, true><<<grid, dim3(512), 0, s>>>(a);
  return launch_status();
}

}  // namespace rcsa
