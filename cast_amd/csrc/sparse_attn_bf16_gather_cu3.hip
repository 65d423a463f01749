// The gathered bf16 attention (Q, K and V rows read through slot maps) as
// three 4-wavefront workgroups per compute unit, for grids with at least two
// full rounds of query blocks per XCD.  In a source of its own: the
// memory-clause scheduler is the one that fits it in 168 VGPRs without spills
// (163; the default and ILP schedulers spill 4-24).
#include "sparse_attn_kernel.h"

namespace rcsa {

int launch_bf16_gather_cu3(AttnArgs& a, dim3 grid, hipStream_t s) {
  sparse_attn_kernel<false, 128, 128, 128, 3, 32, 1, true, true, 3><<<grid, dim3(256), 0, s>>>(a);
  return launch_status();
}

}  // namespace rcsa
