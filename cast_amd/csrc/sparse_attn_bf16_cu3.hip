// bf16 attention kernels of three 4-wavefront workgroups per compute unit that
// need the memory-clause scheduler to fit 168 VGPRs without spills: gathered
// sources (Q, K and V rows read through slot maps; 163 VGPRs) and packed
// sources with validity bytes (160 VGPRs; the default and ILP schedulers
// spill 4-24 VGPRs in both).  Packed sources with validity bits are launched
// from sparse_attn.hip.
#include "sparse_attn_kernel.h"

namespace rcsa {

int launch_bf16_cu3(AttnArgs& a, dim3 grid, bool gather, hipStream_t s) {
  if (gather)
    sparse_attn_kernel<false, 128, 128, 128, 3, 32, 1, true, true, 3><<<grid, dim3(256), 0, s>>>(a);
  else
    sparse_attn_kernel<false, 128, 128, 128, 3, 32, 1, false, false, 3><<<grid, dim3(256), 0, s>>>(a);
  return launch_status();
}

}  // namespace rcsa
