// The int8 attention as three workgroups per compute unit: 4 wavefronts each
// (one per SIMD, 32 query rows apiece, no key halves to merge), the 128-key
// block staged in four 32-key ring steps of 3 x 12.25 KiB, 157 VGPRs (162 with
// V read through the slot map).  The three workgroups on a SIMD set interleave
// their MFMA and VALU phases where the 8-wavefront kernel's two key halves run
// them in step.  The launcher uses this form when every XCD has at least two
// full rounds of query blocks; smaller grids keep the 8-wavefront kernel.
// Built with the default instruction scheduler (the ILP scheduler spills
// SGPRs here and runs 15% slower).
#include "sparse_attn_kernel.h"

namespace rcsa {

int launch_int8_cu3(AttnArgs& a, dim3 grid, bool gather, bool bits, hipStream_t s) {
  constexpr int kThreads = 128 / 32 * 64;  // BLOCK_M / 32 row groups, one key half
  if (gather)
    sparse_attn_kernel<true, 128, 128, 128, 3, 32, 1, true, true, 3>
        <<<grid, dim3(kThreads), 0, s>>>(a);
  else if (bits)
    sparse_attn_kernel<true, 128, 128, 128, 3, 32, 1, true, false, 3>
        <<<grid, dim3(kThreads), 0, s>>>(a);
  else
    sparse_attn_kernel<true, 128, 128, 128, 3, 32, 1, false, false, 3>
        <<<grid, dim3(kThreads), 0, s>>>(a);
  return launch_status();
}

}  // namespace rcsa
