// Fixed-budget top-k block selector (gfx950): one wavefront per row; the
// selection itself is in select_core.h.
#include "select_core.h"

namespace rcsa {

template <int PER, bool RANK>
__global__ void __launch_bounds__(kSelWaves * kWave)
select_kernel(SelArgs a) {
  extern __shared__ uint64_t s_keys[];  // RANK: kSelWaves * max_k
  select_rows<PER, RANK, false>(a, blockIdx.x, s_keys);
}

template <bool RANK>
static void launch_select(const SelArgs& a, hipStream_t stream) {
  const int64_t per = (a.n_k + kWave - 1) / kWave;
  dim3 grid(static_cast<unsigned>((a.n_rows + kSelWaves - 1) / kSelWaves));
  dim3 block(kSelWaves * kWave);
  const size_t lds = RANK ? static_cast<size_t>(kSelWaves * a.max_k) * sizeof(uint64_t) : 0;
  if (per <= 1) select_kernel<1, RANK><<<grid, block, lds, stream>>>(a);
  else if (per <= 2) select_kernel<2, RANK><<<grid, block, lds, stream>>>(a);
  else if (per <= 4) select_kernel<4, RANK><<<grid, block, lds, stream>>>(a);
  else if (per <= 8) select_kernel<8, RANK><<<grid, block, lds, stream>>>(a);
  else if (per <= 16) select_kernel<16, RANK><<<grid, block, lds, stream>>>(a);
  else if (per <= 32) select_kernel<32, RANK><<<grid, block, lds, stream>>>(a);
  else select_kernel<0, RANK><<<grid, block, lds, stream>>>(a);
}

}  // namespace rcsa

using namespace rcsa;

extern "C" int rcsa_select_topk(const float* score, int64_t n_bh, int64_t n_qblocks,
                                int64_t n_kblocks, const int32_t* row_k,
                                int64_t row_k_stride_bh, int64_t k_fixed,
                                const uint8_t* forced, const uint8_t* allowed,
                                int64_t mask_stride_bh, int32_t* indices,
                                int64_t max_k, int32_t* counts, int order,
                                hipStream_t stream) {
  if (!score || !indices || !counts) return RCSA_ERR_NULL;
  if (n_bh <= 0 || n_qblocks <= 0 || n_kblocks <= 0 || max_k <= 0) return RCSA_ERR_SHAPE;
  if (n_kblocks > 65536) return RCSA_ERR_SHAPE;
  if (order != RCSA_ORDER_INDEX && order != RCSA_ORDER_RANK) return RCSA_ERR_SHAPE;
  if (order == RCSA_ORDER_RANK && max_k > 2048) return RCSA_ERR_SHAPE;
  if (mask_stride_bh < 0 || row_k_stride_bh < 0) return RCSA_ERR_STRIDE;
  SelArgs a{score, n_bh * n_qblocks, n_qblocks, n_kblocks, row_k, row_k_stride_bh,
            k_fixed, forced, allowed, mask_stride_bh, indices, max_k, counts,
            nullptr, nullptr, 0};
  if (order == RCSA_ORDER_RANK) launch_select<true>(a, stream);
  else launch_select<false>(a, stream);
  return launch_status();
}
