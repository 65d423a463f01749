// Fixed-budget top-k block selector (gfx950).
//
// One wavefront owns one (head, query block) row.  Every column j gets a
// 64-bit key whose unsigned order is the selection order:
//   bit 62      : column is allowed (0 => key == 0, never selected)
//   bit 61      : column is forced (anchor / local stencil / current chunk)
//   bits 16..47 : order-preserving image of the fp32 score
//   bits  0..15 : 0xffff - j  (lower index wins ties)
// Keys are unique, so the k-th largest key T is found exactly by a 50-step
// MSB-first bisection whose counts are wavefront ballots + popcounts (scalar
// unit, no LDS, no shuffles).  The selected set is {key >= T}; it is written
// in ascending column order by ballot prefix counts, or in rank order.
#include "rcsa_common.h"

namespace rcsa {

struct SelArgs {
  const float* score;
  int64_t n_rows;       // n_bh * n_q
  int64_t n_q, n_k;
  const int32_t* row_k;
  int64_t row_k_stride_bh;
  int64_t k_fixed;
  const uint8_t* forced;
  const uint8_t* allowed;
  int64_t mask_stride_bh;
  int32_t* indices;
  int64_t max_k;
  int32_t* counts;
};

constexpr int kSelWaves = 4;

__device__ __forceinline__ uint64_t column_key(const SelArgs& a, int64_t row,
                                               int64_t bh, int64_t i, int64_t j) {
  if (j >= a.n_k) return 0;
  const int64_t moff = bh * a.mask_stride_bh + i * a.n_k + j;
  if (a.allowed && a.allowed[moff] == 0) return 0;
  const bool forced = a.forced && a.forced[moff] != 0;
  float s = a.score[row * a.n_k + j];
  if (s == 0.0f) s = 0.0f;                          // -0 and +0: one image
  if (s != s) s = __uint_as_float(0x7fc00000u);     // every NaN ranks highest
  const uint32_t u = __float_as_uint(s);
  const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return (1ull << 62) | (static_cast<uint64_t>(forced) << 61) |
         (static_cast<uint64_t>(ord) << 16) | static_cast<uint64_t>(0xffff - j);
}

// PER > 0: keys held in registers (PER per lane, n_k <= 64 * PER).
// PER == 0: keys recomputed from memory on every pass (any n_k <= 65536).
template <int PER, bool RANK>
__global__ void __launch_bounds__(kSelWaves * kWave)
select_kernel(SelArgs a) {
  extern __shared__ uint64_t s_keys[];  // RANK: kSelWaves * max_k
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kSelWaves + wave;
  if (row >= a.n_rows) return;  // whole wavefront exits together
  const int64_t bh = row / a.n_q, i = row % a.n_q;
  const int64_t passes = PER > 0 ? PER : (a.n_k + kWave - 1) / kWave;

  uint64_t keys[PER > 0 ? PER : 1];
  int64_t n_allowed = 0;
  for (int64_t p = 0; p < passes; ++p) {
    const uint64_t key = column_key(a, row, bh, i, lane + kWave * p);
    if (PER > 0) keys[p] = key;
    n_allowed += __popcll(__ballot(key != 0));
  }
  int64_t k = a.row_k ? static_cast<int64_t>(a.row_k[bh * a.row_k_stride_bh + i]) : a.k_fixed;
  k = k < 0 ? 0 : (k > a.max_k ? a.max_k : k);
  const int64_t k_eff = k < n_allowed ? k : n_allowed;
  int32_t* out = a.indices + row * a.max_k;

  uint64_t thr = 0;
  if (k_eff > 0) {
    // bits 48..60 are always zero; skip them
    for (int bit = 62; bit >= 0; --bit) {
      if (bit == 60) bit = 47;
      const uint64_t cand = thr | (1ull << bit);
      int64_t cnt = 0;
      for (int64_t p = 0; p < passes; ++p) {
        const uint64_t key = PER > 0 ? keys[p] : column_key(a, row, bh, i, lane + kWave * p);
        cnt += __popcll(__ballot(key >= cand));
      }
      if (cnt >= k_eff) thr = cand;
    }
    const uint64_t lt_mask = (1ull << lane) - 1ull;
    int64_t base = 0;
    uint64_t* wkeys = s_keys + wave * a.max_k;
    for (int64_t p = 0; p < passes; ++p) {
      const int64_t j = lane + kWave * p;
      const uint64_t key = PER > 0 ? keys[p] : column_key(a, row, bh, i, j);
      const bool sel = key != 0 && key >= thr;
      const uint64_t m = __ballot(sel);
      const int64_t pos = base + __popcll(m & lt_mask);
      if (sel && pos < k_eff) {  // exactly k_eff keys pass: keys are unique
        if (RANK) wkeys[pos] = key;
        else out[pos] = static_cast<int32_t>(j);
      }
      base += __popcll(m);
    }
    if (RANK) {
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      for (int64_t e = lane; e < k_eff; e += kWave) {
        const uint64_t mine = wkeys[e];
        int64_t rank = 0;
        for (int64_t f = 0; f < k_eff; ++f) rank += wkeys[f] > mine;
        out[rank] = static_cast<int32_t>(0xffff - (mine & 0xffffull));
      }
    }
  }
  for (int64_t s = k_eff + lane; s < a.max_k; s += kWave) out[s] = -1;
  if (lane == 0) a.counts[row] = static_cast<int32_t>(k_eff);
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
            k_fixed, forced, allowed, mask_stride_bh, indices, max_k, counts};
  if (order == RCSA_ORDER_RANK) launch_select<true>(a, stream);
  else launch_select<false>(a, stream);
  return launch_status();
}
