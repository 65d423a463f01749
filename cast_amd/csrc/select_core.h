// Fixed-budget top-k selection of one (head, query block) row per wavefront,
// shared by rcsa_select_topk and the fused key-quantiser + selection launch.
//
// Every column j gets a 64-bit key whose unsigned order is the selection order:
//   bit 62      : column is allowed (0 => key == 0, never selected)
//   bit 61      : column is forced (anchor / local stencil / current chunk)
//   bits 16..47 : order-preserving image of the fp32 score
//   bits  0..15 : 0xffff - j  (lower index wins ties)
// Keys are unique, so the k-th largest key T is found exactly by a 50-step
// MSB-first bisection whose counts are wavefront ballots + popcounts (scalar
// unit, no LDS, no shuffles).  The selected set is {key >= T}; it is written
// in ascending column order by ballot prefix counts, or in rank order.
#pragma once
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
  // fused scoring (SCORE kernels): score(row, j) = qhat[row] . khat[bh, j],
  // summed over the head_dim channels in order, written to score when set
  const float* qhat;
  const float* khat;
  int64_t head_dim;
};

constexpr int kSelWaves = 4;

template <bool SCORE>
__device__ __forceinline__ uint64_t column_key(const SelArgs& a, int64_t row,
                                               int64_t bh, int64_t i, int64_t j) {
  if (j >= a.n_k) return 0;
  float s;
  if constexpr (SCORE) {  // the cosine score, in rcsa_block_scores' summation order
    constexpr int kD = 128;  // the fused launch's head_dim: the loads unroll and overlap
    const float4* q = reinterpret_cast<const float4*>(a.qhat + row * kD);
    const float4* k = reinterpret_cast<const float4*>(a.khat + (bh * a.n_k + j) * kD);
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < kD / 4; ++c) {
      const float4 qv = q[c], kv = k[c];
      acc = fmaf(qv.x, kv.x, acc);
      acc = fmaf(qv.y, kv.y, acc);
      acc = fmaf(qv.z, kv.z, acc);
      acc = fmaf(qv.w, kv.w, acc);
    }
    if (a.score) const_cast<float*>(a.score)[row * a.n_k + j] = acc;
    s = acc;
  } else {
    s = a.score[row * a.n_k + j];
  }
  const int64_t moff = bh * a.mask_stride_bh + i * a.n_k + j;
  if (a.allowed && a.allowed[moff] == 0) return 0;
  const bool forced = a.forced && a.forced[moff] != 0;
  if (s == 0.0f) s = 0.0f;                          // -0 and +0: one image
  if (s != s) s = __uint_as_float(0x7fc00000u);     // every NaN ranks highest
  const uint32_t u = __float_as_uint(s);
  const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return (1ull << 62) | (static_cast<uint64_t>(forced) << 61) |
         (static_cast<uint64_t>(ord) << 16) | static_cast<uint64_t>(0xffff - j);
}

// PER > 0: keys held in registers (PER per lane, n_k <= 64 * PER).
// PER == 0: keys recomputed from memory on every pass (any n_k <= 65536).
// SCORE: the scores are computed here (PER > 0 only: each once).
template <int PER, bool RANK, bool SCORE>
__device__ __forceinline__ void select_rows(const SelArgs& a, int64_t block, uint64_t* s_keys) {
  static_assert(!SCORE || PER > 0, "fused scores need the keys in registers");
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int64_t row = block * kSelWaves + wave;
  if (row >= a.n_rows) return;  // whole wavefront exits together
  const int64_t bh = row / a.n_q, i = row % a.n_q;
  const int64_t passes = PER > 0 ? PER : (a.n_k + kWave - 1) / kWave;

  uint64_t keys[PER > 0 ? PER : 1];
  int64_t n_allowed = 0;
  for (int64_t p = 0; p < passes; ++p) {
    const uint64_t key = column_key<SCORE>(a, row, bh, i, lane + kWave * p);
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
        const uint64_t key = PER > 0 ? keys[p] : column_key<SCORE>(a, row, bh, i, lane + kWave * p);
        cnt += __popcll(__ballot(key >= cand));
      }
      if (cnt >= k_eff) thr = cand;
    }
    const uint64_t lt_mask = (1ull << lane) - 1ull;
    int64_t base = 0;
    uint64_t* wkeys = s_keys + wave * a.max_k;
    for (int64_t p = 0; p < passes; ++p) {
      const int64_t j = lane + kWave * p;
      const uint64_t key = PER > 0 ? keys[p] : column_key<SCORE>(a, row, bh, i, j);
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

}  // namespace rcsa
