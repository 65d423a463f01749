// FC-PASM swap router on the device (gfx950): the per-row work of a
// fixed-budget coordinate-swap refinement of a top-k route.
//
// route_proxy_kernel (one workgroup per (bh, current row)): softmax of the
// row's block scores, the pooled attention output o = P v, the row's 2k
// candidate blocks (ranking score + 1e6 local, descending, ties to the lower
// index), the omission proxy of every candidate sketched over channel groups,
// and the row's error (the proxies of the candidates it does not keep).
// route_swap_kernel (one workgroup per (bh, current row)): the best single
// (removed slot, added candidate) exchange of the row under the objective's
// quadratic form, as a value and a flat index slot * n_cand + candidate.
#include "rcsa_common.h"

namespace rcsa {

constexpr int kRouteThreads = 256;
constexpr int kRouteMaxBlocks = 1024;
constexpr int kRouteMaxGroups = 16;
constexpr int kRouteMaxD = 128;
constexpr int kRouteMaxDynFloats = 12288;  // 48 KiB of dynamic LDS per workgroup

// Ascending keys order rankings descending, equal rankings by index ascending.
__device__ __forceinline__ uint64_t rank_key(float r, int i) {
  uint32_t u = __float_as_uint(r);
  u ^= (u & 0x80000000u) ? 0xffffffffu : 0x80000000u;  // monotone in r
  return (static_cast<uint64_t>(0xffffffffu - u) << 32) | static_cast<uint32_t>(i);
}

__device__ float route_block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}
__device__ float route_block_max(float v, float* red) {
  v = wave_max(v);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

struct RouteArgs {
  const float* score;         // [n_bh, n_blocks, n_blocks]
  const float* value;         // [n_bh, n_blocks, D] pooled (mean) values
  const uint8_t* local;       // [n_blocks, n_blocks] protected local edges
  const int32_t* selected;    // [n_bh, n_blocks, max_k]
  const int32_t* counts;      // [n_bh, n_blocks]
  int n_blocks, memory_blocks, D, max_k, n_cand, cand_mult, groups;
  float eps;
  int32_t* cand;              // [n_bh, rows, n_cand]
  float* proxy;               // [n_bh, rows, n_cand, groups]
  float* error;               // [n_bh, rows, groups]
};

__global__ void __launch_bounds__(kRouteThreads)
route_proxy_kernel(RouteArgs a) {
  __shared__ float s_p[kRouteMaxBlocks];
  __shared__ uint64_t s_key[kRouteMaxBlocks];
  __shared__ float s_part[kRouteThreads * 4];
  __shared__ float s_o[kRouteMaxD];
  __shared__ uint8_t s_kept[kRouteMaxBlocks];
  __shared__ float s_red[4];
  extern __shared__ float s_px[];  // the row's proxies, n_cand x groups
  const int N = a.n_blocks, rows = N - a.memory_blocks;
  const int64_t bh = blockIdx.x / rows;
  const int row = a.memory_blocks + static_cast<int>(blockIdx.x % rows);
  const int t = threadIdx.x;
  const float* x = a.score + (bh * N + row) * static_cast<int64_t>(N);
  const uint8_t* loc = a.local + static_cast<int64_t>(row) * N;

  // softmax of the row (fp32, max-subtracted)
  float mx = -INFINITY;
  for (int k = t; k < N; k += kRouteThreads) {
    const float v = x[k];
    s_p[k] = v;
    mx = fmaxf(mx, v);
    s_kept[k] = 0;
  }
  mx = route_block_max(mx, s_red);
  float sum = 0.0f;
  for (int k = t; k < N; k += kRouteThreads) {
    const float e = expf(s_p[k] - mx);
    s_p[k] = e;
    sum += e;
  }
  sum = route_block_sum(sum, s_red);
  const float inv = 1.0f / sum;
  // ranking keys (score + 1e6 local), padded to a power of two
  int np = 1;
  while (np < N) np <<= 1;
  for (int k = t; k < np; k += kRouteThreads)
    s_key[k] = k < N ? rank_key(x[k] + (loc[k] ? 1e6f : 0.0f), k) : ~0ull;
  // kept blocks of the row
  const int cnt = min(max(a.counts[bh * N + row], 0), a.max_k);
  const int32_t* sel = a.selected + (bh * N + row) * static_cast<int64_t>(a.max_k);
  __syncthreads();
  for (int s = t; s < cnt; s += kRouteThreads) {
    const int32_t b = sel[s];
    if (b >= 0 && b < N) s_kept[b] = 1;
  }
  for (int k = t; k < N; k += kRouteThreads) s_p[k] *= inv;
  __syncthreads();

  // o = P v: D / 4 float4 columns, kRouteThreads * 4 / D partial sums over the
  // blocks, four loads in flight per thread
  const int D = a.D;
  const int c4 = D / 4, parts = kRouteThreads / c4;
  const float* v = a.value + bh * static_cast<int64_t>(N) * D;
  {
    const int col = t % c4, part = t / c4;
    const float4* v4 = reinterpret_cast<const float4*>(v) + col;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    int k = part;
    for (; k + 3 * parts < N; k += 4 * parts) {
      float4 w[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) w[u] = v4[static_cast<int64_t>(k + u * parts) * c4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float p = s_p[k + u * parts];
        acc.x = fmaf(p, w[u].x, acc.x);
        acc.y = fmaf(p, w[u].y, acc.y);
        acc.z = fmaf(p, w[u].z, acc.z);
        acc.w = fmaf(p, w[u].w, acc.w);
      }
    }
    for (; k < N; k += parts) {
      const float4 w = v4[static_cast<int64_t>(k) * c4];
      const float p = s_p[k];
      acc.x = fmaf(p, w.x, acc.x);
      acc.y = fmaf(p, w.y, acc.y);
      acc.z = fmaf(p, w.z, acc.z);
      acc.w = fmaf(p, w.w, acc.w);
    }
    reinterpret_cast<float4*>(s_part)[part * c4 + col] = acc;
  }
  // (the sort's first barrier also publishes s_part)
  for (int kk = 2; kk <= np; kk <<= 1) {
    for (int j = kk >> 1; j > 0; j >>= 1) {
      __syncthreads();
      for (int i = t; i < np / 2; i += kRouteThreads) {
        const int lo = ((i & ~(j - 1)) << 1) | (i & (j - 1));
        const int hi = lo | j;
        const bool up = (lo & kk) == 0;
        const uint64_t ka = s_key[lo], kb = s_key[hi];
        if ((ka > kb) == up) {
          s_key[lo] = kb;
          s_key[hi] = ka;
        }
      }
    }
  }
  __syncthreads();
  if (t < D) {
    float o = 0.0f;
    for (int part = 0; part < parts; ++part) o += s_part[part * D + t];
    s_o[t] = o;
  }
  __syncthreads();

  // candidates, their proxies, and the row's error
  const int L = a.n_cand, G = a.groups, gw = D / G;
  const int64_t out_row = bh * rows + (row - a.memory_blocks);
  int32_t* cand = a.cand + out_row * L;
  float* proxy = a.proxy + out_row * static_cast<int64_t>(L) * G;
  const int limit = min(a.cand_mult * cnt, N);
  // proxy of candidate l, group g: p / (1 - p + eps) * mean over the group of (o - v_c)
  auto proxy_of = [&](int l, int g) {
    const int c = static_cast<int>(static_cast<uint32_t>(s_key[l]));
    const float p = s_p[c];
    const float w = p / (1.0f - p + a.eps);
    const float* vc = v + static_cast<int64_t>(c) * D + g * gw;
    float acc = 0.0f;
    if (gw == 8) {  // 16 groups of 128 channels: two 16-byte loads
      const float4 lo = reinterpret_cast<const float4*>(vc)[0];
      const float4 hi = reinterpret_cast<const float4*>(vc)[1];
      const float vv[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
      for (int d = 0; d < 8; ++d) acc += w * (s_o[g * 8 + d] - vv[d]);
    } else {
      for (int d = 0; d < gw; ++d) acc += w * (s_o[g * gw + d] - vc[d]);
    }
    return acc / static_cast<float>(gw);
  };
  for (int e = t; e < L * G; e += kRouteThreads) {
    const int l = e / G, g = e % G;
    const float px = proxy_of(l, g);
    proxy[e] = px;
    s_px[e] = px;
    if (g == 0) cand[l] = static_cast<int>(static_cast<uint32_t>(s_key[l]));
  }
  __syncthreads();
  // the row's error: the proxies of the candidates within its limit that it
  // does not keep, summed in candidate order
  if (t < G) {
    float err = 0.0f;
    for (int l = 0; l < limit && l < L; ++l) {
      const int c = static_cast<int>(static_cast<uint32_t>(s_key[l]));
      if (!s_kept[c]) err += s_px[l * G + t];
    }
    a.error[out_row * G + t] = err;
  }
}

struct SwapArgs {
  const float* proxy;         // [n_bh, rows, n_cand, groups]
  const int32_t* cand;        // [n_bh, rows, n_cand]
  const uint8_t* local;
  const int32_t* selected;
  const int32_t* counts;
  const float* coef;          // [rows]
  const float* linear;        // [n_bh, rows, groups]
  const float* error;         // [n_bh, rows, groups]
  const uint8_t* row_gate;    // [rows] or NULL
  int n_blocks, memory_blocks, max_k, n_cand, cand_mult, groups, same_bank;
  float* best;                // [n_bh, rows]
  int32_t* best_flat;         // [n_bh, rows]
};

__global__ void __launch_bounds__(kRouteThreads)
route_swap_kernel(SwapArgs a) {
  extern __shared__ float s_rem[];                                // removable slots' proxies
  __shared__ int s_slot[kRouteMaxBlocks];                         // their slot numbers
  __shared__ uint8_t s_rmem[kRouteMaxBlocks];                     // removed block in memory
  __shared__ int s_pos[kRouteMaxBlocks];                          // candidate position of a block
  __shared__ uint8_t s_kept[kRouteMaxBlocks];
  __shared__ int s_nrem;
  __shared__ float s_bv[kRouteThreads / kWave];
  __shared__ int s_bf[kRouteThreads / kWave];
  const int N = a.n_blocks, rows = N - a.memory_blocks, M = a.memory_blocks;
  const int64_t bh = blockIdx.x / rows;
  const int rr = static_cast<int>(blockIdx.x % rows), row = M + rr;
  const int t = threadIdx.x;
  const int L = a.n_cand, G = a.groups;
  const int64_t out_row = bh * rows + rr;
  const int32_t* cand = a.cand + out_row * L;
  const float* proxy = a.proxy + out_row * static_cast<int64_t>(L) * G;
  const uint8_t* loc = a.local + static_cast<int64_t>(row) * N;
  const int cnt = min(max(a.counts[bh * N + row], 0), a.max_k);
  const int32_t* sel = a.selected + (bh * N + row) * static_cast<int64_t>(a.max_k);
  for (int k = t; k < N; k += kRouteThreads) {
    s_pos[k] = -1;
    s_kept[k] = 0;
  }
  if (t == 0) s_nrem = 0;
  __syncthreads();
  for (int l = t; l < L; l += kRouteThreads) s_pos[cand[l]] = l;
  for (int s = t; s < cnt; s += kRouteThreads) {
    const int32_t b = sel[s];
    if (b >= 0 && b < N) s_kept[b] = 1;
  }
  __syncthreads();
  // removable slots (kept, not a protected local edge), in any order: equal
  // values are resolved by the flat index, not by this order
  for (int s = t; s < cnt; s += kRouteThreads) {
    const int32_t b = sel[s];
    if (b >= 0 && b < N && !loc[b]) {
      const int n = atomicAdd(&s_nrem, 1);
      s_rmem[n] = b < M;
      s_slot[n] = s;
    }
  }
  __syncthreads();
  const int nrem = s_nrem;
  const bool gated = a.row_gate == nullptr || a.row_gate[rr] != 0;
  for (int e = t; e < nrem * G; e += kRouteThreads) {
    const int i = e / G, g = e % G;
    const int pos = s_pos[sel[s_slot[i]]];
    s_rem[e] = pos >= 0 ? proxy[static_cast<int64_t>(pos) * G + g] : 0.0f;
  }
  __syncthreads();
  const float ca = a.coef[rr];
  float err[kRouteMaxGroups], lin[kRouteMaxGroups];
#pragma unroll
  for (int g = 0; g < kRouteMaxGroups; ++g) {
    err[g] = g < G ? a.error[out_row * G + g] : 0.0f;
    lin[g] = g < G ? a.linear[out_row * G + g] : 0.0f;
  }
  const int limit = min(a.cand_mult * cnt, N);
  float bv = INFINITY;
  int bf = 0x7fffffff;
  if (gated) {
    for (int l = t; l < L; l += kRouteThreads) {
      const int c = cand[l];
      if (l >= limit || s_kept[c]) continue;  // not addable
      float add[kRouteMaxGroups];
#pragma unroll
      for (int g = 0; g < kRouteMaxGroups; ++g)
        add[g] = g < G ? proxy[static_cast<int64_t>(l) * G + g] : 0.0f;
      const uint8_t add_mem = c < M;
      // every lane reads the same removable slot at a time (LDS broadcasts)
      for (int i = 0; i < nrem; ++i) {
        if (a.same_bank && s_rmem[i] != add_mem) continue;
        float imp = 0.0f;
#pragma unroll
        for (int g = 0; g < kRouteMaxGroups; ++g) {
          if (g < G) {
            const float dl = s_rem[i * G + g] - add[g];
            imp += ca * (2.0f * err[g] * dl + dl * dl) + 2.0f * lin[g] * dl;
          }
        }
        const int flat = s_slot[i] * L + l;
        if (imp < bv || (imp == bv && flat < bf)) {
          bv = imp;
          bf = flat;
        }
      }
    }
  }
  // workgroup minimum, ties to the lower flat index
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, kWave);
    const int of = __shfl_xor(bf, o, kWave);
    if (ov < bv || (ov == bv && of < bf)) {
      bv = ov;
      bf = of;
    }
  }
  const int lane = t % kWave, wave = t / kWave;
  if (lane == 0) {
    s_bv[wave] = bv;
    s_bf[wave] = bf;
  }
  __syncthreads();
  if (t == 0) {
    for (int w = 1; w < kRouteThreads / kWave; ++w)
      if (s_bv[w] < bv || (s_bv[w] == bv && s_bf[w] < bf)) {
        bv = s_bv[w];
        bf = s_bf[w];
      }
    a.best[out_row] = bv;
    a.best_flat[out_row] = bv == INFINITY ? -1 : bf;
  }
}

}  // namespace rcsa

using namespace rcsa;

static int route_shapes(int64_t n_bh, int64_t n_blocks, int64_t memory_blocks, int64_t max_k,
                        int64_t n_cand, int64_t groups, int64_t cand_mult) {
  if (n_bh <= 0 || n_blocks <= 0 || n_blocks > kRouteMaxBlocks) return RCSA_ERR_SHAPE;
  if (memory_blocks < 0 || memory_blocks >= n_blocks) return RCSA_ERR_SHAPE;
  if (max_k <= 0 || max_k > n_blocks || n_cand <= 0 || n_cand > n_blocks) return RCSA_ERR_SHAPE;
  if (groups <= 0 || groups > kRouteMaxGroups || cand_mult <= 0) return RCSA_ERR_SHAPE;
  if (n_bh * (n_blocks - memory_blocks) >= (int64_t{1} << 31)) return RCSA_ERR_SHAPE;
  return RCSA_OK;
}

extern "C" int rcsa_route_proxy(const float* score, const float* pooled_value, const uint8_t* local,
                                const int32_t* selected, const int32_t* counts, int64_t n_bh,
                                int64_t n_blocks, int64_t memory_blocks, int64_t head_dim,
                                int64_t max_k, int64_t n_cand, int64_t cand_mult,
                                int64_t sketch_groups, float eps, int32_t* cand, float* proxy,
                                float* error, hipStream_t stream) {
  if (!score || !pooled_value || !local || !selected || !counts || !cand || !proxy || !error)
    return RCSA_ERR_NULL;
  int st = route_shapes(n_bh, n_blocks, memory_blocks, max_k, n_cand, sketch_groups, cand_mult);
  if (st) return st;
  if (!(head_dim == 64 || head_dim == 128) || head_dim % sketch_groups) return RCSA_ERR_SHAPE;
  if (n_cand * sketch_groups > kRouteMaxDynFloats) return RCSA_ERR_SHAPE;
  if (reinterpret_cast<uintptr_t>(pooled_value) & 15u) return RCSA_ERR_ALIGN;
  if (!(eps >= 0.0f)) return RCSA_ERR_SHAPE;
  RouteArgs a{score, pooled_value, local, selected, counts, static_cast<int>(n_blocks),
              static_cast<int>(memory_blocks), static_cast<int>(head_dim),
              static_cast<int>(max_k), static_cast<int>(n_cand), static_cast<int>(cand_mult),
              static_cast<int>(sketch_groups), eps, cand, proxy, error};
  const int64_t grid = n_bh * (n_blocks - memory_blocks);
  const size_t lds = static_cast<size_t>(n_cand * sketch_groups) * sizeof(float);
  route_proxy_kernel<<<dim3(static_cast<unsigned>(grid)), dim3(kRouteThreads), lds, stream>>>(a);
  return launch_status();
}

extern "C" int rcsa_route_best_swap(const float* proxy, const int32_t* cand, const uint8_t* local,
                                    const int32_t* selected, const int32_t* counts,
                                    const float* coef, const float* linear, const float* error,
                                    const uint8_t* row_gate, int64_t n_bh, int64_t n_blocks,
                                    int64_t memory_blocks, int64_t max_k, int64_t n_cand,
                                    int64_t cand_mult, int64_t sketch_groups, int same_bank,
                                    float* best, int32_t* best_flat, hipStream_t stream) {
  if (!proxy || !cand || !local || !selected || !counts || !coef || !linear || !error || !best ||
      !best_flat)
    return RCSA_ERR_NULL;
  int st = route_shapes(n_bh, n_blocks, memory_blocks, max_k, n_cand, sketch_groups, cand_mult);
  if (st) return st;
  // the removable slots' proxies live in LDS; flat indices stay below 2^31
  if (max_k * sketch_groups > kRouteMaxDynFloats) return RCSA_ERR_SHAPE;
  if (max_k * n_cand >= (int64_t{1} << 31)) return RCSA_ERR_SHAPE;
  SwapArgs a{proxy, cand, local, selected, counts, coef, linear, error, row_gate,
             static_cast<int>(n_blocks), static_cast<int>(memory_blocks),
             static_cast<int>(max_k), static_cast<int>(n_cand), static_cast<int>(cand_mult),
             static_cast<int>(sketch_groups), same_bank ? 1 : 0, best, best_flat};
  const int64_t grid = n_bh * (n_blocks - memory_blocks);
  const size_t lds = static_cast<size_t>(max_k * sketch_groups) * sizeof(float);
  route_swap_kernel<<<dim3(static_cast<unsigned>(grid)), dim3(kRouteThreads), lds, stream>>>(a);
  return launch_status();
}
