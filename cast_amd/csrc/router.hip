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

__device__ __forceinline__ int wave_sum_i(int v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
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
  extern __shared__ __attribute__((aligned(16))) float s_rem[];  // removable slots' proxies
  __shared__ int s_slot[kRouteMaxBlocks];                         // their slot numbers
  __shared__ uint8_t s_rmem[kRouteMaxBlocks];                     // removed block in memory
  __shared__ int s_pos[kRouteMaxBlocks];                          // candidate position of a block
  __shared__ uint8_t s_kept[kRouteMaxBlocks];
  __shared__ int s_nrem;
  __shared__ float s_rterm[kRouteMaxBlocks];                      // removable slots' own terms
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
  // The quadratic form of an exchange (removed proxies r, added proxies c,
  // d = r - c) expands as
  //   sum_g ca (2 e_g d_g + d_g^2) + 2 lin_g d_g
  //     = [ca |r|^2 + 2 r.w] + [ca |c|^2 - 2 c.w] - 2 ca (r.c),  w = ca e + lin,
  // so each removable slot and each candidate get one term of their own and a
  // pair costs one dot product over the groups.
  const float ca = a.coef[rr];
  float w[kRouteMaxGroups];
#pragma unroll
  for (int g = 0; g < kRouteMaxGroups; ++g)
    w[g] = g < G ? ca * a.error[out_row * G + g] + a.linear[out_row * G + g] : 0.0f;
  for (int i = t; i < nrem; i += kRouteThreads) {
    float r2 = 0.0f, rw = 0.0f;
#pragma unroll
    for (int g = 0; g < kRouteMaxGroups; ++g) {
      if (g < G) {
        const float r = s_rem[i * G + g];
        r2 = fmaf(r, r, r2);
        rw = fmaf(r, w[g], rw);
      }
    }
    s_rterm[i] = ca * r2 + 2.0f * rw;
  }
  __syncthreads();
  const int limit = min(a.cand_mult * cnt, N);
  const float m2ca = -2.0f * ca;
  float bv = INFINITY;
  int bf = 0x7fffffff;
  if (gated) {
    for (int l = t; l < L; l += kRouteThreads) {
      const int c = cand[l];
      if (l >= limit || s_kept[c]) continue;  // not addable
      float add[kRouteMaxGroups];
      float c2 = 0.0f, cw = 0.0f;
#pragma unroll
      for (int g = 0; g < kRouteMaxGroups; ++g) {
        add[g] = g < G ? proxy[static_cast<int64_t>(l) * G + g] : 0.0f;
        c2 = fmaf(add[g], add[g], c2);
        cw = fmaf(add[g], w[g], cw);
      }
      const float aterm = ca * c2 - 2.0f * cw;
      const uint8_t add_mem = c < M;
      // every lane reads the same removable slot at a time (LDS broadcasts)
      for (int i = 0; i < nrem; ++i) {
        if (a.same_bank && s_rmem[i] != add_mem) continue;
        float dot = 0.0f;
        if (G == kRouteMaxGroups) {
          const float4* r4 = reinterpret_cast<const float4*>(s_rem + i * kRouteMaxGroups);
#pragma unroll
          for (int q = 0; q < kRouteMaxGroups / 4; ++q) {
            const float4 r = r4[q];
            dot = fmaf(r.x, add[4 * q], dot);
            dot = fmaf(r.y, add[4 * q + 1], dot);
            dot = fmaf(r.z, add[4 * q + 2], dot);
            dot = fmaf(r.w, add[4 * q + 3], dot);
          }
        } else {
#pragma unroll
          for (int g = 0; g < kRouteMaxGroups; ++g)
            if (g < G) dot = fmaf(s_rem[i * G + g], add[g], dot);
        }
        const float imp = fmaf(m2ca, dot, s_rterm[i] + aterm);
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

// One swap round's decision and its application, on the device
// (P/fc_pasm_swap_routing.py:935-977): the strongest row is the first minimum
// of best over all (bh, current row) (torch.argmin's order); when the swap limit
// is not reached and its value is below -eps, its exchange replaces the kept
// slot with the candidate and moves the row's error by the removed block's
// proxy (zero when it is not a candidate of the row) minus the added one's.
// Otherwise the refinement stops: later rounds change nothing.
// state (int32): [0] swaps applied, [1] stopped, then per applied swap
// [bh, row, slot, removed block, added block, improvement as float bits].
struct ApplyArgs {
  const float* best;          // [n_bh * rows]
  const int32_t* best_flat;   // [n_bh * rows]
  const int32_t* cand;        // [n_bh, rows, n_cand]
  const float* proxy;         // [n_bh, rows, n_cand, groups]
  int32_t* selected;          // [n_bh, n_blocks, max_k]
  float* error;               // [n_bh, rows, groups]
  int32_t* state;
  int n_bh, n_blocks, memory_blocks, max_k, n_cand, groups, max_swaps, max_records;
  float eps;
};

__global__ void __launch_bounds__(kRouteThreads)
route_apply_kernel(ApplyArgs a) {
  __shared__ float s_bv[kRouteThreads / kWave];
  __shared__ int s_bi[kRouteThreads / kWave];
  __shared__ int s_hit;
  const int t = threadIdx.x;
  const int rows = a.n_blocks - a.memory_blocks;
  const int n = a.n_bh * rows;
  const int swaps = a.state[0];
  if (a.state[1] != 0) return;  // an earlier round stopped (uniform)
  if ((a.max_swaps > 0 && swaps >= a.max_swaps) || swaps >= a.max_records) {
    if (t == 0) a.state[1] = 1;
    return;
  }
  float bv = INFINITY;
  int bi = 0x7fffffff;
  for (int i = t; i < n; i += kRouteThreads) {
    const float v = a.best[i];
    if (v < bv || (v == bv && i < bi)) { bv = v; bi = i; }
  }
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, kWave);
    const int oi = __shfl_xor(bi, o, kWave);
    if (ov < bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
  }
  const int lane = t % kWave, wave = t / kWave;
  if (lane == 0) { s_bv[wave] = bv; s_bi[wave] = bi; }
  if (t == 0) s_hit = 0x7fffffff;
  __syncthreads();
  for (int w = 0; w < kRouteThreads / kWave; ++w)
    if (s_bv[w] < bv || (s_bv[w] == bv && s_bi[w] < bi)) { bv = s_bv[w]; bi = s_bi[w]; }
  // every thread now holds the same (bv, bi); rows with no exchange hold +inf
  if (!(bv < -a.eps) || bi >= n) {
    if (t == 0) a.state[1] = 1;
    return;
  }
  const int fl = a.best_flat[bi];
  if (fl < 0) {
    if (t == 0) a.state[1] = 1;
    return;
  }
  const int bh = bi / rows, rr = bi % rows, row = a.memory_blocks + rr;
  const int slot = fl / a.n_cand, pos = fl % a.n_cand;
  int32_t* sel = a.selected + (static_cast<int64_t>(bh) * a.n_blocks + row) * a.max_k;
  const int32_t* cand = a.cand + static_cast<int64_t>(bi) * a.n_cand;
  const float* proxy = a.proxy + static_cast<int64_t>(bi) * a.n_cand * a.groups;
  const int32_t removed = sel[slot];
  // the removed block's candidate position (its first occurrence), if any
  for (int l = t; l < a.n_cand; l += kRouteThreads)
    if (cand[l] == removed) atomicMin(&s_hit, l);
  __syncthreads();
  const int hit = s_hit;
  if (t < a.groups) {
    const float rem = hit < a.n_cand ? proxy[static_cast<int64_t>(hit) * a.groups + t] : 0.0f;
    const float add = proxy[static_cast<int64_t>(pos) * a.groups + t];
    a.error[static_cast<int64_t>(bi) * a.groups + t] += rem - add;
  }
  if (t == 0) {
    const int32_t added = cand[pos];
    sel[slot] = added;
    int32_t* rec = a.state + 2 + 6 * swaps;
    rec[0] = bh;
    rec[1] = row;
    rec[2] = slot;
    rec[3] = removed;
    rec[4] = added;
    rec[5] = __float_as_int(-bv);
    a.state[0] = swaps + 1;
  }
}

// The checks at the end of a refine (P/fc_pasm_swap_routing.py:983-1033), per
// (bh, row) over the first count entries of the row before
// (base) and after (sel) the refinement, summed into out (int32, zero before):
// [0] rows whose memory-bank count changed, [1] rows with a repeated block,
// [2] local edges the rows keep, [3] rows whose current-bank blocks changed,
// [4] / [5] memory-bank entries before / after, [6] max_k - the smallest
// count, [7] the largest count, [8] the count sum, [9] the local edges of the
// stencil over all rows (what [2] must equal).
struct CheckArgs {
  const int32_t* base;     // [n_bh, n_blocks, max_k]
  const int32_t* sel;      // [n_bh, n_blocks, max_k]
  const int32_t* counts;   // [n_bh, n_blocks]
  const uint8_t* local;    // [n_blocks, n_blocks]
  int n_blocks, memory_blocks, max_k;
  int32_t* out;
};

// One workgroup per (bh, run of kCheckRows rows), one wavefront per row at a
// time (bitmaps in LDS per wavefront); the sums meet in LDS, then ten global
// atomics per workgroup.
constexpr int kCheckRows = 16;
__global__ void __launch_bounds__(kRouteThreads)
route_check_kernel(CheckArgs a) {
  constexpr int kWords = kRouteMaxBlocks / 32;
  constexpr int kWaves = kRouteThreads / kWave;
  __shared__ uint32_t s_seen[kWaves][kWords];   // blocks kept after
  __shared__ uint32_t s_cur0[kWaves][kWords];   // current-bank blocks kept before
  __shared__ int s_acc[10];
  const int N = a.n_blocks, M = a.memory_blocks, K = a.max_k;
  const int runs = (N + kCheckRows - 1) / kCheckRows;
  const int64_t bh = blockIdx.x / runs;
  const int row0 = static_cast<int>(blockIdx.x % runs) * kCheckRows;
  const int row_end = min(row0 + kCheckRows, N);
  const int t = threadIdx.x, lane = t % kWave, wave = t / kWave;
  if (t < 10) s_acc[t] = 0;
  int acc[10] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  for (int row = row0 + wave; row < row_end; row += kWaves) {
    for (int w = lane; w < kWords; w += kWave) { s_seen[wave][w] = 0u; s_cur0[wave][w] = 0u; }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    const int cnt = min(max(a.counts[bh * N + row], 0), K);
    const int32_t* base = a.base + (bh * N + row) * static_cast<int64_t>(K);
    const int32_t* sel = a.sel + (bh * N + row) * static_cast<int64_t>(K);
    const uint8_t* loc = a.local + static_cast<int64_t>(row) * N;
    int hist0 = 0, hist1 = 0, kept_local = 0, dup = 0, cur0 = 0, cur1 = 0, stencil = 0;
    for (int s = lane; s < cnt; s += kWave) {
      const int32_t b0 = base[s], b1 = sel[s];
      hist0 += b0 >= 0 && b0 < M;
      hist1 += b1 >= 0 && b1 < M;
      if (b0 >= M && b0 < N) {
        atomicOr(&s_cur0[wave][b0 / 32], 1u << (b0 % 32));
        ++cur0;
      }
      if (b1 >= 0 && b1 < N) {
        kept_local += loc[b1] != 0;
        const uint32_t bit = 1u << (b1 % 32);
        dup += (atomicOr(&s_seen[wave][b1 / 32], bit) & bit) != 0u;
        cur1 += b1 >= M;
      }
    }
    for (int j = lane; j < N; j += kWave) stencil += loc[j] != 0;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    // current-bank blocks after, as a bitmap, against those before
    int cur_diff = 0;
    for (int w = lane; w < kWords; w += kWave) {
      uint32_t after = s_seen[wave][w];
      const int lo = w * 32;
      if (lo + 32 <= M) after = 0u;
      else if (lo < M) after &= ~((1u << (M - lo)) - 1u);
      cur_diff += after != s_cur0[wave][w];
    }
    hist0 = wave_sum_i(hist0); hist1 = wave_sum_i(hist1);
    dup = wave_sum_i(dup); cur0 = wave_sum_i(cur0); cur1 = wave_sum_i(cur1);
    cur_diff = wave_sum_i(cur_diff);
    acc[0] += hist0 != hist1;
    acc[1] += dup != 0;
    acc[2] += kept_local;  // summed over lanes below
    acc[3] += (cur_diff != 0 || cur0 != cur1);
    acc[4] += hist0;
    acc[5] += hist1;
    acc[6] = max(acc[6], K - cnt);
    acc[7] = max(acc[7], cnt);
    acc[8] += cnt;
    acc[9] += stencil;  // summed over lanes below
    __builtin_amdgcn_wave_barrier();
  }
  acc[2] = wave_sum_i(acc[2]);
  acc[9] = wave_sum_i(acc[9]);
  __syncthreads();
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < 10; ++i) {
      if (i == 6 || i == 7) atomicMax(&s_acc[i], acc[i]);
      else atomicAdd(&s_acc[i], acc[i]);
    }
  }
  __syncthreads();
  if (t < 10) {
    if (t == 6 || t == 7) atomicMax(&a.out[t], s_acc[t]);
    else atomicAdd(&a.out[t], s_acc[t]);
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

extern "C" int rcsa_route_apply_swap(const float* best, const int32_t* best_flat,
                                     const int32_t* cand, const float* proxy, int32_t* selected,
                                     float* error, int32_t* state, int64_t n_bh,
                                     int64_t n_blocks, int64_t memory_blocks, int64_t max_k,
                                     int64_t n_cand, int64_t sketch_groups, int64_t max_swaps,
                                     int64_t max_records, float eps, hipStream_t stream) {
  if (!best || !best_flat || !cand || !proxy || !selected || !error || !state)
    return RCSA_ERR_NULL;
  int st = route_shapes(n_bh, n_blocks, memory_blocks, max_k, n_cand, sketch_groups, 1);
  if (st) return st;
  if (max_swaps < 0 || max_records <= 0 || max_records > 64 || !(eps >= 0.0f))
    return RCSA_ERR_SHAPE;
  const ApplyArgs a{best, best_flat, cand, proxy, selected, error, state,
                    static_cast<int>(n_bh), static_cast<int>(n_blocks),
                    static_cast<int>(memory_blocks), static_cast<int>(max_k),
                    static_cast<int>(n_cand), static_cast<int>(sketch_groups),
                    static_cast<int>(max_swaps < (int64_t{1} << 30) ? max_swaps : 0),
                    static_cast<int>(max_records), eps};
  route_apply_kernel<<<dim3(1), dim3(kRouteThreads), 0, stream>>>(a);
  return launch_status();
}

extern "C" int rcsa_route_check(const int32_t* base, const int32_t* selected,
                                const int32_t* counts, const uint8_t* local, int64_t n_bh,
                                int64_t n_blocks, int64_t memory_blocks, int64_t max_k,
                                int32_t* out, hipStream_t stream) {
  if (!base || !selected || !counts || !local || !out) return RCSA_ERR_NULL;
  if (n_bh <= 0 || n_blocks <= 0 || n_blocks > kRouteMaxBlocks) return RCSA_ERR_SHAPE;
  if (memory_blocks < 0 || memory_blocks > n_blocks || max_k <= 0) return RCSA_ERR_SHAPE;
  if (n_bh * n_blocks >= (int64_t{1} << 31) || n_bh * n_blocks * max_k >= (int64_t{1} << 31))
    return RCSA_ERR_SHAPE;
  const CheckArgs a{base, selected, counts, local, static_cast<int>(n_blocks),
                    static_cast<int>(memory_blocks), static_cast<int>(max_k), out};
  const int64_t grid = n_bh * ((n_blocks + kCheckRows - 1) / kCheckRows);
  route_check_kernel<<<dim3(static_cast<unsigned>(grid)), dim3(kRouteThreads), 0, stream>>>(a);
  return launch_status();
}
