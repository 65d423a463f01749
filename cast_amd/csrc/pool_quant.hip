// Block pooling, cosine block scores and the int8 Q/K quantiser (gfx950).
//
// All three passes over Q/K are HBM-bound streams: one workgroup owns one
// (head, block) tile of block_size tokens x head_dim channels and reads it
// once with 16-byte coalesced loads (a bf16 row of 128 channels is 16 lanes
// x 16 B).  Per-channel partial sums are combined through LDS.
#include "rcsa_common.h"

namespace rcsa {

constexpr int kPoolThreads = 256;

struct PoolArgs {
  const void* x;
  int64_t n_heads;
  int64_t n_blocks;
  int64_t stride_b, stride_h, stride_t;
  const uint8_t* valid;
  float* hat;
  float* bsum;
  float* bmin;
  float* bmax;
  int8_t* x_i8;     // query quantiser output (pool_query only)
  float* x_scale;   // query scales (pool_query only)
};

// Block-wide helpers (kPoolThreads = 4 waves).
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float r = red[0] + red[1] + red[2] + red[3];
  return r;
}
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// One workgroup per (bh, block).  QUANT: fuse the int8 query quantiser.
// STATS: write sum/min/max for the key quantiser.
template <typename T, int D, int BS, bool QUANT, bool STATS>
__global__ void __launch_bounds__(kPoolThreads)
pool_kernel(PoolArgs a) {
  constexpr int CPR = D / 8;                 // 16-byte chunks per token row
  constexpr int RG = kPoolThreads / CPR;     // row groups
  constexpr int ROWS = BS / RG;              // rows per thread
  static_assert(ROWS >= 1 && RG * CPR == kPoolThreads, "tile shape");

  __shared__ float s_sum[RG][D];
  __shared__ float s_min[STATS ? RG : 1][D];
  __shared__ float s_max[STATS ? RG : 1][D];
  __shared__ float s_red[4];

  const int64_t blk = blockIdx.x % a.n_blocks;
  const int64_t bh = blockIdx.x / a.n_blocks;
  const int64_t b_outer = bh / a.n_heads, h = bh % a.n_heads;
  const T* x = static_cast<const T*>(a.x) + b_outer * a.stride_b + h * a.stride_h +
               blk * BS * a.stride_t;
  const int t = threadIdx.x;
  const int c = t % CPR, g = t / CPR;

  const int n_valid = __syncthreads_count(
      t < BS && (a.valid == nullptr || a.valid[blk * BS + t] != 0));

  float vals[QUANT ? ROWS : 1][8];
  bool rv[ROWS];
  float sum[8], mn[8], mx[8];
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) { sum[j] = 0.0f; mn[j] = INFINITY; mx[j] = -INFINITY; }
#pragma unroll
  for (int i = 0; i < ROWS; ++i) {
    const int r = g + RG * i;
    rv[i] = a.valid == nullptr || a.valid[blk * BS + r] != 0;
    float v[8];
    Vec8<T>::load(x + r * a.stride_t + c * 8, v);
    if (rv[i]) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        sum[j] += v[j];
        if (STATS) { mn[j] = fminf(mn[j], v[j]); mx[j] = fmaxf(mx[j], v[j]); }
        if (QUANT) amax = fmaxf(amax, fabsf(v[j]));
      }
    }
    if (QUANT) {
#pragma unroll
      for (int j = 0; j < 8; ++j) vals[i][j] = v[j];
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    s_sum[g][c * 8 + j] = sum[j];
    if (STATS) { s_min[g][c * 8 + j] = mn[j]; s_max[g][c * 8 + j] = mx[j]; }
  }
  __syncthreads();

  float mean = 0.0f;
  if (t < D) {
    float s = 0.0f, lo = INFINITY, hi = -INFINITY;
#pragma unroll 4
    for (int r = 0; r < RG; ++r) {
      s += s_sum[r][t];
      if (STATS) { lo = fminf(lo, s_min[r][t]); hi = fmaxf(hi, s_max[r][t]); }
    }
    const int64_t o = (bh * a.n_blocks + blk) * D + t;
    if (STATS) {
      if (n_valid == 0) { lo = 0.0f; hi = 0.0f; }
      a.bsum[o] = s;
      a.bmin[o] = lo;
      a.bmax[o] = hi;
    }
    mean = s / static_cast<float>(n_valid > 0 ? n_valid : 1);
  }
  const float norm2 = block_sum(t < D ? mean * mean : 0.0f, s_red);
  if (t < D) {
    const float denom = fmaxf(sqrtf(norm2), 1e-12f);
    a.hat[(bh * a.n_blocks + blk) * D + t] = mean / denom;
  }

  if (QUANT) {
    amax = block_max(amax, s_red);
    const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    const float inv = amax > 0.0f ? 127.0f / amax : 1.0f;
    if (t == 0) a.x_scale[bh * a.n_blocks + blk] = scale;
    int8_t* out = a.x_i8 + (bh * a.n_blocks + blk) * BS * D;
#pragma unroll
    for (int i = 0; i < ROWS; ++i) {
      const int r = g + RG * i;
      uint32_t lo = 0, hi = 0;
      if (rv[i]) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          lo |= (static_cast<uint32_t>(quant_i8(vals[i][j], inv)) & 0xffu) << (8 * j);
          hi |= (static_cast<uint32_t>(quant_i8(vals[i][j + 4], inv)) & 0xffu) << (8 * j);
        }
      }
      *reinterpret_cast<uint2*>(out + r * D + c * 8) = make_uint2(lo, hi);
    }
  }
}

// Cosine scores: one workgroup per (bh, 16 query blocks, 64 key blocks).
template <int D>
__global__ void __launch_bounds__(256)
score_kernel(const float* qhat, const float* khat, int64_t nq, int64_t nk,
             float* score) {
  __shared__ float sq[16][D];
  __shared__ float sk[64][D + 1];
  const int64_t tiles_q = (nq + 15) / 16, tiles_k = (nk + 63) / 64;
  const int64_t tk = blockIdx.x % tiles_k;
  const int64_t tq = (blockIdx.x / tiles_k) % tiles_q;
  const int64_t bh = blockIdx.x / (tiles_k * tiles_q);
  const int t = threadIdx.x;
  const float* qb = qhat + (bh * nq + tq * 16) * D;
  const float* kb = khat + (bh * nk + tk * 64) * D;
  for (int e = t; e < 16 * D; e += 256) {
    const int r = e / D, cc = e % D;
    sq[r][cc] = (tq * 16 + r < nq) ? qb[r * D + cc] : 0.0f;
  }
  for (int e = t; e < 64 * D; e += 256) {
    const int r = e / D, cc = e % D;
    sk[r][cc] = (tk * 64 + r < nk) ? kb[r * D + cc] : 0.0f;
  }
  __syncthreads();
  const int qi = t / 16;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int kj = t % 16 + 16 * u;
    float acc = 0.0f;
#pragma unroll 8
    for (int cc = 0; cc < D; ++cc) acc = fmaf(sq[qi][cc], sk[kj][cc], acc);
    const int64_t gi = tq * 16 + qi, gj = tk * 64 + kj;
    if (gi < nq && gj < nk) score[(bh * nq + gi) * nk + gj] = acc;
  }
}

// Per-head key mean over all valid tokens: kmean = sum_b ksum / n_valid_total.
// One workgroup per head; the block loop is unrolled with independent
// partial sums so that many loads are in flight (the pass is latency bound).
template <int D>
__global__ void __launch_bounds__(256)
kmean_kernel(const float* ksum, const uint8_t* valid, int64_t n_blocks,
             int64_t n_tokens, float* kmean) {
  constexpr int G = 256 / D;
  constexpr int U = 8;
  __shared__ float part[G][D];
  __shared__ float s_red[4];
  const int64_t bh = blockIdx.x;
  const int t = threadIdx.x, c = t % D, g = t / D;
  const float* src = ksum + bh * n_blocks * D + c;
  float acc[U];
#pragma unroll
  for (int u = 0; u < U; ++u) acc[u] = 0.0f;
  int64_t b = g;
  for (; b + (U - 1) * G < n_blocks; b += U * G) {
#pragma unroll
    for (int u = 0; u < U; ++u) acc[u] += src[(b + u * G) * D];
  }
  for (; b < n_blocks; b += G) acc[0] += src[b * D];
  float s = 0.0f;
#pragma unroll
  for (int u = 0; u < U; ++u) s += acc[u];
  part[g][c] = s;
  int cnt = 0;
  if (valid == nullptr) {
    cnt = t == 0 ? static_cast<int>(n_tokens) : 0;
  } else {
    int64_t i = t;
    for (; i + 7 * 256 < n_tokens; i += 8 * 256) {
#pragma unroll
      for (int u = 0; u < 8; ++u) cnt += valid[i + u * 256] != 0;
    }
    for (; i < n_tokens; i += 256) cnt += valid[i] != 0;
  }
  const float total = block_sum(static_cast<float>(cnt), s_red);
  if (t < D) {
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < G; ++i) sum += part[i][t];
    kmean[bh * D + t] = sum / fmaxf(total, 1.0f);
  }
}

// Smoothed per-block key quantiser: one workgroup per (bh, block).
template <typename T, int D, int BS>
__global__ void __launch_bounds__(kPoolThreads)
quant_key_kernel(PoolArgs a, const float* kmean, int8_t* k_i8, float* k_scale) {
  constexpr int CPR = D / 8;
  constexpr int RG = kPoolThreads / CPR;
  constexpr int ROWS = BS / RG;
  __shared__ float s_mean[D];
  __shared__ float s_red[4];
  const int64_t blk = blockIdx.x % a.n_blocks;
  const int64_t bh = blockIdx.x / a.n_blocks;
  const int64_t b_outer = bh / a.n_heads, h = bh % a.n_heads;
  const int t = threadIdx.x;
  const int n_valid = __syncthreads_count(
      t < BS && (a.valid == nullptr || a.valid[blk * BS + t] != 0));
  float dev = 0.0f;
  if (t < D) {
    const float m = kmean[bh * D + t];
    s_mean[t] = m;
    const int64_t o = (bh * a.n_blocks + blk) * D + t;
    dev = fmaxf(a.bmax[o] - m, m - a.bmin[o]);
  }
  const float amax = block_max(dev, s_red);  // also publishes s_mean
  const bool live = n_valid > 0 && amax > 0.0f;
  const float scale = live ? amax / 127.0f : 1.0f;
  const float inv = live ? 127.0f / amax : 1.0f;
  if (t == 0) k_scale[bh * a.n_blocks + blk] = scale;

  const T* x = static_cast<const T*>(a.x) + b_outer * a.stride_b + h * a.stride_h +
               blk * BS * a.stride_t;
  int8_t* out = k_i8 + (bh * a.n_blocks + blk) * BS * D;
  const int c = t % CPR, g = t / CPR;
  float m8[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) m8[j] = s_mean[c * 8 + j];
#pragma unroll
  for (int i = 0; i < ROWS; ++i) {
    const int r = g + RG * i;
    const bool ok = a.valid == nullptr || a.valid[blk * BS + r] != 0;
    float v[8];
    Vec8<T>::load(x + r * a.stride_t + c * 8, v);
    uint32_t lo = 0, hi = 0;
    if (ok) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        lo |= (static_cast<uint32_t>(quant_i8(v[j] - m8[j], inv)) & 0xffu) << (8 * j);
        hi |= (static_cast<uint32_t>(quant_i8(v[j + 4] - m8[j + 4], inv)) & 0xffu) << (8 * j);
      }
    }
    *reinterpret_cast<uint2*>(out + r * D + c * 8) = make_uint2(lo, hi);
  }
}

// ---------------------------------------------------------------------------
// Host-side dispatch.

static int check_pool_shape(int dtype, int64_t batch, int64_t n_heads,
                            int64_t n_blocks, int64_t bs, int64_t d,
                            int64_t stride_b, int64_t stride_h, int64_t stride_t) {
  if (dtype != RCSA_BF16 && dtype != RCSA_F32) return RCSA_ERR_DTYPE;
  if (batch <= 0 || n_heads <= 0 || n_blocks <= 0) return RCSA_ERR_SHAPE;
  if (!(d == 64 || d == 128) || !(bs == 64 || bs == 128)) return RCSA_ERR_SHAPE;
  const int64_t vec = dtype == RCSA_BF16 ? 8 : 4;  // elements per 16 bytes
  if (stride_t % vec || stride_h % vec || stride_b % vec) return RCSA_ERR_STRIDE;
  if (stride_t < d) return RCSA_ERR_STRIDE;
  return RCSA_OK;
}

template <typename T, bool QUANT, bool STATS>
static void launch_pool(const PoolArgs& a, int64_t nbh, int64_t bs, int64_t d,
                        hipStream_t s) {
  dim3 grid(static_cast<unsigned>(nbh * a.n_blocks)), block(kPoolThreads);
  if (d == 128 && bs == 128) pool_kernel<T, 128, 128, QUANT, STATS><<<grid, block, 0, s>>>(a);
  else if (d == 128) pool_kernel<T, 128, 64, QUANT, STATS><<<grid, block, 0, s>>>(a);
  else if (bs == 128) pool_kernel<T, 64, 128, QUANT, STATS><<<grid, block, 0, s>>>(a);
  else pool_kernel<T, 64, 64, QUANT, STATS><<<grid, block, 0, s>>>(a);
}

}  // namespace rcsa

using namespace rcsa;

extern "C" int rcsa_pool_query(const void* q, int dtype, int64_t batch,
                               int64_t n_heads, int64_t n_blocks, int64_t block_size,
                               int64_t head_dim, int64_t stride_b, int64_t stride_h,
                               int64_t stride_t, const uint8_t* valid, float* qhat,
                               int8_t* q_i8, float* q_scale, hipStream_t stream) {
  if (!q || !qhat) return RCSA_ERR_NULL;
  if ((q_i8 == nullptr) != (q_scale == nullptr)) return RCSA_ERR_NULL;
  int st = check_pool_shape(dtype, batch, n_heads, n_blocks, block_size, head_dim,
                            stride_b, stride_h, stride_t);
  if (st) return st;
  if (!aligned16(q) || (q_i8 && (reinterpret_cast<uintptr_t>(q_i8) & 7u)))
    return RCSA_ERR_ALIGN;
  PoolArgs a{q, n_heads, n_blocks, stride_b, stride_h, stride_t, valid, qhat,
             nullptr, nullptr, nullptr, q_i8, q_scale};
  const int64_t nbh = batch * n_heads;
  if (dtype == RCSA_BF16) {
    if (q_i8) launch_pool<u16, true, false>(a, nbh, block_size, head_dim, stream);
    else launch_pool<u16, false, false>(a, nbh, block_size, head_dim, stream);
  } else {
    if (q_i8) launch_pool<float, true, false>(a, nbh, block_size, head_dim, stream);
    else launch_pool<float, false, false>(a, nbh, block_size, head_dim, stream);
  }
  return launch_status();
}

extern "C" int rcsa_pool_key(const void* k, int dtype, int64_t batch, int64_t n_heads,
                             int64_t n_blocks, int64_t block_size, int64_t head_dim,
                             int64_t stride_b, int64_t stride_h, int64_t stride_t,
                             const uint8_t* valid, float* khat, float* ksum,
                             float* kmin, float* kmax, hipStream_t stream) {
  if (!k || !khat) return RCSA_ERR_NULL;
  const bool stats = ksum || kmin || kmax;
  if (stats && !(ksum && kmin && kmax)) return RCSA_ERR_NULL;
  int st = check_pool_shape(dtype, batch, n_heads, n_blocks, block_size, head_dim,
                            stride_b, stride_h, stride_t);
  if (st) return st;
  if (!aligned16(k)) return RCSA_ERR_ALIGN;
  PoolArgs a{k, n_heads, n_blocks, stride_b, stride_h, stride_t, valid, khat,
             ksum, kmin, kmax, nullptr, nullptr};
  const int64_t nbh = batch * n_heads;
  if (dtype == RCSA_BF16) {
    if (stats) launch_pool<u16, false, true>(a, nbh, block_size, head_dim, stream);
    else launch_pool<u16, false, false>(a, nbh, block_size, head_dim, stream);
  } else {
    if (stats) launch_pool<float, false, true>(a, nbh, block_size, head_dim, stream);
    else launch_pool<float, false, false>(a, nbh, block_size, head_dim, stream);
  }
  return launch_status();
}

extern "C" int rcsa_block_scores(const float* qhat, const float* khat, int64_t n_bh,
                                 int64_t n_qblocks, int64_t n_kblocks,
                                 int64_t head_dim, float* score, hipStream_t stream) {
  if (!qhat || !khat || !score) return RCSA_ERR_NULL;
  if (n_bh <= 0 || n_qblocks <= 0 || n_kblocks <= 0) return RCSA_ERR_SHAPE;
  if (!(head_dim == 64 || head_dim == 128)) return RCSA_ERR_SHAPE;
  const int64_t tiles = n_bh * ((n_qblocks + 15) / 16) * ((n_kblocks + 63) / 64);
  dim3 grid(static_cast<unsigned>(tiles)), block(256);
  if (head_dim == 128) score_kernel<128><<<grid, block, 0, stream>>>(qhat, khat, n_qblocks, n_kblocks, score);
  else score_kernel<64><<<grid, block, 0, stream>>>(qhat, khat, n_qblocks, n_kblocks, score);
  return launch_status();
}

extern "C" int rcsa_quantize_key(const void* k, int dtype, int64_t batch,
                                 int64_t n_heads, int64_t n_blocks, int64_t block_size,
                                 int64_t head_dim, int64_t stride_b, int64_t stride_h,
                                 int64_t stride_t, const uint8_t* valid,
                                 const float* ksum, const float* kmin,
                                 const float* kmax, float* kmean, int8_t* k_i8,
                                 float* k_scale, hipStream_t stream) {
  if (!k || !ksum || !kmin || !kmax || !kmean || !k_i8 || !k_scale) return RCSA_ERR_NULL;
  int st = check_pool_shape(dtype, batch, n_heads, n_blocks, block_size, head_dim,
                            stride_b, stride_h, stride_t);
  if (st) return st;
  if (!aligned16(k) || (reinterpret_cast<uintptr_t>(k_i8) & 7u)) return RCSA_ERR_ALIGN;
  const int64_t nbh = batch * n_heads;
  const int64_t n_tokens = n_blocks * block_size;
  if (head_dim == 128) kmean_kernel<128><<<dim3(nbh), dim3(256), 0, stream>>>(ksum, valid, n_blocks, n_tokens, kmean);
  else kmean_kernel<64><<<dim3(nbh), dim3(256), 0, stream>>>(ksum, valid, n_blocks, n_tokens, kmean);
  st = launch_status();
  if (st) return st;
  PoolArgs a{k, n_heads, n_blocks, stride_b, stride_h, stride_t, valid, nullptr,
             const_cast<float*>(ksum), const_cast<float*>(kmin),
             const_cast<float*>(kmax), nullptr, nullptr};
  dim3 grid(static_cast<unsigned>(nbh * n_blocks)), block(kPoolThreads);
#define RCSA_QK(T, D, BS) quant_key_kernel<T, D, BS><<<grid, block, 0, stream>>>(a, kmean, k_i8, k_scale)
  if (dtype == RCSA_BF16) {
    if (head_dim == 128 && block_size == 128) RCSA_QK(u16, 128, 128);
    else if (head_dim == 128) RCSA_QK(u16, 128, 64);
    else if (block_size == 128) RCSA_QK(u16, 64, 128);
    else RCSA_QK(u16, 64, 64);
  } else {
    if (head_dim == 128 && block_size == 128) RCSA_QK(float, 128, 128);
    else if (head_dim == 128) RCSA_QK(float, 128, 64);
    else if (block_size == 128) RCSA_QK(float, 64, 128);
    else RCSA_QK(float, 64, 64);
  }
#undef RCSA_QK
  return launch_status();
}
