// Block pooling, cosine block scores and the int8 Q/K quantiser (gfx950).
//
// All three passes over Q/K are HBM-bound streams: one workgroup owns one
// (head, block) tile of block_size tokens x head_dim channels and reads it
// once with 16-byte coalesced loads (a bf16 row of 128 channels is 16 lanes
// x 16 B).  Per-channel partial sums are combined through LDS.
#include "rcsa_common.h"
#include "select_core.h"

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
  uint32_t* mask;   // per-block validity bits (pool_key only, may be NULL)
  // Gather map (MAP kernels only): packed slot s = blk * BS + r reads token
  // slot_tok[s] of x's token axis (stride_t); -1 or a token >= src_len is an
  // empty slot (invalid, never read).
  const int32_t* slot_tok;
  int64_t src_len;
};

// Source of packed row r of block blk, relative to the tile base (x advanced
// to the block's first row without a map, the (b, h) plane with one): the
// row itself, or through the gather map (an empty slot reads token 0, which
// its validity then drops).
template <bool MAP, int BS>
__device__ __forceinline__ int64_t src_row(const PoolArgs& a, int64_t blk, int r) {
  if constexpr (!MAP) {
    return r;
  } else {
    const int32_t tk = a.slot_tok[blk * BS + r];
    return (tk < 0 || tk >= a.src_len) ? 0 : tk;
  }
}
template <bool MAP, int BS>
__device__ __forceinline__ bool slot_valid(const PoolArgs& a, int64_t blk, int r) {
  bool v = a.valid == nullptr || a.valid[blk * BS + r] != 0;
  if constexpr (MAP) {
    const int32_t tk = a.slot_tok[blk * BS + r];
    v = v && tk >= 0 && tk < a.src_len;
  }
  return v;
}

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

// Sum / min / max of v over the row groups that share a wavefront: lanes
// with the same channel chunk (lane % CPR) are combined by xor shuffles.
template <int CPR>
__device__ __forceinline__ float wave_rows_sum(float v) {
#pragma unroll
  for (int o = CPR; o < kWave; o <<= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
template <int CPR>
__device__ __forceinline__ float wave_rows_min(float v) {
#pragma unroll
  for (int o = CPR; o < kWave; o <<= 1) v = fminf(v, __shfl_xor(v, o, kWave));
  return v;
}
template <int CPR>
__device__ __forceinline__ float wave_rows_max(float v) {
#pragma unroll
  for (int o = CPR; o < kWave; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// Raw 16-byte chunks of a tile row (8 elements): bf16 keeps one uint4, fp32 two.
template <typename T>
struct Raw8;
template <>
struct Raw8<u16> {
  uint4 w;
  __device__ __forceinline__ void load(const u16* p) { w = *reinterpret_cast<const uint4*>(p); }
  // Hide the words from value reuse: a second get() then converts again
  // instead of keeping the first pass's floats alive.
  __device__ __forceinline__ void opaque() {
    asm volatile("" : "+v"(w.x), "+v"(w.y), "+v"(w.z), "+v"(w.w));
  }
  __device__ __forceinline__ void get(float* out) const {
    const uint32_t v[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = __uint_as_float(v[i] << 16);
      out[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
    }
  }
};
template <>
struct Raw8<float> {
  float4 a, b;
  __device__ __forceinline__ void load(const float* p) {
    a = reinterpret_cast<const float4*>(p)[0];
    b = reinterpret_cast<const float4*>(p)[1];
  }
  __device__ __forceinline__ void opaque() {
    asm volatile("" : "+v"(a.x), "+v"(a.y), "+v"(a.z), "+v"(a.w));
    asm volatile("" : "+v"(b.x), "+v"(b.y), "+v"(b.z), "+v"(b.w));
  }
  __device__ __forceinline__ void get(float* out) const {
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
  }
};

// One workgroup per (bh, block).  QUANT: fuse the int8 query quantiser.
// STATS: write sum/min/max for the key quantiser.  Every thread issues all
// its row loads first; the block's validity bytes go through LDS while they
// are in flight, and the per-channel partials are reduced across the row
// groups of a wavefront by shuffles before one small LDS pass.
// NORM false: hat receives the valid-weighted block mean itself (the pooled V
// of P/matrix_curvature_phase_frame_weave.py:5700), not its normalised direction.
template <typename T, int D, int BS, bool QUANT, bool STATS, bool MAP, bool NORM = true>
__device__ __forceinline__ void pool_tile(const PoolArgs& a, int64_t tile) {
  constexpr int CPR = D / 8;                 // 16-byte chunks per token row
  constexpr int RG = kPoolThreads / CPR;     // row groups
  constexpr int ROWS = BS / RG;              // rows per thread
  constexpr int NWV = kPoolThreads / kWave;  // wavefronts
  static_assert(ROWS >= 1 && RG * CPR == kPoolThreads && CPR <= kWave, "tile shape");

  __shared__ float s_sum[NWV][D];
  __shared__ float s_min[STATS ? NWV : 1][D];
  __shared__ float s_max[STATS ? NWV : 1][D];
  __shared__ uint8_t s_valid[BS];
  __shared__ float s_red[4];

  const int64_t blk = tile % a.n_blocks;
  const int64_t bh = tile / a.n_blocks;
  const int64_t b_outer = bh / a.n_heads, h = bh % a.n_heads;
  const T* x = static_cast<const T*>(a.x) + b_outer * a.stride_b + h * a.stride_h +
               (MAP ? 0 : blk * BS * a.stride_t);
  const int t = threadIdx.x;
  const int c = t % CPR, g = t / CPR;
  const int lane = t % kWave, wave = t / kWave;

  Raw8<T> raw[ROWS];
#pragma unroll
  for (int i = 0; i < ROWS; ++i)
    raw[i].load(x + src_row<MAP, BS>(a, blk, g + RG * i) * a.stride_t + c * 8);
  bool tv = false;
  if (t < BS) {
    tv = slot_valid<MAP, BS>(a, blk, t);
    s_valid[t] = tv;
  }
  // validity bits of the block (every head shares them: head 0 writes)
  if (!QUANT && a.mask != nullptr && bh == 0 && t < BS) {
    const uint64_t bits = __ballot(tv);
    if (lane == 0) {
      a.mask[blk * (BS / 32) + 2 * wave] = static_cast<uint32_t>(bits);
      if (BS - 64 * wave > 32) a.mask[blk * (BS / 32) + 2 * wave + 1] = static_cast<uint32_t>(bits >> 32);
    }
  }
  const int n_valid = __syncthreads_count(tv);

  float sum[8], mn[8], mx[8];
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) { sum[j] = 0.0f; mn[j] = INFINITY; mx[j] = -INFINITY; }
#pragma unroll
  for (int i = 0; i < ROWS; ++i) {
    if (s_valid[g + RG * i]) {
      float v[8];
      raw[i].get(v);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        sum[j] += v[j];
        if (STATS) { mn[j] = fminf(mn[j], v[j]); mx[j] = fmaxf(mx[j], v[j]); }
        if (QUANT) amax = fmaxf(amax, fabsf(v[j]));
      }
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    sum[j] = wave_rows_sum<CPR>(sum[j]);
    if (STATS) { mn[j] = wave_rows_min<CPR>(mn[j]); mx[j] = wave_rows_max<CPR>(mx[j]); }
  }
  if (lane < CPR) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      s_sum[wave][c * 8 + j] = sum[j];
      if (STATS) { s_min[wave][c * 8 + j] = mn[j]; s_max[wave][c * 8 + j] = mx[j]; }
    }
  }
  if (QUANT) amax = wave_max(amax);
  if (QUANT && lane == 0) s_red[wave] = amax;
  __syncthreads();

  float mean = 0.0f;
  if (t < D) {
    float s = 0.0f, lo = INFINITY, hi = -INFINITY;
#pragma unroll
    for (int w = 0; w < NWV; ++w) {
      s += s_sum[w][t];
      if (STATS) { lo = fminf(lo, s_min[w][t]); hi = fmaxf(hi, s_max[w][t]); }
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
  if (QUANT) amax = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
  if constexpr (NORM) {
    const float norm2 = block_sum(t < D ? mean * mean : 0.0f, s_red);
    if (t < D) {
      const float denom = fmaxf(sqrtf(norm2), 1e-12f);
      a.hat[(bh * a.n_blocks + blk) * D + t] = mean / denom;
    }
  } else if (t < D) {
    a.hat[(bh * a.n_blocks + blk) * D + t] = mean;
  }

  if (QUANT) {
    const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    const float inv = amax > 0.0f ? 127.0f / amax : 1.0f;
    if (t == 0) a.x_scale[bh * a.n_blocks + blk] = scale;
    int8_t* out = a.x_i8 + (bh * a.n_blocks + blk) * BS * D;
#pragma unroll
    for (int i = 0; i < ROWS; ++i) {
      const int r = g + RG * i;
      uint32_t lo = 0, hi = 0;
      if (s_valid[r]) {
        float v[8];
        raw[i].opaque();
        raw[i].get(v);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          lo |= (static_cast<uint32_t>(quant_i8(v[j], inv)) & 0xffu) << (8 * j);
          hi |= (static_cast<uint32_t>(quant_i8(v[j + 4], inv)) & 0xffu) << (8 * j);
        }
      }
      *reinterpret_cast<uint2*>(out + r * D + c * 8) = make_uint2(lo, hi);
    }
  }
}

template <typename T, int D, int BS, bool QUANT, bool STATS>
__global__ void __launch_bounds__(kPoolThreads)
pool_kernel(PoolArgs a) {
  pool_tile<T, D, BS, QUANT, STATS, false>(a, blockIdx.x);
}

// Query pooling (with its int8 quantiser) and key pooling (with the key
// statistics) in one launch: the first q_tiles workgroups take query tiles,
// the rest key tiles.  The short, latency-bound query pass then runs inside
// the HBM-bound key pass instead of before it.
// (QS false: the bf16 path's pooling, no query quantiser and no key statistics)
// VMEAN: the workgroups past the key tiles (from k_end) pool V tiles into
// their block means (the router's pooled values), in the same launch.
template <typename T, int D, int BS, bool MAP, bool QS = true, bool VMEAN = false>
__global__ void __launch_bounds__(kPoolThreads)
pool_qk_kernel(PoolArgs q, PoolArgs k, int64_t q_tiles, PoolArgs v, int64_t k_end) {
  if (blockIdx.x < q_tiles) pool_tile<T, D, BS, QS, false, MAP>(q, blockIdx.x);
  else if (!VMEAN || blockIdx.x < k_end) pool_tile<T, D, BS, false, QS, MAP>(k, blockIdx.x - q_tiles);
  else pool_tile<T, D, BS, false, false, MAP, false>(v, blockIdx.x - k_end);
}

// Cosine scores: one workgroup per (bh, 16 query blocks, 64 key blocks).
// The tiles are loaded with 16-byte loads, all issued before the LDS stores.
template <int D>
__global__ void __launch_bounds__(256)
score_kernel(const float* qhat, const float* khat, int64_t nq, int64_t nk,
             float* score) {
  __shared__ float sq[16][D];
  __shared__ float sk[64][D + 1];
  constexpr int C4 = D / 4;                      // float4 per row
  constexpr int QL = 16 * C4 / 256;              // float4 loads per thread (query tile)
  constexpr int KL = 64 * C4 / 256;              // (key tile)
  const int64_t tiles_q = (nq + 15) / 16, tiles_k = (nk + 63) / 64;
  const int64_t tk = blockIdx.x % tiles_k;
  const int64_t tq = (blockIdx.x / tiles_k) % tiles_q;
  const int64_t bh = blockIdx.x / (tiles_k * tiles_q);
  const int t = threadIdx.x;
  const float4* qb = reinterpret_cast<const float4*>(qhat + (bh * nq + tq * 16) * D);
  const float4* kb = reinterpret_cast<const float4*>(khat + (bh * nk + tk * 64) * D);
  // rows past the end re-read the last row (then zeroed): every load is in bounds
  float4 qv[QL], kv[KL];
  const int q_last = static_cast<int>(min<int64_t>(nq - tq * 16, 16)) - 1;
  const int k_last = static_cast<int>(min<int64_t>(nk - tk * 64, 64)) - 1;
#pragma unroll
  for (int i = 0; i < QL; ++i) {
    const int e = t + 256 * i, r = e / C4;
    qv[i] = qb[min(r, q_last) * C4 + e % C4];
    if (r > q_last) qv[i] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
#pragma unroll
  for (int i = 0; i < KL; ++i) {
    const int e = t + 256 * i, r = e / C4;
    kv[i] = kb[min(r, k_last) * C4 + e % C4];
    if (r > k_last) kv[i] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
#pragma unroll
  for (int i = 0; i < QL; ++i) {
    const int e = t + 256 * i, r = e / C4, cc = (e % C4) * 4;
    sq[r][cc] = qv[i].x; sq[r][cc + 1] = qv[i].y; sq[r][cc + 2] = qv[i].z; sq[r][cc + 3] = qv[i].w;
  }
#pragma unroll
  for (int i = 0; i < KL; ++i) {
    const int e = t + 256 * i, r = e / C4, cc = (e % C4) * 4;
    sk[r][cc] = kv[i].x; sk[r][cc + 1] = kv[i].y; sk[r][cc + 2] = kv[i].z; sk[r][cc + 3] = kv[i].w;
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

// Number of nonzero bytes of a 32-bit word.
__device__ __forceinline__ int nonzero_bytes(uint32_t w) {
  return __popc((((w & 0x7f7f7f7fu) + 0x7f7f7f7fu) | w) & 0x80808080u);
}

// Per-head key mean over all valid tokens: kmean = sum_b ksum / n_valid_total.
// One workgroup per (bh, 16 channels): 16 block lanes per channel, each with
// four independent partial sums, then an LDS reduction.  The valid-token
// count is taken with 16-byte loads.
template <int D>
__global__ void __launch_bounds__(256)
kmean_kernel(const float* ksum, const uint8_t* valid, const int32_t* slot_tok,
             int64_t src_len, int64_t n_blocks, int64_t n_tokens, float* kmean) {
  constexpr int CG = 16;          // channels per workgroup
  constexpr int BL = 256 / CG;    // block lanes
  __shared__ float part[BL][CG + 1];
  __shared__ float s_red[4];
  const int64_t bh = blockIdx.x / (D / CG);
  const int c0 = static_cast<int>(blockIdx.x % (D / CG)) * CG;
  const int t = threadIdx.x, c = t % CG, bl = t / CG;
  const float* src = ksum + bh * n_blocks * D + c0 + c;
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  int64_t b = bl;
  // sixteen loads in flight per pass; the adds keep the four chains' order
  for (; b + 15 * BL < n_blocks; b += 16 * BL) {
    float v[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = src[(b + k * BL) * D];
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[u] += v[4 * g + u];
  }
  for (; b + 3 * BL < n_blocks; b += 4 * BL) {
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[u] += src[(b + u * BL) * D];
  }
  for (; b < n_blocks; b += BL) acc[0] += src[b * D];
  part[bl][c] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  int cnt = 0;
  if (slot_tok != nullptr) {  // gathered keys: a slot counts when it holds a token
    // four slots per 16-byte load (and their four validity bytes per word),
    // eight loads in flight per thread
    const uint32_t src = static_cast<uint32_t>(src_len);
    const bool vec = (reinterpret_cast<uintptr_t>(slot_tok) & 15u) == 0 &&
                     (valid == nullptr || (reinterpret_cast<uintptr_t>(valid) & 3u) == 0);
    const int64_t n4 = vec ? n_tokens / 4 : 0;
    const int4* s4 = reinterpret_cast<const int4*>(slot_tok);
    const uint32_t* v4 = reinterpret_cast<const uint32_t*>(valid);
    auto count4 = [&](int4 w, uint32_t vb) {
      return static_cast<int>(static_cast<uint32_t>(w.x) < src && (vb & 0xffu)) +
             static_cast<int>(static_cast<uint32_t>(w.y) < src && (vb & 0xff00u)) +
             static_cast<int>(static_cast<uint32_t>(w.z) < src && (vb & 0xff0000u)) +
             static_cast<int>(static_cast<uint32_t>(w.w) < src && (vb & 0xff000000u));
    };
    int64_t i0 = t;
    for (; i0 + 7 * 256 < n4; i0 += 8 * 256) {
      int4 w[8];
      uint32_t vb[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        w[k] = s4[i0 + k * 256];
        vb[k] = valid == nullptr ? 0xffffffffu : v4[i0 + k * 256];
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) cnt += count4(w[k], vb[k]);
    }
    for (; i0 < n4; i0 += 256)
      cnt += count4(s4[i0], valid == nullptr ? 0xffffffffu : v4[i0]);
    for (int64_t i = n4 * 4 + t; i < n_tokens; i += 256) {
      const int32_t tk = slot_tok[i];
      cnt += tk >= 0 && tk < src_len && (valid == nullptr || valid[i] != 0);
    }
  } else if (valid == nullptr) {
    cnt = t == 0 ? static_cast<int>(n_tokens) : 0;
  } else if ((reinterpret_cast<uintptr_t>(valid) & 15u) == 0) {
    const int64_t n16 = n_tokens / 16;
    const uint4* v4 = reinterpret_cast<const uint4*>(valid);
    int64_t i0 = t;
    for (; i0 + 3 * 256 < n16; i0 += 4 * 256) {  // four 16-byte loads in flight
      uint4 w[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) w[k] = v4[i0 + k * 256];
#pragma unroll
      for (int k = 0; k < 4; ++k)
        cnt += nonzero_bytes(w[k].x) + nonzero_bytes(w[k].y) + nonzero_bytes(w[k].z) +
               nonzero_bytes(w[k].w);
    }
    for (int64_t i = i0; i < n16; i += 256) {
      const uint4 w = v4[i];
      cnt += nonzero_bytes(w.x) + nonzero_bytes(w.y) + nonzero_bytes(w.z) + nonzero_bytes(w.w);
    }
    for (int64_t i = n16 * 16 + t; i < n_tokens; i += 256) cnt += valid[i] != 0;
  } else {
    for (int64_t i = t; i < n_tokens; i += 256) cnt += valid[i] != 0;
  }
  const float total = block_sum(static_cast<float>(cnt), s_red);  // also publishes part
  if (t < CG) {
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < BL; ++i) sum += part[i][t];
    kmean[bh * D + c0 + t] = sum / fmaxf(total, 1.0f);
  }
}

// Smoothed per-block key quantiser: one workgroup per (bh, block).  The tile
// loads are issued first; the scale (from the block's min/max and the head
// mean) is computed while they are in flight.
template <typename T, int D, int BS, bool MAP>
__device__ __forceinline__ void quant_tile(const PoolArgs& a, const float* kmean, int8_t* k_i8,
                                           float* k_scale, int64_t tile) {
  constexpr int CPR = D / 8;
  constexpr int RG = kPoolThreads / CPR;
  constexpr int ROWS = BS / RG;
  __shared__ float s_mean[D];
  __shared__ uint8_t s_valid[BS];
  __shared__ float s_red[4];
  const int64_t blk = tile % a.n_blocks;
  const int64_t bh = tile / a.n_blocks;
  const int64_t b_outer = bh / a.n_heads, h = bh % a.n_heads;
  const int t = threadIdx.x;
  const int c = t % CPR, g = t / CPR;
  const T* x = static_cast<const T*>(a.x) + b_outer * a.stride_b + h * a.stride_h +
               (MAP ? 0 : blk * BS * a.stride_t);
  Raw8<T> raw[ROWS];
#pragma unroll
  for (int i = 0; i < ROWS; ++i)
    raw[i].load(x + src_row<MAP, BS>(a, blk, g + RG * i) * a.stride_t + c * 8);
  bool tv = false;
  if (t < BS) {
    tv = slot_valid<MAP, BS>(a, blk, t);
    s_valid[t] = tv;
  }
  float dev = 0.0f;
  if (t < D) {
    const float m = kmean[bh * D + t];
    s_mean[t] = m;
    const int64_t o = (bh * a.n_blocks + blk) * D + t;
    dev = fmaxf(a.bmax[o] - m, m - a.bmin[o]);
  }
  const int n_valid = __syncthreads_count(tv);
  const float amax = block_max(dev, s_red);  // also publishes s_mean / s_valid
  const bool live = n_valid > 0 && amax > 0.0f;
  const float scale = live ? amax / 127.0f : 1.0f;
  const float inv = live ? 127.0f / amax : 1.0f;
  if (t == 0) k_scale[bh * a.n_blocks + blk] = scale;

  int8_t* out = k_i8 + (bh * a.n_blocks + blk) * BS * D;
  float m8[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) m8[j] = s_mean[c * 8 + j];
#pragma unroll
  for (int i = 0; i < ROWS; ++i) {
    const int r = g + RG * i;
    uint32_t lo = 0, hi = 0;
    if (s_valid[r]) {
      float v[8];
      raw[i].get(v);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        lo |= (static_cast<uint32_t>(quant_i8(v[j] - m8[j], inv)) & 0xffu) << (8 * j);
        hi |= (static_cast<uint32_t>(quant_i8(v[j + 4] - m8[j + 4], inv)) & 0xffu) << (8 * j);
      }
    }
    // non-temporal: the int8 keys are read back only by the attention, after
    // this pass, so they need not displace cached lines of the key passes
    // (layer call at 3520 q x 38,720 kv, 24 heads: 0.502 against 0.509 ms)
    const v2u packed = {lo, hi};
    __builtin_nontemporal_store(packed, reinterpret_cast<v2u*>(out + r * D + c * 8));
  }
}

template <typename T, int D, int BS, bool MAP>
__global__ void __launch_bounds__(kPoolThreads)
quant_key_kernel(PoolArgs a, const float* kmean, int8_t* k_i8, float* k_scale) {
  quant_tile<T, D, BS, MAP>(a, kmean, k_i8, k_scale, blockIdx.x);
}

// The key quantiser and the block scores + top-k selection in one launch: the
// first n_sel workgroups each score and select kSelWaves rows (latency-bound
// work that then runs inside the HBM-bound key pass), the rest quantise key
// tiles.  No reference counterpart; replaces a side stream and its two
// cross-stream waits.
template <typename T, int D, int BS, bool MAP, int PER>
__global__ void __launch_bounds__(kPoolThreads)
quant_select_kernel(PoolArgs a, const float* kmean, int8_t* k_i8, float* k_scale, SelArgs sel,
                    int64_t n_sel) {
  static_assert(kSelWaves * kWave == kPoolThreads, "one block shape");
  if (blockIdx.x < n_sel) select_rows<PER, false, true>(sel, blockIdx.x, nullptr);
  else quant_tile<T, D, BS, MAP>(a, kmean, k_i8, k_scale, blockIdx.x - n_sel);
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
             nullptr, nullptr, nullptr, q_i8, q_scale, nullptr, nullptr, 0};
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
                             float* kmin, float* kmax, uint32_t* block_mask,
                             hipStream_t stream) {
  if (!k || !khat) return RCSA_ERR_NULL;
  const bool stats = ksum || kmin || kmax;
  if (stats && !(ksum && kmin && kmax)) return RCSA_ERR_NULL;
  int st = check_pool_shape(dtype, batch, n_heads, n_blocks, block_size, head_dim,
                            stride_b, stride_h, stride_t);
  if (st) return st;
  if (!aligned16(k)) return RCSA_ERR_ALIGN;
  if (block_mask && (reinterpret_cast<uintptr_t>(block_mask) & 7u)) return RCSA_ERR_ALIGN;
  PoolArgs a{k, n_heads, n_blocks, stride_b, stride_h, stride_t, valid, khat,
             ksum, kmin, kmax, nullptr, nullptr, block_mask, nullptr, 0};
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

static int pool_query_key_impl(
    const void* q, const void* k, int dtype, int64_t batch, int64_t n_heads,
    int64_t n_qblocks, int64_t n_kblocks, int64_t block_size, int64_t head_dim,
    int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_t, int64_t k_stride_b,
    int64_t k_stride_h, int64_t k_stride_t, const uint8_t* q_valid, const uint8_t* k_valid,
    const int32_t* q_slot_token, int64_t q_src_len, const int32_t* k_slot_token,
    int64_t k_src_len, float* qhat, int8_t* q_i8, float* q_scale, float* khat, float* ksum,
    float* kmin, float* kmax, uint32_t* block_mask, const void* v, int64_t v_stride_b,
    int64_t v_stride_h, int64_t v_stride_t, float* vmean, hipStream_t stream) {
  if (!q || !k || !qhat || !khat) return RCSA_ERR_NULL;
  if ((v == nullptr) != (vmean == nullptr)) return RCSA_ERR_NULL;
  // the quantiser outputs and the key statistics come together or not at all
  const bool qs = q_i8 || q_scale || ksum || kmin || kmax;
  if (qs && !(q_i8 && q_scale && ksum && kmin && kmax)) return RCSA_ERR_NULL;
  // both gathered or neither (one kernel instance serves both tile kinds)
  if ((q_slot_token == nullptr) != (k_slot_token == nullptr)) return RCSA_ERR_NULL;
  const bool map = q_slot_token != nullptr;
  if (map && (q_src_len <= 0 || k_src_len <= 0 || q_src_len >= (int64_t{1} << 31) ||
              k_src_len >= (int64_t{1} << 31)))
    return RCSA_ERR_SHAPE;
  int st = check_pool_shape(dtype, batch, n_heads, n_qblocks, block_size, head_dim,
                            q_stride_b, q_stride_h, q_stride_t);
  if (st) return st;
  st = check_pool_shape(dtype, batch, n_heads, n_kblocks, block_size, head_dim, k_stride_b,
                        k_stride_h, k_stride_t);
  if (st) return st;
  if (v) {  // V: the key layout (slot map, validity, blocks), strides of its own
    st = check_pool_shape(dtype, batch, n_heads, n_kblocks, block_size, head_dim, v_stride_b,
                          v_stride_h, v_stride_t);
    if (st) return st;
    if (!aligned16(v) || !aligned16(vmean)) return RCSA_ERR_ALIGN;
  }
  if (!aligned16(q) || !aligned16(k) || (reinterpret_cast<uintptr_t>(q_i8) & 7u))
    return RCSA_ERR_ALIGN;
  if (block_mask && (reinterpret_cast<uintptr_t>(block_mask) & 7u)) return RCSA_ERR_ALIGN;
  const PoolArgs qa{q, n_heads, n_qblocks, q_stride_b, q_stride_h, q_stride_t, q_valid, qhat,
                    nullptr, nullptr, nullptr, q_i8, q_scale, nullptr, q_slot_token,
                    q_src_len};
  const PoolArgs ka{k, n_heads, n_kblocks, k_stride_b, k_stride_h, k_stride_t, k_valid, khat,
                    ksum, kmin, kmax, nullptr, nullptr, block_mask, k_slot_token, k_src_len};
  const PoolArgs va{v, n_heads, n_kblocks, v_stride_b, v_stride_h, v_stride_t, k_valid, vmean,
                    nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, k_slot_token,
                    k_src_len};
  const int64_t nbh = batch * n_heads;
  const int64_t q_tiles = nbh * n_qblocks;
  const int64_t k_end = q_tiles + nbh * n_kblocks;
  const dim3 grid(static_cast<unsigned>(k_end + (v ? nbh * n_kblocks : 0))), block(kPoolThreads);
#define RCSA_PQK(T_, D_, BS_)                                                     \
  if (v) {                                                                        \
    if (!qs) { if (map) pool_qk_kernel<T_, D_, BS_, true, false, true><<<grid, block, 0, stream>>>(qa, ka, q_tiles, va, k_end); \
               else pool_qk_kernel<T_, D_, BS_, false, false, true><<<grid, block, 0, stream>>>(qa, ka, q_tiles, va, k_end); } \
    else if (map) pool_qk_kernel<T_, D_, BS_, true, true, true><<<grid, block, 0, stream>>>(qa, ka, q_tiles, va, k_end); \
    else pool_qk_kernel<T_, D_, BS_, false, true, true><<<grid, block, 0, stream>>>(qa, ka, q_tiles, va, k_end); \
  } else if (!qs) { if (map) pool_qk_kernel<T_, D_, BS_, true, false><<<grid, block, 0, stream>>>(qa, ka, q_tiles, va, k_end); \
             else pool_qk_kernel<T_, D_, BS_, false, false><<<grid, block, 0, stream>>>(qa, ka, q_tiles, va, k_end); } \
  else if (map) pool_qk_kernel<T_, D_, BS_, true><<<grid, block, 0, stream>>>(qa, ka, q_tiles, va, k_end); \
  else pool_qk_kernel<T_, D_, BS_, false><<<grid, block, 0, stream>>>(qa, ka, q_tiles, va, k_end)
#define RCSA_PQK_T(T_)                                               \
  if (head_dim == 128 && block_size == 128) { RCSA_PQK(T_, 128, 128); } \
  else if (head_dim == 128) { RCSA_PQK(T_, 128, 64); }                  \
  else if (block_size == 128) { RCSA_PQK(T_, 64, 128); }                \
  else { RCSA_PQK(T_, 64, 64); }
  if (dtype == RCSA_BF16) { RCSA_PQK_T(u16) } else { RCSA_PQK_T(float) }
#undef RCSA_PQK_T
#undef RCSA_PQK
  return launch_status();
}

extern "C" int rcsa_pool_query_key(
    const void* q, const void* k, int dtype, int64_t batch, int64_t n_heads,
    int64_t n_qblocks, int64_t n_kblocks, int64_t block_size, int64_t head_dim,
    int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_t, int64_t k_stride_b,
    int64_t k_stride_h, int64_t k_stride_t, const uint8_t* q_valid, const uint8_t* k_valid,
    const int32_t* q_slot_token, int64_t q_src_len, const int32_t* k_slot_token,
    int64_t k_src_len, float* qhat, int8_t* q_i8, float* q_scale, float* khat, float* ksum,
    float* kmin, float* kmax, uint32_t* block_mask, hipStream_t stream) {
  return pool_query_key_impl(q, k, dtype, batch, n_heads, n_qblocks, n_kblocks, block_size,
                             head_dim, q_stride_b, q_stride_h, q_stride_t, k_stride_b,
                             k_stride_h, k_stride_t, q_valid, k_valid, q_slot_token, q_src_len,
                             k_slot_token, k_src_len, qhat, q_i8, q_scale, khat, ksum, kmin,
                             kmax, block_mask, nullptr, 0, 0, 0, nullptr, stream);
}

extern "C" int rcsa_pool_query_key_value(
    const void* q, const void* k, const void* v, int dtype, int64_t batch, int64_t n_heads,
    int64_t n_qblocks, int64_t n_kblocks, int64_t block_size, int64_t head_dim,
    int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_t, int64_t k_stride_b,
    int64_t k_stride_h, int64_t k_stride_t, int64_t v_stride_b, int64_t v_stride_h,
    int64_t v_stride_t, const uint8_t* q_valid, const uint8_t* k_valid,
    const int32_t* q_slot_token, int64_t q_src_len, const int32_t* k_slot_token,
    int64_t k_src_len, float* qhat, int8_t* q_i8, float* q_scale, float* khat, float* ksum,
    float* kmin, float* kmax, uint32_t* block_mask, float* vmean, hipStream_t stream) {
  if (!v || !vmean) return RCSA_ERR_NULL;
  return pool_query_key_impl(q, k, dtype, batch, n_heads, n_qblocks, n_kblocks, block_size,
                             head_dim, q_stride_b, q_stride_h, q_stride_t, k_stride_b,
                             k_stride_h, k_stride_t, q_valid, k_valid, q_slot_token, q_src_len,
                             k_slot_token, k_src_len, qhat, q_i8, q_scale, khat, ksum, kmin,
                             kmax, block_mask, v, v_stride_b, v_stride_h, v_stride_t, vmean,
                             stream);
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

// The key mean, then the quantiser (with sel: fused with the scores + top-k).
static int quantize_key_impl(const void* k, int dtype, int64_t batch, int64_t n_heads,
                             int64_t n_blocks, int64_t block_size, int64_t head_dim,
                             int64_t stride_b, int64_t stride_h, int64_t stride_t,
                             const uint8_t* valid, const int32_t* slot_token, int64_t src_len,
                             const float* ksum, const float* kmin, const float* kmax,
                             float* kmean, int8_t* k_i8, float* k_scale, const SelArgs* sel,
                             hipStream_t stream) {
  if (!k || !ksum || !kmin || !kmax || !kmean || !k_i8 || !k_scale) return RCSA_ERR_NULL;
  // the fused launch exists for the layer call's shape only
  if (sel && !(dtype == RCSA_BF16 && head_dim == 128 && block_size == 128 && n_blocks <= 1024))
    return RCSA_ERR_SHAPE;
  if (slot_token && (src_len <= 0 || src_len >= (int64_t{1} << 31))) return RCSA_ERR_SHAPE;
  int st = check_pool_shape(dtype, batch, n_heads, n_blocks, block_size, head_dim,
                            stride_b, stride_h, stride_t);
  if (st) return st;
  if (!aligned16(k) || (reinterpret_cast<uintptr_t>(k_i8) & 7u)) return RCSA_ERR_ALIGN;
  const int64_t nbh = batch * n_heads;
  const int64_t n_tokens = n_blocks * block_size;
  if (head_dim == 128)
    kmean_kernel<128><<<dim3(nbh * 8), dim3(256), 0, stream>>>(ksum, valid, slot_token, src_len,
                                                               n_blocks, n_tokens, kmean);
  else
    kmean_kernel<64><<<dim3(nbh * 4), dim3(256), 0, stream>>>(ksum, valid, slot_token, src_len,
                                                              n_blocks, n_tokens, kmean);
  st = launch_status();
  if (st) return st;
  PoolArgs a{k, n_heads, n_blocks, stride_b, stride_h, stride_t, valid, nullptr,
             const_cast<float*>(ksum), const_cast<float*>(kmin),
             const_cast<float*>(kmax), nullptr, nullptr, nullptr, slot_token, src_len};
  dim3 block(kPoolThreads);
  if (sel) {
    const int64_t n_sel = (sel->n_rows + kSelWaves - 1) / kSelWaves;
    dim3 grid(static_cast<unsigned>(n_sel + nbh * n_blocks));
#define RCSA_QS(MAP, PER) \
  quant_select_kernel<u16, 128, 128, MAP, PER><<<grid, block, 0, stream>>>(a, kmean, k_i8, k_scale, *sel, n_sel)
    if (n_blocks <= 512) {
      if (slot_token) RCSA_QS(true, 8); else RCSA_QS(false, 8);
    } else {
      if (slot_token) RCSA_QS(true, 16); else RCSA_QS(false, 16);
    }
#undef RCSA_QS
    return launch_status();
  }
  dim3 grid(static_cast<unsigned>(nbh * n_blocks));
#define RCSA_QK(T, D, BS)                                                                   \
  do {                                                                                      \
    if (slot_token) quant_key_kernel<T, D, BS, true><<<grid, block, 0, stream>>>(a, kmean, k_i8, k_scale); \
    else quant_key_kernel<T, D, BS, false><<<grid, block, 0, stream>>>(a, kmean, k_i8, k_scale); \
  } while (0)
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

extern "C" int rcsa_quantize_key(const void* k, int dtype, int64_t batch,
                                 int64_t n_heads, int64_t n_blocks, int64_t block_size,
                                 int64_t head_dim, int64_t stride_b, int64_t stride_h,
                                 int64_t stride_t, const uint8_t* valid,
                                 const int32_t* slot_token, int64_t src_len,
                                 const float* ksum, const float* kmin,
                                 const float* kmax, float* kmean, int8_t* k_i8,
                                 float* k_scale, hipStream_t stream) {
  return quantize_key_impl(k, dtype, batch, n_heads, n_blocks, block_size, head_dim, stride_b,
                           stride_h, stride_t, valid, slot_token, src_len, ksum, kmin, kmax,
                           kmean, k_i8, k_scale, nullptr, stream);
}

extern "C" int rcsa_quantize_key_select(
    const void* k, int dtype, int64_t batch, int64_t n_heads, int64_t n_blocks,
    int64_t block_size, int64_t head_dim, int64_t stride_b, int64_t stride_h, int64_t stride_t,
    const uint8_t* valid, const int32_t* slot_token, int64_t src_len, const float* ksum,
    const float* kmin, const float* kmax, float* kmean, int8_t* k_i8, float* k_scale,
    const float* qhat, const float* khat, int64_t n_qblocks, float* score,
    const int32_t* row_k, int64_t row_k_stride_bh, int64_t k_fixed, const uint8_t* forced,
    const uint8_t* allowed, int64_t mask_stride_bh, int32_t* indices, int64_t max_k,
    int32_t* counts, hipStream_t stream) {
  if (!qhat || !khat || !score || !indices || !counts) return RCSA_ERR_NULL;
  if (n_qblocks <= 0 || max_k <= 0 || batch <= 0 || n_heads <= 0) return RCSA_ERR_SHAPE;
  if (mask_stride_bh < 0 || row_k_stride_bh < 0) return RCSA_ERR_STRIDE;
  if (!aligned16(qhat) || !aligned16(khat)) return RCSA_ERR_ALIGN;
  if (head_dim != 128) return RCSA_ERR_SHAPE;  // the fused scores are unrolled for 128
  const SelArgs sel{score, batch * n_heads * n_qblocks, n_qblocks, n_blocks, row_k,
                    row_k_stride_bh, k_fixed, forced, allowed, mask_stride_bh, indices, max_k,
                    counts, qhat, khat, head_dim};
  return quantize_key_impl(k, dtype, batch, n_heads, n_blocks, block_size, head_dim, stride_b,
                           stride_h, stride_t, valid, slot_token, src_len, ksum, kmin, kmax,
                           kmean, k_i8, k_scale, &sel, stream);
}
