// Shared int8 Q/K/V projection (gfx950): one per-token int8 quantisation of
// the activations, then int8 GEMMs with a dequantising epilogue.
//
// quant_rows_kernel: one wavefront per token row; scale = absmax / 127 (1 for
// an all-zero row), q = rne(x * 127 / absmax) clamped to [-127, 127].
//
// int8_linear_kernel: out[m][n] = bf16(bf16(acc * xs[m] * ws[n]) + bias[n]),
// acc = sum_k x[m][k] w[n][k] in int32.  A workgroup (8 wavefronts, one per CU)
// computes a 256 (tokens) x 256 (channels) tile; each wavefront 64 x 128 as
// 2 x 4 tiles of v_mfma_i32_32x32x32_i8 with the weights as the A operand, so a
// lane ends up holding one token and runs of 4 consecutive channels; lanes l and
// l + 32 swap halves (v_permlane32_swap) so that each stores 8 consecutive
// channels (16 bytes).  Both operands are staged by direct-to-LDS copies through
// a 2-slot ring of 128-byte K steps (64 KiB per slot), so every row a copy reads
// is one whole 128-byte line (half as many L2 requests as 64-byte steps);
// 16-byte chunks of each 128-byte row are XORed by (row / 2) mod 8 so the
// ds_read_b128 operand reads are conflict free.  When the 256 x 256 tiles would
// end in a short round, the rows of that round run as 128 x 128 tiles (each
// wavefront 32 x 64) of the same launch, taken first.  The launch is
// persistent: one workgroup per compute unit walks its XCD's tiles, and the
// copy ring runs on from one 256 x 256 tile to the next, so a tile's first
// copies fly during the previous tile's epilogue (at 38,720 x 3072 x 3072:
// 0.396-0.407 against 0.415-0.421 ms with one workgroup per tile, interleaved
// on one box; holding half of each output tile in registers to store it
// beside the next tile's first MFMAs gained nothing more).
#include <type_traits>

#include "rcsa_common.h"

#define RCSA_QKV_LDS(T, p) ((__attribute__((address_space(3))) T*)(p))

namespace rcsa {

constexpr int kQThreads = 256;       // quantiser: 4 rows per workgroup
constexpr int kGemmThreads = 512;    // 8 wavefronts: 4 (tokens) x 2 (channels)
constexpr int kKS = 128;             // bytes of K per ring step (one 128-byte line per row)

template <typename T>
__device__ __forceinline__ float to_f32(T v) {
  if constexpr (std::is_same<T, float>::value) return v;
  else return bf16_to_f32(v);
}

template <typename T>
__global__ void __launch_bounds__(kQThreads)
quant_rows_kernel(const T* x, int64_t M, int64_t C, int64_t ldx, int8_t* q, float* scale) {
  const int lane = threadIdx.x % kWave;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (kQThreads / kWave) + threadIdx.x / kWave;
  if (row >= M) return;
  const T* xr = x + row * ldx;
  float amax = 0.0f;
  for (int64_t c = lane * 8; c < C; c += kWave * 8) {
    float v[8];
    Vec8<T>::load(xr + c, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
  }
  amax = wave_max(amax);
  const float inv = amax > 0.0f ? 127.0f / amax : 1.0f;
  if (lane == 0) scale[row] = amax > 0.0f ? amax / 127.0f : 1.0f;
  int8_t* qr = q + row * C;
  for (int64_t c = lane * 8; c < C; c += kWave * 8) {
    float v[8];
    Vec8<T>::load(xr + c, v);
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      lo |= (static_cast<uint32_t>(quant_i8(v[j], inv)) & 0xffu) << (8 * j);
      hi |= (static_cast<uint32_t>(quant_i8(v[j + 4], inv)) & 0xffu) << (8 * j);
    }
    *reinterpret_cast<uint2*>(qr + c) = make_uint2(lo, hi);
  }
}

struct LinearArgs {
  const int8_t* x;      // [M, K]
  const float* xs;      // [M]
  const int8_t* w;      // [N, K]
  const float* ws;      // [N]
  const u16* bias;      // [N] bf16 or NULL
  u16* out;             // [M, ldo] bf16
  int64_t M, N, K, ldo;
  // 256 x 256 tiles over rows [0, big_rows), 128 x 128 tiles over [big_rows, M)
  int64_t big_rows;
};

constexpr int kQkvRsrc3 = 0x00020000;  // raw untyped buffer, 32-bit data format

__device__ __forceinline__ void dma16(const int8_t* base, int bytes, uint32_t voff, int soff,
                                      char* dst) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(base), 0, bytes, kQkvRsrc3);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, RCSA_QKV_LDS(void, dst), 16, voff, soff, 0, 0);
}

// chunk XOR of a 128-byte row: (row / 2) mod 8
__device__ __forceinline__ int qkv_swz(int row) { return (row >> 1) & 7; }

// s_waitcnt immediate for vmcnt <= n only (gfx9 encoding)
constexpr int qkv_vmcnt(int n) {
  return (n & 0xf) | (0x7 << 4) | (0xf << 8) | (((n >> 4) & 0x3) << 14);
}

template <int N>
__device__ __forceinline__ void qkv_wait_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

// A workgroup tile of 8 wavefronts (4 along tokens x 2 along channels), each
// TMT x TNT tiles of 32 x 32.
template <int TMT, int TNT>
struct LinTile {
  static constexpr int BM = 4 * 32 * TMT, BN = 2 * 32 * TNT;
  static constexpr int XB = BM * kKS, WB = BN * kKS;          // bytes of a ring step
  static constexpr int XU = XB / 1024 / 8, WU = WB / 1024 / 8;  // 1 KiB copy units per wavefront
  static constexpr int OPS = XU + WU;                         // copies per wavefront and step
  static constexpr int KS = kKS / 32;                         // MFMA k-steps per ring step
  static_assert(XU == WU && XU >= 1, "both tiles are copied by the same rows");
};

using BigTile = LinTile<2, 4>;    // 256 x 256, each wavefront 64 x 128
using SmallTile = LinTile<1, 2>;  // 128 x 128, each wavefront 32 x 64

// The per-lane pieces of a tile shape: copy offsets, operand offsets, the
// k-step's copies and MFMAs, and the dequantising epilogue.
template <int TMT, int TNT>
struct LinLane {
  using T = LinTile<TMT, TNT>;
  int wave, wm, wn, hf, li;
  uint32_t off[T::XU];  // copies: the same rows of both tiles
  // Operand offsets.  Row 32 i + li of a wavefront's rows has the chunk
  // swizzle (li / 2) mod 8 for every i (the rows differ above bit 4), so its
  // 32-row tiles sit 4 KiB apart and one lane offset per k-step serves them
  // all (the 4 KiB steps become instruction immediates).
  int xk[T::KS], wk[T::KS];

  __device__ __forceinline__ explicit LinLane(const LinearArgs& a) {
    const int t = threadIdx.x;
    const int lane = t % kWave;
    wave = __builtin_amdgcn_readfirstlane(t / kWave);
    wm = wave & 3;
    wn = wave >> 2;
    hf = lane >> 5;
    li = lane & 31;
    // each tile is units of 1 KiB (8 rows of 128 bytes); lane l lands at row
    // 8 u + l / 8, chunk l % 8 of its unit and loads the chunk that the
    // swizzle puts there
#pragma unroll
    for (int i = 0; i < T::XU; ++i) {
      const int r = (wave * T::XU + i) * 8 + lane / 8;
      off[i] = static_cast<uint32_t>(r * a.K + ((lane & 7) ^ qkv_swz(r)) * 16);
    }
#pragma unroll
    for (int ks = 0; ks < T::KS; ++ks) {
      const int c = ((ks * 2 + hf) ^ qkv_swz(li)) * 16;
      xk[ks] = (wm * 32 * TMT + li) * kKS + c;
      wk[ks] = T::XB + (wn * 32 * TNT + li) * kKS + c;
    }
  }

  // The copies of k-step s of the operand rows at xb (xbytes readable) and wb
  // (wbytes readable) into dst.  Ranges of 0 bytes read nothing.
  __device__ __forceinline__ void stage(const int8_t* xb, int xbytes, const int8_t* wb,
                                        int wbytes, int s, char* dst) const {
    const int k0 = s * kKS;
#pragma unroll
    for (int i = 0; i < T::XU; ++i)
      dma16(xb, xbytes, off[i], k0, dst + (wave * T::XU + i) * 1024);
#pragma unroll
    for (int i = 0; i < T::WU; ++i)
      dma16(wb, wbytes, off[i], k0, dst + T::XB + (wave * T::WU + i) * 1024);
  }

  // One ring step: the copies of a later step into `fill` first, then the
  // MFMAs of the step in `tile`, each with one operand read of the following
  // k-steps.
  __device__ __forceinline__ void step(v16i (&acc)[TNT][TMT], const char* tile,
                                       const int8_t* fxb, int fxbytes, const int8_t* fwb,
                                       int fwbytes, int fs, char* fill) const {
    stage(fxb, fxbytes, fwb, fwbytes, fs, fill);
#pragma unroll
    for (int ks = 0; ks < T::KS; ++ks) {
      v4i xf[TMT], wf[TNT];
#pragma unroll
      for (int i = 0; i < TMT; ++i)
        xf[i] = *reinterpret_cast<const v4i*>(tile + xk[ks] + i * 32 * kKS);
#pragma unroll
      for (int i = 0; i < TNT; ++i)
        wf[i] = *reinterpret_cast<const v4i*>(tile + wk[ks] + i * 32 * kKS);
#pragma unroll
      for (int tni = 0; tni < TNT; ++tni)
#pragma unroll
        for (int tmi = 0; tmi < TMT; ++tmi)
          acc[tni][tmi] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf[tni], xf[tmi], acc[tni][tmi],
                                                                0, 0, 0);
    }
    constexpr int kReads = TMT + TNT, kMfma = TMT * TNT;
    __builtin_amdgcn_sched_group_barrier(0x020, T::OPS, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, kReads, 0);
#pragma unroll
    for (int i = 0; i < T::KS * kMfma; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (i < (T::KS - 1) * kReads) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
  }

  // epilogue: lane holds token m = li of each 32-token tile and channels
  // 8 g + 4 hf + (0..3) of each 32-channel tile; lanes l and l + 32 swap
  // halves so that each stores 8 consecutive channels (16 bytes)
  __device__ __forceinline__ void store(const LinearArgs& a, const v16i (&acc)[TNT][TMT],
                                        int64_t m0, int64_t n0) const {
#pragma unroll
    for (int tmi = 0; tmi < TMT; ++tmi) {
      const int64_t m = m0 + wm * 32 * TMT + tmi * 32 + li;
      if (m >= a.M) continue;
      const float xs = a.xs[m];
      u16* orow = a.out + m * a.ldo;
#pragma unroll
      for (int tni = 0; tni < TNT; ++tni)
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          uint32_t pk[2][2];
#pragma unroll
          for (int gg = 0; gg < 2; ++gg) {
            const int g = 2 * p + gg;
            const int64_t n = n0 + wn * 32 * TNT + tni * 32 + 8 * g + 4 * hf;
            const float4 ws = *reinterpret_cast<const float4*>(a.ws + n);
            float y[4] = {static_cast<float>(acc[tni][tmi][4 * g + 0]) * xs * ws.x,
                          static_cast<float>(acc[tni][tmi][4 * g + 1]) * xs * ws.y,
                          static_cast<float>(acc[tni][tmi][4 * g + 2]) * xs * ws.z,
                          static_cast<float>(acc[tni][tmi][4 * g + 3]) * xs * ws.w};
            if (a.bias != nullptr) {
              const uint2 bb = *reinterpret_cast<const uint2*>(a.bias + n);
              const float bv[4] = {__uint_as_float(bb.x << 16),
                                   __uint_as_float(bb.x & 0xffff0000u),
                                   __uint_as_float(bb.y << 16),
                                   __uint_as_float(bb.y & 0xffff0000u)};
#pragma unroll
              for (int e = 0; e < 4; ++e) y[e] = bf16_to_f32(f32_to_bf16(y[e])) + bv[e];
            }
            pk[gg][0] = pack_bf16x2(y[0], y[1]);
            pk[gg][1] = pack_bf16x2(y[2], y[3]);
          }
          // lane l (half 0) keeps channels 8(2p) + 0..3 and takes + 4..7 from
          // lane l + 32, which keeps 8(2p + 1) + 4..7 and takes + 0..3
          uint32_t st[4];
#pragma unroll
          for (int w = 0; w < 2; ++w) {
            const auto r = __builtin_amdgcn_permlane32_swap(pk[0][w], pk[1][w], false, false);
            st[w] = r[0];
            st[2 + w] = r[1];
          }
          const int64_t n = n0 + wn * 32 * TNT + tni * 32 + 8 * (2 * p + hf);
          *reinterpret_cast<uint4*>(orow + n) = make_uint4(st[0], st[1], st[2], st[3]);
        }
    }
  }
};

template <int TMT, int TNT>
__device__ __forceinline__ void zero_acc(v16i (&acc)[TNT][TMT]) {
#pragma unroll
  for (int i = 0; i < TNT; ++i)
#pragma unroll
    for (int j = 0; j < TMT; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
}

// Operand rows of a tile and the bytes a copy may read (the rows past M of a
// partial last tile read as zeros).
struct TileSrc {
  const int8_t* xb;
  const int8_t* wb;
  int xbytes, wbytes;
};
template <int TMT, int TNT>
__device__ __forceinline__ TileSrc tile_src(const LinearArgs& a, int64_t m0, int64_t n0) {
  using T = LinTile<TMT, TNT>;
  const int64_t rows_x = a.M - m0 < T::BM ? a.M - m0 : T::BM;
  return {a.x + m0 * a.K, a.w + n0 * a.K, static_cast<int>(rows_x * a.K),
          static_cast<int>(T::BN * a.K)};
}

// One 128 x 128 tile: a 2-slot ring of k-steps (step j in slot j % 2; the
// copies of step j + 1 go out at the start of step j, after every wavefront
// has finished step j - 1 and step j has landed), then the epilogue.
__device__ __forceinline__ void small_tile(const LinearArgs& a, int64_t m0, int64_t n0,
                                           char* s_0, char* s_1) {
  const LinLane<1, 2> L(a);
  const TileSrc src = tile_src<1, 2>(a, m0, n0);
  const int steps = static_cast<int>(a.K / kKS);
  v16i acc[2][1];
  zero_acc<1, 2>(acc);
  L.stage(src.xb, src.xbytes, src.wb, src.wbytes, 0, s_0);
  // past the last step the copies are empty ranges: nothing is read
  auto fill_of = [&](int s) { return s < steps ? src : TileSrc{src.xb, src.wb, 0, 0}; };
  for (int j = 0; j + 1 < steps; j += 2) {
    qkv_wait_barrier<0>();
    const TileSrc f1 = fill_of(j + 1);
    L.step(acc, s_0, f1.xb, f1.xbytes, f1.wb, f1.wbytes, j + 1, s_1);
    qkv_wait_barrier<0>();
    const TileSrc f2 = fill_of(j + 2);
    L.step(acc, s_1, f2.xb, f2.xbytes, f2.wb, f2.wbytes, j + 2, s_0);
  }
  if (steps & 1) {  // the last step of an odd count, in slot 0
    qkv_wait_barrier<0>();
    L.step(acc, s_0, src.xb, 0, src.wb, 0, steps, s_1);
  }
  __builtin_amdgcn_s_waitcnt(qkv_vmcnt(0));
  L.store(a, acc, m0, n0);
}

// XCD-local big tile `work` -> its origin.  Consecutive work items of an XCD
// walk groups of kGroupM token blocks for one channel block, then the next,
// so the 32 workgroups of an XCD share 4 token blocks and 8 weight blocks in
// its L2 (at 38,720 x 3072 x 3072, interleaved on one box: 0.398-0.403 ms with
// 4 blocks per group; 2, 6 and 8: 0.407-0.414, 0.399-0.410 and 0.404-0.409 ms).
__device__ __forceinline__ bool big_tile_of(const LinearArgs& a, int64_t work, int64_t* m0,
                                            int64_t* n0) {
  constexpr int64_t kGroupM = 4;
  const int64_t n_m = (a.big_rows + BigTile::BM - 1) / BigTile::BM;
  const int64_t tiles_n = a.N / BigTile::BN;
  if (work >= n_m * tiles_n) return false;
  const int64_t group = work / (kGroupM * tiles_n), in_group = work % (kGroupM * tiles_n);
  const int64_t group_m = n_m - group * kGroupM < kGroupM ? n_m - group * kGroupM : kGroupM;
  *m0 = (group * kGroupM + in_group % group_m) * BigTile::BM;
  *n0 = (in_group / group_m) * BigTile::BN;
  return true;
}

// The 256 x 256 tiles items first, first + stride, ... of an XCD's per_xcd.
// The ring runs on from tile to tile: with an even k-step count, the last
// step of a tile fills the other slot with the next tile's first step, so
// those copies fly during the epilogue (with an odd count the next tile
// starts its ring after a barrier).
__device__ __forceinline__ void big_tiles(const LinearArgs& a, int64_t xcd, int64_t first,
                                          int64_t stride, int64_t per_xcd, char* s_0,
                                          char* s_1) {
  int64_t item = first, m0 = 0, n0 = 0;
  if (item >= per_xcd || !big_tile_of(a, xcd * per_xcd + item, &m0, &n0)) return;
  const LinLane<2, 4> L(a);
  const int steps = static_cast<int>(a.K / kKS);
  const bool chain = (steps & 1) == 0;
  TileSrc src = tile_src<2, 4>(a, m0, n0);
  L.stage(src.xb, src.xbytes, src.wb, src.wbytes, 0, s_0);
  v16i acc[4][2];
  while (true) {
    zero_acc<2, 4>(acc);
    const int64_t next = item + stride;
    int64_t nm0 = 0, nn0 = 0;
    const bool has_next = next < per_xcd && big_tile_of(a, xcd * per_xcd + next, &nm0, &nn0);
    TileSrc nsrc = tile_src<2, 4>(a, nm0, nn0);
    if (!(has_next && chain)) nsrc.xbytes = nsrc.wbytes = 0;  // the last fill reads nothing
    for (int j = 0; j + 1 < steps; j += 2) {
      qkv_wait_barrier<0>();
      L.step(acc, s_0, src.xb, src.xbytes, src.wb, src.wbytes, j + 1, s_1);
      qkv_wait_barrier<0>();
      // one step call with selected operands (a branch between two calls
      // makes the compiler spill)
      const bool last = j + 2 >= steps;
      L.step(acc, s_1, last ? nsrc.xb : src.xb, last ? nsrc.xbytes : src.xbytes,
             last ? nsrc.wb : src.wb, last ? nsrc.wbytes : src.wbytes, last ? 0 : j + 2, s_0);
    }
    if (!chain) {  // the last step of an odd count, in slot 0
      qkv_wait_barrier<0>();
      L.step(acc, s_0, src.xb, 0, src.wb, 0, steps, s_1);
    }
    L.store(a, acc, m0, n0);
    if (!has_next) break;
    item = next;
    m0 = nm0;
    n0 = nn0;
    src = tile_src<2, 4>(a, m0, n0);
    if (!chain) {  // every wavefront is past its last step before slot 0 refills
      __builtin_amdgcn_s_waitcnt(qkv_vmcnt(0));
      __syncthreads();
      L.stage(src.xb, src.xbytes, src.wb, src.wbytes, 0, s_0);
    }
  }
  __builtin_amdgcn_s_waitcnt(qkv_vmcnt(0));
}

// One workgroup per compute unit (the LDS ring admits one), `per_wg` of them
// on each XCD: workgroup j of XCD x takes the XCD's 128 x 128 tiles j,
// j + per_wg, ... (the rows past big_rows), then its 256 x 256 tiles the
// same way.  The compute units that take a small tile start their big tiles
// a quarter tile later than the others, so the two groups' output stores
// fall beside the other group's MFMAs instead of all at once.
__global__ void __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
int8_linear_kernel(LinearArgs a, int64_t per_wg, int64_t per_xcd_small, int64_t per_xcd_big) {
  __shared__ __attribute__((aligned(1024))) char s_0[BigTile::XB + BigTile::WB];
  __shared__ __attribute__((aligned(1024))) char s_1[BigTile::XB + BigTile::WB];
  const int64_t xcd = blockIdx.x % kNumXcd, j = blockIdx.x / kNumXcd;
  const int64_t tiles_n = a.N / SmallTile::BN;
  const int64_t n_small =
      (a.M - a.big_rows + SmallTile::BM - 1) / SmallTile::BM * tiles_n;
  for (int64_t i = j; i < per_xcd_small; i += per_wg) {
    const int64_t tile = xcd * per_xcd_small + i;
    if (tile >= n_small) break;
    small_tile(a, a.big_rows + tile / tiles_n * SmallTile::BM, tile % tiles_n * SmallTile::BN,
               s_0, s_1);
    __syncthreads();  // every wavefront is done with the slots
  }
  big_tiles(a, xcd, j, per_wg, per_xcd_big, s_0, s_1);
}

}  // namespace rcsa

using namespace rcsa;

extern "C" int rcsa_quantize_rows_int8(const void* x, int dtype, int64_t M, int64_t C, int64_t ldx,
                                       int8_t* q, float* scale, hipStream_t stream) {
  if (!x || !q || !scale) return RCSA_ERR_NULL;
  if (M <= 0 || C <= 0 || C % 8 || ldx < C || ldx % 8) return RCSA_ERR_SHAPE;
  if ((reinterpret_cast<uintptr_t>(x) & 15u) || (reinterpret_cast<uintptr_t>(q) & 7u))
    return RCSA_ERR_ALIGN;
  const int64_t rows_per = kQThreads / kWave;
  const dim3 grid(static_cast<unsigned>((M + rows_per - 1) / rows_per));
  if (dtype == RCSA_BF16)
    quant_rows_kernel<u16><<<grid, dim3(kQThreads), 0, stream>>>(static_cast<const u16*>(x), M, C,
                                                                  ldx, q, scale);
  else if (dtype == RCSA_F32)
    quant_rows_kernel<float><<<grid, dim3(kQThreads), 0, stream>>>(static_cast<const float*>(x), M,
                                                                    C, ldx, q, scale);
  else
    return RCSA_ERR_DTYPE;
  return launch_status();
}

extern "C" int rcsa_int8_linear(const int8_t* x, const float* x_scale, const int8_t* w,
                                const float* w_scale, const void* bias, int64_t M, int64_t N,
                                int64_t K, void* out, int64_t ldo, hipStream_t stream) {
  if (!x || !x_scale || !w || !w_scale || !out) return RCSA_ERR_NULL;
  if (M <= 0 || N <= 0 || K <= 0 || N % BigTile::BN || K % kKS || ldo < N || ldo % 4)
    return RCSA_ERR_SHAPE;
  // the copies address a tile with 32-bit offsets
  if (static_cast<int64_t>(BigTile::BM) * K >= (int64_t{1} << 31)) return RCSA_ERR_SHAPE;
  if ((reinterpret_cast<uintptr_t>(x) & 15u) || (reinterpret_cast<uintptr_t>(w) & 15u) ||
      (reinterpret_cast<uintptr_t>(w_scale) & 15u) || (reinterpret_cast<uintptr_t>(out) & 7u) ||
      (reinterpret_cast<uintptr_t>(bias) & 7u))
    return RCSA_ERR_ALIGN;
  // 256 x 256 tiles, except that a short last round (fewer tiles than half the
  // compute units) is re-cut: the rows its tiles would cover go to 128 x 128
  // tiles, a quarter of the work each, taken first (which also offsets the
  // rounds of the compute units that take one)
  const int64_t big_n = N / BigTile::BN;
  const int64_t all_big = ((M + BigTile::BM - 1) / BigTile::BM) * big_n;
  int64_t big_rows = M;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) == hipSuccess &&
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
      cus > 0) {
    const int64_t rem = all_big % cus;
    const int64_t rows = (all_big - rem) / big_n * BigTile::BM;  // whole row blocks of full rounds
    if (rem != 0 && 2 * rem < cus && rows > 0 && rows < M) big_rows = rows;
  }
  const int64_t big_tiles = ((big_rows + BigTile::BM - 1) / BigTile::BM) * big_n;
  const int64_t small_tiles =
      big_rows < M ? ((M - big_rows + SmallTile::BM - 1) / SmallTile::BM) * (N / SmallTile::BN) : 0;
  if (big_tiles >= (int64_t{1} << 30) || small_tiles >= (int64_t{1} << 30)) return RCSA_ERR_SHAPE;
  LinearArgs a{x, x_scale, w, w_scale, static_cast<const u16*>(bias), static_cast<u16*>(out),
               M, N, K, ldo, big_rows};
  // one workgroup per compute unit, the same number on every XCD
  const int64_t per_wg = cus >= kNumXcd ? cus / kNumXcd : 32;
  const dim3 grid(static_cast<unsigned>(per_wg * kNumXcd));
  int8_linear_kernel<<<grid, dim3(kGemmThreads), 0, stream>>>(
      a, per_wg, (small_tiles + kNumXcd - 1) / kNumXcd, (big_tiles + kNumXcd - 1) / kNumXcd);
  return launch_status();
}
