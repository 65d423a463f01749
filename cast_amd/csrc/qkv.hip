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
// wavefront 32 x 64) of the same launch, dispatched first.
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
  // one launch: 128 x 128 tiles over rows [big_rows, M) on the first
  // gridDim.x - big_grid workgroups, then 256 x 256 tiles over rows [0, big_rows)
  // on the last big_grid
  int64_t big_rows, big_grid;
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

template <int TMT, int TNT>
__device__ __forceinline__ void linear_tile(const LinearArgs& a, int64_t m0, int64_t n0,
                                            char* s_0, char* s_1) {
  using T = LinTile<TMT, TNT>;
  const int t = threadIdx.x, lane = t % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
  const int wm = wave & 3, wn = wave >> 2;

  // copies: each tile is units of 1 KiB (8 rows of 128 bytes); a wavefront
  // copies XU + WU units per ring step.  Lane l lands at row 8 u + l / 8, chunk
  // l % 8 of its unit and loads the chunk that the swizzle puts there.
  const int64_t rows_x = a.M - m0 < T::BM ? a.M - m0 : T::BM;
  const int8_t* xb = a.x + m0 * a.K;
  const int8_t* wb = a.w + n0 * a.K;
  const int xbytes = static_cast<int>(rows_x * a.K), wbytes = static_cast<int>(T::BN * a.K);
  uint32_t off[T::XU];  // the same rows of both tiles
#pragma unroll
  for (int i = 0; i < T::XU; ++i) {
    const int r = (wave * T::XU + i) * 8 + lane / 8;
    off[i] = static_cast<uint32_t>(r * a.K + ((lane & 7) ^ qkv_swz(r)) * 16);
  }
  const int steps = static_cast<int>(a.K / kKS);
  auto stage = [&](int s, char* dst) __attribute__((always_inline)) {
    // past the last step: empty ranges, nothing is read (the slot is never read)
    const bool live = s < steps;
    const int k0 = live ? s * kKS : 0;
#pragma unroll
    for (int i = 0; i < T::XU; ++i)
      dma16(xb, live ? xbytes : 0, off[i], k0, dst + (wave * T::XU + i) * 1024);
#pragma unroll
    for (int i = 0; i < T::WU; ++i)
      dma16(wb, live ? wbytes : 0, off[i], k0, dst + T::XB + (wave * T::WU + i) * 1024);
  };

  // operand read offsets: row r of a tile, chunk c = 2 ks + lane half
  const int hf = lane >> 5, li = lane & 31;
  int xo[TMT][T::KS], wo[TNT][T::KS];
#pragma unroll
  for (int tmi = 0; tmi < TMT; ++tmi)
#pragma unroll
    for (int ks = 0; ks < T::KS; ++ks) {
      const int r = wm * 32 * TMT + tmi * 32 + li;
      xo[tmi][ks] = r * kKS + (((ks * 2 + hf) ^ qkv_swz(r)) * 16);
    }
#pragma unroll
  for (int tni = 0; tni < TNT; ++tni)
#pragma unroll
    for (int ks = 0; ks < T::KS; ++ks) {
      const int r = wn * 32 * TNT + tni * 32 + li;
      wo[tni][ks] = T::XB + r * kKS + (((ks * 2 + hf) ^ qkv_swz(r)) * 16);
    }

  v16i acc[TNT][TMT];
#pragma unroll
  for (int i = 0; i < TNT; ++i)
#pragma unroll
    for (int j = 0; j < TMT; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  stage(0, s_0);
  auto compute = [&](const char* tile, int s_fill, char* fill) __attribute__((always_inline)) {
    stage(s_fill, fill);
#pragma unroll
    for (int ks = 0; ks < T::KS; ++ks) {
      v4i xf[TMT], wf[TNT];
#pragma unroll
      for (int i = 0; i < TMT; ++i) xf[i] = *reinterpret_cast<const v4i*>(tile + xo[i][ks]);
#pragma unroll
      for (int i = 0; i < TNT; ++i) wf[i] = *reinterpret_cast<const v4i*>(tile + wo[i][ks]);
#pragma unroll
      for (int tni = 0; tni < TNT; ++tni)
#pragma unroll
        for (int tmi = 0; tmi < TMT; ++tmi)
          acc[tni][tmi] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf[tni], xf[tmi], acc[tni][tmi],
                                                                0, 0, 0);
    }
    // the copies of the next step first, then the k-step 0 operands, then each
    // MFMA with one operand read of the following k-steps
    constexpr int kReads = TMT + TNT, kMfma = TMT * TNT;
    __builtin_amdgcn_sched_group_barrier(0x020, T::OPS, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, kReads, 0);
#pragma unroll
    for (int i = 0; i < T::KS * kMfma; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (i < (T::KS - 1) * kReads) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
  };
  // ring of two slots: step j lives in slot j % 2; the copies of step j + 1
  // go out at the start of step j, after every wavefront has finished step
  // j - 1 and step j has landed
  for (int j = 0; j + 1 < steps; j += 2) {
    qkv_wait_barrier<0>();
    compute(s_0, j + 1, s_1);
    qkv_wait_barrier<0>();
    compute(s_1, j + 2, s_0);
  }
  if (steps & 1) {  // the last step of an odd count, in slot 0; its copies are empty
    qkv_wait_barrier<0>();
    compute(s_0, steps, s_1);
  }
  __builtin_amdgcn_s_waitcnt(qkv_vmcnt(0));

  // epilogue: lane holds token m = li of each 32-token tile and channels
  // 8 g + 4 hf + (0..3) of each 32-channel tile; lanes l and l + 32 swap
  // halves so that each stores 8 consecutive channels (16 bytes)
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
            const float bv[4] = {__uint_as_float(bb.x << 16), __uint_as_float(bb.x & 0xffff0000u),
                                 __uint_as_float(bb.y << 16), __uint_as_float(bb.y & 0xffff0000u)};
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

using BigTile = LinTile<2, 4>;    // 256 x 256, each wavefront 64 x 128
using SmallTile = LinTile<1, 2>;  // 128 x 128, each wavefront 32 x 64

__global__ void __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
int8_linear_kernel(LinearArgs a) {
  __shared__ __attribute__((aligned(1024))) char s_0[BigTile::XB + BigTile::WB];
  __shared__ __attribute__((aligned(1024))) char s_1[BigTile::XB + BigTile::WB];
  // the 128 x 128 tiles take the first workgroup slots: the compute units that
  // run one start their 256 x 256 tiles a quarter tile later than the others,
  // so the two groups' output stores fall beside the other group's MFMAs
  // instead of all at once (0.417 against 0.428 ms at 38,720 x 3072 x 3072)
  const int64_t small_grid = static_cast<int64_t>(gridDim.x) - a.big_grid;
  const int64_t bid = static_cast<int64_t>(blockIdx.x) >= small_grid
                          ? static_cast<int64_t>(blockIdx.x) - small_grid
                          : static_cast<int64_t>(blockIdx.x) + a.big_grid;
  if (bid < a.big_grid) {
    // XCD-aware order in groups of kGroupM token blocks: consecutive tiles of
    // one XCD walk the group's token blocks for one channel block, then the
    // next channel block, so the 32 workgroups resident on an XCD at once share
    // 4 token blocks and 8 weight blocks in its L2 (at 38,720 x 3072 x 3072:
    // 0.458 ms with 4 blocks per group; 2, 8 and 16: 0.467, 0.462 and 0.469 ms)
    constexpr int64_t kGroupM = 4;
    const int64_t n_m = (a.big_rows + BigTile::BM - 1) / BigTile::BM;
    const int64_t tiles_n = a.N / BigTile::BN;
    const int64_t tile = xcd_remap(bid, n_m * tiles_n);
    if (tile < 0) return;
    const int64_t group = tile / (kGroupM * tiles_n), in_group = tile % (kGroupM * tiles_n);
    const int64_t group_m = n_m - group * kGroupM < kGroupM ? n_m - group * kGroupM : kGroupM;
    const int64_t tm = group * kGroupM + in_group % group_m, tn = in_group / group_m;
    linear_tile<2, 4>(a, tm * BigTile::BM, tn * BigTile::BN, s_0, s_1);
  } else {
    // the rows after big_rows in 128 x 128 tiles: the work of a short last
    // round, which whole 256 x 256 tiles would leave mostly idle
    const int64_t n_m = (a.M - a.big_rows + SmallTile::BM - 1) / SmallTile::BM;
    const int64_t tiles_n = a.N / SmallTile::BN;
    const int64_t tile = xcd_remap(bid - a.big_grid, n_m * tiles_n);
    if (tile < 0) return;
    const int64_t tm = tile / tiles_n, tn = tile % tiles_n;
    linear_tile<1, 2>(a, a.big_rows + tm * SmallTile::BM, tn * SmallTile::BN, s_0, s_1);
  }
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
  // tiles, a quarter of the work each, dispatched first (which also offsets
  // the rounds of the compute units that take one)
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
               M, N, K, ldo, big_rows, xcd_grid(big_tiles)};
  const dim3 grid(static_cast<unsigned>(a.big_grid + (small_tiles ? xcd_grid(small_tiles) : 0)));
  int8_linear_kernel<<<grid, dim3(kGemmThreads), 0, stream>>>(a);
  return launch_status();
}
