// Block-sparse flash attention for gfx950 (MI355X).
//
// Work decomposition: one workgroup = one (batch, head, query block) of
// BLOCK_M rows; it streams only the key blocks named in its block list.
// The workgroup has 2 * BLOCK_M / 32 wavefronts: row group rg (32 query
// rows) x key half kh (BLOCK_N / 2 keys of every block).  The two key halves
// keep independent online-softmax states that are merged once at the end, so
// eight wavefronts share every staged tile (two per SIMD).
//
// Staging: each selected K tile (row-major, 16-byte chunks XOR-swizzled) and
// V tile (row-major, swizzled) is copied global -> LDS with direct-to-LDS
// loads (no VGPR round trip), double buffered: the copy of block i+1 is in
// flight while block i is computed.
//
// Orientation: a wavefront computes S^T = K Q^T with 32x32 MFMAs, so a lane
// owns ONE query row (column lane%32 of the MFMA output).  The K rows fed to
// the A operand are permuted (key_perm) so that lane half h holds the 16
// consecutive keys 16h..16h+15 of each 32-key tile; P^T then feeds the B
// operand of O^T = V^T P^T straight from registers.  The V^T operand comes
// from the row-major V tile through ds_read_b64_tr_b16 (a 16-lane group
// reading a 4x16 block receives its transpose).
//
// Arithmetic: QK^T on v_mfma_i32_32x32x32_i8 (int8) or
// v_mfma_f32_32x32x16_bf16 (bf16); PV on v_mfma_f32_32x32x16_bf16.  In the
// int8 path the i32 accumulator starts at the bit pattern of 1.5 * 2^23, so
// the result read as fp32 is exactly 1.5 * 2^23 + x (|x| < 2^22): the
// int->float conversion is free and folds into the exp2 argument's FMA.
// Softmax is online, fp32, exp2 domain (log2(e) folded into the scale); the
// running max is only moved when a row's max grows by more than 2^8
// (rescaling O is skipped otherwise).  Row sums accumulate the bf16-rounded
// probabilities with v_dot2_f32_bf16, so numerator and denominator use the
// same P.
#include <type_traits>

#include "rcsa_common.h"

namespace rcsa {

typedef __bf16 v4bf __attribute__((ext_vector_type(4)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
#define RCSA_LDS(T, p) ((__attribute__((address_space(3))) T*)(p))

struct AttnArgs {
  const void* q;
  const void* k;
  const u16* v;
  const uint8_t* kvalid;
  float scale_log2;  // sm_scale * log2(e)
  float* lse;
  u16* out;
  const int32_t* idx;
  const int32_t* lens;
  const float* q_scale;
  int64_t q_scale_stride;
  const float* k_scale;
  int64_t k_scale_stride;
  int64_t sqz, sqh, sqm, skz, skh, skn, svz, svh, svn, soz, soh, som;
  int64_t sbz, sbh, sbm, slz, slh, slm;
  int64_t H, q_len, k_len, n_qblocks, n_kblocks, max_k, n_work;
};

constexpr float kTau = 8.0f;               // lazy-rescale threshold, log2 units
constexpr float kMagicF = 12582912.0f;     // 1.5 * 2^23
constexpr int kMagicI = 0x4B400000;        // its fp32 bit pattern

// MFMA row m = 8a + 4h + b of a 32-key tile reads key 16h + 4a + b.
__device__ __forceinline__ int key_perm(int m) {
  return 16 * ((m >> 2) & 1) + 4 * (m >> 3) + (m & 3);
}
// 16-byte chunk swizzles (bank-conflict-free ds_read_b128 of permuted K rows,
// balanced ds_read_b64_tr_b16 over 4-row groups of V).
__device__ __forceinline__ int swz_k(int row) { return (row & 3) | ((row >> 2) & 4); }
__device__ __forceinline__ int swz_v(int row) { return 4 * (row & 3); }

template <bool INT8, int D, int BM, int BN>
struct AttnCfg {
  static constexpr int NRG = BM / 32;            // row groups
  static constexpr int NW = NRG * 2;             // wavefronts
  static constexpr int NT = NW * 64;             // threads
  static constexpr int KB = INT8 ? 1 : 2;        // bytes per K element
  static constexpr int KROW = D * KB;            // bytes per staged K row
  static constexpr int CPR_K = KROW / 16;
  static constexpr int VROW = D * 2;             // bytes per staged V row
  static constexpr int CPR_V = VROW / 16;
  static constexpr int QSTEPS = INT8 ? D / 32 : D / 16;
  static constexpr int HK = BN / 2;              // keys per wavefront per block
  static constexpr int KT = HK / 32;             // 32-key tiles per wavefront
  static constexpr int NDT = D / 32;             // 32-wide head_dim tiles
  static constexpr int KBYTES = BN * KROW;
  static constexpr int VBYTES = BN * VROW;
  static constexpr int BUF = KBYTES + VBYTES;
  static constexpr int UNITS = BUF / 1024;       // 1 KiB direct-load units
  static constexpr int KUNITS = KBYTES / 1024;
  static constexpr int UPW = (UNITS + NW - 1) / NW;
  static constexpr int K_RPU = 1024 / KROW;      // rows per unit
  static constexpr int V_RPU = 1024 / VROW;
  static constexpr int MERGE_WAVE = NDT * 16 * 64 + 128;  // floats
  static constexpr int MERGE = NRG * MERGE_WAVE * 4;     // bytes
  static constexpr int SMEM = 2 * BUF > MERGE ? 2 * BUF : MERGE;
  static_assert(KBYTES % 1024 == 0 && VBYTES % 1024 == 0, "tile is not whole 1 KiB units");
  static_assert(QSTEPS * 2 == CPR_K, "K chunk layout");
};

template <bool INT8, int D, int BM, int BN>
__global__ void __launch_bounds__(BM * 4)  // == AttnCfg::NT
sparse_attn_kernel(AttnArgs a) {
  using C = AttnCfg<INT8, D, BM, BN>;
  typedef typename std::conditional<INT8, v4i, v8bf>::type OpT;
  typedef typename std::conditional<INT8, v16i, v16f>::type AccT;
  __shared__ __attribute__((aligned(1024))) char smem[C::SMEM];

  const int64_t work = xcd_remap(blockIdx.x, a.n_work);
  if (work < 0) return;
  const int64_t qb = work % a.n_qblocks;
  const int64_t bh = work / a.n_qblocks;
  const int64_t b = bh / a.H, h = bh % a.H;

  const int tid = threadIdx.x;
  const int lane = tid % kWave, wave = tid / kWave;
  const int rg = wave % C::NRG, kh = wave / C::NRG;
  const int hf = lane >> 5, lr = lane & 31;
  const int64_t qrow = qb * BM + rg * 32 + lr;
  const bool qrow_ok = qrow < a.q_len;

  // Q operand (B of S^T = K Q^T): lane half hf holds the row's bytes
  // [hf*KROW/2, (hf+1)*KROW/2) as QSTEPS 16-byte steps.
  OpT q_op[C::QSTEPS];
  {
    const char* qp = static_cast<const char*>(a.q) +
                     (b * a.sqz + h * a.sqh + qrow * a.sqm) * C::KB;
#pragma unroll
    for (int st = 0; st < C::QSTEPS; ++st) {
      v4i raw = {0, 0, 0, 0};
      if (qrow_ok) raw = *reinterpret_cast<const v4i*>(qp + (hf * C::QSTEPS + st) * 16);
      q_op[st] = __builtin_bit_cast(OpT, raw);
    }
  }
  const float qs = INT8 ? a.q_scale[bh * a.q_scale_stride + qb] : 1.0f;

  v16f o_acc[C::NDT];
#pragma unroll
  for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) o_acc[dt][r] = 0.0f;
  float m_run = -INFINITY;  // running max (log2 domain), shared by both lane halves
  float l_run = 0.0f;       // this lane's partial row sum

  int64_t cnt = a.lens[b * a.slz + h * a.slh + qb * a.slm];
  cnt = cnt < 0 ? 0 : (cnt > a.max_k ? a.max_k : cnt);
  const int32_t* list = a.idx + b * a.sbz + h * a.sbh + qb * a.sbm;
  const char* kbase = static_cast<const char*>(a.k) + (b * a.skz + h * a.skh) * C::KB;
  const char* vbase = reinterpret_cast<const char*>(a.v + b * a.svz + h * a.svh);
  const int64_t klast = a.k_len - 1;
  const int64_t krow_bytes = a.skn * C::KB, vrow_bytes = a.svn * 2;

  // Direct-to-LDS staging geometry.  Unit u (1 KiB) of a buffer holds K rows
  // (u < KUNITS) or V rows; lane l lands at byte l*16 of its unit, so it
  // loads the swizzled global chunk that belongs there.  Per unit: the tile
  // row this lane copies and that row's in-row byte offset (32-bit: the host
  // bounds one head's K/V below 2 GiB).
  int st_row[C::UPW];
  int st_col[C::UPW];
#pragma unroll
  for (int i = 0; i < C::UPW; ++i) {
    const int u = wave * C::UPW + i;
    if (u < C::KUNITS) {
      st_row[i] = u * C::K_RPU + lane / C::CPR_K;
      st_col[i] = ((lane % C::CPR_K) ^ (swz_k(st_row[i]) & (C::CPR_K - 1))) * 16;
    } else {
      st_row[i] = (u - C::KUNITS) * C::V_RPU + lane / C::CPR_V;
      st_col[i] = ((lane % C::CPR_V) ^ (swz_v(st_row[i]) & (C::CPR_V - 1))) * 16;
    }
  }
  // Rows past k_len re-read the last row (those keys are masked).
  auto stage = [&](int64_t n, int buf) {
    const int64_t key0 = n * BN;
    const bool tail = key0 + BN > a.k_len;
    char* dst = smem + buf * C::BUF;
#pragma unroll
    for (int i = 0; i < C::UPW; ++i) {
      const int u = wave * C::UPW + i;
      if (u < C::UNITS) {
        int64_t key = key0 + st_row[i];
        if (tail) key = min(key, klast);
        const char* src = u < C::KUNITS
            ? kbase + static_cast<uint32_t>(key * krow_bytes + st_col[i])
            : vbase + static_cast<uint32_t>(key * vrow_bytes + st_col[i]);
        __builtin_amdgcn_global_load_lds(src, RCSA_LDS(void, dst + u * 1024), 16, 0, 0);
      }
    }
  };
  auto block_of = [&](int64_t it) -> int64_t {
    const int64_t n = list[it];
    return (n >= 0 && n < a.n_kblocks) ? n : 0;
  };

  // Lane-dependent LDS read offsets.  The swizzles only involve lane bits,
  // so tile/step offsets (32t, 8u, 4q rows) become instruction immediates.
  int k_off[C::QSTEPS];
  {
    const int row = key_perm(lr);  // + kh*HK + 32t: multiples of 32
    const int sw = swz_k(row) & (C::CPR_K - 1);
#pragma unroll
    for (int st = 0; st < C::QSTEPS; ++st)
      k_off[st] = (kh * C::HK + row) * C::KROW + (((hf * C::QSTEPS + st) ^ sw) * 16);
  }
  int v_off[C::NDT];
  {
    const int grp = lane >> 4, gi = lane & 15;
    const int row = 16 * (grp >> 1) + (gi >> 2);  // + kh*HK + 32t + 8u + 4q: multiples of 4
    const int sw = swz_v(row) & (C::CPR_V - 1);
#pragma unroll
    for (int dt = 0; dt < C::NDT; ++dt) {
      const int d = 32 * dt + 16 * (grp & 1) + 4 * (gi & 3);
      v_off[dt] = C::KBYTES + (kh * C::HK + row) * C::VROW + (((d >> 3) ^ sw) * 16) + (d & 7) * 2;
    }
  }

  if (cnt > 0) stage(block_of(0), 0);

  for (int64_t it = 0; it < cnt; ++it) {
    const int64_t n_raw = list[it];
    const bool blk_ok = n_raw >= 0 && n_raw < a.n_kblocks;
    const int64_t n = blk_ok ? n_raw : 0;
    const int buf = static_cast<int>(it & 1);
    __syncthreads();  // block `it` is in LDS; everyone is done with the other buffer
    if (it + 1 < cnt) stage(block_of(it + 1), buf ^ 1);

    const char* tile = smem + buf * C::BUF;
    const int64_t key0 = n * BN + kh * C::HK;

    // validity of this wavefront's HK keys as a uniform bitmask
    const int64_t mykey = key0 + lane;
    const bool kok = blk_ok && lane < C::HK && mykey < a.k_len &&
                     (a.kvalid == nullptr || a.kvalid[mykey] != 0);
    const uint64_t vmask = __ballot(kok);
    const bool all_valid = vmask == (C::HK == 64 ? ~0ull : ((1ull << C::HK) - 1ull));

    // ---- S^T = K Q^T ----
    AccT s_acc[C::KT];
#pragma unroll
    for (int t = 0; t < C::KT; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        if constexpr (INT8) s_acc[t][r] = kMagicI;
        else s_acc[t][r] = 0.0f;
      }
#pragma unroll
      for (int st = 0; st < C::QSTEPS; ++st) {
        const v4i raw = *reinterpret_cast<const v4i*>(tile + k_off[st] + 32 * t * C::KROW);
        if constexpr (INT8) {
          s_acc[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(raw, q_op[st], s_acc[t], 0, 0, 0);
        } else {
          s_acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              __builtin_bit_cast(v8bf, raw), q_op[st], s_acc[t], 0, 0, 0);
        }
      }
    }

    // ---- online softmax: lane half hf, register r <-> key 32t + 16hf + r ----
    // raw value: int8 -> 1.5*2^23 + x read as fp32; bf16 -> the fp32 logit.
    // A masked key's raw value becomes -inf, so max and exp2 need no mask.
    float rv[C::KT][16];
#pragma unroll
    for (int t = 0; t < C::KT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        if constexpr (INT8) rv[t][r] = __int_as_float(s_acc[t][r]);
        else rv[t][r] = s_acc[t][r];
      }
    if (!all_valid) {
      // this lane's 16 keys of each tile as one 32-bit word
      uint32_t bits = 0;
#pragma unroll
      for (int t = 0; t < C::KT; ++t)
        bits |= static_cast<uint32_t>((vmask >> (32 * t + 16 * hf)) & 0xffffull) << (16 * t);
#pragma unroll
      for (int t = 0; t < C::KT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          rv[t][r] = ((bits >> (16 * t + r)) & 1u) ? rv[t][r] : -INFINITY;
    }
    float rmax = -INFINITY;
#pragma unroll
    for (int t = 0; t < C::KT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) rmax = fmaxf(rmax, rv[t][r]);
    rmax = fmaxf(rmax, __shfl_xor(rmax, 32, kWave));
    const float c = INT8 ? a.scale_log2 * qs * a.k_scale[bh * a.k_scale_stride + n]
                         : a.scale_log2;
    const float m_blk = (rmax == -INFINITY) ? -INFINITY
                        : (INT8 ? (rmax - kMagicF) * c : rmax * c);
    if (__ballot(m_blk > m_run + kTau) != 0) {  // wavefront-uniform
      const float m_new = fmaxf(m_run, m_blk);
      const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o_acc[dt][r] *= alpha;
      m_run = m_new;
    }
    const float bias = -(INT8 ? c * kMagicF : 0.0f) - (m_run == -INFINITY ? 0.0f : m_run);

    v8bf p_op[C::KT][2];
#pragma unroll
    for (int t = 0; t < C::KT; ++t)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float e = __builtin_amdgcn_exp2f(fmaf(rv[t][8 * u + j], c, bias));
          p_op[t][u][j] = static_cast<__bf16>(e);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const v2bf pair = {p_op[t][u][2 * j], p_op[t][u][2 * j + 1]};
          const v2bf ones = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};
          l_run = __builtin_amdgcn_fdot2_f32_bf16(pair, ones, l_run, false);
        }
      }

    // ---- O^T += V^T P^T, V^T operand by transposing LDS reads ----
#pragma unroll
    for (int t = 0; t < C::KT; ++t)
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int dt = 0; dt < C::NDT; ++dt) {
          const char* p0 = tile + v_off[dt] + (32 * t + 8 * u) * C::VROW;
          const v4bf lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(RCSA_LDS(v4bf, p0));
          const v4bf hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
              RCSA_LDS(v4bf, p0 + 4 * C::VROW));
          const v8bf v_op = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
          o_acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v_op, p_op[t][u], o_acc[dt],
                                                             0, 0, 0);
        }
  }

  // ---- merge the two key halves, normalise, write O (bf16) and the LSE ----
  const float l_tot = l_run + __shfl_xor(l_run, 32, kWave);
  __syncthreads();  // main loop done everywhere: LDS is free for the merge
  float* mbuf = reinterpret_cast<float*>(smem) + rg * C::MERGE_WAVE;
  if (kh == 1) {
#pragma unroll
    for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) mbuf[(dt * 16 + r) * 64 + lane] = o_acc[dt][r];
    mbuf[C::NDT * 16 * 64 + lane] = m_run;
    mbuf[C::NDT * 16 * 64 + 64 + lane] = l_tot;
  }
  __syncthreads();
  if (kh == 0) {
    const float m_b = mbuf[C::NDT * 16 * 64 + lane];
    const float l_b = mbuf[C::NDT * 16 * 64 + 64 + lane];
    const float m = fmaxf(m_run, m_b);
    const float wa = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m);
    const float wb = m_b == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_b - m);
    const float l = l_tot * wa + l_b * wb;
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    const float fa = wa * inv, fb = wb * inv;
    if (qrow_ok) {
      u16* op = a.out + b * a.soz + h * a.soh + qrow * a.som;
#pragma unroll
      for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float o4[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int r = 4 * g + j;
            o4[j] = o_acc[dt][r] * fa + mbuf[(dt * 16 + r) * 64 + lane] * fb;
          }
          const int d0 = 32 * dt + 8 * g + 4 * hf;
          *reinterpret_cast<uint2*>(op + d0) =
              make_uint2(pack_bf16x2(o4[0], o4[1]), pack_bf16x2(o4[2], o4[3]));
        }
      if (a.lse && hf == 0)
        a.lse[(b * a.H + h) * a.q_len + qrow] =
            l > 0.0f ? (m + __log2f(l)) * 0.69314718055994531f : -INFINITY;
    }
  }
}

template <bool INT8>
static int launch_attn(AttnArgs& a, int64_t D, int64_t BM, int64_t BN, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(xcd_grid(a.n_work)));
#define RCSA_ATTN(D_, BM_, BN_)                                                   \
  if (D == D_ && BM == BM_ && BN == BN_) {                                        \
    sparse_attn_kernel<INT8, D_, BM_, BN_>                                        \
        <<<grid, dim3(AttnCfg<INT8, D_, BM_, BN_>::NT), 0, s>>>(a);               \
    return launch_status();                                                       \
  }
  RCSA_ATTN(128, 128, 128)
  RCSA_ATTN(128, 128, 64)
  RCSA_ATTN(128, 64, 128)
  RCSA_ATTN(128, 64, 64)
  RCSA_ATTN(64, 128, 128)
  RCSA_ATTN(64, 128, 64)
  RCSA_ATTN(64, 64, 128)
  RCSA_ATTN(64, 64, 64)
#undef RCSA_ATTN
  return RCSA_ERR_SHAPE;
}

static int fill_common(AttnArgs& a, const uint8_t* K_valid, float sm_scale, float* M,
                       void* Out, const int32_t* bi, const int32_t* bl,
                       int64_t sqz, int64_t sqh, int64_t sqm, int64_t skz, int64_t skh,
                       int64_t skn, int64_t svz, int64_t svh, int64_t svn, int64_t soz,
                       int64_t soh, int64_t som, int64_t sbz, int64_t sbh, int64_t sbm,
                       int64_t slz, int64_t slh, int64_t slm, int64_t B, int64_t H,
                       int64_t Q_LEN, int64_t K_LEN, int64_t D, int64_t BM, int64_t BN,
                       int64_t max_k, int64_t kvec) {
  if (!Out || !bi || !bl) return RCSA_ERR_NULL;
  if (B <= 0 || H <= 0 || Q_LEN <= 0 || K_LEN <= 0 || max_k < 0) return RCSA_ERR_SHAPE;
  if (!(D == 64 || D == 128) || !(BM == 64 || BM == 128) || !(BN == 64 || BN == 128))
    return RCSA_ERR_SHAPE;
  if (!(sm_scale > 0.0f) || !(sm_scale < INFINITY)) return RCSA_ERR_SHAPE;
  // 16-byte aligned rows: bf16 strides multiple of 8, int8 multiple of 16
  if (sqm % kvec || sqh % kvec || sqz % kvec) return RCSA_ERR_STRIDE;
  if (skn % kvec || skh % kvec || skz % kvec) return RCSA_ERR_STRIDE;
  if (svn % 8 || svh % 8 || svz % 8) return RCSA_ERR_STRIDE;
  if (som % 4 || soh % 4 || soz % 4) return RCSA_ERR_STRIDE;
  if (reinterpret_cast<uintptr_t>(Out) & 7u) return RCSA_ERR_ALIGN;
  a.kvalid = K_valid;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  a.lse = M;
  a.out = static_cast<u16*>(Out);
  a.idx = bi;
  a.lens = bl;
  a.sqz = sqz; a.sqh = sqh; a.sqm = sqm;
  a.skz = skz; a.skh = skh; a.skn = skn;
  a.svz = svz; a.svh = svh; a.svn = svn;
  a.soz = soz; a.soh = soh; a.som = som;
  a.sbz = sbz; a.sbh = sbh; a.sbm = sbm;
  a.slz = slz; a.slh = slh; a.slm = slm;
  a.H = H;
  a.q_len = Q_LEN;
  a.k_len = K_LEN;
  a.n_qblocks = (Q_LEN + BM - 1) / BM;
  a.n_kblocks = (K_LEN + BN - 1) / BN;
  a.max_k = max_k;
  a.n_work = B * H * a.n_qblocks;
  return RCSA_OK;
}

}  // namespace rcsa

using namespace rcsa;

extern "C" int rcsa_sparse_attn_bf16(
    const void* Q, const void* K, const void* V, const uint8_t* K_valid, float sm_scale,
    float* M, void* Out, const int32_t* block_indices, const int32_t* block_indices_lens,
    int64_t stride_qz, int64_t stride_qh, int64_t stride_qm, int64_t stride_kz,
    int64_t stride_kh, int64_t stride_kn, int64_t stride_vz, int64_t stride_vh,
    int64_t stride_vn, int64_t stride_oz, int64_t stride_oh, int64_t stride_om,
    int64_t stride_bz, int64_t stride_bh, int64_t stride_bm, int64_t stride_lz,
    int64_t stride_lh, int64_t stride_lm, int64_t B, int64_t H, int64_t Q_LEN,
    int64_t K_LEN, int64_t HEAD_DIM, int64_t BLOCK_M, int64_t BLOCK_N, int64_t max_k,
    hipStream_t stream) {
  if (!Q || !K || !V) return RCSA_ERR_NULL;
  if (!aligned16(Q) || !aligned16(K) || !aligned16(V)) return RCSA_ERR_ALIGN;
  AttnArgs a{};
  a.q = Q;
  a.k = K;
  a.v = static_cast<const u16*>(V);
  int st = fill_common(a, K_valid, sm_scale, M, Out, block_indices, block_indices_lens,
                       stride_qz, stride_qh, stride_qm, stride_kz, stride_kh, stride_kn,
                       stride_vz, stride_vh, stride_vn, stride_oz, stride_oh, stride_om,
                       stride_bz, stride_bh, stride_bm, stride_lz, stride_lh, stride_lm, B,
                       H, Q_LEN, K_LEN, HEAD_DIM, BLOCK_M, BLOCK_N, max_k, 8);
  if (st) return st;
  if (a.n_work == 0) return RCSA_OK;
  return launch_attn<false>(a, HEAD_DIM, BLOCK_M, BLOCK_N, stream);
}

extern "C" int rcsa_sparse_attn_int8(
    const int8_t* Q, const float* q_scale, int64_t q_scale_stride, const int8_t* K,
    const float* k_scale, int64_t k_scale_stride, const void* V, const uint8_t* K_valid,
    float sm_scale, float* M, void* Out, const int32_t* block_indices,
    const int32_t* block_indices_lens, int64_t stride_qz, int64_t stride_qh,
    int64_t stride_qm, int64_t stride_kz, int64_t stride_kh, int64_t stride_kn,
    int64_t stride_vz, int64_t stride_vh, int64_t stride_vn, int64_t stride_oz,
    int64_t stride_oh, int64_t stride_om, int64_t stride_bz, int64_t stride_bh,
    int64_t stride_bm, int64_t stride_lz, int64_t stride_lh, int64_t stride_lm, int64_t B,
    int64_t H, int64_t Q_LEN, int64_t K_LEN, int64_t HEAD_DIM, int64_t BLOCK_M,
    int64_t BLOCK_N, int64_t max_k, hipStream_t stream) {
  if (!Q || !K || !V || !q_scale || !k_scale) return RCSA_ERR_NULL;
  if (!aligned16(Q) || !aligned16(K) || !aligned16(V)) return RCSA_ERR_ALIGN;
  AttnArgs a{};
  a.q = Q;
  a.k = K;
  a.v = static_cast<const u16*>(V);
  a.q_scale = q_scale;
  a.k_scale = k_scale;
  a.q_scale_stride = q_scale_stride;
  a.k_scale_stride = k_scale_stride;
  int st = fill_common(a, K_valid, sm_scale, M, Out, block_indices, block_indices_lens,
                       stride_qz, stride_qh, stride_qm, stride_kz, stride_kh, stride_kn,
                       stride_vz, stride_vh, stride_vn, stride_oz, stride_oh, stride_om,
                       stride_bz, stride_bh, stride_bm, stride_lz, stride_lh, stride_lm, B,
                       H, Q_LEN, K_LEN, HEAD_DIM, BLOCK_M, BLOCK_N, max_k, 16);
  if (st) return st;
  if (q_scale_stride < a.n_qblocks || k_scale_stride < a.n_kblocks) return RCSA_ERR_STRIDE;
  if (a.n_work == 0) return RCSA_OK;
  return launch_attn<true>(a, HEAD_DIM, BLOCK_M, BLOCK_N, stream);
}
