// Block-sparse flash attention for gfx950 (MI355X).
//
// One workgroup = one (batch, head, query block) = BLOCK_M query rows, one
// wavefront per 32 rows.  The workgroup streams only the key blocks named in
// its block list: each selected K tile and V tile is staged in LDS once and
// shared by all wavefronts.
//
// Orientation: every wavefront computes S^T = K Q^T with 32x32 MFMAs, so a
// lane owns ONE query row (column lane%32 of the MFMA output) and holds 16
// of every 32 keys in registers.  Row max / row sum are then in-lane, plus a
// single exchange with the partner lane (lane ^ 32).  The key rows fed to the
// A operand are permuted (pi below) so that lane half h holds the 16
// CONSECUTIVE keys 16h..16h+15 of each 32-key tile; P^T then feeds the B
// operand of O^T = V^T P^T directly from registers, and the matching V^T
// operand is one 16-byte LDS read.  V is transposed once while it is staged
// into LDS.
//
// QK^T runs on v_mfma_i32_32x32x32_i8 (int8 path) or
// v_mfma_f32_32x32x16_bf16 (bf16 path); PV on v_mfma_f32_32x32x16_bf16.
// Softmax is online, in fp32, in the exp2 domain (log2(e) folded into the
// logit scale).
#include <type_traits>

#include "rcsa_common.h"

namespace rcsa {

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

// Row permutation of the QK A operand (see header comment): MFMA row
// m = 8a + 4h + b feeds key 16h + 4a + b.
__device__ __forceinline__ int key_perm(int m) {
  return 16 * ((m >> 2) & 1) + 4 * (m >> 3) + (m & 3);
}
// 16-byte chunk swizzles that keep the LDS reads bank-conflict free.
__device__ __forceinline__ int swz_k(int row) { return (row & 3) | ((row >> 2) & 4); }
__device__ __forceinline__ int swz_v(int d) { return d + (d >> 3); }

template <bool INT8, int D, int BM, int BN>
__global__ void __launch_bounds__(BM * 2)
sparse_attn_kernel(AttnArgs a) {
  constexpr int NT = BM * 2;                   // threads (BM/32 wavefronts)
  constexpr int KB = INT8 ? 1 : 2;             // bytes per K element
  constexpr int KROW = D * KB;                 // bytes per staged K row
  constexpr int CPR_K = KROW / 16;             // 16-byte chunks per K row
  constexpr int VROW = BN * 2;                 // bytes per staged V^T row
  constexpr int CPR_V = BN / 8;
  constexpr int QSTEPS = INT8 ? D / 32 : D / 16;
  constexpr int NKT = BN / 32;                 // 32-key tiles per block
  constexpr int NDT = D / 32;                  // 32-wide head_dim tiles
  static_assert(QSTEPS * 2 == CPR_K, "K chunk layout");

  __shared__ __attribute__((aligned(16))) char s_k[BN * KROW];
  __shared__ __attribute__((aligned(16))) char s_v[D * VROW];

  const int64_t work = xcd_remap(blockIdx.x, a.n_work);
  if (work < 0) return;
  const int64_t qb = work % a.n_qblocks;
  const int64_t bh = work / a.n_qblocks;
  const int64_t b = bh / a.H, h = bh % a.H;

  const int tid = threadIdx.x;
  const int lane = tid % kWave, wave = tid / kWave;
  const int hf = lane >> 5, lr = lane & 31;
  const int64_t qrow = qb * BM + wave * 32 + lr;
  const bool qrow_ok = qrow < a.q_len;

  // Q operand (B of S^T = K Q^T): lane holds 16 contiguous bytes per step,
  // lane half hf covering the row's bytes [hf*KROW/2, (hf+1)*KROW/2).
  typedef typename std::conditional<INT8, v4i, v8bf>::type OpT;
  typedef typename std::conditional<INT8, v16i, v16f>::type AccT;
  OpT q_op[QSTEPS];
  {
    const char* qp = static_cast<const char*>(a.q) +
                     (b * a.sqz + h * a.sqh + qrow * a.sqm) * KB;
#pragma unroll
    for (int st = 0; st < QSTEPS; ++st) {
      v4i raw = {0, 0, 0, 0};
      if (qrow_ok) raw = *reinterpret_cast<const v4i*>(qp + (hf * QSTEPS + st) * 16);
      q_op[st] = __builtin_bit_cast(OpT, raw);
    }
  }
  const float qs = INT8 ? a.q_scale[bh * a.q_scale_stride + qb] : 1.0f;

  v16f o_acc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) o_acc[dt][r] = 0.0f;
  float m_run = -INFINITY;  // running max, log2 domain
  float l_run = 0.0f;       // partial row sum over this lane's keys

  int64_t cnt = a.lens[b * a.slz + h * a.slh + qb * a.slm];
  cnt = cnt < 0 ? 0 : (cnt > a.max_k ? a.max_k : cnt);
  const int32_t* list = a.idx + b * a.sbz + h * a.sbh + qb * a.sbm;

  const char* kbase = static_cast<const char*>(a.k) + (b * a.skz + h * a.skh) * KB;
  const u16* vbase = a.v + b * a.svz + h * a.svh;

  for (int64_t it = 0; it < cnt; ++it) {
    const int64_t n = list[it];
    if (n < 0 || n >= a.n_kblocks) continue;  // uniform across the workgroup
    const int64_t key0 = n * BN;

    __syncthreads();  // previous tile fully consumed
    // ---- stage K (row-major, chunk-swizzled) ----
#pragma unroll
    for (int pass = 0; pass < (BN * CPR_K + NT - 1) / NT; ++pass) {
      const int e = tid + pass * NT;
      if (e >= BN * CPR_K) break;
      const int row = e / CPR_K, c = e % CPR_K;
      v4i val = {0, 0, 0, 0};
      if (key0 + row < a.k_len)
        val = *reinterpret_cast<const v4i*>(kbase + (key0 + row) * a.skn * KB + c * 16);
      *reinterpret_cast<v4i*>(s_k + row * KROW + ((c ^ (swz_k(row) & (CPR_K - 1))) * 16)) = val;
    }
    // ---- stage V transposed: s_v[d][key] ----
#pragma unroll
    for (int pass = 0; pass < ((BN / 4) * (D / 8) + NT - 1) / NT; ++pass) {
      const int e = tid + pass * NT;
      if (e >= (BN / 4) * (D / 8)) break;
      const int dc = e % (D / 8), kg = e / (D / 8);
      uint4 r4[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t key = key0 + 4 * kg + i;
        r4[i] = key < a.k_len
                    ? *reinterpret_cast<const uint4*>(vbase + key * a.svn + dc * 8)
                    : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int dp = 0; dp < 8; ++dp) {
        uint32_t x[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t w = (dp >> 1) == 0 ? r4[i].x : (dp >> 1) == 1 ? r4[i].y
                           : (dp >> 1) == 2 ? r4[i].z : r4[i].w;
          x[i] = w;
        }
        uint32_t lo, hi;
        if (dp & 1) {
          lo = (x[0] >> 16) | (x[1] & 0xffff0000u);
          hi = (x[2] >> 16) | (x[3] & 0xffff0000u);
        } else {
          lo = (x[0] & 0xffffu) | (x[1] << 16);
          hi = (x[2] & 0xffffu) | (x[3] << 16);
        }
        const int d = dc * 8 + dp;
        const int chunk = (kg >> 1) ^ (swz_v(d) & (CPR_V - 1));
        *reinterpret_cast<uint2*>(s_v + d * VROW + chunk * 16 + (kg & 1) * 8) =
            make_uint2(lo, hi);
      }
    }
    // ---- key validity of this block (uniform bitmasks) ----
    uint64_t vmask[(BN + 63) / 64];
    bool all_valid = true;
#pragma unroll
    for (int w = 0; w < (BN + 63) / 64; ++w) {
      const int64_t key = key0 + w * 64 + lane;
      const bool ok = (w * 64 + lane < BN) && key < a.k_len &&
                      (a.kvalid == nullptr || a.kvalid[key] != 0);
      vmask[w] = __ballot(ok);
      const uint64_t full = (BN - w * 64 >= 64) ? ~0ull : ((1ull << (BN - w * 64)) - 1ull);
      all_valid = all_valid && (vmask[w] == full);
    }
    __syncthreads();

    // ---- S^T = K Q^T ----
    AccT s_acc[NKT];
#pragma unroll
    for (int t = 0; t < NKT; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s_acc[t][r] = 0;
      const int row = 32 * t + key_perm(lr);
      const char* rp = s_k + row * KROW;
      const int sw = swz_k(row) & (CPR_K - 1);
#pragma unroll
      for (int st = 0; st < QSTEPS; ++st) {
        const v4i raw = *reinterpret_cast<const v4i*>(rp + (((hf * QSTEPS + st) ^ sw) * 16));
        if constexpr (INT8) {
          s_acc[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(raw, q_op[st], s_acc[t], 0, 0, 0);
        } else {
          s_acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              __builtin_bit_cast(v8bf, raw), q_op[st], s_acc[t], 0, 0, 0);
        }
      }
    }

    // ---- online softmax (lane half hf, register r <-> key 32t + 16hf + r) ----
    const float c = INT8 ? a.scale_log2 * qs * a.k_scale[bh * a.k_scale_stride + n]
                         : a.scale_log2;
    float p[NKT][16];
    float mx = -INFINITY;
    if (all_valid) {
      if constexpr (INT8) {
        int mi = INT32_MIN;
#pragma unroll
        for (int t = 0; t < NKT; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) mi = max(mi, s_acc[t][r]);
        mx = static_cast<float>(mi) * c;
      } else {
#pragma unroll
        for (int t = 0; t < NKT; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s_acc[t][r]);
        mx *= c;
      }
    } else {
#pragma unroll
      for (int t = 0; t < NKT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kk = 32 * t + 16 * hf + r;
          const bool ok = (vmask[kk >> 6] >> (kk & 63)) & 1ull;
          const float x = static_cast<float>(s_acc[t][r]) * c;
          mx = ok ? fmaxf(mx, x) : mx;
        }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
    // A row with nothing admissible so far keeps m = -inf, alpha = 1 and
    // p = 0 (masked lanes are zeroed below); no divergent branch around MFMA.
    const float m_new = fmaxf(m_run, mx);
    const bool live = m_new != -INFINITY;
    const float alpha = live ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
    const float m_sub = live ? m_new : 0.0f;
    m_run = m_new;
    float lsum = 0.0f;
#pragma unroll
    for (int t = 0; t < NKT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float e = __builtin_amdgcn_exp2f(static_cast<float>(s_acc[t][r]) * c - m_sub);
        if (!all_valid) {
          const int kk = 32 * t + 16 * hf + r;
          e = ((vmask[kk >> 6] >> (kk & 63)) & 1ull) ? e : 0.0f;
        }
        p[t][r] = e;
        lsum += e;
      }
    l_run = l_run * alpha + lsum;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) o_acc[dt][r] *= alpha;

    // ---- O^T += V^T P^T ----
#pragma unroll
    for (int t = 0; t < NKT; ++t) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        v8bf p_op;
#pragma unroll
        for (int j = 0; j < 8; ++j) p_op[j] = static_cast<__bf16>(p[t][8 * u + j]);
        const int chunk = 4 * t + 2 * hf + u;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          const int d = 32 * dt + lr;
          const v8bf v_op = *reinterpret_cast<const v8bf*>(
              s_v + d * VROW + ((chunk ^ (swz_v(d) & (CPR_V - 1))) * 16));
          o_acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v_op, p_op, o_acc[dt], 0, 0, 0);
        }
      }
    }
  }

  // ---- epilogue: normalise, write O (bf16) and the log-sum-exp ----
  const float l_tot = l_run + __shfl_xor(l_run, 32, kWave);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  if (qrow_ok) {
    u16* op = a.out + b * a.soz + h * a.soh + qrow * a.som;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = 32 * dt + 8 * g + 4 * hf;
        const uint32_t lo = pack_bf16x2(o_acc[dt][4 * g] * inv, o_acc[dt][4 * g + 1] * inv);
        const uint32_t hi = pack_bf16x2(o_acc[dt][4 * g + 2] * inv, o_acc[dt][4 * g + 3] * inv);
        *reinterpret_cast<uint2*>(op + d0) = make_uint2(lo, hi);
      }
    if (a.lse && hf == 0) {
      a.lse[(b * a.H + h) * a.q_len + qrow] =
          l_tot > 0.0f ? (m_run + __log2f(l_tot)) * 0.69314718055994531f : -INFINITY;
    }
  }
}

template <bool INT8>
static int launch_attn(AttnArgs& a, int64_t D, int64_t BM, int64_t BN, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(xcd_grid(a.n_work)));
#define RCSA_ATTN(D_, BM_, BN_)                                            \
  if (D == D_ && BM == BM_ && BN == BN_) {                                 \
    sparse_attn_kernel<INT8, D_, BM_, BN_><<<grid, dim3(BM_ * 2), 0, s>>>(a); \
    return launch_status();                                                \
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
  // 16-byte aligned rows: bf16 strides multiple of 8, int8 multiple of 16
  if (sqm % kvec || sqh % kvec || sqz % kvec) return RCSA_ERR_STRIDE;
  if (skn % kvec || skh % kvec || skz % kvec) return RCSA_ERR_STRIDE;
  if (svn % 8 || svh % 8 || svz % 8) return RCSA_ERR_STRIDE;
  if (som % 4 || soh % 4 || soz % 4) return RCSA_ERR_STRIDE;
  if (!aligned16(Out) && (reinterpret_cast<uintptr_t>(Out) & 7u)) return RCSA_ERR_ALIGN;
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
