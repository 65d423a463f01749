// Block-sparse attention kernels for gfx950: the kernel template, its
// helpers and the merge pass, included by the sources that instantiate and
// launch them (sparse_attn.hip, sparse_attn_bf16_gather.hip).
//
// Block-sparse flash attention for gfx950 (MI355X).
//
// Work decomposition: one workgroup = one (batch, head, query block) of
// BLOCK_M rows; it streams only the key blocks named in its block list.
// The workgroup has NKH * BLOCK_M / 32 wavefronts: row group rg (32 query
// rows) x key half kh.  With NKH = 2 the two key halves keep independent
// online-softmax states that are merged once at the end, so eight wavefronts
// share every staged tile (two per SIMD, one workgroup per compute unit).
// With NKH = 1 and WPE = 3 a workgroup of four wavefronts takes whole ring
// steps and three workgroups share a compute unit.
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
// (rescaling O is skipped otherwise).  Row sums accumulate the fp32
// probabilities (P is rounded to bf16 only as the PV operand).
#pragma once
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
  const uint32_t* kmask;  // validity bits per key (32 per word), replaces kvalid
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
  int64_t H, q_len, k_len, n_qblocks, n_kblocks, max_k, block_m;
  // Work: n_items = B*H*n_qblocks query blocks.  XCD x runs query blocks
  // [x xcd_items, (x+1) xcd_items): the first xcd_direct whole, the rest
  // (those that would run in a round leaving compute units idle) in n_split
  // shares each.  Tail query block t of XCD x has tail index
  // x (xcd_items - xcd_direct) + t < n_tail; its shares' normalised partial
  // outputs go to ws_o [n_split][n_tail][block_m][D] (bf16) and their
  // (max, sum) pairs to ws_ml [n_split][n_tail][block_m] for attn_merge_kernel.
  int64_t n_bh, n_items, xcd_items, xcd_direct, n_split, n_tail;
  u16* ws_o;
  float2* ws_ml;
  // Output scatter (nullable): packed query row r goes to row out_tok[r] of
  // Out and M (out_len rows per (b, h)); -1 or a row >= out_len is dropped.
  const int32_t* out_tok;
  int64_t out_len;
  // Gathered sources (GATHER kernels only): packed key slot s reads row
  // kv_tok[s] of a token-major V (and, bf16, K) with kv_len token rows; -1
  // or a row >= kv_len is an empty slot (zeros).  bf16 query row r reads row
  // q_tok[r] of a token-major Q of q_src_len rows (zeros when empty).
  const int32_t* kv_tok;
  int64_t kv_len;
  const int32_t* q_tok;
  int64_t q_src_len;
};

// Output row of packed query row r, or -1 when the row is not written.
__device__ __forceinline__ int64_t out_row(const AttnArgs& a, int64_t r) {
  if (a.out_tok == nullptr) return r;
  const int32_t t = a.out_tok[r];
  return (t < 0 || t >= a.out_len) ? -1 : t;
}

constexpr float kTau = 8.0f;               // lazy-rescale threshold, log2 units
constexpr float kTauPow = 256.0f;          // 2^kTau
constexpr float kMagicF = 12582912.0f;     // 1.5 * 2^23
constexpr int kMagicI = 0x4B400000;        // its fp32 bit pattern

// MFMA row m = 8a + 4h + b of a 32-key tile reads key 16h + 4a + b.
__device__ __forceinline__ int key_perm(int m) {
  return 16 * ((m >> 2) & 1) + 4 * (m >> 3) + (m & 3);
}
// 16-byte chunk swizzles.  LDS serves 256 bytes per clock from 64 four-byte
// banks.  A ds_read_b128 of the K operand serves 16 lanes per clock, which
// read the permuted rows {0-7, 16-23} (or {8-15, 24-31}, plus 32t and the key
// half): rows that share a 256-byte bank line (row / (256 / KROW) equal
// modulo the line) get distinct chunk XORs, so the 16 reads hit 16 distinct
// 16-byte bank groups.  V rows XOR by 4 * (row mod 4), which keeps the
// ds_read_b64_tr_b16 groups of 4 rows conflict free.
template <int KROW>
__device__ __forceinline__ int swz_k(int row) {
  constexpr int RPL = 256 / KROW;     // rows per bank line: 1, 2 or 4
  constexpr int M = KROW / 16 / 2;    // half the chunks of a row
  const int q = row / RPL;
  return (q & (M - 1)) | ((q >> 1) & M);
}
__device__ __forceinline__ int swz_v(int row) { return 4 * (row & 3); }

// s_waitcnt immediate that waits for vmcnt <= n only (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] at [15:14]).
constexpr int vmcnt_imm(int n) {
  return (n & 0xf) | (0x7 << 4) | (0xf << 8) | (((n >> 4) & 0x3) << 14);
}

// Load through the constant address space: read-only inputs (block lists,
// scales) then go through the scalar unit (lgkmcnt) instead of a vector load
// whose vmcnt wait would also drain the direct-to-LDS copies in flight.
template <typename T>
__device__ __forceinline__ T ld_const(const T* p) {
  return *(const __attribute__((address_space(4))) T*)(p);
}

// Wait until at most N vector-memory operations of this wavefront are
// outstanding, then barrier the workgroup.  Unlike __syncthreads(), whose
// workgroup fences drain every outstanding direct-to-LDS copy, this keeps the
// younger ring stages in flight.  The memory clobber keeps the compiler from
// moving LDS accesses across it.
template <int N>
__device__ __forceinline__ void wait_vm_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

// v[lane] + v[lane ^ 32] through v_permlane32_swap.
__device__ __forceinline__ float pair_sum(float v) {
  const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                   false, false);
  return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
}

// max(v[lane], v[lane ^ 32]) through v_permlane32_swap (no LDS round trip).
__device__ __forceinline__ float pair_max(float v) {
  const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                   false, false);
  return fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
}

// Validity bytes of a key block when K_valid is NULL.
#define RCSA_ONES16 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1
static __device__ uint8_t kAllValid[128] = {RCSA_ONES16, RCSA_ONES16, RCSA_ONES16, RCSA_ONES16,
                                     RCSA_ONES16, RCSA_ONES16, RCSA_ONES16, RCSA_ONES16};
#undef RCSA_ONES16

// BNS keys of a block are staged per ring step (BN / BNS steps per selected
// block); NKH key halves split every staged step between wavefronts.  WPE > 0:
// several workgroups share a compute unit, WPE waves per SIMD in all (a
// register budget of 512 / WPE); 0: one workgroup per compute unit.
template <bool INT8, int D, int BM, int BN, int STAGES, int BNS, int NKH, int WPE = 0>
struct AttnCfg {
  static constexpr int NRG = BM / 32;            // row groups
  static constexpr int NW = NRG * NKH;           // wavefronts: row group x key half
  static constexpr int NT = NW * 64;             // threads
  static constexpr int SUB = BN / BNS;           // ring steps per selected block
  static constexpr int KB = INT8 ? 1 : 2;        // bytes per K element
  static constexpr int KROW = D * KB;            // bytes per staged K row
  static constexpr int CPR_K = KROW / 16;
  static constexpr int VROW = D * 2;             // bytes per staged V row
  static constexpr int CPR_V = VROW / 16;
  static constexpr int QSTEPS = INT8 ? D / 32 : D / 16;
  static constexpr int HK = BNS / NKH;           // keys per wavefront per step
  static constexpr int KT = HK / 32;             // 32-key tiles per wavefront
  static constexpr int NDT = D / 32;             // 32-wide head_dim tiles
  static constexpr int KBYTES = BNS * KROW;
  static constexpr int VBYTES = BNS * VROW;
  static constexpr int BUF = KBYTES + VBYTES;    // one ring slot: K tile then V tile
  static constexpr int KUNITS = KBYTES / 1024;   // 1 KiB direct-to-LDS copies
  static constexpr int VUNITS = VBYTES / 1024;
  static constexpr int KUPW = (KUNITS + NW - 1) / NW;  // copies per wavefront
  static constexpr int VUPW = (VUNITS + NW - 1) / NW;
  static constexpr int DMA = KUPW + VUPW;
  static constexpr int K_RPU = 1024 / KROW;      // rows per copy
  static constexpr int V_RPU = 1024 / VROW;
  static constexpr int MW = NDT * 16 * 64 + 128; // floats of one row group's merge partial
  static constexpr int MPER = (NRG + STAGES - 1) / STAGES;  // partials per slot
  // a 3-slot ring's slots are grown to hold the key-half merge partials (the
  // 64-key bf16 ring: 2 x 16.5 KiB in each 32.25 KiB slot); workgroups that
  // share a compute unit have one key half and no merge
  static constexpr int SLOT = (WPE == 0 && STAGES == 3 && MPER * MW * 4 > BUF + 256)
                                  ? MPER * MW * 4 : BUF + 256;
  static constexpr bool MERGE_IN_SLOTS = MPER * MW * 4 <= SLOT;
  // the vmcnt accounting of a 3-deep ring needs the same copy count on every wavefront
  static_assert(STAGES == 2 || (KUNITS % NW == 0 && VUNITS % NW == 0), "uneven copies");
  static_assert(QSTEPS * 2 == CPR_K, "K chunk layout");
  static_assert(STAGES == 2 || STAGES == 3, "ring depth");
  static_assert((NKH == 1 || NKH == 2) && HK % 32 == 0 && BN % BNS == 0, "key split");
  static_assert(BNS <= 256, "validity bytes of one step fit the slot tail");
  static_assert(WPE == 0 || NKH == 1, "workgroups sharing a compute unit merge no key halves");
};

// Direct-to-LDS copy of 16 (4) bytes per lane through a buffer resource over
// [base, base + bytes): a lane whose bytes do not fit below `bytes` reads
// zeros and touches no memory.
// (The LDS destination is passed as a generic pointer: an LDS-typed
// parameter makes the host pass of the kernel templates drop their stubs.)
constexpr int kRsrcWord3 = 0x00020000;  // raw untyped buffer, 32-bit data format
__device__ __forceinline__ void buffer_copy16(char* base, int bytes, uint32_t voff, char* dst) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(base, 0, bytes, kRsrcWord3);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, RCSA_LDS(void, dst), 16, voff, 0, 0, 0);
}
__device__ __forceinline__ void buffer_copy4(char* base, int bytes, uint32_t voff, char* dst) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(base, 0, bytes, kRsrcWord3);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, RCSA_LDS(void, dst), 4, voff, 0, 0, 0);
}

// Waves per SIMD the register budget is sized for: WPE when several
// workgroups share a compute unit, otherwise at least the workgroup's own.
template <int NT, int WPE>
constexpr int attn_waves_min() { return WPE > 0 ? WPE : (NT / 256 > 1 ? NT / 256 : 1); }
template <int WPE>
constexpr int attn_waves_max() { return WPE > 0 ? WPE : 8; }

template <bool INT8, int D, int BM, int BN, int STAGES, int BNS, int NKH, bool MASK,
          bool GATHER = false, int WPE = 0>
__global__ void __launch_bounds__(BM * 2 * NKH)  // == AttnCfg::NT
__attribute__((amdgpu_waves_per_eu(attn_waves_min<BM * 2 * NKH, WPE>(), attn_waves_max<WPE>())))
sparse_attn_kernel(AttnArgs a) {
  using C = AttnCfg<INT8, D, BM, BN, STAGES, BNS, NKH, WPE>;
  typedef typename std::conditional<INT8, v4i, v8bf>::type OpT;
  // A 3-slot ring issues its copies between the PV MFMAs, every wavefront
  // the same kOps copies per ring step (validity bytes included)
  constexpr bool kDmaInPv = STAGES == 3;
  // Rings of several steps per key block run whole rounds of STAGES steps (up
  // to STAGES - 1 masked steps past the list, a fraction of a block); a ring of
  // one step per block stops at the list's end, and so do the gathered rings
  // (their scalar registers spill more with the padded loop, 56 -> 71 SGPRs in
  // the int8 kernel).
  constexpr bool kPadRounds = kDmaInPv && BN / BNS > 1 && !GATHER;
  // validity bytes ride along with the copies unless the caller passes the
  // validity bits (MASK: read with scalar loads instead)
  constexpr bool kValidCopy = kDmaInPv && !MASK;
  constexpr int kOps = C::DMA + (kValidCopy ? 1 : 0);
  // GATHER: every ring step also reads, one step ahead, the slot-map entries
  // of the VUPW V rows (bf16: and the same K rows) its lane copies
  constexpr int kTok = GATHER ? C::VUPW : 0;
  static_assert(!GATHER || (kDmaInPv && MASK), "gathered sources ride the 3-slot ring with bits");
  static_assert(!GATHER || INT8 || (C::KUPW == C::VUPW && C::K_RPU == C::V_RPU &&
                                    C::CPR_K == C::CPR_V), "bf16 K and V rows share tokens");
  typedef typename std::conditional<INT8, v16i, v16f>::type AccT;
  // Ring slots are separate arrays and the loop is unrolled over them, so
  // the compiler can prove that reads of slot j do not alias the copies in
  // flight into the other slots (it would otherwise drain them first).
  __shared__ __attribute__((aligned(1024))) char s_0[C::SLOT];
  __shared__ __attribute__((aligned(1024))) char s_1[C::SLOT];
  __shared__ __attribute__((aligned(1024))) char s_2[STAGES > 2 ? C::SLOT : 16];
  __shared__ __attribute__((aligned(16)))
  char s_m[NKH == 1 || C::MERGE_IN_SLOTS ? 16 : C::NRG * C::MW * 4];

  // Workgroups go to the XCDs round-robin: XCD x runs a contiguous run of
  // query blocks (neighbouring query blocks of a head share its L2), whole
  // ones first, then the shares of its tail query blocks back to back.
  // (32-bit decode: the host keeps work items below 2^31)
  const uint32_t xcd = blockIdx.x % kNumXcd, slot = blockIdx.x / kNumXcd;
  const uint32_t x_items = static_cast<uint32_t>(a.xcd_items);
  const uint32_t x_direct = static_cast<uint32_t>(a.xcd_direct);
  const bool is_share = slot >= x_direct;  // a share of a tail query block
  const uint32_t tailpos = slot - x_direct;
  const uint32_t nsp = is_share ? static_cast<uint32_t>(a.n_split) : 1u;
  const uint32_t split = is_share ? tailpos % nsp : 0u;
  const uint32_t in_xcd = is_share ? x_direct + tailpos / nsp : slot;
  const uint32_t item = xcd * x_items + in_xcd;
  if (in_xcd >= x_items || item >= static_cast<uint32_t>(a.n_items)) return;
  const int64_t tail = static_cast<int64_t>(xcd) * (x_items - x_direct) +
                       (static_cast<int64_t>(in_xcd) - x_direct);
  const uint32_t nqb32 = static_cast<uint32_t>(a.n_qblocks), h32 = static_cast<uint32_t>(a.H);
  const int64_t qb = item % nqb32;
  const uint32_t bh32 = item / nqb32;
  const int64_t bh = bh32;
  const int64_t b = bh32 / h32, h = bh32 % h32;

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // uniform: SGPR arithmetic
  const int rg = wave % C::NRG, kh = wave / C::NRG;
  const int hf = lane >> 5, lr = lane & 31;
  const int64_t qrow = qb * BM + rg * 32 + lr;
  bool qrow_ok = qrow < a.q_len;
  int64_t qsrc = qrow;  // source row of the Q load
  if constexpr (GATHER && !INT8) {  // bf16 queries are read through the query map
    const int32_t t = qrow_ok ? a.q_tok[qrow] : -1;
    qrow_ok = t >= 0 && t < a.q_src_len;
    qsrc = t;
  }

  // Workgroup-uniform list length and query-block scale, through the scalar
  // cache, issued ahead of the Q loads so the two latencies overlap.
  int64_t cnt = ld_const(a.lens + (b * a.slz + h * a.slh + qb * a.slm));
  const float qs = INT8 ? ld_const(a.q_scale + (bh * a.q_scale_stride + qb)) : 1.0f;

  // Q operand (B of S^T = K Q^T): lane half hf holds the row's bytes
  // [hf*KROW/2, (hf+1)*KROW/2) as QSTEPS 16-byte steps.
  OpT q_op[C::QSTEPS];
  {
    const char* qp = static_cast<const char*>(a.q) +
                     (b * a.sqz + h * a.sqh + qsrc * a.sqm) * C::KB;
#pragma unroll
    for (int st = 0; st < C::QSTEPS; ++st) {
      v4i raw = {0, 0, 0, 0};
      if (qrow_ok) raw = *reinterpret_cast<const v4i*>(qp + (hf * C::QSTEPS + st) * 16);
      q_op[st] = __builtin_bit_cast(OpT, raw);
    }
  }
  // Q must be resident before the ring starts: otherwise its pending loads
  // meet the loop's back edge and the compiler drains at the first MFMA.
  // A 3-slot ring waits for them after issuing its two prologue stages
  // (counted below); the other rings wait here.
  if constexpr (!kDmaInPv) __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));

  v16f o_acc[C::NDT];
#pragma unroll
  for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) o_acc[dt][r] = 0.0f;
  float m_run = -INFINITY;  // running max (log2 domain), shared by both lane halves
  float l_run = 0.0f;       // this lane's partial row sum

  cnt = cnt < 0 ? 0 : (cnt > a.max_k ? a.max_k : cnt);
  const int32_t* list = a.idx + b * a.sbz + h * a.sbh + qb * a.sbm;
  {  // this workgroup's share of the list (shares differ by at most one block)
    // (cnt < 2^24 and split < 16: the products fit in 32 bits)
    const uint32_t c32 = static_cast<uint32_t>(cnt);
    const int64_t begin = c32 * split / nsp, end = c32 * (split + 1) / nsp;
    list += begin;
    cnt = end - begin;
  }
  const int steps = static_cast<int>(cnt) * C::SUB;  // ring steps of BNS keys
  const char* kbase = static_cast<const char*>(a.k) + (b * a.skz + h * a.skh) * C::KB;
  const char* vbase = reinterpret_cast<const char*>(a.v + b * a.svz + h * a.svh);
  // Key and block numbers are 32-bit (the host keeps K_LEN below 2^31), so
  // the per-block scalar arithmetic stays on the scalar unit.
  const int klen = static_cast<int>(a.k_len), klast = klen - 1;
  const int nkb = static_cast<int>(a.n_kblocks);
  const int64_t krow_bytes = a.skn * C::KB, vrow_bytes = a.svn * 2;

  // Direct-to-LDS staging: copy u of a K (V) tile holds K_RPU (V_RPU) rows;
  // lane l lands at byte l*16 of it, so it loads the swizzled global chunk
  // that belongs there.  A block's source address is a uniform 64-bit base
  // plus a loop-invariant 32-bit lane offset.
  auto k_row = [&](int i) __attribute__((always_inline)) { return (wave * C::KUPW + i) * C::K_RPU + lane / C::CPR_K; };
  auto v_row = [&](int i) __attribute__((always_inline)) { return (wave * C::VUPW + i) * C::V_RPU + lane / C::CPR_V; };
  auto k_col = [&](int i) __attribute__((always_inline)) { return ((lane % C::CPR_K) ^ (swz_k<C::KROW>(k_row(i)) & (C::CPR_K - 1))) * 16; };
  auto v_col = [&](int i) __attribute__((always_inline)) { return ((lane % C::CPR_V) ^ (swz_v(v_row(i)) & (C::CPR_V - 1))) * 16; };
  // (gathered rows: the row part comes from the slot map at copy time, so
  // only the column part is kept)
  constexpr bool kGatherK = GATHER && !INT8;
  uint32_t k_lo[C::KUPW], v_lo[C::VUPW];
#pragma unroll
  for (int i = 0; i < C::KUPW; ++i)
    k_lo[i] = (kGatherK ? 0u : static_cast<uint32_t>(k_row(i) * krow_bytes)) + k_col(i);
#pragma unroll
  for (int i = 0; i < C::VUPW; ++i)
    v_lo[i] = (GATHER ? 0u : static_cast<uint32_t>(v_row(i) * vrow_bytes)) + v_col(i);
  // Copy step n (BNS keys from key n*BNS; clamped to 0 when invalid) into a
  // slot.  Rows past k_len re-read the last row (those keys are masked).
  // (Named source pointers: an inline pointer expression as this builtin's
  // source argument makes the host pass drop the kernel stub.)
  // Branch-free variant for the 3-slot ring: the copies of a step go through
  // buffer resources that end at the step's last valid row, so each lane
  // keeps its loop-invariant offset and rows past K_LEN land as zeros (those
  // keys are masked); the copies then sit in the caller's basic block
  // between its MFMAs.
  const uint32_t krb = static_cast<uint32_t>(krow_bytes), vrb = static_cast<uint32_t>(vrow_bytes);
  // Gathered rows: lane l of copy i moves a chunk of slot v_row(i) =
  // v_row(0) + i V_RPU of the step, read from the slot map through a buffer
  // resource (map entries past K_LEN read as 0: none are asked for).  A row
  // goes through a resource over the whole (b, h) plane of the token-major
  // source (kv_len rows; the host keeps kv_len x row bytes below 2^31), and an
  // empty slot gets an offset past its end, so it lands as zeros.
  constexpr int kTokArr = kTok > 0 ? kTok : 1;
  const uint32_t kv_rows = static_cast<uint32_t>(a.kv_len);
  const uint32_t tok_lane = static_cast<uint32_t>(v_row(0)) * 4u;
  auto load_tokens = [&](int n, uint32_t (&tk)[kTokArr]) __attribute__((always_inline)) {
    if constexpr (GATHER) {
      const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<int32_t*>(a.kv_tok), 0, n < 0 ? 0 : klen * 4, kRsrcWord3);
      const int key0 = (n < 0 ? 0 : n) * BNS;
#pragma unroll
      for (int i = 0; i < kTok; ++i)
        tk[i] = static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(
            r, static_cast<int>(tok_lane) + i * C::V_RPU * 4, key0 * 4, 0));
    }
  };
  auto row_off = [&](uint32_t t, uint32_t row_bytes, uint32_t col) __attribute__((always_inline)) {
    return t < kv_rows ? t * row_bytes + col : 0x80000000u;
  };
  // A step past the list (n < 0) still issues its copies, so that every
  // ring wait counts the same operations, but through empty buffer ranges:
  // every lane is out of range, nothing is read from memory and the slot,
  // which nobody reads, fills with zeros.
  auto stage_flat = [&](int n, char* dst, const uint32_t (&tk)[kTokArr]) __attribute__((always_inline)) {
    if constexpr (GATHER) {
      char* const kb0 = const_cast<char*>(kbase);
      char* const vb0 = const_cast<char*>(vbase);
      if constexpr (INT8) {  // packed int8 keys: the step's rows as in the flat copy
        int key0 = (n < 0 ? 0 : n) * BNS;
        char* const kbs = kb0 + static_cast<uint64_t>(static_cast<uint32_t>(key0)) * krb;
        const int knum = n < 0 ? 0 : BNS * static_cast<int>(krb);
#pragma unroll
        for (int i = 0; i < C::KUPW; ++i)
          buffer_copy16(kbs, knum, k_lo[i], dst + (wave * C::KUPW + i) * 1024);
      } else {
        const int knum = n < 0 ? 0 : static_cast<int>(kv_rows * krb);
#pragma unroll
        for (int i = 0; i < C::KUPW; ++i)
          buffer_copy16(kb0, knum, row_off(tk[i], krb, k_lo[i]),
                        dst + (wave * C::KUPW + i) * 1024);
      }
      const int vnum = n < 0 ? 0 : static_cast<int>(kv_rows * vrb);
#pragma unroll
      for (int i = 0; i < C::VUPW; ++i)
        buffer_copy16(vb0, vnum, row_off(tk[i], vrb, v_lo[i]),
                      dst + C::KBYTES + (wave * C::VUPW + i) * 1024);
      return;
    }
    int key0 = (n < 0 ? 0 : n) * BNS;
    key0 = key0 > klast ? klast : key0;
    const int left = klen - key0;  // >= 1
    const int rows = n < 0 ? 0 : (left < BNS ? left : BNS);
    // (key0 and the row strides are below 2^31: 32 x 32 -> 64-bit products)
    char* const kb0 = const_cast<char*>(kbase) +
                      static_cast<uint64_t>(static_cast<uint32_t>(key0)) * krb;
    char* const vb0 = const_cast<char*>(vbase) +
                      static_cast<uint64_t>(static_cast<uint32_t>(key0)) * vrb;
    // rows * row bytes < 2^31: row strides stay below 16 MiB
    const int knum = rows * static_cast<int>(krb), vnum = rows * static_cast<int>(vrb);
#pragma unroll
    for (int i = 0; i < C::KUPW; ++i)
      buffer_copy16(kb0, knum, k_lo[i], dst + (wave * C::KUPW + i) * 1024);
#pragma unroll
    for (int i = 0; i < C::VUPW; ++i)
      buffer_copy16(vb0, vnum, v_lo[i], dst + C::KBYTES + (wave * C::VUPW + i) * 1024);
  };
  // validity bytes of step n, 4 per lane from every wavefront (lanes 32-63
  // repeat lanes 0-31 into the tail's unused half), through a buffer that
  // ends at the dword holding the last key (K_valid is readable up to its
  // next 16-byte boundary; bytes of keys past K_LEN are masked anyway)
  auto stage_valid_flat = [&](int n, char* dst) __attribute__((always_inline)) {
    static_assert(BNS <= 128, "validity bytes of a step: 32 lanes x 4");
    const int key0 = (n < 0 ? 0 : n) * BNS;  // a listed block starts below K_LEN
    const bool has = a.kvalid != nullptr;
    char* const vb = has ? reinterpret_cast<char*>(const_cast<uint8_t*>(a.kvalid)) + key0
                         : reinterpret_cast<char*>(kAllValid);
    const int left = n < 0 ? 0 : (has ? klen - key0 : BNS);
    const int vnum = ((left + 3) & ~3) < BNS ? ((left + 3) & ~3) : BNS;
    buffer_copy4(vb, vnum, 4u * (lane & 31), dst + C::BUF);
  };
  auto stage = [&](int n, char* dst) __attribute__((always_inline)) {
    const int64_t key0 = static_cast<int64_t>(n < 0 ? 0 : n) * BNS;
    const bool tail = key0 + BNS > a.k_len;
    const char* kb0 = kbase + key0 * krow_bytes;
    const char* vb0 = vbase + key0 * vrow_bytes;
#pragma unroll
    for (int i = 0; i < C::KUPW; ++i) {
      if (C::KUNITS % C::NW == 0 || wave * C::KUPW + i < C::KUNITS) {  // uniform per wavefront
        const char* src = tail ? kbase + min(key0 + k_row(i), int64_t{klast}) * krow_bytes + k_col(i)
                               : kb0 + k_lo[i];
        __builtin_amdgcn_global_load_lds(
            src, RCSA_LDS(void, dst + (wave * C::KUPW + i) * 1024), 16, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < C::VUPW; ++i) {
      if (C::VUNITS % C::NW == 0 || wave * C::VUPW + i < C::VUNITS) {
        const char* src = tail ? vbase + min(key0 + v_row(i), int64_t{klast}) * vrow_bytes + v_col(i)
                               : vb0 + v_lo[i];
        __builtin_amdgcn_global_load_lds(
            src, RCSA_LDS(void, dst + C::KBYTES + (wave * C::VUPW + i) * 1024), 16, 0, 0);
      }
    }
  };
  // Ring step `it`: step SUB*n + it%SUB of list entry n = list[it / SUB]
  // (-1 = invalid entry), a scalar load.
  auto block_step = [&](int n, int it) __attribute__((always_inline)) -> int {
    // one unsigned compare rejects both -1 padding and entries past the keys
    return static_cast<uint32_t>(n) < static_cast<uint32_t>(nkb) ? n * C::SUB + it % C::SUB : -1;
  };
  auto block_of = [&](int it) __attribute__((always_inline)) -> int {
    return block_step(ld_const(list + it / C::SUB), it);
  };
  auto fetch_scale = [&](int n) __attribute__((always_inline)) -> float {
    return INT8 ? ld_const(a.k_scale + bh * a.k_scale_stride + (n < 0 ? 0 : n / C::SUB))
                : 1.0f;
  };
  // The BNS validity bytes of a step ride along with its copies (BNS/16
  // lanes of wavefront 0, 16 bytes each) into the slot's 256-byte tail;
  // K_valid is 16-byte aligned and readable up to the next 16-byte boundary.
  auto stage_valid = [&](int n, char* dst) __attribute__((always_inline)) {
    if (a.kvalid != nullptr && wave == 0 && lane < BNS / 16) {
      const int64_t key0 = static_cast<int64_t>(n < 0 ? 0 : n) * BNS;
      const int64_t chunk = min(key0 + 16 * lane, (klast / 16) * 16);
      const char* src = reinterpret_cast<const char*>(a.kvalid) + chunk;
      __builtin_amdgcn_global_load_lds(src, RCSA_LDS(void, dst + C::BUF), 16, 0, 0);
    }
  };
  // validity of the wavefront's HK keys of step n from the caller's bits
  // (uniform scalar loads; keys past K_LEN are cleared)
  // (split in two: the raw words, loaded ahead, and the mask of step n)
  auto mask_words = [&](int n) __attribute__((always_inline)) -> uint2 {
    const uint32_t* w = a.kmask + ((n < 0 ? 0 : n) * BNS + kh * C::HK) / 32;
    return make_uint2(ld_const(w), C::HK == 64 ? ld_const(w + 1) : 0u);
  };
  // Only the step holding K_LEN can have keys past it: its keep mask for this
  // wavefront's half is computed once.
  const int tail_step = klen % BNS != 0 ? klen / BNS : -1;
  const uint64_t tail_keep = [&]() -> uint64_t {
    const int left = klen - (klen / BNS * BNS + kh * C::HK);
    return left >= C::HK ? ~0ull : (left <= 0 ? 0ull : ((1ull << left) - 1));
  }();
  auto mask_of = [&](int n, uint2 words) __attribute__((always_inline)) -> uint64_t {
    const uint64_t m = words.x | (static_cast<uint64_t>(words.y) << 32);
    return n < 0 ? 0ull : (n == tail_step ? m & tail_keep : m);
  };
  auto mask_bits = [&](int n) __attribute__((always_inline)) -> uint64_t {
    return mask_of(n, mask_words(n));
  };
  // Validity bits come from the caller when MASK is set; the 3-slot ring is
  // launched with MASK whenever the caller passes bits, so without MASK it
  // always takes the bytes (and drops the bit path at compile time).
  const bool use_bits = MASK || (!kDmaInPv && a.kmask != nullptr);
  // validity of this lane's key in the wavefront's half, from the slot tail
  auto key_valid = [&](int n, const char* tile) __attribute__((always_inline)) -> bool {
    const int key = n * BNS + kh * C::HK + lane;
    if (n < 0 || lane >= C::HK || key >= klen) return false;
    return a.kvalid == nullptr || tile[C::BUF + kh * C::HK + lane] != 0;
  };

  // Lane-dependent LDS read offsets.  The swizzles only involve lane bits,
  // so tile/step offsets (32t, 8u, 4q rows) become instruction immediates.
  int k_off[C::QSTEPS];
  {
    const int row = kh * C::HK + key_perm(lr);  // + 32t
    const int sw = swz_k<C::KROW>(row) & (C::CPR_K - 1);
#pragma unroll
    for (int st = 0; st < C::QSTEPS; ++st)
      k_off[st] = row * C::KROW + (((hf * C::QSTEPS + st) ^ sw) * 16);
  }
  int v_off[C::NDT];
  {
    const int grp = lane >> 4, gi = lane & 15;
    const int row = kh * C::HK + 16 * (grp >> 1) + (gi >> 2);  // + 32t + 8u + 4q
    const int sw = swz_v(row) & (C::CPR_V - 1);
#pragma unroll
    for (int dt = 0; dt < C::NDT; ++dt) {
      const int d = 32 * dt + 16 * (grp & 1) + 4 * (gi & 3);
      v_off[dt] = C::KBYTES + row * C::VROW + (((d >> 3) ^ sw) * 16) + (d & 7) * 2;
    }
  }

  // The first MFMA of every S tile accumulates onto this constant tile (the
  // 1.5 * 2^23 pattern for int8, zero for bf16): no per-block moves.
  AccT c_init;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    if constexpr (INT8) c_init[r] = kMagicI;
    else c_init[r] = 0.0f;
  }

  // One key block from the slot at `tile`.  `bits` is its key-validity mask
  // when the caller passes validity bits; `prefetch` issues scalar loads for
  // later blocks once this block's QK MFMAs are issued (scalar loads return
  // out of order, so any LDS wait behind them waits for them too).
  auto compute = [&](const char* tile, int n, float kscale, uint64_t bits, int n_fill,
                     char* fill, const uint32_t (&fill_tok)[kTokArr],
                     auto&& prefetch) __attribute__((always_inline)) {
    const uint64_t vmask = use_bits ? bits : __ballot(key_valid(n, tile));
    const bool all_valid = vmask == (~0ull >> (64 - C::HK));
    // ---- S^T = K Q^T: every K operand read is issued before the MFMAs ----
    AccT s_acc[C::KT];
    v4i kraw[C::KT][C::QSTEPS];
#pragma unroll
    for (int t = 0; t < C::KT; ++t)
#pragma unroll
      for (int st = 0; st < C::QSTEPS; ++st)
        kraw[t][st] = *reinterpret_cast<const v4i*>(tile + k_off[st] + 32 * t * C::KROW);
#pragma unroll
    for (int st = 0; st < C::QSTEPS; ++st)
#pragma unroll
      for (int t = 0; t < C::KT; ++t) {
        if constexpr (INT8) {
          s_acc[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(kraw[t][st], q_op[st],
                                                           st == 0 ? c_init : s_acc[t], 0, 0, 0);
        } else {
          s_acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              __builtin_bit_cast(v8bf, kraw[t][st]), q_op[st], st == 0 ? c_init : s_acc[t],
              0, 0, 0);
        }
      }
    __builtin_amdgcn_sched_group_barrier(0x100, C::KT * C::QSTEPS, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, C::KT * C::QSTEPS, 0);
    __builtin_amdgcn_sched_barrier(0);
    prefetch();
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
      uint32_t bits = 0;  // this lane's 16 keys of each tile as one word
#pragma unroll
      for (int t = 0; t < C::KT; ++t)
        bits |= static_cast<uint32_t>((vmask >> (32 * t + 16 * hf)) & 0xffffull) << (16 * t);
#pragma unroll
      for (int t = 0; t < C::KT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          rv[t][r] = ((bits >> (16 * t + r)) & 1u) ? rv[t][r] : -INFINITY;
    }
    const float c = INT8 ? a.scale_log2 * qs * kscale : a.scale_log2;
    // Row sums add the fp32 exponentials in four independent chains: the
    // bf16 dot instruction would share the matrix pipe and stall behind the
    // other wavefront's MFMAs, plain adds issue beside them.
    v8bf p_op[C::KT][2];
    auto exps = [&]() __attribute__((always_inline)) -> float {
      const float bias = -(INT8 ? c * kMagicF : 0.0f) - (m_run == -INFINITY ? 0.0f : m_run);
      float lsum[4];  // seeded with the first four terms (0 + e cannot be folded)
#pragma unroll
      for (int t = 0; t < C::KT; ++t)
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int jj = 0; jj < 8; ++jj) {
            const float e = __builtin_amdgcn_exp2f(fmaf(rv[t][8 * u + jj], c, bias));
            p_op[t][u][jj] = static_cast<__bf16>(e);
            if (t == 0 && u == 0 && jj < 4) lsum[jj] = e;
            else lsum[jj & 3] += e;
          }
      return (lsum[0] + lsum[1]) + (lsum[2] + lsum[3]);
    };
    // Exponentials against the running max first.  Every term is >= 0, so a
    // lane's partial sum bounds each of its terms: at most 2^kTau means none
    // of its keys exceeds the running max by more than kTau, and the running
    // max stays (lazy rescale).  Only otherwise, or while a row has no max yet,
    // is the block max reduced (wavefront-uniform branch) and the running max
    // moved, and the exponentials are taken again.  Steady blocks skip the
    // serial max reduction before the first exponential.
    float part = exps();
    if (__ballot(m_run == -INFINITY || !(part <= kTauPow)) != 0) {
      float rmax = -INFINITY;
#pragma unroll
      for (int t = 0; t < C::KT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) rmax = fmaxf(rmax, rv[t][r]);
      rmax = pair_max(rmax);  // with the partner lane (lane ^ 32)
      const float m_blk = (rmax == -INFINITY) ? -INFINITY
                          : (INT8 ? (rmax - kMagicF) * c : rmax * c);
      // lazy rescale: move the running max only when it grows by > 2^kTau
      if (__ballot(m_blk > m_run + kTau) != 0) {  // wavefront-uniform
        const float m_new = fmaxf(m_run, m_blk);
        const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
        l_run *= alpha;
#pragma unroll
        for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) o_acc[dt][r] *= alpha;
        m_run = m_new;
        part = exps();
      }
    }
    l_run += part;
    if constexpr (kDmaInPv) {
      if constexpr (kValidCopy) stage_valid_flat(n_fill, fill);
      stage_flat(n_fill, fill, fill_tok);
    }
    // ---- O^T += V^T P^T, V^T operand by transposing LDS reads; the reads of
    //      the next 16-key step are in flight during this step's MFMAs ----
    auto v_group = [&](int g, v8bf (&op)[C::NDT]) __attribute__((always_inline)) {
      const int t = g >> 1, u = g & 1;
#pragma unroll
      for (int dt = 0; dt < C::NDT; ++dt) {
        const char* p0 = tile + v_off[dt] + (32 * t + 8 * u) * C::VROW;
        const v4bf lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(RCSA_LDS(v4bf, p0));
        const v4bf hi =
            __builtin_amdgcn_ds_read_tr16_b64_v4bf16(RCSA_LDS(v4bf, p0 + 4 * C::VROW));
        op[dt] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
    };
    v8bf vop[2][C::NDT];
    v_group(0, vop[0]);
#pragma unroll
    for (int g = 0; g < 2 * C::KT; ++g) {
      if (g + 1 < 2 * C::KT) v_group(g + 1, vop[(g + 1) & 1]);
#pragma unroll
      for (int dt = 0; dt < C::NDT; ++dt)
        o_acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vop[g & 1][dt], p_op[g >> 1][g & 1],
                                                           o_acc[dt], 0, 0, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * C::NDT, 0);
#pragma unroll
    for (int g = 0; g < 2 * C::KT; ++g)
#pragma unroll
      for (int dt = 0; dt < C::NDT; ++dt) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (g + 1 < 2 * C::KT) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        if (kDmaInPv && g * C::NDT + dt < kOps)
          __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);
      }
  };

  // ---- ring: block j lives in slot j % STAGES; STAGES-1 blocks in flight ----
  // List entries are read one iteration before they are staged (scalar
  // loads whose latency hides behind that iteration's compute).
  int n_m[3] = {-1, -1, -1};
  float ks_m[3] = {1.0f, 1.0f, 1.0f};
  uint2 mk_m[3] = {};  // raw validity words per slot (caller's bits only)
  // slot-map entries of the step that fills each slot (GATHER)
  uint32_t tk_m[3][kTokArr] = {};
  int n_pre = -1;  // next step to stage
  if constexpr (kDmaInPv) {
    // both prologue steps always copy (step 0 stands in past the list), so
    // every wavefront has exactly 2 * kOps copies in flight
#pragma unroll
    for (int sidx = 0; sidx < STAGES - 1; ++sidx) {
      n_m[sidx] = sidx < steps ? block_of(sidx) : -1;
      ks_m[sidx] = fetch_scale(n_m[sidx]);
    }
    if constexpr (GATHER) n_pre = STAGES - 1 < steps ? block_of(STAGES - 1) : -1;
    // gathered: the map reads of the two prologue steps, then their copies,
    // then the map read of step 2.  The first ring wait counts the copies of
    // one step plus one step's map reads as the younger operations, so the
    // map read of step 2 must come after the copies of step 0: the scheduling
    // fence keeps the compiler from hoisting it (loads issue in order).
    load_tokens(n_m[0], tk_m[0]);
    load_tokens(n_m[1], tk_m[1]);
#pragma unroll
    for (int sidx = 0; sidx < STAGES - 1; ++sidx) {
      char* const dst = sidx == 0 ? s_0 : sidx == 1 ? s_1 : s_2;
      if constexpr (kValidCopy) stage_valid_flat(n_m[sidx], dst);
      stage_flat(n_m[sidx], dst, tk_m[sidx]);
      // the copies of step 0 stay older than those of step 1 (the first
      // ring wait leaves one step's copies in flight)
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (GATHER) {
      __builtin_amdgcn_sched_barrier(0);
      load_tokens(n_pre, tk_m[2]);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (use_bits) mk_m[0] = mask_words(n_m[0]);
    if constexpr (!GATHER) n_pre = STAGES - 1 < steps ? block_of(STAGES - 1) : -1;
    // the Q loads (and the first two map reads) precede these 2 kOps copies
    // (and the third map read): with at most that many outstanding, Q has
    // landed and both prologue stages stay in flight
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * kOps + kTok));
  } else {
#pragma unroll
    for (int sidx = 0; sidx < STAGES - 1; ++sidx) {
      if (sidx < steps) {
        char* const dst = sidx == 0 ? s_0 : sidx == 1 ? s_1 : s_2;
        n_m[sidx] = block_of(sidx);
        ks_m[sidx] = fetch_scale(n_m[sidx]);
        stage_valid(n_m[sidx], dst);
        stage(n_m[sidx], dst);
      }
    }
    n_pre = STAGES - 1 < steps ? block_of(STAGES - 1) : -1;
  }
  // 3-slot ring: the list entry of the step after n_pre, as loaded
  // (read only when the list is not empty: an empty list may have no entries)
  int32_t pre_raw =
      (kDmaInPv && steps > 0) ? ld_const(list + (STAGES < steps ? STAGES : 0) / C::SUB) : -1;
  auto iteration = [&](auto slot_c, int j) __attribute__((always_inline)) {
    constexpr int J = decltype(slot_c)::value;
    constexpr int F = (J + STAGES - 1) % STAGES;  // slot of block j + STAGES - 1
    // keep the int8 bias tile in VGPRs (otherwise it lives in SGPRs and is
    // copied into VGPRs for every block's first QK MFMA)
    if constexpr (INT8) asm volatile("" : "+v"(c_init));
    char* const tile = J == 0 ? s_0 : J == 1 ? s_1 : s_2;
    char* const fill = F == 0 ? s_0 : F == 1 ? s_1 : s_2;
    // block j's copies are the oldest in flight; the STAGES-2 younger
    // stages may remain (wavefront 0's extra validity copy is waited too),
    // then every wavefront's copies of block j have landed and slot F is free
    if constexpr (kDmaInPv) {
      wait_vm_barrier<kOps + kTok>();  // every step issues kOps copies (+ kTok map reads)
    } else if constexpr (STAGES == 3) {
      if (j + 1 < steps) wait_vm_barrier<C::DMA>();
      else wait_vm_barrier<0>();
    } else {
      wait_vm_barrier<0>();
    }
    if constexpr (kDmaInPv) {
      // every iteration copies (a step past the list re-copies step 0 into
      // the slot it fills, which nobody reads), so every wait counts the
      // same copies; the K/V copies issue between the PV MFMAs
      // Scalar loads for later blocks go out after this block's QK MFMAs:
      // the scale of block j+2, the list entry of block j+3 and the
      // validity bits of block j+1.
      // Loaded values are only stored here (their first use is a later
      // block's), so no wait lands before this block's softmax.
      constexpr int N1 = (J + 1) % STAGES;  // slot of block j + 1
      const int nf = n_pre;
      n_m[F] = nf;
      n_pre = j + STAGES < steps ? block_step(pre_raw, j + STAGES) : -1;
      const int nxt = j + STAGES + 1 < steps ? j + STAGES + 1 : 0;  // in-bounds entry
      compute(tile, n_m[J], ks_m[J], use_bits ? mask_of(n_m[J], mk_m[J]) : 0ull, nf, fill,
              tk_m[F], [&]() __attribute__((always_inline)) {
                ks_m[F] = fetch_scale(nf);
                pre_raw = ld_const(list + nxt / C::SUB);
                if (use_bits) mk_m[N1] = mask_words(n_m[N1]);
                // map entries of block j + 3, which will fill this block's slot
                load_tokens(n_pre, tk_m[J]);
              });
    } else {
      if (j + STAGES - 1 < steps) {
        n_m[F] = n_pre;
        ks_m[F] = fetch_scale(n_pre);
        stage_valid(n_pre, fill);
        stage(n_pre, fill);
        n_pre = j + STAGES < steps ? block_of(j + STAGES) : -1;
      }
      compute(tile, n_m[J], ks_m[J], use_bits ? mask_bits(n_m[J]) : 0ull, -1, fill, tk_m[F],
              []() __attribute__((always_inline)) {});
    }
  };
  if constexpr (kPadRounds) {
    // Whole rounds of STAGES steps, no exit between them: a step past the list
    // has every key masked (its exponentials are 0, its running max stays), so
    // it adds exactly nothing.  With one loop exit the compiler keeps track of
    // which ring slot each copy in flight writes across the back edge (it waits
    // for exactly the oldest step at the loop header instead of draining every
    // copy) and keeps the loop-carried scalars in registers (int8: 32 -> 3
    // SGPRs spilled; 2-4% faster).
    const int rounds = (steps + STAGES - 1) / STAGES;
    for (int rd = 0; rd < rounds; ++rd) {
      const int j = rd * STAGES;
      iteration(std::integral_constant<int, 0>{}, j);
      iteration(std::integral_constant<int, 1>{}, j + 1);
      iteration(std::integral_constant<int, 2>{}, j + 2);
    }
  } else {
    for (int j = 0; j < steps; j += STAGES) {
      iteration(std::integral_constant<int, 0>{}, j);
      if (j + 1 >= steps) break;
      iteration(std::integral_constant<int, 1>{}, j + 1);
      if constexpr (STAGES > 2) {
        if (j + 2 >= steps) break;
        iteration(std::integral_constant<int, 2>{}, j + 2);
      }
    }
  }

  // the trailing copies (past the list) land before the slots are reused or freed
  if constexpr (kDmaInPv) __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));

  // ---- merge the key halves, normalise, write O (bf16) and the LSE ----
  const float l_tot = pair_sum(l_run);
  float m = m_run, l = l_tot, fa = 1.0f, fb = 0.0f;
  const float* mbuf = nullptr;
  if constexpr (NKH == 2) {
    __syncthreads();  // main loop done everywhere: LDS is free for the merge
    float* mb;
    if constexpr (C::MERGE_IN_SLOTS) {
      const int sl = rg % STAGES;
      mb = reinterpret_cast<float*>(sl == 0 ? s_0 : sl == 1 ? s_1 : s_2) +
           (rg / STAGES) * C::MW;
    } else {
      mb = reinterpret_cast<float*>(s_m) + rg * C::MW;
    }
    if (kh == 1) {
#pragma unroll
      for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) mb[(dt * 16 + r) * 64 + lane] = o_acc[dt][r];
      mb[C::NDT * 16 * 64 + lane] = m_run;
      mb[C::NDT * 16 * 64 + 64 + lane] = l_tot;
    }
    __syncthreads();
    if (kh == 1) return;
    const float m_b = mb[C::NDT * 16 * 64 + lane];
    const float l_b = mb[C::NDT * 16 * 64 + 64 + lane];
    m = fmaxf(m_run, m_b);
    fa = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m);
    fb = m_b == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_b - m);
    l = l_tot * fa + l_b * fb;
    mbuf = mb;
  }
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  fa *= inv;
  fb *= inv;
  // a share writes its normalised partial and (m, l) to the workspace
  const int64_t orow = qrow_ok && nsp == 1 ? out_row(a, qrow) : qrow;
  if (qrow_ok && orow >= 0) {
    const int64_t ws_row = (split * a.n_tail + tail) * BM + (qrow - qb * BM);
    u16* op = nsp == 1 ? a.out + b * a.soz + h * a.soh + orow * a.som : a.ws_o + ws_row * D;
#pragma unroll
    for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float o4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * g + e;
          o4[e] = o_acc[dt][r] * fa;
          if constexpr (NKH == 2) o4[e] += mbuf[(dt * 16 + r) * 64 + lane] * fb;
        }
        const int d0 = 32 * dt + 8 * g + 4 * hf;
        *reinterpret_cast<uint2*>(op + d0) =
            make_uint2(pack_bf16x2(o4[0], o4[1]), pack_bf16x2(o4[2], o4[3]));
      }
    if (hf == 0) {
      if (nsp > 1) {
        a.ws_ml[ws_row] = make_float2(l > 0.0f ? m : -INFINITY, l);
      } else if (a.lse) {
        a.lse[(b * a.H + h) * (a.out_tok ? a.out_len : a.q_len) + orow] =
            l > 0.0f ? (m + __log2f(l)) * 0.69314718055994531f : -INFINITY;
      }
    }
  }
}

// Combine the n_split partial results of every row of the tail query blocks:
//   w_s = l_s 2^(m_s - M),  out = sum_s w_s O_s / sum_s w_s,  lse = ln 2 (M + log2 sum_s w_s)
// One thread per (tail row, 8 channels); rows with no admissible key get 0 / -inf.
template <int D>
__global__ void __launch_bounds__(256)
attn_merge_kernel(AttnArgs a) {
  constexpr int CPR = D / 8;
  const int64_t v = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t rows = a.n_tail * a.block_m;
  if (v >= rows * CPR) return;
  const int c = static_cast<int>(v % CPR);
  const int64_t trow = v / CPR;  // tail * block_m + row in block
  const int64_t tail = trow / a.block_m, r = trow % a.block_m;
  const int64_t per = a.xcd_items - a.xcd_direct;
  const int64_t item = (tail / per) * a.xcd_items + a.xcd_direct + tail % per;
  if (item >= a.n_items) return;
  const int64_t qb = item % a.n_qblocks, bh = item / a.n_qblocks;
  const int64_t qrow = qb * a.block_m + r;
  if (qrow >= a.q_len) return;
  if (a.q_tok != nullptr) {  // a gathered query slot with no token: no share wrote it
    const int32_t t = a.q_tok[qrow];
    if (t < 0 || t >= a.q_src_len) return;
  }
  const int64_t orow = out_row(a, qrow);
  if (orow < 0) return;
  float mx = -INFINITY;
  for (int64_t s = 0; s < a.n_split; ++s) mx = fmaxf(mx, a.ws_ml[s * rows + trow].x);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float wsum = 0.0f;
  if (mx != -INFINITY) {
    for (int64_t s = 0; s < a.n_split; ++s) {
      const float2 ml = a.ws_ml[s * rows + trow];
      if (ml.x == -INFINITY) continue;
      const float w = ml.y * __builtin_amdgcn_exp2f(ml.x - mx);
      wsum += w;
      float o[8];
      Vec8<u16>::load(a.ws_o + (s * rows + trow) * D + c * 8, o);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = fmaf(w, o[j], acc[j]);
    }
  }
  const float inv = wsum > 0.0f ? 1.0f / wsum : 0.0f;
  const int64_t b = bh / a.H, h = bh % a.H;
  u16* op = a.out + b * a.soz + h * a.soh + orow * a.som + c * 8;
  *reinterpret_cast<uint4*>(op) =
      make_uint4(pack_bf16x2(acc[0] * inv, acc[1] * inv), pack_bf16x2(acc[2] * inv, acc[3] * inv),
                 pack_bf16x2(acc[4] * inv, acc[5] * inv), pack_bf16x2(acc[6] * inv, acc[7] * inv));
  if (a.lse && c == 0)
    a.lse[bh * (a.out_tok ? a.out_len : a.q_len) + orow] =
        wsum > 0.0f ? (mx + __log2f(wsum)) * 0.69314718055994531f : -INFINITY;
}

// Launch of the gathered bf16 kernel (3-slot ring of 64-key steps, validity
// bits, Q/K/V rows through slot maps).  It is compiled in its own source with
// the default instruction scheduler: the kernels of sparse_attn.hip are
// scheduled for instruction-level parallelism, which makes this one slower.
int launch_bf16_gather(AttnArgs& a, dim3 grid, hipStream_t s);
// Three 4-wavefront workgroups per compute unit (sparse_attn_int8_cu3.hip,
// sparse_attn_bf16_cu3.hip): int8 with gathered V (bits) or packed sources
// (bits or bytes); bf16 with gathered sources (bits) or packed ones with
// validity bytes.
int launch_int8_cu3(AttnArgs& a, dim3 grid, bool gather, bool bits, hipStream_t s);
int launch_bf16_cu3(AttnArgs& a, dim3 grid, bool gather, hipStream_t s);

}  // namespace rcsa

