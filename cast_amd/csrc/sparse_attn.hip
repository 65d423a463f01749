// Block-sparse flash attention for gfx950 (MI355X): launchers, split plans,
// workspaces and the C ABI.  The kernels are in sparse_attn_kernel.h.
#include <mutex>

#include "sparse_attn_kernel.h"

namespace rcsa {

static int64_t cus_per_xcd();

template <bool INT8>
static int launch_attn(AttnArgs& a, int64_t D, int64_t BM, int64_t BN, hipStream_t s) {
  const int64_t per_xcd = a.xcd_direct + (a.xcd_items - a.xcd_direct) * a.n_split;
  const dim3 grid(static_cast<unsigned>(kNumXcd * per_xcd));
  // the shapes other than D 128 with 128 x 128 blocks double-buffer
#define RCSA_ATTN(D_, BM_, BN_, ST_)                                                   \
  if (D == D_ && BM == BM_ && BN == BN_) {                                              \
    sparse_attn_kernel<INT8, D_, BM_, BN_, ST_, BN_, 2, false><<<grid, dim3(BM_ * 4), 0, s>>>(a); \
    return launch_status();                                                             \
  }
  // gathered sources exist for the 3-slot rings with validity bits only
  if (a.kv_tok != nullptr && !(a.kmask != nullptr && D == 128 && BM == 128 && BN == 128))
    return RCSA_ERR_SHAPE;
  // D 128, 128 x 128 blocks: 3-slot rings.  With at least two full rounds of
  // query blocks per XCD, three 4-wavefront workgroups per compute unit
  // (32-key steps); otherwise one 8-wavefront workgroup (int8: 128-key steps
  // of 48 KiB, bf16: 64-key steps of 32 KiB).  Packed and gathered sources of
  // one shape take the same form, so the two forms of a call stay bit-identical.
  if (D == 128 && BM == 128 && BN == 128) {
    const int64_t cux = cus_per_xcd();
    const bool cu3 = cux > 0 && a.xcd_items >= 2 * cux;
    const bool bits = a.kmask != nullptr, gather = a.kv_tok != nullptr;
    if constexpr (INT8) {
      if (cu3) return launch_int8_cu3(a, grid, gather, bits, s);
      if (gather)
        sparse_attn_kernel<true, 128, 128, 128, 3, 128, 2, true, true><<<grid, dim3(512), 0, s>>>(a);
      else if (bits)
        sparse_attn_kernel<true, 128, 128, 128, 3, 128, 2, true><<<grid, dim3(512), 0, s>>>(a);
      else
        sparse_attn_kernel<true, 128, 128, 128, 3, 128, 2, false><<<grid, dim3(512), 0, s>>>(a);
    } else {
      if (cu3 && bits && !gather)  // built here, for instruction-level parallelism
        sparse_attn_kernel<false, 128, 128, 128, 3, 32, 1, true, false, 3>
            <<<grid, dim3(256), 0, s>>>(a);
      else if (cu3)
        return launch_bf16_cu3(a, grid, gather, s);
      else if (gather)
        return launch_bf16_gather(a, grid, s);
      else if (bits)
        sparse_attn_kernel<false, 128, 128, 128, 3, 64, 2, true><<<grid, dim3(512), 0, s>>>(a);
      else
        sparse_attn_kernel<false, 128, 128, 128, 3, 64, 2, false><<<grid, dim3(512), 0, s>>>(a);
    }
    return launch_status();
  }
  RCSA_ATTN(128, 128, 64, 2)
  RCSA_ATTN(128, 64, 128, 2)
  RCSA_ATTN(128, 64, 64, 2)
  RCSA_ATTN(64, 128, 128, 2)
  RCSA_ATTN(64, 128, 64, 2)
  RCSA_ATTN(64, 64, 128, 2)
  RCSA_ATTN(64, 64, 64, 2)
#undef RCSA_ATTN
  return RCSA_ERR_SHAPE;
}

// Kernel, then (for a split list) the merge of the partial results.
template <bool INT8>
static int launch_attn_split(AttnArgs& a, int64_t D, int64_t BM, int64_t BN, hipStream_t s) {
  int st = launch_attn<INT8>(a, D, BM, BN, s);
  if (st || a.n_split == 1) return st;
  const int64_t threads = a.n_tail * a.block_m * (D / 8);
  const dim3 grid(static_cast<unsigned>((threads + 255) / 256));
  if (D == 128) attn_merge_kernel<128><<<grid, dim3(256), 0, s>>>(a);
  else attn_merge_kernel<64><<<grid, dim3(256), 0, s>>>(a);
  return launch_status();
}

// Compute units per XCD of the current device (0 when it cannot be read);
// one attention workgroup fills a compute unit.
static int64_t cus_per_xcd() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus < kNumXcd)
    return 0;
  return cus / kNumXcd;
}

// Workspace of a split launch: normalised bf16 partials, then (m, l) pairs,
// for n_tail tail query blocks of block_m rows.
static int64_t ws_o_bytes(int64_t n_tail, int64_t block_m, int64_t d, int64_t n_split) {
  return ((n_split * n_tail * block_m * d * 2) + 255) / 256 * 256;
}
// Upper bound for any BLOCK_M in {64, 128}: at most min(8 (cus_per_xcd - 1),
// items + 7) tail query blocks (items counted at BLOCK_M = 64) of at most
// 128 rows.
static int64_t ws_bound(int64_t n_bh, int64_t q_len, int64_t d, int64_t n_split) {
  if (n_split <= 1) return 0;
  int64_t tails = n_bh * ((q_len + 63) / 64) + kNumXcd - 1;
  const int64_t cux = cus_per_xcd();
  if (cux > 0 && kNumXcd * (cux - 1) < tails) tails = kNumXcd * (cux - 1);
  return ws_o_bytes(tails, 128, d, n_split) + n_split * tails * 128 * 8;
}

// Tail query blocks: on each XCD, those past the last full round of its
// compute units (all of them when one round is not filled).  Sets the split
// fields of `a` (no workspace yet); leaves `a` unsplit when every round is full.
// Rounds count one workgroup per compute unit also for the form that runs
// three per compute unit: there the shares of the tail items still land
// beside the direct items' last blocks, and at 24 heads x 28 query blocks x 97
// key blocks the split launch takes 0.375 ms against 0.403 ms unsplit in that
// form (interleaved on one box), so both forms keep this plan.
static int plan_split(AttnArgs& a, int64_t n_split) {
  if (n_split < 1 || n_split > 16) return RCSA_ERR_SHAPE;
  if (n_split == 1) return RCSA_OK;
  const int64_t cux = cus_per_xcd();
  if (cux <= 0) return RCSA_ERR_LAUNCH;
  const int64_t p = a.xcd_items;
  const int64_t direct = p % cux == 0 ? p : p / cux * cux;
  if (direct == p) return RCSA_OK;  // every round full: nothing to split
  a.xcd_direct = direct;
  a.n_split = n_split;
  a.n_tail = kNumXcd * (p - direct);
  return RCSA_OK;
}

// Bytes of workspace a planned split launch uses (0 when unsplit).
static int64_t split_need(const AttnArgs& a, int64_t d) {
  if (a.n_split == 1) return 0;
  return ws_o_bytes(a.n_tail, a.block_m, d, a.n_split) + a.n_split * a.n_tail * a.block_m * 8;
}

// Point the partial outputs and (max, sum) pairs of a planned split at `base`.
static void bind_workspace(AttnArgs& a, int64_t d, char* base) {
  a.ws_o = reinterpret_cast<u16*>(base);
  a.ws_ml = reinterpret_cast<float2*>(base + ws_o_bytes(a.n_tail, a.block_m, d, a.n_split));
}

static int apply_split(AttnArgs& a, int64_t d, int64_t n_split, void* workspace,
                       int64_t workspace_bytes) {
  if (n_split < 1 || n_split > 16) return RCSA_ERR_SHAPE;
  if (n_split == 1) return RCSA_OK;
  if (workspace == nullptr) return RCSA_ERR_NULL;
  if (!aligned16(workspace)) return RCSA_ERR_ALIGN;
  if (workspace_bytes < ws_bound(a.n_bh, a.q_len, d, n_split)) return RCSA_ERR_SHAPE;
  const int st = plan_split(a, n_split);
  if (st || a.n_split == 1) return st;
  bind_workspace(a, d, static_cast<char*>(workspace));
  return RCSA_OK;
}

// ---- the allocation-free entry point's scratch ----
// Device-resident workspace of rcsa_sparse_attn_int8_noalloc: the split
// shares' partial outputs and (max, sum) pairs.  Every GPU the library runs on
// holds its own copy until the process ends.  Host code must not use the
// array's name as an address (it is a host-side stand-in): the device address
// comes from hipGetSymbolAddress, once per device, in scratch_on_device().
constexpr int64_t kScratchBytes = int64_t{32} << 20;
static __device__ __align__(256) char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static char* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch` (looked up on the first call per device).
static int scratch_on_device(char** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return RCSA_ERR_LAUNCH;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr)
      return RCSA_ERR_LAUNCH;
    g_scratch_ptr[dev] = static_cast<char*>(p);
  }
  *out = g_scratch_ptr[dev];
  return RCSA_OK;
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
  // copy addressing multiplies row numbers by the row stride in 24 bits
  if (skn < 0 || svn < 0 || skn * (16 / kvec) >= (1 << 24) || svn * 2 >= (1 << 24))
    return RCSA_ERR_STRIDE;
  if (som % 4 || soh % 4 || soz % 4) return RCSA_ERR_STRIDE;
  if (reinterpret_cast<uintptr_t>(Out) & 7u) return RCSA_ERR_ALIGN;
  // validity bytes are copied in aligned 16-byte chunks (the chunk holding the
  // last byte stays inside the same page, so no padding is needed)
  if (reinterpret_cast<uintptr_t>(K_valid) & 15u) return RCSA_ERR_ALIGN;
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
  a.block_m = BM;
  a.n_bh = B * H;
  a.n_items = B * H * a.n_qblocks;
  // the kernel decodes work items and list shares in 32-bit arithmetic
  if (a.n_items >= (int64_t{1} << 31) || max_k >= (int64_t{1} << 24) ||
      K_LEN >= (int64_t{1} << 31))
    return RCSA_ERR_SHAPE;
  a.xcd_items = (a.n_items + kNumXcd - 1) / kNumXcd;
  a.xcd_direct = a.xcd_items;
  a.n_split = 1;
  a.n_tail = 0;
  return RCSA_OK;
}

// Gathered V (and, with `gather_k`, K) rows: packed key slot s reads token row
// kv_token[s] of a token-major source of kv_len rows (the strides given for
// V/K are then token-major: row stride = token stride).  Needs the validity
// bits and whole key blocks; the (b, h) plane of kv_len rows stays below 2^31
// bytes so that an empty slot's offset lies past it.
static int set_gather(AttnArgs& a, const int32_t* kv_token, int64_t kv_len, int64_t BN,
                      bool gather_k) {
  if (!kv_token) return RCSA_OK;
  if (reinterpret_cast<uintptr_t>(kv_token) & 3u) return RCSA_ERR_ALIGN;
  if (a.kmask == nullptr || kv_len <= 0 || a.k_len % BN != 0) return RCSA_ERR_SHAPE;
  constexpr int64_t kPlane = int64_t{1} << 31;
  if (kv_len * a.svn * 2 >= kPlane || (gather_k && kv_len * a.skn * 2 >= kPlane))
    return RCSA_ERR_SHAPE;
  a.kv_tok = kv_token;
  a.kv_len = kv_len;
  return RCSA_OK;
}

}  // namespace rcsa

using namespace rcsa;

extern "C" int rcsa_sparse_attn_bf16_split(
    const void* Q, const void* K, const void* V, const uint8_t* K_valid,
    const uint32_t* K_block_mask, float sm_scale,
    float* M, void* Out, const int32_t* block_indices, const int32_t* block_indices_lens,
    int64_t stride_qz, int64_t stride_qh, int64_t stride_qm, int64_t stride_kz,
    int64_t stride_kh, int64_t stride_kn, int64_t stride_vz, int64_t stride_vh,
    int64_t stride_vn, int64_t stride_oz, int64_t stride_oh, int64_t stride_om,
    int64_t stride_bz, int64_t stride_bh, int64_t stride_bm, int64_t stride_lz,
    int64_t stride_lh, int64_t stride_lm, int64_t B, int64_t H, int64_t Q_LEN,
    int64_t K_LEN, int64_t HEAD_DIM, int64_t BLOCK_M, int64_t BLOCK_N, int64_t max_k,
    int64_t n_split, void* workspace, int64_t workspace_bytes, const int32_t* q_token,
    int64_t q_tokens, const int32_t* kv_token, int64_t kv_len, const int32_t* out_token,
    int64_t out_len, hipStream_t stream) {
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
  if (K_block_mask) {  // the bits replace the validity bytes
    if (reinterpret_cast<uintptr_t>(K_block_mask) & 3u) return RCSA_ERR_ALIGN;
    a.kmask = K_block_mask;
    a.kvalid = nullptr;
  }
  // gathered: Q rows through q_token, K/V rows through kv_token, O rows out
  // through out_token (or, when it is NULL, through q_token)
  if ((q_token == nullptr) != (kv_token == nullptr)) return RCSA_ERR_SHAPE;
  if (out_token && !q_token) return RCSA_ERR_SHAPE;
  if (q_token) {
    if ((reinterpret_cast<uintptr_t>(q_token) & 3u) ||
        (reinterpret_cast<uintptr_t>(out_token) & 3u))
      return RCSA_ERR_ALIGN;
    if (q_tokens <= 0 || q_tokens >= (int64_t{1} << 31)) return RCSA_ERR_SHAPE;
    if (out_token && (out_len <= 0 || out_len >= (int64_t{1} << 31))) return RCSA_ERR_SHAPE;
    a.q_tok = q_token;
    a.q_src_len = q_tokens;
    a.out_tok = out_token ? out_token : q_token;
    a.out_len = out_token ? out_len : q_tokens;
  }
  st = set_gather(a, kv_token, kv_len, BLOCK_N, true);
  if (st) return st;
  st = apply_split(a, HEAD_DIM, n_split, workspace, workspace_bytes);
  if (st) return st;
  if (a.n_items == 0) return RCSA_OK;
  return launch_attn_split<false>(a, HEAD_DIM, BLOCK_M, BLOCK_N, stream);
}

// The checks and argument set-up the split int8 entry point and its
// allocation-free variant share: everything but where the split's workspace
// comes from.
static int int8_setup(
    AttnArgs& a, const int8_t* Q, const float* q_scale, int64_t q_scale_stride,
    const int8_t* K, const float* k_scale, int64_t k_scale_stride, const void* V,
    const uint8_t* K_valid, const uint32_t* K_block_mask, float sm_scale, float* M, void* Out,
    const int32_t* block_indices, const int32_t* block_indices_lens, int64_t stride_qz,
    int64_t stride_qh, int64_t stride_qm, int64_t stride_kz, int64_t stride_kh,
    int64_t stride_kn, int64_t stride_vz, int64_t stride_vh, int64_t stride_vn,
    int64_t stride_oz, int64_t stride_oh, int64_t stride_om, int64_t stride_bz,
    int64_t stride_bh, int64_t stride_bm, int64_t stride_lz, int64_t stride_lh,
    int64_t stride_lm, int64_t B, int64_t H, int64_t Q_LEN, int64_t K_LEN, int64_t HEAD_DIM,
    int64_t BLOCK_M, int64_t BLOCK_N, int64_t max_k, const int32_t* out_token,
    int64_t out_len, const int32_t* kv_token, int64_t kv_len) {
  if (!Q || !K || !V || !q_scale || !k_scale) return RCSA_ERR_NULL;
  if (!aligned16(Q) || !aligned16(K) || !aligned16(V)) return RCSA_ERR_ALIGN;
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
  if (out_token) {  // Out and M hold out_len rows per (b, h), written through the map
    if (out_len <= 0 || out_len >= (int64_t{1} << 31)) return RCSA_ERR_SHAPE;
    a.out_tok = out_token;
    a.out_len = out_len;
  }
  if (K_block_mask) {  // the bits replace the validity bytes
    if (reinterpret_cast<uintptr_t>(K_block_mask) & 3u) return RCSA_ERR_ALIGN;
    a.kmask = K_block_mask;
    a.kvalid = nullptr;
  }
  return set_gather(a, kv_token, kv_len, BLOCK_N, false);
}

extern "C" int rcsa_sparse_attn_int8_split(
    const int8_t* Q, const float* q_scale, int64_t q_scale_stride, const int8_t* K,
    const float* k_scale, int64_t k_scale_stride, const void* V, const uint8_t* K_valid,
    const uint32_t* K_block_mask, float sm_scale, float* M, void* Out,
    const int32_t* block_indices,
    const int32_t* block_indices_lens, int64_t stride_qz, int64_t stride_qh,
    int64_t stride_qm, int64_t stride_kz, int64_t stride_kh, int64_t stride_kn,
    int64_t stride_vz, int64_t stride_vh, int64_t stride_vn, int64_t stride_oz,
    int64_t stride_oh, int64_t stride_om, int64_t stride_bz, int64_t stride_bh,
    int64_t stride_bm, int64_t stride_lz, int64_t stride_lh, int64_t stride_lm, int64_t B,
    int64_t H, int64_t Q_LEN, int64_t K_LEN, int64_t HEAD_DIM, int64_t BLOCK_M,
    int64_t BLOCK_N, int64_t max_k, int64_t n_split, void* workspace,
    int64_t workspace_bytes, const int32_t* out_token, int64_t out_len, const int32_t* kv_token,
    int64_t kv_len, hipStream_t stream) {
  AttnArgs a{};
  int st = int8_setup(a, Q, q_scale, q_scale_stride, K, k_scale, k_scale_stride, V, K_valid,
                      K_block_mask, sm_scale, M, Out, block_indices, block_indices_lens,
                      stride_qz, stride_qh, stride_qm, stride_kz, stride_kh, stride_kn,
                      stride_vz, stride_vh, stride_vn, stride_oz, stride_oh, stride_om,
                      stride_bz, stride_bh, stride_bm, stride_lz, stride_lh, stride_lm, B, H,
                      Q_LEN, K_LEN, HEAD_DIM, BLOCK_M, BLOCK_N, max_k, out_token, out_len,
                      kv_token, kv_len);
  if (st) return st;
  st = apply_split(a, HEAD_DIM, n_split, workspace, workspace_bytes);
  if (st) return st;
  if (a.n_items == 0) return RCSA_OK;
  return launch_attn_split<true>(a, HEAD_DIM, BLOCK_M, BLOCK_N, stream);
}

// The split int8 entry point with the library's static scratch as its
// workspace: allocates nothing.  Planned exactly like the split entry point;
// a split needing more than kScratchBytes is refused with RCSA_ERR_SCRATCH.
// Calls on one device share the scratch: the caller serialises them (one
// stream, or an event chain between streams).
extern "C" int rcsa_sparse_attn_int8_noalloc(
    const int8_t* Q, const float* q_scale, int64_t q_scale_stride, const int8_t* K,
    const float* k_scale, int64_t k_scale_stride, const void* V, const uint8_t* K_valid,
    const uint32_t* K_block_mask, float sm_scale, float* M, void* Out,
    const int32_t* block_indices,
    const int32_t* block_indices_lens, int64_t stride_qz, int64_t stride_qh,
    int64_t stride_qm, int64_t stride_kz, int64_t stride_kh, int64_t stride_kn,
    int64_t stride_vz, int64_t stride_vh, int64_t stride_vn, int64_t stride_oz,
    int64_t stride_oh, int64_t stride_om, int64_t stride_bz, int64_t stride_bh,
    int64_t stride_bm, int64_t stride_lz, int64_t stride_lh, int64_t stride_lm, int64_t B,
    int64_t H, int64_t Q_LEN, int64_t K_LEN, int64_t HEAD_DIM, int64_t BLOCK_M,
    int64_t BLOCK_N, int64_t max_k, int64_t n_split, const int32_t* out_token,
    int64_t out_len, const int32_t* kv_token, int64_t kv_len, hipStream_t stream) {
  AttnArgs a{};
  int st = int8_setup(a, Q, q_scale, q_scale_stride, K, k_scale, k_scale_stride, V, K_valid,
                      K_block_mask, sm_scale, M, Out, block_indices, block_indices_lens,
                      stride_qz, stride_qh, stride_qm, stride_kz, stride_kh, stride_kn,
                      stride_vz, stride_vh, stride_vn, stride_oz, stride_oh, stride_om,
                      stride_bz, stride_bh, stride_bm, stride_lz, stride_lh, stride_lm, B, H,
                      Q_LEN, K_LEN, HEAD_DIM, BLOCK_M, BLOCK_N, max_k, out_token, out_len,
                      kv_token, kv_len);
  if (st) return st;
  st = plan_split(a, n_split);
  if (st) return st;
  if (split_need(a, HEAD_DIM) > kScratchBytes) return RCSA_ERR_SCRATCH;
  if (a.n_split > 1) {
    // every share writes all its rows' partials and (max, sum) before the
    // merge reads them, so nothing left from an earlier call is read
    char* base = nullptr;
    st = scratch_on_device(&base);
    if (st) return st;
    bind_workspace(a, HEAD_DIM, base);
  }
  if (a.n_items == 0) return RCSA_OK;
  return launch_attn_split<true>(a, HEAD_DIM, BLOCK_M, BLOCK_N, stream);
}

extern "C" int64_t rcsa_attn_noalloc_scratch_bytes(void) { return kScratchBytes; }

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
  return rcsa_sparse_attn_bf16_split(
      Q, K, V, K_valid, nullptr, sm_scale, M, Out, block_indices, block_indices_lens, stride_qz,
      stride_qh, stride_qm, stride_kz, stride_kh, stride_kn, stride_vz, stride_vh, stride_vn,
      stride_oz, stride_oh, stride_om, stride_bz, stride_bh, stride_bm, stride_lz, stride_lh,
      stride_lm, B, H, Q_LEN, K_LEN, HEAD_DIM, BLOCK_M, BLOCK_N, max_k, 1, nullptr, 0,
      nullptr, 0, nullptr, 0, nullptr, 0, stream);
}

extern "C" int rcsa_sparse_attn_int8(
    const int8_t* Q, const float* q_scale, int64_t q_scale_stride, const int8_t* K,
    const float* k_scale, int64_t k_scale_stride, const void* V, const uint8_t* K_valid,
    const uint32_t* K_block_mask, float sm_scale, float* M, void* Out,
    const int32_t* block_indices,
    const int32_t* block_indices_lens, int64_t stride_qz, int64_t stride_qh,
    int64_t stride_qm, int64_t stride_kz, int64_t stride_kh, int64_t stride_kn,
    int64_t stride_vz, int64_t stride_vh, int64_t stride_vn, int64_t stride_oz,
    int64_t stride_oh, int64_t stride_om, int64_t stride_bz, int64_t stride_bh,
    int64_t stride_bm, int64_t stride_lz, int64_t stride_lh, int64_t stride_lm, int64_t B,
    int64_t H, int64_t Q_LEN, int64_t K_LEN, int64_t HEAD_DIM, int64_t BLOCK_M,
    int64_t BLOCK_N, int64_t max_k, const int32_t* out_token, int64_t out_len,
    hipStream_t stream) {
  return rcsa_sparse_attn_int8_split(
      Q, q_scale, q_scale_stride, K, k_scale, k_scale_stride, V, K_valid, K_block_mask,
      sm_scale, M, Out,
      block_indices, block_indices_lens, stride_qz, stride_qh, stride_qm, stride_kz,
      stride_kh, stride_kn, stride_vz, stride_vh, stride_vn, stride_oz, stride_oh, stride_om,
      stride_bz, stride_bh, stride_bm, stride_lz, stride_lh, stride_lm, B, H, Q_LEN, K_LEN,
      HEAD_DIM, BLOCK_M, BLOCK_N, max_k, 1, nullptr, 0, out_token, out_len, nullptr, 0,
      stream);
}

extern "C" int64_t rcsa_attn_workspace_bytes(int64_t B, int64_t H, int64_t Q_LEN,
                                             int64_t HEAD_DIM, int64_t n_split) {
  if (B <= 0 || H <= 0 || Q_LEN <= 0 || HEAD_DIM <= 0 || n_split < 1) return -1;
  return ws_bound(B * H, Q_LEN, HEAD_DIM, n_split);
}

// Split count for B * H * ceil(Q_LEN / BLOCK_M) query blocks on the current
// device.  Each XCD runs ceil(items / 8) of them on its compute units, one
// workgroup per unit at a time: `full` whole rounds, then `rem` tail query
// blocks, which s shares turn into ceil(rem s / units) rounds of
// ceil(max_k / s) key blocks.  Every round also pays a fixed cost (Q load,
// prologue, epilogue, partial write and merge) of about kFixedBlocks key
// blocks, measured over 1..4 shares at 41..152 blocks per list.  A larger
// count must win by 2% and keep at least 2 key blocks per share.
extern "C" int rcsa_attn_split_plan(int64_t B, int64_t H, int64_t Q_LEN, int64_t BLOCK_M,
                                    int64_t max_k, int64_t* n_split) {
  if (!n_split) return RCSA_ERR_NULL;
  if (B <= 0 || H <= 0 || Q_LEN <= 0 || BLOCK_M <= 0 || max_k < 0) return RCSA_ERR_SHAPE;
  const int64_t cux = cus_per_xcd();
  if (cux <= 0) return RCSA_ERR_LAUNCH;
  constexpr double kFixedBlocks = 7.0;
  const int64_t items = B * H * ((Q_LEN + BLOCK_M - 1) / BLOCK_M);
  const int64_t p = (items + kNumXcd - 1) / kNumXcd;
  const int64_t full = p / cux, rem = p % cux;
  int64_t best = 1;
  double best_cost = 0.0;
  for (int64_t s = 1; s <= 8 && rem > 0; ++s) {
    if (s > 1 && max_k < 2 * s) break;
    const double share = static_cast<double>((max_k + s - 1) / s);
    const double cost = static_cast<double>(full) * (kFixedBlocks + max_k) +
                        static_cast<double>((rem * s + cux - 1) / cux) * (kFixedBlocks + share);
    if (s == 1 || cost < best_cost * 0.98) { best = s; best_cost = cost; }
  }
  *n_split = best;
  return RCSA_OK;
}
