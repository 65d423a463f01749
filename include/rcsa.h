/*
 * rcsa.h -- C ABI of the MI355X (gfx950) Reconstruction-Coupled Sparse
 * Attention (RCSA) hot path.
 *
 * Every entry point takes raw device pointers, element counts and strides
 * (in elements, int64), the HIP stream to launch on, and returns an int
 * status (RCSA_OK == 0).  Nothing here allocates device memory: outputs and
 * scratch are owned by the caller.  Nothing here synchronises the stream or
 * reads device memory on the host, so every call is stream-ordered.
 *
 * Reference paths below are relative to the CAST repository, with
 * P/ = src/interaction_accel/methods/proposed/.
 *
 * Tensor conventions (all row-major, last dimension contiguous):
 *   packed Q/K/V    [B, H, L, D]   token-major inside a head; L = blocks * block_size
 *   pooled vectors  [B*H, NB, D]   fp32
 *   block scores    [B*H, NQB, NKB] fp32
 *   block lists     [B, H, NQB, max_k] int32, lens [B, H, NQB] int32
 */
#ifndef RCSA_H_
#define RCSA_H_

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes returned by every entry point. */
enum {
  RCSA_OK = 0,
  RCSA_ERR_NULL = 1,     /* a required pointer is NULL */
  RCSA_ERR_SHAPE = 2,    /* unsupported or inconsistent sizes */
  RCSA_ERR_STRIDE = 3,   /* last dimension not contiguous / misaligned stride */
  RCSA_ERR_DTYPE = 4,    /* unsupported element type code */
  RCSA_ERR_LAUNCH = 5,   /* the HIP runtime rejected the launch */
  RCSA_ERR_ALIGN = 6,    /* a pointer is not 16-byte aligned */
  RCSA_ERR_SCRATCH = 7   /* the request exceeds the library's static scratch */
};

/* Element type codes for inputs that may be bf16 or fp32. */
enum { RCSA_BF16 = 0, RCSA_F32 = 1 };

/* Selection output order. */
enum {
  RCSA_ORDER_INDEX = 0, /* ascending block index (what the attention kernel streams best) */
  RCSA_ORDER_RANK = 1   /* descending rank: forced first, then score desc, index asc */
};

/* Human-readable text for a status code (static storage). */
const char* rcsa_status_string(int status);

/* ABI version: (major << 16) | minor. */
int rcsa_abi_version(void);

/*
 * Pooled query blocks, optionally fused with the int8 query quantiser.
 *
 * Replaces the query half of the masked mean-pool + F.normalize at
 * P/matrix_curvature_phase_frame_weave.py:5685-5700 (native form:
 * P/qk_uncertainty_tangent_attention.py:1013-1022 over the tiling of
 * P/reciprocal_joint_attention.py:64-103):
 *   qhat[bh, b, :] = normalize(sum_{t valid} q[bh, b*bs + t, :] / max(n_valid, 1))
 * with normalize(x) = x / max(||x||_2, 1e-12).
 * valid: uint8 [n_blocks * block_size] shared by every head, or NULL (all valid).
 * When q_i8 and q_scale are both non-NULL the same pass writes the int8
 * query (no reference counterpart; see rcsa_quantize_key):
 *   q_scale[bh, b] = absmax_{t valid, c}(q) / 127   (1 when the block is all zero)
 *   q_i8[bh, b*bs + t, c] = clamp(rne(q / q_scale), -127, 127), 0 on invalid tokens.
 * q is addressed as q[bh_outer * stride_b + bh_inner * stride_h + token * stride_t + c]
 * with bh = bh_outer * n_heads + bh_inner.  head_dim in {64, 128}; block_size in {64, 128}.
 */
int rcsa_pool_query(const void* q, int dtype, int64_t batch, int64_t n_heads,
                    int64_t n_blocks, int64_t block_size, int64_t head_dim,
                    int64_t stride_b, int64_t stride_h, int64_t stride_t,
                    const uint8_t* valid, float* qhat, int8_t* q_i8,
                    float* q_scale, hipStream_t stream);

/*
 * Pooled key blocks plus the per-block statistics the key quantiser needs.
 * Same pooling as rcsa_pool_query (the key half of
 * P/matrix_curvature_phase_frame_weave.py:5685-5700).  Optional outputs
 * (each [B*H, n_blocks, head_dim] fp32, all or none):
 *   ksum = sum over valid tokens, kmin/kmax = min/max over valid tokens
 *   (0 for blocks with no valid token).
 * block_mask (optional, 8-byte aligned): uint32 [n_blocks][block_size / 32],
 *   bit i of word w of block n = validity of token n*block_size + 32w + i
 *   (the form rcsa_sparse_attn_int8 reads; no reference counterpart).
 */
int rcsa_pool_key(const void* k, int dtype, int64_t batch, int64_t n_heads,
                  int64_t n_blocks, int64_t block_size, int64_t head_dim,
                  int64_t stride_b, int64_t stride_h, int64_t stride_t,
                  const uint8_t* valid, float* khat, float* ksum, float* kmin,
                  float* kmax, uint32_t* block_mask, hipStream_t stream);

/*
 * rcsa_pool_query (with q_i8 / q_scale) and rcsa_pool_key (with ksum / kmin /
 * kmax and, if non-NULL, block_mask) in one launch; the outputs are those of
 * the two calls bit for bit.  No reference counterpart: the int8 layer call's
 * pooling pass, so the short query pass runs inside the key pass instead of
 * before it.  Q and K share dtype, batch, heads, block_size and head_dim; each
 * has its own block count, strides and validity.
 *
 * Gathered inputs (both maps non-NULL, or both NULL): q and k are then
 * token-major sources (e.g. [B, L, H, D] with stride_t = H * D) and packed
 * slot s = block * block_size + r reads token slot_token[s] of the source
 * (q_src_len / k_src_len tokens); -1, or a token >= src_len, is an empty
 * (invalid) slot.  The outputs are those of rcsa_pack_tokens followed by the
 * ungathered call, bit for bit, without the packed copies.  Fuses the
 * q[:, flat] / k[:, flat] gathers of P/matrix_curvature_phase_frame_weave.py:5677-5684
 * into the pooling pass; q_valid / k_valid, when given, stay per packed slot.
 *
 * q_i8, q_scale, ksum, kmin and kmax may all be NULL together: then only the
 * pooled blocks (and block_mask) are written — rcsa_pool_query without the
 * quantiser and rcsa_pool_key without the statistics, the bf16 path's pass.
 */
int rcsa_pool_query_key(const void* q, const void* k, int dtype, int64_t batch,
                        int64_t n_heads, int64_t n_qblocks, int64_t n_kblocks,
                        int64_t block_size, int64_t head_dim, int64_t q_stride_b,
                        int64_t q_stride_h, int64_t q_stride_t, int64_t k_stride_b,
                        int64_t k_stride_h, int64_t k_stride_t, const uint8_t* q_valid,
                        const uint8_t* k_valid, const int32_t* q_slot_token,
                        int64_t q_src_len, const int32_t* k_slot_token, int64_t k_src_len,
                        float* qhat, int8_t* q_i8, float* q_scale,
                        float* khat, float* ksum, float* kmin, float* kmax,
                        uint32_t* block_mask, hipStream_t stream);

/*
 * rcsa_pool_query_key plus the block means of V in the same launch:
 * vmean [batch*n_heads][n_kblocks][head_dim] fp32 (16-byte aligned) =
 * sum over the valid tokens of the block / max(valid tokens, 1), the pooled
 * values v_content that the FC-PASM router consumes
 * (P/matrix_curvature_phase_frame_weave.py:5696-5700).  V shares the key
 * layout: block count, validity (k_valid) and slot map (k_slot_token,
 * k_src_len); its strides are its own.  All other arguments and outputs are
 * those of rcsa_pool_query_key.
 */
int rcsa_pool_query_key_value(const void* q, const void* k, const void* v, int dtype,
                              int64_t batch, int64_t n_heads, int64_t n_qblocks,
                              int64_t n_kblocks, int64_t block_size, int64_t head_dim,
                              int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_t,
                              int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_t,
                              int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_t,
                              const uint8_t* q_valid, const uint8_t* k_valid,
                              const int32_t* q_slot_token, int64_t q_src_len,
                              const int32_t* k_slot_token, int64_t k_src_len, float* qhat,
                              int8_t* q_i8, float* q_scale, float* khat, float* ksum,
                              float* kmin, float* kmax, uint32_t* block_mask, float* vmean,
                              hipStream_t stream);

/*
 * Row degrees of a compact woven layer under the closed-loop allocator, on the
 * device (no .item() syncs).  Replaces compact_closed_loop_degrees
 * (P/control_response_cwca_attention.py:1188-1363, with _compact_time_cells
 * :1123-1163 and _redistribute_compact_capacity :1165-1186) and its
 * composition into the layer's degrees (P/matrix_curvature_phase_frame_weave.py:
 * 5727-5817):
 *   curvature [t_src][spatial] fp32 (the compiler's curvature matrix), response
 *   [t_src][spatial] fp32 or NULL (the previous layer's response; ignored when
 *   response_weight == 0), frames [n_frames] int32 current-local active frames,
 *   current_temporal_offset, source_group (the block shape's tt of the CWCA
 *   tiles), compact_group (the compact tt), feedback_form 0 additive,
 *   1 centered multiplicative, 2 centered inverse; fixed_query_budget != 0 gives
 *   every current cell mean_degree.
 * degrees: int32 [total_blocks]; total_blocks == memory_blocks +
 * ceil(n_frames / compact_group) * spatial (the packed rows).  status: int32 [1],
 * written on the device: 0, or the bits RCSA_CL_OUTSIDE_TILES (a profiled frame
 * lies past the curvature tiles), RCSA_CL_EXHAUSTED (a worldline ran out of key
 * capacity: the reference raises "exhausted key capacity") and
 * RCSA_CL_MEMORY_FRAME (a negative, i.e. memory, frame).  spatial <= 1024, at
 * most 64 cells, total_blocks <= 8192.
 */
enum { RCSA_CL_OUTSIDE_TILES = 1, RCSA_CL_EXHAUSTED = 2, RCSA_CL_MEMORY_FRAME = 4 };
int rcsa_closed_loop_degrees(const float* curvature, const float* response, int64_t t_src,
                             int64_t spatial, const int32_t* frames, int64_t n_frames,
                             int64_t current_temporal_offset, int64_t source_group,
                             int64_t compact_group, int64_t mean_degree, int64_t base_degree,
                             int64_t total_blocks, int64_t memory_blocks, float response_weight,
                             int feedback_form, int fixed_query_budget, int32_t* degrees,
                             int32_t* status, hipStream_t stream);

/*
 * Per-row key-block budgets on the device, so no budget is read back to the
 * host.  For every section row s of weights [n_sections][n] (row stride
 * weights_stride): largest-remainder apportionment of total_per_section edges
 * by max(w, 0) in fp32 (raw = total * w / sum w, floors, one more edge to the
 * largest fractional parts, ties to the lower index; a row whose weights sum
 * to <= 0 weighs every entry 1), as P/qk_uncertainty_tangent_attention.py:847-865
 * and :1239-1264 (_apportion_section_matrix).  With cap > 0 every degree is
 * then clamped to cap and the lost edges go, one each and pass after pass, to
 * the lowest-index rows below cap until the row sums to target_total (<= 0:
 * total_per_section) or no row has room, as the saturation at
 * P/matrix_curvature_phase_frame_weave.py:5807-5817.  n <= 8192,
 * total_per_section < 2^24.  degrees: int32 [n_sections][degrees_stride].
 */
int rcsa_row_budgets(const float* weights, int64_t n_sections, int64_t n,
                     int64_t weights_stride, int64_t total_per_section, int64_t cap,
                     int64_t target_total, int32_t* degrees, int64_t degrees_stride,
                     hipStream_t stream);

/*
 * Cosine block scores score[bh, i, j] = <qhat[bh, i], khat[bh, j]>.
 * Replaces torch.matmul(q_content, k_content.transpose(-2, -1)) at
 * P/matrix_curvature_phase_frame_weave.py:5701 and
 * P/qk_uncertainty_tangent_attention.py:1023.
 */
int rcsa_block_scores(const float* qhat, const float* khat, int64_t n_bh,
                      int64_t n_qblocks, int64_t n_kblocks, int64_t head_dim,
                      float* score, hipStream_t stream);

/*
 * Fixed-budget top-k block selection, one wavefront per (bh, query block).
 * Replaces score + 1e6 * local followed by torch.topk
 * (P/matrix_curvature_phase_frame_weave.py:5829-5832) and the native stable
 * descending argsort (P/qk_uncertainty_tangent_attention.py:970-980, 1025-1044).
 * Total order: forced columns first, then higher score, then lower index.
 * Only allowed columns are eligible; counts[row] = min(k_row, n_allowed).
 *   row_k:   int32 k per row, element [bh * row_k_stride_bh + i]; NULL -> k_fixed
 *   forced:  uint8 [NQB, NKB] (+ bh * mask_stride_bh) or NULL (none forced)
 *   allowed: uint8 [NQB, NKB] (+ bh * mask_stride_bh) or NULL (all allowed)
 *   indices: int32 [n_bh, NQB, max_k] (row stride max_k); slots >= count hold -1
 *   counts:  int32 [n_bh, NQB]
 * k values above max_k are clamped to max_k.  n_kblocks <= 65536.
 */
int rcsa_select_topk(const float* score, int64_t n_bh, int64_t n_qblocks,
                     int64_t n_kblocks, const int32_t* row_k,
                     int64_t row_k_stride_bh, int64_t k_fixed,
                     const uint8_t* forced, const uint8_t* allowed,
                     int64_t mask_stride_bh, int32_t* indices, int64_t max_k,
                     int32_t* counts, int order, hipStream_t stream);

/*
 * int8 key quantiser with per-head mean smoothing.  No reference
 * counterpart: the reference feeds bf16 keys to the sparse kernel
 * (P/matrix_jit_spatial_acceleration.py:676-678).  Uses the statistics of
 * rcsa_pool_key:
 *   kmean[bh, c]    = sum_b ksum[bh, b, c] / max(sum_b n_valid(b), 1)
 *   k_scale[bh, b]  = max_c max(kmax - kmean, kmean - kmin) / 127   (1 if 0)
 *   k_i8[bh, t, c]  = clamp(rne((k - kmean) / k_scale), -127, 127), 0 on invalid tokens
 * Softmax is invariant to the per-row constant q . kmean, so attention over
 * the smoothed keys equals attention over the original keys.
 * slot_token (nullable): gathered keys, as for rcsa_pool_query_key (k is the
 * token-major source of src_len tokens; k_i8 stays packed).
 */
int rcsa_quantize_key(const void* k, int dtype, int64_t batch, int64_t n_heads,
                      int64_t n_blocks, int64_t block_size, int64_t head_dim,
                      int64_t stride_b, int64_t stride_h, int64_t stride_t,
                      const uint8_t* valid, const int32_t* slot_token, int64_t src_len,
                      const float* ksum,
                      const float* kmin, const float* kmax, float* kmean,
                      int8_t* k_i8, float* k_scale, hipStream_t stream);

/*
 * rcsa_quantize_key, rcsa_block_scores and rcsa_select_topk (index order) in
 * two launches instead of four: the key mean, then one launch whose first
 * workgroups score and select the rows (one wavefront per row) while the rest
 * quantise the key tiles.  Outputs are those of the separate calls bit for
 * bit (each score is summed over the channels in rcsa_block_scores' order).
 * No reference counterpart: the int8 layer call's form, replacing a side
 * stream and its two cross-stream waits.  qhat [n_bh][n_qblocks][D] and khat
 * [n_bh][n_blocks][D] come from the pooling pass; score receives
 * [n_bh][n_qblocks][n_blocks]; the selection arguments are those of
 * rcsa_select_topk.  bf16 keys, head_dim 128, block_size 128 and n_blocks <=
 * 1024 only (RCSA_ERR_SHAPE otherwise: use the separate calls).
 */
int rcsa_quantize_key_select(const void* k, int dtype, int64_t batch, int64_t n_heads,
                             int64_t n_blocks, int64_t block_size, int64_t head_dim,
                             int64_t stride_b, int64_t stride_h, int64_t stride_t,
                             const uint8_t* valid, const int32_t* slot_token, int64_t src_len,
                             const float* ksum, const float* kmin, const float* kmax,
                             float* kmean, int8_t* k_i8, float* k_scale, const float* qhat,
                             const float* khat, int64_t n_qblocks, float* score,
                             const int32_t* row_k, int64_t row_k_stride_bh, int64_t k_fixed,
                             const uint8_t* forced, const uint8_t* allowed,
                             int64_t mask_stride_bh, int32_t* indices, int64_t max_k,
                             int32_t* counts, hipStream_t stream);

/*
 * Block-sparse flash attention, bf16 Q/K/V, fp32 online softmax.
 * Drop-in for wan.modules.longcat_kernel._attn_fwd_bsa_align as launched by
 * _longcat_active (P/matrix_jit_spatial_acceleration.py:663-729) and
 * _longcat_asymmetric (P/matrix_curvature_phase_frame_weave.py:8847-8917):
 * same argument meaning and order.  For every (b, h, query block m):
 *   out[b,h,i,:] = softmax_j(sm_scale * q_i . k_j) v_j over the key tokens j of
 *   blocks block_indices[b,h,m,0:lens[b,h,m]] with j < K_LEN and K_valid[j] != 0.
 * M (nullable) receives the natural-log log-sum-exp of each row
 * (-inf for a row with no admissible key, whose output row is 0).
 * Indices outside [0, ceil(K_LEN/BLOCK_N)) are skipped; lens are clamped to
 * [0, max_k].  Strides are in elements; every *_k / *_bs stride must be 1;
 * a K or V row (stride_kn, stride_vn) spans less than 16 MiB.
 * HEAD_DIM in {64, 128}; BLOCK_M, BLOCK_N in {64, 128}.
 * Alignment: Q/K/V rows 16-byte aligned, Out 8-byte aligned, K_valid (when
 * not NULL) 16-byte aligned -- it is read in aligned 16-byte chunks, so up
 * to 15 bytes past K_LEN inside the same chunk may be read (never used).
 */
int rcsa_sparse_attn_bf16(const void* Q, const void* K, const void* V,
                          const uint8_t* K_valid, float sm_scale, float* M,
                          void* Out, const int32_t* block_indices,
                          const int32_t* block_indices_lens,
                          int64_t stride_qz, int64_t stride_qh, int64_t stride_qm,
                          int64_t stride_kz, int64_t stride_kh, int64_t stride_kn,
                          int64_t stride_vz, int64_t stride_vh, int64_t stride_vn,
                          int64_t stride_oz, int64_t stride_oh, int64_t stride_om,
                          int64_t stride_bz, int64_t stride_bh, int64_t stride_bm,
                          int64_t stride_lz, int64_t stride_lh, int64_t stride_lm,
                          int64_t B, int64_t H, int64_t Q_LEN, int64_t K_LEN,
                          int64_t HEAD_DIM, int64_t BLOCK_M, int64_t BLOCK_N,
                          int64_t max_k, hipStream_t stream);

/*
 * Block-sparse flash attention with int8 QK^T (i32 MFMA accumulate) and
 * bf16 PV (fp32 MFMA accumulate), fp32 online softmax.  Same contract as
 * rcsa_sparse_attn_bf16 with Q/K replaced by the quantiser outputs:
 *   logits = sm_scale * q_scale[b*H+h, m] * k_scale[b*H+h, n] * (q_i8 . k_i8)
 * q_scale has ceil(Q_LEN/BLOCK_M) entries per head and k_scale
 * ceil(K_LEN/BLOCK_N) entries per head (row strides given).
 * K_block_mask (optional, 4-byte aligned): the key validity as bits, uint32
 * [ceil(K_LEN/BLOCK_N)][BLOCK_N / 32] in rcsa_pool_key's block_mask form;
 * when given it replaces K_valid (which may then be NULL) and the kernel
 * reads it with scalar loads instead of staging validity bytes.
 * out_token (nullable): output scatter.  Row r of the packed query writes row
 * out_token[r] of Out and M, which then hold out_len rows per (b, h) (e.g. a
 * token-major [B, L, H, D] Out with stride_om = H * D); -1, or a row >=
 * out_len, is not written, and no row may appear twice.  Rows of Out that no
 * slot maps to are left as they were.  Fuses output_packed[:, token_to_packed]
 * (P/matrix_curvature_phase_frame_weave.py:6095) into the epilogue.
 */
int rcsa_sparse_attn_int8(const int8_t* Q, const float* q_scale,
                          int64_t q_scale_stride, const int8_t* K,
                          const float* k_scale, int64_t k_scale_stride,
                          const void* V, const uint8_t* K_valid,
                          const uint32_t* K_block_mask, float sm_scale,
                          float* M, void* Out, const int32_t* block_indices,
                          const int32_t* block_indices_lens,
                          int64_t stride_qz, int64_t stride_qh, int64_t stride_qm,
                          int64_t stride_kz, int64_t stride_kh, int64_t stride_kn,
                          int64_t stride_vz, int64_t stride_vh, int64_t stride_vn,
                          int64_t stride_oz, int64_t stride_oh, int64_t stride_om,
                          int64_t stride_bz, int64_t stride_bh, int64_t stride_bm,
                          int64_t stride_lz, int64_t stride_lh, int64_t stride_lm,
                          int64_t B, int64_t H, int64_t Q_LEN, int64_t K_LEN,
                          int64_t HEAD_DIM, int64_t BLOCK_M, int64_t BLOCK_N,
                          int64_t max_k, const int32_t* out_token, int64_t out_len,
                          hipStream_t stream);

/*
 * Split-list variants of the two attention entry points (same arguments,
 * then n_split, workspace, workspace_bytes).  No reference counterpart: the
 * reference launches one program per (query block, B*H).  The query blocks
 * are dealt to the device's 8 XCDs in contiguous runs; on each XCD, those
 * that would run in a last round leaving compute units idle (all of them
 * when the XCD's blocks do not fill one round) have their lists cut into
 * n_split contiguous shares handled by separate workgroups.  The shares'
 * normalised partial outputs and (max, sum) pairs go to the caller's
 * workspace and a second kernel on the same stream combines them:
 *   w_s = l_s 2^(m_s - M),  out = sum_s w_s O_s / sum_s w_s.
 * n_split == 1 is the plain entry point (workspace may be NULL); so is any
 * n_split when every XCD's query blocks fill whole rounds.
 * The bf16 variant also takes K_block_mask (uint32 [NKB, BLOCK_N / 32], bit i of
 * word w of block n = validity of key n * BLOCK_N + 32 w + i, 4-byte aligned,
 * as rcsa_pool_key writes it); when it is not NULL the bits replace K_valid.
 * workspace: 16-byte aligned, at least rcsa_attn_workspace_bytes(...) bytes.
 *
 * Gathered sources (the q[:, flat] / k[:, flat] / v[:, flat] gathers and the
 * scatter back to token rows of P/matrix_curvature_phase_frame_weave.py:
 * 5677-5684 and 6095 fused into the kernel; no reference counterpart as an
 * entry point).  kv_token (int32 [K_LEN], 4-byte aligned; NULL = packed
 * sources) maps packed key slot s to row kv_token[s] of a token-major V
 * ([B, kv_len, H, D]; stride_vn is then the token stride) — for the bf16
 * variant also of K — and -1 (or a row >= kv_len) is an empty slot that reads
 * zeros.  The bf16 variant takes q_token (int32 [Q_LEN]) with it: Q row r is
 * token q_token[r] of a token-major Q of q_tokens rows, and O / M are written
 * to row out_token[r] of [B, out_len, H, D] / [B, H, out_len] (-1 rows are
 * dropped), as out_token does for the int8 variant; with out_token NULL they
 * go to row q_token[r] of q_tokens rows.  Needs K_block_mask,
 * HEAD_DIM 128, BLOCK_M = BLOCK_N = 128, K_LEN a multiple of 128 and
 * kv_len x (V, bf16 also K) row stride below 2^31 bytes; else RCSA_ERR_SHAPE.
 */
int rcsa_sparse_attn_bf16_split(const void* Q, const void* K, const void* V,
                                const uint8_t* K_valid, const uint32_t* K_block_mask,
                                float sm_scale, float* M,
                                void* Out, const int32_t* block_indices,
                                const int32_t* block_indices_lens,
                                int64_t stride_qz, int64_t stride_qh, int64_t stride_qm,
                                int64_t stride_kz, int64_t stride_kh, int64_t stride_kn,
                                int64_t stride_vz, int64_t stride_vh, int64_t stride_vn,
                                int64_t stride_oz, int64_t stride_oh, int64_t stride_om,
                                int64_t stride_bz, int64_t stride_bh, int64_t stride_bm,
                                int64_t stride_lz, int64_t stride_lh, int64_t stride_lm,
                                int64_t B, int64_t H, int64_t Q_LEN, int64_t K_LEN,
                                int64_t HEAD_DIM, int64_t BLOCK_M, int64_t BLOCK_N,
                                int64_t max_k, int64_t n_split, void* workspace,
                                int64_t workspace_bytes, const int32_t* q_token,
                                int64_t q_tokens, const int32_t* kv_token, int64_t kv_len,
                                const int32_t* out_token, int64_t out_len,
                                hipStream_t stream);
int rcsa_sparse_attn_int8_split(const int8_t* Q, const float* q_scale,
                                int64_t q_scale_stride, const int8_t* K,
                                const float* k_scale, int64_t k_scale_stride,
                                const void* V, const uint8_t* K_valid,
                                const uint32_t* K_block_mask, float sm_scale,
                                float* M, void* Out, const int32_t* block_indices,
                                const int32_t* block_indices_lens,
                                int64_t stride_qz, int64_t stride_qh, int64_t stride_qm,
                                int64_t stride_kz, int64_t stride_kh, int64_t stride_kn,
                                int64_t stride_vz, int64_t stride_vh, int64_t stride_vn,
                                int64_t stride_oz, int64_t stride_oh, int64_t stride_om,
                                int64_t stride_bz, int64_t stride_bh, int64_t stride_bm,
                                int64_t stride_lz, int64_t stride_lh, int64_t stride_lm,
                                int64_t B, int64_t H, int64_t Q_LEN, int64_t K_LEN,
                                int64_t HEAD_DIM, int64_t BLOCK_M, int64_t BLOCK_N,
                                int64_t max_k, int64_t n_split, void* workspace,
                                int64_t workspace_bytes, const int32_t* out_token,
                                int64_t out_len, const int32_t* kv_token, int64_t kv_len,
                                hipStream_t stream);

/*
 * The split int8 entry point with no workspace argument: it allocates
 * nothing.  No reference counterpart; it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  The split shares' partial outputs and (max, sum)
 * pairs live in a static device array of rcsa_attn_noalloc_scratch_bytes()
 * bytes (32 MiB) that each GPU holds until the process ends; a split whose
 * workspace would exceed it returns RCSA_ERR_SCRATCH (n_split 3 covers up to
 * 8 * 31 = 248 tail query blocks of 128 rows at HEAD_DIM 128).  Every call on
 * one GPU shares that GPU's array: calls that overlap on one GPU (different
 * streams, or threads) race, so the caller serialises them: one stream per
 * device, or an event recorded after each call and waited on by the stream of
 * the next.  Arguments and results as
 * rcsa_sparse_attn_int8_split.
 */
int rcsa_sparse_attn_int8_noalloc(const int8_t* Q, const float* q_scale,
                                  int64_t q_scale_stride, const int8_t* K,
                                  const float* k_scale, int64_t k_scale_stride,
                                  const void* V, const uint8_t* K_valid,
                                  const uint32_t* K_block_mask, float sm_scale,
                                  float* M, void* Out, const int32_t* block_indices,
                                  const int32_t* block_indices_lens,
                                  int64_t stride_qz, int64_t stride_qh, int64_t stride_qm,
                                  int64_t stride_kz, int64_t stride_kh, int64_t stride_kn,
                                  int64_t stride_vz, int64_t stride_vh, int64_t stride_vn,
                                  int64_t stride_oz, int64_t stride_oh, int64_t stride_om,
                                  int64_t stride_bz, int64_t stride_bh, int64_t stride_bm,
                                  int64_t stride_lz, int64_t stride_lh, int64_t stride_lm,
                                  int64_t B, int64_t H, int64_t Q_LEN, int64_t K_LEN,
                                  int64_t HEAD_DIM, int64_t BLOCK_M, int64_t BLOCK_N,
                                  int64_t max_k, int64_t n_split, const int32_t* out_token,
                                  int64_t out_len, const int32_t* kv_token, int64_t kv_len,
                                  hipStream_t stream);

/* Size in bytes of the static scratch of rcsa_sparse_attn_int8_noalloc. */
int64_t rcsa_attn_noalloc_scratch_bytes(void);

/* Workspace bytes of a split launch on the current device, an upper bound
 * for BLOCK_M in {64, 128} (0 for n_split == 1, -1 on bad sizes). */
int64_t rcsa_attn_workspace_bytes(int64_t B, int64_t H, int64_t Q_LEN, int64_t HEAD_DIM,
                                  int64_t n_split);

/*
 * Split count in 1..8 for the current device.  Each XCD runs
 * ceil(items / 8) of the items = B*H*ceil(Q_LEN/BLOCK_M) query blocks on its
 * compute units (U of them): `full` whole rounds, then `rem` tail blocks.
 * The count s minimises
 *   full * (7 + max_k) + ceil(rem * s / U) * (7 + ceil(max_k / s)),
 * i.e. rounds times the key blocks per workgroup plus a fixed cost of
 * about 7 blocks per workgroup; a larger count must win by 2% and keep at
 * least 2 key blocks per share.  Host-only (reads device attributes).
 */
int rcsa_attn_split_plan(int64_t B, int64_t H, int64_t Q_LEN, int64_t BLOCK_M,
                         int64_t max_k, int64_t* n_split);

/*
 * Gather compact tokens into the packed head-major layout, zeroing invalid
 * slots.  Replaces q[:, flat].transpose(1, 2).contiguous(); q_packed[:, :, ~mask] = 0
 * at P/matrix_curvature_phase_frame_weave.py:5671-5684.
 *   x:      [B, L, H, D]   (strides in elements, last dim contiguous), bf16 or fp32
 *   slot_token: int64 [n_slots]  source token of each packed slot, -1 = invalid
 *   out:    [B, H, n_slots, D] (contiguous), same element type as x
 */
int rcsa_pack_tokens(const void* x, int dtype, int64_t B, int64_t L, int64_t H,
                     int64_t D, int64_t stride_b, int64_t stride_l,
                     int64_t stride_h, const int64_t* slot_token,
                     int64_t n_slots, void* out, hipStream_t stream);

/*
 * Scatter the packed attention output back to token order.  Replaces
 * output_packed[:, token_to_packed] (P/matrix_curvature_phase_frame_weave.py:6095)
 * after the .transpose(1, 2) of :6086-6094.
 *   packed: [B, H, n_slots, D] bf16 (contiguous)
 *   token_slot: int64 [L]  packed slot of each output token
 *   out:    [B, L, H, D] bf16 (contiguous)
 */
int rcsa_unpack_tokens(const void* packed, int64_t B, int64_t H, int64_t n_slots,
                       int64_t D, const int64_t* token_slot, int64_t L, void* out,
                       hipStream_t stream);

/*
 * FC-PASM swap router, the per-row device work of
 * FCPASMLocalCoordinateSwapRouter.refine (P/fc_pasm_swap_routing.py:616-1077).
 *
 * rcsa_route_proxy: for every (bh, current row r >= memory_blocks) of the
 * square block scores score [n_bh][n_blocks][n_blocks] (fp32):
 *   p = softmax(score row) (fp32, max-subtracted), o = p @ pooled_value
 *   (pooled_value fp32 [n_bh][n_blocks][head_dim], the masked block means of V);
 *   cand[bh][r - M][0..n_cand) = the first n_cand blocks by the ranking
 *   score + 1e6 * local (descending, equal rankings by lower block index);
 *   proxy[bh][r - M][l][g] = p_c / (1 - p_c + eps) * mean over channel group g of
 *   (o - pooled_value[c]) for c = cand[l] (estimate_block_omission_error, :64-106);
 *   error[bh][r - M][g] = sum of proxy[l][g] over l < min(cand_mult * count, n_blocks)
 *   whose block the row does not keep (its first count entries of selected).
 * local: uint8 [n_blocks][n_blocks]; selected int32 [n_bh][n_blocks][max_k]; counts
 * int32 [n_bh][n_blocks].  n_blocks <= 1024, head_dim in {64, 128}, sketch_groups
 * <= 16 and divides head_dim, n_cand * sketch_groups <= 12288 (and, for
 * rcsa_route_best_swap, max_k * sketch_groups <= 12288); pooled_value 16-byte
 * aligned.
 *
 * rcsa_route_best_swap: for every (bh, current row), the admissible exchange
 * (a kept slot s whose block is not a local edge, a candidate l < the row's limit
 * that the row does not keep; with same_bank, both in memory or both current;
 * none when row_gate[r - M] == 0) minimising
 *   sum_g coef[r - M] (2 e_g d_g + d_g^2) + 2 linear[bh][r - M][g] d_g,
 *   d = proxy of the removed block (0 if it is not a candidate) - proxy[l],
 *   e = error[bh][r - M]  (the best-swap search of :899-977);
 * best[bh][r - M] = that value (+inf if none), best_flat = s * n_cand + l (-1 if
 * none; equal values go to the lower flat index).  coef fp32 [rows]; linear and
 * error fp32 [n_bh][rows][sketch_groups]; row_gate uint8 [rows] or NULL.
 */
int rcsa_route_proxy(const float* score, const float* pooled_value, const uint8_t* local,
                     const int32_t* selected, const int32_t* counts, int64_t n_bh,
                     int64_t n_blocks, int64_t memory_blocks, int64_t head_dim, int64_t max_k,
                     int64_t n_cand, int64_t cand_mult, int64_t sketch_groups, float eps,
                     int32_t* cand, float* proxy, float* error, hipStream_t stream);
int rcsa_route_best_swap(const float* proxy, const int32_t* cand, const uint8_t* local,
                         const int32_t* selected, const int32_t* counts, const float* coef,
                         const float* linear, const float* error, const uint8_t* row_gate,
                         int64_t n_bh, int64_t n_blocks, int64_t memory_blocks, int64_t max_k,
                         int64_t n_cand, int64_t cand_mult, int64_t sketch_groups,
                         int same_bank, float* best, int32_t* best_flat, hipStream_t stream);

/*
 * One swap round's decision and exchange on the device, replacing the host
 * argmin / scatter / error update of FCPASMLocalCoordinateSwapRouter.refine
 * (P/fc_pasm_swap_routing.py:935-977) so that a refine reads nothing back until
 * its record.  One workgroup: the strongest row is the first minimum of best
 * [n_bh * rows] (rows = n_blocks - memory_blocks); unless state[1] is set, the
 * swap limit max_swaps (> 0) is reached or that minimum is not below -eps, its
 * exchange best_flat = slot * n_cand + l writes cand[l] into the slot of
 * selected [n_bh][n_blocks][max_k] and adds (the removed block's proxy, zero
 * when it is not a candidate of the row) - proxy[l] to the row's error
 * [n_bh][rows][sketch_groups]; otherwise it sets state[1] (stopped).
 * state: int32 [2 + 6 * max_records], zero before the first round:
 * [0] swaps applied, [1] stopped, then per swap (bh, row, slot, removed block,
 * added block, improvement -best as float bits).  max_records <= 64.
 */
int rcsa_route_apply_swap(const float* best, const int32_t* best_flat, const int32_t* cand,
                          const float* proxy, int32_t* selected, float* error, int32_t* state,
                          int64_t n_bh, int64_t n_blocks, int64_t memory_blocks, int64_t max_k,
                          int64_t n_cand, int64_t sketch_groups, int64_t max_swaps,
                          int64_t max_records, float eps, hipStream_t stream);

/*
 * The checks at the end of a refine (P/fc_pasm_swap_routing.py:983-1033) as
 * device sums, so that a refine reads its record back once: over every
 * (bh, row) of the routes before (base) and after (selected), both int32
 * [n_bh][n_blocks][max_k], first min(max(counts, 0), max_k) entries valid,
 * local uint8 [n_blocks][n_blocks] (n_blocks <= 1024), out int32 [10], zero on
 * entry, receives: [0] rows whose memory-bank count changed, [1] rows with a
 * repeated block, [2] local edges kept, [3] rows whose current-bank blocks
 * changed, [4]/[5] memory-bank entries before/after, [6] max_k - the smallest
 * count, [7] the largest count, [8] the count sum, [9] the stencil's local edges
 * over all rows.
 */
int rcsa_route_check(const int32_t* base, const int32_t* selected, const int32_t* counts,
                     const uint8_t* local, int64_t n_bh, int64_t n_blocks,
                     int64_t memory_blocks, int64_t max_k, int32_t* out, hipStream_t stream);

/*
 * Shared int8 Q/K/V projection (P/matrix_shared_int8_qkv.py:19-92): the
 * activations are quantised once per token and reused by the three int8
 * projections.  No reference kernel: the reference calls the upstream Matrix
 * Int8Linear Triton kernels (int8_quantize_triton, int8_gemm_triton), which it
 * does not vendor.
 *
 * rcsa_quantize_rows_int8: x [M][C] (row stride ldx; bf16 or fp32, 16-byte
 * aligned, C and ldx multiples of 8) -> q int8 [M][C] (row stride C, 8-byte
 * aligned), scale fp32 [M]: scale = absmax_c |x| / 127 (1 for an all-zero row),
 * q = clamp(rne(x * 127 / absmax), -127, 127).
 *
 * rcsa_int8_linear: out[m][n] = bf16(bf16(float(acc) * x_scale[m] * w_scale[n])
 * + bias[n]), acc = sum_k x[m][k] w[n][k] (int32), for x int8 [M][K], w int8
 * [N][K] (both 16-byte aligned), w_scale fp32 [N] (16-byte aligned), bias bf16
 * [N] or NULL (then out = bf16(float(acc) * x_scale * w_scale)); out bf16 with
 * row stride ldo (8-byte aligned).  N a multiple of 256, K a multiple of 128.
 * The launch is persistent (one workgroup per compute unit, each with a fixed
 * share of the tiles): it expects the device to itself, and beside other
 * kernels it stays correct but runs as slowly as its latest workgroup.
 */
int rcsa_quantize_rows_int8(const void* x, int dtype, int64_t M, int64_t C, int64_t ldx,
                            int8_t* q, float* scale, hipStream_t stream);
int rcsa_int8_linear(const int8_t* x, const float* x_scale, const int8_t* w, const float* w_scale,
                     const void* bias, int64_t M, int64_t N, int64_t K, void* out, int64_t ldo,
                     hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* RCSA_H_ */
