// PyTorch-ROCm extension over the C ABI of include/rcsa.h: torch custom ops
// (namespace "rcsa") for the entry points of the RCSA layer call (the int8
// Q/K/V projection, the pooling pass, key quantisation + selection, the
// attention) and of the block-sparse attention drop-in.  Each op takes the tensors the Python
// wrapper has shaped and allocated (cast_amd/ops.py), checks them (device,
// dtype, rank, sizes against the launch dimensions), launches on the current
// HIP stream of the tensors' device and raises RuntimeError("<op>: <reason>
// (status N)") on a non-zero status, as the reference's wrappers raise on a
// bad layout.  Every tensor is checked to span the elements the call's dims
// and strides reach, so no argument combination makes a kernel read or write
// past the tensors it was given.  Nothing here allocates device memory or
// synchronises.
//
// The C ABI is bound at load time (rcsa::bind_library) from the library the
// Python side loaded, so one librcsa.so serves both the ctypes binding and
// these ops.
#include <dlfcn.h>

#include <cstdint>
#include <mutex>
#include <string>
#include <vector>

#include <c10/hip/HIPGuard.h>
#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime_api.h>
#include <torch/library.h>

#include "../../include/rcsa.h"

namespace {

struct Api {
  decltype(&rcsa_status_string) status_string = nullptr;
  decltype(&rcsa_pool_query_key) pool_query_key = nullptr;
  decltype(&rcsa_quantize_key_select) quantize_key_select = nullptr;
  decltype(&rcsa_sparse_attn_bf16_split) sparse_attn_bf16_split = nullptr;
  decltype(&rcsa_sparse_attn_int8_split) sparse_attn_int8_split = nullptr;
  decltype(&rcsa_quantize_rows_int8) quantize_rows_int8 = nullptr;
  decltype(&rcsa_int8_linear) int8_linear = nullptr;
};

std::mutex g_mu;
Api g_api;
bool g_bound = false;

template <typename F>
void bind_one(void* h, const char* name, F& slot) {
  void* p = dlsym(h, name);
  TORCH_CHECK(p != nullptr, "rcsa::bind_library: ", name, " is not exported");
  slot = reinterpret_cast<F>(p);
}

void bind_library(const std::string& path) {
  std::lock_guard<std::mutex> lock(g_mu);
  void* h = dlopen(path.c_str(), RTLD_NOW | RTLD_GLOBAL);
  TORCH_CHECK(h != nullptr, "rcsa::bind_library: cannot load ", path, ": ", dlerror());
  Api api;
  bind_one(h, "rcsa_status_string", api.status_string);
  bind_one(h, "rcsa_pool_query_key", api.pool_query_key);
  bind_one(h, "rcsa_quantize_key_select", api.quantize_key_select);
  bind_one(h, "rcsa_sparse_attn_bf16_split", api.sparse_attn_bf16_split);
  bind_one(h, "rcsa_sparse_attn_int8_split", api.sparse_attn_int8_split);
  bind_one(h, "rcsa_quantize_rows_int8", api.quantize_rows_int8);
  bind_one(h, "rcsa_int8_linear", api.int8_linear);
  g_api = api;
  g_bound = true;
}

const Api& api(const char* op) {
  std::lock_guard<std::mutex> lock(g_mu);
  TORCH_CHECK(g_bound, op, ": the RCSA library is not bound (load cast_amd first)");
  return g_api;
}

void check_status(const Api& a, const char* op, int status) {
  TORCH_CHECK(status == 0, op, ": ", a.status_string(status), " (status ", status, ")");
}

// The device every tensor of a call lives on (made current for the call)
// and that device's current stream.
struct Launch {
  c10::hip::HIPGuard guard;
  hipStream_t stream;
  explicit Launch(int device)
      : guard(static_cast<c10::DeviceIndex>(device)),
        stream(c10::hip::getCurrentHIPStream(static_cast<c10::DeviceIndex>(device)).stream()) {}
};

void on_device(const char* op, int& device, const at::Tensor& t, const char* name) {
  TORCH_CHECK(t.defined() && t.is_cuda(), op, ": ", name, " must be a GPU tensor");
  const int d = t.get_device();
  TORCH_CHECK(device < 0 || d == device, op, ": ", name, " is on another GPU");
  device = d;
}

void on_device(const char* op, int& device, const c10::optional<at::Tensor>& t, const char* name) {
  if (t.has_value() && t->defined()) on_device(op, device, *t, name);
}

int device_of(const char* op, int device) {
  TORCH_CHECK(device >= 0, op, ": no GPU tensor");
  return device;
}

void want(const char* op, const at::Tensor& t, at::ScalarType dt, const char* name) {
  TORCH_CHECK(t.scalar_type() == dt, op, ": ", name, " has dtype ", t.scalar_type(),
              ", expected ", dt);
}

// Elements a strided view spans from its first element (0 when empty).
int64_t span(const char* op, const at::Tensor& t, const char* name) {
  if (t.numel() == 0) return 0;
  int64_t s = 1;
  for (int64_t i = 0; i < t.dim(); ++i) {
    TORCH_CHECK(t.stride(i) >= 0, op, ": ", name, " has a negative stride");
    s += (t.size(i) - 1) * t.stride(i);
  }
  return s;
}

// The call reaches `need` elements from the tensor's first element.
void want_numel(const char* op, const at::Tensor& t, int64_t need, const char* name) {
  const int64_t have = span(op, t, name);
  TORCH_CHECK(need <= have, op, ": ", name, " spans ", have, " elements, the call reaches ", need);
}
void want_numel(const char* op, const c10::optional<at::Tensor>& t, int64_t need,
                const char* name) {
  if (t.has_value() && t->defined()) want_numel(op, *t, need, name);
}

// Elements reached by rows [0, n2) of planes [0, n0) x [0, n1) with strides
// (s0, s1, s2) and `inner` unit-stride elements per row.
int64_t reach(const char* op, int64_t n0, int64_t n1, int64_t n2, int64_t inner, int64_t s0,
              int64_t s1, int64_t s2) {
  TORCH_CHECK(s0 >= 0 && s1 >= 0 && s2 >= 0, op, ": strides must not be negative");
  if (n0 <= 0 || n1 <= 0 || n2 <= 0 || inner <= 0) return 0;
  return 1 + (n0 - 1) * s0 + (n1 - 1) * s1 + (n2 - 1) * s2 + (inner - 1);
}

int64_t cdiv(int64_t a, int64_t b) { return b > 0 ? (a + b - 1) / b : 0; }

void want(const char* op, const c10::optional<at::Tensor>& t, at::ScalarType dt,
          const char* name) {
  if (t.has_value() && t->defined()) want(op, *t, dt, name);
}

// One byte per element, read as "!= 0" (bool, uint8 or int8 masks).
void want_bytes(const char* op, const c10::optional<at::Tensor>& t, const char* name) {
  if (!t.has_value() || !t->defined()) return;
  const auto dt = t->scalar_type();
  TORCH_CHECK(dt == at::kBool || dt == at::kByte || dt == at::kChar, op, ": ", name,
              " has dtype ", dt, ", expected a byte mask (bool or uint8)");
}

// The source dtype code of the pooling entry points (RCSA_BF16 / RCSA_F32).
void want_code(const char* op, const at::Tensor& t, int64_t code, const char* name) {
  TORCH_CHECK(code == RCSA_BF16 || code == RCSA_F32, op, ": unknown dtype code ", code);
  want(op, t, code == RCSA_BF16 ? at::kBFloat16 : at::kFloat, name);
}

template <typename T>
T* ptr(const c10::optional<at::Tensor>& t) {
  return (t.has_value() && t->defined()) ? static_cast<T*>(t->data_ptr()) : nullptr;
}

template <typename T>
T* ptr(const at::Tensor& t) {
  return static_cast<T*>(t.data_ptr());
}

void want_len(const char* op, c10::IntArrayRef v, size_t n, const char* name) {
  TORCH_CHECK(v.size() == n, op, ": ", name, " needs ", n, " values");
}

// dims = [B, H, NQ, NK, block_size, D]; strides in elements of the sources
void pool_query_key(const at::Tensor& q, const at::Tensor& k, int64_t dtype, c10::IntArrayRef dims,
                    c10::IntArrayRef q_strides, c10::IntArrayRef k_strides,
                    const c10::optional<at::Tensor>& q_valid,
                    const c10::optional<at::Tensor>& k_valid,
                    const c10::optional<at::Tensor>& q_slot_token, int64_t q_src_len,
                    const c10::optional<at::Tensor>& k_slot_token, int64_t k_src_len,
                    const at::Tensor& qhat, const c10::optional<at::Tensor>& q_i8,
                    const c10::optional<at::Tensor>& q_scale, const at::Tensor& khat,
                    const c10::optional<at::Tensor>& ksum, const c10::optional<at::Tensor>& kmin,
                    const c10::optional<at::Tensor>& kmax, const at::Tensor& block_mask) {
  const char* op = "pool_query_key";
  const Api& a = api(op);
  want_len(op, dims, 6, "dims");
  want_len(op, q_strides, 3, "q_strides");
  want_len(op, k_strides, 3, "k_strides");
  int dev = -1;
  on_device(op, dev, q, "q");
  on_device(op, dev, k, "k");
  on_device(op, dev, q_valid, "q_valid");
  on_device(op, dev, k_valid, "k_valid");
  on_device(op, dev, q_slot_token, "q_slot_token");
  on_device(op, dev, k_slot_token, "k_slot_token");
  on_device(op, dev, qhat, "qhat");
  on_device(op, dev, q_i8, "q_i8");
  on_device(op, dev, q_scale, "q_scale");
  on_device(op, dev, khat, "khat");
  on_device(op, dev, ksum, "ksum");
  on_device(op, dev, kmin, "kmin");
  on_device(op, dev, kmax, "kmax");
  on_device(op, dev, block_mask, "block_mask");
  const int64_t B = dims[0], H = dims[1], NQ = dims[2], NK = dims[3], BS = dims[4], D = dims[5];
  want_code(op, q, dtype, "q");
  want_code(op, k, dtype, "k");
  want_numel(op, q, reach(op, B, H, q_slot_token.has_value() ? q_src_len : NQ * BS, D,
                          q_strides[0], q_strides[1], q_strides[2]), "q");
  want_numel(op, k, reach(op, B, H, k_slot_token.has_value() ? k_src_len : NK * BS, D,
                          k_strides[0], k_strides[1], k_strides[2]), "k");
  want_numel(op, q_valid, NQ * BS, "q_valid");
  want_numel(op, k_valid, NK * BS, "k_valid");
  want_bytes(op, q_valid, "q_valid");
  want_bytes(op, k_valid, "k_valid");
  want(op, q_slot_token, at::kInt, "q_slot_token");
  want(op, k_slot_token, at::kInt, "k_slot_token");
  want(op, q_scale, at::kFloat, "q_scale");
  for (const auto* t : {&ksum, &kmin, &kmax}) want(op, *t, at::kFloat, "key statistics");
  want_numel(op, q_slot_token, NQ * BS, "q_slot_token");
  want_numel(op, k_slot_token, NK * BS, "k_slot_token");
  want(op, qhat, at::kFloat, "qhat");
  want(op, khat, at::kFloat, "khat");
  want(op, block_mask, at::kInt, "block_mask");
  want_numel(op, qhat, B * H * NQ * D, "qhat");
  want_numel(op, khat, B * H * NK * D, "khat");
  want_numel(op, q_i8, B * H * NQ * BS * D, "q_i8");
  want_numel(op, q_scale, B * H * NQ, "q_scale");
  for (const auto* t : {&ksum, &kmin, &kmax}) want_numel(op, *t, B * H * NK * D, "key statistics");
  want_numel(op, block_mask, NK * cdiv(BS, 32), "block_mask");
  if (q_i8.has_value()) want(op, *q_i8, at::kChar, "q_i8");
  const Launch l(device_of(op, dev));
  check_status(a, op, a.pool_query_key(
      q.data_ptr(), k.data_ptr(), static_cast<int>(dtype), B, H, NQ, NK, BS, D, q_strides[0],
      q_strides[1], q_strides[2], k_strides[0], k_strides[1], k_strides[2],
      ptr<const uint8_t>(q_valid), ptr<const uint8_t>(k_valid), ptr<const int32_t>(q_slot_token),
      q_src_len, ptr<const int32_t>(k_slot_token), k_src_len, ptr<float>(qhat),
      ptr<int8_t>(q_i8), ptr<float>(q_scale), ptr<float>(khat), ptr<float>(ksum),
      ptr<float>(kmin), ptr<float>(kmax), ptr<uint32_t>(block_mask), l.stream));
}

// dims = [B, H, NB, block_size, D]; strides of k in elements
void quantize_key_select(const at::Tensor& k, int64_t dtype, c10::IntArrayRef dims,
                         c10::IntArrayRef strides, const c10::optional<at::Tensor>& valid,
                         const c10::optional<at::Tensor>& slot_token, int64_t src_len,
                         const at::Tensor& ksum, const at::Tensor& kmin, const at::Tensor& kmax,
                         const at::Tensor& kmean, const at::Tensor& k_i8,
                         const at::Tensor& k_scale, const at::Tensor& qhat,
                         const at::Tensor& khat, int64_t n_qblocks, const at::Tensor& score,
                         const c10::optional<at::Tensor>& row_k, int64_t row_k_stride_bh,
                         int64_t k_fixed, const c10::optional<at::Tensor>& forced,
                         const c10::optional<at::Tensor>& allowed, int64_t mask_stride_bh,
                         const at::Tensor& indices, int64_t max_k, const at::Tensor& counts) {
  const char* op = "quantize_key_select";
  const Api& a = api(op);
  want_len(op, dims, 5, "dims");
  want_len(op, strides, 3, "strides");
  int dev = -1;
  for (const auto* t : {&k, &ksum, &kmin, &kmax, &kmean, &k_i8, &k_scale, &qhat, &khat, &score,
                        &indices, &counts})
    on_device(op, dev, *t, "a tensor argument");
  on_device(op, dev, valid, "valid");
  on_device(op, dev, slot_token, "slot_token");
  on_device(op, dev, row_k, "row_k");
  on_device(op, dev, forced, "forced");
  on_device(op, dev, allowed, "allowed");
  const int64_t B = dims[0], H = dims[1], NB = dims[2], BS = dims[3], D = dims[4];
  const int64_t BH = B * H, NQ = n_qblocks;
  want_code(op, k, dtype, "k");
  want(op, k_i8, at::kChar, "k_i8");
  want(op, indices, at::kInt, "indices");
  want(op, counts, at::kInt, "counts");
  want_numel(op, k, reach(op, B, H, slot_token.has_value() ? src_len : NB * BS, D, strides[0],
                          strides[1], strides[2]), "k");
  want_numel(op, valid, NB * BS, "valid");
  want_bytes(op, valid, "valid");
  want_bytes(op, forced, "forced");
  want_bytes(op, allowed, "allowed");
  want(op, slot_token, at::kInt, "slot_token");
  want(op, row_k, at::kInt, "row_k");
  for (const auto* t : {&ksum, &kmin, &kmax, &kmean, &k_scale, &qhat, &khat, &score})
    want(op, *t, at::kFloat, "fp32 operand");
  want_numel(op, slot_token, NB * BS, "slot_token");
  for (const auto* t : {&ksum, &kmin, &kmax, &khat}) want_numel(op, *t, BH * NB * D, "key blocks");
  want_numel(op, kmean, BH * D, "kmean");
  want_numel(op, k_i8, BH * NB * BS * D, "k_i8");
  want_numel(op, k_scale, BH * NB, "k_scale");
  want_numel(op, qhat, BH * NQ * D, "qhat");
  want_numel(op, score, BH * NQ * NB, "score");
  TORCH_CHECK(row_k_stride_bh >= 0 && mask_stride_bh >= 0, op, ": strides must not be negative");
  if (NQ > 0) {
    want_numel(op, row_k, (BH - 1) * row_k_stride_bh + NQ, "row_k");
    want_numel(op, forced, (BH - 1) * mask_stride_bh + NQ * NB, "forced");
    want_numel(op, allowed, (BH - 1) * mask_stride_bh + NQ * NB, "allowed");
  }
  want_numel(op, indices, BH * NQ * max_k, "indices");
  want_numel(op, counts, BH * NQ, "counts");
  const Launch l(device_of(op, dev));
  check_status(a, op, a.quantize_key_select(
      k.data_ptr(), static_cast<int>(dtype), B, H, NB, BS, D, strides[0], strides[1], strides[2],
      ptr<const uint8_t>(valid), ptr<const int32_t>(slot_token), src_len, ptr<const float>(ksum),
      ptr<const float>(kmin), ptr<const float>(kmax), ptr<float>(kmean), ptr<int8_t>(k_i8),
      ptr<float>(k_scale), ptr<const float>(qhat), ptr<const float>(khat), n_qblocks,
      ptr<float>(score), ptr<const int32_t>(row_k), row_k_stride_bh, k_fixed,
      ptr<const uint8_t>(forced), ptr<const uint8_t>(allowed), mask_stride_bh,
      ptr<int32_t>(indices), max_k, ptr<int32_t>(counts), l.stream));
}

// Shared checks of the attention ops.  dims = [B, H, Q_LEN, K_LEN, D, BLOCK_M,
// BLOCK_N, max_k]; strides = q, k, v, out, indices, counts (three each).
struct AttnDims {
  int64_t B, H, Lq, Lk, D, BM, BN, max_k;
};

AttnDims attn_dims(const char* op, c10::IntArrayRef dims, c10::IntArrayRef strides,
                   const at::Tensor& indices, const at::Tensor& counts) {
  want_len(op, dims, 8, "dims");
  want_len(op, strides, 18, "strides");
  want(op, indices, at::kInt, "indices");
  want(op, counts, at::kInt, "counts");
  const AttnDims d{dims[0], dims[1], dims[2], dims[3], dims[4], dims[5], dims[6], dims[7]};
  TORCH_CHECK(indices.dim() == 4 && indices.size(3) == d.max_k, op,
              ": indices must be [B, H, query blocks, max_k]");
  TORCH_CHECK(counts.dim() == 3, op, ": counts must be [B, H, query blocks]");
  const int64_t nqb = cdiv(d.Lq, d.BM);
  want_numel(op, indices, reach(op, d.B, d.H, nqb, d.max_k, strides[12], strides[13],
                                strides[14]), "indices");
  want_numel(op, counts, reach(op, d.B, d.H, nqb, 1, strides[15], strides[16], strides[17]),
             "counts");
  return d;
}

// Extents of the operands every attention op shares: the key validity, the
// LSE rows and the slot maps (q_token / kv_token / out_token: rows of the
// token-major sources and output, or none).
void attn_common(const char* op, const AttnDims& d, const c10::optional<at::Tensor>& k_valid,
                 const c10::optional<at::Tensor>& block_mask, const c10::optional<at::Tensor>& lse,
                 int64_t lse_rows, const c10::optional<at::Tensor>& q_token,
                 const c10::optional<at::Tensor>& kv_token,
                 const c10::optional<at::Tensor>& out_token) {
  want_numel(op, k_valid, d.Lk, "k_valid");
  want_numel(op, block_mask, cdiv(d.Lk, d.BN) * cdiv(d.BN, 32), "block_mask");
  want_numel(op, lse, d.B * d.H * lse_rows, "lse");
  want_numel(op, q_token, d.Lq, "q_token");
  want_numel(op, kv_token, d.Lk, "kv_token");
  want_numel(op, out_token, d.Lq, "out_token");
  want_bytes(op, k_valid, "k_valid");
  if (block_mask.has_value()) want(op, *block_mask, at::kInt, "block_mask");
  if (lse.has_value()) want(op, *lse, at::kFloat, "lse");
  for (const auto* t : {&q_token, &kv_token, &out_token})
    if (t->has_value()) want(op, **t, at::kInt, "slot map");
}

void sparse_attn_bf16(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                      const c10::optional<at::Tensor>& k_valid,
                      const c10::optional<at::Tensor>& block_mask, double sm_scale,
                      const c10::optional<at::Tensor>& lse, const at::Tensor& out,
                      const at::Tensor& indices, const at::Tensor& counts, c10::IntArrayRef dims,
                      c10::IntArrayRef strides, int64_t n_split,
                      const c10::optional<at::Tensor>& workspace,
                      const c10::optional<at::Tensor>& q_token, int64_t q_tokens,
                      const c10::optional<at::Tensor>& kv_token, int64_t kv_len,
                      const c10::optional<at::Tensor>& out_token, int64_t out_len) {
  const char* op = "sparse_attn_bf16";
  const Api& a = api(op);
  const AttnDims d = attn_dims(op, dims, strides, indices, counts);
  int dev = -1;
  for (const auto* t : {&q, &k, &v, &out, &indices, &counts}) on_device(op, dev, *t, "a tensor argument");
  on_device(op, dev, k_valid, "k_valid");
  on_device(op, dev, block_mask, "block_mask");
  on_device(op, dev, lse, "lse");
  on_device(op, dev, workspace, "workspace");
  on_device(op, dev, q_token, "q_token");
  on_device(op, dev, kv_token, "kv_token");
  on_device(op, dev, out_token, "out_token");
  for (const auto* t : {&q, &k, &v, &out}) want(op, *t, at::kBFloat16, "q/k/v/out");
  const auto& s = strides;
  const int64_t q_rows = q_token.has_value() ? q_tokens : d.Lq;
  const int64_t kv_rows = kv_token.has_value() ? kv_len : d.Lk;
  // output rows go through out_token, else through q_token (gathered), else packed
  const int64_t o_rows = out_token.has_value() ? out_len : q_rows;
  want_numel(op, q, reach(op, d.B, d.H, q_rows, d.D, s[0], s[1], s[2]), "q");
  want_numel(op, k, reach(op, d.B, d.H, kv_rows, d.D, s[3], s[4], s[5]), "k");
  want_numel(op, v, reach(op, d.B, d.H, kv_rows, d.D, s[6], s[7], s[8]), "v");
  want_numel(op, out, reach(op, d.B, d.H, o_rows, d.D, s[9], s[10], s[11]), "out");
  attn_common(op, d, k_valid, block_mask, lse, o_rows, q_token, kv_token, out_token);
  const int64_t ws_bytes = workspace.has_value() ? workspace->numel() * workspace->element_size() : 0;
  const Launch l(device_of(op, dev));
  check_status(a, op, a.sparse_attn_bf16_split(
      q.data_ptr(), k.data_ptr(), v.data_ptr(), ptr<const uint8_t>(k_valid),
      ptr<const uint32_t>(block_mask), static_cast<float>(sm_scale), ptr<float>(lse),
      out.data_ptr(), ptr<const int32_t>(indices), ptr<const int32_t>(counts), s[0], s[1], s[2],
      s[3], s[4], s[5], s[6], s[7], s[8], s[9], s[10], s[11], s[12], s[13], s[14], s[15], s[16],
      s[17], d.B, d.H, d.Lq, d.Lk, d.D, d.BM, d.BN, d.max_k, n_split, ptr<void>(workspace),
      ws_bytes, ptr<const int32_t>(q_token), q_tokens, ptr<const int32_t>(kv_token), kv_len,
      ptr<const int32_t>(out_token), out_len, l.stream));
}

void sparse_attn_int8(const at::Tensor& q_i8, const at::Tensor& q_scale, int64_t q_scale_stride,
                      const at::Tensor& k_i8, const at::Tensor& k_scale, int64_t k_scale_stride,
                      const at::Tensor& v, const c10::optional<at::Tensor>& k_valid,
                      const c10::optional<at::Tensor>& block_mask, double sm_scale,
                      const c10::optional<at::Tensor>& lse, const at::Tensor& out,
                      const at::Tensor& indices, const at::Tensor& counts, c10::IntArrayRef dims,
                      c10::IntArrayRef strides, int64_t n_split,
                      const c10::optional<at::Tensor>& workspace,
                      const c10::optional<at::Tensor>& out_token, int64_t out_len,
                      const c10::optional<at::Tensor>& kv_token, int64_t kv_len) {
  const char* op = "sparse_attn_int8";
  const Api& a = api(op);
  const AttnDims d = attn_dims(op, dims, strides, indices, counts);
  int dev = -1;
  for (const auto* t : {&q_i8, &q_scale, &k_i8, &k_scale, &v, &out, &indices, &counts})
    on_device(op, dev, *t, "a tensor argument");
  on_device(op, dev, k_valid, "k_valid");
  on_device(op, dev, block_mask, "block_mask");
  on_device(op, dev, lse, "lse");
  on_device(op, dev, workspace, "workspace");
  on_device(op, dev, out_token, "out_token");
  on_device(op, dev, kv_token, "kv_token");
  want(op, q_i8, at::kChar, "q_i8");
  want(op, k_i8, at::kChar, "k_i8");
  want(op, q_scale, at::kFloat, "q_scale");
  want(op, k_scale, at::kFloat, "k_scale");
  want(op, v, at::kBFloat16, "v");
  want(op, out, at::kBFloat16, "out");
  const auto& s = strides;
  const int64_t kv_rows = kv_token.has_value() ? kv_len : d.Lk;
  const int64_t o_rows = out_token.has_value() ? out_len : d.Lq;
  want_numel(op, q_i8, reach(op, d.B, d.H, d.Lq, d.D, s[0], s[1], s[2]), "q_i8");
  want_numel(op, k_i8, reach(op, d.B, d.H, d.Lk, d.D, s[3], s[4], s[5]), "k_i8");
  want_numel(op, v, reach(op, d.B, d.H, kv_rows, d.D, s[6], s[7], s[8]), "v");
  want_numel(op, out, reach(op, d.B, d.H, o_rows, d.D, s[9], s[10], s[11]), "out");
  TORCH_CHECK(q_scale_stride >= 0 && k_scale_stride >= 0, op, ": strides must not be negative");
  if (d.B > 0 && d.H > 0) {
    want_numel(op, q_scale, (d.B * d.H - 1) * q_scale_stride + cdiv(d.Lq, d.BM), "q_scale");
    want_numel(op, k_scale, (d.B * d.H - 1) * k_scale_stride + cdiv(d.Lk, d.BN), "k_scale");
  }
  attn_common(op, d, k_valid, block_mask, lse, o_rows, c10::nullopt, kv_token, out_token);
  const int64_t ws_bytes = workspace.has_value() ? workspace->numel() * workspace->element_size() : 0;
  const Launch l(device_of(op, dev));
  check_status(a, op, a.sparse_attn_int8_split(
      ptr<const int8_t>(q_i8), ptr<const float>(q_scale), q_scale_stride, ptr<const int8_t>(k_i8),
      ptr<const float>(k_scale), k_scale_stride, v.data_ptr(), ptr<const uint8_t>(k_valid),
      ptr<const uint32_t>(block_mask), static_cast<float>(sm_scale), ptr<float>(lse),
      out.data_ptr(), ptr<const int32_t>(indices), ptr<const int32_t>(counts), s[0], s[1], s[2],
      s[3], s[4], s[5], s[6], s[7], s[8], s[9], s[10], s[11], s[12], s[13], s[14], s[15], s[16],
      s[17], d.B, d.H, d.Lq, d.Lk, d.D, d.BM, d.BN, d.max_k, n_split, ptr<void>(workspace),
      ws_bytes, ptr<const int32_t>(out_token), out_len, ptr<const int32_t>(kv_token), kv_len,
      l.stream));
}

// x [M, C] with unit column stride (bf16 or fp32, dtype code as for the pools)
void quantize_rows_int8(const at::Tensor& x, int64_t dtype, const at::Tensor& q,
                        const at::Tensor& scale) {
  const char* op = "quantize_rows_int8";
  const Api& a = api(op);
  int dev = -1;
  for (const auto* t : {&x, &q, &scale}) on_device(op, dev, *t, "a tensor argument");
  TORCH_CHECK(x.dim() == 2 && x.stride(1) == 1, op, ": x must be [M, C] with unit column stride");
  const int64_t M = x.size(0), C = x.size(1);
  want(op, q, at::kChar, "q");
  want(op, scale, at::kFloat, "scale");
  want_numel(op, q, M * C, "q");
  want_numel(op, scale, M, "scale");
  want_code(op, x, dtype, "x");
  const Launch l(device_of(op, dev));
  check_status(a, op, a.quantize_rows_int8(x.data_ptr(), static_cast<int>(dtype), M, C,
                                           x.stride(0), ptr<int8_t>(q), ptr<float>(scale),
                                           l.stream));
}

// x_i8 [M, K], w_i8 [N, K] contiguous int8; out bf16 [M, N] with unit column stride
void int8_linear(const at::Tensor& x_i8, const at::Tensor& x_scale, const at::Tensor& w_i8,
                 const at::Tensor& w_scale, const c10::optional<at::Tensor>& bias,
                 const at::Tensor& out) {
  const char* op = "int8_linear";
  const Api& a = api(op);
  int dev = -1;
  for (const auto* t : {&x_i8, &x_scale, &w_i8, &w_scale, &out})
    on_device(op, dev, *t, "a tensor argument");
  on_device(op, dev, bias, "bias");
  TORCH_CHECK(x_i8.dim() == 2 && w_i8.dim() == 2 && x_i8.is_contiguous() && w_i8.is_contiguous(),
              op, ": x and w must be contiguous 2-D int8 matrices");
  want(op, x_i8, at::kChar, "x");
  want(op, w_i8, at::kChar, "w");
  want(op, x_scale, at::kFloat, "x_scale");
  want(op, w_scale, at::kFloat, "w_scale");
  want(op, out, at::kBFloat16, "out");
  const int64_t M = x_i8.size(0), K = x_i8.size(1), N = w_i8.size(0);
  TORCH_CHECK(w_i8.size(1) == K, op, ": x and w disagree on K");
  want_numel(op, x_scale, M, "x_scale");
  want_numel(op, w_scale, N, "w_scale");
  if (bias.has_value()) {
    want(op, *bias, at::kBFloat16, "bias");
    want_numel(op, *bias, N, "bias");
  }
  TORCH_CHECK(out.dim() == 2 && out.size(0) == M && out.size(1) == N && out.stride(1) == 1, op,
              ": out must be [M, N] with unit column stride");
  const Launch l(device_of(op, dev));
  check_status(a, op, a.int8_linear(ptr<const int8_t>(x_i8), ptr<const float>(x_scale),
                                    ptr<const int8_t>(w_i8), ptr<const float>(w_scale),
                                    ptr<const void>(bias), M, N, K, out.data_ptr(), out.stride(0),
                                    l.stream));
}

}  // namespace

TORCH_LIBRARY(rcsa, m) {
  m.def("bind_library(str path) -> ()", &bind_library);
  m.def(
      "pool_query_key(Tensor q, Tensor k, int dtype, int[] dims, int[] q_strides, int[] k_strides, "
      "Tensor? q_valid, Tensor? k_valid, Tensor? q_slot_token, int q_src_len, "
      "Tensor? k_slot_token, int k_src_len, Tensor(a!) qhat, Tensor(b!)? q_i8, "
      "Tensor(c!)? q_scale, Tensor(d!) khat, Tensor(e!)? ksum, Tensor(f!)? kmin, "
      "Tensor(g!)? kmax, Tensor(h!) block_mask) -> ()",
      &pool_query_key);
  m.def(
      "quantize_key_select(Tensor k, int dtype, int[] dims, int[] strides, Tensor? valid, "
      "Tensor? slot_token, int src_len, Tensor ksum, Tensor kmin, Tensor kmax, Tensor(a!) kmean, "
      "Tensor(b!) k_i8, Tensor(c!) k_scale, Tensor qhat, Tensor khat, int n_qblocks, "
      "Tensor(d!) score, Tensor? row_k, int row_k_stride_bh, int k_fixed, Tensor? forced, "
      "Tensor? allowed, int mask_stride_bh, Tensor(e!) indices, int max_k, "
      "Tensor(f!) counts) -> ()",
      &quantize_key_select);
  m.def(
      "sparse_attn_bf16(Tensor q, Tensor k, Tensor v, Tensor? k_valid, Tensor? block_mask, "
      "float sm_scale, Tensor(a!)? lse, Tensor(b!) out, Tensor indices, Tensor counts, "
      "int[] dims, int[] strides, int n_split, Tensor(c!)? workspace, Tensor? q_token, "
      "int q_tokens, Tensor? kv_token, int kv_len, Tensor? out_token, int out_len) -> ()",
      &sparse_attn_bf16);
  m.def(
      "sparse_attn_int8(Tensor q_i8, Tensor q_scale, int q_scale_stride, Tensor k_i8, "
      "Tensor k_scale, int k_scale_stride, Tensor v, Tensor? k_valid, Tensor? block_mask, "
      "float sm_scale, Tensor(a!)? lse, Tensor(b!) out, Tensor indices, Tensor counts, "
      "int[] dims, int[] strides, int n_split, Tensor(c!)? workspace, Tensor? out_token, "
      "int out_len, Tensor? kv_token, int kv_len) -> ()",
      &sparse_attn_int8);
  m.def("quantize_rows_int8(Tensor x, int dtype, Tensor(a!) q, Tensor(b!) scale) -> ()",
        &quantize_rows_int8);
  m.def(
      "int8_linear(Tensor x_i8, Tensor x_scale, Tensor w_i8, Tensor w_scale, Tensor? bias, "
      "Tensor(a!) out) -> ()",
      &int8_linear);
}
