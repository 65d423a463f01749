// Compact-token <-> packed-block layout copies (HBM-bound gathers).
//
// One thread moves 8 channels so that consecutive threads write consecutive
// chunks of a packed row.
#include "rcsa_common.h"

namespace rcsa {

template <typename T>
__device__ __forceinline__ void store8(T* dst, const float (&f)[8], bool live);

template <>
__device__ __forceinline__ void store8<u16>(u16* dst, const float (&f)[8], bool live) {
  uint4 w = make_uint4(0, 0, 0, 0);
  if (live) {
    w.x = pack_bf16x2(f[0], f[1]);
    w.y = pack_bf16x2(f[2], f[3]);
    w.z = pack_bf16x2(f[4], f[5]);
    w.w = pack_bf16x2(f[6], f[7]);
  }
  *reinterpret_cast<uint4*>(dst) = w;
}

template <>
__device__ __forceinline__ void store8<float>(float* dst, const float (&f)[8], bool live) {
  const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
  reinterpret_cast<float4*>(dst)[0] = live ? make_float4(f[0], f[1], f[2], f[3]) : z;
  reinterpret_cast<float4*>(dst)[1] = live ? make_float4(f[4], f[5], f[6], f[7]) : z;
}

// The packed copy keeps the source element type (a gather, no rounding).
template <typename T>
__global__ void __launch_bounds__(256)
pack_kernel(const T* x, int64_t H, int64_t D, int64_t sb, int64_t sl, int64_t sh,
            const int64_t* slot_token, int64_t n_slots, int64_t L, T* out,
            int64_t total_vec) {
  const int64_t v = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (v >= total_vec) return;
  const int64_t cpr = D / 8;
  const int64_t c = v % cpr;
  const int64_t slot = (v / cpr) % n_slots;
  const int64_t bh = v / (cpr * n_slots);
  const int64_t b = bh / H, h = bh % H;
  const int64_t tok = slot_token[slot];
  const bool live = tok >= 0 && tok < L;
  float f[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (live) Vec8<T>::load(x + b * sb + tok * sl + h * sh + c * 8, f);
  store8<T>(out + (bh * n_slots + slot) * D + c * 8, f, live);
}

__global__ void __launch_bounds__(256)
unpack_kernel(const u16* packed, int64_t H, int64_t n_slots, int64_t D,
              const int64_t* token_slot, int64_t L, u16* out, int64_t total_vec) {
  const int64_t v = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (v >= total_vec) return;
  const int64_t cpr = D / 8;
  const int64_t c = v % cpr;
  const int64_t h = (v / cpr) % H;
  const int64_t tok = (v / (cpr * H)) % L;
  const int64_t b = v / (cpr * H * L);
  const int64_t slot = token_slot[tok];
  uint4 w = make_uint4(0, 0, 0, 0);
  if (slot >= 0 && slot < n_slots)
    w = *reinterpret_cast<const uint4*>(packed + ((b * H + h) * n_slots + slot) * D + c * 8);
  *reinterpret_cast<uint4*>(out + ((b * L + tok) * H + h) * D + c * 8) = w;
}

}  // namespace rcsa

using namespace rcsa;

extern "C" int rcsa_pack_tokens(const void* x, int dtype, int64_t B, int64_t L, int64_t H,
                                int64_t D, int64_t stride_b, int64_t stride_l,
                                int64_t stride_h, const int64_t* slot_token,
                                int64_t n_slots, void* out, hipStream_t stream) {
  if (!x || !slot_token || !out) return RCSA_ERR_NULL;
  if (dtype != RCSA_BF16 && dtype != RCSA_F32) return RCSA_ERR_DTYPE;
  if (B <= 0 || L <= 0 || H <= 0 || n_slots <= 0 || D <= 0 || D % 8) return RCSA_ERR_SHAPE;
  const int64_t vec = dtype == RCSA_BF16 ? 8 : 4;
  if (stride_b % vec || stride_l % vec || stride_h % vec) return RCSA_ERR_STRIDE;
  if (!aligned16(x) || !aligned16(out)) return RCSA_ERR_ALIGN;
  const int64_t total = B * H * n_slots * (D / 8);
  const dim3 grid(static_cast<unsigned>((total + 255) / 256));
  if (dtype == RCSA_BF16)
    pack_kernel<u16><<<grid, dim3(256), 0, stream>>>(static_cast<const u16*>(x), H, D, stride_b,
                                                    stride_l, stride_h, slot_token, n_slots, L,
                                                    static_cast<u16*>(out), total);
  else
    pack_kernel<float><<<grid, dim3(256), 0, stream>>>(static_cast<const float*>(x), H, D,
                                                      stride_b, stride_l, stride_h, slot_token,
                                                      n_slots, L, static_cast<float*>(out),
                                                      total);
  return launch_status();
}

extern "C" int rcsa_unpack_tokens(const void* packed, int64_t B, int64_t H, int64_t n_slots,
                                  int64_t D, const int64_t* token_slot, int64_t L, void* out,
                                  hipStream_t stream) {
  if (!packed || !token_slot || !out) return RCSA_ERR_NULL;
  if (B <= 0 || L <= 0 || H <= 0 || n_slots <= 0 || D <= 0 || D % 8) return RCSA_ERR_SHAPE;
  if (!aligned16(packed) || !aligned16(out)) return RCSA_ERR_ALIGN;
  const int64_t total = B * L * H * (D / 8);
  const dim3 grid(static_cast<unsigned>((total + 255) / 256));
  unpack_kernel<<<grid, dim3(256), 0, stream>>>(static_cast<const u16*>(packed), H, n_slots, D,
                                                token_slot, L, static_cast<u16*>(out), total);
  return launch_status();
}

extern "C" const char* rcsa_status_string(int status) {
  switch (status) {
    case RCSA_OK: return "ok";
    case RCSA_ERR_NULL: return "a required pointer is null";
    case RCSA_ERR_SHAPE: return "unsupported or inconsistent sizes";
    case RCSA_ERR_STRIDE: return "unsupported stride (last dim must be contiguous, rows 16-byte aligned)";
    case RCSA_ERR_DTYPE: return "unsupported dtype code";
    case RCSA_ERR_LAUNCH: return "HIP launch failed";
    case RCSA_ERR_ALIGN: return "pointer not 16-byte aligned";
    case RCSA_ERR_SCRATCH: return "split workspace exceeds the library's static scratch";
    default: return "unknown status";
  }
}

extern "C" int rcsa_abi_version(void) { return 3 << 16; }
