// Per-row key-block budgets on the device (gfx950): largest-remainder
// apportionment of a section's edge budget by non-negative weights, then the
// saturation pass that clamps rows to the key-block count and hands the lost
// edges to the lowest-index rows with capacity.
//
// Restates P/qk_uncertainty_tangent_attention.py:847-865 (apportion),
// :1239-1264 (_apportion_section_matrix) and the saturation of
// P/matrix_curvature_phase_frame_weave.py:5807-5817, in fp32 as the reference
// computes it, so the host never reads a budget back (.item() syncs).
//
// One workgroup per section row; thread t owns the contiguous rows
// [t*chunk, (t+1)*chunk), so index order is thread order and every pass is a
// block-wide exclusive scan.
#include "rcsa_common.h"

namespace rcsa {

constexpr int kBudgetThreads = 256;
constexpr int kBudgetMaxN = 8192;

// Exclusive prefix of v over the workgroup (thread order), and the total.
__device__ __forceinline__ int block_exclusive_scan(int v, int* s_tmp, int* total) {
  const int t = threadIdx.x, lane = t % kWave, wave = t / kWave;
  int incl = v;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int u = __shfl_up(incl, o, kWave);
    if (lane >= o) incl += u;
  }
  __syncthreads();
  if (lane == kWave - 1) s_tmp[wave] = incl;
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kBudgetThreads / kWave; ++w) {
    if (w < wave) before += s_tmp[w];
    all += s_tmp[w];
  }
  *total = all;
  return before + incl - v;
}

// Sum of fp32 values in a fixed order: thread partials (their rows in
// index order), then a pairwise tree over lanes, then the four wavefronts.
__device__ __forceinline__ float block_sum_fixed(float v, float* s_tmp) {
  const int t = threadIdx.x, lane = t % kWave, wave = t / kWave;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const float u = __shfl_xor(v, o, kWave);
    v = (lane & o) ? u + v : v + u;  // the lower lane's partial first
  }
  __syncthreads();
  if (lane == 0) s_tmp[wave] = v;
  __syncthreads();
  return (s_tmp[0] + s_tmp[1]) + (s_tmp[2] + s_tmp[3]);
}

__global__ void __launch_bounds__(kBudgetThreads)
apportion_kernel(const float* weights, int64_t ldw, int n, int total, int cap, int target,
                 int32_t* degrees, int64_t ldd) {
  __shared__ __attribute__((aligned(16))) float s_frac[kBudgetMaxN];
  __shared__ int s_deg[kBudgetMaxN];
  __shared__ float s_f[4];
  __shared__ int s_i[4];
  const int t = threadIdx.x;
  const float* w = weights + static_cast<int64_t>(blockIdx.x) * ldw;
  int32_t* out = degrees + static_cast<int64_t>(blockIdx.x) * ldd;
  const int chunk = (n + kBudgetThreads - 1) / kBudgetThreads;
  const int lo = t * chunk < n ? t * chunk : n;
  const int hi = lo + chunk < n ? lo + chunk : n;

  // w = clamp_min(w, 0) (NaN stays NaN, as torch's clamp_min); a row whose
  // sum is not positive (or NaN) weighs every entry 1
  auto clamp0 = [](float x) { return x < 0.0f ? 0.0f : x; };
  float part = 0.0f;
  for (int i = lo; i < hi; ++i) part += clamp0(w[i]);
  float sum = block_sum_fixed(part, s_f);
  const bool uniform = !(sum > 0.0f);
  if (uniform) sum = static_cast<float>(n);
  const float tot_f = static_cast<float>(total);

  // raw = total * w / sum; floor; fractional part
  int fl_part = 0;
  for (int i = lo; i < hi; ++i) {
    const float wi = uniform ? 1.0f : clamp0(w[i]);
    const float raw = tot_f * wi / sum;
    const float f = floorf(raw);
    s_deg[i] = static_cast<int>(f);
    s_frac[i] = raw - f;
    fl_part += static_cast<int>(f);
  }
  int fl_sum = 0;
  block_exclusive_scan(fl_part, s_i, &fl_sum);  // also publishes s_frac / s_deg
  const int rem = total - fl_sum;

  // one extra edge to the `rem` largest fractional parts, ties to the lower index
  // (rank = entries ahead of i in that order; a straight count over 16-byte
  // LDS reads, unrolled so the reads stay in flight)
  if (rem > 0) {
    const int n4 = n & ~3;
    for (int i = lo; i < hi; ++i) {
      const float fi = s_frac[i];
      int rank = 0;
#pragma unroll 4
      for (int j = 0; j < n4; j += 4) {
        const float4 f = *reinterpret_cast<const float4*>(&s_frac[j]);
        rank += (f.x > fi) || (f.x == fi && j < i);
        rank += (f.y > fi) || (f.y == fi && j + 1 < i);
        rank += (f.z > fi) || (f.z == fi && j + 2 < i);
        rank += (f.w > fi) || (f.w == fi && j + 3 < i);
      }
      for (int j = n4; j < n; ++j) rank += (s_frac[j] > fi) || (s_frac[j] == fi && j < i);
      s_deg[i] += rank < rem;
    }
  }

  // saturation: clamp to cap, then one edge each to the lowest-index rows with
  // capacity, pass after pass, until the target or no capacity is left
  if (cap > 0) {
    int have_part = 0;
    for (int i = lo; i < hi; ++i) {
      const int d = s_deg[i] < cap ? s_deg[i] : cap;
      s_deg[i] = d;
      have_part += d;
    }
    int have = 0;
    block_exclusive_scan(have_part, s_i, &have);
    int missing = target - have;
    while (missing > 0) {  // workgroup-uniform: missing and n_room come from scans
      int room = 0;
      for (int i = lo; i < hi; ++i) room += s_deg[i] < cap;
      int n_room = 0;
      int before = block_exclusive_scan(room, s_i, &n_room);
      if (n_room == 0) break;
      for (int i = lo; i < hi; ++i) {
        if (s_deg[i] < cap) {
          s_deg[i] += before < missing;
          ++before;
        }
      }
      missing -= n_room < missing ? n_room : missing;
    }
  }
  for (int i = lo; i < hi; ++i) out[i] = s_deg[i];
}

}  // namespace rcsa

using namespace rcsa;

extern "C" int rcsa_row_budgets(const float* weights, int64_t n_sections, int64_t n,
                                int64_t weights_stride, int64_t total_per_section,
                                int64_t cap, int64_t target_total, int32_t* degrees,
                                int64_t degrees_stride, hipStream_t stream) {
  if (!weights || !degrees) return RCSA_ERR_NULL;
  if (n_sections <= 0 || n <= 0 || n > kBudgetMaxN || total_per_section <= 0 ||
      total_per_section >= (int64_t{1} << 24) || n_sections >= (int64_t{1} << 31))
    return RCSA_ERR_SHAPE;
  if (cap < 0 || cap >= (int64_t{1} << 24) || target_total >= (int64_t{1} << 30))
    return RCSA_ERR_SHAPE;
  if (weights_stride < n || degrees_stride < n) return RCSA_ERR_STRIDE;
  const int target = target_total > 0 ? static_cast<int>(target_total)
                                      : static_cast<int>(total_per_section);
  apportion_kernel<<<dim3(static_cast<unsigned>(n_sections)), dim3(kBudgetThreads), 0,
                     stream>>>(weights, weights_stride, static_cast<int>(n),
                               static_cast<int>(total_per_section), static_cast<int>(cap),
                               target, degrees, degrees_stride);
  return launch_status();
}
