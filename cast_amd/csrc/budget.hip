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

// Sort key of a fractional part in [0, 1) (or NaN) and its index: ascending
// keys order fractions descending (non-negative floats order as their bits),
// equal fractions by index ascending.
__device__ __forceinline__ uint64_t frac_key(float f, int i) {
  return (static_cast<uint64_t>(0xffffffffu - __float_as_uint(f)) << 32) |
         static_cast<uint32_t>(i);
}

// Ascending bitonic sort of np (a power of two) 64-bit keys in LDS by the
// workgroup; every compare-exchange stage ends at a barrier.
__device__ void bitonic_sort_lds(uint64_t* key, int np) {
  for (int k = 2; k <= np; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < np / 2; i += kBudgetThreads) {
        // the pair (lo, lo + j): lo has bit j clear
        const int lo = ((i & ~(j - 1)) << 1) | (i & (j - 1));
        const int hi = lo | j;
        const bool up = (lo & k) == 0;
        const uint64_t a = key[lo], b = key[hi];
        if ((a > b) == up) {
          key[lo] = b;
          key[hi] = a;
        }
      }
      __syncthreads();
    }
  }
}

__global__ void __launch_bounds__(kBudgetThreads)
apportion_kernel(const float* weights, int64_t ldw, int n, int total, int cap, int target,
                 int32_t* degrees, int64_t ldd) {
  __shared__ uint64_t s_key[kBudgetMaxN];  // (fractional part descending, index) sort keys
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
    s_key[i] = frac_key(raw - f, i);
    fl_part += static_cast<int>(f);
  }
  int fl_sum = 0;
  block_exclusive_scan(fl_part, s_i, &fl_sum);  // also publishes s_key / s_deg
  const int rem = total - fl_sum;

  // one extra edge to the `rem` largest fractional parts, ties to the lower
  // index: a bitonic sort of the keys in LDS, then the first `rem` positions
  if (rem > 0) {
    int np = 1;
    while (np < n) np <<= 1;
    for (int i = n + t; i < np; i += kBudgetThreads) s_key[i] = ~0ull;  // padding sorts last
    __syncthreads();
    bitonic_sort_lds(s_key, np);
    for (int p = t; p < rem && p < n; p += kBudgetThreads)
      s_deg[static_cast<uint32_t>(s_key[p])] += 1;
    __syncthreads();
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

// ---- the closed-loop allocator of a compact woven layer ----
constexpr int kClMaxCells = 64;    // compact current time cells
constexpr int kClMaxFrames = kClMaxCells * 16;
constexpr int kClMaxSpatial = 1024;

struct ClosedLoopArgs {
  const float* curvature;  // [t_src][spatial]
  const float* response;   // [t_src][spatial] or null
  const int32_t* frames;   // [n_frames] current-local frame ids
  int t_src, spatial, n_frames, offset, source_group, compact_group;
  int mean_degree, base_degree, total_blocks, memory_blocks;
  float response_weight;
  int feedback;            // 0 additive, 1 centered multiplicative, 2 centered inverse
  int use_response, fixed_budget;
  int32_t* degrees;        // [total_blocks]
  int32_t* status;         // [1]
};

// One workgroup.  Thread t owns spatial worldlines t, t + 256, ...: the
// column mean of the curvature, the compact time cells of its column, the
// weights 1 + log1p(signal), the largest-remainder split of its worldline's
// residual edges over the cells, base + bonus, and the saturation at the key
// count with redistribution; then the memory rows and the layer-wide
// saturation.  All arithmetic in fp32 in the order the reference writes it.
__global__ void __launch_bounds__(kBudgetThreads) closed_loop_kernel(ClosedLoopArgs a) {
  __shared__ int s_status;
  __shared__ int s_i[4];
  __shared__ int s_deg[kBudgetMaxN];     // the layer's degrees
  __shared__ float s_w[kBudgetMaxN];     // weights of cell c, worldline s at c * spatial + s
  __shared__ float s_fr[kBudgetMaxN];    // their fractional parts
  const int t = threadIdx.x;
  if (t == 0) s_status = 0;
  __syncthreads();
  const int cells = (a.n_frames + a.compact_group - 1) / a.compact_group;
  const float eps = 1.1920928955078125e-07f;  // torch.finfo(float32).eps
  const int n_blocks = a.total_blocks;
  const int S = a.spatial;
  for (int i = t; i < a.memory_blocks; i += kBudgetThreads) s_deg[i] = a.mean_degree;
  for (int sp = t; sp < S; sp += kBudgetThreads) {
    int* const deg = s_deg + a.memory_blocks + sp;  // cell c at deg[c * S]
    float* const w = s_w + sp;
    float* const fr = s_fr + sp;
    // column mean of the curvature (sum over tiles in order, then / t_src)
    float csum = 0.0f;
    for (int r = 0; r < a.t_src; ++r) csum += a.curvature[r * S + sp];
    float cmean = csum / static_cast<float>(a.t_src);
    cmean = cmean < eps ? eps : cmean;
    for (int c = 0; c < cells; ++c) {
      // mean over the cell's frames of the profiled tiles' values (0 for frames
      // before the first profiled tile)
      const int f0 = c * a.compact_group;
      const int f1 = f0 + a.compact_group < a.n_frames ? f0 + a.compact_group : a.n_frames;
      float cs = 0.0f, rs = 0.0f;
      for (int f = f0; f < f1; ++f) {
        const int local = a.frames[f];
        if (local < 0) atomicOr(&s_status, RCSA_CL_MEMORY_FRAME);
        if (local < a.offset) continue;
        const int src = (local - a.offset) / a.source_group;
        if (src >= a.t_src) {
          atomicOr(&s_status, RCSA_CL_OUTSIDE_TILES);
          continue;
        }
        cs += a.curvature[src * S + sp] / cmean;
        if (a.use_response) rs += a.response[src * S + sp];
      }
      const float cnt = static_cast<float>(f1 - f0);
      const float curv = cs / cnt;
      float signal = curv;
      if (a.use_response) {
        const float resp = rs / cnt;
        if (a.feedback == 0) {
          signal = curv + a.response_weight * resp;
        } else {
          const float sign = a.feedback == 2 ? -1.0f : 1.0f;
          signal = curv * expf(sign * a.response_weight * (resp - 1.0f));
        }
      }
      w[c * S] = 1.0f + log1pf(signal);
    }
    if (a.fixed_budget) {
      for (int c = 0; c < cells; ++c) deg[c * S] = a.mean_degree;
      continue;
    }
    // largest remainder of the residual over the cells of this worldline
    const int residual = cells * (a.mean_degree - a.base_degree);
    float sum = 0.0f;
    for (int c = 0; c < cells; ++c) sum += w[c * S] < 0.0f ? 0.0f : w[c * S];
    const bool uniform = !(sum > 0.0f);
    if (uniform) sum = static_cast<float>(cells);
    int fl = 0;
    for (int c = 0; c < cells; ++c) {
      const float wc = uniform ? 1.0f : (w[c * S] < 0.0f ? 0.0f : w[c * S]);
      const float raw = static_cast<float>(residual) * wc / sum;
      const float f = floorf(raw);
      deg[c * S] = static_cast<int>(f);
      fr[c * S] = raw - f;
      fl += static_cast<int>(f);
    }
    const int rem = residual - fl;
    for (int c = 0; c < cells; ++c) {
      int rank = 0;
      for (int e = 0; e < cells; ++e)
        rank += (fr[e * S] > fr[c * S]) || (fr[e * S] == fr[c * S] && e < c);
      deg[c * S] += (rank < rem ? 1 : 0) + a.base_degree;
    }
    // saturate at the key count; the lost edges go to the lowest cells with room
    const int target = cells * a.mean_degree;
    int have = 0;
    for (int c = 0; c < cells; ++c) {
      deg[c * S] = deg[c * S] < n_blocks ? deg[c * S] : n_blocks;
      have += deg[c * S];
    }
    int missing = target - have;
    while (missing > 0) {
      int room = 0;
      for (int c = 0; c < cells; ++c) room += deg[c * S] < n_blocks;
      if (room == 0) {
        atomicOr(&s_status, RCSA_CL_EXHAUSTED);
        break;
      }
      for (int c = 0; c < cells && missing > 0; ++c)
        if (deg[c * S] < n_blocks) {
          ++deg[c * S];
          --missing;
        }
    }
  }
  __syncthreads();
  // the layer: clamp to the key count, then one edge each to the lowest rows
  // with room, pass after pass, up to n_blocks * mean_degree
  const int chunk = (n_blocks + kBudgetThreads - 1) / kBudgetThreads;
  const int lo = t * chunk < n_blocks ? t * chunk : n_blocks;
  const int hi = lo + chunk < n_blocks ? lo + chunk : n_blocks;
  int have_part = 0;
  for (int i = lo; i < hi; ++i) {
    s_deg[i] = s_deg[i] < n_blocks ? s_deg[i] : n_blocks;
    have_part += s_deg[i];
  }
  int have = 0;
  block_exclusive_scan(have_part, s_i, &have);
  int missing = n_blocks * a.mean_degree - have;
  while (missing > 0) {
    int room = 0;
    for (int i = lo; i < hi; ++i) room += s_deg[i] < n_blocks;
    int n_room = 0;
    int before = block_exclusive_scan(room, s_i, &n_room);
    if (n_room == 0) break;
    for (int i = lo; i < hi; ++i)
      if (s_deg[i] < n_blocks) {
        s_deg[i] += before < missing;
        ++before;
      }
    missing -= n_room < missing ? n_room : missing;
  }
  for (int i = lo; i < hi; ++i) a.degrees[i] = s_deg[i];
  __syncthreads();
  if (t == 0) a.status[0] = s_status;
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

extern "C" int rcsa_closed_loop_degrees(
    const float* curvature, const float* response, int64_t t_src, int64_t spatial,
    const int32_t* frames, int64_t n_frames, int64_t current_temporal_offset,
    int64_t source_group, int64_t compact_group, int64_t mean_degree, int64_t base_degree,
    int64_t total_blocks, int64_t memory_blocks, float response_weight, int feedback_form,
    int fixed_query_budget, int32_t* degrees, int32_t* status, hipStream_t stream) {
  if (!curvature || !frames || !degrees || !status) return RCSA_ERR_NULL;
  if (t_src <= 0 || spatial <= 0 || spatial > kClMaxSpatial || n_frames <= 0 ||
      n_frames > kClMaxFrames || source_group <= 0 || compact_group <= 0 ||
      current_temporal_offset < 0 || mean_degree < 0 || base_degree < 0 ||
      base_degree > mean_degree || total_blocks <= 0 || total_blocks > kBudgetMaxN ||
      memory_blocks < 0 || memory_blocks > total_blocks ||
      t_src * spatial >= (int64_t{1} << 30) || feedback_form < 0 || feedback_form > 2)
    return RCSA_ERR_SHAPE;
  const int64_t cells = (n_frames + compact_group - 1) / compact_group;
  if (cells > kClMaxCells || memory_blocks + cells * spatial != total_blocks)
    return RCSA_ERR_SHAPE;
  if (!(response_weight >= 0.0f) || !(response_weight < INFINITY)) return RCSA_ERR_SHAPE;
  ClosedLoopArgs a{};
  a.curvature = curvature;
  a.response = response;
  a.frames = frames;
  a.t_src = static_cast<int>(t_src);
  a.spatial = static_cast<int>(spatial);
  a.n_frames = static_cast<int>(n_frames);
  a.offset = static_cast<int>(current_temporal_offset);
  a.source_group = static_cast<int>(source_group);
  a.compact_group = static_cast<int>(compact_group);
  a.mean_degree = static_cast<int>(mean_degree);
  a.base_degree = static_cast<int>(base_degree);
  a.total_blocks = static_cast<int>(total_blocks);
  a.memory_blocks = static_cast<int>(memory_blocks);
  a.response_weight = response_weight;
  a.feedback = feedback_form;
  a.use_response = response != nullptr && response_weight != 0.0f;
  a.fixed_budget = fixed_query_budget != 0;
  a.degrees = degrees;
  a.status = status;
  closed_loop_kernel<<<dim3(1), dim3(kBudgetThreads), 0, stream>>>(a);
  return launch_status();
}
