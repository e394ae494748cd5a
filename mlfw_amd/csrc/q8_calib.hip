// q8_calib.hip -- calibration observers on the device (gfx950).
//
// The reference calibrates a static activation scale by running the float
// graph on sample batches and feeding every value to a ValueObserver
// (min / max / count) with an optional 2048-bin HistogramCollector
// (src/compiler/analysis/calibration.ts:11-189).  Here the observer state
// lives in device memory and one batch is observed with four launches and
// no host round trip:
//   k_obs_begin    clears the batch min/max keys;
//   k_obs_minmax   NaN-ignoring batch min / max as order keys (atomic max of
//                  the int pattern, HBM-bound, 16-byte loads);
//   k_obs_control  one workgroup applies the reference's decisions in f64:
//                  observer min/max/count, first-batch range, the range
//                  expansion with re-bucketing of the old bins by their
//                  centres, and the range the batch is binned with;
//   k_obs_hist     bins the batch: per-workgroup histogram in LDS (32-bit
//                  counts, up to Q8_OBS_MAX_BINS bins = 32 KiB), flushed
//                  with 64-bit atomics.
// Counts are exact integers (the reference keeps them in a Float64Array).
// Scale selection from the read-back state (minmax / percentile 0.999 /
// KL entropy, calibration.ts:128-187, 246-268) runs on the host in
// q8_capi.hip.
#include "../../include/q8hip.h"
#include "q8_device.h"
#include "q8_internal.h"

namespace q8 {

static constexpr int NT = 256;
static constexpr int KEY_NONE_MIN = 0x7fffffff;       // no value seen (min side)
static constexpr int KEY_NONE_MAX = (int)0x80000000;  // no value seen (max side)

__global__ void k_obs_reset(ObsState* st, int num_bins, int has_hist) {
  unsigned long long* bins = obs_bins(st);
  for (int i = threadIdx.x; i < num_bins; i += blockDim.x) bins[i] = 0ull;
  if (threadIdx.x == 0) {
    st->min_key = KEY_NONE_MIN;
    st->max_key = KEY_NONE_MAX;
    st->bmin_key = KEY_NONE_MIN;
    st->bmax_key = KEY_NONE_MAX;
    st->has_hist = has_hist;
    st->num_bins = num_bins;
    st->initialized = 0;
    st->mode = 0;
    st->count = 0ull;
    st->total_count = 0ull;
    st->range_min = 0.0;
    st->range_max = 0.0;
    st->act_min = 0.0;
    st->act_scale = 0.0;
  }
}

__global__ void k_obs_begin(ObsState* st) {
  st->bmin_key = KEY_NONE_MIN;
  st->bmax_key = KEY_NONE_MAX;
}

__device__ __forceinline__ void minmax_key(float v, int& mn, int& mx) {
  if (v == v) {
    const int k = order_key(v);
    mn = mn < k ? mn : k;
    mx = mx > k ? mx : k;
  }
}

__global__ __launch_bounds__(NT) void k_obs_minmax(const float* __restrict__ x, int64_t n,
                                                   ObsState* st) {
  __shared__ int smn[NT / 64], smx[NT / 64];
  int mn = KEY_NONE_MIN, mx = KEY_NONE_MAX;
  const int64_t stride = (int64_t)gridDim.x * NT;
  const int64_t i0 = blockIdx.x * (int64_t)NT + threadIdx.x;
  if ((reinterpret_cast<uintptr_t>(x) & 15) == 0) {
    const int64_t n4 = n >> 2;
    const v4f* x4 = reinterpret_cast<const v4f*>(x);
    for (int64_t i = i0; i < n4; i += stride) {
      const v4f v = __builtin_nontemporal_load(x4 + i);
      minmax_key(v.x, mn, mx);
      minmax_key(v.y, mn, mx);
      minmax_key(v.z, mn, mx);
      minmax_key(v.w, mn, mx);
    }
    for (int64_t i = (n4 << 2) + i0; i < n; i += stride) minmax_key(x[i], mn, mx);
  } else {
    for (int64_t i = i0; i < n; i += stride) minmax_key(x[i], mn, mx);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const int a = __shfl_xor(mn, o, 64), b = __shfl_xor(mx, o, 64);
    mn = mn < a ? mn : a;
    mx = mx > b ? mx : b;
  }
  if ((threadIdx.x & 63) == 0) {
    smn[threadIdx.x >> 6] = mn;
    smx[threadIdx.x >> 6] = mx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    mn = smn[0];
    mx = smx[0];
    for (int w = 1; w < NT / 64; ++w) {
      mn = mn < smn[w] ? mn : smn[w];
      mx = mx > smx[w] ? mx : smx[w];
    }
    if (mn != KEY_NONE_MIN) atomicMin(&st->bmin_key, mn);
    if (mx != KEY_NONE_MAX) atomicMax(&st->bmax_key, mx);
  }
}

// Math.min(numBins - 1, Math.floor((v - lo) * scale)); -1 when the index is
// NaN (the reference's typed-array store at a NaN index is dropped).
__device__ __forceinline__ int obs_bin(double v, double lo, double scale, int num_bins) {
  const double f = floor((v - lo) * scale);
  if (f != f) return -1;
  return f < (double)(num_bins - 1) ? (int)f : num_bins - 1;
}

// One workgroup: the reference's per-batch decisions (calibration.ts:24-34,
// 58-126) on the reduced batch keys.
__global__ __launch_bounds__(NT) void k_obs_control(ObsState* st, int64_t n) {
  __shared__ int s_expand;
  __shared__ double s_old_min, s_old_w, s_new_min, s_new_scale;
  const int nb = st->num_bins;
  const bool any = st->bmin_key != KEY_NONE_MIN;               // a non-NaN value was seen
  const double bmin = any ? (double)from_order_key(st->bmin_key) : __builtin_inf();
  const double bmax = any ? (double)from_order_key(st->bmax_key) : -__builtin_inf();
  if (threadIdx.x == 0) {
    if (any) {
      st->min_key = st->min_key < st->bmin_key ? st->min_key : st->bmin_key;
      st->max_key = st->max_key > st->bmax_key ? st->max_key : st->bmax_key;
    }
    st->count += (unsigned long long)n;
    s_expand = 0;
    st->mode = 0;
    if (st->has_hist) {
      if (!st->initialized) {                                   // _initRange
        double mn = bmin, mx = bmax;
        if (mn == mx) mx = mn + 1.0;
        st->range_min = mn;
        st->range_max = mx;
        st->initialized = 1;
      }
      const double range = st->range_max - st->range_min;
      if (!(range <= 0.0)) {                                    // a NaN range continues
        if (any && (bmin < st->range_min || bmax > st->range_max)) {
          const double new_min = bmin < st->range_min ? bmin : st->range_min;
          const double new_max = bmax > st->range_max ? bmax : st->range_max;
          const double old_range = st->range_max - st->range_min;
          s_expand = old_range > 0.0 ? 2 : 1;                   // 2: re-bucket the old bins
          s_old_min = st->range_min;
          s_old_w = old_range / nb;
          s_new_min = new_min;
          s_new_scale = nb / (new_max - new_min);
          st->range_min = new_min;
          st->range_max = new_max;
          st->act_min = new_min;
          st->act_scale = s_new_scale;
        } else {
          st->act_min = st->range_min;
          st->act_scale = nb / range;
        }
        st->total_count += (unsigned long long)n;
        st->mode = 1;
      }
    }
  }
  __syncthreads();
  if (s_expand) {
    unsigned long long* bins = obs_bins(st);
    unsigned long long* old = obs_scratch(st);
    for (int i = threadIdx.x; i < nb; i += NT) {
      old[i] = bins[i];
      bins[i] = 0ull;
    }
    __syncthreads();
    if (s_expand == 2) {
      for (int i = threadIdx.x; i < nb; i += NT) {
        const unsigned long long c = old[i];
        if (c == 0ull) continue;
        const double center = s_old_min + (i + 0.5) * s_old_w;
        const int b = obs_bin(center, s_new_min, s_new_scale, nb);
        if (b >= 0) atomicAdd(&bins[b], c);
      }
    }
  }
}

__global__ __launch_bounds__(NT) void k_obs_hist(const float* __restrict__ x, int64_t n,
                                                 ObsState* st) {
  __shared__ unsigned int lhist[Q8_OBS_MAX_BINS];
  if (st->mode != 1) return;                                   // uniform per launch
  const int nb = st->num_bins;
  const double lo = st->act_min, scale = st->act_scale;
  for (int i = threadIdx.x; i < nb; i += NT) lhist[i] = 0u;
  __syncthreads();
  const int64_t stride = (int64_t)gridDim.x * NT;
  const int64_t i0 = blockIdx.x * (int64_t)NT + threadIdx.x;
  auto add = [&](float v) {
    const int b = obs_bin((double)v, lo, scale, nb);
    if (b >= 0) atomicAdd(&lhist[b], 1u);
  };
  if ((reinterpret_cast<uintptr_t>(x) & 15) == 0) {
    const int64_t n4 = n >> 2;
    const v4f* x4 = reinterpret_cast<const v4f*>(x);
    for (int64_t i = i0; i < n4; i += stride) {
      const v4f v = __builtin_nontemporal_load(x4 + i);
      add(v.x);
      add(v.y);
      add(v.z);
      add(v.w);
    }
    for (int64_t i = (n4 << 2) + i0; i < n; i += stride) add(x[i]);
  } else {
    for (int64_t i = i0; i < n; i += stride) add(x[i]);
  }
  __syncthreads();
  unsigned long long* bins = obs_bins(st);
  for (int i = threadIdx.x; i < nb; i += NT)
    if (lhist[i]) atomicAdd(&bins[i], (unsigned long long)lhist[i]);
}

static int grid_for(int64_t work, int64_t per_block, int cap) {
  int64_t g = (work + per_block - 1) / per_block;
  if (g < 1) g = 1;
  return (int)(g > cap ? cap : g);
}

hipError_t launch_obs_reset(ObsState* st, int num_bins, int has_hist, hipStream_t s) {
  hipLaunchKernelGGL(k_obs_reset, dim3(1), dim3(NT), 0, s, st, num_bins, has_hist);
  return hipGetLastError();
}

hipError_t launch_obs_update(ObsState* st, const float* x, int64_t n, hipStream_t s) {
  hipLaunchKernelGGL(k_obs_begin, dim3(1), dim3(1), 0, s, st);
  if (n > 0) {
    const int grid = grid_for((n + 3) / 4, NT * 4, 4096);
    hipLaunchKernelGGL(k_obs_minmax, dim3(grid), dim3(NT), 0, s, x, n, st);
  }
  hipLaunchKernelGGL(k_obs_control, dim3(1), dim3(NT), 0, s, st, n);
  if (n > 0) {
    const int grid = grid_for((n + 3) / 4, NT * 16, 2048);
    hipLaunchKernelGGL(k_obs_hist, dim3(grid), dim3(NT), 0, s, x, n, st);
  }
  return hipGetLastError();
}

}  // namespace q8
