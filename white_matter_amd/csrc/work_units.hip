// Work list of a dense attention problem with per-row bounds (cached
// prefixes of different lengths): the (batch row, query tile) units ordered
// by the number of 64-key tiles their loops visit, largest first, so the
// longest workgroups start first. One workgroup counts the units per load
// (a histogram over load values in LDS), turns the counts into descending
// bin starts with a block scan, and scatters every unit to its bin; the
// order of units with equal loads is unspecified (each unit's result does
// not depend on it). This replaces a sort issued as a sequence of torch
// operations before every ragged prefill launch.
#include "wmx_kernels.h"

namespace wmx {

namespace {

constexpr int kUnitThreads = 1024;
constexpr int kUnitBins = 4096;  // loads beyond kUnitBins - 1 key tiles share the last bin
constexpr int kBinsPerThread = kUnitBins / kUnitThreads;

__device__ __forceinline__ int unit_load(const wmx_attn_args& a, int u, int tiles, int tile) {
  const int b = u / tiles, t = u - b * tiles;
  const int64_t last = min((int64_t)t * tile + tile - 1, (int64_t)a.q_len - 1);
  int64_t bound = (a.row_offset ? (int64_t)a.row_offset[b] : a.query_offset) + (int64_t)a.query_stride * last;
  if (a.row_limit && bound > a.row_limit[b]) bound = a.row_limit[b];
  if (bound > (int64_t)a.kv_len - 1) bound = (int64_t)a.kv_len - 1;
  if (bound < -1) bound = -1;
  const int64_t steps = (bound + 64) / 64;  // 64-key tiles that hold keys 0 .. bound
  return (int)(steps < kUnitBins - 1 ? steps : kUnitBins - 1);
}

__global__ __launch_bounds__(kUnitThreads) void dense_units_kernel(const wmx_attn_args a, int32_t* units, int tile) {
  __shared__ int hist[kUnitBins], cursor[kUnitBins];
  __shared__ int wave_sum[kUnitThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int tiles = (a.q_len + tile - 1) / tile;
  const int n = a.batch * tiles;
  for (int i = tid; i < kUnitBins; i += kUnitThreads) hist[i] = 0;
  __syncthreads();
  for (int u = tid; u < n; u += kUnitThreads) atomicAdd(&hist[unit_load(a, u, tiles, tile)], 1);
  __syncthreads();
  // thread k owns the bins kUnitBins - 1 - kBinsPerThread k - [0, kBinsPerThread):
  // heavier bins belong to lower threads, so an exclusive scan in thread
  // order gives each bin the count of all heavier units
  int local = 0;
#pragma unroll
  for (int i = 0; i < kBinsPerThread; ++i) local += hist[kUnitBins - 1 - kBinsPerThread * tid - i];
  int incl = local;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o);
    if (lane >= o) incl += y;
  }
  if (lane == 63) wave_sum[w] = incl;
  __syncthreads();
  int before = 0;
  for (int i = 0; i < w; ++i) before += wave_sum[i];
  int start = before + incl - local;
#pragma unroll
  for (int i = 0; i < kBinsPerThread; ++i) {
    const int bin = kUnitBins - 1 - kBinsPerThread * tid - i;
    cursor[bin] = start;
    start += hist[bin];
  }
  __syncthreads();
  for (int u = tid; u < n; u += kUnitThreads) {
    const int pos = atomicAdd(&cursor[unit_load(a, u, tiles, tile)], 1);
    const int b = u / tiles;
    units[2 * pos] = b;
    units[2 * pos + 1] = u - b * tiles;
  }
}

}  // namespace

int launch_dense_units(const wmx_attn_args& a, int32_t* units, hipStream_t stream) {
  const int tile = a.query_tile == 256 ? 256 : 128;
  if (a.batch == 0 || a.q_len == 0) return WMX_OK;
  hipLaunchKernelGGL(dense_units_kernel, dim3(1), dim3(kUnitThreads), 0, stream, a, units, tile);
  return WMX_OK;
}

}  // namespace wmx
