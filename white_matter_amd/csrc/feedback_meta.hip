// Per-residue cyclic metadata of packed documents on the device: the
// reference's prepare_feedback_metadata (blocks/_execution/metadata.py:11-55)
// in one kernel, one workgroup per batch row, with no host synchronisation
// (every output size follows from the inputs' shapes).
//
// A run is a maximal sequence of equal document ids in a row (padding ids
// included: each padding run is its own run). Per token t the row's scans give
//   first[t]  the run's first token   (forward max-scan of run starts)
//   end[t]    the run's exclusive end (backward min-scan of run ends)
// kept in the workspace for the gathers that follow. Then, for every group r
// of G (query tokens r, r + G, ... in the model's cyclic schedule; any slots
// here), with d = use_dummy:
//   key_ids[b, j]            -1 for j < d, else id(token j - d), negative ids as -2
//   key_query_end[r, b, j]   count_r for j < d, else
//                            min(ceil(max(end[j - d] - r, 0) / G), count_r)
//   query_ids[r][b, i]       id(slots_r[i]), negative ids as -2
//   query_key_start[r][b, i] first[slots_r[i]] + d
// Slots outside [0, length) read as padding (-2, start 0) instead of faulting.
#include "wmx_kernels.h"

namespace wmx {

namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;

// Inclusive max-scan over the workgroup's threads in thread order; `total`
// receives the maximum over all of them. Every thread must call it.
__device__ int64_t block_max_scan(int64_t x, int64_t& total, int64_t* sh) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int64_t y = __shfl_up(x, o);
    if (lane >= o) x = x > y ? x : y;
  }
  if (lane == 63) sh[w] = x;
  __syncthreads();
  int64_t before = INT64_MIN, all = INT64_MIN;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    const int64_t v = sh[i];
    if (i < w) before = before > v ? before : v;
    all = all > v ? all : v;
  }
  __syncthreads();  // sh is free again
  total = all;
  return before > x ? before : x;
}

__device__ __forceinline__ int64_t doc_at(const wmx_feedback_meta_args& a, int b, int64_t t) {
  const int64_t off = (int64_t)b * a.doc_stride + t;
  return a.doc_dtype == WMX_DTYPE_I32 ? (int64_t)((const int32_t*)a.document_ids)[off]
                                      : ((const int64_t*)a.document_ids)[off];
}

// The id as the metadata stores it: int32, padding (any negative id) as -2.
__device__ __forceinline__ int32_t segment_id(int64_t id) { return id < 0 ? -2 : (int32_t)(uint32_t)(uint64_t)id; }

__global__ __launch_bounds__(kThreads) void feedback_meta_kernel(const wmx_feedback_meta_args a) {
  __shared__ int64_t sh[kWaves];
  const int b = blockIdx.x;
  const int64_t T = a.length;
  int32_t* first = (int32_t*)a.workspace + (int64_t)b * 2 * T;
  int32_t* end = first + T;

  // run starts: token t starts a run when t == 0 or its id differs from t - 1
  int64_t carry = 0;
  for (int64_t t0 = 0; t0 < T; t0 += kThreads) {
    const int64_t t = t0 + threadIdx.x;
    int64_t v = -1;
    if (t < T) v = (t == 0 || doc_at(a, b, t) != doc_at(a, b, t - 1)) ? t : -1;
    int64_t total;
    const int64_t incl = block_max_scan(v, total, sh);
    if (t < T) first[t] = (int32_t)(incl > carry ? incl : carry);
    carry = total > carry ? total : carry;
  }
  // run ends, scanning from the row's end (thread k takes token t1 - 1 - k):
  // token t closes a run when it is the last token or t + 1 has another id;
  // the minimum of those ends over u >= t is a maximum of their negatives
  carry = -T;
  for (int64_t t1 = T; t1 > 0; t1 -= kThreads) {
    const int64_t t = t1 - 1 - threadIdx.x;
    int64_t v = -T;
    if (t >= 0) v = (t == T - 1 || doc_at(a, b, t + 1) != doc_at(a, b, t)) ? -(t + 1) : -T;
    int64_t total;
    const int64_t incl = block_max_scan(v, total, sh);
    if (t >= 0) end[t] = (int32_t)(-(incl > carry ? incl : carry));
    carry = total > carry ? total : carry;
  }
  __syncthreads();  // the row's run bounds are written

  const int d = a.use_dummy;
  const int64_t KL = a.key_length;
  for (int64_t j = threadIdx.x; j < KL; j += kThreads) {
    if (j < d) {
      a.key_ids[(int64_t)b * KL + j] = -1;
      for (int g = 0; g < a.group_count; ++g) {
        const int64_t count = a.group_offsets[g + 1] - a.group_offsets[g];
        a.key_query_end[((int64_t)g * a.batch + b) * KL + j] = (int32_t)count;
      }
      continue;
    }
    const int64_t t = j - d;
    a.key_ids[(int64_t)b * KL + j] = segment_id(doc_at(a, b, t));
    const int64_t e = end[t];
    for (int g = 0; g < a.group_count; ++g) {
      const int64_t count = a.group_offsets[g + 1] - a.group_offsets[g];
      const int64_t behind = e - (a.group_base + g);
      const int64_t q = ((behind > 0 ? behind : 0) + a.groups - 1) / a.groups;
      a.key_query_end[((int64_t)g * a.batch + b) * KL + j] = (int32_t)(q < count ? q : count);
    }
  }
  for (int g = 0; g < a.group_count; ++g) {
    const int64_t o0 = a.group_offsets[g], count = a.group_offsets[g + 1] - o0;
    for (int64_t i = threadIdx.x; i < count; i += kThreads) {
      const int64_t slot = a.slots[o0 + i];
      const bool ok = slot >= 0 && slot < T;
      const int64_t out = (int64_t)a.batch * o0 + (int64_t)b * count + i;
      a.query_ids[out] = ok ? segment_id(doc_at(a, b, slot)) : -2;
      a.query_key_start[out] = ok ? first[slot] + d : 0;
    }
  }
}

}  // namespace

int64_t feedback_meta_workspace_size(const wmx_feedback_meta_args& a) {
  return (int64_t)2 * a.batch * a.length * (int64_t)sizeof(int32_t);
}

int launch_feedback_meta(const wmx_feedback_meta_args& a, hipStream_t stream) {
  if (a.batch == 0) return WMX_OK;
  hipLaunchKernelGGL(feedback_meta_kernel, dim3((unsigned)a.batch), dim3(kThreads), 0, stream, a);
  return WMX_OK;
}

}  // namespace wmx
