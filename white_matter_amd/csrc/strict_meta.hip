// Packed-document schedule builder for gfx950: the reference's
// prepare_strict_causal_metadata (ops/strict_causal_attention.py:75-155) as
// two kernels with one workgroup per batch row. Integer scans over the row's
// slots and queries replace the torch sequence (cumsum, cummax, nonzero,
// repeat_interleave) and its host synchronisations; the caller synchronises
// once, between the passes, to size the outputs.
//
// Per row the count pass computes, over slots s (present = id >= 0):
//   rank[s]      present slots before s (rank[extent] = the row's total)
//   run_rank[s]  rank of the first slot of the run holding (or last before) s;
//                a run is a maximal sequence of present slots with one id,
//                padding slots in between not breaking it
//   sor[r]       slot of the r-th present slot
// and over queries i at slot p = start + i:
//   first = run_rank[p], end = rank[min(p, kv_len)]  (keys of ranks [first, end))
//   valid = id[p] >= 0 and (end > first or a dummy slot leads the keys)
// Valid queries are compacted in order; consecutive ones share a segment while
// first is unchanged and end grows by exactly one; a segment's keys are those
// of its last query, the dummy first.
#include "wmx_kernels.h"

namespace wmx {

namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;

struct MetaLayout {
  int64_t row_ints;  // int32 elements per row
  int64_t rank, run_rank, sor, vq_i, vq_first, vq_end, seg_kend, seg_first;  // offsets in a row
  __host__ __device__ explicit MetaLayout(const wmx_strict_meta_args& a) {
    const int64_t e = a.extent, q = a.query_length;
    rank = 0;
    run_rank = e + 1;
    sor = run_rank + e;
    vq_i = sor + e;
    vq_first = vq_i + q;
    vq_end = vq_first + q;
    seg_kend = vq_end + q;
    seg_first = seg_kend + q;
    row_ints = (seg_first + q + 3) & ~(int64_t)3;  // rows stay 16-byte aligned
  }
};

struct Add {
  __device__ int64_t operator()(int64_t x, int64_t y) const { return x + y; }
  static constexpr int64_t kIdentity = 0;
};
struct Max {
  __device__ int64_t operator()(int64_t x, int64_t y) const { return x > y ? x : y; }
  static constexpr int64_t kIdentity = INT64_MIN;
};

// Inclusive scan of x over the workgroup's 1024 threads in thread order;
// `total` receives the reduction over all of them. Every thread must call it.
template <typename Op>
__device__ int64_t block_scan(int64_t x, int64_t& total, int64_t* sh) {
  const Op op;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int64_t y = __shfl_up(x, o);
    if (lane >= o) x = op(x, y);
  }
  if (lane == 63) sh[w] = x;
  __syncthreads();
  int64_t before = Op::kIdentity, all = Op::kIdentity;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    if (i < w) before = op(before, sh[i]);
    all = op(all, sh[i]);
  }
  __syncthreads();  // sh is free again
  total = all;
  return op(before, x);
}

__device__ __forceinline__ int64_t doc_id(const wmx_strict_meta_args& a, int b, int64_t s) {
  const int64_t off = (int64_t)b * a.doc_stride + s;
  return a.doc_dtype == WMX_DTYPE_I32 ? (int64_t)((const int32_t*)a.document_ids)[off]
                                      : ((const int64_t*)a.document_ids)[off];
}

// Segments of the row's compacted valid queries (nv of them). For each
// compacted query k: brk (it opens a segment), last (it closes one) and the
// closing segment's key count. With FILL the row's outputs are written at the
// given offsets; the totals (segments, keys) are returned either way.
template <bool FILL>
__device__ void segments(const wmx_strict_meta_args& a, int b, const int32_t* ws, int32_t* wsw, const MetaLayout& L,
                         int64_t nv, int64_t qoff, int64_t soff, int64_t koff, int64_t& nseg, int64_t& nkeys,
                         int64_t* sh) {
  const int32_t* vq_i = ws + L.vq_i;
  const int32_t* vq_first = ws + L.vq_first;
  const int32_t* vq_end = ws + L.vq_end;
  int64_t carry_seg = 0, carry_keys = 0;
  for (int64_t k0 = 0; k0 < nv; k0 += kThreads) {
    const int64_t k = k0 + threadIdx.x;
    const bool in = k < nv;
    int64_t f = 0, e = 0;
    bool brk = false, last = false;
    if (in) {
      f = vq_first[k];
      e = vq_end[k];
      brk = k == 0 || vq_first[k - 1] != f || vq_end[k - 1] + 1 != e;
      last = k + 1 == nv || vq_first[k + 1] != f || vq_end[k + 1] != e + 1;
    }
    const int64_t c = last ? (e > f ? e - f : 0) + a.use_dummy : 0;
    int64_t seg_total, key_total;
    const int64_t seg_incl = block_scan<Add>(brk ? 1 : 0, seg_total, sh);
    const int64_t key_incl = block_scan<Add>(c, key_total, sh);
    if (FILL && in) {
      const int64_t sidx = carry_seg + seg_incl - 1;  // this query's segment (row-local)
      a.query_indices[qoff + k] = (int64_t)b * a.query_length + vq_i[k];
      if (brk) {
        a.cu_queries[soff + sidx] = (int32_t)(qoff + k);
        a.cu_keys[soff + sidx] = (int32_t)(koff + carry_keys + key_incl - c);
      }
      if (last) {
        wsw[L.seg_kend + sidx] = (int32_t)(carry_keys + key_incl);
        wsw[L.seg_first + sidx] = (int32_t)f;
      }
    }
    carry_seg += seg_total;
    carry_keys += key_total;
  }
  nseg = carry_seg;
  nkeys = carry_keys;
}

__global__ __launch_bounds__(kThreads) void strict_meta_count_kernel(const wmx_strict_meta_args a) {
  __shared__ int64_t sh[kWaves];
  __shared__ int64_t prev_lds[kThreads];
  const int b = blockIdx.x, tid = threadIdx.x;
  const MetaLayout L(a);
  int32_t* ws = (int32_t*)a.workspace + (int64_t)b * L.row_ints;

  // slots: rank, run_rank, sor
  int64_t carry_rank = 0, carry_prev = -1, carry_rr = 0;
  for (int64_t c0 = 0; c0 < a.extent; c0 += kThreads) {
    const int64_t s = c0 + tid;
    const bool in = s < a.extent;
    const int64_t id = in ? doc_id(a, b, s) : -1;
    const bool pres = in && id >= 0;
    int64_t t_rank, t_prev, t_rr;
    const int64_t rank = carry_rank + block_scan<Add>(pres ? 1 : 0, t_rank, sh) - (pres ? 1 : 0);
    const int64_t pmax = block_scan<Max>(pres ? s : -1, t_prev, sh);
    prev_lds[tid] = pmax;
    __syncthreads();
    int64_t prev = tid > 0 ? prev_lds[tid - 1] : -1;  // last present slot before s
    prev = prev > carry_prev ? prev : carry_prev;
    const bool run_begins = pres && (prev < 0 || doc_id(a, b, prev) != id);
    const int64_t rr_in = block_scan<Max>(run_begins ? rank : 0, t_rr, sh);
    const int64_t run_rank = rr_in > carry_rr ? rr_in : carry_rr;
    if (in) {
      ws[L.rank + s] = (int32_t)rank;
      ws[L.run_rank + s] = (int32_t)run_rank;
      if (pres) ws[L.sor + rank] = (int32_t)s;
    }
    carry_rank += t_rank;
    carry_prev = t_prev > carry_prev ? t_prev : carry_prev;
    carry_rr = t_rr > carry_rr ? t_rr : carry_rr;
    __syncthreads();  // prev_lds is reused by the next chunk
  }
  if (tid == 0) ws[L.rank + a.extent] = (int32_t)carry_rank;
  __syncthreads();  // rank and run_rank are read at arbitrary slots below

  // queries: validity and compaction
  const int64_t start = a.query_start ? a.query_start[b] : a.query_start_scalar;
  const int64_t kv = a.kv_lengths ? a.kv_lengths[b] : INT64_MAX;
  int64_t nv = 0, bad_any = 0;
  for (int64_t i0 = 0; i0 < a.query_length; i0 += kThreads) {
    const int64_t i = i0 + tid;
    const bool in = i < a.query_length;
    const int64_t p = start + i;
    const bool bad = in && (p < 0 || p >= a.extent);
    bool valid = false;
    int64_t first = 0, end = 0;
    if (in && !bad) {
      first = ws[L.run_rank + p];
      int64_t reach = p < kv ? p : kv;
      reach = reach < 0 ? 0 : reach > a.extent ? a.extent : reach;
      end = ws[L.rank + reach];
      valid = doc_id(a, b, p) >= 0 && (end > first || a.use_dummy);
    }
    int64_t t_valid, t_bad;
    const int64_t pos = nv + block_scan<Add>(valid ? 1 : 0, t_valid, sh) - (valid ? 1 : 0);
    block_scan<Max>(bad ? 1 : 0, t_bad, sh);
    if (valid) {
      ws[L.vq_i + pos] = (int32_t)i;
      ws[L.vq_first + pos] = (int32_t)first;
      ws[L.vq_end + pos] = (int32_t)end;
    }
    nv += t_valid;
    bad_any = t_bad > bad_any ? t_bad : bad_any;
  }
  __syncthreads();  // the compacted queries are read by neighbours below

  int64_t nseg, nkeys;
  segments<false>(a, b, ws, ws, L, nv, 0, 0, 0, nseg, nkeys, sh);
  if (tid == 0) {
    a.counts[4 * b + 0] = nv;
    a.counts[4 * b + 1] = nseg;
    a.counts[4 * b + 2] = nkeys;
    a.counts[4 * b + 3] = bad_any;
  }
}

__global__ __launch_bounds__(kThreads) void strict_meta_fill_kernel(const wmx_strict_meta_args a) {
  __shared__ int64_t sh[kWaves];
  const int b = blockIdx.x, tid = threadIdx.x;
  const MetaLayout L(a);
  int32_t* ws = (int32_t*)a.workspace + (int64_t)b * L.row_ints;

  // this row's output offsets: totals of the rows before it
  int64_t q_before = 0, s_before = 0, k_before = 0, q_all = 0, s_all = 0, k_all = 0;
  for (int r = tid; r < a.batch; r += kThreads) {
    const int64_t nq = a.counts[4 * r], ns = a.counts[4 * r + 1], nk = a.counts[4 * r + 2];
    q_all += nq;
    s_all += ns;
    k_all += nk;
    if (r < b) {
      q_before += nq;
      s_before += ns;
      k_before += nk;
    }
  }
  int64_t qoff, soff, koff, q_total, s_total, k_total;
  block_scan<Add>(q_before, qoff, sh);
  block_scan<Add>(s_before, soff, sh);
  block_scan<Add>(k_before, koff, sh);
  block_scan<Add>(q_all, q_total, sh);
  block_scan<Add>(s_all, s_total, sh);
  block_scan<Add>(k_all, k_total, sh);

  const int64_t nv = a.counts[4 * b];
  int64_t nseg, nkeys;
  segments<true>(a, b, ws, ws, L, nv, qoff, soff, koff, nseg, nkeys, sh);
  if (b == a.batch - 1 && tid == 0) {
    a.cu_queries[s_total] = (int32_t)q_total;
    a.cu_keys[s_total] = (int32_t)k_total;
  }
  __syncthreads();  // segment key ends and first ranks are read below

  // keys: key t of the row belongs to the segment whose key end first exceeds t
  const int32_t* seg_kend = ws + L.seg_kend;
  const int32_t* seg_first = ws + L.seg_first;
  const int32_t* sor = ws + L.sor;
  const int64_t key_extent = (int64_t)a.extent + a.use_dummy;
  for (int64_t t0 = tid; t0 < nkeys; t0 += kThreads) {
    int64_t lo = 0, hi = nseg - 1;
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if (seg_kend[mid] > t0) hi = mid;
      else lo = mid + 1;
    }
    const int64_t j = t0 - (lo > 0 ? seg_kend[lo - 1] : 0);
    const int64_t slot = (a.use_dummy && j == 0) ? 0 : sor[seg_first[lo] + j - a.use_dummy] + a.use_dummy;
    a.key_indices[koff + t0] = (int64_t)b * key_extent + slot;
  }
}

}  // namespace

int64_t strict_meta_workspace_size(const wmx_strict_meta_args& a) {
  return (int64_t)a.batch * MetaLayout(a).row_ints * (int64_t)sizeof(int32_t);
}

int launch_strict_meta(const wmx_strict_meta_args& a, bool fill, hipStream_t stream) {
  if (a.batch == 0) return WMX_OK;
  if (fill)
    hipLaunchKernelGGL(strict_meta_fill_kernel, dim3(a.batch), dim3(kThreads), 0, stream, a);
  else
    hipLaunchKernelGGL(strict_meta_count_kernel, dim3(a.batch), dim3(kThreads), 0, stream, a);
  return WMX_OK;
}

}  // namespace wmx
