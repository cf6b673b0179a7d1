// Internal launch interface between the C ABI (capi.hip) and the kernels.
#pragma once

#include <hip/hip_runtime.h>

#include "wmx_device.h"

namespace wmx {

// How a workgroup finds its query and key rows.
enum Mode {
  kDense = 0,   // rows of one batch entry, strided causal bound (+ optional key mask)
  kDoc = 1,     // kDense plus cyclic document metadata
  kVarlen = 2,  // packed segments addressed through flat query/key indices
};

// Backward workspace: the dK/dV accumulators of varlen schedules whose key
// rows repeat, then from a 256-byte boundary the bf16 dS buffer: per query
// head and problem (batch row or segment) a block of keys x ld elements,
// ld = queries rounded up to 128, holding dS^T (element [j * ld + i] for key
// j and query i).
//   keys_unique 0 (any key row may repeat): fp32 rows [2][batch][key slot]
//     [kv head][D] (dK, then dV), accumulated with atomics;
//   keys_unique 2 (only the leading dummy of a batch row repeats): per
//     segment a mark (its dummy's batch row + 1, 0 without one) from offset
//     0, then from a 256-byte boundary fp32 partials [2][segment][kv head][D]
//     that a second kernel sums in segment order (no atomics: the dummy's
//     gradients are the same on every run).
__host__ __device__ inline int64_t bwd_acc_rows(const wmx_attn_args& a) {
  return a.query_indices && a.keys_unique == 0 ? a.key_extent : 0;
}
__host__ __device__ inline bool bwd_dummy_partials(const wmx_attn_args& a) {
  return a.query_indices && a.keys_unique == 2;
}
__host__ __device__ inline int64_t bwd_dummy_mark_bytes(const wmx_attn_args& a) {
  return ((int64_t)a.num_segments * (int64_t)sizeof(int32_t) + 255) & ~(int64_t)255;
}
__host__ __device__ inline int64_t bwd_acc_bytes(const wmx_attn_args& a) {
  const int64_t row = (int64_t)a.kv_heads * a.head_dim * (int64_t)sizeof(float);
  if (bwd_dummy_partials(a)) return bwd_dummy_mark_bytes(a) + 2 * (int64_t)a.num_segments * row;
  return 2 * (int64_t)a.batch * bwd_acc_rows(a) * row;
}
__host__ __device__ inline int64_t bwd_ds_offset(const wmx_attn_args& a) { return (bwd_acc_bytes(a) + 255) & ~(int64_t)255; }
__host__ __device__ inline int64_t ds_ld(int nq) { return ((int64_t)nq + 127) & ~(int64_t)127; }
int64_t bwd_ds_bytes(const wmx_attn_args& a);  // 0 when the layout has no dS buffer
bool bwd_uses_ds(const wmx_attn_args& a);      // the workspace holds the dS buffer

int launch_fwd(const wmx_attn_args& a, hipStream_t stream);
int launch_dense_units(const wmx_attn_args& a, int32_t* units, hipStream_t stream);
int launch_bwd_preprocess(const wmx_attn_args& a, hipStream_t stream);
int64_t bwd_workspace_size(const wmx_attn_args& a);
int64_t bwd_min_workspace_size(const wmx_attn_args& a);
int launch_bwd(const wmx_attn_args& a, hipStream_t stream);
int launch_bwd_seg(const wmx_attn_args& a, hipStream_t stream);  // the f_units segments (attn_bwd_seg.hip)
int launch_bwd_dq(const wmx_attn_args& a, hipStream_t stream);
int launch_bwd_dkv(const wmx_attn_args& a, hipStream_t stream);
int64_t decode_workspace_size(const wmx_decode_args& a);
int decode_num_splits(const wmx_decode_args& a);
int launch_decode(const wmx_decode_args& a, hipStream_t stream);
int launch_kv_store(const wmx_kv_store_args& a, hipStream_t stream);
int launch_kv_store_bwd(const wmx_kv_store_bwd_args& a, hipStream_t stream);
int64_t kv_store_bwd_workspace_size(const wmx_kv_store_bwd_args& a);
int launch_kv_premix(const wmx_kv_mix_args& a, hipStream_t stream);
int launch_kv_mix(const wmx_kv_mix_args& a, hipStream_t stream);
constexpr int kRouterChunk = 1024;  // inputs per partial sum of the router GEMM
inline int64_t kv_router_chunks(const wmx_kv_router_args& a) { return (a.inputs + kRouterChunk - 1) / kRouterChunk; }
inline int64_t kv_router_workspace_size(const wmx_kv_router_args& a) {
  return 2 * kv_router_chunks(a) * (int64_t)a.rows * a.logits * (int64_t)sizeof(float);
}
int launch_kv_router(const wmx_kv_router_args& a, hipStream_t stream);
int64_t strict_meta_workspace_size(const wmx_strict_meta_args& a);
int launch_strict_meta(const wmx_strict_meta_args& a, bool fill, hipStream_t stream);
int64_t feedback_meta_workspace_size(const wmx_feedback_meta_args& a);
int launch_feedback_meta(const wmx_feedback_meta_args& a, hipStream_t stream);

}  // namespace wmx
