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

// Backward workspace: fp32 dK/dV accumulators (varlen schedules whose key
// rows repeat: all rows, or slot 0 only), then from a 256-byte boundary the bf16 dS buffer: per query
// head and problem (batch row or segment) a block of keys x ld elements,
// ld = queries rounded up to 128, holding dS^T (element [j * ld + i] for key
// j and query i).
// Rows of the fp32 dK/dV accumulators per batch row: every key slot when any
// key row may repeat, slot 0 only when only the leading dummy repeats.
__host__ __device__ inline int64_t bwd_acc_rows(const wmx_attn_args& a) {
  if (!a.query_indices || a.keys_unique == 1) return 0;
  return a.keys_unique == 2 ? 1 : a.key_extent;
}
__host__ __device__ inline int64_t bwd_acc_bytes(const wmx_attn_args& a) {
  return (int64_t)2 * a.batch * bwd_acc_rows(a) * a.kv_heads * a.head_dim * (int64_t)sizeof(float);
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
int launch_bwd_dq(const wmx_attn_args& a, hipStream_t stream);
int launch_bwd_dkv(const wmx_attn_args& a, hipStream_t stream);
int64_t decode_workspace_size(const wmx_decode_args& a);
int decode_num_splits(const wmx_decode_args& a);
int launch_decode(const wmx_decode_args& a, hipStream_t stream);
int launch_kv_store(const wmx_kv_store_args& a, hipStream_t stream);
int64_t strict_meta_workspace_size(const wmx_strict_meta_args& a);
int launch_strict_meta(const wmx_strict_meta_args& a, bool fill, hipStream_t stream);
int64_t feedback_meta_workspace_size(const wmx_feedback_meta_args& a);
int launch_feedback_meta(const wmx_feedback_meta_args& a, hipStream_t stream);

}  // namespace wmx
