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

int launch_fwd(const wmx_attn_args& a, hipStream_t stream);
int launch_bwd_preprocess(const wmx_attn_args& a, hipStream_t stream);
int64_t bwd_workspace_size(const wmx_attn_args& a);
int launch_bwd(const wmx_attn_args& a, hipStream_t stream);
int launch_bwd_dq(const wmx_attn_args& a, hipStream_t stream);
int launch_bwd_dkv(const wmx_attn_args& a, hipStream_t stream);
int64_t decode_workspace_size(const wmx_decode_args& a);
int decode_num_splits(const wmx_decode_args& a);
int launch_decode(const wmx_decode_args& a, hipStream_t stream);

}  // namespace wmx
