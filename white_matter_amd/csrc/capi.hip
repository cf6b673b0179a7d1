// extern "C" entry points of libwmx_attn.so (declared in include/wmx_attn.h).
// Each entry point checks what the kernels assume about shapes, strides and
// alignment before anything is launched, so a bad call returns an error code
// instead of reaching the GPU.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "wmx_kernels.h"

// Device scratch of wmx_decode_noalloc: the split-K partials live here instead
// of in a caller-allocated workspace. Each GPU holds its own copy for the life
// of the process. Host code never uses this name as an address: the entry
// point resolves the array's device address once per device with
// hipGetSymbolAddress and passes that pointer to the kernels.
constexpr int64_t kDecodeScratchBytes = WMX_DECODE_NOALLOC_MAX_BYTES;
static __device__ __align__(256) unsigned char scratch[kDecodeScratchBytes];

namespace {

thread_local char g_error[512] = "";

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
bool aligned8(const void* p) { return ((uintptr_t)p & 7u) == 0; }

// Row starts must stay 16-byte aligned for the 16-byte loads.
bool strides_vec8(const int64_t* s, int n) {
  for (int i = 0; i < n; ++i)
    if (s[i] % 8 != 0) return false;
  return true;
}

int check_common(const wmx_attn_args* a, bool backward) {
  if (!a) return fail(WMX_E_INVALID, "args is NULL");
  if (a->head_dim != 64 && a->head_dim != 96 && a->head_dim != 128)
    return fail(WMX_E_UNSUPPORTED, "head_dim %d is not 64, 96 or 128", a->head_dim);
  if (a->batch < 0 || a->q_heads <= 0 || a->kv_heads <= 0 || a->q_len < 0 || a->kv_len < 0)
    return fail(WMX_E_INVALID, "negative or zero shape");
  if (a->q_heads % a->kv_heads != 0) return fail(WMX_E_INVALID, "q_heads %% kv_heads != 0");
  if (a->query_stride < 1) return fail(WMX_E_INVALID, "query_stride must be >= 1");
  if (a->query_tile != 0 && a->query_tile != 128 && a->query_tile != 256)
    return fail(WMX_E_INVALID, "query_tile must be 0, 128 or 256");
  if (a->key_tile != 0 && a->key_tile != 64 && a->key_tile != 128)
    return fail(WMX_E_INVALID, "key_tile must be 0, 64 or 128");
  if (!(a->softmax_scale > 0.f)) return fail(WMX_E_UNSUPPORTED, "softmax_scale must be positive and finite");
  if (!a->q || !a->k || !a->v || !a->o || !a->lse) return fail(WMX_E_INVALID, "q/k/v/o/lse pointer is NULL");
  if (!aligned16(a->q) || !aligned16(a->k) || !aligned16(a->v))
    return fail(WMX_E_INVALID, "q/k/v must be 16-byte aligned");
  if (!aligned8(a->o)) return fail(WMX_E_INVALID, "o must be 8-byte aligned");
  if (!strides_vec8(a->q_stride, 3) || !strides_vec8(a->k_stride, 3) || !strides_vec8(a->v_stride, 3))
    return fail(WMX_E_INVALID, "q/k/v strides must be multiples of 8 elements");
  if (!strides_vec8(a->o_stride, 3)) return fail(WMX_E_INVALID, "o strides must be multiples of 8 elements");
  if (a->query_indices) {
    if (!a->key_indices || !a->cu_queries || !a->cu_keys)
      return fail(WMX_E_INVALID, "varlen schedule needs key_indices, cu_queries and cu_keys");
    if (a->num_segments < 0 || a->max_queries < 0 || a->max_keys < 0 || a->query_extent <= 0 || a->key_extent <= 0)
      return fail(WMX_E_INVALID, "invalid varlen sizes");
    if (a->q_seg) return fail(WMX_E_INVALID, "varlen schedule and document metadata are exclusive");
    if (a->key_mask) return fail(WMX_E_INVALID, "varlen schedule and key_mask are exclusive");
    if (a->row_offset || a->row_limit) return fail(WMX_E_INVALID, "varlen schedule takes no row offsets");
    if (a->k_units && a->num_k_units < 0) return fail(WMX_E_INVALID, "negative work-list length");
    if (a->keys_unique < 0 || a->keys_unique > 2) return fail(WMX_E_INVALID, "keys_unique must be 0, 1 or 2");
    if (a->ds_offsets && a->ds_elements < 0) return fail(WMX_E_INVALID, "negative ds_elements");
    if (a->f_units) {
      if (a->num_f_units < 0) return fail(WMX_E_INVALID, "negative work-list length");
      if (!a->k_units || !a->q_units)
        return fail(WMX_E_INVALID, "f_units needs k_units and q_units (the segments it does not list)");
      if (a->unit_fields != WMX_UNIT_FIELDS)
        return fail(WMX_E_INVALID, "f_units needs entries of WMX_UNIT_FIELDS ints (unit_fields)");
      if (a->q_heads != a->kv_heads) return fail(WMX_E_INVALID, "f_units needs q_heads == kv_heads");
      if (a->keys_unique == 0) return fail(WMX_E_INVALID, "f_units needs keys_unique 1 or 2");
      if ((a->segment_layout & 3) != 3)
        return fail(WMX_E_INVALID, "f_units needs consecutive query and key slots (segment_layout bits 0 and 1)");
      for (const int64_t* st : {a->q_stride, a->k_stride, a->v_stride, a->do_stride})
        if (st[2] < a->head_dim || st[2] >= (int64_t(1) << 23))
          return fail(WMX_E_INVALID, "f_units needs token strides in [head_dim, 2^23) elements");
    }
  } else if (a->k_units || a->ds_offsets || a->f_units) {
    return fail(WMX_E_INVALID, "key work lists, fused segment lists and dS offsets need a varlen schedule");
  }
  if (a->q_units && a->num_q_units < 0) return fail(WMX_E_INVALID, "negative work-list length");
  if (a->q_seg && (!a->k_seg || !a->q_start || !a->k_qend))
    return fail(WMX_E_INVALID, "document metadata needs all four arrays");
  if (a->q_seg && a->key_mask) return fail(WMX_E_INVALID, "document metadata and key_mask are exclusive");
  if (backward) {
    if (!a->dout || !a->delta || !a->dq || !a->dk || !a->dv)
      return fail(WMX_E_INVALID, "dout/delta/dq/dk/dv pointer is NULL");
    if (!aligned16(a->dout)) return fail(WMX_E_INVALID, "dout must be 16-byte aligned");
    if (!aligned8(a->dq) || !aligned8(a->dk) || !aligned8(a->dv))
      return fail(WMX_E_INVALID, "dq/dk/dv must be 8-byte aligned");
    if (!strides_vec8(a->do_stride, 3) || !strides_vec8(a->dq_stride, 3) || !strides_vec8(a->dk_stride, 3) ||
        !strides_vec8(a->dv_stride, 3))
      return fail(WMX_E_INVALID, "gradient strides must be multiples of 8 elements");
    const int64_t need = wmx::bwd_min_workspace_size(*a);
    if (need > 0 && (!a->workspace || a->workspace_bytes < need))
      return fail(WMX_E_WORKSPACE, "backward needs %lld workspace bytes", (long long)need);
    if (a->workspace && !aligned16(a->workspace)) return fail(WMX_E_WORKSPACE, "workspace must be 16-byte aligned");
  }
  return WMX_OK;
}

int launched(int rc) {
  if (rc != WMX_OK) {
    if (rc == WMX_E_UNSUPPORTED) return fail(rc, "unsupported configuration");
    return rc;
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(WMX_E_LAUNCH, "launch failed: %s", hipGetErrorString(e));
  return WMX_OK;
}

// Everything wmx_decode checks except the workspace.
int check_decode(const wmx_decode_args* a) {
  if (!a) return fail(WMX_E_INVALID, "args is NULL");
  if (a->head_dim != 64 && a->head_dim != 96 && a->head_dim != 128)
    return fail(WMX_E_UNSUPPORTED, "head_dim %d is not 64, 96 or 128", a->head_dim);
  if (a->batch < 0 || a->q_heads <= 0 || a->kv_heads <= 0 || a->capacity < 0)
    return fail(WMX_E_INVALID, "negative or zero shape");
  if (a->q_heads % a->kv_heads != 0) return fail(WMX_E_INVALID, "q_heads %% kv_heads != 0");
  if (!a->q || !a->k || !a->v || !a->o) return fail(WMX_E_INVALID, "q/k/v/o pointer is NULL");
  if (!aligned16(a->q) || !aligned16(a->k) || !aligned16(a->v))
    return fail(WMX_E_INVALID, "q/k/v must be 16-byte aligned");
  if (a->q_stride[0] % 8 || a->q_stride[1] % 8 || !strides_vec8(a->k_stride, 3) || !strides_vec8(a->v_stride, 3))
    return fail(WMX_E_INVALID, "q/k/v strides must be multiples of 8 elements");
  if (a->use_dummy != 0 && a->use_dummy != 1) return fail(WMX_E_INVALID, "use_dummy must be 0 or 1");
  return WMX_OK;
}

// Device address of `scratch` on the current device, resolved once per device
// (with that device current) and kept.
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxScratchDevices] = {};

int decode_scratch(void* stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(WMX_E_LAUNCH, "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(WMX_E_UNSUPPORTED, "device %d is beyond the %d devices the static scratch serves", dev, kMaxScratchDevices);
  int sdev = dev;
  e = hipStreamGetDevice((hipStream_t)stream, &sdev);
  if (e != hipSuccess) return fail(WMX_E_INVALID, "hipStreamGetDevice failed: %s", hipGetErrorString(e));
  if (sdev != dev) return fail(WMX_E_INVALID, "the stream belongs to device %d, the current device is %d", sdev, dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(WMX_E_LAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return WMX_OK;
}

int check_strict_meta(const wmx_strict_meta_args* a, bool fill) {
  if (!a) return fail(WMX_E_INVALID, "args is NULL");
  if (a->batch < 0 || a->extent < 0 || a->query_length < 0) return fail(WMX_E_INVALID, "negative shape");
  if (a->use_dummy != 0 && a->use_dummy != 1) return fail(WMX_E_INVALID, "use_dummy must be 0 or 1");
  if (a->doc_dtype != WMX_DTYPE_I32 && a->doc_dtype != WMX_DTYPE_I64)
    return fail(WMX_E_INVALID, "document_ids must be WMX_DTYPE_I32 or WMX_DTYPE_I64");
  if (a->batch == 0) return WMX_OK;
  if ((a->extent > 0 && !a->document_ids) || !a->counts) return fail(WMX_E_INVALID, "document_ids/counts pointer is NULL");
  if (a->doc_stride < a->extent) return fail(WMX_E_INVALID, "doc_stride is smaller than extent");
  const int64_t need = wmx::strict_meta_workspace_size(*a);
  if (!a->workspace || a->workspace_bytes < need || !aligned16(a->workspace))
    return fail(WMX_E_WORKSPACE, "schedule builder needs %lld workspace bytes", (long long)need);
  if (fill && (!a->query_indices || !a->key_indices || !a->cu_queries || !a->cu_keys))
    return fail(WMX_E_INVALID, "fill needs query_indices, key_indices, cu_queries and cu_keys");
  return WMX_OK;
}

int check_feedback_meta(const wmx_feedback_meta_args* a) {
  if (!a) return fail(WMX_E_INVALID, "args is NULL");
  if (a->batch < 0 || a->length < 0 || a->key_length < 0) return fail(WMX_E_INVALID, "negative shape");
  if (a->use_dummy != 0 && a->use_dummy != 1) return fail(WMX_E_INVALID, "use_dummy must be 0 or 1");
  if (a->doc_dtype != WMX_DTYPE_I32 && a->doc_dtype != WMX_DTYPE_I64)
    return fail(WMX_E_INVALID, "document_ids must be WMX_DTYPE_I32 or WMX_DTYPE_I64");
  if ((int64_t)a->key_length > (int64_t)a->length + a->use_dummy)
    return fail(WMX_E_INVALID, "key_length %d exceeds the dummy-shifted extent %d", a->key_length,
                a->length + a->use_dummy);
  if (a->groups < 1) return fail(WMX_E_INVALID, "groups must be >= 1");
  if (a->group_count < 1 || a->group_count > WMX_FEEDBACK_MAX_GROUPS)
    return fail(WMX_E_INVALID, "group_count must be in [1, %d]", WMX_FEEDBACK_MAX_GROUPS);
  if (a->group_base < 0 || (int64_t)a->group_base + a->group_count > a->groups)
    return fail(WMX_E_INVALID, "groups [group_base, group_base + group_count) must lie in [0, groups)");
  if (a->group_offsets[0] != 0) return fail(WMX_E_INVALID, "group_offsets[0] must be 0");
  for (int g = 0; g < a->group_count; ++g)
    if (a->group_offsets[g + 1] < a->group_offsets[g]) return fail(WMX_E_INVALID, "group_offsets must be nondecreasing");
  if (a->batch == 0) return WMX_OK;
  if (a->length > 0 && (!a->document_ids || a->doc_stride < a->length))
    return fail(WMX_E_INVALID, "document_ids is NULL or doc_stride is smaller than length");
  if (a->key_length > 0 && (!a->key_ids || !a->key_query_end))
    return fail(WMX_E_INVALID, "key_ids/key_query_end pointer is NULL");
  if (a->group_offsets[a->group_count] > 0 && (!a->slots || !a->query_ids || !a->query_key_start))
    return fail(WMX_E_INVALID, "slots/query_ids/query_key_start pointer is NULL");
  const int64_t need = wmx::feedback_meta_workspace_size(*a);
  if (need > 0 && (!a->workspace || a->workspace_bytes < need || !aligned16(a->workspace)))
    return fail(WMX_E_WORKSPACE, "feedback metadata needs %lld workspace bytes", (long long)need);
  return WMX_OK;
}

}  // namespace

extern "C" {

int wmx_abi_version(void) { return WMX_ABI_VERSION; }
size_t wmx_attn_args_size(void) { return sizeof(wmx_attn_args); }
size_t wmx_decode_args_size(void) { return sizeof(wmx_decode_args); }
const char* wmx_last_error(void) { return g_error; }

int wmx_attn_fwd(const wmx_attn_args* args, void* stream) {
  int rc = check_common(args, false);
  if (rc != WMX_OK) return rc;
  if (args->batch == 0 || args->q_len == 0) return WMX_OK;
  return launched(wmx::launch_fwd(*args, (hipStream_t)stream));
}

int wmx_attn_bwd_preprocess(const wmx_attn_args* args, void* stream) {
  if (!args) return fail(WMX_E_INVALID, "args is NULL");
  if (args->head_dim != 64 && args->head_dim != 96 && args->head_dim != 128)
    return fail(WMX_E_UNSUPPORTED, "head_dim %d is not 64, 96 or 128", args->head_dim);
  if (!args->o || !args->dout || !args->delta) return fail(WMX_E_INVALID, "o/dout/delta pointer is NULL");
  if (!aligned16(args->o) || !aligned16(args->dout)) return fail(WMX_E_INVALID, "o/dout must be 16-byte aligned");
  if (!strides_vec8(args->o_stride, 3) || !strides_vec8(args->do_stride, 3))
    return fail(WMX_E_INVALID, "o/dout strides must be multiples of 8 elements");
  return launched(wmx::launch_bwd_preprocess(*args, (hipStream_t)stream));
}

int64_t wmx_attn_bwd_workspace_size(const wmx_attn_args* args) {
  return args ? wmx::bwd_workspace_size(*args) : 0;
}

int64_t wmx_attn_bwd_min_workspace_size(const wmx_attn_args* args) {
  return args ? wmx::bwd_min_workspace_size(*args) : 0;
}

int wmx_attn_bwd(const wmx_attn_args* args, void* stream) {
  int rc = check_common(args, true);
  if (rc != WMX_OK) return rc;
  if (!aligned16(args->o)) return fail(WMX_E_INVALID, "o must be 16-byte aligned for the backward");
  if (args->batch == 0 || args->q_len == 0) return WMX_OK;
  return launched(wmx::launch_bwd(*args, (hipStream_t)stream));
}

int wmx_attn_bwd_dq(const wmx_attn_args* args, void* stream) {
  int rc = check_common(args, true);
  if (rc != WMX_OK) return rc;
  if (args->batch == 0 || args->q_len == 0) return WMX_OK;
  return launched(wmx::launch_bwd_dq(*args, (hipStream_t)stream));
}

int wmx_attn_bwd_dkv(const wmx_attn_args* args, void* stream) {
  int rc = check_common(args, true);
  if (rc != WMX_OK) return rc;
  if (args->batch == 0 || args->q_len == 0) return WMX_OK;
  return launched(wmx::launch_bwd_dkv(*args, (hipStream_t)stream));
}

int wmx_kv_pool_store(const wmx_kv_store_args* a, void* stream) {
  if (!a) return fail(WMX_E_INVALID, "args is NULL");
  if (a->head_dim != 64 && a->head_dim != 96 && a->head_dim != 128)
    return fail(WMX_E_UNSUPPORTED, "kv store head_dim %d is not 64, 96 or 128", a->head_dim);
  if (a->batch < 0 || a->channels < 0 || a->heads < 0 || a->tokens < 0 || a->pool_slots < 0)
    return fail(WMX_E_INVALID, "negative shape");
  for (int dt : {a->key_dtype, a->value_dtype, a->weight_dtype, a->rope_dtype})
    if (dt != WMX_DTYPE_F32 && dt != WMX_DTYPE_BF16) return fail(WMX_E_INVALID, "dtype must be WMX_DTYPE_F32 or WMX_DTYPE_BF16");
  if (!(a->eps >= 0.f)) return fail(WMX_E_INVALID, "eps must be >= 0");
  if ((int64_t)a->batch * a->channels * a->heads * a->tokens == 0) return WMX_OK;
  if (!a->key || !a->k_norm_weight || !a->cos || !a->sin || !a->key_pool || !a->slots)
    return fail(WMX_E_INVALID, "kv store pointer is NULL");
  if (!a->value != !a->value_pool) return fail(WMX_E_INVALID, "value and value_pool are given together");
  if (!aligned16(a->key) || !aligned16(a->value) || !aligned16(a->k_norm_weight) || !aligned16(a->cos) ||
      !aligned16(a->sin) || !aligned16(a->key_pool) || !aligned16(a->value_pool) || !aligned8(a->slots))
    return fail(WMX_E_INVALID, "kv store operands must be 16-byte aligned");
  if (!strides_vec8(a->key_stride, 4) || !strides_vec8(a->value_stride, 4) || !strides_vec8(a->key_pool_stride, 4) ||
      !strides_vec8(a->value_pool_stride, 4) || !strides_vec8(a->rope_stride, 2))
    return fail(WMX_E_INVALID, "kv store strides must be multiples of 8 elements");
  return launched(wmx::launch_kv_store(*a, (hipStream_t)stream));
}

static int check_kv_mix(const wmx_kv_mix_args* a, bool premix) {
  if (!a) return fail(WMX_E_INVALID, "args is NULL");
  if (a->batch < 0 || a->tokens < 0) return fail(WMX_E_INVALID, "negative shape");
  if (a->num_sources < 1 || a->num_sources > WMX_KV_MIX_MAX_SOURCES)
    return fail(WMX_E_UNSUPPORTED, "kv mix num_sources %d is not in [1, %d]", a->num_sources, WMX_KV_MIX_MAX_SOURCES);
  if (a->hidden < 8 || a->hidden % 8 || a->hidden > WMX_KV_MIX_MAX_HIDDEN)
    return fail(WMX_E_UNSUPPORTED, "kv mix hidden %d is not a multiple of 8 in [8, %d]", a->hidden, WMX_KV_MIX_MAX_HIDDEN);
  if (a->channels < 1) return fail(WMX_E_INVALID, "kv mix channels must be >= 1");
  for (int dt : {a->source_dtype, a->weight_dtype})
    if (dt != WMX_DTYPE_F32 && dt != WMX_DTYPE_BF16) return fail(WMX_E_INVALID, "dtype must be WMX_DTYPE_F32 or WMX_DTYPE_BF16");
  if (!(a->eps >= 0.f) || !(a->mix_eps >= 0.f)) return fail(WMX_E_INVALID, "eps and mix_eps must be >= 0");
  if ((int64_t)a->batch * a->tokens == 0) return WMX_OK;
  for (int side = 0; side < 2; ++side) {
    if (!a->premixed[side]) return fail(WMX_E_INVALID, "kv mix pointer is NULL");
    if (premix ? !a->pre_mix[side] : (!a->alpha[side] || !a->gain[side] || !a->mixed[side]))
      return fail(WMX_E_INVALID, "kv mix pointer is NULL");
    if (!aligned16(a->premixed[side]) || !aligned16(a->pre_mix[side]) || !aligned16(a->gain[side]) ||
        !aligned16(a->mixed[side]) || ((uintptr_t)a->alpha[side] & 1u))
      return fail(WMX_E_INVALID, "kv mix operands must be 16-byte aligned (alpha 2-byte)");
  }
  return WMX_OK;
}

int wmx_kv_premix(const wmx_kv_mix_args* a, void* stream) {
  int rc = check_kv_mix(a, true);
  if (rc != WMX_OK || (int64_t)a->batch * a->tokens == 0) return rc;
  if (!a->sources) return fail(WMX_E_INVALID, "kv mix sources is NULL");
  if (!aligned16(a->sources) || !strides_vec8(a->source_stride, 3))
    return fail(WMX_E_INVALID, "kv mix sources must be 16-byte aligned with strides of multiples of 8 elements");
  return launched(wmx::launch_kv_premix(*a, (hipStream_t)stream));
}

int wmx_kv_mix(const wmx_kv_mix_args* a, void* stream) {
  int rc = check_kv_mix(a, false);
  if (rc != WMX_OK || (int64_t)a->batch * a->tokens == 0) return rc;
  if (a->alpha_stride < (int64_t)a->channels * a->num_sources)
    return fail(WMX_E_INVALID, "kv mix alpha_stride must cover the C*S logits of a token");
  return launched(wmx::launch_kv_mix(*a, (hipStream_t)stream));
}

static int check_kv_router(const wmx_kv_router_args* a) {
  if (!a) return fail(WMX_E_INVALID, "args is NULL");
  if (a->rows < 0) return fail(WMX_E_INVALID, "negative shape");
  if (a->inputs < 64 || a->inputs % 64)
    return fail(WMX_E_UNSUPPORTED, "kv router inputs %d is not a positive multiple of 64", a->inputs);
  if (a->logits < 1 || a->logits > WMX_KV_ROUTER_MAX_LOGITS)
    return fail(WMX_E_UNSUPPORTED, "kv router logits %d is not in [1, %d]", a->logits, WMX_KV_ROUTER_MAX_LOGITS);
  if (a->source_width != 0) {
    if (a->source_width < 0 || a->source_width % 64 || a->inputs % a->source_width)
      return fail(WMX_E_UNSUPPORTED, "kv router source_width %d must be a multiple of 64 dividing inputs",
                  a->source_width);
    if (a->source_start < 0 || a->source_stride < 1) return fail(WMX_E_INVALID, "kv router source start/stride");
    const int64_t blocks = a->inputs / a->source_width;
    const int64_t last = (int64_t)a->source_start + (blocks - 1) * a->source_stride;
    if (a->row_stride < 0 || a->row_stride % 8 || (last + 1) * a->source_width > a->row_stride)
      return fail(WMX_E_INVALID, "kv router row_stride %d does not hold the selected sources", a->row_stride);
  }
  return WMX_OK;
}

int64_t wmx_kv_router_workspace_size(const wmx_kv_router_args* a) {
  return check_kv_router(a) == WMX_OK ? wmx::kv_router_workspace_size(*a) : 0;
}

int wmx_kv_router(const wmx_kv_router_args* a, void* stream) {
  int rc = check_kv_router(a);
  if (rc != WMX_OK || a->rows == 0) return rc;
  for (int side = 0; side < 2; ++side) {
    if (!a->premixed[side] || !a->weight[side] || !a->alpha[side]) return fail(WMX_E_INVALID, "kv router pointer is NULL");
    if (!aligned16(a->premixed[side]) || !aligned16(a->weight[side]) || ((uintptr_t)a->alpha[side] & 1u) ||
        ((uintptr_t)a->bias[side] & 1u))
      return fail(WMX_E_INVALID, "kv router operands must be 16-byte aligned (alpha and bias 2-byte)");
  }
  const int64_t need = wmx::kv_router_workspace_size(*a);
  if (!a->workspace || a->workspace_bytes < need || !aligned16(a->workspace))
    return fail(WMX_E_WORKSPACE, "kv router needs %lld workspace bytes", (long long)need);
  return launched(wmx::launch_kv_router(*a, (hipStream_t)stream));
}

size_t wmx_kv_router_args_size(void) { return sizeof(wmx_kv_router_args); }

size_t wmx_kv_store_args_size(void) { return sizeof(wmx_kv_store_args); }

size_t wmx_kv_mix_args_size(void) { return sizeof(wmx_kv_mix_args); }

size_t wmx_kv_store_bwd_args_size(void) { return sizeof(wmx_kv_store_bwd_args); }

int64_t wmx_kv_store_bwd_workspace_size(const wmx_kv_store_bwd_args* a) {
  return a ? wmx::kv_store_bwd_workspace_size(*a) : 0;
}

int wmx_kv_store_bwd(const wmx_kv_store_bwd_args* a, void* stream) {
  if (!a) return fail(WMX_E_INVALID, "args is NULL");
  if (a->head_dim != 64 && a->head_dim != 96 && a->head_dim != 128)
    return fail(WMX_E_UNSUPPORTED, "kv store head_dim %d is not 64, 96 or 128", a->head_dim);
  if (a->batch < 0 || a->channels < 0 || a->heads < 0 || a->tokens < 0) return fail(WMX_E_INVALID, "negative shape");
  for (int dt : {a->key_dtype, a->weight_dtype, a->rope_dtype})
    if (dt != WMX_DTYPE_F32 && dt != WMX_DTYPE_BF16) return fail(WMX_E_INVALID, "dtype must be WMX_DTYPE_F32 or WMX_DTYPE_BF16");
  if (!(a->eps >= 0.f)) return fail(WMX_E_INVALID, "eps must be >= 0");
  if (a->channels == 0) return WMX_OK;
  if (!a->k_norm_weight || !a->grad_weight) return fail(WMX_E_INVALID, "kv store backward pointer is NULL");
  const int64_t need = wmx::kv_store_bwd_workspace_size(*a);
  if (need > 0) {
    if (!a->key || !a->grad_out || !a->cos || !a->sin || !a->grad_key || !a->workspace)
      return fail(WMX_E_INVALID, "kv store backward pointer is NULL");
    if (a->workspace_bytes < need) return fail(WMX_E_WORKSPACE, "workspace %lld < %lld bytes", (long long)a->workspace_bytes, (long long)need);
  }
  if (!aligned16(a->key) || !aligned16(a->grad_out) || !aligned16(a->k_norm_weight) || !aligned16(a->cos) ||
      !aligned16(a->sin) || !aligned16(a->grad_key) || !aligned16(a->workspace) || !aligned16(a->grad_weight))
    return fail(WMX_E_INVALID, "kv store backward operands must be 16-byte aligned");
  if (!strides_vec8(a->key_stride, 4) || !strides_vec8(a->grad_out_stride, 4) || !strides_vec8(a->grad_key_stride, 4) ||
      !strides_vec8(a->rope_stride, 2))
    return fail(WMX_E_INVALID, "kv store backward strides must be multiples of 8 elements");
  return launched(wmx::launch_kv_store_bwd(*a, (hipStream_t)stream));
}

size_t wmx_strict_meta_args_size(void) { return sizeof(wmx_strict_meta_args); }


int64_t wmx_strict_meta_workspace_size(const wmx_strict_meta_args* a) {
  return a ? wmx::strict_meta_workspace_size(*a) : 0;
}

int wmx_strict_meta_count(const wmx_strict_meta_args* a, void* stream) {
  if (const int rc = check_strict_meta(a, false)) return rc;
  return launched(wmx::launch_strict_meta(*a, false, (hipStream_t)stream));
}

int wmx_strict_meta_fill(const wmx_strict_meta_args* a, void* stream) {
  if (const int rc = check_strict_meta(a, true)) return rc;
  return launched(wmx::launch_strict_meta(*a, true, (hipStream_t)stream));
}

int wmx_dense_units(const wmx_attn_args* a, int32_t* units, void* stream) {
  if (!a) return fail(WMX_E_INVALID, "args is NULL");
  if (a->batch < 0 || a->q_len < 0 || a->kv_len < 0) return fail(WMX_E_INVALID, "negative shape");
  if (a->query_indices || a->q_seg) return fail(WMX_E_INVALID, "work lists of dense problems only");
  if (a->query_stride < 1) return fail(WMX_E_INVALID, "query_stride must be >= 1");
  if (a->query_tile != 0 && a->query_tile != 128 && a->query_tile != 256)
    return fail(WMX_E_INVALID, "query_tile must be 0, 128 or 256");
  const int64_t tile = a->query_tile == 256 ? 256 : 128;
  const int64_t n = (int64_t)a->batch * ((a->q_len + tile - 1) / tile);
  if (n > INT32_MAX / 2) return fail(WMX_E_UNSUPPORTED, "work list of %lld units is too long", (long long)n);
  if (n > 0 && !units) return fail(WMX_E_INVALID, "units pointer is NULL");
  return launched(wmx::launch_dense_units(*a, units, (hipStream_t)stream));
}

size_t wmx_feedback_meta_args_size(void) { return sizeof(wmx_feedback_meta_args); }

int64_t wmx_feedback_meta_workspace_size(const wmx_feedback_meta_args* args) {
  return args ? wmx::feedback_meta_workspace_size(*args) : 0;
}

int wmx_feedback_meta(const wmx_feedback_meta_args* a, void* stream) {
  if (const int rc = check_feedback_meta(a)) return rc;
  return launched(wmx::launch_feedback_meta(*a, (hipStream_t)stream));
}

int64_t wmx_decode_workspace_size(const wmx_decode_args* args) {
  return args ? wmx::decode_workspace_size(*args) : 0;
}

int32_t wmx_decode_num_splits(const wmx_decode_args* args) { return args ? wmx::decode_num_splits(*args) : 0; }

int wmx_decode(const wmx_decode_args* a, void* stream) {
  if (const int rc = check_decode(a)) return rc;
  const int64_t need = wmx::decode_workspace_size(*a);
  if (!a->workspace || a->workspace_bytes < need || !aligned16(a->workspace))
    return fail(WMX_E_WORKSPACE, "decode needs %lld workspace bytes", (long long)need);
  if (a->batch == 0 || a->capacity == 0) {
    // nothing visible: the caller's zero-filled output stands
    return WMX_OK;
  }
  return launched(wmx::launch_decode(*a, (hipStream_t)stream));
}

int wmx_decode_noalloc(const wmx_decode_args* a, void* stream) {
  if (const int rc = check_decode(a)) return rc;
  wmx_decode_args b = *a;
  if (wmx::decode_workspace_size(b) > kDecodeScratchBytes) {
    // fewer splits, so that their partials fit the scratch (one split needs
    // none: it writes the output itself)
    const int64_t per_split = (int64_t)b.batch * b.q_heads * (b.head_dim + 2) * (int64_t)sizeof(float);
    const int64_t fit = kDecodeScratchBytes / per_split;
    b.num_splits = (int32_t)(fit < 1 ? 1 : fit);
  }
  if (b.batch == 0 || b.capacity == 0) return WMX_OK;
  void* ptr = nullptr;
  if (const int rc = decode_scratch(stream, &ptr)) return rc;
  b.workspace = ptr;
  b.workspace_bytes = kDecodeScratchBytes;
  b.counters = nullptr;  // the splits are merged by a second kernel
  return launched(wmx::launch_decode(b, (hipStream_t)stream));
}

}  // extern "C"
