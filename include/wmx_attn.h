/*
 * wmx_attn.h - C ABI of the MI355X (gfx950) attention library libwmx_attn.so.
 *
 * The library holds the hand-written CDNA4 HIP kernels behind WhiteMatter's
 * two attention operators, `cyclic_attention` and `strict_causal_attention`.
 * Every entry point:
 *   - takes plain device pointers, element strides and sizes (no C++ types),
 *   - launches asynchronously on the given hipStream_t (passed as void*),
 *   - allocates nothing: outputs and workspaces come from the caller,
 *   - returns 0 on success or a negative WMX_E* code; wmx_last_error() then
 *     returns a thread-local message naming the failed check.
 *
 * Tensors are bf16 (Q/K/V/O and gradients) with unit stride along head_dim.
 * Logical shapes follow the reference operators: Q (B, Hq, Tq, D) and
 * K/V (B, Hkv, Tk, D) with Hq % Hkv == 0; query head h reads KV head h / (Hq/Hkv).
 *
 * Reference interfaces replaced (paths in Cy-47/White-Matter):
 *   wmx_attn_fwd      src/white_matter/ops/cyclic_attention/_tilelang/registration.py:123-140
 *                     (TileLang kernels forward.py:15-133, document_forward.py:17-165),
 *                     src/white_matter/ops/strict_causal_attention.py:397-442
 *                     (flash_attn_varlen_func / TorchFlashVarlen / flash_attn_func),
 *                     src/white_matter/ops/flash_attention.py:125-145,170-211
 *   wmx_attn_bwd_preprocess
 *                     src/white_matter/ops/cyclic_attention/_tilelang/backward_preprocess.py:34-49
 *   wmx_attn_bwd      src/white_matter/ops/cyclic_attention/_tilelang/registration.py:143-161
 *                     (backward_query.py, backward_key_value.py, document_backward_*.py),
 *                     src/white_matter/ops/flash_attention.py:147-167,213-236
 *   wmx_decode        src/white_matter/ops/flash_attention.py:15-49 (flash_attn_with_kvcache),
 *                     src/white_matter/ops/flash_attention.py:52-103 (torch_flash_decode),
 *                     src/white_matter/ops/strict_causal_attention.py:238-263,338-358
 */
#ifndef WMX_ATTN_H
#define WMX_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WMX_ABI_VERSION 13

enum {
  WMX_OK = 0,
  WMX_E_INVALID = -1,     /* argument check failed */
  WMX_E_UNSUPPORTED = -2, /* head_dim or layout the kernels do not implement */
  WMX_E_WORKSPACE = -3,   /* workspace missing or too small */
  WMX_E_LAUNCH = -4       /* HIP reported an error at launch */
};

/*
 * Arguments shared by the forward and backward entry points.
 *
 * Visibility of key slot j to query row i (all modes):
 *   j <= lim(i), lim(i) = min(offset_b + query_stride * i, limit_b)
 *   or (keep_slot0 and j == 0),
 *   and key_mask[b, j] when key_mask is given,
 *   and the document rule when q_seg/k_seg/q_start/k_qend are given:
 *   (q_seg[i] == k_seg[j] and j >= q_start[i] or k_seg[j] == -1) and i < k_qend[j].
 * offset_b is row_offset[b] when row_offset is given, else query_offset;
 * limit_b is row_limit[b] when row_limit is given, else unbounded.
 * Rows with no visible key produce a zero output, lse = +inf and zero gradients.
 *
 * Varlen mode (query_indices != NULL): segment s holds queries
 * query_indices[cu_queries[s] : cu_queries[s+1]] (flat b * query_extent + t)
 * and keys key_indices[cu_keys[s] : cu_keys[s+1]] (flat b * key_extent + slot);
 * local key j is visible to local query i iff
 * j <= (nk - 1) - query_stride * (nq - 1 - i): the segment's last query sees
 * all its keys, each earlier query query_stride fewer (bottom-right causal at
 * query_stride 1; strided cyclic queries of one document above 1; query_offset
 * is unused). Output rows not named by any segment are left untouched, so
 * callers zero-fill o/dq/dk/dv first.
 */
typedef struct wmx_attn_args {
  const void* q;
  const void* k;
  const void* v;
  void* o;              /* bf16, logical (B, Hq, Tq, D), strides o_stride */
  float* lse;           /* fp32 (B, Hq, Tq) contiguous; natural log; +inf for empty rows */
  const void* dout;     /* bf16 gradient of o, strides do_stride (backward only) */
  float* delta;         /* fp32 (B, Hq, Tq) contiguous; rowsum(dout * o) (backward) */
  void* dq;
  void* dk;
  void* dv;
  void* workspace;      /* device scratch for the backward (see wmx_attn_bwd_workspace_size) */
  int64_t workspace_bytes;
  /* element strides [batch, head, token]; head_dim stride is 1 */
  int64_t q_stride[3];
  int64_t k_stride[3];
  int64_t v_stride[3];
  int64_t o_stride[3];
  int64_t do_stride[3];
  int64_t dq_stride[3];
  int64_t dk_stride[3];
  int64_t dv_stride[3];
  int32_t batch;
  int32_t q_heads;
  int32_t kv_heads;
  int32_t q_len;
  int32_t kv_len;
  int32_t head_dim;     /* 64, 96 or 128 */
  int32_t query_stride;
  int32_t query_offset;
  const int32_t* row_offset;  /* optional (B,) */
  const int32_t* row_limit;   /* optional (B,) */
  const uint8_t* key_mask;    /* optional (B, Tk) bool rows */
  int64_t key_mask_stride;
  int32_t keep_slot0;
  int32_t keys_unique;        /* varlen: 1 = no key row appears in two segments;
                               * 2 = only slot 0 of a batch row (a leading dummy
                               * every segment of the row holds) repeats: its
                               * dK/dV go through fp32 accumulators, the other
                               * rows are stored directly; 0 = any row may repeat
                               * (fp32 accumulators for all) */
  const int32_t* q_seg;       /* optional cyclic document metadata, int32 contiguous */
  const int32_t* k_seg;
  const int32_t* q_start;
  const int32_t* k_qend;
  const int64_t* query_indices;  /* optional varlen schedule */
  const int64_t* key_indices;
  const int32_t* cu_queries;
  const int32_t* cu_keys;
  int32_t num_segments;
  int32_t max_queries;        /* largest segment query count */
  int32_t max_keys;           /* largest segment key count */
  int32_t query_extent;       /* T: row width of flat query indices */
  int32_t key_extent;         /* N: row width of flat key indices */
  int32_t segment_layout;     /* varlen bit 0: each segment's queries are consecutive
                                 slots of one row; bit 1: its keys 1.. are consecutive
                                 slots following key 1 (key 0 may be the dummy) */
  float softmax_scale;
  /* Optional work lists, [count][2] int32 (segment or batch row, 128-row
   * tile), in the order the kernels should take them (heaviest first). With
   * them the kernels visit exactly these units; without them every (segment,
   * tile < max / 128) pair, most of which are empty for short segments, or
   * every (batch row, tile) pair from the last tile down. k_units needs a
   * varlen schedule. */
  const int32_t* q_units;     /* query tiles: forward and dQ */
  const int32_t* k_units;     /* key tiles: dK/dV */
  int32_t num_q_units;
  int32_t num_k_units;
  /* Optional varlen dS layout (see wmx_attn_bwd_workspace_size), int64
   * [num_segments + 1]: segment s's dS block starts ds_offsets[s] elements
   * into each query head's region and holds keys(s) x pad128(queries(s))
   * elements, ds_offsets[0] = 0, ds_elements = ds_offsets[num_segments].
   * NULL: varlen backward passes recompute dQ without a dS buffer. */
  const int64_t* ds_offsets;
  int64_t ds_elements;
  /* Forward query rows per workgroup: 0 or 128 (4 waves), or 256 (8 waves:
   * each key/value tile serves twice the rows, for few query tiles over long
   * key ranges such as a chunk after a cached prefix). q_units tiles count in
   * these rows. The backward kernels are unaffected. */
  int32_t query_tile;
  /* Ints per entry of q_units and k_units: 0 or 2 for (segment or batch row,
   * tile) pairs; WMX_UNIT_FIELDS (varlen schedules only) for entries that
   * also carry their segment's bounds, so a workgroup reads one entry instead
   * of cu_queries, cu_keys and the index arrays one after another (fields
   * below; the row and slots are those of the segment's index elements 0 and
   * 1, slot 1 being slot 0 + 1 for a one-element side; the dS offset is
   * ds_offsets[segment] as two int32 halves). */
  int32_t unit_fields;
  /* dK/dV key rows per workgroup: 0 or 128 (eight waves, one workgroup per
   * CU), or 64 (four waves, two workgroups per CU: one workgroup's setup
   * overlaps the other's tile loop). k_units tiles count in these rows. */
  int32_t key_tile;
  /* Optional fused backward of short segments (13th ABI revision; varlen,
   * q_heads == kv_heads, keys_unique 1 or 2, entries of WMX_UNIT_FIELDS ints
   * as unit_fields): one workgroup per listed segment and head holds all of
   * its queries (1 .. 128) and computes its dQ, dK and dV in one pass over its
   * keys (at least one), without the dS buffer. The backward then runs the
   * key- and query-tiled kernels on k_units and q_units only, which must be
   * given and must not name the listed segments; the forward ignores f_units.
   * Heaviest first (most 64-key tiles). */
  const int32_t* f_units;
  int32_t num_f_units;
} wmx_attn_args;

enum {
  WMX_UNIT_SEGMENT = 0,
  WMX_UNIT_TILE = 1,
  WMX_UNIT_QUERY_START = 2, /* cu_queries[segment] */
  WMX_UNIT_QUERIES = 3,
  WMX_UNIT_KEY_START = 4,   /* cu_keys[segment] */
  WMX_UNIT_KEYS = 5,
  WMX_UNIT_QUERY_ROW = 6,   /* query_indices[start] / query_extent */
  WMX_UNIT_QUERY_SLOT0 = 7,
  WMX_UNIT_QUERY_SLOT1 = 8,
  WMX_UNIT_KEY_ROW = 9,     /* key_indices[start] / key_extent */
  WMX_UNIT_KEY_SLOT0 = 10,
  WMX_UNIT_KEY_SLOT1 = 11,
  WMX_UNIT_DS_LO = 12,      /* ds_offsets[segment], low and high 32 bits */
  WMX_UNIT_DS_HI = 13,
  WMX_UNIT_FIELDS = 16
};

/*
 * Single-query decode over a KV pool (no gradient).
 * Query head h of row b attends to slots j of KV head h / (Hq/Hkv) with
 *   j < len_b,  len_b = clamp(min(start_b, kvlen_b), 0, capacity - dummy) + dummy,
 * or, when key_mask is given, key_mask[b, j] and j < min(start_b, kvlen_b) + dummy.
 * start_b is query_start[b] when given, else query_start_scalar; kvlen_b is
 * kv_lengths[b] when given, else unbounded.
 * The work is split over num_splits key ranges per (b, kv head) whose partial
 * (o, max, sum) rows live in the workspace and are merged by the last split
 * to finish (with counters) or by a second kernel (without).
 */
typedef struct wmx_decode_args {
  const void* q;        /* bf16 (B, Hq, 1, D) */
  const void* k;        /* bf16 (B, Hkv, capacity, D) */
  const void* v;
  void* o;              /* bf16 output, logical (B, Hq, D) */
  const int64_t* query_start;   /* optional (B,) int64 */
  const int64_t* kv_lengths;    /* optional (B,) int64 */
  const uint8_t* key_mask;      /* optional (B, capacity) bool rows */
  int64_t key_mask_stride;
  void* workspace;
  int64_t workspace_bytes;
  int64_t q_stride[2];  /* [batch, head] */
  int64_t k_stride[3];  /* [batch, head, slot] */
  int64_t v_stride[3];
  int64_t o_stride[2];  /* [batch, head] */
  int64_t query_start_scalar;
  int32_t batch;
  int32_t q_heads;
  int32_t kv_heads;
  int32_t capacity;
  int32_t head_dim;
  int32_t use_dummy;
  int32_t num_splits;   /* <= 0: chosen by the library */
  float softmax_scale;
  /* Optional, batch * kv_heads int32, zero on entry and left zero: with it
   * the last split of each (row, KV head) to finish merges the splits (one
   * launch per call) where the launch is short (at most 1024 workgroups, 64
   * splits); otherwise, and without it, a second kernel does. The outputs are
   * bit-identical. Calls that share counters must not overlap (calls in
   * order on one stream do not). */
  int32_t* counters;
  /* Nonzero: query_start[0] and kv_lengths[0] hold every row's values (a
   * pool's one shared length read in place, without a per-row copy). */
  int32_t lengths_broadcast;
} wmx_decode_args;

/*
 * KV-pool store: the step that writes a group's keys and values into the
 * pool (reference modules/kv_pool.py:163-172 `_apply_k_norm_rope` and the
 * `.to(V.dtype)` cast of :216, then blocks/_execution/cyclic.py:448-458
 * `_write_pool`'s two index_copy_ along the token axis). For every row
 * (b, c, h, t):
 *   x  = key[b, c, h, t, :]
 *   y  = r(x * rsqrt(mean(x^2) + eps))            (the mean in fp32)
 *   y  = r(y * r(w[c, :]))
 *   k' = r(r(y * r(cos[b, t, :])) + r(rot(y) * r(sin[b, t, :])))
 *        rot(y) = (-y[D/2:], y[:D/2])
 *   key_pool[b, c, h, slots[t], :]   = bf16(k')
 *   value_pool[b, c, h, slots[t], :] = bf16(value[b, c, h, t, :])
 * where r() rounds to the key dtype (identity for fp32), as the reference
 * evaluates each step in the key dtype. Slots must be distinct; a slot
 * outside [0, N) is not written. value and value_pool may both be NULL
 * (keys only).
 */
enum { WMX_DTYPE_F32 = 0, WMX_DTYPE_BF16 = 1 };

typedef struct wmx_kv_store_args {
  const void* key;           /* (B, C, H, T, D), dtype key_dtype */
  const void* value;         /* (B, C, H, T, D), dtype value_dtype, or NULL */
  const void* k_norm_weight; /* (C, D) contiguous, dtype weight_dtype */
  const void* cos;           /* (B, T, D), dtype rope_dtype */
  const void* sin;           /* same shape and strides as cos */
  void* key_pool;            /* bf16 (B, C, H, N, D) */
  void* value_pool;          /* bf16 (B, C, H, N, D), or NULL */
  const int64_t* slots;      /* (T) pool slot of token t, in [0, N) */
  /* element strides; head_dim stride is 1 */
  int64_t key_stride[4];     /* [batch, channel, head, token] */
  int64_t value_stride[4];
  int64_t key_pool_stride[4];
  int64_t value_pool_stride[4];
  int64_t rope_stride[2];    /* [batch, token] */
  int32_t key_dtype;         /* WMX_DTYPE_F32 or WMX_DTYPE_BF16 */
  int32_t value_dtype;
  int32_t weight_dtype;
  int32_t rope_dtype;
  int32_t batch;
  int32_t channels;
  int32_t heads;
  int32_t tokens;
  int32_t head_dim;          /* 64, 96 or 128 */
  int32_t pool_slots;        /* N */
  float eps;
  /* Nonzero: cos and sin are (N, D) tables of rows by pool slot, and token t
   * of every batch row reads row slots[t] (rope_stride[1] apart; rope_stride[0]
   * is unused), so a decode step needs no gather of its rows. */
  int32_t rope_by_slot;
} wmx_kv_store_args;

/*
 * Gradient of the store's key transform k' = rope(rms_norm(key) * w[c]) for
 * training (the autograd of the reference's `_apply_k_norm_rope` and its cast,
 * modules/kv_pool.py:163-172, 216). With g = grad_out[b, c, h, t, :] and the
 * forward's y = x / sqrt(mean(x^2) + eps), u = y * w[c]:
 *   du = g * cos + rot^T(g * sin),  rot^T(z) = (z[D/2:], -z[:D/2])
 *   grad_key  = (du * w[c] - y * mean(du * w[c] * y)) / sqrt(mean(x^2) + eps)
 *   grad_weight[c, :] = sum over b, h, t of du * y
 * in fp32 (no intermediate rounding). grad_weight is summed through
 * per-workgroup parts in the workspace in a fixed order: the same bits on
 * every run.
 */
typedef struct wmx_kv_store_bwd_args {
  const void* key;            /* (B, C, H, T, D) forward input, dtype key_dtype */
  const void* grad_out;       /* bf16 (B, C, H, T, D): gradient of the bf16 keys */
  const void* k_norm_weight;  /* (C, D) contiguous, dtype weight_dtype */
  const void* cos;            /* (B, T, D), dtype rope_dtype */
  const void* sin;            /* same shape and strides as cos */
  void* grad_key;             /* (B, C, H, T, D), dtype key_dtype */
  float* grad_weight;         /* fp32 (C, D) contiguous, overwritten */
  void* workspace;            /* wmx_kv_store_bwd_workspace_size bytes */
  int64_t workspace_bytes;
  int64_t key_stride[4];      /* element strides [batch, channel, head, token] */
  int64_t grad_out_stride[4];
  int64_t grad_key_stride[4];
  int64_t rope_stride[2];     /* [batch, token] */
  int32_t key_dtype;          /* WMX_DTYPE_F32 or WMX_DTYPE_BF16 */
  int32_t weight_dtype;
  int32_t rope_dtype;
  int32_t batch;
  int32_t channels;
  int32_t heads;
  int32_t tokens;
  int32_t head_dim;           /* 64, 96 or 128 */
  float eps;
} wmx_kv_store_bwd_args;

/*
 * KV-pool producer, the token-local steps ahead of the per-channel projection
 * (reference modules/kv_pool.py:97-160 `KVPool._project`, the bf16 inference
 * form of :108-136; modules/routing.py:77-124 `Router.forward`,
 * `_RoutedMixer.forward`). For token n = b * T + t with sources
 * x[s] = sources[b, t, s, :] (S rows of `hidden`) and each side (0 K, 1 V):
 *   wmx_kv_premix:
 *     premixed[side][n, s, :] = bf16(x[s] * (1 / sqrt(mean(x[s]^2) + eps)) * pre_mix[side][s, :])
 *   the router logits alpha[side][n, c * S + s] are the caller's GEMM of the
 *   premixed row (B*T, S*hidden) by the router weight, plus its bias;
 *   wmx_kv_mix:
 *     m = bf16(sum over s ascending of alpha[side][n, c * S + s] * premixed[side][n, s, :])
 *     mixed[side][c, n, :] = bf16(m * (1 / sqrt(mean(m^2) + mix_eps)) * gain[side][c, :])
 * with fp32 arithmetic throughout (the sources are read as fp32 whatever their
 * dtype). mixed[side] is the (C, B*T, hidden) input of the per-channel
 * projection GEMM.
 */
#define WMX_KV_MIX_MAX_SOURCES 512
#define WMX_KV_MIX_MAX_HIDDEN 4096

typedef struct wmx_kv_mix_args {
  const void* sources;        /* (B, T, S, hidden), dtype source_dtype, unit stride along hidden */
  int64_t source_stride[3];   /* element strides [batch, token, source]; 0 repeats one row */
  const void* pre_mix[2];     /* (S, hidden) contiguous, dtype weight_dtype: K side, V side */
  void* premixed[2];          /* bf16 (B*T, S*hidden) contiguous */
  const void* alpha[2];       /* bf16 (B*T, C*S), rows alpha_stride elements apart */
  int64_t alpha_stride;
  const void* gain[2];        /* (C, hidden) contiguous, dtype weight_dtype */
  void* mixed[2];             /* bf16 (C, B*T, hidden) contiguous */
  int32_t source_dtype;       /* WMX_DTYPE_F32 or WMX_DTYPE_BF16 */
  int32_t weight_dtype;       /* of pre_mix and gain */
  int32_t batch;
  int32_t tokens;
  int32_t num_sources;        /* S, 1 .. WMX_KV_MIX_MAX_SOURCES */
  int32_t hidden;             /* a multiple of 8, at most WMX_KV_MIX_MAX_HIDDEN */
  int32_t channels;           /* C >= 1 */
  float eps;
  float mix_eps;
} wmx_kv_mix_args;

/*
 * The router logits between the two producer steps, for both sides in one
 * launch: alpha[side] = bf16(premixed[side] . weight[side]^T + bias[side])
 * (reference modules/routing.py:77-115 `Router.forward`, the bf16 nn.Linear
 * over the premixed row). Each workgroup multiplies 128 rows by all logits
 * over one 1024-input chunk on the MFMA units (fp32 sums of bf16 products);
 * the chunks' fp32 partial sums go to the workspace and a second kernel adds
 * them in chunk order with the bias and rounds once to bf16. The library GEMM
 * of this shape (few logits, long inputs) runs on 32 workgroups.
 */
#define WMX_KV_ROUTER_MAX_LOGITS 256

typedef struct wmx_kv_router_args {
  const void* premixed[2];    /* bf16 (rows, inputs) contiguous, K side and V side */
  const void* weight[2];      /* bf16 (logits, inputs) contiguous */
  const void* bias[2];        /* bf16 (logits,), or NULL for none */
  void* alpha[2];             /* bf16 (rows, logits) contiguous */
  void* workspace;            /* wmx_kv_router_workspace_size bytes, 16-byte aligned */
  int64_t workspace_bytes;
  int32_t rows;               /* B*T */
  int32_t inputs;             /* the product's width, a positive multiple of 64 */
  int32_t logits;             /* C*S, 1 .. WMX_KV_ROUTER_MAX_LOGITS */
  /* The reference Router's strided source view (modules/routing.py:46-99,
   * router_layer_stride): with source_width > 0 a row's inputs are its
   * blocks of source_width elements at sources source_start,
   * source_start + source_stride, ... (inputs / source_width of them), read
   * in place from the premixed rows, row_stride elements apart. With
   * source_width 0 the inputs are a row's first `inputs` elements and rows
   * are `inputs` apart (row_stride ignored). source_width is a multiple of 64. */
  int32_t row_stride;
  int32_t source_width;
  int32_t source_start;
  int32_t source_stride;
} wmx_kv_router_args;

/*
 * Packed-document schedule builder on the device: the reference's
 * prepare_strict_causal_metadata (ops/strict_causal_attention.py:75-155),
 * whose torch sequence synchronises with the host at every data-dependent
 * size (the position check, three nonzero, repeat_interleave). Here two
 * kernels (one workgroup per batch row) share one workspace:
 *   wmx_strict_meta_count  per-slot ranks, run-start ranks and the rank -> slot
 *                          map, the row's valid queries compacted, and
 *                          counts[b] = {valid queries, segments, keys,
 *                          1 if a query position lies outside [0, extent)};
 *   wmx_strict_meta_fill   (after the caller has read counts, checked the flag
 *                          and allocated the outputs) query_indices,
 *                          key_indices, cu_queries and cu_keys, rows in order.
 * Outputs are bit-identical to the reference's: query i of row b is
 * b * query_length + i; key index b * (extent + use_dummy) + slot (+1 past
 * the dummy, which is slot 0 and every segment's first key).
 */
enum { WMX_DTYPE_I32 = 2, WMX_DTYPE_I64 = 3 };

typedef struct wmx_strict_meta_args {
  const void* document_ids;   /* (B, extent) of doc_dtype, rows doc_stride elements apart */
  const int64_t* query_start; /* (B) first query slot per row, or NULL: query_start_scalar */
  const int64_t* kv_lengths;  /* (B) or NULL */
  void* workspace;            /* wmx_strict_meta_workspace_size bytes, 16-byte aligned */
  int64_t* counts;            /* (B, 4), written by count, read by fill */
  int64_t* query_indices;     /* fill: sum of counts[:, 0] */
  int64_t* key_indices;       /* fill: sum of counts[:, 2] */
  int32_t* cu_queries;        /* fill: sum of counts[:, 1] + 1 */
  int32_t* cu_keys;           /* fill: sum of counts[:, 1] + 1 */
  int64_t doc_stride;
  int64_t query_start_scalar;
  int64_t workspace_bytes;
  int32_t doc_dtype;          /* WMX_DTYPE_I32 or WMX_DTYPE_I64 */
  int32_t batch;
  int32_t extent;
  int32_t query_length;
  int32_t use_dummy;          /* 0 or 1 */
} wmx_strict_meta_args;

/*
 * Per-residue cyclic metadata of packed documents on the device: replaces the
 * reference's prepare_feedback_metadata (blocks/_execution/metadata.py:11-55),
 * its torch sequence (cummax / flipped cummin run bounds, index_select, div)
 * issued once per residue. One kernel, one workgroup per batch row, no host
 * synchronisation. For the groups r = group_base .. group_base + group_count - 1
 * of G = groups (the model's query tokens r, r + G, ...; any slots here), with
 * d = use_dummy and runs = maximal sequences of equal ids in a row:
 *   key_ids[b, j]                -1 for j < d, else id(token j - d), negative as -2
 *   key_query_end[g, b, j]       count_g for j < d, else
 *                                min(ceil(max(run_end(j - d) - r, 0) / G), count_g)
 *   query_ids[B*o_g + b*count_g + i]        id(slots[o_g + i]), negative as -2
 *   query_key_start[B*o_g + b*count_g + i]  run_start(slots[o_g + i]) + d
 * with o_g = group_offsets[g], count_g = o_{g+1} - o_g (group g's outputs are a
 * contiguous (B, count_g) block). Slots outside [0, length) give -2 and 0.
 */
#define WMX_FEEDBACK_MAX_GROUPS 64

typedef struct wmx_feedback_meta_args {
  const void* document_ids;   /* (B, length) of doc_dtype, rows doc_stride elements apart */
  const int64_t* slots;       /* the groups' query slots, group g at [group_offsets[g], group_offsets[g+1]) */
  void* workspace;            /* wmx_feedback_meta_workspace_size bytes (per-token run bounds) */
  int32_t* key_ids;           /* (B, key_length) */
  int32_t* key_query_end;     /* (group_count, B, key_length) */
  int32_t* query_ids;         /* B * group_offsets[group_count] */
  int32_t* query_key_start;   /* B * group_offsets[group_count] */
  int64_t doc_stride;
  int64_t workspace_bytes;
  int64_t group_offsets[WMX_FEEDBACK_MAX_GROUPS + 1]; /* group_offsets[0] = 0, nondecreasing */
  int32_t doc_dtype;          /* WMX_DTYPE_I32 or WMX_DTYPE_I64 */
  int32_t batch;
  int32_t length;
  int32_t key_length;         /* <= length + use_dummy */
  int32_t groups;             /* G >= 1: the cyclic stride */
  int32_t group_base;         /* residue of this call's first group */
  int32_t group_count;        /* 1 .. WMX_FEEDBACK_MAX_GROUPS */
  int32_t use_dummy;          /* 0 or 1 */
} wmx_feedback_meta_args;

/* Library identity and struct layout checks for FFI bindings. */
int wmx_abi_version(void);
size_t wmx_attn_args_size(void);
size_t wmx_decode_args_size(void);
size_t wmx_kv_store_args_size(void);
size_t wmx_kv_mix_args_size(void);
size_t wmx_kv_store_bwd_args_size(void);
size_t wmx_kv_router_args_size(void);
size_t wmx_strict_meta_args_size(void);
size_t wmx_feedback_meta_args_size(void);
const char* wmx_last_error(void);

/* Forward: o and lse. (see replaced interfaces above) */
int wmx_attn_fwd(const wmx_attn_args* args, void* stream);

/* Work list of a dense problem (no varlen schedule, no documents) for
 * args->q_units: the (batch row, query tile) pairs, tiles of query_tile rows
 * (128 when 0), ordered by how many 64-key tiles their rows reach under
 * query_offset / row_offset / row_limit / query_stride, largest first,
 * written as int32 pairs to units[0 .. 2 * batch * ceil(q_len / tile)).
 * One kernel on the stream, no host synchronisation; the order of units with
 * equal loads is unspecified. Replaces the host-side ordering a ragged
 * prefill would need (the reference's FlashAttention varlen call orders its
 * own work: ops/strict_causal_attention.py:443-458). */
int wmx_dense_units(const wmx_attn_args* args, int32_t* units, void* stream);

/* delta[b,h,i] = sum_d dout[b,h,i,d] * o[b,h,i,d] in fp32. */
int wmx_attn_bwd_preprocess(const wmx_attn_args* args, void* stream);

/* Workspace bytes for the fastest backward of these arguments (0 when it
 * needs none): the fp32 dK/dV accumulators of varlen schedules whose key rows
 * repeat (required), then, from a 256-byte aligned offset, the bf16 dS
 * buffer that the dK/dV kernel writes and the dQ kernel reads (a
 * keys x pad128(queries) block per batch row or segment and query head; for
 * varlen schedules laid out by ds_offsets) when it totals at most 4 GiB.
 * wmx_attn_bwd_min_workspace_size is the required part: a workspace between
 * the two sizes runs the backward without the dS buffer, recomputing S and
 * dP in the dQ kernel. */
int64_t wmx_attn_bwd_workspace_size(const wmx_attn_args* args);
int64_t wmx_attn_bwd_min_workspace_size(const wmx_attn_args* args);

/* Backward: delta, then dk and dv (and dS), then dq (with a dS buffer), or
 * delta, dq, dk and dv (without). */
int wmx_attn_bwd(const wmx_attn_args* args, void* stream);

/* The two halves of wmx_attn_bwd, for callers that schedule or time them
 * separately; both read the delta that wmx_attn_bwd_preprocess wrote.
 * wmx_attn_bwd_dkv writes dk/dv (key-parallel) and, with a dS workspace, dS;
 * wmx_attn_bwd_dq writes dq (query-parallel) from that dS, so it runs after
 * wmx_attn_bwd_dkv on the same workspace (without a dS workspace it
 * recomputes and has no order). */
int wmx_attn_bwd_dq(const wmx_attn_args* args, void* stream);
int wmx_attn_bwd_dkv(const wmx_attn_args* args, void* stream);

/* Workspace bytes wmx_decode needs, and the split count it will use. */
int64_t wmx_decode_workspace_size(const wmx_decode_args* args);
int32_t wmx_decode_num_splits(const wmx_decode_args* args);

/* Single-query decode forward. */
int wmx_decode(const wmx_decode_args* args, void* stream);

/*
 * wmx_decode without a workspace: the split-K partials go to a static device
 * array of WMX_DECODE_NOALLOC_MAX_BYTES that the library holds on each GPU it
 * runs on until the process ends (args->workspace, workspace_bytes and
 * counters are ignored; a second kernel merges the splits). No counterpart in
 * the reference: this entry point is for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc). It calls no allocating routine. The partials of s splits take
 * batch * q_heads * s * (head_dim + 2) * 4 bytes; where the split count
 * wmx_decode would use (wmx_decode_num_splits) needs more than the maximum,
 * this call uses the largest count that fits (at least one: a single split
 * needs no scratch), and its outputs then differ from wmx_decode's by the
 * summation order of the splits; otherwise they are bit-identical. Every call
 * on one GPU shares that GPU's array, so calls that overlap on one GPU
 * (concurrent streams, or threads) race; calls in order on one stream do not.
 * The array's first use on a device resolves its address there
 * (hipGetSymbolAddress) with that device current; the stream must belong to
 * the current device.
 */
#define WMX_DECODE_NOALLOC_MAX_BYTES ((int64_t)8 << 20)
int wmx_decode_noalloc(const wmx_decode_args* args, void* stream);

/* KV-pool store (see wmx_kv_store_args): one pass over the group's keys and
 * values, writing the pool slots. Replaces the reference's eager sequence of
 * rms_norm, weight, RoPE, casts and index_copy_ (modules/kv_pool.py:163-172,
 * 216; blocks/_execution/cyclic.py:448-458). */
int wmx_kv_pool_store(const wmx_kv_store_args* args, void* stream);

/* Backward of the store's key transform (see wmx_kv_store_bwd_args): replaces
 * the autograd of the reference's eager rms_norm, weight and RoPE steps
 * (modules/kv_pool.py:163-172) where training projects keys. */
int64_t wmx_kv_store_bwd_workspace_size(const wmx_kv_store_bwd_args* args);
int wmx_kv_store_bwd(const wmx_kv_store_bwd_args* args, void* stream);

/* KV-pool producer (see wmx_kv_mix_args). wmx_kv_premix replaces the source
 * RMS norm and the pre-mix products with their bf16 casts (reference
 * modules/kv_pool.py:15-19 `_premix`, :103-123); wmx_kv_mix replaces the routed
 * mixture, the mix norm and the gain with its cast and permute (reference
 * modules/routing.py:117-124 `_RoutedMixer.forward`, modules/kv_pool.py:22-25
 * `_projection_input`, :129-136). Outputs are fully overwritten. */
int wmx_kv_premix(const wmx_kv_mix_args* args, void* stream);
int wmx_kv_mix(const wmx_kv_mix_args* args, void* stream);

/* Router logits of both sides (see wmx_kv_router_args): replace the two
 * nn.Linear calls of the reference's routers (modules/routing.py:108-115).
 * The workspace holds 2 x ceil(inputs / 1024) x rows x logits fp32 partial
 * sums. */
int64_t wmx_kv_router_workspace_size(const wmx_kv_router_args* args);
int wmx_kv_router(const wmx_kv_router_args* args, void* stream);

/* Packed-document schedule (see wmx_strict_meta_args): replaces the torch
 * sequence of prepare_strict_causal_metadata (reference
 * ops/strict_causal_attention.py:75-155). */
int64_t wmx_strict_meta_workspace_size(const wmx_strict_meta_args* args);
int wmx_strict_meta_count(const wmx_strict_meta_args* args, void* stream);
int wmx_strict_meta_fill(const wmx_strict_meta_args* args, void* stream);

/* Per-residue cyclic metadata (see wmx_feedback_meta_args): replaces the torch
 * sequence of prepare_feedback_metadata (reference
 * blocks/_execution/metadata.py:11-55). */
int64_t wmx_feedback_meta_workspace_size(const wmx_feedback_meta_args* args);
int wmx_feedback_meta(const wmx_feedback_meta_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* WMX_ATTN_H */
